"""Greedy MTP acceptance on the device, and the drafter call surface (hsd/mtp.py,
hsd/model.py:366-443).

`greedy_accept` replaces the host round trip of model.py:419-427: the target's argmax per
verified row, the number of accepted drafts a (first mismatch, else k), the emitted
tokens draft[:a] + [tgt[a]], and -- when given the shared Mamba ring index -- the
rollback cur += a+1, all queued on the stream.

The MTP head's forward (enorm/hnorm/eh_proj, one attention block, one MoE block,
mtp.py:44-88) is not part of this hot path; `ScriptedDrafter` keeps the head's call
surface (`__call__(h, toks) -> (pred, hn)`, `trim`, `reset`) and proposes scripted
drafts, which is how acceptance is forced in the benchmarks.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as N


def greedy_accept(draft, logits, cur=None, nslab=4):
    """draft [k] int32, logits [k+1, V] (bf16/f16/f32) -> dict of device int32 tensors:
    tgt [k+1] (first argmax per row), tokens [k+1] (emitted, -1 padded), n_accept [1],
    n_keep [1] (= a+1). With `cur` (the Mamba ring index), also applies the rollback."""
    logits = N.contig(logits)
    k = logits.shape[0] - 1
    V = logits.shape[1]
    dev = logits.device
    draft = N.contig(draft.to(torch.int32)) if k > 0 else torch.zeros(1, dtype=torch.int32, device=dev)
    out = {n: torch.empty(s, dtype=torch.int32, device=dev)
           for n, s in (("tgt", k + 1), ("tokens", k + 1), ("n_accept", 1), ("n_keep", 1))}
    N.call("hsd_greedy_accept", N.ptr(logits), N.dtype_tag(logits.dtype), k, V, N.ptr(draft),
           N.ptr(out["tgt"]), N.ptr(out["tokens"]), N.ptr(out["n_accept"]), N.ptr(out["n_keep"]),
           N.ptr(cur), nslab, N.stream(dev))
    return out


class ScriptedDrafter:
    """The MTPHead call surface (mtp.py:67-88) with scripted drafts: for each step the
    drafter is told the true continuation and an accept count, and proposes the true
    tokens for the accepted positions and a guaranteed-wrong token at the first rejected
    one (forced acceptance). hn is passed through unchanged."""

    def __init__(self, vocab: int, n_draft: int = 2):
        self.vocab, self.n_draft = vocab, n_draft
        self.reset()

    def reset(self):
        self.rows = 0

    def trim(self, n):
        """Drop the last n rows of the head's (notional) cache."""
        self.rows = max(0, self.rows - n)

    def script(self, true_next, n_accept):
        """true_next: the next n_draft true tokens; n_accept in [0, n_draft]."""
        d = [int(t) for t in true_next[:self.n_draft]]
        if n_accept < self.n_draft:
            d[n_accept] = (d[n_accept] + 1) % self.vocab
        self._next = d

    def __call__(self, h, toks):
        self.rows += int(h.shape[0])
        d = torch.tensor(self._next, dtype=torch.int32, device=h.device)
        return d, h


def scripted_accepts(n_steps, probs, seed):
    """Accepted-draft counts per step from a seeded categorical (probs over 0..k)."""
    rng = np.random.default_rng(seed)
    return rng.choice(len(probs), size=n_steps, p=np.asarray(probs) / np.sum(probs)).astype(np.int64)
