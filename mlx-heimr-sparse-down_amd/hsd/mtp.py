"""Greedy MTP acceptance on the device, and the drafter call surface (hsd/mtp.py,
hsd/model.py:366-443).

`greedy_accept` replaces the host round trip of model.py:419-427: the target's argmax per
verified row, the number of accepted drafts a (first mismatch, else k), the emitted
tokens draft[:a] + [tgt[a]], and -- when given the shared Mamba ring index -- the
rollback cur += a+1, all queued on the stream.

`MTPHead` is the head's call surface (mtp.py:41-88: `__call__(h, toks) -> (pred, hn)`,
`trim`, `reset`) over a hsd.model.NemotronModel's own one-layer head (enorm/hnorm/eh_proj,
one attention block, one MoE block, final_norm, the target's lm_head and argmax), with
its own KV cache. `ScriptedDrafter` has the same surface and proposes scripted drafts,
which is how acceptance is forced in the benchmarks.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as N


def greedy_accept(draft, logits, cur=None, nslab=4):
    """draft [k] int32, logits [k+1, V] (bf16/f16/f32) -> dict of device int32 tensors:
    tgt [k+1] (first argmax per row), tokens [k+1] (emitted, -1 padded), n_accept [1],
    n_keep [1] (= a+1). With `cur` -- a hsd.mamba.MambaCache (its ring index and slab
    count) or the ring index tensor itself -- also applies the rollback cur += a+1."""
    if hasattr(cur, "cur") and hasattr(cur, "nslab"):
        cur, nslab = cur.cur, cur.nslab
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


class MTPHead:
    """hsd/mtp.py:41-88 on a hsd.model.NemotronModel built with its MTP head (the random
    init's head stands in for the published checkpoint; head_dir is accepted for the
    signature and must be None). prenorm records which hidden state the caller feeds
    (model.py:382): the model's own speculative loop feeds the pre-norm_f state."""

    def __init__(self, target, head_dir=None, prenorm=True):
        if getattr(target, "mtp", None) is None:
            raise N.HSDError("MTPHead needs a NemotronModel built with its MTP head (cfg.mtp)")
        if head_dir is not None:
            raise N.HSDError("the synthetic model's head is built with it; head_dir must be None")
        from . import nn
        self.target, self.prenorm = target, prenorm
        self.eps = target.cfg.eps
        c = target.cfg
        self.kv = nn.KVCache(c.kv_heads, c.max_seq, target.device, c.head_dim)
        self._pos = torch.zeros(1, dtype=torch.int32, device=target.device)
        self._buf = target._make_buffers(3)
        self.bytes = target.mtp.nbytes()
        self.reset()

    def reset(self):
        """An empty KV cache."""
        self.rows = 0
        self._pos.zero_()

    def trim(self, n):
        """Drop the last n rows of the head's cache (the speculative rows after a verify)."""
        self.rows = max(0, self.rows - int(n))
        self._pos.fill_(self.rows)

    def __call__(self, h, toks):
        """h [R, D] bf16: the target's hidden state at R confirmed positions; toks [R]
        int32: the token that follows each row's position -> (pred [R] int32, the argmax
        of the head's logits: the token two positions ahead of each row; hn [R, D] bf16,
        the head's own normed hidden state, for chaining). The rows are appended to the
        head's cache, 3 at a time."""
        from . import nn
        R = h.shape[0]
        if self.rows + R > self.kv.smax:
            raise N.HSDError(f"the head's cache holds {self.kv.smax} rows")
        m, b = self.target, self._buf
        toks = N.contig(toks.to(torch.int32))
        pred = torch.empty(R, dtype=torch.int32, device=h.device)
        hn = torch.empty((R, m.cfg.hidden), dtype=torch.bfloat16, device=h.device)
        st = N.stream(h.device)
        for r0 in range(0, R, 3):
            n = min(3, R - r0)
            x = b["x"][:n]
            x.copy_(h[r0:r0 + n])
            m.mtp_rows(x, toks[r0:r0 + n], b, self.kv, self._pos, keys=b["keys"][:n])
            nn.argmax(b["keys"][:n], n, out=pred[r0:r0 + n])
            hn[r0:r0 + n].copy_(b["hn"][:n])
            N.call("hsd_seq_add", N.ptr(self._pos), 0, n, st)
        self.rows += R
        return pred, hn


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
