"""Sparse MoE down projection for decode on the neuron-major layout (hsd/decode.py).

The down projection of one MoE layer for B token rows,

    y[b] = sum_k gain[b,k] * W_{sel[b,k]} h[b,k] + gain[b,topk] * W_shared h[b,shared],

read only over the neurons whose ReLU^2 activation is nonzero: libhsd's
`hsd_sparse_down_decode` compacts each 64-neuron group's live rows with wave ballots,
reads only those rows' 4-bit words and the group's bf16 scale/bias vectors (if the group
has a live row), accumulates in fp32, and sums the partials in a fixed order.
"""
from __future__ import annotations

import torch

from . import _native as N


def _workspace(nbytes, device, workspace):
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < nbytes:
            raise N.HSDError(f"workspace too small: need {nbytes} bytes")
        return workspace
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def sparse_down(h, sel, gains, pw, ps, pb, spw, sps, spb, *, F, FS, D, topk,
                sl=928, unr=2, nds=3, out_dtype=None, loadsc=1, dense=False,
                live_masks=None, status=None, workspace=None):
    """hsd/decode.py:164-186. Down projection over the live rows only.

    h [B, topk*F + FS] (bf16/f16/f32), sel [B, topk] int32 (the routed experts),
    gains [B, topk+1] f32 (routing scores, then 1 for the shared expert) -> y [B, D]
    (out_dtype, default h.dtype). pw [E, F, D/8], ps/pb [E, F/64, D]; spw [FS, D/8],
    sps/spb [FS/64, D] (hsd.layout.to_neuron_major).

    sl / unr / nds are the reference's Metal tuning knobs; the HIP kernel's geometry is
    fixed (128-output chunks x 8-group parts, 32 parts per token row at the reference
    shape), so they are accepted and ignored.
    dense=True: the dense-h control -- the same kernel reading every row (bit-identical
    result for finite inputs). live_masks: optional [B, topk*F/64 + FS/64] int64 tensor
    that receives the canonical live mask of every 64-group. status: optional int32 [1]
    tensor ORed with 1 when an expert id is out of range (that slot then contributes 0).
    """
    del sl, unr, nds
    if not loadsc:
        raise ValueError("loadsc=0 (skip scales/biases) is a benchmark-only mode of the reference "
                         "(decode.py:25-27) and gives wrong results; it is not provided")
    h = N.contig(h)
    B = h.shape[0]
    if h.shape[1] != topk * F + FS:
        raise N.HSDError(f"h has {h.shape[1]} columns, expected topk*F + FS = {topk * F + FS}")
    sel = N.contig(sel.to(torch.int32))
    gains = N.contig(gains.to(torch.float32))
    E = pw.shape[0]
    od = out_dtype or h.dtype
    y = torch.empty((B, D), dtype=od, device=h.device)
    nbytes = N.lib().hsd_sparse_down_workspace_bytes(B, D, F, FS, topk)
    ws = _workspace(nbytes, h.device, workspace)
    if live_masks is not None and (live_masks.dtype != torch.int64 or not live_masks.is_contiguous()
                                   or live_masks.numel() < B * (topk * F // 64 + FS // 64)):
        raise N.HSDError("live_masks must be a contiguous int64 tensor of B*(topk*F/64 + FS/64) entries")
    N.call("hsd_sparse_down_decode", N.ptr(h), N.dtype_tag(h.dtype), N.ptr(sel), N.ptr(gains),
           N.ptr(N.as_words(N.contig(pw))), N.ptr(N.contig(ps)), N.ptr(N.contig(pb)),
           N.ptr(N.as_words(N.contig(spw))), N.ptr(N.contig(sps)), N.ptr(N.contig(spb)),
           N.ptr(y), N.dtype_tag(od), B, D, F, FS, topk, E, 1 if dense else 0,
           N.ptr(live_masks), N.ptr(status), N.ptr(ws), ws.numel(), N.stream(h.device))
    return y


def dense_down(h, sel, gains, w, s, b, sw, ss, sb, *, F, FS, D, topk, out_dtype=None, status=None):
    """The dense 4-bit down projection on the checkpoint's STOCK layout (w [E, D, F/8],
    s/b [E, D, F/64]; shared [D, FS/8], [D, FS/64]) -- what dense mode computes with
    mlx-lm's quantised matmuls (model.py:132-133). Reads every byte of the 7 selected
    matrices; the comparator of the sparse kernel."""
    h = N.contig(h)
    B = h.shape[0]
    sel = N.contig(sel.to(torch.int32))
    gains = N.contig(gains.to(torch.float32))
    od = out_dtype or h.dtype
    y = torch.empty((B, D), dtype=od, device=h.device)
    N.call("hsd_dense_down_decode", N.ptr(h), N.dtype_tag(h.dtype), N.ptr(sel), N.ptr(gains),
           N.ptr(N.as_words(N.contig(w))), N.ptr(N.contig(s)), N.ptr(N.contig(b)),
           N.ptr(N.as_words(N.contig(sw))), N.ptr(N.contig(ss)), N.ptr(N.contig(sb)),
           N.ptr(y), N.dtype_tag(od), B, D, F, FS, topk, w.shape[0], N.ptr(status), N.stream(h.device))
    return y
