"""Sparse MoE down projection for prefill on the neuron-major layout (hsd/prefill.py).

The (token, expert-slot) pairs of a chunk are sorted by expert into tiles of tt slots
(`build_tiles`), the union of the neurons live in any slot of a tile is compacted
(`build_union`), and a bf16 MFMA grouped GEMM over each tile's union rows, with the B
tiles dequantised from the 4-bit layout in LDS, forms the partials that are summed per
token (`sparse_down_prefill`). All on the device, no host readback.
"""
from __future__ import annotations

import torch

from . import _native as N
from .decode import _workspace


def num_tiles(T, topk, E, tt):
    """The fixed tile count NT = T*topk//tt + E + ceil(T/tt) (prefill.py:266, 275)."""
    return T * topk // tt + E + (T + tt - 1) // tt


def build_tiles(sel, E, tt, status=None):
    """hsd/prefill.py:247-278. sel [T, topk] int32 -> (tile_e [NT] int32, tile_slot [NT*tt]
    int32): slots t*topk+k stably sorted by expert (ties by slot id) in tiles of tt, then
    the shared expert's ceil(T/tt) tiles (expert id E) over the tokens; -1 padding."""
    sel = N.contig(sel.to(torch.int32))
    T, K = sel.shape
    NT = num_tiles(T, K, E, tt)
    tile_e = torch.empty(NT, dtype=torch.int32, device=sel.device)
    tile_slot = torch.empty(NT * tt, dtype=torch.int32, device=sel.device)
    ws = _workspace(N.lib().hsd_prefill_tiles_workspace_bytes(T, K, E), sel.device, None)
    N.call("hsd_prefill_tiles", N.ptr(sel), T, K, E, tt, N.ptr(tile_e), N.ptr(tile_slot),
           N.ptr(status), N.ptr(ws), ws.numel(), N.stream(sel.device))
    return tile_e, tile_slot


def build_union(h, tile_e, tile_slot, *, F, FS, topk, E, tt, kc=32, nth=256):
    """hsd/prefill.py:281-291. The ascending union of live neurons per tile, -1 padded to
    UMAX = ceil(FS/kc)*kc -> (ulist [NT, UMAX] int32, ucount [NT] int32). nth is the
    reference's threadgroup size and is ignored."""
    del nth
    h = N.contig(h)
    T = h.shape[0]
    NT = tile_e.shape[0]
    umax = (FS + kc - 1) // kc * kc
    ulist = torch.empty((NT, umax), dtype=torch.int32, device=h.device)
    ucount = torch.empty(NT, dtype=torch.int32, device=h.device)
    N.call("hsd_prefill_union", N.ptr(h), N.dtype_tag(h.dtype), N.ptr(N.contig(tile_e)),
           N.ptr(N.contig(tile_slot)), N.ptr(ulist), N.ptr(ucount), T, F, FS, topk, E, tt, NT,
           umax, N.stream(h.device))
    return ulist, ucount


def sparse_down_prefill(h, sel, gains, pw, ps, pb, spw, sps, spb, *, F, FS, D, topk, E,
                        tt=32, nb=64, kc=32, nsg=4, tiles=None, union=None, out_dtype=None,
                        workspace=None):
    """hsd/prefill.py:294-321. h [T, topk*F + FS] bf16, sel [T, topk] int32,
    gains [T, topk+1] f32 -> y [T, D] (out_dtype, default h.dtype). tt in {32, 64}:
    slots per tile. nb / kc / nsg are Metal tile knobs, accepted and ignored (the HIP
    GEMM uses one wavefront per 128-column block (64 for tt=64) and 16-row k-blocks).
    The GEMM's A operand is bf16: an f16 or f32 h is rounded to bf16 first (the reference
    rounds its A tile to half, prefill.py:113), so such inputs agree to bf16 precision;
    the live rows (exact zeros) are the same either way."""
    del nb, nsg
    od = out_dtype or h.dtype
    if h.dtype in (torch.float16, torch.float32):
        h = h.to(torch.bfloat16)
    elif h.dtype != torch.bfloat16:
        raise N.HSDError("sparse_down_prefill takes bf16, f16 or f32 activations")
    h = N.contig(h)
    T = h.shape[0]
    tile_e, tile_slot = tiles if tiles is not None else build_tiles(sel, E, tt)
    ulist, ucount = union if union is not None else build_union(h, tile_e, tile_slot, F=F, FS=FS,
                                                                topk=topk, E=E, tt=tt, kc=kc)
    NT = tile_e.shape[0]
    gains = N.contig(gains.to(torch.float32))
    y = torch.empty((T, D), dtype=od, device=h.device)
    ws = _workspace(N.lib().hsd_prefill_gemm_workspace_bytes(T, D, F, FS, topk, E, tt), h.device,
                    workspace)
    sel = N.contig(sel.to(torch.int32))
    N.call("hsd_prefill_gemm", N.ptr(h), N.ptr(sel), N.ptr(gains), N.ptr(N.contig(tile_e)), N.ptr(N.contig(tile_slot)),
           N.ptr(N.contig(ulist)), N.ptr(N.contig(ucount)), N.ptr(N.as_words(N.contig(pw))),
           N.ptr(N.contig(ps)), N.ptr(N.contig(pb)), N.ptr(N.as_words(N.contig(spw))),
           N.ptr(N.contig(sps)), N.ptr(N.contig(spb)), N.ptr(y), N.dtype_tag(od), T, D, F, FS, topk,
           E, tt, NT, ulist.shape[1], N.ptr(ws), ws.numel(), N.stream(h.device))
    return y
