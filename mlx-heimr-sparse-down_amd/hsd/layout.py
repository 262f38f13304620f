"""The neuron-major permutation of the quantised down projections (hsd/layout.py).

mlx-lm's affine 4-bit layout of a down projection W[out=D, in=F] is

    w  [.., D, F/8]  uint32   8 nibbles of one output row per word, low nibble first
    s  [.., D, F/64] bf16     scales per 64-neuron group
    b  [.., D, F/64] bf16     biases

and the neuron-major layout that the decode and prefill kernels read is

    pw [.., F, D/8]  uint32   row i = neuron i, word w packs W[8w .. 8w+7, i]
    ps [.., F/64, D] bf16
    pb [.., F/64, D] bf16

The nibble part is an exact, self-inverse 8x8 nibble-block transpose done by one HIP
kernel (libhsd `hsd_permute_nibbles`); the scales and biases are moved bit for bit by
`hsd_transpose_u16`. No value is re-quantised and no transient buffer is needed.
"""
from __future__ import annotations

import torch

from . import _native as N


def nibble_transpose(w: torch.Tensor) -> torch.Tensor:
    """hsd/layout.py:34-50. [.., R, C/8] uint32/int32 -> [.., C, R/8] (same dtype) with
    out[.., c, wo] packing W[8*wo + n, c] at nibble n. Exact and self-inverse."""
    w = N.contig(w)
    words = N.as_words(w)
    *lead, R, CW = w.shape
    if R % 8:
        raise N.HSDError(f"nibble_transpose: rows ({R}) must be a multiple of 8")
    out = torch.empty((*lead, CW * 8, R // 8), dtype=torch.int32, device=w.device)
    batch = 1
    for d in lead:
        batch *= d
    N.call("hsd_permute_nibbles", N.ptr(words), N.ptr(out), batch, R, CW, N.stream(w.device))
    return out.view(w.dtype) if w.dtype != torch.int32 else out


def transpose_last2(x: torch.Tensor) -> torch.Tensor:
    """Bit-exact swap of the last two axes of a 16-bit tensor, into a contiguous tensor
    (the scale/bias half of hsd/layout.py:72-73)."""
    x = N.contig(N.as_u16(x))
    *lead, R, C = x.shape
    out = torch.empty((*lead, C, R), dtype=x.dtype, device=x.device)
    batch = 1
    for d in lead:
        batch *= d
    N.call("hsd_transpose_u16", N.ptr(x), N.ptr(out), batch, R, C, N.stream(x.device))
    return out


def to_neuron_major(w: torch.Tensor, s: torch.Tensor, b: torch.Tensor, chunk: int = 16):
    """hsd/layout.py:53-74: the checkpoint layout (w [.., D, F/8], s/b [.., D, F/64]) ->
    (pw [.., F, D/8], ps [.., F/64, D], pb [.., F/64, D]). `chunk` is accepted for API
    compatibility: the device permutation needs no transient, so it is not chunked."""
    del chunk
    return nibble_transpose(w), transpose_last2(s), transpose_last2(b)
