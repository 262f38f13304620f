"""The dense pieces of a Nemotron-H decode step around the hot path, over libhsd: the
quantised (and bf16) projections with their fused norms and residual adds, the greedy
argmax of lm_head, the quantised embedding, the MTP head's input norm and GQA attention
over a KV cache (hsd/model.py:223-230, 281-288, 333-346; hsd/mtp.py:81-88).

Every function takes device tensors, allocates its outputs with torch on the current
stream (or writes into `out=`), and raises hsd._native.HSDError when libhsd refuses the
call. A token row is computed the same way whatever the number of rows, so verify rows
equal decode rows bit for bit.
"""
from __future__ import annotations

import math

import torch

from . import _native as N

MAX_ROWS = 4


class QWeight:
    """A projection's weight: affine 4-bit group-64 (w [O, I/8] int32 words, scales/biases
    [O, I/64] bf16 -- mlx's QuantizedLinear) or bf16 (w [O, I], scales None)."""

    def __init__(self, w, scales=None, biases=None):
        self.w, self.scales, self.biases = w, scales, biases
        self.q4 = scales is not None
        if self.q4:
            self.O, self.I = w.shape[0], w.shape[1] * 8
        else:
            if w.dtype != torch.bfloat16:
                raise N.HSDError("an unquantised weight must be bf16")
            self.O, self.I = w.shape

    @property
    def kind(self):
        return N.W_Q4 if self.q4 else N.W_BF16

    def nbytes(self):
        n = self.w.numel() * self.w.element_size()
        if self.q4:
            n += 2 * self.scales.numel() * 2
        return n


def argmax_slots(O, q4=True):
    return int(N.lib().hsd_linear_argmax_slots(O, N.W_Q4 if q4 else N.W_BF16))


def linear(x, W: QWeight, *, norm=None, eps=1e-5, gate=None, gated_z=False, residual=None, out=None,
           out_dtype=torch.bfloat16, xn_out=None, argmax_keys=None):
    """y = xn W^T for x [B, I] (B <= 4; longer inputs go 4 rows at a time).
    norm (bf16 [I]): xn = rms_norm(x, norm, eps) (mx.fast.rms_norm); with `gate` as well,
    x is the f32 SSM output and xn the Mamba-2 gated RMSNorm of x * silu(gate) per group of
    512; gated_z=True: x is mamba.ssm_rows(..., gated=True)'s z (its rows carry the
    16-channel sums of z^2 past column I) and xn the same gated norm.
    residual: y = bf16(residual + bf16(xn W^T)) (out may be residual). argmax_keys
    ([B, slots] int64): the greedy argmax's per-workgroup keys instead of y (y still
    written when out is given). xn_out: receives xn (bf16 [B, I])."""
    B = x.shape[0]
    if B > MAX_ROWS and gated_z:
        raise N.HSDError(f"the gated_z prologue takes at most {MAX_ROWS} rows")
    if B > MAX_ROWS:
        if argmax_keys is not None:
            raise N.HSDError(f"argmax takes at most {MAX_ROWS} rows")
        y = out if out is not None else torch.empty((B, W.O), dtype=out_dtype, device=x.device)
        for r in range(0, B, MAX_ROWS):
            sl = slice(r, r + MAX_ROWS)
            linear(x[sl], W, norm=norm, eps=eps, gate=None if gate is None else gate[sl],
                   residual=None if residual is None else residual[sl], out=y[sl], out_dtype=out_dtype,
                   xn_out=None if xn_out is None else xn_out[sl])
        return y
    if x.shape[1] != W.I:
        raise N.HSDError(f"linear: x has {x.shape[1]} columns, the weight {W.I} inputs")
    if gated_z:
        xk = N.X_GATED_Z
        if x.dtype != torch.float32 or norm is None or gate is not None or x.stride(0) < W.I + W.I // 16:
            raise N.HSDError("gated_z takes ssm_rows(gated=True)'s z (rows of I + I/16 values) and a norm weight")
    elif gate is not None:
        xk = N.X_GATED
        if x.dtype != torch.float32 or norm is None:
            raise N.HSDError("the gated norm takes the f32 SSM output and a norm weight")
    else:
        xk = N.X_RMS if norm is not None else N.X_BF16
        if x.dtype != torch.bfloat16:
            raise N.HSDError("linear takes bf16 activations")
    if argmax_keys is not None:
        yk = N.Y_ARGMAX
        y = out
    elif residual is not None:
        yk = N.Y_RESID
        y = out if out is not None else torch.empty((B, W.O), dtype=torch.bfloat16, device=x.device)
    else:
        yk = N.Y_F32 if out_dtype == torch.float32 else N.Y_BF16
        y = out if out is not None else torch.empty((B, W.O), dtype=out_dtype, device=x.device)
    if y is not None and (y.stride(1) != 1 or (y.dtype == torch.float32) != (yk == N.Y_F32)):
        raise N.HSDError("linear: out must have unit column stride and the requested dtype")
    N.call("hsd_linear", N.ptr(x), x.stride(0), xk, N.ptr(gate), 0 if gate is None else gate.stride(0), N.ptr(norm),
           float(eps), N.ptr(W.w), N.ptr(W.scales), N.ptr(W.biases), W.kind, N.ptr(y),
           0 if y is None else y.stride(0), yk, N.ptr(residual), 0 if residual is None else residual.stride(0),
           N.ptr(xn_out), 0 if xn_out is None else xn_out.stride(0), N.ptr(argmax_keys),
           0 if argmax_keys is None else argmax_keys.stride(0), B, W.O, W.I, N.stream(x.device))
    return y


def argmax(keys, B=None, out=None):
    """tok [B] int32 from the per-workgroup keys of linear(..., argmax_keys=keys)."""
    B = keys.shape[0] if B is None else B
    out = out if out is not None else torch.empty(B, dtype=torch.int32, device=keys.device)
    N.call("hsd_argmax_keys", N.ptr(keys), keys.stride(0), keys.shape[1], B, N.ptr(out), N.stream(keys.device))
    return out


def embed(tok, W: QWeight, out=None, status=None):
    """The quantised embedding rows of tok [B] int32 (model.py:223-224) -> [B, D] bf16."""
    B = tok.shape[0]
    D = W.I
    out = out if out is not None else torch.empty((B, D), dtype=torch.bfloat16, device=tok.device)
    N.call("hsd_embed_q4", N.ptr(tok), B, N.ptr(W.w), N.ptr(W.scales), N.ptr(W.biases), W.O, D, N.ptr(out),
           out.stride(0), N.ptr(status), N.stream(tok.device))
    return out


def pair_norm(e, h, we, wh, eps=1e-5, out=None):
    """concat(rms_norm(e, we), rms_norm(h, wh)) -> [B, 2D] bf16 (the MTP head's input,
    mtp.py:81-83)."""
    B, D = e.shape
    out = out if out is not None else torch.empty((B, 2 * D), dtype=torch.bfloat16, device=e.device)
    N.call("hsd_pair_norm", N.ptr(e), e.stride(0), N.ptr(h), h.stride(0), N.ptr(we), N.ptr(wh), float(eps), B, D,
           N.ptr(out), out.stride(0), N.stream(e.device))
    return out


def head_input(tok, h, W: QWeight, we, wh, eps=1e-5, out=None, status=None, chain=None):
    """concat(rms_norm(embed(tok), we), rms_norm(h, wh)) -> [B, 2D] bf16 in one launch
    (embed then pair_norm, the same bits; mtp.py:81-83 on the head's token rows). chain =
    (keys [1, slots] int64, seq, d1 [>= 1] int32): the chained call (model.py:408-414), tok
    unused: the token is the argmax of keys, written to d1[0], and seq's HEAD_POS2 advances as
    hsd_mtp_chain does; h is then the selected row's normed hidden row [1, D]."""
    B, D = h.shape
    out = out if out is not None else torch.empty((B, 2 * D), dtype=torch.bfloat16, device=h.device)
    keys, seq, d1 = chain if chain is not None else (None, None, None)
    N.call("hsd_head_input", None if chain is not None else N.ptr(tok), N.ptr(keys),
           0 if keys is None else keys.shape[-1], N.ptr(W.w), N.ptr(W.scales), N.ptr(W.biases), W.O, N.ptr(h),
           h.stride(0), N.ptr(we), N.ptr(wh), float(eps), B, D, N.ptr(seq), N.ptr(d1), N.ptr(out), out.stride(0),
           N.ptr(status), N.stream(h.device))
    return out


class KVCache:
    """One attention layer's cache: K and V [HKV, smax, HD] bf16. The length lives on the
    device (an int32 the step kernels advance), so trimming after a rejected draft
    (KVCache.trim, model.py:355) is a smaller length and nothing is copied."""

    def __init__(self, hkv, smax, device, head_dim=128):
        self.smax = smax
        self.k = torch.zeros((hkv, smax, head_dim), dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)


def attention(qkv, cache: KVCache, pos, *, n_heads, n_kv_heads, head_dim=128, scale=None, out=None, workspace=None,
              status=None):
    """GQA attention of B <= 4 rows at positions pos .. pos+B-1 (pos: device int32 [1], the
    cache length before the call) over keys 0 .. pos+r; the rows' keys and values (in qkv
    [B, (HQ + 2 HKV) * HD]: q | k | v) are appended to the cache. -> [B, HQ * HD] bf16."""
    B = qkv.shape[0]
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    out = out if out is not None else torch.empty((B, n_heads * head_dim), dtype=torch.bfloat16, device=qkv.device)
    nbytes = N.lib().hsd_attn_workspace_bytes(B, n_heads, cache.smax)
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=qkv.device)
    N.call("hsd_attn_decode", N.ptr(qkv), qkv.stride(0), B, N.ptr(cache.k), N.ptr(cache.v), cache.smax, N.ptr(pos),
           N.ptr(out), out.stride(0), n_heads, n_kv_heads, head_dim, float(scale), N.ptr(status), N.ptr(workspace),
           workspace.numel() * workspace.element_size(), N.stream(qkv.device))
    return out
