"""Multi-row Mamba-2 steps with rollback, for speculative decoding (hsd/mamba.py).

A Mamba-2 layer's recurrent state is a (conv state, ssm state) pair. Here it lives in a
ring of `nslab` slabs per layer (ssm [nslab, H, P, N] fp32, conv [nslab, K-1, CD] bf16)
and a device int32 `cur` names the current slab. A verify of L rows writes the state
after every row into its own slab (per-row checkpoints in HBM), so the rollback to the
first n_keep rows is `cur += n_keep` on the device -- no recompute (the reference
recomputes the SSM over the kept prefix, mamba.py:47-56) and no host round trip. One
`cur` can be shared by every Mamba layer of a model, so one rollback (or the greedy
acceptance kernel) moves all of them.

A row is computed by the same instruction sequence whatever L is: a verify of L rows is
bit-identical to L single-row steps.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as N
from .decode import _workspace

CONV_K = 4


@dataclass
class Mamba2Mixer:
    """The parameters of one Mamba-2 mixer (the attributes mamba.py:24-43 reads from
    mlx-lm's mixer): conv_w [CD, K] bf16, conv_b [CD] bf16, A_log / dt_bias / D [H] f32,
    norm_w [H*P] bf16 (the gated RMSNorm's weight). The block around it (pre-norm,
    in_proj, out_proj) is hsd.model.MambaBlock."""
    conv_w: torch.Tensor
    conv_b: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    D: torch.Tensor
    norm_w: torch.Tensor
    num_heads: int = 64
    head_dim: int = 64
    ssm_state_size: int = 128
    n_groups: int = 8
    norm_group: int = 512
    eps: float = 1e-5
    time_step_limit: tuple = (0.0, float("inf"))

    @property
    def intermediate_size(self):
        return self.num_heads * self.head_dim

    @property
    def conv_dim(self):
        return self.intermediate_size + 2 * self.n_groups * self.ssm_state_size


class MambaCache:
    """The state ring of one Mamba-2 layer. `cur` is a device int32 [1] tensor; pass the
    same tensor to every layer of a model to move them together."""

    def __init__(self, mixer: Mamba2Mixer, device, nslab=4, cur=None, conv_state=None, ssm_state=None):
        H, P, Nst, CD = mixer.num_heads, mixer.head_dim, mixer.ssm_state_size, mixer.conv_dim
        self.nslab = nslab
        self.ssm = torch.zeros((nslab, H, P, Nst), dtype=torch.float32, device=device)
        self.conv = torch.zeros((nslab, CONV_K - 1, CD), dtype=torch.bfloat16, device=device)
        self.cur = cur if cur is not None else torch.zeros(1, dtype=torch.int32, device=device)
        if conv_state is not None or ssm_state is not None:
            c = int(self.cur.item())
            if conv_state is not None:
                self.conv[c].copy_(conv_state)
            if ssm_state is not None:
                self.ssm[c].copy_(ssm_state)

    def state(self):
        """(conv_state [K-1, CD] bf16, ssm_state [H, P, N] f32) at the current slab (reads
        cur on the host: a synchronising debug/test accessor, not for the hot loop)."""
        c = int(self.cur.item())
        return self.conv[c], self.ssm[c]


def verify_rows(mixer: Mamba2Mixer, proj, cache: MambaCache, out_dtype=torch.bfloat16, workspace=None,
                status=None):
    """The fused conv + SSM + gated-norm update of L rows from the in_proj output
    proj [L, 2*H*P + 2*G*N + H] (gate | conv input | dt, mamba.py:27), writing the per-row
    checkpoints. -> y [L, H*P] (the gated RMSNorm output that out_proj consumes).
    status: optional int32 [1], ORed with 2 when the ring index is corrupt (y is then NaN)."""
    if proj.dtype != torch.bfloat16:
        raise N.HSDError("the Mamba-2 verify takes the bf16 in_proj output")
    proj = N.contig(proj)
    L = proj.shape[0]
    H, P, Nst, G = mixer.num_heads, mixer.head_dim, mixer.ssm_state_size, mixer.n_groups
    DI, CD = mixer.intermediate_size, mixer.conv_dim
    ld = proj.shape[1]
    if ld != DI + CD + H:
        raise N.HSDError(f"proj has {ld} columns, expected {DI + CD + H}")
    y = torch.empty((L, DI), dtype=out_dtype, device=proj.device)
    ws = _workspace(N.lib().hsd_mamba_workspace_bytes(L, H, P), proj.device, workspace)
    base = proj.data_ptr()
    es = proj.element_size()
    import ctypes
    gate_p = ctypes.c_void_p(base)
    conv_p = ctypes.c_void_p(base + DI * es)
    dt_p = ctypes.c_void_p(base + (DI + CD) * es)
    lo, hi = mixer.time_step_limit
    N.call("hsd_mamba_verify", conv_p, ld, dt_p, ld, gate_p, ld,
           N.ptr(N.contig(mixer.conv_w)), N.ptr(N.contig(mixer.conv_b)), N.ptr(N.contig(mixer.A_log)),
           N.ptr(N.contig(mixer.dt_bias)), N.ptr(N.contig(mixer.D)), N.ptr(N.contig(mixer.norm_w)),
           N.ptr(cache.ssm), N.ptr(cache.conv), N.ptr(cache.cur), cache.nslab, N.ptr(y),
           N.dtype_tag(out_dtype), L, H, P, Nst, G, mixer.norm_group, float(mixer.eps), float(lo),
           float(hi), N.ptr(status), N.ptr(ws), ws.numel(), N.stream(proj.device))
    return y


def ssm_rows(mixer: Mamba2Mixer, proj, cache: MambaCache, out=None, status=None, gated=False):
    """The conv + SSM update of L rows from the in_proj output proj [L, 2*H*P + 2*G*N + H]
    (gate | conv input | dt) with the per-row checkpoints written, without the gated norm:
    -> y [L, H*P] f32 (sum_n S C + D x), which out_proj consumes through nn.linear's gated
    norm prologue (with the gate columns of proj).
    gated=True: the gate applied here (hsd_mamba_ssm_gated) -> z [L, H*P] f32 = y silu(gate),
    a view of rows of H*P + H*P/16 values whose tail holds each 16 channels' sum of z^2;
    out_proj then takes it with nn.linear(..., gated_z=True)."""
    if proj.dtype != torch.bfloat16:
        raise N.HSDError("the Mamba-2 update takes the bf16 in_proj output")
    L = proj.shape[0]
    H, P, Nst, G = mixer.num_heads, mixer.head_dim, mixer.ssm_state_size, mixer.n_groups
    DI, CD = mixer.intermediate_size, mixer.conv_dim
    if proj.shape[1] < DI + CD + H or proj.stride(1) != 1:
        raise N.HSDError(f"proj needs {DI + CD + H} unit-stride columns")
    es = proj.element_size()
    import ctypes
    conv_p = ctypes.c_void_p(proj.data_ptr() + DI * es)
    dt_p = ctypes.c_void_p(proj.data_ptr() + (DI + CD) * es)
    lo, hi = mixer.time_step_limit
    if gated:
        zw = DI + DI // 16
        if out is None:
            out = torch.empty((L, zw), dtype=torch.float32, device=proj.device)
        if out.dtype != torch.float32 or out.shape[0] < L or out.stride(1) != 1 or out.stride(0) < zw:
            raise N.HSDError(f"ssm_rows(gated=True) needs f32 rows of at least {zw} values")
        N.call("hsd_mamba_ssm_gated", conv_p, proj.stride(0), dt_p, proj.stride(0), N.ptr(proj), proj.stride(0),
               N.ptr(N.contig(mixer.conv_w)), N.ptr(N.contig(mixer.conv_b)), N.ptr(N.contig(mixer.A_log)),
               N.ptr(N.contig(mixer.dt_bias)), N.ptr(N.contig(mixer.D)), N.ptr(cache.ssm), N.ptr(cache.conv),
               N.ptr(cache.cur), cache.nslab, N.ptr(out), out.stride(0), L, H, P, Nst, G, float(lo), float(hi),
               N.ptr(status), N.stream(proj.device))
        return out[:L, :DI]
    y = out if out is not None else torch.empty((L, DI), dtype=torch.float32, device=proj.device)
    N.call("hsd_mamba_ssm", conv_p, proj.stride(0), dt_p, proj.stride(0), N.ptr(N.contig(mixer.conv_w)),
           N.ptr(N.contig(mixer.conv_b)), N.ptr(N.contig(mixer.A_log)), N.ptr(N.contig(mixer.dt_bias)),
           N.ptr(N.contig(mixer.D)), N.ptr(cache.ssm), N.ptr(cache.conv), N.ptr(cache.cur), cache.nslab, N.ptr(y), L,
           H, P, Nst, G, float(lo), float(hi), N.ptr(status), N.stream(proj.device))
    return y


def mamba_verify(block, x3, cache, records):
    """hsd/mamba.py:19-44. One Mamba-2 block on x3 [1, L, *] with the cache advanced by L
    rows (the per-row checkpoints written), remembering in `records` what mamba_rollback
    needs.

    `block` with the reference's structure -- `.norm_w` (the block pre-norm, mamba.py:25),
    `.in_proj` / `.out_proj` (4-bit nn.QWeight) and `.mixer` (a Mamba2Mixer), such as
    hsd.model.MambaBlock: x3 is the block input [1, L, D] and the result is
    x3 + out_proj(gated_norm(ssm(conv(in_proj(norm(x3)))))) (mamba.py:25-44), in bf16.
    A bare Mamba2Mixer (the kernel-level form): x3 is the in_proj output
    [1, L, 2*H*P + 2*G*N + H] and the result the gated-norm output y [1, L, H*P]."""
    x = N.contig(x3[0])
    L = x.shape[0]
    if hasattr(block, "in_proj") and hasattr(block, "norm_w") and hasattr(block, "rows"):
        m = block.mixer
        buf = dict(proj=torch.empty((L, block.in_proj.O), dtype=torch.bfloat16, device=x.device),
                   y_pre=torch.empty((L, m.intermediate_size + m.intermediate_size // 16), dtype=torch.float32,
                                     device=x.device))
        out = x.clone()
        block.rows(out, buf, cache)
        records.append((cache, L))
        return out[None]
    m = getattr(block, "mixer", block)
    y = verify_rows(m, x, cache)
    records.append((cache, L))
    return y[None]


def mamba_rollback(records, n_keep, n_keep_dev=None, status=None):
    """hsd/mamba.py:47-56. After mamba_verify on L rows, put every cache in `records` at
    the state after its first n_keep rows: cur += n_keep on the device. A `cur` shared by
    several caches is moved once. n_keep_dev (a device int32 [1], e.g. from
    hsd.mtp.greedy_accept) overrides the host n_keep; a device value outside [0, L] leaves
    the caches where they are and ORs 2 into `status` (optional int32 [1])."""
    seen = set()
    for cache, L in records:
        if id(cache.cur) in seen:
            continue
        seen.add(id(cache.cur))
        if n_keep_dev is None and not 0 <= n_keep <= L:
            raise N.HSDError(f"n_keep {n_keep} outside [0, {L}]")
        N.call("hsd_mamba_select_row", N.ptr(cache.cur), N.ptr(n_keep_dev),
               0 if n_keep_dev is not None else int(n_keep), L, cache.nslab, N.ptr(status),
               N.stream(cache.cur.device))
