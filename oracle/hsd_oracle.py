"""CPU oracle for the hsd hot path -- TEST INFRASTRUCTURE ONLY.

This module is a NumPy restatement of the reference's arithmetic for the four
hot-path parts (layout permutation, sparse decode down projection, prefill tile
order / union / grouped down projection, Mamba-2 multi-row verify + rollback,
greedy acceptance). It exists to CHECK the HIP library: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it. The product path (the `hsd` package and `libhsd.so`) never calls it.

Every function cites the reference file:line it restates (paths relative to the
reference repository root). Conventions:

* bf16 tensors are carried as raw uint16 bit patterns; `bf16_to_f32` /
  `f32_to_bf16` convert (round-to-nearest-even, NaN -> 0x7FC0).
* Float results are accumulated in float64 and returned as float32, so the
  oracle is a tighter yardstick than the fp32 kernels it checks.

Pinning status (what checks each function beyond its own formula) is listed in
`PINNING` at the bottom; the tests in tests/test_oracle_*.py implement those
checks.
"""
from __future__ import annotations

import numpy as np

GS = 64  # quantisation group along the neuron (reduction) axis, layout.py:3-7


# --------------------------------------------------------------------------- bf16
def bf16_to_f32(bits):
    """uint16 bf16 bit patterns -> float32 (exact)."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x):
    """float -> uint16 bf16 bits, round to nearest even; every NaN -> 0x7FC0."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), rounded).astype(np.uint16)


def round_bf16(x):
    """float -> float32 holding the nearest bf16 value."""
    return bf16_to_f32(f32_to_bf16(x))


# ------------------------------------------------------------------ a1/a2 layout
def unpack_nibbles(w):
    """[.., R, C/8] uint32 -> [.., R, C] uint8, nibble i%8 of word i//8 at bits 4*(i%8)
    (the MLX affine 4-bit packing, layout.py:3-7). Little-endian bytes: byte j of a word
    holds nibbles 2j (low half) and 2j+1 (high half)."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.uint32))
    by = w.view(np.uint8).reshape(*w.shape, 4)
    nib = np.stack([by & np.uint8(0xF), by >> np.uint8(4)], axis=-1)   # [.., R, CW, 4, 2]
    return nib.reshape(*w.shape[:-1], w.shape[-1] * 8)


def pack_nibbles(q):
    """Inverse of unpack_nibbles: [.., R, C] values 0..15 -> [.., R, C/8] uint32."""
    q = np.ascontiguousarray(np.asarray(q, dtype=np.uint8))
    *lead, R, C = q.shape
    pairs = q.reshape(*lead, R, C // 8, 4, 2)
    by = (pairs[..., 0] | (pairs[..., 1] << np.uint8(4))).astype(np.uint8)
    return np.ascontiguousarray(by).view(np.uint32).reshape(*lead, R, C // 8)


def nibble_transpose(w):
    """hsd/layout.py:34-50. [.., R, C/8] u32 -> [.., C, R/8] u32 with
    out[.., c, wo] packing W[8*wo + n, c] at nibble n (low nibble first). Exact and
    self-inverse. Restated through a byte-level unpack / pack rather than the
    reference's shift-and-sum."""
    q = unpack_nibbles(w)                           # [.., R, C]  W[r, c]
    qt = np.swapaxes(q, -1, -2)                     # [.., C, R]
    return pack_nibbles(qt)


def to_neuron_major(w, s, b):
    """hsd/layout.py:53-74: (w [.., D, F/8], s/b [.., D, F/64]) ->
    (pw [.., F, D/8], ps/pb [.., F/64, D]); scales/biases are moved bit for bit."""
    pw = nibble_transpose(w)
    ps = np.ascontiguousarray(np.swapaxes(np.asarray(s), -1, -2))
    pb = np.ascontiguousarray(np.swapaxes(np.asarray(b), -1, -2))
    return pw, ps, pb


def dequantize(w, s, b, dtype=np.float64):
    """MLX affine dequantisation on the stock layout (layout.py:3-7, 26-28):
    W[.., o, i] = scale[.., o, i//64] * q + bias[.., o, i//64]; s/b are bf16 bits."""
    q = unpack_nibbles(w).astype(dtype)
    sf = np.repeat(bf16_to_f32(s).astype(dtype), GS, axis=-1)
    bf = np.repeat(bf16_to_f32(b).astype(dtype), GS, axis=-1)
    return sf * q + bf


# ------------------------------------------------ MoE front end: up projection + ReLU^2
def up_proj_f64(x, w, s, b):
    """One stock-layout 4-bit projection applied to x (the `transpose=True` product of
    mx.gather_qmm / mx.quantized_matmul, model.py:117-120): u[.., o] = sum_i W[o, i] x[i]
    with W = s * q + b (layout.py:3-7). x float [.., I]; w [O, I/8] u32, s/b [O, I/64]
    bf16 bits -> float64 [.., O]."""
    W = dequantize(w, s, b)
    return np.asarray(x, dtype=np.float64) @ W.T


def relu2_bf16(u):
    """model.py:49-50 `square(relu(x))` on a bf16 tensor: u rounded to bf16 (the product's
    output dtype), relu, the square rounded to bf16. NaN stays NaN. -> bf16 bits."""
    ub = bf16_to_f32(f32_to_bf16(np.asarray(u, dtype=np.float32))).astype(np.float64)
    r = np.where(np.isnan(ub), ub, np.maximum(ub, 0.0))
    return f32_to_bf16((r * r).astype(np.float32))


def up_relu2(x_bits, sel, w1, s1, b1, sw1, ss1, sb1, *, F, FS, topk, E=None):
    """The MoE front end after the router (model.py:110-121) followed by pack's layout
    (model.py:123-129): for token b, routed slot k uses expert sel[b, k]'s up projection
    (w1 [E, F, D/8], s1/b1 [E, F, D/64]) and the shared expert its own (sw1 [FS, D/8],
    ss1/sb1 [FS, D/64]); h = relu2(x @ W^T) in bf16 (test_layout_decode.py:111-120).
    -> hcat [B, topk*F + FS] bf16 bits. A routed id outside [0, E) gives a zero slot (hsd
    indexes the weights with it unchecked)."""
    x = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16)).astype(np.float64)
    B = x.shape[0]
    E = w1.shape[0] if E is None else E
    out = np.zeros((B, topk * F + FS), dtype=np.uint16)
    for bi in range(B):
        for k in range(topk):
            e = int(sel[bi, k])
            if 0 <= e < E:
                out[bi, k * F:(k + 1) * F] = relu2_bf16(up_proj_f64(x[bi], w1[e], s1[e], b1[e]))
        out[bi, topk * F:] = relu2_bf16(up_proj_f64(x[bi], sw1, ss1, sb1))
    return out


# -------------------------------------------------------------- a5 compaction
def live_masks(hcat, F, FS, topk):
    """Canonical compaction of hsd/decode.py:84-101 (Appendix A.3 of the hot-path
    spec): for every slot (topk routed, then the shared expert) and every 64-group, a
    uint64 mask with bit j set iff float(h[g*64 + j]) != 0 (+0 and -0 dead, NaN live).
    Returns [B, topk*F/64 + FS/64] uint64; the ascending live list of a slot is the
    set bits in group order."""
    h = np.asarray(hcat, dtype=np.float32)
    B = h.shape[0]
    live = (h != 0) | np.isnan(h)
    ng = h.shape[1] // GS
    bits = live.reshape(B, ng, GS).astype(np.uint64) << np.arange(GS, dtype=np.uint64)
    return np.bitwise_or.reduce(bits, axis=-1).astype(np.uint64)


# ------------------------------------------------------- a6/a7/a8 sparse decode
def _slot_views(hcat, sel_b, k, pw, ps, pb, spw, sps, spb, F, FS, topk):
    if k < topk:
        e = int(sel_b[k])
        return hcat[k * F:(k + 1) * F], pw[e], ps[e], pb[e]
    return hcat[topk * F: topk * F + FS], spw, sps, spb


def sparse_down(hcat, sel, gains, pw, ps, pb, spw, sps, spb, *, F, FS, D, topk, dense=False):
    """hsd/decode.py:164-186 with the arithmetic of decode.py:105-144 (Appendix A.4):
    per slot and live 64-group, acc[o] = sum over live rows of h_i * q_{i,o} and
    hsum = sum of h_i; out[o] += s_g[o]*acc[o] + b_g[o]*hsum; part = gain * out; y = the
    sum of the slot parts in slot order. Only live rows and live groups are touched.
    `dense=True` treats every row as live (the dense-h control of bench/decode_layers.py
    :163-168). hcat: [B, topk*F+FS] float32 values; sel [B, topk]; gains [B, topk+1];
    weights in the neuron-major layout (uint32 / bf16 bits). -> y [B, D] float32."""
    h = np.asarray(hcat, dtype=np.float32)
    B = h.shape[0]
    y = np.zeros((B, D), dtype=np.float64)
    for bi in range(B):
        for k in range(topk + 1):
            hk, wk, sk, bk = _slot_views(h[bi], sel[bi], k, pw, ps, pb, spw, sps, spb, F, FS, topk)
            n = hk.shape[0]
            live = np.ones(n, dtype=bool) if dense else ((hk != 0) | np.isnan(hk))
            out = np.zeros(D, dtype=np.float64)
            for g in range(n // GS):
                idx = np.flatnonzero(live[g * GS:(g + 1) * GS]) + g * GS
                if idx.size == 0:
                    continue                      # dead group: its scales/biases are not read
                q = unpack_nibbles(wk[idx]).astype(np.float64)        # [nl, D]
                hv = hk[idx].astype(np.float64)
                acc = hv @ q
                hsum = hv.sum()
                out += bf16_to_f32(sk[g]).astype(np.float64) * acc + bf16_to_f32(bk[g]).astype(np.float64) * hsum
            y[bi] += np.float64(np.float32(gains[bi, k])) * out
    return y.astype(np.float32)


def dense_reference(hcat, sel, gains, w, s, b, sw, ss, sb, *, F, FS, D, topk):
    """tests/test_layout_decode.py:128-142: dequantise the selected down projections in
    the STOCK layout (w [E, D, F/8], s/b [E, D, F/64]; shared [D, FS/8], [D, FS/64]) and
    form y = sum_k gain_k * W_k h_k + gain_s * W_s h_s, in float64."""
    h = np.asarray(hcat, dtype=np.float64)
    B = h.shape[0]
    Ws = dequantize(sw, ss, sb)
    y = np.zeros((B, D))
    for bi in range(B):
        for k in range(topk):
            W = dequantize(w[int(sel[bi, k])], s[int(sel[bi, k])], b[int(sel[bi, k])])
            y[bi] += float(np.float32(gains[bi, k])) * (W @ h[bi, k * F:(k + 1) * F])
        y[bi] += float(np.float32(gains[bi, topk])) * (Ws @ h[bi, topk * F:topk * F + FS])
    return y


def touched_bytes(hcat, F, FS, topk, D, dense=False):
    """The byte model of bench/common.py:16-19, 78-83 plus I/O: per slot, live rows x D/2
    + live 64-groups x 4D (bf16 scales + biases), plus h, sel, gains and the bf16 y."""
    m = live_masks(hcat, F, FS, topk)
    B = m.shape[0]
    if dense:
        rows = B * (topk * F + FS)
        groups = m.size
    else:
        rows = int(sum(bin(int(v)).count("1") for v in m.reshape(-1)))
        groups = int(np.count_nonzero(m))
    io = B * ((topk * F + FS) * 2 + topk * 4 + (topk + 1) * 4 + D * 2)
    return rows * (D // 2) + groups * (4 * D) + io


# ------------------------------------------------------------ a9 tiles / a10 union
def build_tiles(sel, E, tt):
    """hsd/prefill.py:247-278 (Appendix A.5). Slots t*topk+k stably sorted by expert;
    ceil(count_e/tt) tiles per expert in expert order, then ceil(T/tt) shared tiles
    (expert id E) over tokens 0..T-1; a fixed NT = T*topk//tt + E + ceil(T/tt); -1 pads.
    -> (tile_e [NT] int32, tile_slot [NT*tt] int32)."""
    sel = np.asarray(sel, dtype=np.int64)
    T, K = sel.shape
    flat = sel.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)[:E]
    ntile = (counts + tt - 1) // tt
    tile_base = np.cumsum(ntile) - ntile
    exp_start = np.cumsum(counts) - counts
    nt_routed = T * K // tt + E
    tile_e = np.full(nt_routed, -1, dtype=np.int32)
    tile_slot = np.full(nt_routed * tt, -1, dtype=np.int32)
    for e in range(E):
        tile_e[tile_base[e]:tile_base[e] + ntile[e]] = e
    for j, slot in enumerate(order):
        e = flat[slot]
        rank = j - exp_start[e]
        tile_slot[(tile_base[e] + rank // tt) * tt + rank % tt] = slot
    nt_shared = (T + tt - 1) // tt
    sh_e = np.full(nt_shared, E, dtype=np.int32)
    ar = np.arange(nt_shared * tt)
    sh_slot = np.where(ar < T, ar, -1).astype(np.int32)
    return np.concatenate([tile_e, sh_e]), np.concatenate([tile_slot, sh_slot])


def slot_h_offset(s, shared, NR, F, topk):
    """The row offset into hcat [T, NR] of slot s (prefill.py:70, 109)."""
    if s < 0:
        return -1
    return s * NR + topk * F if shared else (s // topk) * NR + (s % topk) * F


def build_union(hcat, tile_e, tile_slot, *, F, FS, topk, E, tt, kc=32):
    """hsd/prefill.py:48-93, 281-291 (Appendix A.6): per tile, the ascending columns
    c < (FS if shared else F) live in any of its valid slots, -1 padded to
    UMAX = ceil(FS/kc)*kc; empty tiles (expert -1) are all -1 with count 0.
    -> (ulist [NT, UMAX] int32, ucount [NT] int32)."""
    h = np.asarray(hcat, dtype=np.float32)
    NR = h.shape[1]
    hf = h.reshape(-1)
    NT = tile_e.shape[0]
    umax = (FS + kc - 1) // kc * kc
    ulist = np.full((NT, umax), -1, dtype=np.int32)
    ucount = np.zeros(NT, dtype=np.int32)
    for t in range(NT):
        e = int(tile_e[t])
        if e < 0:
            continue
        shared = e >= E
        FF = FS if shared else F
        live = np.zeros(FF, dtype=bool)
        for m in range(tt):
            off = slot_h_offset(int(tile_slot[t * tt + m]), shared, NR, F, topk)
            if off >= 0:
                seg = hf[off:off + FF]
                live |= (seg != 0) | np.isnan(seg)
        cols = np.flatnonzero(live).astype(np.int32)
        ulist[t, :cols.size] = cols
        ucount[t] = cols.size
    return ulist, ucount


def dequant_rows(pw_e, ps_e, pb_e, rows):
    """Neuron-major rows -> float64 [len(rows), D]: s[g(r)] * q + b[g(r)]."""
    q = unpack_nibbles(pw_e[rows]).astype(np.float64)
    g = np.asarray(rows) // GS
    return bf16_to_f32(ps_e[g]).astype(np.float64) * q + bf16_to_f32(pb_e[g]).astype(np.float64)


def sparse_down_prefill(hcat, sel, gains, pw, ps, pb, spw, sps, spb, *, F, FS, D, topk, E, tt=32,
                        kc=32, tiles=None, union=None):
    """hsd/prefill.py:294-321 (Appendix A.7): part[t*(topk+1)+k] =
    gain[t,k] * sum_{c in union(tile)} h_{t,k}[c] * W_e[c, :]; y[t] = sum_k part in slot
    order. Float64 here; -> (y [T, D] float32, part [T*(topk+1), D] float32)."""
    h = np.asarray(hcat, dtype=np.float32)
    T, NR = h.shape
    tile_e, tile_slot = tiles if tiles is not None else build_tiles(sel, E, tt)
    ulist, ucount = union if union is not None else build_union(h, tile_e, tile_slot, F=F, FS=FS,
                                                                topk=topk, E=E, tt=tt, kc=kc)
    hf = h.reshape(-1).astype(np.float64)
    part = np.zeros((T * (topk + 1), D), dtype=np.float64)
    for t in range(tile_e.shape[0]):
        e = int(tile_e[t])
        if e < 0 or ucount[t] == 0:
            continue
        shared = e >= E
        cols = ulist[t, :ucount[t]]
        W = dequant_rows(spw, sps, spb, cols) if shared else dequant_rows(pw[e], ps[e], pb[e], cols)
        for m in range(tt):
            s = int(tile_slot[t * tt + m])
            if s < 0:
                continue
            off = slot_h_offset(s, shared, NR, F, topk)
            gi = s * (topk + 1) + topk if shared else (s // topk) * (topk + 1) + s % topk
            part[gi] = float(np.float32(gains.reshape(-1)[gi])) * (hf[off + cols] @ W)
    y = part.reshape(T, topk + 1, D).sum(axis=1)
    return y.astype(np.float32), part.astype(np.float32)


# ------------------------------------------------------- a14-a16 Mamba-2 verify
def softplus(x):
    return np.logaddexp(np.asarray(x, dtype=np.float64), 0.0)


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def mamba_verify(conv_in, dt_raw, gate, conv_w, conv_b, A_log, dt_bias, Dp, norm_w,
                 conv_state, ssm_state, *, n_groups=8, eps=1e-5, dt_lo=0.0, dt_hi=np.inf,
                 norm_group=512):
    """hsd/mamba.py:19-44 with mlx-lm's ssm_update restated from the Mamba-2 recurrence
    (Appendix A.8). L rows processed sequentially from (conv_state [3, CD] bf16 values,
    ssm_state [H, P, N] fp32):
      window_r = padded[r:r+4] with padded = concat(conv_state, conv_in)   (mamba.py:29-31)
      co = silu(sum_j conv_w[:, j] * window_r[j] + conv_b)                  (mamba.py:32)
      x, B, C = split(co, [H*P, H*P + G*N])                                 (mamba.py:33-37)
      dt = clip(softplus(dt_raw + dt_bias), lo, hi); dA = exp(-exp(A_log) * dt)
      S <- dA * S + (x * dt) B^T ;  y = S C + bf16(D) x                     (mamba.py:38-41)
      out = rmsnorm_{groups of 512}(y * silu(gate)) * norm_w                (mamba.py:43)
    Inputs are float arrays (bf16 values); returns dict with y [L, H*P] (normed, f32),
    y_pre [L, H*P] (before the gate/norm), conv_states [L, 3, CD] (after each row) and
    ssm_states [L, H, P, N] float32 (after each row)."""
    conv_in = np.asarray(conv_in, dtype=np.float64)
    L, CD = conv_in.shape
    H = A_log.shape[0]
    Nst = ssm_state.shape[-1]
    P = ssm_state.shape[1]
    DI = H * P
    hpg = H // n_groups
    padded = np.concatenate([np.asarray(conv_state, dtype=np.float64), conv_in], axis=0)
    W = np.asarray(conv_w, dtype=np.float64)
    S = np.asarray(ssm_state, dtype=np.float64).copy()
    A = -np.exp(np.asarray(A_log, dtype=np.float64))
    # D enters ssm_update rounded to the activations' dtype, bf16 (m.D.astype(hs4.dtype),
    # mamba.py:38)
    Dr = round_bf16(np.asarray(Dp, dtype=np.float32)).astype(np.float64)
    out = dict(y=np.zeros((L, DI), np.float32), y_pre=np.zeros((L, DI), np.float32),
               conv_states=np.zeros((L, 3, CD), np.float32),
               ssm_states=np.zeros((L, H, P, Nst), np.float32))
    for r in range(L):
        win = padded[r:r + 4]                                         # [4, CD]
        co = silu((W.T * win).sum(axis=0) + np.asarray(conv_b, dtype=np.float64))
        x = co[:DI].reshape(H, P)
        Bm = co[DI:DI + n_groups * Nst].reshape(n_groups, Nst)
        Cm = co[DI + n_groups * Nst:DI + 2 * n_groups * Nst].reshape(n_groups, Nst)
        dt = np.clip(softplus(np.asarray(dt_raw[r], dtype=np.float64) + dt_bias), dt_lo, dt_hi)
        dA = np.exp(A * dt)
        Bh = np.repeat(Bm, hpg, axis=0)                                # [H, N]
        Ch = np.repeat(Cm, hpg, axis=0)
        S = dA[:, None, None] * S + (x * dt[:, None])[:, :, None] * Bh[:, None, :]
        y = np.einsum("hpn,hn->hp", S, Ch) + Dr[:, None] * x
        z = y.reshape(-1) * silu(np.asarray(gate[r], dtype=np.float64))
        zg = z.reshape(-1, norm_group)
        zn = zg / np.sqrt((zg * zg).mean(axis=1, keepdims=True) + eps)
        out["y"][r] = (zn.reshape(-1) * np.asarray(norm_w, dtype=np.float64)).astype(np.float32)
        out["y_pre"][r] = y.reshape(-1).astype(np.float32)
        out["conv_states"][r] = padded[r + 1:r + 4].astype(np.float32)
        out["ssm_states"][r] = S.astype(np.float32)
        S = S.astype(np.float32).astype(np.float64)    # the state is stored as fp32 between rows
    return out


def mamba_rollback(verify_out, conv_state0, ssm_state0, n_keep):
    """hsd/mamba.py:47-56: the (conv, ssm) state after the first n_keep rows of a verify;
    n_keep = 0 gives the starting state back."""
    if n_keep == 0:
        return np.asarray(conv_state0, np.float32), np.asarray(ssm_state0, np.float32)
    return verify_out["conv_states"][n_keep - 1], verify_out["ssm_states"][n_keep - 1]


# ----------------------------------------------------------- a18 acceptance
def argmax_first(logits):
    """mx.argmax over the last axis: the first index of the maximum (model.py:419)."""
    return np.argmax(np.asarray(logits, dtype=np.float32), axis=-1).astype(np.int32)


def greedy_accept(draft, tgt):
    """hsd/model.py:423-425 (Appendix A.9): a = the first i < k with draft[i] != tgt[i],
    else k; emitted tokens draft[:a] + [tgt[a]]; the caches keep a+1 rows.
    -> (a, emitted list, n_keep)."""
    k = len(draft)
    a = next((i for i in range(k) if int(draft[i]) != int(tgt[i])), k)
    return a, [int(t) for t in draft[:a]] + [int(tgt[a])], a + 1


# ------------------------------------------- the rest of a decode step (end to end)
def rms_norm_bf16(x, w, eps=1e-5):
    """mx.fast.rms_norm(x, w, eps) on bf16 (the block pre-norms, model.py:114, mamba.py:25;
    the MTP head's norms, mtp.py:81-86): t = bf16(x / sqrt(mean(x^2) + eps)), out =
    bf16(t * w). x, w bf16 values (float arrays) over the last axis -> bf16 bits."""
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    t = round_bf16((x * inv).astype(np.float32)).astype(np.float64)
    return f32_to_bf16((t * np.asarray(w, dtype=np.float64)).astype(np.float32))


def gated_rms_norm_bf16(y, gate, w, eps=1e-5, group=512):
    """The Mamba-2 gated RMSNorm in front of out_proj (mamba.py:43, mlx-lm's
    MambaRMSNormGated): z = y * silu(gate); per group of `group` elements t = bf16(z /
    sqrt(mean(z^2) + eps)); out = bf16(t * w). -> bf16 bits."""
    z = np.asarray(y, dtype=np.float64) * silu(np.asarray(gate, dtype=np.float64))
    shp = z.shape
    zg = z.reshape(*shp[:-1], shp[-1] // group, group)
    inv = 1.0 / np.sqrt((zg * zg).mean(axis=-1, keepdims=True) + eps)
    t = round_bf16((zg * inv).reshape(shp).astype(np.float32)).astype(np.float64)
    return f32_to_bf16((t * np.asarray(w, dtype=np.float64)).astype(np.float32))


def linear_q4(x, w, s, b):
    """mlx quantized_matmul(x, w, s, b, transpose=True) in float64: x [B, I] values, w
    [O, I/8] u32, s/b [O, I/64] bf16 bits -> [B, O]."""
    return up_proj_f64(x, w, s, b)


def linear_bf16(x, w_bits):
    """x @ W.T with W [O, I] bf16 bits, float64."""
    return np.asarray(x, dtype=np.float64) @ bf16_to_f32(w_bits).astype(np.float64).T


def argmax_bf16(y):
    """mx.argmax of bf16 outputs (lm_head then argmax, model.py:302, 419): the first index
    of the largest bf16-rounded value; NaN beats every number."""
    v = round_bf16(np.asarray(y, dtype=np.float32))
    v = np.atleast_2d(v)
    out = np.empty(v.shape[0], dtype=np.int32)
    for r in range(v.shape[0]):
        nan = np.flatnonzero(np.isnan(v[r]))
        out[r] = nan[0] if nan.size else int(np.argmax(v[r]))
    return out


def embed_q4(tok, w, s, b):
    """The quantised embedding (model.py:223-224): row tok of W = s q + b, the exact value
    rounded to fp32 then to bf16. -> [B, D] bf16 bits; a token outside [0, V) gives 0."""
    V = w.shape[0]
    D = w.shape[1] * 8
    out = np.zeros((len(tok), D), dtype=np.uint16)
    for i, t in enumerate(tok):
        if 0 <= int(t) < V:
            out[i] = f32_to_bf16(dequantize(w[int(t)], s[int(t)], b[int(t)]).astype(np.float32))
    return out


def attention(q, k, v, scale):
    """Scaled dot-product attention of one query row over its visible keys, per query
    head (float64): q [HQ, HD], k/v [HKV, S, HD] -> [HQ, HD]; query head h uses kv head
    h // (HQ // HKV). The reference's block calls mx.fast.scaled_dot_product_attention
    (mlx-lm NemotronH attention, model.py:287, 343)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    HQ, HKV = q.shape[0], k.shape[0]
    out = np.zeros_like(q)
    for h in range(HQ):
        g = h // (HQ // HKV)
        sc = (k[g] @ q[h]) * scale
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v[g]
    return out


def sigmoid_f32(x):
    """1 / (1 + exp(-x)) in float32 arithmetic."""
    x = np.asarray(x, dtype=np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))).astype(np.float32)


def router_topk(logits, bias, topk, scale=1.0, norm_topk=True):
    """The MoE router of the Nemotron-H family as mlx-lm runs it after `x @ gate.T`
    (model.py:115; restated from the family's published gate: sigmoid scores, a selection
    bias, top-k, normalised and scaled weights): score = sigmoid(logit) (fp32), choice =
    score + bias; sel = the topk largest choices in descending order, equal choices by
    the smaller expert id (mlx's argpartition leaves the order open: parity unpinned);
    gain = score / (sum of the selected scores + 1e-20) * scale (norm_topk) or score *
    scale. logits [B, E] float (bf16 values) -> (sel [B, topk] int32, gains [B, topk])."""
    lg = np.atleast_2d(np.asarray(logits, dtype=np.float32))
    B, E = lg.shape
    sc = sigmoid_f32(lg)
    ch = (sc + (np.zeros(E, np.float32) if bias is None else np.asarray(bias, np.float32))).astype(np.float32)
    ch = np.where(np.isnan(ch), np.float32(-np.inf), ch)          # a NaN choice ranks last
    sel = np.zeros((B, topk), dtype=np.int32)
    gains = np.zeros((B, topk), dtype=np.float64)
    for r in range(B):
        order = sorted(range(E), key=lambda e: (-float(ch[r, e]), e))[:topk]
        sel[r] = order
        sv = sc[r, order].astype(np.float64)
        gains[r] = sv / (sv.sum() + 1e-20) * scale if norm_topk else sv * scale
    return sel, gains


# ------------------------------------- one decode row through the hybrid's blocks
def _vals(bits):
    return bf16_to_f32(np.asarray(bits, dtype=np.uint16)).astype(np.float64)


def residual_add_bf16(x_bits, y):
    """x + mixer(x) in bf16 (model.py:139, mamba.py:44): bf16(x + bf16(y)) -> bits."""
    return f32_to_bf16((_vals(x_bits) + round_bf16(np.asarray(y, np.float32)).astype(np.float64)).astype(np.float32))


def mamba_block_step(x_bits, w, conv_state, ssm_state, *, n_groups=8, eps=1e-5):
    """One decode row through a Mamba-2 block (mamba.py:19-44 with L = 1): rms_norm,
    in_proj (4-bit), split gate | conv input | dt, the conv + SSM step (mamba_verify), the
    gated RMSNorm, out_proj (4-bit), the residual add. w: norm_w, in_w/in_s/in_b, out_w/
    out_s/out_b, conv_w, conv_b (bf16 values), A_log, dt_bias, D, gnorm_w. -> (x bits,
    conv_state, ssm_state)."""
    xn = rms_norm_bf16(_vals(x_bits), _vals(w["norm_w"]), eps)
    proj = round_bf16(linear_q4(_vals(xn)[None], w["in_w"], w["in_s"], w["in_b"]).astype(np.float32))[0]
    H = np.asarray(w["A_log"]).shape[0]
    DI = np.asarray(w["gnorm_w"]).shape[0]
    CD = np.asarray(w["conv_b"]).shape[0]
    gate, cin, dt = proj[:DI], proj[DI:DI + CD], proj[DI + CD:DI + CD + H]
    out = mamba_verify(cin[None], dt[None], gate[None], w["conv_w"], w["conv_b"], w["A_log"], w["dt_bias"], w["D"],
                       np.ones(DI), conv_state, ssm_state, n_groups=n_groups, eps=eps)
    g = gated_rms_norm_bf16(out["y_pre"], gate[None], _vals(w["gnorm_w"]), eps, DI // n_groups)
    y = linear_q4(_vals(g), w["out_w"], w["out_s"], w["out_b"])[0]
    return residual_add_bf16(x_bits, y), out["conv_states"][0], out["ssm_states"][0]


def attn_block_step(x_bits, w, k_cache, v_cache, *, n_heads, n_kv_heads, head_dim=128, eps=1e-5):
    """One decode row through the attention block at position P = k_cache.shape[1]
    (model.py:287): rms_norm, the q|k|v projection (4-bit), the new key/value appended,
    scaled dot-product attention over keys 0..P (bf16 output), o_proj (4-bit), residual.
    k_cache/v_cache [HKV, P, HD] values. -> (x bits, k_cache, v_cache) with P + 1 rows."""
    xn = rms_norm_bf16(_vals(x_bits), _vals(w["norm_w"]), eps)
    qkv = round_bf16(linear_q4(_vals(xn)[None], w["qkv_w"], w["qkv_s"], w["qkv_b"]).astype(np.float32))[0]
    QD, KD = n_heads * head_dim, n_kv_heads * head_dim
    q = qkv[:QD].reshape(n_heads, head_dim)
    k = np.concatenate([k_cache, qkv[QD:QD + KD].reshape(n_kv_heads, 1, head_dim)], axis=1)
    v = np.concatenate([v_cache, qkv[QD + KD:QD + 2 * KD].reshape(n_kv_heads, 1, head_dim)], axis=1)
    o = round_bf16(attention(q, k, v, 1.0 / np.sqrt(head_dim)).reshape(-1).astype(np.float32))
    y = linear_q4(o[None], w["o_w"], w["o_s"], w["o_b"])[0]
    return residual_add_bf16(x_bits, y), k, v


def moe_block_step(x_bits, w, *, topk, routed_scale, norm_topk=True, eps=1e-5):
    """One decode row through the MoE block (model.py:110-139): rms_norm, the bf16 gate
    and the router (router_topk), the selected and shared 4-bit up projections with
    ReLU^2 (up_relu2), the sparse down projection on the neuron-major layout
    (sparse_down), the residual add. -> x bits."""
    xn = rms_norm_bf16(_vals(x_bits), _vals(w["norm_w"]), eps)
    logits = round_bf16(linear_bf16(_vals(xn)[None], w["gate"]).astype(np.float32))
    sel, g = router_topk(logits, w["e_bias"], topk, routed_scale, norm_topk)
    gains = np.concatenate([g.astype(np.float32), np.ones((1, 1), np.float32)], axis=1)
    F, FS = w["w1"].shape[1], w["sw1"].shape[0]
    hcat = up_relu2(xn[None], sel, w["w1"], w["s1"], w["b1"], w["sw1"], w["ss1"], w["sb1"], F=F, FS=FS, topk=topk)
    D = w["pw"].shape[2] * 8
    y = sparse_down(bf16_to_f32(hcat), sel, gains, w["pw"], w["ps"], w["pb"], w["spw"], w["sps"], w["spb"], F=F,
                    FS=FS, D=D, topk=topk)[0]
    return residual_add_bf16(x_bits, y)


def lm_head_logits(x_bits, norm_f, w, s, b, eps=1e-5):
    """lm_head(norm_f(x)) (model.py:229-230) in float64 from the bf16 normed row."""
    xn = rms_norm_bf16(_vals(x_bits), _vals(norm_f), eps)
    return linear_q4(_vals(xn)[None], w, s, b)[0]


PINNING = {
    "up_proj_f64": "brute force on tiny shapes (scalar loops over words and nibbles); the nibble order "
                   "is unpack_nibbles', pinned with the layout",
    "relu2_bf16": "special values (negative, -0, +0, NaN) and exact squares of bf16 values",
    "up_relu2": "slot layout of pack (model.py:123-129) by construction from up_proj_f64 and relu2_bf16; "
                "a bad id gives a zero slot",
    "nibble_transpose": "closed form on tiny shapes (scalar loop), self-inverse, hand-made known answer, "
                        "dequantisation invariance (test_layout_decode.py:70-83)",
    "to_neuron_major": "dequantisation invariance; scales/biases moved bit for bit",
    "live_masks": "brute force (flatnonzero) incl. all-dead, all-live, +-0, NaN, last-group single live",
    "sparse_down": "textbook dequantised GEMV (test_layout_decode.py:128-142) on the stock layout; "
                   "zero h -> exactly 0; dense-h == all-live; linearity in the gains",
    "build_tiles": "hand-computed small case; invariants (each slot once, homogeneous tiles, NT formula, "
                   "shared tiles last)",
    "build_union": "brute force on small cases",
    "sparse_down_prefill": "per-slot textbook GEMV (independent of tiling); invariance to tt",
    "mamba_verify": "closed forms: impulse response of the conv (orientation), state 0 single step, "
                    "dA=1/B=0 identity, A_log -> large forgets the state; multi-row == sequential rows. "
                    "mlx-lm ssm_update's time_step_limit default and intermediate precisions: "
                    "parity unpinned (mlx-lm is not available here)",
    "greedy_accept": "brute force over all draft/target combinations",
    "rms_norm_bf16": "closed forms: a constant-magnitude row normalises to +-w exactly; scale invariance "
                     "under powers of two (eps = 0); a hand-computed known answer",
    "gated_rms_norm_bf16": "closed form: a group of constant |y| and constant gate gives +-w whatever "
                           "silu's value; groups are independent",
    "linear_q4": "brute force on tiny shapes (scalar loops over words and nibbles)",
    "argmax_bf16": "ties to the first index, NaN first, bf16 rounding ties; brute force",
    "embed_q4": "closed form: one dequantised row, exactly representable values round trip",
    "attention": "closed forms: one visible key returns its value row; equal keys average the value "
                 "rows; a dominant key selects its value row; GQA head grouping",
    "mamba_block_step / attn_block_step / moe_block_step / lm_head_logits": "compositions of the pinned "
                                                                              "functions above in the blocks' "
                                                                              "order (model.py, mamba.py)",
    "router_topk": "brute force over every subset of size topk on small E; normalised gains sum to the "
                   "scale; order and tie rule by construction. The gate's exact form in mlx-lm 0.31.3 "
                   "(nemotron_h) is not in the container: parity unpinned against it",
}
