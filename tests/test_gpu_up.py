"""GPU parity of the MoE front end after the router (hsd/model.py:110-121, 49-50): the
4-bit up projections of the selected and shared experts, ReLU^2, in pack's hcat layout
(model.py:123-129), with the canonical live masks.

Bars:
* h bit-identical to the oracle's relu2(bf16(u)) wherever the float64 pre-activation u
  is farther than the kernel's fp32 accumulation error from a bf16 rounding boundary.
  The error bound is 2^-20 M + 2^-23 |u| with M = sum_i (|s| (16 + q) + |b - 16 s|) |x_i|,
  the magnitude of every partial sum the kernel forms (u = 16 s sum (1 + q/16) x +
  (b - 16 s) sum x per 32-input piece: 16 roundings at the full magnitude, the depth of
  one piece's dot2 chain; the cross-piece sum adds far less). Within that distance
  of a boundary h must lie between relu2 of the two neighbouring bf16 values (the
  fraction of such elements is printed; at least 99 % are bit-identical overall);
* integer work bit-exact: the live masks equal those of the kernel's own h;
* a routed id outside [0, E): status flag, that slot exactly 0, the others unchanged.
"""
import numpy as np
import pytest
import torch

from hsd import decode, layout, synth as S
from hsd.moe import up_relu2
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
D, F, FS, K, E = 2688, 1856, 3712, 6, 128


def inputs(seed, B, E=E, D=D):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16((rng.standard_normal((B, D)) * 0.5).astype(np.float32))
    sel = np.stack([rng.permutation(E)[:K] for _ in range(B)]).astype(np.int32)
    return x, sel


def masks_of(h_bits):
    live = (h_bits & 0x7FFF) != 0
    w = 1 << np.arange(64, dtype=np.uint64)
    return (live.reshape(live.shape[0], -1, 64).astype(np.uint64) * w).sum(-1, dtype=np.uint64).reshape(-1)


def check(h, ref, x_bits, sel, lay, F, FS, topk):
    """h, ref [B, topk*F + FS] bf16 bits (kernel, oracle); the bar in the module doc."""
    assert np.mean(h == ref) >= 0.99
    x = O.bf16_to_f32(x_bits).astype(np.float64)
    n_edge = 0
    for b in range(x.shape[0]):
        slots = [(k * F, lay["w1"][e], lay["s1"][e], lay["b1"][e]) for k, e in enumerate(sel[b])]
        slots.append((topk * F, lay["sw1"], lay["ss1"], lay["sb1"]))
        for off, w, sc, bi in slots:
            q = O.unpack_nibbles(w).astype(np.float64)
            sf = np.repeat(O.bf16_to_f32(sc).astype(np.float64), 64, axis=-1)
            bf = np.repeat(O.bf16_to_f32(bi).astype(np.float64), 64, axis=-1)
            u = (sf * q + bf) @ x[b]
            m = (np.abs(sf) * (16 + q) + np.abs(bf - 16 * sf)) @ np.abs(x[b])
            err = 2.0 ** -20 * m + 2.0 ** -23 * np.abs(u)
            lo, mid, hi = O.relu2_bf16(u - err), O.relu2_bf16(u), O.relu2_bf16(u + err)
            got = h[b, off:off + len(u)]
            edge = lo != hi
            assert np.array_equal(got[~edge], mid[~edge])
            gv = O.bf16_to_f32(got[edge])
            assert np.all((O.bf16_to_f32(lo[edge]) <= gv) & (gv <= O.bf16_to_f32(hi[edge])))
            n_edge += int(edge.sum())
    print(f"bit-identical {np.mean(h == ref):.5f}; within the accumulation error of a bf16 boundary "
          f"{n_edge / h.size:.4f}")


@pytest.fixture(scope="module")
def up(dev):
    lay = S.moe_up_np(5)
    return lay, {k: S.to_device(v, dev) for k, v in lay.items()}


def test_up_relu2_matches_oracle(up, dev):
    lay, dv = up
    x, sel = inputs(6, 2)
    masks = torch.zeros(2 * (K * F + FS) // 64, dtype=torch.int64, device=dev)
    h = up_relu2(S.to_device(x, dev), S.to_device(sel, dev), dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"],
                 dv["sb1"], topk=K, live_masks=masks)
    hb = h.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.up_relu2(x, sel, lay["w1"], lay["s1"], lay["b1"], lay["sw1"], lay["ss1"], lay["sb1"], F=F, FS=FS, topk=K)
    check(hb, ref, x, sel, lay, F, FS, K)
    assert np.array_equal(masks.cpu().numpy().view(np.uint64), masks_of(hb))


def test_rows_do_not_depend_on_batch(up, dev):
    """A token row's h and mask bits are the same in a call of 1, 3 or 6 rows (the shared
    expert's blocks take tiles of up to 4 rows: at B = 6 a tile of 4 and one of 2)."""
    lay, dv = up
    x, sel = inputs(13, 6)
    args = (dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"], dv["sb1"])
    nm = (K * F + FS) // 64

    def run(lo, hi):
        m = torch.zeros((hi - lo) * nm, dtype=torch.int64, device=dev)
        h = up_relu2(S.to_device(x[lo:hi], dev), S.to_device(sel[lo:hi], dev), *args, topk=K, live_masks=m)
        return h.view(torch.int16).cpu().numpy(), m.cpu().numpy()

    h6, m6 = run(0, 6)
    for lo, hi in [(0, 3), (3, 6), (2, 3), (5, 6), (0, 1)]:
        h, m = run(lo, hi)
        assert np.array_equal(h, h6[lo:hi]), (lo, hi)
        assert np.array_equal(m, m6[lo * nm:hi * nm]), (lo, hi)
    ref = O.up_relu2(x, sel, lay["w1"], lay["s1"], lay["b1"], lay["sw1"], lay["ss1"], lay["sb1"], F=F, FS=FS, topk=K)
    check(h6.view(np.uint16), ref, x, sel, lay, F, FS, K)


def test_bad_expert_id(up, dev):
    lay, dv = up
    x, sel = inputs(7, 1)
    bad = sel.copy()
    bad[0, 3] = E + 9
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    args = (dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"], dv["sb1"])
    h = up_relu2(S.to_device(x, dev), S.to_device(bad, dev), *args, topk=K, status=status)
    h0 = up_relu2(S.to_device(x, dev), S.to_device(sel, dev), *args, topk=K)
    assert int(status.item()) == 1
    assert torch.all(h[0, 3 * F:4 * F].view(torch.int16) == 0)
    keep = torch.ones(K * F + FS, dtype=torch.bool, device=dev)
    keep[3 * F:4 * F] = False
    assert torch.equal(h[0, keep].view(torch.int16), h0[0, keep].view(torch.int16))


def test_small_shape(dev):
    """D=256 (8 pieces per row: most lanes idle), F=128, FS=192, 4 experts, top-2."""
    d, f, fs, e, k = 256, 128, 192, 4, 2
    lay = S.moe_up_np(8, n_experts=e, d=d, f=f, fs=fs)
    dv = {n: S.to_device(v, dev) for n, v in lay.items()}
    rng = np.random.default_rng(9)
    x = O.f32_to_bf16((rng.standard_normal((3, d)) * 0.5).astype(np.float32))
    sel = np.stack([rng.permutation(e)[:k] for _ in range(3)]).astype(np.int32)
    h = up_relu2(S.to_device(x, dev), S.to_device(sel, dev), dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"],
                 dv["sb1"], topk=k)
    ref = O.up_relu2(x, sel, lay["w1"], lay["s1"], lay["b1"], lay["sw1"], lay["ss1"], lay["sb1"], F=f, FS=fs, topk=k)
    check(h.view(torch.int16).cpu().numpy().view(np.uint16), ref, x, sel, lay, f, fs, k)


def test_large_d_instance(dev):
    """D=3584 takes the kernel instance sized for D <= 4096 (the reference shape's 2688
    takes the one for D <= 3072): F=128, FS=192, 4 experts, top-2."""
    d, f, fs, e, k = 3584, 128, 192, 4, 2
    lay = S.moe_up_np(11, n_experts=e, d=d, f=f, fs=fs)
    dv = {n: S.to_device(v, dev) for n, v in lay.items()}
    rng = np.random.default_rng(12)
    x = O.f32_to_bf16((rng.standard_normal((3, d)) * 0.5).astype(np.float32))
    sel = np.stack([rng.permutation(e)[:k] for _ in range(3)]).astype(np.int32)
    h = up_relu2(S.to_device(x, dev), S.to_device(sel, dev), dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"],
                 dv["sb1"], topk=k)
    ref = O.up_relu2(x, sel, lay["w1"], lay["s1"], lay["b1"], lay["sw1"], lay["ss1"], lay["sb1"], F=f, FS=fs, topk=k)
    check(h.view(torch.int16).cpu().numpy().view(np.uint16), ref, x, sel, lay, f, fs, k)


def test_front_end_feeds_the_down_projection(up, dev):
    """hcat from the front end goes straight into the sparse down projection; its live
    masks are the ones the down kernel derives from the same hcat."""
    lay, dv = up
    x, sel = inputs(10, 1)
    m_up = torch.zeros((K * F + FS) // 64, dtype=torch.int64, device=dev)
    h = up_relu2(S.to_device(x, dev), S.to_device(sel, dev), dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"],
                 dv["sb1"], topk=K, live_masks=m_up)
    down = S.moe_layer_np(11)
    dd = {k2: S.to_device(v, dev) for k2, v in down.items()}
    nm = layout.to_neuron_major(dd["w"], dd["s"], dd["b"]) + layout.to_neuron_major(dd["sw"], dd["ss"], dd["sb"])
    gains = torch.cat([torch.rand((1, K), device=dev), torch.ones((1, 1), device=dev)], dim=1)
    m_dn = torch.zeros_like(m_up)
    decode.sparse_down(h, S.to_device(sel, dev), gains, *nm, F=F, FS=FS, D=D, topk=K, live_masks=m_dn)
    assert torch.equal(m_up, m_dn)
