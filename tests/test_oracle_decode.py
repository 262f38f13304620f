"""Pins the oracle's sparse decode down projection (hsd/decode.py:37-186): canonical
compaction by brute force incl. the edge cases, the sum by the textbook dequantised
GEMV of tests/test_layout_decode.py:128-142 on the STOCK layout (an independent formula:
full dequantisation, no group factorisation, no skipping), exact zero for a zero h,
skip-exactness (dense-h == sparse) and linearity in the gains."""
import numpy as np
import pytest

from oracle import hsd_oracle as O
from hsd import synth as S

SMALL = dict(E=8, D=256, F=192, FS=384, topk=3)


def small_case(seed, B=2, zero_frac=0.9, **kw):
    c = dict(SMALL, **kw)
    lay = S.moe_layer_np(seed, n_experts=c["E"], d=c["D"], f=c["F"], fs=c["FS"])
    h, sel, gains = S.decode_inputs_np(seed + 1, B=B, zero_frac=zero_frac, n_experts=c["E"], f=c["F"],
                                       fs=c["FS"], topk=c["topk"])
    pw, ps, pb = O.to_neuron_major(lay["w"], lay["s"], lay["b"])
    spw, sps, spb = O.to_neuron_major(lay["sw"], lay["ss"], lay["sb"])
    return c, lay, O.bf16_to_f32(h), sel, gains, (pw, ps, pb, spw, sps, spb)


def test_live_masks_brute_force_and_edges():
    F, FS, topk = 128, 192, 2
    rng = np.random.default_rng(0)
    h = np.where(rng.random((3, topk * F + FS)) < 0.2, 1.0, 0.0).astype(np.float32)
    h[1] = 0.0                                  # all dead
    h[2] = 1.0                                  # all live
    h[0, 5] = -0.0                              # -0 is dead
    h[0, 6] = np.nan                            # NaN is live
    h[0, F - 1] = 3.0                           # single live neuron in the last group of a slot
    m = O.live_masks(h, F, FS, topk)
    for b in range(3):
        for g in range(m.shape[1]):
            seg = h[b, 64 * g:64 * (g + 1)]
            want = sum(1 << j for j in range(64) if (seg[j] != 0 or np.isnan(seg[j])))
            assert int(m[b, g]) == want
    assert not (int(m[0, 0]) >> 5) & 1 and (int(m[0, 0]) >> 6) & 1
    assert np.all(m[1] == 0) and np.all(m[2] == np.uint64(2 ** 64 - 1))


@pytest.mark.parametrize("zero_frac", [0.0, 0.7, 0.9, 0.97])
def test_sparse_down_matches_textbook_dequantised_gemv(zero_frac):
    c, lay, h, sel, gains, nm = small_case(3, zero_frac=zero_frac)
    y = O.sparse_down(h, sel, gains, *nm, F=c["F"], FS=c["FS"], D=c["D"], topk=c["topk"])
    ref = O.dense_reference(h, sel, gains, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"], lay["sb"],
                            F=c["F"], FS=c["FS"], D=c["D"], topk=c["topk"])
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_sparse_down_zero_h_is_exactly_zero_and_skip_is_exact():
    c, lay, h, sel, gains, nm = small_case(5)
    kw = dict(F=c["F"], FS=c["FS"], D=c["D"], topk=c["topk"])
    assert np.all(O.sparse_down(np.zeros_like(h), sel, gains, *nm, **kw) == 0.0)
    # skipping dead rows changes nothing: the all-rows (dense-h) sum equals the sparse one
    assert np.array_equal(O.sparse_down(h, sel, gains, *nm, **kw),
                          O.sparse_down(h, sel, gains, *nm, dense=True, **kw))


def test_sparse_down_linear_in_gains():
    c, lay, h, sel, gains, nm = small_case(7, B=1)
    kw = dict(F=c["F"], FS=c["FS"], D=c["D"], topk=c["topk"])
    y = O.sparse_down(h, sel, gains, *nm, **kw).astype(np.float64)
    parts = []
    for k in range(c["topk"] + 1):
        g = np.zeros_like(gains)
        g[:, k] = gains[:, k]
        parts.append(O.sparse_down(h, sel, g, *nm, **kw).astype(np.float64))
    assert np.allclose(sum(parts), y, rtol=1e-5, atol=1e-6 * np.abs(y).max())
    g2 = gains.copy()
    g2[:, 0] *= 2
    y2 = O.sparse_down(h, sel, g2, *nm, **kw).astype(np.float64)
    assert np.allclose(y2 - y, parts[0], rtol=1e-4, atol=1e-5 * np.abs(y).max())


def test_touched_bytes_model():
    """bench/common.py:16-19, 78-83: live rows x D/2 + live groups x 4D (+ I/O)."""
    F, FS, topk, D = 128, 128, 1, 256
    h = np.zeros((1, topk * F + FS), np.float32)
    h[0, [0, 1, 70]] = 1.0          # slot 0: rows 0, 1 (group 0), 70 (group 1)
    h[0, F + 3] = 1.0               # shared: row 3 (group 0)
    io = (topk * F + FS) * 2 + topk * 4 + (topk + 1) * 4 + D * 2
    assert O.touched_bytes(h, F, FS, topk, D) == 4 * (D // 2) + 3 * 4 * D + io
    assert O.touched_bytes(h, F, FS, topk, D, dense=True) == (topk * F + FS) * (D // 2) + 4 * 4 * D + io
