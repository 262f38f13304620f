"""Pins the oracle's layout permutation (hsd/layout.py:34-74) without the reference:
scalar closed form, a hand-made known answer, self-inverse, and dequantisation
invariance (the check of tests/test_layout_decode.py:70-83)."""
import numpy as np
import pytest

from oracle import hsd_oracle as O


def scalar_nibble_transpose(w):
    """out[.., c, wo] = sum_n W[8*wo+n, c] << 4n, element by element (layout.py:35-36)."""
    *lead, R, CW = w.shape
    flat = w.reshape(-1, R, CW)
    out = np.zeros((flat.shape[0], CW * 8, R // 8), dtype=np.uint32)
    for b in range(flat.shape[0]):
        for c in range(CW * 8):
            for wo in range(R // 8):
                v = 0
                for n in range(8):
                    r = 8 * wo + n
                    nib = (int(flat[b, r, c // 8]) >> (4 * (c % 8))) & 0xF
                    v |= nib << (4 * n)
                out[b, c, wo] = v
    return out.reshape(*lead, CW * 8, R // 8)


@pytest.mark.parametrize("shape", [(5, 24, 9), (8, 2), (2, 16, 3), (40, 1)])
def test_nibble_transpose_matches_scalar_closed_form(shape):
    rng = np.random.default_rng(0)
    w = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(O.nibble_transpose(w), scalar_nibble_transpose(w))


def test_nibble_transpose_known_answer():
    # W[r, c] = (r + c) % 16 for an 8 x 8 block: stock word r packs W[r, 0..7] low nibble first
    W = (np.arange(8)[:, None] + np.arange(8)[None, :]) % 16
    w = np.array([[sum(int(W[r, c]) << (4 * c) for c in range(8))] for r in range(8)], dtype=np.uint32)
    out = O.nibble_transpose(w)
    assert out.shape == (8, 1)
    # neuron-major word c packs W[0..7, c]; W symmetric here, so out == w; and a concrete word
    assert out[0, 0] == 0x76543210 and out[1, 0] == 0x87654321
    assert np.array_equal(out, w)
    # an asymmetric block: only W[2, 5] = 0xA set
    w2 = np.zeros((8, 1), np.uint32)
    w2[2, 0] = 0xA << (4 * 5)
    o2 = O.nibble_transpose(w2)
    assert o2[5, 0] == 0xA << (4 * 2) and np.count_nonzero(o2) == 1


@pytest.mark.parametrize("shape", [(5, 24, 9), (3, 64, 16), (2688, 29)])
def test_nibble_transpose_self_inverse(shape):
    rng = np.random.default_rng(1)
    w = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    t = O.nibble_transpose(w)
    assert t.shape == (*shape[:-2], shape[-1] * 8, shape[-2] // 8)
    assert np.array_equal(O.nibble_transpose(t), w)


def test_to_neuron_major_dequantises_identically():
    rng = np.random.default_rng(2)
    E, D, F = 3, 128, 192
    w = rng.integers(0, 2 ** 32, size=(E, D, F // 8), dtype=np.uint64).astype(np.uint32)
    s = O.f32_to_bf16(rng.uniform(0.005, 0.02, size=(E, D, F // 64)))
    b = O.f32_to_bf16(rng.normal(0, 0.01, size=(E, D, F // 64)))
    pw, ps, pb = O.to_neuron_major(w, s, b)
    assert pw.shape == (E, F, D // 8) and ps.shape == (E, F // 64, D)
    ref = O.dequantize(w, s, b)                                  # [E, D, F]
    back = O.dequantize(O.nibble_transpose(pw), np.swapaxes(ps, -1, -2), np.swapaxes(pb, -1, -2))
    assert np.array_equal(back, ref)
    # neuron-major row i dequantised directly is column i of the stock matrix
    rows = O.dequant_rows(pw[1], ps[1], pb[1], np.arange(F))
    assert np.array_equal(rows, ref[1].T)


def test_bf16_roundtrip_and_rounding():
    x = np.array([1.0, -2.5, 3.14159, 1e-8, 65504.0, np.inf, -np.inf, 0.0, -0.0], np.float32)
    b = O.f32_to_bf16(x)
    assert O.bf16_to_f32(b)[0] == 1.0 and O.bf16_to_f32(b)[1] == -2.5
    assert O.bf16_to_f32(b)[2] == np.float32(3.140625)          # RNE of 3.14159
    assert np.isinf(O.bf16_to_f32(b)[5]) and O.bf16_to_f32(b)[6] < 0
    assert b[8] == 0x8000
    assert O.f32_to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0
    # ties to even: 1 + 2^-8 lies halfway between bf16 1.0 and 1.0078125 -> 1.0
    assert O.bf16_to_f32(O.f32_to_bf16(np.array([1 + 2 ** -8], np.float32)))[0] == 1.0
    assert O.bf16_to_f32(O.f32_to_bf16(np.array([1 + 3 * 2 ** -8], np.float32)))[0] == np.float32(1 + 2 ** -6)
