"""Pins the oracle's MoE front end after the router (hsd/model.py:110-121: the routed
experts' 4-bit up projection by gather_qmm, the shared expert's up_proj, ReLU^2) by
brute force on tiny shapes and by special values, not by restating its formula."""
import numpy as np

from oracle import hsd_oracle as O


def brute_up(x, w, s, b):
    """u[o] = sum_i (s[o, i//64] * nibble(w[o, i//8], i%8) + b[o, i//64]) * x[i], scalar
    loops over words and nibbles (low nibble first)."""
    O_, IW = w.shape
    u = np.zeros(O_)
    for o in range(O_):
        acc = 0.0
        for wi in range(IW):
            word = int(w[o, wi])
            for n in range(8):
                i = 8 * wi + n
                q = (word >> (4 * n)) & 0xF
                sc = float(O.bf16_to_f32(np.uint16(s[o, i // 64])))
                bi = float(O.bf16_to_f32(np.uint16(b[o, i // 64])))
                acc += (sc * q + bi) * float(x[i])
        u[o] = acc
    return u


def rand_proj(rng, rows, cols):
    w = rng.integers(0, 2 ** 32, size=(rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    s = O.f32_to_bf16(rng.uniform(0.005, 0.02, size=(rows, cols // 64)).astype(np.float32))
    b = O.f32_to_bf16(rng.normal(0, 0.01, size=(rows, cols // 64)).astype(np.float32))
    return w, s, b


def test_up_proj_brute_force():
    rng = np.random.default_rng(0)
    w, s, b = rand_proj(rng, 5, 128)
    x = rng.standard_normal(128)
    assert np.allclose(O.up_proj_f64(x, w, s, b), brute_up(x, w, s, b), rtol=1e-12, atol=1e-12)


def test_up_proj_orientation():
    """One nibble set: output o sees input i only through W[o, i]."""
    w = np.zeros((3, 16), dtype=np.uint32)
    w[1, 2] = np.uint32(7 << 12)                    # W[1, 8*2 + 3] has q = 7
    s = np.full((3, 2), O.f32_to_bf16(np.float32(0.5)), dtype=np.uint16)
    b = np.zeros((3, 2), dtype=np.uint16)
    x = np.zeros(128)
    x[19] = 2.0
    assert np.array_equal(O.up_proj_f64(x, w, s, b), [0.0, 7.0, 0.0])


def test_relu2_special_values():
    u = np.array([-3.0, -0.0, 0.0, 1.5, np.nan, 3.0], dtype=np.float32)
    h = O.relu2_bf16(u)
    assert h[0] == 0 and h[1] == 0 and h[2] == 0
    assert O.bf16_to_f32(h[3]) == 2.25 and O.bf16_to_f32(h[5]) == 9.0
    assert np.isnan(O.bf16_to_f32(h[4]))
    # u rounds to bf16 before the square: 1 + 2^-9 -> 1.0 (ties to even), squared 1.0
    assert O.bf16_to_f32(O.relu2_bf16(np.array([1.0 + 2 ** -9], np.float32))[0]) == 1.0
    # the square rounds to bf16: 1.0078125^2 = 1.01568603515625 -> 1.015625
    assert O.bf16_to_f32(O.relu2_bf16(np.array([1.0078125], np.float32))[0]) == 1.015625


def test_up_relu2_slot_layout_and_bad_id():
    rng = np.random.default_rng(1)
    E, F, FS, D, K = 3, 64, 128, 128, 2
    w1, s1, b1 = (np.stack(a) for a in zip(*[rand_proj(rng, F, D) for _ in range(E)]))
    sw1, ss1, sb1 = rand_proj(rng, FS, D)
    x = O.f32_to_bf16(rng.standard_normal((2, D)).astype(np.float32))
    sel = np.array([[2, 0], [1, 7]], dtype=np.int32)            # 7: out of range
    h = O.up_relu2(x, sel, w1, s1, b1, sw1, ss1, sb1, F=F, FS=FS, topk=K)
    xf = O.bf16_to_f32(x).astype(np.float64)
    for bi in range(2):
        for k in range(K):
            e = sel[bi, k]
            want = O.relu2_bf16(brute_up(xf[bi], w1[e], s1[e], b1[e])) if e < E else np.zeros(F, np.uint16)
            assert np.array_equal(h[bi, k * F:(k + 1) * F], want)
        assert np.array_equal(h[bi, K * F:], O.relu2_bf16(brute_up(xf[bi], sw1, ss1, sb1)))
