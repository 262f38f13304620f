"""Pins the oracle's restatement of the decode step's other pieces (norms, projections,
argmax, embedding, attention, router) with checks the mathematics fixes: closed forms,
invariants and brute force -- not by retyping the formulas."""
import itertools

import numpy as np

from hsd import synth as S
from oracle import hsd_oracle as O


def bf(x):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(x, dtype=np.float32)))


def test_rms_norm_closed_forms():
    w = bf(np.linspace(0.5, 2.0, 64))
    # a row of constant magnitude normalises to +-1 (eps = 0), so the output is +-w exactly
    x = bf(np.where(np.arange(64) % 3 == 0, -0.75, 0.75))
    out = O.bf16_to_f32(O.rms_norm_bf16(x, w, eps=0.0))
    assert np.array_equal(out, bf(np.sign(x) * w))
    # invariance under a power-of-two scale (eps = 0)
    rng = np.random.default_rng(0)
    x = bf(rng.standard_normal(256))
    w2 = bf(rng.uniform(0.5, 1.5, 256))
    assert np.array_equal(O.rms_norm_bf16(x, w2, eps=0.0), O.rms_norm_bf16(bf(x * 8.0), w2, eps=0.0))
    # known answer: x = [3, 4]: mean square 12.5, x / sqrt(12.5) = [0.8485.., 1.1313..]
    out = O.bf16_to_f32(O.rms_norm_bf16(np.array([3.0, 4.0]), np.array([1.0, 1.0]), eps=0.0))
    assert np.array_equal(out, bf([3 / np.sqrt(12.5), 4 / np.sqrt(12.5)]))


def test_gated_norm_closed_form():
    # each group of 512: |y| constant and the gate constant -> z has constant magnitude, so
    # the group normalises to sign(y) sign(gate) w whatever the magnitude of silu(gate) is
    # (silu(g) has the sign of g)
    rng = np.random.default_rng(1)
    w = bf(rng.uniform(0.5, 1.5, 1024))
    mags = [0.3, 7.0]
    y = np.concatenate([mags[g] * np.where(rng.random(512) < 0.5, -1.0, 1.0) for g in range(2)]).astype(np.float32)
    gate = np.concatenate([np.full(512, 1.7), np.full(512, -0.4)])
    out = O.bf16_to_f32(O.gated_rms_norm_bf16(y[None], bf(gate)[None], w, eps=0.0))[0]
    assert np.array_equal(out, bf(np.sign(y) * np.sign(gate) * w))


def test_linear_q4_brute_force():
    rng = np.random.default_rng(2)
    O_, I = 4, 128
    w, s, b = S.down_proj_np(rng, (), O_, I)
    x = bf(rng.standard_normal((2, I)))
    got = O.linear_q4(x, w, s, b)
    sv, bv = O.bf16_to_f32(s), O.bf16_to_f32(b)
    for r in range(2):
        for o in range(O_):
            acc = 0.0
            for i in range(I):
                q = (int(w[o, i // 8]) >> (4 * (i % 8))) & 0xF
                acc += float(x[r, i]) * (float(sv[o, i // 64]) * q + float(bv[o, i // 64]))
            assert abs(got[r, o] - acc) <= 1e-9 * (1 + abs(acc))


def test_argmax_bf16_rules():
    # bf16 rounding makes 1.0 and 1.001 equal: the first index wins
    assert O.argmax_bf16(np.array([0.5, 1.001, 1.0, -3.0]))[0] == 1
    assert O.argmax_bf16(np.array([0.5, 1.0, 1.001]))[0] == 1
    assert O.argmax_bf16(np.array([0.5, np.nan, 9.0, np.nan]))[0] == 1
    rng = np.random.default_rng(3)
    v = rng.standard_normal((5, 300)).astype(np.float32)
    got = O.argmax_bf16(v)
    for r in range(5):
        rb = bf(v[r])
        best = max(range(300), key=lambda i: (rb[i], -i))
        assert got[r] == best


def test_embed_closed_form():
    rng = np.random.default_rng(4)
    w, s, b = S.down_proj_np(rng, (), 10, 128)
    out = O.embed_q4(np.array([3, 9, 10, -1]), w, s, b)
    for i, t in enumerate((3, 9)):
        row = O.dequantize(w[t], s[t], b[t])
        assert np.array_equal(O.bf16_to_f32(out[i]), bf(row))
    assert not out[2].any() and not out[3].any()
    # a scale of 1 and bias 0: the nibbles themselves
    s1 = np.full_like(s, O.f32_to_bf16(np.float32(1.0)))
    b0 = np.zeros_like(b)
    q = O.unpack_nibbles(w[5]).astype(np.float32)
    assert np.array_equal(O.bf16_to_f32(O.embed_q4(np.array([5]), w, s1, b0)[0]), q)


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    HQ, HKV, HD, Sn = 4, 2, 8, 5
    q = rng.standard_normal((HQ, HD))
    v = rng.standard_normal((HKV, Sn, HD))
    # one visible key: the output is its value row
    k1 = rng.standard_normal((HKV, 1, HD))
    out = O.attention(q, k1, v[:, :1], 0.3)
    for h in range(HQ):
        assert np.allclose(out[h], v[h // 2, 0], atol=1e-12)
    # equal keys: the mean of the value rows
    ke = np.repeat(rng.standard_normal((HKV, 1, HD)), Sn, axis=1)
    out = O.attention(q, ke, v, 0.3)
    for h in range(HQ):
        assert np.allclose(out[h], v[h // 2].mean(axis=0), atol=1e-12)
    # a dominant key selects its value row (kv head grouping h // 2)
    kd = rng.standard_normal((HKV, Sn, HD)) * 1e-3
    kd[:, 3] = 0.0
    qd = np.zeros((HQ, HD))
    qd[:, 0] = 1.0
    kd[:, 3, 0] = 1e4
    out = O.attention(qd, kd, v, 1.0)
    for h in range(HQ):
        assert np.allclose(out[h], v[h // 2, 3], atol=1e-9)


def test_router_topk_brute_force():
    rng = np.random.default_rng(6)
    E, K = 9, 3
    for _ in range(20):
        lg = bf(rng.standard_normal((1, E)) * 2)
        bias = rng.standard_normal(E).astype(np.float32) * 0.1
        sel, gains = O.router_topk(lg, bias, K, scale=2.5)
        sc = 1 / (1 + np.exp(-lg[0].astype(np.float64)))
        ch = sc + bias
        best = max(itertools.combinations(range(E), K), key=lambda c: sum(ch[list(c)]))
        assert sorted(sel[0].tolist()) == sorted(best)
        assert list(sel[0]) == sorted(best, key=lambda e: -ch[e])          # descending choice
        assert abs(gains[0].sum() - 2.5) < 1e-9                             # normalised, then scaled
        assert np.allclose(gains[0] / 2.5, sc[sel[0]] / sc[sel[0]].sum(), rtol=1e-6)
    # equal choices: the smaller expert id first
    sel, _ = O.router_topk(np.zeros((1, 6)), None, 4)
    assert sel[0].tolist() == [0, 1, 2, 3]
    sel, g = O.router_topk(np.zeros((1, 6)), None, 2, scale=1.0, norm_topk=False)
    assert np.allclose(g, 0.5)
