"""Pins the oracle's prefill pieces (hsd/prefill.py:48-321): a hand-computed tile order,
the tile invariants, the union by brute force, and the grouped down projection by the
per-slot textbook dequantised GEMV (independent of tiles, unions and tt)."""
import numpy as np
import pytest

from oracle import hsd_oracle as O
from hsd import synth as S


def test_build_tiles_hand_computed():
    # T=3 tokens, topk=2, E=3, tt=2. slots: 0:e1 1:e0 2:e1 3:e2 4:e1 5:e0
    sel = np.array([[1, 0], [1, 2], [1, 0]], np.int32)
    te, ts = O.build_tiles(sel, E=3, tt=2)
    # counts e0=2 e1=3 e2=1 -> tiles e0:1, e1:2, e2:1 -> 4 routed; NT_routed = 3*2//2 + 3 = 6
    # shared: ceil(3/2) = 2 tiles of expert 3
    assert te.tolist() == [0, 1, 1, 2, -1, -1, 3, 3]
    assert ts.tolist() == [1, 5, 0, 2, 4, -1, 3, -1, -1, -1, -1, -1, 0, 1, 2, -1]


@pytest.mark.parametrize("T,tt", [(64, 32), (512, 32), (512, 64), (37, 32)])
def test_build_tiles_invariants(T, tt):
    rng = np.random.default_rng(T + tt)
    E, K = 128, 6
    sel = S.zipf_sel_np(rng, T, E, K)
    te, ts = O.build_tiles(sel, E, tt)
    NT = T * K // tt + E + (T + tt - 1) // tt
    assert te.shape == (NT,) and ts.shape == (NT * tt,)
    nt_routed = T * K // tt + E
    routed = ts[:nt_routed * tt]
    assert sorted(routed[routed >= 0].tolist()) == list(range(T * K))   # every slot once
    flat = sel.reshape(-1)
    prev = -1
    for t in range(nt_routed):
        slots = ts[t * tt:(t + 1) * tt]
        v = slots[slots >= 0]
        if te[t] < 0:
            assert v.size == 0
            continue
        assert v.size > 0 and np.all(flat[v] == te[t])                    # homogeneous
        assert te[t] >= prev                                             # experts ascending
        assert np.all(np.diff(v) > 0)                                    # stable order
        prev = te[t]
    assert np.all(te[nt_routed:] == E)                                   # shared tiles last
    sh = ts[nt_routed * tt:]
    assert sh[:T].tolist() == list(range(T)) and np.all(sh[T:] == -1)


def test_build_union_brute_force():
    rng = np.random.default_rng(4)
    E, K, F, FS, T, tt = 16, 2, 128, 192, 40, 8
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    h = np.where(rng.random((T, K * F + FS)) < 0.05, 1.0, 0.0).astype(np.float32)
    te, ts = O.build_tiles(sel, E, tt)
    ul, uc = O.build_union(h, te, ts, F=F, FS=FS, topk=K, E=E, tt=tt)
    assert ul.shape == (te.shape[0], 192)
    for t in range(te.shape[0]):
        if te[t] < 0:
            assert uc[t] == 0 and np.all(ul[t] == -1)
            continue
        shared = te[t] == E
        width = FS if shared else F
        cols = set()
        for s in ts[t * tt:(t + 1) * tt]:
            if s < 0:
                continue
            row = h[s] [K * F:] if shared else h[s // K][(s % K) * F:(s % K + 1) * F]
            cols |= {c for c in range(width) if row[c] != 0}
        assert uc[t] == len(cols)
        assert ul[t, :uc[t]].tolist() == sorted(cols) and np.all(ul[t, uc[t]:] == -1)


@pytest.mark.parametrize("tt", [8, 16])
def test_prefill_matches_per_slot_textbook(tt):
    E, K, F, FS, D, T = 8, 2, 128, 192, 128, 24
    lay = S.moe_layer_np(11, n_experts=E, d=D, f=F, fs=FS)
    h, sel, gains = S.prefill_inputs_np(12, T=T, zero_frac=0.8, n_experts=E, f=F, fs=FS, topk=K)
    h = O.bf16_to_f32(h)
    pw, ps, pb = O.to_neuron_major(lay["w"], lay["s"], lay["b"])
    spw, sps, spb = O.to_neuron_major(lay["sw"], lay["ss"], lay["sb"])
    y, part = O.sparse_down_prefill(h, sel, gains, pw, ps, pb, spw, sps, spb, F=F, FS=FS, D=D,
                                    topk=K, E=E, tt=tt)
    ref = O.dense_reference(h, sel, gains, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"], lay["sb"],
                            F=F, FS=FS, D=D, topk=K)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    assert part.shape == (T * (K + 1), D)
