"""GPU parity of the Mamba-2 multi-row verify with per-row checkpoints and rollback
(hsd/mamba.py:19-56) and of the device greedy acceptance (hsd/model.py:419-427), at the
Nemotron-3.5 Mamba-2 shape (64 heads x head_dim 64, state 128, 8 groups, conv 4, fp32 state).

Bars: the verify of L rows is BIT-IDENTICAL to L single-row calls (y, ssm and conv
checkpoints); against the float64 oracle the fp32 states are within 1e-4 relative and
the bf16 outputs within |y - ref| <= 2e-2 + 1e-2*|ref|; the rollback restores exactly the
checkpoint of the kept prefix; acceptance integers are exact."""
import itertools

import numpy as np
import pytest
import torch

from hsd import mamba as M, mtp, synth as S
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
H, P, N, G = 64, 64, 128, 8
DI, CD = H * P, H * P + 2 * G * N


def make(dev, seed):
    p = S.mamba_params_np(seed)
    mixer = M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                          A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                          D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev))
    cache = M.MambaCache(mixer, dev, nslab=4, conv_state=S.to_device(p["conv_state"], dev),
                         ssm_state=torch.from_numpy(p["ssm_state"]).to(dev))
    return p, mixer, cache


def oracle(p, rows, cs=None, ss=None):
    r = O.bf16_to_f32(rows)
    return O.mamba_verify(r[:, DI:DI + CD], r[:, DI + CD:], r[:, :DI], O.bf16_to_f32(p["conv_w"]),
                          O.bf16_to_f32(p["conv_b"]), p["A_log"], p["dt_bias"], p["D"], O.bf16_to_f32(p["norm_w"]),
                          O.bf16_to_f32(p["conv_state"]) if cs is None else cs,
                          p["ssm_state"] if ss is None else ss, n_groups=G)


@pytest.mark.parametrize("L", [1, 2, 3])
def test_verify_matches_oracle(dev, L):
    p, mixer, cache = make(dev, 1)
    rows = S.mamba_rows_np(np.random.default_rng(2), L)
    y = M.verify_rows(mixer, S.to_device(rows, dev), cache)
    ref = oracle(p, rows)
    yh = y.float().cpu().numpy()
    assert np.all(np.abs(yh - ref["y"]) <= 2e-2 + 1e-2 * np.abs(ref["y"]))
    for r in range(L):
        slab = (0 + 1 + r) % 4
        st = cache.ssm[slab].cpu().numpy()
        err = np.abs(st - ref["ssm_states"][r]).max() / np.abs(ref["ssm_states"][r]).max()
        assert err <= 1e-4, (r, err)
        cv = S.to_host(cache.conv[slab])
        assert np.array_equal(O.bf16_to_f32(cv), ref["conv_states"][r])


def test_verify_bit_identical_to_single_rows_and_rollback(dev):
    p, mixer, cache = make(dev, 3)
    rows = S.mamba_rows_np(np.random.default_rng(4), 3)
    rd = S.to_device(rows, dev)
    y3 = M.verify_rows(mixer, rd, cache)
    ssm3 = cache.ssm.clone()
    conv3 = cache.conv.clone()
    _, mixer1, c1 = make(dev, 3)
    ys = []
    for r in range(3):
        ys.append(M.verify_rows(mixer1, rd[r:r + 1], c1))
        M.mamba_rollback([(c1, 1)], 1)                     # accept the single row
    assert torch.equal(torch.cat(ys), y3)
    for r in range(3):
        assert torch.equal(c1.ssm[(1 + r) % 4], ssm3[(1 + r) % 4])
        assert torch.equal(c1.conv[(1 + r) % 4], conv3[(1 + r) % 4])
    # rollback of the 3-row verify to each prefix names the right checkpoint
    for n_keep in range(4):
        cache.cur.zero_()
        M.mamba_rollback([(cache, 3)], n_keep)
        cs, ss = cache.state()
        if n_keep == 0:
            assert np.array_equal(ss.cpu().numpy(), p["ssm_state"])
        else:
            assert torch.equal(ss, ssm3[n_keep % 4])


def test_verify_then_rollback_then_single_step_equals_single_steps(dev):
    """verify(3) -> rollback to 2 -> one more row == 3 single rows (the reference's test
    tests/test_verify_rollback.py:333-344, here bit-exact)."""
    p, mixer, cache = make(dev, 5)
    rows = S.mamba_rows_np(np.random.default_rng(6), 4)
    rd = S.to_device(rows, dev)
    M.verify_rows(mixer, rd[:3], cache)
    M.mamba_rollback([(cache, 3)], 2)
    y_next = M.verify_rows(mixer, rd[3:4], cache)
    M.mamba_rollback([(cache, 1)], 1)
    _, mixer1, c1 = make(dev, 5)
    for r in (0, 1, 3):
        y1 = M.verify_rows(mixer1, rd[r:r + 1], c1)
        M.mamba_rollback([(c1, 1)], 1)
    assert torch.equal(y1, y_next)
    assert torch.equal(c1.state()[1], cache.state()[1])


def test_greedy_accept_on_device(dev):
    V = 1000
    rng = np.random.default_rng(7)
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    for draft in itertools.product((3, 5), repeat=2):
        logits = rng.standard_normal((3, V)).astype(np.float32)
        logits[0, 3] = logits[1, 5] = 50.0           # target argmax: 3, 5, then whatever row 2 says
        logits[2, 17] = logits[2, 18] = 60.0          # a tie: the first index wins
        for dt in (torch.float32, torch.bfloat16):
            cur.zero_()
            out = mtp.greedy_accept(torch.tensor(draft, dtype=torch.int32, device=dev),
                                    torch.from_numpy(logits).to(dev).to(dt), cur=cur, nslab=4)
            tgt = O.argmax_first(torch.from_numpy(logits).to(dt).float().numpy())
            a, emitted, n_keep = O.greedy_accept(draft, tgt)
            assert out["tgt"].cpu().tolist() == tgt.tolist()
            assert int(out["n_accept"].item()) == a and int(out["n_keep"].item()) == n_keep
            assert out["tokens"].cpu().tolist()[:a + 1] == emitted
            assert int(cur.item()) == n_keep % 4
