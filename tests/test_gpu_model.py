"""The whole decode loop on the GPU (hsd/model.py:291-443): a reduced random-init
Nemotron-H hybrid ("MEM*EME", hidden 512, 16 experts, vocab 4096, the MTP head) run with
the MoE down projection dense, sparse, and sparse + MTP-2 verify and rollback.

Bars (bit-exact integer outputs):
* greedy tokens identical for dense, sparse, sparse + MTP-2 with scripted acceptance
  (the true token where the mask accepts, a wrong one where it rejects), and sparse +
  MTP-2 with the head's own drafts (speculative decoding is exact whatever it drafts);
* replayed graphs equal eager steps;
* verify_step(3) then rollback(n_keep) then single steps leaves every cache and the
  hidden state bit-identical to single steps only.
"""
import numpy as np
import pytest
import torch

from hsd import _native as N
from hsd import model as Mdl
from hsd import mtp

pytestmark = pytest.mark.gpu
CFG = Mdl.ModelConfig(hidden=512, pattern="MEM*EME", vocab=4096, n_experts=16, topk=6, moe_inter=256,
                      shared_inter=512, max_seq=256, mtp=True)
PROMPT = np.random.default_rng(0).integers(0, CFG.vocab, 20).astype(np.int32)
NTOK = 24


@pytest.fixture(scope="module")
def model(dev):
    m = Mdl.NemotronModel(CFG, mode="sparse", seed=3, device=dev)
    print(f"measured zero fractions per MoE block: {[round(z, 3) for z in m.zero_frac_measured]}", flush=True)
    return m


def tokens(gen):
    out = [t for t, _ in gen]
    return out


@pytest.fixture(scope="module")
def dense_tokens(model):
    model.set_mode("dense")
    t = tokens(model.generate(PROMPT, max_tokens=NTOK))
    model.set_mode("sparse")
    print(f"dense tokens: {t}", flush=True)
    return t


def test_sparsity_is_calibrated(model):
    z = np.array(model.zero_frac_measured)
    assert np.all((z > 0.8) & (z < 0.97)), z


def test_sparse_equals_dense(model, dense_tokens):
    assert tokens(model.generate(PROMPT, max_tokens=NTOK)) == dense_tokens


def test_graph_equals_eager(model, dense_tokens):
    assert tokens(model.generate(PROMPT, max_tokens=NTOK, graph=False)) == dense_tokens


@pytest.mark.parametrize("probs", [(0.2, 0.34, 0.46), (0.06, 0.2, 0.74), (1.0, 0.0, 0.0), (0.0, 0.0, 1.0)])
def test_mtp_scripted_equals_dense(model, dense_tokens, probs):
    acc = mtp.scripted_accepts(64, probs, seed=5)
    out = list(model.generate_mtp(PROMPT, max_tokens=NTOK, script=dense_tokens, accepts=acc))
    toks = [t for t, _ in out]
    stats = out[-1][1]
    print(f"accepts {probs}: steps {stats['spec']['steps']}, mean accepted {stats['spec']['accepted_mean']:.2f}")
    assert toks == dense_tokens
    # the realised acceptance follows the script exactly
    n, i, want = 1, 0, []
    while n < NTOK:
        want.append(int(acc[i]))
        n += int(acc[i]) + 1
        i += 1
    assert stats["spec"]["steps"] == len(want)
    assert abs(stats["spec"]["accepted_mean"] - np.mean(want)) < 1e-9


def test_mtp_own_drafts_equals_dense(model, dense_tokens):
    out = list(model.generate_mtp(PROMPT, max_tokens=NTOK))
    assert [t for t, _ in out] == dense_tokens
    out_e = list(model.generate_mtp(PROMPT, max_tokens=NTOK, graph=False))
    assert [t for t, _ in out_e] == dense_tokens


def snapshot(cache):
    parts = [cache.seq.clone()]
    for lc in cache.layers:
        if lc is None:
            continue
        if hasattr(lc, "ssm"):
            c = int(cache.cur.item())
            parts += [lc.ssm[c].clone(), lc.conv[c].clone()]
        else:
            n = int(cache.pos.item())
            parts += [lc.k[:, :n].clone(), lc.v[:, :n].clone()]
    return parts


def test_verify_rollback_equals_single_steps(model):
    dev = model.device
    ids = torch.from_numpy(np.array([5, 77, 901, 4000], dtype=np.int32)).to(dev)
    for n_keep in (1, 2, 3):
        a = model.make_cache(cap=8)
        b = model.make_cache(cap=8)
        model.prefill(PROMPT, a, with_head=False, graph=False)
        model.prefill(PROMPT, b, with_head=False, graph=False)
        # a: verify 3 rows, roll back to n_keep, then single steps for the rest
        xa = model.verify_step(model.embed(ids[:3]), a).clone()
        model.rollback(a, n_keep, 3)
        for r in range(n_keep, 4):
            xa_r = model.step(model.embed(ids[r:r + 1]).clone(), a)
            N.call("hsd_seq_add", N.ptr(a.seq), N.SEQ_POS, 1, N.stream(dev))
            N.call("hsd_mamba_select_row", N.ptr(a.cur), None, 1, 1, Mdl.NSLAB, None, N.stream(dev))
        # b: single steps only
        xb = []
        for r in range(4):
            xb.append(model.step(model.embed(ids[r:r + 1]).clone(), b).clone())
            N.call("hsd_seq_add", N.ptr(b.seq), N.SEQ_POS, 1, N.stream(dev))
            N.call("hsd_mamba_select_row", N.ptr(b.cur), None, 1, 1, Mdl.NSLAB, None, N.stream(dev))
        torch.cuda.synchronize(dev)
        for r in range(n_keep):
            assert torch.equal(xa[r:r + 1].view(torch.int16), xb[r].view(torch.int16)), f"verify row {r}"
        assert torch.equal(xa_r.view(torch.int16), xb[3].view(torch.int16))
        sa, sb = snapshot(a), snapshot(b)
        assert len(sa) == len(sb)
        for u, v in zip(sa, sb):
            assert torch.equal(u.view(torch.uint8), v.view(torch.uint8))
