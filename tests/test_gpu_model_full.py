"""The end-to-end workload at its real shape (hsd/model.py:366-443; the reference's own
check is tests/test_end_to_end.py:67-97): the 52-layer Nemotron-3.5-Lightning-30B-A3B
hybrid (23 Mamba-2, 23 MoE with 128 experts top-6 and the neuron-major 4-bit down
projection, 6 GQA attention; hidden 2688, vocab 131072, the one-layer MTP head),
random-init, a seeded 2048-token random prompt, then greedy decoding with the down
projection dense (the dense-h control), sparse, and sparse + MTP-2 verify and rollback.

Bar (integer outputs, bit-exact): the first NTOK greedy tokens are identical in every
mode: dense == sparse == sparse + MTP-2 with scripted acceptance at a mean of 1.26 and
1.68 accepted drafts (the true token where the script accepts, a wrong one where it
rejects), and sparse + MTP-2 with the head's own drafts. The realised acceptance follows
the script. No kernel raises the sequence's device status word.
"""
import numpy as np
import pytest
import torch

from hsd import _native as N
from hsd import model as Mdl
from hsd import mtp

pytestmark = pytest.mark.gpu
PROMPT_LEN = 2048
NTOK = 96
# the two scripted acceptance mixes of the benchmark: P(0, 1, 2 drafts accepted)
MIXES = {"mean 1.26": (0.2, 0.34, 0.46), "mean 1.68": (0.06, 0.2, 0.74)}


@pytest.fixture(scope="module")
def model(dev):
    cfg = Mdl.ModelConfig()
    assert (len(cfg.pattern), cfg.hidden, cfg.vocab, cfg.n_experts) == (52, 2688, 131072, 128)
    m = Mdl.NemotronModel(cfg, mode="sparse", seed=0, device=dev)
    print(f"full-shape model: {m.nbytes() / 1e9:.2f} GB of weights; MoE zero fractions "
          f"{min(m.zero_frac_measured):.3f}..{max(m.zero_frac_measured):.3f}", flush=True)
    yield m
    del m
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def prompt():
    return np.random.default_rng(11).integers(0, Mdl.ModelConfig().vocab, PROMPT_LEN).astype(np.int32)


@pytest.fixture(scope="module")
def dense_tokens(model, prompt):
    model.set_mode("dense")
    toks = [t for t, _ in model.generate(prompt, max_tokens=NTOK)]
    model.set_mode("sparse")
    print(f"dense tokens[:16]: {toks[:16]}", flush=True)
    return toks


def test_prompt_fills_the_caches(model, prompt):
    s = model.session(prompt, cap=4)
    st = s.state()
    assert st[N.SEQ_POS] == PROMPT_LEN and st[N.SEQ_N] == 1
    assert int(s.cache.status.item()) == 0


def test_sparse_equals_dense(model, prompt, dense_tokens):
    model.set_mode("sparse")
    assert [t for t, _ in model.generate(prompt, max_tokens=NTOK)] == dense_tokens


@pytest.mark.parametrize("mix", sorted(MIXES))
def test_mtp2_scripted_equals_dense(model, prompt, dense_tokens, mix):
    model.set_mode("sparse")
    acc = mtp.scripted_accepts(256, MIXES[mix], seed=5)
    out = list(model.generate_mtp(prompt, max_tokens=NTOK, script=dense_tokens, accepts=acc))
    toks, stats = [t for t, _ in out], out[-1][1]
    print(f"MTP-2 {mix}: {stats['spec']['steps']} steps, mean accepted {stats['spec']['accepted_mean']:.3f}, "
          f"{stats['decode_tps']:.0f} tok/s", flush=True)
    assert toks == dense_tokens
    n, i, want = 1, 0, []
    while n < NTOK:
        want.append(int(acc[i]))
        n += int(acc[i]) + 1
        i += 1
    assert stats["spec"]["steps"] == len(want)
    assert abs(stats["spec"]["accepted_mean"] - np.mean(want)) < 1e-9


def test_mtp2_own_drafts_equals_dense(model, prompt, dense_tokens):
    model.set_mode("sparse")
    out = list(model.generate_mtp(prompt, max_tokens=NTOK))
    stats = out[-1][1]
    print(f"MTP-2 own drafts: mean accepted {stats['spec']['accepted_mean']:.3f}", flush=True)
    assert [t for t, _ in out][:NTOK] == dense_tokens
