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


def host_weights(model):
    """The reduced model's weights as host arrays in the oracle's conventions."""
    from hsd import synth as S
    u32 = lambda t: S.to_host(t).view(np.uint32)
    out = []
    for t, blk in zip(model.cfg.pattern, model.blocks):
        if t == "M":
            m = blk.mixer
            out.append(dict(norm_w=S.to_host(blk.norm_w), in_w=u32(blk.in_proj.w), in_s=S.to_host(blk.in_proj.scales),
                            in_b=S.to_host(blk.in_proj.biases), out_w=u32(blk.out_proj.w),
                            out_s=S.to_host(blk.out_proj.scales), out_b=S.to_host(blk.out_proj.biases),
                            conv_w=m.conv_w.float().cpu().numpy(), conv_b=m.conv_b.float().cpu().numpy(),
                            A_log=m.A_log.cpu().numpy(), dt_bias=m.dt_bias.cpu().numpy(), D=m.D.cpu().numpy(),
                            gnorm_w=S.to_host(m.norm_w)))
        elif t == "*":
            out.append(dict(norm_w=S.to_host(blk.norm_w), qkv_w=u32(blk.qkv.w), qkv_s=S.to_host(blk.qkv.scales),
                            qkv_b=S.to_host(blk.qkv.biases), o_w=u32(blk.o_proj.w), o_s=S.to_host(blk.o_proj.scales),
                            o_b=S.to_host(blk.o_proj.biases)))
        else:
            out.append(dict(norm_w=S.to_host(blk.norm_w), gate=S.to_host(blk.gate.w), e_bias=blk.e_bias.cpu().numpy(),
                            w1=u32(blk.w1), s1=S.to_host(blk.s1), b1=S.to_host(blk.b1), sw1=u32(blk.sw1),
                            ss1=S.to_host(blk.ss1), sb1=S.to_host(blk.sb1), pw=u32(blk.pw), ps=S.to_host(blk.ps),
                            pb=S.to_host(blk.pb), spw=u32(blk.spw), sps=S.to_host(blk.sps), spb=S.to_host(blk.spb)))
    return out


def test_decode_step_matches_oracle(model):
    """One decode step of the whole reduced model against the oracle's composition of the
    blocks (float64 sums, bf16 activations between ops), from the GPU's caches after the
    prompt: the final hidden row and the logits within 3e-2 of their scale, and the same
    greedy token unless the top two logits are closer than that."""
    from hsd import synth as S
    from oracle import hsd_oracle as O
    c = model.cfg
    model.set_mode("sparse")
    cache = model.make_cache(cap=8)
    x_last = model.prefill(PROMPT, cache, with_head=False, graph=False)
    model._first_token(x_last, cache)
    torch.cuda.synchronize()
    seq = cache.state()
    tok0, P, cur = seq[N.SEQ_TOK], seq[N.SEQ_POS], seq[N.SEQ_CUR]
    states = []
    for t, lc in zip(c.pattern, cache.layers):
        if t == "M":
            states.append((lc.conv[cur].float().cpu().numpy(), lc.ssm[cur].cpu().numpy()))
        elif t == "*":
            states.append((lc.k[:, :P].float().cpu().numpy(), lc.v[:, :P].float().cpu().numpy()))
        else:
            states.append(None)
    model._decode_step(cache)
    buf = model._bufs[1]
    x_gpu = buf["x"].float().cpu().numpy()[0]
    logits_gpu = model.logits(buf["x"]).float().cpu().numpy()[0]
    torch.cuda.synchronize()
    # the oracle from the same token and states
    E = model.embedding
    x = O.embed_q4(np.array([tok0]), S.to_host(E.w).view(np.uint32), S.to_host(E.scales), S.to_host(E.biases))[0]
    for t, w, st in zip(c.pattern, host_weights(model), states):
        if t == "M":
            x, _, _ = O.mamba_block_step(x, w, st[0], st[1], n_groups=c.n_groups, eps=c.eps)
        elif t == "*":
            x, _, _ = O.attn_block_step(x, w, st[0], st[1], n_heads=c.attn_heads, n_kv_heads=c.kv_heads, eps=c.eps)
        else:
            x = O.moe_block_step(x, w, topk=c.topk, routed_scale=c.routed_scale, eps=c.eps)
    x_ref = O.bf16_to_f32(x)
    lg = O.lm_head_logits(x, S.to_host(model.norm_f), S.to_host(model.lm_head.w).view(np.uint32),
                          S.to_host(model.lm_head.scales), S.to_host(model.lm_head.biases), c.eps)
    ex = np.abs(x_gpu - x_ref).max() / np.abs(x_ref).max()
    el = np.abs(logits_gpu - lg).max() / np.abs(lg).max()
    print(f"decode step vs oracle: hidden max rel err {ex:.2e}, logits {el:.2e}")
    assert ex <= 3e-2 and el <= 3e-2
    top = np.sort(lg)[::-1]
    if top[0] - top[1] > 6e-2 * np.abs(lg).max():
        assert int(np.argmax(logits_gpu)) == int(np.argmax(lg))
