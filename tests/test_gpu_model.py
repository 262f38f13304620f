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

from . import hostw

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
    for t, w, st in zip(c.pattern, hostw.model_blocks(model), states):
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


def test_mtp_head_call_surface(model):
    """hsd.mtp.MTPHead (mtp.py:41-88): rows in chunks equal single rows bit for bit,
    trim drops rows, reset empties the cache; the first row against the oracle's head
    (pair norm, eh_proj, attention over itself, MoE, final norm, lm_head)."""
    from hsd import synth as S
    from oracle import hsd_oracle as O
    dev = model.device
    c = model.cfg
    rng = np.random.default_rng(77)
    hb = O.f32_to_bf16(rng.standard_normal((5, c.hidden)).astype(np.float32))
    h = S.to_device(hb, dev)
    toks = torch.from_numpy(rng.integers(0, c.vocab, 5).astype(np.int32)).to(dev)
    head = mtp.MTPHead(model)
    pred, hn = head(h, toks)
    assert head.rows == 5
    single = mtp.MTPHead(model)
    for r in range(5):
        p1, h1 = single(h[r:r + 1], toks[r:r + 1])
        assert int(p1[0]) == int(pred[r])
        assert torch.equal(h1[0].view(torch.int16), hn[r].view(torch.int16))
    head.trim(2)
    p2, h2 = head(h[3:5], toks[3:5])
    assert torch.equal(p2, pred[3:5]) and torch.equal(h2.view(torch.int16), hn[3:5].view(torch.int16))
    head.reset()
    p3, h3 = head(h[:1], toks[:1])
    assert int(p3[0]) == int(pred[0])
    # the oracle's head on row 0 (an empty cache: attention over the row itself)
    hd = model.mtp
    E = model.embedding
    e = O.embed_q4(np.array([int(toks[0])]), S.to_host(E.w).view(np.uint32), S.to_host(E.scales),
                   S.to_host(E.biases))[0]
    pair = np.concatenate([O.rms_norm_bf16(O._vals(e), O._vals(S.to_host(hd.enorm)), c.eps),
                           O.rms_norm_bf16(O._vals(hb[0]), O._vals(S.to_host(hd.hnorm)), c.eps)])
    x = O.f32_to_bf16(O.linear_bf16(O._vals(pair)[None], S.to_host(hd.eh_proj.w))[0].astype(np.float32))
    HKV, HD = c.kv_heads, c.head_dim
    x, _, _ = O.attn_block_step(x, hostw.attn_block(hd.attn), np.zeros((HKV, 0, HD)), np.zeros((HKV, 0, HD)),
                                n_heads=c.attn_heads, n_kv_heads=HKV, eps=c.eps)
    x = O.moe_block_step(x, hostw.moe_block(hd.moe), topk=c.topk, routed_scale=c.routed_scale, eps=c.eps)
    hn_ref = O.bf16_to_f32(O.rms_norm_bf16(O._vals(x), O._vals(S.to_host(hd.final_norm)), c.eps))
    got = hn[0].float().cpu().numpy()
    err = np.abs(got - hn_ref).max() / np.abs(hn_ref).max()
    print(f"MTP head row 0 vs oracle: hn max rel err {err:.2e}")
    assert err <= 3e-2
    lg = O.lm_head_logits(x, S.to_host(hd.final_norm), S.to_host(model.lm_head.w).view(np.uint32),
                          S.to_host(model.lm_head.scales), S.to_host(model.lm_head.biases), c.eps)
    top = np.sort(lg)[::-1]
    if top[0] - top[1] > 6e-2 * np.abs(lg).max():
        assert int(pred[0]) == int(np.argmax(lg))


def test_cache_bounds_are_checked(model):
    """A prompt plus generation that would pass the attention caches' max_seq rows is
    refused on the host before any kernel runs, and a step that would pass them is
    refused before it is launched; a kernel's flag in the cache's status word raises."""
    c = model.cfg
    with pytest.raises(N.HSDError, match="max_seq"):
        model.session(np.zeros(c.max_seq - 4, np.int32), cap=8)
    with pytest.raises(N.HSDError, match="max_seq"):
        # 3-row prefill steps: a max_seq-token prompt's last step would write 2 rows past it
        model.prefill(np.zeros(c.max_seq, np.int32), model.make_cache(cap=4), graph=False)
    s = model.session(PROMPT, cap=8)
    with pytest.raises(N.HSDError, match="attention cache"):
        s.step(c.max_seq)
    s.step(2)
    assert s.emitted() == 3
    s.cache.status.fill_(N.STATUS_BAD_STATE)
    with pytest.raises(N.HSDError, match="overflow"):
        s.cache.check_status("test")
