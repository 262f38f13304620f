"""GPU parity of the per-block call surfaces: hsd.mamba.mamba_verify on a whole Mamba-2
block (mamba.py:19-44: pre-norm, in_proj, conv + SSM, gated norm, out_proj, residual)
with mamba_rollback, and the MoE block's decode_sparse / decode_dense / prefill_sparse
(model.py:110-175), on a reduced random-init block (hidden 512, 16 experts, F 256,
FS 512; the Mamba mixer at its real 64 x 64 x 128, 8 groups).

Bars:
* each row within the bf16 bound |x - ref| <= 2e-2 + 1e-2 |ref| of the oracle's block
  step (float64 sums, bf16 activations between the ops), the state after every row
  (conv state bf16, ssm state f32) within 2e-2 + 1e-2 |ref|;
* bit-exact: a verify of L rows == L single-row verifies (outputs and checkpoints);
  rollback to n_keep == the state after n_keep single rows; decode_sparse ==
  decode_dense; decode_sparse rows independent of B;
* prefill_sparse (the MFMA grouped GEMM, another summation order) within the bf16
  bound of decode_sparse and of the oracle.
"""
import numpy as np
import pytest
import torch

from hsd import mamba as M
from hsd import model as Mdl
from hsd import synth as S
from oracle import hsd_oracle as O

from . import hostw

pytestmark = pytest.mark.gpu
CFG = Mdl.ModelConfig(hidden=512, pattern="ME", vocab=4096, n_experts=16, topk=6, moe_inter=256, shared_inter=512,
                      max_seq=256, mtp=False)


def close(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= 2e-2 + 1e-2 * np.abs(ref))


@pytest.fixture(scope="module")
def blocks(dev):
    init = Mdl._Init(21, dev)
    mb = Mdl.MambaBlock(CFG, init)
    eb = Mdl.MoEBlock(CFG, init)
    eb.norm_w[0] = 0.3                       # a moderate bias-channel offset: some zeros, some live
    return mb, eb


def rand_rows(seed, L, dev, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((L, CFG.hidden)) * scale).astype(np.float32)
    x[:, 0] = 1.875                           # the bias channel the embedding sets
    bits = O.f32_to_bf16(x)
    return bits, S.to_device(bits, dev)


def start_state(seed, mixer, dev):
    rng = np.random.default_rng(seed)
    conv = O.f32_to_bf16((rng.standard_normal((3, mixer.conv_dim)) * 0.5).astype(np.float32))
    ssm = (rng.standard_normal((mixer.num_heads, mixer.head_dim, mixer.ssm_state_size)) * 0.1).astype(np.float32)
    return conv, ssm


def fresh_cache(mixer, dev, conv, ssm):
    return M.MambaCache(mixer, dev, nslab=4, conv_state=S.to_device(conv, dev),
                        ssm_state=torch.from_numpy(ssm).to(dev))


def test_mamba_verify_block_matches_oracle(blocks, dev):
    mb, _ = blocks
    conv, ssm = start_state(30, mb.mixer, dev)
    xb, xd = rand_rows(31, 3, dev)
    cache = fresh_cache(mb.mixer, dev, conv, ssm)
    records = []
    out = M.mamba_verify(mb, xd[None], cache, records)
    assert out.shape == (1, 3, CFG.hidden) and records == [(cache, 3)]
    got = out[0].float().cpu().numpy()
    w = hostw.mamba_block(mb)
    cs, ss, states = O.bf16_to_f32(conv), ssm, []
    for r in range(3):
        xr, cs, ss = O.mamba_block_step(xb[r], w, cs, ss, n_groups=CFG.n_groups, eps=CFG.eps)
        states.append((cs, ss))
        ref = O.bf16_to_f32(xr)
        d, dr = got[r] - O.bf16_to_f32(xb[r]), ref - O.bf16_to_f32(xb[r])
        err = np.abs(d - dr).max()
        print(f"row {r}: max |update - ref| {err:.3e} (max |update| {np.abs(dr).max():.3f})")
        assert close(got[r], ref)
        assert err <= 3e-2 * np.abs(dr).max()          # the block's own contribution, not hidden by x
    # roll back to each n_keep: the state after that many rows
    for n_keep in (1, 2, 3):
        c2 = fresh_cache(mb.mixer, dev, conv, ssm)
        rec = []
        M.mamba_verify(mb, xd[None], c2, rec)
        M.mamba_rollback(rec, n_keep)
        cv, sv = c2.state()
        assert close(cv.float().cpu().numpy(), states[n_keep - 1][0])
        assert close(sv.cpu().numpy(), states[n_keep - 1][1])


def test_mamba_verify_rows_equal_single_rows(blocks, dev):
    mb, _ = blocks
    conv, ssm = start_state(32, mb.mixer, dev)
    _, xd = rand_rows(33, 3, dev)
    ca = fresh_cache(mb.mixer, dev, conv, ssm)
    ra = []
    ya = M.mamba_verify(mb, xd[None], ca, ra)
    M.mamba_rollback(ra, 2)
    cb = fresh_cache(mb.mixer, dev, conv, ssm)
    for r in range(2):
        rb = []
        yb = M.mamba_verify(mb, xd[None, r:r + 1], cb, rb)
        M.mamba_rollback(rb, 1)
        assert torch.equal(ya[0, r].view(torch.int16), yb[0, 0].view(torch.int16))
    for u, v in zip(ca.state(), cb.state()):
        assert torch.equal(u.contiguous().view(torch.uint8), v.contiguous().view(torch.uint8))
    # the bare mixer form is the kernel-level verify: in_proj output in, gated-norm output out
    proj = torch.randn((2, CFG.in_proj_dim), device=dev).to(torch.bfloat16)
    cm = fresh_cache(mb.mixer, dev, conv, ssm)
    y = M.mamba_verify(mb.mixer, proj[None], cm, [])
    assert y.shape == (1, 2, CFG.mamba_inner)


@pytest.mark.parametrize("B", [1, 3])
def test_moe_decode_sparse_matches_oracle(blocks, dev, B):
    _, eb = blocks
    xb, xd = rand_rows(40 + B, B, dev)
    y = eb.decode_sparse(xd)
    assert torch.equal(xd.view(torch.int16), S.to_device(xb, dev).view(torch.int16))   # x not written
    yd = eb.decode_dense(xd)
    assert torch.equal(y.view(torch.int16), yd.view(torch.int16))
    w = hostw.moe_block(eb)
    got = y.float().cpu().numpy()
    for r in range(B):
        ref = O.bf16_to_f32(O.moe_block_step(xb[r], w, topk=CFG.topk, routed_scale=CFG.routed_scale, eps=CFG.eps))
        d = got[r] - O.bf16_to_f32(xb[r])
        dr = ref - O.bf16_to_f32(xb[r])
        print(f"B={B} row {r}: max |moe - ref| {np.abs(d - dr).max():.3e} (max |moe| {np.abs(dr).max():.3f})")
        assert close(got[r], ref)
        assert np.abs(d - dr).max() <= 3e-2 * np.abs(dr).max()
        if B > 1:
            y1 = eb.decode_sparse(xd[r:r + 1])
            assert torch.equal(y1[0].view(torch.int16), y[r].view(torch.int16))
    # the front end's pieces repack into the same result
    inds, scores, h, hs = eb.front(xd)
    hcat, sel, gains = eb.pack(inds, scores, h, hs)
    assert hcat.shape == (B, CFG.topk * CFG.moe_inter + CFG.shared_inter) and torch.all(gains[:, -1] == 1)
    frac = float((hcat == 0).float().mean().item())
    print(f"zero fraction of hcat: {frac:.3f}")
    assert 0.05 < frac < 0.995


def test_moe_prefill_sparse(blocks, dev):
    _, eb = blocks
    T = 40
    xb, xd = rand_rows(50, T, dev)
    yp = eb.prefill_sparse(xd)
    yd = eb.decode_sparse(xd)
    gp, gd = yp.float().cpu().numpy(), yd.float().cpu().numpy()
    assert close(gp, gd)
    w = hostw.moe_block(eb)
    for r in (0, 17, T - 1):
        ref = O.bf16_to_f32(O.moe_block_step(xb[r], w, topk=CFG.topk, routed_scale=CFG.routed_scale, eps=CFG.eps))
        assert close(gp[r], ref)
    assert torch.equal(eb.prefill(xd, mode="dense").view(torch.int16), yd.view(torch.int16))
