"""GPU parity of the MoE front end with the router (hsd_moe_route_up_relu2: the gate's
top-k fused into the up projection, model.py:110-121) and of the SSM-only Mamba entry
(hsd_mamba_ssm, the conv + SSM half of mamba.py:19-44 that the model feeds to out_proj).

Bars: the selected experts equal the oracle's bit for bit (rows whose k-th and (k+1)-th
choices lie within 1e-6 -- an fp32 exp rounding apart -- are reported and skipped);
gains within 1e-6 relative; hcat equal bit for bit to hsd_moe_up_relu2 given the same
experts; the written sel/gains are what the down projection reads. y_pre within
2e-2 + 1e-2 |ref| of the float64 oracle and bit-identical to hsd_mamba_verify's input to
its norm (the same kernel)."""
import numpy as np
import pytest
import torch

from hsd import mamba as M, moe, synth as S, nn
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
D, F, FS, E, K = 2688, 1856, 3712, 128, 6


@pytest.fixture(scope="module")
def up(dev):
    u = S.moe_up_np(5)
    return u, {k: S.to_device(v, dev) for k, v in u.items()}


@pytest.mark.parametrize("B", [1, 3, 6])
def test_router_topk_and_front_end(dev, up, B):
    u, ud = up
    rng = np.random.default_rng(40 + B)
    x = O.f32_to_bf16(rng.standard_normal((B, D)).astype(np.float32))
    logits = O.f32_to_bf16(rng.standard_normal((B, E)).astype(np.float32) * 2)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    xd = S.to_device(x, dev)
    hcat, sel, gains = moe.route_up_relu2(xd, S.to_device(logits, dev), torch.from_numpy(bias).to(dev),
                                          ud["w1"], ud["s1"], ud["b1"], ud["sw1"], ud["ss1"], ud["sb1"], topk=K,
                                          routed_scale=2.5, norm_topk=True)
    rsel, rg = O.router_topk(O.bf16_to_f32(logits), bias, K, scale=2.5)
    sel_h, g_h = sel.cpu().numpy(), gains.cpu().numpy()
    ch = O.sigmoid_f32(O.bf16_to_f32(logits)) + bias
    for r in range(B):
        srt = np.sort(ch[r])[::-1]
        if srt[K - 1] - srt[K] < 1e-6:
            print(f"row {r}: near tie at the k-th choice, skipped")
            continue
        assert sel_h[r].tolist() == rsel[r].tolist()
        assert np.allclose(g_h[r, :K], rg[r], rtol=1e-6, atol=0)
        assert g_h[r, K] == 1.0
    # the router alone gives the same selection and gains
    s2, g2 = moe.router_topk(S.to_device(logits, dev), torch.from_numpy(bias).to(dev), topk=K, routed_scale=2.5)
    assert torch.equal(s2, sel) and torch.equal(g2.view(torch.int32), gains.view(torch.int32))
    # the up projection with those experts is hsd_moe_up_relu2's, bit for bit
    h2 = moe.up_relu2(xd, sel, ud["w1"], ud["s1"], ud["b1"], ud["sw1"], ud["ss1"], ud["sb1"], topk=K)
    assert torch.equal(hcat.view(torch.int16), h2.view(torch.int16))
    # rows are independent of B
    if B > 1:
        h1, s1, g1 = moe.route_up_relu2(xd[1:2], S.to_device(logits[1:2], dev), torch.from_numpy(bias).to(dev),
                                        ud["w1"], ud["s1"], ud["b1"], ud["sw1"], ud["ss1"], ud["sb1"], topk=K,
                                        routed_scale=2.5)
        assert torch.equal(h1.view(torch.int16), hcat[1:2].view(torch.int16))
        assert torch.equal(s1, sel[1:2]) and torch.equal(g1.view(torch.int32), gains[1:2].view(torch.int32))


def test_router_without_bias_at_an_odd_offset(dev, up):
    """No selection bias (e_bias None: the kernels then load a word of the logits in its
    place and drop it) and logits starting at an odd element (a 2-byte aligned view)."""
    u, ud = up
    B = 3
    rng = np.random.default_rng(47)
    x = O.f32_to_bf16(rng.standard_normal((B, D)).astype(np.float32))
    logits = O.f32_to_bf16(rng.standard_normal((B, E)).astype(np.float32) * 2)
    buf = torch.zeros(B * E + 1, dtype=torch.bfloat16, device=dev)
    buf[1:] = S.to_device(logits, dev).reshape(-1)
    lv = buf[1:].view(B, E)
    assert lv.data_ptr() % 4 == 2
    hcat, sel, gains = moe.route_up_relu2(S.to_device(x, dev), lv, None, ud["w1"], ud["s1"], ud["b1"], ud["sw1"],
                                          ud["ss1"], ud["sb1"], topk=K, routed_scale=2.5, norm_topk=True)
    rsel, rg = O.router_topk(O.bf16_to_f32(logits), np.zeros(E, np.float32), K, scale=2.5)
    sel_h, g_h = sel.cpu().numpy(), gains.cpu().numpy()
    ch = O.sigmoid_f32(O.bf16_to_f32(logits))
    for r in range(B):
        srt = np.sort(ch[r])[::-1]
        if srt[K - 1] - srt[K] < 1e-6:
            print(f"row {r}: near tie at the k-th choice, skipped")
            continue
        assert sel_h[r].tolist() == rsel[r].tolist()
        assert np.allclose(g_h[r, :K], rg[r], rtol=1e-6, atol=0)
    s2, g2 = moe.router_topk(lv, None, topk=K, routed_scale=2.5)
    assert torch.equal(s2, sel) and torch.equal(g2.view(torch.int32), gains.view(torch.int32))


def test_ssm_only_entry(dev):
    p = S.mamba_params_np(9)
    mk = lambda: M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                               A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                               D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev))
    mixer = mk()
    rows = S.mamba_rows_np(np.random.default_rng(10), 3)
    rd = S.to_device(rows, dev)
    c1 = M.MambaCache(mixer, dev, conv_state=S.to_device(p["conv_state"], dev),
                      ssm_state=torch.from_numpy(p["ssm_state"]).to(dev))
    y_pre = M.ssm_rows(mixer, rd, c1)
    r = O.bf16_to_f32(rows)
    DI, CD = 4096, 6144
    ref = O.mamba_verify(r[:, DI:DI + CD], r[:, DI + CD:], r[:, :DI], O.bf16_to_f32(p["conv_w"]),
                         O.bf16_to_f32(p["conv_b"]), p["A_log"], p["dt_bias"], p["D"], O.bf16_to_f32(p["norm_w"]),
                         O.bf16_to_f32(p["conv_state"]), p["ssm_state"])
    got = y_pre.cpu().numpy()
    assert np.all(np.abs(got - ref["y_pre"]) <= 2e-2 + 1e-2 * np.abs(ref["y_pre"]))
    # the same checkpoints as the full verify
    c2 = M.MambaCache(mixer, dev, conv_state=S.to_device(p["conv_state"], dev),
                      ssm_state=torch.from_numpy(p["ssm_state"]).to(dev))
    M.verify_rows(mixer, rd, c2)
    assert torch.equal(c1.ssm.view(torch.int32), c2.ssm.view(torch.int32))
    assert torch.equal(c1.conv.view(torch.int16), c2.conv.view(torch.int16))


def test_ssm_gated_entry(dev):
    """hsd_mamba_ssm_gated: z = y * silu(gate) against the plain entry's y (same state,
    same checkpoints), the 16-channel sums of z^2 against float64 sums of the returned z,
    and the out_proj prologue that consumes them (HSD_X_GATED_Z) against the oracle's
    gated norm; a row of a 3-row call equals that row alone, bit for bit."""
    p = S.mamba_params_np(13)
    mixer = M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                          A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                          D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev))
    rows = S.mamba_rows_np(np.random.default_rng(14), 3)
    rd = S.to_device(rows, dev)
    DI = 4096
    fresh = lambda: M.MambaCache(mixer, dev, conv_state=S.to_device(p["conv_state"], dev),
                                 ssm_state=torch.from_numpy(p["ssm_state"]).to(dev))
    c1, c2 = fresh(), fresh()
    y = M.ssm_rows(mixer, rd, c1).cpu().numpy().astype(np.float64)
    zbuf = torch.full((3, DI + DI // 16 + 4), float("nan"), dtype=torch.float32, device=dev)  # strided rows
    z = M.ssm_rows(mixer, rd, c2, out=zbuf, gated=True)
    assert torch.equal(c1.ssm.view(torch.int32), c2.ssm.view(torch.int32))
    assert torch.equal(c1.conv.view(torch.int16), c2.conv.view(torch.int16))
    zh = z.cpu().numpy().astype(np.float64)
    g = O.bf16_to_f32(rows[:, :DI]).astype(np.float64)
    zref = y * O.silu(g)
    assert np.all(np.abs(zh - zref) <= 1e-5 * np.abs(zref) + 1e-6 * np.abs(y))
    part = zbuf[:, DI:DI + DI // 16].cpu().numpy().astype(np.float64)
    pref = (zh * zh).reshape(3, DI // 16, 16).sum(-1)
    assert np.all(np.abs(part - pref) <= 1e-5 * pref + 1e-30)
    assert torch.isnan(zbuf[:, DI + DI // 16:]).all()          # nothing past the partials
    # the consumer: out_proj's gated norm from z and the partials
    I, O_ = DI, 2688
    rng = np.random.default_rng(15)
    w, s, b = S.down_proj_np(rng, (), O_, I)
    W = nn.QWeight(S.to_device(w, dev), S.to_device(s, dev), S.to_device(b, dev))
    nw = O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32))
    res = torch.zeros((3, O_), dtype=torch.bfloat16, device=dev)
    xn = torch.empty((3, I), dtype=torch.bfloat16, device=dev)
    out = nn.linear(z, W, norm=S.to_device(nw, dev), gated_z=True, residual=res, xn_out=xn)
    xn_h = S.to_host(xn)
    want = O.gated_rms_norm_bf16(y, g, O.bf16_to_f32(nw), 1e-5)
    a, bb = xn_h.astype(np.int32), want.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    sb = np.where(bb & 0x8000, -(bb & 0x7FFF), bb & 0x7FFF)
    print(f"gated_z norm: identical {np.mean(a == bb):.4f}")
    assert np.all(np.abs(sa - sb) <= 1) and np.mean(a == bb) >= 0.99
    ref = O.linear_q4(O.bf16_to_f32(xn_h), w, s, b)
    assert np.all(np.abs(out.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))
    for r in range(3):
        res1 = torch.zeros((1, O_), dtype=torch.bfloat16, device=dev)
        o1 = nn.linear(z[r:r + 1], W, norm=S.to_device(nw, dev), gated_z=True, residual=res1)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), f"row {r}"


def test_corrupt_ring_index_is_reported(dev):
    p = S.mamba_params_np(11)
    mixer = M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                          A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                          D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev))
    cache = M.MambaCache(mixer, dev)
    cache.cur.fill_(7)                                       # outside [0, nslab)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    before = cache.ssm.clone()
    y = M.verify_rows(mixer, S.to_device(S.mamba_rows_np(np.random.default_rng(12), 2), dev), cache, status=status)
    assert int(status.item()) == 2
    assert torch.isnan(y.float()).all()
    assert torch.equal(cache.ssm, before)
    # the gated entry: z and its partial sums NaN, the same status bit
    st1 = torch.zeros(1, dtype=torch.int32, device=dev)
    zbuf = torch.zeros((2, 4096 + 256), dtype=torch.float32, device=dev)
    M.ssm_rows(mixer, S.to_device(S.mamba_rows_np(np.random.default_rng(12), 2), dev), cache, out=zbuf,
               gated=True, status=st1)
    assert int(st1.item()) == 2 and torch.isnan(zbuf).all()
    assert torch.equal(cache.ssm, before)
    # a device n_keep beyond the verify's rows leaves the ring where it is
    cache.cur.zero_()
    st2 = torch.zeros(1, dtype=torch.int32, device=dev)
    M.mamba_rollback([(cache, 2)], 0, n_keep_dev=torch.tensor([3], dtype=torch.int32, device=dev), status=st2)
    assert int(cache.cur.item()) == 0 and int(st2.item()) == 2
