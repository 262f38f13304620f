"""GPU parity of hsd_linear -- the projections of a decode step (mlx quantized_matmul with
transpose=True: Mamba in/out_proj, attention q/k/v/o, lm_head; bf16 router gate and MTP
eh_proj) with the fused rms_norm / gated-norm prologues and the residual / argmax
epilogues.

Bars:
* the fused norms (xn_out) equal the oracle's bf16 within one bf16 ulp, and at least
  99 % of the elements are bit-identical;
* y against the float64 oracle applied to the kernel's own xn: max|y - ref| <= 1e-4 *
  max|ref| (fp32 accumulation over up to 6144 inputs); bf16 outputs within the north-star
  bound |y - ref| <= 2e-2 + 1e-2 |ref|;
* bit-exact: every row of a B-row call equals that row alone; the bf16, residual and
  argmax epilogues equal bf16(f32 output), bf16(res + bf16(y)) and the first argmax of
  the bf16 outputs.
"""
import numpy as np
import pytest
import torch

from hsd import _native as N, nn, synth as S
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu


def q4_weight(seed, O_, I, dev, scale=None):
    rng = np.random.default_rng(seed)
    w, s, b = S.down_proj_np(rng, (), O_, I)
    if scale is not None:
        s = O.f32_to_bf16(O.bf16_to_f32(s) * scale)
        b = O.f32_to_bf16(O.bf16_to_f32(b) * scale)
    return (w, s, b), nn.QWeight(S.to_device(w, dev), S.to_device(s, dev), S.to_device(b, dev))


def bf16_rows(rng, B, I, dev, scale=1.0):
    x = O.f32_to_bf16(rng.standard_normal((B, I)).astype(np.float32) * scale)
    return x, S.to_device(x, dev)


def ulp_close(a_bits, b_bits):
    """Element-wise |a - b| <= 1 bf16 ulp, and the fraction of bit-identical elements."""
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.all(np.abs(sa - sb) <= 1), float(np.mean(a == b))


@pytest.mark.parametrize("I,O_", [(2688, 2688), (4096, 1024), (3584, 512), (2688, 10304), (2688, 20480), (4096, 16384),
                                  (1024, 96)])
def test_rms_linear_matches_oracle(dev, I, O_):
    """(2688, 20480) and (4096, 16384): more 16-row blocks than resident workgroups, so a
    workgroup runs several blocks in turn; (1024, 96): 32 pieces a row, one pass."""
    (w, s, b), W = q4_weight(10 + I, O_, I, dev)
    rng = np.random.default_rng(20)
    nw = O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32))
    x, xd = bf16_rows(rng, 3, I, dev, 2.0)
    xn = torch.empty((3, I), dtype=torch.bfloat16, device=dev)
    y = nn.linear(xd, W, norm=S.to_device(nw, dev), eps=1e-5, out_dtype=torch.float32, xn_out=xn)
    xn_h = S.to_host(xn)
    ok, same = ulp_close(xn_h, O.rms_norm_bf16(O.bf16_to_f32(x), O.bf16_to_f32(nw), 1e-5))
    print(f"I={I} O={O_}: xn within 1 ulp {ok}, identical {same:.4f}")
    assert ok and same >= 0.99
    ref = O.linear_q4(O.bf16_to_f32(xn_h), w, s, b)
    yh = y.cpu().numpy()
    scale = np.abs(ref).max()
    print(f"  max rel err {np.abs(yh - ref).max() / scale:.2e}")
    assert np.abs(yh - ref).max() <= 1e-4 * scale


def test_rows_are_independent_and_epilogues_agree(dev):
    I, O_ = 2688, 4608
    (w, s, b), W = q4_weight(31, O_, I, dev)
    rng = np.random.default_rng(32)
    nw = S.to_device(O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32)), dev)
    _, xd = bf16_rows(rng, 4, I, dev)
    y4 = nn.linear(xd, W, norm=nw, out_dtype=torch.float32)
    for r in range(4):
        y1 = nn.linear(xd[r:r + 1], W, norm=nw, out_dtype=torch.float32)
        assert torch.equal(y1.view(torch.int32), y4[r:r + 1].view(torch.int32)), f"row {r}"
    y3 = nn.linear(xd[:3], W, norm=nw, out_dtype=torch.float32)
    assert torch.equal(y3.view(torch.int32), y4[:3].view(torch.int32))
    yb = nn.linear(xd, W, norm=nw)                                      # bf16 epilogue
    assert torch.equal(yb.view(torch.int16), y4.to(torch.bfloat16).view(torch.int16))
    for r in range(4):                      # one row: 2 rows per wavefront; four rows: 4
        y1b = nn.linear(xd[r:r + 1], W, norm=nw)
        assert torch.equal(y1b.view(torch.int16), yb[r:r + 1].view(torch.int16)), f"row {r}"
    # argmax epilogue: the first index of the largest bf16 output, per row
    slots = nn.argmax_slots(O_)
    keys = torch.empty((4, slots), dtype=torch.int64, device=dev)
    logits = torch.empty((4, O_), dtype=torch.bfloat16, device=dev)
    nn.linear(xd, W, norm=nw, argmax_keys=keys, out=logits)
    tok = nn.argmax(keys).cpu().numpy()
    assert torch.equal(logits.view(torch.int16), yb.view(torch.int16))
    assert tok.tolist() == O.argmax_bf16(yb.float().cpu().numpy()).tolist()


@pytest.mark.parametrize("I", [2688, 4096])
def test_many_blocks_matrix_core_path(dev, I):
    """O past 2048 blocks of 16 rows takes the MFMA kernel (lm_head's path): the oracle on
    the first and last 1024 rows, rows independent of B, and the bf16 / residual / argmax
    epilogues against the f32 output."""
    O_ = 33024
    (w, s, b), W = q4_weight(61 + I, O_, I, dev)
    rng = np.random.default_rng(62)
    nw = O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32))
    nwd = S.to_device(nw, dev)
    x, xd = bf16_rows(rng, 3, I, dev, 2.0)
    xn = torch.empty((3, I), dtype=torch.bfloat16, device=dev)
    y3 = nn.linear(xd, W, norm=nwd, out_dtype=torch.float32, xn_out=xn)
    xn_h = S.to_host(xn)
    yh = y3.cpu().numpy()
    for rows in (slice(0, 1024), slice(O_ - 1024, O_)):
        ref = O.linear_q4(O.bf16_to_f32(xn_h), w[rows], s[rows], b[rows])
        assert np.abs(yh[:, rows] - ref).max() <= 1e-4 * np.abs(ref).max()
    for r in range(3):
        y1 = nn.linear(xd[r:r + 1], W, norm=nwd, out_dtype=torch.float32)
        assert torch.equal(y1.view(torch.int32), y3[r:r + 1].view(torch.int32)), f"row {r}"
    yb = nn.linear(xd, W, norm=nwd)
    assert torch.equal(yb.view(torch.int16), y3.to(torch.bfloat16).view(torch.int16))
    keys = torch.empty((3, nn.argmax_slots(O_)), dtype=torch.int64, device=dev)
    nn.linear(xd, W, norm=nwd, argmax_keys=keys)
    assert nn.argmax(keys).cpu().numpy().tolist() == O.argmax_bf16(yb.float().cpu().numpy()).tolist()
    res = S.to_device(O.f32_to_bf16(rng.standard_normal((3, O_)).astype(np.float32)), dev)
    yp = nn.linear(xd, W)
    out = res.clone()
    nn.linear(xd, W, residual=out, out=out)
    assert torch.equal(out.view(torch.int16), (res.float() + yp.float()).to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("I,O_", [(2688, 131072), (2688, 33024), (1024, 40960)])
def test_one_row_argmax_ring(dev, I, O_):
    """One or three token rows of argmax keys with no logits (the decode and verify steps'
    lm_head) take the LDS-ring kernel: each row's token equals the first argmax of the same
    row's bf16 logits from the register kernel (and of the oracle's), alone and among three
    rows; equal logits give the smallest index; a NaN logit wins; every key slot is
    written; xn_out equals the three-row call's."""
    (w, s, b), W = q4_weight(71 + O_, O_, I, dev)
    rng = np.random.default_rng(72)
    nwd = S.to_device(O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32)), dev)
    x, xd = bf16_rows(rng, 3, I, dev, 2.0)
    slots = nn.argmax_slots(O_)
    xn3 = torch.empty((3, I), dtype=torch.bfloat16, device=dev)
    y3 = nn.linear(xd, W, norm=nwd, xn_out=xn3)                      # bf16 logits, 3 rows
    keys3 = torch.full((3, slots), -1, dtype=torch.int64, device=dev)
    nn.linear(xd, W, norm=nwd, argmax_keys=keys3)
    assert int((keys3 == -1).sum().item()) == 0
    tok3 = nn.argmax(keys3).cpu().numpy().tolist()
    want = O.argmax_bf16(y3.float().cpu().numpy()).tolist()
    assert tok3 == want
    for r in range(3):
        keys = torch.full((1, slots), -1, dtype=torch.int64, device=dev)
        xn1 = torch.empty((1, I), dtype=torch.bfloat16, device=dev)
        nn.linear(xd[r:r + 1], W, norm=nwd, argmax_keys=keys, xn_out=xn1)
        assert int(nn.argmax(keys).item()) == want[r], f"row {r}"
        assert torch.equal(xn1.view(torch.int16), xn3[r:r + 1].view(torch.int16))
        assert int((keys == -1).sum().item()) == 0                  # every slot written
    rows = slice(O_ - 1024, O_)
    ref = O.linear_q4(O.bf16_to_f32(S.to_host(xn3)), w[rows], s[rows], b[rows])
    assert np.abs(y3[:, rows].float().cpu().numpy() - ref).max() <= 2e-2 + 1e-2 * np.abs(ref).max()
    # equal rows: the first index wins; a NaN scale in one row: that row wins
    wt, st, bt = (np.broadcast_to(a[5:6], a.shape).copy() for a in (w, s, b))
    Wt = nn.QWeight(S.to_device(wt, dev), S.to_device(st, dev), S.to_device(bt, dev))
    keys = torch.empty((1, slots), dtype=torch.int64, device=dev)
    nn.linear(xd[:1], Wt, norm=nwd, argmax_keys=keys)
    assert int(nn.argmax(keys).item()) == 0
    nn.linear(xd, Wt, norm=nwd, argmax_keys=keys3)
    assert nn.argmax(keys3).cpu().numpy().tolist() == [0, 0, 0]
    st[O_ - 3, 1] = 0x7FC0
    Wt = nn.QWeight(S.to_device(wt, dev), S.to_device(st, dev), S.to_device(bt, dev))
    nn.linear(xd[:1], Wt, norm=nwd, argmax_keys=keys)
    assert int(nn.argmax(keys).item()) == O_ - 3
    nn.linear(xd, Wt, norm=nwd, argmax_keys=keys3)
    assert nn.argmax(keys3).cpu().numpy().tolist() == [O_ - 3] * 3


def test_residual_epilogue(dev):
    I, O_ = 4096, 2688
    (w, s, b), W = q4_weight(41, O_, I, dev)
    rng = np.random.default_rng(42)
    x, xd = bf16_rows(rng, 3, I, dev)
    res = S.to_device(O.f32_to_bf16(rng.standard_normal((3, O_)).astype(np.float32) * 4), dev)
    y = nn.linear(xd, W)                                                 # plain bf16 x, bf16 y
    ref = O.linear_q4(O.bf16_to_f32(x), w, s, b)
    assert np.all(np.abs(y.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))
    out = res.clone()
    nn.linear(xd, W, residual=out, out=out)                              # in place, as the model does
    want = (res.float() + y.float()).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    # one token row takes 2 rows per wavefront at this shape, three rows 4: the same bits
    for r in range(3):
        o1 = res[r:r + 1].clone()
        nn.linear(xd[r:r + 1], W, residual=o1, out=o1)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), f"row {r}"


@pytest.mark.parametrize("B", [2, 4])
def test_residual_epilogue_token_rows(dev, B):
    """Two and four token rows of a residual projection with few blocks (the one-row kernel
    over the token rows): each row equals that row alone, and the bf16 output plus the
    residual."""
    I, O_ = 4096, 2688
    _, W = q4_weight(45, O_, I, dev)
    rng = np.random.default_rng(46 + B)
    x, xd = bf16_rows(rng, B, I, dev)
    res = S.to_device(O.f32_to_bf16(rng.standard_normal((B, O_)).astype(np.float32) * 4), dev)
    y = nn.linear(xd, W)
    out = res.clone()
    nn.linear(xd, W, residual=out, out=out)
    assert torch.equal(out.view(torch.int16), (res.float() + y.float()).to(torch.bfloat16).view(torch.int16))
    for r in range(B):
        o1 = res[r:r + 1].clone()
        nn.linear(xd[r:r + 1], W, residual=o1, out=o1)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), f"row {r}"


def test_residual_epilogue_many_blocks(dev):
    """More 16-row blocks than resident workgroups (a workgroup runs several blocks in
    turn), so each block's residual is loaded with that block's weights: equal to the bf16
    output plus the residual, and every row of the three-row call to that row alone. (The
    residual epilogue takes 4-bit weights only.)"""
    I, O_ = 2688, 20480
    rng = np.random.default_rng(43)
    _, W = q4_weight(44, O_, I, dev)
    x, xd = bf16_rows(rng, 3, I, dev)
    res = S.to_device(O.f32_to_bf16(rng.standard_normal((3, O_)).astype(np.float32) * 4), dev)
    y = nn.linear(xd, W)
    out = res.clone()
    nn.linear(xd, W, residual=out, out=out)
    want = (res.float() + y.float()).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    for r in range(3):
        o1 = res[r:r + 1].clone()
        nn.linear(xd[r:r + 1], W, residual=o1, out=o1)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), f"row {r}"


def test_gated_norm_prologue(dev):
    I, O_ = 4096, 2688
    (w, s, b), W = q4_weight(51, O_, I, dev)
    rng = np.random.default_rng(52)
    y_pre = rng.standard_normal((2, I)).astype(np.float32) * 3
    gate = O.f32_to_bf16(rng.standard_normal((2, I)).astype(np.float32))
    gate_buf = torch.zeros((2, I + 64), dtype=torch.bfloat16, device=dev)  # a strided gate, as in_proj's
    gate_buf[:, 64:] = S.to_device(gate, dev)
    nw = O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32))
    res = torch.zeros((2, O_), dtype=torch.bfloat16, device=dev)
    xn = torch.empty((2, I), dtype=torch.bfloat16, device=dev)
    # the gated norm is instantiated with the residual epilogue only (out_proj)
    out = nn.linear(torch.from_numpy(y_pre).to(dev), W, norm=S.to_device(nw, dev), gate=gate_buf[:, 64:],
                    residual=res, xn_out=xn)
    xn_h = S.to_host(xn)
    ok, same = ulp_close(xn_h, O.gated_rms_norm_bf16(y_pre, O.bf16_to_f32(gate), O.bf16_to_f32(nw), 1e-5))
    print(f"gated norm: within 1 ulp {ok}, identical {same:.4f}")
    assert ok and same >= 0.99
    ref = O.linear_q4(O.bf16_to_f32(xn_h), w, s, b)
    assert np.all(np.abs(out.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))


@pytest.mark.parametrize("I,O_,B", [(2688, 128, 1), (2688, 128, 3), (5376, 2688, 3)])
def test_bf16_weights(dev, I, O_, B):
    rng = np.random.default_rng(60 + I + B)
    wb = O.f32_to_bf16((rng.standard_normal((O_, I)) * 0.02).astype(np.float32))
    W = nn.QWeight(S.to_device(wb, dev))
    x, xd = bf16_rows(rng, B, I, dev)
    y = nn.linear(xd, W)
    ref = O.linear_bf16(O.bf16_to_f32(x), wb)
    assert np.all(np.abs(y.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))
    if I == 2688:                                                        # the router: rms prologue
        nw = O.f32_to_bf16(rng.uniform(0.5, 1.5, I).astype(np.float32))
        xn = torch.empty((B, I), dtype=torch.bfloat16, device=dev)
        y = nn.linear(xd, W, norm=S.to_device(nw, dev), xn_out=xn)
        ref = O.linear_bf16(O.bf16_to_f32(S.to_host(xn)), wb)
        assert np.all(np.abs(y.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))
        for r in range(B):
            assert torch.equal(nn.linear(xd[r:r + 1], W, norm=S.to_device(nw, dev)).view(torch.int16),
                               y[r:r + 1].view(torch.int16))


def test_embed_rows(dev):
    rng = np.random.default_rng(70)
    V, D = 1000, 2688
    w, s, b = S.down_proj_np(rng, (), V, D)
    W = nn.QWeight(S.to_device(w, dev), S.to_device(s, dev), S.to_device(b, dev))
    tok = np.array([0, 999, 17, 1000], dtype=np.int32)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    out = nn.embed(torch.from_numpy(tok).to(dev), W, status=status)
    assert np.array_equal(S.to_host(out), O.embed_q4(tok, w, s, b))
    assert int(status.item()) == 4                                       # token 1000 is outside [0, V)


def test_pair_norm(dev):
    rng = np.random.default_rng(80)
    D = 2688
    e, ed = bf16_rows(rng, 3, D, dev)
    h, hd = bf16_rows(rng, 3, D, dev, 5.0)
    we = O.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    wh = O.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    out = S.to_host(nn.pair_norm(ed, hd, S.to_device(we, dev), S.to_device(wh, dev)))
    ref = np.concatenate([O.rms_norm_bf16(O.bf16_to_f32(e), O.bf16_to_f32(we)),
                          O.rms_norm_bf16(O.bf16_to_f32(h), O.bf16_to_f32(wh))], axis=1)
    ok, same = ulp_close(out, ref)
    assert ok and same >= 0.99


def test_head_input_equals_embed_then_pair_norm(dev):
    """hsd_head_input (the MTP head's embedding and pair norm in one launch) equals
    hsd_embed_q4 then hsd_pair_norm bit for bit: on token rows (a token outside the table
    embeds as zeros and sets the status bit), and for the chained call, whose token is the
    argmax of a keys row (d1 and HEAD_POS2 as hsd_mtp_chain writes them)."""
    rng = np.random.default_rng(81)
    V, D = 1000, 2688
    w, s, b = S.down_proj_np(rng, (), V, D)
    W = nn.QWeight(S.to_device(w, dev), S.to_device(s, dev), S.to_device(b, dev))
    h, hd = bf16_rows(rng, 3, D, dev, 5.0)
    we = S.to_device(O.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)), dev)
    wh = S.to_device(O.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32)), dev)
    tok = torch.tensor([5, 999, 1000], dtype=torch.int32, device=dev)
    st1 = torch.zeros(1, dtype=torch.int32, device=dev)
    st2 = torch.zeros(1, dtype=torch.int32, device=dev)
    want = nn.pair_norm(nn.embed(tok, W, status=st1), hd, we, wh)
    got = nn.head_input(tok, hd, W, we, wh, status=st2)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert int(st1.item()) == 4 and int(st2.item()) == 4
    # the chained call: keys of one row (the per-workgroup keys of an argmax linear)
    slots = 512
    vals = rng.integers(0, 1 << 30, slots, dtype=np.int64)      # (order bits << 32) | ~index
    keys = torch.from_numpy(((vals << 32) | (~np.arange(slots, dtype=np.int64) & 0xFFFFFFFF)).reshape(1, slots)).to(dev)
    for R in (1, 2, 3):
        seq = torch.zeros(N.SEQ_LEN, dtype=torch.int32, device=dev)
        seq[N.SEQ_R] = R
        seq[N.SEQ_HEAD_POS] = 40
        seq2 = seq.clone()
        d1a = torch.zeros(4, dtype=torch.int32, device=dev)
        d1b = torch.zeros(4, dtype=torch.int32, device=dev)
        h2 = torch.empty((1, D), dtype=torch.bfloat16, device=dev)
        N.call("hsd_mtp_chain", N.ptr(keys), 0, slots, N.ptr(hd[1:2]), 0, D, N.ptr(seq), N.ptr(d1a), N.ptr(h2),
               N.stream(dev))
        want = nn.pair_norm(nn.embed(d1a[:1], W), h2, we, wh)
        got = nn.head_input(None, hd[1:2], W, we, wh, chain=(keys, seq2, d1b))
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), R
        assert torch.equal(d1a, d1b) and torch.equal(seq, seq2), R


@pytest.mark.parametrize("scripted", [False, True])
def test_verify_input_equals_draft_ids_then_embed(dev, scripted):
    """hsd_verify_input (the verify ids and their embedding rows in one launch) equals
    hsd_draft_ids then hsd_embed_q4 bit for bit, with the head's own drafts and with
    scripted acceptance."""
    rng = np.random.default_rng(82)
    V, D = 1000, 2688
    w, s, b = S.down_proj_np(rng, (), V, D)
    W = nn.QWeight(S.to_device(w, dev), S.to_device(s, dev), S.to_device(b, dev))
    slots = 512
    vals = rng.integers(0, 1 << 30, slots, dtype=np.int64)      # (order bits << 32) | ~token
    idx = (rng.permutation(slots) % V).astype(np.int64)
    keys2 = torch.from_numpy(((vals << 32) | (~idx & 0xFFFFFFFF)).reshape(1, slots)).to(dev)
    d1 = torch.tensor([321], dtype=torch.int32, device=dev)
    script = torch.from_numpy(rng.integers(0, V, 64).astype(np.int32)).to(dev) if scripted else None
    accepts = torch.tensor([0, 1, 2, 1], dtype=torch.int32, device=dev) if scripted else None
    for step in range(4):
        seq = torch.zeros(N.SEQ_LEN, dtype=torch.int32, device=dev)
        seq[N.SEQ_TOK] = 777
        seq[N.SEQ_N] = 5 + 2 * step
        seq[N.SEQ_STEPS] = step
        args = (N.ptr(d1), N.ptr(keys2), slots, 2, N.ptr(seq), N.ptr(script), 0 if script is None else script.numel(),
                N.ptr(accepts), 0 if accepts is None else accepts.numel(), V)
        ids_a = torch.full((4,), -1, dtype=torch.int32, device=dev)
        N.call("hsd_draft_ids", *args, N.ptr(ids_a), N.stream(dev))
        want = nn.embed(ids_a[:3], W)
        ids_b = torch.full((4,), -1, dtype=torch.int32, device=dev)
        got = torch.empty((3, D), dtype=torch.bfloat16, device=dev)
        st = torch.zeros(1, dtype=torch.int32, device=dev)
        N.call("hsd_verify_input", *args, N.ptr(W.w), N.ptr(W.scales), N.ptr(W.biases), D, N.ptr(ids_b), N.ptr(got),
               got.stride(0), N.ptr(st), N.stream(dev))
        assert torch.equal(ids_a, ids_b), step
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        assert int(st.item()) == 0
