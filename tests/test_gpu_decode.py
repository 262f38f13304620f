"""GPU parity of the sparse decode down projection (hsd/decode.py:37-186) at the
Nemotron-3.5 MoE shape (D=2688, F=1856, FS=3712, top-6 of 128 + shared, affine 4-bit g64).

Bars:
* integer work bit-exact: the canonical live masks equal the oracle's;
* fp32 output within max|y - ref| <= 1e-5 * max|ref| of the float64 oracle;
* bf16 output within the bf16 parity bound |y - ref| <= 2e-2 + 1e-2 * |ref|;
* bit-exact: dense-h control == sparse (skipping exact zeros is exact), and every row
  of a B-row call == the same row alone (verify rows == single rows).
"""
import numpy as np
import pytest
import torch

from hsd import decode, layout, synth as S
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
D, F, FS, TOPK = 2688, 1856, 3712, 6
KW = dict(F=F, FS=FS, D=D, topk=TOPK)


@pytest.fixture(scope="module")
def layer(dev):
    lay = S.moe_layer_np(7)
    dv = {k: S.to_device(v, dev) for k, v in lay.items()}
    pw, ps, pb = layout.to_neuron_major(dv["w"], dv["s"], dv["b"])
    spw, sps, spb = layout.to_neuron_major(dv["sw"], dv["ss"], dv["sb"])
    nm_np = O.to_neuron_major(lay["w"], lay["s"], lay["b"]) + O.to_neuron_major(lay["sw"], lay["ss"], lay["sb"])
    return dict(np=lay, dev=dv, nm=(pw, ps, pb, spw, sps, spb), nm_np=nm_np)


def run_case(layer, dev, seed, B, zero_frac, out_dtype=torch.float32, h_dtype=torch.bfloat16, **kw):
    h, sel, gains = S.decode_inputs_np(seed, B=B, zero_frac=zero_frac)
    hd = S.to_device(h, dev).to(h_dtype)
    y = decode.sparse_down(hd, S.to_device(sel, dev), S.to_device(gains, dev), *layer["nm"], out_dtype=out_dtype,
                           **KW, **kw)
    return h, sel, gains, hd, y


@pytest.mark.parametrize("zero_frac", [0.0, 0.7, 0.85, 0.9, 0.95, 0.97, 1.0])
def test_sparse_down_matches_oracle(layer, dev, zero_frac):
    h, sel, gains, hd, y = run_case(layer, dev, 11, 1, zero_frac)
    ref = O.sparse_down(O.bf16_to_f32(h), sel, gains, *layer["nm_np"], **KW)
    yh = y.cpu().numpy()
    scale = max(np.abs(ref).max(), 1e-30)
    print(f"zero_frac {zero_frac}: max|ref| {scale:.3f}  max rel err {np.abs(yh - ref).max() / scale:.2e}")
    if zero_frac == 1.0:
        assert np.all(yh == 0.0)
    else:
        assert np.abs(yh - ref).max() <= 1e-5 * scale


def test_bf16_output_and_textbook_reference(layer, dev):
    h, sel, gains, hd, y = run_case(layer, dev, 12, 1, 0.9, out_dtype=torch.bfloat16)
    lay = layer["np"]
    ref = O.dense_reference(O.bf16_to_f32(h), sel, gains, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"],
                            lay["sb"], **KW)
    yh = y.float().cpu().numpy()
    assert np.all(np.abs(yh - ref) <= 2e-2 + 1e-2 * np.abs(ref))


def test_live_masks_bit_exact(layer, dev):
    h, sel, gains = S.decode_inputs_np(13, B=3, zero_frac=0.9)
    h[0, :64] = 0                                   # an all-dead group
    h[1, 5] = 0x8000                                # -0.0 is dead
    h[2, TOPK * F - 1] = S.bf16_bits(2.0)           # last neuron of the last routed slot
    masks = torch.zeros(3 * (TOPK * F // 64 + FS // 64), dtype=torch.int64, device=dev)
    decode.sparse_down(S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev), *layer["nm"],
                       live_masks=masks, **KW)
    want = O.live_masks(O.bf16_to_f32(h), F, FS, TOPK).reshape(-1)
    assert np.array_equal(masks.cpu().numpy().view(np.uint64), want)


@pytest.mark.parametrize("zero_frac", [0.5, 0.9])
def test_dense_h_control_is_bit_identical(layer, dev, zero_frac):
    h, sel, gains, hd, y = run_case(layer, dev, 14, 2, zero_frac)
    yd = decode.sparse_down(hd, S.to_device(sel, dev), S.to_device(gains, dev), *layer["nm"],
                            out_dtype=torch.float32, dense=True, **KW)
    assert torch.equal(y, yd)


def test_rows_independent_of_batch(layer, dev):
    h, sel, gains, hd, y3 = run_case(layer, dev, 15, 3, 0.9)
    for b in range(3):
        y1 = decode.sparse_down(hd[b:b + 1], S.to_device(sel[b:b + 1], dev), S.to_device(gains[b:b + 1], dev),
                                *layer["nm"], out_dtype=torch.float32, **KW)
        assert torch.equal(y1[0], y3[b])


def test_many_rows(layer, dev):
    """24 rows in one call (16128 workgroups, several rounds of what is resident): every row
    equals the same row alone, bit for bit; rows against the oracle; live masks bit-exact;
    a bad id in one row flagged and skipped; dense-h control equal."""
    B = 24
    h, sel, gains = S.decode_inputs_np(18, B=B, zero_frac=0.9)
    sel[7, 1] = 4000
    hd, seld, gd = S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev)
    masks = torch.zeros(B * (TOPK * F // 64 + FS // 64), dtype=torch.int64, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    y = decode.sparse_down(hd, seld, gd, *layer["nm"], out_dtype=torch.float32, live_masks=masks, status=status,
                           **KW)
    yd = decode.sparse_down(hd, seld, gd, *layer["nm"], out_dtype=torch.float32, dense=True, **KW)
    assert int(status.item()) == 1
    assert torch.equal(y, yd)
    for b in range(B):
        y1 = decode.sparse_down(hd[b:b + 1], seld[b:b + 1], gd[b:b + 1], *layer["nm"], out_dtype=torch.float32,
                                **KW)
        assert torch.equal(y1[0], y[b]), f"row {b}"
    g0 = gains.copy()
    g0[7, 1] = 0.0
    s0 = sel.copy()
    s0[7, 1] = 0
    hf = O.bf16_to_f32(h)
    for b in (0, 7, B - 1):
        ref = O.sparse_down(hf[b:b + 1], s0[b:b + 1], g0[b:b + 1], *layer["nm_np"], **KW)
        assert np.abs(y[b].cpu().numpy() - ref[0]).max() <= 1e-5 * np.abs(ref).max(), f"row {b}"
    want = O.live_masks(hf, F, FS, TOPK).reshape(B, -1)
    got = masks.cpu().numpy().view(np.uint64).reshape(B, -1)
    ok = np.ones(B, dtype=bool)
    ok[7] = False                                   # a bad id's slot reports no live rows
    assert np.array_equal(got[ok], want[ok])


@pytest.mark.parametrize("h_dtype", [torch.float32, torch.float16])
def test_other_activation_dtypes(layer, dev, h_dtype):
    h, sel, gains, hd, y = run_case(layer, dev, 16, 1, 0.9, h_dtype=h_dtype)
    hv = hd.float().cpu().numpy()
    ref = O.sparse_down(hv, sel, gains, *layer["nm_np"], **KW)
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


def test_bad_expert_id_is_flagged_and_skipped(layer, dev):
    h, sel, gains = S.decode_inputs_np(17, B=1, zero_frac=0.9)
    bad = sel.copy()
    bad[0, 2] = 999
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    y = decode.sparse_down(S.to_device(h, dev), S.to_device(bad, dev), S.to_device(gains, dev), *layer["nm"],
                           out_dtype=torch.float32, status=status, **KW)
    assert int(status.item()) == 1
    g0 = gains.copy()
    g0[0, 2] = 0.0
    ref = O.sparse_down(O.bf16_to_f32(h), sel, g0, *layer["nm_np"], **KW)
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("h_dtype", [torch.bfloat16, torch.float32])
def test_dense_stock_comparator(layer, dev, h_dtype):
    """bf16 h takes the GEMV-shaped kernel (pieces of the 7 slots' rows per lane), f32 h the
    element-wise one; both against the oracle's dequantise-then-mat-vec (float64), and a
    bad expert id adds nothing and sets the status bit."""
    h, sel, gains = S.decode_inputs_np(18, B=2, zero_frac=0.9)
    dv = layer["dev"]
    hd = S.to_device(h, dev).to(h_dtype)
    lay = layer["np"]
    y = decode.dense_down(hd, S.to_device(sel, dev), S.to_device(gains, dev), dv["w"], dv["s"],
                          dv["b"], dv["sw"], dv["ss"], dv["sb"], out_dtype=torch.float32, **KW)
    ref = O.dense_reference(O.bf16_to_f32(h), sel, gains, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"],
                            lay["sb"], **KW)
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    bad = sel.copy()
    bad[1, 4] = -3
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    yb = decode.dense_down(hd, S.to_device(bad, dev), S.to_device(gains, dev), dv["w"], dv["s"], dv["b"], dv["sw"],
                           dv["ss"], dv["sb"], out_dtype=torch.float32, status=status, **KW)
    g0 = gains.copy()
    g0[1, 4] = 0.0
    ref_b = O.dense_reference(O.bf16_to_f32(h), sel, g0, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"],
                              lay["sb"], **KW)
    assert int(status.item()) == 1
    assert np.abs(yb.cpu().numpy() - ref_b).max() <= 1e-5 * np.abs(ref_b).max()


@pytest.mark.parametrize("zero_frac", [0.85, 0.9, 0.95])
def test_hot_neurons_match_oracle(layer, dev, zero_frac):
    """The hot-neuron activation model (a fixed 5 % of each slot's neurons live with
    p = 0.6, the rest at the rate that keeps the mean zero fraction), B = 3."""
    rng = np.random.default_rng(15)
    hot_mask = rng.random(TOPK * F + FS) < 0.05
    p_hot, p_cold = S.hot_cold_rates(zero_frac)
    h, sel, gains = S.decode_inputs_np(16, B=3, zero_frac=zero_frac, hot=(hot_mask, p_hot, p_cold))
    y = decode.sparse_down(S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev), *layer["nm"],
                           out_dtype=torch.float32, **KW)
    ref = O.sparse_down(O.bf16_to_f32(h), sel, gains, *layer["nm_np"], **KW)
    yh = y.cpu().numpy()
    scale = np.abs(ref).max()
    print(f"hot neurons, zero_frac {zero_frac}: measured {np.mean(h == 0):.3f}, "
          f"max rel err {np.abs(yh - ref).max() / scale:.2e}")
    assert np.abs(yh - ref).max() <= 1e-5 * scale
