"""GPU: the MoE block's down-projection surface (hsd/model.py:89-175) end to end after
the front end: build_layout (one resident layout), pack, sparse decode, the dense
comparator on the stock layout and the sparse prefill, each against the float64 oracle
(max |y - ref| <= 1e-5 of the output scale for decode, 1e-4 for the bf16-MFMA prefill)
and against the lower-level calls they wrap (bit-exact)."""
import numpy as np
import pytest
import torch

from hsd import decode, synth as S
from hsd.moe import MoEDown, build_layouts
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
D, F, FS, K, E = 2688, 1856, 3712, 6, 128


def make_block(lay, dev, **kw):
    dv = {k: S.to_device(v, dev) for k, v in lay.items()}
    return MoEDown(dict(weight=dv["w"], scales=dv["s"], biases=dv["b"]),
                   dict(weight=dv["sw"], scales=dv["ss"], biases=dv["sb"]), topk=K, **kw)


def front_outputs(hcat_bits, sel, gains, dev):
    """Split synthetic (hcat, sel, gains) into what the front end returns: inds, scores,
    h [B, K, 1, F], hs [B, FS]."""
    hc = S.to_device(hcat_bits, dev)
    B = hc.shape[0]
    return (S.to_device(sel, dev).long(), S.to_device(gains, dev)[:, :K],
            hc[:, :K * F].reshape(B, K, 1, F), hc[:, K * F:])


@pytest.fixture(scope="module")
def lay():
    return S.moe_layer_np(31)


def test_decode_sparse_and_dense(lay, dev):
    blk = make_block(lay, dev, decode_kw=dict(out_dtype=torch.float32))
    h, sel, gains = S.decode_inputs_np(41, B=2, zero_frac=0.9)
    inds, scores, hh, hs = front_outputs(h, sel, gains, dev)
    x = torch.zeros((2, D), dtype=torch.float32, device=dev)
    ref = O.dense_reference(O.bf16_to_f32(h), sel, gains, lay["w"], lay["s"], lay["b"], lay["sw"], lay["ss"],
                            lay["sb"], F=F, FS=FS, D=D, topk=K)
    yd = blk.decode_dense(x, inds, scores, hh, hs).cpu().numpy()
    assert np.abs(yd - ref).max() <= 1e-5 * np.abs(ref).max()
    build_layouts([blk], single_layout=True)
    assert blk.has_layout and not blk.stock_layout
    ys = blk.decode_sparse(x, inds, scores, hh, hs)
    assert np.abs(ys.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    hcat, s2, g2 = blk.pack(inds, scores, hh, hs)
    direct = decode.sparse_down(hcat, s2, g2, *blk.w_routed, *blk.w_shared, F=F, FS=FS, D=D, topk=K,
                                out_dtype=torch.float32)
    assert torch.equal(ys, x + direct)


def test_residual_in_activation_dtype(lay, dev):
    blk = make_block(lay, dev)
    blk.build_layout()
    h, sel, gains = S.decode_inputs_np(42, B=1, zero_frac=0.9)
    inds, scores, hh, hs = front_outputs(h, sel, gains, dev)
    x = torch.randn((1, D), device=dev).to(torch.bfloat16)
    y = blk.decode_sparse(x, inds, scores, hh, hs)
    assert y.dtype == torch.bfloat16
    hcat, s2, g2 = blk.pack(inds, scores, hh, hs)
    direct = decode.sparse_down(hcat, s2, g2, *blk.w_routed, *blk.w_shared, F=F, FS=FS, D=D, topk=K)
    assert torch.equal(y, x + direct.to(x.dtype))


@pytest.mark.parametrize("tt", [32, 64])
def test_prefill_sparse(lay, dev, tt):
    blk = make_block(lay, dev, prefill_kw=dict(tt=tt, out_dtype=torch.float32))
    blk.build_layout()
    T = 96
    h, sel, gains = S.prefill_inputs_np(43, T=T, zero_frac=0.9)
    inds, scores, hh, hs = front_outputs(h, sel, gains, dev)
    x = torch.zeros((T, D), dtype=torch.float32, device=dev)
    y = blk.prefill_sparse(x, inds, scores, hh.reshape(T, K, F), hs).cpu().numpy()
    nm = O.to_neuron_major(lay["w"], lay["s"], lay["b"]) + O.to_neuron_major(lay["sw"], lay["ss"], lay["sb"])
    ref, _ = O.sparse_down_prefill(O.bf16_to_f32(h), sel, gains, *nm, F=F, FS=FS, D=D, topk=K, E=E, tt=tt)
    assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max()
