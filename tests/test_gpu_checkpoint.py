"""GPU: MoE layers loaded from a synthetic MLX-format checkpoint (hsd.checkpoint;
tests/test_layout_decode.py:24-35, hsd/model.py:182-252).

* sparse mode: each layer's neuron-major layout equals the oracle's permutation of the
  checkpoint bytes bit for bit, and the stock down projections are released
  (one resident layout, AGENTS.md:47-49);
* the loaded layer computes what the lower-level calls compute on the same bytes: decode
  bit-identical to decode.sparse_down on the oracle-permuted weights, and within 1e-5 of
  the output scale of the float64 oracle; the front end bit-identical to moe.up_relu2 on
  the checkpoint's up projections;
* with single_layout=False both layouts stay and dense decode matches the oracle."""
import numpy as np
import pytest
import torch

from hsd import checkpoint as C
from hsd import decode, synth as S
from hsd.moe import up_relu2
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
E, D, F, FS, K = 8, 256, 128, 192, 2


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckg")
    arrays = S.write_checkpoint(str(d), 17, pattern="EME", n_experts=E, d=D, f=F, fs=FS, topk=K, shards=2)
    return str(d), arrays


def front_outputs(h, sel, gains, dev):
    hc = S.to_device(h, dev)
    B = hc.shape[0]
    return (S.to_device(sel, dev).long(), S.to_device(gains, dev)[:, :K],
            hc[:, :K * F].reshape(B, K, 1, F), hc[:, K * F:])


def test_sparse_load_permutes_and_releases(ckpt, dev):
    d, arrays = ckpt
    layers = C.load_moe_layers(d, dev, mode="sparse", single_layout=True)
    assert sorted(layers) == [0, 2]
    for l, ml in layers.items():
        blk, dn = ml.down, arrays[l]["down"]
        assert blk.has_layout and not blk.stock_layout and blk.fc2 is None and blk.shared_down is None
        want = O.to_neuron_major(dn["w"], dn["s"], dn["b"]) + O.to_neuron_major(dn["sw"], dn["ss"], dn["sb"])
        for got, w in zip(blk.w_routed + blk.w_shared, want):
            g = S.to_host(got)
            g = g.view(np.uint32) if g.dtype == np.int32 else g
            assert g.shape == w.shape and np.array_equal(g, w)


def test_loaded_layer_decode_and_front(ckpt, dev):
    d, arrays = ckpt
    layers = C.load_moe_layers(d, dev)
    for l, ml in layers.items():
        blk, dn, up = ml.down, arrays[l]["down"], arrays[l]["up"]
        h, sel, gains = S.decode_inputs_np(60 + l, B=2, zero_frac=0.9, n_experts=E, f=F, fs=FS, topk=K)
        inds, scores, hh, hs = front_outputs(h, sel, gains, dev)
        x = torch.zeros((2, D), dtype=torch.float32, device=dev)
        blk.decode_kw = dict(out_dtype=torch.float32)
        y = blk.decode_sparse(x, inds, scores, hh, hs)
        nm = [S.to_device(a, dev) for a in O.to_neuron_major(dn["w"], dn["s"], dn["b"])
              + O.to_neuron_major(dn["sw"], dn["ss"], dn["sb"])]
        hcat, s2, g2 = blk.pack(inds, scores, hh, hs)
        direct = decode.sparse_down(hcat, s2, g2, *nm, F=F, FS=FS, D=D, topk=K, out_dtype=torch.float32)
        assert torch.equal(y, x + direct)
        ref = O.sparse_down(O.bf16_to_f32(h), sel, gains, *O.to_neuron_major(dn["w"], dn["s"], dn["b"]),
                            *O.to_neuron_major(dn["sw"], dn["ss"], dn["sb"]), F=F, FS=FS, D=D, topk=K)
        assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
        rng = np.random.default_rng(70 + l)
        xb = S.to_device(O.f32_to_bf16((rng.standard_normal((2, D)) * 0.5).astype(np.float32)), dev)
        inds2 = torch.from_numpy(np.stack([rng.permutation(E)[:K] for _ in range(2)]).astype(np.int32)).to(dev)
        got = ml.front(xb, inds2)
        u = {k: S.to_device(v, dev) for k, v in up.items()}
        want = up_relu2(xb, inds2, u["w1"], u["s1"], u["b1"], u["sw1"], u["ss1"], u["sb1"], topk=K)
        assert got.shape == (2, K * F + FS) and torch.equal(got, want)


def test_both_layouts_when_not_single(ckpt, dev):
    d, arrays = ckpt
    layers = C.load_moe_layers(d, dev, single_layout=False, layers=[2])
    ml = layers[2]
    blk, dn = ml.down, arrays[2]["down"]
    assert blk.has_layout and blk.stock_layout
    h, sel, gains = S.decode_inputs_np(80, B=1, zero_frac=0.9, n_experts=E, f=F, fs=FS, topk=K)
    inds, scores, hh, hs = front_outputs(h, sel, gains, dev)
    x = torch.zeros((1, D), dtype=torch.float32, device=dev)
    blk.decode_kw = dict(out_dtype=torch.float32)
    yd = blk.decode_dense(x, inds, scores, hh, hs).cpu().numpy()
    ys = blk.decode_sparse(x, inds, scores, hh, hs).cpu().numpy()
    ref = O.dense_reference(O.bf16_to_f32(h), sel, gains, dn["w"], dn["s"], dn["b"], dn["sw"], dn["ss"],
                            dn["sb"], F=F, FS=FS, D=D, topk=K)
    assert np.abs(yd - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.abs(ys - ref).max() <= 1e-5 * np.abs(ref).max()
