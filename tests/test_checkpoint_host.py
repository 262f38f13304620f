"""The checkpoint reader (hsd.checkpoint; tests/test_layout_decode.py:24-35, hsd/model.py:182-252)
on the CPU: a synthetic MLX-format checkpoint written with safetensors is read back with
every tensor's bytes intact, under the names test_layout_decode.py:27-31 uses, from an
index with several shards and from a single file; the MoE layers come from the config's
pattern; and malformed checkpoints fail with an error that names the problem. "dense" mode
needs no kernel, so it is exercised here too."""
import json
import os

import numpy as np
import pytest
import torch

from hsd import _native as N
from hsd import checkpoint as C
from hsd import synth as S

E, D, F, FS, K = 4, 128, 128, 192, 2


def host_bits(t):
    return S.to_host(t) if t.dtype == torch.bfloat16 else t.view(torch.int32).numpy().view(np.uint32)


@pytest.fixture(scope="module", params=[2, 1], ids=["index", "single"])
def ckpt(request, tmp_path_factory):
    d = tmp_path_factory.mktemp(f"ck{request.param}")
    arrays = S.write_checkpoint(str(d), 5, pattern="MEM*E", n_experts=E, d=D, f=F, fs=FS, topk=K,
                                shards=request.param)
    return str(d), arrays, request.param


def test_names_follow_the_checkpoint_convention():
    n = C.moe_tensor_names(10)
    assert len(n) == 12 and len(set(n)) == 12
    assert n[:3] == [f"backbone.layers.10.mixer.switch_mlp.fc1.{k}" for k in ("weight", "scales", "biases")]
    assert n[3] == "backbone.layers.10.mixer.switch_mlp.fc2.weight"
    assert n[6] == "backbone.layers.10.mixer.shared_experts.up_proj.weight"
    assert n[11] == "backbone.layers.10.mixer.shared_experts.down_proj.biases"


def test_layers_and_bytes_round_trip(ckpt):
    d, arrays, shards = ckpt
    ck = C.Checkpoint(d)
    assert ck.layer_kinds == ["mamba", "moe", "mamba", "attention", "moe"]
    assert ck.moe_layers == [1, 4] == sorted(arrays)
    assert len(set(ck.weight_map.values())) == shards
    for l in ck.moe_layers:
        t = ck.moe_layer(l)
        n = C.moe_tensor_names(l)
        dn, up = arrays[l]["down"], arrays[l]["up"]
        want = [up["w1"], up["s1"], up["b1"], dn["w"], dn["s"], dn["b"],
                up["sw1"], up["ss1"], up["sb1"], dn["sw"], dn["ss"], dn["sb"]]
        for name, w in zip(n, want):
            got = host_bits(t[name])
            assert got.shape == w.shape and got.dtype == w.dtype, name
            assert np.array_equal(got, w), name
        assert C.check_moe_shapes(t, l, ck.config) == (E, D, F, FS)


@pytest.fixture(scope="module")
def index_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("cki")
    S.write_checkpoint(str(d), 5, pattern="MEM*E", n_experts=E, d=D, f=F, fs=FS, topk=K, shards=3)
    return str(d)


def test_moe_layers_without_config(index_ckpt, tmp_path):
    d = index_ckpt
    for fn in os.listdir(d):
        if fn != "config.json":
            os.symlink(os.path.join(d, fn), tmp_path / fn)
    ck = C.Checkpoint(str(tmp_path))
    assert ck.config == {} and ck.layer_kinds is None
    assert ck.moe_layers == [1, 4]       # from the tensor names


def test_dense_mode_keeps_the_stock_layout(ckpt):
    d, arrays, _ = ckpt
    layers = C.load_moe_layers(d, "cpu", mode="dense")
    assert sorted(layers) == [1, 4]
    for l, ml in layers.items():
        blk = ml.down
        assert (blk.E, blk.D, blk.F, blk.FS, blk.topk) == (E, D, F, FS, K)
        assert blk.stock_layout and not blk.has_layout
        assert np.array_equal(host_bits(blk.fc2["weight"]), arrays[l]["down"]["w"])
        assert np.array_equal(host_bits(ml.up["sw1"]), arrays[l]["up"]["sw1"])
        with pytest.raises(N.HSDError, match="layout"):
            blk.decode_sparse(None, None, None, None, None)


def test_missing_tensor_is_named(index_ckpt, tmp_path):
    d = index_ckpt
    idx = json.load(open(os.path.join(d, C.INDEX)))
    gone = "backbone.layers.4.mixer.shared_experts.down_proj.scales"
    del idx["weight_map"][gone]
    for fn in os.listdir(d):
        if fn != C.INDEX:
            os.symlink(os.path.join(d, fn), tmp_path / fn)
    json.dump(idx, open(tmp_path / C.INDEX, "w"))
    ck = C.Checkpoint(str(tmp_path))
    ck.moe_layer(1)
    with pytest.raises(N.HSDError, match=gone.replace(".", r"\.")):
        ck.moe_layer(4)


def test_rejects_other_quantisations_and_shapes(tmp_path):
    S.write_checkpoint(str(tmp_path), 9, pattern="E", n_experts=E, d=D, f=F, fs=FS, topk=K, shards=1)
    cfg = json.load(open(tmp_path / "config.json"))
    ck = C.Checkpoint(str(tmp_path))
    t = ck.moe_layer(0)
    # a config that disagrees with the tensors
    with pytest.raises(N.HSDError, match="moe_intermediate_size"):
        C.check_moe_shapes(t, 0, dict(cfg, moe_intermediate_size=F + 64))
    # a group size the kernels do not read
    bad = dict(t)
    name = "backbone.layers.0.mixer.switch_mlp.fc2.scales"
    bad[name] = torch.zeros((E, D, F // 32), dtype=torch.bfloat16)
    with pytest.raises(N.HSDError, match="fc2 scales"):
        C.check_moe_shapes(bad, 0)
    bad = dict(t)
    bad["backbone.layers.0.mixer.switch_mlp.fc2.weight"] = torch.zeros((E, D, F // 8), dtype=torch.float32)
    with pytest.raises(N.HSDError, match="32-bit words"):
        C.check_moe_shapes(bad, 0)
    json.dump(dict(cfg, quantization=dict(group_size=32, bits=4)), open(tmp_path / "config.json", "w"))
    with pytest.raises(N.HSDError, match="group 64"):
        C.Checkpoint(str(tmp_path))
    with pytest.raises(N.HSDError, match="neither"):
        C.Checkpoint(str(tmp_path / "nowhere"))
    with pytest.raises(N.HSDError, match="mode"):
        C.load_moe_layers(str(tmp_path), "cpu", mode="fast")
