"""The MoE layers of an MLX 4-bit checkpoint: read straight from its safetensors
(tests/test_layout_decode.py:24-35, load_moe_layer) and, for sparse mode, permuted into
the neuron-major layout at load time, one layer at a time, with the checkpoint's own down
layout released before the next layer is read (hsd/model.py:182-252, NemotronModel
__init__ + set_mode; AGENTS.md:47-49: exactly one down layout resident).

Checkpoint format (the names of test_layout_decode.py:27-31; the config keys of
model.py:64-69 and 200-201):
  model.safetensors.index.json  {"weight_map": {tensor name: shard file}}, or one
                                model.safetensors without an index
  config.json                   hidden_size, moe_intermediate_size,
                                moe_shared_expert_intermediate_size, n_routed_experts,
                                num_experts_per_tok, hybrid_override_pattern ("M" Mamba,
                                "*" attention, "E" MoE), quantization {group_size, bits}
  backbone.layers.{l}.mixer.switch_mlp.fc1.{weight,scales,biases}
      routed up projections   [E, F, D/8] u32, [E, F, D/64] bf16
  backbone.layers.{l}.mixer.switch_mlp.fc2.{weight,scales,biases}
      routed down projections [E, D, F/8] u32, [E, D, F/64] bf16
  backbone.layers.{l}.mixer.shared_experts.up_proj.{weight,scales,biases}
      [FS, D/8] u32, [FS, D/64] bf16
  backbone.layers.{l}.mixer.shared_experts.down_proj.{weight,scales,biases}
      [D, FS/8] u32, [D, FS/64] bf16
Only affine 4-bit with group 64 is accepted (the format every kernel here reads). Tensors
are read with safetensors' own reader, which executes nothing from the file.
"""
from __future__ import annotations

import json
import os

import torch
from safetensors import safe_open

from . import _native as N
from . import moe

INDEX = "model.safetensors.index.json"
SINGLE = "model.safetensors"
PARTS = ("weight", "scales", "biases")
GROUP_SIZE, BITS = 64, 4
LAYER_KINDS = {"M": "mamba", "*": "attention", "E": "moe"}   # model.py:201


def moe_tensor_names(layer):
    """The 12 tensors of MoE layer `layer`, in test_layout_decode.py:28-31's order: fc1,
    fc2, then the shared expert's up_proj and down_proj, each weight, scales, biases."""
    p = f"backbone.layers.{layer}.mixer"
    return ([f"{p}.switch_mlp.fc1.{k}" for k in PARTS] + [f"{p}.switch_mlp.fc2.{k}" for k in PARTS]
            + [f"{p}.shared_experts.{n}.{k}" for n in ("up_proj", "down_proj") for k in PARTS])


class Checkpoint:
    """A checkpoint directory: the tensor -> shard map and config.json (if present)."""

    def __init__(self, model_dir):
        self.dir = str(model_dir)
        index = os.path.join(self.dir, INDEX)
        single = os.path.join(self.dir, SINGLE)
        if os.path.exists(index):
            with open(index) as f:
                self.weight_map = dict(json.load(f)["weight_map"])
        elif os.path.exists(single):
            with safe_open(single, framework="pt") as f:
                self.weight_map = {k: SINGLE for k in f.keys()}
        else:
            raise N.HSDError(f"{self.dir}: neither {INDEX} nor {SINGLE}")
        cfg = os.path.join(self.dir, "config.json")
        self.config = {}
        if os.path.exists(cfg):
            with open(cfg) as f:
                self.config = json.load(f)
        q = self.config.get("quantization")
        if q is not None and (q.get("group_size") != GROUP_SIZE or q.get("bits") != BITS):
            raise N.HSDError(f"only affine {BITS}-bit, group {GROUP_SIZE} checkpoints are supported, got {q}")

    @property
    def layer_kinds(self):
        """Per layer "mamba" / "attention" / "moe" from hybrid_override_pattern, or None."""
        pat = self.config.get("hybrid_override_pattern")
        if pat is None:
            return None
        try:
            return [LAYER_KINDS[c] for c in pat]
        except KeyError as err:
            raise N.HSDError(f"hybrid_override_pattern: unknown layer kind {err}") from None

    @property
    def moe_layers(self):
        """Indices of the MoE layers: from the config's pattern, else every layer that has a
        routed down projection."""
        kinds = self.layer_kinds
        if kinds is not None:
            return [l for l, k in enumerate(kinds) if k == "moe"]
        out = set()
        for name in self.weight_map:
            if name.startswith("backbone.layers.") and name.endswith(".mixer.switch_mlp.fc2.weight"):
                out.add(int(name.split(".")[2]))
        return sorted(out)

    def read(self, names, device="cpu"):
        """{name: tensor} for `names`, each shard opened once; raises naming what is missing."""
        missing = [n for n in names if n not in self.weight_map]
        if missing:
            raise N.HSDError(f"{self.dir}: missing tensors {missing}")
        by_file = {}
        for n in names:
            by_file.setdefault(self.weight_map[n], []).append(n)
        out = {}
        for fn in sorted(by_file):
            with safe_open(os.path.join(self.dir, fn), framework="pt") as f:
                for n in by_file[fn]:
                    out[n] = f.get_tensor(n).to(device)
        return out

    def moe_layer(self, layer, device="cpu"):
        """test_layout_decode.py:24-35: one MoE layer's 12 quantised tensors, checked for a
        consistent 4-bit, group-64 shape set."""
        t = self.read(moe_tensor_names(layer), device)
        check_moe_shapes(t, layer, self.config)
        return t


def _expect(cond, layer, what):
    if not cond:
        raise N.HSDError(f"MoE layer {layer}: {what}")


def check_moe_shapes(t, layer, config=None):
    """Shapes and dtypes of one MoE layer's tensors (keyed as moe_tensor_names) against one
    another and, where config.json gives them, against the config. Returns (E, D, F, FS)."""
    n = moe_tensor_names(layer)
    w1, s1, b1, w2, s2, b2, su, ssu, sbu, sd, ssd, sbd = (t[k] for k in n)
    for k in (w1, w2, su, sd):
        _expect(k.dtype in (torch.uint32, torch.int32), layer, f"packed weights must be 32-bit words, got {k.dtype}")
    for k in (s1, b1, s2, b2, ssu, sbu, ssd, sbd):
        _expect(k.dtype == torch.bfloat16, layer, f"scales and biases must be bf16, got {k.dtype}")
    _expect(w2.dim() == 3 and w1.dim() == 3 and sd.dim() == 2 and su.dim() == 2, layer,
            "routed weights must be [E, rows, words] and shared ones [rows, words]")
    E, D, F = w2.shape[0], w2.shape[1], w2.shape[2] * 8
    FS = sd.shape[1] * 8
    _expect(tuple(w1.shape) == (E, F, D // 8) and D % 8 == 0, layer, f"fc1 weight {tuple(w1.shape)} vs fc2 {tuple(w2.shape)}")
    _expect(tuple(s1.shape) == tuple(b1.shape) == (E, F, D // GROUP_SIZE), layer, "fc1 scales/biases shape")
    _expect(tuple(s2.shape) == tuple(b2.shape) == (E, D, F // GROUP_SIZE), layer, "fc2 scales/biases shape")
    _expect(tuple(sd.shape) == (D, FS // 8), layer, "shared down_proj weight shape")
    _expect(tuple(su.shape) == (FS, D // 8), layer, "shared up_proj weight shape")
    _expect(tuple(ssu.shape) == tuple(sbu.shape) == (FS, D // GROUP_SIZE), layer, "shared up_proj scales/biases shape")
    _expect(tuple(ssd.shape) == tuple(sbd.shape) == (D, FS // GROUP_SIZE), layer, "shared down_proj scales/biases shape")
    cfg = config or {}
    for key, val in (("hidden_size", D), ("moe_intermediate_size", F),
                     ("moe_shared_expert_intermediate_size", FS), ("n_routed_experts", E)):
        if key in cfg:
            _expect(cfg[key] == val, layer, f"config {key}={cfg[key]} but the tensors give {val}")
    return E, D, F, FS


class MoELayer:
    """One loaded MoE layer: `down` (moe.MoEDown, the down projections and their layouts)
    and the up projections the front end reads (fc1 and the shared up_proj, stock layout)."""

    def __init__(self, layer, down, up):
        self.layer = layer
        self.down = down
        self.up = up          # dict: w1, s1, b1, sw1, ss1, sb1

    def front(self, x, inds, live_masks=None, status=None):
        """model.py:110-121 after the router: hcat = ReLU^2 of the selected experts' and
        the shared expert's up projections of x (moe.up_relu2)."""
        u = self.up
        return moe.up_relu2(x, inds, u["w1"], u["s1"], u["b1"], u["sw1"], u["ss1"], u["sb1"],
                            topk=self.down.topk, live_masks=live_masks, status=status)


def load_moe_layers(model_dir, device, *, mode="sparse", single_layout=True, layers=None, topk=None,
                    decode_kw=None, prefill_kw=None):
    """NemotronModel.__init__ + set_mode for the MoE layers (model.py:182-252): each MoE
    layer's tensors read onto `device`; in "sparse" mode its neuron-major layout is built
    right after it is read and, with single_layout, its stock down projections released
    before the next layer is read, so the transient stays one layer's down weights.
    "dense" mode keeps the stock layout only. topk defaults to the config's
    num_experts_per_tok. Returns {layer: MoELayer}."""
    if mode not in ("dense", "sparse"):
        raise N.HSDError(f"mode must be 'dense' or 'sparse', got {mode!r}")
    ck = model_dir if isinstance(model_dir, Checkpoint) else Checkpoint(model_dir)
    if topk is None:
        topk = ck.config.get("num_experts_per_tok")
        if topk is None:
            raise N.HSDError("topk: not given and config.json has no num_experts_per_tok")
    ids = ck.moe_layers if layers is None else list(layers)
    out = {}
    for l in ids:
        t = ck.moe_layer(l, device)
        n = moe_tensor_names(l)
        w1, s1, b1, w2, s2, b2, su, ssu, sbu, sd, ssd, sbd = (t.pop(k) for k in n)
        down = moe.MoEDown(dict(weight=w2, scales=s2, biases=b2), dict(weight=sd, scales=ssd, biases=sbd),
                           topk=topk, decode_kw=decode_kw, prefill_kw=prefill_kw)
        del w2, s2, b2, sd, ssd, sbd
        if mode == "sparse":
            down.build_layout(drop_stock=single_layout)
        out[l] = MoELayer(l, down, dict(w1=w1, s1=s1, b1=b1, sw1=su, ss1=ssu, sb1=sbu))
    return out
