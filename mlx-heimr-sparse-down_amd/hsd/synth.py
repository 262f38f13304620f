"""Seeded synthetic workloads at the Nemotron-3.5-Lightning-30B-A3B shapes.

No checkpoint is available, so weights and activations are drawn from fixed
distributions:

* down projections: affine 4-bit, group 64, uniform random nibbles (uniform uint32
  words), scales ~ U(0.005, 0.02), biases ~ N(0, 0.01), bf16; STOCK layout
  (w [E, D, F/8], s/b [E, D, F/64]) -- the neuron-major layout is made on the device by
  hsd.layout;
* decode activations h = ReLU^2-like: a Bernoulli(1 - zero_frac) live mask, live values
  bf16(|N(0,1)|^2), dead values exactly +0; optional "hot neuron" variant (a fixed 5 %
  of each expert's neurons fire with p = 0.6, the rest at the rate that keeps the
  overall live fraction);
* routing: top-6 of 128 without replacement, uniform (decode) or Zipf(1.1) popularity
  over a seeded permutation of the experts (prefill); gains ~ U(0, 1), shared gain 1;
* Mamba-2: A_log = log U(1, 16), dt_bias ~ N(0, 0.5), D ~ U(0.5, 1.5), conv w/b ~
  N(0, 0.2), conv state ~ N(0, 1), ssm state ~ N(0, 0.1) fp32, per-row in_proj outputs
  ~ N(0, 1), norm weight ~ U(0.5, 1.5).

NumPy generators (`*_np`) give host arrays (bf16 as uint16 bits) that the CPU oracle and
the device see identically; `*_torch` generators draw the large benchmark tensors
directly on the device.
"""
from __future__ import annotations

import numpy as np
import torch

D, F, FS, E, TOPK, GS = 2688, 1856, 3712, 128, 6, 64
MAMBA = dict(H=64, P=64, N=128, G=8, K=4)


def bf16_bits(x):
    """float -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_values(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_device(a, device):
    """numpy -> torch on device: uint16 -> bfloat16 (bit pattern), uint32 -> int32 (bits),
    uint64 -> int64, others as is."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(device)
    if a.dtype == np.uint64:
        return torch.from_numpy(a.view(np.int64)).to(device)
    return torch.from_numpy(a).to(device)


def to_host(t):
    """Inverse of to_device: bf16 -> uint16 bits, int32 words -> uint32."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


# ----------------------------------------------------------------- MoE down proj
def down_proj_np(rng, lead, rows, cols):
    """One stock-layout 4-bit projection W[rows, cols] (rows = outputs): w [*lead, rows,
    cols/8] uint32, s / b [*lead, rows, cols/64] bf16 bits."""
    w = rng.integers(0, 2 ** 32, size=(*lead, rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    s = bf16_bits(rng.uniform(0.005, 0.02, size=(*lead, rows, cols // GS)))
    b = bf16_bits(rng.normal(0.0, 0.01, size=(*lead, rows, cols // GS)))
    return w, s, b


def moe_layer_np(seed, n_experts=E, d=D, f=F, fs=FS):
    """The stock-layout down projections of one MoE layer: routed (w, s, b) [E, D, ...]
    and shared (sw, ss, sb) [D, ...]."""
    rng = np.random.default_rng(seed)
    w, s, b = down_proj_np(rng, (n_experts,), d, f)
    sw, ss, sb = down_proj_np(rng, (), d, fs)
    return dict(w=w, s=s, b=b, sw=sw, ss=ss, sb=sb)


def proj_torch(gen, device, lead, rows, cols):
    """down_proj_np's distributions drawn on the device: w [*lead, rows, cols/8] (int32 bit
    patterns), s / b [*lead, rows, cols/64] bf16."""
    w = torch.randint(-2 ** 31, 2 ** 31, (*lead, rows, cols // 8), dtype=torch.int32,
                      device=device, generator=gen)
    s = (torch.rand((*lead, rows, cols // GS), device=device, generator=gen) * 0.015 + 0.005).to(torch.bfloat16)
    b = (torch.randn((*lead, rows, cols // GS), device=device, generator=gen) * 0.01).to(torch.bfloat16)
    return w, s, b


def moe_layer_torch(gen, device, n_experts=E, d=D, f=F, fs=FS):
    """moe_layer_np's distributions drawn on the device (benchmark scale: 364.8 MB per
    layer). Words are int32 bit patterns."""
    w, s, b = proj_torch(gen, device, (n_experts,), d, f)
    sw, ss, sb = proj_torch(gen, device, (), d, fs)
    return dict(w=w, s=s, b=b, sw=sw, ss=ss, sb=sb)


def moe_up_np(seed, n_experts=E, d=D, f=F, fs=FS):
    """The stock-layout up projections of one MoE layer (rows = outputs): routed (w1, s1,
    b1) [E, F, ...] over D inputs, shared (sw1, ss1, sb1) [FS, ...]."""
    rng = np.random.default_rng(seed)
    w1, s1, b1 = down_proj_np(rng, (n_experts,), f, d)
    sw1, ss1, sb1 = down_proj_np(rng, (), fs, d)
    return dict(w1=w1, s1=s1, b1=b1, sw1=sw1, ss1=ss1, sb1=sb1)


def moe_up_torch(gen, device, n_experts=E, d=D, f=F, fs=FS):
    """moe_up_np's distributions drawn on the device (int32 words)."""
    w1, s1, b1 = proj_torch(gen, device, (n_experts,), f, d)
    sw1, ss1, sb1 = proj_torch(gen, device, (), fs, d)
    return dict(w1=w1, s1=s1, b1=b1, sw1=sw1, ss1=ss1, sb1=sb1)


def write_checkpoint(model_dir, seed, *, pattern="MEME", n_experts=E, d=D, f=F, fs=FS, topk=TOPK,
                     shards=2):
    """A synthetic MLX-format checkpoint of random 4-bit MoE layers: config.json, the
    shard files and model.safetensors.index.json (shards > 1) or one model.safetensors,
    with the names hsd.checkpoint reads. Layers marked "E" in `pattern` get a MoE layer
    (moe_layer_np + moe_up_np, seeds seed + 2l and seed + 2l + 1); other layers get one
    small placeholder tensor each. Returns {layer: {"down": moe_layer_np dict, "up":
    moe_up_np dict}} (host arrays, bf16 as uint16 bits)."""
    import json
    import os
    from safetensors.torch import save_file

    def tens(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
        return torch.from_numpy(a)

    os.makedirs(model_dir, exist_ok=True)
    tensors, arrays = {}, {}
    for l, kind in enumerate(pattern):
        p = f"backbone.layers.{l}.mixer"
        if kind != "E":
            tensors[f"{p}.placeholder"] = torch.zeros(4, dtype=torch.float32)
            continue
        dn = moe_layer_np(seed + 2 * l, n_experts, d, f, fs)
        up = moe_up_np(seed + 2 * l + 1, n_experts, d, f, fs)
        arrays[l] = dict(down=dn, up=up)
        for k, (wk, sk, bk), src in (("switch_mlp.fc1", ("w1", "s1", "b1"), up),
                                     ("switch_mlp.fc2", ("w", "s", "b"), dn),
                                     ("shared_experts.up_proj", ("sw1", "ss1", "sb1"), up),
                                     ("shared_experts.down_proj", ("sw", "ss", "sb"), dn)):
            tensors[f"{p}.{k}.weight"] = tens(src[wk])
            tensors[f"{p}.{k}.scales"] = tens(src[sk])
            tensors[f"{p}.{k}.biases"] = tens(src[bk])
    names = sorted(tensors)
    if shards <= 1:
        save_file(tensors, os.path.join(model_dir, "model.safetensors"), metadata={"format": "mlx"})
    else:
        wmap = {}
        for i in range(shards):
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            part = {n: tensors[n] for n in names[i::shards]}
            save_file(part, os.path.join(model_dir, fn), metadata={"format": "mlx"})
            wmap.update({n: fn for n in part})
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as fh:
            json.dump({"metadata": {}, "weight_map": wmap}, fh)
    cfg = dict(hidden_size=d, moe_intermediate_size=f, moe_shared_expert_intermediate_size=fs,
               n_routed_experts=n_experts, num_experts_per_tok=topk, hybrid_override_pattern=pattern,
               quantization=dict(group_size=GS, bits=4))
    with open(os.path.join(model_dir, "config.json"), "w") as fh:
        json.dump(cfg, fh)
    return arrays


def live_mask_np(rng, shape, zero_frac, hot=None):
    """Bernoulli(1 - zero_frac) live mask; `hot` = (hot_mask [.., width], p_hot, p_cold)
    gives per-neuron rates instead."""
    if hot is None:
        return rng.random(shape) >= zero_frac
    hot_mask, p_hot, p_cold = hot
    p = np.where(hot_mask, p_hot, p_cold)
    return rng.random(shape) < p


def hot_cold_rates(zero_frac, hot_frac=0.05, p_hot=0.6):
    """p_cold so that hot_frac*p_hot + (1-hot_frac)*p_cold = 1 - zero_frac."""
    return p_hot, max(0.0, ((1.0 - zero_frac) - hot_frac * p_hot) / (1.0 - hot_frac))


def relu2_values_np(rng, live):
    """bf16(|N(0,1)|^2) where live, exact +0 elsewhere -> uint16 bits."""
    v = np.abs(rng.standard_normal(live.shape)).astype(np.float32) ** 2
    v = np.where(live, v, np.float32(0.0))
    return bf16_bits(v)


def decode_inputs_np(seed, B=1, zero_frac=0.9, n_experts=E, f=F, fs=FS, topk=TOPK, hot=None):
    """hcat [B, topk*F + FS] (bf16 bits), sel [B, topk] int32 (distinct, uniform), gains
    [B, topk+1] f32 (U(0, 1), then 1.0 for the shared expert)."""
    rng = np.random.default_rng(seed)
    sel = np.stack([rng.permutation(n_experts)[:topk] for _ in range(B)]).astype(np.int32)
    gains = np.concatenate([rng.uniform(0, 1, size=(B, topk)), np.ones((B, 1))], axis=1).astype(np.float32)
    live = live_mask_np(rng, (B, topk * f + fs), zero_frac, hot)
    return relu2_values_np(rng, live), sel, gains


def zipf_sel_np(rng, T, n_experts=E, topk=TOPK, a=1.1):
    """T tokens x topk distinct experts, p(expert) proportional to rank^-a over a seeded
    permutation of the experts."""
    perm = rng.permutation(n_experts)
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -a
    p /= p.sum()
    sel = np.empty((T, topk), dtype=np.int32)
    for t in range(T):
        sel[t] = perm[rng.choice(n_experts, size=topk, replace=False, p=p)]
    return sel


def prefill_inputs_np(seed, T=512, zero_frac=0.9, n_experts=E, f=F, fs=FS, topk=TOPK, zipf=1.1):
    rng = np.random.default_rng(seed)
    sel = zipf_sel_np(rng, T, n_experts, topk, zipf) if zipf else \
        np.stack([rng.permutation(n_experts)[:topk] for _ in range(T)]).astype(np.int32)
    gains = np.concatenate([rng.uniform(0, 1, size=(T, topk)), np.ones((T, 1))], axis=1).astype(np.float32)
    live = live_mask_np(rng, (T, topk * f + fs), zero_frac)
    return relu2_values_np(rng, live), sel, gains


# ----------------------------------------------------------------- Mamba-2
def mamba_params_np(seed, H=64, P=64, N=128, G=8, K=4):
    rng = np.random.default_rng(seed)
    DI = H * P
    CD = DI + 2 * G * N
    return dict(
        A_log=np.log(rng.uniform(1, 16, size=H)).astype(np.float32),
        dt_bias=rng.normal(0, 0.5, size=H).astype(np.float32),
        D=rng.uniform(0.5, 1.5, size=H).astype(np.float32),
        conv_w=bf16_bits(rng.normal(0, 0.2, size=(CD, K))),
        conv_b=bf16_bits(rng.normal(0, 0.2, size=CD)),
        norm_w=bf16_bits(rng.uniform(0.5, 1.5, size=DI)),
        conv_state=bf16_bits(rng.normal(0, 1, size=(K - 1, CD))),
        ssm_state=rng.normal(0, 0.1, size=(H, P, N)).astype(np.float32),
    )


def mamba_rows_np(rng, L, H=64, P=64, N=128, G=8):
    """L rows of the in_proj output (gate | conv input | dt) as bf16 bits."""
    DI = H * P
    CD = DI + 2 * G * N
    return bf16_bits(rng.standard_normal((L, DI + CD + H)))
