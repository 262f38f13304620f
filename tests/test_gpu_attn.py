"""GPU parity of hsd_attn_decode: GQA attention (32 query / 2 kv heads, head_dim 128) of
B <= 4 rows over a KV cache whose length lives on the device (mlx-lm's attention block
with KVCache as hsd's decode and verify steps run it, model.py:287, 343, 355).

Bars: the bf16 output within |o - ref| <= 2e-2 + 1e-2 |ref| of the float64 oracle (keys
0 .. P+r per row); the new rows' keys/values are in the cache bit for bit; a B-row call
equals B single-row calls at consecutive positions bit for bit; a cache that would
overflow writes zeros and sets the status bit."""
import math

import numpy as np
import pytest
import torch

from hsd import nn, synth as S
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu
HQ, HKV, HD, SMAX = 32, 2, 128, 4096
QKV = (HQ + 2 * HKV) * HD
SCALE = 1.0 / math.sqrt(HD)


def setup(dev, seed, P, B, smax=SMAX, hkv=HKV):
    rng = np.random.default_rng(seed)
    cache = nn.KVCache(hkv, smax, dev)
    kc = O.f32_to_bf16(rng.standard_normal((hkv, smax, HD)).astype(np.float32))
    vc = O.f32_to_bf16(rng.standard_normal((hkv, smax, HD)).astype(np.float32))
    cache.k.copy_(S.to_device(kc, dev))
    cache.v.copy_(S.to_device(vc, dev))
    qkv = O.f32_to_bf16(rng.standard_normal((B, (HQ + 2 * hkv) * HD)).astype(np.float32) * 2)
    pos = torch.tensor([P], dtype=torch.int32, device=dev)
    return cache, kc, vc, qkv, pos


def oracle_rows(kc, vc, qkv, P, hkv=HKV):
    B = qkv.shape[0]
    k = O.bf16_to_f32(kc).copy()
    v = O.bf16_to_f32(vc).copy()
    q = O.bf16_to_f32(qkv)
    out = np.zeros((B, HQ * HD))
    for r in range(B):
        k[:, P + r] = q[r, HQ * HD:(HQ + hkv) * HD].reshape(hkv, HD)
        v[:, P + r] = q[r, (HQ + hkv) * HD:].reshape(hkv, HD)
        out[r] = O.attention(q[r, :HQ * HD].reshape(HQ, HD), k[:, :P + r + 1], v[:, :P + r + 1], SCALE).reshape(-1)
    return out, k, v


@pytest.mark.parametrize("P,B,smax", [(0, 1, SMAX), (0, 3, SMAX), (5, 1, SMAX), (63, 3, SMAX), (64, 2, SMAX),
                                      (2047, 3, SMAX), (2300, 4, SMAX), (4094, 3, 8192),
                                      (5000, 3, 8192), (8190, 2, 8192)])
def test_attention_matches_oracle(dev, P, B, smax):
    """Contexts past 2048 keys (more than 64 chunks of 32) take the combine's second
    load phase; P = 4094, B = 3 puts the third row's last key (4096) first in its chunk."""
    cache, kc, vc, qkv, pos = setup(dev, 100 + P + B, P, B, smax)
    out = nn.attention(S.to_device(qkv, dev), cache, pos, n_heads=HQ, n_kv_heads=HKV)
    ref, k, v = oracle_rows(kc, vc, qkv, P)
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    print(f"P={P} B={B}: max err {err.max():.3e}")
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref))
    # the new rows are in the cache bit for bit; the rest is untouched
    kh, vh = O.bf16_to_f32(S.to_host(cache.k)), O.bf16_to_f32(S.to_host(cache.v))
    assert np.array_equal(kh[:, :P + B], k[:, :P + B]) and np.array_equal(vh[:, :P + B], v[:, :P + B])
    assert np.array_equal(kh[:, P + B:], O.bf16_to_f32(kc)[:, P + B:])


@pytest.mark.parametrize("P,smax", [(0, SMAX), (62, SMAX), (700, SMAX), (4094, 8192), (6143, 8192)])
def test_verify_rows_equal_single_rows(dev, P, smax):
    cache, kc, vc, qkv, pos = setup(dev, 200 + P, P, 3, smax)
    qd = S.to_device(qkv, dev)
    out3 = nn.attention(qd, cache, pos, n_heads=HQ, n_kv_heads=HKV)
    cache1, _, _, _, pos1 = setup(dev, 200 + P, P, 3, smax)
    for r in range(3):
        o1 = nn.attention(qd[r:r + 1], cache1, pos1, n_heads=HQ, n_kv_heads=HKV)
        assert torch.equal(o1.view(torch.int16), out3[r:r + 1].view(torch.int16)), f"row {r}"
        pos1 += 1
    assert torch.equal(cache1.k.view(torch.int16), cache.k.view(torch.int16))


@pytest.mark.parametrize("hkv", [4, 8])
def test_other_head_ratios(dev, hkv):
    """8 and 4 query heads per kv head (the workgroups then hold 8 or 4 heads): against
    the oracle, and a 3-row call equal to single rows."""
    P = 1000
    cache, kc, vc, qkv, pos = setup(dev, 400 + hkv, P, 3, hkv=hkv)
    qd = S.to_device(qkv, dev)
    out = nn.attention(qd, cache, pos, n_heads=HQ, n_kv_heads=hkv)
    ref, _, _ = oracle_rows(kc, vc, qkv, P, hkv=hkv)
    assert np.all(np.abs(out.float().cpu().numpy() - ref) <= 2e-2 + 1e-2 * np.abs(ref))
    cache1, _, _, _, pos1 = setup(dev, 400 + hkv, P, 3, hkv=hkv)
    for r in range(3):
        o1 = nn.attention(qd[r:r + 1], cache1, pos1, n_heads=HQ, n_kv_heads=hkv)
        assert torch.equal(o1.view(torch.int16), out[r:r + 1].view(torch.int16)), f"row {r}"
        pos1 += 1


def test_full_cache_is_refused_on_device(dev):
    cache, kc, vc, qkv, pos = setup(dev, 300, SMAX - 2, 3)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    out = nn.attention(S.to_device(qkv, dev), cache, pos, n_heads=HQ, n_kv_heads=HKV, status=status)
    assert int(status.item()) == 2
    assert not out.float().abs().sum().item()
    assert torch.equal(cache.k.view(torch.int16), S.to_device(kc, dev).view(torch.int16))
