"""GPU parity of the layout permutation (hsd/layout.py:34-74): bit-exact against the
oracle on the reference's test shapes (tests/test_layout_decode.py:59) and the real
layer shapes, self-inverse on the device, scales/biases moved bit for bit."""
import numpy as np
import pytest
import torch

from hsd import layout, synth as S
from oracle import hsd_oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(5, 24, 9), (2688, 232), (1856, 336), (3712, 336), (3, 2688, 232), (2688, 464), (8, 7)]


@pytest.mark.parametrize("shape", SHAPES)
def test_nibble_transpose_bit_exact_and_self_inverse(dev, shape):
    rng = np.random.default_rng(sum(shape))
    w = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint64).astype(np.uint32)
    wd = S.to_device(w, dev)
    t = layout.nibble_transpose(wd)
    assert tuple(t.shape) == (*shape[:-2], shape[-1] * 8, shape[-2] // 8)
    assert np.array_equal(S.to_host(t).view(np.uint32), O.nibble_transpose(w))
    back = layout.nibble_transpose(t)
    assert torch.equal(back, wd)


def test_to_neuron_major_full_layer(dev):
    """All 128 routed experts + the shared expert of one layer at the real shape; the
    oracle checks a sample of experts, the device checks self-inverse on all."""
    lay = S.moe_layer_np(100)
    w, s, b = (S.to_device(lay[k], dev) for k in ("w", "s", "b"))
    pw, ps, pb = layout.to_neuron_major(w, s, b)
    assert tuple(pw.shape) == (128, 1856, 336) and tuple(ps.shape) == (128, 29, 2688)
    for e in (0, 77, 127):
        assert np.array_equal(S.to_host(pw[e]).view(np.uint32), O.nibble_transpose(lay["w"][e]))
        assert np.array_equal(S.to_host(ps[e]), lay["s"][e].T)
        assert np.array_equal(S.to_host(pb[e]), lay["b"][e].T)
    assert torch.equal(layout.nibble_transpose(pw), w)
    assert torch.equal(layout.transpose_last2(ps), s)
    sw = S.to_device(lay["sw"], dev)
    spw, sps, spb = layout.to_neuron_major(sw, S.to_device(lay["ss"], dev), S.to_device(lay["sb"], dev))
    assert np.array_equal(S.to_host(spw).view(np.uint32), O.nibble_transpose(lay["sw"]))
    assert np.array_equal(S.to_host(sps), lay["ss"].T)
