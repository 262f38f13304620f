"""Host logic of the MoE block's down-projection surface (hsd/model.py:89-139): pack's
layout (model.py:123-129: routed slots then the shared expert, gains = scores then 1)
against its closed form, and the mode guards. CPU tensors only: no kernel runs here."""
import numpy as np
import pytest
import torch

from hsd import _native as N
from hsd.moe import MoEDown, build_layouts

E, D, F, FS, K = 8, 256, 128, 192, 2


def block():
    w = torch.zeros((E, D, F // 8), dtype=torch.int32)
    s = torch.zeros((E, D, F // 64), dtype=torch.int16)
    sw = torch.zeros((D, FS // 8), dtype=torch.int32)
    ss = torch.zeros((D, FS // 64), dtype=torch.int16)
    return MoEDown(dict(weight=w, scales=s, biases=s.clone()), dict(weight=sw, scales=ss, biases=ss.clone()),
                   topk=K)


def test_shapes_from_stock_layout():
    b = block()
    assert (b.E, b.D, b.F, b.FS, b.topk) == (E, D, F, FS, K)
    assert b.stock_layout and not b.has_layout


def test_pack_matches_closed_form():
    rng = np.random.default_rng(3)
    B = 3
    h = torch.from_numpy(rng.standard_normal((B, K, 1, F)).astype(np.float32)).to(torch.bfloat16)
    hs = torch.from_numpy(rng.standard_normal((B, FS)).astype(np.float32)).to(torch.bfloat16)
    inds = torch.from_numpy(rng.integers(0, E, (B, K)))
    scores = torch.from_numpy(rng.uniform(0, 1, (B, K)).astype(np.float64))
    hcat, sel, gains = block().pack(inds, scores, h, hs)
    want = np.concatenate([h.float().numpy().reshape(B, K * F), hs.float().numpy()], axis=1)
    assert hcat.dtype == torch.bfloat16 and hcat.shape == (B, K * F + FS)
    assert np.array_equal(hcat.float().numpy(), want)
    # slot k of token b at [k F, (k+1) F), the shared expert after the routed slots
    assert np.array_equal(hcat[1, F:2 * F].float().numpy(), h[1, 1, 0].float().numpy())
    assert sel.dtype == torch.int32 and np.array_equal(sel.numpy(), inds.numpy())
    assert gains.dtype == torch.float32 and gains.shape == (B, K + 1)
    assert np.array_equal(gains[:, :K].numpy(), scores.numpy().astype(np.float32))
    assert np.all(gains[:, K].numpy() == 1.0)


def test_pack_rejects_wrong_shapes():
    with pytest.raises(N.HSDError):
        block().pack(torch.zeros((1, K), dtype=torch.int64), torch.zeros((1, K)),
                     torch.zeros((1, K, F + 1)), torch.zeros((1, FS)))


def test_sparse_mode_needs_the_layout():
    b = block()
    x = torch.zeros((1, D))
    with pytest.raises(N.HSDError, match="build_layout"):
        b.decode_sparse(x, torch.zeros((1, K), dtype=torch.int64), torch.zeros((1, K)),
                        torch.zeros((1, K, F)), torch.zeros((1, FS)))


def test_dense_mode_needs_the_stock_layout():
    b = block()
    b.drop_stock()
    assert not b.stock_layout and b.fc2 is None
    with pytest.raises(N.HSDError, match="dense mode"):
        b.decode_dense(torch.zeros((1, D)), torch.zeros((1, K), dtype=torch.int64), torch.zeros((1, K)),
                       torch.zeros((1, K, F)), torch.zeros((1, FS)))
    with pytest.raises(N.HSDError, match="dropped"):
        b.build_layout()


def test_build_layouts_skips_built_blocks():
    class Done:
        has_layout = True

        def build_layout(self, drop_stock=True):
            raise AssertionError("not rebuilt")
    assert len(build_layouts([Done(), Done()])) == 2
