"""The entry points inside HIP graphs: no entry allocates device memory through the HIP
API, synchronises or records a memset, so a captured call replays the eager call. Each
graph is replayed several times with eager work and synchronisations between replays,
and every replay is compared with the eager result bit for bit (the kernels are
deterministic: fixed summation orders, no float atomics)."""
import numpy as np
import pytest
import torch

from hsd import _native as N, decode, layout, mamba as M, prefill, synth as S
from hsd.moe import up_relu2

pytestmark = pytest.mark.gpu
D, F, FS, K, E = 2688, 1856, 3712, 6, 128


def capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                   # warm the allocator outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with N.capture_guard(), torch.cuda.graph(g):
        out = fn()
    return g, out


def replays(g, out, want, n=3):
    for i in range(n):
        torch.randn(1 << 20, device=want.device).sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


@pytest.fixture(scope="module")
def down(dev):
    lay = S.moe_layer_np(3)
    dv = {k: S.to_device(v, dev) for k, v in lay.items()}
    return layout.to_neuron_major(dv["w"], dv["s"], dv["b"]) + layout.to_neuron_major(dv["sw"], dv["ss"], dv["sb"])


def test_decode_graph(dev, down):
    h, sel, gains = (S.to_device(a, dev) for a in S.decode_inputs_np(21, B=1, zero_frac=0.9))
    ws = torch.empty(decode.N.lib().hsd_sparse_down_workspace_bytes(1, D, F, FS, K), dtype=torch.uint8, device=dev)
    run = lambda: decode.sparse_down(h, sel, gains, *down, F=F, FS=FS, D=D, topk=K,  # noqa: E731
                                     out_dtype=torch.float32, workspace=ws)
    want = run().clone()
    g, out = capture(run)
    replays(g, out, want)


def test_prefill_graph(dev, down):
    T = 128
    h, sel, gains = (S.to_device(a, dev) for a in S.prefill_inputs_np(22, T=T, zero_frac=0.9))

    def run():
        tiles = prefill.build_tiles(sel, E, 32)
        union = prefill.build_union(h, *tiles, F=F, FS=FS, topk=K, E=E, tt=32)
        return prefill.sparse_down_prefill(h, sel, gains, *down, F=F, FS=FS, D=D, topk=K, E=E, tt=32,
                                           tiles=tiles, union=union, out_dtype=torch.float32)
    want = run().clone()
    g, out = capture(run)
    replays(g, out, want)


def test_front_end_graph(dev):
    lay = S.moe_up_np(23)
    dv = {k: S.to_device(v, dev) for k, v in lay.items()}
    rng = np.random.default_rng(24)
    x = (torch.from_numpy(rng.standard_normal((1, D)).astype(np.float32)) * 0.5).to(torch.bfloat16).to(dev)
    sel = S.to_device(np.stack([rng.permutation(E)[:K]]).astype(np.int32), dev)
    run = lambda: up_relu2(x, sel, dv["w1"], dv["s1"], dv["b1"], dv["sw1"], dv["ss1"], dv["sb1"], topk=K)  # noqa: E731
    want = run().clone()
    g, out = capture(run)
    replays(g, out, want)


def test_mamba_verify_rollback_graph(dev):
    """A verify + rollback step captured once; K replays from a state equal K eager steps
    from the same state (the ring index and the checkpoint slabs advance on the device)."""
    p = S.mamba_params_np(25)

    def make():
        mixer = M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                              A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                              D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev))
        cache = M.MambaCache(mixer, dev, nslab=4, conv_state=S.to_device(p["conv_state"], dev),
                             ssm_state=torch.from_numpy(p["ssm_state"]).to(dev))
        return mixer, cache
    rows = S.to_device(S.mamba_rows_np(np.random.default_rng(26), 3), dev)
    keep = torch.tensor([2], dtype=torch.int32, device=dev)
    ws = torch.empty(M.N.lib().hsd_mamba_workspace_bytes(3, 64, 64), dtype=torch.uint8, device=dev)

    def step(mixer, cache):
        y = M.verify_rows(mixer, rows, cache, workspace=ws)
        M.mamba_rollback([(cache, 3)], 0, n_keep_dev=keep)
        return y

    me, ce = make()
    eager = []
    for _ in range(4):
        eager.append(step(me, ce).clone())
    torch.cuda.synchronize()
    mg, cg = make()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), N.capture_guard():
        with torch.cuda.graph(g):
            yg = step(mg, cg)      # recorded, not run: the state is still the initial one
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(4):
        torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, eager[i]), f"step {i}"
    assert torch.equal(cg.cur, ce.cur)
    assert torch.equal(cg.ssm, ce.ssm) and torch.equal(cg.conv, ce.conv)
