"""The no-allocation sparse decode entry point (hsd_sparse_down_decode_noalloc) against
the workspace entry point it shares kernels with (hsd_sparse_down_decode), through the C
ABI: bit-identical outputs, live masks and status on two calls in a row (the second with
fewer rows, so its partial sums reuse the static scratch the first call filled), and the
size limit reported as an error."""
import numpy as np
import pytest
import torch

from hsd import _native as N
from hsd import layout, synth as S

pytestmark = pytest.mark.gpu
D, F, FS, TOPK = 2688, 1856, 3712, 6


@pytest.fixture(scope="module")
def layer(dev):
    lay = S.moe_layer_np(21)
    dv = {k: S.to_device(v, dev) for k, v in lay.items()}
    return layout.to_neuron_major(dv["w"], dv["s"], dv["b"]) + layout.to_neuron_major(dv["sw"], dv["ss"], dv["sb"])


def call(name, h, sel, gains, nm, B, y_dtype, dense=0, ws=None):
    y = torch.empty((B, D), dtype=y_dtype, device=h.device)
    masks = torch.zeros(B * (TOPK * F // 64 + FS // 64), dtype=torch.int64, device=h.device)
    status = torch.zeros(1, dtype=torch.int32, device=h.device)
    args = [N.ptr(h), N.dtype_tag(h.dtype), N.ptr(sel), N.ptr(gains), N.ptr(N.as_words(nm[0])), N.ptr(nm[1]),
            N.ptr(nm[2]), N.ptr(N.as_words(nm[3])), N.ptr(nm[4]), N.ptr(nm[5]), N.ptr(y), N.dtype_tag(y_dtype),
            B, D, F, FS, TOPK, nm[0].shape[0], dense, N.ptr(masks), N.ptr(status)]
    if ws is not None:
        args += [N.ptr(ws), ws.numel()]
    N.call(name, *args, N.stream(h.device))
    return y, masks, status


@pytest.mark.parametrize("y_dtype", [torch.float32, torch.bfloat16])
def test_noalloc_equals_workspace_entry(layer, dev, y_dtype):
    for i, (B, zf) in enumerate(((4, 0.9), (2, 0.7))):     # second call: fewer rows
        h, sel, gains = S.decode_inputs_np(300 + i, B=B, zero_frac=zf)
        sel[B - 1, 0] = 1000                                  # one bad id: status bit and a zero slot
        hd, seld, gd = S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev)
        ws = torch.empty(N.lib().hsd_sparse_down_workspace_bytes(B, D, F, FS, TOPK), dtype=torch.uint8, device=dev)
        ref = call("hsd_sparse_down_decode", hd, seld, gd, layer, B, y_dtype, ws=ws)
        got = call("hsd_sparse_down_decode_noalloc", hd, seld, gd, layer, B, y_dtype)
        torch.cuda.synchronize()
        print(f"call {i}: B={B} zero_frac={zf} max|y|={ref[0].float().abs().max().item():.3f}", flush=True)
        assert torch.equal(got[0].view(torch.int16) if y_dtype == torch.bfloat16 else got[0].view(torch.int32),
                           ref[0].view(torch.int16) if y_dtype == torch.bfloat16 else ref[0].view(torch.int32))
        assert torch.equal(got[1], ref[1])
        assert int(got[2].item()) == int(ref[2].item()) == N.STATUS_BAD_EXPERT


def test_noalloc_dense_control_equals_sparse(layer, dev):
    h, sel, gains = S.decode_inputs_np(310, B=3, zero_frac=0.9)
    hd, seld, gd = S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev)
    ys = call("hsd_sparse_down_decode_noalloc", hd, seld, gd, layer, 3, torch.float32)[0].clone()
    yd = call("hsd_sparse_down_decode_noalloc", hd, seld, gd, layer, 3, torch.float32, dense=1)[0]
    torch.cuda.synchronize()
    assert torch.equal(ys.view(torch.int32), yd.view(torch.int32))


def test_noalloc_rejects_rows_beyond_the_scratch(layer, dev):
    B = 13                                                   # 13 x 32 parts x 2688 x 4 B > 4 MiB
    h = torch.zeros((B, TOPK * F + FS), dtype=torch.bfloat16, device=dev)
    sel = torch.zeros((B, TOPK), dtype=torch.int32, device=dev)
    gains = torch.ones((B, TOPK + 1), dtype=torch.float32, device=dev)
    y = torch.empty((B, D), dtype=torch.float32, device=dev)
    nm = layer
    rc = N.lib().hsd_sparse_down_decode_noalloc(
        N.ptr(h), 0, N.ptr(sel), N.ptr(gains), N.ptr(N.as_words(nm[0])), N.ptr(nm[1]), N.ptr(nm[2]),
        N.ptr(N.as_words(nm[3])), N.ptr(nm[4]), N.ptr(nm[5]), N.ptr(y), 2, B, D, F, FS, TOPK, nm[0].shape[0], 0,
        None, None, N.stream(dev))
    assert rc == -2 and b"static scratch" in N.lib().hsd_last_error()


# The child process of test_noalloc_first_call_inside_graph_capture: its first
# hsd_sparse_down_decode_noalloc call (the one that looks up the device's scratch address)
# is made while a HIP graph is being captured; the graph is replayed three times with eager
# calls of the workspace entry point in between, and every replay's output must equal that
# entry point's bit for bit.
CHILD = r'''
import sys
sys.path[:0] = sys.argv[1:3]
import torch
from hsd import _native as N, layout, synth as S
dev = torch.device("cuda:0")
E, D, F, FS, K, B = 8, 256, 192, 384, 3, 3
lay = S.moe_layer_np(5, n_experts=E, d=D, f=F, fs=FS)
dv = {k: S.to_device(v, dev) for k, v in lay.items()}
nm = layout.to_neuron_major(dv["w"], dv["s"], dv["b"]) + layout.to_neuron_major(dv["sw"], dv["ss"], dv["sb"])
ins = []
for i in range(3):
    h, sel, gains = S.decode_inputs_np(40 + i, B=B, zero_frac=0.9, n_experts=E, f=F, fs=FS, topk=K)
    ins.append([S.to_device(a, dev) for a in (h, sel, gains)])
cur = [t.clone() for t in ins[0]]
y = torch.empty((B, D), dtype=torch.float32, device=dev)
ws = torch.empty(N.lib().hsd_sparse_down_workspace_bytes(B, D, F, FS, K), dtype=torch.uint8, device=dev)
def args(h, sel, gains, out):
    return [N.ptr(h), N.dtype_tag(h.dtype), N.ptr(sel), N.ptr(gains), N.ptr(N.as_words(nm[0])), N.ptr(nm[1]),
            N.ptr(nm[2]), N.ptr(N.as_words(nm[3])), N.ptr(nm[4]), N.ptr(nm[5]), N.ptr(out), N.dtype_tag(out.dtype),
            B, D, F, FS, K, E, 0, None, None]
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s):
        N.call("hsd_sparse_down_decode_noalloc", *args(*cur, y), N.stream(dev))
torch.cuda.current_stream().wait_stream(s)
for i in range(3):
    for c, t in zip(cur, ins[i]):
        c.copy_(t)
    g.replay()
    ref = torch.empty_like(y)
    N.call("hsd_sparse_down_decode", *args(*cur, ref), N.ptr(ws), ws.numel(), N.stream(dev))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32)), f"replay {i} differs"
    print(f"replay {i}: equal, max|y| {ref.abs().max().item():.4f}", flush=True)
print("ok", flush=True)
'''


def test_noalloc_first_call_inside_graph_capture(dev):
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", CHILD, root, os.path.join(root, "mlx-heimr-sparse-down_amd")],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok")
