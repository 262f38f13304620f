"""Benchmark of the hsd hot path on one MI355X.

Default (python bench.py [--steps K --warmup W]): one JSON line whose headline is the
end-to-end workload -- batch-1 greedy decode of a random-init Nemotron-H hybrid at the
Nemotron-3.5-Lightning-30B-A3B shape (52 layers: 23 Mamba-2, 23 MoE with 128 experts top-6
and the 4-bit neuron-major down projection, 6 GQA attention; vocab 131072; 4-bit g64; the
one-layer MTP head), a 2048-token seeded random prompt, then 256 tokens: `value` is the
decode tok/s of sparse down + MTP-2 with scripted acceptance at a mean of 1.26 accepted
drafts; dense down, sparse down and the 1.68 acceptance are reported beside it, with the
check that all four produce the same greedy tokens. A step is one speculative step
(the head's two drafts, the 3-row verify through the 52 layers, the acceptance and the
rollback), replayed from one captured graph; inputs and weights are resident in HBM.

`roofline` is the sparse down projection's (the hot path of the metric), from the 23-layer
decode sweep; `workloads` holds the decode sweep, the prefill grouped GEMM, the MTP
verify + rollback over 23 Mamba-2 layers and the MoE front end, each with its roofline and
its CPU baseline (the NumPy oracle on the host cores, a bounded sample).

--workload e2e|decode|prefill|mtp|up|proj prints one of them alone (proj: the step's projections
and attention, each alone; calib: the counter calibration copy); --workload step --mode
mtp|sparse|dense replays one captured step of the model (for per-kernel profiles).
"""
from __future__ import annotations

import argparse
import math
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-heimr-sparse-down_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from hsd import decode, layout, mamba as M, model as Mdl, moe, mtp, prefill, synth as S  # noqa: E402
from hsd import _native as N  # noqa: E402

METRIC = "batch-1 decode tok/s (sparse+MTP2); sparse-down HBM GB/s vs peak"
DECODE_METRIC = "sparse down projection, 23 MoE layers, batch 1: HBM GB/s on touched bytes"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.txt")


def pmc_traffic(workload):
    """HBM bytes per dispatch of a workload's kernel(s), from the committed rocprofv3 counter
    summary: FETCH_SIZE x fetch_factor + WRITE_SIZE x write_factor (KiB per dispatch, factors
    from a device copy of known size). None when the summary or its line is absent."""
    try:
        lines = open(TRAFFIC_SUMMARY).read().splitlines()
    except OSError:
        return None
    fields = {}
    for ln in lines:
        tok = ln.split()
        if tok[:1] == ["calibration"]:
            fields["cal"] = dict(t.split("=", 1) for t in tok[1:])
        elif tok[:2] == ["traffic", workload]:
            fields["kib"] = dict(t.split("=", 1) for t in tok[2:])
    if "cal" not in fields or "kib" not in fields:
        return None
    cal, kib = fields["cal"], fields["kib"]
    return int(1024 * (float(kib["fetch_kib"]) * float(cal["fetch_factor"])
                       + float(kib["write_kib"]) * float(cal["write_factor"])))
def pmc_mfma_util(kernel):
    """The kernel's matrix-core utilisation (MFMA busy cycles over SIMD cycles of the
    dispatch) from the committed counter summary, or None."""
    try:
        for ln in open(os.path.join(ROOT, "profiles", "mfma_utilisation.txt")):
            tok = ln.split()
            if tok[:2] == ["mfma", kernel]:
                return float(tok[2].split("=", 1)[1])
    except OSError:
        pass
    return None


NL = 23                      # MoE layers
D, F, FS, E, K = S.D, S.F, S.FS, S.E, S.TOPK
NR = K * F + FS


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_info():
    model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(cpu_count=os.cpu_count(), affinity=len(os.sched_getaffinity(0)), cpu_model=model,
                omp_threads=os.environ.get("OMP_NUM_THREADS"))


# ------------------------------------------------------------------ decode
def touched_bytes_dev(h):
    """bench/common.py:16-19, 78-83 byte model on the device: h [..., NR] ->
    [...] int64 bytes (live rows x D/2 + live groups x 4D + I/O)."""
    live = (h != 0)
    rows = live.sum(-1)
    groups = live.view(*h.shape[:-1], NR // 64, 64).any(-1).sum(-1)
    io = NR * 2 + K * 4 + (K + 1) * 4 + D * 2
    return rows.to(torch.int64) * (D // 2) + groups.to(torch.int64) * (4 * D) + io


def dense_bytes():
    return NR * (D // 2) + (NR // 64) * 4 * D + NR * 2 + K * 4 + (K + 1) * 4 + D * 2


def make_layers(dev, seed, keep_stock):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    layers, permute_ms, permute_bytes = [], 0.0, 0
    for l in range(NL):
        st = S.moe_layer_torch(gen, dev)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        nm = layout.to_neuron_major(st["w"], st["s"], st["b"]) + layout.to_neuron_major(st["sw"], st["ss"], st["sb"])
        e1.record()
        torch.cuda.synchronize()
        permute_ms += e0.elapsed_time(e1)
        permute_bytes += 2 * sum(t.numel() * t.element_size() for t in nm)
        layers.append(dict(nm=nm, stock=st if keep_stock else None))
        if not keep_stock:
            del st
    return layers, permute_ms, permute_bytes


def make_decode_inputs(dev, seed, ntok, zero_frac, hot=False):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if hot:
        p_hot, p_cold = S.hot_cold_rates(zero_frac)
        hot_mask = torch.rand((NL, E, F), device=dev, generator=gen) < 0.05
        hot_sh = torch.rand((NL, FS), device=dev, generator=gen) < 0.05
    sel = torch.stack([torch.stack([torch.randperm(E, device=dev, generator=gen)[:K] for _ in range(NL)])
                       for _ in range(ntok)]).to(torch.int32)                        # [ntok, NL, K]
    gains = torch.cat([torch.rand((ntok, NL, K), device=dev, generator=gen),
                       torch.ones((ntok, NL, 1), device=dev)], dim=-1).float()
    u = torch.rand((ntok, NL, NR), device=dev, generator=gen)
    if hot:
        hm = torch.cat([hot_mask[torch.arange(NL, device=dev)[None, :, None], sel.long()].reshape(ntok, NL, K * F),
                        hot_sh[None].expand(ntok, NL, FS)], dim=-1)
        live = u < torch.where(hm, torch.tensor(p_hot, device=dev), torch.tensor(p_cold, device=dev))
    else:
        live = u >= zero_frac
    v = torch.randn((ntok, NL, NR), device=dev, generator=gen) ** 2
    h = torch.where(live, v, torch.zeros_like(v)).to(torch.bfloat16)
    return h.contiguous(), sel.contiguous(), gains.contiguous()


def capture_steps(fn_layer, ntok):
    """One HIP graph per token: the 23 layer calls of a decode step."""
    graphs = []
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for t in range(min(2, ntok)):          # warm the allocator outside capture
            for l in range(NL):
                fn_layer(t, l)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for t in range(ntok):
        g = torch.cuda.CUDAGraph()
        with N.capture_guard(), torch.cuda.graph(g):
            for l in range(NL):
                fn_layer(t, l)
        graphs.append(g)
    torch.cuda.synchronize()
    return graphs


def time_graphs(graphs, steps, warmup):
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def time_graphs_cold(graphs, steps, flush):
    """Per step: overwrite a flush buffer larger than the 256 MB Infinity Cache, then time
    only the step's graph with events."""
    tot = 0.0
    for i in range(steps):
        flush.fill_(float(i))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graphs[i % len(graphs)].replay()
        e1.record()
        torch.cuda.synchronize()
        tot += e0.elapsed_time(e1)
    return tot


def launch_floors(dev, nbytes, ntok, steps, warm):
    """What one call cannot beat on this machine, timed like the calls (graphs of NL
    back-to-back launches, ntok graphs rotated): a one-element fill (the launch floor), and
    a copy of the call's algorithmic byte count from a pool larger than the 256 MB Infinity
    Cache (one launch streaming that many bytes from HBM, plus the same written back)."""
    tiny = torch.zeros(1, device=dev)
    n4 = max(nbytes // 4, 64)
    pool = torch.ones((ntok, NL, n4), dtype=torch.float32, device=dev)
    dst = torch.empty(n4, dtype=torch.float32, device=dev)
    g_fill = capture_steps(lambda t, l: tiny.fill_(float(l)), ntok)
    us_fill = 1e3 * time_graphs(g_fill, steps, warm) / (steps * NL)
    g_copy = capture_steps(lambda t, l: dst.copy_(pool[t, l]), ntok)
    us_copy = 1e3 * time_graphs(g_copy, steps, warm) / (steps * NL)
    del g_fill, g_copy, pool
    return dict(empty_launch_us=round(us_fill, 3), two_launch_us=round(2 * us_fill, 3),
                stream_copy_us=round(us_copy, 3), stream_copy_bytes=int(4 * n4),
                note="a call of two dependent launches cannot beat two_launch_us; stream_copy_us is one "
                     "launch reading the call's byte count from HBM and writing it back")


def cpu_baseline_decode(layers, h, sel, gains, budget_s=15.0):
    """The oracle (NumPy, float64 accumulation) on host cores over a bounded sample of the
    same workload: token-layers in order until ~budget_s of CPU time."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    done_bytes, cpu_s, n = 0, 0.0, 0
    ntok = h.shape[0]
    t = 0
    while cpu_s < budget_s and t < ntok:
        for l in range(NL):
            nm = layers[l]["nm"]
            s_h = sel[t, l].cpu().numpy()
            pw = {int(e): S.to_host(nm[0][int(e)]).view(np.uint32) for e in s_h}
            ps = {int(e): S.to_host(nm[1][int(e)]) for e in s_h}
            pb = {int(e): S.to_host(nm[2][int(e)]) for e in s_h}
            hv = h[t, l].float().cpu().numpy()[None]
            g = gains[t, l].cpu().numpy()[None]
            spw, sps, spb = (S.to_host(x) for x in nm[3:6])
            spw = spw.view(np.uint32)
            idx = np.arange(K, dtype=np.int32)[None]
            pwa = np.stack([pw[int(e)] for e in s_h])
            psa = np.stack([ps[int(e)] for e in s_h])
            pba = np.stack([pb[int(e)] for e in s_h])
            t0 = time.perf_counter()
            O.sparse_down(hv, idx, g, pwa, psa, pba, spw, sps, spb, F=F, FS=FS, D=D, topk=K)
            cpu_s += time.perf_counter() - t0
            done_bytes += int(touched_bytes_dev(h[t, l]).item())
            n += 1
            if cpu_s >= budget_s:
                break
        t += 1
    info = cpu_info()
    return dict(value=round(done_bytes / cpu_s / 1e9, 4), unit="GB/s", cores=info["affinity"], kind="port",
                sample=f"{n} token-layers of the same workload (NumPy oracle sparse_down, float64 accumulate)",
                ms_per_token_layer=round(1e3 * cpu_s / n, 3), **{k: v for k, v in info.items()})


def cpu_baseline_decode_formula(layers, h, sel, gains, budget_s=8.0):
    """The reference's own formula on host cores (test_layout_decode.py:128-142): the 7
    selected stock-layout matrices dequantised in full, then the mat-vecs (the oracle's
    float64 dense_reference), over token-layers in order until ~budget_s."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    cpu_s, n, done_bytes = 0.0, 0, 0
    t = 0
    while cpu_s < budget_s and t < h.shape[0]:
        for l in range(NL):
            st = layers[l]["stock"]
            s_h = sel[t, l].cpu().numpy()
            w = np.stack([S.to_host(st["w"][int(e)]).view(np.uint32) for e in s_h])
            sc = np.stack([S.to_host(st["s"][int(e)]) for e in s_h])
            bi = np.stack([S.to_host(st["b"][int(e)]) for e in s_h])
            sw, ss, sb = S.to_host(st["sw"]).view(np.uint32), S.to_host(st["ss"]), S.to_host(st["sb"])
            hv = h[t, l].float().cpu().numpy()[None]
            g = gains[t, l].cpu().numpy()[None]
            idx = np.arange(K, dtype=np.int32)[None]
            t0 = time.perf_counter()
            O.dense_reference(hv, idx, g, w, sc, bi, sw, ss, sb, F=F, FS=FS, D=D, topk=K)
            cpu_s += time.perf_counter() - t0
            done_bytes += int(touched_bytes_dev(h[t, l]).item())
            n += 1
            if cpu_s >= budget_s:
                break
        t += 1
    return dict(value=round(done_bytes / cpu_s / 1e9, 4), unit="GB/s (touched bytes)",
                ms_per_token_layer=round(1e3 * cpu_s / n, 3),
                sample=f"{n} token-layers: full dequantisation of the 7 selected matrices + mat-vec (float64)")


def bench_decode(args):
    dev = torch.device("cuda:0")
    log(f"[decode] building {NL} MoE layers (stock 4-bit, permuting to neuron-major on device)")
    layers, perm_ms, perm_bytes = make_layers(dev, args.seed, keep_stock=not args.no_dense)
    log(f"[decode] layout permute: {perm_ms:.1f} ms for {NL} layers ({perm_bytes / perm_ms / 1e6:.0f} GB/s r+w)")
    ntok = args.ntok
    h, sel, gains = make_decode_inputs(dev, args.seed + 1, ntok, args.zero_frac, hot=args.hot)
    tb = touched_bytes_dev(h)                                                      # [ntok, NL]
    ws = [torch.empty(N.lib().hsd_sparse_down_workspace_bytes(1, D, F, FS, K), dtype=torch.uint8, device=dev)
          for _ in range(NL)]
    kw = dict(F=F, FS=FS, D=D, topk=K)

    def sparse_layer(t, l, dense=False):
        return decode.sparse_down(h[t, l:l + 1], sel[t, l:l + 1], gains[t, l:l + 1],
                                  *layers[l]["nm"], dense=dense, workspace=ws[l], **kw)

    log(f"[decode] capturing {ntok} token graphs x {NL} layers")
    graphs = capture_steps(sparse_layer, ntok)
    steps, warm = args.steps, args.warmup
    ms = time_graphs(graphs, steps, warm)
    idx = torch.arange(steps, device=dev) % ntok
    bytes_timed = int(tb[idx].sum().item())
    gbs = bytes_timed / (ms * 1e-3) / 1e9
    ms_step = ms / steps
    per_launch_bytes = bytes_timed / (steps * NL)
    per_launch_us = 1e3 * ms / (steps * NL)
    log(f"[decode] sparse: {ms_step * 1e3:.1f} us/token (23 layers), {gbs:.0f} GB/s touched, "
        f"{per_launch_bytes / 1e6:.2f} MB/layer")
    extra = {}
    floor = launch_floors(dev, int(per_launch_bytes), ntok, steps, warm)
    log(f"[decode] floors: empty launch {floor['empty_launch_us']:.2f} us, one-launch copy of "
        f"{per_launch_bytes / 1e6:.2f} MB {floor['stream_copy_us']:.2f} us; the call: {per_launch_us:.2f} us")
    # dense-h control: the same kernel reading every row
    if not args.no_control:
        graphs_dh = capture_steps(lambda t, l: sparse_layer(t, l, dense=True), min(ntok, 8))
        ms_dh = time_graphs(graphs_dh, steps, warm)
        extra["dense_h_control"] = dict(us_per_token=round(1e3 * ms_dh / steps, 2),
                                        gbs=round(dense_bytes() * NL * steps / (ms_dh * 1e-3) / 1e9, 1))
        del graphs_dh
    if not args.no_dense:
        def dense_layer(t, l):
            st = layers[l]["stock"]
            return decode.dense_down(h[t, l][None], sel[t, l][None], gains[t, l][None], st["w"], st["s"], st["b"],
                                     st["sw"], st["ss"], st["sb"], **kw)
        graphs_d = capture_steps(dense_layer, min(ntok, 8))
        ms_d = time_graphs(graphs_d, steps, warm)
        extra["dense_4bit_stock"] = dict(us_per_token=round(1e3 * ms_d / steps, 2),
                                         gbs=round(dense_bytes() * NL * steps / (ms_d * 1e-3) / 1e9, 1),
                                         speedup_sparse_vs_dense=round(ms_d / ms, 3))
        del graphs_d
        log(f"[decode] dense 4-bit (stock layout): {1e3 * ms_d / steps:.1f} us/token; sparse speedup {ms_d / ms:.2f}x")
    sweep = batch_sweep(args, dev, layers, kw) if args.batch_sweep else []
    if sweep:
        extra["batch_sweep"] = sweep
    if args.cold:
        flush = torch.empty(1 << 28, dtype=torch.float32, device=dev)                 # 1 GiB
        ncold = min(steps, 64)
        ms_c = time_graphs_cold(graphs, ncold, flush)
        bc = int(tb[torch.arange(ncold, device=dev) % ntok].sum().item())
        extra["cold"] = dict(us_per_token=round(1e3 * ms_c / ncold, 2), gbs=round(bc / (ms_c * 1e-3) / 1e9, 1),
                             note="1 GiB flush written between tokens, outside the timed interval")
        log(f"[decode] cold: {1e3 * ms_c / ncold:.1f} us/token, {bc / (ms_c * 1e-3) / 1e9:.0f} GB/s")
        del flush
    cpu = cpu_baseline_decode(layers, h, sel, gains, budget_s=args.cpu_budget) if args.cpu_budget > 0 else None
    if cpu is not None and not args.no_dense:
        cpu["reference_formula"] = cpu_baseline_decode_formula(layers, h, sel, gains, budget_s=args.cpu_budget / 2)
    achieved = per_launch_bytes / (per_launch_us * 1e-6) / 1e9
    rec = dict(metric=DECODE_METRIC, value=round(gbs, 2), unit="GB/s", n_gpus=1, steps=steps, warmup=warm,
               ms_per_step=round(ms_step, 5), higher_is_better=True, scaling="weak", vs_baseline=None,
               dtype="f32 (4-bit weights, bf16 scales/activations)", data="synthetic",
               config=dict(workload="decode sweep: 23 MoE layers, batch 1, sparse 4-bit down projection",
                           zero_frac=args.zero_frac, hot_neurons=bool(args.hot), experts=E, topk=K, D=D, F=F,
                           FS=FS, group=64, tokens_rotated=ntok, weights_gb=round(NL * 364.8e6 / 1e9, 2)),
               roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                             frac=round(achieved / HBM_PEAK_GBS, 4), traffic=pmc_traffic("decode"),
                             kernel="k_sparse_down_part + k_sum_parts (one decode call)",
                             bytes_per_launch=int(per_launch_bytes), us_per_launch=round(per_launch_us, 3),
                             floor=floor),
               cpu_baseline=cpu,
               down_proj_tok_s=round(1e3 / ms_step, 1),
               layout_permute=dict(ms_23_layers=round(perm_ms, 2), gbs_rw=round(perm_bytes / perm_ms / 1e6, 1)),
               **extra)
    return rec


def batch_sweep(args, dev, layers, kw, ntok=8):
    """The same 23-layer sparse down projection with B token rows per call (B independent
    tokens, each with its own experts and activations: several sequences decoded at once),
    timed like the batch-1 sweep (graphs of 23 calls, ntok graphs rotated). Bytes are the
    per-row byte model summed over the rows (the rows' experts and live rows differ; the
    shared expert's scales are counted once per row)."""
    out = []
    steps, warm = max(20, args.steps // 2), args.warmup
    for B in [int(v) for v in args.batch_sweep.split(",") if v]:
        hb, sb, gb = make_decode_inputs(dev, args.seed + 101 + B, ntok * B, args.zero_frac)
        hb = hb.view(ntok, B, NL, NR).transpose(1, 2).contiguous()            # [ntok, NL, B, NR]
        sb = sb.view(ntok, B, NL, K).transpose(1, 2).contiguous()
        gb = gb.view(ntok, B, NL, K + 1).transpose(1, 2).contiguous()
        tbb = touched_bytes_dev(hb).sum(-1)                                   # [ntok, NL]
        wsb = [torch.empty(N.lib().hsd_sparse_down_workspace_bytes(B, D, F, FS, K), dtype=torch.uint8, device=dev)
               for _ in range(NL)]
        graphs = capture_steps(lambda t, l: decode.sparse_down(hb[t, l], sb[t, l], gb[t, l], *layers[l]["nm"],
                                                               workspace=wsb[l], **kw), ntok)
        ms = time_graphs(graphs, steps, warm)
        nbytes = int(tbb[torch.arange(steps, device=dev) % ntok].sum().item())
        us_call = 1e3 * ms / (steps * NL)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append(dict(rows=B, us_per_call=round(us_call, 3), mb_per_call=round(nbytes / (steps * NL) / 1e6, 2),
                        gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4)))
        log(f"[decode] {B} rows per call: {us_call:.2f} us, {nbytes / (steps * NL) / 1e6:.1f} MB, {gbs:.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")
        del graphs, hb, sb, gb, wsb
    return out


# ------------------------------------------------------------------ prefill
def cpu_baseline_prefill(layers, chunks, args, tokens=32):
    """The oracle's grouped matmul (sparse_down_prefill: per tile, the union rows
    dequantised, float64) on host cores for the first `tokens` tokens of the first chunk of
    layer 0 (the same tile order and unions), as algorithmic TFLOP/s."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    l, h, sel, gains = chunks[0]
    hh = S.to_host(h[:tokens])
    ss, gg = sel[:tokens].cpu().numpy(), gains[:tokens].cpu().numpy()
    nm = layers[l]["nm"]
    used = sorted(set(int(e) for e in ss.reshape(-1)))
    pw = np.zeros((E, F, D // 8), np.uint32)
    ps = np.zeros((E, F // 64, D), np.uint16)
    pb = np.zeros((E, F // 64, D), np.uint16)
    for e in used:
        pw[e] = S.to_host(nm[0][e]).view(np.uint32)
        ps[e] = S.to_host(nm[1][e])
        pb[e] = S.to_host(nm[2][e])
    spw, sps, spb = S.to_host(nm[3]).view(np.uint32), S.to_host(nm[4]), S.to_host(nm[5])
    te, ts = O.build_tiles(ss, E, args.tt)
    ul, uc = O.build_union(O.bf16_to_f32(hh), te, ts, F=F, FS=FS, topk=K, E=E, tt=args.tt)
    nvalid = (ts.reshape(-1, args.tt) >= 0).sum(1)
    flops = int((2 * D * nvalid.astype(np.int64) * uc.astype(np.int64)).sum())
    t0 = time.perf_counter()
    O.sparse_down_prefill(O.bf16_to_f32(hh), ss, gg, pw, ps, pb, spw, sps, spb, F=F, FS=FS, D=D, topk=K, E=E,
                          tt=args.tt, tiles=(te, ts), union=(ul, uc))
    sec = time.perf_counter() - t0
    info = cpu_info()
    return dict(value=round(flops / sec / 1e12, 6), unit="TFLOP/s", cores=info["affinity"], kind="port",
                sample=f"{tokens} tokens of one 512-token chunk of one layer (NumPy oracle grouped matmul over the "
                       f"union rows, float64)", seconds=round(sec, 3), **info)


def bench_prefill(args):
    dev = torch.device("cuda:0")
    nl = args.layers
    T, chunk, tt = 2048, 512, args.tt
    log(f"[prefill] {nl} layers, T={T} in chunks of {chunk}, tt={tt}")
    layers, _, _ = make_layers(dev, args.seed, keep_stock=False) if nl == NL else (None, 0, 0)
    if layers is None:
        gen = torch.Generator(device=dev)
        gen.manual_seed(args.seed)
        layers = []
        for l in range(nl):
            st = S.moe_layer_torch(gen, dev)
            layers.append(dict(nm=layout.to_neuron_major(st["w"], st["s"], st["b"]) +
                               layout.to_neuron_major(st["sw"], st["ss"], st["sb"])))
            del st
    chunks = []
    for l in range(nl):
        for c in range(T // chunk):
            h, sel, gains = S.prefill_inputs_np(args.seed + 1000 * l + c, T=chunk, zero_frac=args.zero_frac)
            chunks.append((l, S.to_device(h, dev), S.to_device(sel, dev), S.to_device(gains, dev)))
    # algorithmic FLOPs from the device's own union counts
    flops, ws = 0, None
    prep = []
    for (l, h, sel, gains) in chunks:
        te, ts = prefill.build_tiles(sel, E, tt)
        ul, uc = prefill.build_union(h, te, ts, F=F, FS=FS, topk=K, E=E, tt=tt)
        nvalid = (ts.view(-1, tt) >= 0).sum(1)
        flops += int((2 * D * nvalid.long() * uc.long()).sum().item())
        prep.append((te, ts, ul, uc))
    ws = torch.empty(N.lib().hsd_prefill_gemm_workspace_bytes(chunk, D, F, FS, K, E, tt), dtype=torch.uint8,
                     device=dev)

    def run(i, with_tiles):
        l, h, sel, gains = chunks[i]
        te, ts, ul, uc = prep[i]
        if with_tiles:
            return prefill.sparse_down_prefill(h, sel, gains, *layers[l]["nm"], F=F, FS=FS, D=D, topk=K, E=E,
                                               tt=tt, workspace=ws)
        return prefill.sparse_down_prefill(h, sel, gains, *layers[l]["nm"], F=F, FS=FS, D=D, topk=K, E=E, tt=tt,
                                           tiles=(te, ts), union=(ul, uc), workspace=ws)

    for i in range(len(chunks)):
        run(i, True)
    torch.cuda.synchronize()
    res = {}
    for with_tiles in (False, True):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for rep in range(args.steps):
            for i in range(len(chunks)):
                run(i, with_tiles)
        e1.record()
        torch.cuda.synchronize()
        res[with_tiles] = e0.elapsed_time(e1) / args.steps
    ms_gemm, ms_all = res[False], res[True]
    tflops = flops / (ms_gemm * 1e-3) / 1e12
    wbytes = nl * 364.8e6 * (T // chunk)
    log(f"[prefill] grouped GEMM {ms_gemm:.2f} ms per prompt ({tflops:.1f} TFLOP/s algorithmic); with tiles+union "
        f"{ms_all:.2f} ms -> {T / (ms_all * 1e-3):.0f} tok/s")
    cpu = cpu_baseline_prefill(layers, chunks, args) if args.cpu_budget > 0 else None
    return dict(metric="prefill down-projection TFLOP/s (bf16 MFMA, algorithmic union FLOPs)",
                value=round(tflops, 2), unit="TFLOP/s", n_gpus=1, steps=args.steps, warmup=1,
                ms_per_step=round(ms_all, 4), higher_is_better=True, scaling="weak", vs_baseline=None,
                dtype="bf16 MFMA, f32 accumulate", data="synthetic",
                config=dict(workload="prefill: 2048-token prompt in chunks of 512, Zipf(1.1) top-6 routing",
                            layers=nl, tt=tt, zero_frac=args.zero_frac),
                roofline=dict(bound="mfma", achieved=round(tflops, 2), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                              frac=round(tflops / BF16_PEAK_TFLOPS, 4), traffic=pmc_traffic("prefill"),
                              hbm_frac_dense_weights=round(wbytes / (ms_gemm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              mfma_busy_frac=pmc_mfma_util("k_gemm"),
                              mfma_busy_note="k_gemm's MFMA busy cycles over its SIMD cycles, from rocprofv3 "
                                             "counters (profiles/mfma_utilisation.txt)"),
                cpu_baseline=cpu,
                prefill_tok_s=round(T / (ms_all * 1e-3), 1), gflop_per_prompt=round(flops / 1e9, 2))


# ------------------------------------------------------------------ MTP verify
def cpu_baseline_mtp(args, per_layer, layers=4):
    """The oracle's sequential Mamba-2 recurrence (mamba_verify: conv, SSM over 3 rows with
    every row's state kept, gated norm; float64) on host cores for `layers` layer-steps, as
    GB/s over the same byte model."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    rng = np.random.default_rng(args.seed)
    DI, CD = 4096, 6144
    sec = 0.0
    for l in range(layers):
        p = S.mamba_params_np(args.seed + l)
        r = O.bf16_to_f32(S.mamba_rows_np(rng, 3))
        t0 = time.perf_counter()
        O.mamba_verify(r[:, DI:DI + CD], r[:, DI + CD:], r[:, :DI], O.bf16_to_f32(p["conv_w"]),
                       O.bf16_to_f32(p["conv_b"]), p["A_log"], p["dt_bias"], p["D"], O.bf16_to_f32(p["norm_w"]),
                       O.bf16_to_f32(p["conv_state"]), p["ssm_state"])
        sec += time.perf_counter() - t0
    info = cpu_info()
    return dict(value=round(per_layer * layers / sec / 1e9, 4), unit="GB/s", cores=info["affinity"], kind="port",
                sample=f"{layers} layer-steps of 3 rows (NumPy oracle recurrence, float64)",
                ms_per_layer_step=round(1e3 * sec / layers, 2), **info)


def mamba_layer_bytes(cfg, L):
    """Algorithmic bytes of one Mamba-2 layer-step of L rows. "ssm": the conv + SSM update
    as the model runs it (hsd_mamba_ssm_gated): the fp32 state read once and written once
    per row (the checkpoints), the conv window read and L checkpoints written, the conv
    weights, the L rows' conv inputs, dt and gate read and z with its sums of squares
    written. "block": that plus in_proj and out_proj (4-bit weights once, RMS norm and
    gated-norm weights) and the residual row read and written."""
    D, H, P, N_, G = cfg.hidden, cfg.mamba_heads, cfg.mamba_head_dim, cfg.ssm_state, cfg.n_groups
    DI, CD = cfg.mamba_inner, cfg.conv_dim
    state = H * P * N_ * 4
    ssm = (state + L * state + 3 * CD * 2 + L * 3 * CD * 2 + CD * 5 * 2 + 3 * H * 4
           + L * (CD + H + DI) * 2 + L * (DI + DI // 16) * 4)
    block = ssm + _q4(cfg.in_proj_dim, D) + _q4(D, DI) + 2 * D + 2 * DI + 2 * L * D * 2
    return dict(ssm=ssm, block=block)


def bench_mtp(args):
    """MTP verify + rollback over 23 Mamba-2 layers on the model's own path: each step runs
    3 rows through every layer's block (in_proj with the RMS norm fused, the conv + SSM
    update with the gate applied and every row's state checkpointed, out_proj with the
    gated norm and the residual fused), then rolls the shared ring index back to the
    scripted number of kept rows, P(0, 1, 2 drafts accepted) = (0.15, 0.35, 0.50). The
    headline is the conv + SSM part (hsd_mamba_ssm_gated, the verify the survey's byte
    model counts); the whole block is timed beside it."""
    dev = torch.device("cuda:0")
    cfg = Mdl.ModelConfig()
    init = Mdl._Init(args.seed, dev)
    blocks = [Mdl.MambaBlock(cfg, init) for _ in range(NL)]
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    caches = []
    for l, b in enumerate(blocks):
        p = S.mamba_params_np(args.seed + l)
        caches.append(M.MambaCache(b.mixer, dev, nslab=Mdl.NSLAB, cur=cur, conv_state=S.to_device(p["conv_state"], dev),
                                   ssm_state=torch.from_numpy(p["ssm_state"]).to(dev)))
    L, nsteps, D = 3, 64, cfg.hidden
    rng = np.random.default_rng(args.seed)
    xs = [S.to_device(S.bf16_bits(rng.standard_normal((L, D))), dev) for _ in range(nsteps)]
    projs = [S.to_device(S.mamba_rows_np(rng, L), dev) for _ in range(NL)]
    accepts = mtp.scripted_accepts(nsteps, (0.15, 0.35, 0.50), args.seed)
    nkeep = torch.tensor(accepts + 1, dtype=torch.int32, device=dev)
    buf = dict(proj=torch.zeros((L, cfg.in_proj_dim), dtype=torch.bfloat16, device=dev),
               y_pre=torch.zeros((L, cfg.mamba_inner + cfg.mamba_inner // 16), dtype=torch.float32, device=dev))
    st = N.stream(dev)

    def rollback(i):
        N.call("hsd_mamba_select_row", N.ptr(cur), N.ptr(nkeep[i:i + 1]), 0, L, Mdl.NSLAB, None, st)

    def step_block(i):
        for l in range(NL):
            blocks[l].rows(xs[i], buf, caches[l])
        rollback(i)

    def step_ssm(i):
        for l in range(NL):
            M.ssm_rows(blocks[l].mixer, projs[l], caches[l], out=buf["y_pre"], gated=True)
        rollback(i)

    def capture(fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn(0)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gs = []
        for i in range(nsteps):
            g = torch.cuda.CUDAGraph()
            with N.capture_guard(), torch.cuda.graph(g):
                fn(i)
            gs.append(g)
        return gs

    g_ssm = capture(step_ssm)
    ms = time_graphs(g_ssm, args.steps, args.warmup)
    del g_ssm
    g_blk = capture(step_block)
    ms_blk = time_graphs(g_blk, args.steps, args.warmup)
    del g_blk
    lb = mamba_layer_bytes(cfg, L)
    gbs = lb["ssm"] * NL * args.steps / (ms * 1e-3) / 1e9
    gbs_blk = lb["block"] * NL * args.steps / (ms_blk * 1e-3) / 1e9
    us, us_blk = 1e3 * ms / args.steps, 1e3 * ms_blk / args.steps
    log(f"[mtp] verify(3)+rollback, 23 Mamba-2 layers: conv + SSM (hsd_mamba_ssm_gated) {us:.1f} us/step, "
        f"{gbs:.0f} GB/s; whole block (in_proj, conv + SSM, out_proj) {us_blk:.1f} us/step, {gbs_blk:.0f} GB/s")
    cpu = cpu_baseline_mtp(args, lb["ssm"]) if args.cpu_budget > 0 else None
    roof_us = lb["ssm"] * NL / HBM_PEAK_GBS / 1e3
    return dict(metric="MTP-2 verify + rollback, 23 Mamba-2 layers (conv + SSM update): HBM GB/s", value=round(gbs, 2),
                unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup, ms_per_step=round(ms / args.steps, 5),
                higher_is_better=True, scaling="weak", vs_baseline=None, dtype="f32 state, bf16 I/O",
                data="synthetic",
                config=dict(workload="MTP verify + rollback: 23 Mamba-2 layers (64 heads x 64, state 128, 8 groups, "
                                     "conv 4), 3 rows per step, P(0,1,2)=(.15,.35,.5); the model's path "
                                     "(hsd_mamba_ssm_gated; the whole block beside it)"),
                roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                              frac=round(gbs / HBM_PEAK_GBS, 4), traffic=pmc_traffic("mtp"),
                              bytes_per_layer_step=lb["ssm"], us_per_step=round(us, 2),
                              roof_us_per_step=round(roof_us, 2)),
                block=dict(us_per_step=round(us_blk, 2), gbs=round(gbs_blk, 1),
                           frac=round(gbs_blk / HBM_PEAK_GBS, 4), bytes_per_layer_step=lb["block"],
                           traffic_per_layer_step=pmc_traffic("mtp_block"),
                           roof_us_per_step=round(lb["block"] * NL / HBM_PEAK_GBS / 1e3, 2),
                           note="in_proj (RMS norm fused) + hsd_mamba_ssm_gated + out_proj (gated norm and "
                                "residual fused), 23 layers, then the rollback"),
                cpu_baseline=cpu)


# ------------------------------------------------------------------ MoE front end
def cpu_baseline_up(ups, x, sel, per_call, calls=3):
    """The oracle's front end (up_relu2: the 7 up projections dequantised, float64, then
    ReLU^2 in bf16) on host cores for `calls` token-layers, as GB/s over the same bytes."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    sec = 0.0
    for c in range(calls):
        u = ups[c]
        s_h = sel[c, c].cpu().numpy()
        w1 = np.stack([S.to_host(u["w1"][int(e)]).view(np.uint32) for e in s_h])
        s1 = np.stack([S.to_host(u["s1"][int(e)]) for e in s_h])
        b1 = np.stack([S.to_host(u["b1"][int(e)]) for e in s_h])
        sw1, ss1, sb1 = S.to_host(u["sw1"]).view(np.uint32), S.to_host(u["ss1"]), S.to_host(u["sb1"])
        xb = S.to_host(x[c, c:c + 1])
        t0 = time.perf_counter()
        O.up_relu2(xb, np.arange(K, dtype=np.int32)[None], w1, s1, b1, sw1, ss1, sb1, F=F, FS=FS, topk=K)
        sec += time.perf_counter() - t0
    info = cpu_info()
    return dict(value=round(per_call * calls / sec / 1e9, 4), unit="GB/s", cores=info["affinity"], kind="port",
                sample=f"{calls} token-layers (NumPy oracle up projections + ReLU^2, float64)",
                ms_per_token_layer=round(1e3 * sec / calls, 2), **info)


def bench_up(args):
    dev = torch.device("cuda:0")
    nl = args.layers
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 7)
    ups = [S.moe_up_torch(gen, dev) for _ in range(nl)]
    downs, _, _ = make_layers(dev, args.seed, keep_stock=False)
    ntok = args.ntok
    x = (torch.randn((ntok, nl, D), device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    sel = torch.stack([torch.stack([torch.randperm(E, device=dev, generator=gen)[:K] for _ in range(nl)])
                       for _ in range(ntok)]).to(torch.int32)
    gains = torch.cat([torch.rand((ntok, nl, K), device=dev, generator=gen),
                       torch.ones((ntok, nl, 1), device=dev)], dim=-1).float()
    hbuf = [None] * nl
    ws = [torch.empty(N.lib().hsd_sparse_down_workspace_bytes(1, D, F, FS, K), dtype=torch.uint8, device=dev)
          for _ in range(nl)]

    def up_layer(t, l):
        u = ups[l]
        hbuf[l] = moe.up_relu2(x[t, l:l + 1], sel[t, l:l + 1], u["w1"], u["s1"], u["b1"], u["sw1"], u["ss1"],
                               u["sb1"], topk=K)

    def chain_layer(t, l):
        up_layer(t, l)
        decode.sparse_down(hbuf[l], sel[t, l:l + 1], gains[t, l:l + 1], *downs[l]["nm"], F=F, FS=FS, D=D, topk=K,
                           workspace=ws[l])

    graphs = capture_steps(up_layer, ntok) if nl == NL else None
    if graphs is None:
        raise SystemExit("--workload up times all 23 layers")
    ms = time_graphs(graphs, args.steps, args.warmup)
    per_call = NR * (D // 2 + 4 * (D // 64)) + D * 2 + NR * 2 + K * 4
    gbs = per_call * nl * args.steps / (ms * 1e-3) / 1e9
    del graphs
    cgraphs = capture_steps(chain_layer, ntok)
    cms = time_graphs(cgraphs, args.steps, args.warmup)
    log(f"[up] front end (up projections + ReLU^2), 23 layers: {1e3 * ms / args.steps:.1f} us/token, "
        f"{gbs:.0f} GB/s over {per_call / 1e6:.2f} MB/layer")
    log(f"[up] front end + sparse down, 23 layers: {1e3 * cms / args.steps:.1f} us/token")
    cpu = cpu_baseline_up(ups, x, sel, per_call) if args.cpu_budget > 0 else None
    return dict(metric="MoE front end (4-bit up projections + ReLU^2), batch 1, 23 layers: HBM GB/s",
                value=round(gbs, 2), unit="GB/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
                ms_per_step=round(ms / args.steps, 5), higher_is_better=True, scaling="weak", vs_baseline=None,
                dtype="bf16 x, 4-bit weights, f32 accumulate (bf16 dot2)", data="synthetic",
                config=dict(workload="MoE front end after the router: 6 routed + shared up projections, ReLU^2, "
                                     "batch 1, 23 layers", experts=E, topk=K, D=D, F=F, FS=FS,
                            tokens_rotated=ntok),
                roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                              frac=round(gbs / HBM_PEAK_GBS, 4), traffic=pmc_traffic("up"),
                              kernel="k_moe_up", bytes_per_launch=per_call,
                              us_per_launch=round(1e3 * ms / args.steps / nl, 3)),
                cpu_baseline=cpu,
                front_plus_down_us_per_token=round(1e3 * cms / args.steps, 2))


# ------------------------------------------------------------------ end to end
def _host_block_weights(model, l):
    """Block l's weights as host arrays in the oracle's conventions."""
    u32 = lambda t: S.to_host(t).view(np.uint32)
    t, blk = model.cfg.pattern[l], model.blocks[l]
    if t == "M":
        m = blk.mixer
        return dict(norm_w=S.to_host(blk.norm_w), in_w=u32(blk.in_proj.w), in_s=S.to_host(blk.in_proj.scales),
                    in_b=S.to_host(blk.in_proj.biases), out_w=u32(blk.out_proj.w), out_s=S.to_host(blk.out_proj.scales),
                    out_b=S.to_host(blk.out_proj.biases), conv_w=m.conv_w.float().cpu().numpy(),
                    conv_b=m.conv_b.float().cpu().numpy(), A_log=m.A_log.cpu().numpy(),
                    dt_bias=m.dt_bias.cpu().numpy(), D=m.D.cpu().numpy(), gnorm_w=S.to_host(m.norm_w))
    if t == "*":
        return dict(norm_w=S.to_host(blk.norm_w), qkv_w=u32(blk.qkv.w), qkv_s=S.to_host(blk.qkv.scales),
                    qkv_b=S.to_host(blk.qkv.biases), o_w=u32(blk.o_proj.w), o_s=S.to_host(blk.o_proj.scales),
                    o_b=S.to_host(blk.o_proj.biases))
    return dict(norm_w=S.to_host(blk.norm_w), gate=S.to_host(blk.gate.w), e_bias=blk.e_bias.cpu().numpy(),
                w1=u32(blk.w1), s1=S.to_host(blk.s1), b1=S.to_host(blk.b1), sw1=u32(blk.sw1), ss1=S.to_host(blk.ss1),
                sb1=S.to_host(blk.sb1), pw=u32(blk.pw), ps=S.to_host(blk.ps), pb=S.to_host(blk.pb), spw=u32(blk.spw),
                sps=S.to_host(blk.sps), spb=S.to_host(blk.spb))


def cpu_baseline_e2e(model, sess, lm_rows=8192):
    """The oracle's decode step on host cores, sampled: one decode row through one Mamba-2,
    one MoE and one attention block (the attention over the session's cached keys) and
    lm_head over `lm_rows` of its rows, each timed, then scaled to the 52-layer step
    (23 / 23 / 6 blocks, the whole vocabulary) -> tok/s."""
    sys.path.insert(0, ROOT)
    from oracle import hsd_oracle as O
    c = model.cfg
    pat = c.pattern
    seq = sess.state()
    P, cur = seq[N.SEQ_POS], seq[N.SEQ_CUR]
    E_ = model.embedding
    x = O.embed_q4(np.array([seq[N.SEQ_TOK]]), S.to_host(E_.w).view(np.uint32), S.to_host(E_.scales),
                   S.to_host(E_.biases))[0]
    t = {}
    for kind in "ME*":
        l = pat.index(kind)
        w = _host_block_weights(model, l)
        lc = sess.cache.layers[l]
        t0 = time.perf_counter()
        if kind == "M":
            O.mamba_block_step(x, w, lc.conv[cur].float().cpu().numpy(), lc.ssm[cur].cpu().numpy(),
                               n_groups=c.n_groups, eps=c.eps)
        elif kind == "*":
            k = lc.k[:, :P].float().cpu().numpy()
            v = lc.v[:, :P].float().cpu().numpy()
            t0 = time.perf_counter()
            O.attn_block_step(x, w, k, v, n_heads=c.attn_heads, n_kv_heads=c.kv_heads, eps=c.eps)
        else:
            O.moe_block_step(x, w, topk=c.topk, routed_scale=c.routed_scale, eps=c.eps)
        t[kind] = time.perf_counter() - t0
        del w
    lw = S.to_host(model.lm_head.w[:lm_rows]).view(np.uint32)
    t0 = time.perf_counter()
    O.lm_head_logits(x, S.to_host(model.norm_f), lw, S.to_host(model.lm_head.scales[:lm_rows]),
                     S.to_host(model.lm_head.biases[:lm_rows]), c.eps)
    t_lm = (time.perf_counter() - t0) * c.vocab / lm_rows
    per_tok = pat.count("M") * t["M"] + pat.count("E") * t["E"] + pat.count("*") * t["*"] + t_lm
    info = cpu_info()
    return dict(value=round(1.0 / per_tok, 5), unit="tok/s", cores=info["affinity"], kind="port",
                sample=f"one decode row through one Mamba-2, one MoE and one attention block (keys 0..{P}) and "
                       f"{lm_rows} lm_head rows with the NumPy oracle (float64), scaled to the 52-layer step",
                seconds_per_token=round(per_tok, 3),
                block_seconds=dict(mamba=round(t["M"], 4), moe=round(t["E"], 4), attention=round(t["*"], 4),
                                   lm_head=round(t_lm, 4)), **info)


def graph_node_counts(model, fn):
    """Node types of one captured step (a capture of fn() that is counted and dropped,
    never replayed): {"kernel": launches per step, ...} from hipGraphGetNodes /
    hipGraphNodeGetType on the HIP runtime torch has loaded."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")
    g = model._capture(fn, keep_graph=True)
    raw = ctypes.c_void_p(g.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(raw, None, ctypes.byref(n)) != 0:
        return None
    nodes = (ctypes.c_void_p * n.value)()
    if hip.hipGraphGetNodes(raw, nodes, ctypes.byref(n)) != 0:
        return None
    names = {0: "kernel", 1: "memcpy", 2: "memset", 5: "empty"}
    out = {}
    for nd in nodes:
        t = ctypes.c_int(-1)
        hip.hipGraphNodeGetType(ctypes.c_void_p(nd), ctypes.byref(t))
        k = names.get(t.value, f"type{t.value}")
        out[k] = out.get(k, 0) + 1
    del g
    return out


def empty_launch_us(dev, n, reps=50):
    """One graph of n back-to-back one-element fills (the launch floor of an n-kernel
    step, timed like the steps: the graph replayed reps times) -> us per launch."""
    tiny = torch.zeros(1, device=dev)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s), N.capture_guard():
        tiny.fill_(0.0)
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                tiny.fill_(float(i))
    torch.cuda.current_stream(dev).wait_stream(s)
    ms = time_graphs([g], reps, 5)
    del g
    return 1e3 * ms / (reps * n)


def _q4(O, I):
    """Bytes of a 4-bit group-64 projection: nibbles plus bf16 scale and bias per group."""
    return O * I // 2 + O * (I // 64) * 4


def pass_bytes(cfg, B, P, z):
    """Algorithmic HBM bytes of one pass of B token rows (positions P .. P+B-1) through the
    52 layers, by block kind: every weight byte the pass needs once, the Mamba states read
    once and written once per row (the checkpoints), the attention keys and values of the
    prefix read once and the rows' own written, and the MoE experts the rows select
    (routed experts: the expected number of distinct ones among B rows' top-k; down
    projection: live rows x D/2 + live 64-groups x 4D at zero fraction z, the shared
    expert's rows counted once per live row of any row). Activations between kernels are
    not counted (they are KB)."""
    D, H, Pd, Ns, G = cfg.hidden, cfg.mamba_heads, cfg.mamba_head_dim, cfg.ssm_state, cfg.n_groups
    CD, DI = cfg.conv_dim, cfg.mamba_inner
    E, k, F, FS = cfg.n_experts, cfg.topk, cfg.moe_inter, cfg.shared_inter
    state = H * Pd * Ns * 4
    mamba = (_q4(cfg.in_proj_dim, D) + _q4(D, DI) + 2 * D + 2 * DI + CD * 5 * 2 + 3 * H * 4
             + state + B * state + 3 * CD * 2 + B * 3 * CD * 2)
    d = E * (1.0 - (1.0 - k / E) ** B)                          # distinct routed experts
    up = d * _q4(F, D) + _q4(FS, D)
    live_g = 1.0 - z ** 64
    down = (D // 2) * (B * k * F * (1.0 - z) + FS * (1.0 - z ** B)) + 4 * D * live_g * (d * F // 64 + FS // 64)
    moe = E * D * 2 + 2 * D + E * 4 + up + down
    kv = cfg.kv_heads * cfg.head_dim * 2
    attn = _q4(cfg.qkv_dim, D) + _q4(D, cfg.attn_heads * cfg.head_dim) + 2 * D + 2 * kv * P + 2 * kv * B
    pat = cfg.pattern
    return dict(mamba=pat.count("M") * mamba, moe=pat.count("E") * moe, attention=pat.count("*") * attn)


def step_bytes(cfg, kind, P, z):
    """Algorithmic bytes of one captured step at cache length P, by part. kind "decode":
    the embedding row, the 52 layers at one row, lm_head (norm_f fused). kind "mtp": the
    head's call over the three rows the last verify confirmed (eh_proj, its attention and
    MoE blocks) and lm_head on the draft row, the chained call at one row with lm_head
    again, then the 3-row verify through the 52 layers and lm_head at three rows: lm_head's
    198 MB are read three times, as three dependent passes (each needs the previous one's
    argmax)."""
    D, V = cfg.hidden, cfg.vocab
    lm = _q4(V, D) + 2 * D
    emb_row = D // 2 + (D // 64) * 4
    out = {}
    if kind == "decode":
        out.update(pass_bytes(cfg, 1, P, z))
        out["embedding"] = emb_row
        out["lm_head"] = lm
    else:
        p3 = pass_bytes(cfg, 3, P, z)
        out.update(p3)
        cfg1 = Mdl.ModelConfig(**{**cfg.__dict__, "pattern": "*E"})
        h3, h1 = pass_bytes(cfg1, 3, P, z), pass_bytes(cfg1, 1, P, z)
        eh = 2 * D * D * 2 + 2 * 2 * D
        out["mtp_head"] = h3["attention"] + h3["moe"] + h1["attention"] + h1["moe"] + 2 * eh
        out["embedding"] = 7 * emb_row                        # the head's 3 + 1 rows, the verify's 3
        out["lm_head"] = 3 * lm
    out["total"] = sum(out.values())
    return out


def e2e_roofline(model, kind, ms_per_step, P, launches, launch_us):
    z = float(np.mean(model.zero_frac_measured))
    b = step_bytes(model.cfg, kind, P, z)
    gbs = b["total"] / (ms_per_step * 1e-3) / 1e9
    floor_ms = launches * launch_us * 1e-3 if launches else None
    return dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4),
                traffic=None, bytes_per_step=int(b["total"]),
                bytes_by_part={k: int(v) for k, v in b.items() if k != "total"},
                ms_per_step=ms_per_step, roof_ms_per_step=round(b["total"] / HBM_PEAK_GBS / 1e9 * 1e3, 4),
                cache_len=int(P), moe_zero_frac=round(z, 4), launches_per_step=launches,
                empty_launch_us=round(launch_us, 3),
                launch_floor_ms=None if floor_ms is None else round(floor_ms, 4),
                launch_floor_frac_of_step=None if floor_ms is None else round(floor_ms / ms_per_step, 4),
                note="bytes: every weight byte the step needs once (lm_head once per dependent pass), Mamba "
                     "states read and checkpoints written, the attention prefix read, the selected experts' "
                     "up rows and the down projection's live rows and groups; launch floor: the step's kernel "
                     "launches (graph nodes) x the measured launch time of an empty kernel in a graph")


def bench_e2e(args):
    dev = torch.device("cuda:0")
    cfg = Mdl.ModelConfig()
    t0 = time.time()
    model = Mdl.NemotronModel(cfg, mode="sparse", seed=args.seed)
    torch.cuda.synchronize()
    init_s = time.time() - t0
    log(f"[e2e] model: {len(cfg.pattern)} layers + MTP head, {model.nbytes() / 1e9:.2f} GB, built and calibrated "
        f"in {init_s:.1f} s; MoE zero fractions {min(model.zero_frac_measured):.3f}..{max(model.zero_frac_measured):.3f}")
    prompt = np.random.default_rng(args.seed + 11).integers(0, cfg.vocab, args.prompt).astype(np.int32)
    T, G, W = len(prompt), args.gen, max(args.warmup, 0)
    # out_tokens room for the warm-up and timed steps of an MTP run (up to 3 tokens each)
    cap = max(G, 1 + 3 * (W + max(args.steps, 0))) + 8
    runs, nodes = {}, {}

    def finish(s, n_to):
        """Untimed steps after the timed window until n_to tokens are emitted."""
        while s.emitted() < n_to:
            s.step(1)

    def plain(mode):
        model.set_mode(mode)
        s = model.session(prompt, cap=cap)
        s.step(W)
        n0 = s.emitted()
        k = args.steps if args.steps > 0 else max(G - n0, 1)
        sec = s.step(k)
        n1 = s.emitted()
        finish(s, G)
        r = dict(tok_s=round((n1 - n0) / sec, 2), ms_per_token=round(1e3 * sec / k, 4), steps=k, warmup=W,
                 timed_tokens=[n0, n1], cache_len_mid=T + (n0 + n1) // 2,
                 generation_tok_s=round((s.emitted() - 1) / s.decode_s, 2), generation_tokens=s.emitted(),
                 prompt_tok_s=round(T / s.prompt_s, 1))
        log(f"[e2e] {mode}: {r['tok_s']:.1f} tok/s over tokens {n0}..{n1} ({r['ms_per_token']:.3f} ms/token), "
            f"{r['generation_tok_s']:.1f} tok/s over the whole generation, prefill {r['prompt_tok_s']:.0f} tok/s")
        return r, s

    runs["dense"], s = plain("dense")
    dense_toks = s.tokens(G)
    del s
    runs["sparse"], s = plain("sparse")
    runs["sparse"]["tokens_equal_dense"] = s.tokens(G) == dense_toks
    runs["sparse"]["tokens_compared"] = G
    nodes["decode"] = graph_node_counts(model, s.step_fn)
    cpu = cpu_baseline_e2e(model, s) if args.cpu_budget > 0 else None
    del s
    model.set_mode("sparse")
    for name, probs in (("mtp2_prose", (0.2, 0.34, 0.46)), ("mtp2_code", (0.06, 0.2, 0.74))):
        acc = mtp.scripted_accepts(8192, probs, seed=args.seed + 5)
        s = model.session(prompt, mtp=True, cap=cap, script=dense_toks, accepts=acc)
        s.step(W)
        n0, st0 = s.emitted(), s.state()
        if args.steps > 0:
            k = args.steps
        else:                                    # the steps that bring the generation to G tokens
            k, n = 0, n0
            while n < G:
                n += int(acc[W + k]) + 1
                k += 1
        sec = s.step(k)
        st1 = s.state()
        n1 = s.emitted()
        finish(s, G)
        toks = s.tokens(G)
        acc_mean = (st1[N.SEQ_ACC_SUM] - st0[N.SEQ_ACC_SUM]) / k
        runs[name] = dict(tok_s=round((n1 - n0) / sec, 2), ms_per_step=round(1e3 * sec / k, 4), steps=k, warmup=W,
                          timed_tokens=[n0, n1], cache_len_mid=T + (n0 + n1) // 2,
                          accepted_mean=round(acc_mean, 4), tokens_per_step=round((n1 - n0) / k, 4),
                          scripted_probs=list(probs), tokens_equal_dense=toks == dense_toks, tokens_compared=G,
                          generation_tok_s=round((s.emitted() - 1) / s.decode_s, 2), generation_tokens=s.emitted(),
                          generation_steps=s.steps, prompt_tok_s=round(T / s.prompt_s, 1))
        if "mtp" not in nodes:
            nodes["mtp"] = graph_node_counts(model, s.step_fn)
        log(f"[e2e] sparse + MTP-2 ({name}, mean accepted {acc_mean:.2f}): {runs[name]['tok_s']:.1f} tok/s over "
            f"tokens {n0}..{n1}, {runs[name]['ms_per_step']:.3f} ms/step; {runs[name]['generation_tok_s']:.1f} tok/s "
            f"over the whole generation; {G} tokens equal dense: {runs[name]['tokens_equal_dense']}")
        del s
    launch_us = empty_launch_us(dev, max(nodes["mtp"].get("kernel", 1) if nodes.get("mtp") else 200, 1))
    head = runs["mtp2_prose"]
    e2e_roof = dict(
        mtp2_step=e2e_roofline(model, "mtp", head["ms_per_step"], head["cache_len_mid"],
                               (nodes.get("mtp") or {}).get("kernel"), launch_us),
        decode_step=e2e_roofline(model, "decode", runs["sparse"]["ms_per_token"], runs["sparse"]["cache_len_mid"],
                                 (nodes.get("decode") or {}).get("kernel"), launch_us))
    for k_, r_ in e2e_roof.items():
        log(f"[e2e] roofline {k_}: {r_['bytes_per_step'] / 1e9:.3f} GB per step, {r_['achieved']:.0f} GB/s "
            f"({r_['frac']:.1%} of HBM); {r_['launches_per_step']} launches x {r_['empty_launch_us']:.2f} us = "
            f"{r_['launch_floor_ms']} ms launch floor of {r_['ms_per_step']} ms")
    rec = dict(metric=METRIC, value=head["tok_s"], unit="tok/s", n_gpus=1, steps=head["steps"], warmup=W,
               ms_per_step=head["ms_per_step"], higher_is_better=True, scaling="weak", vs_baseline=None,
               dtype="f32 accumulate (4-bit weights, bf16 activations)", data="synthetic",
               config=dict(workload="end to end: random-init Nemotron-H hybrid, 52 layers (23 Mamba-2, 23 MoE "
                                    "128x top-6, 6 GQA 32/2) + 1-layer MTP head, 4-bit g64, vocab 131072; "
                                    "2048-token random prompt, 256 greedy tokens; sparse down + MTP-2, scripted "
                                    "acceptance at mean 1.26/2",
                           prompt_tokens=T, gen_tokens=G, layers=len(cfg.pattern), hidden=cfg.hidden,
                           vocab=cfg.vocab, experts=cfg.n_experts, topk=cfg.topk,
                           weights_gb=round(model.nbytes() / 1e9, 2),
                           moe_zero_frac=round(float(np.mean(model.zero_frac_measured)), 4),
                           timed=f"{W} untimed warm-up steps, then {head['steps']} timed steps (tokens "
                                 f"{head['timed_tokens'][0]}..{head['timed_tokens'][1]}); every run is then stepped "
                                 f"on untimed to {G} tokens, and all {G} are compared with dense decode"),
               roofline=None, e2e_roofline=e2e_roof, graph_nodes=nodes, cpu_baseline=cpu, e2e=runs,
               all_tokens_equal=all(r.get("tokens_equal_dense", True) for r in runs.values()),
               reference_published={"sparse+MTP2 tok/s, Apple M5 Pro, real checkpoint and text (README.md:19)": 153})
    del model
    torch.cuda.empty_cache()
    return rec


def bench_step(args):
    """One captured step of the end-to-end model replayed `--steps` times after a
    `--prompt`-token prefill: --mode mtp (the head's own two drafts, the 3-row verify, the
    acceptance and the rollback; the kernels of a step do not depend on how many drafts are
    accepted), sparse or dense (a plain decode step). For per-kernel profiles of a step."""
    cfg = Mdl.ModelConfig()
    model = Mdl.NemotronModel(cfg, mode="dense" if args.mode == "dense" else "sparse", seed=args.seed)
    prompt = np.random.default_rng(args.seed + 11).integers(0, cfg.vocab, args.prompt).astype(np.int32)
    K = args.steps if args.steps > 0 else 200
    per = 3 if args.mode == "mtp" else 1               # tokens a step can emit
    s = model.session(prompt, mtp=args.mode == "mtp", cap=per * (K + max(args.warmup, 0)) + 8)
    s.step(max(args.warmup, 0))
    sec = s.step(K)
    log(f"[step] {args.mode}: {1e3 * sec / K:.3f} ms per step over {K} steps after a {len(prompt)}-token prompt")
    return dict(metric=f"captured {args.mode} step time", value=round(1e3 * sec / K, 4), unit="ms/step", n_gpus=1,
                steps=K, warmup=args.warmup, ms_per_step=round(1e3 * sec / K, 4), higher_is_better=False,
                scaling="weak", vs_baseline=None, dtype="f32 accumulate (4-bit weights, bf16 activations)",
                data="synthetic", config=dict(workload=f"one {args.mode} step of the 52-layer random-init model",
                                              prompt_tokens=len(prompt)))


# ------------------------------------------------------------------ the step's other kernels
def bench_proj(args):
    """The other kernels of a decode / verify step, each on its own, timed like the decode
    sweep (graphs of 23 calls, distinct weight sets rotated so that the calls read HBM, not
    the 256 MB memory-side cache): every 4-bit and bf16 projection of the model with the
    prologue and epilogue the model fuses into it, at one token row (a decode step) and
    three (a verify step), and the attention over a 2100-key cache. Per kernel: us per
    call, algorithmic bytes (weights once, inputs and outputs) and the fraction of the HBM
    roof."""
    from hsd import nn
    dev = torch.device("cuda:0")
    cfg = Mdl.ModelConfig()
    init = Mdl._Init(args.seed, dev)
    D, DI = cfg.hidden, cfg.mamba_inner
    ncall = 23
    steps, warm = max(args.steps, 10), max(args.warmup, 2)
    out = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 7)

    def rows(B, n, dt=torch.bfloat16, lo=-1.0, hi=1.0):
        return (torch.rand((B, n), device=dev, generator=gen) * (hi - lo) + lo).to(dt)

    def timed(name, key, B, nbytes, fn):
        graphs = capture_steps(lambda t, l: fn(l), 2)
        ms = time_graphs(graphs, steps, warm)
        del graphs
        us = 1e3 * ms / (steps * ncall)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append(dict(kernel=name, rows=B, us_per_call=round(us, 3), mb_per_call=round(nbytes / 1e6, 3),
                        gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4),
                        traffic=pmc_traffic(f"proj:{key}:{B}")))
        log(f"[proj] {name:36s} rows {B}: {us:7.2f} us, {nbytes / 1e6:7.2f} MB, {gbs:6.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")

    specs = [  # name, key, O, I, 4-bit, prologue, epilogue
        ("Mamba in_proj (RMS norm)", "in_proj", cfg.in_proj_dim, D, True, "rms", "bf16"),
        ("Mamba out_proj (gated norm, residual)", "out_proj", D, DI, True, "gated_z", "resid"),
        ("attention q|k|v (RMS norm)", "qkv", cfg.qkv_dim, D, True, "rms", "bf16"),
        ("attention o_proj (residual)", "o_proj", D, cfg.attn_heads * cfg.head_dim, True, "none", "resid"),
        ("MoE router gate, bf16 (RMS norm)", "gate", cfg.n_experts, D, False, "rms", "bf16"),
        ("MTP eh_proj, bf16", "eh_proj", D, 2 * D, False, "none", "bf16"),
        ("lm_head (RMS norm, argmax)", "lm_head", cfg.vocab, D, True, "rms", "argmax"),
    ]
    for name, key, O, I, q4, pro, epi in specs:
        wbytes = _q4(O, I) if q4 else O * I * 2
        nsets = min(ncall, max(2, -(-700_000_000 // wbytes)))
        Ws = [nn.QWeight(*init.q4(O, I, 1.0 / math.sqrt(I))) if q4 else nn.QWeight(init.bf16(O, I, std=I ** -0.5))
              for _ in range(nsets)]
        normw = init.uniform(I)
        for B in (1, 3):
            if pro == "gated_z":                          # z rows with their sums of squares past I
                x = rows(B, I + I // 16, torch.float32, 0.1, 1.0)[:, :I]
            else:
                x = rows(B, I)
            res = rows(B, O) if epi == "resid" else None
            keys = torch.empty((B, nn.argmax_slots(O, q4)), dtype=torch.int64, device=dev) if epi == "argmax" else None
            y = None if epi == "argmax" else torch.empty((B, O), dtype=torch.bfloat16, device=dev)
            xn = torch.empty((B, I), dtype=torch.bfloat16, device=dev) if pro == "rms" and not q4 else None
            io = B * I * (4 if pro == "gated_z" else 2) + B * O * 2 * (2 if epi == "resid" else 1) + \
                (2 * I if pro != "none" else 0) + (B * keys.shape[1] * 8 if keys is not None else 0)

            def call(l, W=Ws, x=x, res=res, keys=keys, y=y, xn=xn, pro=pro, epi=epi, normw=normw):
                w = W[l % len(W)]
                nn.linear(x, w, norm=normw if pro != "none" else None, eps=cfg.eps, gated_z=pro == "gated_z",
                          residual=res if epi == "resid" else None, out=y if epi != "argmax" else None,
                          argmax_keys=keys, xn_out=xn)
            timed(name, key, B, wbytes + io, call)
        del Ws
        torch.cuda.empty_cache()
    # attention over a 2100-key cache (6 layers' caches rotated)
    P = 2100
    kvs = [nn.KVCache(cfg.kv_heads, cfg.max_seq, dev, cfg.head_dim) for _ in range(6)]
    for kv in kvs:
        kv.k.normal_(generator=gen)
        kv.v.normal_(generator=gen)
    pos = torch.tensor([P], dtype=torch.int32, device=dev)
    for B in (1, 3):
        qkv = rows(B, cfg.qkv_dim)
        o = torch.empty((B, cfg.attn_heads * cfg.head_dim), dtype=torch.bfloat16, device=dev)
        ws = torch.empty(N.lib().hsd_attn_workspace_bytes(B, cfg.attn_heads, cfg.max_seq), dtype=torch.uint8,
                         device=dev)
        nbytes = 2 * cfg.kv_heads * cfg.head_dim * 2 * (P + B) + B * cfg.qkv_dim * 2 + B * cfg.attn_heads * cfg.head_dim * 2

        def att(l, qkv=qkv, o=o, ws=ws):
            # the cache length stays P: the call writes rows P .. P+B-1 and a replay rewrites them
            nn.attention(qkv, kvs[l % len(kvs)], pos, n_heads=cfg.attn_heads, n_kv_heads=cfg.kv_heads,
                         head_dim=cfg.head_dim, out=o, workspace=ws)
        timed(f"attention, {P} keys (part + combine)", "attention", B, nbytes, att)
    return dict(metric="the step's projections and attention, each alone: HBM GB/s", value=None, unit="GB/s",
                n_gpus=1, steps=steps, warmup=warm, ms_per_step=None, higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="f32 accumulate (4-bit or bf16 weights, bf16 activations)", data="synthetic",
                config=dict(workload="graphs of 23 calls over rotated weight sets, 1 and 3 token rows"),
                kernels=out)


def bench_calib(args):
    """The counter calibration workload: a 268435456-byte device-to-device copy (torch
    copy_), six times. Its FETCH_SIZE and WRITE_SIZE per dispatch against the 256 MiB read
    and written give the factors that turn those counters into bytes."""
    dev = torch.device("cuda:0")
    n = 1 << 26
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(6):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 6
    gbs = 2 * 4 * n / (ms * 1e-3) / 1e9
    log(f"[calib] 256 MiB copy: {ms * 1e3:.1f} us, {gbs:.0f} GB/s read + write")
    return dict(metric="256 MiB device copy (counter calibration)", value=round(gbs, 1), unit="GB/s", n_gpus=1,
                steps=6, warmup=0, ms_per_step=round(ms, 4), higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="f32", data="synthetic", config=dict(workload="copy", bytes=4 * n))


def _sub(rec):
    """A workload's record inside the combined line (the fields the run record repeats dropped)."""
    drop = ("n_gpus", "higher_is_better", "scaling", "vs_baseline", "data")
    return {k: v for k, v in rec.items() if k not in drop}


def bench_all(args):
    import copy
    rec = bench_e2e(args)
    torch.cuda.empty_cache()
    sub = {}
    for name, fn, steps, warm in (("decode_sparse_down", bench_decode, 200, 20), ("prefill", bench_prefill, 3, 1),
                                  ("mtp_verify_rollback", bench_mtp, 200, 20), ("moe_front_end", bench_up, 200, 20)):
        a = copy.copy(args)
        a.steps, a.warmup = steps, warm
        if name == "decode_sparse_down":
            a.cold = True
        sub[name] = _sub(fn(a))
        torch.cuda.empty_cache()
    dec = sub["decode_sparse_down"]
    rec["roofline"] = dict(dec["roofline"], workload="decode_sparse_down",
                           note="the sparse down projection (the metric's 'sparse-down HBM GB/s vs peak'), from the "
                                "23-layer decode sweep at 90 % zeros, warm; the cold figure is in workloads")
    rec["workloads"] = sub
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0,
                    help="timed steps (0: the workload's default; end to end: the steps that make 256 tokens)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="all",
                    choices=("all", "e2e", "decode", "prefill", "mtp", "up", "step", "calib", "proj"))
    ap.add_argument("--mode", default="mtp", choices=("mtp", "sparse", "dense"), help="step: which step")
    ap.add_argument("--prompt", type=int, default=2048, help="end to end: prompt tokens")
    ap.add_argument("--gen", type=int, default=256, help="end to end: generated tokens")
    ap.add_argument("--zero-frac", type=float, default=0.9)
    ap.add_argument("--hot", action="store_true", help="hot-neuron activation variant")
    ap.add_argument("--ntok", type=int, default=32, help="distinct tokens rotated (one graph each)")
    ap.add_argument("--cold", action="store_true", help="also time with a cache flush between tokens")
    ap.add_argument("--batch-sweep", default="3,8,16,32,64",
                    help="decode: token rows per call to time besides batch 1 (comma list; empty: skip)")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense 4-bit comparator")
    ap.add_argument("--no-control", action="store_true",
                    help="decode: skip the dense-h control (so a profile holds the sparse calls only)")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle time (0: skip)")
    ap.add_argument("--layers", type=int, default=NL)
    ap.add_argument("--tt", type=int, default=32)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    if args.workload not in ("all", "e2e", "step", "calib", "proj"):
        defaults = dict(decode=(200, 20), prefill=(3, 1), mtp=(200, 20), up=(200, 20))[args.workload]
        if args.steps <= 0:
            args.steps, args.warmup = defaults
    fn = dict(all=bench_all, e2e=bench_e2e, decode=bench_decode, prefill=bench_prefill, mtp=bench_mtp,
              up=bench_up, step=bench_step, calib=bench_calib, proj=bench_proj)[args.workload]
    rec = fn(args)
    rec["device"] = torch.cuda.get_device_name(0)
    rec["torch"] = torch.__version__
    rec["hip"] = torch.version.hip
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
