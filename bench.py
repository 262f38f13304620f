"""Benchmark of the hsd hot path on one MI355X.

Default workload (python bench.py [--steps K --warmup W]): the 23-layer batch-1 decode
sweep at the Nemotron-3.5-Lightning-30B-A3B MoE shape -- 128 experts, top-6 uniform
routing per layer and token, routed D=2688 x F=1856 and shared D x 3712 down
projections in affine 4-bit g64 (8.39 GB of neuron-major weights resident), ReLU^2
activations with 90 % exact zeros. A step = one token through the 23 sparse down
projections (captured once per token as a HIP graph and replayed). `value` is GB/s over
the bytes actually touched (live rows x D/2 + live 64-groups x 4D + I/O) for the whole
timed region; inputs are resident in HBM.

Other workloads, each printing one JSON line of its own:
  --workload prefill   2048-token prompt in chunks of 512, Zipf(1.1) routing, 23 layers
  --workload mtp       MTP-2 verify (3 rows) + rollback over 23 Mamba-2 layers
  --workload up        the MoE front end after the router: 4-bit up projections of the 6
                       selected and the shared expert + ReLU^2 into hcat, 23 layers,
                       batch 1; also the front end followed by the sparse down projection
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-heimr-sparse-down_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from hsd import decode, layout, mamba as M, moe, mtp, prefill, synth as S  # noqa: E402
from hsd import _native as N  # noqa: E402

METRIC = "batch-1 decode tok/s (sparse+MTP2); sparse-down HBM GB/s vs peak"
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
        with torch.cuda.graph(g):
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
    # dense-h control: the same kernel reading every row
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
    achieved = per_launch_bytes / (per_launch_us * 1e-6) / 1e9
    rec = dict(metric=METRIC, value=round(gbs, 2), unit="GB/s", n_gpus=1, steps=steps, warmup=warm,
               ms_per_step=round(ms_step, 5), higher_is_better=True, scaling="weak", vs_baseline=None,
               dtype="f32 (4-bit weights, bf16 scales/activations)", data="synthetic",
               config=dict(workload="decode sweep: 23 MoE layers, batch 1, sparse 4-bit down projection",
                           zero_frac=args.zero_frac, hot_neurons=bool(args.hot), experts=E, topk=K, D=D, F=F,
                           FS=FS, group=64, tokens_rotated=ntok, weights_gb=round(NL * 364.8e6 / 1e9, 2)),
               roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                             frac=round(achieved / HBM_PEAK_GBS, 4), traffic=pmc_traffic("decode"),
                             kernel="k_sparse_down_part + k_sum_parts (one decode call)",
                             bytes_per_launch=int(per_launch_bytes), us_per_launch=round(per_launch_us, 3)),
               cpu_baseline=cpu,
               down_proj_tok_s=round(1e3 / ms_step, 1),
               layout_permute=dict(ms_23_layers=round(perm_ms, 2), gbs_rw=round(perm_bytes / perm_ms / 1e6, 1)),
               **extra)
    return rec


# ------------------------------------------------------------------ prefill
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
    return dict(metric="prefill down-projection TFLOP/s (bf16 MFMA, algorithmic union FLOPs)",
                value=round(tflops, 2), unit="TFLOP/s", n_gpus=1, steps=args.steps, warmup=1,
                ms_per_step=round(ms_all, 4), higher_is_better=True, scaling="weak", vs_baseline=None,
                dtype="bf16 MFMA, f32 accumulate", data="synthetic",
                config=dict(workload="prefill: 2048-token prompt in chunks of 512, Zipf(1.1) top-6 routing",
                            layers=nl, tt=tt, zero_frac=args.zero_frac),
                roofline=dict(bound="mfma", achieved=round(tflops, 2), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                              frac=round(tflops / BF16_PEAK_TFLOPS, 4), traffic=pmc_traffic("prefill"),
                              hbm_frac_dense_weights=round(wbytes / (ms_gemm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)),
                prefill_tok_s=round(T / (ms_all * 1e-3), 1), gflop_per_prompt=round(flops / 1e9, 2))


# ------------------------------------------------------------------ MTP verify
def bench_mtp(args):
    dev = torch.device("cuda:0")
    nl = NL
    mixers, caches = [], []
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    for l in range(nl):
        p = S.mamba_params_np(args.seed + l)
        mixers.append(M.Mamba2Mixer(conv_w=S.to_device(p["conv_w"], dev), conv_b=S.to_device(p["conv_b"], dev),
                                    A_log=S.to_device(p["A_log"], dev), dt_bias=S.to_device(p["dt_bias"], dev),
                                    D=S.to_device(p["D"], dev), norm_w=S.to_device(p["norm_w"], dev)))
        caches.append(M.MambaCache(mixers[-1], dev, nslab=4, cur=cur,
                                   conv_state=S.to_device(p["conv_state"], dev),
                                   ssm_state=torch.from_numpy(p["ssm_state"]).to(dev)))
    rng = np.random.default_rng(args.seed)
    nsteps = 64
    rows = S.to_device(np.stack([S.mamba_rows_np(rng, 3) for _ in range(nsteps)]), dev)   # [steps, 3, 10304]
    accepts = mtp.scripted_accepts(nsteps, (0.15, 0.35, 0.50), args.seed)
    nkeep = torch.tensor(accepts + 1, dtype=torch.int32, device=dev)
    ws = torch.empty(N.lib().hsd_mamba_workspace_bytes(3, 64, 64), dtype=torch.uint8, device=dev)

    def step(i):
        recs = []
        for l in range(nl):
            M.verify_rows(mixers[l], rows[i], caches[l], workspace=ws)
            recs.append((caches[l], 3))
        M.mamba_rollback(recs[:1], 0, n_keep_dev=nkeep[i:i + 1])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(0)
    torch.cuda.current_stream().wait_stream(s)
    graphs = []
    for i in range(nsteps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    ms = time_graphs(graphs, args.steps, args.warmup)
    per_layer = 2097152 + 3 * 2097152 + 3 * 6144 * 2 + 3 * 3 * 6144 * 2 + 3 * 10304 * 2 + 3 * 4096 * 2
    gbs = per_layer * nl * args.steps / (ms * 1e-3) / 1e9
    log(f"[mtp] verify(3)+rollback, 23 Mamba-2 layers: {1e3 * ms / args.steps:.1f} us/step, {gbs:.0f} GB/s")
    return dict(metric="MTP-2 verify + rollback, 23 Mamba-2 layers: HBM GB/s", value=round(gbs, 2), unit="GB/s",
                n_gpus=1, steps=args.steps, warmup=args.warmup, ms_per_step=round(ms / args.steps, 5),
                higher_is_better=True, scaling="weak", vs_baseline=None, dtype="f32 state, bf16 I/O",
                data="synthetic",
                config=dict(workload="MTP verify + rollback: 23 Mamba-2 layers, 3 rows, P(0,1,2)=(.15,.35,.5)"),
                roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                              frac=round(gbs / HBM_PEAK_GBS, 4), traffic=pmc_traffic("mtp"),
                              bytes_per_layer_step=per_layer))


# ------------------------------------------------------------------ MoE front end
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
                front_plus_down_us_per_token=round(1e3 * cms / args.steps, 2))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="decode", choices=("decode", "prefill", "mtp", "up"))
    ap.add_argument("--zero-frac", type=float, default=0.9)
    ap.add_argument("--hot", action="store_true", help="hot-neuron activation variant")
    ap.add_argument("--ntok", type=int, default=32, help="distinct tokens rotated (one graph each)")
    ap.add_argument("--cold", action="store_true", help="also time with a cache flush between tokens")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense 4-bit comparator")
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
    fn = dict(decode=bench_decode, prefill=bench_prefill, mtp=bench_mtp, up=bench_up)[args.workload]
    rec = fn(args)
    rec["device"] = torch.cuda.get_device_name(0)
    rec["torch"] = torch.__version__
    rec["hip"] = torch.version.hip
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
