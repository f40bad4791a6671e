"""Benchmark: packed varlen causal GQA attention fwd+bwd on one MI355X.

Workload (the one the metric is quoted on): Qwen2.5-1.5B attention shape,
12 query heads, 2 key/value heads, head_dim 128, fp16, batch 4 x 512 tokens, every document full
length (causal). One step = 28 layer-equivalent calls (forward + backward each) over 28 distinct
resident buffer sets, launched as one captured HIP graph. Inputs are N(0, 1), synthetic.

Metric: causal-FLOP throughput, F = 3.5 * 4 * Hq * D * sum L(L+1)/2 per call (forward + backward,
the backward's recomputation of P not counted), in TFLOP/s and as a fraction of the MI355X dense
fp16 MFMA peak. The dominant kernel's duration is measured with HIP events on the stream it runs
on (each kernel captured alone, 28 launches per graph replay) and reported against its roofline
(HBM or MFMA, whichever its arithmetic intensity puts first against the ridge point), with the HBM
traffic that rocprofv3 --pmc measured for it (profiles/hbm_traffic_<workload>.md). The
CPU baseline is the oracle (numpy fp32) on one layer call of the same shape, on this host's cores.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 2]
    python bench.py --pmc-probe          # untimed launches for rocprofv3 --pmc passes
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "varlen attn fwd+bwd TFLOP/s (causal FLOPs) at Qwen2.5-1.5B shape; % MFMA peak"
PEAK_MFMA_TFLOPS = {"float16": 2516.6, "bfloat16": 2516.6}  # dense, 256 CU x 2.4 GHz x 4096
PEAK_HBM_GBS = 8000.0
LAYER_CALLS = 28


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", type=int, default=2)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--pmc-probe", action="store_true",
                   help="launch a 256 MiB fp32 copy-like kernel and each attention kernel once per "
                        "buffer set, untimed, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    return p.parse_args()


class LayerSet:
    """One layer-equivalent buffer set: inputs, outputs, lse and the backward workspace."""

    def __init__(self, torch, att, lengths, hq, hkv, dtype, qk_scale, seed, plan):
        n = sum(lengths)
        dev = torch.device("cuda")
        g = torch.Generator(device=dev).manual_seed(seed)
        self.q = (torch.randn(n, hq, 128, device=dev, generator=g) * qk_scale).to(dtype)
        self.k = (torch.randn(n, hkv, 128, device=dev, generator=g) * qk_scale).to(dtype)
        self.v = torch.randn(n, hkv, 128, device=dev, generator=g).to(dtype)
        self.do = torch.randn(n, hq, 128, device=dev, generator=g).to(dtype)
        self.out = torch.empty_like(self.q)
        self.lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
        self.dq = torch.empty_like(self.q)
        self.dk = torch.empty_like(self.k)
        self.dv = torch.empty_like(self.v)
        self.ws, _ = att.bwd_workspace(n, hq, hkv, dev)
        self.n, self.hq, self.hkv = n, hq, hkv
        self.plan = plan


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` as measured by rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE (each scaled by the same counter's reading on a copy kernel of known size), read from
    the committed profile summary; None when no measurement is committed."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch:" and parts[1] == kernel:
                return int(parts[2])
    return None


def roofline(flops, nbytes, us, peak_tflops, peak_gbs=PEAK_HBM_GBS):
    """Roofline position of a kernel from its algorithmic FLOPs and HBM bytes per launch and its
    average launch duration: the ceiling is HBM bandwidth when the arithmetic intensity is below
    the ridge point peak_tflops / peak_gbs, else the MFMA peak."""
    intensity = flops / nbytes
    ridge = peak_tflops * 1e12 / (peak_gbs * 1e9)
    secs = us * 1e-6
    mfma_tflops = flops / secs / 1e12
    if intensity >= ridge:
        bound, achieved, peak, unit = "mfma", mfma_tflops, peak_tflops, "TFLOP/s"
    else:
        bound, achieved, peak, unit = "hbm", nbytes / secs / 1e9, peak_gbs, "GB/s"
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "arithmetic_intensity": round(intensity, 1),
            "ridge": round(ridge, 1), "mfma_tflops": round(mfma_tflops, 2),
            "mfma_frac": round(mfma_tflops / peak_tflops, 4)}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the attention path needs no "
                                   "collective; run with --gpus 1 (see the sharding note in the "
                                   "design document)"}))
        sys.exit(2)

    import numpy as np
    import torch

    from hackaton_amd import _lib
    from hackaton_amd import attention as att
    from hackaton_amd import workloads as wl

    lib = _lib.lib()
    cfg = wl.CONFIGS[args.config]
    lengths = wl.config_lengths(args.config)
    hq, hkv = cfg["hq"], cfg["hkv"]
    dtype = wl.torch_dtype(cfg["dtype"])
    dcode = {torch.float16: _lib.VA_F16, torch.bfloat16: _lib.VA_BF16}[dtype]
    scale = 128 ** -0.5
    dev = torch.device("cuda")
    torch.cuda.set_device(0)
    cu = att._cu_seqlens(lengths, dev)
    plan = att._plan(cu, hq, hkv)
    sets = [LayerSet(torch, att, lengths, hq, hkv, dtype, cfg["qk_scale"], 1000 + i, plan)
            for i in range(LAYER_CALLS)]
    torch.cuda.synchronize()

    def fwd(s, stream):
        _lib.check(lib.va_fwd(s.q.data_ptr(), s.k.data_ptr(), s.v.data_ptr(), s.out.data_ptr(),
                              s.lse.data_ptr(), plan.fwd_items.data_ptr(), plan.n_fwd, s.n, hq,
                              hkv, 128, scale, dcode, stream), "va_fwd")

    def bwd(s, stream, stage=-1):
        argv = (s.do.data_ptr(), s.q.data_ptr(), s.k.data_ptr(), s.v.data_ptr(),
                s.out.data_ptr(), s.lse.data_ptr(), plan.bwd_items.data_ptr(), plan.n_bwd, s.n,
                hq, hkv, 128, scale, dcode, s.dq.data_ptr(), s.dk.data_ptr(), s.dv.data_ptr(),
                s.ws.data_ptr(), s.ws.numel(), stream)
        if stage < 0:
            _lib.check(lib.va_bwd(*argv), "va_bwd")
        else:
            _lib.check(lib.va_bwd_stage(stage, *argv), "va_bwd_stage")

    def step():
        stream = torch.cuda.current_stream().cuda_stream
        for s in sets:
            fwd(s, stream)
            bwd(s, stream)

    if args.pmc_probe:
        # calibration kernel of known traffic: y = x * 1 over 64 Mi fp32 (256 MiB read, 256 MiB
        # written), then every attention kernel once per buffer set
        x = torch.randn(64 << 20, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            torch.mul(x, 1.0, out=y)
        stream = torch.cuda.current_stream().cuda_stream
        for s in sets:
            fwd(s, stream)
        for s in sets:
            bwd(s, stream, _lib.VA_BWD_MAIN)
        for s in sets:
            bwd(s, stream, _lib.VA_BWD_FINISH)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": cfg["name"], "copy_read_bytes": x.numel() * 4,
                          "copy_write_bytes": y.numel() * 4, "launches_per_kernel": len(sets)}),
              flush=True)
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph.replay()
    torch.cuda.synchronize()

    # ---- timed region: K graph replays -------------------------------------------------------
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_per_step = start.elapsed_time(end) / args.steps

    flops_call = wl.attention_flops(lengths, hq)
    flops_step = flops_call * LAYER_CALLS
    tflops = flops_step / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_MFMA_TFLOPS[cfg["dtype"]]

    # ---- dominant-kernel timing: HIP events on the launch stream ------------------------------
    # Each kernel is captured alone, 28 launches back to back (one per buffer set), and the graph
    # is replayed between two events recorded on the stream the replays run on; the average
    # launch duration is the elapsed time over the number of launches.
    def kernel_graph(launch):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            st = torch.cuda.current_stream().cuda_stream
            for s in sets:
                launch(s, st)
        return g

    def timed(g, reps=10):
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (reps * len(sets))

    g_fwd = kernel_graph(fwd)
    g_bwd = kernel_graph(lambda s, st: bwd(s, st, _lib.VA_BWD_MAIN))
    g_fin = kernel_graph(lambda s, st: bwd(s, st, _lib.VA_BWD_FINISH))
    fwd_us, bwd_us, fin_us = timed(g_fwd), timed(g_bwd), timed(g_fin)
    fwd_flops = wl.forward_flops(lengths, hq)
    bwd_flops = 2.5 * fwd_flops
    n_tok = sum(lengths)
    kernels = {
        "fwd_kernel": dict(us=fwd_us, flops=fwd_flops,
                           bytes=wl.forward_bytes(n_tok, hq, hkv)),
        "bwd_kernel": dict(us=bwd_us, flops=bwd_flops,
                           bytes=wl.backward_main_bytes(n_tok, hq, hkv)),
        "bwd_gqa_sum_kernel": dict(us=fin_us, flops=0.0,
                                   bytes=wl.gqa_sum_bytes(n_tok, hq, hkv)),
    }
    dom_name = max(kernels, key=lambda k: kernels[k]["us"])
    dom = kernels[dom_name]
    roofline_ = {"kernel": dom_name,
                 **roofline(dom["flops"], dom["bytes"], dom["us"], peak),
                 "traffic": measured_traffic(dom_name, cfg["name"]), "avg_us": round(dom["us"], 3),
                 "flops_per_launch": dom["flops"], "algorithmic_bytes": dom["bytes"]}

    # ---- CPU baseline: the oracle on one layer call of the same shape ------------------------
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import attention_oracle as orc
        try:
            from threadpoolctl import threadpool_info
            threads = max([i.get("num_threads", 1) for i in threadpool_info()
                           if i.get("user_api") == "blas"] or [1])
        except Exception:
            threads = os.cpu_count() or 1
        q, k, v, do = wl.make_inputs(lengths, hq, hkv, torch.float32, seed=0,
                                     qk_scale=cfg["qk_scale"])
        q, k, v, do = (t.numpy() for t in (q, k, v, do))
        cuh = orc.cu_seqlens_from_lengths(lengths)
        reps, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds or reps == 0:
            t1 = time.perf_counter()
            o, lse = orc.attention_forward(q, k, v, cuh, scale, dtype=np.float32)
            orc.attention_backward(q, k, v, o, lse, do, cuh, scale, dtype=np.float32)
            t_cpu += time.perf_counter() - t1
            reps += 1
        cpu = {"value": round(flops_call * reps / t_cpu / 1e12, 5), "unit": "TFLOP/s",
               "cores": int(threads), "kind": "port",
               "sample": f"{reps} layer call(s) of the benchmark shape ({len(lengths)} docs, "
                         f"{sum(lengths)} tokens, {hq}/{hkv} heads) fwd+bwd, numpy fp32 oracle, "
                         f"{t_cpu:.1f} s, BLAS threads {threads}"}

    result = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float16": "fp16", "bfloat16": "bf16"}[cfg["dtype"]],
        "data": "synthetic N(0,1) q/k/v/dO, 28 resident buffer sets",
        "config": {"workload": cfg["name"], "tokens": sum(lengths), "docs": len(lengths),
                   "hq": hq, "hkv": hkv, "head_dim": 128, "layer_calls": LAYER_CALLS,
                   "causal_flops_per_step": flops_step},
        "pct_mfma_peak": round(100 * tflops / peak, 3),
        "wall_ms_per_step": round(wall_ms, 5),
        "kernels_us": {k: round(v["us"], 3) for k, v in kernels.items()},
        "kernels_tflops": {k: round(v["flops"] / (v["us"] * 1e-6) / 1e12, 2)
                           for k, v in kernels.items() if v["flops"]},
        "roofline": roofline_,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
