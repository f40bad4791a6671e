"""Benchmark: packed varlen causal GQA attention fwd+bwd on one MI355X.

Workload (the one the metric is quoted on): Qwen2.5-1.5B attention shape,
12 query heads, 2 key/value heads, head_dim 128, fp16, batch 4 x 512 tokens, every document full
length (causal). One step = 28 layer-equivalent calls (forward + backward each) over 28 distinct
resident buffer sets, launched as one captured HIP graph. Inputs are N(0, 1), synthetic.

Metric: causal-FLOP throughput, F = 3.5 * 4 * Hq * D * sum L(L+1)/2 per call (forward + backward,
the backward's recomputation of P not counted), in TFLOP/s and as a fraction of the MI355X dense
fp16 MFMA peak. The dominant kernel's duration is measured with HIP events on the stream it runs
on (queue pre-filled so launch latency is not timed) and reported against its roofline. The CPU
baseline is the oracle (numpy fp32) on one layer call of the same shape, on this host's cores.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 2]
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

    # ---- dominant-kernel timing: HIP events on the launch stream, queue pre-filled -----------
    def timed(launch, reps=3):
        stream = torch.cuda.current_stream()
        evs = []
        for _ in range(reps):
            try:
                torch.cuda._sleep(20_000_000)  # holds the queue while the launches are enqueued
            except Exception:
                pass
            for s in sets:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                launch(s, stream, a, b)
                evs.append((a, b))
        torch.cuda.synchronize()
        times = [a.elapsed_time(b) * 1e3 for a, b in evs]
        return float(np.mean(times)), float(np.median(times))

    def fwd_launch(s, stream, a, b):
        a.record()
        fwd(s, stream.cuda_stream)
        b.record()

    def bwd_main_launch(s, stream, a, b):
        a.record()
        bwd(s, stream.cuda_stream, _lib.VA_BWD_MAIN)
        b.record()
        bwd(s, stream.cuda_stream, _lib.VA_BWD_FINISH)

    fwd_us, fwd_med = timed(fwd_launch)
    bwd_us, bwd_med = timed(bwd_main_launch)
    fwd_flops = wl.forward_flops(lengths, hq)
    bwd_flops = 2.5 * fwd_flops
    kernels = {
        "fwd_kernel": dict(us=fwd_us, median_us=fwd_med, flops=fwd_flops,
                           tflops=fwd_flops / (fwd_us * 1e-6) / 1e12),
        "bwd_kernel": dict(us=bwd_us, median_us=bwd_med, flops=bwd_flops,
                           tflops=bwd_flops / (bwd_us * 1e-6) / 1e12),
    }
    dom_name = max(kernels, key=lambda k: kernels[k]["us"])
    dom = kernels[dom_name]
    roofline = {"kernel": dom_name, "bound": "mfma", "achieved": round(dom["tflops"], 2),
                "peak": peak, "unit": "TFLOP/s", "frac": round(dom["tflops"] / peak, 4),
                "traffic": None, "avg_us": round(dom["us"], 3),
                "flops_per_launch": dom["flops"]}

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
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
