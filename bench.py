"""Benchmark: packed varlen causal GQA attention fwd+bwd on one MI355X.

Headline workload (the one the metric is quoted on): Qwen2.5-1.5B
attention shape, 12 query heads, 2 key/value heads, head_dim 128, fp16, batch 4 x 512 tokens, every
document full length (causal). One step = 28 layer-equivalent calls (forward + backward each) over
28 distinct resident buffer sets, launched as one captured HIP graph. Inputs are N(0, 1),
synthetic.

Metric: causal-FLOP throughput, F = 3.5 * 4 * Hq * D * sum L(L+1)/2 per call (forward + backward,
the backward's recomputation of P not counted), in TFLOP/s and as a fraction of the MI355X dense
fp16 MFMA peak.

Also reported on the same JSON line:
* kernels_us: median per-launch duration of each kernel (each kernel captured alone, one launch
  per buffer set, >= 20 timed replays between HIP events on the stream the kernels run on);
* roofline: the dominant kernel against its ceiling, with the algorithmic bytes of the pass it
  computes (forward: q, k, v read, O and lse written; backward: q, k, v, O, dO, lse read, dq and
  dk/dv written at Hkv width) and the HBM traffic that rocprofv3 --pmc measured for it
  (profiles/hbm_traffic_<workload>.md);
* by_config: the same fwd+bwd call timed at BASELINE configurations 3-5;
* installed_path: PackedAttention (rotation, attention forward, attention backward, inverse
  rotation) as the decoder layer calls it, at the headline configuration (host
  and device lengths) and at configurations 3-5 (host lengths), beside the bare kernels' time;
* cpu_baseline: the reference's own CPU-runnable math (torch CPU scaled_dot_product_attention in
  fp32, forward + autograd backward, GQA through enable_gqa), in the two constructions the
  reference tests use, at BASELINE configuration 1 and at the headline shape.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 2]
    python bench.py --pmc-probe          # untimed launches for rocprofv3 --pmc passes
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "varlen attn fwd+bwd TFLOP/s (causal FLOPs) at Qwen2.5-1.5B shape; % MFMA peak"
PEAK_MFMA_TFLOPS = {"float16": 2516.6, "bfloat16": 2516.6}  # dense, 256 CU x 2.4 GHz x 4096
PEAK_HBM_GBS = 8000.0
LAYER_CALLS = 28
MIN_REPS = 20
SET_BYTES_TARGET = 1 << 30  # buffer sets per configuration: at least this much resident memory


def parse(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", type=int, default=2)
    p.add_argument("--reps", type=int, default=25, help="timed replays per kernel median (>= 20)")
    p.add_argument("--by-config", default="3,4,5",
                   help="other BASELINE configurations to time (comma list, empty for none)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-installed-path", action="store_true")
    p.add_argument("--pmc-probe", action="store_true",
                   help="launch a 256 MiB fp32 copy-like kernel and each attention kernel once per "
                        "buffer set, untimed, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    return p.parse_args(argv)


# ------------------------------------------------------------------------------------------------
# report helpers (pure functions, tested on the CPU)
# ------------------------------------------------------------------------------------------------
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
    launch duration: the ceiling is HBM bandwidth when the arithmetic intensity is below the ridge
    point peak_tflops / peak_gbs, else the MFMA peak."""
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


def kernel_models(lengths, hq, hkv, elem=2):
    """Algorithmic FLOPs and bytes per launch of each kernel of one fwd+bwd call. The backward's
    bytes (dk/dv at Hkv width) belong to the pass, charged to its main kernel; a separate GQA sum
    and the row statistics pass have no algorithmic work of their own."""
    from hackaton_amd import workloads as wl

    n = int(sum(lengths))
    fwd_flops = wl.forward_flops(lengths, hq)
    fwd = dict(flops=fwd_flops, bytes=wl.forward_bytes(n, hq, hkv, elem))
    return {
        "fwd_kernel": fwd,
        "fwd_lean_kernel": dict(fwd),  # the many-item forward: same work
        "bwd_kernel": dict(flops=2.5 * fwd_flops, bytes=wl.backward_bytes(n, hq, hkv, elem)),
        "bwd_gqa_sum_kernel": dict(flops=0.0, bytes=0),
        "bwd_stats_kernel": dict(flops=0.0, bytes=0),
    }


def by_config_list(args):
    """The other BASELINE configurations to time (--by-config)."""
    return [int(x) for x in args.by_config.split(",") if x.strip()]


def median_us(samples_ms, launches):
    """Median per-launch duration in microseconds of timed replays of `launches` launches each."""
    return statistics.median(samples_ms) * 1e3 / launches


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


# ------------------------------------------------------------------------------------------------
# CPU baseline: torch CPU SDPA in fp32, as the reference's tests build it
# ------------------------------------------------------------------------------------------------
def sdpa_padded_call(q, k, v, grad, lengths, scale):
    """Forward + autograd backward of the reference test's construction
    (solution/test_attention.py:95-106): zero-padded dense SDPA with a `tril & real` mask, here
    with Hkv key/value heads through enable_gqa. Returns out (N, Hq*D) and the three gradients."""
    import torch

    batch, seq = len(lengths), max(lengths)
    hq, hkv, dim = q.shape[1], k.shape[1], q.shape[2]
    real = torch.zeros(batch, seq, dtype=torch.bool)
    for row, length in enumerate(lengths):
        real[row, :length] = True
    rows = torch.nonzero(real.reshape(-1), as_tuple=True)[0]
    mask = torch.ones(seq, seq, dtype=torch.bool).tril()[None, None] & real[:, None, None]
    leaves = [x.detach().requires_grad_() for x in (q, k, v)]

    def padded(x):
        full = torch.zeros(batch * seq, x.shape[1], dim, dtype=x.dtype)
        return full.index_copy(0, rows, x).view(batch, seq, x.shape[1], dim).transpose(1, 2)

    out = torch.nn.functional.scaled_dot_product_attention(
        *[padded(x) for x in leaves], attn_mask=mask, scale=scale, enable_gqa=hq != hkv)
    out = out.transpose(1, 2).reshape(batch * seq, hq * dim)[rows]
    out.backward(grad)
    return out.detach(), [x.grad for x in leaves]


def sdpa_per_document_call(q, k, v, grad, lengths, scale):
    """Forward + autograd backward of per-document causal SDPA (is_causal=True, enable_gqa) on
    the packed rows. Returns out (N, Hq*D) and the three gradients."""
    import torch

    hq, hkv, dim = q.shape[1], k.shape[1], q.shape[2]
    leaves = [x.detach().requires_grad_() for x in (q, k, v)]
    outs, s = [], 0
    for length in lengths:
        e = s + length
        qd, kd, vd = (x[s:e].transpose(0, 1)[None] for x in leaves)
        o = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd, is_causal=True,
                                                             scale=scale, enable_gqa=hq != hkv)
        outs.append(o[0].transpose(0, 1).reshape(length, hq * dim))
        s = e
    out = torch.cat(outs)
    out.backward(grad)
    return out.detach(), [x.grad for x in leaves]


def time_cpu(fn, args, warmup=2, reps=5, budget_s=2.5):
    """Best of at least `reps` timed calls, repeated until `budget_s` seconds of timed work (so the
    whole CPU sample is ~10 s of CPU work: 2 configurations x 2 constructions)."""
    for _ in range(warmup):
        fn(*args)
    best, spent, n = math.inf, 0.0, 0
    while n < reps or spent < budget_s:
        t0 = time.perf_counter()
        fn(*args)
        dt = time.perf_counter() - t0
        best, spent, n = min(best, dt), spent + dt, n + 1
    return best


def measure_ceilings(reps=5):
    """The two ceilings the roofline fractions are quoted against, measured on this box with the
    library's probes (va_probe_mfma, va_probe_copy): dense 32x32x16 MFMA issue rate in fp16 and
    bf16 (4096 work-groups of 4 waves, 4 independent accumulators per wave) and the streaming rate
    of a 1 GiB device copy (read + written bytes), each the median of `reps` launches timed with
    HIP events on the launch stream."""
    import torch

    from hackaton_amd import _lib

    lib = _lib.lib()
    st = torch.cuda.current_stream()
    # 16 waves per SIMD over the kernel, ~4 ms per launch: the launch's own cost is under 1%
    blocks, iters = 4096, 4000
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    flops = blocks * 4 * iters * 4 * 32 * 32 * 16 * 2

    def timed(launch):
        launch()
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(st)
            launch()
            b.record(st)
            b.synchronize()
            times.append(a.elapsed_time(b))
        return sorted(times)[len(times) // 2]

    out = {}
    for name, code in (("mfma_f16_tflops", _lib.VA_F16), ("mfma_bf16_tflops", _lib.VA_BF16)):
        ms = timed(lambda: _lib.check(lib.va_probe_mfma(code, blocks, iters, sink.data_ptr(),
                                                        st.cuda_stream), "va_probe_mfma"))
        out[name] = round(flops / (ms * 1e-3) / 1e12, 1)
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    # one round of 4 chunks per thread (65536 work-groups: the best of 1024-65536 on the box)
    ms = timed(lambda: _lib.check(lib.va_probe_copy(src.data_ptr(), dst.data_ptr(), n, 65536,
                                                    st.cuda_stream), "va_probe_copy"))
    out["hbm_copy_gbs"] = round(2 * n / (ms * 1e-3) / 1e9, 1)
    out["datasheet"] = {"mfma_tflops": PEAK_MFMA_TFLOPS["float16"], "hbm_gbs": PEAK_HBM_GBS}
    out["method"] = ("va_probe_mfma: 4096 work-groups x 4 waves x 4000 rounds of 4 independent "
                     "v_mfma_f32_32x32x16; va_probe_copy: 1 GiB (4x the 256 MB last-level "
                     "cache), 65536 work-groups, 16 B per lane, read + write bytes; median of 5 "
                     "launches")
    del src, dst, sink
    torch.cuda.empty_cache()
    return out


def cpu_baseline(configs=(1, 2)):
    """The reference's CPU-runnable math on this host's cores (fp32, forward + backward), both
    constructions, at each configuration's shape; the faster construction of the last
    configuration (the headline shape) is the reported value."""
    import torch

    from hackaton_amd import workloads as wl

    threads = cpu_threads()
    torch.set_num_threads(threads)
    scale = 128 ** -0.5
    detail, total = {}, 0.0
    for cfg in configs:
        c = wl.CONFIGS[cfg]
        lengths = wl.config_lengths(cfg)
        q, k, v, do = wl.make_inputs(lengths, c["hq"], c["hkv"], torch.float32, seed=0,
                                     qk_scale=c["qk_scale"])
        grad = do.reshape(do.shape[0], -1)
        flops = wl.attention_flops(lengths, c["hq"])
        row = {}
        for name, fn in (("padded_masked", sdpa_padded_call),
                         ("per_document_causal", sdpa_per_document_call)):
            t0 = time.perf_counter()
            secs = time_cpu(fn, (q, k, v, grad, lengths, scale))
            total += time.perf_counter() - t0
            row[name] = {"ms": round(secs * 1e3, 3), "tflops": round(flops / secs / 1e12, 5)}
        best = max(row.values(), key=lambda x: x["tflops"])
        detail[f"config{cfg}"] = {"lengths": lengths, "hq": c["hq"], "hkv": c["hkv"],
                                  "flops": flops, **row, "best_tflops": best["tflops"]}
    last = detail[f"config{configs[-1]}"]
    return {"value": last["best_tflops"], "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": (f"torch CPU scaled_dot_product_attention fp32 fwd+autograd bwd, GQA via "
                       f"enable_gqa, padded tril&real mask (solution/test_attention.py:95-106) and "
                       f"per-document is_causal, faster of the two, best of >= 5 calls and "
                       f">= 2.5 s per construction after 2 warm-ups, "
                       f"one layer call of configuration {configs[-1]}'s shape; configuration 1 "
                       f"also timed; {threads} threads of {os.cpu_count()} logical CPUs, "
                       f"{cpu_model()}; {total:.1f} s of CPU work"),
            "cpu_model": cpu_model(), "logical_cpus": os.cpu_count(),
            "torch_threads": torch.get_num_threads(), "configs": detail}


# ------------------------------------------------------------------------------------------------
# GPU timing
# ------------------------------------------------------------------------------------------------
class LayerSet:
    """One layer-equivalent buffer set: inputs, outputs, lse and the backward workspace."""

    def __init__(self, torch, att, lengths, hq, hkv, dtype, qk_scale, seed):
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
        if att.bwd_workspace_needed(hq, hkv):
            self.ws, _ = att.bwd_workspace(n, hq, hkv, dev)
        else:  # Hq == Hkv: the kernels write dK/dV directly
            self.ws = torch.empty(0, dtype=torch.uint8, device=dev)
        self.n = n

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in
                   (self.q, self.k, self.v, self.do, self.out, self.lse, self.dq, self.dk,
                    self.dv, self.ws))


class Workload:
    """Buffer sets, plan and launch closures of one BASELINE configuration."""

    def __init__(self, cfg, n_sets=None):
        import torch

        from hackaton_amd import _lib
        from hackaton_amd import attention as att
        from hackaton_amd import workloads as wl

        self.torch, self.lib, self._lib, self.att = torch, _lib.lib(), _lib, att
        c = wl.CONFIGS[cfg]
        self.cfg, self.c = cfg, c
        self.lengths = wl.config_lengths(cfg)
        self.hq, self.hkv = c["hq"], c["hkv"]
        self.dtype = wl.torch_dtype(c["dtype"])
        self.dcode = {torch.float16: _lib.VA_F16, torch.bfloat16: _lib.VA_BF16}[self.dtype]
        self.scale = 128 ** -0.5
        dev = torch.device("cuda")
        self.plan = att._plan(att._cu_seqlens(self.lengths, dev), self.hq, self.hkv)
        first = LayerSet(torch, att, self.lengths, self.hq, self.hkv, self.dtype, c["qk_scale"],
                         1000)
        if n_sets is None:
            n_sets = max(2, min(LAYER_CALLS, -(-SET_BYTES_TARGET // first.nbytes())))
        self.sets = [first] + [LayerSet(torch, att, self.lengths, self.hq, self.hkv, self.dtype,
                                        c["qk_scale"], 1000 + i) for i in range(1, n_sets)]
        self.flops_call = wl.attention_flops(self.lengths, self.hq)
        torch.cuda.synchronize()

    def fwd(self, s, stream):
        p = self.plan
        self._lib.check(self.lib.va_fwd(s.q.data_ptr(), s.k.data_ptr(), s.v.data_ptr(),
                                        s.out.data_ptr(), s.lse.data_ptr(), p.fwd_items.data_ptr(),
                                        p.n_fwd, s.n, self.hq, self.hkv, 128, self.scale,
                                        self.dcode, stream), "va_fwd")

    def bwd(self, s, stream, stage=-1):
        p = self.plan
        argv = (s.do.data_ptr(), s.q.data_ptr(), s.k.data_ptr(), s.v.data_ptr(),
                s.out.data_ptr(), s.lse.data_ptr(), p.bwd_items.data_ptr(), p.n_bwd, s.n,
                self.hq, self.hkv, 128, self.scale, self.dcode, s.dq.data_ptr(), s.dk.data_ptr(),
                s.dv.data_ptr(), s.ws.data_ptr() if s.ws.numel() else None, s.ws.numel(), stream)
        stages = self.att.bwd_stages(self.plan, True, s.ws.numel() > 0) if stage < 0 else [stage]
        for st in stages:
            self._lib.check(self.lib.va_bwd_stage(st, *argv), "va_bwd_stage")

    def main_stage(self):
        """The backward's main kernel stage: reading the row statistics pass's output where the
        plan runs that pass."""
        return self._lib.VA_BWD_MAIN_STATS if self.plan.bwd_stats else self._lib.VA_BWD_MAIN

    def call(self, s, stream):
        self.fwd(s, stream)
        self.bwd(s, stream)

    def graph(self, launch):
        """One captured graph of `launch` over every buffer set."""
        torch = self.torch
        stream = torch.cuda.current_stream().cuda_stream
        for s in self.sets:  # warm-up outside the capture
            launch(s, stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            st = torch.cuda.current_stream().cuda_stream
            for s in self.sets:
                launch(s, st)
        g.replay()
        torch.cuda.synchronize()
        return g

    def replay_ms(self, g, reps):
        """Per-replay times (ms) of `reps` replays, each between two HIP events recorded on the
        stream the replays run on."""
        torch = self.torch
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        torch.cuda.synchronize()
        evs[0].record()
        for i in range(reps):
            g.replay()
            evs[i + 1].record()
        torch.cuda.synchronize()
        return [evs[i].elapsed_time(evs[i + 1]) for i in range(reps)]

    def kernel_us(self, reps):
        """Median per-launch duration of each kernel, captured alone."""
        lib = self._lib
        out = {}
        fwd_name = "fwd_lean_kernel" if lib.fwd_many_items(sum(self.lengths), self.hq) else \
            "fwd_kernel"
        # the row statistics pass (where the plan runs it) before the main kernel that reads them
        for name, launch in ((fwd_name, self.fwd),
                             ("bwd_stats_kernel", lambda s, st: self.bwd(s, st, lib.VA_BWD_STATS)),
                             ("bwd_kernel", lambda s, st: self.bwd(s, st, self.main_stage())),
                             ("bwd_gqa_sum_kernel",
                              lambda s, st: self.bwd(s, st, self.plan.bwd_finish_stage))):
            if name == "bwd_gqa_sum_kernel" and not self.gqa_sum_launched():
                continue
            if name == "bwd_stats_kernel" and not self.plan.bwd_stats:
                continue
            g = self.graph(launch)
            out[name] = median_us(self.replay_ms(g, reps), len(self.sets))
            del g
        return out

    def gqa_sum_launched(self):
        """The GQA sum runs unless Hq == Hkv or group items cover every key tile of the plan."""
        return self.plan.bwd_finish


def time_config(cfg, reps):
    """fwd+bwd call time (median over replays of a graph over the buffer sets) and kernel times
    at one configuration."""
    import torch

    w = Workload(cfg)
    g = w.graph(w.call)
    call_us = median_us(w.replay_ms(g, reps), len(w.sets))
    del g
    kus = w.kernel_us(reps)
    peak = PEAK_MFMA_TFLOPS[w.c["dtype"]]
    tflops = w.flops_call / (call_us * 1e-6) / 1e12
    res = {"workload": w.c["name"], "tokens": sum(w.lengths), "docs": len(w.lengths),
           "hq": w.hq, "hkv": w.hkv, "dtype": w.c["dtype"], "buffer_sets": len(w.sets),
           "call_us": round(call_us, 3), "tflops": round(tflops, 2),
           "pct_mfma_peak": round(100 * tflops / peak, 3),
           "kernels_us": {k: round(v, 3) for k, v in kus.items()}}
    del w
    torch.cuda.empty_cache()
    return res


def time_installed_path(cfg, reps, with_device_lengths=False):
    """PackedAttention as the patched decoder layer calls it (rotation, attention forward, attention
    backward and the inverse rotation, in its epilogues or as a pass of its own) at one
    configuration, captured in a graph with
    its autograd backward; with host lengths (cached host plan) and, if asked, device lengths
    (cu_seqlens and plan built on the device in every call). Each document is one padded batch
    row of the decoder's input (b_idx = document, t_idx = position), as the reference's packed
    step forms them for right-padded rows (solution/packed.py:156-172)."""
    import torch

    from hackaton_amd import attention as att
    from hackaton_amd import workloads as wl

    c = wl.CONFIGS[cfg]
    lengths = wl.config_lengths(cfg)
    hq, hkv, n = c["hq"], c["hkv"], sum(lengths)
    dtype = wl.torch_dtype(c["dtype"])
    dev = torch.device("cuda")
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)],
                        device=dev)
    b_idx, t_idx = (rows // seq).to(torch.int32), (rows % seq).to(torch.int32)
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, device=dev).float() / 128))
    emb = torch.arange(seq, device=dev).float()[:, None] * inv[None]
    emb = torch.cat((emb, emb), -1)[None]
    cos, sin = emb.cos(), emb.sin()
    # projections and their gradient, plus what the layer keeps (rotated q/k/v, O, lse)
    set_bytes = 2 * n * (hq + 2 * hkv) * 128 * 2 + 2 * n * hq * 128 * 2 + 4 * hq * n
    n_sets = max(2, min(LAYER_CALLS, -(-SET_BYTES_TARGET // set_bytes)))
    sets = []
    for i in range(n_sets):
        g = torch.Generator(device=dev).manual_seed(2000 + i)
        qk = c["qk_scale"]
        q = (torch.randn(n, hq * 128, device=dev, generator=g) * qk).to(dtype).requires_grad_()
        k = (torch.randn(n, hkv * 128, device=dev, generator=g) * qk).to(dtype).requires_grad_()
        v = torch.randn(n, hkv * 128, device=dev, generator=g).to(dtype).requires_grad_()
        grad = torch.randn(n, hq * 128, device=dev, generator=g).to(dtype)
        sets.append((q, k, v, grad))
    flops = wl.attention_flops(lengths, hq) * n_sets
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    res = {"workload": c["name"], "buffer_sets": n_sets,
           "backward": (("inverse rotation in the backward kernels' epilogues; "
                         + ("GQA sum of rotated partials" if plan.bwd_finish else
                            "group items write dK/dV at Hkv width, no GQA sum"))
                        if att.rotary_epilogues(n, hq) else
                        "per-head partials summed by the inverse rotation pass"),
           "row_statistics_pass": bool(plan.bwd_stats)}
    variants = [("host_lengths", lengths)]
    if with_device_lengths:
        variants.append(("device_lengths", torch.tensor(lengths, device=dev)))
    for label, lens in variants:
        def step():  # gradients returned, not accumulated into .grad (no add kernels)
            for q, k, v, grad in sets:
                out = att.packed_attention(q, k, v, cos, sin, b_idx, t_idx, seq, hq, hkv, lens,
                                           128 ** -0.5)
                torch.autograd.grad(out, (q, k, v), grad)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        graph.replay()
        torch.cuda.synchronize()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        evs[0].record()
        for i in range(reps):
            graph.replay()
            evs[i + 1].record()
        torch.cuda.synchronize()
        ms = statistics.median(evs[i].elapsed_time(evs[i + 1]) for i in range(reps))
        res[label] = {"call_us": round(ms * 1e3 / n_sets, 3),
                      "tflops": round(flops / (ms * 1e-3) / 1e12, 2)}
        del graph
    del sets
    torch.cuda.empty_cache()
    return res


INSTALLED_NOTE = ("layer calls over resident buffer sets per replay, projections (N, H*128) in "
                  "the configuration's dtype, RoPE tables of theta 1e6; includes the rotation and "
                  "its inverse, not the projections; bare_call_us is the same configuration's "
                  "fwd+bwd kernels alone (by_config)")


def main(argv=None):
    args = parse(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the attention path needs no "
                                   "collective; run with --gpus 1 (see the sharding note in the "
                                   "design document)"}))
        sys.exit(2)
    reps = max(args.reps, MIN_REPS)

    import torch

    from hackaton_amd import workloads as wl

    torch.cuda.set_device(0)
    w = Workload(args.config, n_sets=LAYER_CALLS)
    cfg = w.c
    print(f"[bench] configuration {args.config} ({cfg['name']}), {len(w.sets)} buffer sets",
          flush=True)

    if args.pmc_probe:
        # calibration kernel of known traffic: y = x * 1 over 64 Mi fp32 (256 MiB read, 256 MiB
        # written), then every attention kernel once per buffer set
        dev = torch.device("cuda")
        x = torch.randn(64 << 20, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            torch.mul(x, 1.0, out=y)
        stream = torch.cuda.current_stream().cuda_stream
        for s in w.sets:
            w.fwd(s, stream)
        if w.plan.bwd_stats:
            for s in w.sets:
                w.bwd(s, stream, w._lib.VA_BWD_STATS)
        for s in w.sets:
            w.bwd(s, stream, w.main_stage())
        if w.gqa_sum_launched():
            for s in w.sets:
                w.bwd(s, stream, w.plan.bwd_finish_stage)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": cfg["name"], "copy_read_bytes": x.numel() * 4,
                          "copy_write_bytes": y.numel() * 4, "launches_per_kernel": len(w.sets)}),
              flush=True)
        return

    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(args.warmup):
        for s in w.sets:
            w.call(s, stream)
    torch.cuda.synchronize()
    graph = w.graph(w.call)

    # ---- timed region: K graph replays, each 28 layer calls ----------------------------------
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
    del graph
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.4f} ms per step", flush=True)

    flops_step = w.flops_call * LAYER_CALLS
    tflops = flops_step / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_MFMA_TFLOPS[cfg["dtype"]]

    # ---- kernel durations: median of >= 20 replays, HIP events on the launch stream ----------
    kus = w.kernel_us(reps)
    models = kernel_models(w.lengths, w.hq, w.hkv)
    dom_name = max(kus, key=lambda k: kus[k])
    dom = models[dom_name]
    traffic = measured_traffic(dom_name, cfg["name"])
    roofline_ = {"kernel": dom_name,
                 **roofline(dom["flops"], dom["bytes"], kus[dom_name], peak),
                 "traffic": traffic, "avg_us": round(kus[dom_name], 3),
                 "timing": f"median of {reps} graph replays of {len(w.sets)} launches",
                 "flops_per_launch": dom["flops"], "algorithmic_bytes": dom["bytes"],
                 "traffic_over_algorithmic": (round(traffic / dom["bytes"], 3)
                                              if traffic and dom["bytes"] else None)}
    print(f"[bench] kernels {json.dumps({k: round(v, 3) for k, v in kus.items()})}", flush=True)

    by_config = {f"config{args.config}": {
        "workload": cfg["name"], "tokens": sum(w.lengths), "docs": len(w.lengths),
        "hq": w.hq, "hkv": w.hkv, "dtype": cfg["dtype"], "buffer_sets": len(w.sets),
        "call_us": round(ms_per_step * 1e3 / LAYER_CALLS, 3), "tflops": round(tflops, 2),
        "pct_mfma_peak": round(100 * tflops / peak, 3),
        "kernels_us": {k: round(v, 3) for k, v in kus.items()}}}
    del w
    torch.cuda.empty_cache()
    for cfg_other in by_config_list(args):
        if cfg_other == args.config:
            continue
        by_config[f"config{cfg_other}"] = time_config(cfg_other, reps)
        print(f"[bench] config {cfg_other}: {json.dumps(by_config[f'config{cfg_other}'])}",
              flush=True)

    installed = None
    if not args.no_installed_path:
        installed = {"note": INSTALLED_NOTE}
        for cfg_i in [args.config] + [c for c in by_config_list(args) if c != args.config]:
            r = time_installed_path(cfg_i, reps, with_device_lengths=cfg_i == args.config)
            bare = by_config.get(f"config{cfg_i}", {}).get("call_us")
            if bare:
                r["bare_call_us"] = bare
                r["over_bare"] = round(r["host_lengths"]["call_us"] / bare, 3)
            installed[f"config{cfg_i}"] = r
            print(f"[bench] installed path config {cfg_i}: {json.dumps(r)}", flush=True)

    ceilings = measure_ceilings()
    print(f"[bench] measured ceilings {json.dumps(ceilings)}", flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline((1, args.config))
        print("[bench] cpu baseline done", flush=True)

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
        "config": {"workload": cfg["name"], "tokens": sum(wl.config_lengths(args.config)),
                   "docs": len(wl.config_lengths(args.config)), "hq": cfg["hq"],
                   "hkv": cfg["hkv"], "head_dim": 128, "layer_calls": LAYER_CALLS,
                   "causal_flops_per_step": flops_step},
        "pct_mfma_peak": round(100 * tflops / peak, 3),
        "wall_ms_per_step": round(wall_ms, 5),
        "kernels_us": {k: round(v, 3) for k, v in kus.items()},
        "kernels_tflops": {k: round(models[k]["flops"] / (v * 1e-6) / 1e12, 2)
                           for k, v in kus.items() if models[k]["flops"]},
        "roofline": roofline_,
        "ceilings_measured": ceilings,
        "by_config": by_config,
        "installed_path": installed,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
