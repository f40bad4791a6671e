"""CPU checks of bench.py's reporting: the roofline classification, the one-GPU refusal, the
lookup of committed HBM traffic, and the per-launch FLOP and byte models it divides by."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from hackaton_amd import workloads as wl  # noqa: E402


def test_ridge_point_is_peak_ratio():
    r = bench.roofline(flops=1.0, nbytes=1.0, us=1.0, peak_tflops=2516.6)
    assert r["ridge"] == pytest.approx(2516.6e12 / 8000e9, abs=0.05)   # 314.6 FLOP/B


def test_below_ridge_is_hbm_bound():
    # 100 FLOP per byte, 1 GB in 1 ms -> 1000 GB/s of 8000, 100 TFLOP/s of MFMA.
    r = bench.roofline(flops=100e9, nbytes=1e9, us=1000.0, peak_tflops=2516.6)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["achieved"] == pytest.approx(1000.0)
    assert r["frac"] == pytest.approx(0.125)
    assert r["mfma_tflops"] == pytest.approx(100.0)
    assert r["mfma_frac"] == pytest.approx(100.0 / 2516.6, abs=1e-4)


def test_above_ridge_is_mfma_bound():
    # 1000 FLOP per byte, 1e12 FLOP in 1 ms -> 1000 TFLOP/s.
    r = bench.roofline(flops=1e12, nbytes=1e9, us=1000.0, peak_tflops=2516.6)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2516.6
    assert r["achieved"] == pytest.approx(1000.0)
    assert r["frac"] == pytest.approx(1000.0 / 2516.6, abs=1e-4)
    assert r["arithmetic_intensity"] == pytest.approx(1000.0)


def test_config2_kernels_sit_below_the_ridge():
    lengths = wl.config_lengths(2)
    cfg = wl.CONFIGS[2]
    models = bench.kernel_models(lengths, cfg["hq"], cfg["hkv"])
    ridge = 2516.6e12 / 8000e9
    for name in ("fwd_kernel", "bwd_kernel"):
        assert models[name]["flops"] / models[name]["bytes"] < ridge
    # the backward's arithmetic intensity at 4 x 512 tokens: 8.07 GFLOP over 29.56 MB
    bwd = models["bwd_kernel"]
    assert bwd["bytes"] == 2048 * 14432
    assert bwd["flops"] / bwd["bytes"] == pytest.approx(273.0, abs=0.5)


def test_causal_pairs_match_mask_count():
    lengths = [1, 7, 64, 130, 0, 3]
    mask = 0
    for L in lengths:
        mask += int(np.tril(np.ones((L, L), dtype=np.int64)).sum())
    assert wl.causal_pairs(lengths) == mask


def test_byte_models_by_hand():
    # Hq=12, Hkv=2, D=128, fp16, one token:
    #   q 12*128*2 = 3072, k+v 2*2*128*2 = 1024, O 3072, lse 12*4 = 48.
    assert wl.forward_bytes(1, 12, 2) == 3072 + 1024 + 3072 + 48
    #   backward: reads q (3072), k+v (1024), O and dO (2*3072), lse and delta (2*48); writes
    #   dq (3072) and dk+dv at Hkv width (1024).
    assert wl.backward_bytes(1, 12, 2) == 3072 + 1024 + 2 * 3072 + 96 + 3072 + 1024 == 14432
    assert wl.forward_bytes(1, 12, 2) + wl.backward_bytes(1, 12, 2) == 21648
    assert wl.algorithmic_bytes(7, 12, 2) == 7 * 21648
    #   per-head dK/dV partials: 2 tensors x 12 heads; GQA reduction reads them, writes 2*2 heads.
    assert wl.partial_write_bytes(1, 12, 2) == 24 * 128 * 2
    assert wl.gqa_sum_bytes(1, 12, 2) == (24 + 4) * 128 * 2
    assert wl.gqa_sum_bytes(5, 4, 4) == 0 and wl.partial_write_bytes(5, 4, 4) == 0


def test_forward_flops_by_hand():
    # One document of 2 tokens: 3 causal pairs, two products of 2*D FLOPs per pair and head.
    assert wl.forward_flops([2], 1, 128) == 3 * 2 * 2 * 128
    assert wl.attention_flops([2], 1, 128) == pytest.approx(3.5 * 3 * 2 * 2 * 128)


def test_measured_traffic_reads_committed_profile():
    name = wl.CONFIGS[2]["name"]
    for kernel in ("fwd_kernel", "bwd_kernel", "bwd_gqa_sum_kernel"):
        t = bench.measured_traffic(kernel, name)
        assert isinstance(t, int) and t > 0
    assert bench.measured_traffic("no_such_kernel", name) is None
    assert bench.measured_traffic("fwd_kernel", "no_such_workload") is None


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert p.returncode == 2
    msg = json.loads(p.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_median_per_launch():
    assert bench.median_us([1.0, 3.0, 2.0], 28) == pytest.approx(2.0e3 / 28)


@pytest.mark.parametrize("lengths,hq,hkv", [([9, 1, 4], 4, 2), ([6, 3], 2, 2)])
def test_cpu_baseline_constructions_match_the_oracle(lengths, hq, hkv):
    """Both CPU-baseline constructions (the reference test's padded tril & real mask and
    per-document is_causal) compute the oracle's outputs and gradients."""
    import torch

    from oracle import attention_oracle as orc

    q, k, v, do = wl.make_inputs(lengths, hq, hkv, torch.float32, seed=4)
    grad = do.reshape(do.shape[0], -1)
    cu = orc.cu_seqlens_from_lengths(lengths)
    f64 = [t.double().numpy() for t in (q, k, v, do)]
    o_ref, lse = orc.attention_forward(f64[0], f64[1], f64[2], cu, 0.3)
    refs = orc.attention_backward(f64[0], f64[1], f64[2], o_ref, lse, f64[3], cu, 0.3)
    for fn in (bench.sdpa_padded_call, bench.sdpa_per_document_call):
        out, grads = fn(q, k, v, grad, lengths, 0.3)
        np.testing.assert_allclose(out.numpy().reshape(o_ref.shape), o_ref, atol=1e-5)
        for mine, ref in zip(grads, refs):
            np.testing.assert_allclose(mine.numpy(), ref, atol=1e-5)


def test_cpu_baseline_reports_cores_and_model(monkeypatch):
    """The CPU leg states the threads it used, the logical CPU count and the CPU model; run on a
    tiny configuration so that the test stays fast."""
    import torch

    monkeypatch.setitem(wl.CONFIGS, 99, dict(name="tiny", hq=4, hkv=2, dtype="float16",
                                             qk_scale=1.0))
    real = wl.config_lengths
    monkeypatch.setattr(wl, "config_lengths", lambda c, seed=0: [5, 3] if c == 99 else real(c))
    threads = torch.get_num_threads()
    try:
        r = bench.cpu_baseline((99,))
    finally:
        torch.set_num_threads(threads)
    assert r["unit"] == "TFLOP/s" and r["value"] > 0 and r["cores"] >= 1
    assert r["cpu_model"] and r["logical_cpus"] >= 1
    row = r["configs"]["config99"]
    assert set(row) >= {"padded_masked", "per_document_causal", "best_tflops"}
