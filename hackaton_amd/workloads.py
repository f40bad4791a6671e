"""Synthetic workloads of the benchmark configurations and their algorithmic FLOP / byte counts.

Document lengths are drawn with numpy.random.default_rng(seed); values (Q, K, V, dO) with a CPU
torch.Generator seeded the same, cast once to the element type. Rows never share a document:
greedy packing fills rows in order and truncates the document that overflows a row so the row is
filled exactly; rows are then concatenated on the packed token axis.
"""

import math

import numpy as np
import torch

HEAD_DIM = 128
LOGNORMAL_SIGMA = 0.75  # not fixed by the benchmark description; recorded here


def pack_greedy(doc_lengths, rows, row_tokens):
    """Documents in order into `rows` rows of `row_tokens`; the overflowing document is cut to
    fill the row exactly, a new row starts with the next document. Returns the packed lengths
    (a list whose sum is <= rows * row_tokens)."""
    out = []
    row, used = 0, 0
    for length in doc_lengths:
        length = int(length)
        while length > 0 and row < rows:
            take = min(length, row_tokens - used)
            out.append(take)
            used += take
            length = 0  # the remainder of a cut document is dropped
            if used == row_tokens:
                row, used = row + 1, 0
        if row >= rows:
            break
    return out


def lognormal_docs(rng, median, lo, hi, total):
    """Log-normal lengths (median, sigma LOGNORMAL_SIGMA) clipped to [lo, hi], enough to cover
    `total` tokens."""
    docs, s = [], 0
    while s < total:
        x = int(np.clip(round(rng.lognormal(math.log(median), LOGNORMAL_SIGMA)), lo, hi))
        docs.append(x)
        s += x
    return docs


CONFIGS = {
    1: dict(name="cpu_ref_1p5b_fp32", hq=12, hkv=2, dtype="float32", qk_scale=1.0),
    2: dict(name="qwen2.5-1.5b_4x512_causal_fp16", hq=12, hkv=2, dtype="float16", qk_scale=1.0,
            layer_calls=28),
    3: dict(name="qwen2.5-1.5b_packed_lognormal180_4x2048_fp16", hq=12, hkv=2, dtype="float16",
            qk_scale=1.0),
    4: dict(name="qwen2.5-1.5b_packed_64docs_16384_bf16_qk3", hq=12, hkv=2, dtype="bfloat16",
            qk_scale=3.0),
    5: dict(name="qwen2.5-7b_packed_lognormal400_4x8192_bf16", hq=28, hkv=4, dtype="bfloat16",
            qk_scale=1.0),
}


def config_lengths(cfg, seed=0):
    """Packed document lengths of benchmark configuration `cfg` (1..5)."""
    rng = np.random.default_rng(seed)
    if cfg == 1:
        return [int(x) for x in rng.integers(64, 512, size=4, endpoint=True)]
    if cfg == 2:
        return [512] * 4
    if cfg == 3:
        return pack_greedy(lognormal_docs(rng, 180, 16, 512, 4 * 2048 + 512), 4, 2048)
    if cfg == 4:
        docs = [int(x) for x in rng.integers(8, 512, size=64, endpoint=True)]
        return pack_greedy(docs, 1, 16384)
    if cfg == 5:
        return pack_greedy(lognormal_docs(rng, 400, 32, 4096, 4 * 8192 + 4096), 4, 8192)
    raise ValueError(f"unknown configuration {cfg}")


def torch_dtype(name):
    return {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}[name]


def make_inputs(lengths, hq, hkv, dtype, seed=0, qk_scale=1.0, device="cpu"):
    """q (N, hq, D), k, v (N, hkv, D), dout (N, hq, D) drawn from N(0, 1) (q, k times qk_scale),
    cast once to `dtype`, then moved to `device`."""
    n = int(sum(lengths))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, hq, HEAD_DIM, generator=g) * qk_scale
    k = torch.randn(n, hkv, HEAD_DIM, generator=g) * qk_scale
    v = torch.randn(n, hkv, HEAD_DIM, generator=g)
    do = torch.randn(n, hq, HEAD_DIM, generator=g)
    return [t.to(dtype).to(device) for t in (q, k, v, do)]


def causal_pairs(lengths):
    return sum(int(x) * (int(x) + 1) // 2 for x in lengths if int(x) > 0)


def attention_flops(lengths, hq, d=HEAD_DIM):
    """Causal FLOPs of one forward + backward: 3.5 * 4 * Hq * D * sum L (L + 1) / 2 (the forward is
    2 products of 2 FLOPs per pair and head dimension, the backward 5; recompute not counted)."""
    return 3.5 * 4.0 * hq * d * causal_pairs(lengths)


def forward_flops(lengths, hq, d=HEAD_DIM):
    return 4.0 * hq * d * causal_pairs(lengths)


def algorithmic_bytes(n_tokens, hq, hkv, elem=2, d=HEAD_DIM):
    """HBM bytes one forward + backward must move at least (inputs read once, outputs written
    once): forward reads q, k, v, writes O and lse; backward reads q, k, v, O, dO, lse, writes dq,
    dk, dv (delta is recomputed from O and dO)."""
    fwd = n_tokens * ((hq + 2 * hkv) * d * elem + hq * d * elem + 4 * hq)
    bwd = n_tokens * ((hq + 2 * hkv) * d * elem + 2 * hq * d * elem + 8 * hq
                      + (hq + 2 * hkv) * d * elem)
    return fwd + bwd


def backward_bytes(n_tokens, hq, hkv, elem=2, d=HEAD_DIM):
    """HBM bytes one attention backward must move at least: reads q, k, v, O, dO and lse (and the
    row statistic delta, counted like lse), writes dq, dk and dv at their own widths (dK/dV have
    Hkv heads: the GQA sum is part of the backward)."""
    return n_tokens * ((hq + 2 * hkv) * d * elem + 2 * hq * d * elem + 8 * hq
                       + (hq + 2 * hkv) * d * elem)


def partial_write_bytes(n_tokens, hq, hkv, elem=2, d=HEAD_DIM):
    """Bytes of per-query-head dK/dV partials one backward writes (and the GQA sum reads back)
    when the query heads of a group are split over work items: an intermediate of this
    implementation, not algorithmic traffic."""
    if hq == hkv:
        return 0
    return n_tokens * 2 * hq * d * elem


def forward_bytes(n_tokens, hq, hkv, elem=2, d=HEAD_DIM):
    return n_tokens * ((hq + 2 * hkv) * d * elem + hq * d * elem + 4 * hq)


def gqa_sum_bytes(n_tokens, hq, hkv, elem=2, d=HEAD_DIM):
    """HBM bytes a separate GQA reduction moves: reads the per-head dK/dV partials, writes dK/dV
    (the dK/dV writes are algorithmic; the partial reads are not)."""
    if hq == hkv:
        return 0
    return n_tokens * 2 * (hq + hkv) * d * elem
