"""Randomised GPU parity of the packed attention path: seeded random batches (document counts,
lengths with the tile-boundary and empty-document edges, GQA shapes from G = 1 to G = 8, fp16 and
bf16) through varlen_attention, each checked against the CPU oracle with the tolerances of
test_gpu_attention.py, against the same batch with device-side lengths (bitwise: the device plan
must give the host plan's results) and against a second run (bitwise: the path is deterministic).

The cases come from a fixed seed, so a failure names a reproducible case; they cover what the
hand-written cases do not combine: the host planner's choice of per-head, pair and group items
and of the forward kernel, for random mixes of short and long documents.
"""

import numpy as np
import pytest
import torch

from hackaton_amd import attention as att
from hackaton_amd import workloads as wl
from tests.test_gpu_attention import (SCALE, banner, check_all, check_packed_attention, oracle,
                                      run_varlen)

pytestmark = pytest.mark.gpu

# (Hq, Hkv): the benchmark shapes (G = 6, 7), the reference's expanded form (G = 1), and G = 2,
# 4 and 8
SHAPES = [(12, 2), (28, 4), (8, 8), (6, 3), (4, 1), (16, 2)]
# lengths with a tile edge: the 64 / 128-row tiles of the kernels and the 32-row steps
EDGES = [0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 384, 511, 512]


def fuzz_cases(n=24, seed=20261202):
    """Every fourth case is a long batch (up to 16 documents, 5,200 tokens), long enough at 16 and
    28 query heads for the pair and group backward items and the many-item forward kernel."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        hq, hkv = SHAPES[i % len(SHAPES)]
        dtype = torch.float16 if rng.random() < 0.6 else torch.bfloat16
        long_batch = i % 4 == 3
        max_tokens = 5200 if long_batch else 1500
        lengths = []
        for _ in range(int(rng.integers(10, 17) if long_batch else rng.integers(1, 9))):
            r = rng.random()
            if r < 0.35:
                lengths.append(int(rng.choice(EDGES)))
            elif r < 0.85:
                lengths.append(int(rng.integers(1, 400)))
            else:
                lengths.append(int(rng.integers(400, 900)))
        while sum(lengths) > max_tokens:
            lengths.pop()
        if sum(lengths) == 0:
            lengths.append(int(rng.integers(1, 300)))
        cases.append((i, lengths, hq, hkv, dtype))
    return cases


@pytest.mark.parametrize("i,lengths,hq,hkv,dtype", fuzz_cases())
def test_random_batches_match_oracle_device_lengths_and_rerun(i, lengths, hq, hkv, dtype):
    banner("fuzz", i, lengths, hq, hkv, dtype)
    n = sum(lengths)
    q, k, v, do = wl.make_inputs([x for x in lengths if x], hq, hkv, dtype, seed=1000 + i)
    host = run_varlen(q, k, v, do, lengths)
    check_all(host[0], host[1:], oracle(q, k, v, do, lengths), dtype, n, hq)
    again = run_varlen(q, k, v, do, lengths)
    for a, b in zip(host, again):
        assert torch.equal(a, b), "second run differs"
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.varlen_attention(qd, kd, vd, torch.tensor(lengths, device="cuda"), SCALE)
    out.backward(do.cuda().reshape(out.shape))
    torch.cuda.synchronize()
    for a, b in zip(host, (out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu())):
        assert torch.equal(a, b), "device lengths differ from host lengths"


def packed_fuzz_cases(n=12, seed=20261203):
    """Batches for the installed path: short lists (the per-head partials and the inverse rotation
    pass) and, every third case, lists long enough for the rotary epilogues (ceil(N / 128) Hq >=
    512)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        hq, hkv = SHAPES[(i + 1) % len(SHAPES)]
        dtype = torch.float16 if rng.random() < 0.5 else torch.bfloat16
        long_batch = i % 3 == 2
        target = (512 // hq + 2) * 128 if long_batch else int(rng.integers(50, 1200))
        lengths = []
        while sum(lengths) < target:
            lengths.append(int(rng.choice(EDGES)) if rng.random() < 0.3
                           else int(rng.integers(1, 700)))
        cases.append((i, lengths, hq, hkv, dtype))
    return cases


@pytest.mark.parametrize("i,lengths,hq,hkv,dtype", packed_fuzz_cases())
def test_random_batches_through_packed_attention_match_oracle(i, lengths, hq, hkv, dtype):
    banner("packed fuzz", i, len(lengths), sum(lengths), hq, hkv, dtype,
           "rotary epilogues" if att.rotary_epilogues(sum(lengths), hq) else "partials route")
    check_packed_attention(lengths, hq, hkv, dtype, seed=2000 + i)
