"""Writes the committed golden vectors of the varlen attention path.

The reference ships no golden files for this path (its tests draw seeded CUDA inputs, which the
CPU cannot regenerate), so the fixtures are produced by the CPU oracle, which tests/test_oracle.py
pins to torch's SDPA/autograd, the reference test's masked-SDPA construction, transformers'
rotary embedding, closed forms and finite differences. The lengths include the reference test's
pattern of a long, medium and a 1-token document (solution/test_attention.py:84).

Inputs are stored in their 16-bit form (bf16 as raw uint16 bits); expected outputs in fp32,
computed in fp64 from exactly those 16-bit values.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention_oracle as orc  # noqa: E402

CASES = {
    "fp16_g6": dict(lengths=[37, 12, 1, 20], hq=6, hkv=1, dtype=torch.float16, qk=1.0, seed=11),
    "bf16_g7_peaky": dict(lengths=[45, 3, 17], hq=7, hkv=1, dtype=torch.bfloat16, qk=3.0,
                          seed=12),
}


def to_store(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def make(name, lengths, hq, hkv, dtype, qk, seed):
    n = sum(lengths)
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n, hq, 128, generator=g) * qk).to(dtype)
    k = (torch.randn(n, hkv, 128, generator=g) * qk).to(dtype)
    v = torch.randn(n, hkv, 128, generator=g).to(dtype)
    do = torch.randn(n, hq, 128, generator=g).to(dtype)
    f64 = [t.double().numpy() for t in (q, k, v, do)]
    cu = orc.cu_seqlens_from_lengths(lengths)
    scale = 128 ** -0.5
    o, lse = orc.attention_forward(f64[0], f64[1], f64[2], cu, scale)
    dq, dk, dv = orc.attention_backward(f64[0], f64[1], f64[2], o, lse, f64[3], cu, scale)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"), lengths=np.asarray(lengths, dtype=np.int32),
        hq=hq, hkv=hkv, dtype=str(dtype).replace("torch.", ""), scale=scale,
        q=to_store(q), k=to_store(k), v=to_store(v), do=to_store(do),
        o=o.astype(np.float32), lse=lse.astype(np.float32), dq=dq.astype(np.float32),
        dk=dk.astype(np.float32), dv=dv.astype(np.float32))


def load(name):
    """Fixture as a dict; 16-bit inputs returned as torch tensors of their dtype."""
    z = np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False)
    dtype = getattr(torch, str(z["dtype"]))
    out = {key: z[key] for key in z.files}
    for key in ("q", "k", "v", "do"):
        raw = torch.from_numpy(z[key].copy())
        out[key] = raw.view(torch.bfloat16) if dtype == torch.bfloat16 else raw
    out["dtype"] = dtype
    out["lengths"] = [int(x) for x in z["lengths"]]
    return out


if __name__ == "__main__":
    for case, cfg in CASES.items():
        make(case, **cfg)
        print("wrote", case)
