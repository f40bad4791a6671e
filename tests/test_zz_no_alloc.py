"""va_bwd_noalloc: the attention backward with its dK/dV partials in the library's static device
scratch instead of a workspace argument, checked through the C ABI against va_bwd (the same
kernels on the same inputs: bitwise equal), on two calls in a row, the second one smaller, so the
second reuses the scratch the first one filled. (Its refusal of sizes beyond the scratch needs no
GPU and is tested in test_abi.py.)"""

import pytest
import torch

from hackaton_amd import _lib
from hackaton_amd import attention as att
from hackaton_amd import workloads as wl

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def noalloc_fn():
    return att.lib().va_bwd_noalloc


def backward_both_ways(lengths, hq, hkv, dtype, seed):
    dev = torch.device("cuda")
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(lengths, hq, hkv, dtype, seed=seed))
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    out, lse = att.attention_forward(q, k, v, plan, SCALE)
    ref = att.attention_backward(do, q, k, v, out, lse, plan, SCALE)  # va_bwd with a workspace
    n = q.shape[0]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    code = _lib.VA_F16 if dtype == torch.float16 else _lib.VA_BF16
    rc = noalloc_fn()(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                      lse.data_ptr(), plan.bwd_items.data_ptr(), plan.n_bwd, n, hq, hkv, 128,
                      SCALE, code, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), att._stream())
    att.check(rc, "va_bwd_noalloc")
    torch.cuda.synchronize()
    return ref, (dq, dk, dv)


def test_noalloc_backward_matches_va_bwd_twice_in_a_row():
    for lengths, hq, hkv, dtype in (([512, 300, 77, 1], 12, 2, torch.float16),
                                    ([200, 33], 12, 2, torch.float16),
                                    ([130, 5], 28, 4, torch.bfloat16)):
        print(f"\n[case] va_bwd_noalloc {lengths} {hq}/{hkv} {dtype}", flush=True)
        ref, got = backward_both_ways(lengths, hq, hkv, dtype, seed=sum(lengths))
        for name, a, b in zip(("dq", "dk", "dv"), ref, got):
            assert torch.equal(a, b), name
