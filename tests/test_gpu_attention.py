"""GPU parity of the HIP attention path against the CPU oracle, the golden vectors and the
reference's own PyTorch constructions (solution/test_attention.py, test_offload.py).

Tolerances (element type of the inputs; the oracle runs in fp64 on the same 16-bit values):
  fp16: O max-abs <= 2e-3; dQ/dK/dV max|err| / max|ref| <= 1e-2 (and assert_close rtol=atol=1e-2
        as the reference test); lse max-abs <= 1e-3.
  bf16: O max-abs <= 1.6e-2; dQ/dK/dV max|err| / max|ref| <= 5e-2; lse max-abs <= 1e-2
        (fp16 bounds x 8 for the 3 fewer mantissa bits; no reference counterpart: the reference
        computes in fp16 only).
"""

import ctypes

import numpy as np
import pytest
import torch

from hackaton_amd import attention as att
from hackaton_amd import workloads as wl
from oracle import attention_oracle as orc
from tests.golden.make_golden import CASES as GOLDEN, load as load_golden

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
TOL = {torch.float16: dict(o=2e-3, g=1e-2, lse=1e-3), torch.bfloat16: dict(o=1.6e-2, g=5e-2,
                                                                             lse=1e-2)}


def banner(*what):
    print("\n[case]", *what, flush=True)


def run_varlen(q, k, v, do, lengths, scale=SCALE):
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.varlen_attention(qd, kd, vd, lengths, scale)
    out.backward(do.cuda().reshape(out.shape))
    torch.cuda.synchronize()
    return out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()


def oracle(q, k, v, do, lengths, scale=SCALE):
    f64 = [t.double().numpy() for t in (q, k, v, do)]
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(f64[0], f64[1], f64[2], cu, scale)
    dq, dk, dv = orc.attention_backward(f64[0], f64[1], f64[2], o, lse, f64[3], cu, scale)
    return o, lse, dq, dk, dv


def rel(mine, ref):
    """max|err| / max|ref|, with max|ref| floored at 0.1 so that an exactly-zero gradient (dQ of
    a 1-token document: dS = P (dP - delta) = 0) is judged on an absolute scale."""
    ref = np.asarray(ref, dtype=np.float64)
    err = np.max(np.abs(np.asarray(mine, dtype=np.float64) - ref))
    return float(err / max(np.max(np.abs(ref)), 0.1))


def check_all(out, grads, ref, dtype, n, hq):
    tol = TOL[dtype]
    o_ref, _lse, dq_ref, dk_ref, dv_ref = ref
    err_o = float(np.max(np.abs(out.float().numpy().reshape(n, hq, 128) - o_ref)))
    assert err_o <= tol["o"], f"O max-abs {err_o}"
    for name, mine, theirs in zip("qkv", grads, (dq_ref, dk_ref, dv_ref)):
        r = rel(mine.float().numpy(), theirs)
        assert r <= tol["g"], f"d{name} rel {r}"
        if dtype == torch.float16:
            torch.testing.assert_close(mine.float(), torch.from_numpy(theirs).float(), rtol=1e-2,
                                       atol=1e-2)


CASES = [
    ([64, 37, 50, 12], 12, 2, torch.float16),
    ([334, 200, 100, 7], 12, 2, torch.float16),
    ([64, 37, 50, 12], 12, 12, torch.float16),      # reference's expanded K/V form (G = 1)
    ([1], 12, 2, torch.float16),
    ([1, 1, 1, 2, 3], 4, 1, torch.float16),
    ([127, 128, 129, 255, 256, 257], 12, 2, torch.float16),
    ([300, 45, 1], 28, 4, torch.bfloat16),          # 7B heads, G = 7
    ([64, 37, 50, 12], 12, 2, torch.bfloat16),
    ([1000, 24], 12, 2, torch.float16),
    ([334, 0, 200, 100, 7], 12, 2, torch.float16),  # an empty document between others
    ([0, 5, 0, 33], 4, 2, torch.bfloat16),          # empty first and inner documents
]


@pytest.mark.parametrize("lengths,hq,hkv,dtype", CASES)
def test_varlen_matches_oracle(lengths, hq, hkv, dtype):
    banner("varlen", lengths, hq, hkv, dtype)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=sum(lengths))
    out, *grads = run_varlen(q, k, v, do, lengths)
    check_all(out, grads, oracle(q, k, v, do, lengths), dtype, sum(lengths), hq)


def padded_fwd_plan(plan, min_items):
    """The forward items of `plan` followed by empty items up to `min_items` (which the kernels
    skip), as a device-built plan pads its list."""
    items = torch.zeros(max(min_items, plan.n_fwd), 4, dtype=torch.int32, device="cuda")
    items[: plan.n_fwd] = plan.fwd_items[: plan.n_fwd]
    return items


@pytest.mark.parametrize("lengths,hq,hkv,dtype", CASES + [([300, 45, 1, 128], 12, 2, "peaky")])
def test_many_item_forward_matches_oracle(lengths, hq, hkv, dtype):
    """The forward kernel that runs for many items (ceil(N / 128) Hq >= VA_FWD_MANY_ITEMS = 512;
    one wave per query strip over all key tiles, no halves to merge), forced on small cases with
    va_fwd_kernel(VA_FWD_MANY) over the plan padded with empty items: O and lse against the
    oracle, and the backward run from them."""
    qk = 3.0 if dtype == "peaky" else 1.0
    dtype = torch.bfloat16 if dtype == "peaky" else dtype
    banner("many-item forward", lengths, hq, hkv, dtype, qk)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=sum(lengths) + 1, qk_scale=qk)
    n = sum(lengths)
    dev = torch.device("cuda")
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    items = padded_fwd_plan(plan, 512)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    out = torch.empty_like(qd)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    att.check(att.lib().va_fwd_kernel(att._lib.VA_FWD_MANY, qd.data_ptr(), kd.data_ptr(),
                                      vd.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                      items.data_ptr(), items.shape[0], n, hq, hkv, 128, SCALE,
                                      0 if dtype == torch.float16 else 1, att._stream()),
              "va_fwd_kernel")
    dq, dk, dv = att.attention_backward(do.to(dev), qd, kd, vd, out, lse, plan, SCALE)
    torch.cuda.synchronize()
    ref = oracle(q, k, v, do, lengths)
    err_lse = float(np.max(np.abs(lse.cpu().numpy() - ref[1])))
    assert err_lse <= TOL[dtype]["lse"], err_lse
    check_all(out.cpu(), (dq.cpu(), dk.cpu(), dv.cpu()), ref, dtype, n, hq)


@pytest.mark.parametrize("lengths,hq,hkv,dtype", [([512] * 4, 12, 2, torch.float16),
                                                   ([450, 450, 60], 12, 2, torch.bfloat16),
                                                   ([200, 70, 33], 28, 4, torch.bfloat16)])
def test_narrow_forward_items_match_the_oracle(lengths, hq, hkv, dtype):
    """The host plan splits the last tile of the longest documents into narrow 64-query items
    (VA_PLAN_FWD_NARROW: configuration 2's 48 longest items, partial second halves of 450-token
    documents, G = 7): O and lse of both forward kernels over that list (the 8-wave kernel's
    four-phase walk, the many-item kernel over the list padded with empty items) against the
    oracle, and against the same kernel over the unsplit list to rounding."""
    banner("narrow forward", lengths, hq, hkv, dtype)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=sum(lengths) + hq)
    n = sum(lengths)
    dev = torch.device("cuda")
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    narrow = (plan.fwd_items[: plan.n_fwd, 3] & (1 << 22)) != 0
    assert bool(narrow.any())
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    plain = torch.from_numpy(att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_FWD)).to(dev)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    code = 0 if dtype == torch.float16 else 1
    ref = oracle(q, k, v, do, lengths)

    def run(kernel, items):
        out = torch.full_like(qd, float("nan"))
        lse = torch.full((hq, n), float("nan"), dtype=torch.float32, device=dev)
        att.check(att.lib().va_fwd_kernel(kernel, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                          out.data_ptr(), lse.data_ptr(), items.data_ptr(),
                                          items.shape[0], n, hq, hkv, 128, SCALE, code,
                                          att._stream()), "va_fwd_kernel")
        torch.cuda.synchronize()
        return out, lse
    for kernel, items, unsplit in ((att._lib.VA_FWD_WIDE, plan.fwd_items[: plan.n_fwd], plain),
                                   (att._lib.VA_FWD_MANY, padded_fwd_plan(plan, 512), plain)):
        out, lse = run(kernel, items)
        err_o = float(np.max(np.abs(out.cpu().float().numpy().reshape(n, hq, 128) - ref[0])))
        err_lse = float(np.max(np.abs(lse.cpu().numpy() - ref[1])))
        assert err_o <= TOL[dtype]["o"] and err_lse <= TOL[dtype]["lse"], (kernel, err_o, err_lse)
        out2, lse2 = run(kernel, unsplit)
        assert float((out.float() - out2.float()).abs().max()) <= TOL[dtype]["o"], kernel
        assert float((lse - lse2).abs().max()) <= TOL[dtype]["lse"], kernel


class _Plan:
    """A plan object for attention_forward / attention_backward from explicit item lists."""

    def __init__(self, fwd, bwd, total):
        self.fwd_items, self.n_fwd = fwd, fwd.shape[0]
        self.bwd_items, self.n_bwd = bwd, bwd.shape[0]
        self.total = total

    def partial_bwd(self):
        return self.bwd_items, self.n_bwd


@pytest.mark.parametrize("lengths,hq,hkv,dtype", CASES + [([300, 45, 1, 128], 12, 2, "peaky")])
def test_pair_backward_matches_oracle(lengths, hq, hkv, dtype):
    """The backward plan with two query heads per kv and q item (VA_PLAN_BWD_PAIRS, what VA_PLAN_BWD
    takes for long lists), forced on small cases: dQ/dK/dV against the oracle, and bitwise equal
    over two runs."""
    qk = 3.0 if dtype == "peaky" else 1.0
    dtype = torch.bfloat16 if dtype == "peaky" else dtype
    banner("pair backward", lengths, hq, hkv, dtype, qk)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=sum(lengths) + 2, qk_scale=qk)
    n = sum(lengths)
    dev = torch.device("cuda")
    base = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    cu = np.concatenate([[0], np.cumsum([x for x in lengths if x])]).astype(np.int32)
    pair_items = torch.from_numpy(att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_BWD_PAIRS))
    plan = _Plan(base.fwd_items[: base.n_fwd], pair_items.to(dev), n)
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    out, lse = att.attention_forward(qd, kd, vd, plan, SCALE)
    runs = [att.attention_backward(dod, qd, kd, vd, out, lse, plan, SCALE) for _ in range(2)]
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    ref = oracle(q, k, v, do, lengths)
    check_all(out.cpu(), tuple(t.cpu() for t in runs[0]), ref, dtype, n, hq)


GROUP_CASES = CASES + [([300, 45, 1, 128], 12, 2, "peaky"),
                       # long enough for pair items: group items of 2, 3 and 6 heads (G = 6), and
                       # of 7 beside pair tiles (G = 7)
                       ([300] * 12 + [64] * 10, 12, 2, torch.float16),
                       ([250] * 10 + [40] * 30, 28, 4, torch.bfloat16)]


@pytest.mark.parametrize("kind", ["all", "auto"])
@pytest.mark.parametrize("lengths,hq,hkv,dtype", GROUP_CASES)
def test_group_backward_matches_oracle(lengths, hq, hkv, dtype, kind):
    """Backward plans with GQA group items (one kv item over all G query heads of a group, writing
    dK/dV at Hkv width): every key tile grouped (VA_PLAN_BWD_GROUPS_ALL), and the planner's mix
    of group tiles and per-head or pair tiles (VA_PLAN_BWD_GROUPS, where the GQA sum must skip
    the group tiles' rows). dQ/dK/dV against the oracle, and bitwise equal over two runs."""
    qk = 3.0 if dtype == "peaky" else 1.0
    dtype = torch.bfloat16 if dtype == "peaky" else dtype
    banner("group backward", kind, lengths, hq, hkv, dtype, qk)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=sum(lengths) + 4, qk_scale=qk)
    n = sum(lengths)
    dev = torch.device("cuda")
    base = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    cu = np.concatenate([[0], np.cumsum([x for x in lengths if x])]).astype(np.int32)
    code = att._lib.VA_PLAN_BWD_GROUPS_ALL if kind == "all" else att._lib.VA_PLAN_BWD_GROUPS
    items = att.build_plan_host(cu, hq, hkv, code)
    kv = items[(items[:, 3] >> 24) == 0]
    if hq > hkv and kind == "all":
        assert len(kv) and ((kv[:, 3] >> 21) & 1).all()
    if kind == "auto" and len(lengths) == 22:  # the subsets this case exists for
        heads = {((w >> 12) & 0xFF) + 1 for w in kv[:, 3].tolist() if (w >> 21) & 1}
        assert heads == {2, 3, 6}, heads
    plan = _Plan(base.fwd_items[: base.n_fwd], torch.from_numpy(items).to(dev), n)
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    out, lse = att.attention_forward(qd, kd, vd, plan, SCALE)
    runs = [att.attention_backward(dod, qd, kd, vd, out, lse, plan, SCALE) for _ in range(2)]
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    ref = oracle(q, k, v, do, lengths)
    check_all(out.cpu(), tuple(t.cpu() for t in runs[0]), ref, dtype, n, hq)


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_golden_vectors(name):
    z = load_golden(name)
    banner("golden", name)
    lengths = z["lengths"]
    out, *grads = run_varlen(z["q"], z["k"], z["v"], z["do"], lengths, float(z["scale"]))
    ref = (z["o"], z["lse"], z["dq"], z["dk"], z["dv"])
    check_all(out, grads, ref, z["dtype"], sum(lengths), int(z["hq"]))


def test_lse_matches_oracle():
    lengths, hq, hkv = [300, 45, 1, 128], 12, 2
    banner("lse", lengths)
    for dtype, qk in ((torch.float16, 1.0), (torch.bfloat16, 3.0)):
        q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=3, qk_scale=qk)
        plan = att._plan(att._cu_seqlens(lengths, torch.device("cuda")), hq, hkv)
        _out, lse = att.attention_forward(q.cuda(), k.cuda(), v.cuda(), plan, SCALE)
        torch.cuda.synchronize()
        _o, lse_ref, *_ = oracle(q, k, v, do, lengths)
        err = float(np.max(np.abs(lse.cpu().numpy() - lse_ref)))
        assert err <= TOL[dtype]["lse"], (dtype, err)


def test_reference_padded_masked_sdpa_construction():
    """solution/test_attention.py:84-116 as the reference states it: fp16 varlen vs zero-padded
    dense SDPA with a `tril & real` mask over H = 12 expanded heads (here evaluated in fp32 on
    the CPU), same tolerances."""
    for lengths in ([64, 37, 50, 12], [334, 200, 100, 7]):
        banner("reference-construction", lengths)
        torch.manual_seed(0)
        batch, seq, heads, dim = len(lengths), max(lengths), 12, 128
        real = torch.zeros(batch, seq, dtype=torch.bool)
        for row, length in enumerate(lengths):
            real[row, :length] = True
        rows = torch.nonzero(real.reshape(-1), as_tuple=True)[0]
        n = rows.numel()
        qkv = [torch.randn(n, heads, dim).half() for _ in range(3)]
        grad = torch.randn(n, heads * dim).half()
        mask = torch.ones(seq, seq, dtype=torch.bool).tril()[None, None] & real[:, None, None]
        leaves = [x.float().requires_grad_() for x in qkv]

        def padded(x):
            full = torch.zeros(batch * seq, heads, dim, dtype=x.dtype)
            return full.index_copy(0, rows, x).view(batch, seq, heads, dim).transpose(1, 2)

        ref = torch.nn.functional.scaled_dot_product_attention(
            *[padded(x) for x in leaves], attn_mask=mask, scale=dim ** -0.5)
        ref = ref.transpose(1, 2).reshape(batch * seq, heads * dim)[rows]
        ref.backward(grad.float())
        out, *grads = run_varlen(*qkv, grad, lengths, dim ** -0.5)
        torch.testing.assert_close(out.float(), ref.detach(), rtol=2e-3, atol=2e-3)
        for mine, leaf in zip(grads, leaves):
            torch.testing.assert_close(mine.float(), leaf.grad, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_benchmark_configs_match_oracle(cfg):
    """Full-size parity at the benchmark configurations with 1.5B heads. Configuration 1 is the
    reference's CPU-runnable case (fp32, 4 documents U[64, 512], seed 0 -> [445, 349, 293, 185]):
    the HIP path runs it on the same values rounded once to fp16."""
    c = wl.CONFIGS[cfg]
    lengths = wl.config_lengths(cfg)
    dtype = torch.float16 if c["dtype"] == "float32" else wl.torch_dtype(c["dtype"])
    if cfg == 1:
        assert lengths == [445, 349, 293, 185]
    banner("config", cfg, len(lengths), sum(lengths), dtype)
    q, k, v, do = wl.make_inputs(lengths, c["hq"], c["hkv"], dtype, seed=0,
                                 qk_scale=c["qk_scale"])
    out, *grads = run_varlen(q, k, v, do, lengths)
    check_all(out, grads, oracle(q, k, v, do, lengths), dtype, sum(lengths), c["hq"])


def config5_checked_documents(lengths):
    """Documents of configuration 5 checked against the oracle: one at every length decile (the
    shortest, the 10th, ..., 90th percentile and the longest), the three longest, the first and
    the last."""
    order = sorted(range(len(lengths)), key=lambda i: lengths[i])
    deciles = [order[min(len(order) - 1, (len(order) - 1) * p // 10)] for p in range(11)]
    return sorted(set(deciles + order[-3:] + [0, len(lengths) - 1]))


def test_7b_config_documents_match_oracle():
    """Configuration 5 (7B heads, 67 documents up to 1740 tokens) at full size on the GPU (the
    group-item backward list and the row statistics pass, as the benchmark runs it), checked
    against the oracle on every query and key/value head of one document per length decile, the
    three longest, the first and the last."""
    lengths = wl.config_lengths(5)
    c = wl.CONFIGS[5]
    dtype = wl.torch_dtype(c["dtype"])
    banner("config", 5, len(lengths), sum(lengths))
    plan = att._plan(att._cu_seqlens(lengths, torch.device("cuda")), c["hq"], c["hkv"])
    assert plan.bwd_stats and not plan.bwd_finish
    q, k, v, do = wl.make_inputs(lengths, c["hq"], c["hkv"], dtype, seed=0)
    out, dq, dk, dv = run_varlen(q, k, v, do, lengths)
    cu = orc.cu_seqlens_from_lengths(lengths)
    docs = config5_checked_documents(lengths)
    assert len(docs) >= 11
    o_all = out.reshape(-1, c["hq"], 128)
    for d in docs:
        s, e = int(cu[d]), int(cu[d + 1])
        sl = slice(s, e)
        print(f"  document {d}: tokens {s}..{e}", flush=True)
        ref = oracle(q[sl], k[sl], v[sl], do[sl], [e - s])
        check_all(o_all[sl], (dq[sl], dk[sl], dv[sl]), ref, dtype, e - s, c["hq"])


def test_forward_and_backward_are_bitwise_deterministic():
    """The attention kernels use no atomics: dQ and the per-head dK/dV partials are each written
    by one work-group and the GQA sum adds the partials in head order, so repeated calls agree
    bit for bit."""
    lengths, hq, hkv = [512, 300, 77], 12, 2
    banner("determinism", lengths)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, torch.float16, seed=5)
    a = run_varlen(q, k, v, do, lengths)
    b = run_varlen(q, k, v, do, lengths)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_graph_replays_match_eager():
    """Forward + backward captured in one HIP graph (as the benchmark runs them): every replay,
    with eager work and a synchronisation before it and the outputs overwritten in between,
    gives bitwise the eager results (no memset nodes, nothing that only the first replay sets)."""
    lengths, hq, hkv = [512, 300, 77], 12, 2
    banner("graph replay", lengths)
    dev = torch.device("cuda")
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(lengths, hq, hkv, torch.float16, seed=9))
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)

    def step():
        out, lse = att.attention_forward(q, k, v, plan, SCALE)
        return (out, lse) + tuple(att.attention_backward(do, q, k, v, out, lse, plan, SCALE))

    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for r in range(3):
        for t in captured:
            t.fill_(float("nan"))
        torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("out", "lse", "dq", "dk", "dv"), captured, eager):
            assert torch.equal(x, y), f"replay {r}: {name} differs from eager"


@pytest.mark.parametrize("lengths", [[0], [0, 0, 0]])
def test_empty_batch(lengths):
    """No tokens. Host lengths: ValueError, as the reference's max() over no lengths
    (solution/attention.py:239-242). Device lengths (no host read, so no such check): no launch,
    empty outputs and gradients of the right shapes."""
    banner("empty", lengths)
    q, k, v, do = wl.make_inputs(lengths, 12, 2, torch.float16, seed=0)
    assert q.shape[0] == 0
    with pytest.raises(ValueError):
        run_varlen(q, k, v, do, lengths)
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.varlen_attention(qd, kd, vd, torch.tensor(lengths, device="cuda"), SCALE)
    out.backward(do.cuda().reshape(out.shape))
    torch.cuda.synchronize()
    assert out.shape == (0, 12 * 128)
    assert qd.grad.shape == q.shape and kd.grad.shape == k.shape and vd.grad.shape == v.shape


def test_qkv_rotate_matches_transformers():
    """solution/test_attention.py:40-81 restated: rotation + fp16 cast + repeat_kv, both layouts,
    against transformers' formula (fp32, CPU), output 2e-3 and grads rtol 2e-3 / atol 2e-2."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb, repeat_kv

    for (lengths, seq), padded in [(([64, 37, 50, 12], 64), False), (([64, 37, 50, 12], 64), True),
                                   (([334, 200, 100, 7], 334), False),
                                   (([334, 200, 100, 7], 334), True)]:
        banner("qkv_rotate", lengths, padded)
        torch.manual_seed(0)
        batch, heads, kv_heads, dim = len(lengths), 12, 2, 128
        real = torch.zeros(batch, seq, dtype=torch.bool)
        for row, length in enumerate(lengths):
            real[row, :length] = True
        rows = torch.nonzero(real.reshape(-1), as_tuple=True)[0]
        b_idx, t_idx = (rows // seq).to(torch.int32), (rows % seq).to(torch.int32)
        n = rows.numel()
        q = torch.randn(n, heads * dim, requires_grad=True)
        k = torch.randn(n, kv_heads * dim, requires_grad=True)
        v = torch.randn(n, kv_heads * dim, requires_grad=True)
        inv_freq = 1.0 / (1000000.0 ** (torch.arange(0, dim, 2).float() / dim))
        freqs = torch.arange(seq).float()[:, None] * inv_freq[None]
        emb = torch.cat((freqs, freqs), dim=-1)
        cos, sin = emb.cos()[None], emb.sin()[None]
        grads = [torch.randn(batch, heads, seq, dim).half() for _ in range(3)]

        def to_padded(x):
            full = torch.zeros(batch * seq, x.shape[-1])
            return full.index_copy(0, rows, x).view(batch, seq, -1)

        q4 = to_padded(q).view(batch, seq, heads, dim).transpose(1, 2)
        k4 = to_padded(k).view(batch, seq, kv_heads, dim).transpose(1, 2)
        v4 = to_padded(v).view(batch, seq, kv_heads, dim).transpose(1, 2)
        qe, ke = apply_rotary_pos_emb(q4, k4, cos.expand(batch, seq, dim),
                                      sin.expand(batch, seq, dim))
        ref = (qe.half(), repeat_kv(ke, heads // kv_heads).half(),
               repeat_kv(v4, heads // kv_heads).half())
        torch.autograd.backward(ref, grads)
        ref_grads = [t.grad.clone() for t in (q, k, v)]

        def packed(x):
            return x.transpose(1, 2).reshape(batch * seq, heads, dim)[rows]

        qd, kd, vd = (t.detach().cuda().requires_grad_() for t in (q, k, v))
        out = att.qkv_rotate(qd, kd, vd, cos.cuda(), sin.cuda(), b_idx.cuda(), t_idx.cuda(), batch,
                             seq, heads, kv_heads, padded)
        if padded:
            torch.autograd.backward(out, [g.cuda() for g in grads])
            refs = ref
        else:
            torch.autograd.backward(out, [packed(g).cuda() for g in grads])
            refs = [packed(x) for x in ref]
        for mine, theirs in zip(out, refs):
            torch.testing.assert_close(mine.detach().cpu().float(), theirs.detach().float(),
                                       rtol=2e-3, atol=2e-3)
        for mine, theirs in zip((qd.grad, kd.grad, vd.grad), ref_grads):
            torch.testing.assert_close(mine.cpu(), theirs, rtol=2e-3, atol=2e-2)


def test_pack_rows_matches_indexing():
    """solution/test_attention.py:119-137: exact."""
    banner("pack_rows")
    torch.manual_seed(0)
    lengths, seq, heads, dim = [50, 20, 33], 64, 12, 128
    real = torch.zeros(len(lengths), seq, dtype=torch.bool)
    for row, length in enumerate(lengths):
        real[row, :length] = True
    rows = torch.nonzero(real.reshape(-1), as_tuple=True)[0]
    b_idx, t_idx = (rows // seq).to(torch.int32).cuda(), (rows % seq).to(torch.int32).cuda()
    attn = torch.randn(len(lengths), heads, seq, dim, dtype=torch.float16, device="cuda",
                       requires_grad=True)
    grad = torch.randn(rows.numel(), heads * dim, dtype=torch.float16, device="cuda")
    ref = attn.permute(0, 2, 1, 3).reshape(-1, heads * dim)[rows.cuda()]
    ref.backward(grad)
    ref_grad = attn.grad.clone()
    attn.grad = None
    out = att.pack_rows(attn, b_idx, t_idx)
    out.backward(grad)
    torch.testing.assert_close(out, ref, rtol=0, atol=0)
    torch.testing.assert_close(attn.grad, ref_grad, rtol=0, atol=0)


def rope_tables(seq, dim=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    emb = torch.arange(seq).float()[:, None] * torch.rand(dim // 2, generator=g)
    emb = torch.cat((emb, emb), dim=-1)[None]
    return emb.cos(), emb.sin()


PACKED_CASES = [
    # per-head backward list, rotated partials summed by the GQA sum without row flags
    ("small", [70, 33, 51, 1, 200], 12, 2, torch.float16),
    ("small", [70, 33, 51, 1, 200], 12, 2, torch.bfloat16),
    # configuration 3's documents: group items of 6, 3 and 2 heads beside pair items, flagged sum
    ("config3", wl.config_lengths(3), 12, 2, torch.float16),
    # configuration 4's documents: group items write rotated dK and dV at Hkv width, no GQA sum
    ("config4", wl.config_lengths(4), 12, 2, torch.bfloat16),
    # the first 8 documents of configuration 5 (7B heads): the row statistics pass
    ("config5[:8]", wl.config_lengths(5)[:8], 28, 4, torch.bfloat16),
    # expanded K/V (Hq == Hkv): dK/dV written directly, no workspace
    ("mha", [70, 33, 51, 1, 200], 4, 4, torch.float16),
]


@pytest.mark.parametrize("name,lengths,heads,kv_heads,dtype", PACKED_CASES,
                         ids=[f"{c[0]}-{c[4]}" for c in PACKED_CASES])
def test_packed_attention_matches_oracle(name, lengths, heads, kv_heads, dtype):
    """Rotation + attention of the packed rows (PackedAttention, the inverse rotation in the
    backward kernels' epilogues) against the oracle: fp32 rotation rounded once to the compute
    type, fp64 attention, fp32 inverse rotation. Each case checks first that the plan has the
    backward shape it is there for."""
    banner("packed_attention", name, len(lengths), sum(lengths), heads, kv_heads, dtype)
    plan = att._plan(att._cu_seqlens(lengths, torch.device("cuda")), heads, kv_heads)
    words = plan.bwd_items.cpu().numpy()[:, 3]
    kv_shapes = set(((words[(words >> 24) == 0] >> 20) & 3).tolist())  # 0 head, 1 pair, 2 group
    q_shapes = set(((words[(words >> 24) == 1] >> 20) & 3).tolist())
    n = sum(lengths)
    # short lists: the partials route and the inverse rotation pass; long: the rotary epilogues
    assert att.rotary_epilogues(n, heads) == (name not in ("small", "mha"))
    if name == "small":  # per-head q items, per-head and group kv items
        assert q_shapes == {0} and kv_shapes == {0, 2} and plan.bwd_finish
    elif name == "config3":  # pair q items, group kv items of 6, 3 and 2 heads, flagged sum
        assert q_shapes == {1} and kv_shapes == {2} and plan.bwd_finish
    elif name == "config4":  # group kv items of the whole group everywhere: no GQA sum
        assert kv_shapes == {2} and not plan.bwd_finish and not plan.bwd_stats
    elif name == "mha":
        assert q_shapes == {0} and kv_shapes == {0} and not plan.bwd_finish
    else:  # every kv shape, the row statistics pass
        assert kv_shapes == {0, 1, 2} and plan.bwd_stats
    check_packed_attention(lengths, heads, kv_heads, dtype)


def check_packed_attention(lengths, heads, kv_heads, dtype, seed=1):
    """packed_attention forward and backward on random projections of the packed rows of
    `lengths` (right-padded batch, rotary tables of test length) against the oracle's fp32
    rotation, fp64 attention and fp32 inverse rotation."""
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)])
    b_idx, t_idx = (rows // seq).to(torch.int32), (rows % seq).to(torch.int32)
    n = rows.numel()
    cos, sin = rope_tables(seq)
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n, heads * 128, generator=g) * 0.5).to(dtype)
    k = (torch.randn(n, kv_heads * 128, generator=g) * 0.5).to(dtype)
    v = torch.randn(n, kv_heads * 128, generator=g).to(dtype)
    do = torch.randn(n, heads * 128, generator=g).to(dtype)
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.packed_attention(qd, kd, vd, cos.cuda(), sin.cuda(), b_idx.cuda(), t_idx.cuda(), seq,
                               heads, kv_heads, lengths, SCALE)
    out.backward(do.cuda())
    torch.cuda.synchronize()
    # oracle: rotate in fp32, round once to the compute type, attention in fp64
    qr = torch.from_numpy(orc.rope_forward(q.float().numpy(), cos.numpy(), sin.numpy(), b_idx,
                                           t_idx, heads)).to(dtype)
    kr = torch.from_numpy(orc.rope_forward(k.float().numpy(), cos.numpy(), sin.numpy(), b_idx,
                                           t_idx, kv_heads)).to(dtype)
    vr = v.view(n, kv_heads, 128)
    o_ref, _lse, dq_ref, dk_ref, dv_ref = oracle(qr, kr, vr, do.view(n, heads, 128), lengths)
    dq_in = orc.rope_backward(dq_ref, cos.numpy(), sin.numpy(), b_idx, t_idx)
    dk_in = orc.rope_backward(dk_ref, cos.numpy(), sin.numpy(), b_idx, t_idx)
    dv_in = dv_ref.reshape(n, -1)
    tol = TOL[dtype]
    err = float(np.max(np.abs(out.detach().cpu().float().numpy().reshape(n, heads, 128) - o_ref)))
    assert err <= tol["o"], err
    for which, mine, theirs in (("q", qd.grad, dq_in), ("k", kd.grad, dk_in),
                                ("v", vd.grad, dv_in)):
        r = rel(mine.cpu().float().numpy(), theirs)
        assert r <= tol["g"], (which, r)


@pytest.mark.parametrize("lengths", [[334, 200, 0, 100, 7], wl.config_lengths(3)[:30] + [0]])
def test_packed_attention_device_lengths_match_host_lengths(lengths):
    """packed_attention with the lengths as a device tensor (device cu_seqlens and plans, no host
    read) gives bitwise the host-lengths output and projection gradients: the two lists hold the
    same items. Short lists take the partials route and the inverse rotation pass; the 30
    documents of configuration 3 (ceil(N / 128) Hq >= 512) the rotary epilogues and the flagged
    GQA sum over the group list."""
    heads, kv_heads = 12, 2
    banner("packed_attention device lengths", len(lengths), sum(lengths))
    n_real = sum(lengths)
    assert att.rotary_epilogues(n_real, heads) == (len(lengths) > 5)
    real = [x for x in lengths if x]
    seq = max(real)
    rows = torch.tensor([b * seq + t for b, length in enumerate(real) for t in range(length)])
    b_idx, t_idx = (rows // seq).to(torch.int32).cuda(), (rows % seq).to(torch.int32).cuda()
    n = rows.numel()
    cos, sin = (t.cuda() for t in rope_tables(seq, seed=3))
    g = torch.Generator().manual_seed(8)
    q = torch.randn(n, heads * 128, generator=g).half().cuda()
    k = torch.randn(n, kv_heads * 128, generator=g).half().cuda()
    v = torch.randn(n, kv_heads * 128, generator=g).half().cuda()
    do = torch.randn(n, heads * 128, generator=g).half().cuda()
    res = []
    for lens in (lengths, torch.tensor(lengths, device="cuda")):
        leaves = [t.clone().requires_grad_() for t in (q, k, v)]
        out = att.packed_attention(*leaves, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lens,
                                   SCALE)
        out.backward(do)
        torch.cuda.synchronize()
        res.append([out.detach()] + [t.grad for t in leaves])
    for a, b in zip(*res):
        assert torch.equal(a, b)


HEAD_MASK = (1 << 12) - 1  # item word: kind << 24 | group << 21 | pair << 20 | (S-1) << 12 | head


def plan_work(kind, a, e, s, w):
    """The planners' work measure of an item: keys visited (forward); MFMAs per wave per
    iteration plus the item's fixed cost (backward; a pair item's halves take every step, a
    group item's the steps of its S heads)."""
    if kind in (0, 6):  # VA_PLAN_FWD, VA_PLAN_FWD_NARROW (a narrow item: its whole tile's)
        return min(a + 128, e) - s
    if w >> 24 == 0:
        steps = (e - a + 31) // 32
        if (w >> 21) & 1:
            return ((((w >> 12) & 0xFF) + 1) * steps + 1) // 2 * 32 + 39
        return (steps if (w >> 20) & 1 else (steps + 1) // 2) * 32 + 39
    return ((min(a + 128, e) - s + 31) // 32 + 1) // 2 * (48 if (w >> 20) & 1 else 24) + 30


def check_device_xcd_layout(items, kind, hq, hkv, pairs=False):
    """The items of one (tile, kind, GQA group) sit a constant stride apart, at most 8 (one XCD),
    and the groups come longest first by the work measure in buckets of 8. Empty items (the
    rows a pair plan or group items leave free) are skipped; a tile's G / S group items of S heads
    form its combo."""
    g = hq // hkv
    combos = {}
    for pos, (a, e, s, w) in enumerate(items.tolist()):
        if (a, e, s, w) == (0, 0, 0, 0):
            continue
        combos.setdefault((a, e, s, w >> 24, (w & HEAD_MASK) // g), []).append((pos, w))
    firsts = []
    for key, entries in combos.items():
        pos = [p for p, _ in entries]
        w_first = entries[0][1]
        grouped = (w_first >> 21) & 1
        n_heads = ((w_first >> 12) & 0xFF) + 1
        assert len(pos) == (g // n_heads if grouped else (g if not pairs else (g + 1) // 2)), key
        steps = {b - a for a, b in zip(pos, pos[1:])}
        assert len(steps) <= 1 and all(0 < x <= 8 for x in steps), (key, pos)
        w0 = (key[3] << 24) | ((1 << 20) if pairs and g > 1 and not grouped else 0)
        if grouped:
            w0 = w_first
        firsts.append((pos[0], plan_work(kind, key[0], key[1], key[2], w0) // 8))
    work = [w for _, w in sorted(firsts)]
    assert work == sorted(work, reverse=True)


@pytest.mark.parametrize("lengths", [[64, 37, 50, 12], [334, 0, 200, 100, 7], [1000, 24],
                                     [1, 1, 1, 2, 3], [512] * 4,
                                     [300] * 12 + [64] * 10])  # pair list: group items of 2, 3, 6
def test_device_plan_matches_host_plan(lengths):
    """The plans built on the device from device lengths hold the host plans' items (as a set: the
    order inside a work bucket is free) in the same XCD layout, then empty items up to their
    capacity; zero lengths make no items; the cu_seqlens written with them is the prefix sum. The
    entry point that starts from a device cu_seqlens builds the same items."""
    banner("device plan", lengths)
    hq, hkv = 12, 2
    dev = torch.device("cuda")
    n = sum(lengths)
    dplan = att.DevicePlan(torch.tensor(lengths, device=dev), n, hq, hkv)
    torch.cuda.synchronize()
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    assert dplan.cu.cpu().numpy().tolist() == cu.tolist()
    groups = att._lib.VA_PLAN_BWD_GROUPS
    tiles = sum(-(-x // 128) for x in lengths if x > 0)
    pairs = 2 * tiles * hq >= att._lib.VA_BWD_PAIR_MIN_ITEMS
    part_items, part_n = dplan.partial_bwd()
    narrow = att._lib.VA_PLAN_FWD_NARROW
    for kind, items, count in ((narrow, dplan.fwd_items, dplan.n_fwd), (1, part_items, part_n),
                               (groups, dplan.bwd_items, dplan.n_bwd)):
        host = att.build_plan_host(cu, hq, hkv, kind)
        got = items.cpu().numpy()[:count]
        if kind == groups or (kind == 1 and pairs):  # rows left empty inside the blocks
            real = [tuple(x) for x in got.tolist() if any(x)]
            assert sorted(real) == sorted(map(tuple, host.tolist()))
            check_device_xcd_layout(got, kind, hq, hkv, pairs=pairs)
        else:
            real, empty = got[: len(host)], got[len(host):]
            assert sorted(map(tuple, real.tolist())) == sorted(map(tuple, host.tolist()))
            assert not empty.any()
            check_device_xcd_layout(real, kind, hq, hkv)
        again = torch.empty_like(items)
        att.check(att.lib().va_plan_build_device(dplan.cu.data_ptr(), len(lengths), n, hq, hkv,
                                                 kind, again.data_ptr(), count, att._stream()),
                  "va_plan_build_device")
        torch.cuda.synchronize()
        again = again.cpu().numpy()[:count]
        assert sorted(map(tuple, again.tolist())) == sorted(map(tuple, got.tolist()))
    # the pair plan (two heads per kv item) from the device cu_seqlens: the host pair plan's items
    # plus empty items (the free rows of the kv blocks and the slots past the real items)
    count = dplan.n_bwd
    pair_items = torch.empty_like(dplan.bwd_items)
    att.check(att.lib().va_plan_build_device(dplan.cu.data_ptr(), len(lengths), n, hq, hkv,
                                             att._lib.VA_PLAN_BWD_PAIRS, pair_items.data_ptr(),
                                             count, att._stream()), "va_plan_build_device")
    torch.cuda.synchronize()
    got = pair_items.cpu().numpy()[:count]
    host = att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_BWD_PAIRS)
    real = [tuple(x) for x in got.tolist() if any(x)]
    assert sorted(real) == sorted(map(tuple, host.tolist()))
    check_device_xcd_layout(got, 1, hq, hkv, pairs=True)
    # every key tile as group items, from the device cu_seqlens
    all_items = torch.empty_like(dplan.bwd_items)
    att.check(att.lib().va_plan_build_device(dplan.cu.data_ptr(), len(lengths), n, hq, hkv,
                                             att._lib.VA_PLAN_BWD_GROUPS_ALL,
                                             all_items.data_ptr(), count, att._stream()),
              "va_plan_build_device")
    torch.cuda.synchronize()
    got = all_items.cpu().numpy()[:count]
    host = att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_BWD_GROUPS_ALL)
    assert sorted(tuple(x) for x in got.tolist() if any(x)) == sorted(map(tuple, host.tolist()))
    check_device_xcd_layout(got, 1, hq, hkv, pairs=pairs)


def test_device_lengths_plan_is_rebuilt_inside_a_captured_graph():
    """A graph captured with device lengths contains the plan build: after the lengths tensor is
    overwritten in place, a replay attends over the new documents (the plan cached by the eager
    call before the capture is not reused inside it)."""
    banner("device lengths under graph capture")
    dev = torch.device("cuda")
    first, second = [300, 200, 100], [100, 250, 250]
    hq, hkv = 12, 2
    q, k, v, _do = (t.to(dev) for t in wl.make_inputs(first, hq, hkv, torch.float16, seed=8))
    lens = torch.tensor(first, device=dev)
    eager_first = att.varlen_attention(q, k, v, lens, SCALE)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = att.varlen_attention(q, k, v, lens, SCALE)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(captured, eager_first)
    lens.copy_(torch.tensor(second, device=dev))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(captured, att.varlen_attention(q, k, v, second, SCALE))
    assert not torch.equal(captured, eager_first)


@pytest.mark.parametrize("lengths,hq,hkv", [
    ([334, 200, 0, 100, 7], 12, 2),
    # many short documents: the device list's capacity (648) and the host list (360 items) lie on
    # either side of VA_FWD_MANY_ITEMS; both paths still run the same forward kernel
    ([100] * 30, 12, 2),
    # zero lengths beside 43 documents: the host drops them, the device counts them, and both
    # take pair items by the tiles of the non-empty documents
    ([0] * 10 + [100] * 43, 12, 2),
    ([0, 300, 0, 45, 1], 28, 4),
])
def test_device_lengths_run_without_host_reads_and_match_host_lengths(lengths, hq, hkv):
    """varlen_attention with the lengths as a device tensor (device cu_seqlens and plan, no host
    read) gives bitwise the host-lengths results: both paths choose the forward kernel from the
    sizes and the backward's pair shape from the tiles of the non-empty documents."""
    banner("device lengths", len(lengths), sum(lengths), hq, hkv)
    q, k, v, do = wl.make_inputs([x for x in lengths if x], hq, hkv, torch.float16, seed=5)
    host = run_varlen(q, k, v, do, lengths)
    dev_lengths = torch.tensor(lengths, device="cuda")
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.varlen_attention(qd, kd, vd, dev_lengths, SCALE)
    out.backward(do.cuda().reshape(out.shape))
    torch.cuda.synchronize()
    for a, b in zip(host, (out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu())):
        assert torch.equal(a, b)


@pytest.mark.parametrize("lengths,n_rows", [([334, 200, 100], 700), ([100, 0, 50, 0], 230)])
def test_device_lengths_summing_below_n_extend_the_last_document(lengths, n_rows):
    """Device lengths whose sum falls short of the rows cannot be checked without a host read (the
    host path raises ValueError): the device plan ends the last document at N, so every output and
    gradient row is written, bitwise as host lengths whose last document takes the rest."""
    hq, hkv = 12, 2
    banner("device lengths below N", lengths, n_rows)
    extended = list(lengths)
    extended[-1] += n_rows - sum(lengths)
    q, k, v, do = wl.make_inputs([x for x in extended if x], hq, hkv, torch.float16, seed=9)
    assert q.shape[0] == n_rows
    with pytest.raises(ValueError):
        run_varlen(q, k, v, do, lengths)
    host = run_varlen(q, k, v, do, extended)
    qd, kd, vd = (t.cuda().requires_grad_() for t in (q, k, v))
    out = att.varlen_attention(qd, kd, vd, torch.tensor(lengths, device="cuda"), SCALE)
    out.backward(do.cuda().reshape(out.shape))
    torch.cuda.synchronize()
    for a, b in zip(host, (out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu())):
        assert torch.equal(a, b)


def test_packed_attention_save_policies_agree_bitwise():
    """Keeping O / lse for the backward ("outputs") gives the same output and gradients, bit for
    bit, as recomputing the forward in the backward ("inputs", the reference's choice), and keeps
    the rotated operands plus O and lse instead of the projections."""
    lengths, heads, kv_heads, dtype = [70, 33, 51, 1, 200], 12, 2, torch.float16
    banner("packed_attention save policies", lengths)
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)])
    b_idx, t_idx = (rows // seq).to(torch.int32).cuda(), (rows % seq).to(torch.int32).cuda()
    n = rows.numel()
    cos, sin = (t.cuda() for t in rope_tables(seq))
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(n, heads * 128, generator=g) * 0.5).to(dtype).cuda()
    k = (torch.randn(n, kv_heads * 128, generator=g) * 0.5).to(dtype).cuda()
    v = torch.randn(n, kv_heads * 128, generator=g).to(dtype).cuda()
    do = torch.randn(n, heads * 128, generator=g).to(dtype).cuda()
    results = {}
    try:
        for policy in ("inputs", "outputs"):
            att.set_save_policy(policy)
            qd, kd, vd = (t.clone().requires_grad_() for t in (q, k, v))
            out = att.packed_attention(qd, kd, vd, cos, sin, b_idx, t_idx, seq, heads, kv_heads,
                                       lengths, SCALE)
            saved = [t.shape for t in out.grad_fn.saved_tensors]
            out.backward(do)
            torch.cuda.synchronize()
            results[policy] = (out.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu(),
                               saved)
    finally:
        att.set_save_policy("outputs")
    for a, b in zip(results["inputs"][:4], results["outputs"][:4]):
        assert torch.equal(a, b)
    assert results["inputs"][4] == [q.shape, k.shape, v.shape]
    assert results["outputs"][4] == [(n, heads, 128), (n, kv_heads, 128), (n, kv_heads, 128),
                                     (n, heads, 128), (heads, n)]
    with pytest.raises(ValueError):
        att.set_save_policy("everything")


def test_packed_attention_offloaded_matches_plain_autograd(monkeypatch):
    """solution/test_offload.py:68-106: three offloaded layers (two of them evicted to host memory
    and brought back, one prefetched), forward bitwise equal, grads within 1e-2 of 3x the single
    call."""
    from hackaton_amd import offload

    monkeypatch.setattr(offload, "KEEP_BYTES", 1 << 20)
    banner("offload")
    torch.manual_seed(0)
    lengths, heads, kv_heads, dim = [70, 33, 51], 12, 2, 128
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)])
    b_idx = (rows // seq).to(torch.int32).cuda()
    t_idx = (rows % seq).to(torch.int32).cuda()
    n = rows.numel()
    cos, sin = (t.cuda() for t in rope_tables(seq))
    q = (torch.randn(n, heads * dim, device="cuda") * 0.3).half().requires_grad_()
    k = (torch.randn(n, kv_heads * dim, device="cuda") * 0.3).half().requires_grad_()
    v = (torch.randn(n, kv_heads * dim, device="cuda") * 0.3).half().requires_grad_()
    grad = torch.randn(n, heads * dim, device="cuda").half()
    query, key, value = att.qkv_rotate(q, k, v, cos, sin, b_idx, t_idx, 0, seq, heads, kv_heads)
    ref = att.varlen_attention(query, key, value, lengths, dim ** -0.5)
    ref.backward(grad)
    ref_grads = [t.grad.clone() for t in (q, k, v)]
    for t in (q, k, v):
        t.grad = None
    offload.OFFLOADER.begin(q.device)
    outs = [att.packed_attention(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths,
                                 dim ** -0.5) for _ in range(3)]
    offload.OFFLOADER.end()
    torch.autograd.backward(outs, [grad] * 3)
    # the packed path runs GQA-native (K/V not expanded, each K/V head read for its G query
    # heads) on bitwise the same rotated values, and every forward item does the same arithmetic
    # in the same order: the outputs are equal bit for bit (solution/test_offload.py:104)
    assert torch.equal(outs[0].detach(), ref.detach())
    assert torch.equal(outs[0].detach(), outs[2].detach())
    for t, theirs in zip((q, k, v), ref_grads):
        torch.testing.assert_close(t.grad.float(), 3 * theirs.float(), rtol=1e-2, atol=1e-2)


def test_kernels_skip_items_of_a_plan_for_other_sizes():
    """A work list built for more query heads and more tokens than the launch: the kernels skip
    every item whose head or rows fall outside the launch, so nothing is written outside the
    launch's output tensors (each is a view inside a larger NaN-filled buffer whose margins must
    stay NaN), and the items that do fit still compute their rows correctly (per-head items; the
    group items of a list built for G = 6 do not fit G = 2 and are skipped: canaries only)."""
    banner("mismatched plan")
    dev = torch.device("cuda")
    small, big = [200, 100], [200, 100, 300]
    hq_small, hq_big, hkv = 4, 12, 2
    n = sum(small)
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(small, hq_small, hkv, torch.float16, seed=2))
    plan_big = att._plan(att._cu_seqlens(big, dev), hq_big, hkv)
    pad = 1 << 16

    def canaried(shape, dtype):
        fill = 0xA5 if dtype == torch.uint8 else float("nan")
        buf = torch.full((pad + int(np.prod(shape)) + pad,), fill, dtype=dtype, device=dev)
        return buf, buf[pad: pad + int(np.prod(shape))].view(shape)

    lib = att.lib()
    ob, out = canaried((n, hq_small, 128), torch.float16)
    lb, lse = canaried((hq_small, n), torch.float32)
    att.check(lib.va_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                         plan_big.fwd_items.data_ptr(), plan_big.n_fwd, n, hq_small, hkv, 128,
                         SCALE, 0, att._stream()), "va_fwd")
    qb, dq = canaried((n, hq_small, 128), torch.float16)
    ws_bytes = att.bwd_workspace(n, hq_small, hkv, q.device)[0].numel()
    wb, ws = canaried((ws_bytes,), torch.uint8)
    kb, dk = canaried((n, hkv, 128), torch.float16)
    vb, dv = canaried((n, hkv, 128), torch.float16)
    part_items, n_part = plan_big.partial_bwd()
    for items_b, n_b in ((plan_big.bwd_items, plan_big.n_bwd), (part_items, n_part)):
        att.check(lib.va_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             out.data_ptr(), lse.data_ptr(), items_b.data_ptr(), n_b, n,
                             hq_small, hkv, 128, SCALE, 0, dq.data_ptr(), dk.data_ptr(),
                             dv.data_ptr(), ws.data_ptr(), ws_bytes, att._stream()), "va_bwd")
    torch.cuda.synchronize()
    for buf in (ob, lb, qb, kb, vb):
        assert torch.isnan(buf[:pad].float()).all() and torch.isnan(buf[-pad:].float()).all()
    assert bool((wb[:pad] == 0xA5).all()) and bool((wb[-pad:] == 0xA5).all())
    # the first two documents are the same in both plans: their rows are right
    ref = oracle(q.cpu(), k.cpu(), v.cpu(), do.cpu(), small)
    check_all(out.cpu(), (dq.cpu(), dk.cpu(), dv.cpu()), ref, torch.float16, n, hq_small)
    # the many-item forward kernel (the same list padded with empty items) skips the same items
    items = padded_fwd_plan(plan_big, 512)
    ob2, out2 = canaried((n, hq_small, 128), torch.float16)
    lb2, lse2 = canaried((hq_small, n), torch.float32)
    att.check(lib.va_fwd_kernel(att._lib.VA_FWD_MANY, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                out2.data_ptr(), lse2.data_ptr(), items.data_ptr(), items.shape[0],
                                n, hq_small, hkv, 128, SCALE, 0, att._stream()), "va_fwd_kernel")
    torch.cuda.synchronize()
    for buf in (ob2, lb2):
        assert torch.isnan(buf[:pad].float()).all() and torch.isnan(buf[-pad:].float()).all()
    err_o = float(np.max(np.abs(out2.cpu().float().numpy() - ref[0])))
    assert err_o <= TOL[torch.float16]["o"], err_o


@pytest.mark.parametrize("cfg", [2, 3])
def test_gqa_sum_without_flags_matches_flagged_sum(cfg):
    """VA_BWD_FINISH_HEADS (the GQA sum that reads no row flags) on a list without group items
    gives bitwise the flagged sum's dK/dV; the plans choose it exactly when their backward list has
    no group items (configuration 2's list; configuration 3's has group tiles)."""
    lengths, c = wl.config_lengths(cfg), wl.CONFIGS[cfg]
    hq, hkv = c["hq"], c["hkv"]
    banner("flag-free GQA sum", cfg, len(lengths))
    dev = torch.device("cuda")
    plan = att._plan(att._cu_seqlens(lengths, dev), hq, hkv)
    lib = att.lib()
    if cfg == 3:
        assert plan.bwd_finish_stage == att._lib.VA_BWD_FINISH
        items, n_items = plan.partial_bwd()  # the same documents without group items
    else:
        assert plan.bwd_finish_stage == att._lib.VA_BWD_FINISH_HEADS
        items, n_items = plan.bwd_items, plan.n_bwd
    n = sum(lengths)
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(lengths, hq, hkv, torch.float16, seed=4))
    out = torch.empty_like(q)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    att.check(lib.va_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                         plan.fwd_items.data_ptr(), plan.n_fwd, n, hq, hkv, 128, SCALE, 0,
                         att._stream()), "va_fwd")
    ws = att.bwd_workspace(n, hq, hkv, dev)[0]
    dq = torch.empty_like(q)
    res = []
    for stage in (att._lib.VA_BWD_FINISH, att._lib.VA_BWD_FINISH_HEADS):
        dk, dv = torch.full_like(k, float("nan")), torch.full_like(v, float("nan"))
        argv = (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                lse.data_ptr(), items.data_ptr(), n_items, n, hq, hkv, 128, SCALE, 0,
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
                att._stream())
        att.check(lib.va_bwd_stage(att._lib.VA_BWD_MAIN, *argv), "va_bwd_stage")
        att.check(lib.va_bwd_stage(stage, *argv), "va_bwd_stage")
        res.append((dk, dv))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a, b)


STATS_CASES = [
    ([512, 300, 77, 1], 12, 2, torch.float16, att._lib.VA_PLAN_BWD),         # per-head items
    (wl.config_lengths(3), 12, 2, torch.float16, att._lib.VA_PLAN_BWD),      # pair items
    (wl.config_lengths(3), 12, 2, torch.float16, att._lib.VA_PLAN_BWD_GROUPS),
    ([300, 45, 1, 128], 28, 4, torch.bfloat16, att._lib.VA_PLAN_BWD_GROUPS_ALL),
    ([64, 37, 50, 12], 12, 12, torch.float16, att._lib.VA_PLAN_BWD),        # Hq == Hkv
    ([5, 33], 4, 2, torch.bfloat16, att._lib.VA_PLAN_BWD),
]


@pytest.mark.parametrize("lengths,hq,hkv,dtype,kind", STATS_CASES)
def test_row_statistics_pass_gives_bitwise_the_in_kernel_statistics(lengths, hq, hkv, dtype,
                                                                      kind):
    """VA_BWD_STATS + VA_BWD_MAIN_STATS (lse log2 e and rowsum(dO * O) formed once per row by a
    pass of their own) against VA_BWD_MAIN (formed by every item that stages the row): same
    arithmetic, so dQ, dK/dV and the per-head partials agree bit for bit, for every item shape."""
    banner("row statistics pass", len(lengths), sum(lengths), hq, hkv, dtype, kind)
    dev = torch.device("cuda")
    lib = att.lib()
    n = sum(lengths)
    cu = orc.cu_seqlens_from_lengths(lengths)
    items_np = att.build_plan_host(cu, hq, hkv, kind)
    items = torch.from_numpy(items_np).to(dev)
    fwd = torch.from_numpy(att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_FWD)).to(dev)
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(lengths, hq, hkv, dtype, seed=11))
    code = att._lib.VA_F16 if dtype == torch.float16 else att._lib.VA_BF16
    out = torch.empty_like(q)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    att.check(lib.va_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                         fwd.data_ptr(), fwd.shape[0], n, hq, hkv, 128, SCALE, code,
                         att._stream()), "va_fwd")
    grouped = kind in (att._lib.VA_PLAN_BWD_GROUPS, att._lib.VA_PLAN_BWD_GROUPS_ALL)
    res = []
    for stages in ([att._lib.VA_BWD_MAIN], [att._lib.VA_BWD_STATS, att._lib.VA_BWD_MAIN_STATS]):
        ws = torch.full((att.bwd_workspace(n, hq, hkv, dev)[0].numel(),), 255, dtype=torch.uint8,
                        device=dev)
        offs = att.bwd_workspace(n, hq, hkv, dev)[1]
        dq = torch.full_like(q, float("nan"))
        dk, dv = torch.full_like(k, float("nan")), torch.full_like(v, float("nan"))
        outs = [(dk, dv)] if (grouped or hq == hkv) else [(dk, dv), (None, None)]
        for dk_o, dv_o in outs:
            argv = (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                    lse.data_ptr(), items.data_ptr(), items.shape[0], n, hq, hkv, 128, SCALE,
                    code, dq.data_ptr(), _ptr_or_none(dk_o), _ptr_or_none(dv_o), ws.data_ptr(),
                    ws.numel(), att._stream())
            for st in stages + ([att._lib.VA_BWD_FINISH] if dk_o is not None else []):
                att.check(lib.va_bwd_stage(st, *argv), "va_bwd_stage")
            torch.cuda.synchronize()
            part = n * hq * 128 * 2
            parts = [ws[o: o + part].clone() for o in offs] if dk_o is None else []
            res.append([dq.clone(), dk.clone(), dv.clone(), *parts])
    half = len(res) // 2
    for a, b in zip(res[:half], res[half:]):
        for x, y in zip(a, b):
            if x.is_floating_point():
                assert not torch.isnan(x.float()).any()
            assert torch.equal(x, y)


def _ptr_or_none(t):
    return t.data_ptr() if t is not None else None


def test_device_plan_writes_cu_seqlens_without_a_forward_plan():
    """va_plan_build_device_lengths with only the backward plan requested still writes
    cu_seqlens_out (the backward's work-group writes it when there is no forward plan)."""
    lengths, hq, hkv = [334, 0, 200, 100, 7], 12, 2
    banner("device plan cu_seqlens, backward only", lengths)
    dev = torch.device("cuda")
    n = sum(lengths)
    cap = np.zeros(1, dtype=np.int64)
    att.check(att.lib().va_plan_capacity(n, len(lengths), hq, att._lib.VA_PLAN_BWD,
                                         cap.ctypes.data_as(att._lib._pi64)), "va_plan_capacity")
    items = torch.empty(int(cap[0]), 4, dtype=torch.int32, device=dev)
    cu = torch.full((len(lengths) + 1,), -7, dtype=torch.int32, device=dev)
    lens = torch.tensor(lengths, dtype=torch.int64, device=dev)
    att.check(att.lib().va_plan_build_device_lengths(lens.data_ptr(), len(lengths), n, hq, hkv,
                                                     None, 0, items.data_ptr(), int(cap[0]),
                                                     cu.data_ptr(), att._stream()),
              "va_plan_build_device_lengths")
    torch.cuda.synchronize()
    assert cu.cpu().tolist() == np.concatenate([[0], np.cumsum(lengths)]).tolist()
    host = att.build_plan_host(np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32), hq,
                               hkv, att._lib.VA_PLAN_BWD)
    got = [tuple(x) for x in items.cpu().numpy().tolist() if any(x)]
    assert sorted(got) == sorted(map(tuple, host.tolist()))


@pytest.mark.parametrize("lengths,hq,hkv,kind", [
    (wl.config_lengths(3), 12, 2, att._lib.VA_PLAN_BWD_GROUPS),      # S = 6, 3 and 2 tiles
    ([300, 45, 1, 128], 28, 4, att._lib.VA_PLAN_BWD_GROUPS_ALL),
    ([512, 300, 77, 1], 12, 2, att._lib.VA_PLAN_BWD_GROUPS_ALL),
])
def test_group_items_without_outputs_leave_exact_partials(lengths, hq, hkv, kind):
    """A group-item list run with dk = dv = NULL (the partials are the result): each group item
    writes its heads' sum into its first head's partial and zeros into the others', so the sum of
    all G partials of a row (VA_BWD_FINISH_HEADS, no row flags) is bitwise the dK/dV that the same
    list writes with outputs (group items at Hkv width, the flagged GQA sum for S < G)."""
    banner("group items without outputs", len(lengths), sum(lengths), hq, hkv, kind)
    dev = torch.device("cuda")
    lib = att.lib()
    n = sum(lengths)
    cu = orc.cu_seqlens_from_lengths(lengths)
    items = torch.from_numpy(att.build_plan_host(cu, hq, hkv, kind)).to(dev)
    fwd = torch.from_numpy(att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_FWD)).to(dev)
    q, k, v, do = (t.to(dev) for t in wl.make_inputs(lengths, hq, hkv, torch.float16, seed=13))
    out = torch.empty_like(q)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    att.check(lib.va_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                         fwd.data_ptr(), fwd.shape[0], n, hq, hkv, 128, SCALE, 0, att._stream()),
              "va_fwd")
    res = []
    for outputs in (True, False):
        ws = torch.full((att.bwd_workspace(n, hq, hkv, dev)[0].numel(),), 0x7f, dtype=torch.uint8,
                        device=dev)  # stale partials: 0x7f7f is a NaN in fp16
        dq = torch.empty_like(q)
        dk, dv = torch.full_like(k, float("nan")), torch.full_like(v, float("nan"))

        def argv(with_out):
            return (do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                    lse.data_ptr(), items.data_ptr(), items.shape[0], n, hq, hkv, 128, SCALE, 0,
                    dq.data_ptr(), dk.data_ptr() if with_out else None,
                    dv.data_ptr() if with_out else None, ws.data_ptr(), ws.numel(),
                    att._stream())
        if outputs:
            att.check(lib.va_bwd(*argv(True)), "va_bwd")
        else:
            att.check(lib.va_bwd_stage(att._lib.VA_BWD_MAIN, *argv(False)), "va_bwd_stage")
            att.check(lib.va_bwd_stage(att._lib.VA_BWD_FINISH_HEADS, *argv(True)), "va_bwd_stage")
        torch.cuda.synchronize()
        res.append((dq.clone(), dk.clone(), dv.clone()))
    for a, b in zip(*res):
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a, b)


ROTARY_CASES = [
    ([70, 33, 51, 1, 200], 12, 2, torch.float16, att._lib.VA_PLAN_BWD_HEADS, True),
    ([70, 33, 51, 1, 200], 12, 2, torch.float16, att._lib.VA_PLAN_BWD_PAIRS, True),
    ([70, 33, 51, 1, 200], 12, 2, torch.float16, att._lib.VA_PLAN_BWD_PAIRS, False),
    ([180] * 45, 12, 2, torch.float16, att._lib.VA_PLAN_BWD_GROUPS, True),     # S = 6, 3, 2
    ([180] * 45, 12, 2, torch.float16, att._lib.VA_PLAN_BWD_GROUPS, False),
    ([300, 45, 1, 128], 28, 4, torch.bfloat16, att._lib.VA_PLAN_BWD_GROUPS_ALL, True),
    ([64, 37, 50, 12], 4, 4, torch.float16, att._lib.VA_PLAN_BWD, True),         # Hq == Hkv
]


@pytest.mark.parametrize("lengths,hq,hkv,dtype,kind,outputs", ROTARY_CASES)
def test_rotary_backward_matches_oracle(lengths, hq, hkv, dtype, kind, outputs):
    """va_bwd_rotary_stage (the inverse rotation in the backward kernels' epilogues) against the
    oracle's backward followed by its inverse rotation (solution/attention.py:113-134), for every
    item shape: per-head q items (their halves split the (d, d + 64) pairs), pair items, group
    items of S < G and S = G heads, Hq == Hkv, and without outputs (rotated per-head partials
    summed by VA_BWD_FINISH_HEADS). Tables of random frequencies; rows by document, as the
    decoder's packed call forms them. The row statistics pass is used for one half of the cases."""
    banner("rotary backward", len(lengths), sum(lengths), hq, hkv, dtype, kind, outputs)
    dev = torch.device("cuda")
    lib = att.lib()
    n = sum(lengths)
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)])
    b_idx, t_idx = (rows // seq).to(torch.int32), (rows % seq).to(torch.int32)
    cos, sin = rope_tables(seq, seed=hq + n)
    tab, keep = att.rotary_tables(cos.to(dev), sin.to(dev), b_idx.to(dev), t_idx.to(dev))
    cu = orc.cu_seqlens_from_lengths(lengths)
    items = torch.from_numpy(att.build_plan_host(cu, hq, hkv, kind)).to(dev)
    fwd = torch.from_numpy(att.build_plan_host(cu, hq, hkv, att._lib.VA_PLAN_FWD)).to(dev)
    q, k, v, do = wl.make_inputs(lengths, hq, hkv, dtype, seed=n + hq)
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    code = att._lib.VA_F16 if dtype == torch.float16 else att._lib.VA_BF16
    out = torch.empty_like(qd)
    lse = torch.empty(hq, n, dtype=torch.float32, device=dev)
    att.check(lib.va_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                         lse.data_ptr(), fwd.data_ptr(), fwd.shape[0], n, hq, hkv, 128, SCALE, code,
                         att._stream()), "va_fwd")
    ws = att.bwd_workspace(n, hq, hkv, dev)[0]
    dq = torch.full_like(qd, float("nan"))
    dk, dv = torch.full_like(kd, float("nan")), torch.full_like(vd, float("nan"))
    stats = len(lengths) % 2 == 1

    def argv(with_out):
        return (dod.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                lse.data_ptr(), items.data_ptr(), items.shape[0], n, hq, hkv, 128, SCALE, code,
                dq.data_ptr(), dk.data_ptr() if with_out else None,
                dv.data_ptr() if with_out else None, ws.data_ptr(), ws.numel(), att._stream())
    if stats:
        att.check(lib.va_bwd_rotary_stage(att._lib.VA_BWD_STATS, ctypes.byref(tab), *argv(outputs)),
                  "va_bwd_rotary_stage")
    main = att._lib.VA_BWD_MAIN_STATS if stats else att._lib.VA_BWD_MAIN
    att.check(lib.va_bwd_rotary_stage(main, ctypes.byref(tab), *argv(outputs)),
              "va_bwd_rotary_stage")
    if hq != hkv:
        finish = att._lib.VA_BWD_FINISH if outputs else att._lib.VA_BWD_FINISH_HEADS
        att.check(lib.va_bwd_stage(finish, *argv(True)), "va_bwd_stage")
    torch.cuda.synchronize()
    o_ref, _lse, dq_ref, dk_ref, dv_ref = oracle(q, k, v, do, lengths)
    refs = (orc.rope_backward(dq_ref, cos.numpy(), sin.numpy(), b_idx, t_idx).reshape(n, hq, 128),
            orc.rope_backward(dk_ref, cos.numpy(), sin.numpy(), b_idx, t_idx).reshape(n, hkv, 128),
            dv_ref)
    for which, mine, ref in zip("qkv", (dq, dk, dv), refs):
        r = rel(mine.cpu().float().numpy(), ref)
        assert r <= TOL[dtype]["g"], (which, r)


def test_rope_forward_passes_v_through_when_it_needs_no_cast():
    """The packed rotation without expansion leaves the value rows out of the kernel when v is
    already in the compute type (v is returned as a view of itself); q and k come out bitwise as
    when the kernel also casts v (an fp32 v)."""
    lengths, heads, kv_heads = [70, 33, 200], 12, 2
    banner("rope forward, v as it is", lengths)
    seq = max(lengths)
    rows = torch.tensor([b * seq + t for b, length in enumerate(lengths) for t in range(length)])
    b_idx, t_idx = ((rows // seq).to(torch.int32).cuda(), (rows % seq).to(torch.int32).cuda())
    n = rows.numel()
    cos, sin = (t.cuda() for t in rope_tables(seq, seed=4))
    g = torch.Generator().manual_seed(2)
    q = torch.randn(n, heads * 128, generator=g).half().cuda()
    k = torch.randn(n, kv_heads * 128, generator=g).half().cuda()
    v = torch.randn(n, kv_heads * 128, generator=g).half().cuda()
    qa, ka, va = att.rope_forward(q, k, v, cos, sin, b_idx, t_idx, heads, kv_heads,
                                  torch.float16)
    # the same rotation with the value rows copied by the kernel
    qb, kb = torch.empty_like(qa), torch.empty_like(ka)
    vb = torch.empty(n, kv_heads, 128, dtype=torch.float16, device="cuda")
    tab_cos, tab_sin = cos.float().contiguous(), sin.float().contiguous()
    att.check(att.lib().va_rope_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), tab_cos.data_ptr(),
                                    tab_sin.data_ptr(), 0, 128, b_idx.data_ptr(),
                                    t_idx.data_ptr(), qb.data_ptr(), kb.data_ptr(),
                                    vb.data_ptr(), n, heads, kv_heads, 128, 0, 0, 0, 0, 0,
                                    att._stream()), "va_rope_fwd")
    torch.cuda.synchronize()
    assert va.data_ptr() == v.data_ptr() and va.shape == (n, kv_heads, 128)
    assert torch.equal(qa, qb) and torch.equal(ka, kb)
    assert torch.equal(va, vb) and torch.equal(vb.reshape(n, -1), v)
    with pytest.raises(ValueError, match="share a dtype"):
        att.rope_forward(q, k, v.float(), cos, sin, b_idx, t_idx, heads, kv_heads, torch.float16)


def test_ceiling_probes_run_and_copy_exactly():
    """The benchmark's ceiling probes: va_probe_mfma runs in fp16 and bf16 and leaves a finite
    value per thread; va_probe_copy copies a buffer (with a ragged tail past its last full
    stride) exactly."""
    banner("ceiling probes")
    lib = att._lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.full((8 * 256,), float("nan"), device="cuda")
    for code in (att._lib.VA_F16, att._lib.VA_BF16):
        att._lib.check(lib.va_probe_mfma(code, 8, 10, sink.data_ptr(), stream), "va_probe_mfma")
        torch.cuda.synchronize()
        assert bool(torch.isfinite(sink).all())
    n = 3 * 256 * 16 * 4 * 16 + 48  # bytes: three grid strides of 4 chunks and a short tail
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros_like(src)
    att._lib.check(lib.va_probe_copy(src.data_ptr(), dst.data_ptr(), n, 16, stream),
                   "va_probe_copy")
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
