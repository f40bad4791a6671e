"""Pins the CPU oracle (oracle/attention_oracle.py) to things that do not retype its formulas:
torch's own scaled_dot_product_attention and autograd, the reference test's padded masked-SDPA
construction (solution/test_attention.py:95-106), transformers' rotary embedding and repeat_kv,
brute-force loops, closed forms, adjoint identities and finite differences."""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_oracle as orc

SCALE = 128 ** -0.5


def rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float64) * scale).numpy()


def sdpa_per_doc(q, k, v, lengths, scale, grad=None):
    """torch SDPA (fp64, causal, enable_gqa) per document: out (N,Hq,D) and grads."""
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    outs, s = [], 0
    for length in lengths:
        e = s + length
        o = F.scaled_dot_product_attention(qt[s:e].transpose(0, 1)[None],
                                           kt[s:e].transpose(0, 1)[None],
                                           vt[s:e].transpose(0, 1)[None], is_causal=True,
                                           scale=scale, enable_gqa=True)
        outs.append(o[0].transpose(0, 1))
        s = e
    out = torch.cat(outs)
    grads = None
    if grad is not None:
        out.backward(torch.tensor(grad))
        grads = [x.grad.numpy() for x in (qt, kt, vt)]
    return out.detach().numpy(), grads


CASES = [([64, 37, 50, 12], 4, 2), ([17, 1, 9], 6, 1), ([33, 20], 4, 4), ([5, 8, 1, 1], 6, 2)]


@pytest.mark.parametrize("lengths,hq,hkv", CASES)
def test_forward_matches_torch_sdpa(lengths, hq, hkv):
    n = sum(lengths)
    q, k, v = rand((n, hq, 128), 1), rand((n, hkv, 128), 2), rand((n, hkv, 128), 3)
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, SCALE)
    ref, _ = sdpa_per_doc(q, k, v, lengths, SCALE)
    np.testing.assert_allclose(o, ref, rtol=1e-12, atol=1e-12)
    # lse: torch.logsumexp of the masked logits built by torch
    g = hq // hkv
    s = 0
    for length in lengths:
        e = s + length
        qt = torch.tensor(q[s:e]).transpose(0, 1)
        kt = torch.tensor(k[s:e]).repeat_interleave(g, dim=1).transpose(0, 1)
        logits = qt @ kt.transpose(1, 2) * SCALE
        logits = logits.masked_fill(~torch.ones(length, length, dtype=torch.bool).tril(),
                                    float("-inf"))
        np.testing.assert_allclose(lse[:, s:e], torch.logsumexp(logits, -1).numpy(), rtol=1e-12,
                                   atol=1e-12)
        s = e


@pytest.mark.parametrize("lengths,hq,hkv", CASES)
def test_backward_matches_torch_autograd(lengths, hq, hkv):
    n = sum(lengths)
    q, k, v = rand((n, hq, 128), 4), rand((n, hkv, 128), 5), rand((n, hkv, 128), 6)
    do = rand((n, hq, 128), 7)
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, SCALE)
    dq, dk, dv = orc.attention_backward(q, k, v, o, lse, do, cu, SCALE)
    _, (rq, rk, rv) = sdpa_per_doc(q, k, v, lengths, SCALE, grad=do)
    for mine, theirs in ((dq, rq), (dk, rk), (dv, rv)):
        np.testing.assert_allclose(mine, theirs, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("lengths", [[64, 37, 50, 12], [34, 20, 10, 7]])
def test_forward_backward_match_reference_test_construction(lengths):
    """The reference test's ground truth: zero-padded dense SDPA with a `tril & real` mask over
    expanded (H = 12) heads (solution/test_attention.py:89-110), here in fp64 on the CPU."""
    batch, seq, heads, dim = len(lengths), max(lengths), 12, 128
    n = sum(lengths)
    q, k, v, do = (rand((n, heads, dim), 10 + i) for i in range(4))
    real = torch.zeros(batch, seq, dtype=torch.bool)
    for row, length in enumerate(lengths):
        real[row, :length] = True
    rows = torch.nonzero(real.reshape(-1), as_tuple=True)[0]
    mask = torch.ones(seq, seq, dtype=torch.bool).tril()[None, None] & real[:, None, None]
    leaves = [torch.tensor(x, requires_grad=True) for x in (q, k, v)]

    def padded(x):
        full = torch.zeros(batch * seq, heads, dim, dtype=x.dtype)
        return full.index_copy(0, rows, x).view(batch, seq, heads, dim).transpose(1, 2)

    ref = F.scaled_dot_product_attention(*[padded(x) for x in leaves], attn_mask=mask,
                                         scale=dim ** -0.5)
    ref = ref.transpose(1, 2).reshape(batch * seq, heads * dim)[rows]
    ref.backward(torch.tensor(do).reshape(n, heads * dim))
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, dim ** -0.5)
    np.testing.assert_allclose(o.reshape(n, -1), ref.detach().numpy(), rtol=1e-10, atol=1e-10)
    grads = orc.attention_backward(q, k, v, o, lse, do, cu, dim ** -0.5)
    for mine, leaf in zip(grads, leaves):
        np.testing.assert_allclose(mine, leaf.grad.numpy(), rtol=1e-10, atol=1e-10)


def test_brute_force_loops():
    """Pure-Python softmax attention on a tiny GQA case."""
    lengths, hq, hkv, d = [3, 1, 4], 4, 2, 5
    n = sum(lengths)
    q, k, v = rand((n, hq, d), 20), rand((n, hkv, d), 21), rand((n, hkv, d), 22)
    scale = 0.37
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, scale)
    s = 0
    for length in lengths:
        for h in range(hq):
            kvh = h // (hq // hkv)
            for i in range(s, s + length):
                logits = [scale * sum(q[i, h, c] * k[j, kvh, c] for c in range(d))
                          for j in range(s, i + 1)]
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                tot = sum(w)
                for c in range(d):
                    ref = sum(w[jj] * v[s + jj, kvh, c] for jj in range(len(w))) / tot
                    assert abs(o[i, h, c] - ref) < 1e-12
                assert abs(lse[h, i] - (mx + math.log(tot))) < 1e-12
        s += length


def test_closed_forms():
    hq, hkv, d = 4, 2, 128
    # a length-1 document: O = V row, lse = scale * q.k
    lengths = [1, 6]
    n = sum(lengths)
    q, k, v = rand((n, hq, d), 30), rand((n, hkv, d), 31), rand((n, hkv, d), 32)
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, SCALE)
    for h in range(hq):
        np.testing.assert_allclose(o[0, h], v[0, h // 2], rtol=0, atol=1e-14)
        np.testing.assert_allclose(lse[h, 0], SCALE * q[0, h] @ k[0, h // 2], rtol=1e-13)
    # constant keys within a document: O = prefix mean of V, and dQ = 0 (rowsum(dS) = 0)
    k2 = k.copy()
    k2[1:] = k2[1]
    o2, lse2 = orc.attention_forward(q, k2, v, cu, SCALE)
    for i in range(1, n):
        for h in range(hq):
            np.testing.assert_allclose(o2[i, h], v[1:i + 1, h // 2].mean(axis=0), atol=1e-12)
    do = rand((n, hq, d), 33)
    dq, _, _ = orc.attention_backward(q, k2, v, o2, lse2, do, cu, SCALE)
    np.testing.assert_allclose(dq[1:], 0.0, atol=1e-12)
    # V = 1 everywhere: O = 1 (rows of P sum to 1)
    o3, _ = orc.attention_forward(q, k, np.ones_like(v), cu, SCALE)
    np.testing.assert_allclose(o3, 1.0, atol=1e-13)


def test_backward_finite_differences():
    lengths, hq, hkv, d = [4, 3], 4, 2, 8
    n = sum(lengths)
    q, k, v = rand((n, hq, d), 40), rand((n, hkv, d), 41), rand((n, hkv, d), 42)
    do = rand((n, hq, d), 43)
    cu = orc.cu_seqlens_from_lengths(lengths)
    o, lse = orc.attention_forward(q, k, v, cu, 0.7)
    grads = orc.attention_backward(q, k, v, o, lse, do, cu, 0.7)
    eps = 1e-6
    for which in range(3):
        direction = rand((q, k, v)[which].shape, 50 + which)
        plus = [q, k, v]
        minus = [q, k, v]
        plus[which] = plus[which] + eps * direction
        minus[which] = minus[which] - eps * direction
        fd = (np.sum(do * orc.attention_forward(*plus, cu, 0.7)[0])
              - np.sum(do * orc.attention_forward(*minus, cu, 0.7)[0])) / (2 * eps)
        assert abs(fd - np.sum(grads[which] * direction)) < 1e-6 * max(1.0, abs(fd))


def test_rope_matches_transformers():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb, repeat_kv
    lengths, seq, heads, kv_heads, dim = [5, 3, 7], 7, 4, 2, 128
    batch = len(lengths)
    rows = [b * seq + t for b, length in enumerate(lengths) for t in range(length)]
    b_idx = np.array([r // seq for r in rows], dtype=np.int32)
    t_idx = np.array([r % seq for r in rows], dtype=np.int32)
    n = len(rows)
    inv_freq = 1.0 / (1000000.0 ** (torch.arange(0, dim, 2).float() / dim))
    for per_batch in (False, True):
        pos = torch.arange(seq).float()[None].repeat(batch if per_batch else 1, 1)
        if per_batch:
            pos = pos + torch.arange(batch)[:, None] * 3.0
        freqs = pos[..., None] * inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        cos, sin = emb.cos(), emb.sin()  # (1 or B, T, D)
        q = rand((n, heads * dim), 60).astype(np.float32)
        k = rand((n, kv_heads * dim), 61).astype(np.float32)
        qpad = torch.zeros(batch * seq, heads * dim)
        qpad[rows] = torch.tensor(q)
        kpad = torch.zeros(batch * seq, kv_heads * dim)
        kpad[rows] = torch.tensor(k)
        q4 = qpad.view(batch, seq, heads, dim).transpose(1, 2)
        k4 = kpad.view(batch, seq, kv_heads, dim).transpose(1, 2)
        cexp = cos.expand(batch, seq, dim)
        sexp = sin.expand(batch, seq, dim)
        qr, kr = apply_rotary_pos_emb(q4, k4, cexp, sexp)
        qr = qr.transpose(1, 2).reshape(batch * seq, heads, dim)[rows].numpy()
        kr = repeat_kv(kr, heads // kv_heads).transpose(1, 2).reshape(batch * seq, heads, dim)
        kr = kr[rows].numpy()
        mine_q = orc.rope_forward(q, cos.numpy(), sin.numpy(), b_idx, t_idx, heads)
        mine_k = orc.gqa_expand(orc.rope_forward(k, cos.numpy(), sin.numpy(), b_idx, t_idx,
                                                 kv_heads), heads)
        np.testing.assert_allclose(mine_q, qr, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(mine_k, kr, rtol=1e-6, atol=1e-6)
        # backward: the adjoint of the forward rotation, <R x, y> = <x, R^T y>
        dy = rand((n, heads, dim), 62).astype(np.float32)
        lhs = float(np.sum(mine_q.astype(np.float64) * dy))
        rhs = float(np.sum(q.astype(np.float64)
                           * orc.rope_backward(dy, cos.numpy(), sin.numpy(), b_idx, t_idx)))
        assert abs(lhs - rhs) < 1e-3 * max(1.0, abs(lhs))
        # and torch autograd of transformers' rotation gives the same gradient
        qleaf = torch.tensor(q, requires_grad=True)
        qp = torch.zeros(batch * seq, heads * dim).index_copy(0, torch.tensor(rows), qleaf)
        qr2, _ = apply_rotary_pos_emb(qp.view(batch, seq, heads, dim).transpose(1, 2), k4, cexp,
                                      sexp)
        packed = qr2.transpose(1, 2).reshape(batch * seq, heads, dim)[rows]
        packed.backward(torch.tensor(dy))
        np.testing.assert_allclose(orc.rope_backward(dy, cos.numpy(), sin.numpy(), b_idx, t_idx),
                                   qleaf.grad.numpy(), rtol=1e-5, atol=1e-5)


def test_gqa_expand_reduce_adjoint():
    from transformers.models.qwen2.modeling_qwen2 import repeat_kv
    x = rand((9, 2, 16), 70)
    ex = orc.gqa_expand(x, 6)
    ref = repeat_kv(torch.tensor(x).transpose(0, 1)[None], 3)[0].transpose(0, 1).numpy()
    np.testing.assert_array_equal(ex, ref)
    y = rand((9, 6, 16), 71)
    lhs = np.sum(ex * y)
    rhs = np.sum(x * orc.gqa_reduce(y, 2))
    assert abs(lhs - rhs) < 1e-4 * max(1.0, abs(lhs))


def test_pack_rows_matches_indexing():
    lengths, seq, heads, dim = [50, 20, 33], 64, 3, 16
    rows = [b * seq + t for b, length in enumerate(lengths) for t in range(length)]
    b_idx = np.array([r // seq for r in rows])
    t_idx = np.array([r % seq for r in rows])
    attn = rand((len(lengths), heads, seq, dim), 80)
    ref = attn.transpose(0, 2, 1, 3).reshape(-1, heads * dim)[rows]
    np.testing.assert_array_equal(orc.pack_rows(attn, b_idx, t_idx), ref)
    back = orc.unpack_rows(ref, b_idx, t_idx, len(lengths), heads, seq)
    mask = np.zeros((len(lengths), seq), dtype=bool)
    for b, length in enumerate(lengths):
        mask[b, :length] = True
    np.testing.assert_array_equal(back.transpose(0, 2, 1, 3)[mask], attn.transpose(0, 2, 1, 3)[mask])
    assert np.all(back.transpose(0, 2, 1, 3)[~mask] == 0)


def test_cu_seqlens_drops_zero_lengths():
    np.testing.assert_array_equal(orc.cu_seqlens_from_lengths([3, 0, 5, 0]), [0, 3, 8])
    assert orc.cu_seqlens_from_lengths([]).tolist() == [0]
    assert orc.causal_pairs(orc.cu_seqlens_from_lengths([3, 8])) == 6 + 36


def test_flops_formula_counts_pairs():
    # 4 x 512 causal, Hq = 12: F = 3.5 * 4 * 12 * 128 * 4 * 512 * 513 / 2
    cu = orc.cu_seqlens_from_lengths([512] * 4)
    assert orc.attention_flops(cu, 12, 128) == pytest.approx(11.30e9, rel=1e-3)
    brute = sum(1 for length in [7, 3] for i, j in itertools.product(range(length), repeat=2)
                if j <= i)
    assert orc.causal_pairs(orc.cu_seqlens_from_lengths([7, 3])) == brute
