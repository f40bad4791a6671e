"""CPU oracle for packed variable-length causal GQA attention (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it. The shipped path (`hackaton_amd`) runs the HIP
kernels and raises when they are missing.

It restates, in numpy, the arithmetic of the reference path:

* `cu_seqlens_from_lengths`   solution/attention.py:195-209 and :239 (drop zero lengths, int32
                              prefix sums).
* `rope_forward`              solution/attention.py:57-83 (fp32 rotation y1 = x1*c1 - x2*s1,
                              y2 = x2*c2 + x1*s2, rounded once; cos/sin row `b*scb + t*sct`).
* `rope_backward`             solution/attention.py:106-134 (sum of the G copies, then the inverse
                              rotation dx1 = dy1*c1 + dy2*s2, dx2 = dy2*c2 - dy1*s1).
* `attention_forward`         the arithmetic of aten::_efficient_attention_forward as called at
                              solution/attention.py:221-222: per-document causal softmax attention
                              (custom_mask_type=1, top-left), scale given, log-sum-exp per row.
                              GQA head mapping h -> h // G is transformers' repeat_kv
                              (modeling_qwen2.py:138-147, restated at test_attention.py:26-27).
* `attention_backward`        aten::_efficient_attention_backward at solution/attention.py:230-232
                              followed by the GQA sum of solution/attention.py:113-134.
* `pack_rows` / `unpack_rows` solution/attention.py:288-325 (exact gather / zero-filled scatter).

Pinning (tests/test_oracle.py): every function here is checked against something that does not
retype its formula: torch's own scaled_dot_product_attention (forward and autograd backward, fp64),
the reference test's padded masked-SDPA construction (test_attention.py:95-106), transformers'
apply_rotary_pos_emb/repeat_kv, brute-force pure-Python loops, closed forms (length-1 documents,
constant keys), invariants (rows of P sum to 1, rowsum(dS) = 0) and central finite differences of
the forward for the backward. The log-sum-exp output of `attention_forward` is pinned by the
closed form of length-1 documents, by torch.logsumexp over the masked logits and by a
brute-force loop.

All arithmetic is in the dtype requested (float64 for checking, float32 for the CPU baseline).
Layouts: q (N, Hq, D), k/v (N, Hkv, D), o (N, Hq, D), lse (Hq, N).
"""

import numpy as np


def cu_seqlens_from_lengths(lengths):
    """[0, l0, l0+l1, ...] as int32, zero lengths dropped (solution/attention.py:198-209, :239)."""
    lens = [int(x) for x in lengths if int(x) > 0]
    cu = np.zeros(len(lens) + 1, dtype=np.int32)
    if lens:
        cu[1:] = np.cumsum(np.asarray(lens, dtype=np.int64)).astype(np.int32)
    return cu


def _docs(cu):
    cu = np.asarray(cu, dtype=np.int64)
    return [(int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1) if cu[i + 1] > cu[i]]


def _causal_mask(n):
    """True where key j <= query i (top-left causal, custom_mask_type=1)."""
    return np.tril(np.ones((n, n), dtype=bool))


def attention_forward(q, k, v, cu, scale, dtype=np.float64):
    """Per-document causal GQA attention. Returns (o (N,Hq,D), lse (Hq,N)) in `dtype`.

    Follows aten::_efficient_attention_forward as solution/attention.py:221-222 calls it:
    softmax(scale * q k^T + causal mask) v within each document of cu_seqlens; lse is the natural
    log-sum-exp of the scaled, masked logits of each row."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    n, hq, d = q.shape
    hkv = k.shape[1]
    assert hq % hkv == 0, "query heads must be a multiple of key/value heads"
    g = hq // hkv
    o = np.zeros((n, hq, d), dtype=dtype)
    lse = np.full((hq, n), np.nan, dtype=dtype)
    kv_of = np.arange(hq) // g  # repeat_kv: query head h reads key/value head h // G
    for s, e in _docs(cu):
        length = e - s
        qh = q[s:e].transpose(1, 0, 2)                     # (Hq, L, D)
        kh = k[s:e][:, kv_of].transpose(1, 2, 0)           # (Hq, D, L)
        vh = v[s:e][:, kv_of].transpose(1, 0, 2)           # (Hq, L, D)
        logits = np.matmul(qh, kh) * dtype(scale)          # (Hq, L, L)
        logits = np.where(_causal_mask(length)[None], logits, -np.inf)
        m = logits.max(axis=-1, keepdims=True)
        p = np.exp(logits - m)
        denom = p.sum(axis=-1, keepdims=True)
        o[s:e] = (np.matmul(p, vh) / denom).transpose(1, 0, 2)
        lse[:, s:e] = (m + np.log(denom))[..., 0]
    return o, lse


def attention_backward(q, k, v, o, lse, do, cu, scale, dtype=np.float64):
    """Gradients (dq (N,Hq,D), dk (N,Hkv,D), dv (N,Hkv,D)) of attention_forward.

    P is recomputed from lse (as aten::_efficient_attention_backward does, attention.py:230-232);
    dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)), dQ = scale dS K, dK = scale dS^T Q,
    then dK/dV of the G query heads sharing a key/value head are summed (attention.py:113-134)."""
    q, k, v, o, do = (np.asarray(x, dtype=dtype) for x in (q, k, v, o, do))
    lse = np.asarray(lse, dtype=dtype)
    n, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    kv_of = np.arange(hq) // g
    dq = np.zeros_like(q)
    dk = np.zeros((n, hkv, d), dtype=dtype)
    dv = np.zeros((n, hkv, d), dtype=dtype)
    for s, e in _docs(cu):
        length = e - s
        qh = q[s:e].transpose(1, 0, 2)
        kh = k[s:e][:, kv_of].transpose(1, 0, 2)
        vh = v[s:e][:, kv_of].transpose(1, 0, 2)
        oh = o[s:e].transpose(1, 0, 2)
        doh = do[s:e].transpose(1, 0, 2)
        logits = np.matmul(qh, kh.transpose(0, 2, 1)) * dtype(scale)
        p = np.exp(logits - lse[:, s:e, None])
        p = np.where(_causal_mask(length)[None], p, 0.0)
        dvh = np.matmul(p.transpose(0, 2, 1), doh)                  # (Hq, L, D)
        dp = np.matmul(doh, vh.transpose(0, 2, 1))                   # (Hq, L, L)
        delta = (doh * oh).sum(axis=-1, keepdims=True)               # (Hq, L, 1)
        ds = p * (dp - delta)
        dqh = np.matmul(ds, kh) * dtype(scale)
        dkh = np.matmul(ds.transpose(0, 2, 1), qh) * dtype(scale)
        dq[s:e] = dqh.transpose(1, 0, 2)
        for h in range(hq):
            dk[s:e, kv_of[h]] += dkh[h]
            dv[s:e, kv_of[h]] += dvh[h]
    return dq, dk, dv


def _cos_sin_rows(cos, sin, b_idx, t_idx):
    """cos/sin row of each packed token: row `b` of (B, T, D) tables, or row 0 of (1, T, D)
    tables (attention.py:45-49 and :160, scb = 0 when cos.shape[0] == 1)."""
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    b = np.asarray(b_idx, dtype=np.int64)
    t = np.asarray(t_idx, dtype=np.int64)
    if cos.shape[0] == 1:
        b = np.zeros_like(b)
    return cos[b, t], sin[b, t]


def rope_forward(x, cos, sin, b_idx, t_idx, heads):
    """Rotate packed projections x (N, heads*D) with the reference's fp32 formula
    (attention.py:57-63): returns float32 (N, heads, D); the caller rounds once."""
    x = np.asarray(x, dtype=np.float32)
    n = x.shape[0]
    d = x.shape[1] // heads
    half = d // 2
    c, s = _cos_sin_rows(cos, sin, b_idx, t_idx)       # (N, D)
    c1, c2, s1, s2 = c[:, None, :half], c[:, None, half:], s[:, None, :half], s[:, None, half:]
    xh = x.reshape(n, heads, d)
    x1, x2 = xh[..., :half], xh[..., half:]
    return np.concatenate((x1 * c1 - x2 * s1, x2 * c2 + x1 * s2), axis=-1)


def rope_backward(dy, cos, sin, b_idx, t_idx):
    """Inverse rotation of a gradient dy (N, heads, D) in fp32 (attention.py:106-134):
    dx1 = dy1*c1 + dy2*s2, dx2 = dy2*c2 - dy1*s1. Returns float32 (N, heads*D)."""
    dy = np.asarray(dy, dtype=np.float32)
    n, heads, d = dy.shape
    half = d // 2
    c, s = _cos_sin_rows(cos, sin, b_idx, t_idx)
    c1, c2, s1, s2 = c[:, None, :half], c[:, None, half:], s[:, None, :half], s[:, None, half:]
    dy1, dy2 = dy[..., :half], dy[..., half:]
    return np.concatenate((dy1 * c1 + dy2 * s2, dy2 * c2 - dy1 * s1), axis=-1).reshape(n, heads * d)


def gqa_expand(x, heads):
    """(N, Hkv, D) -> (N, heads, D), query head h reading kv head h // G (attention.py:71-83)."""
    x = np.asarray(x)
    g = heads // x.shape[1]
    return x[:, np.arange(heads) // g]


def gqa_reduce(dx, kv_heads):
    """(N, heads, D) -> (N, kv_heads, D): sum of the G copies in fp32 (attention.py:113-134)."""
    dx = np.asarray(dx, dtype=np.float32)
    n, heads, d = dx.shape
    return dx.reshape(n, kv_heads, heads // kv_heads, d).sum(axis=2)


def pack_rows(attn, b_idx, t_idx):
    """(B, H, T, D) -> (N, H*D) rows of the real tokens (attention.py:297-298)."""
    attn = np.asarray(attn)
    b = np.asarray(b_idx, dtype=np.int64)
    t = np.asarray(t_idx, dtype=np.int64)
    return attn[b, :, t, :].reshape(len(b), -1)


def unpack_rows(grad, b_idx, t_idx, batch, heads, seq):
    """(N, H*D) -> (B, H, T, D), zeros at padding (attention.py:299-300, :322)."""
    grad = np.asarray(grad)
    b = np.asarray(b_idx, dtype=np.int64)
    t = np.asarray(t_idx, dtype=np.int64)
    n = grad.shape[0]
    d = grad.shape[1] // heads
    out = np.zeros((batch, heads, seq, d), dtype=grad.dtype)
    out[b, :, t, :] = grad.reshape(n, heads, d)
    return out


def causal_pairs(cu):
    """P = sum over documents of L (L + 1) / 2: the allowed (query, key) pairs per head."""
    return sum((e - s) * (e - s + 1) // 2 for s, e in _docs(cu))


def attention_flops(cu, hq, d):
    """Causal FLOPs of one forward + backward: F = 3.5 * 4 * Hq * D * P (recompute not counted)."""
    return 3.5 * 4.0 * hq * d * causal_pairs(cu)
