"""Packed (padding-free) varlen causal GQA attention on MI355X: the reference's autograd surface
(solution/attention.py) over hand-written gfx950 HIP kernels reached through the C ABI.

Public surface, same names, argument order and number of returned gradients as the reference:

    qkv_rotate(q, k, v, cos, sin, b_idx, t_idx, batch, seq, heads, kv_heads, padded=False)
                                    solution/attention.py:191 (QKVRotate 150-188)
    varlen_attention(query, key, value, lengths, scale)
                                    solution/attention.py:236-242 (VarlenAttention 212-233)
    packed_attention(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths, scale)
                                    solution/attention.py:282-285 (PackedAttention 250-279)
    pack_rows(attn, b_idx, t_idx)   solution/attention.py:328 (PackRows 303-325)

Differences that keep the drop-in contract:
* `varlen_attention` accepts key/value with Hkv heads (GQA-native: the kernels read each key/value
  head once for its G query heads) as well as the reference's expanded Hq-head form.
* `packed_attention` rotates q and k without expanding K/V to the query heads and runs the
  attention on Hkv key/value heads; its backward sums dK/dV over each GQA group in fp32 (the
  reference sums its expanded fp16 copies, solution/attention.py:113-134) and rotates dQ and dK
  back, in the backward kernels' epilogues for long lists, else in a pass of its own. The
  backward is deterministic.
* fp16 and bf16 inputs both run on the MFMA kernels (the reference computes in fp16 only).

Every op requires the HIP library and CUDA (HIP) tensors; there is no other implementation.
"""

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check, lib
from .offload import OFFLOADER

HEAD_DIM = 128

_DTYPES = {torch.float16: _lib.VA_F16, torch.bfloat16: _lib.VA_BF16, torch.float32: _lib.VA_F32}


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(stream):
    return stream.cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _require_device(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("hackaton_amd attention runs on the GPU only: got a tensor on "
                             f"{t.device}")


def _attn_dtype(t):
    if t.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"attention inputs must be float16 or bfloat16, got {t.dtype}")
    return _DTYPES[t.dtype]


# ------------------------------------------------------------------------------------------------
# cu_seqlens and work plans
# ------------------------------------------------------------------------------------------------
_CU_SEQLENS = {}
_PLANS = {}


def _cu_seqlens(lengths, device):
    """Document start offsets (and the total) as an int32 device tensor, one tensor per distinct
    list of lengths and device, reused by every layer of a step (solution/attention.py:198-209).
    The host copy of the offsets is attached to the tensor, so the planner never reads the GPU."""
    key = (device, tuple(lengths))
    cu = _CU_SEQLENS.get(key)
    if cu is None:
        if len(_CU_SEQLENS) > 16:
            _CU_SEQLENS.clear()
        offsets = [0]
        for length in lengths:
            offsets.append(offsets[-1] + int(length))
        cu = torch.tensor(offsets, dtype=torch.int32, device=device)
        cu._va_offsets = tuple(offsets)
        _CU_SEQLENS[key] = cu
    return cu


class Plan:
    """Device work lists of the forward and backward kernels for one (cu_seqlens, Hq, Hkv). The
    forward list splits its longest items into narrow ones where it is short (VA_PLAN_FWD_NARROW);
    the backward list takes GQA group items where they do not lengthen it (VA_PLAN_BWD_GROUPS); a
    backward that leaves per-head dK/dV partials to its caller takes `partial_bwd()`, the list
    without them."""

    __slots__ = ("fwd_items", "n_fwd", "bwd_items", "n_bwd", "total", "offsets", "_hq", "_hkv",
                 "_part", "bwd_finish", "bwd_finish_stage", "bwd_stats")

    def __init__(self, offsets, hq, hkv, device):
        cu = np.ascontiguousarray(np.asarray(offsets, dtype=np.int32))
        self.offsets = tuple(int(x) for x in cu)
        self.total = int(cu[-1])
        self._hq, self._hkv = hq, hkv
        bwd_kind = _lib.VA_PLAN_BWD_GROUPS if hq > hkv else _lib.VA_PLAN_BWD
        # the forward list with its longest items split in two where it leaves CUs idle
        host_fwd = build_plan_host(cu, hq, hkv, _lib.VA_PLAN_FWD_NARROW)
        host_bwd = build_plan_host(cu, hq, hkv, bwd_kind)
        self.n_fwd, self.n_bwd = host_fwd.shape[0], host_bwd.shape[0]
        self.fwd_items = torch.from_numpy(host_fwd).to(device)
        self.bwd_items = torch.from_numpy(host_bwd).to(device)
        self._part = None if hq > hkv else (self.bwd_items, self.n_bwd)
        # whether the backward needs its GQA sum: not when every key tile's group items take the
        # whole GQA group (item word: group bit 21, heads - 1 in bits 12-19)
        kv = host_bwd[(host_bwd[:, 3] >> 24) == 0]
        grouped = ((kv[:, 3] >> 21) & 1) == 1
        whole = grouped & ((((kv[:, 3] >> 12) & 0xFF) + 1) == hq // hkv)
        self.bwd_finish = hq > hkv and not bool(whole.all())
        # the GQA sum of a list without group items reads no row flags (VA_BWD_FINISH_HEADS)
        self.bwd_finish_stage = _lib.VA_BWD_FINISH if bool(grouped.any()) else \
            _lib.VA_BWD_FINISH_HEADS
        # the backward's row statistics in a pass of their own where the documents are long
        # enough for it to pay (va_plan_bwd_row_stats)
        self.bwd_stats = bwd_row_stats(cu)

    def partial_bwd(self):
        """(items, n) of the backward list without group items (built on first use)."""
        if self._part is None:
            cu = np.asarray(self.offsets, dtype=np.int32)
            host = build_plan_host(cu, self._hq, self._hkv, _lib.VA_PLAN_BWD)
            self._part = (torch.from_numpy(host).to(self.bwd_items.device), host.shape[0])
        return self._part


def bwd_row_stats(cu):
    """Whether the backward's row statistics {lse log2 e, rowsum(dO * O)} pay for a pass of their
    own over these documents (the C planner's rule: on average VA_BWD_STATS_MIN_TILES or more
    128-key tiles cover each query row)."""
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    use = np.zeros(1, dtype=np.int32)
    check(lib().va_plan_bwd_row_stats(cu.ctypes.data_as(_lib._pi32), cu.shape[0] - 1,
                                      use.ctypes.data_as(_lib._pi32)), "va_plan_bwd_row_stats")
    return bool(use[0])


def build_plan_host(cu, hq, hkv, kind):
    """Work items (n, 4) int32 from the C planner (host only)."""
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    n_docs = cu.shape[0] - 1
    n = np.zeros(1, dtype=np.int64)
    cu_p = cu.ctypes.data_as(_lib._pi32)
    check(lib().va_plan_size(cu_p, n_docs, hq, hkv, kind, n.ctypes.data_as(_lib._pi64)),
          "va_plan_size")
    items = np.zeros((max(int(n[0]), 1), 4), dtype=np.int32)
    written = np.zeros(1, dtype=np.int64)
    check(lib().va_plan_build(cu_p, n_docs, hq, hkv, kind, items.ctypes.data_as(_lib._pi32),
                              int(n[0]), written.ctypes.data_as(_lib._pi64)), "va_plan_build")
    return items[: int(n[0])]


class DevicePlan:
    """Work lists and cu_seqlens built on the device from device lengths: no host read. One launch
    (va_plan_build_device_lengths) builds cu_seqlens, the forward list (VA_PLAN_FWD_NARROW, as the
    host plan's) and the backward list
    without GQA group items; with Hq > Hkv a second (va_plan_build_device from that cu_seqlens)
    builds the backward list with them (VA_PLAN_BWD_GROUPS), and the first one serves a backward
    that leaves per-head partials to its caller. Each list has the capacity that the host-known
    sizes bound; its slots past the real items are empty items that the kernels skip."""

    __slots__ = ("fwd_items", "n_fwd", "bwd_items", "n_bwd", "total", "cu", "_part",
                 "bwd_finish", "bwd_finish_stage", "bwd_stats", "__weakref__")

    def __init__(self, lengths, n_tokens, hq, hkv):
        lengths = lengths.reshape(-1)
        if lengths.dtype != torch.int64:
            lengths = lengths.to(torch.int64)
        lengths = lengths.contiguous()
        n_docs = lengths.numel()
        self.total = int(n_tokens)
        dev = lengths.device
        caps = []
        for kind in (_lib.VA_PLAN_FWD_NARROW, _lib.VA_PLAN_BWD):
            cap = np.zeros(1, dtype=np.int64)
            check(lib().va_plan_capacity(n_tokens, n_docs, hq, kind, cap.ctypes.data_as(_lib._pi64)),
                  "va_plan_capacity")
            caps.append(int(cap[0]))
        self.n_fwd, self.n_bwd = caps
        self.fwd_items = torch.empty(max(self.n_fwd, 1), 4, dtype=torch.int32, device=dev)
        part = torch.empty(max(self.n_bwd, 1), 4, dtype=torch.int32, device=dev)
        self.cu = torch.empty(n_docs + 1, dtype=torch.int32, device=dev)
        check(lib().va_plan_build_device_lengths(
            lengths.data_ptr() if n_docs else None, n_docs, n_tokens, hq, hkv,
            self.fwd_items.data_ptr(), self.n_fwd, part.data_ptr(), self.n_bwd,
            self.cu.data_ptr(), _stream()), "va_plan_build_device_lengths")
        self._part = (part, self.n_bwd)
        self.bwd_items = part
        self.bwd_finish = hq > hkv  # the device list's group tiles are not known here
        self.bwd_finish_stage = _lib.VA_BWD_FINISH
        self.bwd_stats = False  # the document lengths are not known on the host
        if hq > hkv and n_docs > 0:
            self.bwd_items = torch.empty_like(part)
            check(lib().va_plan_build_device(self.cu.data_ptr(), n_docs, n_tokens, hq, hkv,
                                             _lib.VA_PLAN_BWD_GROUPS, self.bwd_items.data_ptr(),
                                             self.n_bwd, _stream()), "va_plan_build_device")
        self.cu._va_plan = self

    def partial_bwd(self):
        """(items, n) of the backward list without group items."""
        return self._part


def _capture_id():
    cid = ctypes.c_uint64(0)
    check(lib().va_stream_capture_id(_stream(), ctypes.byref(cid)), "va_stream_capture_id")
    return cid.value


def _device_plan(lengths, n_tokens, hq, hkv):
    """The device plan of a device lengths tensor, built once and reused by every layer that gets
    the same tensor (unchanged since: its version counter is part of the key). A plan built while
    a graph is being captured is reused only inside that same capture, and one built outside any
    capture never inside one: a captured graph then always contains the plan build its replays
    need."""
    key = (lengths._version, int(n_tokens), hq, hkv, _capture_id())
    cache = getattr(lengths, "_va_plans", None)
    if cache is None:
        cache = {}
        lengths._va_plans = cache
    plan = cache.get(key)
    if plan is None:
        if len(cache) > 8:
            cache.clear()
        plan = cache[key] = DevicePlan(lengths, n_tokens, hq, hkv)
    return plan


def _plan(cu_seqlens, hq, hkv):
    device_plan = getattr(cu_seqlens, "_va_plan", None)
    if device_plan is not None:
        return device_plan
    offsets = getattr(cu_seqlens, "_va_offsets", None)
    if offsets is None:  # a cu_seqlens tensor not made by _cu_seqlens: read it (one sync)
        offsets = tuple(int(x) for x in cu_seqlens.cpu().tolist())
    key = (cu_seqlens.device, offsets, hq, hkv)
    plan = _PLANS.get(key)
    if plan is None:
        if len(_PLANS) > 32:
            _PLANS.clear()
        plan = _PLANS[key] = Plan(offsets, hq, hkv, cu_seqlens.device)
    return plan


# ------------------------------------------------------------------------------------------------
# attention forward / backward through the C ABI
# ------------------------------------------------------------------------------------------------
def attention_forward(query, key, value, plan, scale):
    """(out (N, Hq, D), lse (Hq, N) fp32) of packed causal attention; query (N, Hq, D),
    key/value (N, Hkv, D), all contiguous, same 16-bit dtype."""
    _require_device(query, key, value)
    dtype = _attn_dtype(query)
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("query, key and value must share a dtype")
    n, hq, d = query.shape
    hkv = key.shape[1]
    if key.shape != (n, hkv, d) or value.shape != key.shape:
        raise ValueError(f"shape mismatch: q {tuple(query.shape)} k {tuple(key.shape)} "
                         f"v {tuple(value.shape)}")
    if n != plan.total:
        raise ValueError(f"{n} tokens but cu_seqlens covers {plan.total}")
    out = torch.empty_like(query)
    lse = torch.empty(hq, n, dtype=torch.float32, device=query.device)
    check(lib().va_fwd(_ptr(query), _ptr(key), _ptr(value), _ptr(out), _ptr(lse),
                       _ptr(plan.fwd_items), plan.n_fwd, n, hq, hkv, d, float(scale), dtype,
                       _stream()), "va_fwd")
    return out, lse


def bwd_workspace_needed(hq, hkv, outputs=True):
    """Whether the backward needs its workspace (per-query-head dK/dV partials, row flags and row
    statistics): not when Hq == Hkv and dK/dV are returned, which the kernels then write directly
    (the reference's expanded-K/V call, solution/attention.py:230-232)."""
    return hq != hkv or not outputs


def bwd_workspace(n, hq, hkv, device):
    """Workspace of the backward (per-query-head dK/dV partials, row flags, row statistics) and
    the byte offsets of the two partial arrays."""
    offsets = np.zeros(2, dtype=np.int64)
    nbytes = np.zeros(1, dtype=np.int64)
    check(lib().va_bwd_workspace_layout(n, hq, hkv, HEAD_DIM, offsets.ctypes.data_as(_lib._pi64),
                                        nbytes.ctypes.data_as(_lib._pi64)),
          "va_bwd_workspace_layout")
    return torch.empty(int(nbytes[0]), dtype=torch.uint8, device=device), [int(x) for x in offsets]


def bwd_stages(plan, outputs=True, workspace=True):
    """The va_bwd_stage calls of one backward over `plan`: the row-statistics pass where the plan
    says it pays (it needs the workspace), the main kernel, and the GQA sum unless the plan's group
    items wrote every dK/dV row, Hq == Hkv, or the per-head partials are the result."""
    stats = workspace and getattr(plan, "bwd_stats", False)
    stages = [_lib.VA_BWD_STATS, _lib.VA_BWD_MAIN_STATS] if stats else [_lib.VA_BWD_MAIN]
    if outputs and getattr(plan, "bwd_finish", True):
        stages.append(getattr(plan, "bwd_finish_stage", _lib.VA_BWD_FINISH))
    return stages


def attention_backward(grad, query, key, value, out, lse, plan, scale, outputs=True, rope=None):
    """dq, dk, dv of packed causal attention (dk/dv summed over each GQA group), deterministic.
    With outputs=False returns dq and the per-query-head dK/dV partials (N, Hq, D) in the element
    type (plus the workspace that holds them), for a caller that sums them itself. With `rope`
    (rotary_tables(...)) dq and dk come out rotated back to the projections' frame by the
    kernels' epilogues (va_bwd_rotary_stage)."""
    n, hq, d = query.shape
    hkv = key.shape[1]
    dtype = _attn_dtype(query)
    grad = grad.reshape(out.shape)
    if grad.dtype != query.dtype:
        grad = grad.to(query.dtype)
    grad = grad.contiguous()
    dq = torch.empty_like(query)
    if outputs:
        dk, dv = torch.empty_like(key), torch.empty_like(value)
    else:
        dk = dv = None
    if bwd_workspace_needed(hq, hkv, outputs):
        ws, offs = bwd_workspace(n, hq, hkv, query.device)
    else:
        ws, offs = None, None
    items, n_items = (plan.bwd_items, plan.n_bwd) if outputs else plan.partial_bwd()
    argv = (_ptr(grad), _ptr(query), _ptr(key), _ptr(value), _ptr(out), _ptr(lse),
            _ptr(items), n_items, n, hq, hkv, d, float(scale), dtype,
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ws.numel() if ws is not None else 0,
            _stream())
    for stage in bwd_stages(plan, outputs, ws is not None):
        if rope is None:
            check(lib().va_bwd_stage(stage, *argv), "va_bwd_stage")
        else:
            check(lib().va_bwd_rotary_stage(stage, ctypes.byref(rope[0]), *argv),
                  "va_bwd_rotary_stage")
    if outputs:
        return dq, dk, dv
    part = n * hq * d * 2

    def view(off):
        return ws[off: off + part].view(query.dtype).view(n, hq, d)

    return dq, view(offs[0]), view(offs[1]), ws


class VarlenAttention(torch.autograd.Function):
    """Autograd node of the attention itself: one forward launch over all documents of the packed
    rows, and the backward launches, driven by a work plan built from `cu_seqlens`. Query rows
    (N, H, D); key/value rows (N, Hkv, D) with Hkv dividing H (Hkv = H is the expanded form the
    reference passes). Returns (N, H * D). Replaces solution/attention.py:212-233."""

    @staticmethod
    def forward(ctx, query, key, value, cu_seqlens, max_len, scale):
        plan = _plan(cu_seqlens, query.shape[1], key.shape[1])
        out, lse = attention_forward(query, key, value, plan, scale)
        ctx.save_for_backward(query, key, value, out, lse, cu_seqlens)
        ctx.max_len, ctx.scale, ctx.plan = max_len, scale, plan
        return out.reshape(query.shape[0], query.shape[1] * query.shape[2])

    @staticmethod
    def backward(ctx, grad):
        query, key, value, out, lse, _cu = ctx.saved_tensors
        dq, dk, dv = attention_backward(grad, query, key, value, out, lse, ctx.plan, ctx.scale)
        return dq, dk, dv, None, None, None


def _lengths_cu(lengths, device, hq, hkv, n_tokens):
    """cu_seqlens for `lengths`: a host list (zero lengths dropped, as solution/attention.py:239;
    the plan is built on the host and cached) or a device tensor (cu_seqlens and both plans are
    built on the device by one launch, cached on the tensor: no host read, no synchronisation)."""
    if isinstance(lengths, torch.Tensor) and lengths.is_cuda:
        return _device_plan(lengths, n_tokens, hq, hkv).cu, None
    lengths = [int(length) for length in lengths if int(length) > 0]
    if not lengths:  # the reference's max() of no lengths raises ValueError too (attention.py:242)
        raise ValueError("varlen attention: every length is zero (no tokens to attend over)")
    return _cu_seqlens(lengths, device), max(lengths)


def varlen_attention(query, key, value, lengths, scale):
    """Packed rows hold documents back to back, document i being the next `lengths[i]` rows; each
    query row attends causally to the rows of its own document only. Returns (N, H * D).
    `lengths` is a host list (zero entries are skipped) or a device tensor, in which case the
    document offsets and the work plan are built on the GPU with no host read.
    Same call as solution/attention.py:236-242."""
    cu_seqlens, max_len = _lengths_cu(lengths, query.device, query.shape[1], key.shape[1],
                                      query.shape[0])
    return VarlenAttention.apply(query.contiguous(), key.contiguous(), value.contiguous(),
                                 cu_seqlens, max_len, scale)


# ------------------------------------------------------------------------------------------------
# rotary embedding
# ------------------------------------------------------------------------------------------------
def _rope_strides(cos):
    scb = 0 if cos.shape[0] == 1 else cos.stride(0)
    return scb, cos.stride(1)


def _tables(cos, sin):
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    if cos.shape != sin.shape or cos.dim() != 3 or cos.shape[-1] != HEAD_DIM:
        raise ValueError(f"cos/sin must be (1 or B, T, {HEAD_DIM}), got {tuple(cos.shape)}")
    return cos, sin


def rotary_tables(cos, sin, b_idx, t_idx):
    """The va_rope_tables of a packed call (fp32 cos/sin (1 or B, T, D), int32 token rows and
    positions) and the tensors it points to (kept alive beside it)."""
    _require_device(cos, sin, b_idx, t_idx)
    cos, sin = _tables(cos, sin)
    b_idx = b_idx.to(torch.int32).contiguous()
    t_idx = t_idx.to(torch.int32).contiguous()
    scb, sct = _rope_strides(cos)
    tab = _lib.RopeTables(cos.data_ptr(), sin.data_ptr(), scb, sct, b_idx.data_ptr(),
                          t_idx.data_ptr())
    return tab, (cos, sin, b_idx, t_idx)


def rope_forward(q, k, v, cos, sin, b_idx, t_idx, heads, kv_heads, out_dtype, layout=0,
                 expand=False, batch=0, seq=0):
    """Rotated q, k and cast v as three tensors of `out_dtype`, in the packed (N, H, D) or the
    zero-filled padded (B, H, T, D) layout; K/V keep kv_heads unless `expand`. A packed,
    unexpanded v already in `out_dtype` is returned as a view of itself (the kernel leaves the
    value rows out)."""
    _require_device(q, k, v, cos, sin, b_idx, t_idx)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    cos, sin = _tables(cos, sin)
    n = q.shape[0]
    kvo = heads if expand else kv_heads
    if q.shape[1] != heads * HEAD_DIM or k.shape[1] != kv_heads * HEAD_DIM or v.shape != k.shape:
        raise ValueError("projection shapes do not match heads * head_dim")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    v_as_is = layout == _lib.VA_LAYOUT_PACKED and not expand and v.dtype == out_dtype
    if layout == _lib.VA_LAYOUT_PADDED:
        qo = torch.zeros(batch, heads, seq, HEAD_DIM, dtype=out_dtype, device=q.device)
        ko, vo = torch.zeros_like(qo), torch.zeros_like(qo)
    else:
        qo = torch.empty(n, heads, HEAD_DIM, dtype=out_dtype, device=q.device)
        ko = torch.empty(n, kvo, HEAD_DIM, dtype=out_dtype, device=q.device)
        vo = v.view(n, kv_heads, HEAD_DIM) if v_as_is else torch.empty_like(ko)
    scb, sct = _rope_strides(cos)
    check(lib().va_rope_fwd(_ptr(q), _ptr(k), None if v_as_is else _ptr(v), _ptr(cos), _ptr(sin),
                            scb, sct, _ptr(b_idx), _ptr(t_idx), _ptr(qo), _ptr(ko),
                            None if v_as_is else _ptr(vo), n, heads, kv_heads, HEAD_DIM, seq,
                            _DTYPES[q.dtype], _DTYPES[out_dtype], layout, int(expand), _stream()),
          "va_rope_fwd")
    return qo, ko, vo


def rope_backward(dq, dk, dv, cos, sin, b_idx, t_idx, heads, kv_heads, out_dtype, layout=0,
                  expand=False, seq=0):
    """Projection gradients (N, heads*D), (N, kv_heads*D) x2 in `out_dtype` from the gradients of
    the rotated tensors (expanded ones are summed over each GQA group first)."""
    n = b_idx.shape[0]
    dq, dk, dv = dq.contiguous(), dk.contiguous(), dv.contiguous()
    cos, sin = _tables(cos, sin)
    dq_in = torch.empty(n, heads * HEAD_DIM, dtype=out_dtype, device=dq.device)
    dk_in = torch.empty(n, kv_heads * HEAD_DIM, dtype=out_dtype, device=dq.device)
    dv_in = torch.empty_like(dk_in)
    scb, sct = _rope_strides(cos)
    if not (dq.dtype == dk.dtype == dv.dtype):
        raise ValueError("gradient dtypes differ")
    check(lib().va_rope_bwd(_ptr(dq), _ptr(dk), _ptr(dv), _ptr(cos), _ptr(sin), scb, sct,
                            _ptr(b_idx), _ptr(t_idx), _ptr(dq_in), _ptr(dk_in), _ptr(dv_in), n,
                            heads, kv_heads, HEAD_DIM, seq, _DTYPES[dq.dtype], _DTYPES[out_dtype],
                            layout, int(expand), _stream()), "va_rope_bwd")
    return dq_in, dk_in, dv_in


class QKVRotate(torch.autograd.Function):
    """Rotary embedding of the query and key projections plus the fp16 cast of the values, with
    key/value heads repeated to the query-head count. Projections come in as packed rows
    (N, heads * D); the three results are packed (N, heads, D) rows, or a zero-filled
    (B, heads, T, D) batch when `padded` is set. Backward: the inverse rotation, after summing the
    repeated heads. Same outputs and 12 returned gradients as solution/attention.py:150-188."""

    @staticmethod
    def forward(ctx, q, k, v, cos, sin, b_idx, t_idx, batch, seq, heads, kv_heads, padded):
        layout = _lib.VA_LAYOUT_PADDED if padded else _lib.VA_LAYOUT_PACKED
        qo, ko, vo = rope_forward(q, k, v, cos, sin, b_idx, t_idx, heads, kv_heads,
                                  torch.float16, layout, True, batch, seq)
        ctx.save_for_backward(cos, sin, b_idx, t_idx)
        ctx.meta = (seq, heads, kv_heads, q.dtype, layout)
        return qo, ko, vo

    @staticmethod
    def backward(ctx, dq, dk, dv):
        cos, sin, b_idx, t_idx = ctx.saved_tensors
        seq, heads, kv_heads, dtype, layout = ctx.meta
        dq_in, dk_in, dv_in = rope_backward(dq.half(), dk.half(), dv.half(), cos, sin, b_idx,
                                            t_idx, heads, kv_heads, dtype, layout, True, seq)
        return dq_in, dk_in, dv_in, None, None, None, None, None, None, None, None, None


def qkv_rotate(q, k, v, cos, sin, b_idx, t_idx, batch, seq, heads, kv_heads, padded=False):
    return QKVRotate.apply(q, k, v, cos, sin, b_idx, t_idx, batch, seq, heads, kv_heads, padded)


# ------------------------------------------------------------------------------------------------
# rotation + attention of the packed rows (the decoder layer's call)
# ------------------------------------------------------------------------------------------------
def _compute_dtype(proj_dtype):
    """Element type the attention runs in: bf16 projections stay bf16, everything else runs in
    fp16 like the reference (solution/attention.py:21-22: one rounding to fp16 after the rotation)."""
    return torch.bfloat16 if proj_dtype == torch.bfloat16 else torch.float16


def _attend(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths, scale):
    """Rotation (no K/V expansion) + varlen attention; returns (out (N,Hq,D), lse, rotated q/k/v,
    plan). solution/attention.py:245-247."""
    cu, _max_len = _lengths_cu(lengths, q.device, heads, kv_heads, q.shape[0])
    plan = _plan(cu, heads, kv_heads)
    qr, kr, vr = rope_forward(q, k, v, cos, sin, b_idx, t_idx, heads, kv_heads,
                              _compute_dtype(q.dtype))
    out, lse = attention_forward(qr, kr, vr, plan, scale)
    return out, lse, (qr, kr, vr), plan


# What PackedAttention keeps for its backward when it does not offload: "outputs" keeps the
# rotated q/k/v, O and the log-sum-exp in HBM and skips the forward recomputation (one attention
# forward and one rotation fewer per layer and step, for N * Hq * D * e + 4 * Hq * N bytes more
# per layer: 6.4 MB per 2048-token layer at the 1.5B shape in fp16); "inputs" keeps q/k/v and recomputes
# the rotation and the forward in the backward, as solution/attention.py:250-279 does. Both give
# the same gradients bit for bit (the forward is deterministic). With offload the inputs go to
# host memory and the forward is recomputed either way (the offloader's contract).
SAVE_POLICY = "outputs"
_SAVE_POLICIES = ("outputs", "inputs")


def set_save_policy(policy):
    """Select what PackedAttention keeps for its backward: "outputs" (default) or "inputs"."""
    global SAVE_POLICY
    if policy not in _SAVE_POLICIES:
        raise ValueError(f"save policy must be one of {_SAVE_POLICIES}, got {policy!r}")
    SAVE_POLICY = policy


def rotary_epilogues(n_tokens, heads):
    """Whether PackedAttention's backward rotates dQ and dK back in the attention kernels'
    epilogues (va_bwd_rotary_stage) rather than leaving per-head partials to the standalone
    inverse rotation. The epilogues read the fp32 tables (1 KB per row) once per query head and
    row, where the standalone pass reads them once per token, but save that pass's round trip of
    dQ and the partials: they pay where the lists hold many items (ceil(N / 128) Hq >=
    VA_FWD_MANY_ITEMS; measured at configurations 3-5: 125 -> 114, 231 -> 223, 1419 -> 1394 us per
    layer call), and lose at a few long items (configuration 2: 50.0 -> 51.9 us), whose epilogues
    then set the time. A rule of the sizes only, so host and device lengths take the same route."""
    return _lib.fwd_many_items(n_tokens, heads)


class PackedAttention(torch.autograd.Function):
    """Autograd node of the decoder layer's call: rotary embedding, then causal attention of every
    document of the packed rows; returns (N, heads * D) in the compute type.

    The backward runs the attention backward kernels and the inverse rotation: in the kernels'
    epilogues (dQ and dK rotated back in fp32 before their one rounding) where the lists are long,
    else as a pass of its own that sums per-query-head dK/dV partials over each GQA group in fp32
    while it rotates (rotary_epilogues). What is kept for it follows
    SAVE_POLICY: the rotated operands, O and lse ("outputs"), or only the three projections,
    recomputing the rotation and the forward like solution/attention.py:250-279 ("inputs", and
    always when `offload` moves them to pinned host memory). Returns the three projection
    gradients and 10 Nones."""

    @staticmethod
    def forward(ctx, q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths, scale,
                offload):
        with torch.no_grad():
            out, lse, rot, plan = _attend(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads,
                                          lengths, scale)
        ctx.consts = (cos, sin, b_idx, t_idx)
        ctx.meta = (seq, heads, kv_heads, lengths, scale)
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        ctx.saved_outputs = False
        if offload:
            ctx.item = OFFLOADER.save(q, k, v)
        elif SAVE_POLICY == "outputs":
            ctx.saved_outputs = True
            ctx.plan = plan
            ctx.save_for_backward(*rot, out, lse)
        else:
            ctx.save_for_backward(q, k, v)
        return out.reshape(out.shape[0], out.shape[1] * out.shape[2]).to(_compute_dtype(q.dtype))

    @staticmethod
    def backward(ctx, dout):
        cos, sin, b_idx, t_idx = ctx.consts
        seq, heads, kv_heads, lengths, scale = ctx.meta
        if ctx.saved_outputs:
            qr, kr, vr, out, lse = ctx.saved_tensors
            plan = ctx.plan
        else:
            q, k, v = OFFLOADER.load(ctx.item) if hasattr(ctx, "item") else ctx.saved_tensors
            out, lse, (qr, kr, vr), plan = _attend(q, k, v, cos, sin, b_idx, t_idx, seq, heads,
                                                   kv_heads, lengths, scale)
        q_dtype, k_dtype, v_dtype = ctx.dtypes
        n = qr.shape[0]
        if rotary_epilogues(n, heads):
            # the inverse rotation in the attention backward's epilogues: dq and dk come out as
            # the projections' gradients, dK/dV summed over each GQA group by group items or the
            # GQA sum of rotated partials (solution/attention.py:113-134 sums expanded copies)
            dq, dk, dv = attention_backward(dout, qr, kr, vr, out, lse, plan, scale,
                                            rope=rotary_tables(cos, sin, b_idx, t_idx))
            dq, dk, dv = dq.reshape(n, -1), dk.reshape(n, -1), dv.reshape(n, -1)
        else:
            # dq and the per-query-head dK/dV partials; the inverse rotation sums the partials
            # over each GQA group in fp32 while it rotates (as attention.py:113-134 sums copies)
            dq_r, dk_part, dv_part, _ws = attention_backward(dout, qr, kr, vr, out, lse, plan,
                                                             scale, outputs=False)
            dq, dk, dv = rope_backward(dq_r, dk_part, dv_part, cos, sin, b_idx, t_idx, heads,
                                       kv_heads, q_dtype, expand=True)
        grads = (dq.to(q_dtype), dk.to(k_dtype), dv.to(v_dtype))
        return (*grads, None, None, None, None, None, None, None, None, None, None)


def packed_attention(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths, scale):
    offload = OFFLOADER.wants(q, k, v) and (q.requires_grad or k.requires_grad or v.requires_grad)
    return PackedAttention.apply(q, k, v, cos, sin, b_idx, t_idx, seq, heads, kv_heads, lengths,
                                 scale, offload)


# ------------------------------------------------------------------------------------------------
# padded -> packed rows (fallback layout)
# ------------------------------------------------------------------------------------------------
class PackRows(torch.autograd.Function):
    """Gathers the real tokens of a padded (B, H, T, D) attention result into packed
    (N, H * D) rows for the output projection; the backward scatters the row gradients back into
    a zero-filled padded tensor. Used by the masked fallback. solution/attention.py:303-325."""

    @staticmethod
    def forward(ctx, attn, b_idx, t_idx):
        _require_device(attn, b_idx, t_idx)
        batch, heads, seq, dim = attn.shape
        attn = attn.contiguous()
        out = torch.empty(b_idx.shape[0], heads * dim, dtype=attn.dtype, device=attn.device)
        check(lib().va_pack_rows(_ptr(attn), _ptr(out), _ptr(b_idx), _ptr(t_idx), b_idx.shape[0],
                                 heads, seq, dim, attn.element_size(), 0, _stream()),
              "va_pack_rows")
        ctx.save_for_backward(b_idx, t_idx)
        ctx.meta = (batch, heads, seq, dim)
        return out

    @staticmethod
    def backward(ctx, grad):
        b_idx, t_idx = ctx.saved_tensors
        batch, heads, seq, dim = ctx.meta
        grad = grad.contiguous()
        padded = torch.zeros(batch, heads, seq, dim, dtype=grad.dtype, device=grad.device)
        check(lib().va_pack_rows(_ptr(grad), _ptr(padded), _ptr(b_idx), _ptr(t_idx),
                                 b_idx.shape[0], heads, seq, dim, grad.element_size(), 1,
                                 _stream()), "va_pack_rows")
        return padded, None, None


def pack_rows(attn, b_idx, t_idx):
    return PackRows.apply(attn, b_idx, t_idx)
