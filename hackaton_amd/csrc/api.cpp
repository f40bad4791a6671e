// C-ABI entry points: argument validation, then the kernel launchers. Nothing here allocates,
// frees or synchronises; every launch goes to the caller's stream.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/varlen_attn.h"
#include "va_api_internal.h"
#include "va_kernels.h"

static_assert(va::kFwdLeanMinItems == VA_FWD_MANY_ITEMS, "forward kernel switch: header and kernels");
static_assert(va::kBwdPairMinItems == VA_BWD_PAIR_MIN_ITEMS && VA_PLAN_BWD_HEADS == 2 &&
                  VA_PLAN_BWD_PAIRS == 3 && VA_PLAN_BWD_GROUPS == 4 &&
                  VA_PLAN_BWD_GROUPS_ALL == 5,
              "backward plan kinds: header and planners");

namespace va {

char* last_error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

}  // namespace va

namespace {

constexpr int32_t kAbiVersion = 1;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int hip_fail(hipError_t e, const char* what) {
  va::fail((int)e, "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

int check_attn_shape(int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim) {
  if (head_dim != va::kHeadDim)
    return va::fail(VA_ESHAPE, "head_dim=%d, the kernels are built for %d", head_dim, va::kHeadDim);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return va::fail(VA_ESHAPE, "Hq=%d must be a positive multiple of Hkv=%d", hq, hkv);
  if (total_tokens < 0 || total_tokens > INT32_MAX / 2)
    return va::fail(VA_ESHAPE, "total_tokens=%lld out of range", (long long)total_tokens);
  if (total_tokens * (int64_t)hq > INT32_MAX)
    return va::fail(VA_ESHAPE, "total_tokens * Hq exceeds the 32-bit row index");
  return VA_OK;
}

int check_dtype16(int32_t dtype) {
  if (dtype != VA_F16 && dtype != VA_BF16)
    return va::fail(VA_EDTYPE, "dtype %d: attention runs on VA_F16 or VA_BF16", dtype);
  return VA_OK;
}

int check_ptrs(std::initializer_list<const void*> ptrs, const char* what) {
  for (const void* p : ptrs) {
    if (p == nullptr) return va::fail(VA_EINVAL, "%s: NULL buffer", what);
    if (!aligned16(p)) return va::fail(VA_EINVAL, "%s: buffer not 16-byte aligned", what);
  }
  return VA_OK;
}

int64_t round256(int64_t x) { return (x + 255) & ~int64_t(255); }


}  // namespace

extern "C" const char* va_last_error(void) { return va::last_error_buffer(); }
extern "C" int32_t va_abi_version(void) { return kAbiVersion; }
extern "C" int32_t va_head_dim(void) { return va::kHeadDim; }

extern "C" int va_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                      const int32_t* items, int64_t n_items, int64_t total_tokens, int32_t hq,
                      int32_t hkv, int32_t head_dim, float scale, int32_t dtype, void* stream) {
  return va_fwd_kernel(VA_FWD_AUTO, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                       head_dim, scale, dtype, stream);
}

extern "C" int va_fwd_kernel(int32_t kernel, const void* q, const void* k, const void* v,
                             void* out, float* lse, const int32_t* items, int64_t n_items,
                             int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim,
                             float scale, int32_t dtype, void* stream) {
  if (kernel != VA_FWD_AUTO && kernel != VA_FWD_WIDE && kernel != VA_FWD_MANY)
    return va::fail(VA_EINVAL, "va_fwd_kernel: kernel %d", kernel);
  int rc = check_attn_shape(total_tokens, hq, hkv, head_dim);
  if (rc) return rc;
  if ((rc = check_dtype16(dtype))) return rc;
  if (n_items < 0 || n_items > INT32_MAX) return va::fail(VA_EINVAL, "n_items out of range");
  if (!std::isfinite(scale) || scale <= 0.f)
    return va::fail(VA_EINVAL, "scale must be finite and positive");
  if (n_items == 0 || total_tokens == 0) return VA_OK;
  if ((rc = check_ptrs({q, k, v, out, lse, items}, "va_fwd"))) return rc;
  if (kernel == VA_FWD_AUTO)
    kernel = (total_tokens + va::kFwdBlockM - 1) / va::kFwdBlockM * hq >= VA_FWD_MANY_ITEMS
                 ? VA_FWD_MANY
                 : VA_FWD_WIDE;
  va::FwdArgs a{q, k, v, out, lse, items, n_items, total_tokens, hq, hkv, scale, dtype,
                (hipStream_t)stream, kernel};
  hipError_t e = va::launch_fwd(a);
  return e == hipSuccess ? VA_OK : hip_fail(e, "va_fwd launch");
}

extern "C" int va_bwd_workspace_layout(int64_t total_tokens, int32_t hq, int32_t hkv,
                                       int32_t head_dim, int64_t offsets[2], int64_t* bytes) {
  int rc = check_attn_shape(total_tokens, hq, hkv, head_dim);
  if (rc) return rc;
  if (offsets == nullptr || bytes == nullptr) return va::fail(VA_EINVAL, "NULL output");
  const int64_t part = round256(total_tokens * hq * head_dim * 2);
  offsets[0] = 0;     // per-query-head dK partials (N, Hq, D), element type
  offsets[1] = part;  // per-query-head dV partials
  // then (N) uint32 row flags at 2 part: which rows a GQA group item finished itself; then
  // (Hq, N) x 2 fp32 row statistics {lse log2 e, rowsum(dO * O)} of the row-statistics pass
  *bytes = 2 * part + round256(total_tokens * 4) + round256(total_tokens * hq * 8);
  return VA_OK;
}

namespace va {

int bwd_checked(int32_t stage, const void* dout, const void* q, const void* k, const void* v,
                const void* out, const float* lse, const int32_t* items, int64_t n_items,
                int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim, float scale,
                int32_t dtype, void* dq, void* dk, void* dv, void* workspace,
                int64_t workspace_bytes, void* stream, const va_rope_tables* rope) {
  int rc = check_attn_shape(total_tokens, hq, hkv, head_dim);
  if (rc) return rc;
  va::RopeTab tab{nullptr, nullptr, nullptr, nullptr, 0, 0};
  if (rope != nullptr) {
    if (rope->cos == nullptr || rope->sin == nullptr || rope->b_idx == nullptr ||
        rope->t_idx == nullptr)
      return va::fail(VA_EINVAL, "va_bwd_rotary_stage: NULL rotary table or index");
    if (!aligned16(rope->cos) || !aligned16(rope->sin))
      return va::fail(VA_EINVAL, "va_bwd_rotary_stage: cos/sin not 16-byte aligned");
    if (rope->cos_batch_stride < 0 || rope->cos_seq_stride < 0 ||
        rope->cos_batch_stride % 4 != 0 || rope->cos_seq_stride % 4 != 0 ||
        rope->cos_batch_stride > INT32_MAX || rope->cos_seq_stride > INT32_MAX)
      return va::fail(VA_EINVAL,
                      "va_bwd_rotary_stage: cos/sin strides must be non-negative multiples of 4");
    tab = va::RopeTab{rope->cos, rope->sin, rope->b_idx, rope->t_idx,
                      (int)rope->cos_batch_stride, (int)rope->cos_seq_stride};
  }
  if ((rc = check_dtype16(dtype))) return rc;
  if (n_items < 0 || n_items > INT32_MAX) return va::fail(VA_EINVAL, "n_items out of range");
  if (!std::isfinite(scale) || scale <= 0.f)
    return va::fail(VA_EINVAL, "scale must be finite and positive");
  if ((dk == nullptr) != (dv == nullptr))
    return va::fail(VA_EINVAL, "va_bwd: dk and dv must both be given or both be NULL");
  // With Hq == Hkv and outputs given, the per-head dK/dV are the outputs: no workspace needed.
  const bool direct = dk != nullptr && hq == hkv;
  int64_t offs[2], need = 0;
  va_bwd_workspace_layout(total_tokens, hq, hkv, head_dim, offs, &need);
  if (total_tokens == 0) return VA_OK;
  if (!direct && workspace_bytes < need)
    return va::fail(VA_ECAPACITY, "workspace %lld bytes, need %lld", (long long)workspace_bytes,
                    (long long)need);
  if ((rc = check_ptrs({dout, q, k, v, out, lse, dq}, "va_bwd"))) return rc;
  if (n_items > 0 && (rc = check_ptrs({items}, "va_bwd items"))) return rc;
  if (dk != nullptr && (rc = check_ptrs({dk, dv}, "va_bwd outputs"))) return rc;
  if (!direct && (rc = check_ptrs({workspace}, "va_bwd workspace"))) return rc;
  char* ws = static_cast<char*>(workspace);
  void* dk_part = direct ? dk : static_cast<void*>(ws + offs[0]);
  void* dv_part = direct ? dv : static_cast<void*>(ws + offs[1]);
  uint32_t* flags = direct ? nullptr : reinterpret_cast<uint32_t*>(ws + 2 * offs[1]);
  // The row statistics exist for the stages that write or read them (they need the workspace).
  const bool with_stats = stage == VA_BWD_STATS || stage == VA_BWD_MAIN_STATS;
  if (with_stats && direct && (rc = check_ptrs({workspace}, "va_bwd workspace (statistics)")))
    return rc;
  if (with_stats && direct && workspace_bytes < need)
    return va::fail(VA_ECAPACITY, "workspace %lld bytes, the row statistics need %lld",
                    (long long)workspace_bytes, (long long)need);
  float* stats = with_stats ? reinterpret_cast<float*>(ws + 2 * offs[1] + round256(total_tokens * 4))
                            : nullptr;
  va::BwdArgs a{dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv, scale, dtype,
                dq, dk_part, dv_part, dk, dv, flags, stats, (hipStream_t)stream, tab};
  const int kstage = stage == VA_BWD_MAIN_STATS ? 1 : stage == VA_BWD_STATS ? 4 : stage;
  hipError_t e = stage < 0 ? va::launch_bwd(a) : va::launch_bwd_stage(a, kstage);
  return e == hipSuccess ? VA_OK : hip_fail(e, "va_bwd launch");
}

}  // namespace va

extern "C" int va_bwd(const void* dout, const void* q, const void* k, const void* v,
                      const void* out, const float* lse, const int32_t* items, int64_t n_items,
                      int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim, float scale,
                      int32_t dtype, void* dq, void* dk, void* dv, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  return va::bwd_checked(-1, dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                         head_dim, scale, dtype, dq, dk, dv, workspace, workspace_bytes, stream,
                         nullptr);
}

extern "C" int va_bwd_stage(int32_t stage, const void* dout, const void* q, const void* k,
                            const void* v, const void* out, const float* lse,
                            const int32_t* items, int64_t n_items, int64_t total_tokens,
                            int32_t hq, int32_t hkv, int32_t head_dim, float scale, int32_t dtype,
                            void* dq, void* dk, void* dv, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (stage != VA_BWD_MAIN && stage != VA_BWD_FINISH && stage != VA_BWD_FINISH_HEADS &&
      stage != VA_BWD_STATS && stage != VA_BWD_MAIN_STATS)
    return va::fail(VA_EINVAL, "va_bwd_stage: stage %d", stage);
  return va::bwd_checked(stage, dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                         head_dim, scale, dtype, dq, dk, dv, workspace, workspace_bytes, stream,
                         nullptr);
}

extern "C" int va_bwd_rotary_stage(int32_t stage, const va_rope_tables* rope, const void* dout,
                                   const void* q, const void* k, const void* v, const void* out,
                                   const float* lse, const int32_t* items, int64_t n_items,
                                   int64_t total_tokens, int32_t hq, int32_t hkv,
                                   int32_t head_dim, float scale, int32_t dtype, void* dq,
                                   void* dk, void* dv, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  if (stage != VA_BWD_MAIN && stage != VA_BWD_FINISH && stage != VA_BWD_FINISH_HEADS &&
      stage != VA_BWD_STATS && stage != VA_BWD_MAIN_STATS)
    return va::fail(VA_EINVAL, "va_bwd_rotary_stage: stage %d", stage);
  if (rope == nullptr) return va::fail(VA_EINVAL, "va_bwd_rotary_stage: rope is NULL");
  return va::bwd_checked(stage, dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                         head_dim, scale, dtype, dq, dk, dv, workspace, workspace_bytes, stream,
                         rope);
}

namespace {

int rope_common(const void* x0, const void* x1, const void* x2, const float* cos,
                const float* sin, const int32_t* b_idx, const int32_t* t_idx, void* y0, void* y1,
                void* y2, int64_t n_tokens, int32_t heads, int32_t kv_heads, int32_t head_dim,
                int32_t seq, int32_t in_dtype, int32_t out_dtype, int32_t layout, int32_t expand,
                const char* what) {
  if (head_dim != va::kHeadDim)
    return va::fail(VA_ESHAPE, "%s: head_dim=%d, built for %d", what, head_dim, va::kHeadDim);
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0)
    return va::fail(VA_ESHAPE, "%s: heads=%d must be a positive multiple of kv_heads=%d", what,
                    heads, kv_heads);
  if (n_tokens < 0 || n_tokens > INT32_MAX) return va::fail(VA_ESHAPE, "%s: n_tokens", what);
  if (in_dtype < VA_F16 || in_dtype > VA_F32 || out_dtype < VA_F16 || out_dtype > VA_F32)
    return va::fail(VA_EDTYPE, "%s: dtype", what);
  if (layout != VA_LAYOUT_PACKED && layout != VA_LAYOUT_PADDED)
    return va::fail(VA_EINVAL, "%s: layout %d", what, layout);
  if (expand != 0 && expand != 1) return va::fail(VA_EINVAL, "%s: expand %d", what, expand);
  if (layout == VA_LAYOUT_PADDED && (seq <= 0 || !expand))
    return va::fail(VA_EINVAL, "%s: padded layout needs seq > 0 and expand = 1", what);
  if (n_tokens == 0) return VA_OK;
  // The value rows may be left out (both pointers NULL) of a forward that expands nothing: v then
  // needs neither rotation nor expansion, and a caller whose v is already in out_dtype uses it as
  // it is.
  const bool no_v = x2 == nullptr && y2 == nullptr;
  if (no_v && (expand || std::strcmp(what, "va_rope_fwd") != 0))
    return va::fail(VA_EINVAL, "%s: the value rows may only be left out of va_rope_fwd without "
                               "expand", what);
  for (const void* p : {x0, x1, (const void*)cos, (const void*)sin, (const void*)b_idx,
                        (const void*)t_idx, (const void*)y0, (const void*)y1}) {
    if (p == nullptr) return va::fail(VA_EINVAL, "%s: NULL buffer", what);
  }
  if (!no_v && (x2 == nullptr || y2 == nullptr))
    return va::fail(VA_EINVAL, "%s: NULL buffer", what);
  // 16-byte lane accesses: tensor bases and the cos/sin row starts must be 16-byte aligned.
  for (const void* p : {x0, x1, x2, (const void*)cos, (const void*)sin, (const void*)y0,
                        (const void*)y1, (const void*)y2}) {
    if (p != nullptr && !aligned16(p))
      return va::fail(VA_EINVAL, "%s: buffer not 16-byte aligned", what);
  }
  return VA_OK;
}

}  // namespace

extern "C" int va_rope_fwd(const void* q, const void* k, const void* v, const float* cos,
                           const float* sin, int64_t cos_batch_stride, int64_t cos_seq_stride,
                           const int32_t* b_idx, const int32_t* t_idx, void* q_out, void* k_out,
                           void* v_out, int64_t n_tokens, int32_t heads, int32_t kv_heads,
                           int32_t head_dim, int32_t seq, int32_t in_dtype, int32_t out_dtype,
                           int32_t layout, int32_t expand, void* stream) {
  int rc = rope_common(q, k, v, cos, sin, b_idx, t_idx, q_out, k_out, v_out, n_tokens, heads,
                       kv_heads, head_dim, seq, in_dtype, out_dtype, layout, expand,
                       "va_rope_fwd");
  if (rc || n_tokens == 0) return rc;
  if (cos_batch_stride % 4 != 0 || cos_seq_stride % 4 != 0 || cos_batch_stride < 0 ||
      cos_seq_stride < 0)
    return va::fail(VA_EINVAL, "va_rope_fwd: cos/sin strides must be non-negative multiples of 4");
  va::RopeArgs a{q, k, v, cos, sin, cos_batch_stride, cos_seq_stride, b_idx, t_idx,
                 q_out, k_out, v_out, n_tokens, heads, kv_heads, seq, in_dtype, out_dtype,
                 layout, expand, (hipStream_t)stream};
  hipError_t e = va::launch_rope_fwd(a);
  return e == hipSuccess ? VA_OK : hip_fail(e, "va_rope_fwd launch");
}

extern "C" int va_rope_bwd(const void* dq, const void* dk, const void* dv, const float* cos,
                           const float* sin, int64_t cos_batch_stride, int64_t cos_seq_stride,
                           const int32_t* b_idx, const int32_t* t_idx, void* dq_in, void* dk_in,
                           void* dv_in, int64_t n_tokens, int32_t heads, int32_t kv_heads,
                           int32_t head_dim, int32_t seq, int32_t in_dtype, int32_t out_dtype,
                           int32_t layout, int32_t expand, void* stream) {
  int rc = rope_common(dq, dk, dv, cos, sin, b_idx, t_idx, dq_in, dk_in, dv_in, n_tokens, heads,
                       kv_heads, head_dim, seq, in_dtype, out_dtype, layout, expand,
                       "va_rope_bwd");
  if (rc || n_tokens == 0) return rc;
  if (cos_batch_stride % 4 != 0 || cos_seq_stride % 4 != 0 || cos_batch_stride < 0 ||
      cos_seq_stride < 0)
    return va::fail(VA_EINVAL, "va_rope_bwd: cos/sin strides must be non-negative multiples of 4");
  va::RopeArgs a{dq, dk, dv, cos, sin, cos_batch_stride, cos_seq_stride, b_idx, t_idx,
                 dq_in, dk_in, dv_in, n_tokens, heads, kv_heads, seq, in_dtype, out_dtype,
                 layout, expand, (hipStream_t)stream};
  hipError_t e = va::launch_rope_bwd(a);
  return e == hipSuccess ? VA_OK : hip_fail(e, "va_rope_bwd launch");
}

extern "C" int va_pack_rows(const void* src, void* dst, const int32_t* b_idx,
                            const int32_t* t_idx, int64_t n_tokens, int32_t heads, int32_t seq,
                            int32_t head_dim, int32_t elem_bytes, int32_t mode, void* stream) {
  if (mode != 0 && mode != 1) return va::fail(VA_EINVAL, "va_pack_rows: mode %d", mode);
  if (elem_bytes != 2 && elem_bytes != 4) return va::fail(VA_EDTYPE, "va_pack_rows: elem_bytes");
  if (heads <= 0 || seq <= 0 || head_dim <= 0 || n_tokens < 0 || n_tokens > INT32_MAX ||
      heads > 65535)
    return va::fail(VA_ESHAPE, "va_pack_rows: sizes");
  const int64_t row_bytes = (int64_t)head_dim * elem_bytes;
  if (row_bytes % 16 != 0 || row_bytes / 16 > 1024)
    return va::fail(VA_ESHAPE, "va_pack_rows: head_dim * elem_bytes must be a multiple of 16");
  if (n_tokens == 0) return VA_OK;
  int rc = check_ptrs({src, dst, b_idx, t_idx}, "va_pack_rows");
  if (rc) return rc;
  hipError_t e = va::launch_pack_rows(src, dst, b_idx, t_idx, n_tokens, heads, seq,
                                      (int)row_bytes, mode, (hipStream_t)stream);
  return e == hipSuccess ? VA_OK : hip_fail(e, "va_pack_rows launch");
}
