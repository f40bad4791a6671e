// Rotary embedding and row packing kernels around the attention (memory-bound, one pass each).
//
// rope_fwd_kernel   y = rotate(x) in fp32, rounded once to the output type, for q (heads) and k
//                   (kv heads); v is cast. Output layout packed (N, H, D) or padded (B, H, T, D);
//                   with `expand` K/V are written for every query head (the reference's
//                   qkv_rotate semantics), without it K/V keep their kv heads (what the GQA-native
//                   attention kernels read).
// rope_bwd_kernel   the inverse rotation of dq and dk and the cast of dv, after summing the G
//                   copies (or per-head partials) of dk/dv in fp32 when they are per query head;
//                   output in the projection type.
// pack_rows_kernel  (B, H, T, D) <-> (N, H*D) gather / scatter of whole 16-byte chunks.
//
// Access pattern: a (token, head) row of D = 128 elements is handled by 8 consecutive lanes; lane
// j of the row takes elements [8j, 8j + 8) of the first half and the matching 8 of the second
// half, so every 16-bit load or store is one 16-byte access per lane (fp32 data: two), and the 8
// lanes of a row cover its 256 bytes (16-bit) in two contiguous 128-byte runs. A work-group of
// 256 threads covers 32 rows. The element types are template parameters (no run-time branch per
// element).
#include <type_traits>

#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace {

enum { kF16 = 0, kBF16 = 1, kF32 = 2 };
constexpr int D = kHeadDim, HALF = kHeadDim / 2;
constexpr int kLanesPerRow = HALF / 8;    // 8 lanes x 8 pairs
constexpr int kRopeThreads = 256;
constexpr int kRowsPerGroup = kRopeThreads / kLanesPerRow;

template <int DT>
__device__ inline void load8(const void* base, long elem, float (&x)[8]) {
  if constexpr (DT == kF32) {
    const f32x4* p = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + elem);
    const f32x4 a = p[0], b = p[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + elem);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      x[e] = DT == kF16 ? F16::to_f32(half_of(w, e)) : BF16::to_f32(half_of(w, e));
  }
}

template <int DT>
__device__ inline void store8(void* base, long elem, const float (&x)[8]) {
  if constexpr (DT == kF32) {
    f32x4* p = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + elem);
    p[0] = f32x4{x[0], x[1], x[2], x[3]};
    p[1] = f32x4{x[4], x[5], x[6], x[7]};
  } else {
    using E = std::conditional_t<DT == kF16, F16, BF16>;
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(base) + elem) =
        pack8<E>(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
  }
}

__device__ inline void load_table8(const float* t, long elem, float (&x)[8]) {
  const f32x4* p = reinterpret_cast<const f32x4*>(t + elem);
  const f32x4 a = p[0], b = p[1];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = a[e];
    x[4 + e] = b[e];
  }
}

// Row (in elements of D) of head `head` of token (b, t, pid) in the packed or padded layout.
__device__ inline long out_row(int layout, long pid, int b, int t, int heads, int seq, int head) {
  return layout == 0 ? pid * heads + head : ((long)b * heads + head) * seq + t;
}

struct RowLane {
  long pid;
  int slot, j;
  bool valid;
};
__device__ inline RowLane row_lane(long n_tokens, int slots) {
  const long row = (long)blockIdx.x * kRowsPerGroup + threadIdx.x / kLanesPerRow;
  RowLane r;
  r.pid = row / slots;
  r.slot = (int)(row - r.pid * slots);
  r.j = threadIdx.x % kLanesPerRow;
  r.valid = r.pid < n_tokens;
  return r;
}

// Rows: every token's q heads, then k heads, then v heads.
template <int IN, int OUT>
__global__ __launch_bounds__(kRopeThreads) void rope_fwd_kernel(RopeArgs a) {
  const int slots = a.heads + 2 * a.kv_heads;
  const RowLane rl = row_lane(a.n_tokens, slots);
  if (!rl.valid) return;
  const long pid = rl.pid;
  const int slot = rl.slot, c0 = 8 * rl.j;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const int rep = a.heads / a.kv_heads;
  const int out_heads = (a.expand || slot < a.heads) ? a.heads : a.kv_heads;
  float y1[8], y2[8];
  int head, copies;
  void* y;
  if (slot < a.heads + a.kv_heads) {  // q or k: rotate in fp32
    const bool is_q = slot < a.heads;
    head = is_q ? slot : slot - a.heads;
    const void* x = is_q ? a.x0 : a.x1;
    const long xrow = (pid * (is_q ? a.heads : a.kv_heads) + head) * D;
    float x1[8], x2[8], cs1[8], cs2[8], sn1[8], sn2[8];
    load8<IN>(x, xrow + c0, x1);
    load8<IN>(x, xrow + HALF + c0, x2);
    const long cb = (long)b * a.cos_batch_stride + (long)t * a.cos_seq_stride;
    load_table8(a.cos, cb + c0, cs1);
    load_table8(a.cos, cb + HALF + c0, cs2);
    load_table8(a.sin, cb + c0, sn1);
    load_table8(a.sin, cb + HALF + c0, sn2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y1[e] = x1[e] * cs1[e] - x2[e] * sn1[e];
      y2[e] = x2[e] * cs2[e] + x1[e] * sn2[e];
    }
    y = is_q ? a.y0 : a.y1;
    copies = (!is_q && a.expand) ? rep : 1;
    if (is_q) {
      const long orow = out_row(a.layout, pid, b, t, out_heads, a.seq, head) * D;
      store8<OUT>(y, orow + c0, y1);
      store8<OUT>(y, orow + HALF + c0, y2);
      return;
    }
  } else {  // v: cast
    head = slot - a.heads - a.kv_heads;
    const long xrow = (pid * a.kv_heads + head) * D;
    load8<IN>(a.x2, xrow + c0, y1);
    load8<IN>(a.x2, xrow + HALF + c0, y2);
    y = a.y2;
    copies = a.expand ? rep : 1;
  }
  for (int r = 0; r < copies; ++r) {  // k / v: once per query head of the group when expanding
    const int oh = a.expand ? head * rep + r : head;
    const long orow = out_row(a.layout, pid, b, t, out_heads, a.seq, oh) * D;
    store8<OUT>(y, orow + c0, y1);
    store8<OUT>(y, orow + HALF + c0, y2);
  }
}

// Inputs: x0 = dq, x1 = dk, x2 = dv in `layout`, with `heads` heads for dq and
// (expand ? heads : kv_heads) heads for dk/dv. Outputs y0 (N, heads*D), y1/y2 (N, kv_heads*D).
template <int IN, int OUT>
__global__ __launch_bounds__(kRopeThreads) void rope_bwd_kernel(RopeArgs a) {
  const int slots = a.heads + 2 * a.kv_heads;
  const RowLane rl = row_lane(a.n_tokens, slots);
  if (!rl.valid) return;
  const long pid = rl.pid;
  const int slot = rl.slot, c0 = 8 * rl.j;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const int rep = a.heads / a.kv_heads;
  const int in_kv_heads = a.expand ? a.heads : a.kv_heads;
  int head, in_heads, copies;
  const void* x;
  if (slot < a.heads) {
    head = slot; x = a.x0; in_heads = a.heads; copies = 1;
  } else if (slot < a.heads + a.kv_heads) {
    head = slot - a.heads; x = a.x1; in_heads = in_kv_heads; copies = a.expand ? rep : 1;
  } else {
    head = slot - a.heads - a.kv_heads; x = a.x2; in_heads = in_kv_heads;
    copies = a.expand ? rep : 1;
  }
  float d1[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float d2[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < copies; ++r) {  // the G copies of a key/value head, summed in fp32
    const int ih = (slot >= a.heads && a.expand) ? head * rep + r : head;
    const long irow = out_row(a.layout, pid, b, t, in_heads, a.seq, ih) * D;
    float u1[8], u2[8];
    load8<IN>(x, irow + c0, u1);
    load8<IN>(x, irow + HALF + c0, u2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      d1[e] += u1[e];
      d2[e] += u2[e];
    }
  }
  const bool is_v = slot >= a.heads + a.kv_heads;
  float o1[8], o2[8];
  if (!is_v) {  // inverse rotation
    float cs1[8], cs2[8], sn1[8], sn2[8];
    const long cb = (long)b * a.cos_batch_stride + (long)t * a.cos_seq_stride;
    load_table8(a.cos, cb + c0, cs1);
    load_table8(a.cos, cb + HALF + c0, cs2);
    load_table8(a.sin, cb + c0, sn1);
    load_table8(a.sin, cb + HALF + c0, sn2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = d1[e] * cs1[e] + d2[e] * sn2[e];
      o2[e] = d2[e] * cs2[e] - d1[e] * sn1[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = d1[e];
      o2[e] = d2[e];
    }
  }
  void* y = slot < a.heads ? a.y0 : (is_v ? a.y2 : a.y1);
  const int out_heads = slot < a.heads ? a.heads : a.kv_heads;
  const long orow = (pid * out_heads + head) * D;
  store8<OUT>(y, orow + c0, o1);
  store8<OUT>(y, orow + HALF + c0, o2);
}

// grid (N, heads) x (row_chunks) threads; 16-byte chunks of one (token, head) row.
__global__ void pack_rows_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                 const int32_t* __restrict__ b_idx,
                                 const int32_t* __restrict__ t_idx, int heads, int seq,
                                 int row_chunks, int mode) {
  const long pid = blockIdx.x;
  const int head = blockIdx.y;
  const int c = threadIdx.x;
  if (c >= row_chunks) return;
  const long padded = (((long)b_idx[pid] * heads + head) * seq + t_idx[pid]) * row_chunks + c;
  const long packed = (pid * heads + head) * row_chunks + c;
  if (mode == 0) dst[packed] = src[padded];
  else dst[padded] = src[packed];
}

template <int IN, int OUT>
hipError_t launch_rope_t(const RopeArgs& a, bool fwd) {
  const long rows = a.n_tokens * (long)(a.heads + 2 * a.kv_heads);
  const unsigned groups = (unsigned)((rows + kRowsPerGroup - 1) / kRowsPerGroup);
  if (fwd) {
    hipLaunchKernelGGL((rope_fwd_kernel<IN, OUT>), dim3(groups), dim3(kRopeThreads), 0, a.stream,
                       a);
  } else {
    hipLaunchKernelGGL((rope_bwd_kernel<IN, OUT>), dim3(groups), dim3(kRopeThreads), 0, a.stream,
                       a);
  }
  return hipGetLastError();
}

template <int IN>
hipError_t launch_rope_out(const RopeArgs& a, bool fwd) {
  switch (a.out_dtype) {
    case kF16: return launch_rope_t<IN, kF16>(a, fwd);
    case kBF16: return launch_rope_t<IN, kBF16>(a, fwd);
    default: return launch_rope_t<IN, kF32>(a, fwd);
  }
}

hipError_t launch_rope(const RopeArgs& a, bool fwd) {
  if (a.n_tokens == 0) return hipSuccess;
  switch (a.in_dtype) {
    case kF16: return launch_rope_out<kF16>(a, fwd);
    case kBF16: return launch_rope_out<kBF16>(a, fwd);
    default: return launch_rope_out<kF32>(a, fwd);
  }
}

}  // namespace

hipError_t launch_rope_fwd(const RopeArgs& a) { return launch_rope(a, true); }
hipError_t launch_rope_bwd(const RopeArgs& a) { return launch_rope(a, false); }

hipError_t launch_pack_rows(const void* src, void* dst, const int32_t* b_idx, const int32_t* t_idx,
                            int64_t n_tokens, int heads, int seq, int row_bytes, int mode,
                            hipStream_t stream) {
  if (n_tokens == 0) return hipSuccess;
  const int chunks = row_bytes / 16;
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)n_tokens, heads), dim3(chunks), 0, stream,
                     (const u32x4*)src, (u32x4*)dst, b_idx, t_idx, heads, seq, chunks, mode);
  return hipGetLastError();
}

}  // namespace va
