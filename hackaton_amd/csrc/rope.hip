// Rotary embedding and row packing kernels around the attention (memory-bound, one pass each).
//
// rope_fwd_kernel   y = rotate(x) in fp32, rounded once to the output type, for q (heads) and k
//                   (kv heads); v is cast. Output layout packed (N, H, D) or padded (B, H, T, D);
//                   with `expand` K/V are written for every query head (the reference's
//                   qkv_rotate semantics), without it K/V keep their kv heads (what the GQA-native
//                   attention kernels read).
// rope_bwd_kernel   the inverse rotation of dq and dk and the cast of dv, after summing the G
//                   copies of dk/dv when they are expanded; input fp32 accumulators or 16-bit
//                   gradients, output in the projection type.
// pack_rows_kernel  (B, H, T, D) <-> (N, H*D) gather / scatter of whole 16-byte chunks.
#include "va_common.h"
#include "va_kernels.h"

namespace va {

enum { kF16 = 0, kBF16 = 1, kF32 = 2 };

__device__ inline float load_elem(const void* p, long i, int dt) {
  if (dt == kF32) return reinterpret_cast<const float*>(p)[i];
  const uint16_t x = reinterpret_cast<const uint16_t*>(p)[i];
  return dt == kF16 ? F16::to_f32(x) : BF16::to_f32(x);
}
__device__ inline void store_elem(void* p, long i, int dt, float x) {
  if (dt == kF32) {
    reinterpret_cast<float*>(p)[i] = x;
  } else {
    reinterpret_cast<uint16_t*>(p)[i] = dt == kF16 ? F16::from_f32(x) : BF16::from_f32(x);
  }
}

// Output row (in elements of D) of head `head` of token (b, t, pid).
__device__ inline long out_row(int layout, long pid, int b, int t, int heads, int seq, int head) {
  return layout == 0 ? pid * heads + head : ((long)b * heads + head) * seq + t;
}

// grid (N, heads + 2 kv_heads) x 64 threads; thread i handles the pair (i, i + 64).
__global__ __launch_bounds__(64) void rope_fwd_kernel(RopeArgs a) {
  const long pid = blockIdx.x;
  const int slot = blockIdx.y;
  const int i = threadIdx.x;
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const long cb = (long)b * a.cos_batch_stride + (long)t * a.cos_seq_stride;
  const int rep = a.heads / a.kv_heads;
  const int out_heads = (a.expand || slot < a.heads) ? a.heads : a.kv_heads;
  if (slot < a.heads + a.kv_heads) {  // q or k: rotate
    const bool is_q = slot < a.heads;
    const int head = is_q ? slot : slot - a.heads;
    const void* x = is_q ? a.x0 : a.x1;
    const long xrow = pid * (is_q ? a.heads : a.kv_heads) * D + (long)head * D;
    const float x1 = load_elem(x, xrow + i, a.in_dtype);
    const float x2 = load_elem(x, xrow + HALF + i, a.in_dtype);
    const float c1 = a.cos[cb + i], c2 = a.cos[cb + HALF + i];
    const float s1 = a.sin[cb + i], s2 = a.sin[cb + HALF + i];
    const float y1 = x1 * c1 - x2 * s1;
    const float y2 = x2 * c2 + x1 * s2;
    void* y = is_q ? a.y0 : a.y1;
    const int copies = (!is_q && a.expand) ? rep : 1;
    for (int r = 0; r < copies; ++r) {
      const int oh = is_q ? head : (a.expand ? head * rep + r : head);
      const long orow = out_row(a.layout, pid, b, t, out_heads, a.seq, oh) * D;
      store_elem(y, orow + i, a.out_dtype, y1);
      store_elem(y, orow + HALF + i, a.out_dtype, y2);
    }
  } else {  // v: cast (and copy per query head when expanding)
    const int head = slot - a.heads - a.kv_heads;
    const long xrow = pid * a.kv_heads * D + (long)head * D;
    const float v1 = load_elem(a.x2, xrow + i, a.in_dtype);
    const float v2 = load_elem(a.x2, xrow + HALF + i, a.in_dtype);
    const int copies = a.expand ? rep : 1;
    for (int r = 0; r < copies; ++r) {
      const int oh = a.expand ? head * rep + r : head;
      const long orow = out_row(a.layout, pid, b, t, out_heads, a.seq, oh) * D;
      store_elem(a.y2, orow + i, a.out_dtype, v1);
      store_elem(a.y2, orow + HALF + i, a.out_dtype, v2);
    }
  }
}

// grid (N, heads + 2 kv_heads) x 64 threads. Inputs: x0 = dq, x1 = dk, x2 = dv in `layout`, with
// `heads` heads for dq and (expand ? heads : kv_heads) heads for dk/dv. Outputs y0 (N, heads*D),
// y1/y2 (N, kv_heads*D) in out_dtype.
__global__ __launch_bounds__(64) void rope_bwd_kernel(RopeArgs a) {
  const long pid = blockIdx.x;
  const int slot = blockIdx.y;
  const int i = threadIdx.x;
  constexpr int D = kHeadDim, HALF = kHeadDim / 2;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const long cb = (long)b * a.cos_batch_stride + (long)t * a.cos_seq_stride;
  const int rep = a.heads / a.kv_heads;
  const int in_kv_heads = a.expand ? a.heads : a.kv_heads;
  float d1 = 0.f, d2 = 0.f;
  int head;
  const void* x;
  int in_heads;
  int copies;
  if (slot < a.heads) {
    head = slot; x = a.x0; in_heads = a.heads; copies = 1;
  } else if (slot < a.heads + a.kv_heads) {
    head = slot - a.heads; x = a.x1; in_heads = in_kv_heads; copies = a.expand ? rep : 1;
  } else {
    head = slot - a.heads - a.kv_heads; x = a.x2; in_heads = in_kv_heads;
    copies = a.expand ? rep : 1;
  }
  for (int r = 0; r < copies; ++r) {
    const int ih = (slot >= a.heads && a.expand) ? head * rep + r : head;
    const long irow = out_row(a.layout, pid, b, t, in_heads, a.seq, ih) * D;
    d1 += load_elem(x, irow + i, a.in_dtype);
    d2 += load_elem(x, irow + HALF + i, a.in_dtype);
  }
  const bool is_v = slot >= a.heads + a.kv_heads;
  float o1 = d1, o2 = d2;
  if (!is_v) {
    const float c1 = a.cos[cb + i], c2 = a.cos[cb + HALF + i];
    const float s1 = a.sin[cb + i], s2 = a.sin[cb + HALF + i];
    o1 = d1 * c1 + d2 * s2;
    o2 = d2 * c2 - d1 * s1;
  }
  void* y = slot < a.heads ? a.y0 : (is_v ? a.y2 : a.y1);
  const int out_heads = slot < a.heads ? a.heads : a.kv_heads;
  const long orow = (pid * out_heads + head) * D;
  store_elem(y, orow + i, a.out_dtype, o1);
  store_elem(y, orow + HALF + i, a.out_dtype, o2);
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

hipError_t launch_rope_fwd(const RopeArgs& a) {
  if (a.n_tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_fwd_kernel, dim3((unsigned)a.n_tokens, a.heads + 2 * a.kv_heads),
                     dim3(64), 0, a.stream, a);
  return hipGetLastError();
}

hipError_t launch_rope_bwd(const RopeArgs& a) {
  if (a.n_tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_bwd_kernel, dim3((unsigned)a.n_tokens, a.heads + 2 * a.kv_heads),
                     dim3(64), 0, a.stream, a);
  return hipGetLastError();
}

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
