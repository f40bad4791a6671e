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
// Access pattern: one wave per token. A (token, head) row of D = 128 elements is handled by 8
// consecutive lanes; lane j of the row takes elements [8j, 8j + 8) of the first half and the
// matching 8 of the second half, so every 16-bit load or store is one 16-byte access per lane
// (fp32 data: two), and the 8 lanes of a row cover its 256 bytes (16-bit) in two contiguous
// 128-byte runs. The wave's 8 lane groups take 16 heads of the token per pass; the token's
// position is read once per wave and its cos / sin chunks once per pass, not once per head. The
// element types
// are template parameters (no run-time branch per element).
#include <type_traits>

#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace {

enum { kF16 = 0, kBF16 = 1, kF32 = 2 };
constexpr int D = kHeadDim, HALF = kHeadDim / 2;
constexpr int kRopeThreads = 256;
constexpr int kTokensPerGroup = kRopeThreads / 64;  // one wave per token

// Device-memory (global address space) pointers: accesses through them are global loads and stores.
#define VA_GLOBAL __attribute__((address_space(1)))
using gcvoid = const VA_GLOBAL void*;
using gvoid = VA_GLOBAL void*;

// 8 elements of a row as loaded: one 16-byte vector for 16-bit types, two for fp32. Loads are kept
// raw and converted at the point of use, so a load issued under a branch needs no wait there.
template <int DT>
struct Raw8 {
  u32x4 w[DT == kF32 ? 2 : 1];
};

template <int DT>
__device__ inline Raw8<DT> load_raw8(gcvoid base, long elem) {
  Raw8<DT> r;
  const VA_GLOBAL u32x4* p = reinterpret_cast<const VA_GLOBAL u32x4*>(
      reinterpret_cast<const VA_GLOBAL uint8_t*>(base) + elem * (DT == kF32 ? 4 : 2));
#pragma unroll
  for (int i = 0; i < (DT == kF32 ? 2 : 1); ++i) r.w[i] = p[i];
  return r;
}

template <int DT>
__device__ inline void cvt8(const Raw8<DT>& r, float (&x)[8]) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // Element copied out first: a bit cast applied to a vector-element lvalue reads element 0.
      const uint32_t u = r.w[e / 4][e % 4];
      x[e] = __builtin_bit_cast(float, u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      x[e] = DT == kF16 ? F16::to_f32(half_of(r.w[0], e)) : BF16::to_f32(half_of(r.w[0], e));
  }
}

template <int DT>
__device__ inline void store8(gvoid base, long elem, const float (&x)[8]) {
  if constexpr (DT == kF32) {
    VA_GLOBAL f32x4* p =
        reinterpret_cast<VA_GLOBAL f32x4*>(reinterpret_cast<VA_GLOBAL float*>(base) + elem);
    p[0] = f32x4{x[0], x[1], x[2], x[3]};
    p[1] = f32x4{x[4], x[5], x[6], x[7]};
  } else {
    using E = std::conditional_t<DT == kF16, F16, BF16>;
    *reinterpret_cast<VA_GLOBAL u32x4*>(reinterpret_cast<VA_GLOBAL uint16_t*>(base) + elem) =
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

// One wave per token: lane j = lane & 7 takes elements [8j, 8j + 8) of both halves of a row, and
// the wave's 8 lane groups take rows (heads) r, r + 8, ... of the token. The token's position, and
// its cos / sin chunks, are read once per wave and kept for all of its heads.
struct TokenLanes {
  long pid;
  int j, r0;
  bool valid;
};
__device__ inline TokenLanes token_lanes(long n_tokens) {
  TokenLanes tl;
  tl.pid = (long)blockIdx.x * kTokensPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  tl.j = threadIdx.x & 7;
  tl.r0 = (threadIdx.x & 63) >> 3;
  tl.valid = tl.pid < n_tokens;
  return tl;
}

// Kernel-argument values chosen per lane are laundered through an empty asm first, so that the
// compiler cannot turn the choice of value into a choice of argument address, which would copy the
// whole argument block to scratch memory.
template <typename T>
__device__ inline T uniform(T v) {
  asm("" : "+s"(v));  // not volatile: free to be hoisted and shared, so choices stay selects
  return v;
}
// Kernel-argument pointers are device memory: cast to the global address space first and laundered
// after, so that a per-lane choice among them is a choice of global pointers.
__device__ inline gcvoid pick3(bool first, bool last, const void* p0, const void* p1,
                               const void* p2) {
  gcvoid g0 = uniform((gcvoid)p0), g1 = uniform((gcvoid)p1), g2 = uniform((gcvoid)p2);
  return first ? g0 : (last ? g2 : g1);
}
__device__ inline gvoid pick3(bool first, bool last, void* p0, void* p1, void* p2) {
  gvoid g0 = uniform((gvoid)p0), g1 = uniform((gvoid)p1), g2 = uniform((gvoid)p2);
  return first ? g0 : (last ? g2 : g1);
}

struct Tables {
  float cs1[8], cs2[8], sn1[8], sn2[8];
};
__device__ inline void load_tables(const RopeArgs& a, int b, int t, int c0, Tables& tb) {
  const long cb = (long)b * a.cos_batch_stride + (long)t * a.cos_seq_stride;
  load_table8(a.cos, cb + c0, tb.cs1);
  load_table8(a.cos, cb + HALF + c0, tb.cs2);
  load_table8(a.sin, cb + c0, tb.sn1);
  load_table8(a.sin, cb + HALF + c0, tb.sn2);
}

// Rows of a token: its q heads (slots [0, heads)), then k heads, then v heads.
struct Slot {
  bool is_q, is_v;
  int head;
};
__device__ inline Slot slot_of(const RopeArgs& a, int slot) {
  Slot r;
  r.is_q = slot < a.heads;
  r.is_v = slot >= a.heads + a.kv_heads;
  r.head = r.is_q ? slot : (r.is_v ? slot - a.heads - a.kv_heads : slot - a.heads);
  return r;
}

// Forward: both halves of a row of q (N, heads, D), k or v (N, kv_heads, D).
template <int IN>
struct RowIn {
  Raw8<IN> h1, h2;
};
template <int IN>
__device__ inline RowIn<IN> fwd_load(const RopeArgs& a, long pid, int c0, int slot) {
  const Slot sl = slot_of(a, slot);
  const gcvoid x = pick3(sl.is_q, sl.is_v, a.x0, a.x1, a.x2);
  const long xrow = (pid * (sl.is_q ? uniform(a.heads) : uniform(a.kv_heads)) + sl.head) * D;
  return RowIn<IN>{load_raw8<IN>(x, xrow + c0), load_raw8<IN>(x, xrow + HALF + c0)};
}

// q and k rows are rotated in fp32, v rows cast; k / v rows are stored once per query head of the
// group when expanding.
template <int IN, int OUT>
__device__ inline void fwd_store(const RopeArgs& a, long pid, int b, int t, int c0, int slot,
                                 const Tables& tb, const RowIn<IN>& in) {
  const Slot sl = slot_of(a, slot);
  const int rep = a.heads / a.kv_heads;
  const int out_heads = (a.expand || sl.is_q) ? uniform(a.heads) : uniform(a.kv_heads);
  const int copies = (!sl.is_q && a.expand) ? rep : 1;
  const gvoid y = pick3(sl.is_q, sl.is_v, a.y0, a.y1, a.y2);
  float x1[8], x2[8], y1[8], y2[8];
  cvt8<IN>(in.h1, x1);
  cvt8<IN>(in.h2, x2);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r1, r2;
    rope_rotate(x1[e], x2[e], tb.cs1[e], tb.cs2[e], tb.sn1[e], tb.sn2[e], r1, r2);
    y1[e] = sl.is_v ? x1[e] : r1;
    y2[e] = sl.is_v ? x2[e] : r2;
  }
  for (int r = 0; r < copies; ++r) {
    const int oh = (!sl.is_q && a.expand) ? sl.head * rep + r : sl.head;
    const long orow = out_row(a.layout, pid, b, t, out_heads, a.seq, oh) * D;
    store8<OUT>(y, orow + c0, y1);
    store8<OUT>(y, orow + HALF + c0, y2);
  }
}

// Each lane group handles two rows per pass: both rows, then the token's cos / sin chunks, are
// loaded before either row is stored, so a wave has the reads of 16 rows in flight (all 16 rows
// of a 12 + 2 + 2 head token in one pass). The tables are read again per pass, from cache.
template <int IN, int OUT>
__global__ __launch_bounds__(kRopeThreads) void rope_fwd_kernel(RopeArgs a) {
  const TokenLanes tl = token_lanes(a.n_tokens);
  if (!tl.valid) return;
  const long pid = tl.pid;
  const int c0 = 8 * tl.j;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const int slots = a.heads + (a.x2 != nullptr ? 2 : 1) * a.kv_heads;  // no value rows: x2 null
  for (int s0 = tl.r0; s0 < slots; s0 += 16) {
    const int s1 = s0 + 8;
    const RowIn<IN> u = fwd_load<IN>(a, pid, c0, s0);
    RowIn<IN> w;
    if (s1 < slots) w = fwd_load<IN>(a, pid, c0, s1);
    Tables tb;
    load_tables(a, b, t, c0, tb);
    fwd_store<IN, OUT>(a, pid, b, t, c0, s0, tb, u);
    if (s1 < slots) fwd_store<IN, OUT>(a, pid, b, t, c0, s1, tb, w);
  }
}

// Backward, inputs: x0 = dq, x1 = dk, x2 = dv in `layout`, with `heads` heads for dq and
// (expand ? heads : kv_heads) heads for dk/dv. Outputs y0 (N, heads*D), y1/y2 (N, kv_heads*D).
// Row `slot`'s gradient (its first copy when expanded).
template <int IN>
__device__ inline RowIn<IN> bwd_load(const RopeArgs& a, long pid, int b, int t, int c0, int slot,
                                     int copy) {
  const Slot sl = slot_of(a, slot);
  const int in_heads = sl.is_q ? uniform(a.heads) : uniform(a.expand ? a.heads : a.kv_heads);
  const int ih = (!sl.is_q && a.expand) ? sl.head * (a.heads / a.kv_heads) + copy : sl.head;
  const gcvoid x = pick3(sl.is_q, sl.is_v, a.x0, a.x1, a.x2);
  const long irow = out_row(a.layout, pid, b, t, in_heads, a.seq, ih) * D;
  return RowIn<IN>{load_raw8<IN>(x, irow + c0), load_raw8<IN>(x, irow + HALF + c0)};
}

// The G copies of a key/value head summed in fp32 when expanded, then the inverse rotation of dq
// and dk rows, the cast of dv rows.
template <int IN, int OUT>
__device__ inline void bwd_store(const RopeArgs& a, long pid, int b, int t, int c0, int slot,
                                 const Tables& tb, const RowIn<IN>& in) {
  const Slot sl = slot_of(a, slot);
  float d1[8], d2[8];
  cvt8<IN>(in.h1, d1);
  cvt8<IN>(in.h2, d2);
  const int copies = (!sl.is_q && a.expand) ? a.heads / a.kv_heads : 1;
  // The other copies in batches of 7, every load of a batch issued before its first add: one
  // memory round trip per batch instead of one per copy.
  constexpr int kBatch = 7;
  for (int r0 = 1; r0 < copies; r0 += kBatch) {
    RowIn<IN> more[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (r0 + i < copies) more[i] = bwd_load<IN>(a, pid, b, t, c0, slot, r0 + i);
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (r0 + i < copies) {
        float u1[8], u2[8];
        cvt8<IN>(more[i].h1, u1);
        cvt8<IN>(more[i].h2, u2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          d1[e] += u1[e];
          d2[e] += u2[e];
        }
      }
  }
  float o1[8], o2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r1, r2;
    rope_unrotate(d1[e], d2[e], tb.cs1[e], tb.cs2[e], tb.sn1[e], tb.sn2[e], r1, r2);
    o1[e] = sl.is_v ? d1[e] : r1;
    o2[e] = sl.is_v ? d2[e] : r2;
  }
  const gvoid y = pick3(sl.is_q, sl.is_v, a.y0, a.y1, a.y2);
  const long orow = (pid * (sl.is_q ? uniform(a.heads) : uniform(a.kv_heads)) + sl.head) * D;
  store8<OUT>(y, orow + c0, o1);
  store8<OUT>(y, orow + HALF + c0, o2);
}

template <int IN, int OUT>
__global__ __launch_bounds__(kRopeThreads) void rope_bwd_kernel(RopeArgs a) {
  const TokenLanes tl = token_lanes(a.n_tokens);
  if (!tl.valid) return;
  const long pid = tl.pid;
  const int c0 = 8 * tl.j;
  const int b = a.b_idx[pid], t = a.t_idx[pid];
  const int slots = a.heads + 2 * a.kv_heads;
  for (int s0 = tl.r0; s0 < slots; s0 += 16) {
    const int s1 = s0 + 8;
    const RowIn<IN> u = bwd_load<IN>(a, pid, b, t, c0, s0, 0);
    RowIn<IN> w;
    if (s1 < slots) w = bwd_load<IN>(a, pid, b, t, c0, s1, 0);
    Tables tb;
    load_tables(a, b, t, c0, tb);
    bwd_store<IN, OUT>(a, pid, b, t, c0, s0, tb, u);
    if (s1 < slots) bwd_store<IN, OUT>(a, pid, b, t, c0, s1, tb, w);
  }
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
  const unsigned groups = (unsigned)((a.n_tokens + kTokensPerGroup - 1) / kTokensPerGroup);
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
