// Backward kernels of packed varlen causal GQA attention for gfx950.
//
//  bwd_pre_kernel    delta[h][t] = sum_d dO * O (fp32) and clears the fp32 dQ/dK/dV accumulators.
//  bwd_kernel        one work-group = NW waves x 32 keys of one document (a key tile) and a run of
//                    query heads of one GQA group. K and V of the wave's keys stay in registers;
//                    for every 32-query step from the key tile's first key to the document end it
//                    stages Q and dO (row-major and transposed) in LDS, recomputes
//                    P = exp2(S scale log2e - lse log2e), and accumulates dV += P^T dO and
//                    dK += dS^T Q in registers (dS = P (dP - delta), dP = dO V^T). dS goes through
//                    LDS so the work-group computes dQ = dS K for its keys, added to the fp32 dQ
//                    accumulator with global atomics. dK/dV are added once per work item to fp32
//                    accumulators, which sums the query heads of a GQA group.
//  bwd_post_kernel   casts the fp32 accumulators to the element type.
#include "va_common.h"
#include "va_kernels.h"

namespace va {

// ---------------------------------------------------------------------------------------------
// delta + accumulator clear: 16 lanes per (token, head) row, 8 elements per lane.
// ---------------------------------------------------------------------------------------------
template <class E>
__global__ __launch_bounds__(256) void bwd_pre_kernel(
    const uint16_t* __restrict__ o, const uint16_t* __restrict__ dout, float* __restrict__ delta,
    float* __restrict__ dq_acc, float* __restrict__ dk_acc, float* __restrict__ dv_acc,
    int n_tokens, int hq, int hkv) {
  const long row = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const long rows = (long)n_tokens * hq;
  float acc = 0.f;
  if (row < rows) {
    const long t = row / hq;
    const int h = (int)(row - t * hq);
    const u32x4 a = gload16(o + row * kHeadDim + 8 * sub);
    const u32x4 b = gload16(dout + row * kHeadDim + 8 * sub);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += E::to_f32(half_of(a, e)) * E::to_f32(half_of(b, e));
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4* dq4 = reinterpret_cast<f32x4*>(dq_acc + row * kHeadDim + 8 * sub);
    dq4[0] = z;
    dq4[1] = z;
    if (h < hkv) {
      const long kr = t * hkv + h;
      f32x4* dk4 = reinterpret_cast<f32x4*>(dk_acc + kr * kHeadDim + 8 * sub);
      f32x4* dv4 = reinterpret_cast<f32x4*>(dv_acc + kr * kHeadDim + 8 * sub);
      dk4[0] = z;
      dk4[1] = z;
      dv4[0] = z;
      dv4[1] = z;
    }
  }
  acc += __shfl_xor(acc, 8, 16);
  acc += __shfl_xor(acc, 4, 16);
  acc += __shfl_xor(acc, 2, 16);
  acc += __shfl_xor(acc, 1, 16);
  if (row < rows && sub == 0) {
    const long t = row / hq;
    const int h = (int)(row - t * hq);
    delta[(long)h * n_tokens + t] = acc;
  }
}

// ---------------------------------------------------------------------------------------------
// Main backward kernel.
// ---------------------------------------------------------------------------------------------
namespace bwd {
constexpr int NW = kBwdWaves;   // waves, 32 keys each
constexpr int BN = 32 * NW;     // keys per work item
constexpr int BQ = kBwdBlockQ;  // queries per step
constexpr int D = kHeadDim;
constexpr int LD = D + 8;       // row stride (halfs) of the Q, dO and K tiles
constexpr int LDT = BQ + 16;    // row stride (halfs) of the dS^T tile (rows = keys)
constexpr int NT = NW * 64;
constexpr int QTILE = BQ * LD;
// LDS map (halfs): Q[2 stages], dO[2 stages], K, dS^T; then lse2/delta floats [2 stages][BQ].
constexpr int OFF_Q = 0;
constexpr int OFF_DO = OFF_Q + 2 * QTILE;
constexpr int OFF_K = OFF_DO + 2 * QTILE;
constexpr int OFF_DST = OFF_K + BN * LD;
constexpr int HALFS = OFF_DST + BN * LDT;
constexpr int STAGE_CHUNKS = 2 * BQ * 16;        // Q and dO 16-byte chunks per step
constexpr int SPT = STAGE_CHUNKS / NT;            // per thread
static_assert(SPT * NT == STAGE_CHUNKS, "staging split");
}  // namespace bwd

template <class E>
__global__ __launch_bounds__(bwd::NT, 1) void bwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, float* __restrict__ dq_acc,
    float* __restrict__ dk_acc, float* __restrict__ dv_acc, const int4* __restrict__ items,
    int n_tokens, int hq, int hkv, float scale, float scale_log2) {
  using namespace bwd;
  __shared__ __attribute__((aligned(16))) uint16_t smem_raw[HALFS];
  __shared__ __attribute__((aligned(16))) float stat_raw[2][2][BQ];  // [stage][lse2 | delta][row]
  lds_u16* smem = (lds_u16*)smem_raw;

  const int4 it = items[blockIdx.x];
  const int k0 = it.x, doc_end = it.y, h_begin = it.z, h_count = it.w;
  const int group = hq / hkv;
  const int kvh = h_begin / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int src = lane & 15, grp = lane >> 4;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;

  const int kw0 = k0 + 32 * wave;   // first key of this wave
  const int my_key = kw0 + l32;

  // K and V of this lane's key as MFMA B operands (column = key, k slots = d), rows clamped.
  u32x4 kf[8], vf[8];
  {
    const long row = min(my_key, doc_end - 1);
    const uint16_t* kp = k + row * kvrow + kvh * D + 8 * hi;
    const uint16_t* vp = v + row * kvrow + kvh * D + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      kf[kk] = gload16(kp + 16 * kk);
      vf[kk] = gload16(vp + 16 * kk);
    }
  }
  // The key tile, row-major, in LDS (B operand of dQ = dS K through transposed reads).
  {
    const int srow = tid >> 4, scol = 8 * (tid & 15);
#pragma unroll
    for (int i = 0; i < BN / 16; ++i) {
      const long row = min(k0 + srow + 16 * i, doc_end - 1);
      st128(smem + OFF_K + (srow + 16 * i) * LD + scol,
            gload16(k + row * kvrow + kvh * D + scol));
    }
  }

  // Staging of one query step (Q and dO rows, lse * log2e and delta) through registers.
  const int s_tensor = tid / (NT / 2);              // threads [0, NT/2): Q, the rest: dO
  const int s_unit = tid % (NT / 2);
  const int s_row = s_unit >> 4, s_col = 8 * (s_unit & 15);
  constexpr int SROWS = (NT / 2) / 16;              // rows covered per staging pass
  u32x4 sreg[SPT];
  float st_lse = 0.f, st_del = 0.f;
  auto gload_step = [&](int h, int qs0) {
    const uint16_t* base = (s_tensor ? dout : q) + h * D + s_col;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const long row = min(qs0 + s_row + SROWS * i, doc_end - 1);
      sreg[i] = gload16(base + row * qrow);
    }
    if (tid < BQ) {
      const int row = qs0 + tid;
      const bool ok = row < doc_end;
      st_lse = ok ? lse[(long)h * n_tokens + row] * kLog2e : INFINITY;
      st_del = ok ? delta[(long)h * n_tokens + row] : 0.f;
    }
  };
  auto store_step = [&](int stage) {
    lds_u16* base = smem + (s_tensor ? OFF_DO : OFF_Q) + stage * QTILE + s_row * LD + s_col;
#pragma unroll
    for (int i = 0; i < SPT; ++i) st128(base + SROWS * i * LD, sreg[i]);
    if (tid < BQ) {
      stat_raw[stage][0][tid] = st_lse;
      stat_raw[stage][1][tid] = st_del;
    }
  };

  // Per-lane LDS read bases (halfs).
  const int rm_read = perm32(l32) * LD + 8 * hi;                              // rows = queries
  const int tr_read = (8 * hi + 2 * (src >> 2)) * LD + 16 * (grp & 1) + 4 * (src & 3);
  const int dst_read = OFF_DST + (8 * hi + 2 * (src >> 2)) * LDT + 16 * (grp & 1) + 4 * (src & 3);
  const int dst_write = OFF_DST + (32 * wave + l32) * LDT + 8 * hi;

  f32x16 dkacc[4], dvacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  // The (head, query step) sequence of this work item.
  const int steps_per_head = (doc_end - k0 + BQ - 1) / BQ;
  const int n_steps = steps_per_head * h_count;
  auto step_head = [&](int s) { return h_begin + s / steps_per_head; };
  auto step_q0 = [&](int s) { return k0 + (s % steps_per_head) * BQ; };

  gload_step(step_head(0), step_q0(0));
  store_step(0);
  if (n_steps > 1) gload_step(step_head(1), step_q0(1));
  __syncthreads();

  for (int s = 0; s < n_steps; ++s) {
    const int stage = s & 1;
    const int h = step_head(s), qs0 = step_q0(s);
    const lds_u16* qs = smem + OFF_Q + stage * QTILE;
    const lds_u16* dos = smem + OFF_DO + stage * QTILE;

    // S = Q K^T and dP = dO V^T (rows = queries, columns = this wave's keys).
    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      sacc = E::mfma(ld128(qs + rm_read + 16 * kk), kf[kk], sacc);
      pacc = E::mfma(ld128(dos + rm_read + 16 * kk), vf[kk], pacc);
    }
    // register j <-> query qs0 + reg_row(j, hi) = qs0 + 16 (j >> 3) + 8 hi + (j & 7).
    float p[16], ds[16];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int r0 = 16 * c + 8 * hi;
      const lds_f32x4* st = reinterpret_cast<const lds_f32x4*>(
          (__attribute__((address_space(3))) float*)&stat_raw[stage][0][0]);
      const f32x4 l0 = st[r0 / 4], l1 = st[r0 / 4 + 1];
      const f32x4 d0 = st[(BQ + r0) / 4], d1 = st[(BQ + r0) / 4 + 1];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 8 * c + e;
        const float lv = e < 4 ? l0[e] : l1[e - 4];
        p[j] = fast_exp2(fmaf(sacc[j], scale_log2, -lv));
        ds[j] = e < 4 ? d0[e] : d1[e - 4];
      }
    }
    if (kw0 + 31 > qs0) {  // the step crosses this wave's diagonal: key > query -> P = 0
      const int lim = my_key - qs0;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (reg_row(j, hi) < lim) p[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) ds[j] = p[j] * (pacc[j] - ds[j]);

    // dV += P^T dO and dK += dS^T Q: A = this lane's key row (k = queries), B via tr reads.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4 pa = pack8_tr<E>(p + 8 * c);
      const u32x4 da = pack8_tr<E>(ds + 8 * c);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int off = tr_read + 16 * c * LD + 32 * db;
        dvacc[db] = E::mfma(pa, ldtr8(dos + off, LD), dvacc[db]);
        dkacc[db] = E::mfma(da, ldtr8(qs + off, LD), dkacc[db]);
      }
    }
    // dS^T rows (this lane's key), queries in natural order.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int j0 = 8 * c;
      st128(smem + dst_write + 16 * c,
            pack8<E>(ds[j0], ds[j0 + 1], ds[j0 + 2], ds[j0 + 3], ds[j0 + 4], ds[j0 + 5],
                     ds[j0 + 6], ds[j0 + 7]));
    }
    // Next step's Q/dO into the other stage (its readers finished before the last barrier).
    if (s + 1 < n_steps) {
      store_step(stage ^ 1);
      if (s + 2 < n_steps) gload_step(step_head(s + 2), step_q0(s + 2));
    }
    __syncthreads();

    // dQ rows [qs0, qs0 + 32), columns [32 w, 32 w + 32) = dS (32 x BN) K (BN x 32).
    {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int kc = 0; kc < BN / 16; ++kc) {
        const u32x4 a = ldtr8(smem + dst_read + 16 * kc * LDT, LDT);
        const u32x4 b = ldtr8(smem + OFF_K + tr_read + 16 * kc * LD + 32 * wave, LD);
        acc = E::mfma(a, b, acc);
      }
      // register j <-> query qs0 + 8 (j >> 2) + 4 hi + (j & 3), column 32 w + l32.
      float* dqp = dq_acc + (long)qs0 * qrow + (long)h * D + 32 * wave + l32;
      const int rows_left = doc_end - qs0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = 8 * (j >> 2) + 4 * hi + (j & 3);
        if (r < rows_left) atomicAdd(dqp + (long)r * qrow, acc[j] * scale);
      }
    }
    __syncthreads();
  }

  // dK, dV of this wave's keys: register j <-> key kw0 + 8 (j >> 2) + 4 hi + (j & 3), column
  // d = 32 db + l32.
  if (kw0 < doc_end) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = kw0 + 8 * (j >> 2) + 4 * hi + (j & 3);
        if (key < doc_end) {
          const long off = ((long)key * hkv + kvh) * D + 32 * db + l32;
          atomicAdd(dk_acc + off, dkacc[db][j] * scale);
          atomicAdd(dv_acc + off, dvacc[db][j]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// fp32 accumulators -> element type, 8 elements per thread.
// ---------------------------------------------------------------------------------------------
template <class E>
__global__ __launch_bounds__(256) void bwd_post_kernel(const float* __restrict__ src,
                                                       uint16_t* __restrict__ dst, long n8) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const f32x4 a = reinterpret_cast<const f32x4*>(src)[2 * i];
  const f32x4 b = reinterpret_cast<const f32x4*>(src)[2 * i + 1];
  gstore16(dst + 8 * i, pack8<E>(a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]));
}

template <class E>
static hipError_t launch_bwd_prepare_t(const BwdArgs& a) {
  const long rows = a.n_tokens * a.hq;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(bwd_pre_kernel<E>, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0,
                     a.stream, (const uint16_t*)a.out, (const uint16_t*)a.dout, a.delta,
                     a.dq_acc, a.dk_acc, a.dv_acc, (int)a.n_tokens, a.hq, a.hkv);
  return hipGetLastError();
}

template <class E>
static hipError_t launch_bwd_main_t(const BwdArgs& a) {
  if (a.n_items == 0) return hipSuccess;
  hipLaunchKernelGGL((bwd_kernel<E>), dim3((unsigned)a.n_items), dim3(bwd::NT),
                     0, a.stream, (const uint16_t*)a.q, (const uint16_t*)a.k,
                     (const uint16_t*)a.v, (const uint16_t*)a.dout, a.lse, a.delta, a.dq_acc,
                     a.dk_acc, a.dv_acc, (const int4*)a.items, (int)a.n_tokens, a.hq, a.hkv,
                     a.scale, a.scale * kLog2e);
  return hipGetLastError();
}

template <class E>
static hipError_t launch_bwd_finish_t(const BwdArgs& a) {
  const struct {
    const float* src;
    void* dst;
    long n;
  } outs[3] = {{a.dq_acc, a.dq, a.n_tokens * a.hq * kHeadDim},
               {a.dk_acc, a.dk, a.n_tokens * a.hkv * kHeadDim},
               {a.dv_acc, a.dv, a.n_tokens * a.hkv * kHeadDim}};
  for (const auto& t : outs) {
    if (t.dst == nullptr || t.n == 0) continue;
    const long n8 = t.n / 8;
    hipLaunchKernelGGL(bwd_post_kernel<E>, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                       a.stream, t.src, (uint16_t*)t.dst, n8);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_bwd_stage(const BwdArgs& a, int stage) {
  const bool bf = a.dtype != 0;
  switch (stage) {
    case 0: return bf ? launch_bwd_prepare_t<BF16>(a) : launch_bwd_prepare_t<F16>(a);
    case 1: return bf ? launch_bwd_main_t<BF16>(a) : launch_bwd_main_t<F16>(a);
    default: return bf ? launch_bwd_finish_t<BF16>(a) : launch_bwd_finish_t<F16>(a);
  }
}

hipError_t launch_bwd(const BwdArgs& a) {
  for (int stage = 0; stage < 3; ++stage) {
    hipError_t e = launch_bwd_stage(a, stage);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace va
