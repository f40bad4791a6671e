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
template <class E, int NW>
__global__ __launch_bounds__(NW * 64, 1) void bwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, float* __restrict__ dq_acc,
    float* __restrict__ dk_acc, float* __restrict__ dv_acc, const int4* __restrict__ items,
    int n_tokens, int hq, int hkv, float scale, float scale_log2) {
  constexpr int BN = 32 * NW;    // keys per work item
  constexpr int BQ = kBwdBlockQ; // queries per step
  constexpr int D = kHeadDim;
  constexpr int NT = NW * 64;
  constexpr int NCH = BN / 8;    // 16-byte chunks per row of the dS and K^T tiles
  static_assert(BQ == 32, "the query step is one 32-row MFMA block");
  static_assert(4 % NW == 0 || NW % 4 == 0, "d blocks per wave");

  __shared__ __attribute__((aligned(16))) uint16_t qs[BQ * D];     // Q rows, swz8
  __shared__ __attribute__((aligned(16))) uint16_t qt[D * BQ];     // Q^T rows (d), swz4
  __shared__ __attribute__((aligned(16))) uint16_t dos[BQ * D];    // dO rows
  __shared__ __attribute__((aligned(16))) uint16_t dot_[D * BQ];   // dO^T rows (d)
  __shared__ __attribute__((aligned(16))) uint16_t dss[BQ * BN];   // dS rows (query), keys
  __shared__ __attribute__((aligned(16))) uint16_t kt[D * BN];     // K^T rows (d), keys
  __shared__ __attribute__((aligned(16))) float lse_s[BQ];
  __shared__ __attribute__((aligned(16))) float del_s[BQ];

  const int4 it = items[blockIdx.x];
  const int k0 = it.x, doc_end = it.y, h_begin = it.z, h_count = it.w;
  const int group = hq / hkv;
  const int kvh = h_begin / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;

  const int kw0 = k0 + 32 * wave;   // first key of this wave
  const int my_key = kw0 + l32;
  const bool key_valid = my_key < doc_end;
  const bool wave_live = kw0 < doc_end;

  // K and V of this lane's key as MFMA B operands (k slots = d).
  u32x4 kf[8], vf[8];
  {
    const uint16_t* kp = k + (long)(key_valid ? my_key : k0) * kvrow + kvh * D + 8 * hi;
    const uint16_t* vp = v + (long)(key_valid ? my_key : k0) * kvrow + kvh * D + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      kf[kk] = key_valid ? gload16(kp + 16 * kk) : u32x4{0, 0, 0, 0};
      vf[kk] = key_valid ? gload16(vp + 16 * kk) : u32x4{0, 0, 0, 0};
    }
  }
  // K^T of the whole key tile in LDS (B operand of dQ = dS K).
  {
    constexpr int UNITS = (BN / 4) * 16;
    for (int u = tid; u < UNITS; u += NT) {
      const int kq = u >> 4, col8 = u & 15;
      u32x4 r4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 4 * kq + r;
        r4[r] = key < doc_end ? gload16(k + (long)key * kvrow + kvh * D + 8 * col8)
                              : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w[0] = (uint32_t)half_of(r4[0], e) | ((uint32_t)half_of(r4[1], e) << 16);
        w[1] = (uint32_t)half_of(r4[2], e) | ((uint32_t)half_of(r4[3], e) << 16);
        *reinterpret_cast<u32x2*>(kt + tile_off<NCH>(8 * col8 + e, 4 * kq)) = w;
      }
    }
  }

  f32x16 dkacc[4], dvacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  for (int hh = 0; hh < h_count; ++hh) {
    const int h = h_begin + hh;
    for (int qs0 = k0; qs0 < doc_end; qs0 += BQ) {
      __syncthreads();  // the previous step's readers of qs/qt/dos/dot/dss/lse_s are done
      // Stage Q and dO rows [qs0, qs0 + 32) of head h: row-major and transposed.
      for (int u = tid; u < 2 * (BQ / 4) * 16; u += NT) {
        const int which = u >> 7;            // 0: Q, 1: dO
        const int unit = u & 127;
        const int qq = unit >> 4, col8 = unit & 15;
        const uint16_t* src = which ? dout : q;
        u32x4 r4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = qs0 + 4 * qq + r;
          r4[r] = row < doc_end ? gload16(src + (long)row * qrow + h * D + 8 * col8)
                                : u32x4{0, 0, 0, 0};
        }
        uint16_t* rm = which ? dos : qs;
        uint16_t* tr = which ? dot_ : qt;
#pragma unroll
        for (int r = 0; r < 4; ++r) lds_write16(rm, tile_off<16>(4 * qq + r, 8 * col8), r4[r]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          u32x2 w;
          w[0] = (uint32_t)half_of(r4[0], e) | ((uint32_t)half_of(r4[1], e) << 16);
          w[1] = (uint32_t)half_of(r4[2], e) | ((uint32_t)half_of(r4[3], e) << 16);
          *reinterpret_cast<u32x2*>(tr + tile_off<4>(8 * col8 + e, 4 * qq)) = w;
        }
      }
      if (tid < BQ) {
        const int row = qs0 + tid;
        const bool ok = row < doc_end;
        lse_s[tid] = ok ? lse[(long)h * n_tokens + row] * kLog2e : INFINITY;
        del_s[tid] = ok ? delta[(long)h * n_tokens + row] : 0.f;
      }
      __syncthreads();

      const bool active = wave_live && kw0 <= qs0 + BQ - 1;
      if (active) {
        f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int off = tile_off<16>(perm32(l32), 16 * kk + 8 * hi);
          sacc = E::mfma(lds_read16(qs, off), kf[kk], sacc);
          pacc = E::mfma(lds_read16(dos, off), vf[kk], pacc);
        }
        // register j <-> query qs0 + reg_row(j, hi), key my_key
        const bool diag = kw0 + 31 > qs0;
        float p[16], ds[16];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int r0 = 16 * c + 8 * hi;
          const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse_s + r0);
          const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse_s + r0 + 4);
          const f32x4 d0 = *reinterpret_cast<const f32x4*>(del_s + r0);
          const f32x4 d1 = *reinterpret_cast<const f32x4*>(del_s + r0 + 4);
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            const int j = 8 * c + s;
            const float lv = s < 4 ? l0[s] : l1[s - 4];
            const float dv = s < 4 ? d0[s] : d1[s - 4];
            float pv = fast_exp2(sacc[j] * scale_log2 - lv);
            if (diag && my_key > qs0 + r0 + s) pv = 0.f;
            p[j] = pv;
            ds[j] = pv * (pacc[j] - dv);
          }
        }
        u32x4 pp[2], dsp[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int j0 = 8 * c;
          pp[c] = pack8<E>(p[j0], p[j0 + 1], p[j0 + 2], p[j0 + 3], p[j0 + 4], p[j0 + 5],
                           p[j0 + 6], p[j0 + 7]);
          dsp[c] = pack8<E>(ds[j0], ds[j0 + 1], ds[j0 + 2], ds[j0 + 3], ds[j0 + 4], ds[j0 + 5],
                            ds[j0 + 6], ds[j0 + 7]);
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int off = tile_off<4>(32 * db + perm32(l32), 16 * c + 8 * hi);
            dvacc[db] = E::mfma(pp[c], lds_read16(dot_, off), dvacc[db]);
            dkacc[db] = E::mfma(dsp[c], lds_read16(qt, off), dkacc[db]);
          }
        }
        // dS (queries x keys) to LDS, in the element type (the precision the MFMA consumes).
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          dss[tile_off<NCH>(reg_row(j, hi), 32 * wave + l32)] = E::from_f32(ds[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) dss[tile_off<NCH>(reg_row(j, hi), 32 * wave + l32)] = 0;
      }
      __syncthreads();

      // dQ rows [qs0, qs0 + 32) = dS (32 x BN) . K (BN x 128): each wave owns 128 / NW columns.
      constexpr int DB_PER_WAVE = 4 / NW > 0 ? 4 / NW : 1;
      if (wave < 4) {
#pragma unroll
        for (int i = 0; i < DB_PER_WAVE; ++i) {
          const int db = wave * DB_PER_WAVE + i;
          f32x16 acc = f32x16{};
#pragma unroll
          for (int kc = 0; kc < BN / 16; ++kc) {
            const u32x4 a = lds_read16(dss, tile_off<NCH>(perm32(l32), 16 * kc + 8 * hi));
            const u32x4 b = lds_read16(kt, tile_off<NCH>(32 * db + perm32(l32), 16 * kc + 8 * hi));
            acc = E::mfma(a, b, acc);
          }
          float* dqp = dq_acc + (long)h * D + 32 * db + perm32(l32);
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int row = qs0 + reg_row(j, hi);
            if (row < doc_end) atomicAdd(dqp + (long)row * qrow, acc[j] * scale);
          }
        }
      }
    }
  }

  // dK, dV of this wave's keys: register j <-> key kw0 + 8 (j >> 2) + 4 hi + (j & 3),
  // column d = 32 db + perm32(l32).
  if (wave_live) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = 32 * db + perm32(l32);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = kw0 + 8 * (j >> 2) + 4 * hi + (j & 3);
        if (key < doc_end) {
          const long off = ((long)key * hkv + kvh) * D + d;
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
  hipLaunchKernelGGL((bwd_kernel<E, kBwdWaves>), dim3((unsigned)a.n_items), dim3(kBwdWaves * 64),
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
