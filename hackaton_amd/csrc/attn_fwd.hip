// Forward kernel of packed varlen causal GQA attention for gfx950.
//
// One work-group = one work item of the plan: NW waves x 32 queries of one document and one query
// head. The K/V tiles of the document (BN = 64 keys) stream through LDS (double buffered, K
// row-major, V transposed so the P.V product reads 8 consecutive keys per lane); Q stays in
// registers. Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 so that one lane owns one
// query: the online softmax (running max / sum, exp2 with scale*log2(e) folded in) is in-lane plus
// one cross-half exchange. O^T = V^T P^T accumulates in fp32; per-row log-sum-exp is written to
// lse[h][token] (natural log). Causal masking is applied only on tiles that cross the diagonal;
// tiles past the diagonal are never loaded (the plan bounds the key range by the last query).
#include "va_common.h"
#include "va_kernels.h"

namespace va {

constexpr int kFwdBN = 64;

template <class E, int NW>
__global__ __launch_bounds__(NW * 64, 2) void fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ lse,
    const int4* __restrict__ items, int n_tokens, int hq, int hkv, float scale_log2) {
  constexpr int BM = 32 * NW;
  constexpr int BN = kFwdBN;
  constexpr int D = kHeadDim;
  constexpr int NT = NW * 64;
  constexpr int KCH = BN * 16 / NT;    // 16-byte K chunks per thread per tile
  constexpr int VU = (BN / 4) * 16 / NT;  // (key quad, d chunk) units per thread per tile
  static_assert(KCH * NT == BN * 16 && VU * NT == (BN / 4) * 16, "tile split");

  __shared__ __attribute__((aligned(16))) uint16_t ks[2][BN * D];  // K rows, 16 chunks, swz8
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][D * BN];  // V^T rows (d), 8 chunks

  const int4 it = items[blockIdx.x];
  const int q0 = it.x, doc_end = it.y, doc_start = it.z, h = it.w;
  const int group = hq / hkv;
  const int kvh = h / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;

  const int wq0 = q0 + 32 * wave;             // first query of this wave
  const int my_q = wq0 + l32;
  const bool q_valid = my_q < doc_end;
  const bool wave_live = wq0 < doc_end;

  u32x4 qf[8];
  {
    const uint16_t* qp = q + (long)(q_valid ? my_q : q0) * qrow + h * D + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      qf[kk] = q_valid ? gload16(qp + 16 * kk) : u32x4{0, 0, 0, 0};
    }
  }

  const int kv_end = min(q0 + BM, doc_end);
  const int n_tiles = (kv_end - doc_start + BN - 1) / BN;

  u32x4 kreg[KCH];
  u32x4 vreg[VU][4];
  const uint16_t* kbase = k + kvh * D;
  const uint16_t* vbase = v + kvh * D;

  auto load_tile = [&](int t) {
    const int kv0 = doc_start + t * BN;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * NT;
      const int key = kv0 + (c >> 4);
      kreg[i] = key < doc_end ? gload16(kbase + (long)key * kvrow + 8 * (c & 15))
                              : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = tid + i * NT;
      const int key = kv0 + 4 * (u >> 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vreg[i][r] = key + r < doc_end
                         ? gload16(vbase + (long)(key + r) * kvrow + 8 * (u & 15))
                         : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * NT;
      lds_write16(ks[buf], tile_off<16>(c >> 4, 8 * (c & 15)), kreg[i]);
    }
#pragma unroll
    for (int i = 0; i < VU; ++i) {
      const int u = tid + i * NT;
      const int kq = u >> 4, col8 = u & 15;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w[0] = (uint32_t)half_of(vreg[i][0], e) | ((uint32_t)half_of(vreg[i][1], e) << 16);
        w[1] = (uint32_t)half_of(vreg[i][2], e) | ((uint32_t)half_of(vreg[i][3], e) << 16);
        *reinterpret_cast<u32x2*>(vt[buf] + tile_off<8>(8 * col8 + e, 4 * kq)) = w;
      }
    }
  };

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    const int kv0 = doc_start + t * BN;
    if (t + 1 < n_tiles) load_tile(t + 1);

    if (wave_live && kv0 <= wq0 + 31) {
      f32x16 sacc[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        sacc[b] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const u32x4 a = lds_read16(ks[buf], tile_off<16>(32 * b + perm32(l32), 16 * kk + 8 * hi));
          sacc[b] = E::mfma(a, qf[kk], sacc[b]);
        }
      }
      const bool diag = kv0 + BN - 1 > wq0;
      float mt = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float x = sacc[b][j] * scale_log2;
          if (diag && kv0 + 32 * b + reg_row(j, hi) > my_q) x = -INFINITY;
          sacc[b][j] = x;
          mt = fmaxf(mt, x);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = fast_exp2(sacc[b][j] - m_use);
          sacc[b][j] = p;
          rs += p;
        }
      }
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;

#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int j0 = 8 * c;
          const u32x4 pf = pack8<E>(sacc[b][j0], sacc[b][j0 + 1], sacc[b][j0 + 2], sacc[b][j0 + 3],
                                    sacc[b][j0 + 4], sacc[b][j0 + 5], sacc[b][j0 + 6],
                                    sacc[b][j0 + 7]);
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const u32x4 a = lds_read16(vt[buf], tile_off<8>(32 * db + perm32(l32),
                                                            32 * b + 16 * c + 8 * hi));
            oacc[db] = E::mfma(a, pf, oacc[db]);
          }
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (q_valid) {
    const float inv = 1.f / l_tot;
    uint16_t* op = o + (long)my_q * qrow + h * D;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int j0 = 8 * c;
        const f32x16& a = oacc[db];
        const u32x4 w = pack8<E>(a[j0] * inv, a[j0 + 1] * inv, a[j0 + 2] * inv, a[j0 + 3] * inv,
                                 a[j0 + 4] * inv, a[j0 + 5] * inv, a[j0 + 6] * inv,
                                 a[j0 + 7] * inv);
        gstore16(op + 32 * db + 16 * c + 8 * hi, w);
      }
    }
    if (hi == 0) lse[(long)h * n_tokens + my_q] = (m_run + fast_log2(l_tot)) * kLn2;
  }
}

template <class E, int NW>
static hipError_t launch_fwd_t(const FwdArgs& a) {
  if (a.n_items == 0) return hipSuccess;
  hipLaunchKernelGGL((fwd_kernel<E, NW>), dim3((unsigned)a.n_items), dim3(NW * 64), 0, a.stream,
                     (const uint16_t*)a.q, (const uint16_t*)a.k, (const uint16_t*)a.v,
                     (uint16_t*)a.out, a.lse, (const int4*)a.items, (int)a.n_tokens, a.hq, a.hkv,
                     a.scale * kLog2e);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdArgs& a) {
  return a.dtype == 0 ? launch_fwd_t<F16, kFwdWaves>(a) : launch_fwd_t<BF16, kFwdWaves>(a);
}

}  // namespace va
