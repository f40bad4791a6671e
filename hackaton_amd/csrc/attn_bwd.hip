// Backward of packed varlen causal GQA attention for gfx950: one atomic-free, deterministic launch
// over two kinds of work items, plus the GQA sum of dK/dV when query heads share key/value heads.
//
//  kv item   128 keys of one document x one query head, 8 waves: 4 key strips of 32 x 2 halves
//            that take alternate 32-query steps (two waves per SIMD). Per step: S = Q K^T and
//            dP = dO V^T (rows = queries), P = exp2(S scale log2e - lse log2e), dS = P (dP - delta),
//            dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T read by ds_read_b64_tr_b16, so that
//            a lane holds 8 consecutive d of one key per 8 accumulator registers. delta =
//            rowsum(dO * O) is computed by the staging threads. The halves add their partial
//            dK/dV through LDS (half 0 finishes dK, half 1 dV) and write them once, 16-byte rows
//            straight from registers, per query head: into dK/dV themselves when
//            Hq == Hkv, else into per-head partials that the finish pass (or the rotary backward)
//            sums over each GQA group, as the reference sums its expanded copies.
//  q item    128 queries of one document x one query head, 8 waves: 4 query strips x 2 halves that
//            take alternate 32-key tiles. Per tile: S^T = K Q^T and dP^T = V dO^T (one query per
//            lane, lse and delta in-lane), dS^T, dQ^T += K^T dS^T. The halves add their dQ through
//            LDS and write it once in the element type.
//  finish    dK/dV = sum over the G query heads of each group of the per-head partials.
#include <type_traits>

#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace bwd {
constexpr int NS = 4;           // strips of 32 per work item
constexpr int NW = 2 * NS;      // two halves
constexpr int NT = NW * 64;
constexpr int D = kHeadDim;
constexpr int LD = D + 8;       // row stride (halfs) of every row-major LDS tile
constexpr int BK = 32 * NS;     // keys per kv item
constexpr int BQ = 32;          // queries per kv-item step
constexpr int QB = 32 * NS;     // queries per q item
constexpr int BT = 32;          // keys per q-item tile
constexpr int ROWT = 32 * LD;   // halfs of a 32-row tile
// kv item LDS (halfs): K[128], V[128], Q[stage][half], dO[stage][half]; stats floats apart.
constexpr int KV_OFF_K = 0;
constexpr int KV_OFF_V = KV_OFF_K + BK * LD;
constexpr int KV_OFF_Q = KV_OFF_V + BK * LD;
constexpr int KV_OFF_DO = KV_OFF_Q + 4 * ROWT;
constexpr int KV_HALFS = KV_OFF_DO + 4 * ROWT;
// q item LDS (halfs): [stage][K0, V0, K1, V1] 32-row tiles.
constexpr int Q_PAIR = 4 * ROWT;
constexpr int Q_HALFS = 2 * Q_PAIR;
constexpr int HALFS = KV_HALFS > Q_HALFS ? KV_HALFS : Q_HALFS;
static_assert(BK == kBwdBlockN && QB == kBwdBlockM && BQ == kBwdBlockQ, "plan tile sizes");
constexpr int kKindKV = 0, kKindQ = 1;
constexpr int kHeadMask = kItemHeadMask;  // item word: see kItemGroupBit
// Transposed operand reads (Q^T, dO^T, K^T): the second 16-lane group of a wave reads 64 columns
// (d) over the first (TRG), so that the 32 lanes one LDS cycle serves hit 64 distinct banks of
// the 272-byte rows; 16 columns over, as the accumulator layout would suggest, they overlapped on
// 24 of 32 banks (measured at config 2: bank conflicts 16.3% -> 2.0% of the backward's LDS cycles,
// LDS active cycles -15%, time unchanged). An accumulator db then holds, in its registers
// [8 c, 8 c + 8), d = 16 db + 64 c + 8 hi + 0..7 (TRB = 16 columns per db).
constexpr int TRG = 64, TRB = 16;
// The 16-byte chunk i of store_rows32<16> (d = 8 (2 i + hi) + 0..7) that registers [8 c, 8 c + 8)
// of accumulator db fill; and the accumulator / register group that fill chunk i of the 64-column
// block b (store_rows32<8>, d = 64 b + 8 (2 i + hi) + 0..7).
__device__ __host__ constexpr int acc_chunk(int db, int c) { return db + 4 * c; }
__device__ __host__ constexpr int block_db(int /*b*/, int i) { return i; }
__device__ __host__ constexpr int block_c(int b, int /*i*/) { return b; }
}  // namespace bwd

// --------------------------------------------------------------------------------------------
// kv item: dK, dV of 128 keys for one query head, or (pair items) for two query heads h, h + 1
// of one GQA group: then half j takes head h + j over every query step, so the halves share the
// K/V tile, never exchange accumulators, and each writes both partials of its head.
// --------------------------------------------------------------------------------------------
// SHAPE (item word bits 20-21): 0 per head, 1 pair, 2 group; a template constant, so that each
// shape's step loop carries no unit / head arithmetic of the others (per-head items: no division
// by the step count, no pair selects).
template <class E, int SHAPE, bool PREP, bool ROPE>
__device__ __forceinline__ void bwd_kv_item(
    lds_u16* smem, float (&stat)[2][2][2][bwd::BQ], const int4 it,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ out,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse,
    uint16_t* __restrict__ dk_part, uint16_t* __restrict__ dv_part, uint16_t* __restrict__ dk_out,
    uint16_t* __restrict__ dv_out, uint32_t* __restrict__ flags, int n_tokens, int hq, int hkv,
    float scale, float scale_log2, const f32x2* __restrict__ stats, const RopeTab& rope,
    int* trow_lds) {
  using namespace bwd;
  const int k0 = it.x, doc_end = it.y, h = it.w & kHeadMask;
  constexpr bool pair = SHAPE == 1;
  // Group items walk heads h .. h + S - 1 in sequence (S = G: the whole GQA group).
  constexpr bool grouped = SHAPE == 2;
  const int S = grouped ? ((it.w >> kItemHeadsShift) & 0xff) + 1 : 1;
  const int G = hq / hkv;
  const int kvh = h / G;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int half = wave / NS, strip = wave % NS;
  const int src = lane & 15, grp = lane >> 4;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;
  const int kw0 = k0 + 32 * strip;
  const int my_key = kw0 + l32;
  // Rotary table row of this lane's key, looked up with the prologue's loads and parked in LDS
  // (a register held across the step loop would spill there), so that the epilogue's table loads
  // wait for no other memory access.
  if constexpr (ROPE) trow_lds[tid] = (int)rope_row(rope, min(my_key, doc_end - 1));

  // K and V tiles, row-major, rows clamped to the document: loaded here, stored to LDS once the
  // first step pair's loads are in flight too (one memory round trip for the whole prologue).
  u32x4 kvr[2 * (BK / 32)];
  const int kv_srow = tid >> 4, kv_scol = 8 * (tid & 15);
#pragma unroll
  for (int i = 0; i < BK / 32; ++i) {
    const long g = (long)min(k0 + kv_srow + 32 * i, doc_end - 1) * kvrow + kvh * D + kv_scol;
    kvr[2 * i] = gload16(k + g);
    kvr[2 * i + 1] = gload16(v + g);
  }

  const int n_steps = (doc_end - k0 + BQ - 1) / BQ;
  // Units of work: (head, step) in head-major order, over one head or (group items) the S heads
  // h .. h + S - 1. Iterations of the step loop: a pair of units (the halves take alternate units),
  // or one step of each head of a pair item.
  const int n_units = S * n_steps;
  const int n_iter = pair ? n_steps : (n_units + 1) / 2;
  auto unit_of = [&](int p, int j) { return min(2 * p + j, n_units - 1); };  // clamped: loads
  // Group items decode unit 2 p + j into (head offset, step) without a division per iteration:
  // nx_* hold the two units of the iteration whose rows are loaded next and advance by two units
  // per iteration (at most two head changes, n_steps >= 1); cur_* hold the computed iteration's.
  // A head offset of S or more is past the last unit (loads take the last unit's rows).
  int nx_ho[2] = {0, n_steps > 1 ? 0 : 1}, nx_s[2] = {0, n_steps > 1 ? 1 : 0};
  int cur_ho[2] = {0, 0}, cur_s[2] = {0, 0};
  auto advance2 = [&](int& ho, int& st) {
    st += 2;
    if (st >= n_steps) {
      st -= n_steps;
      ++ho;
    }
    if (st >= n_steps) {
      st -= n_steps;
      ++ho;
    }
  };
  // Step and head of unit j of iteration p (grouped: of the iteration loaded next).
  auto step_of = [&](int p, int j) {
    if constexpr (grouped) return nx_ho[j] < S ? nx_s[j] : n_steps - 1;
    else return pair ? p : unit_of(p, j);
  };
  auto head_of = [&](int p, int j) {
    if constexpr (grouped) return h + min(nx_ho[j], S - 1);
    else return pair ? h + j : h;
  };
  // The computed iteration p's unit j: its step, and whether it exists and has queries at or
  // after this strip's keys.
  auto cur_step = [&](int p, int j) {
    if constexpr (grouped) return cur_s[j];
    else return step_of(p, j);
  };
  auto live = [&](int p, int j) {
    if constexpr (grouped) {
      if (cur_ho[j] >= S) return false;
    } else if (!pair && 2 * p + j >= n_units) {
      return false;
    }
    return kw0 <= k0 + cur_step(p, j) * BQ + BQ - 1;
  };

  // Staging of a step pair: thread chunk i is (step half i >> 1, tensor i & 1 = Q / dO), row
  // tid >> 4, 16-byte column tid & 15, through buffer loads bounded at the document end (rows past
  // it read as zeros; their lse is +inf, so P = 0). The O chunk of the same row stays in registers
  // until the store, where its dot product with the dO chunk gives delta = rowsum(dO * O): the
  // loads are then complete and the dot product does not stall the step.
  const int s_row = tid >> 4, s_col = 8 * (tid & 15);
  const int s_voff = (s_row * (int)qrow + s_col) * 2;  // from the unit's (first row, head)
  u32x4 sreg[4], oreg[PREP ? 1 : 2];
  float st_lse = 0.f;
  f32x2 st_pre = f32x2{0.f, 0.f};
  int st_row = 0;
  auto gload_pair = [&](int p) {
    int row0[2];
    long lrow[2];
#pragma unroll
    for (int sh = 0; sh < 2; ++sh) {
      // The unit's head column is in the descriptor's base (wave-uniform), so the per-lane offset
      // is the same for every unit.
      const int hs = head_of(p, sh);
      row0[sh] = k0 + min(step_of(p, sh), n_steps - 1) * BQ;
      lrow[sh] = (long)hs * n_tokens;
      const long base = (long)row0[sh] * qrow + (long)hs * D;
      const long bytes = ((long)(doc_end - row0[sh] - 1) * qrow + D) * 2;
      sreg[2 * sh] = bload16(make_rsrc(q + base, bytes), s_voff);
      sreg[2 * sh + 1] = bload16(make_rsrc(dout + base, bytes), s_voff);
      if constexpr (!PREP) oreg[sh] = bload16(make_rsrc(out + base, bytes), s_voff);
    }
    if (tid < 64) {  // raw value: scaled at the store, so that no wait follows the loads here
      const int sh = tid >> 5;
      st_row = (sh ? row0[1] : row0[0]) + (tid & 31);
      const long at = (sh ? lrow[1] : lrow[0]) + min(st_row, doc_end - 1);
      if constexpr (PREP) st_pre = stats[at];
      else st_lse = lse[at];
    }
  };
  auto store_pair = [&](int stage) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      st128(smem + ((i & 1) ? KV_OFF_DO : KV_OFF_Q) + (stage * 2 + (i >> 1)) * ROWT +
                s_row * LD + s_col,
            sreg[i]);
    if constexpr (PREP) {  // lse log2 e and delta from the row-statistics pass
      if (tid < 64) {
        const bool in = st_row < doc_end;
        stat[stage][0][tid >> 5][tid & 31] = in ? st_pre[0] : INFINITY;
        stat[stage][1][tid >> 5][tid & 31] = in ? st_pre[1] : 0.f;
      }
    } else {
#pragma unroll
      for (int sh = 0; sh < 2; ++sh) {  // delta: sum over the 16 threads that share a row
        float d = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) d = E::dot2(oreg[sh][w], sreg[2 * sh + 1][w], d);
        d = sum_rows16(d);
        if ((tid & 15) == 0) stat[stage][1][sh][s_row] = d;
      }
      if (tid < 64)
        stat[stage][0][tid >> 5][tid & 31] = st_row < doc_end ? st_lse * kLog2e : INFINITY;
    }
  };

  const int rm_read = perm32(l32) * LD + 8 * hi;                 // A rows = queries
  const int kv_read = (32 * strip + l32) * LD + 8 * hi;          // B columns = keys
  // Q^T / dO^T rows (d) through transposed reads, columns in the order that makes the 8
  // registers [8c, 8c + 8) of a dK^T / dV^T accumulator 8 consecutive d (16-byte stores); the
  // second 16-lane group TRG columns over the first.
  const int tr_read = (8 * hi + 2 * (src >> 2)) * LD + TRG * (grp & 1) +
                      4 * ((((src & 3) & 1) << 1) | ((src & 3) >> 1));

  f32x16 dkacc[4], dvacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  if (half) __builtin_amdgcn_s_setprio(1);  // see the forward kernel: issue ties between halves
  gload_pair(0);
#pragma unroll
  for (int i = 0; i < BK / 32; ++i) {
    st128(smem + KV_OFF_K + (kv_srow + 32 * i) * LD + kv_scol, kvr[2 * i]);
    st128(smem + KV_OFF_V + (kv_srow + 32 * i) * LD + kv_scol, kvr[2 * i + 1]);
  }
  store_pair(0);
  __syncthreads();
  for (int p = 0; p < n_iter; ++p) {
    const int stage = p & 1;
    if constexpr (grouped) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        cur_ho[j] = nx_ho[j];
        cur_s[j] = nx_s[j];
        advance2(nx_ho[j], nx_s[j]);
      }
    }
    if (p + 1 < n_iter) gload_pair(p + 1);
    const int qs0 = k0 + cur_step(p, half) * BQ;
    if (live(p, half)) {
      const lds_u16* qs = smem + KV_OFF_Q + (stage * 2 + half) * ROWT;
      const lds_u16* dos = smem + KV_OFF_DO + (stage * 2 + half) * ROWT;
      // S = Q K^T and dP = dO V^T: 16 MFMAs, both operands of each read from LDS 3 MFMAs ahead.
      f32x16 sacc = f32x16{}, pacc = f32x16{};
      auto opa = [&](int i) {  // MFMA i: kk = i >> 1, S (i even) or dP (i odd)
        return ld128(((i & 1) ? dos : qs) + rm_read + 16 * (i >> 1));
      };
      auto opb = [&](int i) {
        return ld128(smem + ((i & 1) ? KV_OFF_V : KV_OFF_K) + kv_read + 16 * (i >> 1));
      };
      u32x4 ra[3], rb[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        ra[i] = opa(i);
        rb[i] = opb(i);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i & 1) pacc = E::mfma(ra[i % 3], rb[i % 3], pacc);
        else sacc = E::mfma(ra[i % 3], rb[i % 3], sacc);
        if (i + 3 < 16) {
          ra[i % 3] = opa(i + 3);
          rb[i % 3] = opb(i + 3);
        }
      }
      VA_SCHED(kSchedDsRead, 6);
#pragma unroll
      for (int i = 0; i < 13; ++i) {
        VA_SCHED(kSchedMfma, 1);
        VA_SCHED(kSchedDsRead, 2);
      }
      VA_SCHED(kSchedMfma, 3);
      // register j <-> query qs0 + reg_row(j, hi); P overwrites S, dS overwrites dP.
      const lds_f32x4* st = reinterpret_cast<const lds_f32x4*>(
          (__attribute__((address_space(3))) float*)&stat[stage][0][half][0]);
      // The dV / dK operands do not depend on the softmax: their first reads go out before it.
      auto opt = [&](int i) {  // MFMA i: c = i >> 3, db = (i >> 1) & 3, dV (i even) / dK (odd)
        return ldtr8(((i & 1) ? qs : dos) + tr_read + 16 * (i >> 3) * LD + TRB * ((i >> 1) & 3), LD);
      };
      u32x4 rt[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) rt[i] = opt(i);
      __builtin_amdgcn_sched_barrier(0);
      auto softmax = [&](auto masked) {
        const int lim = my_key - qs0;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int g4 = 0; g4 < 2; ++g4) {
            const int r0 = 16 * c + 8 * hi + 4 * g4;
            const f32x4 l4 = st[r0 / 4];
            const f32x4 d4 = st[(2 * BQ + r0) / 4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int j = 8 * c + 4 * g4 + e;
              float pv = fast_exp2(fmaf(sacc[j], scale_log2, -l4[e]));
              if (masked && reg_row(j, hi) < lim) pv = 0.f;  // key > query
              sacc[j] = pv;
              pacc[j] = pv * (pacc[j] - d4[e]);
            }
          }
      };
      if (kw0 + 31 > qs0) softmax(std::true_type{});  // the step crosses this strip's diagonal
      else softmax(std::false_type{});
      // dV^T += dO^T P and dK^T += Q^T dS: 16 MFMAs (c, db, dV / dK), the transposed operands
      // read 3 MFMAs ahead.
      u32x4 pa[2], da[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pv8[8], dv8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv8[e] = sacc[8 * c + e];
          dv8[e] = pacc[8 * c + e];
        }
        pa[c] = pack8_tr<E>(pv8);
        da[c] = pack8_tr<E>(dv8);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int c = i >> 3, db = (i >> 1) & 3;
        if (i & 1) dkacc[db] = E::mfma(rt[i % 3], da[c], dkacc[db]);
        else dvacc[db] = E::mfma(rt[i % 3], pa[c], dvacc[db]);
        if (i + 3 < 16) rt[i % 3] = opt(i + 3);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads 3 MFMAs ahead: not sunk to their use
      }
    }
    if (p + 1 < n_iter) store_pair(stage ^ 1);
    __syncthreads();
  }

  // dK^T / dV^T: registers [8c, 8c + 8) of lane (l32, hi) of accumulator db hold key kw0 + l32
  // and d = 16 db + 64 c + 8 hi + 0..7 (chunk acc_chunk(db, c) of the key's row).
  // The halves swap one tensor each through LDS (16-byte chunks, same lane order): half 0 adds
  // half 1's dK and writes dK (scaled), half 1 adds half 0's dV and writes dV.
  lds_f32x4* xs = reinterpret_cast<lds_f32x4*>(
      (__attribute__((address_space(3))) float*)(smem));
  auto slot = [&](int tensor, int db, int j4) { return ((tensor * NS + strip) * 16 + 4 * db + j4) * 64 + lane; };
  static_assert(2 * NS * 16 * 64 * 16 <= HALFS * 2, "dK/dV exchange fits in LDS");
  // The finished 32 x 128 tile goes out through this wave's own exchange slot (read just before,
  // by this wave only) as a row-major LDS tile, so that each 16-byte global store instruction
  // writes 4 whole rows instead of 32-byte pieces of 32 rows.
  // Rows go to `part` at row stride `rs` heads, head `hd` (per-head partials, or a group item's
  // dK/dV at Hkv width).
  auto finish = [&](f32x16(&mine)[4], const f32x16(&other)[4], float mul, uint16_t* part, int rs,
                    int hd) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4)
        xs[slot(half ^ 1, db, j4)] = f32x4{other[db][4 * j4], other[db][4 * j4 + 1],
                                           other[db][4 * j4 + 2], other[db][4 * j4 + 3]};
    __syncthreads();
    u32x4 w[8];  // chunk acc_chunk(db, c): registers [8 c, 8 c + 8) of key kw0 + l32
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      float x[16];
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 y = xs[slot(half, db, j4)];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * j4 + e] = (mine[db][4 * j4 + e] + y[e]) * mul;
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
        w[acc_chunk(db, c)] = pack8<E>(x[8 * c], x[8 * c + 1], x[8 * c + 2], x[8 * c + 3],
                                       x[8 * c + 4], x[8 * c + 5], x[8 * c + 6], x[8 * c + 7]);
    }
    store_rows32<16>(reinterpret_cast<lds_u16*>(&xs[slot(half, 0, 0) - lane]), w, lane,
                    [&](int r) { return part + ((long)(kw0 + r) * rs + hd) * D; }, doc_end - kw0);
  };
  // With rotary tables the halves split the columns instead of the tensors: half H finishes dK
  // and dV for accumulators db = 2 H, 2 H + 1 with both column halves c, i.e. the (d, d + 64)
  // pairs that the inverse rotation of dK mixes (registers [8 c, 8 c + 8) hold d = 16 db + 64 c +
  // 8 hi + 0..7), so each half rotates half of dK with the tables of 16 pairs, loaded before the
  // exchange. Same exchange volume; each tensor goes out as two 64-byte runs per row.
  auto xslot = [&](int dst, int t, int j, int j4) {
    return (((dst * NS + strip) * 2 + t) * 8 + 4 * j + j4) * 64 + lane;
  };
  auto finish_rot = [&](auto half_c, uint16_t* kout, uint16_t* vout, int rs, int hd) {
    constexpr int H = decltype(half_c)::value;
    const int trow = trow_lds[tid];
    Tab8 tab[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) tab[j] = load_tab8(rope, trow, 16 * (2 * H + j) + 8 * hi);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          const f32x16& a = t ? dvacc[2 * (1 - H) + j] : dkacc[2 * (1 - H) + j];
          xs[xslot(H ^ 1, t, j, j4)] = f32x4{a[4 * j4], a[4 * j4 + 1], a[4 * j4 + 2], a[4 * j4 + 3]};
        }
    __syncthreads();
    u32x4 wk[4], wv[4];  // w[j + 2 c]: registers [8 c, 8 c + 8) of accumulator 2 H + j
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float xk[16], xv[16];
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 yk = xs[xslot(H, 0, j, j4)], yv = xs[xslot(H, 1, j, j4)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xk[4 * j4 + e] = (dkacc[2 * H + j][4 * j4 + e] + yk[e]) * scale;
          xv[4 * j4 + e] = dvacc[2 * H + j][4 * j4 + e] + yv[e];
        }
      }
      rope_unrotate8(tab[j], xk);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        wk[j + 2 * c] = pack8<E>(xk[8 * c], xk[8 * c + 1], xk[8 * c + 2], xk[8 * c + 3],
                                 xk[8 * c + 4], xk[8 * c + 5], xk[8 * c + 6], xk[8 * c + 7]);
        wv[j + 2 * c] = pack8<E>(xv[8 * c], xv[8 * c + 1], xv[8 * c + 2], xv[8 * c + 3],
                                 xv[8 * c + 4], xv[8 * c + 5], xv[8 * c + 6], xv[8 * c + 7]);
      }
    }
    // through two row tiles in this wave's own (just read) exchange slots; tile column
    // t = 16 j + 32 c + 8 hi + e holds d = t + 32 H + 32 c
    lds_u16* tk = reinterpret_cast<lds_u16*>(&xs[xslot(H, 0, 0, 0) - lane]);
    lds_u16* tv = reinterpret_cast<lds_u16*>(&xs[xslot(H, 1, 0, 0) - lane]);
    static_assert(32 * (8 * 8 + 8) * 2 <= 8 * 64 * 16, "a row tile fits in one tensor's slots");
    auto cols = [](int col) { return col + 32 * H + (col >= 32 ? 32 : 0); };
    store_rows32<8>(tk, wk, lane, [&](int r) { return kout + ((long)(kw0 + r) * rs + hd) * D; },
                    doc_end - kw0, cols);
    store_rows32<8>(tv, wv, lane, [&](int r) { return vout + ((long)(kw0 + r) * rs + hd) * D; },
                    doc_end - kw0, cols);
  };
  // The GQA sum reads how many heads each partial of a row sums (S; G: a group item wrote the
  // row's dK/dV itself): every key row belongs to one tile, whose items of the GQA group's first
  // head write its flag. Without outputs every head's partial holds a share (zeros beside a
  // group item's sum, below): 1, so that any later sum adds all G.
  if (flags != nullptr && h % G == 0 && tid < BK && k0 + tid < doc_end)
    flags[k0 + tid] = dk_out != nullptr ? S : 1;
  if constexpr (pair) {
    // Each half holds the whole dK/dV of its head: both go out through this wave's own row tile
    // (the LDS stages are free after the loop's last barrier), dK scaled.
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar: no VGPR kept
    const int head_w = pair ? h + (wv >> 2) : h;                         // across the loop
    lds_u16* tile = smem + wv * 32 * (8 * 8 + 8);
    static_assert(NW * 32 * (8 * 8 + 8) <= HALFS, "per-wave row tiles fit in LDS");
    // 64 columns at a time (db 2 c2, 2 c2 + 1), so that few registers are live beside the
    // accumulators.
    auto store = [&](const f32x16(&acc)[4], float mul, uint16_t* part) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        u32x4 w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x16& a = acc[block_db(c2, i)];
          const int c = block_c(c2, i);
          w[i] = pack8<E>(a[8 * c] * mul, a[8 * c + 1] * mul, a[8 * c + 2] * mul,
                          a[8 * c + 3] * mul, a[8 * c + 4] * mul, a[8 * c + 5] * mul,
                          a[8 * c + 6] * mul, a[8 * c + 7] * mul);
        }
        store_rows32<8>(tile, w, lane,
                        [&](int r) {
                          return part + ((long)(kw0 + r) * hq + head_w) * D + 64 * c2;
                        },
                        doc_end - kw0);
      }
    };
    if constexpr (ROPE) {  // dK back to the projection's frame, in place (next tables ahead)
      const int trow = trow_lds[tid];
      Tab8 t0 = load_tab8(rope, trow, 8 * hi), t1;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        if (db + 1 < 4) t1 = load_tab8(rope, trow, 16 * (db + 1) + 8 * hi);
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = dkacc[db][i];
        rope_unrotate8(t0, x);
#pragma unroll
        for (int i = 0; i < 16; ++i) dkacc[db][i] = x[i];
        t0 = t1;
      }
    }
    store(dkacc, scale, dk_part);
    store(dvacc, 1.f, dv_part);
    return;
  }
  if (S == G && dk_out != nullptr) {
    if constexpr (ROPE) {
      if (half) finish_rot(std::integral_constant<int, 1>{}, dk_out, dv_out, hkv, kvh);
      else finish_rot(std::integral_constant<int, 0>{}, dk_out, dv_out, hkv, kvh);
    } else if (half) {
      finish(dvacc, dkacc, 1.f, dv_out, hkv, kvh);
    } else {
      finish(dkacc, dvacc, scale, dk_out, hkv, kvh);
    }
  } else {
    if constexpr (ROPE) {
      if (half) finish_rot(std::integral_constant<int, 1>{}, dk_part, dv_part, hq, h);
      else finish_rot(std::integral_constant<int, 0>{}, dk_part, dv_part, hq, h);
    } else if (half) {
      finish(dvacc, dkacc, 1.f, dv_part, hq, h);
    } else {
      finish(dkacc, dvacc, scale, dk_part, hq, h);
    }
    if constexpr (grouped) {
      // No outputs: the caller sums all G per-head partials of each row, so the item's other
      // heads' partials hold zeros (its sum went into head h's), and that sum is exact.
      if (dk_out == nullptr) {
        // half j clears tensor j (dK / dV) of the other heads
        uint16_t* part = half ? dv_part : dk_part;
        for (int x = 1; x < S; ++x)
          for (int i = lane; i < 32 * (D / 8); i += 64) {
            const int r = i / (D / 8), c = i % (D / 8);
            if (kw0 + r < doc_end)
              gstore16(part + ((long)(kw0 + r) * hq + h + x) * D + 8 * c, u32x4{0u, 0u, 0u, 0u});
          }
      }
    }
  }
}

// --------------------------------------------------------------------------------------------
// q item: dQ of 128 queries for one query head, or (pair items) for two query heads h, h + 1 of
// one GQA group: then half j takes head h + j over both tiles of every pair, so the halves share
// the K/V tiles, never exchange dQ, and each writes all 128 columns of its head.
// --------------------------------------------------------------------------------------------
template <class E, bool PAIR, bool PREP, bool ROPE>
__device__ __forceinline__ void bwd_q_item(
    lds_u16* smem, const int4 it, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, uint16_t* __restrict__ dq, int n_tokens, int hq, int hkv,
    float scale, float scale_log2, float* stat_f, const f32x2* __restrict__ stats,
    const RopeTab& rope, int* trow_lds) {
  using namespace bwd;
  const int q0 = it.x, doc_end = it.y, doc_start = it.z, h = it.w & kHeadMask;
  constexpr bool pair = PAIR;
  const int kvh = h / (hq / hkv);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int half = wave / NS, strip = wave % NS;
  const int src = lane & 15, grp = lane >> 4;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;
  const int wq0 = q0 + 32 * strip;
  const int my_q = wq0 + l32;
  // Rotary table row of this lane's query, looked up with the prologue's loads, parked in LDS.
  if constexpr (ROPE) trow_lds[tid] = (int)rope_row(rope, min(my_q, doc_end - 1));

  const int kv_end = min(q0 + QB, doc_end);
  const int n_tiles = (kv_end - doc_start + BT - 1) / BT;
  const int n_pairs = (n_tiles + 1) / 2;

  // Staging of a tile pair: chunk i is (tile i >> 1, tensor i & 1 = K / V), row tid >> 4.
  const int srow = tid >> 4, scol = 8 * (tid & 15);
  u32x4 sr[4];
  const int voff = (srow * (int)kvrow + kvh * D + scol) * 2;
  auto gload_pair = [&](int p) {  // buffer loads bounded at the document end (zero rows: masked)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      const int row0 = doc_start + (2 * p + t2) * BT;
      const long bytes = ((long)(doc_end - row0 - 1) * kvrow + (long)(kvh + 1) * D) * 2;
      sr[2 * t2] = bload16(make_rsrc(k + (long)row0 * kvrow, bytes), voff);
      sr[2 * t2 + 1] = bload16(make_rsrc(v + (long)row0 * kvrow, bytes), voff);
    }
  };
  auto store_pair = [&](int stage) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st128(smem + stage * Q_PAIR + i * ROWT + srow * LD + scol, sr[i]);
  };

  gload_pair(0);  // in flight together with the Q / dO / O loads below

  // Q and dO of the item's 128 queries: coalesced buffer loads (16 lanes per row, rows past the
  // document end read as zeros), staged in LDS after the two K / V stages; O only for delta =
  // rowsum(dO * O), reduced over the 16 lanes of a row. Each lane then reads its query's Q and
  // dO rows as B operands (k slots = d), lse and delta from the 256-float stat area.
  // A pair item stages its second head's Q / dO in the K / V stages (free until the first pair
  // is stored, after every wave has read its rows back) and its lse / delta in stat_f[2 QB ..).
  constexpr int QT_OFF = Q_HALFS;
  static_assert(Q_HALFS + 2 * QB * LD <= HALFS, "Q / dO tiles of a q item fit in LDS");
  static_assert(2 * QB * LD <= Q_HALFS, "a second head's Q / dO tiles fit in the K / V stages");
  auto stage_head = [&](int hh, int off_q, float* st) {
    const long bytes = ((long)(doc_end - q0 - 1) * qrow + (long)(hh + 1) * D) * 2;
    const brsrc rq = make_rsrc(q + (long)q0 * qrow, bytes);
    const brsrc rd = make_rsrc(dout + (long)q0 * qrow, bytes);
    const brsrc ro = make_rsrc(out + (long)q0 * qrow, bytes);
    u32x4 xq[QB / 32], xd[QB / 32], xo[PREP ? 1 : QB / 32];
#pragma unroll
    for (int i = 0; i < QB / 32; ++i) {
      const int off = ((srow + 32 * i) * (int)qrow + hh * D + scol) * 2;
      xq[i] = bload16(rq, off);
      xd[i] = bload16(rd, off);
      if constexpr (!PREP) xo[i] = bload16(ro, off);
    }
    if constexpr (PREP) {  // lse log2 e and delta from the row-statistics pass
      if (tid < QB) {
        const bool in = q0 + tid < doc_end;
        const f32x2 x = stats[(long)hh * n_tokens + min(q0 + tid, doc_end - 1)];
        st[tid] = in ? x[0] : INFINITY;
        st[QB + tid] = in ? x[1] : 0.f;
      }
    } else if (tid < QB) {
      st[tid] = q0 + tid < doc_end ? lse[(long)hh * n_tokens + q0 + tid] * kLog2e : INFINITY;
    }
#pragma unroll
    for (int i = 0; i < QB / 32; ++i) {
      st128(smem + off_q + (srow + 32 * i) * LD + scol, xq[i]);
      st128(smem + off_q + QB * LD + (srow + 32 * i) * LD + scol, xd[i]);
      if constexpr (!PREP) {
        float d = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) d = E::dot2(xo[i][w], xd[i][w], d);
        d = sum_rows16(d);
        if ((tid & 15) == 0) st[QB + srow + 32 * i] = d;
      }
    }
  };
  stage_head(h, QT_OFF, stat_f);
  if (pair) stage_head(h + 1, 0, stat_f + 2 * QB);

  // LDS read bases inside a tile slot (K at 2 slot, V at 2 slot + 1): K / V rows as A operands
  // (rows = keys through perm32, k = d); K^T through transposed reads with the column order that
  // keeps output registers d-contiguous (dQ^T accumulators laid out as dK^T / dV^T above).
  const int ka_read = perm32(l32) * LD + 8 * hi;
  const int va_read = ROWT + perm32(l32) * LD + 8 * hi;
  const int kt_read = (8 * hi + 2 * (src >> 2)) * LD + TRG * (grp & 1) +
                      4 * ((((src & 3) & 1) << 1) | ((src & 3) >> 1));

  f32x16 dqacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) dqacc[db] = f32x16{};

  if (half) __builtin_amdgcn_s_setprio(1);  // see the forward kernel: issue ties between halves
  if (!pair) store_pair(0);
  __syncthreads();
  u32x4 qf[8], df[8];
  const bool second = pair && half;  // this half's head was staged in the K / V stages
  {
    const int off_q = second ? 0 : QT_OFF;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      qf[kk] = ld128(smem + off_q + (32 * strip + l32) * LD + 16 * kk + 8 * hi);
      df[kk] = ld128(smem + off_q + QB * LD + (32 * strip + l32) * LD + 16 * kk + 8 * hi);
    }
  }
  const float* st = stat_f + (second ? 2 * QB : 0);
  const float lse2 = st[32 * strip + l32], dlt = st[QB + 32 * strip + l32];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    settle(qf[kk]);
    settle(df[kk]);
  }
  if (pair) {  // every wave holds its rows: the first K / V pair may now take the stages
    __syncthreads();
    store_pair(0);
    __syncthreads();
  }
  const int my_head = pair ? h + half : h;
  // Tile t of the stage's slot `slot` (0: K0 V0, 1: K1 V1): S^T, dP^T, dS^T, dQ^T += K^T dS^T.
  auto qtile = [&](int stage, int t, int slot) {
    const int kv0 = doc_start + t * BT;
    if (t < n_tiles && kv0 <= wq0 + 31) {
      const lds_u16* base = smem + stage * Q_PAIR + 2 * slot * ROWT;
      // S^T = K Q^T and dP^T = V dO^T: 16 MFMAs, the K / V operand read 3 MFMAs ahead.
      f32x16 sacc = f32x16{}, pacc = f32x16{};
      auto opa = [&](int i) {  // MFMA i: kk = i >> 1, S (i even) or dP (i odd)
        return ld128(base + ((i & 1) ? va_read : ka_read) + 16 * (i >> 1));
      };
      u32x4 ra[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) ra[i] = opa(i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i & 1) pacc = E::mfma(ra[i % 3], df[i >> 1], pacc);
        else sacc = E::mfma(ra[i % 3], qf[i >> 1], sacc);
        if (i + 3 < 16) ra[i % 3] = opa(i + 3);
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead: not sunk to their use
      }
      // dQ^T operands (K^T, transposed reads) do not depend on the softmax: the first go out now.
      auto opt = [&](int i) {  // MFMA i: c = i >> 2, db = i & 3
        return ldtr8(base + kt_read + 16 * (i >> 2) * LD + TRB * (i & 3), LD);
      };
      u32x4 rt[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) rt[i] = opt(i);
      __builtin_amdgcn_sched_barrier(0);
      // register j <-> key kv0 + reg_row(j, hi), query my_q.
      float ds[16];
      auto softmax = [&](auto masked) {
        const int lim = my_q - kv0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float pv = fast_exp2(fmaf(sacc[j], scale_log2, -lse2));
          if (masked && reg_row(j, hi) > lim) pv = 0.f;  // key > query
          ds[j] = pv * (pacc[j] - dlt);
        }
      };
      if (kv0 + 31 > wq0) softmax(std::true_type{});  // the tile crosses this strip's diagonal
      else softmax(std::false_type{});
      const u32x4 bf[2] = {pack8_tr<E>(ds), pack8_tr<E>(ds + 8)};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dqacc[i & 3] = E::mfma(rt[i % 3], bf[i >> 2], dqacc[i & 3]);
        if (i + 3 < 8) rt[i % 3] = opt(i + 3);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  for (int p = 0; p < n_pairs; ++p) {
    const int stage = p & 1;
    if (p + 1 < n_pairs) gload_pair(p + 1);
    if (pair) {
      qtile(stage, 2 * p, 0);
      qtile(stage, 2 * p + 1, 1);
    } else {
      qtile(stage, 2 * p + half, half);
    }
    if (p + 1 < n_pairs) store_pair(stage ^ 1);
    __syncthreads();
  }

  if (pair) {
    if constexpr (ROPE) {  // dQ back to the projection's frame, in place
      // The two halves hold the same 32 rows of their strip (heads h and h + 1): each loads the
      // tables of two of the four accumulators' d ranges and both read all four back from LDS
      // (free after the loop's last barrier), so each table row is read once per item.
      lds_f32x4* xt = reinterpret_cast<lds_f32x4*>(
          (__attribute__((address_space(3))) float*)(smem));
      auto tslot = [&](int db, int m) { return ((strip * 4 + db) * 8 + m) * 64 + lane; };
      static_assert(NS * 4 * 8 * 64 * 16 <= HALFS * 2, "rotary tables fit in LDS");
      const int trow = trow_lds[tid];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int db = 2 * half + j;
        const Tab8 t = load_tab8(rope, trow, 16 * db + 8 * hi);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          xt[tslot(db, i)] = t.c1[i];
          xt[tslot(db, 2 + i)] = t.c2[i];
          xt[tslot(db, 4 + i)] = t.s1[i];
          xt[tslot(db, 6 + i)] = t.s2[i];
        }
      }
      __syncthreads();
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        Tab8 t;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          t.c1[i] = xt[tslot(db, i)];
          t.c2[i] = xt[tslot(db, 2 + i)];
          t.s1[i] = xt[tslot(db, 4 + i)];
          t.s2[i] = xt[tslot(db, 6 + i)];
        }
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = dqacc[db][i];
        rope_unrotate8(t, x);
#pragma unroll
        for (int i = 0; i < 16; ++i) dqacc[db][i] = x[i];
      }
      __syncthreads();  // every wave has its tables before the row tiles reuse the LDS
    }
    // Each half holds its head's whole dQ^T: 64 columns at a time through this wave's own row
    // tile (the LDS is free after the loop's last barrier), scaled.
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    lds_u16* tile = smem + wv * 32 * (8 * 8 + 8);
    static_assert(NW * 32 * (8 * 8 + 8) <= HALFS, "per-wave row tiles fit in LDS");
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      u32x4 w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x16& a = dqacc[block_db(c2, i)];
        const int c = block_c(c2, i);
        w[i] = pack8<E>(a[8 * c] * scale, a[8 * c + 1] * scale, a[8 * c + 2] * scale,
                        a[8 * c + 3] * scale, a[8 * c + 4] * scale, a[8 * c + 5] * scale,
                        a[8 * c + 6] * scale, a[8 * c + 7] * scale);
      }
      store_rows32<8>(tile, w, lane,
                      [&](int r) { return dq + (long)(wq0 + r) * qrow + my_head * D + 64 * c2; },
                      doc_end - wq0);
    }
    return;
  }

  // The halves swap partial dQ^T columns (16-byte chunks, same lane order): half h finishes
  // d in [64 h, 64 h + 64) of its strip's 32 queries and writes them as whole 128-byte row halves
  // through its own exchange slot as an LDS row tile. The half is a template constant in each
  // branch, so the accumulator indices are compile-time (a runtime index would move them to
  // scratch memory).
  lds_f32x4* xq = reinterpret_cast<lds_f32x4*>((__attribute__((address_space(3))) float*)(smem));
  auto qslot = [&](int dst_half, int i, int j2) {
    return (((dst_half * NS + strip) * 4 + i) * 2 + j2) * 64 + lane;
  };
  auto finish = [&](auto half_c) {
    constexpr int H = decltype(half_c)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        const f32x16& a = dqacc[block_db(H ^ 1, i)];
        const int r = 8 * block_c(H ^ 1, i) + 4 * j2;
        xq[qslot(H ^ 1, i, j2)] = f32x4{a[r], a[r + 1], a[r + 2], a[r + 3]};
      }
    __syncthreads();
    u32x4 w[4];  // chunk i of the 64 columns from 64 H: registers of block_db / block_c(H, i)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x16& a = dqacc[block_db(H, i)];
      const int c = block_c(H, i);
      float x[8];
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        const f32x4 y = xq[qslot(H, i, j2)];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * j2 + e] = (a[8 * c + 4 * j2 + e] + y[e]) * scale;
      }
      w[i] = pack8<E>(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
    }
    store_rows32<8>(reinterpret_cast<lds_u16*>(&xq[qslot(H, 0, 0) - lane]), w, lane,
                    [&](int r) { return dq + (long)(wq0 + r) * qrow + h * D + 64 * H; },
                    doc_end - wq0);
  };
  // With rotary tables half H finishes instead accumulators db = 2 H, 2 H + 1 with both column
  // halves c, i.e. the (d, d + 64) pairs that the inverse rotation mixes: d in [32 H, 32 H + 32)
  // and [64 + 32 H, 96 + 32 H), two 64-byte runs per row. Same exchange volume.
  auto finish_rot = [&](auto half_c) {
    constexpr int H = decltype(half_c)::value;
    const int trow = trow_lds[tid];
    Tab8 tab[2];  // issued before the exchange, which hides their latency
#pragma unroll
    for (int j = 0; j < 2; ++j) tab[j] = load_tab8(rope, trow, 16 * (2 * H + j) + 8 * hi);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2) {
          const f32x16& a = dqacc[2 * (1 - H) + j];
          const int r = 8 * c + 4 * j2;
          xq[qslot(H ^ 1, 2 * j + c, j2)] = f32x4{a[r], a[r + 1], a[r + 2], a[r + 3]};
        }
    __syncthreads();
    u32x4 w[4];  // w[j + 2 c]: registers [8 c, 8 c + 8) of accumulator 2 H + j
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f32x16& a = dqacc[2 * H + j];
      float x[16];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2) {
          const f32x4 y = xq[qslot(H, 2 * j + c, j2)];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            x[8 * c + 4 * j2 + e] = (a[8 * c + 4 * j2 + e] + y[e]) * scale;
        }
      rope_unrotate8(tab[j], x);
#pragma unroll
      for (int c = 0; c < 2; ++c)
        w[j + 2 * c] = pack8<E>(x[8 * c], x[8 * c + 1], x[8 * c + 2], x[8 * c + 3],
                                x[8 * c + 4], x[8 * c + 5], x[8 * c + 6], x[8 * c + 7]);
    }
    // tile column t = 16 j + 32 c + 8 hi + e holds d = t + 32 H + 32 c
    store_rows32<8>(reinterpret_cast<lds_u16*>(&xq[qslot(H, 0, 0) - lane]), w, lane,
                    [&](int r) { return dq + (long)(wq0 + r) * qrow + h * D; }, doc_end - wq0,
                    [](int col) { return col + 32 * H + (col >= 32 ? 32 : 0); });
  };
  if constexpr (ROPE) {
    if (half) finish_rot(std::integral_constant<int, 1>{});
    else finish_rot(std::integral_constant<int, 0>{});
  } else if (half) {
    finish(std::integral_constant<int, 1>{});
  } else {
    finish(std::integral_constant<int, 0>{});
  }
}

// PREP: lse log2 e and delta come from the row-statistics pass (`stats`); otherwise the items
// load O beside dO and form delta themselves. ROPE: dQ and dK are rotated back with `rope`'s
// tables before they are stored.
template <class E, bool PREP, bool ROPE>
// Arguments in the order the work-group needs them: the first 14 dwords are preloaded into
// SGPRs at launch (-amdgpu-kernarg-preload-count), so the work item's load starts at once.
__global__ __launch_bounds__(bwd::NT, 1) void bwd_kernel(
    const int4* __restrict__ items, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, int hq, int hkv,
    const float* __restrict__ lse, uint16_t* __restrict__ dq, uint16_t* __restrict__ dk_part,
    uint16_t* __restrict__ dv_part, int n_tokens, float scale, float scale_log2,
    uint16_t* __restrict__ dk_out, uint16_t* __restrict__ dv_out, uint32_t* __restrict__ flags,
    const f32x2* __restrict__ stats, RopeTab rope) {
  __shared__ __attribute__((aligned(16))) uint16_t smem_raw[bwd::HALFS];
  __shared__ __attribute__((aligned(16))) float stat[2][2][2][bwd::BQ];  // [stage][lse|del][half]
  __shared__ __attribute__((aligned(16))) float qstat[4 * bwd::QB];  // q items: [head][lse|del]
  __shared__ int trow_lds[ROPE ? bwd::NT : 1];  // rotary table row of each thread's key / query
  lds_u16* smem = (lds_u16*)smem_raw;
  const int4 it = items[blockIdx.x];
  // Empty slots of a device-built plan, and items that do not fit this launch (a plan built for
  // other sizes), are skipped: nothing outside [0, n_tokens) x [0, hq) is ever addressed.
  const int kind = it.w >> 24, h = it.w & bwd::kHeadMask, shape = (it.w >> 20) & 15;
  // Pair items (shape 1) take heads h, h + 1 of one GQA group; group items (shape 2, kv only)
  // heads h .. h + S - 1 (S >= 2 dividing G, h a multiple of S).
  const int G = hq / hkv, S = ((it.w >> kItemHeadsShift) & 0xff) + 1;
  if (it.x >= it.y || it.z < 0 || it.x < it.z || it.y > n_tokens || h >= hq ||
      (kind != bwd::kKindKV && kind != bwd::kKindQ) || shape > 2 ||
      (shape < 2 && S != 1) ||
      (shape == 1 && (h + 1 >= hq || h / G != (h + 1) / G)) ||
      (shape == 2 && (kind != bwd::kKindKV || S < 2 || G % S != 0 || h % S != 0)))
    return;
  if (kind == bwd::kKindKV) {
    if (shape == 0)
      bwd_kv_item<E, 0, PREP, ROPE>(smem, stat, it, q, k, v, out, dout, lse, dk_part, dv_part, dk_out,
                              dv_out, flags, n_tokens, hq, hkv, scale, scale_log2, stats,
                              rope, trow_lds);
    else if (shape == 1)
      bwd_kv_item<E, 1, PREP, ROPE>(smem, stat, it, q, k, v, out, dout, lse, dk_part, dv_part, dk_out,
                              dv_out, flags, n_tokens, hq, hkv, scale, scale_log2, stats,
                              rope, trow_lds);
    else
      bwd_kv_item<E, 2, PREP, ROPE>(smem, stat, it, q, k, v, out, dout, lse, dk_part, dv_part, dk_out,
                              dv_out, flags, n_tokens, hq, hkv, scale, scale_log2, stats,
                              rope, trow_lds);
  } else if (shape == 0) {
    bwd_q_item<E, false, PREP, ROPE>(smem, it, q, k, v, out, dout, lse, dq, n_tokens, hq, hkv, scale,
                               scale_log2, qstat, stats, rope, trow_lds);
  } else {
    bwd_q_item<E, true, PREP, ROPE>(smem, it, q, k, v, out, dout, lse, dq, n_tokens, hq, hkv, scale,
                              scale_log2, qstat, stats, rope, trow_lds);
  }
}

// --------------------------------------------------------------------------------------------
// Row statistics of the backward, once per (query head, row): {lse log2 e, delta = rowsum(dO * O)}
// in fp32, with the arithmetic of the items' own staging (16 threads per row, v_dot2 over each
// thread's 8 elements, then the 16-lane DPP sum), so that the main kernel's results do not depend
// on where delta was formed. Rows are taken in the statistics' own (head, token) order, 64 per
// work-group, 4 per thread (8 loads of O / dO and 4 of lse in flight each): lse is read and the
// statistics written as whole lines, while each O / dO row is a contiguous 256 bytes anyway. In
// the token-major order of O / dO the 8-byte statistics of one line came from several
// work-groups (config 5: 98-100 us against 92).
// --------------------------------------------------------------------------------------------
constexpr int kStatThreads = 256, kStatRows = 64;
template <class E>
__global__ __launch_bounds__(kStatThreads) void bwd_stats_kernel(
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, f32x2* __restrict__ stats, int n_tokens, int hq) {
  const int tid = threadIdx.x;
  const long rows = (long)n_tokens * hq;
  const long r0 = (long)blockIdx.x * kStatRows + (tid >> 4);
  const int col = 8 * (tid & 15);
  constexpr int R = kStatRows / (kStatThreads / 16);
  u32x4 o[R], g[R];
  float l[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const long r = min(r0 + 16 * i, rows - 1);  // h * n_tokens + token
    const int h = (int)(r / n_tokens), token = (int)(r - (long)h * n_tokens);
    const long at = ((long)token * hq + h) * kHeadDim + col;
    l[i] = lse[r];
    o[i] = gload16(out + at);
    g[i] = gload16(dout + at);
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float d = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) d = E::dot2(o[i][w], g[i][w], d);
    d = sum_rows16(d);
    const long r = r0 + 16 * i;
    if ((tid & 15) == 0 && r < rows) stats[r] = f32x2{l[i] * kLog2e, d};
  }
}

// --------------------------------------------------------------------------------------------
// dK/dV = sum over the G query heads of each key/value head of the per-head partials (fp32 sum
// of the 16-bit partials, one rounding); 8 elements per thread, 128 threads per work-group
// (measured at config 2: 4.60 us against 4.68 with 256, 4.78 with 512, 5.14 with 1024).
// --------------------------------------------------------------------------------------------
constexpr int kSumThreads = 128;
template <class E>
__global__ __launch_bounds__(kSumThreads) void bwd_gqa_sum_kernel(const uint16_t* __restrict__ dk_part,
                                                          const uint16_t* __restrict__ dv_part,
                                                          uint16_t* __restrict__ dk,
                                                          uint16_t* __restrict__ dv, long n8,
                                                          int hq, int hkv,
                                                          const uint32_t* __restrict__ flags) {
  long i = (long)blockIdx.x * kSumThreads + threadIdx.x;
  const uint16_t* src = dk_part;
  uint16_t* dst = dk;
  if (i >= n8) {
    i -= n8;
    src = dv_part;
    dst = dv;
    if (i >= n8) return;
  }
  // i indexes 8-element chunks of (N, Hkv, D): row r = token * Hkv + kvh, chunk c of 16.
  const long r = i >> 4;
  const int c = (int)(i & 15);
  const long token = r / hkv;
  const int kvh = (int)(r - token * hkv);
  // Partials of this row: G / S of them, S heads apart (S = 1: one per head); S = G: a group
  // item wrote the row itself.
  const int S = flags != nullptr ? max((int)flags[token], 1) : 1;
  if (S >= hq / hkv) return;
  const int g = hq / hkv, n = g / S;
  const uint16_t* p = src + (token * hq + (long)kvh * g) * kHeadDim + 8 * c;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // All loads of a batch go out before the first add (one memory round trip per 8 partials).
  for (int x0 = 0; x0 < n; x0 += 8) {
    u32x4 w[8];
#pragma unroll
    for (int x = 0; x < 8; ++x)
      if (x0 + x < n) w[x] = gload16(p + (long)(x0 + x) * S * kHeadDim);
#pragma unroll
    for (int x = 0; x < 8; ++x)
      if (x0 + x < n) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += E::to_f32(half_of(w[x], e));
      }
  }
  gstore16(dst + 8 * i, pack8<E>(acc[0], acc[1], acc[2], acc[3], acc[4], acc[5], acc[6], acc[7]));
}

template <class E>
static hipError_t launch_bwd_stats_t(const BwdArgs& a) {
  if (a.n_tokens == 0 || a.stats == nullptr) return hipSuccess;
  const dim3 grid((unsigned)((a.n_tokens * a.hq + kStatRows - 1) / kStatRows));
  hipLaunchKernelGGL(bwd_stats_kernel<E>, grid, dim3(kStatThreads), 0, a.stream,
                     (const uint16_t*)a.out, (const uint16_t*)a.dout, a.lse, (f32x2*)a.stats,
                     (int)a.n_tokens, a.hq);
  return hipGetLastError();
}

// PREP: the row statistics are in a.stats already (written by launch_bwd_stats_t); ROPE: a.rope
// holds the rotary tables.
template <class E, bool PREP, bool ROPE>
static hipError_t launch_bwd_main_t(const BwdArgs& a) {
  if (a.n_items == 0) return hipSuccess;
  hipLaunchKernelGGL((bwd_kernel<E, PREP, ROPE>), dim3((unsigned)a.n_items), dim3(bwd::NT), 0,
                     a.stream, (const int4*)a.items, (const uint16_t*)a.q, (const uint16_t*)a.k,
                     (const uint16_t*)a.v, (const uint16_t*)a.out, (const uint16_t*)a.dout, a.hq,
                     a.hkv, a.lse, (uint16_t*)a.dq, (uint16_t*)a.dk_part, (uint16_t*)a.dv_part,
                     (int)a.n_tokens, a.scale, a.scale * kLog2e, (uint16_t*)a.dk,
                     (uint16_t*)a.dv, a.flags, (const f32x2*)a.stats, a.rope);
  return hipGetLastError();
}

// heads_only: the list has no group items, every row sums its G per-head partials (flags unread).
template <class E>
static hipError_t launch_bwd_finish_t(const BwdArgs& a, bool heads_only) {
  if (a.dk == nullptr || a.dk_part == a.dk) return hipSuccess;  // partials are the result
  const long n8 = a.n_tokens * a.hkv * kHeadDim / 8;
  if (n8 == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((2 * n8 + kSumThreads - 1) / kSumThreads);
  hipLaunchKernelGGL(bwd_gqa_sum_kernel<E>, dim3(blocks), dim3(kSumThreads), 0,
                     a.stream, (const uint16_t*)a.dk_part, (const uint16_t*)a.dv_part,
                     (uint16_t*)a.dk, (uint16_t*)a.dv, n8, a.hq, a.hkv,
                     heads_only ? nullptr : a.flags);
  return hipGetLastError();
}

hipError_t launch_bwd_stage(const BwdArgs& a, int stage) {
  const bool bf = a.dtype != 0;
  if (stage == 4) return bf ? launch_bwd_stats_t<BF16>(a) : launch_bwd_stats_t<F16>(a);
  if (stage == 1) {
    const bool prep = a.stats != nullptr, rope = a.rope.cos != nullptr;
    if (bf) {
      if (rope) return prep ? launch_bwd_main_t<BF16, true, true>(a)
                            : launch_bwd_main_t<BF16, false, true>(a);
      return prep ? launch_bwd_main_t<BF16, true, false>(a) : launch_bwd_main_t<BF16, false, false>(a);
    }
    if (rope) return prep ? launch_bwd_main_t<F16, true, true>(a)
                          : launch_bwd_main_t<F16, false, true>(a);
    return prep ? launch_bwd_main_t<F16, true, false>(a) : launch_bwd_main_t<F16, false, false>(a);
  }
  const bool heads_only = stage == 3;
  return bf ? launch_bwd_finish_t<BF16>(a, heads_only) : launch_bwd_finish_t<F16>(a, heads_only);
}

hipError_t launch_bwd(const BwdArgs& a) {
  for (int stage = 1; stage < 3; ++stage) {
    hipError_t e = launch_bwd_stage(a, stage);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace va
