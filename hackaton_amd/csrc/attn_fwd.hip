// Forward kernel of packed varlen causal GQA attention for gfx950.
//
// One work-group = one work item of the plan: 128 queries (4 strips of 32) of one document and one
// query head, run by 8 waves in two halves. Half h (waves 4h .. 4h + 3) processes the key tiles
// t = h, h + 2, h + 4, ... (64 keys each) for the 4 query strips, so two waves share each SIMD
// and the key range of the work item is split in two. The halves run out of phase: half 1
// computes S^T of its next tile at the end of a pair, so a pair starts with half 0's S^T MFMAs
// beside half 1's softmax. At the end the halves swap their unnormalised partial O through LDS
// and publish (m, l); each half finishes 64 of the 128 columns, half 0 also the log-sum-exp.
//
// Per wave: Q (copied once into LDS, read back as each lane's row) stays in registers as the MFMA B
// operand; S^T = K Q^T (v_mfma_f32_32x32x16) puts one query per lane, so the online softmax is
// in-lane plus one v_permlane32_swap; O^T += V^T P^T reads V^T straight from the row-major tile
// with ds_read_b64_tr_b16. K/V tiles stream through two LDS stages of tile pairs, copied straight
// from HBM into LDS by buffer loads that write LDS (256-byte rows, 16-byte chunks XOR-swizzled by
// swz16 so that the K and V^T reads hit disjoint banks); the next pair's copies are in flight
// while the current pair is computed, one barrier per pair. Loads are buffer loads bounded at the
// document end: rows past it read as zeros (masked keys, zero P). The running maximum moves
// lazily (only when a tile exceeds it by more than 2^8), so P stays below 256 and the O / l
// rescale is skipped on most tiles. Results leave through non-temporal stores.
#include <type_traits>

#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace fwd {
constexpr int NS = 4;           // query strips of 32 per work item
constexpr int BM = 32 * NS;     // queries per work item
constexpr int NW = 2 * NS;      // waves: two halves over the key tiles
constexpr int NT = NW * 64;
constexpr int BN = 64;          // keys per tile
constexpr int D = kHeadDim;
constexpr int TILE = BN * D;    // halfs per K or V tile: 256-byte rows, chunks swizzled by swz16
constexpr int PAIR = 4 * TILE;  // K0, V0, K1, V1 of one tile pair
constexpr float kRescaleLog2 = 8.f;     // largest P before the running maximum must move
static_assert(NT == 512 && BN == 64, "pair copy map: 2 groups of 4 rows per wave and tile");
static_assert(BM == kFwdBlockM, "the plan's query tile");
}  // namespace fwd

// --------------------------------------------------------------------------------------------
// Narrow item of the 8-wave forward (kItemNarrowBit): 64 queries of one head, 8 waves = 2 query
// strips x 4 key phases (wave w: strip w & 1, phase w >> 1). The keys go in quads of 128, the
// K and V of a 64-key tile pair copied into a stage as a wide item's pairs are (K0, V0, K1, V1);
// phase j takes the quad's 32-key tile j (rows 32 (j & 1) of the pair's tile j >> 1). A wave
// then walks a quarter of the item's keys, half as many quads as a wide item's waves walk tile
// pairs, with half a pair's MFMA work in each: the plan gives its longest items this shape when
// the list leaves CUs idle. At the end the four phases of a strip merge (m, l, O) through LDS
// and phase j finishes the 32 columns [32 j, 32 j + 32) of its strip.
// --------------------------------------------------------------------------------------------
template <class E>
__device__ __forceinline__ void fwd_narrow_item(
    lds_u16* smem, uint16_t* smem_raw, int q0, int doc_end, int doc_start, int h,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int hq, int hkv, uint16_t* __restrict__ o,
    float* __restrict__ lse, int n_tokens, float scale_log2) {
  using namespace fwd;
  const int group = hq / hkv;
  const int kvh = h / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int strip = wave & 1, phase = wave >> 1;
  const int src = lane & 15, grp = lane >> 4;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;
  const int wq0 = q0 + 32 * strip;
  const int my_q = wq0 + l32;
  const bool q_valid = my_q < doc_end;
  const int ws = __builtin_amdgcn_readfirstlane(wave);
  const int wq0_u = __builtin_amdgcn_readfirstlane(wq0);
  const int kv_end = min(q0 + 64, doc_end);
  const int n_quads = (kv_end - doc_start + 2 * BN - 1) / (2 * BN);

  // Copies (straight from HBM into LDS, swizzled rows as in the wide item): every wave moves row
  // groups 2 w and 2 w + 1 (4 rows each) of each 64-row tile, 8 instructions per quad; rows past
  // the document end read as zeros.
  int coff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 4 * (2 * wave + j) + (lane >> 4);
    coff[j] = (r * (int)kvrow + 8 * ((lane & 15) ^ swz16(r))) * 2;
  }
  auto copy_tile = [&](int t, int x, uint32_t dst) {  // 64-key tile t of K (x = 0) or V
    const int row0 = doc_start + t * BN;
    const long base = (long)row0 * kvrow + kvh * D;
    const long bytes = ((long)(doc_end - row0 - 1) * kvrow + D) * 2;
    const u32x4 r = make_rsrc4((x ? v : k) + base, bytes);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16_opaque(r, dst + 4 * (2 * ws + j) * D * 2, coff[j]);
  };
  auto copy_quad = [&](int p, int stage) {
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr(smem + stage * PAIR));
#pragma unroll
    for (int i = 0; i < 4; ++i) copy_tile(2 * p + (i >> 1), i & 1, dst + i * TILE * 2);
  };

  int koff[8], toff[4][2];
  {
    const int r = perm32(l32), f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = r * D + 8 * ((2 * kk + hi) ^ f);
    const int sg = (((src & 3) & 1) << 1) | ((src & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int rr = 8 * hi + 2 * (src >> 2) + e;
        const int lc = 2 * (grp & 1) + 4 * db + (sg >> 1);
        toff[db][e] = rr * D + 8 * (lc ^ swz16(rr)) + 4 * (sg & 1);
      }
  }

  u32x4 qf[8];
  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  // S^T of the phase's 32-key tile (K rows at `kb`): 8 MFMAs, K operands read 4 ahead.
  auto s_blk = [&](const lds_u16* kb, f32x16& s) {
    s = f32x16{};
    u32x4 ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = ld128(kb + koff[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s = E::mfma(ka[i & 3], qf[i], s);
      if (i + 4 < 8) ka[i & 3] = ld128(kb + koff[i + 4]);
    }
  };
  // Mask, online softmax and O^T += V^T P^T of the tile (V rows at `vb`, keys from kv0).
  auto pv_blk = [&](const lds_u16* vb, int kv0, f32x16& s) {
    auto v_read = [&](int i) {  // i = (c, db): keys 16 c .. 16 c + 15, d block db
      const lds_u16* p = vb + 16 * (i >> 2) * D;
      const u32x2 x = ldtr(p + toff[i & 3][0]), y = ldtr(p + toff[i & 3][1]);
      return u32x4{x[0], x[1], y[0], y[1]};
    };
    u32x4 va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = v_read(i);
    if (kv0 + 31 > wq0_u) {  // the tile crosses this strip's diagonal: key > query -> -inf
      const int lim = my_q - kv0;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (reg_row(j, hi) > lim) s[j] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) mt = fmaxf(mt, s[j]);
    mt = max_with_other_half(mt) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(mt > m_run + kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float rs = 0.f;
    u32x4 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(s[8 * c + e], scale_log2, -m_use));
      pf[c] = pack8_tr<E>(p);
#pragma unroll
      for (int w = 0; w < 4; ++w) rs = E::sum2(pf[c][w], rs);
    }
    l_run += rs;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      oacc[i & 3] = E::mfma(va[i & 3], pf[i >> 2], oacc[i & 3]);
      if (i + 4 < 8) va[i & 3] = v_read(i + 4);
    }
  };

  // Q of the 64 queries into the second stage (every wave 2 row groups of 4 rows), quad 0 into
  // the first; every lane reads its query's row back as its B operand.
  {
    const long bytes = ((long)(doc_end - q0 - 1) * qrow + (long)(h + 1) * D) * 2;
    const u32x4 rq = make_rsrc4(q + (long)q0 * qrow, bytes);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = 4 * (2 * wave + j) + (lane >> 4);
      dma16_opaque(rq, lds_addr(smem + PAIR + 4 * (2 * ws + j) * D),
                   (r * (int)qrow + h * D + 8 * ((lane & 15) ^ swz16(r))) * 2);
    }
  }
  copy_quad(0, 0);
  wait_vmcnt<0>();
  __syncthreads();
  {
    const int r = 32 * strip + l32, f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = ld128(smem + PAIR + r * D + 8 * ((2 * kk + hi) ^ f));
  }
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) settle(qf[kk]);
  __syncthreads();  // every wave holds its Q before the loop overwrites the second stage
  const bool strip_live = wq0_u < doc_end;
  const int ph = __builtin_amdgcn_readfirstlane(phase);
  for (int p = 0; p < n_quads; ++p) {
    const int stage = p & 1;
    const int kv0 = doc_start + 32 * (4 * p + ph);
    const lds_u16* kb = smem + stage * PAIR + (ph >> 1) * 2 * TILE + 32 * (ph & 1) * D;
    if (strip_live && kv0 < kv_end && kv0 <= wq0_u + 31) {
      f32x16 s;
      s_blk(kb, s);
      if (p + 1 < n_quads) copy_quad(p + 1, stage ^ 1);
      pv_blk(kb + TILE, kv0, s);
    } else if (p + 1 < n_quads) {
      copy_quad(p + 1, stage ^ 1);
    }
    wait_vmcnt<0>();  // this wave's copies of the next quad have landed in LDS
    __syncthreads();
  }

  // Merge of the four phases of each strip (the stages are free after the last barrier): phase
  // j sends its partial O of the other phases' columns (16-byte chunks, same lane order) and
  // publishes (m, l); phase J then finishes d in [32 J, 32 J + 32), the phases' terms added in
  // phase order.
  lds_f32x4* xo = reinterpret_cast<lds_f32x4*>((__attribute__((address_space(3))) float*)(smem));
  constexpr int kSlots = 2 * 4 * 3 * 4 * 64;  // [strip][dst][src, dst left out][j4][lane]
  float* xs = reinterpret_cast<float*>(smem_raw) + kSlots * 4;  // [strip][phase][m | l][lane]
  static_assert((kSlots * 4 + 2 * 4 * 2 * 64) * 4 <= 2 * PAIR * 2, "narrow merge fits in LDS");
  auto xslot = [&](int dst, int from, int j4) {
    return (((strip * 4 + dst) * 3 + from - (from > dst ? 1 : 0)) * 4 + j4) * 64 + lane;
  };
  auto merge = [&](auto phase_c) {
    constexpr int J = decltype(phase_c)::value;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      if (db == J) continue;
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4)
        xo[xslot(db, J, j4)] = f32x4{oacc[db][4 * j4], oacc[db][4 * j4 + 1],
                                     oacc[db][4 * j4 + 2], oacc[db][4 * j4 + 3]};
    }
    xs[((strip * 4 + J) * 2 + 0) * 64 + lane] = m_run;
    xs[((strip * 4 + J) * 2 + 1) * 64 + lane] = l_run;
    __syncthreads();
    float mk[4], lk[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      mk[f] = xs[((strip * 4 + f) * 2 + 0) * 64 + lane];
      lk[f] = xs[((strip * 4 + f) * 2 + 1) * 64 + lane];
    }
    const float m_tot = fmaxf(fmaxf(mk[0], mk[1]), fmaxf(mk[2], mk[3]));
    const float m_use = m_tot == -INFINITY ? 0.f : m_tot;
    float sk[4], lsum = 0.f;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      sk[f] = fast_exp2(mk[f] - m_use);
      lsum += lk[f] * sk[f];
    }
    const float l_tot = sum_with_other_half(lsum);
    const float inv = 1.f / l_tot;
    float x[16];
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const f32x4 y = f == J ? f32x4{oacc[J][4 * j4], oacc[J][4 * j4 + 1], oacc[J][4 * j4 + 2],
                                       oacc[J][4 * j4 + 3]}
                               : xo[xslot(J, f, j4)];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += y[e] * sk[f];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * j4 + e] = acc[e] * inv;
    }
    u32x4 w[2];  // chunk c: d = 32 J + 16 c + 8 hi + 0..7 of query wq0 + l32
#pragma unroll
    for (int c = 0; c < 2; ++c)
      w[c] = pack8<E>(x[8 * c], x[8 * c + 1], x[8 * c + 2], x[8 * c + 3], x[8 * c + 4],
                      x[8 * c + 5], x[8 * c + 6], x[8 * c + 7]);
    // Whole 64-byte row runs through this wave's own exchange slots (read above by this wave
    // only) as an LDS row tile.
    store_rows32<4>(reinterpret_cast<lds_u16*>(&xo[(strip * 4 + J) * 3 * 4 * 64]), w, lane,
                    [&](int r) { return o + (long)(wq0 + r) * qrow + h * D + 32 * J; },
                    doc_end - wq0);
    if (J == 0 && q_valid && hi == 0)
      __builtin_nontemporal_store((m_tot + fast_log2(l_tot)) * kLn2, &lse[(long)h * n_tokens + my_q]);
  };
  switch (ph) {
    case 0: merge(std::integral_constant<int, 0>{}); break;
    case 1: merge(std::integral_constant<int, 1>{}); break;
    case 2: merge(std::integral_constant<int, 2>{}); break;
    default: merge(std::integral_constant<int, 3>{}); break;
  }
}

template <class E>
// Arguments in the order the work-group needs them: the first 14 dwords are preloaded into
// SGPRs at launch (-amdgpu-kernarg-preload-count), so the work item's load starts at once.
__global__ __launch_bounds__(fwd::NT, 1) void fwd_kernel(
    const int4* __restrict__ items, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int hq, int hkv,
    uint16_t* __restrict__ o, float* __restrict__ lse, int n_tokens, float scale_log2) {
  using namespace fwd;
  __shared__ __attribute__((aligned(16))) uint16_t smem_raw[2 * PAIR];
  lds_u16* smem = (lds_u16*)smem_raw;

  const int4 it = items[blockIdx.x];
  const int q0 = it.x, doc_end = it.y, doc_start = it.z, h = it.w & kItemHeadMask;
  // Empty slots of a device-built plan, and items that do not fit this launch (a plan built for
  // other sizes), are skipped: nothing outside [0, n_tokens) x [0, hq) is ever addressed.
  if ((it.w & ~(kItemHeadMask | kItemNarrowBit)) != 0 || q0 >= doc_end || doc_start < 0 ||
      q0 < doc_start || doc_end > n_tokens || h >= hq)
    return;
  if ((it.w & kItemNarrowBit) != 0) {
    fwd_narrow_item<E>(smem, smem_raw, q0, doc_end, doc_start, h, q, k, v, hq, hkv, o, lse,
                       n_tokens, scale_log2);
    return;
  }
  const int group = hq / hkv;
  const int kvh = h / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int half = wave / NS, strip = wave % NS;
  const int src = lane & 15, grp = lane >> 4;   // transposed-read group and source lane
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;

  const int wq0 = q0 + 32 * strip;
  const int my_q = wq0 + l32;
  const bool q_valid = my_q < doc_end;

  u32x4 qf[8];  // Q fragment: B operand of S^T = K Q^T (filled from LDS before the loop)

  const int kv_end = min(q0 + BM, doc_end);
  const int n_tiles = (kv_end - doc_start + BN - 1) / BN;
  const int n_pairs = (n_tiles + 1) / 2;

  // Copy of one tile pair straight from HBM into LDS (buffer loads that write LDS, no staging
  // registers): one instruction moves 4 rows (a row group) of a tile (K0, V0, K1, V1); lane i
  // lands in chunk slot i & 15 of row i >> 4 of the group, so it fetches logical chunk
  // (i & 15) ^ swz16(row). Loads are bounded at the document end: rows past it read as zeros
  // (masked keys, zero P).
  // One half copies (half 1 the first pair, half 0 the others): a copy instruction stalls its
  // wave on the memory queue until the CU takes it. Wave (h, s) moves row groups g = 2 s + j and
  // 2 (s + 4) + j (j = 0, 1) of each tile, 4 rows per instruction.
  const int ws = __builtin_amdgcn_readfirstlane(strip);
  int coff[4];  // [jj]: bytes from the tile's first row, row group 2 (s + 4 (jj >> 1)) + (jj & 1)
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int r = 4 * (2 * (strip + 4 * (jj >> 1)) + (jj & 1)) + (lane >> 4);
    coff[jj] = (r * (int)kvrow + 8 * ((lane & 15) ^ swz16(r))) * 2;
  }
  // Copy of key tile `t` of tensor x (K, V) into the tile slot at LDS byte address `dst`.
  auto copy_tile = [&](int t, int x, uint32_t dst) {
    const int row0 = doc_start + t * BN;
    const long base = (long)row0 * kvrow + kvh * D;
    const long bytes = ((long)(doc_end - row0 - 1) * kvrow + D) * 2;
    const u32x4 r = make_rsrc4((x ? v : k) + base, bytes);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      dma16_opaque(r, dst + ((8 * (ws + 4 * (jj >> 1)) + 4 * (jj & 1)) * D) * 2, coff[jj]);
  };
  // The stage of pair p holds K0, V0, V1 of the pair and K1 of the NEXT pair (slots K0, V0, K1,
  // V1): half 1 computes S^T of its next tile at the end of a pair, after its O^T += V^T P^T, so
  // that at the start of the following pair its softmax (VALU) runs while half 0 computes its S^T
  // (MFMA) on the same SIMD. The K1 copy is left out when that tile does not exist.
  // In the loop, half 0 issues the copies of the next pair, after its S^T MFMAs: the copy
  // instructions stall the issuing wave while the CU takes 64 KB per pair (~1,100 cycles at the
  // CU's fill rate), and half 0 has that slack (half 1 carries the S^T of the next tile).
  auto copy_pair = [&](int p, int stage) {
    const uint32_t dst = lds_addr(smem + stage * PAIR);
    copy_tile(2 * p, 0, dst);
    copy_tile(2 * p, 1, dst + TILE * 2);
    copy_tile(2 * p + 1, 1, dst + 3 * TILE * 2);
    if (2 * p + 3 < n_tiles) copy_tile(2 * p + 3, 0, dst + 2 * TILE * 2);
  };

  // Per-lane LDS read offsets (halfs) inside a tile. K (A operand of S^T): row perm32(l32)
  // (+32 b), logical chunk 2 kk + hi. V^T (transposed reads): row 8 hi + 2 (src >> 2) + e
  // (+16 c + 32 b), logical column 16 (grp & 1) + 32 db + 4 sg, sg the column order that keeps
  // output registers d-contiguous. Adding 16 c + 32 b to a row keeps its swizzle.
  int koff[8], toff[4][2];
  {
    const int r = perm32(l32), f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = r * D + 8 * ((2 * kk + hi) ^ f);
    const int sg = (((src & 3) & 1) << 1) | ((src & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int rr = 8 * hi + 2 * (src >> 2) + e;
        const int lc = 2 * (grp & 1) + 4 * db + (sg >> 1);
        toff[db][e] = rr * D + 8 * (lc ^ swz16(rr)) + 4 * (sg & 1);
      }
  }

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  // S^T of one 64-key tile (K at `kb`): 16 MFMAs over (kk, b), each K operand read from LDS 4
  // MFMAs ahead of its use.
  auto s_tile = [&](const lds_u16* kb, f32x16(&s)[2]) {
    s[0] = f32x16{};
    s[1] = f32x16{};
    u32x4 ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = ld128(kb + koff[i >> 1] + 32 * (i & 1) * D);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = i >> 1, b = i & 1;
      s[b] = E::mfma(ka[i & 3], qf[kk], s[b]);
      if (i + 4 < 16) ka[i & 3] = ld128(kb + koff[(i + 4) >> 1] + 32 * ((i + 4) & 1) * D);
    }
    VA_SCHED(kSchedDsRead, 4);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      VA_SCHED(kSchedMfma, 1);
      VA_SCHED(kSchedDsRead, 1);
    }
    VA_SCHED(kSchedMfma, 4);
  };
  // The rest of a tile for this wave: mask, online softmax, O^T += V^T P^T (V of the tile in the
  // stage's V slot of this half).
  auto pv_tile = [&](int stage, int t, f32x16(&s)[2]) {
    const int kv0 = doc_start + t * BN;
    // The first V^T operands of O^T += V^T P^T, read while the softmax runs.
    const lds_u16* vb = smem + stage * PAIR + (2 * half + 1) * TILE;
    auto v_read = [&](int i) {  // i = (b, c, db) in MFMA order
      const int b = i >> 3, c = (i >> 2) & 1, db = i & 3;
      const lds_u16* p = vb + (32 * b + 16 * c) * D;
      const u32x2 x = ldtr(p + toff[db][0]), y = ldtr(p + toff[db][1]);
      return u32x4{x[0], x[1], y[0], y[1]};
    };
    u32x4 va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = v_read(i);
    if (kv0 + BN - 1 > wq0) {  // the tile crosses this strip's diagonal: key > query -> -inf
      const int lim = my_q - kv0;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (32 * b + reg_row(j, hi) > lim) s[b][j] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) mt = fmaxf(mt, s[b][j]);
    mt = max_with_other_half(mt) * scale_log2;
    // The reference maximum m_run moves only when some lane's tile maximum exceeds it by more
    // than kRescaleLog2 (always on the first tile): P values then stay below 2^kRescaleLog2 and
    // the O / l rescale is skipped on most tiles. When it moves, every lane takes its exact
    // running maximum.
    if (__builtin_amdgcn_ballot_w64(mt > m_run + kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;  // a lane with no visible key yet
    float rs = 0.f;
    u32x4 pf[2][2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(s[b][8 * c + e], scale_log2, -m_use));
        pf[b][c] = pack8_tr<E>(p);
#pragma unroll
        for (int w = 0; w < 4; ++w) rs = E::sum2(pf[b][c][w], rs);
      }
    l_run += rs;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = i >> 3, c = (i >> 2) & 1, db = i & 3;
      oacc[db] = E::mfma(va[i & 3], pf[b][c], oacc[db]);
      if (i + 4 < 16) va[i & 3] = v_read(i + 4);
    }
  };

  // The two waves of a SIMD come from different halves; the younger one (half 1) would otherwise
  // lose every issue tie and finish each pair last, keeping the others at the barrier.
  if (half) __builtin_amdgcn_s_setprio(1);
  // Q of the item's 128 queries, copied straight into the second LDS stage (free until the loop
  // copies the second tile pair) as swizzled 256-byte rows, by the waves of half 0 while half 1
  // copies the first tile pair: wave (0, s) moves its strip's rows 32 s .. 32 s + 31, 4 per
  // instruction. Rows past the document end read as zeros. Each lane then reads its query's row
  // as the B operand of S^T = K Q^T (column = this lane's query, k slots = d).
  static_assert(BM * D <= PAIR, "the Q tile fits in one stage");
  if (half == 0) {
    const long bytes = ((long)(doc_end - q0 - 1) * qrow + (long)(h + 1) * D) * 2;
    const u32x4 rq = make_rsrc4(q + (long)q0 * qrow, bytes);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 32 * strip + 4 * j + (lane >> 4);
      dma16_opaque(rq, lds_addr(smem + PAIR + (32 * ws + 4 * j) * D),
                   (r * (int)qrow + h * D + 8 * ((lane & 15) ^ swz16(r))) * 2);
    }
  }
  if (half == 1) copy_pair(0, 0);
  if (half == 1 && 1 < n_tiles) copy_tile(1, 0, lds_addr(smem + PAIR + 2 * TILE));
  wait_vmcnt<0>();
  __syncthreads();
  {
    const int r = 32 * strip + l32, f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = ld128(smem + PAIR + r * D + 8 * ((2 * kk + hi) ^ f));
  }
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) settle(qf[kk]);
  // Tiles entirely past this strip's diagonal are skipped (their P would be all zero).
  // (wave-uniform: the strip's first query through readfirstlane, so the branches are scalar)
  const int wq0_u = __builtin_amdgcn_readfirstlane(wq0);
  auto visible = [&](int t) { return t < n_tiles && doc_start + t * BN <= wq0_u + 31; };
  // The halves run separate loops (same barriers), so that half 1's S^T carried across a
  // barrier takes no registers in half 0's loop.
  if (half == 0) {
    __syncthreads();  // every wave holds its Q before the loop overwrites the second stage
    for (int p = 0; p < n_pairs; ++p) {
      const int stage = p & 1;
      const int t = 2 * p;
      if (visible(t)) {
        f32x16 s[2];
        s_tile(smem + stage * PAIR, s);
        if (p + 1 < n_pairs) copy_pair(p + 1, stage ^ 1);
        pv_tile(stage, t, s);
      } else if (p + 1 < n_pairs) {
        copy_pair(p + 1, stage ^ 1);
      }
      wait_vmcnt<0>();  // this wave's copies of the next pair have landed in LDS
      __syncthreads();
    }
  } else {
    f32x16 s[2];
    if (visible(1)) s_tile(smem + PAIR + 2 * TILE, s);
    __syncthreads();  // every wave holds its Q, half 1 its first S^T, before stage 1 is reused
    for (int p = 0; p < n_pairs; ++p) {
      const int stage = p & 1;
      const int t = 2 * p + 1;
      if (visible(t)) pv_tile(stage, t, s);
      if (visible(t + 2)) s_tile(smem + stage * PAIR + 2 * TILE, s);  // K1 of pair p + 1
      __syncthreads();
    }
  }

  // Merge the two halves through LDS (same lane order: the partner wave holds the same (query,
  // d) registers). Each half finishes half of the d columns: half h sends its partial O of the
  // other half's columns, 16-byte chunks, and both publish (m, l).
  lds_f32x4* xo = reinterpret_cast<lds_f32x4*>((__attribute__((address_space(3))) float*)(smem_raw));
  float* xs = reinterpret_cast<float*>(smem_raw) + NS * 2 * 2 * 4 * 64 * 4;  // [strip][half][m|l][lane]
  static_assert((NS * 2 * 2 * 4 * 64 * 4 + NS * 2 * 2 * 64) * 4 <= 2 * PAIR * 2, "merge fits in LDS");
  auto slot = [&](int dst_half, int db2, int j4) {
    return (((strip * 2 + dst_half) * 2 + db2) * 4 + j4) * 64 + lane;
  };
  // Accumulator indices must be compile-time constants (a runtime index would move oacc to
  // scratch memory): the half is a template constant in each branch.
  auto merge = [&](auto half_c) {
    constexpr int H = decltype(half_c)::value;
#pragma unroll
    for (int db2 = 0; db2 < 2; ++db2) {
      const int db = 2 * (H ^ 1) + db2;  // the partner's columns
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4)
        xo[slot(H ^ 1, db2, j4)] = f32x4{oacc[db][4 * j4], oacc[db][4 * j4 + 1],
                                         oacc[db][4 * j4 + 2], oacc[db][4 * j4 + 3]};
    }
    xs[((strip * 2 + H) * 2 + 0) * 64 + lane] = m_run;
    xs[((strip * 2 + H) * 2 + 1) * 64 + lane] = l_run;
    __syncthreads();
    const float m_b = xs[((strip * 2 + (H ^ 1)) * 2 + 0) * 64 + lane];
    const float l_b = xs[((strip * 2 + (H ^ 1)) * 2 + 1) * 64 + lane];
    const float m_tot = fmaxf(m_run, m_b);
    const float m_use = m_tot == -INFINITY ? 0.f : m_tot;
    const float sa = fast_exp2(m_run - m_use), sb = fast_exp2(m_b - m_use);
    const float l_tot = sum_with_other_half(l_run * sa + l_b * sb);
    const float inv = 1.f / l_tot;
    const float ca = sa * inv, cb = sb * inv;
    u32x4 w[4];  // chunk 2 db2 + c: d = 64 H + 32 db2 + 16 c + 8 hi + 0..7 of query wq0 + l32
#pragma unroll
    for (int db2 = 0; db2 < 2; ++db2) {
      const int db = 2 * H + db2;
      float x[16];
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 y = xo[slot(H, db2, j4)];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * j4 + e] = oacc[db][4 * j4 + e] * ca + y[e] * cb;
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
        w[2 * db2 + c] = pack8<E>(x[8 * c], x[8 * c + 1], x[8 * c + 2], x[8 * c + 3],
                                  x[8 * c + 4], x[8 * c + 5], x[8 * c + 6], x[8 * c + 7]);
    }
    // Whole 128-byte row halves through this wave's own exchange slot (read above by this wave
    // only) as an LDS row tile.
    store_rows32<8>(reinterpret_cast<lds_u16*>(&xo[slot(H, 0, 0) - lane]), w, lane,
                    [&](int r) { return o + (long)(wq0 + r) * qrow + h * D + 64 * H; },
                    doc_end - wq0);
    if (!q_valid) return;
    if (H == 0 && hi == 0)
      __builtin_nontemporal_store((m_tot + fast_log2(l_tot)) * kLn2, &lse[(long)h * n_tokens + my_q]);
  };
  if (half) merge(std::integral_constant<int, 1>{});
  else merge(std::integral_constant<int, 0>{});
}

// --------------------------------------------------------------------------------------------
// Forward for many work items: 4 waves per work item (one per query strip, each over all of the
// item's key tiles), 64 KB of LDS, so two work-groups share a CU. The two waves of a SIMD then
// come from different work items with their own barriers: one's MFMAs overlap the other's
// softmax without any phase arrangement, one item's start (loads) and end (stores) overlap the
// other's tiles, and no item merges halves at its end. Used when the plan has enough items to
// give every CU two (kFwdLeanMinItems).
// --------------------------------------------------------------------------------------------
namespace fwdl {
constexpr int NW = fwd::NS;     // waves = query strips
constexpr int NT = NW * 64;
constexpr int BN = fwd::BN, D = fwd::D, TILE = fwd::TILE;
constexpr int STAGE = 2 * TILE;  // K, V of one 64-key tile
constexpr int BM = fwd::BM;
static_assert(BM * D <= STAGE, "the Q tile fits in one stage");
}  // namespace fwdl

template <class E>
__global__ __launch_bounds__(fwdl::NT, 2) void fwd_lean_kernel(
    const int4* __restrict__ items, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int hq, int hkv,
    uint16_t* __restrict__ o, float* __restrict__ lse, int n_tokens, float scale_log2) {
  using namespace fwdl;
  __shared__ __attribute__((aligned(16))) uint16_t smem_raw[2 * STAGE];
  lds_u16* smem = (lds_u16*)smem_raw;

  const int4 it = items[blockIdx.x];
  const int q0 = it.x, doc_end = it.y, doc_start = it.z, h = it.w & kItemHeadMask;
  if ((it.w & ~(kItemHeadMask | kItemNarrowBit)) != 0 || q0 >= doc_end || doc_start < 0 ||
      q0 < doc_start || doc_end > n_tokens || h >= hq)
    return;
  // A narrow item's 64 queries are strips 0 and 1 (strips 2 and 3 only copy and meet the
  // barriers); q_end bounds the item's queries and keys.
  const int q_end = min(q0 + ((it.w & kItemNarrowBit) != 0 ? BM / 2 : BM), doc_end);
  const int group = hq / hkv;
  const int kvh = h / group;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
  const int strip = wave;
  const int src = lane & 15, grp = lane >> 4;
  const long qrow = (long)hq * D, kvrow = (long)hkv * D;
  const int wq0 = q0 + 32 * strip;
  const int my_q = wq0 + l32;
  const bool q_valid = my_q < q_end;
  const int ws = __builtin_amdgcn_readfirstlane(strip);
  const int wq0_u = __builtin_amdgcn_readfirstlane(wq0);

  const int kv_end = q_end;
  const int n_tiles = (kv_end - doc_start + BN - 1) / BN;

  // Copy of tile t (K and V) into a stage: wave s moves row groups 4 s .. 4 s + 3 (4 rows each)
  // of both tensors, 8 instructions; lane i lands in chunk slot i & 15 of row i >> 4 of the group
  // and fetches logical chunk (i & 15) ^ swz16(row). Rows past the document end read as zeros.
  int coff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * (4 * strip + j) + (lane >> 4);
    coff[j] = (r * (int)kvrow + 8 * ((lane & 15) ^ swz16(r))) * 2;
  }
  auto copy_tile = [&](int t, int stage) {
    const int row0 = doc_start + t * BN;
    const long base = (long)row0 * kvrow + kvh * D;
    const long bytes = ((long)(doc_end - row0 - 1) * kvrow + D) * 2;
    const uint32_t dst = lds_addr(smem + stage * STAGE);
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const u32x4 r = make_rsrc4((x ? v : k) + base, bytes);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dma16_opaque(r, dst + (x * TILE + 4 * (4 * ws + j) * D) * 2, coff[j]);
    }
  };

  int koff[8], toff[4][2];
  {
    const int r = perm32(l32), f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = r * D + 8 * ((2 * kk + hi) ^ f);
    const int sg = (((src & 3) & 1) << 1) | ((src & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int rr = 8 * hi + 2 * (src >> 2) + e;
        const int lc = 2 * (grp & 1) + 4 * db + (sg >> 1);
        toff[db][e] = rr * D + 8 * (lc ^ swz16(rr)) + 4 * (sg & 1);
      }
  }

  u32x4 qf[8];
  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  // S^T of one 64-key tile (K at `kb`): 16 MFMAs, each K operand read 4 MFMAs ahead.
  auto s_tile = [&](const lds_u16* kb, f32x16(&s)[2]) {
    s[0] = f32x16{};
    s[1] = f32x16{};
    u32x4 ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = ld128(kb + koff[i >> 1] + 32 * (i & 1) * D);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = i >> 1, b = i & 1;
      s[b] = E::mfma(ka[i & 3], qf[kk], s[b]);
      if (i + 4 < 16) ka[i & 3] = ld128(kb + koff[(i + 4) >> 1] + 32 * ((i + 4) & 1) * D);
    }
    VA_SCHED(kSchedDsRead, 4);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      VA_SCHED(kSchedMfma, 1);
      VA_SCHED(kSchedDsRead, 1);
    }
    VA_SCHED(kSchedMfma, 4);
  };
  // Mask, online softmax and O^T += V^T P^T of tile t (V at `vb`), as in the two-half kernel.
  auto pv_tile = [&](const lds_u16* vb, int t, f32x16(&s)[2]) {
    const int kv0 = doc_start + t * BN;
    auto v_read = [&](int i) {
      const int b = i >> 3, c = (i >> 2) & 1, db = i & 3;
      const lds_u16* p = vb + (32 * b + 16 * c) * D;
      const u32x2 x = ldtr(p + toff[db][0]), y = ldtr(p + toff[db][1]);
      return u32x4{x[0], x[1], y[0], y[1]};
    };
    u32x4 va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = v_read(i);
    if (kv0 + BN - 1 > wq0_u) {
      const int lim = my_q - kv0;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (32 * b + reg_row(j, hi) > lim) s[b][j] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) mt = fmaxf(mt, s[b][j]);
    mt = max_with_other_half(mt) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(mt > m_run + fwd::kRescaleLog2)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float rs = 0.f;
    u32x4 pf[2][2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(s[b][8 * c + e], scale_log2, -m_use));
        pf[b][c] = pack8_tr<E>(p);
#pragma unroll
        for (int w = 0; w < 4; ++w) rs = E::sum2(pf[b][c][w], rs);
      }
    l_run += rs;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = i >> 3, c = (i >> 2) & 1, db = i & 3;
      oacc[db] = E::mfma(va[i & 3], pf[b][c], oacc[db]);
      if (i + 4 < 16) va[i & 3] = v_read(i + 4);
    }
  };

  // Q (32 KB) into the second stage, tile 0 into the first; every lane reads its query's row.
  {
    const long bytes = ((long)(doc_end - q0 - 1) * qrow + (long)(h + 1) * D) * 2;
    const u32x4 rq = make_rsrc4(q + (long)q0 * qrow, bytes);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 32 * strip + 4 * j + (lane >> 4);
      dma16_opaque(rq, lds_addr(smem + STAGE + (32 * ws + 4 * j) * D),
                   (r * (int)qrow + h * D + 8 * ((lane & 15) ^ swz16(r))) * 2);
    }
  }
  copy_tile(0, 0);
  wait_vmcnt<0>();
  __syncthreads();
  {
    const int r = 32 * strip + l32, f = swz16(r);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = ld128(smem + STAGE + r * D + 8 * ((2 * kk + hi) ^ f));
  }
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) settle(qf[kk]);
  __syncthreads();  // every wave holds its Q before the loop overwrites the second stage
  // A strip past the document's end (the last item of a document whose length is not a multiple
  // of 128) has no query to compute: its wave only copies and meets the barriers, and leaves its
  // SIMD to the other work-group's wave.
  const bool strip_live = wq0_u < q_end;
  auto visible = [&](int t) { return strip_live && doc_start + t * BN <= wq0_u + 31; };
  for (int t = 0; t < n_tiles; ++t) {
    const int stage = t & 1;
    // The next tile's copies go out after this tile's S^T MFMAs (the wave waits for S anyway).
    if (visible(t)) {
      f32x16 s[2];
      s_tile(smem + stage * STAGE, s);
      if (t + 1 < n_tiles) copy_tile(t + 1, stage ^ 1);
      pv_tile(smem + stage * STAGE + TILE, t, s);
    } else if (t + 1 < n_tiles) {
      copy_tile(t + 1, stage ^ 1);
    }
    wait_vmcnt<0>();  // this wave's copies of the next tile have landed in LDS
    __syncthreads();
  }

  // O = O^T / l per query, written as whole 256-byte rows through this wave's own LDS row tile
  // (the stages are free after the last barrier); lse = (m + log2 l) ln 2.
  const float l_tot = sum_with_other_half(l_run);
  const float inv = 1.f / l_tot;
  u32x4 w[8];  // chunk 2 db + c: d = 32 db + 16 c + 8 hi + 0..7 of query wq0 + l32
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int c = 0; c < 2; ++c)
      w[2 * db + c] = pack8<E>(oacc[db][8 * c] * inv, oacc[db][8 * c + 1] * inv,
                               oacc[db][8 * c + 2] * inv, oacc[db][8 * c + 3] * inv,
                               oacc[db][8 * c + 4] * inv, oacc[db][8 * c + 5] * inv,
                               oacc[db][8 * c + 6] * inv, oacc[db][8 * c + 7] * inv);
  static_assert(NW * 32 * (8 * 16 + 8) * 2 <= 2 * STAGE * 2, "row tiles fit in LDS");
  store_rows32<16>(smem + strip * 32 * (8 * 16 + 8), w, lane,
                   [&](int r) { return o + (long)(wq0 + r) * qrow + h * D; }, q_end - wq0);
  if (q_valid && hi == 0) {
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    __builtin_nontemporal_store((m_use + fast_log2(l_tot)) * kLn2, &lse[(long)h * n_tokens + my_q]);
  }
}

template <class E>
static hipError_t launch_fwd_t(const FwdArgs& a) {
  if (a.n_items == 0) return hipSuccess;
  if (a.kernel == 2) {
    hipLaunchKernelGGL((fwd_lean_kernel<E>), dim3((unsigned)a.n_items), dim3(fwdl::NT), 0,
                       a.stream, (const int4*)a.items, (const uint16_t*)a.q, (const uint16_t*)a.k,
                       (const uint16_t*)a.v, a.hq, a.hkv, (uint16_t*)a.out, a.lse,
                       (int)a.n_tokens, a.scale * kLog2e);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((fwd_kernel<E>), dim3((unsigned)a.n_items), dim3(fwd::NT), 0, a.stream,
                     (const int4*)a.items, (const uint16_t*)a.q, (const uint16_t*)a.k,
                     (const uint16_t*)a.v, a.hq, a.hkv, (uint16_t*)a.out, a.lse, (int)a.n_tokens,
                     a.scale * kLog2e);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdArgs& a) {
  return a.dtype == 0 ? launch_fwd_t<F16>(a) : launch_fwd_t<BF16>(a);
}

}  // namespace va
