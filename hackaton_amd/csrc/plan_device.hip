// Work plans built on the device, for callers whose document lengths are only on the GPU: no host
// read, so no stream synchronisation (the reference reads them back with lengths.tolist() at
// solution/packed.py:170-172).
//
// One launch, one 1024-thread work-group per plan kind (forward, backward). Each work-group takes
// the document bounds (from a device cu_seqlens, or from device lengths through a saturating
// prefix sum), clamps them into [0, n_tokens], makes them non-decreasing and ends the last
// document at n_tokens (rows past the lengths' sum join it); counts each
// document's tiles and prefix-sums the counts in LDS; sorts the tile candidates by the host
// planner's work measure (counting sort, buckets of 8), longest first; and writes one item per
// (candidate, query head) in the host planner's XCD layout: every candidate is Hkv combos (one
// per GQA group), combos are dealt 8 at a time as the columns of a G x 8 block, so that the G
// heads of a group run on one XCD and share its L2. Candidates inside a bucket come in atomic
// order: every item is computed on its own, so the order changes no result. Each plan is
// `capacity` items long; slots past the real items hold empty items that the attention kernels
// skip at once.
#include <climits>

#include "../../include/varlen_attn.h"
#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace {

constexpr int PT = 1024;           // threads of a planning work-group
constexpr int kBuckets = 4096;     // work buckets of 8
constexpr int kTile = kFwdBlockM;  // rows of a forward query tile, a kv key tile, a q query tile
constexpr int kXcds = 8;           // work-group i runs on XCD i mod 8
static_assert(kBwdBlockN == kTile && kBwdBlockM == kTile, "one tile size for every item kind");
constexpr int DPB = (kPlanMaxDocs + 1 + PT - 1) / PT;  // document bounds per thread
constexpr int BPT = kBuckets / PT;                      // buckets per thread

__device__ inline int tiles_of(int len) { return len <= 0 ? 0 : (len + kTile - 1) / kTile; }

// Inclusive block scan of one value per thread (Hillis-Steele over LDS): sum, max or sum
// saturated at `cap` (values in [0, cap], cap < 2^31, so no partial sum overflows 64 bits).
enum { kScanSum, kScanMax, kScanSatSum };
template <int kOp>
__device__ long long block_scan(long long x, long long* buf, long long cap = 0) {
  const int t = threadIdx.x;
  buf[t] = x;
  __syncthreads();
  for (int off = 1; off < PT; off <<= 1) {
    const long long y = t >= off ? buf[t - off] : (kOp == kScanMax ? LLONG_MIN : 0);
    __syncthreads();
    long long r;
    if (kOp == kScanMax) r = max(buf[t], y);
    else if (kOp == kScanSum) r = buf[t] + y;
    else r = min(buf[t] + y, cap);
    buf[t] = r;
    __syncthreads();
  }
  const long long r = buf[t];
  __syncthreads();
  return r;
}

// At most one of `cu` (int32, n_docs + 1 bounds) and `lengths` (int64, n_docs) is non-null (both
// null only when n_docs is 0).
// Work-group 0 builds the forward plan, work-group 1 the backward plan; a null item pointer skips
// that kind. cu_out (when non-null) is written by work-group 0, or by work-group 1 when there is
// no forward plan.
__global__ __launch_bounds__(PT) void plan_kernel(const int32_t* __restrict__ cu,
                                                  const int64_t* __restrict__ lengths, int n_docs,
                                                  int n_tokens, int hq, int hkv,
                                                  int4* __restrict__ fwd_items, long fwd_capacity,
                                                  int4* __restrict__ bwd_items, long bwd_capacity,
                                                  int bwd_kind, int bwd_groups, int fwd_narrow,
                                                  int32_t* __restrict__ cu_out) {
  __shared__ int s_bound[kPlanMaxDocs + 1];  // clamped, non-decreasing document bounds
  __shared__ int s_tbase[kPlanMaxDocs + 1];  // exclusive prefix of the per-document tile counts
  __shared__ int s_mbase[kPlanMaxDocs + 1];  // exclusive prefix count of the longest documents
  __shared__ int s_cnt[kBuckets];
  __shared__ long long s_scan[PT];
  const int tid = threadIdx.x;
  const int kind = blockIdx.x == 0 ? VA_PLAN_FWD : VA_PLAN_BWD;
  int4* items = kind == VA_PLAN_FWD ? fwd_items : bwd_items;
  const long capacity = kind == VA_PLAN_FWD ? fwd_capacity : bwd_capacity;
  if (items == nullptr) return;  // uniform over the work-group
  const int group = hq / hkv;

  // Document bounds, DPB per thread.
  if (lengths != nullptr) {
    // bound_0 = 0, bound_d = min(sum of the first d lengths (each clamped into [0, N]), N)
    long long run[DPB];
    long long s = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;  // run[i] = sum of lengths[tid*DPB .. d - 1]
      run[i] = s;
      long long x = (d < n_docs) ? lengths[d] : 0;
      x = x < 0 ? 0 : (x > n_tokens ? n_tokens : x);
      s = min(s + x, (long long)n_tokens);
    }
    const long long incl = block_scan<kScanSatSum>(s, s_scan, n_tokens);
    const long long excl = tid > 0 ? s_scan[tid - 1] : 0;
    (void)incl;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d <= n_docs) s_bound[d] = (int)min(excl + run[i], (long long)n_tokens);
    }
  } else {
    // bound_d = max over d' <= d of min(max(cu[d'], 0), N)
    int run[DPB];
    int m = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      int x = (cu != nullptr && d <= n_docs) ? cu[d] : 0;  // no documents: both inputs null
      x = x < 0 ? 0 : (x > n_tokens ? n_tokens : x);
      m = max(m, x);
      run[i] = m;
    }
    block_scan<kScanMax>(m, s_scan);  // s_scan holds the inclusive prefix maxima
    const int prev = tid > 0 ? (int)s_scan[tid - 1] : 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d <= n_docs) s_bound[d] = max(prev, run[i]);
    }
  }
  // Every row belongs to a document: rows past the last bound (lengths summing below n_tokens)
  // join the last document, so no output or gradient row is left unwritten.
  __syncthreads();  // every bound written before the last one is replaced
  if (tid == 0 && n_docs > 0) s_bound[n_docs] = n_tokens;
  for (int b = tid; b < kBuckets; b += PT) s_cnt[b] = 0;
  __syncthreads();
  // cu_out comes from the forward's work-group, or from the backward's when no forward plan is
  // built (either item pointer may be null)
  if (cu_out != nullptr && (fwd_items != nullptr ? kind == VA_PLAN_FWD : kind == VA_PLAN_BWD))
    for (int d = tid; d <= n_docs; d += PT) cu_out[d] = s_bound[d];

  // Tile counts and their exclusive prefix sum (DPB documents per thread).
  {
    int cnt[DPB];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      cnt[i] = d < n_docs ? tiles_of(s_bound[d + 1] - s_bound[d]) : 0;
      sum += cnt[i];
    }
    const int incl = (int)block_scan<kScanSum>(sum, s_scan);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d <= n_docs) s_tbase[d] = run;
      run += cnt[i];
    }
  }
  __syncthreads();
  const int n_tiles = s_tbase[n_docs];
  // VA_PLAN_FWD_NARROW (plan.cpp's rule): the last tile of every document of the maximal length
  // splits into narrow 64-query items when (T + those documents) Hq <= 256 CUs; the second
  // halves (of last tiles over 64 queries) are the candidates n_tiles .. n_tiles + n_second - 1.
  int narrow_len = 0, n_second = 0;
  if (kind == VA_PLAN_FWD && fwd_narrow) {
    long long lmax = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d < n_docs) lmax = max(lmax, (long long)(s_bound[d + 1] - s_bound[d]));
    }
    block_scan<kScanMax>(lmax, s_scan);
    lmax = s_scan[PT - 1];
    __syncthreads();
    int cnt[DPB];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      cnt[i] = d < n_docs && lmax > 0 && s_bound[d + 1] - s_bound[d] == lmax;
      sum += cnt[i];
    }
    const int incl = (int)block_scan<kScanSum>(sum, s_scan);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d <= n_docs) s_mbase[d] = run;
      run += cnt[i];
    }
    __syncthreads();
    const int n_max = s_mbase[n_docs];
    if (lmax > 0 && (long long)(n_tiles + n_max) * hq <= kPlanCus) {
      narrow_len = (int)lmax;
      n_second = narrow_len - kTile * (tiles_of(narrow_len) - 1) > kTile / 2 ? n_max : 0;
    }
  }
  const int n_cand = kind == VA_PLAN_FWD ? n_tiles + n_second : 2 * n_tiles;
  // kv items of two heads each: the host planner's rule over the same tile count
  const bool pairs = kind == VA_PLAN_BWD && bwd_plan_pairs(n_tiles, hq, hkv, bwd_kind);

  // Candidate c -> (document, tile, is_q): kv tiles first, then q tiles (backward). Forward
  // candidates past the tiles are the second narrow halves (is_q = 1 marks them there), in the
  // order of their documents.
  auto decode = [&](int c, int& doc, int& t, int& is_q) {
    is_q = c >= n_tiles;
    const bool second = kind == VA_PLAN_FWD && is_q;
    const int ct = second ? c - n_tiles : (is_q ? c - n_tiles : c);
    const int* base = second ? s_mbase : s_tbase;
    int lo = 0, hi = n_docs - 1;  // last document with base <= ct
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (base[mid] <= ct) lo = mid;
      else hi = mid - 1;
    }
    doc = lo;
    t = second ? tiles_of(s_bound[lo + 1] - s_bound[lo]) - 1 : ct - s_tbase[lo];
  };
  // The host planner's work measures (plan.cpp): of a per-head item (w1) and of a pair item (w2)
  // of the candidate; `steps` the query steps of a kv candidate (0 for the others).
  auto works = [&](int doc, int t, int is_q, long& w1, long& w2, long& steps) {
    const long s = s_bound[doc], e = s_bound[doc + 1];
    steps = 0;
    if (kind == VA_PLAN_FWD) {
      w1 = w2 = min(s + (long)(t + 1) * kTile, e) - s;
    } else if (!is_q) {
      steps = (e - (s + (long)t * kTile) + kBwdBlockQ - 1) / kBwdBlockQ;
      w1 = (steps + 1) / 2 * 32 + kPlanKvItemCost;
      w2 = steps * 32 + kPlanKvItemCost;
    } else {
      const long kv_end = min(s + (long)(t + 1) * kTile, e);
      const long tiles = (kv_end - s + kBwdTileK - 1) / kBwdTileK;
      w1 = (tiles + 1) / 2 * 24 + kPlanQItemCost;
      w2 = (tiles + 1) / 2 * 48 + kPlanQItemCost;
    }
  };
  // Group plans: a kv candidate becomes G / S group items per GQA group, S the largest head count
  // whose item's work is at most the longest item of the list without groups, or that list's
  // work per CU (bwd_group_heads, as in plan.cpp).
  const bool groups = kind == VA_PLAN_BWD && bwd_groups != 0 && group >= 2;
  long long group_cap = -1;
  if (groups) {
    if (bwd_groups == 2) {
      group_cap = LLONG_MAX;
    } else {
      long long longest = 0, total = 0;
      for (int c = tid; c < n_cand; c += PT) {
        int doc, t, is_q;
        decode(c, doc, t, is_q);
        long w1, w2, steps;
        works(doc, t, is_q, w1, w2, steps);
        long per = 0;  // the candidate's items over one GQA group
        for (int r = 0; r < (pairs ? (group + 1) / 2 : group); ++r)
          per += (pairs && 2 * r + 1 < group) ? w2 : w1;
        longest = max(longest, (long long)(pairs ? w2 : w1));
        total += per * hkv;
      }
      block_scan<kScanMax>(longest, s_scan);
      longest = s_scan[PT - 1];
      __syncthreads();
      block_scan<kScanSum>(total, s_scan);
      total = s_scan[PT - 1];
      __syncthreads();
      group_cap = max(longest, total / kPlanCus);
    }
  }
  auto group_heads = [&](int doc, int t, int is_q) {  // S of the candidate's group items, or 0
    if (!groups || is_q) return 0;
    long w1, w2, steps;
    works(doc, t, is_q, w1, w2, steps);
    return bwd_group_heads(steps, group, group_cap, pairs);
  };
  // The work measure in buckets of 8.
  auto bucket = [&](int doc, int t, int is_q) {
    long w1, w2, steps;
    works(doc, t, is_q, w1, w2, steps);
    const int sub = group_heads(doc, t, is_q);
    const long work = sub > 0 ? bwd_group_work(steps, sub) : (pairs ? w2 : w1);
    const long b = work >> 3;
    return (int)(b >= kBuckets ? kBuckets - 1 : b);
  };

  for (int c = tid; c < n_cand; c += PT) {
    int doc, t, is_q;
    decode(c, doc, t, is_q);
    atomicAdd(&s_cnt[bucket(doc, t, is_q)], 1);
  }
  __syncthreads();
  // Bucket starts, longest first: start[b] = number of candidates in the buckets above b.
  {
    int cnt[BPT];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      cnt[i] = s_cnt[kBuckets - 1 - (tid * BPT + i)];
      tot += cnt[i];
    }
    const int incl = (int)block_scan<kScanSum>(tot, s_scan);
    int run = incl - tot;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      s_cnt[kBuckets - 1 - (tid * BPT + i)] = run;
      run += cnt[i];
    }
  }
  __syncthreads();
  // Candidate at sorted position `pos` holds combos pos * Hkv + g (g = GQA group); combo j sits
  // in column j % 8 of block j / 8, which spans 8 G slots (fewer columns in the last block);
  // head r of the group goes to row r. In a pair plan a combo's row r < ceil(G / 2) holds the
  // item of heads 2 r, 2 r + 1 (the last head of an odd group alone) and its other rows stay
  // empty items; a group candidate's combo holds its G / S group items (heads S r) in rows
  // r < G / S, empty items below.
  const long n_combos = (long)n_cand * hkv;
  for (int c = tid; c < n_cand; c += PT) {
    int doc, t, is_q;
    decode(c, doc, t, is_q);
    const long pos = atomicAdd(&s_cnt[bucket(doc, t, is_q)], 1);
    const int s = s_bound[doc], e = s_bound[doc + 1];
    const int sub = group_heads(doc, t, is_q);
    // a forward candidate's narrow items: the last tile of a longest document (is_q: its second
    // half, 64 queries on)
    const bool narrow = kind == VA_PLAN_FWD && narrow_len > 0 && e - s == narrow_len &&
                        t == tiles_of(narrow_len) - 1;
    const int q_first = s + t * kTile + (kind == VA_PLAN_FWD && is_q ? kTile / 2 : 0);
    const int fwd_bits = narrow ? kItemNarrowBit : 0;
    for (int g = 0; g < hkv; ++g) {
      const long combo = pos * hkv + g;
      const long blk = combo / kXcds, col = combo % kXcds;
      const long ncols = min((long)kXcds, n_combos - blk * kXcds);
      for (int r = 0; r < group; ++r) {
        const long slot = blk * kXcds * group + r * ncols + col;
        int4 item = kind == VA_PLAN_FWD ? int4{q_first, e, s, fwd_bits | (g * group + r)}
                                        : int4{s + t * kTile, e, s, (is_q << 24) | (g * group + r)};
        if (sub > 0) {
          item = r < group / sub
                     ? int4{s + t * kTile, e, s,
                            kItemGroupBit | ((sub - 1) << kItemHeadsShift) | (g * group + r * sub)}
                     : int4{0, 0, 0, 0};
        } else if (pairs) {
          const int h2 = 2 * r;
          item = h2 < group ? int4{s + t * kTile, e, s,
                                   (is_q << 24) | (h2 + 1 < group ? kItemPairBit : 0) |
                                       (g * group + h2)}
                            : int4{0, 0, 0, 0};
        }
        if (slot < capacity) items[slot] = item;
      }
    }
  }
  for (long slot = (long)n_cand * hq + tid; slot < capacity; slot += PT) items[slot] = int4{0, 0, 0, 0};
}

}  // namespace

hipError_t launch_plan_device(const int32_t* cu, const int64_t* lengths, int n_docs, int n_tokens,
                              int hq, int hkv, int32_t* fwd_items, long fwd_capacity,
                              int32_t* bwd_items, long bwd_capacity, int bwd_kind,
                              int bwd_groups, int fwd_narrow, int32_t* cu_out, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(2), dim3(PT), 0, stream, cu, lengths, n_docs, n_tokens, hq,
                     hkv, (int4*)fwd_items, fwd_capacity, (int4*)bwd_items, bwd_capacity,
                     bwd_kind, bwd_groups, fwd_narrow, cu_out);
  return hipGetLastError();
}

}  // namespace va
