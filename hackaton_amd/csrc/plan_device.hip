// Work plans built on the device from a device cu_seqlens, for callers whose document lengths are
// only on the GPU: no host read, so no stream synchronisation (the reference reads them back with
// lengths.tolist() at solution/packed.py:170-172).
//
// One work-group of 1024 threads: per-document tile counts and their prefix sum in LDS, then a
// counting sort of the tile candidates by work (the host planner's work measure, in buckets of 8)
// longest first, then one work item per (candidate, query head). Items inside a bucket come in
// atomic order: every item is computed on its own, so the order changes no result. The plan is
// `capacity` items long; slots past the real items hold empty items that the attention kernels
// skip at once. Document bounds are clamped into [0, n_tokens] and made non-decreasing, so that
// any cu_seqlens content yields in-bounds items.
#include <climits>

#include "../../include/varlen_attn.h"
#include "va_common.h"
#include "va_kernels.h"

namespace va {

namespace {

constexpr int PT = 1024;           // threads of the planning work-group
constexpr int kBuckets = 4096;     // work buckets of 8
constexpr int kTile = kFwdBlockM;  // rows of a forward query tile, a kv key tile, a q query tile
static_assert(kBwdBlockN == kTile && kBwdBlockM == kTile, "one tile size for every item kind");
constexpr int DPB = (kPlanMaxDocs + 1 + PT - 1) / PT;  // document bounds per thread
constexpr int BPT = kBuckets / PT;                      // buckets per thread

__device__ inline int tiles_of(int len) { return len <= 0 ? 0 : (len + kTile - 1) / kTile; }

// Inclusive block scan of one value per thread (Hillis-Steele over LDS): sum, or max.
template <bool kMax>
__device__ int block_scan(int x, int* buf) {
  const int t = threadIdx.x;
  buf[t] = x;
  __syncthreads();
  for (int off = 1; off < PT; off <<= 1) {
    const int y = t >= off ? buf[t - off] : (kMax ? INT_MIN : 0);
    __syncthreads();
    buf[t] = kMax ? max(buf[t], y) : buf[t] + y;
    __syncthreads();
  }
  const int r = buf[t];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(PT) void plan_kernel(const int32_t* __restrict__ cu, int n_docs,
                                                  int n_tokens, int hq, int kind,
                                                  int4* __restrict__ items, long capacity) {
  __shared__ int s_bound[kPlanMaxDocs + 1];  // clamped, non-decreasing document bounds
  __shared__ int s_tbase[kPlanMaxDocs + 1];  // exclusive prefix of the per-document tile counts
  __shared__ int s_cnt[kBuckets];
  __shared__ int s_scan[PT];
  const int tid = threadIdx.x;

  // bound_d = max over d' <= d of min(max(cu[d'], 0), n_tokens): thread runs of DPB bounds, then
  // a block max-scan of the run maxima.
  {
    int run[DPB];
    int m = 0;
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      int x = d <= n_docs ? cu[d] : 0;
      x = x < 0 ? 0 : (x > n_tokens ? n_tokens : x);
      m = max(m, x);
      run[i] = m;
    }
    block_scan<true>(m, s_scan);  // s_scan now holds the inclusive prefix maxima
    const int prev = tid > 0 ? s_scan[tid - 1] : 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < DPB; ++i) {
      const int d = tid * DPB + i;
      if (d <= n_docs) s_bound[d] = max(prev, run[i]);
    }
  }
  for (int b = tid; b < kBuckets; b += PT) s_cnt[b] = 0;
  __syncthreads();

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
    const int incl = block_scan<false>(sum, s_scan);
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
  const int n_cand = kind == VA_PLAN_FWD ? n_tiles : 2 * n_tiles;

  // Candidate c -> (document, tile, is_q): kv tiles first, then q tiles (backward).
  auto decode = [&](int c, int& doc, int& t, int& is_q) {
    is_q = c >= n_tiles;
    const int ct = is_q ? c - n_tiles : c;
    int lo = 0, hi = n_docs - 1;  // last document with tbase <= ct (it has tiles)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_tbase[mid] <= ct) lo = mid;
      else hi = mid - 1;
    }
    doc = lo;
    t = ct - s_tbase[lo];
  };
  // The host planner's work measures (plan.cpp), in buckets of 8.
  auto bucket = [&](int doc, int t, int is_q) {
    const long s = s_bound[doc], e = s_bound[doc + 1];
    long work;
    if (kind == VA_PLAN_FWD) {
      work = min(s + (long)(t + 1) * kTile, e) - s;
    } else if (!is_q) {
      const long steps = (e - (s + (long)t * kTile) + kBwdBlockQ - 1) / kBwdBlockQ;
      work = (steps + 1) / 2 * 32 + kPlanKvItemCost;
    } else {
      const long kv_end = min(s + (long)(t + 1) * kTile, e);
      const long tiles = (kv_end - s + kBwdTileK - 1) / kBwdTileK;
      work = (tiles + 1) / 2 * 24 + kPlanQItemCost;
    }
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
    const int incl = block_scan<false>(tot, s_scan);
    int run = incl - tot;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      s_cnt[kBuckets - 1 - (tid * BPT + i)] = run;
      run += cnt[i];
    }
  }
  __syncthreads();
  for (int c = tid; c < n_cand; c += PT) {
    int doc, t, is_q;
    decode(c, doc, t, is_q);
    const long pos = atomicAdd(&s_cnt[bucket(doc, t, is_q)], 1);
    const int s = s_bound[doc], e = s_bound[doc + 1];
    for (int h = 0; h < hq; ++h) {
      const long slot = pos * hq + h;
      if (slot < capacity) items[slot] = int4{s + t * kTile, e, s, (is_q << 24) | h};
    }
  }
  for (long slot = (long)n_cand * hq + tid; slot < capacity; slot += PT) items[slot] = int4{0, 0, 0, 0};
}

}  // namespace

hipError_t launch_plan_device(const int32_t* cu, int n_docs, int n_tokens, int hq, int kind,
                              int32_t* items, long capacity, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(PT), 0, stream, cu, n_docs, n_tokens, hq, kind,
                     (int4*)items, capacity);
  return hipGetLastError();
}

}  // namespace va
