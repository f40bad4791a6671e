// Host-side work planning for the varlen attention kernels (no GPU calls).
//
// The plan turns cu_seqlens into a list of work items, one per (tile, query head): tiles never
// cross a document boundary and never start past the causal diagonal, so fully masked causal
// tiles and cross-document tiles are never launched. Items are ordered by decreasing work
// (longest-processing-time first): the hardware dispatcher hands work-groups out in index order,
// so the longest tiles start first and the short ones fill the tail.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <vector>

#include "../../include/varlen_attn.h"
#include "va_api_internal.h"
#include "va_kernels.h"

namespace {

struct Item {
  int32_t a, b, c, d;
  int64_t work;
};

int check_cu(const int32_t* cu, int32_t n_docs) {
  if (n_docs < 0) return va::fail(VA_EINVAL, "n_docs < 0");
  if (cu == nullptr) return va::fail(VA_EINVAL, "cu_seqlens is NULL");
  if (cu[0] != 0) return va::fail(VA_ESEQ, "cu_seqlens[0] != 0");
  for (int32_t i = 0; i < n_docs; ++i) {
    if (cu[i + 1] < cu[i]) return va::fail(VA_ESEQ, "cu_seqlens decreases at %d", i);
  }
  return VA_OK;
}

int check_heads(int32_t hq, int32_t hkv) {
  if (hq <= 0 || hkv <= 0) return va::fail(VA_ESHAPE, "heads must be positive (%d, %d)", hq, hkv);
  if (hq % hkv != 0) return va::fail(VA_ESHAPE, "Hq=%d is not a multiple of Hkv=%d", hq, hkv);
  if (hq > 4096) return va::fail(VA_ESHAPE, "Hq=%d out of range", hq);
  return VA_OK;
}

constexpr int64_t kKvItemCost = va::kPlanKvItemCost;
constexpr int64_t kQItemCost = va::kPlanQItemCost;

bool is_plan_kind(int32_t kind) {
  return kind == VA_PLAN_FWD || kind == VA_PLAN_BWD || kind == VA_PLAN_BWD_HEADS ||
         kind == VA_PLAN_BWD_PAIRS || kind == VA_PLAN_BWD_GROUPS || kind == VA_PLAN_BWD_GROUPS_ALL ||
         kind == VA_PLAN_FWD_NARROW;
}
bool is_fwd_kind(int32_t kind) { return kind == VA_PLAN_FWD || kind == VA_PLAN_FWD_NARROW; }
bool is_group_kind(int32_t kind) {
  return kind == VA_PLAN_BWD_GROUPS || kind == VA_PLAN_BWD_GROUPS_ALL;
}
int32_t item_head(int32_t d) { return d & va::kItemHeadMask; }

// 128-row tiles of the documents (sum of ceil(length / 128); empty documents have none).
int64_t doc_tiles(const int32_t* cu, int32_t n_docs) {
  int64_t t = 0;
  for (int32_t i = 0; i < n_docs; ++i)
    if (cu[i + 1] > cu[i]) t += ((int64_t)cu[i + 1] - cu[i] + va::kBwdBlockN - 1) / va::kBwdBlockN;
  return t;
}

// VA_PLAN_FWD_NARROW: the length of the documents whose last 128-query tile is split into two
// narrow items, or 0. The split is taken when the list, split, still gives every item a CU of its
// own: a short list (configuration 2: 192 items on 256 CUs) is as long as its longest items
// (measured: without them the forward's span fell from 12.4 to 10.1 us), and a narrow item runs
// their key tiles in half the chain.
int32_t narrow_length(const int32_t* cu, int32_t n_docs, int32_t hq, int32_t kind) {
  if (kind != VA_PLAN_FWD_NARROW) return 0;
  int32_t longest = 0;
  int64_t count = 0;
  for (int32_t i = 0; i < n_docs; ++i) {
    const int32_t len = cu[i + 1] - cu[i];
    if (len > longest) {
      longest = len;
      count = 0;
    }
    if (len == longest && len > 0) ++count;
  }
  if (longest == 0 || (doc_tiles(cu, n_docs) + count) * hq > va::kPlanCus) return 0;
  return longest;
}

std::vector<Item> make_items(const int32_t* cu, int32_t n_docs, int32_t hq, int32_t hkv,
                             int32_t kind) {
  std::vector<Item> items;
  const bool pairs =
      !is_fwd_kind(kind) && va::bwd_plan_pairs(doc_tiles(cu, n_docs), hq, hkv, kind);
  const int32_t group = hq / hkv, rows = pairs ? (group + 1) / 2 : group;
  // Group plans: the largest group-item work that keeps the plan about as long as its VA_PLAN_BWD
  // form: that list's longest item, or its work per CU when that is more (measured at configs
  // 3-5: half the work per CU as the bound left config 4 7% slower, the longest item alone 8%;
  // 1.5x and 2x the work per CU made config 3 26% and 59% slower, every key tile at S = G 50%).
  int64_t group_cap = -1;
  if (is_group_kind(kind) && group >= 2) {
    if (kind == VA_PLAN_BWD_GROUPS_ALL) {
      group_cap = INT64_MAX;
    } else {
      int64_t longest = 0, total = 0;
      for (const Item& x : make_items(cu, n_docs, hq, hkv, VA_PLAN_BWD)) {
        longest = std::max(longest, x.work);
        total += x.work;
      }
      group_cap = std::max(longest, total / va::kPlanCus);
    }
  }
  const int32_t narrow = narrow_length(cu, n_docs, hq, kind);
  for (int32_t i = 0; i < n_docs; ++i) {
    const int32_t s = cu[i], e = cu[i + 1];
    if (e <= s) continue;
    if (is_fwd_kind(kind)) {
      for (int32_t q0 = s; q0 < e; q0 += va::kFwdBlockM) {
        const int32_t kv_end = std::min<int64_t>((int64_t)q0 + va::kFwdBlockM, e);
        const int64_t work = kv_end - s;  // keys visited by the tile
        if (e - s == narrow && kv_end == e) {  // the last tile of a longest document: split
          for (int32_t q1 = q0; q1 < e; q1 += va::kFwdBlockM / 2)
            for (int32_t h = 0; h < hq; ++h) items.push_back({q1, e, s, va::kItemNarrowBit | h, work});
          continue;
        }
        for (int32_t h = 0; h < hq; ++h) items.push_back({q0, e, s, h, work});
      }
    } else {
      // Work of a backward item: MFMAs per wave per step pair (kv items: 32 for each pair of
      // 32-query steps; q items: 24 for each pair of 32-key tiles) plus the item's fixed cost
      // (prologue and epilogue) in the same unit. Item durations measured in the benchmark's
      // graph at 4 x 512 tokens: ~2.4 us per kv step pair + ~3.0 us per kv item, ~1.9 us per q
      // tile pair + ~2.4 us per q item; hence 39 and 30. Without the fixed cost a kv item over
      // 384 queries (18.7 us) ties with a q item over 512 keys (17.3 us), and the XCD layout
      // below deals the heavier ones to the same XCDs in every block.
      // A pair item's halves each take one head over every step: twice a per-head item's steps.
      // A group item's halves take its S heads' steps in sequence, two per step pair; a key tile
      // takes the largest S whose item fits the cap (bwd_group_heads), G / S items per GQA group.
      for (int32_t k0 = s; k0 < e; k0 += va::kBwdBlockN) {
        const int64_t steps = ((int64_t)e - k0 + va::kBwdBlockQ - 1) / va::kBwdBlockQ;
        const int sub = group_cap >= 0 ? va::bwd_group_heads(steps, group, group_cap, pairs) : 0;
        if (sub > 0) {
          const int64_t work = va::bwd_group_work(steps, sub);
          for (int32_t g = 0; g < hkv; ++g)
            for (int32_t j = 0; j < group / sub; ++j)
              items.push_back({k0, e, s,
                               va::kItemGroupBit | ((sub - 1) << va::kItemHeadsShift) |
                                   (g * group + j * sub),
                               work});
          continue;
        }
        for (int32_t g = 0; g < hkv; ++g)
          for (int32_t r = 0; r < rows; ++r) {
            const bool pair = pairs && 2 * r + 1 < group;
            const int32_t h = g * group + (pairs ? 2 * r : r);
            const int64_t work = (pair ? steps : (steps + 1) / 2) * 32 + kKvItemCost;
            items.push_back({k0, e, s, (pair ? va::kItemPairBit : 0) | h, work});
          }
      }
      for (int32_t q0 = s; q0 < e; q0 += va::kBwdBlockM) {
        const int64_t kv_end = std::min<int64_t>((int64_t)q0 + va::kBwdBlockM, e);
        const int64_t tiles = (kv_end - s + va::kBwdTileK - 1) / va::kBwdTileK;
        for (int32_t g = 0; g < hkv; ++g)
          for (int32_t r = 0; r < rows; ++r) {
            const bool pair = pairs && 2 * r + 1 < group;
            const int32_t h = g * group + (pairs ? 2 * r : r);
            const int64_t work = (tiles + 1) / 2 * (pair ? 48 : 24) + kQItemCost;
            items.push_back({q0, e, s, (1 << 24) | (pair ? va::kItemPairBit : 0) | h, work});
          }
      }
    }
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& x, const Item& y) { return x.work > y.work; });
  return items;
}

// The dispatcher hands work-group i to XCD i mod kXcds, and each XCD has its own L2. The G query
// heads of a GQA group read the same K/V tiles, so the G items of one (tile, kind, group) are
// placed kXcds apart: they run on one XCD at about the same time and share its L2. Groups are
// taken in list order (longest first), kXcds at a time, as the columns of a block of G rows.
constexpr int kXcds = 8;

std::vector<Item> xcd_order(const std::vector<Item>& v, int32_t group) {
  if (group <= 1) return v;
  std::vector<std::vector<Item>> combos;
  for (const Item& x : v) {
    const Item* last = combos.empty() ? nullptr : &combos.back().front();
    const int32_t h = item_head(x.d), kind = x.d >> 24;
    if (last != nullptr && (int32_t)combos.back().size() < group && last->a == x.a &&
        last->b == x.b && last->c == x.c && (last->d >> 24) == kind &&
        item_head(last->d) / group == h / group) {
      combos.back().push_back(x);
    } else {
      combos.push_back({x});
    }
  }
  std::vector<Item> out;
  out.reserve(v.size());
  // A block takes up to 8 consecutive combos of one size (pair plans mix kv combos of G / 2
  // items with q combos of G), so that every combo's items sit one stride apart.
  for (size_t c0 = 0; c0 < combos.size();) {
    size_t c1 = c0 + 1;
    while (c1 < combos.size() && c1 - c0 < (size_t)kXcds && combos[c1].size() == combos[c0].size())
      ++c1;
    for (size_t r = 0; r < combos[c0].size(); ++r)
      for (size_t c = c0; c < c1; ++c) out.push_back(combos[c][r]);
    c0 = c1;
  }
  return out;
}

int64_t count_items(const int32_t* cu, int32_t n_docs, int32_t hq, int32_t hkv, int32_t kind) {
  if (is_group_kind(kind) || kind == VA_PLAN_FWD_NARROW)
    return (int64_t)make_items(cu, n_docs, hq, hkv, kind).size();
  int64_t n = 0;
  const bool pairs =
      kind != VA_PLAN_FWD && va::bwd_plan_pairs(doc_tiles(cu, n_docs), hq, hkv, kind);
  const int64_t kv_per_tile = pairs ? (int64_t)hkv * ((hq / hkv + 1) / 2) : hq;  // per kind
  for (int32_t i = 0; i < n_docs; ++i) {
    const int64_t len = (int64_t)cu[i + 1] - cu[i];
    if (len <= 0) continue;
    if (kind == VA_PLAN_FWD) {
      n += (len + va::kFwdBlockM - 1) / va::kFwdBlockM * hq;
    } else {
      n += (len + va::kBwdBlockN - 1) / va::kBwdBlockN * kv_per_tile;
      n += (len + va::kBwdBlockM - 1) / va::kBwdBlockM * kv_per_tile;
    }
  }
  return n;
}

}  // namespace

extern "C" int va_plan_size(const int32_t* cu_seqlens, int32_t n_docs, int32_t hq, int32_t hkv,
                            int32_t kind, int64_t* n_items) {
  if (n_items == nullptr) return va::fail(VA_EINVAL, "n_items is NULL");
  if (!is_plan_kind(kind)) return va::fail(VA_EINVAL, "bad plan kind %d", kind);
  int rc = check_heads(hq, hkv);
  if (rc) return rc;
  rc = check_cu(cu_seqlens, n_docs);
  if (rc) return rc;
  *n_items = count_items(cu_seqlens, n_docs, hq, hkv, kind);
  return VA_OK;
}

extern "C" int va_plan_build(const int32_t* cu_seqlens, int32_t n_docs, int32_t hq, int32_t hkv,
                             int32_t kind, int32_t* items, int64_t capacity, int64_t* n_items) {
  int64_t n = 0;
  int rc = va_plan_size(cu_seqlens, n_docs, hq, hkv, kind, &n);
  if (rc) return rc;
  if (n_items) *n_items = n;
  if (n > capacity) return va::fail(VA_ECAPACITY, "plan needs %lld items, capacity %lld",
                                    (long long)n, (long long)capacity);
  if (n > 0 && items == nullptr) return va::fail(VA_EINVAL, "items is NULL");
  const std::vector<Item> v = xcd_order(make_items(cu_seqlens, n_docs, hq, hkv, kind), hq / hkv);
  for (size_t i = 0; i < v.size(); ++i) {
    items[4 * i + 0] = v[i].a;
    items[4 * i + 1] = v[i].b;
    items[4 * i + 2] = v[i].c;
    items[4 * i + 3] = v[i].d;
  }
  return VA_OK;
}

extern "C" int va_plan_bwd_row_stats(const int32_t* cu_seqlens, int32_t n_docs, int32_t* use) {
  int rc = check_cu(cu_seqlens, n_docs);
  if (rc) return rc;
  if (use == nullptr) return va::fail(VA_EINVAL, "va_plan_bwd_row_stats: NULL output");
  // sum over rows of the number of 128-key tiles at or before the row's tile
  int64_t rows = 0, covered = 0;
  for (int32_t i = 0; i < n_docs; ++i) {
    const int64_t len = (int64_t)cu_seqlens[i + 1] - cu_seqlens[i];
    const int64_t full = len / va::kBwdBlockN, rest = len % va::kBwdBlockN;
    covered += (int64_t)va::kBwdBlockN * full * (full + 1) / 2 + rest * (full + 1);
    rows += len;
  }
  *use = rows > 0 && covered >= (int64_t)VA_BWD_STATS_MIN_TILES * rows;
  return VA_OK;
}

extern "C" int va_plan_capacity(int64_t n_tokens, int32_t n_docs, int32_t hq, int32_t kind,
                                int64_t* capacity) {
  if (capacity == nullptr) return va::fail(VA_EINVAL, "capacity is NULL");
  if (!is_plan_kind(kind)) return va::fail(VA_EINVAL, "bad plan kind %d", kind);
  if (n_tokens < 0 || n_tokens > INT32_MAX / 2)
    return va::fail(VA_ESHAPE, "n_tokens=%lld out of range", (long long)n_tokens);
  if (n_docs < 0 || n_docs > va::kPlanMaxDocs)
    return va::fail(VA_ESHAPE, "n_docs=%d out of range [0, %d]", n_docs, va::kPlanMaxDocs);
  if (hq <= 0 || hq > 4096) return va::fail(VA_ESHAPE, "Hq=%d out of range", hq);
  const int64_t tiles = (n_tokens + va::kFwdBlockM - 1) / va::kFwdBlockM + n_docs;
  // A narrow forward plan adds at most one item per document and head (a second half), and only
  // to a list that then holds at most kPlanCus items.
  *capacity = kind == VA_PLAN_FWD ? tiles * hq
              : kind == VA_PLAN_FWD_NARROW
                  ? std::max<int64_t>(tiles * hq, std::min<int64_t>(va::kPlanCus, (tiles + n_docs) * hq))
                  : tiles * hq * 2;
  return VA_OK;
}

namespace {

int check_device_plan(int64_t n_tokens, int32_t n_docs, int32_t hq, int32_t hkv, int32_t kind,
                      const int32_t* items, int64_t capacity) {
  int64_t need = 0;
  int rc = va_plan_capacity(n_tokens, n_docs, hq, kind, &need);
  if (rc) return rc;
  if (items == nullptr) return va::fail(VA_EINVAL, "device plan items are NULL");
  if (((uintptr_t)items & 15u) != 0) return va::fail(VA_EINVAL, "items_device not 16-byte aligned");
  if (capacity < need)
    return va::fail(VA_ECAPACITY, "device plan needs capacity %lld, got %lld", (long long)need,
                    (long long)capacity);
  return VA_OK;
}

}  // namespace

extern "C" int va_plan_build_device(const int32_t* cu_seqlens_device, int32_t n_docs,
                                    int64_t n_tokens, int32_t hq, int32_t hkv, int32_t kind,
                                    int32_t* items_device, int64_t capacity, void* stream) {
  int rc = check_heads(hq, hkv);
  if (rc) return rc;
  if (!is_plan_kind(kind)) return va::fail(VA_EINVAL, "bad plan kind %d", kind);
  if (cu_seqlens_device == nullptr) return va::fail(VA_EINVAL, "cu_seqlens_device is NULL");
  if ((rc = check_device_plan(n_tokens, n_docs, hq, hkv, kind, items_device, capacity))) return rc;
  const bool fwd = is_fwd_kind(kind);
  const hipError_t e = va::launch_plan_device(
      cu_seqlens_device, nullptr, n_docs, (int)n_tokens, hq, hkv, fwd ? items_device : nullptr,
      capacity, fwd ? nullptr : items_device, capacity, kind,
      kind == VA_PLAN_BWD_GROUPS ? 1 : (kind == VA_PLAN_BWD_GROUPS_ALL ? 2 : 0),
      kind == VA_PLAN_FWD_NARROW, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return va::fail((int)e, "va_plan_build_device launch: %s", hipGetErrorString(e));
  return VA_OK;
}

extern "C" int va_plan_build_device_lengths(const int64_t* lengths_device, int32_t n_docs,
                                            int64_t n_tokens, int32_t hq, int32_t hkv,
                                            int32_t* fwd_items_device, int64_t fwd_capacity,
                                            int32_t* bwd_items_device, int64_t bwd_capacity,
                                            int32_t* cu_seqlens_out, void* stream) {
  int rc = check_heads(hq, hkv);
  if (rc) return rc;
  if (lengths_device == nullptr && n_docs > 0) return va::fail(VA_EINVAL, "lengths_device is NULL");
  if (fwd_items_device == nullptr && bwd_items_device == nullptr)
    return va::fail(VA_EINVAL, "no plan requested");
  if (fwd_items_device != nullptr &&
      (rc = check_device_plan(n_tokens, n_docs, hq, hkv, VA_PLAN_FWD_NARROW, fwd_items_device,
                              fwd_capacity)))
    return rc;
  if (bwd_items_device != nullptr &&
      (rc = check_device_plan(n_tokens, n_docs, hq, hkv, VA_PLAN_BWD, bwd_items_device,
                              bwd_capacity)))
    return rc;
  const hipError_t e = va::launch_plan_device(
      nullptr, lengths_device, n_docs, (int)n_tokens, hq, hkv, fwd_items_device, fwd_capacity,
      bwd_items_device, bwd_capacity, VA_PLAN_BWD, 0, 1, cu_seqlens_out, (hipStream_t)stream);
  if (e != hipSuccess)
    return va::fail((int)e, "va_plan_build_device_lengths launch: %s", hipGetErrorString(e));
  return VA_OK;
}

extern "C" int va_stream_capture_id(void* stream, uint64_t* capture_id) {
  if (capture_id == nullptr) return va::fail(VA_EINVAL, "capture_id is NULL");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  const hipError_t e = hipStreamGetCaptureInfo((hipStream_t)stream, &status, &id);
  if (e != hipSuccess) return va::fail((int)e, "hipStreamGetCaptureInfo: %s", hipGetErrorString(e));
  *capture_id = status == hipStreamCaptureStatusActive ? (uint64_t)id : 0;
  return VA_OK;
}
