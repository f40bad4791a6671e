// Host-side launch descriptors shared by the kernel translation units and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace va {

constexpr int kHeadDim = 128;  // Qwen2.5-1.5B / 7B head size; the kernels are built for it

// Tile geometry; the plan builder (plan.cpp) emits work items for exactly these shapes.
constexpr int kFwdWaves = 4;                 // forward: 32 queries per wave
constexpr int kFwdBlockM = 32 * kFwdWaves;   // queries per forward work item
// From this many 128-query tiles x query heads on (ceil(N / 128) Hq >= VA_FWD_MANY_ITEMS, a lower
// bound of the forward list's length that host and device plans share), the 4-wave forward (two
// work-groups per CU) runs instead of the 8-wave one: every CU then gets at least two items.
constexpr int kFwdLeanMinItems = 512;
constexpr int kBwdBlockN = 128;  // keys per backward kv work item
constexpr int kBwdBlockQ = 32;   // queries per kv-item step
constexpr int kBwdBlockM = 128;  // queries per backward q work item
constexpr int kBwdTileK = 32;    // keys per q-item tile
constexpr int kPlanMaxDocs = 8192;  // documents a device-built plan takes (LDS-resident bounds)
// Fixed cost of a backward kv / q item (prologue, epilogue) in the planners' work unit, MFMAs per
// wave per step pair: 32 per kv step pair, 24 per q tile pair (from in-graph item durations).
constexpr int kPlanKvItemCost = 39;
constexpr int kPlanQItemCost = 30;
constexpr int kPlanCus = 256;  // compute units the plans balance work over (MI355X)
// VA_PLAN_BWD takes two query heads per item (pair items, Hq > Hkv) once the per-head list
// would be this long (2 T Hq items, T the 128-row tiles of the documents: every CU then holds
// several).
constexpr int kBwdPairMinItems = 1024;
// Item word: kind << 24 | group << 21 | pair << 20 | (heads - 1) << 12 | head.
constexpr int kItemPairBit = 1 << 20;
constexpr int kItemHeadMask = (1 << 12) - 1;  // head < Hq <= 4096
constexpr int kItemHeadsShift = 12;
// A kv item over S query heads h .. h + S - 1 of one GQA group (group items, S >= 2 dividing G):
// its halves walk the S heads' steps in sequence. With S = G it writes dK/dV of the key tile at
// Hkv width (the tile needs no per-head partials and no GQA sum); with S < G it writes the sum of
// its S heads into the partial of head h, and the GQA sum adds G / S partials for the tile's rows.
constexpr int kItemGroupBit = 1 << 21;
// A narrow forward item (VA_PLAN_FWD_NARROW): 64 queries instead of 128, run by the 8-wave
// forward as 2 query strips x 4 key phases, so that its chain of key tiles is half a 128-query
// item's. The host plan splits its longest items so when the list leaves CUs idle.
constexpr int kItemNarrowBit = 1 << 22;
// Planners' work measure of a group item over S heads of a kv tile with `steps` query steps: the
// halves take ceil(S steps / 2) step pairs.
__host__ __device__ inline int64_t bwd_group_work(int64_t steps, int s) {
  return (s * steps + 1) / 2 * 32 + kPlanKvItemCost;
}
// The head count of a key tile's group items: the largest S >= 2 dividing G whose group item's
// work is at most `cap`, or 0 (the tile keeps per-head or pair items). S < G only in long lists
// (`subsets`: those with pair items, several items per CU), where the total work sets the time:
// in a short list (config 2) items of S < G over its shorter tiles made the backward slower
// (measured +3.5%), each as long as the longest items.
__host__ __device__ inline int bwd_group_heads(int64_t steps, int group, int64_t cap, bool subsets) {
  for (int s = group; s >= 2; --s)
    if (group % s == 0 && bwd_group_work(steps, s) <= cap) return s;
    else if (!subsets) break;
  return 0;
}
// Whether a backward plan of `kind` has pair items; `tiles` = sum over the documents of
// ceil(length / 128) (empty documents have none), which the host planner and the device planner
// both count from the same bounds, so that host and device plans of one batch take the same shape.
__host__ __device__ inline bool bwd_plan_pairs(int64_t tiles, int32_t hq, int32_t hkv, int kind) {
  if (kind == 2 || hkv <= 0 || hq / hkv < 2) return false;  // VA_PLAN_BWD_HEADS, or no group
  if (kind == 3) return true;                                  // VA_PLAN_BWD_PAIRS
  return 2 * tiles * (int64_t)hq >= kBwdPairMinItems;
}

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  const int32_t* items;  // int4 per work item: {q0, doc_end, doc_start, head}
  int64_t n_items;
  int64_t n_tokens;
  int hq, hkv;
  float scale;
  int dtype;
  hipStream_t stream;
  int kernel;  // 1: the 8-wave forward, 2: the many-item (4-wave) forward
};

// Rotary tables of the attention kernels' epilogues: fp32 cos / sin rows (1 or B, T, 128) at
// b * scb + t * sct (elements, multiples of 4), b = b_idx[token], t = t_idx[token].
struct RopeTab {
  const float* cos;
  const float* sin;
  const int32_t* b_idx;
  const int32_t* t_idx;
  int scb, sct;
};

struct BwdArgs {
  const void* dout;
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const float* lse;
  const int32_t* items;  // int4 per work item: kv {k0, doc_end, -, head}, q {q0, doc_end,
                         // doc_start, (1 << 24) | head}
  int64_t n_items;
  int64_t n_tokens;
  int hq, hkv;
  float scale;
  int dtype;
  void* dq;         // (n_tokens, hq, 128), written by the q items
  void* dk_part;    // (n_tokens, hq, 128) per-query-head dK (== dk when hq == hkv)
  void* dv_part;
  void* dk;         // (n_tokens, hkv, 128) GQA sums, or null to keep the per-head partials
  void* dv;
  uint32_t* flags;  // (n_tokens) 1 where a group item wrote dK/dV itself (the GQA sum skips the
                    // row), 0 where per-head partials hold it; null when Hq == Hkv
  float* stats;     // (hq, n_tokens) x {lse log2 e, rowsum(dO * O)} written by the row-statistics
                    // pass before the main kernel, or null: the main kernel forms them itself
  hipStream_t stream;
  RopeTab rope;  // cos null: none; else dQ and dK are written rotated back to the projections'
                 // frame
};

struct RopeArgs {
  const void* x0;        // forward: q, k, v projections; backward: gradients
  const void* x1;
  const void* x2;
  const float* cos;      // (1 or B, T, D) fp32
  const float* sin;
  int64_t cos_batch_stride;  // 0 when cos has one row of tables
  int64_t cos_seq_stride;
  const int32_t* b_idx;
  const int32_t* t_idx;
  void* y0;
  void* y1;
  void* y2;
  int64_t n_tokens;
  int heads, kv_heads;
  int seq;               // padded layout: T
  int in_dtype;          // dtype of x (0 f16, 1 bf16, 2 f32)
  int out_dtype;         // dtype of y
  int layout;            // 0 packed (N, H, D); 1 padded (B, H, T, D)
  int expand;            // 1: write K/V for every query head (reference qkv_rotate semantics)
  hipStream_t stream;
};

hipError_t launch_fwd(const FwdArgs& a);
hipError_t launch_bwd(const BwdArgs& a);
// stage 1 main (reads a.stats when non-null), 2 finish, 3 finish (no flags), 4 row statistics
hipError_t launch_bwd_stage(const BwdArgs& a, int stage);
hipError_t launch_rope_fwd(const RopeArgs& a);
hipError_t launch_rope_bwd(const RopeArgs& a);
hipError_t launch_pack_rows(const void* src, void* dst, const int32_t* b_idx, const int32_t* t_idx,
                            int64_t n_tokens, int heads, int seq, int row_bytes, int mode,
                            hipStream_t stream);

// Device-built plans (plan_device.hip): from a device cu_seqlens or from device lengths (exactly
// one non-null); each requested plan (non-null items) is `capacity` items, real ones first, empty
// ones after; cu_out (nullable) receives the clamped document bounds.
// bwd_kind: the backward plan kind whose pair rule applies (bwd_plan_pairs over the tiles that the
// device counts).
hipError_t launch_plan_device(const int32_t* cu, const int64_t* lengths, int n_docs, int n_tokens,
                              int hq, int hkv, int32_t* fwd_items, long fwd_capacity,
                              int32_t* bwd_items, long bwd_capacity, int bwd_kind,
                              int bwd_groups, int fwd_narrow,
                              int32_t* cu_out, hipStream_t stream);

}  // namespace va
