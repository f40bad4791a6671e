/*
 * varlen_attn.h - C ABI of the MI355X (gfx950) packed variable-length causal GQA attention.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, launches asynchronously on
 * the caller's HIP stream (`stream` is a hipStream_t, NULL = default stream), never allocates and
 * never synchronises. Device buffers are owned by the caller. Return value: 0 on success, a
 * negative VA_E* code for an argument error (nothing launched), or a positive hipError_t when a
 * launch failed; `va_last_error()` describes the last failure of the calling thread.
 *
 * Layouts (row-major, contiguous, 16-byte aligned):
 *   q, out, dq      (N, Hq, 128)   16-bit (dtype VA_F16 or VA_BF16)
 *   k, v, dk, dv    (N, Hkv, 128)  16-bit; GQA: query head h reads key/value head h / (Hq/Hkv)
 *   lse             (Hq, N)        fp32, natural-log log-sum-exp of each query row
 *   cu_seqlens      (n_docs + 1)   int32 host array, cu[0] = 0, non-decreasing; document i is
 *                                  rows [cu[i], cu[i+1]) of the packed token axis
 *   work items      int32 x 4 each in device memory: built on the host by va_plan_build (and
 *                   copied to the device by the caller) or on the device by va_plan_build_device.
 *                   The kernels skip an item whose head is not below Hq or whose rows do not lie
 *                   in [0, total_tokens), so a plan made for other sizes cannot write out of
 *                   bounds (it computes nothing useful either).
 *
 * Reference interfaces replaced (mergentlegen/hackaton, solution/attention.py):
 *   va_plan_build       _cu_seqlens (195-209) + the tile walk inside the aten kernel
 *   va_fwd              torch.ops.aten._efficient_attention_forward(q, k, v, None, cu, cu,
 *                       max_len, max_len, 0.0, 1, True, scale=) at 221-222 (causal top-left,
 *                       log-sum-exp returned)
 *   va_bwd              torch.ops.aten._efficient_attention_backward(grad, q, k, v, None, out, cu,
 *                       cu, max_len, max_len, lse, 0.0, seed, offset, 1, False, scale=) at
 *                       230-232, plus the GQA sum of dk/dv of qkv_kernel mode 1 (113-134)
 *   va_rope_fwd         qkv_kernel mode 0 (_qkv_forward, 36-83; launched at 168-170)
 *   va_rope_bwd         qkv_kernel mode 1 (_qkv_backward, 86-134; launched at 185-187)
 *   va_pack_rows        pack_kernel (288-300; launched at 311-312 and 323-324)
 */
#ifndef VARLEN_ATTN_H_
#define VARLEN_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  VA_OK = 0,
  VA_EINVAL = -1,    /* null pointer, negative size, misaligned buffer, bad enum value */
  VA_ESHAPE = -2,    /* head_dim != 128, Hq not a multiple of Hkv, sizes out of range */
  VA_EDTYPE = -3,    /* unsupported element type */
  VA_ESEQ = -4,      /* cu_seqlens not starting at 0, decreasing, or beyond the token count */
  VA_ECAPACITY = -5  /* output buffer too small (plan items, workspace) */
};

enum { VA_F16 = 0, VA_BF16 = 1, VA_F32 = 2 };
enum { VA_PLAN_FWD = 0, VA_PLAN_BWD = 1, VA_PLAN_BWD_HEADS = 2, VA_PLAN_BWD_PAIRS = 3,
       VA_PLAN_BWD_GROUPS = 4, VA_PLAN_BWD_GROUPS_ALL = 5, VA_PLAN_FWD_NARROW = 6 };
enum { VA_BWD_PAIR_MIN_ITEMS = 1024 };
enum { VA_LAYOUT_PACKED = 0, VA_LAYOUT_PADDED = 1 };
enum { VA_BWD_MAIN = 1, VA_BWD_FINISH = 2, VA_BWD_FINISH_HEADS = 3, VA_BWD_STATS = 4,
       VA_BWD_MAIN_STATS = 5 };

const char* va_last_error(void);
int32_t va_abi_version(void);
int32_t va_head_dim(void);

/* ---- work plan (host only; no GPU call) ------------------------------------------------------
 * Work items for the forward (kind VA_PLAN_FWD: one per 128-query tile x query head) or the
 * backward (one per 128-key tile for dK/dV and one per 128-query tile for dQ, each x query
 * head (VA_PLAN_BWD_HEADS) or x pair of query heads of one GQA group, the last head of an odd
 * group alone (VA_PLAN_BWD_PAIRS); VA_PLAN_BWD takes pairs when Hq > Hkv
 * and the per-head list would hold 2 T Hq >= VA_BWD_PAIR_MIN_ITEMS items, T = the sum over the
 * documents of ceil(length / 128), heads otherwise; a device-built plan applies the same rule to
 * the same count) over the documents of cu_seqlens, longest first. The items of one tile
 * and GQA group sit 8 apart in the list (work-group i runs on XCD i mod 8), so that the heads
 * sharing K/V run on one XCD and share its L2. Fully masked causal tiles and cross-document tiles
 * never appear. VA_PLAN_BWD_GROUPS is VA_PLAN_BWD with GQA group items where they do not lengthen
 * the plan: a key tile gets, per GQA group, G / S kv items over S query heads each (S >= 2
 * dividing G: the largest whose item does no more work than the longest item of the VA_PLAN_BWD
 * list, or than that list's work per CU (256 CUs); S < G only in lists with pair items). An item
 * of S = G heads writes the tile's dK/dV itself (Hkv width): no per-head partials, nothing for
 * the GQA sum; one of S < G heads writes the sum of its heads into the first head's partial.
 * Item word: kind << 24 | narrow << 22 | group << 21 | pair << 20 | (S - 1) << 12 | head.
 * VA_PLAN_FWD_NARROW is VA_PLAN_FWD whose longest items are split in two
 * 64-query items (narrow bit 22) when the list is short enough to leave CUs idle: for the
 * last 128-query tile of every document of the maximal length L, when (T + the number of such
 * documents) x Hq <= 256 (T as below). Both forward kernels run narrow items; the 8-wave one
 * walks a narrow item's keys in four phases, so that its chain of key tiles is half as long.
 * VA_PLAN_BWD_GROUPS_ALL gives every key tile S = G. Group plans need Hq > Hkv; with dk = dv =
 * NULL their per-head partials hold each group item's sum in its first head (see va_bwd). Every
 * plan kind gives the same outputs up to rounding
 * (a pair item sums a head's steps or tiles in one sequence instead of two halves, a group item
 * its heads' in one); each is deterministic.
 * Replaces: solution/attention.py:195-209 (_cu_seqlens, cached per lengths by the caller). */
int va_plan_size(const int32_t* cu_seqlens, int32_t n_docs, int32_t hq, int32_t hkv, int32_t kind,
                 int64_t* n_items);
int va_plan_build(const int32_t* cu_seqlens, int32_t n_docs, int32_t hq, int32_t hkv, int32_t kind,
                  int32_t* items, int64_t capacity, int64_t* n_items);

/* Whether the backward's row statistics pay for a pass of their own (VA_BWD_STATS, then
 * VA_BWD_MAIN_STATS instead of VA_BWD_MAIN) over the documents of cu_seqlens: *use = 1 when the
 * query rows are covered by VA_BWD_STATS_MIN_TILES or more 128-key tiles on average (a row's
 * tiles are those at or before its own in its document: each one's kv item stages the row).
 * The pass reads O and dO once (2 Hq D e bytes per row); without it every kv item that covers a
 * row loads its O beside dO to form rowsum(dO * O). Host only, no GPU call. No counterpart in
 * the reference (its aten kernel's internal choice). */
enum { VA_BWD_STATS_MIN_TILES = 3 };
int va_plan_bwd_row_stats(const int32_t* cu_seqlens, int32_t n_docs, int32_t* use);

/* ---- work plan built on the device --------------------------------------------------------------
 * For callers whose document lengths live on the GPU: the plan is built from a device cu_seqlens
 * by one kernel on `stream`, with no host read (the reference reads the lengths back with
 * lengths.tolist(), solution/packed.py:170-172, before _cu_seqlens at attention.py:195-209).
 * va_plan_capacity gives, from host-known sizes only, the number of items such a plan has:
 * ceil(n_tokens / 128) + n_docs tiles per query head (VA_PLAN_FWD_NARROW: n_docs more, its
 * second halves, up to 256 items in all), twice that for the backward kinds (a pair plan leaves
 * the slots of its missing kv rows empty).
 * va_plan_build_device writes exactly `capacity` items (int32 x 4) to device memory: the real
 * ones longest first, then empty items that va_fwd / va_bwd skip, so the kernels take n_items =
 * capacity. Document bounds are clamped into [0, n_tokens] and made non-decreasing on the device,
 * and the last document ends at n_tokens: rows past the lengths' sum (which the host planner
 * rejects, and which a device plan cannot report without a host read) join the last document, so
 * every output and gradient row is written. n_docs <= 8192. */
int va_plan_capacity(int64_t n_tokens, int32_t n_docs, int32_t hq, int32_t kind, int64_t* capacity);
int va_plan_build_device(const int32_t* cu_seqlens_device, int32_t n_docs, int64_t n_tokens,
                         int32_t hq, int32_t hkv, int32_t kind, int32_t* items_device,
                         int64_t capacity, void* stream);

/* The same plans straight from the per-document lengths (int64, as a mask's row sums give them):
 * one launch builds cu_seqlens (into cu_seqlens_out, n_docs + 1 int32, when it is non-NULL), the
 * forward plan (kind VA_PLAN_FWD_NARROW, capacity from va_plan_capacity of that kind) and the
 * backward plan (VA_PLAN_BWD; either item pointer may be NULL to skip that kind). Each
 * length is clamped into [0, n_tokens] and the bounds saturate at n_tokens.
 * Replaces: lengths.tolist() at solution/packed.py:170-172 and _cu_seqlens at
 * solution/attention.py:195-209, on the device. */
int va_plan_build_device_lengths(const int64_t* lengths_device, int32_t n_docs, int64_t n_tokens,
                                 int32_t hq, int32_t hkv, int32_t* fwd_items_device,
                                 int64_t fwd_capacity, int32_t* bwd_items_device,
                                 int64_t bwd_capacity, int32_t* cu_seqlens_out, void* stream);

/* Capture id of the stream's active graph capture, 0 when the stream is not capturing. A utility
 * with no counterpart in the reference: callers that cache device plans across layers key the
 * cache on it, so that a plan built inside one capture is reused only inside that capture. */
int va_stream_capture_id(void* stream, uint64_t* capture_id);

/* ---- attention forward ------------------------------------------------------------------------
 * out = softmax(scale q k^T + causal mask per document) v, lse = log-sum-exp of each row;
 * scale must be finite and > 0 (D^-0.5 in the reference).
 * From ceil(total_tokens / 128) * Hq >= VA_FWD_MANY_ITEMS on (a lower bound of the list's length
 * that depends on the sizes only, so host and device plans of one batch pick the same kernel)
 * va_fwd runs its many-item kernel (4 waves per item, two work-groups per CU) instead of the
 * 8-wave one; both compute the same function (results agree to rounding, each is deterministic).
 * va_fwd_kernel is va_fwd with the kernel named: VA_FWD_AUTO (va_fwd's choice), VA_FWD_WIDE (the
 * 8-wave kernel) or VA_FWD_MANY (the many-item kernel), for callers that time or test one of them.
 * Replaces: solution/attention.py:221-222 (aten::_efficient_attention_forward). */
enum { VA_FWD_MANY_ITEMS = 512 };
enum { VA_FWD_AUTO = 0, VA_FWD_WIDE = 1, VA_FWD_MANY = 2 };
int va_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
           const int32_t* items, int64_t n_items, int64_t total_tokens, int32_t hq, int32_t hkv,
           int32_t head_dim, float scale, int32_t dtype, void* stream);
int va_fwd_kernel(int32_t kernel, const void* q, const void* k, const void* v, void* out,
                  float* lse, const int32_t* items, int64_t n_items, int64_t total_tokens,
                  int32_t hq, int32_t hkv, int32_t head_dim, float scale, int32_t dtype,
                  void* stream);

/* ---- attention backward -----------------------------------------------------------------------
 * Deterministic and atomic-free. dq (N, Hq, 128) is always written. dk/dv (N, Hkv, 128) are the
 * sums over each GQA group of per-query-head partials (N, Hq, 128, element type) that live in the
 * workspace at the offsets va_bwd_workspace_layout reports; with dk = dv = NULL the partials are
 * the result (a rotary backward can sum them, as the reference sums its expanded copies; a group
 * item then writes its heads' sum into the partial of its first head and zeros into its other
 * heads', so that the sum over each GQA group's partials is exact for every plan kind). Past the
 * two partial arrays the workspace holds one uint32 flag
 * per row, marking the rows whose dK/dV a group item wrote, then the row statistics of
 * VA_BWD_STATS. With Hq == Hkv and dk/dv given, va_bwd uses no workspace. The caller's O and lse
 * come from va_fwd; rowsum(dO * O) is computed inside.
 * Replaces: solution/attention.py:230-232 (aten::_efficient_attention_backward) and the GQA
 * reduction of dk/dv at solution/attention.py:113-134. */
int va_bwd_workspace_layout(int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim,
                            int64_t offsets[2], int64_t* bytes);
int va_bwd(const void* dout, const void* q, const void* k, const void* v, const void* out,
           const float* lse, const int32_t* items, int64_t n_items, int64_t total_tokens,
           int32_t hq, int32_t hkv, int32_t head_dim, float scale, int32_t dtype, void* dq,
           void* dk, void* dv, void* workspace, int64_t workspace_bytes, void* stream);

/* The same backward for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same inputs and outputs as va_bwd, no workspace: the dK/dV partials live in a static
 * device array of the library (va_bwd_noalloc_max_bytes() = 66 MiB per GPU, held until the
 * process ends: partials and row flags), so total_tokens * Hq must not exceed 131072 at head_dim 128 (VA_ECAPACITY
 * otherwise, before any launch); dk and dv must be given. Calls nothing that allocates. Calls
 * that overlap on one GPU (two streams or two threads) race on the shared array. */
int64_t va_bwd_noalloc_max_bytes(void);
int va_bwd_noalloc(const void* dout, const void* q, const void* k, const void* v, const void* out,
                   const float* lse, const int32_t* items, int64_t n_items, int64_t total_tokens,
                   int32_t hq, int32_t hkv, int32_t head_dim, float scale, int32_t dtype, void* dq,
                   void* dk, void* dv, void* stream);

/* The same backward in its two stages, for callers that time or overlap them separately:
 * VA_BWD_MAIN (dQ and the per-head dK/dV partials) and VA_BWD_FINISH (the GQA sums into dk/dv;
 * nothing when they are NULL or Hq == Hkv). VA_BWD_STATS writes the row statistics
 * {lse log2 e, rowsum(dO * O)} (fp32, (Hq, N) pairs) into the workspace's last region, and
 * VA_BWD_MAIN_STATS is VA_BWD_MAIN reading them instead of loading O (the caller runs VA_BWD_STATS
 * first, on the same stream and workspace; both need the workspace even when Hq == Hkv): the
 * results are bitwise those of VA_BWD_MAIN, which forms the same statistics with the same
 * arithmetic. VA_BWD_FINISH_HEADS is VA_BWD_FINISH for a list
 * without group items (VA_PLAN_BWD, VA_PLAN_BWD_HEADS, VA_PLAN_BWD_PAIRS, or a VA_PLAN_BWD_GROUPS
 * list in which the planner grouped no key tile): every key row then sums its G per-head
 * partials, so the row flags that group items leave are not read (one dependent memory round
 * trip less); after a list with group items it would sum stale partials. Any other stage value
 * is VA_EINVAL. Same arguments as va_bwd.
 * Replaces: the same reference call as va_bwd (solution/attention.py:230-232). */
int va_bwd_stage(int32_t stage, const void* dout, const void* q, const void* k, const void* v,
                 const void* out, const float* lse, const int32_t* items, int64_t n_items,
                 int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim, float scale,
                 int32_t dtype, void* dq, void* dk, void* dv, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* The backward with the inverse rotary embedding in its epilogues, for a caller whose q and k are
 * rotated projections (the decoder layer's packed call): dq and dk come out as the gradients of
 * the projections before the rotation, dv as before. The main stages (VA_BWD_MAIN,
 * VA_BWD_MAIN_STATS) rotate each finished dQ row and each dK row or per-head dK partial back
 * with the tables, in fp32 before the one rounding (the rotation is linear, so the GQA sum of
 * rotated partials is the rotated sum); the other stages are va_bwd_stage's. The tables are those
 * of va_rope_bwd (fp32, row b * cos_batch_stride + t * cos_seq_stride for the token's b_idx and
 * t_idx, strides non-negative multiples of 4, cos/sin 16-byte aligned); the caller guarantees
 * that every token's row lies inside them. Arguments otherwise as va_bwd_stage.
 * Replaces: solution/attention.py:230-232 followed by the inverse rotation of qkv_kernel mode 1
 * (attention.py:86-134, launched at 185-187) for dq and dk. */
typedef struct va_rope_tables {
  const float* cos;
  const float* sin;
  int64_t cos_batch_stride;
  int64_t cos_seq_stride;
  const int32_t* b_idx;
  const int32_t* t_idx;
} va_rope_tables;
int va_bwd_rotary_stage(int32_t stage, const va_rope_tables* rope, const void* dout,
                        const void* q, const void* k, const void* v, const void* out,
                        const float* lse, const int32_t* items, int64_t n_items,
                        int64_t total_tokens, int32_t hq, int32_t hkv, int32_t head_dim,
                        float scale, int32_t dtype, void* dq, void* dk, void* dv, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* ---- rotary embedding -------------------------------------------------------------------------
 * Forward: q (N, heads*D), k, v (N, kv_heads*D) in in_dtype (VA_F16/VA_BF16/VA_F32); cos, sin
 * fp32 tables indexed at b*cos_batch_stride + t*cos_seq_stride (b, t from b_idx/t_idx, int32).
 * Rotation in fp32, rounded once to out_dtype. layout VA_LAYOUT_PACKED writes (N, H, D),
 * VA_LAYOUT_PADDED writes (B, H, seq, D) (caller zero-fills). expand=1 writes K/V for all `heads`
 * (reference qkv_rotate semantics); expand=0 keeps kv_heads (GQA-native attention input).
 * v and v_out may both be NULL in a forward without expand: only the q and k rows are written
 * (for a caller whose v is already in out_dtype and uses it as it is).
 * Backward: the inverse rotation (and the sum of the G copies when expand=1); dq/dk/dv read in
 * in_dtype from `layout`, written (N, H*D) in out_dtype. Every tensor base must be 16-byte aligned
 * and the cos/sin strides (in elements) non-negative multiples of 4: each lane moves 16 bytes.
 * Replaces: solution/attention.py:36-134 (qkv_kernel modes 0 and 1). */
int va_rope_fwd(const void* q, const void* k, const void* v, const float* cos, const float* sin,
                int64_t cos_batch_stride, int64_t cos_seq_stride, const int32_t* b_idx,
                const int32_t* t_idx, void* q_out, void* k_out, void* v_out, int64_t n_tokens,
                int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t seq, int32_t in_dtype,
                int32_t out_dtype, int32_t layout, int32_t expand, void* stream);
int va_rope_bwd(const void* dq, const void* dk, const void* dv, const float* cos,
                const float* sin, int64_t cos_batch_stride, int64_t cos_seq_stride,
                const int32_t* b_idx, const int32_t* t_idx, void* dq_in, void* dk_in,
                void* dv_in, int64_t n_tokens, int32_t heads, int32_t kv_heads, int32_t head_dim,
                int32_t seq, int32_t in_dtype, int32_t out_dtype, int32_t layout, int32_t expand,
                void* stream);

/* ---- row packing ------------------------------------------------------------------------------
 * mode 0: (B, heads, seq, head_dim) -> (N, heads*head_dim) rows of the real tokens (exact);
 * mode 1: the reverse scatter into a caller-zeroed (B, heads, seq, head_dim) buffer.
 * Replaces: solution/attention.py:288-300 (pack_kernel). */
int va_pack_rows(const void* src, void* dst, const int32_t* b_idx, const int32_t* t_idx,
                 int64_t n_tokens, int32_t heads, int32_t seq, int32_t head_dim,
                 int32_t elem_bytes, int32_t mode, void* stream);

/* ---- machine-ceiling probes (diagnostics) ----------------------------------------------------
 * No counterpart in the reference: the benchmark measures with them the two ceilings it quotes
 * its roofline fractions against, on the box it runs on, beside the data-sheet figures.
 * va_probe_mfma: `blocks` work-groups of 256 threads, each wave issuing `iters` rounds of 4
 * independent v_mfma_f32_32x32x16 (VA_F16 or VA_BF16) MFMAs, i.e. blocks * 4 * iters * 4 * 32768
 * FLOPs; `sink` (blocks * 256 floats) receives one value per thread. va_probe_copy: dst = src over
 * `bytes` (a multiple of 16, both 16-byte aligned), 16 bytes per lane, `blocks` work-groups of
 * 256 threads striding over the buffer. */
int va_probe_mfma(int32_t dtype, int32_t blocks, int32_t iters, float* sink, void* stream);
int va_probe_copy(const void* src, void* dst, int64_t bytes, int32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VARLEN_ATTN_H_ */
