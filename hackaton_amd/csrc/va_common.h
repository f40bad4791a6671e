// Shared device helpers for the gfx950 varlen attention kernels: element types, the
// v_mfma_f32_32x32x16_{f16,bf16} wrappers, the lane <-> row maps of a 32x32 MFMA block and the
// XOR swizzles of the LDS tiles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "va_kernels.h"

namespace va {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Element tag: 16-bit storage, fp32 arithmetic.
struct F16 {
  static constexpr int kId = 0;
  __device__ static inline float to_f32(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  __device__ static inline uint16_t from_f32(float x) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // acc + the two 16-bit values packed in x (v_dot2_f32_f16 with (1, 1)).
  __device__ static inline float sum2(uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), f16x2_t{1, 1}, acc, false);
  }
  // acc + x.lo * y.lo + x.hi * y.hi in fp32 (v_dot2_f32_f16).
  __device__ static inline float dot2(uint32_t x, uint32_t y, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, y),
                                  acc, false);
  }
};

struct BF16 {
  static constexpr int kId = 1;
  __device__ static inline float to_f32(uint16_t x) {
    return __builtin_bit_cast(float, (uint32_t)x << 16);
  }
  __device__ static inline uint16_t from_f32(float x) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // acc + the two 16-bit values packed in x (v_dot2_f32_bf16 with (1, 1)).
  __device__ static inline float sum2(uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), bf16x2_t{1, 1}, acc,
                                           false);
  }
  // acc + x.lo * y.lo + x.hi * y.hi in fp32 (v_dot2_f32_bf16).
  __device__ static inline float dot2(uint32_t x, uint32_t y, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x),
                                           __builtin_bit_cast(bf16x2_t, y), acc, false);
  }
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> one register of two 16-bit values, round to nearest even
// (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 on gfx950).
template <class E>
__device__ inline uint32_t pack2(float lo, float hi) {
  if constexpr (E::kId == 0) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
}

// Eight fp32 values -> one MFMA operand register quad (8 x 16-bit).
template <class E>
__device__ inline u32x4 pack8(float a0, float a1, float a2, float a3, float a4, float a5,
                              float a6, float a7) {
  u32x4 r;
  r[0] = pack2<E>(a0, a1);
  r[1] = pack2<E>(a2, a3);
  r[2] = pack2<E>(a4, a5);
  r[3] = pack2<E>(a6, a7);
  return r;
}

// Value of lane (l ^ 32) combined with this lane's own. v_permlane32_swap exchanges the upper 32
// lanes of its first operand with the lower 32 lanes of its second: with both holding x, lane l
// ends up with {x[l], x[l ^ 32]} across the two registers. The instruction is emitted through
// inline asm (with the 2 wait states a VALU-written source needs): the compiler's model of the
// intrinsic treats the two results as interchangeable and drops one of them.
__device__ inline void swap_halves(float x, float& r0, float& r1) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ inline float max_with_other_half(float x) {
  float r0, r1;
  swap_halves(x, r0, r1);
  return fmaxf(r0, r1);
}
__device__ inline float sum_with_other_half(float x) {
  float r0, r1;
  swap_halves(x, r0, r1);
  return r0 + r1;
}
// Sum over each group of 16 lanes (a DPP row), the same value in all 16: four DPP adds (swap
// within pairs, within quads, mirror within 8, mirror within 16) instead of LDS permutes.
template <int kCtrl>
__device__ inline float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}
__device__ inline float sum_rows16(float x) {
  x += dpp_mov<0xb1>(x);   // quad_perm [1, 0, 3, 2]
  x += dpp_mov<0x4e>(x);   // quad_perm [2, 3, 0, 1]
  x += dpp_mov<0x141>(x);  // row_half_mirror
  x += dpp_mov<0x140>(x);  // row_mirror
  return x;
}

// ---------------------------------------------------------------------------------------------
// 32x32x16 MFMA block layout (64 lanes, lane = 32 * hi + l32):
//   A operand (32 rows x 16 k): lane supplies row l32, k slots [8 hi, 8 hi + 8)
//   B operand (16 k x 32 cols): lane supplies col l32, k slots [8 hi, 8 hi + 8)
//   C/D (32 x 32, 16 fp32 per lane): register j holds row 8 (j >> 2) + 4 hi + (j & 3), col l32
// The k order inside one MFMA is free as long as A and B agree, so every operand that is a
// reduction axis of the next product is loaded with rows permuted by `perm32`: then register j
// of lane half hi holds logical row `reg_row(j, hi)` = 16 (j >> 3) + 8 hi + (j & 7), i.e. the 8
// registers [8c, 8c + 8) are 8 consecutive rows, exactly the k slots of the next MFMA.
// ---------------------------------------------------------------------------------------------
__device__ __host__ inline int perm32(int r) {  // physical row r = 8g + 4h + i -> logical row
  const int g = r >> 3, h = (r >> 2) & 1, i = r & 3;
  return 16 * (g >> 1) + 8 * h + 4 * (g & 1) + i;
}
__device__ __host__ inline int reg_row(int j, int hi) { return 16 * (j >> 3) + 8 * hi + (j & 7); }

// ---------------------------------------------------------------------------------------------
// LDS access through address-space-3 pointers, so that per-lane bases plus compile-time offsets
// fold into the ds instruction's immediate offset.
//
// ds_read_b64_tr_b16 (gfx950 transposed read): within each group of 16 lanes, source lane i reads
// 4 consecutive 16-bit values at its address; destination lane j receives element (j & 3) of the
// values read by source lanes 4e + (j >> 2), e = 0..3. With source lane i pointing at row
// (r0 + 2 (i >> 2)) and columns [c0 + 4 (i & 3), +4), lane j receives column c0 + j of the 4 rows
// r0, r0 + 2, r0 + 4, r0 + 6: a column of a row-major tile, i.e. 4 k slots of an MFMA operand
// whose k axis runs along the tile's rows. Two such reads (r0 and r0 + 1) give the 8 k slots of
// one 32x32x16 operand in the slot order {0, 2, 4, 6, 1, 3, 5, 7}.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ inline u32x4 ld128(const lds_u16* p) { return *reinterpret_cast<const lds_u32x4*>(p); }
__device__ inline void st128(lds_u16* p, u32x4 v) { *reinterpret_cast<lds_u32x4*>(p) = v; }
__device__ inline u32x2 ldtr(const lds_u16* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (lds_s16x4*)const_cast<lds_u16*>(p)));
}
// One 8-slot operand from two transposed reads at rows r0 (slots 0,2,4,6) and r0 + 1 (1,3,5,7).
__device__ inline u32x4 ldtr8(const lds_u16* p_r0, int row_stride) {
  const u32x2 a = ldtr(p_r0), b = ldtr(p_r0 + row_stride);
  return u32x4{a[0], a[1], b[0], b[1]};
}
// Register operand in the matching slot order: values v[0..7] of 8 consecutive k indices.
template <class E>
__device__ inline u32x4 pack8_tr(const float* v) {
  return pack8<E>(v[0], v[2], v[4], v[6], v[1], v[3], v[5], v[7]);
}

__device__ inline u32x4 gload16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Raw buffer resource over [base, base + bytes) (wave-uniform operands, built in SGPRs): a load at
// a byte offset >= bytes returns zeros, which bounds a tile's rows without per-lane clamping, and
// the per-lane offset is a 32-bit VGPR that stays fixed while the base moves tile by tile.
// 0x00020000: the gfx9 buffer descriptor's dword-3 format field for untyped 32-bit data.
typedef __amdgpu_buffer_rsrc_t brsrc;
__device__ inline brsrc make_rsrc(const void* base, long bytes) {
  const int n = bytes <= 0 ? 0 : (bytes >= 0x7fffffffL ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
__device__ inline u32x4 bload16(brsrc r, int byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
// Buffer load straight into LDS (gfx950 buffer_load_dwordx4 ... lds): lane i's 16 bytes land at
// lds_byte + 16 i (M0 holds the wave-uniform base), rows past the buffer's end as zeros;
// completion is counted by vmcnt. Issued as inline assembly, invisible to the compiler's
// wait-count tracking: the compiler treats an LDS-writing buffer load as a possible writer of
// every later transposed LDS read and waits for it to land before each one, which would
// serialise the copy of the next tile with the MFMAs of the current one. Callers order the copies
// themselves: wait_vmcnt and a barrier before any wave reads the destination, and the destination
// not read by any wave since the last barrier. `rsrc` is a buffer descriptor in SGPRs
// (make_rsrc4), `lds_byte` the LDS byte address of lane 0's 16 bytes.
__device__ inline void dma16_opaque(u32x4 rsrc, uint32_t lds_byte, int byte_off) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_byte), "v"(byte_off), "s"(rsrc)
               : "m0");
}
__device__ inline u32x4 make_rsrc4(const void* base, long bytes) {
  const unsigned long long a = (unsigned long long)base;
  const int n = bytes <= 0 ? 0 : (bytes >= 0x7fffffffL ? 0x7fffffff : (int)bytes);
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, (uint32_t)n, 0x00020000u};
}
__device__ inline uint32_t lds_addr(const lds_u16* p) { return (uint32_t)(uintptr_t)p; }
// s_waitcnt vmcnt(N): at most N vector-memory operations of this wave still outstanding.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// XOR swizzle of the 16 chunks (16 bytes each) of a 256-byte LDS row r: chunk c is stored at
// c ^ swz16(r). swz16 is a bijection on r mod 16, so the 16 rows that one ds_read_b128 group of
// lanes reads through perm32 hit 16 different chunks; and for the rows {r0 + 2m} (m = 0..3) of a
// ds_read_b64_tr_b16 group, bits 2-3 of the swizzle are m, so 4 aligned chunks of each row land
// on 4 disjoint bank groups.
__device__ __host__ inline int swz16(int r) {
  return (((r >> 1) & 3) << 2) | ((r & 1) << 1) | ((r >> 3) & 1);
}
// Result stores are non-temporal (`nt`): the kernels write each output once and never read it
// back, so the lines stream out during the kernel instead of sitting dirty in L2 until the
// write-back at the kernel's end (config 2: forward -1.4 us, backward -1.5 us per call).
__device__ inline void gstore16(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Stores a wave's 32 rows x 8C columns (16-bit) through an LDS row tile (32 x (8C + 8) halfs,
// used by this wave only): lane (l32, hi) holds in w[i] the columns 8 (2 i + hi) + 0..7 of row
// l32. Each global store instruction then writes 64 / C whole rows of 16 C bytes (C lanes x 16
// bytes per row) instead of 32-byte pieces of 32 rows. Rows >= n_rows are skipped; row_ptr(r)
// is the global address of column 0 of row r, and tile column c (a multiple of 8) goes to
// global column col_map(c).
struct SameColumn {
  __device__ int operator()(int col) const { return col; }
};
template <int C, class RowPtr, class ColMap = SameColumn>
__device__ inline void store_rows32(lds_u16* tile, const u32x4 (&w)[C / 2], int lane,
                                    RowPtr row_ptr, int n_rows, ColMap col_map = ColMap{}) {
  static_assert(C == 4 || C == 8 || C == 16, "32, 64 or 128 columns");
  constexpr int LT = 8 * C + 8;
  const int l32 = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int i = 0; i < C / 2; ++i) st128(tile + l32 * LT + 8 * (2 * i + hi), w[i]);
  const int r0 = lane / C, col = 8 * (lane % C);
#pragma unroll
  for (int i = 0; i < C / 2; ++i) {
    const int r = (64 / C) * i + r0;
    const u32x4 v = ld128(tile + r * LT + col);
    if (r < n_rows) gstore16(row_ptr(r) + col_map(col), v);
  }
}

__device__ inline uint16_t half_of(const u32x4& v, int e) {
  const uint32_t w = v[e >> 1];
  return (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu));
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier (LLVM AMDGPU IGroupLP).
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedVmemRead = 0x020,
              kSchedDsRead = 0x100, kSchedDsWrite = 0x200;
#define VA_SCHED(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Makes the wave wait here until the loads that write `v` have landed. Operands loaded once before
// a loop and used inside it must be complete at the loop entry: otherwise the counter-based wait
// inserted before their first use in the loop also waits, on every iteration, for the loads that
// the loop itself has issued since (the wait counters complete in order).
__device__ inline void settle(const u32x4& v) { asm volatile("" ::"v"(v)); }

// ---------------------------------------------------------------------------------------------
// Rotary embedding of a (x[d], x[d + 64]) pair in fp32 with tables c1 = cos[d], c2 = cos[d + 64],
// s1 = sin[d], s2 = sin[d + 64] (solution/attention.py:57-63), and its inverse, the gradient of the
// unrotated pair (attention.py:125-134). Written with explicit fused multiply-adds, so that every
// kernel that rotates (the standalone rotary kernels and the attention kernels' epilogues) rounds
// the same way.
// ---------------------------------------------------------------------------------------------
__device__ inline void rope_rotate(float x1, float x2, float c1, float c2, float s1, float s2,
                                   float& y1, float& y2) {
  y1 = __builtin_fmaf(x1, c1, -(x2 * s1));
  y2 = __builtin_fmaf(x2, c2, x1 * s2);
}
__device__ inline void rope_unrotate(float d1, float d2, float c1, float c2, float s1, float s2,
                                     float& o1, float& o2) {
  o1 = __builtin_fmaf(d1, c1, d2 * s2);
  o2 = __builtin_fmaf(d2, c2, -(d1 * s1));
}

// The table row (element offset) of a packed token.
__device__ inline long rope_row(const RopeTab& r, int token) {
  return (long)r.b_idx[token] * r.scb + (long)r.t_idx[token] * r.sct;
}
// The tables of 8 (d, d + 64) pairs, d = d0 .. d0 + 7 (d0 < 64, a multiple of 8), of one row:
// loaded apart from their use, so that an epilogue can issue them before it waits for anything.
struct Tab8 {
  f32x4 c1[2], c2[2], s1[2], s2[2];
};
__device__ inline Tab8 load_tab8(const RopeTab& r, long row, int d0) {
  const f32x4* c1 = reinterpret_cast<const f32x4*>(r.cos + row + d0);
  const f32x4* c2 = reinterpret_cast<const f32x4*>(r.cos + row + 64 + d0);
  const f32x4* s1 = reinterpret_cast<const f32x4*>(r.sin + row + d0);
  const f32x4* s2 = reinterpret_cast<const f32x4*>(r.sin + row + 64 + d0);
  return Tab8{{c1[0], c1[1]}, {c2[0], c2[1]}, {s1[0], s1[1]}, {s2[0], s2[1]}};
}
// Inverse rotation, in place, of the 8 (x[e], x[8 + e]) pairs of one lane: x[e] holds element
// d0 + e of a row, x[8 + e] element d0 + 64 + e, `t` their tables.
__device__ inline void rope_unrotate8(const Tab8& t, float* x) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    rope_unrotate(x[e], x[8 + e], t.c1[e >> 2][e & 3], t.c2[e >> 2][e & 3], t.s1[e >> 2][e & 3],
                  t.s2[e >> 2][e & 3], x[e], x[8 + e]);
}
__device__ inline void rope_unrotate8(const RopeTab& r, long row, int d0, float* x) {
  rope_unrotate8(load_tab8(r, row, d0), x);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace va
