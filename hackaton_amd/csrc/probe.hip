// Throughput probes of the two machine ceilings that the benchmark quotes its roofline fractions
// against, measured on the box instead of taken from the data sheet: the issue rate of dense
// v_mfma_f32_32x32x16_{f16,bf16} (the instruction every attention kernel here is built on) and the
// HBM streaming rate of a 16-byte-per-lane copy. Diagnostic entry points for bench.py and for
// callers that calibrate a machine; they have no counterpart in the reference.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/varlen_attn.h"
#include "va_api_internal.h"
#include "va_common.h"

namespace va {
namespace {

constexpr int kProbeThreads = 256;  // 4 waves, one per SIMD of the CU that takes the block

// Every wave issues `iters` rounds of 4 MFMAs into 4 independent accumulators (a 32x32x16 MFMA
// occupies the SIMD's matrix pipe for 32 cycles at its peak rate and its result is read only
// 4 issues later, so the pipe never waits on a dependency); the operands come from the thread
// index so that nothing folds, and one float per thread leaves the kernel so that nothing is
// dead.
template <class E>
__global__ __launch_bounds__(kProbeThreads) void mfma_probe_kernel(int iters, float* __restrict__ sink) {
  const uint32_t t = threadIdx.x + 1u;
  const u32x4 a = u32x4{0x3c003c00u ^ t, 0x3c003c00u, 0x38003800u, 0x3c00u ^ (t << 16)};
  const u32x4 b = u32x4{0x38003800u, 0x3c003c00u ^ t, 0x3c003c00u, 0x38003800u};
  f32x16 c0 = f32x16{}, c1 = f32x16{}, c2 = f32x16{}, c3 = f32x16{};
  for (int i = 0; i < iters; ++i) {
    c0 = E::mfma(a, b, c0);
    c1 = E::mfma(b, a, c1);
    c2 = E::mfma(a, a, c2);
    c3 = E::mfma(b, b, c3);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  sink[(long)blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

// dst = src, 16 bytes per lane, grid-stride: each thread loads 4 chunks (4 strides apart) before
// it stores them, so that every wave keeps 4 loads in flight.
__global__ __launch_bounds__(kProbeThreads) void copy_probe_kernel(const u32x4* __restrict__ src,
                                                                   u32x4* __restrict__ dst,
                                                                   long n16) {
  const long stride = (long)gridDim.x * kProbeThreads;
  for (long i = (long)blockIdx.x * kProbeThreads + threadIdx.x; i < n16; i += 4 * stride) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i + j * stride < n16) v[j] = src[i + j * stride];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i + j * stride < n16) __builtin_nontemporal_store(v[j], dst + i + j * stride);
  }
}

}  // namespace
}  // namespace va

extern "C" int va_probe_mfma(int32_t dtype, int32_t blocks, int32_t iters, float* sink,
                             void* stream) {
  if (dtype != VA_F16 && dtype != VA_BF16)
    return va::fail(VA_EDTYPE, "va_probe_mfma: dtype %d (VA_F16 or VA_BF16)", dtype);
  if (blocks <= 0 || iters <= 0)
    return va::fail(VA_EINVAL, "va_probe_mfma: blocks and iters must be positive");
  if (sink == nullptr) return va::fail(VA_EINVAL, "va_probe_mfma: sink is NULL");
  if (dtype == VA_F16)
    hipLaunchKernelGGL(va::mfma_probe_kernel<va::F16>, dim3(blocks), dim3(va::kProbeThreads), 0,
                       (hipStream_t)stream, iters, sink);
  else
    hipLaunchKernelGGL(va::mfma_probe_kernel<va::BF16>, dim3(blocks), dim3(va::kProbeThreads), 0,
                       (hipStream_t)stream, iters, sink);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VA_OK : va::fail((int)e, "va_probe_mfma launch: %s", hipGetErrorString(e));
}

extern "C" int va_probe_copy(const void* src, void* dst, int64_t bytes, int32_t blocks,
                             void* stream) {
  if (src == nullptr || dst == nullptr) return va::fail(VA_EINVAL, "va_probe_copy: NULL buffer");
  if (bytes < 0 || bytes % 16 != 0 || blocks <= 0)
    return va::fail(VA_EINVAL, "va_probe_copy: bytes must be a multiple of 16, blocks positive");
  if (((uintptr_t)src | (uintptr_t)dst) % 16 != 0)
    return va::fail(VA_EINVAL, "va_probe_copy: buffers must be 16-byte aligned");
  if (bytes == 0) return VA_OK;
  hipLaunchKernelGGL(va::copy_probe_kernel, dim3(blocks), dim3(va::kProbeThreads), 0,
                     (hipStream_t)stream, (const va::u32x4*)src, (va::u32x4*)dst, bytes / 16);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VA_OK : va::fail((int)e, "va_probe_copy launch: %s", hipGetErrorString(e));
}
