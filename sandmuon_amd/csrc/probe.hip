// MFMA peak probe (a measurement aid, no counterpart in the reference): the
// sustained dense MFMA rate of the device and the engine clock it holds
// under that load, for the roofline denominators of the S8 GEMMs.
//
// Every wave issues `iters` rounds of kChains independent MFMAs on
// register operands (no memory traffic in the loop; kChains accumulator
// chains cover the MFMA latency) and, from lane 0 of wave 0, stores the
// block's s_memtime (engine clock cycles) and s_memrealtime (a constant
// 100 MHz counter) at its start and end, from which the host derives the
// clock the chip held.  The accumulators feed one store per lane, which a
// caller-visible value depends on, so the loop is not removed.
#include "common.h"

namespace smx {

typedef __bf16 bf16x8p __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8p __attribute__((ext_vector_type(8)));
typedef float f32x16p __attribute__((ext_vector_type(16)));

constexpr int kProbeThreads = 512;  // 8 waves, two per SIMD
constexpr int kChains = 4;

template <int DT>
__global__ void __launch_bounds__(kProbeThreads) mfma_peak_kernel(int64_t iters, uint64_t *times, float *sink) {
  const int lane = threadIdx.x & 63;
  f32x16p acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[c][e] = 0.f;
  // Small operands (exact in every format) so the accumulators stay finite.
  const float base = 1.0f / 1024.0f * static_cast<float>((lane & 7) + 1);
  bf16x8p ab;
  f16x8p ah;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    ab[q] = static_cast<__bf16>(base);
    ah[q] = static_cast<_Float16>(base);
  }
  const float af = base, bf = -base;
  uint64_t t0 = 0, r0 = 0;
  if (threadIdx.x == 0) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
      if constexpr (DT == SMX_BF16) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, ab, acc[c], 0, 0, 0);
      else if constexpr (DT == SMX_F16) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ah, acc[c], 0, 0, 0);
      else acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(af, bf, acc[c], 0, 0, 0);
    }
  }
  if (threadIdx.x == 0) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    uint64_t *t = times + 4 * static_cast<int64_t>(blockIdx.x);
    t[0] = t0;
    t[1] = t1;
    t[2] = r0;
    t[3] = r1;
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[c][e];
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = s;
}

}  // namespace smx

using namespace smx;

extern "C" int smx_mfma_peak(int32_t dtype, int32_t blocks, int64_t iters, uint64_t *times, float *sink,
                             void *stream) {
  SMX_REQUIRE(dtype == SMX_F32 || dtype == SMX_BF16 || dtype == SMX_F16, SMX_EDTYPE,
              "mfma_peak: dtype must be SMX_F32, SMX_BF16 or SMX_F16");
  SMX_REQUIRE(blocks >= 1 && iters >= 1, SMX_EINVAL, "mfma_peak: need blocks >= 1 and iters >= 1");
  SMX_REQUIRE(times && sink, SMX_EINVAL, "mfma_peak: times and sink are required");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SMX_BF16)
    hipLaunchKernelGGL(mfma_peak_kernel<SMX_BF16>, dim3(blocks), dim3(kProbeThreads), 0, st, iters, times, sink);
  else if (dtype == SMX_F16)
    hipLaunchKernelGGL(mfma_peak_kernel<SMX_F16>, dim3(blocks), dim3(kProbeThreads), 0, st, iters, times, sink);
  else
    hipLaunchKernelGGL(mfma_peak_kernel<SMX_F32>, dim3(blocks), dim3(kProbeThreads), 0, st, iters, times, sink);
  return check_launch("mfma_peak");
}
