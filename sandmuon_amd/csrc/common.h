// Shared device/host helpers for the SandMuon gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/sandmuon_amd.h"

namespace smx {

// ------------------------------------------------------------ errors ---
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int check_launch(const char *what);
// Writes `bytes` (a multiple of 4) from host memory `src` to device memory
// `dst` in order on `st`, through the kernel arguments of one small launch
// per 3840 bytes: no host memory is read after the call returns, and the
// host never waits for the device (a hipMemcpyAsync from pinned memory was
// seen to block the calling thread for milliseconds, long enough to leave
// the GPU idle behind it).
int upload_table(void *dst, const void *src, size_t bytes, hipStream_t st);

#define SMX_REQUIRE(cond, code, msg)                                        \
  do {                                                                      \
    if (!(cond)) return ::smx::fail((code), (msg));                         \
  } while (0)

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// ------------------------------------------------------- element I/O ---
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even FP32 -> BF16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, sizeof(v));
  return static_cast<float>(v);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void *p, int64_t i) {
  if constexpr (DT == SMX_F32) {
    return static_cast<const float *>(p)[i];
  } else if constexpr (DT == SMX_BF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  } else {
    return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  }
}

// A parameter element of dtype `dt` (SMX_F32, SMX_BF16 or SMX_F16).
__device__ __forceinline__ float load_any(const void *p, int dt, int64_t i) {
  if (dt == SMX_F32) return load_elem<SMX_F32>(p, i);
  if (dt == SMX_BF16) return load_elem<SMX_BF16>(p, i);
  return load_elem<SMX_F16>(p, i);
}

// v rounded to nearest even in dtype `dt` and widened back to FP32.
__device__ __forceinline__ float round_to(int dt, float v) {
  if (dt == SMX_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dt == SMX_F16) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

// Stores v (already representable in `dt`, see round_to) as dtype `dt`.
__device__ __forceinline__ void store_any(void *p, int dt, int64_t i, float v) {
  if (dt == SMX_F32) {
    static_cast<float *>(p)[i] = v;
  } else if (dt == SMX_BF16) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  } else {
    const _Float16 h = static_cast<_Float16>(v);
    static_cast<_Float16 *>(p)[i] = h;
  }
}

// ---------------------------------------------------- wave reductions ---
// Sum over the 64 lanes of a fully active wave, the same value in every
// lane.  Within each row of 16 lanes four DPP moves (quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror) pair every lane with
// its partner, so every lane of a row ends with the row sum; the four row
// sums are then read from lanes 0, 16, 32 and 48 and added in a fixed
// order.  No LDS round trips.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, dpp_mov<CTRL>(__builtin_bit_cast(uint32_t, v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_mov(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_mov<CTRL>(static_cast<uint32_t>(b)), hi = dpp_mov<CTRL>(static_cast<uint32_t>(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
template <typename T>
__device__ __forceinline__ T read_lane(T v, int lane) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
    return __builtin_bit_cast(T, lo | (hi << 32));
  }
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "float or double");
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}

// Block-wide sum; every thread receives the result.  `scratch` must hold
// one T per wave (blockDim.x / 64 <= 16).
template <typename T>
__device__ __forceinline__ T block_sum(T v, T *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  T t = 0;
  for (int w = 0; w < nw; ++w) t += scratch[w];
  return t;
}

}  // namespace smx
