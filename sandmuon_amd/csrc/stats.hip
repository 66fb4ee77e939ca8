// Per-channel statistics for the SandMuon hooks and their step-time finish.
//
//  * stats_accumulate: the hook bodies of sandmuon/optimizer.py:156-168 and
//    :171-177 (sum of x^2, and sum of x for the rank-one A variant), as one
//    HBM pass.  Each block owns a (row chunk, column tile) and adds its FP32
//    partial into slot row `chunk`, so the result is deterministic and no
//    atomics or tail combine are needed in the hook.
//  * stats_fold: sum += sum over slot rows (FP64), slots zeroed.
//  * stats_finish: _finish_a/_finish_b (sandmuon/optimizer.py:182-222) with
//    rank1_inverse_sqrt (:27-35) and diagonal_inverse_sqrt (:19-24).
#include "common.h"

#include <algorithm>
#include <cfloat>
#include <vector>

namespace smx {

constexpr int kStatsThreads = 512;
constexpr int kStatsWaves = kStatsThreads / 64;

template <int DT, int VEC>
struct VecLoad;

template <>
struct VecLoad<SMX_F32, 4> {
  __device__ __forceinline__ static void load(const void *p, int64_t i, float *v) {
    float4 q = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
};

template <int DT>
struct VecLoad2B8 {
  __device__ __forceinline__ static void load(const void *p, int64_t i, float *v) {
    uint4 q = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == SMX_BF16) {
        v[2 * k] = __uint_as_float(w[k] << 16);
        v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      } else {
        v[2 * k] = f16_bits_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
        v[2 * k + 1] = f16_bits_to_f32(static_cast<uint16_t>(w[k] >> 16));
      }
    }
  }
};
template <>
struct VecLoad<SMX_BF16, 8> : VecLoad2B8<SMX_BF16> {};
template <>
struct VecLoad<SMX_F16, 8> : VecLoad2B8<SMX_F16> {};

template <int DT>
struct VecLoad1 {
  __device__ __forceinline__ static void load(const void *p, int64_t i, float *v) {
    v[0] = load_elem<DT>(p, i);
  }
};
template <>
struct VecLoad<SMX_F32, 1> : VecLoad1<SMX_F32> {};
template <>
struct VecLoad<SMX_BF16, 1> : VecLoad1<SMX_BF16> {};
template <>
struct VecLoad<SMX_F16, 1> : VecLoad1<SMX_F16> {};

// What a launch produces besides sum(x^2) into the slot rows.
enum StatsMode : int {
  kSqOnly = 0,    // B side, diagonal A
  kSqFirst = 1,   // rank-one A: sum(x) into its own slot rows
  kSqColsum = 2,  // sum(x) of this call's rows into per-chunk partials (a bias gradient)
};

struct StatsArgs {
  const void *x;
  int64_t rows, cols, row_stride, rows_per_chunk;
  float *slots_sq;
  float *first;        // kSqFirst: slot rows of sum(x); kSqColsum: per-chunk partials, plain stores
  void *cast_out;      // CAST: low-precision copy of x
  int64_t out_stride;
};

template <int CAST, int VEC>
__device__ __forceinline__ void store_cast(void *out, int64_t i, const float *v) {
  uint16_t h[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    if constexpr (CAST == SMX_BF16) {
      h[k] = f32_to_bf16_bits(v[k]);
    } else {
      const _Float16 f = static_cast<_Float16>(v[k]);
      __builtin_memcpy(&h[k], &f, sizeof(f));
    }
  }
  uint16_t *o = static_cast<uint16_t *>(out) + i;
  if constexpr (VEC == 4) {
    *reinterpret_cast<uint2 *>(o) = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                               h[2] | (static_cast<uint32_t>(h[3]) << 16));
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = h[k];
  }
}

// grid = (column tiles, row chunks); block = kStatsThreads.
// A column tile is CT lanes x VEC channels; a wave covers 64/CT rows per
// step, the block kStatsWaves*64/CT rows per step.  CAST (SMX_BF16 or
// SMX_F16, fp32 input only) also writes x converted, as the mixed-precision
// cast in front of a Linear would.  MODE and CAST change nothing in how
// sum(x^2) is formed, so every variant adds the same bits to the slots.
template <int DT, int VEC, int CT, int MODE, int CAST>
__global__ void __launch_bounds__(kStatsThreads) stats_accumulate_kernel(StatsArgs a) {
  constexpr bool FIRST = MODE != kSqOnly;
  constexpr int RPW = 64 / CT;                 // rows per wave step
  constexpr int GROUPS = kStatsWaves * RPW;    // row groups per block
  constexpr int TW = CT * VEC;                 // channels per tile
  __shared__ float red_sq[GROUPS][TW];
  __shared__ float red_first[FIRST ? GROUPS : 1][FIRST ? TW : 1];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int group = wave * RPW + lane / CT;
  const int64_t vcol = static_cast<int64_t>(blockIdx.x) * CT + (lane % CT);
  const int64_t col0 = vcol * VEC;
  const int64_t r_begin = static_cast<int64_t>(blockIdx.y) * a.rows_per_chunk;
  const int64_t r_end = min(a.rows, r_begin + a.rows_per_chunk);
  const bool empty = r_begin >= r_end;
  // An empty chunk adds nothing; with kSqColsum it still writes its zero
  // partial.
  if (MODE != kSqColsum && empty) return;
  const bool active = col0 < a.cols;

  float acc_sq[VEC], acc_first[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) { acc_sq[k] = 0.f; acc_first[k] = 0.f; }

  if (active) {
    // Loads in flight per thread: 2 for the narrow tiles (measured 8% faster
    // on 768-wide bf16 inputs), 4 otherwise.
    constexpr int U = CT == 16 ? 2 : 4;
    int64_t r = r_begin + group;
    for (; r + (U - 1) * GROUPS < r_end; r += U * GROUPS) {
      float v[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u)
        VecLoad<DT, VEC>::load(a.x, (r + u * GROUPS) * a.row_stride + col0, v[u]);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          acc_sq[k] = fmaf(v[u][k], v[u][k], acc_sq[k]);
          if constexpr (FIRST) acc_first[k] += v[u][k];
        }
      if constexpr (CAST != 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) store_cast<CAST, VEC>(a.cast_out, (r + u * GROUPS) * a.out_stride + col0, v[u]);
      }
    }
    for (; r < r_end; r += GROUPS) {
      float v[VEC];
      VecLoad<DT, VEC>::load(a.x, r * a.row_stride + col0, v);
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        acc_sq[k] = fmaf(v[k], v[k], acc_sq[k]);
        if constexpr (FIRST) acc_first[k] += v[k];
      }
      if constexpr (CAST != 0) store_cast<CAST, VEC>(a.cast_out, r * a.out_stride + col0, v);
    }
  }
  const int cl = (lane % CT) * VEC;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    red_sq[group][cl + k] = acc_sq[k];
    if constexpr (FIRST) red_first[group][cl + k] = acc_first[k];
  }
  __syncthreads();
  const int64_t tile_col0 = static_cast<int64_t>(blockIdx.x) * TW;
  const int64_t row_off = static_cast<int64_t>(blockIdx.y) * a.cols + tile_col0;
  float *slot_sq = a.slots_sq + row_off;
  float *first = FIRST ? a.first + row_off : nullptr;
  for (int c = threadIdx.x; c < TW; c += kStatsThreads) {
    if (tile_col0 + c >= a.cols) break;
    float s = 0.f, f = 0.f;
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
      s += red_sq[g][c];
      if constexpr (FIRST) f += red_first[g][c];
    }
    if (!empty) slot_sq[c] += s;
    if constexpr (MODE == kSqFirst) first[c] += f;
    if constexpr (MODE == kSqColsum) first[c] = f;
  }
}

template <int DT, int VEC, int CT, int MODE, int CAST>
static void launch_acc(StatsArgs a, int32_t n_slots, hipStream_t st) {
  const int64_t vcols = ceil_div(a.cols, VEC);
  dim3 grid(static_cast<unsigned>(ceil_div(vcols, CT)), static_cast<unsigned>(n_slots));
  a.rows_per_chunk = ceil_div(a.rows, n_slots);
  hipLaunchKernelGGL((stats_accumulate_kernel<DT, VEC, CT, MODE, CAST>), grid, dim3(kStatsThreads), 0, st, a);
}

template <int DT, int VEC, int MODE, int CAST>
static void dispatch_ct(const StatsArgs &a, int32_t n_slots, hipStream_t st) {
  // The widest column tile that still gives >= 6 tiles, so that a hook call
  // of 16K rows puts >= 768 blocks (24 waves per CU) in flight.
  const int64_t vcols = ceil_div(a.cols, VEC);
  if (vcols >= 6 * 64)
    launch_acc<DT, VEC, 64, MODE, CAST>(a, n_slots, st);
  else if (vcols >= 6 * 32)
    launch_acc<DT, VEC, 32, MODE, CAST>(a, n_slots, st);
  else
    launch_acc<DT, VEC, 16, MODE, CAST>(a, n_slots, st);
}

template <int MODE, int CAST>
static void dispatch_dtype(const StatsArgs &a, int dtype, int32_t n_slots, hipStream_t st) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(a.x);
  if (dtype == SMX_F32) {
    bool v4 = a.cols % 4 == 0 && a.row_stride % 4 == 0 && addr % 16 == 0;
    if (CAST != 0) v4 = v4 && a.out_stride % 4 == 0 && reinterpret_cast<uintptr_t>(a.cast_out) % 8 == 0;
    if (v4) dispatch_ct<SMX_F32, 4, MODE, CAST>(a, n_slots, st);
    else dispatch_ct<SMX_F32, 1, MODE, CAST>(a, n_slots, st);
    return;
  }
  if constexpr (CAST == 0) {
    const bool v8 = a.cols % 8 == 0 && a.row_stride % 8 == 0 && addr % 16 == 0;
    if (dtype == SMX_BF16) {
      if (v8) dispatch_ct<SMX_BF16, 8, MODE, 0>(a, n_slots, st);
      else dispatch_ct<SMX_BF16, 1, MODE, 0>(a, n_slots, st);
    } else {
      if (v8) dispatch_ct<SMX_F16, 8, MODE, 0>(a, n_slots, st);
      else dispatch_ct<SMX_F16, 1, MODE, 0>(a, n_slots, st);
    }
  }
}

// colsum[c] = sum over the n_parts partial rows (stride cols) in FP64.
// grid = ceil(cols / 64) blocks of 256: wave w sums rows w, w+4, ... of 64
// columns (one 256-byte row segment per load, 8 loads in flight); the four
// wave sums are added in wave order, so the result is deterministic.
__global__ void __launch_bounds__(256)
colsum_fold_kernel(const float *__restrict__ partial, int64_t cols, int32_t n_parts, float *__restrict__ colsum) {
  constexpr int kFold = 8;
  __shared__ double part[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  double t = 0.0;
  if (c < cols) {
    int p = wave;
    for (; p + 4 * (kFold - 1) < n_parts; p += 4 * kFold) {
      float v[kFold];
#pragma unroll
      for (int u = 0; u < kFold; ++u) v[u] = partial[static_cast<int64_t>(p + 4 * u) * cols + c];
#pragma unroll
      for (int u = 0; u < kFold; ++u) t += static_cast<double>(v[u]);
    }
    for (; p < n_parts; p += 4) t += static_cast<double>(partial[static_cast<int64_t>(p) * cols + c]);
  }
  part[wave][lane] = t;
  __syncthreads();
  if (wave == 0 && c < cols)
    colsum[c] = static_cast<float>((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]));
}

// ------------------------------------------------------------- fold ---
// grid = ceil(n / 256) blocks of 256: sum[c] += sum_p slots[p][c] (FP64).
__device__ __forceinline__ void fold_channel(float *sum, float *slots, int64_t n, int32_t n_slots,
                                             int64_t c) {
  double t = 0.0;
  for (int p = 0; p < n_slots; ++p) {
    float *s = slots + static_cast<int64_t>(p) * n + c;
    t += static_cast<double>(*s);
    *s = 0.f;
  }
  sum[c] = static_cast<float>(static_cast<double>(sum[c]) + t);
}

__global__ void __launch_bounds__(256)
stats_fold_kernel(float *sum_sq, float *slots_sq, float *sum_first, float *slots_first, int64_t n,
                  int32_t n_slots) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= n) return;
  fold_channel(sum_sq, slots_sq, n, n_slots, c);
  if (sum_first) fold_channel(sum_first, slots_first, n, n_slots, c);
}

// ----------------------------------------------------------- finish ---
constexpr int kFinishBatch = 32;  // descriptors per launch (by value)
struct FinishPack {
  smx_finish_desc d[kFinishBatch];
  int32_t n;
};
static_assert(sizeof(FinishPack) <= 4000, "FinishPack is passed by value in the kernel arguments");

// Fold pass over a batch of descriptors: grid.x enumerates 64-channel
// chunks of every vector, grid.y = descriptor.  Wave w of kFoldWaves sums
// slots w, w + kFoldWaves, ... of the chunk (coalesced 256-byte rows, all
// loads of the wave in flight together) and zeroes them; the wave partials
// are combined in a fixed order (FP64).
constexpr int kFoldWaves = 8;

__global__ void __launch_bounds__(64 * kFoldWaves) finish_fold_kernel(FinishPack pack) {
  __shared__ double part[2][kFoldWaves][64];
  const smx_finish_desc &d = pack.d[blockIdx.y];
  if (static_cast<int64_t>(blockIdx.x) * 64 >= d.n) return;  // uniform per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool ok = c < d.n;
  const int nv = d.kind == 1 ? 2 : 1;
  for (int v = 0; v < nv; ++v) {
    float *slots = v ? d.slots_first : d.slots_sq;
    double t = 0.0;
    if (ok) {
#pragma unroll 16
      for (int p = wave; p < d.n_slots; p += kFoldWaves) {
        float *s = slots + static_cast<int64_t>(p) * d.n + c;
        t += static_cast<double>(*s);
        *s = 0.f;
      }
    }
    part[v][wave][lane] = t;
  }
  __syncthreads();
  if (wave == 0 && ok) {
    for (int v = 0; v < nv; ++v) {
      float *sum = v ? d.sum_first : d.sum_sq;
      double t = 0.0;
#pragma unroll
      for (int w = 0; w < kFoldWaves; ++w) t += part[v][w][lane];
      sum[c] = static_cast<float>(static_cast<double>(sum[c]) + t);
    }
  }
}

__device__ __forceinline__ float ema_update(float e, float x, float beta, float omb) {
  // e.mul_(beta).add_(x, alpha=1-beta), both coefficients rounded from double
  return e * beta + x * omb;
}

// One block of kFinishThreads per descriptor.
constexpr int kFinishThreads = 1024;

__global__ void __launch_bounds__(kFinishThreads) finish_kernel(FinishPack pack, float beta, float omb) {
  __shared__ double scratch[16];
  const smx_finish_desc &d = pack.d[blockIdx.x];
  const int64_t n = d.n;
  const float cnt = static_cast<float>(d.count);
  const int t = threadIdx.x;
  if (d.kind == 2) {
    // b = sum/count; b /= max(mean(b), tiny); EMA; diagonal inverse sqrt.
    double part = 0.0;
    for (int64_t c = t; c < n; c += kFinishThreads) part += static_cast<double>(d.sum_sq[c] / cnt);
    const float bmean = static_cast<float>(block_sum(part, scratch) / static_cast<double>(n));
    const float den = fmaxf(bmean, FLT_MIN);
    double epart = 0.0;
    for (int64_t c = t; c < n; c += kFinishThreads) {
      const float b = (d.sum_sq[c] / cnt) / den;
      const float e = d.first ? b : ema_update(d.ema[c], b, beta, omb);
      d.ema[c] = e;
      epart += static_cast<double>(e);
    }
    const float em = static_cast<float>(block_sum(epart, scratch) / static_cast<double>(n));
    const float emc = fmaxf(em, FLT_MIN);
    for (int64_t c = t; c < n; c += kFinishThreads) {
      const float r = fmaxf(d.ema[c], em * 1e-6f) / emc;
      d.inv[c] = rsqrtf(fmaxf(r, 1e-6f));
      d.sum_sq[c] = 0.f;
    }
    return;
  }
  // A side: second = sum/count; EMA (first copies); factor.
  double epart = 0.0;
  for (int64_t c = t; c < n; c += kFinishThreads) {
    const float second = d.sum_sq[c] / cnt;
    const float e = d.first ? second : ema_update(d.ema[c], second, beta, omb);
    d.ema[c] = e;
    epart += static_cast<double>(e);
    if (d.kind == 1) {
      const float mean = d.sum_first[c] / cnt;
      d.mean_ema[c] = d.first ? mean : ema_update(d.mean_ema[c], mean, beta, omb);
      d.sum_first[c] = 0.f;
    }
    d.sum_sq[c] = 0.f;
  }
  const float em = static_cast<float>(block_sum(epart, scratch) / static_cast<double>(n));
  if (d.kind == 0) {
    const float emc = fmaxf(em, FLT_MIN);
    for (int64_t c = t; c < n; c += kFinishThreads) {
      const float r = fmaxf(d.ema[c], em * 1e-6f) / emc;
      d.inv[c] = rsqrtf(fmaxf(r, 1e-6f));
    }
    return;
  }
  // rank-one: q = max(mean(e), tiny); var = max(e - m^2, 0);
  // inv = rsqrt(max(var/q, 1e-6)); z = inv*m/sqrt(q); rho = sqrt(1+|z|^2);
  // kappa = -1/(rho(rho+1)).
  const float q = fmaxf(em, FLT_MIN);
  const float sq = sqrtf(q);
  double zpart = 0.0;
  for (int64_t c = t; c < n; c += kFinishThreads) {
    const float m = d.mean_ema[c];
    const float var = fmaxf(d.ema[c] - m * m, 0.f);
    const float inv = rsqrtf(fmaxf(var / q, 1e-6f));
    const float z = inv * (m / sq);
    d.inv[c] = inv;
    d.z[c] = z;
    zpart += static_cast<double>(z) * static_cast<double>(z);
  }
  const double zz = block_sum(zpart, scratch);
  if (t == 0) {
    const float rho = sqrtf(1.0f + static_cast<float>(zz));
    d.kappa[0] = -1.0f / (rho * (rho + 1.0f));
  }
}

}  // namespace smx

using namespace smx;

static int check_rows(const char *who, const void *x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                      const float *slots_sq, int32_t n_slots) {
  const std::string w(who);
  SMX_REQUIRE(rows >= 0 && cols >= 1, SMX_ESHAPE, w + ": need rows >= 0 and cols >= 1");
  SMX_REQUIRE(rows == 0 || x, SMX_EINVAL, w + ": null input");
  SMX_REQUIRE(rows == 0 || slots_sq, SMX_EINVAL, w + ": null slots_sq");
  SMX_REQUIRE(row_stride >= cols || rows <= 1, SMX_ESHAPE, w + ": row_stride must be >= cols");
  SMX_REQUIRE(n_slots >= 1 && n_slots <= 65535, SMX_EINVAL, w + ": n_slots in [1, 65535]");
  SMX_REQUIRE(dtype == SMX_F32 || dtype == SMX_BF16 || dtype == SMX_F16, SMX_EDTYPE,
              w + ": dtype must be f32, bf16 or f16");
  return SMX_OK;
}

extern "C" int smx_stats_accumulate(const void *x, int dtype, int64_t rows, int64_t cols,
                                    int64_t row_stride, float *slots_sq, float *slots_first,
                                    int32_t n_slots, void *stream) {
  int rc = check_rows("stats_accumulate", x, dtype, rows, cols, row_stride, slots_sq, n_slots);
  if (rc) return rc;
  if (rows == 0) return SMX_OK;  // empty microbatch: nothing to add
  const StatsArgs a{x, rows, cols, row_stride, 0, slots_sq, slots_first, nullptr, 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (slots_first) dispatch_dtype<kSqFirst, 0>(a, dtype, n_slots, st);
  else dispatch_dtype<kSqOnly, 0>(a, dtype, n_slots, st);
  return check_launch("stats_accumulate");
}

extern "C" int smx_stats_cast(const void *x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                              float *slots_sq, float *slots_first, int32_t n_slots, void *out,
                              int out_dtype, int64_t out_stride, void *stream) {
  int rc = check_rows("stats_cast", x, dtype, rows, cols, row_stride, slots_sq, n_slots);
  if (rc) return rc;
  SMX_REQUIRE(dtype == SMX_F32, SMX_EDTYPE, "stats_cast: the input must be f32");
  SMX_REQUIRE(out_dtype == SMX_BF16 || out_dtype == SMX_F16, SMX_EDTYPE, "stats_cast: out_dtype must be bf16 or f16");
  SMX_REQUIRE(rows == 0 || out, SMX_EINVAL, "stats_cast: null output");
  SMX_REQUIRE(out_stride >= cols || rows <= 1, SMX_ESHAPE, "stats_cast: out_stride must be >= cols");
  if (rows == 0) return SMX_OK;
  const StatsArgs a{x, rows, cols, row_stride, 0, slots_sq, slots_first, out, out_stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == SMX_BF16) {
    if (slots_first) dispatch_dtype<kSqFirst, SMX_BF16>(a, dtype, n_slots, st);
    else dispatch_dtype<kSqOnly, SMX_BF16>(a, dtype, n_slots, st);
  } else {
    if (slots_first) dispatch_dtype<kSqFirst, SMX_F16>(a, dtype, n_slots, st);
    else dispatch_dtype<kSqOnly, SMX_F16>(a, dtype, n_slots, st);
  }
  return check_launch("stats_cast");
}

extern "C" int64_t smx_stats_colsum_workspace_bytes(int64_t cols, int32_t n_slots) {
  if (cols < 1 || n_slots < 1) return -1;
  return round_up(static_cast<int64_t>(n_slots) * cols * 4, 256);
}

extern "C" int smx_stats_colsum(const void *x, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                                float *slots_sq, int32_t n_slots, float *colsum, void *workspace,
                                int64_t workspace_bytes, void *stream) {
  int rc = check_rows("stats_colsum", x, dtype, rows, cols, row_stride, slots_sq, n_slots);
  if (rc) return rc;
  SMX_REQUIRE(slots_sq && colsum && workspace, SMX_EINVAL, "stats_colsum: null slots_sq, colsum or workspace");
  const int64_t need = smx_stats_colsum_workspace_bytes(cols, n_slots);
  SMX_REQUIRE(workspace_bytes >= need, SMX_EWORKSPACE,
              "stats_colsum: workspace of " + std::to_string(workspace_bytes) + " bytes, need " + std::to_string(need));
  SMX_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SMX_EALIGN, "stats_colsum: workspace must be 256-byte aligned");
  float *partial = static_cast<float *>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // rows == 0 still launches: every chunk is empty, its partial zero.
  const StatsArgs a{x, rows, cols, rows ? row_stride : cols, 0, slots_sq, partial, nullptr, 0};
  dispatch_dtype<kSqColsum, 0>(a, dtype, n_slots, st);
  rc = check_launch("stats_colsum");
  if (rc) return rc;
  hipLaunchKernelGGL(colsum_fold_kernel, dim3(static_cast<unsigned>(ceil_div(cols, 64))), dim3(256), 0, st,
                     partial, cols, n_slots, colsum);
  return check_launch("stats_colsum(fold)");
}

extern "C" int smx_stats_fold(float *sum_sq, float *slots_sq, float *sum_first, float *slots_first,
                              int64_t n, int32_t n_slots, void *stream) {
  SMX_REQUIRE(sum_sq && slots_sq, SMX_EINVAL, "stats_fold: null pointer");
  SMX_REQUIRE((sum_first == nullptr) == (slots_first == nullptr), SMX_EINVAL,
              "stats_fold: sum_first and slots_first must both be set or both NULL");
  SMX_REQUIRE(n >= 1 && n_slots >= 1, SMX_ESHAPE, "stats_fold: n >= 1 and n_slots >= 1");
  hipLaunchKernelGGL(stats_fold_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), sum_sq, slots_sq, sum_first, slots_first, n,
                     n_slots);
  return check_launch("stats_fold");
}

extern "C" int smx_stats_finish(const smx_finish_desc *descs, int32_t n_desc, double beta,
                                void *stream) {
  SMX_REQUIRE(n_desc >= 0, SMX_EINVAL, "stats_finish: n_desc < 0");
  SMX_REQUIRE(n_desc == 0 || descs, SMX_EINVAL, "stats_finish: null descriptor table");
  for (int32_t i = 0; i < n_desc; ++i) {
    const smx_finish_desc &d = descs[i];
    SMX_REQUIRE(d.kind >= 0 && d.kind <= 2, SMX_EINVAL, "stats_finish: kind must be 0, 1 or 2");
    SMX_REQUIRE(d.n >= 1 && d.count >= 1 && d.n_slots >= 1, SMX_ESHAPE,
                "stats_finish: need n >= 1, count >= 1, n_slots >= 1");
    SMX_REQUIRE(d.sum_sq && d.slots_sq && d.ema && d.inv, SMX_EINVAL,
                "stats_finish: sum_sq, slots_sq, ema and inv are required");
    if (d.kind == 1)
      SMX_REQUIRE(d.sum_first && d.slots_first && d.mean_ema && d.z && d.kappa, SMX_EINVAL,
                  "stats_finish: rank-one descriptor needs sum_first, slots_first, mean_ema, z, kappa");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int32_t b = 0; b < n_desc; b += kFinishBatch) {
    FinishPack pack{};
    pack.n = std::min<int32_t>(kFinishBatch, n_desc - b);
    int64_t nmax = 1;
    for (int i = 0; i < pack.n; ++i) {
      pack.d[i] = descs[b + i];
      nmax = std::max<int64_t>(nmax, pack.d[i].n);
    }
    hipLaunchKernelGGL(finish_fold_kernel, dim3(static_cast<unsigned>(ceil_div(nmax, 64)), pack.n),
                       dim3(64 * kFoldWaves), 0, st, pack);
    int rc = check_launch("stats_finish(fold)");
    if (rc) return rc;
    hipLaunchKernelGGL(finish_kernel, dim3(pack.n), dim3(kFinishThreads), 0, st, pack, static_cast<float>(beta),
                       static_cast<float>(1.0 - beta));
    rc = check_launch("stats_finish");
    if (rc) return rc;
  }
  return SMX_OK;
}
