// Per-channel statistics for the SandMuon hooks and their step-time finish.
//
//  * stats_accumulate: the hook bodies of sandmuon/optimizer.py:156-168 and
//    :171-177 (sum of x^2, and sum of x for the rank-one A variant), as one
//    HBM pass, for one input or for a batch of queued hook inputs in one
//    launch (one job per input).  An input is cut into row chunks of at
//    least kStatsMinChunkRows rows; each block owns a (job, row chunk,
//    column tile) and adds its FP32 partial into slot row `chunk` of the
//    job, so the result is deterministic, depends on the job alone (not on
//    the other jobs of the launch), and no atomics or tail combine are
//    needed.  The same kernel takes the statistic inside a Linear's input
//    cast (CAST) and bias-gradient column sum (kSqColsum), and the statistic
//    of a GELU's output inside the GELU (XF, kSqDefer*): the A statistic of
//    the Linear the GELU feeds, as per-chunk partials that the Linear's
//    forward adds into its slot rows (stats_add_partials).
//  * stats_fold: sum += sum over slot rows (FP64), slots zeroed.
//  * stats_finish: _finish_a/_finish_b (sandmuon/optimizer.py:182-222) with
//    rank1_inverse_sqrt (:27-35) and diagonal_inverse_sqrt (:19-24).
#include "common.h"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cstring>
#include <type_traits>
#include <vector>

namespace smx {

constexpr int kStatsThreads = 512;
constexpr int kStatsWaves = kStatsThreads / 64;
constexpr int kStatsMaxTW = 256; // widest column tile (channels)

// What a job produces besides sum(x^2) into the slot rows.
enum StatsMode : int {
  kSqOnly = 0,    // B side, diagonal A
  kSqFirst = 1,   // rank-one A: sum(x) into its own slot rows
  kSqColsum = 2,  // sum(x) of this call's rows into per-chunk partials (a bias gradient)
  kSqDefer = 3,       // sum(x^2) into per-chunk partials (plain stores), added to slot rows later
  kSqFirstDefer = 4,  // kSqDefer, and sum(x) into per-chunk partials too
};
constexpr int kStatsModes = 5;

// Elementwise transform of the input before the statistic (XF): none; the
// exact GELU of the input, rounded to the input dtype and stored in
// cast_out (the statistic is that of the stored, rounded values); or a copy
// of the input into cast_out (a relayout: the input is read through an
// InMap, the copy is row-major).
enum StatsXform : int { kXfNone = 0, kXfGelu = 1, kXfCopy = 2 };
constexpr int kStatsXforms = 3;

// Where input element (row, col) of a job lives, relative to J.x:
// (row - row0) * J.row_stride + col(col).  A row-major input has row0 = 0
// and col(c) = c; a relayout input holds its columns as heads of hd
// channels, hs elements apart (col(c) = (c / hd) * hs + c % hd).
struct InMap {
  int64_t row0 = 0, hd = 0, hs = 0;
  __device__ __forceinline__ int64_t col(int64_t c) const { return hd ? (c / hd) * hs + c % hd : c; }
};

// torch's exact GELU in FP32 (x * 0.5 * (1 + erf(x / sqrt(2))), evaluated
// left to right), without contraction.
__device__ __forceinline__ float gelu_erf(float x) {
  const float e = erff(__fmul_rn(x, static_cast<float>(M_SQRT1_2)));
  return __fmul_rn(__fmul_rn(x, 0.5f), __fadd_rn(1.0f, e));
}

// Element access of one lane's VEC consecutive channels: `raw` loads their
// bits (16 bytes for the vector forms, one element otherwise) and `cvt`
// widens them to FP32.  Keeping the raw bits in registers until they are
// consumed lets the next batch of loads be issued first.  The loads are
// non-temporal (the `nt` cache policy): every input byte is read once, and
// a streaming read of HBM runs 13-15% faster with that hint on this part
// (7.0-7.2 against 6.1-6.4 TB/s over 1-4 GiB).
template <int DT, int VEC>
struct Elems {
  using Raw = std::conditional_t<VEC == 1, uint32_t, uint4>;
  static constexpr int kSize = DT == SMX_F32 ? 4 : 2;
  static_assert(VEC == 1 || VEC * kSize == 16, "vector forms load 16 bytes");
  __device__ __forceinline__ static Raw raw(const void *p, int64_t i) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const char *b = static_cast<const char *>(p) + i * kSize;
    if constexpr (VEC > 1) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(b));
      return make_uint4(v.x, v.y, v.z, v.w);
    } else if constexpr (kSize == 4) {
      return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(b));
    } else {
      return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(b));
    }
  }
  __device__ __forceinline__ static float one(uint32_t w) {
    if constexpr (DT == SMX_F32) return __uint_as_float(w);
    else if constexpr (DT == SMX_BF16) return __uint_as_float(w << 16);
    else return f16_bits_to_f32(static_cast<uint16_t>(w));
  }
  __device__ __forceinline__ static void cvt(const Raw &q, float *v) {
    if constexpr (VEC == 1) {
      v[0] = one(q);
    } else {
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (DT == SMX_F32) {
          v[k] = __uint_as_float(w[k]);
        } else if constexpr (DT == SMX_BF16) {
          v[2 * k] = __uint_as_float(w[k] << 16);
          v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        } else {
          typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
          typedef float float2_t __attribute__((ext_vector_type(2)));
          const float2_t f = __builtin_convertvector(__builtin_bit_cast(half2_t, w[k]), float2_t);
          v[2 * k] = f.x;
          v[2 * k + 1] = f.y;
        }
      }
    }
  }
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
  if constexpr (VEC == 8) {
    *reinterpret_cast<uint4 *>(o) = make_uint4(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                               h[2] | (static_cast<uint32_t>(h[3]) << 16),
                                               h[4] | (static_cast<uint32_t>(h[5]) << 16),
                                               h[6] | (static_cast<uint32_t>(h[7]) << 16));
  } else if constexpr (VEC == 4) {
    *reinterpret_cast<uint2 *>(o) = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                               h[2] | (static_cast<uint32_t>(h[3]) << 16));
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = h[k];
  }
}

// One statistics job: a [rows, cols] input split into n_chunks row chunks
// (chunk p adds into slot row p) and column tiles of CT lanes x VEC
// channels; it occupies blocks [block_begin, block_begin + tiles*n_chunks)
// of a launch.
struct StatsJob {
  const void *x;
  float *sq;
  float *first;     // kSqFirst: slot rows of sum(x); kSqColsum, kSqFirstDefer: per-chunk partials, plain stores
  void *cast_out;   // CAST: low-precision copy of x; XF: the transformed x
  int64_t rows, cols, row_stride, out_stride, rows_per_chunk;
  int32_t block_begin, tiles, code, pad_;
};
// Jobs per launch, passed by value: 44 takes a 1 GiB queue of 25 MB hook
// inputs (768-wide bf16, 16384 rows) in one launch.
constexpr int kStatsJobs = 44;
struct StatsPack {
  StatsJob job[kStatsJobs];
  int32_t n;
};
static_assert(sizeof(StatsPack) <= 4000, "StatsPack is passed by value in the kernel arguments");

// The block (tile, chunk) of a job.  A wave covers 64/CT rows per step, the
// block kStatsWaves*64/CT rows.  Each lane sums its rows in order, with
// U loads in flight and the next batch issued before the current one
// is consumed; lanes holding the same channels are then added by xor
// shuffles, the waves in wave order, and the sum is added to the slot row,
// whose old value was loaded at the start of the block (the deferred modes
// store the chunk's sum instead, to be added to the slot row later by one
// FP32 addition, the same one).  CAST (fp32 input only) also writes x
// converted to bf16/f16, as the mixed-precision cast in front of a Linear
// would.  MODE and CAST change nothing in how sum(x^2) is formed, so every
// variant adds the same bits to the slots; with XF the statistic is that of
// the transformed values a later read of the output would load.
template <int DT, int VEC, int CT, int U, int MODE, int CAST, int XF>
__device__ __forceinline__ void stats_tile(const StatsJob &J, int64_t tile, int64_t chunk, float *red,
                                           const InMap &m = InMap{}) {
  using E = Elems<DT, VEC>;
  using Raw = typename E::Raw;
  constexpr bool FIRST = MODE != kSqOnly && MODE != kSqDefer;
  constexpr bool DEFER = MODE == kSqDefer || MODE == kSqFirstDefer;
  static_assert(XF == kXfNone || (CAST == 0 && DT != SMX_F32 && DEFER && VEC == 8),
                "the GELU and copy forms: 16-bit vector input, deferred");
  constexpr int RPW = 64 / CT;
  constexpr int GROUPS = kStatsWaves * RPW;
  constexpr int TW = CT * VEC;
  static_assert(TW <= kStatsMaxTW && TW <= kStatsThreads, "one owner thread per channel");

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int group = wave * RPW + lane / CT;
  const int64_t col0 = (tile * CT + lane % CT) * VEC;
  const int64_t r_begin = chunk * J.rows_per_chunk;
  const int64_t r_end = min(J.rows, r_begin + J.rows_per_chunk);
  const bool empty = r_begin >= r_end;
  // An empty chunk adds nothing; with kSqColsum it still writes its zero
  // partial.  Uniform per block.
  if (MODE != kSqColsum && empty) return;
  const int64_t tile_col0 = tile * TW;
  const int64_t row_off = chunk * J.cols + tile_col0;
  const int c = threadIdx.x;
  const bool own = c < TW && tile_col0 + c < J.cols;
  float old_sq = 0.f, old_first = 0.f;
  if (!DEFER && own && !empty) old_sq = J.sq[row_off + c];
  if constexpr (MODE == kSqFirst)
    if (own) old_first = J.first[row_off + c];

  float acc_sq[VEC], acc_first[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) { acc_sq[k] = 0.f; acc_first[k] = 0.f; }

  if (!empty && col0 < J.cols) {
    int64_t r = r_begin + group;
    const int64_t colx = m.col(col0);  // the input offset of the lane's channels
    auto issue = [&](Raw (&q)[U], int64_t &rq) {
      rq = r;
#pragma unroll
      for (int u = 0; u < U; ++u) q[u] = E::raw(J.x, (r + u * GROUPS - m.row0) * J.row_stride + colx);
      r += U * GROUPS;
    };
    auto eat1 = [&](const Raw &q, int64_t row) {
      if constexpr (XF == kXfCopy) {
        uint16_t *o = static_cast<uint16_t *>(J.cast_out) + row * J.out_stride + col0;
        *reinterpret_cast<uint4 *>(o) = q;
      }
      float v[VEC];
      E::cvt(q, v);
      if constexpr (XF == kXfGelu) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          float g = gelu_erf(v[k]);
          // The FP32 result is rounded to the 16-bit type as a separate step
          // (torch rounds its FP32 result): the compiler would otherwise fold
          // the last multiply into a mixed FMA that rounds to f16 once.
          asm volatile("" : "+v"(g));
          if constexpr (DT == SMX_BF16) v[k] = bf16_bits_to_f32(f32_to_bf16_bits(g));
          else v[k] = f16_bits_to_f32(__builtin_bit_cast(uint16_t, static_cast<_Float16>(g)));
        }
        store_cast<DT, VEC>(J.cast_out, row * J.out_stride + col0, v);
      }
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        acc_sq[k] = fmaf(v[k], v[k], acc_sq[k]);
        if constexpr (FIRST) acc_first[k] += v[k];
      }
      if constexpr (CAST != 0) store_cast<CAST, VEC>(J.cast_out, row * J.out_stride + col0, v);
    };
    // The scheduling barriers keep the batches in issue order: without them
    // the compiler starts consuming the newest batch before issuing the
    // next one, so each iteration waits for every load (vmcnt(0)) and a
    // wave's loads run dry.
    auto eat = [&](const Raw (&q)[U], int64_t rq) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) eat1(q[u], rq + u * GROUPS);
      __builtin_amdgcn_sched_barrier(0);
    };
    const int64_t n_rows = r < r_end ? (r_end - r + GROUPS - 1) / GROUPS : 0;
    const int64_t nb = n_rows / U;
    Raw A[U], B[U];
    int64_t ra = 0, rb = 0;
    if (nb > 0) {
      issue(A, ra);
      int64_t k = 1;
      for (; k + 1 < nb; k += 2) {
        issue(B, rb);
        eat(A, ra);
        issue(A, ra);
        eat(B, rb);
      }
      if (k < nb) {
        issue(B, rb);
        eat(A, ra);
        eat(B, rb);
      } else {
        eat(A, ra);
      }
    }
    for (; r < r_end; r += GROUPS) eat1(E::raw(J.x, (r - m.row0) * J.row_stride + colx), r);
  }
  // Lanes l, l + CT, ... of a wave hold the same channels.
#pragma unroll
  for (int off = CT; off < 64; off <<= 1)
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      acc_sq[k] += __shfl_xor(acc_sq[k], off);
      if constexpr (FIRST) acc_first[k] += __shfl_xor(acc_first[k], off);
    }
  float *red_sq = red, *red_first = red + kStatsWaves * kStatsMaxTW;
  if (lane < CT) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      red_sq[wave * TW + lane * VEC + k] = acc_sq[k];
      if constexpr (FIRST) red_first[wave * TW + lane * VEC + k] = acc_first[k];
    }
  }
  __syncthreads();
  if (own) {
    float s = 0.f, f = 0.f;
#pragma unroll
    for (int w = 0; w < kStatsWaves; ++w) {
      s += red_sq[w * TW + c];
      if constexpr (FIRST) f += red_first[w * TW + c];
    }
    if (!empty) J.sq[row_off + c] = DEFER ? s : old_sq + s;
    if constexpr (MODE == kSqFirst) J.first[row_off + c] = old_first + f;
    if constexpr (MODE == kSqColsum || MODE == kSqFirstDefer) J.first[row_off + c] = f;
  }
}

// Element forms of a job: the vector forms load 16 bytes per lane, the
// scalar forms one element (64-lane tiles) for inputs whose width, row
// stride or address is not 16-byte aligned.
enum StatsForm : int { kF32V4 = 0, kBf16V8, kF16V8, kF32V1, kBf16V1, kF16V1, kNumForms };
__host__ __device__ constexpr int stats_code(int form, int mode, int cast, int xf = kXfNone) {
  return ((form * kStatsModes + mode) * 3 + cast) * kStatsXforms + xf;
}

// CT: lanes across a column tile (32 for the vector forms: 128 f32 or 256
// 16-bit channels; 16 lanes measured 2% slower on the cfg4 hook inputs).
// U: loads per lane per register batch
// (the f16 form widens its batch early, so it keeps two loads per batch to
// stay within the register budget the other forms set).
template <int FORM>
struct FormTraits;
template <> struct FormTraits<kF32V4> { static constexpr int DT = SMX_F32, VEC = 4, CT = 32, U = 4; };
template <> struct FormTraits<kBf16V8> { static constexpr int DT = SMX_BF16, VEC = 8, CT = 32, U = 4; };
template <> struct FormTraits<kF16V8> { static constexpr int DT = SMX_F16, VEC = 8, CT = 32, U = 2; };
template <> struct FormTraits<kF32V1> { static constexpr int DT = SMX_F32, VEC = 1, CT = 64, U = 4; };
template <> struct FormTraits<kBf16V1> { static constexpr int DT = SMX_BF16, VEC = 1, CT = 64, U = 4; };
template <> struct FormTraits<kF16V1> { static constexpr int DT = SMX_F16, VEC = 1, CT = 64, U = 4; };

template <int FORM>
constexpr int64_t tile_channels() { return FormTraits<FORM>::VEC * FormTraits<FORM>::CT; }
constexpr int64_t kTileChannels[kNumForms] = {tile_channels<kF32V4>(),  tile_channels<kBf16V8>(),
                                              tile_channels<kF16V8>(),  tile_channels<kF32V1>(),
                                              tile_channels<kBf16V1>(), tile_channels<kF16V1>()};

// Row chunks hold at least this many rows (fewer slot rows are then used):
// a block then streams 256 KB, so its start and its reduction weigh less
// (measured against 128 and 256 rows on the cfg4 hook inputs).  The chunking depends on the job alone, so a job adds the same
// bits whether it is launched alone or with others.
constexpr int64_t kStatsMinChunkRows = 512;

// The GELU form keeps two loads per batch: its erf evaluations need the
// registers (it has a kernel of its own, so the hook kernel keeps its
// register budget).
template <int FORM, int MODE, int CAST, int XF>
__device__ __forceinline__ void run_tile(const StatsJob &J, int64_t tile, int64_t chunk, float *red,
                                         const InMap &m = InMap{}) {
  using F = FormTraits<FORM>;
  stats_tile<F::DT, F::VEC, F::CT, XF == kXfGelu ? 2 : F::U, MODE, CAST, XF>(J, tile, chunk, red, m);
}

// The job of block b of a launch: block_begin grows with the job index, so
// the index is the count of later jobs that begin at or before the block
// (unrolled, so the scalar loads of every begin are issued together).
__device__ __forceinline__ int stats_job_of(const StatsPack &pack, int b) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < kStatsJobs; ++i) j += (i < pack.n && b >= pack.job[i].block_begin) ? 1 : 0;
  return j;
}

// grid.x = sum over the jobs of tiles * n_chunks; block = kStatsThreads.
// Four waves per SIMD (two blocks per CU): on the cfg4 hook inputs 0.3-0.7%
// faster than six (three blocks per CU) with the same code and bits; three
// waves per SIMD (one block) was 8% slower.
__global__ void __launch_bounds__(kStatsThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) stats_accumulate_kernel(StatsPack pack) {
  __shared__ float red[2 * kStatsWaves * kStatsMaxTW];
  const int b = static_cast<int>(blockIdx.x);
  // A copy of the block's job (scalar registers): a reference into the pack
  // makes the compiler copy the whole pack to scratch memory.
  const StatsJob J = pack.job[stats_job_of(pack, b)];
  const int64_t local = b - J.block_begin;
  const int64_t tile = local % J.tiles, chunk = local / J.tiles;
#define SMX_STATS_CASE(FORM, MODE, CAST) \
  case stats_code(FORM, MODE, CAST): run_tile<FORM, MODE, CAST, kXfNone>(J, tile, chunk, red); break;

#define SMX_STATS_MODES(FORM)          \
  SMX_STATS_CASE(FORM, kSqOnly, 0)     \
  SMX_STATS_CASE(FORM, kSqFirst, 0)    \
  SMX_STATS_CASE(FORM, kSqColsum, 0)
#define SMX_STATS_CASTS(FORM)                 \
  SMX_STATS_CASE(FORM, kSqOnly, SMX_BF16)     \
  SMX_STATS_CASE(FORM, kSqFirst, SMX_BF16)    \
  SMX_STATS_CASE(FORM, kSqOnly, SMX_F16)      \
  SMX_STATS_CASE(FORM, kSqFirst, SMX_F16)
  switch (J.code) {
    SMX_STATS_MODES(kF32V4)
    SMX_STATS_MODES(kBf16V8)
    SMX_STATS_MODES(kF16V8)
    SMX_STATS_MODES(kF32V1)
    SMX_STATS_MODES(kBf16V1)
    SMX_STATS_MODES(kF16V1)
    SMX_STATS_CASTS(kF32V4)
    SMX_STATS_CASTS(kF32V1)
    default: break;
  }
#undef SMX_STATS_CASTS
#undef SMX_STATS_MODES
#undef SMX_STATS_CASE
}

// The GELU jobs (smx_stats_gelu), in a kernel of their own.
__global__ void __launch_bounds__(kStatsThreads) stats_gelu_kernel(StatsPack pack) {
  __shared__ float red[2 * kStatsWaves * kStatsMaxTW];
  const int b = static_cast<int>(blockIdx.x);
  // A copy of the block's job (scalar registers): a reference into the pack
  // makes the compiler copy the whole pack to scratch memory.
  const StatsJob J = pack.job[stats_job_of(pack, b)];
  const int64_t local = b - J.block_begin;
  const int64_t tile = local % J.tiles, chunk = local / J.tiles;
#define SMX_STATS_GELU(FORM)                                                                   \
  case stats_code(FORM, kSqDefer, 0, kXfGelu):                                                 \
    run_tile<FORM, kSqDefer, 0, kXfGelu>(J, tile, chunk, red);                                 \
    break;                                                                                     \
  case stats_code(FORM, kSqFirstDefer, 0, kXfGelu):                                            \
    run_tile<FORM, kSqFirstDefer, 0, kXfGelu>(J, tile, chunk, red);                            \
    break;
  switch (J.code) {
    SMX_STATS_GELU(kBf16V8)
    SMX_STATS_GELU(kF16V8)
    default: break;
  }
#undef SMX_STATS_GELU
}

// A relayout job (smx_stats_relayout): a [batch, seq, heads, head_dim]
// view with strides (sb, job.row_stride, hs, 1) copied row-major into
// job.cast_out as [batch * seq, heads * head_dim], with the statistic of
// the copy.  A row chunk lies inside one sequence (seq is a multiple of
// job.rows_per_chunk), where consecutive rows are job.row_stride apart.
struct RelayoutArgs {
  StatsJob job;
  int64_t seq, sb, hd, hs;
};

__global__ void __launch_bounds__(kStatsThreads) stats_relayout_kernel(RelayoutArgs a) {
  __shared__ float red[2 * kStatsWaves * kStatsMaxTW];
  StatsJob J = a.job;
  const int64_t local = blockIdx.x;
  const int64_t tile = local % J.tiles, chunk = local / J.tiles;
  const int64_t r0 = chunk * J.rows_per_chunk;  // the chunk's first row: sequence b, position t0
  const int64_t b = r0 / a.seq, t0 = r0 % a.seq;
  J.x = static_cast<const char *>(J.x) + (b * a.sb + t0 * J.row_stride) * 2;  // 16-bit elements
  const InMap m{r0, a.hd, a.hs};
#define SMX_STATS_COPY(FORM)                                                                   \
  case stats_code(FORM, kSqDefer, 0, kXfCopy):                                                 \
    run_tile<FORM, kSqDefer, 0, kXfCopy>(J, tile, chunk, red, m);                              \
    break;                                                                                     \
  case stats_code(FORM, kSqFirstDefer, 0, kXfCopy):                                            \
    run_tile<FORM, kSqFirstDefer, 0, kXfCopy>(J, tile, chunk, red, m);                         \
    break;
  switch (J.code) {
    SMX_STATS_COPY(kBf16V8)
    SMX_STATS_COPY(kF16V8)
    default: break;
  }
#undef SMX_STATS_COPY
}

// Host side: one job per input, launched in packs of kStatsJobs.
struct StatsInput {
  const void *x;
  int dtype;
  int64_t rows, cols, row_stride;
  float *sq, *first;
  int32_t n_slots;
  int mode, cast;
  void *cast_out;
  int64_t out_stride;
  int xf = kXfNone;
};

static int stats_form(const StatsInput &in) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(in.x);
  if (in.dtype == SMX_F32) {
    bool v4 = in.cols % 4 == 0 && in.row_stride % 4 == 0 && addr % 16 == 0;
    if (in.cast) v4 = v4 && in.out_stride % 4 == 0 && reinterpret_cast<uintptr_t>(in.cast_out) % 8 == 0;
    return v4 ? kF32V4 : kF32V1;
  }
  const bool v8 = in.cols % 8 == 0 && in.row_stride % 8 == 0 && addr % 16 == 0;
  if (in.dtype == SMX_BF16) return v8 ? kBf16V8 : kBf16V1;
  return v8 ? kF16V8 : kF16V1;
}

static int stats_launch(const StatsInput *in, int n, hipStream_t st, const char *who) {
  StatsPack pack{};
  int64_t blocks = 0;
  auto flush = [&]() -> int {
    if (pack.n == 0) return SMX_OK;
    if (pack.job[0].code % kStatsXforms == kXfGelu)
      hipLaunchKernelGGL(stats_gelu_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kStatsThreads), 0, st, pack);
    else
      hipLaunchKernelGGL(stats_accumulate_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kStatsThreads), 0, st,
                         pack);
    pack.n = 0;
    blocks = 0;
    return check_launch(who);
  };
  for (int i = 0; i < n; ++i) {
    const StatsInput &s = in[i];
    const int form = stats_form(s);
    const int64_t tiles = ceil_div(s.cols, kTileChannels[form]);
    const int64_t rows_per_chunk = std::max<int64_t>(ceil_div(s.rows, s.n_slots), kStatsMinChunkRows);
    // Chunks that hold rows; colsum writes a zero partial into every slot
    // row, so it keeps one block per slot row.
    const int64_t chunks = s.mode == kSqColsum ? s.n_slots : std::max<int64_t>(ceil_div(s.rows, rows_per_chunk), 1);
    const int64_t nb = tiles * chunks;
    if (pack.n == kStatsJobs || blocks + nb > INT32_MAX || (pack.n > 0 && pack.job[0].code % kStatsXforms != s.xf)) {
      int rc = flush();
      if (rc) return rc;
    }
    StatsJob &J = pack.job[pack.n++];
    J.x = s.x;
    J.sq = s.sq;
    J.first = s.first;
    J.cast_out = s.cast_out;
    J.rows = s.rows;
    J.cols = s.cols;
    J.row_stride = s.row_stride;
    J.out_stride = s.out_stride;
    J.rows_per_chunk = rows_per_chunk;
    J.block_begin = static_cast<int32_t>(blocks);
    J.tiles = static_cast<int32_t>(tiles);
    J.code = stats_code(form, s.mode, s.cast, s.xf);
    blocks += nb;
  }
  return flush();
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

__device__ __forceinline__ void finish_fold(const smx_finish_desc &d) {
  __shared__ double part[2][kFoldWaves][64];
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

__global__ void __launch_bounds__(64 * kFoldWaves) finish_fold_kernel(FinishPack pack) {
  finish_fold(pack.d[blockIdx.y]);
}

// The same over a descriptor table in device memory (any number of
// descriptors in one launch), the block's descriptor copied to registers.
__global__ void __launch_bounds__(64 * kFoldWaves) finish_fold_table_kernel(const smx_finish_desc *table) {
  const smx_finish_desc d = table[blockIdx.y];
  finish_fold(d);
}

__device__ __forceinline__ float ema_update(float e, float x, float beta, float omb) {
  // e.mul_(beta).add_(x, alpha=1-beta), both coefficients rounded from double
  return e * beta + x * omb;
}

// One block of kFinishThreads per descriptor.
constexpr int kFinishThreads = 1024;

__device__ __forceinline__ void finish_one(const smx_finish_desc &d, float beta, float omb) {
  __shared__ double scratch[16];
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

__global__ void __launch_bounds__(kFinishThreads) finish_kernel(FinishPack pack, float beta, float omb) {
  finish_one(pack.d[blockIdx.x], beta, omb);
}

__global__ void __launch_bounds__(kFinishThreads) finish_table_kernel(const smx_finish_desc *table, float beta,
                                                                      float omb) {
  const smx_finish_desc d = table[blockIdx.x];
  finish_one(d, beta, omb);
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
  const StatsInput in{x, dtype, rows, cols, row_stride, slots_sq, slots_first, n_slots,
                      slots_first ? kSqFirst : kSqOnly, 0, nullptr, 0};
  return stats_launch(&in, 1, static_cast<hipStream_t>(stream), "stats_accumulate");
}

extern "C" int32_t smx_stats_slot_rows(int64_t rows, int32_t n_slots) {
  if (rows < 0 || n_slots < 1) return -1;
  if (rows == 0) return 0;
  const int64_t rows_per_chunk = std::max<int64_t>(ceil_div(rows, n_slots), kStatsMinChunkRows);
  return static_cast<int32_t>(ceil_div(rows, rows_per_chunk));
}

extern "C" int smx_stats_accumulate_batch(const smx_stats_desc *descs, int32_t n_desc, void *stream) {
  SMX_REQUIRE(n_desc >= 0 && (n_desc == 0 || descs), SMX_EINVAL, "stats_accumulate_batch: bad descriptor table");
  std::vector<StatsInput> in;
  in.reserve(n_desc);
  for (int32_t i = 0; i < n_desc; ++i) {
    const smx_stats_desc &d = descs[i];
    const std::string who = "stats_accumulate_batch[" + std::to_string(i) + "]";
    int rc = check_rows(who.c_str(), d.x, d.dtype, d.rows, d.cols, d.row_stride, d.slots_sq, d.n_slots);
    if (rc) return rc;
    // Jobs of one launch run concurrently: no two may add into the same
    // slot rows.
    const uintptr_t lo = reinterpret_cast<uintptr_t>(d.slots_sq);
    const uintptr_t hi = lo + static_cast<uintptr_t>(d.n_slots) * d.cols * 4;
    for (int32_t k = 0; k < i; ++k) {
      const smx_stats_desc &e = descs[k];
      for (const float *p : {e.slots_sq, e.slots_first}) {
        if (!p) continue;
        const uintptr_t elo = reinterpret_cast<uintptr_t>(p);
        const uintptr_t ehi = elo + static_cast<uintptr_t>(e.n_slots) * e.cols * 4;
        for (const float *q : {d.slots_sq, d.slots_first}) {
          if (!q) continue;
          const uintptr_t qlo = reinterpret_cast<uintptr_t>(q);
          const uintptr_t qhi = qlo + (hi - lo);
          SMX_REQUIRE(qhi <= elo || ehi <= qlo, SMX_EINVAL,
                      who + ": slot rows overlap those of descriptor " + std::to_string(k));
        }
      }
    }
    if (d.rows == 0) continue;  // empty microbatch: nothing to add
    in.push_back(StatsInput{d.x, d.dtype, d.rows, d.cols, d.row_stride, d.slots_sq, d.slots_first, d.n_slots,
                            d.slots_first ? kSqFirst : kSqOnly, 0, nullptr, 0});
  }
  return stats_launch(in.data(), static_cast<int>(in.size()), static_cast<hipStream_t>(stream),
                      "stats_accumulate_batch");
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
  const StatsInput in{x, dtype, rows, cols, row_stride, slots_sq, slots_first, n_slots,
                      slots_first ? kSqFirst : kSqOnly, out_dtype, out, out_stride};
  return stats_launch(&in, 1, static_cast<hipStream_t>(stream), "stats_cast");
}

extern "C" int smx_stats_gelu(const void *x, int dtype, int64_t rows, int64_t cols, int64_t row_stride, void *out,
                              int64_t out_stride, float *part_sq, float *part_first, int32_t n_slots, void *stream) {
  int rc = check_rows("stats_gelu", x, dtype, rows, cols, row_stride, part_sq, n_slots);
  if (rc) return rc;
  SMX_REQUIRE(dtype == SMX_BF16 || dtype == SMX_F16, SMX_EDTYPE, "stats_gelu: the input must be bf16 or f16");
  SMX_REQUIRE(rows == 0 || out, SMX_EINVAL, "stats_gelu: null output");
  SMX_REQUIRE(out_stride >= cols || rows <= 1, SMX_ESHAPE, "stats_gelu: out_stride must be >= cols");
  SMX_REQUIRE(cols % 8 == 0 && row_stride % 8 == 0 && out_stride % 8 == 0 &&
                  reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
              SMX_EALIGN, "stats_gelu: cols and row strides must be multiples of 8 elements, x and out 16-byte aligned");
  if (rows == 0) return SMX_OK;
  StatsInput in{x, dtype, rows, cols, row_stride, part_sq, part_first, n_slots,
                part_first ? kSqFirstDefer : kSqDefer, 0, out, out_stride};
  in.xf = kXfGelu;
  return stats_launch(&in, 1, static_cast<hipStream_t>(stream), "stats_gelu");
}

extern "C" int smx_stats_relayout(const void *x, int dtype, int64_t batch, int64_t seq, int64_t heads,
                                  int64_t head_dim, int64_t batch_stride, int64_t seq_stride, int64_t head_stride,
                                  void *out, float *part_sq, float *part_first, int32_t n_slots, void *stream) {
  SMX_REQUIRE(dtype == SMX_BF16 || dtype == SMX_F16, SMX_EDTYPE, "stats_relayout: the input must be bf16 or f16");
  SMX_REQUIRE(batch >= 1 && seq >= 1 && heads >= 1 && head_dim >= 1, SMX_ESHAPE,
              "stats_relayout: batch, seq, heads and head_dim must be >= 1");
  SMX_REQUIRE(x && out && part_sq, SMX_EINVAL, "stats_relayout: null input, output or partials");
  SMX_REQUIRE(n_slots >= 1 && n_slots <= 65535, SMX_EINVAL, "stats_relayout: n_slots in [1, 65535]");
  SMX_REQUIRE(head_dim % 8 == 0 && batch_stride % 8 == 0 && seq_stride % 8 == 0 && head_stride % 8 == 0 &&
                  reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
              SMX_EALIGN,
              "stats_relayout: head_dim and the strides must be multiples of 8 elements, x and out 16-byte aligned");
  const int64_t rows = batch * seq, cols = heads * head_dim;
  const int64_t rows_per_chunk = std::max<int64_t>(ceil_div(rows, n_slots), kStatsMinChunkRows);
  SMX_REQUIRE(seq % rows_per_chunk == 0, SMX_ESHAPE,
              "stats_relayout: seq must be a multiple of the row chunk (" + std::to_string(rows_per_chunk) + " rows)");
  const int form = dtype == SMX_BF16 ? kBf16V8 : kF16V8;
  RelayoutArgs a{};
  StatsJob &J = a.job;
  J.x = x;
  J.sq = part_sq;
  J.first = part_first;
  J.cast_out = out;
  J.rows = rows;
  J.cols = cols;
  J.row_stride = seq_stride;
  J.out_stride = cols;
  J.rows_per_chunk = rows_per_chunk;
  J.block_begin = 0;
  J.tiles = static_cast<int32_t>(ceil_div(cols, kTileChannels[form]));
  J.code = stats_code(form, part_first ? kSqFirstDefer : kSqDefer, 0, kXfCopy);
  a.seq = seq;
  a.sb = batch_stride;
  a.hd = head_dim;
  a.hs = head_stride;
  const int64_t blocks = static_cast<int64_t>(J.tiles) * (rows / rows_per_chunk);
  SMX_REQUIRE(blocks < INT32_MAX, SMX_ESHAPE, "stats_relayout: too many blocks for one launch");
  hipLaunchKernelGGL(stats_relayout_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kStatsThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("stats_relayout");
}

// slots[i] += part[i] over n elements (the FP32 addition a statistics call
// makes into its slot rows), for sq and, when given, first.
__global__ void __launch_bounds__(256) stats_add_partials_kernel(float *slots_sq, const float *part_sq, float *slots_first,
                                                                 const float *part_first, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  slots_sq[i] = slots_sq[i] + part_sq[i];
  if (slots_first) slots_first[i] = slots_first[i] + part_first[i];
}

extern "C" int smx_stats_add_partials(float *slots_sq, const float *part_sq, float *slots_first, const float *part_first,
                                      int64_t cols, int32_t n_rows, void *stream) {
  SMX_REQUIRE(cols >= 1 && n_rows >= 0, SMX_ESHAPE, "stats_add_partials: need cols >= 1 and n_rows >= 0");
  SMX_REQUIRE(n_rows == 0 || (slots_sq && part_sq), SMX_EINVAL, "stats_add_partials: null slots_sq or part_sq");
  SMX_REQUIRE((slots_first == nullptr) == (part_first == nullptr), SMX_EINVAL,
              "stats_add_partials: slots_first and part_first must both be set or both NULL");
  const int64_t n = cols * n_rows;
  if (n == 0) return SMX_OK;
  hipLaunchKernelGGL(stats_add_partials_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), slots_sq, part_sq, slots_first, part_first, n);
  return check_launch("stats_add_partials");
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
  const StatsInput in{x, dtype, rows, cols, rows ? row_stride : cols, slots_sq, partial, n_slots,
                      kSqColsum, 0, nullptr, 0};
  rc = stats_launch(&in, 1, st, "stats_colsum");
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

static int check_finish_descs(const smx_finish_desc *descs, int32_t n_desc) {
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
  return SMX_OK;
}

extern "C" int smx_stats_finish(const smx_finish_desc *descs, int32_t n_desc, double beta,
                                void *stream) {
  if (const int rc = check_finish_descs(descs, n_desc)) return rc;
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

extern "C" size_t smx_stats_finish_table_bytes(int32_t n_desc) {
  return n_desc > 0 ? static_cast<size_t>(n_desc) * sizeof(smx_finish_desc) : 0;
}

extern "C" int smx_stats_finish_staged(const smx_finish_desc *descs, int32_t n_desc, double beta, void *dev_table,
                                       size_t table_bytes, void *stream) {
  if (const int rc = check_finish_descs(descs, n_desc)) return rc;
  if (n_desc == 0) return SMX_OK;
  SMX_REQUIRE(n_desc <= 65535, SMX_EINVAL, "stats_finish_staged: at most 65535 descriptors");
  const size_t need = smx_stats_finish_table_bytes(n_desc);
  SMX_REQUIRE(dev_table && table_bytes >= need, SMX_EWORKSPACE,
              "stats_finish_staged: dev_table needs smx_stats_finish_table_bytes(n_desc) bytes");
  int64_t nmax = 1;
  for (int32_t i = 0; i < n_desc; ++i) nmax = std::max<int64_t>(nmax, descs[i].n);
  SMX_REQUIRE(ceil_div(nmax, 64) <= INT32_MAX, SMX_ESHAPE, "stats_finish_staged: vector too long");
  hipStream_t st = static_cast<hipStream_t>(stream);
  static_assert(sizeof(smx_finish_desc) % 4 == 0, "the table is uploaded as 32-bit words");
  if (const int rc = upload_table(dev_table, descs, need, st)) return rc;
  const auto *table = static_cast<const smx_finish_desc *>(dev_table);
  hipLaunchKernelGGL(finish_fold_table_kernel, dim3(static_cast<unsigned>(ceil_div(nmax, 64)), n_desc),
                     dim3(64 * kFoldWaves), 0, st, table);
  int rc = check_launch("stats_finish_staged(fold)");
  if (rc) return rc;
  hipLaunchKernelGGL(finish_table_kernel, dim3(n_desc), dim3(kFinishThreads), 0, st, table, static_cast<float>(beta),
                     static_cast<float>(1.0 - beta));
  return check_launch("stats_finish_staged");
}
