// S8 polar map on gfx950 MFMA: sandmuon/optimizer.py:69-93 with the
// constants of sandmuon/coefficients.py:3-11.
//
// Per matrix (oriented r <= c, unnormalised whitened input V in x0/xt0 and
// its squared Frobenius norm as partials in `fro`) and stage k = 1..5:
//   GRAM    G  = X X^T                 (stage 1: times 1/||V||^2)
//   SQUARE  stage 1: G2 = G G  -> p buffer, plus Schatten-8 partials
//           stage k: P  = a I + b G + c (G G)            -> p buffer
//   APPLY   stage 1: X' = P1 V / (||V|| s),  P1 = a I + b G/s^2 + c G2/s^4
//                    formed in the A-operand loader; s = 1.35 ||G2||_F^(1/4)
//           stage k: X' = P X
// Every product is C = A B^T with A, B row-major and K contiguous: the
// Gram uses X twice, the square uses the symmetric G twice, the apply uses
// P and X^T.  The apply epilogue therefore writes the new iterate in both
// layouts (X and X^T).  Gram and square only compute upper-triangle tiles
// and store each off-diagonal tile twice (tile and mirror).
//
// Arithmetic modes:
//   SMX_S8_FP32       v_mfma_f32_32x32x2_f32, FP32 operands in LDS.
//   SMX_S8_COMP_BF16  each FP32 operand is split into BF16 hi + lo when it
//                     is staged to LDS; acc += hi*lo + lo*hi + hi*hi with
//                     v_mfma_f32_32x32x16_bf16 (the compensated product of
//                     reproduction/odl/ops/bf16_compensated_mm_fast.py:
//                     60-66, applied in all five stages with FP32 storage
//                     of every intermediate).
//
// Block: 256x256 output tile, 4 waves (2 x 2, one per SIMD), each wave
// 128x128 (4 x 4 MFMA 32x32 tiles, 256 accumulators).  Operands stream into a 4-stage LDS ring (K = 16 per
// stage, 32 KB) with direct-to-LDS 16-byte loads issued three stages ahead.
// In compensated mode every operand is stored by its producer as BF16
// hi/lo planes (put_operand), so the inner loop is LDS reads + MFMAs; only
// the stage-1 polynomial operand is formed and split in registers.
#include "s8.h"

#include <algorithm>
#include <cmath>
#include <vector>

namespace smx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;     // 4 waves, one per SIMD
constexpr int kWaves = kThreads / 64;
constexpr int kSubM = 4, kSubN = 4; // 32x32 MFMA tiles per wave (128 x 128)
constexpr int kBK = 16;            // K per pipeline stage
constexpr int kF32Tile = 16384;    // 256 x 16 FP32 operand tile
constexpr int kB16Tile = 8192;     // 256 x 16 BF16 plane tile
constexpr int kStages = 4;         // LDS ring depth (3 stages in flight)
constexpr int kPolyStages = 3;     // ring depth when A is formed from (G, G2)
constexpr int kStageBytes = 2 * kF32Tile;          // A + B (FP32, or 4 BF16 planes)
constexpr int kPolyStageBytes = 3 * kF32Tile;      // G + G2 + B
constexpr int kRingBytes = kStages * kStageBytes > kPolyStages * kPolyStageBytes ? kStages * kStageBytes
                                                                                 : kPolyStages * kPolyStageBytes;

enum Phase { kGram = 0, kSquare = 1, kApply = 2 };

struct StageArgs {
  S8Layout L;
  int32_t seg_off[kMaxClasses + 1];  // block offsets (multiples of 8)
  int32_t seg_cls[kMaxClasses];
  int32_t n_seg;
  int32_t stage;  // 1..5
  float a, b, c;
};

struct PolyArgs {
  float a, b, c;     // stage-1 coefficients
  float is2, is4;    // 1/s^2, 1/s^4
  int64_t r;         // logical rows (identity only on real rows)
  int64_t row0;      // first global row of the A tile
};

// A K-contiguous GEMM operand: FP32 rows of `ld` elements, or BF16 hi/lo
// planes (lo at hi + plane elements).
struct Opnd {
  const void *p;
  int64_t ld;
  int64_t plane;
};

// ------------------------------------------------------- LDS layouts ---
// FP32 tile [256][16]: four 16-byte chunks per row, logical chunk kc at
// slot kc ^ swz4(r).  BF16 plane tile [256][16]: two chunks per row, slot
// c ^ swz2(r).  Both make the fragment reads (8 or 16 consecutive rows, one
// chunk) conflict-free for 32- and 64-bank LDS.
__device__ __forceinline__ int swz4(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }
__device__ __forceinline__ int swz2(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }
__device__ __forceinline__ int f32_off(int r, int kc) { return (r * 4 + (kc ^ swz4(r))) << 4; }
__device__ __forceinline__ int b16_off(int r, int c) { return (r * 2 + (c ^ swz2(r))) << 4; }

// One 16-byte direct-to-LDS load per lane: lane l writes LDS[m0 + 16 l].
// Issued from asm so the compiler does not treat later LDS reads as
// aliasing the in-flight load (it would wait for every outstanding load);
// the ring's waits are explicit (wait_vm).  M0 is an input operand.
__device__ __forceinline__ void dma16(const void *src, char *lds_wave_base) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_wave_base));
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

// This wave's share of an FP32 tile (rows row0.., K k0..k0+15): LDS chunk
// p = (wave*N+i)*64 + lane is stored slot p&3 of row p>>2.
__device__ __forceinline__ void dma_f32(const float *__restrict__ M, int64_t ld, int64_t row0, int64_t k0,
                                        char *tile) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int N = 16 / kWaves;  // 1 KB loads per wave
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int p = (wave * N + i) * 64 + lane;
    const int row = p >> 2;
    const int kc = (p & 3) ^ swz4(row);
    dma16(M + (row0 + row) * ld + k0 + kc * 4, tile + (wave * N + i) * 1024);
  }
}

// This wave's share of a BF16 plane tile: LDS chunk p = (wave*N+i)*64 +
// lane is stored slot p&1 of row p>>1.
__device__ __forceinline__ void dma_b16(const uint16_t *__restrict__ M, int64_t ld, int64_t row0, int64_t k0,
                                        char *tile) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int N = 8 / kWaves;  // 1 KB loads per wave
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int p = (wave * N + i) * 64 + lane;
    const int row = p >> 1;
    const int c = (p & 1) ^ swz2(row);
    dma16(M + (row0 + row) * ld + k0 + c * 8, tile + (wave * N + i) * 1024);
  }
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if constexpr (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if constexpr (N == 24) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else if constexpr (N == 36) asm volatile("s_waitcnt vmcnt(36)" ::: "memory");
  else static_assert(N == 0, "unsupported vmcnt");
}

__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// The 8 consecutive K values (k = 8h .. 8h+7 of the stage) of row r.
__device__ __forceinline__ void read8(const char *tile, int r, int h, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(tile + f32_off(r, 2 * h));
  const f32x4 b = *reinterpret_cast<const f32x4 *>(tile + f32_off(r, 2 * h + 1));
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ bf16x8 read_b16(const char *tile, int r, int h) {
  return *reinterpret_cast<const bf16x8 *>(tile + b16_off(r, h));
}

__device__ __forceinline__ void split8(const float (&v)[8], bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = static_cast<__bf16>(v[e]);
    hi[e] = h;
    lo[e] = static_cast<__bf16>(v[e] - static_cast<float>(h));
  }
}

// ----------------------------------------------------------- compute ---
// Register fragments of one 16-deep K stage for this wave's 128 x 128
// sub-tile: BF16 hi/lo pairs (compensated mode) or FP32 (FP32 mode).  The
// A fragments of row block i are dead once row i's MFMAs are issued and are
// reloaded in place with the next stage; the B fragments, used by every
// row, are double-buffered.
template <int MODE>
struct AFrag;
template <>
struct AFrag<SMX_S8_COMP_BF16> {
  bf16x8 h, l;
};
template <>
struct AFrag<SMX_S8_FP32> {
  float v[8];
};
template <int MODE>
struct BFrags;
template <>
struct BFrags<SMX_S8_COMP_BF16> {
  bf16x8 h[kSubN], l[kSubN];
};
template <>
struct BFrags<SMX_S8_FP32> {
  float v[kSubN][8];
};

// LDS -> registers, A row block i of one stage.
//  COMP, plain: BF16 hi/lo planes.
//  POLY       : A = P1 = a I + (b G)/s^2 + (c G2)/s^4 formed from FP32 G and
//               G2 tiles (and split in compensated mode).
//  FP32       : FP32 tile.
template <int MODE, bool POLY>
__device__ __forceinline__ void load_a(const char *st, int wm, int i, int64_t k0, const PolyArgs &pa,
                                       AFrag<MODE> &f) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const int r = wm * (32 * kSubM) + i * 32 + lr;
  if constexpr (MODE == SMX_S8_FP32 || POLY) {
    float av[8];
    read8(st, r, lh, av);
    if constexpr (POLY) {
      float w[8];
      read8(st + kF32Tile, r, lh, w);
      const int64_t grow = pa.row0 + r;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t gk = k0 + 8 * lh + e;
        const float eye = (grow == gk && grow < pa.r) ? pa.a : 0.f;
        av[e] = (eye + (pa.b * av[e]) * pa.is2) + (pa.c * w[e]) * pa.is4;
      }
    }
    if constexpr (MODE == SMX_S8_COMP_BF16) {
      split8(av, f.h, f.l);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f.v[e] = av[e];
    }
  } else {
    f.h = read_b16(st, r, lh);
    f.l = read_b16(st + kB16Tile, r, lh);
  }
}

template <int MODE, bool POLY>
__device__ __forceinline__ void load_b(const char *st, int wn, BFrags<MODE> &f) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  constexpr bool A_F32 = MODE == SMX_S8_FP32 || POLY;
  const char *bt = st + (POLY ? 2 * kF32Tile : (A_F32 ? kF32Tile : 2 * kB16Tile));
#pragma unroll
  for (int j = 0; j < kSubN; ++j) {
    const int r = wn * (32 * kSubN) + j * 32 + lr;
    if constexpr (MODE == SMX_S8_COMP_BF16) {
      f.h[j] = read_b16(bt, r, lh);
      f.l[j] = read_b16(bt + kB16Tile, r, lh);
    } else {
      read8(bt, r, lh, f.v[j]);
    }
  }
}

// MFMAs of row block i: acc[i][j] += A_i B_j^T over the stage's 16 K.
template <int MODE>
__device__ __forceinline__ void mma_row(const AFrag<MODE> &a, const BFrags<MODE> &b, f32x16 (&acc)[kSubN]) {
  if constexpr (MODE == SMX_S8_COMP_BF16) {
    // Corrections first, then hi*hi.
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.l[j], acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.l, b.h[j], acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.h, b.h[j], acc[j], 0, 0, 0);
  } else {
    // Lane half h supplies k = 8h + q to MFMA q (the same permutation for
    // both operands, so every k is paired exactly once).
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < kSubN; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[q], b.v[j][q], acc[j], 0, 0, 0);
  }
}

// Issues one stage: A (or G, G2 in POLY) and B into the ring slot.
template <int MODE, bool POLY>
__device__ __forceinline__ void issue_stage(const Opnd &A, const Opnd &A2, const Opnd &B, int64_t arow0,
                                            int64_t brow0, int64_t k0, char *st) {
  if constexpr (MODE == SMX_S8_FP32 || POLY) {
    dma_f32(static_cast<const float *>(A.p), A.ld, arow0, k0, st);
    if constexpr (POLY) dma_f32(static_cast<const float *>(A2.p), A2.ld, arow0, k0, st + kF32Tile);
  } else {
    const uint16_t *a = static_cast<const uint16_t *>(A.p);
    dma_b16(a, A.ld, arow0, k0, st);
    dma_b16(a + A.plane, A.ld, arow0, k0, st + kB16Tile);
  }
  char *bt = st + (POLY ? 2 * kF32Tile : (MODE == SMX_S8_FP32 ? kF32Tile : 2 * kB16Tile));
  if constexpr (MODE == SMX_S8_FP32) {
    dma_f32(static_cast<const float *>(B.p), B.ld, brow0, k0, bt);
  } else {
    const uint16_t *b = static_cast<const uint16_t *>(B.p);
    dma_b16(b, B.ld, brow0, k0, bt);
    dma_b16(b + B.plane, B.ld, brow0, k0, bt + kB16Tile);
  }
}

// Waits until at most `pending` stages of this wave's loads are in flight
// (each stage is L loads; loads complete in issue order).
template <int L>
__device__ __forceinline__ void wait_stages(int pending) {
  if (pending >= 3) wait_vm<3 * L>();
  else if (pending == 2) wait_vm<2 * L>();
  else if (pending == 1) wait_vm<L>();
  else wait_vm<0>();
}

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// C[256 x 256] = A[arow0.., :K] * B[brow0.., :K]^T.
//
// Two pipelines overlap the MFMAs:
//  * a ring of S LDS slots filled by direct-to-LDS loads, S stages ahead of
//    the fragment reads;
//  * register fragments: while the MFMAs of stage kt run, the fragments of
//    stage kt+1 are read from LDS (B into the other buffer up front, each A
//    row block right after its last MFMA of stage kt).
// Iteration kt: wait for this wave's loads of stage kt+1 and for its own
// outstanding LDS reads (those of stage kt, so slot kt is free); a block
// barrier makes every wave's loads of kt+1 visible and every wave's reads
// of kt finished; refill slot kt with stage kt+S; MFMAs of stage kt
// interleaved with the reads of stage kt+1.
template <int MODE, bool POLY, int PAR>
__device__ __forceinline__ void pipe_iter(const Opnd &A, const Opnd &A2, const Opnd &B, int64_t arow0,
                                          int64_t brow0, const PolyArgs &pa, char *smem, int kt, int nk, int wm,
                                          int wn, AFrag<MODE> (&af)[kSubM], BFrags<MODE> (&bf)[2],
                                          f32x16 (&acc)[kSubM][kSubN]) {
  constexpr int S = POLY ? kPolyStages : kStages;
  constexpr int SB = POLY ? kPolyStageBytes : kStageBytes;
  constexpr int L = POLY ? 12 : 8;
  const bool more = kt + 1 < nk;
  if (more) wait_stages<L>(min(S - 2, nk - 2 - kt));
  wait_lds();
  block_barrier();
  if (kt + S < nk)
    issue_stage<MODE, POLY>(A, A2, B, arow0, brow0, static_cast<int64_t>(kt + S) * kBK, smem + (kt % S) * SB);
  const char *nxt = smem + ((kt + 1) % S) * SB;
  const int64_t k1 = static_cast<int64_t>(kt + 1) * kBK;
  if (more) load_b<MODE, POLY>(nxt, wn, bf[PAR ^ 1]);
#pragma unroll
  for (int i = 0; i < kSubM; ++i) {
    mma_row<MODE>(af[i], bf[PAR], acc[i]);
    if (more) load_a<MODE, POLY>(nxt, wm, i, k1, pa, af[i]);
  }
}

template <int MODE, bool POLY>
__device__ __forceinline__ void gemm_256(const Opnd &A, const Opnd &A2, const Opnd &B, int64_t K, int64_t arow0,
                                         int64_t brow0, PolyArgs pa, char *smem, f32x16 (&acc)[kSubM][kSubN]) {
  constexpr int S = POLY ? kPolyStages : kStages;
  constexpr int SB = POLY ? kPolyStageBytes : kStageBytes;
  constexpr int L = POLY ? 12 : 8;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  pa.row0 = arow0;
#pragma unroll
  for (int i = 0; i < kSubM; ++i)
#pragma unroll
    for (int j = 0; j < kSubN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int nk = static_cast<int>(K / kBK);
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < nk) issue_stage<MODE, POLY>(A, A2, B, arow0, brow0, static_cast<int64_t>(s) * kBK, smem + s * SB);
  wait_stages<L>(min(S - 1, nk - 1));
  block_barrier();
  AFrag<MODE> af[kSubM];
  BFrags<MODE> bf[2];
  load_b<MODE, POLY>(smem, wn, bf[0]);
#pragma unroll
  for (int i = 0; i < kSubM; ++i) load_a<MODE, POLY>(smem, wm, i, 0, pa, af[i]);
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    pipe_iter<MODE, POLY, 0>(A, A2, B, arow0, brow0, pa, smem, kt, nk, wm, wn, af, bf, acc);
    pipe_iter<MODE, POLY, 1>(A, A2, B, arow0, brow0, pa, smem, kt + 1, nk, wm, wn, af, bf, acc);
  }
  if (kt < nk) pipe_iter<MODE, POLY, 0>(A, A2, B, arow0, brow0, pa, smem, kt, nk, wm, wn, af, bf, acc);
  block_barrier();
}

// ---------------------------------------------------------- scalars ---
// Sum of a small FP64 partial array by wave 0; result broadcast.
__device__ double sum_parts(const double *p, int n, double *bcast) {
  if (threadIdx.x < 64) {
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 64) s += p[i];
    s = wave_sum(s);
    if (threadIdx.x == 0) *bcast = s;
  }
  __syncthreads();
  const double v = *bcast;
  __syncthreads();
  return v;
}

__device__ __forceinline__ int fro_parts_used(const S8Mat &m) {
  return static_cast<int>(ceil_div(m.prow(), kRowsPerPart));
}

// ------------------------------------------------------------ kernel ---
template <int MODE, int PHASE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
s8_stage_kernel(StageArgs args) {
  __shared__ __attribute__((aligned(16))) char smem[kRingBytes];
  __shared__ double dscratch[16];
  __shared__ double bcast;
  constexpr bool PL = MODE == SMX_S8_COMP_BF16;  // operands stored as BF16 planes

  // Segment (class) of this block and its XCD-contiguous tile index.
  const int b = blockIdx.x;
  int seg = 0;
  while (seg + 1 < args.n_seg && b >= args.seg_off[seg + 1]) ++seg;
  const S8Class K = args.L.cls[args.seg_cls[seg]];
  const int jb = b - args.seg_off[seg];
  const int per = (args.seg_off[seg + 1] - args.seg_off[seg]) / 8;
  const int64_t L = static_cast<int64_t>(jb % 8) * per + jb / 8;
  const int64_t tpm = PHASE == kApply ? static_cast<int64_t>(K.tiles_m) * K.tiles_n : sym_tiles(K.tiles_m);
  if (L >= tpm * K.count) return;
  const int slot = static_cast<int>(L / tpm);
  const int64_t tix = L % tpm;
  int64_t tm, tn;
  if constexpr (PHASE == kApply) {
    tm = tix / K.tiles_n;
    tn = tix % K.tiles_n;
  } else {
    int64_t rem = tix;
    tm = 0;
    while (rem >= K.tiles_m - tm) { rem -= K.tiles_m - tm; ++tm; }
    tn = tm + rem;
  }
  const S8Mat M{K, slot};
  const int stage = args.stage;
  const bool odd = (stage & 1) != 0;
  float *x_in = odd ? M.x0() : M.x1();
  float *xt_in = odd ? M.xt0() : M.xt1();
  float *x_out = odd ? M.x1() : M.x0();
  float *xt_out = odd ? M.xt1() : M.xt0();
  const int64_t nx = K.rp * K.cp, ng = K.rp * K.rp;

  f32x16 acc[kSubM][kSubN];
  PolyArgs pa{};
  float scale = 1.f;
  const Opnd none{nullptr, 0, 0};
  if constexpr (PHASE == kGram) {
    if (stage == 1) {
      const double f = sum_parts(M.fro(), fro_parts_used(M), &bcast);
      scale = f > 0.0 ? static_cast<float>(1.0 / f) : 0.f;
    }
    const Opnd X{x_in, K.cp, nx};
    gemm_256<MODE, false>(X, none, X, K.cp, tm * kTile, tn * kTile, pa, smem, acc);
  } else if constexpr (PHASE == kSquare) {
    const Opnd G{PL ? M.gs() : M.g(), K.rp, ng};
    gemm_256<MODE, false>(G, none, G, K.rp, tm * kTile, tn * kTile, pa, smem, acc);
  } else {
    const Opnd XT{xt_in, K.rp, nx};
    if (stage == 1) {
      const double f = sum_parts(M.fro(), fro_parts_used(M), &bcast);
      const double sq = sum_parts(M.sch(), static_cast<int>(sym_tiles(K.tiles_m)), &bcast);
      pa.a = args.a; pa.b = args.b; pa.c = args.c; pa.r = K.r;
      if (f > 0.0 && sq > 0.0) {
        // s = max(1.35 * ||G2||_F^(1/4), 1e-30) on the normalised G2.
        const float s = fmaxf(static_cast<float>(kS8Margin * pow(sq, 0.125)), 1e-30f);
        const float s2 = s * s;
        pa.is2 = 1.0f / s2;
        pa.is4 = 1.0f / (s2 * s2);
        scale = static_cast<float>(1.0 / (sqrt(f) * static_cast<double>(s)));
      } else {
        pa.is2 = 0.f; pa.is4 = 0.f; scale = 0.f;
      }
      gemm_256<MODE, true>(Opnd{M.g(), K.rp, 0}, Opnd{M.p(), K.rp, 0}, XT, K.rp, tm * kTile, tn * kTile, pa,
                           smem, acc);
    } else {
      gemm_256<MODE, false>(Opnd{M.p(), K.rp, ng}, none, XT, K.rp, tm * kTile, tn * kTile, pa, smem, acc);
    }
  }

  // ------------------------------------------------------- epilogue ---
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t R0 = tm * kTile, C0 = tn * kTile;
  float sq_local = 0.f;
#pragma unroll
  for (int i = 0; i < kSubM; ++i)
#pragma unroll
    for (int j = 0; j < kSubN; ++j) {
      const int64_t col = C0 + wn * (32 * kSubN) + j * 32 + lr;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t row = R0 + wm * (32 * kSubM) + i * 32 + 8 * k + 4 * lh;  // rows row..row+3
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc[i][j][4 * k + q];
        if constexpr (PHASE == kGram) {
          float *G = M.g();
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[q] *= scale;
            G[(row + q) * K.rp + col] = v[q];
            if constexpr (PL) put_operand(M.gs(), ng, (row + q) * K.rp + col, v[q], true);
          }
          if (tm != tn) {
            *reinterpret_cast<float4 *>(G + col * K.rp + row) = make_float4(v[0], v[1], v[2], v[3]);
            if constexpr (PL) put_operand4(M.gs(), ng, col * K.rp + row, v, true);
          }
        } else if constexpr (PHASE == kSquare) {
          float *P = M.p();
          const bool planes = PL && stage != 1;  // stage 1 keeps FP32 G2
          if (stage == 1) {
#pragma unroll
            for (int q = 0; q < 4; ++q) sq_local = fmaf(v[q], v[q], sq_local);
          } else {
            const float *G = M.g();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t rr = row + q;
              const float eye = (rr == col && rr < K.r) ? args.a : 0.f;
              v[q] = (eye + args.b * G[rr * K.rp + col]) + args.c * v[q];
            }
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) put_operand(P, ng, (row + q) * K.rp + col, v[q], planes);
          if (tm != tn) put_operand4(P, ng, col * K.rp + row, v, planes);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] *= scale;
          const bool last = stage == 5;
          // The stage-5 result is FP32 in parameter layout only.
          if (!last || !M.flip()) {
#pragma unroll
            for (int q = 0; q < 4; ++q) put_operand(x_out, nx, (row + q) * K.cp + col, v[q], PL && !last);
          }
          if (!last || M.flip()) put_operand4(xt_out, nx, col * K.rp + row, v, PL && !last);
        }
      }
      // Keep the scheduler from hoisting every accumulator read to the top
      // of the epilogue (256 values would not fit in the VGPRs).
      __builtin_amdgcn_sched_barrier(0);
    }
  if constexpr (PHASE == kSquare) {
    if (stage == 1) {
      const double s = block_sum(static_cast<double>(sq_local), dscratch);
      if (threadIdx.x == 0) M.sch()[tix] = (tm == tn ? 1.0 : 2.0) * s;
    }
  }
}

// ------------------------------------------------------------- host ---
template <int PHASE>
static int launch_phase(const S8Layout &Lay, int stage, hipStream_t st) {
  StageArgs a{};
  a.L = Lay;
  a.stage = stage;
  const auto &co = kS8Coefficients[stage - 1];
  a.a = static_cast<float>(co[0]);
  a.b = static_cast<float>(co[1]);
  a.c = static_cast<float>(co[2]);
  // Order classes by per-tile cost (K length), most expensive first.
  std::vector<int> order(Lay.n_classes);
  for (int i = 0; i < Lay.n_classes; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
    const int64_t kx = PHASE == kGram ? Lay.cls[x].cp : Lay.cls[x].rp;
    const int64_t ky = PHASE == kGram ? Lay.cls[y].cp : Lay.cls[y].rp;
    return kx > ky;
  });
  int32_t off = 0;
  a.n_seg = 0;
  for (int ci : order) {
    const S8Class &k = Lay.cls[ci];
    if (k.count == 0) continue;
    const int64_t tpm = PHASE == kApply ? static_cast<int64_t>(k.tiles_m) * k.tiles_n : sym_tiles(k.tiles_m);
    const int64_t nt = round_up(tpm * k.count, 8);
    a.seg_off[a.n_seg] = off;
    a.seg_cls[a.n_seg] = ci;
    ++a.n_seg;
    off += static_cast<int32_t>(nt);
  }
  a.seg_off[a.n_seg] = off;
  if (off == 0) return SMX_OK;
  if (Lay.mode == SMX_S8_COMP_BF16)
    hipLaunchKernelGGL((s8_stage_kernel<SMX_S8_COMP_BF16, PHASE>), dim3(off), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((s8_stage_kernel<SMX_S8_FP32, PHASE>), dim3(off), dim3(kThreads), 0, st, a);
  return check_launch(PHASE == kGram ? "s8 gram" : PHASE == kSquare ? "s8 square" : "s8 apply");
}

int run_s8_stages(const S8Layout &Lay, hipStream_t st) {
  for (int stage = 1; stage <= 5; ++stage) {
    int rc = launch_phase<kGram>(Lay, stage, st);
    if (!rc) rc = launch_phase<kSquare>(Lay, stage, st);
    if (!rc) rc = launch_phase<kApply>(Lay, stage, st);
    if (rc) return rc;
  }
  return SMX_OK;
}

bool plan_s8(const int64_t *r, const int64_t *c, const bool *flips, int32_t n, int mode, char *base,
             S8Plan &plan, int32_t *cls_of, int32_t *slot_of) {
  S8Layout &Lay = plan.layout;
  Lay = S8Layout{};
  Lay.mode = mode;
  // Classes by oriented shape in order of first appearance; transposed
  // parameters take the low slots of their class.
  std::vector<int> ncount, nflip;
  for (int32_t i = 0; i < n; ++i) {
    int ci = -1;
    for (int k = 0; k < Lay.n_classes; ++k)
      if (Lay.cls[k].r == r[i] && Lay.cls[k].c == c[i]) { ci = k; break; }
    if (ci < 0) {
      if (Lay.n_classes == kMaxClasses) return false;
      ci = Lay.n_classes++;
      Lay.cls[ci].r = r[i];
      Lay.cls[ci].c = c[i];
      ncount.push_back(0);
      nflip.push_back(0);
    }
    cls_of[i] = ci;
    ncount[ci]++;
    if (flips[i]) nflip[ci]++;
  }
  std::vector<int> next_flip(Lay.n_classes, 0), next_plain(Lay.n_classes, 0);
  for (int k = 0; k < Lay.n_classes; ++k) next_plain[k] = nflip[k];
  for (int32_t i = 0; i < n; ++i) {
    const int ci = cls_of[i];
    slot_of[i] = flips[i] ? next_flip[ci]++ : next_plain[ci]++;
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~static_cast<size_t>(255);
    return base ? base + o : nullptr;
  };
  for (int k = 0; k < Lay.n_classes; ++k) {
    S8Class &C = Lay.cls[k];
    C.count = ncount[k];
    C.n_flip = nflip[k];
    C.rp = round_up(C.r, kTile);
    C.cp = round_up(C.c, kTile);
    C.tiles_m = static_cast<int32_t>(C.rp / kTile);
    C.tiles_n = static_cast<int32_t>(C.cp / kTile);
    C.parts = static_cast<int32_t>(ceil_div(C.cp, kRowsPerPart));
    const size_t xs = static_cast<size_t>(C.count) * C.rp * C.cp * sizeof(float);
    const size_t gs = static_cast<size_t>(C.count) * C.rp * C.rp * sizeof(float);
    C.x0 = reinterpret_cast<float *>(take(xs));
    C.xt0 = reinterpret_cast<float *>(take(xs));
    C.x1 = reinterpret_cast<float *>(take(xs));
    C.xt1 = reinterpret_cast<float *>(take(xs));
    C.g = reinterpret_cast<float *>(take(gs));
    C.gs = reinterpret_cast<float *>(take(gs));
    C.p = reinterpret_cast<float *>(take(gs));
    C.u = reinterpret_cast<float *>(take(static_cast<size_t>(C.count) * C.cp * sizeof(float)));
    C.fro = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * C.parts * sizeof(double)));
    C.mb = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * C.parts * sizeof(double)));
    C.sch = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * sym_tiles(C.tiles_m) * sizeof(double)));
  }
  plan.bytes = off;
  return true;
}

}  // namespace smx
