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
// Block: 256x256 output tile, 8 waves (2 x 4), each wave 128x64 (4 x 2
// MFMA 32x32 tiles); K step 32, double-buffered LDS (2 x 64 KB).
#include "s8.h"

#include <algorithm>
#include <cmath>
#include <vector>

namespace smx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kBK = 32;
constexpr int kLdsBuf = 65536;  // bytes per pipeline buffer

enum Phase { kGram = 0, kSquare = 1, kApply = 2 };

struct StageArgs {
  S8Layout L;
  int32_t seg_off[kMaxClasses + 1];  // block offsets (multiples of 8)
  int32_t seg_cls[kMaxClasses];
  int32_t n_seg;
  int32_t stage;  // 1..5
  float a, b, c;
};

// ---------------------------------------------------------- operands ---
struct PolyArgs {
  float a, b, c;     // stage-1 coefficients
  float is2, is4;    // 1/s^2, 1/s^4
  int64_t r;         // logical rows (identity only on real rows)
};

// Loads the kThreads-share of a 256 x 32 FP32 tile starting at (row0, k0):
// thread t reads rows t/8 + 64q, columns (t%8)*4 .. +3.
template <bool POLY>
__device__ __forceinline__ void load_a_tile(const float *__restrict__ A, const float *__restrict__ A2,
                                            int64_t ld, int64_t row0, int64_t k0, const PolyArgs &pa,
                                            float4 (&out)[4]) {
  const int t = threadIdx.x;
  const int64_t col = k0 + (t & 7) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = row0 + (t >> 3) + 64 * q;
    float4 v = *reinterpret_cast<const float4 *>(A + row * ld + col);
    if constexpr (POLY) {
      // P1 = a I + (b G)/s^2 + (c G2)/s^4, evaluated left to right.
      const float4 w = *reinterpret_cast<const float4 *>(A2 + row * ld + col);
      float g[4] = {v.x, v.y, v.z, v.w}, g2[4] = {w.x, w.y, w.z, w.w};
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float eye = (row == col + e && row < pa.r) ? pa.a : 0.f;
        p[e] = (eye + (pa.b * g[e]) * pa.is2) + (pa.c * g2[e]) * pa.is4;
      }
      v = make_float4(p[0], p[1], p[2], p[3]);
    }
    out[q] = v;
  }
}

__device__ __forceinline__ void load_b_tile(const float *__restrict__ B, int64_t ld, int64_t row0,
                                            int64_t k0, float4 (&out)[4]) {
  const int t = threadIdx.x;
  const int64_t col = k0 + (t & 7) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = row0 + (t >> 3) + 64 * q;
    out[q] = *reinterpret_cast<const float4 *>(B + row * ld + col);
  }
}

// ------------------------------------------------------ LDS staging ---
// COMP layout of one buffer: planes Ah, Al, Bh, Bl of [256][32] bf16 (64 B
// rows, four 16-B chunks; chunk index XOR ((row>>1)&3)).
// FP32 layout: planes A, B of [256][32] f32 (128 B rows, eight chunks;
// chunk index XOR (row&7)).
__device__ __forceinline__ int comp_off(int row, int ch) { return row * 64 + ((ch ^ ((row >> 1) & 3)) << 4); }
__device__ __forceinline__ int f32_off(int row, int ch) { return row * 128 + ((ch ^ (row & 7)) << 4); }

__device__ __forceinline__ void split4(float4 v, uint2 &hi, uint2 &lo) {
  float x[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = f32_to_bf16_bits(x[e]);
    l[e] = f32_to_bf16_bits(x[e] - bf16_bits_to_f32(h[e]));
  }
  hi = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
  lo = make_uint2(l[0] | (static_cast<uint32_t>(l[1]) << 16), l[2] | (static_cast<uint32_t>(l[3]) << 16));
}

template <int MODE>
__device__ __forceinline__ void store_tiles(char *buf, const float4 (&ra)[4], const float4 (&rb)[4]) {
  const int t = threadIdx.x;
  if constexpr (MODE == SMX_S8_COMP_BF16) {
    const int ch = (t & 7) >> 1, half = (t & 1) * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = (t >> 3) + 64 * q;
      const int off = comp_off(row, ch) + half;
      uint2 h, l;
      split4(ra[q], h, l);
      *reinterpret_cast<uint2 *>(buf + 0 * 16384 + off) = h;
      *reinterpret_cast<uint2 *>(buf + 1 * 16384 + off) = l;
      split4(rb[q], h, l);
      *reinterpret_cast<uint2 *>(buf + 2 * 16384 + off) = h;
      *reinterpret_cast<uint2 *>(buf + 3 * 16384 + off) = l;
    }
  } else {
    const int ch = t & 7;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = (t >> 3) + 64 * q;
      const int off = f32_off(row, ch);
      *reinterpret_cast<float4 *>(buf + off) = ra[q];
      *reinterpret_cast<float4 *>(buf + 32768 + off) = rb[q];
    }
  }
}

// ----------------------------------------------------------- compute ---
template <int MODE>
__device__ __forceinline__ void compute_tile(const char *buf, int wm, int wn, f32x16 (&acc)[4][2]) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  if constexpr (MODE == SMX_S8_COMP_BF16) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ch = s * 2 + lh;
      bf16x8 ah[4], al[4], bh[2], bl[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = comp_off(wm * 128 + i * 32 + lr, ch);
        ah[i] = *reinterpret_cast<const bf16x8 *>(buf + off);
        al[i] = *reinterpret_cast<const bf16x8 *>(buf + 16384 + off);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int off = comp_off(wn * 64 + j * 32 + lr, ch);
        bh[j] = *reinterpret_cast<const bf16x8 *>(buf + 32768 + off);
        bl[j] = *reinterpret_cast<const bf16x8 *>(buf + 49152 + off);
      }
      // Corrections first, then hi*hi (per K step).
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
      const int ch = kg * 2 + lh;
      f32x4 av[4], bv[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        av[i] = *reinterpret_cast<const f32x4 *>(buf + f32_off(wm * 128 + i * 32 + lr, ch));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = *reinterpret_cast<const f32x4 *>(buf + 32768 + f32_off(wn * 64 + j * 32 + lr, ch));
      // Lane half h supplies k = 8kg + 4h + q to MFMA q: the same K
      // permutation for both operands, so every k is paired exactly once.
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][q], bv[j][q], acc[i][j], 0, 0, 0);
    }
  }
}

template <int MODE, bool POLY>
__device__ __forceinline__ void gemm_256(const float *__restrict__ A, const float *__restrict__ A2,
                                         const float *__restrict__ B, int64_t K, int64_t arow0,
                                         int64_t brow0, const PolyArgs &pa, char *smem,
                                         f32x16 (&acc)[4][2]) {
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int nk = static_cast<int>(K / kBK);
  float4 ra[4], rb[4];
  load_a_tile<POLY>(A, A2, K, arow0, 0, pa, ra);
  load_b_tile(B, K, brow0, 0, rb);
  store_tiles<MODE>(smem, ra, rb);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) {
      load_a_tile<POLY>(A, A2, K, arow0, static_cast<int64_t>(kt + 1) * kBK, pa, ra);
      load_b_tile(B, K, brow0, static_cast<int64_t>(kt + 1) * kBK, rb);
    }
    compute_tile<MODE>(smem + (kt & 1) * kLdsBuf, wm, wn, acc);
    if (more) store_tiles<MODE>(smem + ((kt + 1) & 1) * kLdsBuf, ra, rb);
    __syncthreads();
  }
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
__global__ void __launch_bounds__(kThreads) s8_stage_kernel(StageArgs args) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kLdsBuf];
  __shared__ double dscratch[16];
  __shared__ double bcast;

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

  f32x16 acc[4][2];
  PolyArgs pa{};
  float scale = 1.f;
  if constexpr (PHASE == kGram) {
    if (stage == 1) {
      const double f = sum_parts(M.fro(), fro_parts_used(M), &bcast);
      scale = f > 0.0 ? static_cast<float>(1.0 / f) : 0.f;
    }
    gemm_256<MODE, false>(x_in, nullptr, x_in, K.cp, tm * kTile, tn * kTile, pa, smem, acc);
  } else if constexpr (PHASE == kSquare) {
    gemm_256<MODE, false>(M.g(), nullptr, M.g(), K.rp, tm * kTile, tn * kTile, pa, smem, acc);
  } else {
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
      gemm_256<MODE, true>(M.g(), M.p(), xt_in, K.rp, tm * kTile, tn * kTile, pa, smem, acc);
    } else {
      gemm_256<MODE, false>(M.p(), nullptr, xt_in, K.rp, tm * kTile, tn * kTile, pa, smem, acc);
    }
  }

  // ------------------------------------------------------- epilogue ---
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 2, wn = wave & 3;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t R0 = tm * kTile, C0 = tn * kTile;
  float sq_local = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = C0 + wn * 64 + j * 32 + lr;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t row = R0 + wm * 128 + i * 32 + 8 * k + 4 * lh;  // rows row..row+3
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc[i][j][4 * k + q];
        if constexpr (PHASE == kGram) {
          float *G = M.g();
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[q] *= scale;
            G[(row + q) * K.rp + col] = v[q];
          }
          if (tm != tn) *reinterpret_cast<float4 *>(G + col * K.rp + row) = make_float4(v[0], v[1], v[2], v[3]);
        } else if constexpr (PHASE == kSquare) {
          float *P = M.p();
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
          for (int q = 0; q < 4; ++q) P[(row + q) * K.rp + col] = v[q];
          if (tm != tn) *reinterpret_cast<float4 *>(P + col * K.rp + row) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] *= scale;
          const bool last = stage == 5;
          if (!last || !M.flip()) {
#pragma unroll
            for (int q = 0; q < 4; ++q) x_out[(row + q) * K.cp + col] = v[q];
          }
          if (!last || M.flip())
            *reinterpret_cast<float4 *>(xt_out + col * K.rp + row) = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
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
