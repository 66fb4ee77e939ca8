// Workspace layout shared by the matrix-step kernels (whiten, S8 GEMMs,
// mapback).  Matrices are grouped in classes of equal oriented shape
// (r <= c); every class buffer is padded to multiples of kTile so that the
// GEMM tiles never need bounds checks.  Padding holds zeros.
//
// Two iteration forms.  Each stage's P_k is a polynomial in the stage's
// Gram G_k = X_k X_k^T, so every P_k and G_k commute.  A class with
// cp == rp runs the stages on the iterate (X-space): G = X X^T, P from G,
// X <- P X.  A wider class (cp > rp, Gram space) runs them on r x r
// matrices, G_{k+1} = P_k G_k P_k and Q_k = P_k Q_{k-1}, in two segments:
// stages 1-2 from X0 (then X2 = Q2 X0), stages 3-5 from a fresh Gram of
// X2 (then X5 = Q X2).  A Gram carried forward keeps the absolute rounding
// of the Gram it started from, which the small eigenvalues of a
// long-tailed spectrum cannot afford over more than two or three stages;
// the fresh Gram of X2 restores their relative precision.  For r x c with
// c = 4r this takes a third fewer MFMA FLOPs than X-space.
#pragma once

#include "common.h"

namespace smx {

constexpr int kTile = 256;        // apply tile rows and buffer padding
constexpr int kSymTile = 128;     // Gram / square output tile edge
constexpr int kMaxClasses = 8;    // shape classes per GEMM launch
// Parameter columns per stage-5 row-sum partial: a wave's 64 output columns
// of an apply tile, or (transposed parameter) 64 of its output rows (two
// strips per wave of a 256-row tile, one per wave of a 128-row tile).
constexpr int kStripT = 64, kStripM = 64;

// Fixed S8 recipe: sandmuon/coefficients.py:3-11.
constexpr double kS8Margin = 1.35;
constexpr double kS8Coefficients[5][3] = {
    {11.062126275847973, -56.051653229128085, 72.32081107619855},
    {4.100720073616268, -2.9324183165353577, 0.5339692084282731},
    {3.930310192522361, -2.873509793709714, 0.5366557527206212},
    {3.280567968245866, -2.414925589994015, 0.48635134757825227},
    {2.282741575232451, -1.6302296637355072, 0.40275720810675486},
};

// Per-matrix scalars (S8Class::cst): ||V||^2 of the whitened input (the
// S8 normalisation; the total of the whiten partials, or of the input for
// the stand-alone map), sum z^2 and sum (a z)^2 of the rank-one term, and
// ||U||^2 of the mapped-back direction (the graft).
constexpr int kCstFro = 0, kCstZZ = 1, kCstAZ = 2, kCstU = 3, kCst = 4;

struct S8Class {
  int64_t r, c;        // oriented logical dims, r <= c
  int64_t rp, cp;      // padded dims
  int32_t count;       // matrices in the class
  int32_t n_flip;      // slots [0, n_flip) hold transposed parameters
  int32_t tiles_m;     // rp / kTile
  int32_t tiles_n;     // cp / kTile
  int32_t parts;       // per-block partial slots per matrix (2 cp: two partials
                       // for each of the at most cp blocks a whiten launch gives one matrix)
  int32_t tiles_s;     // rp / kSymTile
  int32_t gs;          // Gram-space iteration (cp > rp): the stages run on r x r
                       // products and X0 is applied once, at stage 5
  // Iterate buffers (4 bytes per element), oriented layout only: tiled
  // operands (tiled_index), FP32 in SMX_S8_FP32 mode and interleaved BF16
  // hi/lo (put_operand) or FP16 in the others, except the stage-5 result,
  // which is a row-major FP32 matrix.
  float *x0, *x1;      // [count][rp][cp] ping, pong (Gram space: X0, then X2)
  float *xf;           // [n_flip][cp][rp] stage-5 result of transposed parameters
                       // (parameter layout); the others end in x1 (X-space)
                       // or x0 (Gram space)
  float *g;            // [count][rp][rp] Gram (tiled operand)
  float *p;            // [count][rp][rp] stage 1: FP32 G2; later: P (tiled, like every operand)
  float *t, *qa, *qb;  // Gram-space classes only, [count][rp][rp] each (operand
                       // form): T = P G, and the accumulated product Q of a
                       // segment's stage polynomials (qa, qb: ping-pong)
  float *u;            // [count][cp] per param-row rank-one coefficient
  double *fro;         // [count][parts] whiten: per-block partial sums (two kinds)
  double *mb;          // [count][parts] mapback: per-block partial sums of U^2
  double *sch;         // [count][sym_tiles(tiles_s)] Schatten partials (one per upper-triangle Gram tile)
  double *cst;         // [count][kCst] per-matrix scalars (see the kCst* indices)
  // Matrix step only (S8Layout::rowsums): the A factor diagonal and the
  // rank-one vector (NULL without one) of each slot's matrix, and the
  // stage-5 row-sum partials of the mapback: per parameter row and strip
  // of kStripT parameter columns (kStripM for a transposed parameter), the
  // sums of Q z, (a Q)^2 and (a Q)(a z).
  const float **colv;  // [count][2]: inv_col, z
  float *mrp;          // [count][3][rp * cp / kStripT]
};

struct S8Layout {
  S8Class cls[kMaxClasses];
  int32_t n_classes;
  int32_t mode;
  int32_t rowsums;  // the stage-5 apply writes the mapback row-sum partials (matrix step)
};

__host__ __device__ inline int64_t sym_tiles(int64_t t) { return t * (t + 1) / 2; }

// Per-matrix views of a class slot.
struct S8Mat {
  S8Class k_;
  int32_t slot;
  __host__ __device__ const S8Class *kp() const { return &k_; }
  __host__ __device__ bool flip() const { return slot < kp()->n_flip; }
  __host__ __device__ float *x0() const { return kp()->x0 + slot * kp()->rp * kp()->cp; }
  __host__ __device__ float *x1() const { return kp()->x1 + slot * kp()->rp * kp()->cp; }
  // Valid for flip() only.
  __host__ __device__ float *xf() const { return kp()->xf + slot * kp()->rp * kp()->cp; }
  // The stage-5 result in parameter layout [prow_pad][pcol_pad].
  __host__ __device__ float *result() const { return flip() ? xf() : kp()->gs ? x0() : x1(); }
  __host__ __device__ float *g() const { return kp()->g + slot * kp()->rp * kp()->rp; }
  __host__ __device__ float *p() const { return kp()->p + slot * kp()->rp * kp()->rp; }
  __host__ __device__ float *t() const { return kp()->t + slot * kp()->rp * kp()->rp; }
  __host__ __device__ float *qa() const { return kp()->qa + slot * kp()->rp * kp()->rp; }
  __host__ __device__ float *qb() const { return kp()->qb + slot * kp()->rp * kp()->rp; }
  __host__ __device__ float *u() const { return kp()->u + slot * kp()->cp; }
  __host__ __device__ double *fro() const { return kp()->fro + static_cast<int64_t>(slot) * kp()->parts; }
  __host__ __device__ double *mb() const { return kp()->mb + static_cast<int64_t>(slot) * kp()->parts; }
  __host__ __device__ double *sch() const { return kp()->sch + slot * sym_tiles(kp()->tiles_s); }
  __host__ __device__ double *cst() const { return kp()->cst + kCst * static_cast<int64_t>(slot); }
  __host__ __device__ const float *acol() const { return kp()->colv[2 * slot]; }
  __host__ __device__ const float *zcol() const { return kp()->colv[2 * slot + 1]; }
  __host__ __device__ const float **colv() const { return kp()->colv + 2 * slot; }
  // Row-sum partials: k = 0 (Q z), 1 ((a Q)^2), 2 ((a Q)(a z)), each
  // [strips()][prow_pad] (a strip's rows contiguous).
  __host__ __device__ int64_t mrp_size() const { return kp()->rp * kp()->cp / kStripT; }
  __host__ __device__ float *mrp(int k) const { return kp()->mrp + (3 * static_cast<int64_t>(slot) + k) * mrp_size(); }
  __host__ __device__ int64_t strips() const { return flip() ? kp()->rp / kStripM : kp()->cp / kStripT; }
  // Parameter layout: rows x cols (the transpose of the oriented layout
  // for transposed parameters).
  __host__ __device__ int64_t prow() const { return flip() ? kp()->c : kp()->r; }
  __host__ __device__ int64_t pcol() const { return flip() ? kp()->r : kp()->c; }
  __host__ __device__ int64_t prow_pad() const { return flip() ? kp()->cp : kp()->rp; }
  __host__ __device__ int64_t pcol_pad() const { return flip() ? kp()->rp : kp()->cp; }
};

// GEMM operand buffers hold ld K columns per row (ld a multiple of 16 for
// the 4-byte forms, of 32 for FP16) and rows padded to multiples of kTile.
// In compensated mode an element v is stored as two BF16 values, hi =
// bf16(v) and lo = bf16(v - hi) (round to nearest even), interleaved per
// 16-element K group: 16 hi values, then the 16 matching lo values.  The
// buffer has the byte size of its FP32 form and the 16-element K group of a
// row is one contiguous 64-byte run in both forms (32 elements in FP16).
// Those runs are tiled: the runs of group k of 16 consecutive rows
// (16 i .. 16 i + 15) form one contiguous 1 KB piece, and the pieces of a
// row block follow each other in K order, so every 1 KB direct-to-LDS load
// of a 16-deep K stage reads one piece, 8 whole 128-byte lines, and the K
// groups of a K-major stage (16 rows, many columns) are consecutive pieces.
// A 16-row block takes the bytes of 16 rows, so whole row blocks sit where
// they would in a row-major buffer.  The stage-5 result of the map is not an
// operand: it is a plain row-major FP32 matrix.
// tiled_index: the FP32 element index of (row, col) in a tiled operand of
// ld columns.  plane_hi: the BF16 index of the hi half of an element at FP32
// index idx (its lo half is 16 further).
__host__ __device__ inline int64_t tiled_index(int64_t row, int64_t col, int64_t ld) {
  return ((((row >> 4) * (ld >> 4)) + (col >> 4)) << 8) + ((row & 15) << 4) + (col & 15);
}
__device__ __forceinline__ int64_t plane_hi(int64_t idx) { return 2 * (idx & ~int64_t{15}) + (idx & 15); }

__device__ __forceinline__ uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ __forceinline__ uint16_t bf16_lo_bits(float v) {
  return bf16_bits(v - static_cast<float>(static_cast<__bf16>(v)));
}

// Operand-form stores at the FP32 element index idx (tiled_index of the
// element; the elements of one store lie in one 16-element group).
__device__ __forceinline__ void put_operand(float *base, int64_t idx, float v, bool planes) {
  if (planes) {
    uint16_t *h = reinterpret_cast<uint16_t *>(base) + plane_hi(idx);
    h[0] = bf16_bits(v);
    h[16] = bf16_lo_bits(v);
  } else {
    base[idx] = v;
  }
}

// Four consecutive elements starting at idx (idx % 4 == 0).
__device__ __forceinline__ void put_operand4(float *base, int64_t idx, const float (&v)[4], bool planes) {
  if (planes) {
    uint16_t *h = reinterpret_cast<uint16_t *>(base) + plane_hi(idx);
    *reinterpret_cast<uint2 *>(h) = make_uint2(bf16_bits(v[0]) | (uint32_t(bf16_bits(v[1])) << 16),
                                               bf16_bits(v[2]) | (uint32_t(bf16_bits(v[3])) << 16));
    *reinterpret_cast<uint2 *>(h + 16) = make_uint2(bf16_lo_bits(v[0]) | (uint32_t(bf16_lo_bits(v[1])) << 16),
                                                    bf16_lo_bits(v[2]) | (uint32_t(bf16_lo_bits(v[3])) << 16));
  } else {
    *reinterpret_cast<float4 *>(base + idx) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// The global address space: stores through such a pointer are global
// (not FLAT) instructions.
#define SMX_GLOBAL __attribute__((address_space(1)))

// Operand-form store of four consecutive elements per lane, lanes in pairs
// (lane ^ 1 holds the next four): in BF16 planes the even lane writes the
// pair's 8 hi values and the odd lane their 8 lo values, 16 bytes each, so
// that the 4 lanes of a 16-element group fill its 64 bytes in one store
// instruction (as FP32 does); each lane writes alone where its partner's
// columns lie outside the row.  idx = the lane's first element (idx % 4 == 0).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void put_operand4_paired(SMX_GLOBAL float *base, int64_t idx, const float (&v)[4],
                                                    bool planes, bool pair) {
  if (!planes) {
    *reinterpret_cast<SMX_GLOBAL f32x4v *>(base + idx) = f32x4v{v[0], v[1], v[2], v[3]};
    return;
  }
  const uint32_t h0 = bf16_bits(v[0]) | (uint32_t(bf16_bits(v[1])) << 16);
  const uint32_t h1 = bf16_bits(v[2]) | (uint32_t(bf16_bits(v[3])) << 16);
  const uint32_t l0 = bf16_lo_bits(v[0]) | (uint32_t(bf16_lo_bits(v[1])) << 16);
  const uint32_t l1 = bf16_lo_bits(v[2]) | (uint32_t(bf16_lo_bits(v[3])) << 16);
  const bool odd = (threadIdx.x & 1) != 0;
  // the partner's hi (to an even lane) or lo (to an odd lane)
  const uint32_t x0 = dpp_mov<0xB1>(odd ? h0 : l0), x1 = dpp_mov<0xB1>(odd ? h1 : l1);
  SMX_GLOBAL uint16_t *h = reinterpret_cast<SMX_GLOBAL uint16_t *>(base) + plane_hi(idx);
  if (pair) {
    if (odd)  // lo of the pair: the even lane's four, then this lane's
      *reinterpret_cast<SMX_GLOBAL u32x4v *>(h + 16 - 4) = u32x4v{x0, x1, l0, l1};
    else
      *reinterpret_cast<SMX_GLOBAL u32x4v *>(h) = u32x4v{h0, h1, x0, x1};
  } else {
    *reinterpret_cast<SMX_GLOBAL u32x2v *>(h) = u32x2v{h0, h1};
    *reinterpret_cast<SMX_GLOBAL u32x2v *>(h + 16) = u32x2v{l0, l1};
  }
}

// Eight consecutive elements starting at idx (idx % 8 == 0): one 16-byte
// store per BF16 half, or two for FP32.
__device__ __forceinline__ void put_operand8(float *base, int64_t idx, const float (&v)[8], bool planes) {
  if (planes) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hw[e] = bf16_bits(v[2 * e]) | (static_cast<uint32_t>(bf16_bits(v[2 * e + 1])) << 16);
      lw[e] = bf16_lo_bits(v[2 * e]) | (static_cast<uint32_t>(bf16_lo_bits(v[2 * e + 1])) << 16);
    }
    uint16_t *h = reinterpret_cast<uint16_t *>(base) + plane_hi(idx);
    *reinterpret_cast<uint4 *>(h) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *reinterpret_cast<uint4 *>(h + 16) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  } else {
    *reinterpret_cast<float4 *>(base + idx) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4 *>(base + idx + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Host-side planning of a set of matrices into classes.
struct S8Plan {
  S8Layout layout;
  size_t bytes = 0;
};

// Compute the class layout for oriented shapes; `flips[i]` marks matrices
// whose parameter layout is the transpose of the oriented shape.  Fills
// class/slot of each matrix.  Returns false if more than kMaxClasses shapes.
bool plan_s8(const int64_t *r, const int64_t *c, const bool *flips, int32_t n, int mode,
             char *base, S8Plan &plan, int32_t *cls_of, int32_t *slot_of);

// Run the five S8 stages on a planned layout whose x0 and input norms
// (cst()[kCstFro]) are filled.  The result of each matrix is in S8Mat::result().
int run_s8_stages(const S8Layout &layout, hipStream_t st);

}  // namespace smx
