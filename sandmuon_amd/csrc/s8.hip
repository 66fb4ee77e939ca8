// S8 polar map on gfx950 MFMA: sandmuon/optimizer.py:69-93 with the
// constants of sandmuon/coefficients.py:3-11.
//
// Per matrix (oriented r <= c, unnormalised whitened input V in x0 and
// its squared Frobenius norm as partials in `fro`) and stage k = 1..5:
//   GRAM    G  = X X^T                 (stage 1: times 1/||V||^2)
//   SQUARE  stage 1: G2 = G G  -> p buffer, plus Schatten-8 partials
//           stage k: P  = c (G G + (b/c) G) + a I             -> p buffer
//   POLY1   stage 1 only: P1 = a I + b G/s^2 + c G2/s^4 -> p buffer,
//           s = max(1.35 ||G2||_F^(1/4), 1e-30) (elementwise kernel)
//   APPLY   stage 1: X' = P1 V / (||V|| s);  stage k: X' = P X
// A Gram-space class (cp > rp, see s8.h) replaces most per-stage Grams and
// applies by products of r x r matrices, in two segments:
//   stage 1: GRAM (X0), SQUARE, POLY1 (P1 -> qa = Q1), SYM T = P1 G,
//            SYM G = T P1 / s^2
//   stage 2: SQUARE (P2), APPLY Q2 = P2 Q1 (-> qb), APPLY X2 = Q2 X0 /
//            (||V|| s) (-> x1)
//   stage 3: GRAM (X2), SQUARE (P3 -> qa = Q3), SYM T = P3 G, SYM G = T P3
//   stage 4: SQUARE (P4), SYM T = P4 G, SYM G = T P4, APPLY Q4 = P4 Q3 (-> qb)
//   stage 5: SQUARE (P5), APPLY Q5 = P5 Q4 (-> qa), APPLY X5 = Q5 X2 (-> x0,
//            or xf for a transposed parameter)
// T = P G and T P are symmetric (P is a polynomial in G, computed from the
// same G) and are computed as C = A B^T on upper-triangle tiles like the
// Gram.  Q' = P Q is not mirrored: Q spans a wide range of eigenvalues (1
// to ~1300), and the rounding of P makes P and Q commute only to that
// range's precision, so Q' is the full product with Q as the K-major
// operand of an apply tile (a mirrored Q' costs ~6x in accuracy).
// The Gram (C = X X^T) and the square (C = G G, G symmetric) read both
// operands as K-contiguous rows.  The apply (C = P X) reads P the same way
// and X itself as a K-major operand: its LDS tile holds 16 rows of X and
// the MFMA fragments are gathered with the 16-bit transposed LDS read
// (ds_read_b64_tr_b16), so the iterate is only ever stored in one layout.
// Every operand is tiled (s8.h: 1 KB pieces of 16 rows x one 64-byte K
// group), so each 1 KB direct-to-LDS load of either kind reads one piece:
// 8 whole 128-byte lines, where the rows' 64-byte runs of a row-major layout
// touched 16 lines (cfg4 S8 10% faster).
// Gram and square only compute upper-triangle tiles and store each
// off-diagonal tile twice (tile and mirror).  The (b/c) G term of the square
// is accumulated by extra MFMAs from the B fragments (one_hot), so no
// epilogue reads G.
//
// Arithmetic modes:
//   SMX_S8_FP32       v_mfma_f32_32x32x2_f32 on FP32 operands.
//   SMX_S8_COMP_BF16  every operand is stored by its producer as BF16 hi +
//                     lo (put_operand); acc += hi*lo + lo*hi + hi*hi with
//                     v_mfma_f32_32x32x16_bf16 (the compensated product of
//                     reproduction/odl/ops/bf16_compensated_mm_fast.py:
//                     60-66, applied in all five stages with FP32
//                     accumulation of every intermediate).  Stages whose
//                     bit is clear in smx_s8_comp_mask (default 0x1f: none)
//                     run as kS8HiOnly: the same stored operands, acc +=
//                     hi*hi.
//   SMX_S8_MIXED      stages 1 and 2 as SMX_S8_COMP_BF16 (kernels of
//                     mode kS8CompMix); stages 3-5 of an X-space class as
//                     kS8F16: operands stored as FP16 (2 bytes per element)
//                     and v_mfma_f32_32x32x16_f16 with FP32 accumulation.
//                     Stage 1 maps the raw input, whose range only BF16's
//                     exponent holds; from stage 2 on every operand is
//                     normalised (|X| <= 1, G and P bounded, far below the
//                     FP16 maximum), where FP16's 11-bit significand rounds
//                     8x finer than a plain BF16 product, at a third of the
//                     compensated MFMAs and half the operand bytes.  Stage
//                     2 stays compensated: FP16 rounding there is what the
//                     later stages amplify most.  A Gram-space class stays
//                     compensated in every stage: its stages 3-5 carry the
//                     Gram G = X X^T, whose spectrum is the square of the
//                     iterate's, and an FP16 G loses the small eigenvalues
//                     (1.1e-2 from the FP32 map on matrices whose singular
//                     values decay as i^-1.5, against 3.4e-3 for the same
//                     stages on an X-space class).
//
// Operand forms (what a producer writes, chosen by the mode of the product
// that reads it, out_form): FP32, interleaved BF16 hi/lo ("planes"; the
// byte size of FP32), or FP16.  An FP16 operand has 2 ld bytes per row;
// in units of 4 bytes (the unit of the load offsets) it is an operand of
// ld / 2 columns whose 32-deep K stages move the 64 bytes per row that a
// 16-deep stage of the 4-byte forms moves (its pieces: 16 rows x 32 K), so
// the row-major loads, the LDS ring and the fragment reads are those of the
// planes form (chunk h: K 8h .. 8h+7 of the first 16, chunk 2 + h: of the
// second 16).
//
// Block: 256x128 output tile, 4 waves (2 x 2, one per SIMD), each wave
// 128x64 (4 x 2 MFMA 32x32 tiles, 128 accumulator registers), and two
// blocks per CU, so one block's epilogue and prologue overlap the other's
// MFMAs.  Operands stream into a 3-stage LDS ring (K = 16 per stage, 24 KB)
// with direct-to-LDS 16-byte loads issued two stages ahead.  The epilogue
// stages each 32x32 accumulator block through LDS and writes row vectors
// (the transposed orientation too for Gram/square mirror tiles and for the
// stage-5 result of a transposed parameter).
#include "s8.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

namespace smx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Phase { kGram = 0, kSquare = 1, kApply = 2, kPoly1 = 3, kSpan = 4, kSym = 5 };  // kSpan: timing record of a whole S8 run
// SYM products of a Gram-space class (per segment of a SYM launch).
// The product of a segment of a SYM or APPLY launch: PG / TP of a
// Gram-space class (SYM); X' = P X of an X-space class, Q' = P Q and the
// final X5 = Q X0 of a Gram-space class (APPLY).
enum SegOp { kOpPG = 0, kOpTP = 1, kOpApplyX = 2, kOpApplyQ = 3, kOpApplyMid = 4, kOpApplyFinal = 5 };

// The Gram-space schedule (see the header): Gram at stages 1 and 3, SYM
// products at stages 1, 3 and 4, Q' = P Q at stages 2, 4 and 5, X2 = Q2 X0
// after stage 2, X5 = Q5 X2 after stage 5.  A segment's first stage (1, 3)
// keeps its P in qa: it is the segment's first Q.
__host__ __device__ constexpr bool gs_gram(int stage) { return stage == 1 || stage == 3; }
__host__ __device__ constexpr bool gs_sym(int stage) { return stage == 1 || stage == 3 || stage == 4; }
__host__ __device__ constexpr bool gs_apply_q(int stage) { return stage == 2 || stage == 4 || stage == 5; }
constexpr int kMaxSeg = 2 * kMaxClasses;

// Internal MFMA modes of one GEMM launch (the public modes are SMX_S8_FP32,
// SMX_S8_COMP_BF16 and the recipe SMX_S8_MIXED):
//   kS8HiOnly  a plain BF16 stage of the compensated recipe: the operands in
//              their stored hi/lo form, only the hi*hi product issued;
//   kS8F16     FP16 operands, two 32x32x16 FP16 MFMAs per 32-deep K stage;
//   kS8CompMix the compensated products of SMX_S8_MIXED: the K loop of
//              SMX_S8_COMP_BF16, whose kernels alone also compile an FP16
//              epilogue (kept out of the compensated recipe's kernels, whose
//              code would otherwise outgrow the instruction cache).
constexpr int kS8HiOnly = 3;
constexpr int kS8F16 = 4;
constexpr int kS8CompMix = 5;
__host__ __device__ constexpr bool is_comp(int m) { return m == SMX_S8_COMP_BF16 || m == kS8CompMix; }
// Bit k-1 set: stage k of SMX_S8_COMP_BF16 is compensated.
static int g_comp_mask = 0x1f;

// Operand forms.
enum Form { kFormF32 = 0, kFormPlanes = 1, kFormF16 = 2, kFormAny = 3 };  // kFormAny: an epilogue's run-time choice
__host__ __device__ constexpr int form_of(int gemm_mode) {
  return gemm_mode == SMX_S8_FP32 ? kFormF32 : gemm_mode == kS8F16 ? kFormF16 : kFormPlanes;
}

// The MFMA mode of one product of the map (phase, stage and, for SYM and
// APPLY, its SegOp) under the run's public `mode` and compensation mask.
__host__ __device__ constexpr int gemm_mode(int mode, int mask, int phase, int stage, int op, bool gs) {
  return mode == SMX_S8_FP32 ? SMX_S8_FP32
         : mode == SMX_S8_COMP_BF16 ? (((mask >> (stage - 1)) & 1) ? SMX_S8_COMP_BF16 : kS8HiOnly)
         : (stage <= 2 || gs) ? kS8CompMix
                              : kS8F16;
}

// The output forms a GEMM kernel of MFMA mode `gm` and phase `phase`
// compiles (each kernel keeps only these epilogues): a Gram feeds its
// stage's square (same mode); a square writes FP32 G2 at stage 1, else P
// for its stage's products; the SYM products feed products of their own
// mode; an apply feeds the next stage (in SMX_S8_MIXED the compensated
// stage-2 apply of an X-space class writes the FP16 iterate of stage 3),
// Q2 / X2, or the FP32 result.
__host__ __device__ constexpr bool form_compiled(int gm, int phase, int form) {
  return gm == SMX_S8_FP32 ? form == kFormF32
         : gm == kS8F16 ? (form == kFormF16 || (form == kFormF32 && phase == kApply))
         : form == kFormPlanes || (form == kFormF32 && (phase == kSquare || phase == kApply)) ||
               (form == kFormF16 && gm == kS8CompMix && phase == kApply);
}

// The form a product's output is stored in: that of the product that reads
// it (the Gram feeds its stage's square; the square feeds its stage's apply
// or Q' = P Q, and at stages 3 and 4 the SYM products of the same mode; PG
// feeds TP, TP the next stage's square; an iterate feeds the next stage's
// Gram and apply; Q2 feeds X2, Q4 and Q5 the next Q' and X5; X2 the
// stage-3 Gram and X5).  The stage-1 square's G2 and the stage-5 result
// are FP32.
__host__ __device__ constexpr int out_form(int mode, int mask, int phase, int stage, int op, bool gs) {
  return phase == kGram ? form_of(gemm_mode(mode, mask, kSquare, stage, -1, gs))
         : phase == kSquare ? (stage == 1 ? kFormF32
                                          : form_of(gemm_mode(mode, mask, kApply, stage, gs ? kOpApplyQ : kOpApplyX, gs)))
         : phase == kPoly1 ? form_of(gemm_mode(mode, mask, kApply, 1, kOpApplyX, gs))
         : phase == kSym ? (op == kOpPG ? form_of(gemm_mode(mode, mask, kSym, stage, kOpTP, gs))
                                        : form_of(gemm_mode(mode, mask, kSquare, stage + 1, -1, gs)))
         : op == kOpApplyX ? (stage == 5 ? kFormF32 : form_of(gemm_mode(mode, mask, kGram, stage + 1, -1, gs)))
         : op == kOpApplyQ ? form_of(gemm_mode(mode, mask, kApply, stage == 2 ? 2 : 5,
                                               stage == 2 ? kOpApplyMid : stage == 4 ? kOpApplyQ : kOpApplyFinal, gs))
         : op == kOpApplyMid ? form_of(gemm_mode(mode, mask, kGram, 3, -1, gs))
                             : kFormF32;
}
// Tile geometry policy (smx_s8_tile_geometry): 0 automatic (pick_geo),
// 1 256 x 256 tiles for every GEMM launch, 2 never 256 x 256.
static int g_tile_policy = 0;

constexpr int kSubN = 2;            // 32x32 MFMA column tiles per wave (64 columns)
constexpr int kBK = 16;             // K per pipeline stage

// Block tile geometries.  Each wave computes 32 kSubM x 64 outputs
// (kSubM x kSubN MFMA 32x32 tiles); the waves of a block are 2 x kWavesN.
//   kGeoM  256 x 128, 4 waves of 128 x 64, two blocks per CU;
//   kGeoS  128 x 128, 4 waves of 64 x 64, three blocks per CU;
//   kGeoL  256 x 256, 8 waves of 128 x 64 (two per SIMD), one block per CU.
// The wave tile, and so the LDS fragment reads per MFMA, is the same in M
// and L; an L block moves a third fewer operand bytes into LDS per MFMA
// (its 256 A rows serve 256 B rows: cfg5 S8 7% faster).  A round of the
// device's block slots does the same work in M and L; the host picks the
// geometry per launch (pick_geo).
enum TileGeo { kGeoM = 0, kGeoS = 1, kGeoL = 2 };
template <int TM, int TN>
struct Geo {
  static constexpr int kTileM = TM, kTileN = TN;
  static constexpr int kSubM = TM / 64;             // 32x32 MFMA row tiles per wave
  static constexpr int kWavesN = TN / (32 * kSubN);
  static constexpr int kWaves = 2 * kWavesN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kOpA = TM * kBK * 4;       // A operand tile TM x 16 (4 bytes per element)
  static constexpr int kOpB = TN * kBK * 4;       // B operand tile TN x 16
  static constexpr int kStageBytes = kOpA + kOpB;
  // LDS ring depth (kStages - 1 stages in flight): 3 where two or three
  // blocks share a CU's LDS, 4 for the one 256 x 256 block per CU.
  static constexpr int kStages = TN == 256 ? 4 : 3;
  static constexpr int kRingBytes = kStages * kStageBytes;
  static constexpr int kLoadsA = kOpA / 1024 / kWaves;  // 1 KB loads per wave
  static constexpr int kLoadsB = kOpB / 1024 / kWaves;
  static constexpr int kLoadsPerStage = kLoadsA + kLoadsB;
  static constexpr int kKmRow = TN * 4;           // bytes of a K row of the K-major B tile
  static constexpr int kKmRowH = TN * 2;          // the same for FP16 operands (32 K rows per stage)
  static constexpr int kWavesPerEU = TM == 128 ? 3 : 2;
  static constexpr int kGeo = TN == 256 ? kGeoL : TM == 128 ? kGeoS : kGeoM;
};
using GeoM = Geo<256, 128>;
using GeoS = Geo<128, 128>;
using GeoL = Geo<256, 256>;
// (kGeoS: the Gram, the square, the SYM products and the applies at cfg4,
// and generally a launch whose small tiles take fewer rounds of the CUs'
// block slots, allowing for their lower rate: the smaller tile moves a
// third more operand bytes per MFMA, and a round of it takes 0.9 of a round
// of the larger one.  At 768 x 768 the square's 12
// half-tiles per matrix need two rounds of 512 slots, its 21 small tiles
// 1.5 rounds of 768 (cfg4: 104 against 117 us per launch); at 2048 x 2048
// the larger tile wins.)

struct StageArgs {
  S8Layout L;
  int32_t seg_off[kMaxSeg + 1];  // block offsets (multiples of 8)
  int32_t seg_cls[kMaxSeg];
  int32_t seg_op[kMaxSeg];       // SYM / APPLY launches: the product of the segment (SegOp)
  int32_t seg_slot0[kMaxSeg];    // the segment's matrices: slots slot0 .. slot0 + cnt - 1 of its class
  int32_t seg_cnt[kMaxSeg];
  int32_t n_seg;
  int32_t stage;  // 1..5
  int32_t sq_geo;    // TileGeo of this run's square (the stage-1 Schatten partials are per square tile)
  int32_t mask;      // compensated stages of SMX_S8_COMP_BF16 (bit k-1: stage k)
  float a, b, c;
  float b_over_c;
};

// A K-contiguous GEMM operand with rows of `ld` elements: FP32, or BF16
// hi/lo interleaved per 16-element K group (put_operand).
struct Opnd {
  const void *p;
  int64_t ld;
};

// ------------------------------------------------------- LDS layouts ---
// Operand tile [256 rows][16 K]: four 16-byte chunks per row (FP32: k 0-3,
// 4-7, 8-11, 12-15; interleaved BF16: hi k 0-7, hi k 8-15, lo k 0-7, lo k
// 8-15), logical chunk kc at slot kc ^ swz4(r).  Fragment reads (one chunk
// of 32 consecutive rows per lane half) are conflict-free for 32- and
// 64-bank LDS.
__device__ __forceinline__ int swz4(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }
__device__ __forceinline__ int f32_off(int r, int kc) { return (r * 4 + (kc ^ swz4(r))) << 4; }

// Bits 2 and 3 of a row (or column) index within a 32-row fragment block,
// swapped.  The B fragments are read with this permutation of their 32 rows,
// so that in the accumulator of C^T = B A^T (the operands of every MFMA
// are passed B first) register 4 k + q of lane (r, h) holds column
// 16 (k >> 1) + 8 h + 4 (k & 1) + q of row r: each lane holds 8
// consecutive columns of each 16-column K group of its row, which the
// epilogue stores directly as row vectors.
__device__ __forceinline__ int sw23(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }
// FP32 mode keeps the natural order: its outputs are FP32, whose 16-byte
// quads of columns 8 k + 4 h .. + 3 already give the two lanes of a row 32
// contiguous bytes per store.
template <int MODE>
__device__ __forceinline__ int frag_row(int p) { return MODE == SMX_S8_FP32 ? p : sw23(p); }

// One 16-byte direct-to-LDS load per lane from sbase + voff (scalar base,
// per-lane 32-bit byte offset): lane l writes LDS[m0 + 16 l].  Issued from
// asm so the compiler does not treat later LDS reads as aliasing the
// in-flight load (it would wait for every outstanding load); the ring's
// waits are explicit (wait_vm).  M0 is an input operand; the s_nop is the
// wait state an LDS DMA needs after a scalar write of M0, which the
// compiler cannot see through the asm.
__device__ __forceinline__ void dma16(uint32_t voff, const void *sbase, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

// Per-lane byte offsets of this wave's N loads of one operand tile; a
// stage at K offset k0 only moves the scalar base.
template <int N>
struct TileOffsets {
  uint32_t v[N];
};

// Row-major operand tile (rows row0.. of a tiled operand with ld columns,
// one 16-deep K stage): load q = wave*N + i reads the stage's 1 KB piece of
// rows row0 + 16 q .. + 15, lane l filling LDS slot l & 3 of tile row
// 16 q + (l >> 2) with logical chunk (l & 3) ^ swz4(row) of that row
// (swz4 only sees bits 1-3 of the row).  The scalar base of a stage at K
// offset k0 (4-byte units) moves by 64 k0 bytes: k0 / 16 pieces.
template <int N>
__device__ __forceinline__ TileOffsets<N> tile_offsets(int64_t ld, int64_t row0, int wave) {
  const int lane = threadIdx.x & 63, m = lane >> 2;
  const uint32_t in_piece = static_cast<uint32_t>(m * 64 + (((lane & 3) ^ swz4(m)) << 4));
  TileOffsets<N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int64_t blk = (row0 >> 4) + wave * N + i;  // 16-row block
    t.v[i] = static_cast<uint32_t>(blk * (ld >> 4) * 1024) + in_piece;
  }
  return t;
}

// K-major tile (the apply's B: the stage's K rows, columns n0 .. n0 + TN - 1
// of a tiled operand with ld columns; KMROW = 4 TN bytes, 2 TN for FP16):
// TN / 16 pieces, [piece][16 rows][64 bytes] in LDS.  Load q = wave*N + i
// reads piece q: K group n0 / 16 + q of the stage's 16-row block (FP16, 32
// K rows and 32 columns per group: pieces q < TN / 32 from the first row
// block, the others from the second), lane l filling slot l & 3 of the
// piece's row l >> 2 with logical chunk (l & 3) ^ swzt.  The scalar base of
// a stage at K offset k0 moves by 4 k0 ld bytes (whole row blocks).
// swzt: 2 ((row >> 1 ^ piece) & 1) (FP16: 2 ((row >> 1) & 1); FP32, whose
// 4-byte reads are not on the MFMA-bound path's critical side, none, which
// leaves its fragment addresses one register and constants).  A transposed
// read of 16 lanes takes two chunks of each of 4 consecutive rows of one
// piece: rows 4t and 4t + 2 share their bank positions modulo 128 bytes, and
// the swizzle puts their chunks on different halves of the row (32 banks
// serving 16 lanes); 32 lanes read the same rows of two adjacent pieces
// (FP16: the other two chunks of the same piece), which the piece term puts
// on different halves too (64 banks serving 32 lanes).
__device__ __forceinline__ int swzt(int row, int piece) { return 2 * (((row >> 1) ^ piece) & 1); }
__device__ __forceinline__ int swzt_h(int row) { return 2 * ((row >> 1) & 1); }

// (F16: an FP16 operand; ld and n0 are in 4-byte units, i.e. half the
// element counts, and a stage holds 32 K rows.)
enum KmSwz { kKmSwzNone = 0, kKmSwzT = 1, kKmSwzH = 2 };
template <int N, int KMROW, int SWZ>
__device__ __forceinline__ TileOffsets<N> tile_offsets_km(int64_t ld, int64_t n0, int wave) {
  constexpr bool F16 = SWZ == kKmSwzH;
  constexpr int kBlockPieces = KMROW / 64;  // pieces per 16-row block: TN / 16, FP16 TN / 32
  const int lane = threadIdx.x & 63, m = lane >> 2;
  TileOffsets<N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int q = wave * N + i;
    const int hb = F16 ? q / kBlockPieces : 0, jj = F16 ? q % kBlockPieces : q;
    const int sw = SWZ == kKmSwzH ? swzt_h(m) : SWZ == kKmSwzT ? swzt(m, q) : 0;
    t.v[i] = static_cast<uint32_t>((hb * (ld >> 4) + (n0 >> 4) + jj) * 1024 + m * 64 + (((lane & 3) ^ sw) << 4));
  }
  return t;
}

// f(std::integral_constant<int, 0>{}) .. f(std::integral_constant<int, N - 1>{}),
// expanded at compile time.
template <class F, int... I>
__device__ __forceinline__ void static_for_seq(F &f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// A wave-uniform pointer in scalar registers: the direct-to-LDS loads take
// their base from an SGPR pair, and in some kernels the compiler does not
// prove a base built from the kernel arguments uniform (it is: every
// pointer of a tile derives from the block index and kernel arguments).
// Applied once per tile to the operand bases.
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int N>
__device__ __forceinline__ void dma_tile(const TileOffsets<N> &t, const char *sbase, uint32_t lds) {
#pragma unroll
  for (int i = 0; i < N; ++i) dma16(t.v[i], sbase, lds + i * 1024);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else static_assert(N == 0, "unsupported vmcnt");
}

__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// The 8 consecutive K values (k = 8h .. 8h+7 of the stage) of row r (FP32).
__device__ __forceinline__ void read8(const char *tile, int r, int h, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(tile + f32_off(r, 2 * h));
  const f32x4 b = *reinterpret_cast<const f32x4 *>(tile + f32_off(r, 2 * h + 1));
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Chunk kc of row r as 8 BF16 values.
__device__ __forceinline__ bf16x8 read_b16(const char *tile, int r, int kc) {
  return *reinterpret_cast<const bf16x8 *>(tile + f32_off(r, kc));
}

// ------------------------------------------- K-major operand tile (apply) ---
// [piece][16 K rows][64 bytes] (tile_offsets_km): piece j holds the
// columns 16 j .. 16 j + 15 of the tile (FP16: 32 j .. 32 j + 31 of 16 K
// rows, the stage's second 16 rows after the first), a 64-byte row of it in
// 16-byte chunks, logical chunk c at slot c ^ swzt.  Logical chunks follow
// the global bytes: interleaved BF16 2 plane + half (plane 0 hi / 1 lo,
// columns 8 half .. 8 half + 7 of the piece); FP32 and FP16 in column order.

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) char lds_char;

// An LDS pointer of a generic pointer into __shared__ memory; arithmetic on
// it lets constant offsets fold into the LDS instructions' offset field.
__device__ __forceinline__ lds_char *to_lds(const char *p) { return (lds_char *)(const_cast<char *>(p)); }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane 4a + b receives
// element b of the 4-element (8-byte) reads addressed by lanes a, a + 4,
// a + 8 and a + 12, in that order.
__device__ __forceinline__ i16x4 read_tr16(lds_char *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)p);
}

// ----------------------------------------------------------- compute ---
// Register fragments of one K stage for this wave's 128 x 128 sub-tile:
// BF16 hi/lo pairs (compensated mode, 16 K), FP16 values of K 0-15 and
// 16-31 (kS8F16, 32 K) or FP32 (FP32 mode, 16 K).  The
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
template <>
struct AFrag<kS8HiOnly> : AFrag<SMX_S8_COMP_BF16> {};
template <>
struct AFrag<kS8F16> : AFrag<SMX_S8_COMP_BF16> {};  // h: K 0-15, l: K 16-31 (FP16 bits)
template <>
struct AFrag<kS8CompMix> : AFrag<SMX_S8_COMP_BF16> {};
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
template <>
struct BFrags<kS8HiOnly> : BFrags<SMX_S8_COMP_BF16> {};
template <>
struct BFrags<kS8F16> : BFrags<SMX_S8_COMP_BF16> {};
template <>
struct BFrags<kS8CompMix> : BFrags<SMX_S8_COMP_BF16> {};

// Both 16-byte chunks of a row's K slice are read (the lo plane, or FP16's
// second 16 K).
template <int MODE>
constexpr bool two_chunks() { return is_comp(MODE) || MODE == kS8F16; }

// LDS -> registers: A row block i, and the four B column blocks, of one
// stage.  Lane (r, h) takes K = 8h .. 8h+7 of its row: chunks h (hi) and
// 2 + h (lo) of the interleaved form, chunks 2h and 2h + 1 of FP32.
template <int MODE, class G>
__device__ __forceinline__ void load_a(const char *st, int wm, int i, AFrag<MODE> &f) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const int r = wm * (32 * G::kSubM) + i * 32 + lr;
  if constexpr (MODE != SMX_S8_FP32) {
    f.h = read_b16(st, r, lh);
    if constexpr (two_chunks<MODE>()) f.l = read_b16(st, r, 2 + lh);
  } else {
    read8(st, r, lh, f.v);
  }
}

template <int MODE, class G>
__device__ __forceinline__ void load_b(const char *st, int wn, BFrags<MODE> &f) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const char *bt = st + G::kOpA;
#pragma unroll
  for (int j = 0; j < kSubN; ++j) {
    const int r = wn * (32 * kSubN) + j * 32 + frag_row<MODE>(lr);
    if constexpr (MODE != SMX_S8_FP32) {
      f.h[j] = read_b16(bt, r, lh);
      if constexpr (two_chunks<MODE>()) f.l[j] = read_b16(bt, r, 2 + lh);
    } else {
      read8(bt, r, lh, f.v[j]);
    }
  }
}

// The four B column blocks of one stage from a K-major tile (apply).  Lane
// (n, h) needs B[k = 8h .. 8h+7][sw23(n)] (the permuted fragment rows of
// sw23).  Interleaved BF16: per plane, two transposed reads of 4 K rows
// each; lane s of a 16-lane group g addresses row 8 (g >> 1) + 4 r +
// (s >> 2), columns 16 (g & 1) + 4 c .. + 3 of the 32-column block with
// c = sw23(4 (s & 3)) / 4 (the two bits of s & 3 swapped), so lane
// 16 (g & 1) + 4 a + b of the block receives column 16 (g & 1) + 4 c(a) + b
// = sw23 of its index at the 4 rows.  Column block j of wave wn is pieces
// 4 wn + 2 j and 4 wn + 2 j + 1 (g & 1 picks one), logical chunk 2 plane +
// (c >> 1) = 2 plane + (s & 1), byte 8 (c & 1) = 8 ((s >> 1) & 1) of it.
// The swizzle of rows k and k + 4 is the same, and its piece term is g & 1,
// so the per-lane offsets (wn included) are one per plane (o[plane][0]) and
// every read adds a constant.  FP16: lane s of group g addresses row
// 8 (g >> 1) + (s >> 2) (+4 for the second read, + the second row block's
// pieces for the second 16 K), columns 16 (g & 1) + 4 c .. + 3 of piece
// 2 wn + j (32 columns), i.e. chunk 2 (g & 1) + (s & 1), byte
// 8 ((s >> 1) & 1); o[j][0] holds the offset of block j.  FP32: eight
// 4-byte reads.  (The 16 lanes of a read address the same bytes as with
// unpermuted columns, in another lane order: the same banks.)
struct BkmLane {
  uint32_t o[2][2];
};
__device__ __forceinline__ BkmLane bkm_lane(int wn) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 15;
  const int k = 8 * (g >> 1) + (s >> 2);
  const int sw = swzt(k, g & 1);  // the same for rows k and k + 4
  BkmLane L;
#pragma unroll
  for (int pl = 0; pl < 2; ++pl) {
    L.o[pl][0] = static_cast<uint32_t>((4 * wn + (g & 1)) * 1024 + k * 64 + 8 * ((s >> 1) & 1) +
                                       (((2 * pl + (s & 1)) ^ sw) << 4));
    L.o[pl][1] = 0;
  }
  return L;
}

__device__ __forceinline__ BkmLane bkm_lane_f16(int wn) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 15;
  const int k = 8 * (g >> 1) + (s >> 2);
  const int sw = swzt_h(k);  // the same for rows k + 4 and the second row block
  BkmLane L;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    L.o[j][0] = static_cast<uint32_t>((2 * wn + j) * 1024 + k * 64 + 8 * ((s >> 1) & 1) +
                                      (((2 * (g & 1) + (s & 1)) ^ sw) << 4));
    L.o[j][1] = 0;
  }
  return L;
}

template <int MODE, class G>
__device__ __forceinline__ void load_b_km(const char *st, int wn, BFrags<MODE> &f, const BkmLane &L) {
  constexpr int kOpA = G::kOpA;
  const int lane = threadIdx.x & 63;
  const char *bt = st + kOpA;
  if constexpr (MODE == kS8F16) {
    static_assert(kSubN == 2, "one lane offset per 32-column block");
    constexpr int kBlockBytes = G::kKmRowH / 64 * 1024;  // the pieces of one 16-row block
#pragma unroll
    for (int j = 0; j < kSubN; ++j) {
      lds_char *q = to_lds(st) + L.o[j][0];
      asm volatile("" : "+v"(q));
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        lds_char *p = q + (kOpA + half * kBlockBytes);
        const i16x4 lo = read_tr16(p), hi = read_tr16(p + 4 * 64);
        const bf16x8 v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        if (half == 0) f.h[j] = v;
        else f.l[j] = v;
      }
    }
  } else if constexpr (MODE != SMX_S8_FP32) {
    // Two base addresses per stage; the empty asm keeps the compiler from
    // pre-adding every read's constant offset into a register of its own
    // instead of using the instructions' offset field.
    lds_char *q[2];
#pragma unroll
    for (int pl = 0; pl < 2; ++pl) {
      q[pl] = to_lds(st) + L.o[pl][0];
      asm volatile("" : "+v"(q[pl]));
    }
#pragma unroll
    for (int j = 0; j < kSubN; ++j) {
#pragma unroll
      for (int pl = 0; pl < (is_comp(MODE) ? 2 : 1); ++pl) {
        lds_char *p = q[pl] + (kOpA + 2 * j * 1024);
        const i16x4 lo = read_tr16(p), hi = read_tr16(p + 4 * 64);
        const bf16x8 v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        if (pl == 0) f.h[j] = v;
        else f.l[j] = v;
      }
    }
  } else {
    // (FP32 mode, natural column order: frag_row.)  Lane (n, h), n =
    // 64 wn + 32 j + (lane & 31): piece 4 wn + 2 j + ((lane >> 4) & 1),
    // element 4 ((lane >> 2) & 3) + (lane & 3) of rows 8 h + q (no swizzle).
    const char *base = bt + (4 * wn + ((lane >> 4) & 1)) * 1024 + 512 * (lane >> 5) + 4 * (lane & 15);
#pragma unroll
    for (int j = 0; j < kSubN; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) f.v[j][q] = *reinterpret_cast<const float *>(base + 2048 * j + 64 * q);
  }
}

template <int MODE, class G, bool BKM>
__device__ __forceinline__ void load_b_any(const char *st, int wn, BFrags<MODE> &f, const BkmLane &L) {
  if constexpr (BKM) load_b_km<MODE, G>(st, wn, f, L);
  else load_b<MODE, G>(st, wn, f);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f16x8 as_f16(bf16x8 v) { return __builtin_bit_cast(f16x8, v); }

// MFMAs of row block i: acc[i][j] += A_i B_j^T over the stage's K.
template <int MODE>
__device__ __forceinline__ void mma_row(const AFrag<MODE> &a, const BFrags<MODE> &b, f32x16 (&acc)[kSubN]) {
  // (B first: the accumulator holds C^T = B A^T, lane r of it row r of C.)
  if constexpr (is_comp(MODE)) {
    // Corrections first, then hi*hi.
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.l[j], a.h, acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.h[j], a.l, acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.h[j], a.h, acc[j], 0, 0, 0);
  } else if constexpr (MODE == kS8HiOnly) {
#pragma unroll
    for (int j = 0; j < kSubN; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.h[j], a.h, acc[j], 0, 0, 0);
  } else if constexpr (MODE == kS8F16) {
    // K 0-15, then K 16-31 of the stage.
#pragma unroll
    for (int j = 0; j < kSubN; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.h[j]), as_f16(a.h), acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < kSubN; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.l[j]), as_f16(a.l), acc[j], 0, 0, 0);
  } else {
    // Lane half h supplies k = 8h + q to MFMA q (the same permutation for
    // both operands, so every k is paired exactly once).
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < kSubN; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b.v[j][q], a.v[q], acc[j], 0, 0, 0);
  }
}

// acc += s G over this wave's own output rows (square phase of stages 2-5,
// whose product is P = a I + b G + c G G = c (G G + (b/c) G) + a I).  The
// Gram is symmetric, so the B fragments of the stage whose K range covers
// rows R..R+15 of the wave hold G[R + k][col] in accumulator layout; an A
// fragment that is s on the diagonal k = row - R (a scaled one-hot row)
// adds s G to those accumulator rows with the ordinary (compensated) MFMAs.
template <int MODE>
__device__ __forceinline__ AFrag<MODE> one_hot(float s, int r0) {
  const int lane = threadIdx.x & 63;
  const int e = (lane & 31) - r0 - 8 * (lane >> 5);  // position of k = row - R in this lane's 8
  AFrag<MODE> f;
  if constexpr (MODE == kS8F16) {
    // s as the FP16 pair hi + lo (22 bits), hi in h, lo in l.
    const _Float16 sh = static_cast<_Float16>(s);
    const _Float16 sl = static_cast<_Float16>(s - static_cast<float>(sh));
    const _Float16 z = static_cast<_Float16>(0.f);
    f16x8 h, l;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      h[q] = q == e ? sh : z;
      l[q] = q == e ? sl : z;
    }
    f.h = __builtin_bit_cast(bf16x8, h);
    f.l = __builtin_bit_cast(bf16x8, l);
  } else if constexpr (MODE != SMX_S8_FP32) {
    const __bf16 sh = static_cast<__bf16>(s);
    const __bf16 sl = static_cast<__bf16>(s - static_cast<float>(sh));
    const __bf16 z = static_cast<__bf16>(0.f);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      f.h[q] = q == e ? sh : z;
      f.l[q] = q == e ? sl : z;
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) f.v[q] = q == e ? s : 0.f;
  }
  return f;
}

// acc[i] += s G over the rows of the one-hot window stage: the compensated
// recipe's three products of the (hi, lo) scalar and B planes; a plain BF16
// stage the scalar's hi and lo against B's hi plane (a BF16 scalar alone
// would misscale the linear term of P by up to 2^-9); FP16 the scalar's hi
// and lo against the stage's first 16 K (rows r0 = 0 .. 15 of the block)
// and its second 16 K (rows 16 .. 31); FP32 one product.
template <int MODE>
__device__ __forceinline__ void mma_one_hot(float s, int sel, const BFrags<MODE> &b, f32x16 (&acc)[kSubN]) {
  if constexpr (MODE == kS8F16) {
    const AFrag<MODE> o0 = one_hot<MODE>(s, 0), o1 = one_hot<MODE>(s, 16);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) {
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.h[j]), as_f16(o0.h), acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.h[j]), as_f16(o0.l), acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.l[j]), as_f16(o1.h), acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16(b.l[j]), as_f16(o1.l), acc[j], 0, 0, 0);
    }
  } else if constexpr (MODE == kS8HiOnly) {
    const AFrag<MODE> o = one_hot<MODE>(s, (sel & 1) * 16);
#pragma unroll
    for (int j = 0; j < kSubN; ++j) {
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.h[j], o.h, acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b.h[j], o.l, acc[j], 0, 0, 0);
    }
  } else {
    mma_row<MODE>(one_hot<MODE>(s, (sel & 1) * 16), b, acc);
  }
}

// Issues one stage (A and B tiles) into a ring slot.  `lds` is the slot's
// LDS byte address plus this wave's first A chunk (wave-uniform); the
// wave's B chunks start kOpA bytes later, less the difference of the
// wave's A and B shares.  BKM: B is K-major (its stage is 16 rows further
// down).
template <class G>
struct WaveOffsets {
  TileOffsets<G::kLoadsA> a;
  TileOffsets<G::kLoadsB> b;
  uint32_t b_lds;  // LDS byte offset of the wave's B chunks from its A chunks
};
// KMSTEP: K rows of a K-major stage per 4-byte unit of k0 (2 for FP16,
// whose 32-row stages advance k0 by 16).
template <class G, bool BKM, int KMSTEP>
__device__ __forceinline__ void issue_stage(const Opnd &A, const Opnd &B, const WaveOffsets<G> &o, int64_t k0,
                                            uint32_t lds) {
  dma_tile(o.a, static_cast<const char *>(A.p) + 64 * k0, lds);
  dma_tile(o.b, static_cast<const char *>(B.p) + (BKM ? 4 * k0 * B.ld * KMSTEP : 64 * k0), lds + o.b_lds);
}

// Waits until at most `pending` stages of this wave's loads are in flight
// (loads complete in issue order).
template <class G>
__device__ __forceinline__ void wait_stages(int pending) {
  constexpr int L = G::kLoadsPerStage;
  static_assert(G::kStages == 3 || G::kStages == 4, "at most three stages in flight");
  if constexpr (G::kStages == 4) {
    if (pending >= 3) {
      wait_vm<3 * L>();
      return;
    }
  }
  if (pending >= 2) wait_vm<2 * L>();
  else if (pending == 1) wait_vm<L>();
  else wait_vm<0>();
}

// lgkmcnt(0) (vmcnt and expcnt left at their maxima) as a builtin, so the
// compiler's own wait-count tracking sees the LDS reads complete; an asm
// wait would leave them pending in its model and it would then insert
// lgkmcnt waits before later MFMAs that stall on unrelated newer reads.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// C[TM x TN] = A[arow0.., :K] * B[brow0.., :K]^T (BKM: A[arow0.., :K] *
// B[:K, brow0..]), geometry G.
//
// Two pipelines overlap the MFMAs:
//  * a ring of G::kStages LDS slots filled by direct-to-LDS loads, kStages
//    stages ahead of the fragment reads;
//  * register fragments: while the MFMAs of stage kt run, the fragments of
//    stage kt+1 are read from LDS (B into the other buffer up front, each A
//    row block right after its last MFMA of stage kt).
// Iteration kt: wait for this wave's loads of stage kt+1 and for its own
// outstanding LDS reads (those of stage kt, so slot kt is free); a block
// barrier makes every wave's loads of kt+1 visible and every wave's reads
// of kt finished; refill slot kt with stage kt+kStages; MFMAs of stage kt
// interleaved with the reads of stage kt+1.
// SEL >= 0: this stage is stage SEL of the wave's one_hot window (rows
// 16 SEL .. 16 SEL + 15 of the wave, accumulator block SEL / 2; FP16: rows
// 32 SEL .. 32 SEL + 31, accumulator block SEL).
// STEADY: kt + kStages < nk, so a next stage exists, the refill is due and
// kStages - 2 stages may stay in flight (no run-time conditions).
template <int MODE, class G, int SEL, int PAR, bool STEADY, bool BKM>
__device__ __forceinline__ void pipe_iter(const Opnd &A, const Opnd &B, const WaveOffsets<G> &o, const BkmLane &bl,
                                          uint32_t lds0, float sel_s, char *smem, int kt, int nk, int wm, int wn,
                                          AFrag<MODE> (&af)[G::kSubM], BFrags<MODE> (&bf)[2],
                                          f32x16 (&acc)[G::kSubM][kSubN]) {
  constexpr int S = G::kStages;
  const bool more = STEADY || kt + 1 < nk;
  if constexpr (STEADY) {
    wait_vm<(S - 2) * G::kLoadsPerStage>();
  } else {
    if (more) wait_stages<G>(min(S - 2, nk - 2 - kt));
  }
  wait_lds();
  block_barrier();
  if (STEADY || kt + S < nk)
    issue_stage<G, BKM, MODE == kS8F16 ? 2 : 1>(A, B, o, static_cast<int64_t>(kt + S) * kBK,
                                                lds0 + (kt % S) * G::kStageBytes);
  const char *nxt = smem + ((kt + 1) % S) * G::kStageBytes;
  if (more) load_b_any<MODE, G, BKM>(nxt, wn, bf[PAR ^ 1], bl);
  // (Raising the wave's priority around its MFMAs, s_setprio 1, made the
  // Gram launches 5% faster with 256 x 128 tiles; with the current tiles it
  // made the S8 runs 0.5-1% slower, so the waves keep the default.)
#pragma unroll
  for (int i = 0; i < G::kSubM; ++i) {
    mma_row<MODE>(af[i], bf[PAR], acc[i]);
    if (more) load_a<MODE, G>(nxt, wm, i, af[i]);
  }
  if constexpr (SEL >= 0) mma_one_hot<MODE>(sel_s, SEL, bf[PAR], acc[MODE == kS8F16 ? SEL : SEL >> 1]);
}

// ACCG: also accumulate sel_s * G over the wave's rows (square phase; A and
// B are the same symmetric G, K = rows of G).  BKM: B is a K-major
// row-major operand (C = A B, apply), brow0 its first column.  Row pitches
// (ld), K and brow0 are in elements; an FP16 operand (MODE kS8F16) is
// addressed in 4-byte units, half of each.
template <int MODE, class G, bool ACCG, bool BKM, bool UB = false>
__device__ __forceinline__ void gemm_tile(const Opnd &A_in, const Opnd &B_in, int64_t K, int64_t arow0, int64_t brow0,
                                          float sel_s, char *smem, f32x16 (&acc)[G::kSubM][kSubN]) {
  constexpr int kSubM = G::kSubM;
  constexpr bool F16 = MODE == kS8F16;
  constexpr int kU = F16 ? 2 : 1;  // elements per 4-byte unit
  static_assert((kSubM == 4 || kSubM == 2) && kBK == 16, "the one_hot window is 2 kSubM stages of 16 rows");
  // (UB: pass the operand bases through readfirstlane, for the kernels in
  // which the compiler keeps them in vector registers: see uniform_ptr.)
  const Opnd A{UB ? uniform_ptr(A_in.p) : A_in.p, A_in.ld / kU}, B{UB ? uniform_ptr(B_in.p) : B_in.p, B_in.ld / kU};
  static_assert((8 * kSubN) % 16 == 0, "the wave's K-major column offset must be whole chunk groups");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wm = wave / G::kWavesN, wn = wave % G::kWavesN;  // 2 x kWavesN waves
#pragma unroll
  for (int i = 0; i < kSubM; ++i)
#pragma unroll
    for (int j = 0; j < kSubN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int nk = static_cast<int>(K / (kBK * kU));
  WaveOffsets<G> o;
  o.a = tile_offsets<G::kLoadsA>(A.ld, arow0, wave);
  o.b = BKM ? tile_offsets_km<G::kLoadsB, F16 ? G::kKmRowH : G::kKmRow,
                              F16 ? kKmSwzH : MODE == SMX_S8_FP32 ? kKmSwzNone : kKmSwzT>(B.ld, brow0 / kU, wave)
            : tile_offsets<G::kLoadsB>(B.ld, brow0, wave);
  o.b_lds = static_cast<uint32_t>(G::kOpA + wave * (G::kLoadsB - G::kLoadsA) * 1024);
  // used by the K-major B path only
  const BkmLane bl = F16 ? bkm_lane_f16(wn) : bkm_lane(wn);
  // LDS byte address of the ring plus this wave's first A chunk.
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem)) + wave * G::kLoadsA * 1024;
#pragma unroll
  for (int s = 0; s < G::kStages; ++s)
    if (s < nk) issue_stage<G, BKM, kU>(A, B, o, static_cast<int64_t>(s) * kBK, lds0 + s * G::kStageBytes);
  wait_stages<G>(min(G::kStages - 1, nk - 1));
  block_barrier();
  AFrag<MODE> af[kSubM];
  BFrags<MODE> bf[2];
  load_b_any<MODE, G, BKM>(smem, wn, bf[0], bl);
#pragma unroll
  for (int i = 0; i < kSubM; ++i) load_a<MODE, G>(smem, wm, i, af[i]);
#define SMX_PIPE(SEL, PAR, KT, STEADY) \
  pipe_iter<MODE, G, SEL, PAR, STEADY, BKM>(A, B, o, bl, lds0, sel_s, smem, KT, nk, wm, wn, af, bf, acc)
  // Stages [kt, to) in pairs (kt and `to` even): branch-free while a refill
  // is due, then the general form.
  const int steady_end = nk - G::kStages;
  auto run = [&](int &kt, int to) {
    for (; kt + 1 < min(to, steady_end); kt += 2) {
      SMX_PIPE(-1, 0, kt, true);
      SMX_PIPE(-1, 1, kt + 1, true);
    }
    for (; kt + 1 < to; kt += 2) {
      SMX_PIPE(-1, 0, kt, false);
      SMX_PIPE(-1, 1, kt + 1, false);
    }
  };
  int kt = 0;
  if constexpr (ACCG) {
    // The wave's rows are K stages kt0 .. kt0 + kWin - 1 (kt0 = first row /
    // 16, or / 32 for FP16: even, so the stage parity matches the unrolled
    // pairs).
    constexpr int kWin = (F16 ? 1 : 2) * kSubM;
    const int kt0 = static_cast<int>((arow0 + wm * (32 * kSubM)) / (kBK * kU));
    run(kt, kt0);
    SMX_PIPE(0, 0, kt0, false);
    SMX_PIPE(1, 1, kt0 + 1, false);
    if constexpr (kWin >= 4) {
      SMX_PIPE(2, 0, kt0 + 2, false);
      SMX_PIPE(3, 1, kt0 + 3, false);
    }
    if constexpr (kWin == 8) {
      SMX_PIPE(4, 0, kt0 + 4, false);
      SMX_PIPE(5, 1, kt0 + 5, false);
      SMX_PIPE(6, 0, kt0 + 6, false);
      SMX_PIPE(7, 1, kt0 + 7, false);
    }
    kt = kt0 + kWin;
  }
  run(kt, nk);
#undef SMX_PIPE
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

// Stage-1 scalars of a matrix: ||V||^2 (the input's total, kCstFro) and the
// Schatten scale s = max(1.35 ||G2||_F^(1/4), 1e-30) of the normalised G2
// (sandmuon/optimizer.py:80-84).  ok = false for a zero matrix.
struct Stage1Scalars {
  double fro2;
  float s;
  bool ok;
};
// Tiles of a symmetric r x r result (Gram, square, SYM) in a geometry: the
// upper-triangle 256 x 256 blocks (kGeoL), each as two 128-column halves
// (kGeoM), or the upper-triangle 128 x 128 tiles (kGeoS).
__host__ __device__ inline int64_t square_tiles(const S8Class &k, int geo) {
  return geo == kGeoS ? sym_tiles(k.tiles_s) : geo == kGeoL ? sym_tiles(k.tiles_m) : 2 * sym_tiles(k.tiles_m);
}

__device__ Stage1Scalars stage1_scalars(const S8Mat &M, int sq_geo, double *bcast) {
  Stage1Scalars r;
  r.fro2 = M.cst()[kCstFro];
  const double sq = sum_parts(M.sch(), static_cast<int>(square_tiles(*M.kp(), sq_geo)), bcast);
  r.ok = r.fro2 > 0.0 && sq > 0.0;
  r.s = r.ok ? fmaxf(static_cast<float>(kS8Margin * pow(sq, 0.125)), 1e-30f) : 1.f;
  return r;
}

// Block -> (class, XCD-contiguous tile index).  Blocks are dealt to the
// XCDs round robin, so consecutive logical tiles (the tiles of one matrix)
// share an L2 when L = (jb % 8) * per + jb / 8.
struct TileRef {
  const S8Class *k;
  int64_t L;
  int op;     // SegOp of the segment (SYM and APPLY launches)
  int slot0;  // the segment's first slot and number of matrices
  int cnt;
};
__device__ __forceinline__ TileRef tile_of(const StageArgs &args) {
  const int b = blockIdx.x;
  int seg = 0;
  while (seg + 1 < args.n_seg && b >= args.seg_off[seg + 1]) ++seg;
  const int jb = b - args.seg_off[seg];
  const int per = (args.seg_off[seg + 1] - args.seg_off[seg]) / 8;
  return TileRef{&args.L.cls[args.seg_cls[seg]], static_cast<int64_t>(jb % 8) * per + jb / 8, args.seg_op[seg],
                 args.seg_slot0[seg], args.seg_cnt[seg]};
}

// Epilogue staging: a 32 x 32 FP32 block per orientation per wave, rows
// padded to 36 floats (16-byte aligned row vectors).
constexpr int kEpStride = 36;
constexpr int kEpBlock = 32 * kEpStride;
template <class G>
constexpr bool epilogue_fits() {
  // per wave two staging blocks; the apply adds the tile's a and z vectors
  return (G::kWaves * 2 * kEpBlock + 2 * (G::kTileM > G::kTileN ? G::kTileM : G::kTileN)) * 4 <= G::kRingBytes;
}
static_assert(epilogue_fits<GeoM>() && epilogue_fits<GeoS>() && epilogue_fits<GeoL>(),
              "epilogue staging and the row-sum column vectors must fit in the operand ring");

__device__ __forceinline__ void ep_read8(const float *s, int row, int col, float (&w)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(s + row * kEpStride + col);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(s + row * kEpStride + col + 4);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// ------------------------------------------------------------ kernel ---
// Output tiles are TM x TN: tm counts TM-row blocks, tn TN-column blocks.
// The Gram, the square and the SYM products compute the upper triangle of
// their symmetric result (square_tiles): 256 x 256 tiles are its
// upper-triangle blocks (tn >= tm, row by row); 256 x 128 tiles the
// halves of those blocks (tix = 2 * block index + half); 128 x 128 tiles
// its upper-triangle 128 x 128 tiles.  A diagonal block or tile is
// computed whole; an off-diagonal one also writes its mirror.
__host__ __device__ inline int64_t phase_tiles(const S8Class &k, int phase, int geo, int op = -1) {
  if (phase == kApply)
    return static_cast<int64_t>(geo == kGeoS ? k.tiles_s : k.tiles_m) *
           ((op == kOpApplyQ ? k.rp : k.cp) / (geo == kGeoL ? 256 : 128));
  return square_tiles(k, geo);
}

template <int MODE, int PHASE, int TM, int TN>
__global__ void __launch_bounds__((Geo<TM, TN>::kThreads))
__attribute__((amdgpu_waves_per_eu(Geo<TM, TN>::kWavesPerEU, Geo<TM, TN>::kWavesPerEU)))
s8_stage_kernel(StageArgs args) {
  using Gm = Geo<TM, TN>;
  constexpr int kSubM = Gm::kSubM, kTileN = Gm::kTileN, kThreads = Gm::kThreads, kWaves = Gm::kWaves;
  __shared__ __attribute__((aligned(16))) char smem[Gm::kRingBytes];
  __shared__ double dscratch[16];
  __shared__ double bcast;

  const TileRef ref = tile_of(args);
  const S8Class &K = *ref.k;
  const int64_t tpm = phase_tiles(K, PHASE, Gm::kGeo, ref.op);
  if (ref.L >= tpm * ref.cnt) return;
  const int slot = ref.slot0 + static_cast<int>(ref.L / tpm);
  const int64_t tix = ref.L % tpm;
  int64_t tm, tn;
  bool diag = false;  // symmetric result: a diagonal block or tile (or a half of one)
  if constexpr (PHASE == kApply) {
    // Column-major over the output: consecutive tiles (one XCD's L2) share
    // a column block of X and cycle through P's row blocks, so each X block
    // is fetched once (0.54 GB per cfg4 apply launch against 0.77 GB
    // row-major; the launch time is the same).
    const int64_t nrow = Gm::kGeo == kGeoS ? K.tiles_s : K.tiles_m;  // row tiles
    tn = tix / nrow;
    tm = tix % nrow;
  } else if constexpr (Gm::kGeo == kGeoM) {
    int64_t rem = tix >> 1;
    tm = 0;
    while (rem >= K.tiles_m - tm) { rem -= K.tiles_m - tm; ++tm; }
    const int64_t tb = tm + rem;
    tn = 2 * tb + (tix & 1);
    diag = tb == tm;
  } else {
    const int64_t nt = Gm::kGeo == kGeoL ? K.tiles_m : K.tiles_s;  // tiles per row and column
    int64_t rem = tix;
    tm = 0;
    while (rem >= nt - tm) { rem -= nt - tm; ++tm; }
    tn = tm + rem;
    diag = tn == tm;
  }
  const S8Mat M{K, slot};
  const int stage = args.stage;
  const bool odd = (stage & 1) != 0;
  // The stage-5 result of the matrix step also leaves row sums for the
  // mapback (see the epilogue); the A factor and rank-one entries of the
  // tile's parameter columns are loaded two per thread, here in the
  // compensated modes, so their latency hides under the K loop (the FP32
  // kernel has no two registers to spare and loads them after it), and
  // pass through LDS to the epilogue.
  const bool rsum = PHASE == kApply && stage == 5 && args.L.rowsums != 0 &&
                    (ref.op == kOpApplyX || ref.op == kOpApplyFinal);
  const int64_t rs_c0 = M.flip() ? tm * Gm::kTileM : tn * kTileN;  // first parameter column of the tile
  const int rs_w = M.flip() ? Gm::kTileM : kTileN;                 // parameter columns of the tile
  float colv_pre[2] = {0.f, 0.f};
  auto load_colv = [&]() {
    const float *acol = M.acol(), *zcol = M.zcol();
    const int64_t pcols = M.pcol();
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int idx = static_cast<int>(threadIdx.x) + kThreads * v;  // [vector][column]
      const int64_t col = rs_c0 + idx % rs_w;
      const float *src = idx < rs_w ? acol : zcol;
      if (idx < 2 * rs_w && src && col < pcols) colv_pre[v] = src[col];
    }
  };
  constexpr bool kColvEarly = MODE != SMX_S8_FP32;
  if (kColvEarly && rsum) load_colv();
  float *x_in = odd ? M.x0() : M.x1();
  float *x_out = odd ? M.x1() : M.x0();

  f32x16 acc[kSubM][kSubN];
  float scale = 1.f;
  float *sym_out = nullptr;  // SYM: the product's destination
  // Gram space (see the header): a segment's first Q sits in qa; Q' = P Q
  // goes qa -> qb at stages 2 and 4 and qb -> qa at stage 5.
  float *q_in = stage == 5 ? M.qb() : M.qa();
  float *q_out = stage == 5 ? M.qa() : M.qb();
  if constexpr (PHASE == kSym) {
    float *pk = stage == 1 || stage == 3 ? M.qa() : M.p();
    const float *A, *B;
    if (ref.op == kOpPG) {
      A = pk; B = M.g(); sym_out = M.t();
    } else {
      A = M.t(); B = pk; sym_out = M.g();
      if (stage == 1) {
        // G1 = P1 G0 P1 / s^2
        const Stage1Scalars sc = stage1_scalars(M, args.sq_geo, &bcast);
        scale = sc.ok ? 1.0f / (sc.s * sc.s) : 0.f;
      }
    }
    gemm_tile<MODE, Gm, false, false, MODE == kS8CompMix>(Opnd{A, K.rp}, Opnd{B, K.rp}, K.rp, tm * Gm::kTileM,
                                                         tn * kTileN, 0.f, smem, acc);
  } else if constexpr (PHASE == kGram) {
    if (stage == 1) {
      const double f = M.cst()[kCstFro];
      scale = f > 0.0 ? static_cast<float>(1.0 / f) : 0.f;
    }
    // A Gram-space class takes its stage-3 Gram of X2 from x1.
    const Opnd X{K.gs && stage == 3 ? M.x1() : x_in, K.cp};
    gemm_tile<MODE, Gm, false, false>(X, X, K.cp, tm * Gm::kTileM, tn * kTileN, 0.f, smem, acc);
  } else if constexpr (PHASE == kSquare) {
    const Opnd G{M.g(), K.rp};
    // (the square kernels run at the VGPR budget, where the compiler keeps
    // the operand bases in vector registers)
    constexpr bool kUB = true;
    if (stage == 1) {
      gemm_tile<MODE, Gm, false, false, kUB>(G, G, K.rp, tm * Gm::kTileM, tn * kTileN, 0.f, smem, acc);
    } else {
      // acc = G G + (b/c) G; the epilogue forms P = c acc + a I.
      scale = args.c;
      gemm_tile<MODE, Gm, true, false, kUB>(G, G, K.rp, tm * Gm::kTileM, tn * kTileN, args.b_over_c, smem, acc);
    }
  } else {
    // X-space: X' = P X (stage 1: X' = P1 V / (||V|| s)).  Gram space:
    // Q' = P Q; X2 = Q2 V / (||V|| s), V in x0; X5 = Q5 X2, X2 in x1.
    const int op = ref.op;
    const bool gq = op == kOpApplyQ, mid = op == kOpApplyMid, fin = op == kOpApplyFinal;
    if (stage == 1 || mid) {
      const Stage1Scalars sc = stage1_scalars(M, args.sq_geo, &bcast);
      scale = sc.ok ? static_cast<float>(1.0 / (sqrt(sc.fro2) * static_cast<double>(sc.s))) : 0.f;
    }
    const float *A = mid ? M.qb() : fin ? M.qa() : M.p();
    const Opnd B = gq ? Opnd{q_in, K.rp} : Opnd{mid ? M.x0() : fin ? M.x1() : x_in, K.cp};
    // B = X (or Q) rows k (K-major), columns of the tile.
    gemm_tile<MODE, Gm, false, true>(Opnd{A, K.rp}, B, K.rp, tm * Gm::kTileM, tn * kTileN, 0.f, smem, acc);
  }

  // ------------------------------------------------------- epilogue ---
  // Each lane holds, per 32x32 accumulator block, 8 consecutive columns of
  // each 16-column K group of one row (sw23; FP32 mode: four quads of 4
  // columns), which it stores directly as row vectors: 16 bytes per store,
  // the two lanes of a row 32 contiguous bytes of it (FP32 row-major
  // results of the other modes: 16).  A transposed output (the mirror of an off-diagonal
  // symmetric tile, the stage-5 result of a transposed parameter) goes
  // through wave-private LDS: written by column, read back as rows of 8
  // elements per lane.
  //   GRAM    tile -> G, transpose -> G (halves of off-diagonal blocks)
  //   SQUARE  stage 1: G2 (FP32) -> p; stage k: P = c acc + a I -> p
  //   APPLY   tile -> X' (stage 5, transposed parameter: transpose -> xf)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / Gm::kWavesN, wn = wave % Gm::kWavesN;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t R0 = tm * Gm::kTileM + wm * (32 * kSubM), C0 = tn * kTileN + wn * (32 * kSubN);
  const bool last = stage == 5;
  float *dst_t, *dst_m;
  int64_t ld_t, ld_m;
  bool do_t, do_m;
  // The output's form is that of the product that reads it (out_form); a
  // transposed stage-5 result (dst_m) is FP32 as the stage-5 form is.
  const int form = out_form(args.L.mode, args.mask, PHASE, stage, ref.op, K.gs != 0);
  if constexpr (PHASE == kApply) {
    if (ref.op == kOpApplyQ) {
      dst_t = q_out; ld_t = K.rp;
      dst_m = nullptr; ld_m = K.rp;
      do_t = true;
      do_m = false;
    } else if (ref.op == kOpApplyMid) {
      dst_t = M.x1(); ld_t = K.cp;  // X2, an operand of the stage-3 Gram and the final apply
      dst_m = nullptr; ld_m = K.rp;
      do_t = true;
      do_m = false;
    } else {
      const bool xf = last && M.flip();
      dst_t = ref.op == kOpApplyFinal ? M.x0() : x_out; ld_t = K.cp;
      dst_m = xf ? M.xf() : nullptr; ld_m = K.rp;
      do_t = !xf;
      do_m = xf;
    }
  } else {
    // A Gram-space square at stage 3 writes P3 to qa: it is Q3.
    float *sq_out = K.gs && stage == 3 ? M.qa() : M.p();
    dst_t = dst_m = PHASE == kSym ? sym_out : PHASE == kGram ? M.g() : sq_out;
    ld_t = ld_m = K.rp;
    do_t = true;
    do_m = !diag;
  }
  // Every output is a tiled operand except the stage-5 result (row-major
  // FP32: the mapback's and the stand-alone map's input).
  const bool tiled_t = !(PHASE == kApply && last && (ref.op == kOpApplyX || ref.op == kOpApplyFinal));
  const bool tiled_m = PHASE != kApply;
  const bool eye = PHASE == kSquare && stage != 1;  // add a I on the diagonal
  // the wave's staging block of a transposed output: [column][row]
  float *const U = reinterpret_cast<float *>(smem) + wave * 2 * kEpBlock;
  float sq_local = 0.f;
  // The stage-5 result of the matrix step: per parameter row, partial sums
  // of Q z, (a Q)^2 and (a Q)(a z) over a strip of parameter columns (the
  // wave's 64 output columns; for a transposed parameter, 64 of its output
  // rows), reduced over the lanes that hold the row (the two lanes of a
  // directly stored row, the 8 of a staged transposed one) and stored for
  // the mapback (its row coefficients and graft norm), so no later pass
  // reads Q for them.
  static_assert(PHASE != kApply || (kStripT == 32 * kSubN && (32 * kSubM) % kStripM == 0),
                "a row-sum strip is one wave's share of an apply tile");
  const int64_t prows = M.prow_pad();
  // a and z of the tile's parameter columns in LDS past the staging blocks
  // (the operand ring is free once the K loop is done).
  float *const colv_lds = reinterpret_cast<float *>(smem) + kWaves * 2 * kEpBlock;
  if (rsum) {
    if (!kColvEarly) load_colv();
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int idx = static_cast<int>(threadIdx.x) + kThreads * v;
      if (idx < 2 * rs_w) colv_lds[idx] = colv_pre[v];
    }
    __syncthreads();
  }
  // Read-back of a staged (transposed) block: 8 lanes per row of a 32 x 32
  // block, each the 16-byte chunk
  // `ech` of the row's 128 bytes (32 columns), so that every store
  // instruction writes 8 whole rows of the block: full 128-byte lines (a
  // burst of such stores runs 25% faster than one of 32-byte pieces).  In
  // operand form the chunk is plane (ech >> 1) & 1 of columns
  // 16 (ech >> 2) + 8 (ech & 1) .. + 7; in FP32 columns 4 ech .. 4 ech + 3.
  const int er = lane >> 3, ech = lane & 7;
  // the lane's chunk: tiled, byte 16 (ech & 3) of the row's K group ech >> 2;
  // row-major, byte 16 ech of the row's 128 bytes
  const int ech_t = ((ech >> 2) << 10) + ((ech & 3) << 4), ech_r = ech << 4;
  const bool lo_plane = ((ech >> 1) & 1) != 0;
  const int ec8 = 16 * (ech >> 2) + 8 * (ech & 1), ec4 = 4 * ech;
  float rs[kSubN][4][3];
#pragma unroll
  for (int j = 0; j < kSubN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) rs[j][q][0] = rs[j][q][1] = rs[j][q][2] = 0.f;
  // The row-sum partials of one row (FP32 output, four columns per lane),
  // reduced over the row's 8 lanes and stored by the first.
  auto accum4 = [&](const float (&w)[4], int64_t gc, float (&r)[3]) {
    const int o = static_cast<int>(gc - rs_c0);
    const f32x4 a4 = *reinterpret_cast<const f32x4 *>(colv_lds + o);
    const f32x4 z4 = *reinterpret_cast<const f32x4 *>(colv_lds + rs_w + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float aw = a4[e] * w[e];
      r[0] = fmaf(w[e], z4[e], r[0]);
      r[1] = fmaf(aw, aw, r[1]);
      r[2] = fmaf(aw, a4[e] * z4[e], r[2]);
    }
  };
  auto emit = [&](int64_t prow, int64_t strip, float (&r)[3]) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      r[k] += dpp_mov<0xB1>(r[k]);   // quad_perm [1,0,3,2]
      r[k] += dpp_mov<0x4E>(r[k]);   // quad_perm [2,3,0,1]
      r[k] += dpp_mov<0x141>(r[k]);  // row_half_mirror: the row's 8 lanes
    }
    if (ech == 0)
#pragma unroll
      for (int k = 0; k < 3; ++k) M.mrp(k)[strip * prows + prow] = r[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) r[k] = 0.f;
  };
  // Row `row` of a staged block (S) to global row gr, columns gc0 .. gc0 + 31
  // (gc0 a multiple of 32) in form FM: one 16-byte store per lane (FP32,
  // planes), or one 8-byte store of the lane's four columns (FP16: the
  // row's 64 bytes).  A tiled output (`tl`; planes and FP16 always are)
  // puts the row's two 64-byte K groups (one for FP16) in their pieces, so
  // the 8 rows of a store instruction fill two 512-byte halves of pieces.
  // (FM = kFormAny: planes or FP32 chosen at run time by `form`, one loop
  // for both, in the kernels that produce no FP16.)
  auto put_row = [&](auto fm_c, const float *S, int row, int64_t gr, int64_t gc0, float *dst, int64_t ld, bool tl,
                     float (&r)[3], bool acc_r) {
    constexpr int FM = decltype(fm_c)::value;
    if constexpr (FM == kFormF16) {
      const f32x4 v4 = *reinterpret_cast<const f32x4 *>(S + row * kEpStride + ec4);
      float w[4] = {v4.x, v4.y, v4.z, v4.w};
      if (eye)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (gr == gc0 + ec4 + e && gr < K.r) w[e] += args.a;
      uint32_t b[2];
#pragma unroll
      for (int e = 0; e < 2; ++e)
        b[e] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(w[2 * e]))) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(w[2 * e + 1]))) << 16);
      // (32-column pieces: group gc0 / 32 at 32 gc0 bytes of the row block)
      const int64_t off = (gr & ~int64_t{15}) * (2 * ld) + ((gr & 15) << 6) + 32 * gc0 + 8 * ech;
      *reinterpret_cast<uint2 *>(reinterpret_cast<char *>(dst) + off) = make_uint2(b[0], b[1]);
      return;
    }
    const bool pl = FM == kFormPlanes || (FM == kFormAny && form == kFormPlanes);
    // Row block, row in it, columns: (gr & ~15) 4 ld + (gr & 15) rs + gc0 cs
    // + the lane's chunk, rs = 64 and cs = 64 tiled (group gc0 / 16 at
    // 1024 gc0 / 16 bytes of the row block), rs = 4 ld and cs = 4 row-major.
    const bool t = pl || tl;
    const int64_t off = (gr & ~int64_t{15}) * (4 * ld) + (gr & 15) * (t ? 64 : 4 * ld) + gc0 * (t ? 64 : 4) +
                        (t ? ech_t : ech_r);
    char *out = reinterpret_cast<char *>(dst) + off;
    if (pl) {
      float w[8];
      ep_read8(S, row, ec8, w);
      if (eye)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (gr == gc0 + ec8 + e && gr < K.r) w[e] += args.a;
      uint32_t b[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t x0 = lo_plane ? bf16_lo_bits(w[2 * e]) : bf16_bits(w[2 * e]);
        const uint16_t x1 = lo_plane ? bf16_lo_bits(w[2 * e + 1]) : bf16_bits(w[2 * e + 1]);
        b[e] = x0 | (static_cast<uint32_t>(x1) << 16);
      }
      *reinterpret_cast<uint4 *>(out) = make_uint4(b[0], b[1], b[2], b[3]);
    } else {
      const f32x4 v4 = *reinterpret_cast<const f32x4 *>(S + row * kEpStride + ec4);
      float w[4] = {v4.x, v4.y, v4.z, v4.w};
      if (eye)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (gr == gc0 + ec4 + e && gr < K.r) w[e] += args.a;
      *reinterpret_cast<float4 *>(out) = make_float4(w[0], w[1], w[2], w[3]);
      if (acc_r) accum4(w, gc0 + ec4, r);
    }
  };
  // Register e of a block holds column col16(e) of the lane's row (FP32
  // mode: the natural MFMA order, 8 (e >> 2) + 4 lh + (e & 3)).
  auto col16 = [&](int e) {
    return MODE == SMX_S8_FP32 ? 8 * (e >> 2) + 4 * lh + (e & 3) : 16 * (e >> 3) + 8 * lh + (e & 7);
  };
  // The lane's 16 values w of row gr, columns cb + col16(e) (cb a multiple
  // of 32), stored in form FM: planes and FP16 put each K group's 8 columns
  // of the lane at their place in the group's row (planes: 16 bytes of hi at
  // 16 lh, 16 of lo at 32 + 16 lh; FP16: 16 bytes at 16 lh of the 32-column
  // piece's half g); FP32 (tiled, or row-major for the stage-5 result) as
  // 16-byte quads of columns.
  auto put_direct = [&](auto fm_c, const float (&w)[16], int64_t gr, int64_t cb, float *dst, int64_t ld, bool tl) {
    constexpr int FM = decltype(fm_c)::value;
    char *const out = reinterpret_cast<char *>(dst);
    if constexpr (FM == kFormF16) {
      const int64_t base = (gr & ~int64_t{15}) * (2 * ld) + ((gr & 15) << 6) + 32 * cb + 16 * lh;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        uint32_t b[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          b[e] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(w[8 * g + 2 * e]))) |
                 (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(w[8 * g + 2 * e + 1])))
                  << 16);
        *reinterpret_cast<uint4 *>(out + base + 32 * g) = make_uint4(b[0], b[1], b[2], b[3]);
      }
      return;
    }
    const bool pl = FM == kFormPlanes || (FM == kFormAny && form == kFormPlanes);
    if (pl) {
      const int64_t base = (gr & ~int64_t{15}) * (4 * ld) + ((gr & 15) << 6) + 64 * cb + 16 * lh;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        uint32_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          h[e] = bf16_bits(w[8 * g + 2 * e]) | (static_cast<uint32_t>(bf16_bits(w[8 * g + 2 * e + 1])) << 16);
          l[e] = bf16_lo_bits(w[8 * g + 2 * e]) | (static_cast<uint32_t>(bf16_lo_bits(w[8 * g + 2 * e + 1])) << 16);
        }
        *reinterpret_cast<uint4 *>(out + base + 1024 * g) = make_uint4(h[0], h[1], h[2], h[3]);
        *reinterpret_cast<uint4 *>(out + base + 1024 * g + 32) = make_uint4(l[0], l[1], l[2], l[3]);
      }
    } else {
      // each quad of 4 consecutive columns c = col16(4 e4) .. + 3: tiled,
      // byte 4 (c & 15) of the row of K group c >> 4; row-major, byte 4 c
      const int64_t base = tl ? (gr & ~int64_t{15}) * (4 * ld) + ((gr & 15) << 6) + 64 * cb : gr * (4 * ld) + 4 * cb;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int c = col16(4 * e4), e = 4 * e4;
        *reinterpret_cast<float4 *>(out + base + (tl ? 1024 * (c >> 4) + 4 * (c & 15) : 4 * c)) =
            make_float4(w[e], w[e + 1], w[e + 2], w[e + 3]);
      }
    }
  };
  // The block loop, specialised for the output form (one copy per form the
  // launch's mode can produce, so that each keeps only its own registers).
  auto epilogue = [&](auto fm_c) {
    constexpr int FM = decltype(fm_c)::value;
    // the row sums come with the FP32 result only (rsum implies it)
    const bool rs_on = (FM == kFormF32 || FM == kFormAny) && rsum;
    // Row sums of the lane's row over the wave's strip (its kSubN blocks),
    // for a parameter that is not transposed.
    float rsd[3] = {0.f, 0.f, 0.f};
    // (expanded at compile time: a rolled block loop indexes acc at run
    // time, which moves every accumulator of the kernel to scratch memory)
    static_for<kSubM * kSubN>([&](auto blk_c) {
      constexpr int blk = decltype(blk_c)::value, i = blk / kSubN, j = blk % kSubN;
      const int64_t gr = R0 + i * 32 + lr, cb = C0 + j * 32;
      float w[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        w[e] = acc[i][j][e] * scale;
        // stage 1's FP32 G2: its squared entries feed the Schatten scale
        if constexpr (PHASE == kSquare && (FM == kFormF32 || FM == kFormAny)) sq_local = fmaf(w[e], w[e], sq_local);
        if (do_m) U[col16(e) * kEpStride + lr] = w[e];
      }
      if (do_t) {
        if (eye)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (gr == cb + col16(e) && gr < K.r) w[e] += args.a;
        put_direct(fm_c, w, gr, cb, dst_t, ld_t, tiled_t);
        if (rs_on) {
          // a and z of the lane's columns, then the row's two lanes (lh)
          const int o = static_cast<int>(cb - rs_c0);
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int oc = o + col16(4 * e4);
            const f32x4 a4 = *reinterpret_cast<const f32x4 *>(colv_lds + oc);
            const f32x4 z4 = *reinterpret_cast<const f32x4 *>(colv_lds + rs_w + oc);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x = w[4 * e4 + e], aw = a4[e] * x;
              rsd[0] = fmaf(x, z4[e], rsd[0]);
              rsd[1] = fmaf(aw, aw, rsd[1]);
              rsd[2] = fmaf(aw, a4[e] * z4[e], rsd[2]);
            }
          }
          if (j == kSubN - 1) {
#pragma unroll
            for (int k = 0; k < 3; ++k) rsd[k] += __shfl_xor(rsd[k], 32);
            if (lh == 0)
#pragma unroll
              for (int k = 0; k < 3; ++k) M.mrp(k)[(C0 / kStripT) * prows + gr] = rsd[k];
#pragma unroll
            for (int k = 0; k < 3; ++k) rsd[k] = 0.f;
          }
        }
      }
      if (do_m) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = er + 8 * q;
          const int64_t gm = cb + row;
          put_row(fm_c, U, row, gm, R0 + i * 32, dst_m, ld_m, tiled_m, rs[j][q], rs_on);
          if (rs_on && (i + 1) % (kStripM / 32) == 0) emit(gm, (R0 + 32 * (i + 1) - kStripM) / kStripM, rs[j][q]);
        }
      }
      // Keep the scheduler from hoisting every accumulator read to the top
      // of the epilogue (the values would not fit in the VGPRs).
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // Only the forms this launch kind can produce are compiled (the host
  // checks every launch's forms against the same table, form_compiled).
  constexpr bool kPlanes = form_compiled(MODE, PHASE, kFormPlanes);
  constexpr bool kF16 = form_compiled(MODE, PHASE, kFormF16);
  constexpr bool kF32 = form_compiled(MODE, PHASE, kFormF32);
  if constexpr (PHASE == kSquare && kPlanes && kF32 && !kF16) {
    // one loop for both forms, as compact as a kernel of one form
    epilogue(std::integral_constant<int, kFormAny>{});
  } else if (kPlanes && form == kFormPlanes) {
    if constexpr (kPlanes) epilogue(std::integral_constant<int, kFormPlanes>{});
  } else if (kF16 && form == kFormF16) {
    if constexpr (kF16) epilogue(std::integral_constant<int, kFormF16>{});
  } else {
    if constexpr (kF32) epilogue(std::integral_constant<int, kFormF32>{});
  }
  if constexpr (PHASE == kSquare) {
    if (stage == 1) {
      const double s = block_sum(static_cast<double>(sq_local), dscratch);
      if (threadIdx.x == 0) M.sch()[tix] = (diag ? 1.0 : 2.0) * s;
    }
  }
}

// Stage-1 polynomial operand (sandmuon/optimizer.py:84-86) over the r x r
// matrices of a class: P1 = a I + (b G)/s^2 + (c G2)/s^4 from the
// normalised G and the FP32 G2 of the square phase, written over G2 in the
// p buffer in operand form (into qa, as Q1, for a Gram-space class).  G,
// G2 and P1 are tiled alike, so the pass runs over their 64-byte runs in
// memory order, and only the diagonal term needs an element's row and
// column.  A block takes kPolyChunk consecutive runs of one matrix, four
// lanes per group, each lane a quarter (4 elements: 16 bytes of FP32, 8 of
// each BF16 half), so that every load and store instruction of a wave
// covers 16 whole groups (1 KB); a thread takes kPolyUnits quarters.  All
// loads are issued before the block sums the stage-1 scalars, which they do
// not depend on.  (In place for an X-space class: the lanes of a group are
// one wave's, and a group's loads complete before any of its stores.)
constexpr int kPolyUnits = 4;
constexpr int kPolyChunk = 256 * kPolyUnits / 4;  // groups per block

__host__ __device__ inline int64_t poly_blocks_per_matrix(const S8Class &k) {
  return k.rp * k.rp / 16 / kPolyChunk;  // rp is a multiple of 256
}

template <int MODE>
__global__ void __launch_bounds__(256) s8_poly1_kernel(StageArgs args) {
  __shared__ double bcast;
  constexpr bool PL = MODE == SMX_S8_COMP_BF16;
  const TileRef ref = tile_of(args);
  const S8Class &K = *ref.k;
  const int64_t tpm = poly_blocks_per_matrix(K);
  if (ref.L >= tpm * ref.cnt) return;
  const S8Mat M{K, ref.slot0 + static_cast<int>(ref.L / tpm)};
  const int64_t g0 = (ref.L % tpm) * kPolyChunk;  // first group of the block
  const int64_t gpr = K.rp / 16;                   // groups per row
  const int qt = threadIdx.x & 3;                  // the lane's quarter of its groups
  const float *G = M.g();
  const float *P = M.p();                                           // FP32 G2
  SMX_GLOBAL float *Pout = (SMX_GLOBAL float *)(K.gs ? M.qa() : M.p());  // Gram space: P1 is Q1
  int64_t grp[kPolyUnits];
  float4 w4[kPolyUnits];
  uint2 gh[kPolyUnits], gl[kPolyUnits];  // BF16 hi and lo of the quarter, or its FP32 G
#pragma unroll
  for (int k = 0; k < kPolyUnits; ++k) {
    grp[k] = g0 + (threadIdx.x + 256 * k) / 4;
    const int64_t idx = grp[k] * 16 + 4 * qt;
    w4[k] = *reinterpret_cast<const float4 *>(P + idx);
    if constexpr (PL) {
      const char *gb = reinterpret_cast<const char *>(G + grp[k] * 16);
      gh[k] = *reinterpret_cast<const uint2 *>(gb + 8 * qt);
      gl[k] = *reinterpret_cast<const uint2 *>(gb + 32 + 8 * qt);
    } else {
      const uint4 g = *reinterpret_cast<const uint4 *>(G + idx);
      gh[k] = make_uint2(g.x, g.y);
      gl[k] = make_uint2(g.z, g.w);
    }
  }
  const Stage1Scalars sc = stage1_scalars(M, args.sq_geo, &bcast);
  const float s2 = sc.s * sc.s;
  const float is2 = sc.ok ? 1.0f / s2 : 0.f, is4 = sc.ok ? 1.0f / (s2 * s2) : 0.f;
#pragma unroll
  for (int k = 0; k < kPolyUnits; ++k) {
    const float w[4] = {w4[k].x, w4[k].y, w4[k].z, w4[k].w};
    float g[4];
    if constexpr (PL) {
      const uint32_t hw[2] = {gh[k].x, gh[k].y}, lw[2] = {gl[k].x, gl[k].y};
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        g[2 * e] = __uint_as_float(hw[e] << 16) + __uint_as_float(lw[e] << 16);
        g[2 * e + 1] = __uint_as_float(hw[e] & 0xffff0000u) + __uint_as_float(lw[e] & 0xffff0000u);
      }
    } else {
      g[0] = __uint_as_float(gh[k].x); g[1] = __uint_as_float(gh[k].y);
      g[2] = __uint_as_float(gl[k].x); g[3] = __uint_as_float(gl[k].y);
    }
    // (tiled: run u is row 16 (u / 16 / gpr) + u % 16 of K group (u / 16) % gpr)
    const int64_t pc = grp[k] >> 4;
    const int64_t row = (pc / gpr) * 16 + (grp[k] & 15), col = (pc % gpr) * 16 + 4 * qt;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float eye = (row == col + e && row < K.r) ? args.a : 0.f;
      v[e] = (eye + (args.b * g[e]) * is2) + (args.c * w[e]) * is4;
    }
    put_operand4_paired(Pout, grp[k] * 16 + 4 * qt, v, PL, true);
  }
}

// ------------------------------------------------------------- host ---
// Optional per-launch event timing (smx_s8_timing).
struct LaunchTiming {
  int level = 0;  // 0 off, 1 every launch and every run, 2 runs only
  std::vector<hipEvent_t> start, stop;
  std::vector<int32_t> phase;
  std::vector<double> flops;
  size_t used = 0;
};
static LaunchTiming g_timing;

// Opens a record (start event on `st`) and returns its index in `slot`
// (-1 when the recorder does not record this kind); timing_end closes it.
// Records nest.
static int timing_begin(hipStream_t st, int &slot, bool whole_run) {
  slot = -1;
  if (g_timing.level == 0 || (g_timing.level == 2 && !whole_run)) return SMX_OK;
  if (g_timing.used == g_timing.start.size()) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)
      return fail(SMX_ELAUNCH, "s8 timing: hipEventCreate failed");
    g_timing.start.push_back(a);
    g_timing.stop.push_back(b);
    g_timing.phase.push_back(0);
    g_timing.flops.push_back(0.0);
  }
  slot = static_cast<int>(g_timing.used++);
  g_timing.phase[slot] = -1;  // open
  if (hipEventRecord(g_timing.start[slot], st) != hipSuccess)
    return fail(SMX_ELAUNCH, "s8 timing: hipEventRecord failed");
  return SMX_OK;
}

static int timing_end(int slot, hipStream_t st, int phase, double flops) {
  if (slot < 0) return SMX_OK;
  if (hipEventRecord(g_timing.stop[slot], st) != hipSuccess)
    return fail(SMX_ELAUNCH, "s8 timing: hipEventRecord failed");
  g_timing.phase[slot] = phase;
  g_timing.flops[slot] = flops;
  return SMX_OK;
}


// The segments of one launch, in class order by per-tile cost (K length,
// most expensive first, so long-K tiles start first and short tiles fill
// the remaining CUs).  A Gram-space class takes the Gram at stages 1 and 3
// only; SYM and APPLY launches take one segment per class and product in
// `ops` that applies to it at this stage (the Gram-space schedule above;
// APPLY: X' = P X for an X-space class).
struct Seg {
  int cls;
  int op;
  int lo, hi;  // slots
};

// The MFMA mode of one product of a launch (gemm_mode under the run's mode
// and the process-wide compensation mask).
static int seg_mode(const S8Layout &Lay, int phase, int stage, const Seg &sg) {
  return gemm_mode(Lay.mode, g_comp_mask, phase, stage, sg.op, Lay.cls[sg.cls].gs != 0);
}

// The matrices of one launch chain: slots lo[c] .. hi[c] - 1 of class c.
struct SlotSet {
  int32_t lo[kMaxClasses] = {}, hi[kMaxClasses] = {};
  bool empty() const {
    for (int i = 0; i < kMaxClasses; ++i)
      if (hi[i] > lo[i]) return false;
    return true;
  }
};
static std::vector<Seg> launch_segments(const S8Layout &Lay, const SlotSet &set, int phase, int stage,
                                        const std::vector<int> &ops) {
  std::vector<int> order(Lay.n_classes);
  for (int i = 0; i < Lay.n_classes; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
    const int64_t kx = phase == kGram ? Lay.cls[x].cp : Lay.cls[x].rp;
    const int64_t ky = phase == kGram ? Lay.cls[y].cp : Lay.cls[y].rp;
    return kx > ky;
  });
  std::vector<Seg> segs;
  for (int ci : order) {
    const S8Class &k = Lay.cls[ci];
    const int lo = set.lo[ci], hi = set.hi[ci];
    if (hi <= lo) continue;
    if (phase == kSym || phase == kApply) {
      for (int op : ops) {
        const bool takes = phase == kSym ? k.gs != 0 && gs_sym(stage)
                           : op == kOpApplyX ? k.gs == 0
                           : op == kOpApplyQ ? k.gs != 0 && gs_apply_q(stage)
                           : op == kOpApplyMid ? k.gs != 0 && stage == 2
                                               : k.gs != 0 && stage == 5;
        if (takes) segs.push_back(Seg{ci, op, lo, hi});
      }
      continue;
    }
    if (k.gs && phase == kGram && !gs_gram(stage)) continue;
    segs.push_back(Seg{ci, -1, lo, hi});
  }
  return segs;
}

// MFMA FLOPs of one launch in MFMA mode `mode`: computed tiles x 2 * TM *
// TN * K (x3 compensated), plus the square phase's one-hot MFMAs: per wave
// and 32x32 column tile, 2 kSubM window stages of 3 (compensated), 2
// (plain BF16: the scalar's hi and lo) or 1 (FP32) 16-deep products, or
// kSubM stages of 4 (FP16: hi and lo over each 16 K of a 32-deep stage).
static double launch_flops(int mode, int phase, int stage, int geo, const S8Layout &Lay,
                           const std::vector<Seg> &segs) {
  if (phase == kPoly1) return 0.0;
  const double prod = is_comp(mode) ? 3.0 : 1.0;
  const int tm = geo == kGeoS ? 128 : 256, tn = geo == kGeoL ? 256 : 128, waves = geo == kGeoL ? 8 : 4;
  const int sub_m = tm / 64;
  const double onehot = is_comp(mode) ? 6.0 * sub_m : mode == kS8HiOnly ? 4.0 * sub_m
                        : mode == kS8F16 ? 4.0 * sub_m : 2.0 * sub_m;
  double f = 0.0;
  for (const Seg &sg : segs) {
    const S8Class &k = Lay.cls[sg.cls];
    const double tiles = static_cast<double>(phase_tiles(k, phase, geo, sg.op));
    const double K = phase == kGram ? static_cast<double>(k.cp) : static_cast<double>(k.rp);
    const double cnt = sg.hi - sg.lo;
    f += cnt * tiles * 2.0 * tm * tn * K * prod;
    if (phase == kSquare && stage != 1) f += cnt * tiles * waves * onehot * kSubN * 2.0 * 32 * 32 * kBK;
  }
  return f;
}

static int64_t device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 256;
  return cus[dev];
}

// The tile geometry of one launch over `segs`.  256 x 256 tiles when the
// launch has at least 1.5 of them per CU: those blocks move a third fewer
// operand bytes per MFMA (cfg5 S8 7% faster).  With fewer, each CU holds
// one or two blocks of the launch and nothing of it to overlap a block's
// prologue and epilogue with (cfg4 Gram, square and SYM launches 15-60%
// slower; with tiled operands the cfg4 applies, 0.6-2.2 tiles per CU, are
// 1-2% faster as 256 x 128 tiles, two blocks per CU).  Otherwise 128 x 128
// tiles when they take fewer rounds of the CUs' block slots (three per CU,
// a round counted 0.9 of one of two 256 x 128 blocks per CU), else
// 256 x 128 (the cfg4 applies take 128 x 128 tiles: S8 runs 2% shorter
// than with 256 x 128).
static int pick_geo(const S8Layout &Lay, int phase, const std::vector<Seg> &segs) {
  if (g_tile_policy == 1) return kGeoL;
  const int64_t cus = device_cus();
  int64_t tiles[3] = {0, 0, 0};
  for (const Seg &sg : segs) {
    const S8Class &k = Lay.cls[sg.cls];
    const int64_t cnt = sg.hi - sg.lo;
    for (int g = 0; g < 3; ++g) tiles[g] += cnt * phase_tiles(k, phase, g, sg.op);
  }
  {
    static int thr_apply = getenv("SMX_XL_APPLY") ? atoi(getenv("SMX_XL_APPLY")) : 15;
    static int thr_other = getenv("SMX_XL_OTHER") ? atoi(getenv("SMX_XL_OTHER")) : 15;
    const int thr = phase == kApply ? thr_apply : thr_other;
    if (g_tile_policy == 0 && 10 * tiles[kGeoL] >= thr * cus) return kGeoL;
  }
  {
    const double r_m = static_cast<double>(ceil_div(tiles[kGeoM], 2 * cus));
    const double r_s = static_cast<double>(ceil_div(tiles[kGeoS], 3 * cus));
    if (0.9 * r_s < r_m) return kGeoS;
  }
  return kGeoM;
}

// One phase launch of a stage kernel in geometry `geo`.
template <int MODE, int PHASE>
static void launch_stage(int geo, int32_t blocks, const StageArgs &a, hipStream_t st) {
  if (geo == kGeoS) {
    hipLaunchKernelGGL((s8_stage_kernel<MODE, PHASE, 128, 128>), dim3(blocks), dim3(GeoS::kThreads), 0, st, a);
    return;
  }
  if (geo == kGeoL)
    hipLaunchKernelGGL((s8_stage_kernel<MODE, PHASE, 256, 256>), dim3(blocks), dim3(GeoL::kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((s8_stage_kernel<MODE, PHASE, 256, 128>), dim3(blocks), dim3(GeoM::kThreads), 0, st, a);
}

// sq_geo: the geometry of the run's square launches (the stage-1 Schatten
// partials are per square tile).  The segments of a phase whose products
// run in different MFMA modes (SMX_S8_MIXED at stages 3-5: an X-space
// class in FP16, a Gram-space class compensated) go to one launch per
// mode.
template <int PHASE>
static int launch_phase(const S8Layout &Lay, const SlotSet &set, int stage, int sq_geo, hipStream_t st, double &flops,
                        const std::vector<int> &ops = {}) {
  const std::vector<Seg> all = launch_segments(Lay, set, PHASE, stage, ops);
  std::vector<int> modes;
  for (const Seg &sg : all) {
    const int m = seg_mode(Lay, PHASE, stage, sg);
    if (std::find(modes.begin(), modes.end(), m) == modes.end()) modes.push_back(m);
  }
  for (const int mode : modes) {
    std::vector<Seg> segs;
    for (const Seg &sg : all)
      if (seg_mode(Lay, PHASE, stage, sg) == mode) segs.push_back(sg);
    StageArgs a{};
    a.L = Lay;
    a.stage = stage;
    a.sq_geo = sq_geo;
    a.mask = g_comp_mask;
    const auto &co = kS8Coefficients[stage - 1];
    a.a = static_cast<float>(co[0]);
    a.b = static_cast<float>(co[1]);
    a.c = static_cast<float>(co[2]);
    a.b_over_c = static_cast<float>(co[1] / co[2]);
    if (static_cast<int>(segs.size()) > kMaxSeg) return fail(SMX_EINVAL, "s8: too many launch segments");
    if (PHASE != kPoly1)
      for (const Seg &sg : segs)
        if (!form_compiled(mode, PHASE, out_form(Lay.mode, g_comp_mask, PHASE, stage, sg.op, Lay.cls[sg.cls].gs != 0)))
          return fail(SMX_EINVAL, "s8: no epilogue for the output form of this product");
    const int geo =
        PHASE == kSquare ? sq_geo : PHASE == kPoly1 ? kGeoM : pick_geo(Lay, PHASE, segs);
    int32_t off = 0;
    a.n_seg = 0;
    for (const Seg &sg : segs) {
      const S8Class &k = Lay.cls[sg.cls];
      const int64_t tpm = PHASE == kPoly1 ? poly_blocks_per_matrix(k) : phase_tiles(k, PHASE, geo, sg.op);
      const int64_t nt = round_up(tpm * (sg.hi - sg.lo), 8);
      a.seg_off[a.n_seg] = off;
      a.seg_cls[a.n_seg] = sg.cls;
      a.seg_op[a.n_seg] = sg.op;
      a.seg_slot0[a.n_seg] = sg.lo;
      a.seg_cnt[a.n_seg] = sg.hi - sg.lo;
      ++a.n_seg;
      off += static_cast<int32_t>(nt);
    }
    a.seg_off[a.n_seg] = off;
    if (off == 0) continue;
    int slot = -1;
    int rc = timing_begin(st, slot, false);
    if (rc) return rc;
    if constexpr (PHASE == kPoly1) {
      if (mode != SMX_S8_FP32)
        hipLaunchKernelGGL(s8_poly1_kernel<SMX_S8_COMP_BF16>, dim3(off), dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL(s8_poly1_kernel<SMX_S8_FP32>, dim3(off), dim3(256), 0, st, a);
      rc = check_launch("s8 stage-1 polynomial");
    } else {
      if (mode == SMX_S8_COMP_BF16) launch_stage<SMX_S8_COMP_BF16, PHASE>(geo, off, a, st);
      else if (mode == kS8CompMix) launch_stage<kS8CompMix, PHASE>(geo, off, a, st);
      else if (mode == kS8HiOnly) launch_stage<kS8HiOnly, PHASE>(geo, off, a, st);
      else if (mode == kS8F16) launch_stage<kS8F16, PHASE>(geo, off, a, st);
      else launch_stage<SMX_S8_FP32, PHASE>(geo, off, a, st);
      rc = check_launch(PHASE == kGram ? "s8 gram" : PHASE == kSquare ? "s8 square" : PHASE == kSym ? "s8 sym"
                                                                                                  : "s8 apply");
    }
    if (rc) return rc;
    const double f = launch_flops(mode, PHASE, stage, geo, Lay, segs);
    flops += f;
    rc = timing_end(slot, st, PHASE, f);
    if (rc) return rc;
  }
  return SMX_OK;
}

// Stage `stage` of the S8 map over the matrices of `set`: one launch per
// phase; Gram-space classes add their two SYM products before the apply
// launch at stages 1, 3 and 4, and an apply of their own after it at stages
// 2 (X2) and 5 (X5).
static int run_s8_set_stage(const S8Layout &Lay, const SlotSet &set, int stage, hipStream_t st, double &flops) {
  auto cnt = [&](int i) { return static_cast<int64_t>(set.hi[i] - set.lo[i]); };
  // The square covers every matrix of the set at every stage, so its
  // geometry (and the stage-1 Schatten partials) is the same for the run.
  const int sq_geo = pick_geo(Lay, kSquare, launch_segments(Lay, set, kSquare, stage, {}));
  bool any_gs = false;
  for (int i = 0; i < Lay.n_classes; ++i) any_gs = any_gs || (Lay.cls[i].gs && cnt(i) > 0);
  int rc = SMX_OK;
  {
    rc = launch_phase<kGram>(Lay, set, stage, sq_geo, st, flops);
    if (!rc) rc = launch_phase<kSquare>(Lay, set, stage, sq_geo, st, flops);
    if (!rc && stage == 1) rc = launch_phase<kPoly1>(Lay, set, stage, sq_geo, st, flops);
    if (!rc && any_gs && gs_sym(stage)) {
      rc = launch_phase<kSym>(Lay, set, stage, sq_geo, st, flops, {kOpPG});
      if (!rc) rc = launch_phase<kSym>(Lay, set, stage, sq_geo, st, flops, {kOpTP});
    }
    if (!rc) rc = launch_phase<kApply>(Lay, set, stage, sq_geo, st, flops, {kOpApplyX, kOpApplyQ});
    if (!rc && any_gs && (stage == 2 || stage == 5))
      rc = launch_phase<kApply>(Lay, set, stage, sq_geo, st, flops, {stage == 2 ? kOpApplyMid : kOpApplyFinal});
  }
  return rc;
}

// The launch chains of an S8 run beyond the first (which runs on the
// caller's stream): further streams of the device (default priority), each
// with the events of its fork and join, created once per device.
constexpr int kChains = 2;
struct ForkStream {
  hipStream_t aux[kChains - 1] = {};
  hipEvent_t fork = nullptr, join[kChains - 1] = {};
};
static std::mutex g_fork_lock;
static ForkStream g_fork[64];

// The caller holds g_fork_lock from the fork record to the join wait: the
// streams and events of a device are shared, so two host threads running
// S8 on one device would otherwise interleave their fork and join records
// (one chain waiting on the other caller's fork).
static int fork_stream(ForkStream *&out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(SMX_ELAUNCH, "s8: no current HIP device");
  ForkStream &f = g_fork[dev];
  if (!f.fork) {
    bool ok = hipEventCreateWithFlags(&f.fork, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; ok && i < kChains - 1; ++i)
      ok = hipStreamCreateWithFlags(&f.aux[i], hipStreamNonBlocking) == hipSuccess &&
           hipEventCreateWithFlags(&f.join[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      f.fork = nullptr;
      return fail(SMX_ELAUNCH, "s8: cannot create the launch chains' streams and events");
    }
  }
  out = &f;
  return SMX_OK;
}

// The whole S8 run.  The matrices are independent until the run ends, so
// they go to kChains launch chains: a class of at least kSplitCount
// matrices is split into kChains near-equal parts, one to each chain, and a
// smaller class whole to the chain with the least work so far (r^2 c per
// matrix, largest classes first).  The first chain runs on the caller's
// stream, the others on further streams forked from it and joined back
// before the run ends: the blocks of one chain's launches fill the CUs
// that the others' leave idle (a launch's tail, tiles that take longer than
// the rest).  The chains do not wait for each other between stages: such
// waits kept them in step but cost about 12 us per stage boundary on each
// chain plus the faster chain's idle time (cfg4 S8 2.35 against 2.25 ms,
// the median over 8 processes of 18 steps each).  The launch recorder gets
// one record for the run, on the caller's stream.
constexpr int kSplitCount = 2 * kChains;

int run_s8_stages(const S8Layout &Lay, hipStream_t st) {
  int slot = -1;
  int rc = timing_begin(st, slot, true);
  if (rc) return rc;
  std::vector<int> order;
  for (int i = 0; i < Lay.n_classes; ++i)
    if (Lay.cls[i].count) order.push_back(i);
  auto work = [&](int i, int n) {
    const S8Class &k = Lay.cls[i];
    return static_cast<double>(n) * k.rp * k.rp * k.cp;
  };
  std::stable_sort(order.begin(), order.end(),
                   [&](int x, int y) { return work(x, Lay.cls[x].count) > work(y, Lay.cls[y].count); });
  SlotSet set[kChains];
  double load[kChains] = {};
  for (int i : order) {
    const int c = Lay.cls[i].count;
    if (c >= kSplitCount) {
      int lo = 0;
      for (int t = 0; t < kChains; ++t) {
        const int n = c / kChains + (t < c % kChains ? 1 : 0);
        set[t].lo[i] = lo;
        set[t].hi[i] = lo + n;
        load[t] += work(i, n);
        lo += n;
      }
    } else {
      int t = 0;
      for (int u = 1; u < kChains; ++u)
        if (load[u] < load[t]) t = u;
      set[t].lo[i] = 0;
      set[t].hi[i] = c;
      load[t] += work(i, c);
    }
  }
  int chains = 0;  // chains with work (the first always has some)
  for (int t = 0; t < kChains; ++t)
    if (!set[t].empty()) chains = t + 1;
  double flops = 0.0;
  if (chains <= 1) {
    for (int stage = 1; stage <= 5 && !rc; ++stage) rc = run_s8_set_stage(Lay, set[0], stage, st, flops);
  } else {
    // Only enqueues happen under the lock.
    std::lock_guard<std::mutex> lock(g_fork_lock);
    ForkStream *f = nullptr;
    rc = fork_stream(f);
    if (!rc && hipEventRecord(f->fork, st) != hipSuccess) rc = fail(SMX_ELAUNCH, "s8: fork of the launch chains failed");
    for (int t = 1; t < chains && !rc; ++t)
      if (hipStreamWaitEvent(f->aux[t - 1], f->fork, 0) != hipSuccess)
        rc = fail(SMX_ELAUNCH, "s8: fork of the launch chains failed");
    // The chains are enqueued a stage at a time each, so that every chain
    // starts while the host is still enqueuing the others.
    for (int stage = 1; stage <= 5 && !rc; ++stage)
      for (int t = chains - 1; t >= 0 && !rc; --t)
        if (!set[t].empty()) rc = run_s8_set_stage(Lay, set[t], stage, t ? f->aux[t - 1] : st, flops);
    // Join even after a failed launch, so the caller's stream never runs
    // ahead of work already on the other streams.
    for (int t = 1; f && t < chains; ++t)
      if ((hipEventRecord(f->join[t - 1], f->aux[t - 1]) != hipSuccess ||
           hipStreamWaitEvent(st, f->join[t - 1], 0) != hipSuccess) && !rc)
        rc = fail(SMX_ELAUNCH, "s8: join of the launch chains failed");
  }
  if (rc) return rc;
  return timing_end(slot, st, kSpan, flops);
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
    C.tiles_s = static_cast<int32_t>(C.rp / kSymTile);
    C.parts = static_cast<int32_t>(2 * C.cp);
    C.gs = C.cp > C.rp ? 1 : 0;
    const size_t xs = static_cast<size_t>(C.count) * C.rp * C.cp * sizeof(float);
    const size_t gs = static_cast<size_t>(C.count) * C.rp * C.rp * sizeof(float);
    C.x0 = reinterpret_cast<float *>(take(xs));
    C.x1 = reinterpret_cast<float *>(take(xs));
    C.xf = reinterpret_cast<float *>(take(static_cast<size_t>(C.n_flip) * C.rp * C.cp * sizeof(float)));
    C.g = reinterpret_cast<float *>(take(gs));
    C.p = reinterpret_cast<float *>(take(gs));
    C.t = C.gs ? reinterpret_cast<float *>(take(gs)) : nullptr;
    C.qa = C.gs ? reinterpret_cast<float *>(take(gs)) : nullptr;
    C.qb = C.gs ? reinterpret_cast<float *>(take(gs)) : nullptr;
    C.u = reinterpret_cast<float *>(take(static_cast<size_t>(C.count) * C.cp * sizeof(float)));
    C.fro = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * C.parts * sizeof(double)));
    C.mb = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * C.parts * sizeof(double)));
    C.sch = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * sym_tiles(C.tiles_s) * sizeof(double)));
    C.cst = reinterpret_cast<double *>(take(static_cast<size_t>(C.count) * kCst * sizeof(double)));
    C.colv = reinterpret_cast<const float **>(take(static_cast<size_t>(C.count) * 2 * sizeof(float *)));
    C.mrp = reinterpret_cast<float *>(take(static_cast<size_t>(C.count) * 3 * (C.rp * C.cp / kStripT) * sizeof(float)));
  }
  plan.bytes = off;
  return true;
}

}  // namespace smx

using smx::g_timing;

extern "C" int smx_s8_comp_stages(int32_t k) {
  SMX_REQUIRE(k >= 0 && k <= 5, SMX_EINVAL, "s8 compensated stages: k must be in [0, 5]");
  int prev = 0;  // leading compensated stages of the previous mask
  while (prev < 5 && ((smx::g_comp_mask >> prev) & 1)) ++prev;
  smx::g_comp_mask = (1 << k) - 1;
  return prev;
}

extern "C" int smx_s8_comp_mask(int32_t mask) {
  SMX_REQUIRE(mask >= 0 && mask <= 0x1f, SMX_EINVAL, "s8 compensation mask: must be in [0, 0x1f]");
  const int prev = smx::g_comp_mask;
  smx::g_comp_mask = mask;
  return prev;
}

extern "C" int smx_s8_tile_geometry(int32_t policy) {
  SMX_REQUIRE(policy >= 0 && policy <= 2, SMX_EINVAL, "s8 tile geometry: policy must be 0, 1 or 2");
  const int prev = smx::g_tile_policy;
  smx::g_tile_policy = policy;
  return prev;
}

extern "C" int smx_s8_timing(int32_t enable) {
  SMX_REQUIRE(enable >= 0 && enable <= 2, SMX_EINVAL, "s8 timing: enable must be 0, 1 or 2");
  g_timing.level = enable;
  if (enable) g_timing.used = 0;
  return SMX_OK;
}

extern "C" int32_t smx_s8_timing_read(float *ms, int32_t *phase, double *flops, int32_t capacity) {
  SMX_REQUIRE(capacity >= 0, SMX_EINVAL, "s8 timing: negative capacity");
  const int32_t n = static_cast<int32_t>(std::min<size_t>(g_timing.used, static_cast<size_t>(capacity)));
  for (int32_t i = 0; i < n; ++i) {
    SMX_REQUIRE(g_timing.phase[i] >= 0, SMX_EINVAL, "s8 timing: a record is still open");
    if (hipEventSynchronize(g_timing.stop[i]) != hipSuccess)
      return smx::fail(SMX_ELAUNCH, "s8 timing: hipEventSynchronize failed");
    float t = 0.f;
    if (hipEventElapsedTime(&t, g_timing.start[i], g_timing.stop[i]) != hipSuccess)
      return smx::fail(SMX_ELAUNCH, "s8 timing: hipEventElapsedTime failed");
    if (ms) ms[i] = t;
    if (phase) phase[i] = g_timing.phase[i];
    if (flops) flops[i] = g_timing.flops[i];
  }
  return n;
}
