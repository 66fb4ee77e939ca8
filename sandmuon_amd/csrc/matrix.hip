// Matrix update around the S8 map (parameter layout, W is rows x cols):
//
//   whiten  (sandmuon/optimizer.py:244-248, :249-264, :290-296, rank1_whiten
//            :38-45): m' = b m + (1-b) g;  S = b m' + (1-b) g;
//            V = (D_b S D_a)(I + kappa z z^T)
//   mapback (rank1_mapback :48-60, _graft_direction :63-66, update :314-315):
//            U = D_b Q (I + kappa z z^T) D_a;
//            W -= lr * sqrt(rows) * U / max(||U||_F, FLT_MIN)
//
// In parameter layout the A factor always acts on columns (input channels)
// and B on rows, whichever orientation the S8 map uses; the whiten kernels
// write the oriented iterate X (r x c, r <= c).
//
// Launch structure.  A small prep launch copies the host's per-matrix job
// records into a table in the workspace; every row kernel then covers all
// matrices of the call in one launch (up to kLaunchJobs), finding its job
// from a table of first blocks in its kernel arguments.  A row is handled
// by `wpr` waves (1, 2 or 4, so that a lane holds at most kMaxSlices float4
// of it), a 256-thread block by 4 / wpr rows.  Sums over a matrix (||V||^2
// for the S8 normalisation, ||U||^2 for the graft) are per-block FP64
// partials, added in a fixed order: ||V||^2 by a one-block-per-matrix
// launch after the whiten, ||U||^2 (a few dozen partials) by every block of
// mapback_apply for itself.  (Adding them in the matrix's last block
// instead needs a device-scope release per block, which on this part
// writes back the L2: that made the whiten launch six times slower.)
//
// whiten        two passes per row: momentum update, u_i = b_i sum_j S_ij a_j z_j
//               and the row's ||V_i||^2 in closed form
//               (||V_i||^2 = b_i^2 sum_j (S_ij a_j)^2 + (2 kappa + kappa^2 |z|^2) u_i^2);
//               then V stored to X (S a and z of the pass kept in registers).
// whiten_flip   the same for a transposed parameter, 16 rows per block (one
//               16-element K group of the oriented iterate), V written
//               transposed through LDS.
// mapback_norm  u_i = sum_j Q_ij z_j and ||U_i||^2 in closed form, from the
//               row-sum partials that the S8 map's stage-5 apply leaves
//               beside its result (Q itself is read once, by the apply).
// mapback_apply W -= lr * scale * U.
#include "s8.h"

#include <algorithm>
#include <climits>
#include <cfloat>
#include <cmath>
#include <memory>
#include <vector>

namespace smx {

constexpr int kRowThreads = 256;   // row kernels: 4 waves
constexpr int kMaxSlices = 3;      // float4 per lane per row kept in registers
constexpr int kKeptSlices = 8;     // whiten_rows_kept: float4 of y per lane (4 waves: 8192 columns)
constexpr int kKeptBatch = 8;      // whiten_rows_kept: slices' loads in flight together (all: 1756 us per
                                   // cfg5 launch at 161 VGPRs, against 1881 with 4 and 1963 with 2)
constexpr int kFlipRows = 16;      // transposed whiten: rows per block (one K group)
constexpr int kFlipThreads = 64 * kFlipRows;
constexpr int kFlipChunk = 256 * kMaxSlices;  // transposed whiten: columns per LDS chunk

struct MatJob {
  smx_matrix_desc d;
  float *x;          // whiten: the oriented iterate, a tiled S8 operand ([prow_pad][pcol_pad], or
                     // for a transposed parameter [pcol_pad][prow_pad])
  const float *q;    // mapback: the S8 result in parameter layout ([prow_pad][pcol_pad])
  float *u;          // [prow_pad] rank-one row coefficients
  double *fro;       // whiten per-block partials of ||V||^2
  double *mb;        // mapback per-block partials of ||U||^2
  double *cst;       // kCst per-matrix scalars
  const float **colv;  // the S8 class's slot entry for (inv_col, z)
  const float *mrp;  // stage-5 row-sum partials (3 arrays of mrp_size) [strips][prow_pad]
  int64_t mrp_size;
  int32_t prow_pad, pcol_pad;
  int32_t planes;    // whiten: X as interleaved BF16 hi/lo (comp mode)
  int32_t wpr;       // waves per row
  int32_t slices;    // float4 per lane over a row: ceil(cols / 4 / (64 wpr))
  int32_t cvec;      // float4 column vectors: cols % 4 == 0, inv_col and z 16-byte aligned
  int32_t wvec;      // whiten float4 path: cvec, F32 gradient, gradient and momentum aligned
  int32_t mvec;      // mapback_apply float4 path: cvec, F32 parameter, aligned
  int32_t strips;    // row-sum partials per parameter row
  int32_t flip;      // a transposed parameter
};

constexpr int kLaunchJobs = 128;
struct JobRange {
  const MatJob *jobs;          // the launch's first job in the table
  int32_t start[kLaunchJobs];  // first block of each job; INT32_MAX past the last
  int32_t n;
};
static_assert(sizeof(JobRange) <= 4000, "JobRange is passed by value in the kernel arguments");

// The job of block b: the number of jobs after the first whose first block
// is <= b (start[] ascends), 16 independent compares at a time.
__device__ __forceinline__ int find_job(const JobRange &r, int b) {
  int k = 0;
  for (int c = 0; c < kLaunchJobs; c += 16) {
    if (r.start[c] > b) break;
#pragma unroll
    for (int t = 0; t < 16; ++t) k += (c + t > 0 && b >= r.start[c + t]) ? 1 : 0;
  }
  return k;
}

// The job as the row kernels hold it, with every pointer in the global
// address space (SMX_GLOBAL): a pointer read from memory (the job table) is
// a generic pointer to the compiler, and accesses through it would be FLAT
// instructions, which also count against the LDS / scalar wait counter and
// address with a 64-bit VGPR pair per access.
struct DevDesc {
  SMX_GLOBAL void *param;
  const SMX_GLOBAL void *grad;
  SMX_GLOBAL float *momentum;
  const SMX_GLOBAL float *inv_row, *inv_col, *z, *kappa;
  int64_t rows, cols;
  double lr, momentum_beta;
  int32_t grad_dtype, param_dtype;
};
struct DevJob {
  DevDesc d;
  SMX_GLOBAL float *x;
  const SMX_GLOBAL float *q;
  SMX_GLOBAL float *u;
  SMX_GLOBAL double *fro, *mb, *cst;
  const SMX_GLOBAL float *mrp;
  int64_t mrp_size;
  int64_t prow_pad, pcol_pad;
  int32_t planes, wpr, slices, cvec, wvec, mvec, strips, flip;
};

// Copied from the table once, before any store of the kernel, so that its
// fields stay in registers.
__device__ __forceinline__ DevJob load_job(const MatJob *table, int jid) {
  const MatJob J = table[jid];
  DevJob D;
  D.d.param = (SMX_GLOBAL void *)J.d.param;
  D.d.grad = (const SMX_GLOBAL void *)J.d.grad;
  D.d.momentum = (SMX_GLOBAL float *)J.d.momentum;
  D.d.inv_row = (const SMX_GLOBAL float *)J.d.inv_row;
  D.d.inv_col = (const SMX_GLOBAL float *)J.d.inv_col;
  D.d.z = (const SMX_GLOBAL float *)J.d.z;
  D.d.kappa = (const SMX_GLOBAL float *)J.d.kappa;
  D.d.rows = J.d.rows;
  D.d.cols = J.d.cols;
  D.d.lr = J.d.lr;
  D.d.momentum_beta = J.d.momentum_beta;
  D.d.grad_dtype = J.d.grad_dtype;
  D.d.param_dtype = J.d.param_dtype;
  D.x = (SMX_GLOBAL float *)J.x;
  D.q = (const SMX_GLOBAL float *)J.q;
  D.u = (SMX_GLOBAL float *)J.u;
  D.fro = (SMX_GLOBAL double *)J.fro;
  D.mb = (SMX_GLOBAL double *)J.mb;
  D.cst = (SMX_GLOBAL double *)J.cst;
  D.mrp = (const SMX_GLOBAL float *)J.mrp;
  D.mrp_size = J.mrp_size;
  D.strips = J.strips;
  D.prow_pad = J.prow_pad;
  D.pcol_pad = J.pcol_pad;
  D.planes = J.planes;
  D.wpr = J.wpr;
  D.slices = J.slices;
  D.cvec = J.cvec;
  D.wvec = J.wvec;
  D.mvec = J.mvec;
  D.flip = J.flip;
  return D;
}

template <typename P>
__device__ __forceinline__ float4 ld4(P p, int q) { return ((const float4 *)p)[q]; }
template <typename P>
__device__ __forceinline__ void st4(P p, int q, float4 v) { ((float4 *)p)[q] = v; }

__device__ __forceinline__ float load_grad(const void *g, int dt, int64_t i) {
  if (dt == SMX_F32) return static_cast<const float *>(g)[i];
  if (dt == SMX_BF16) return load_elem<SMX_BF16>(g, i);
  return load_elem<SMX_F16>(g, i);
}

// --------------------------------------------------------------- prep ---
constexpr int kPrepBatch = 19;
struct PrepPack {
  MatJob j[kPrepBatch];
  MatJob *table;  // destination of j[0]
  int32_t n;
};
static_assert(sizeof(PrepPack) <= 4000, "PrepPack is passed by value in the kernel arguments");
static_assert(sizeof(MatJob) % 4 == 0, "the prep kernel copies jobs as 32-bit words");

// One 64-thread block per job: the record into the table, and the slot's
// column vectors for the stage-5 row sums of the S8 map.
__global__ void __launch_bounds__(64) matrix_prep_kernel(PrepPack pack) {
  const MatJob &J = pack.j[blockIdx.x];
  const uint32_t *src = reinterpret_cast<const uint32_t *>(&J);
  uint32_t *dst = reinterpret_cast<uint32_t *>(pack.table + blockIdx.x);
  for (int k = threadIdx.x; k < static_cast<int>(sizeof(MatJob) / 4); k += 64) dst[k] = src[k];
  if (threadIdx.x == 0) {
    J.colv[0] = J.d.inv_col;
    J.colv[1] = J.d.z;
  }
}

// Blocks per matrix of the row kernels (host MatJob or device DevJob).
// Row groups (4 / wpr rows, one per wave group) per whiten block: a job
// whose row fits the lanes' registers takes kWhitenGroups of them in turn,
// the next group's loads in flight while the current one is reduced and
// stored; the other jobs take one.  One group per block is the fastest on
// the cfg4 shapes (more blocks, each issuing all its loads at once): 139 us
// per step against 147 with two groups and 153 with four.
constexpr int kWhitenGroups = 1;
template <typename Job>
__host__ __device__ inline bool whiten_pipelined(const Job &j) {
  return !j.flip && j.wvec && j.slices <= kMaxSlices;
}
template <typename Job>
__host__ __device__ inline int64_t whiten_blocks(const Job &j) {
  return j.flip ? j.prow_pad / kFlipRows : j.prow_pad / (4 / j.wpr) / (whiten_pipelined(j) ? kWhitenGroups : 1);
}
template <typename Job>
__host__ __device__ inline int64_t mapback_blocks(const Job &j) { return ceil_div(j.d.rows, 4 / j.wpr); }
template <typename Job>
__host__ __device__ inline int64_t norm_blocks(const Job &j) { return ceil_div(j.d.rows, kRowThreads / 4); }

// One block per job, after the whiten: the FP64 sums of the job's
// per-block partials (thread t takes partials t, t + 256, ..., then a
// fixed-order block sum), the rank-one constants sum z^2 and sum (a z)^2,
// and ||V||^2 = sum b^2 |S a|^2 + (2 kappa + kappa^2 sum z^2) sum u^2 from the
// whiten's two partials.
constexpr int kTotalThreads = 256;
constexpr int kTotalUnroll = 12;  // column loads in flight per thread (3072 columns in one pass)

// Block-wide sums of N values at once (fixed order: wave sums, then the
// waves in order); every thread receives them.
template <int N>
__device__ __forceinline__ void block_sums(double (&v)[N], double (*scratch)[kTotalThreads / 64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = wave_sum(v[k]);
  if (lane == 0)
#pragma unroll
    for (int k = 0; k < N; ++k) scratch[k][wave] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kTotalThreads / 64; ++w) t += scratch[k][w];
    v[k] = t;
  }
}

__global__ void __launch_bounds__(kTotalThreads) matrix_total_kernel(const MatJob *jobs) {
  __shared__ double scratch[4][kTotalThreads / 64];
  const DevJob J = load_job(jobs, blockIdx.x);
  const DevDesc &d = J.d;
  const SMX_GLOBAL double *parts = J.fro;
  const int64_t nblk = whiten_blocks(J);
  const bool r1 = d.z != nullptr;  // uniform per block
  // Every load of the thread first (partials, then z and a), then the sums.
  double s[4] = {0.0, 0.0, 0.0, 0.0};  // partials (kind 0, kind 1), sum z^2, sum (a z)^2
  for (int64_t k0 = threadIdx.x; k0 < nblk; k0 += kTotalThreads * 4) {
    double v[2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t k = k0 + kTotalThreads * u;
      v[0][u] = k < nblk ? parts[k] : 0.0;
      v[1][u] = k < nblk ? parts[nblk + k] : 0.0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s[0] += v[0][u];
      s[1] += v[1][u];
    }
  }
  if (r1) {
    for (int64_t j0 = threadIdx.x; j0 < d.cols; j0 += kTotalThreads * kTotalUnroll) {
      float z[kTotalUnroll], a[kTotalUnroll];
#pragma unroll
      for (int u = 0; u < kTotalUnroll; ++u) {
        const int64_t j = j0 + kTotalThreads * u;
        z[u] = j < d.cols ? d.z[j] : 0.f;
        a[u] = j < d.cols ? d.inv_col[j] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kTotalUnroll; ++u) {
        const double zd = z[u], t = static_cast<double>(a[u]) * zd;
        s[2] += zd * zd;
        s[3] += t * t;
      }
    }
  }
  block_sums<4>(s, scratch);
  if (threadIdx.x != 0) return;
  // s[0] = sum b^2 |S a|^2, s[1] = sum u^2
  const double kappa = r1 ? d.kappa[0] : 0.0;
  J.cst[kCstZZ] = s[2];
  J.cst[kCstAZ] = s[3];
  J.cst[kCstFro] = s[0] + (2.0 * kappa + kappa * kappa * s[2]) * s[1];
}

// ------------------------------------------------------------- whiten ---
// Row geometry of a block: 4 / wpr rows, wave w on row w / wpr, covering
// float4 wr * 64 + lane + 64 wpr t (wr = w % wpr, slice t) of it.
// The row and the wave's place in it are wave-uniform (scalar registers,
// so row base addresses are too); offsets within a row are 32-bit.
struct RowPos {
  int64_t i;    // parameter row
  int q0;       // this lane's first float4 of the row
  int span;     // float4 between a lane's slices
  int wr, rib;  // wave within the row, row within the block
};
__device__ __forceinline__ RowPos row_pos(const DevJob &J, int blk) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = J.wpr;
  RowPos p;
  p.rib = wave / W;
  p.wr = wave % W;
  p.i = static_cast<int64_t>(blk) * (4 / W) + p.rib;
  p.q0 = p.wr * 64 + lane;
  p.span = 64 * W;
  return p;
}

// Sums of a row over its waves (the same value in every wave of the row):
// red[wave][k] holds each wave's partials; fixed order over the waves.
template <int N>
__device__ __forceinline__ void row_sums(double (&v)[N], double (*red)[4], const RowPos &p, int W) {
  if (W == 1) return;  // uniform per block
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int k = 0; k < N; ++k) red[wave][k] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) {
    double s = 0.0;
    for (int w = 0; w < W; ++w) s += red[p.rib * W + w][k];
    v[k] = s;
  }
}

// The block's partials of the rows' b^2 |S a|^2 and u^2 (its rows in
// order) -> parts[blk] and parts[nblk + blk].
__device__ __forceinline__ void block_part(const DevJob &J, double vy, double vu, const RowPos &p, int blk, int nblk,
                                           SMX_GLOBAL double *parts, double (*rp)[4]) {
  if ((threadIdx.x & 63) == 0 && p.wr == 0) {
    rp[0][p.rib] = vy;
    rp[1][p.rib] = vu;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    double t = 0.0;
    for (int r = 0; r < 4 / J.wpr; ++r) t += rp[threadIdx.x][r];
    parts[threadIdx.x * nblk + blk] = t;
  }
}

// Operand-form bytes of a row group staged in LDS before they go to the
// tiled X: rows of up to 768 columns four at a time (up to 1536 two, up to
// 3072 one at a time), each row's bytes in row-major operand form at a pitch
// of 64 bytes more than the row, so that the 16 lanes reading 16-byte
// chunks of 4 rows hit distinct banks.
constexpr int kWhitenStageBytes = 4 * (768 * 4 + 64);

// The 16 bytes a lane of put_operand4_paired's lane pairs writes, and their
// byte offset in the row: FP32 the lane's four values; BF16 planes the
// pair's eight hi values (even lane) or lo values (odd lane).  col = the
// lane's first column (a multiple of 4).
__device__ __forceinline__ u32x4v operand_chunk(const float (&v)[4], bool planes, int64_t col, int64_t &off) {
  if (!planes) {
    off = 4 * col;
    return u32x4v{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  }
  const uint32_t h0 = bf16_bits(v[0]) | (uint32_t(bf16_bits(v[1])) << 16);
  const uint32_t h1 = bf16_bits(v[2]) | (uint32_t(bf16_bits(v[3])) << 16);
  const uint32_t l0 = bf16_lo_bits(v[0]) | (uint32_t(bf16_lo_bits(v[1])) << 16);
  const uint32_t l1 = bf16_lo_bits(v[2]) | (uint32_t(bf16_lo_bits(v[3])) << 16);
  const bool odd = (threadIdx.x & 1) != 0;
  const uint32_t x0 = dpp_mov<0xB1>(odd ? h0 : l0), x1 = dpp_mov<0xB1>(odd ? h1 : l1);
  off = 2 * (plane_hi(col) + (odd ? 16 - 4 : 0));
  return odd ? u32x4v{x0, x1, l0, l1} : u32x4v{h0, h1, x0, x1};
}

// Rows whose float4 fit kMaxSlices per lane (the float4 path): the block
// takes kWhitenGroups row groups in turn.  a and z are the same for every
// row a lane sees and are loaded once; the g and m' of group k + 1 are
// loaded while group k is reduced and stored.  The group's X goes through
// LDS (`xs`, one buffer per group parity) and is stored as the rows'
// consecutive 64-byte runs of each K group: with two or four rows per group
// whole 128-byte lines of the tiled X, where each wave's own row would leave
// half lines.
template <bool R1>
__device__ __forceinline__ void whiten_rows_pipelined(const DevJob &J, int blk, double (*red)[4][4],
                                                      double (*rp)[4], char (*xs)[kWhitenStageBytes]) {
  const DevDesc &d = J.d;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = J.wpr, rib = wave / W, wr = wave % W, rpg = 4 / W;
  const int q0 = wr * 64 + lane, span = 64 * W;
  const int n4 = static_cast<int>(d.cols / 4), pc4 = static_cast<int>(J.pcol_pad / 4);
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const float kappa = R1 ? d.kappa[0] : 0.f;
  const bool planes = J.planes != 0;
  const int64_t row0 = static_cast<int64_t>(blk) * kWhitenGroups * rpg + rib;
  const int pitch = 4 * static_cast<int>(J.pcol_pad) + 64;
  float4 a[kMaxSlices], z[kMaxSlices];
  float bb[kWhitenGroups];
#pragma unroll
  for (int t = 0; t < kMaxSlices; ++t) {
    const int q = q0 + span * t;
    a[t] = z[t] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < J.slices && q < n4) {
      a[t] = ld4(d.inv_col, q);
      if constexpr (R1) z[t] = ld4(d.z, q);
    }
  }
#pragma unroll
  for (int k = 0; k < kWhitenGroups; ++k) {
    const int64_t i = row0 + k * rpg;
    bb[k] = i < d.rows ? d.inv_row[i] : 0.f;
  }
  float4 g[2][kMaxSlices], m[2][kMaxSlices];
  auto load_rows = [&](int k, float4 (&gg)[kMaxSlices], float4 (&mm)[kMaxSlices]) {
    const int64_t i = row0 + k * rpg;
    if (i >= d.rows) return;
    const SMX_GLOBAL float *grow = (const SMX_GLOBAL float *)d.grad + i * d.cols;
    const SMX_GLOBAL float *mrow = d.momentum + i * d.cols;
#pragma unroll
    for (int t = 0; t < kMaxSlices; ++t) {
      const int q = q0 + span * t;
      if (t < J.slices && q < n4) {
        gg[t] = ld4(grow, q);
        mm[t] = ld4(mrow, q);
      }
    }
  };
  load_rows(0, g[0], m[0]);
  double vy = 0.0, vu = 0.0;  // the b^2 |S a|^2 and u^2 of the wave group's rows, in order
#pragma unroll
  for (int k = 0; k < kWhitenGroups; ++k) {
    const int c = k & 1;
    if (k + 1 < kWhitenGroups) load_rows(k + 1, g[c ^ 1], m[c ^ 1]);
    const int64_t i = row0 + k * rpg;
    const bool live = i < d.rows;
    SMX_GLOBAL float *mrow = d.momentum + i * d.cols;
    float y2 = 0.f, yz = 0.f;
    float4 y[kMaxSlices];
#pragma unroll
    for (int t = 0; t < kMaxSlices; ++t) {
      const int q = q0 + span * t;
      y[t] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (live && t < J.slices && q < n4) {
        const float4 gg = g[c][t], aa = a[t];
        float4 mm = m[c][t];
        mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
        mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
        st4(mrow, q, mm);
        float4 yy;
        yy.x = fmaf(mm.x, beta, gg.x * omb) * aa.x; yy.y = fmaf(mm.y, beta, gg.y * omb) * aa.y;
        yy.z = fmaf(mm.z, beta, gg.z * omb) * aa.z; yy.w = fmaf(mm.w, beta, gg.w * omb) * aa.w;
        y2 = fmaf(yy.x, yy.x, fmaf(yy.y, yy.y, fmaf(yy.z, yy.z, fmaf(yy.w, yy.w, y2))));
        if constexpr (R1) {
          const float4 zz = z[t];
          yz = fmaf(yy.x, zz.x, fmaf(yy.y, zz.y, fmaf(yy.z, zz.z, fmaf(yy.w, zz.w, yz))));
        }
        y[t] = yy;
      }
    }
    double v[2] = {static_cast<double>(wave_sum(y2)), static_cast<double>(wave_sum(yz))};
    if (W > 1) {  // uniform per block; red[k & 1] alternates, so one barrier per group suffices
      if (lane == 0) {
        red[k & 1][wave][0] = v[0];
        red[k & 1][wave][1] = v[1];
      }
      __syncthreads();
      v[0] = v[1] = 0.0;
      for (int w = 0; w < W; ++w) {
        v[0] += red[k & 1][rib * W + w][0];
        v[1] += red[k & 1][rib * W + w][1];
      }
    }
    const float b = bb[k];
    float ku = 0.f;
    if (live) {
      const double bd = b;
      const double u = bd * v[1];
      ku = R1 ? kappa * static_cast<float>(u) : 0.f;
      vy += bd * bd * v[0];
      vu += u * u;
      if (lane == 0 && wr == 0) J.u[i] = static_cast<float>(u);
    }
    // V_ij = b_i y_j + kappa u_i z_j, zeros in padding rows and columns
    // (the S8 operand: tiled, row i's K group 4 q / 16 in its piece)
#pragma unroll
    for (int t = 0; t < kMaxSlices; ++t) {
      const int q = q0 + span * t;
      if (t < J.slices && q < pc4) {
        float w[4] = {0.f, 0.f, 0.f, 0.f};
        if (live && q < n4) {
          const float4 yy = y[t], zz = z[t];
          w[0] = fmaf(ku, zz.x, b * yy.x); w[1] = fmaf(ku, zz.y, b * yy.y);
          w[2] = fmaf(ku, zz.z, b * yy.z); w[3] = fmaf(ku, zz.w, b * yy.w);
        }
        // pc4 is a multiple of 4 and q0 + span t steps by lanes, so both
        // lanes of a pair are inside the row or both outside
        int64_t off;
        const u32x4v c = operand_chunk(w, planes, 4 * static_cast<int64_t>(q), off);
        *reinterpret_cast<u32x4v *>(xs[k & 1] + rib * pitch + off) = c;
      }
    }
    {
      // (one barrier per group: a buffer is rewritten two groups later,
      // after every thread has passed the next group's barrier)
      __syncthreads();
      // The group's rows lie in one 16-row block of the tiled X: K group g
      // at 1 KB g from the group's first run, row r 64 r bytes further.
      const int64_t first = row0 - rib + k * rpg;
      SMX_GLOBAL char *gp = reinterpret_cast<SMX_GLOBAL char *>(J.x) + 4 * tiled_index(first, 0, J.pcol_pad);
      const int lg = W == 1 ? 2 : W == 2 ? 1 : 0;  // log2 rpg
      for (int ci = threadIdx.x; ci < (pc4 << lg); ci += kRowThreads) {
        const int c = ci & 3, r = (ci >> 2) & (rpg - 1), g = ci >> (2 + lg);
        const u32x4v v = *reinterpret_cast<const u32x4v *>(xs[k & 1] + r * pitch + 64 * g + 16 * c);
        *reinterpret_cast<SMX_GLOBAL u32x4v *>(gp + (1024 * g + 64 * r + 16 * c)) = v;
      }
    }
  }
  if (lane == 0 && wr == 0) {
    rp[0][rib] = vy;
    rp[1][rib] = vu;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    double t = 0.0;
    for (int r = 0; r < rpg; ++r) t += rp[threadIdx.x][r];
    J.fro[threadIdx.x * whiten_blocks(J) + blk] = t;
  }
}

// The other rows (wide rows in passes of kMaxSlices float4, or a
// gradient without the float4 path): one row group per block.
template <bool R1>
__device__ __forceinline__ void whiten_rows_single(const DevJob &J, int blk, double (*red)[4], double (*rp)[4]) {
  const DevDesc &d = J.d;
  const RowPos p = row_pos(J, blk);
  const int lane = threadIdx.x & 63;
  const bool live = p.i < d.rows;
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const float kappa = R1 ? d.kappa[0] : 0.f;
  const bool planes = J.planes != 0;
  SMX_GLOBAL float *mrow = live ? d.momentum + p.i * d.cols : nullptr;
  const int pc4 = static_cast<int>(J.pcol_pad / 4);

  // ---- pass 1: m' (stored), y = S a of the lane's columns, and the row's
  // sum y^2 and y.z.
  float y2 = 0.f, yz = 0.f;
  if (J.wvec) {
    const int n4 = static_cast<int>(d.cols / 4);
    const SMX_GLOBAL float *grow = live ? (const SMX_GLOBAL float *)d.grad + p.i * d.cols : nullptr;
    // Slices [t0, t0 + kMaxSlices) of the row.
    auto pass1 = [&](int t0) {
      float4 g[kMaxSlices], m[kMaxSlices], a[kMaxSlices], z[kMaxSlices];
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int q = p.q0 + p.span * (t0 + t);
        if (q < n4) {
          a[t] = ld4(d.inv_col, q);
          if constexpr (R1) z[t] = ld4(d.z, q);
          if (live) {
            g[t] = ld4(grow, q);
            m[t] = ld4(mrow, q);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int q = p.q0 + p.span * (t0 + t);
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f), zz4 = y;
        if (q < n4) {
          const float4 aa = a[t];
          if constexpr (R1) zz4 = z[t];
          if (live) {
            float4 mm = m[t];
            const float4 gg = g[t];
            mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
            mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
            st4(mrow, q, mm);
            y.x = fmaf(mm.x, beta, gg.x * omb) * aa.x; y.y = fmaf(mm.y, beta, gg.y * omb) * aa.y;
            y.z = fmaf(mm.z, beta, gg.z * omb) * aa.z; y.w = fmaf(mm.w, beta, gg.w * omb) * aa.w;
            y2 = fmaf(y.x, y.x, fmaf(y.y, y.y, fmaf(y.z, y.z, fmaf(y.w, y.w, y2))));
            if constexpr (R1) yz = fmaf(y.x, zz4.x, fmaf(y.y, zz4.y, fmaf(y.z, zz4.z, fmaf(y.w, zz4.w, yz))));
          }
        }
      }
    };
    for (int t0 = 0; t0 < J.slices; t0 += kMaxSlices) pass1(t0);
  } else {
    for (int j = p.q0; j < d.cols; j += p.span) {
      const float a = d.inv_col[j];
      float zj = 0.f;
      if constexpr (R1) zj = d.z[j];
      if (live) {
        const float g = load_grad((const void *)d.grad, d.grad_dtype, p.i * d.cols + j);
        const float m = fmaf(mrow[j], beta, g * omb);
        mrow[j] = m;
        const float y = fmaf(m, beta, g * omb) * a;
        y2 = fmaf(y, y, y2);
        if constexpr (R1) yz = fmaf(y, zj, yz);
      }
    }
  }
  double v[2] = {static_cast<double>(wave_sum(y2)), static_cast<double>(wave_sum(yz))};
  row_sums<2>(v, red, p, J.wpr);
  double vy = 0.0, vu = 0.0;  // the row's b^2 |S a|^2 and u^2
  float b = 0.f, ku = 0.f;
  if (live) {
    const double bd = d.inv_row[p.i];
    const double u = bd * v[1];
    b = d.inv_row[p.i];
    ku = R1 ? kappa * static_cast<float>(u) : 0.f;
    vy = bd * bd * v[0];
    vu = u * u;
    if (lane == 0 && p.wr == 0) J.u[p.i] = static_cast<float>(u);
  }

  // ---- pass 2: V_ij = b_i y_j + kappa u_i z_j (zeros in padding rows and
  // columns) in operand form.
  if (J.wvec) {
    // Wide rows: m' and g again (the row was just read and written).
    const int n4 = static_cast<int>(d.cols / 4);
    const SMX_GLOBAL float *grow = live ? (const SMX_GLOBAL float *)d.grad + p.i * d.cols : nullptr;
    for (int q0 = p.q0; q0 < pc4; q0 += p.span * kMaxSlices) {
      float4 g[kMaxSlices], m[kMaxSlices], a[kMaxSlices], z[kMaxSlices];
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int q = q0 + p.span * t;
        if (live && q < n4) {
          g[t] = ld4(grow, q);
          m[t] = ld4(mrow, q);
          a[t] = ld4(d.inv_col, q);
          if constexpr (R1) z[t] = ld4(d.z, q);
        }
      }
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int q = q0 + p.span * t;
        if (q >= pc4) continue;
        float w[4] = {0.f, 0.f, 0.f, 0.f};
        if (live && q < n4) {
          const float gs[4] = {g[t].x, g[t].y, g[t].z, g[t].w}, ms[4] = {m[t].x, m[t].y, m[t].z, m[t].w};
          const float as[4] = {a[t].x, a[t].y, a[t].z, a[t].w};
          float zs[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (R1) {
            zs[0] = z[t].x; zs[1] = z[t].y; zs[2] = z[t].z; zs[3] = z[t].w;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = fmaf(ku, zs[e], b * (fmaf(ms[e], beta, gs[e] * omb) * as[e]));
        }
        put_operand4((float *)J.x, tiled_index(p.i, 4 * q, J.pcol_pad), w, planes);
      }
    }
  } else {
    for (int j = p.q0; j < J.pcol_pad; j += p.span) {
      float x = 0.f;
      if (live && j < d.cols) {
        const float g = load_grad((const void *)d.grad, d.grad_dtype, p.i * d.cols + j);
        const float y = fmaf(mrow[j], beta, g * omb) * d.inv_col[j];
        x = b * y;
        if constexpr (R1) x = fmaf(ku, d.z[j], x);
      }
      put_operand((float *)J.x, tiled_index(p.i, j, J.pcol_pad), x, planes);
    }
  }
  block_part(J, vy, vu, p, blk, static_cast<int>(whiten_blocks(J)), J.fro, rp);
}

// Rows of more than kMaxSlices float4 per lane with the float4 path whose
// padded row is at most kKeptSlices float4 per lane (4 waves per row: up
// to 8192 columns): pass 1 keeps y = S a of every slice in registers, so
// pass 2 forms V without reading g and m' again (24 -> 16 bytes per
// element).  Loads go kKeptBatch slices at a time (every slice at once).
template <bool R1>
__device__ __forceinline__ void whiten_rows_kept(const DevJob &J, int blk, double (*red)[4], double (*rp)[4]) {
  const DevDesc &d = J.d;
  const RowPos p = row_pos(J, blk);
  const bool live = p.i < d.rows;
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const float kappa = R1 ? d.kappa[0] : 0.f;
  const bool planes = J.planes != 0;
  const int n4 = static_cast<int>(d.cols / 4), pc4 = static_cast<int>(J.pcol_pad / 4);
  SMX_GLOBAL float *mrow = d.momentum + p.i * d.cols;
  const SMX_GLOBAL float *grow = (const SMX_GLOBAL float *)d.grad + p.i * d.cols;
  float4 y[kKeptSlices];
  float y2 = 0.f, yz = 0.f;
#pragma unroll
  for (int t0 = 0; t0 < kKeptSlices; t0 += kKeptBatch) {
    float4 g[kKeptBatch], m[kKeptBatch], a[kKeptBatch], z[kKeptBatch];
#pragma unroll
    for (int tb = 0; tb < kKeptBatch; ++tb) {
      const int q = p.q0 + p.span * (t0 + tb);
      if (live && q < n4) {
        g[tb] = ld4(grow, q);
        m[tb] = ld4(mrow, q);
        a[tb] = ld4(d.inv_col, q);
        if constexpr (R1) z[tb] = ld4(d.z, q);
      }
    }
#pragma unroll
    for (int tb = 0; tb < kKeptBatch; ++tb) {
      const int q = p.q0 + p.span * (t0 + tb);
      float4 yy = make_float4(0.f, 0.f, 0.f, 0.f);
      if (live && q < n4) {
        const float4 gg = g[tb], aa = a[tb];
        float4 mm = m[tb];
        mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
        mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
        st4(mrow, q, mm);
        yy.x = fmaf(mm.x, beta, gg.x * omb) * aa.x; yy.y = fmaf(mm.y, beta, gg.y * omb) * aa.y;
        yy.z = fmaf(mm.z, beta, gg.z * omb) * aa.z; yy.w = fmaf(mm.w, beta, gg.w * omb) * aa.w;
        y2 = fmaf(yy.x, yy.x, fmaf(yy.y, yy.y, fmaf(yy.z, yy.z, fmaf(yy.w, yy.w, y2))));
        if constexpr (R1) {
          const float4 zz = z[tb];
          yz = fmaf(yy.x, zz.x, fmaf(yy.y, zz.y, fmaf(yy.z, zz.z, fmaf(yy.w, zz.w, yz))));
        }
      }
      y[t0 + tb] = yy;
    }
  }
  double v[2] = {static_cast<double>(wave_sum(y2)), static_cast<double>(wave_sum(yz))};
  row_sums<2>(v, red, p, J.wpr);
  double vy = 0.0, vu = 0.0;  // the row's b^2 |S a|^2 and u^2
  float b = 0.f, ku = 0.f;
  if (live) {
    const double bd = d.inv_row[p.i];
    const double u = bd * v[1];
    b = d.inv_row[p.i];
    ku = R1 ? kappa * static_cast<float>(u) : 0.f;
    vy = bd * bd * v[0];
    vu = u * u;
    if ((threadIdx.x & 63) == 0 && p.wr == 0) J.u[p.i] = static_cast<float>(u);
  }
  // V_ij = b_i y_j + kappa u_i z_j, zeros in padding rows and columns.  q
  // has the parity of the lane and pc4 is even, so both lanes of a pair
  // are inside the padded row or both outside.
#pragma unroll
  for (int t = 0; t < kKeptSlices; ++t) {
    const int q = p.q0 + p.span * t;
    if (q >= pc4) continue;
    float w[4] = {0.f, 0.f, 0.f, 0.f};
    if (live && q < n4) {
      float4 zz = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (R1) zz = ld4(d.z, q);
      w[0] = fmaf(ku, zz.x, b * y[t].x); w[1] = fmaf(ku, zz.y, b * y[t].y);
      w[2] = fmaf(ku, zz.z, b * y[t].z); w[3] = fmaf(ku, zz.w, b * y[t].w);
    }
    put_operand4_paired(J.x, tiled_index(p.i, 4 * static_cast<int64_t>(q), J.pcol_pad), w, planes, true);
  }
  block_part(J, vy, vu, p, blk, static_cast<int>(whiten_blocks(J)), J.fro, rp);
}

template <bool R1, bool WIDE>
__global__ void __launch_bounds__(kRowThreads) whiten_kernel(JobRange range) {
  __shared__ double red[2][4][4];  // row sums over the waves of a row
  __shared__ double rp[2][4];
  __shared__ __attribute__((aligned(16))) char xs[2][kWhitenStageBytes];
  const int jid = find_job(range, blockIdx.x);
  const DevJob J = load_job(range.jobs, jid);
  const int blk = blockIdx.x - range.start[jid];
  if constexpr (WIDE)
    whiten_rows_kept<R1>(J, blk, red[0], rp);
  else if (whiten_pipelined(J))
    whiten_rows_pipelined<R1>(J, blk, red, rp, xs);
  else
    whiten_rows_single<R1>(J, blk, red[0], rp);
}

// Transposed parameters whose row is one chunk (the float4 path, at most
// kFlipChunk columns): one wave per row, kFlipRows rows per block.  a and z
// (the same for every row) are loaded once into LDS, which leaves every g
// and m load of a lane in flight together (6 float4) within the 64 VGPRs
// that let a CU hold two 1024-thread blocks.  The LDS tile row of a wave
// holds b y = b S a, then V = b y + kappa u z; the block's 16 rows are one
// 16-element K group of every X row, so each 64 lanes write one whole 1 KB
// piece of the tiled X (16 X rows, 4 lanes per row).
template <bool R1>
__global__ void __launch_bounds__(kFlipThreads) whiten_flip_kept_kernel(JobRange range) {
  __shared__ float tile[kFlipRows][kFlipChunk + 4];
  __shared__ double rp[2][kFlipRows];
  __shared__ float4 colv[2][kFlipChunk / 4];  // a, z
  const int jid = find_job(range, blockIdx.x);
  const DevJob J = load_job(range.jobs, jid);
  const DevDesc &d = J.d;
  // (blocks of one XCD take consecutive groups, as in whiten_flip_kernel)
  const int nb = static_cast<int>(whiten_blocks(J));
  const int jb = blockIdx.x - range.start[jid];
  const int blk = (jb & 7) * (nb / 8) + (jb >> 3);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the row: wave-uniform
  const int64_t i0 = static_cast<int64_t>(blk) * kFlipRows;
  const int64_t i = i0 + wave;
  const bool live = i < d.rows;
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const float kappa = R1 ? d.kappa[0] : 0.f;
  const bool planes = J.planes != 0;
  const int n4 = static_cast<int>(d.cols / 4);
  SMX_GLOBAL float *mrow = d.momentum + i * d.cols;
  const SMX_GLOBAL float *grow = (const SMX_GLOBAL float *)d.grad + i * d.cols;
  {
    const int t = threadIdx.x, h = kFlipChunk / 4;
    if (t < n4) colv[0][t] = ld4(d.inv_col, t);
    if (R1 && t >= h && t - h < n4) colv[1][t - h] = ld4(d.z, t - h);
  }
  float4 g[kMaxSlices], m[kMaxSlices];
#pragma unroll
  for (int t = 0; t < kMaxSlices; ++t) {
    const int q = lane + 64 * t;
    if (live && q < n4) {
      g[t] = ld4(grow, q);
      m[t] = ld4(mrow, q);
    }
  }
  const float b = live ? d.inv_row[i] : 0.f;
  __syncthreads();
  float y2 = 0.f, yz = 0.f;
#pragma unroll
  for (int t = 0; t < kMaxSlices; ++t) {
    const int q = lane + 64 * t;
    float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live && q < n4) {
      const float4 aa = colv[0][q], gg = g[t];
      float4 mm = m[t];
      mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
      mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
      st4(mrow, q, mm);
      y.x = fmaf(mm.x, beta, gg.x * omb) * aa.x; y.y = fmaf(mm.y, beta, gg.y * omb) * aa.y;
      y.z = fmaf(mm.z, beta, gg.z * omb) * aa.z; y.w = fmaf(mm.w, beta, gg.w * omb) * aa.w;
      y2 = fmaf(y.x, y.x, fmaf(y.y, y.y, fmaf(y.z, y.z, fmaf(y.w, y.w, y2))));
      if constexpr (R1) {
        const float4 zz4 = colv[1][q];
        yz = fmaf(y.x, zz4.x, fmaf(y.y, zz4.y, fmaf(y.z, zz4.z, fmaf(y.w, zz4.w, yz))));
      }
    }
    *reinterpret_cast<float4 *>(&tile[wave][4 * q]) = make_float4(b * y.x, b * y.y, b * y.z, b * y.w);
  }
  const double Y2 = wave_sum(y2), YZ = wave_sum(yz);
  double vy = 0.0, vu = 0.0;  // the row's b^2 |S a|^2 and u^2
  if (live) {
    const double bd = b;
    const double u = bd * YZ;
    vy = bd * bd * Y2;
    vu = u * u;
    if (lane == 0) J.u[i] = static_cast<float>(u);
    if constexpr (R1) {
      const float ku = kappa * static_cast<float>(u);
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int q = lane + 64 * t;
        if (q < n4) {
          float4 *v = reinterpret_cast<float4 *>(&tile[wave][4 * q]);
          const float4 z = colv[1][q];
          float4 w = *v;
          w.x = fmaf(ku, z.x, w.x); w.y = fmaf(ku, z.y, w.y); w.z = fmaf(ku, z.z, w.z); w.w = fmaf(ku, z.w, w.w);
          *v = w;
        }
      }
    }
  }
  __syncthreads();
  const int qq = threadIdx.x & 3;  // 4-row quarter of the K group
#pragma unroll
  for (int r = 0; r < kFlipChunk / 256; ++r) {
    const int jj = (threadIdx.x >> 2) + 256 * r;  // X row
    if (jj < J.pcol_pad) {
      const float w[4] = {tile[4 * qq][jj], tile[4 * qq + 1][jj], tile[4 * qq + 2][jj], tile[4 * qq + 3][jj]};
      // (the 4 lanes of an X row are in it together, so lane pairs are whole)
      put_operand4_paired(J.x, tiled_index(jj, i0 + 4 * qq, J.prow_pad), w, planes, true);
    }
  }
  if (lane == 0) {
    rp[0][wave] = vy;
    rp[1][wave] = vu;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    double t = 0.0;
    for (int r = 0; r < kFlipRows; ++r) t += rp[threadIdx.x][r];
    J.fro[threadIdx.x * nb + blk] = t;
  }
}

// Transposed parameters, the other rows: one wave per row, kFlipRows rows
// per block, the row in chunks of kFlipChunk columns (kMaxSlices float4 per
// lane); pass 2 reads g and m' again.  Pass 2 stages each chunk of V in LDS
// as whiten_flip_kept_kernel does.
template <bool R1>
__global__ void __launch_bounds__(kFlipThreads) whiten_flip_kernel(JobRange range) {
  __shared__ float tile[kFlipRows][kFlipChunk + 4];
  __shared__ double rp[2][kFlipRows];
  const int jid = find_job(range, blockIdx.x);
  const DevJob J = load_job(range.jobs, jid);
  const DevDesc &d = J.d;
  // Row group of the block: the hardware deals blocks to the 8 XCDs in
  // turn, and the blocks of one XCD take consecutive groups (adjacent K
  // pieces of X).  (Every job's first block and block count are multiples
  // of 8.)
  const int jb = blockIdx.x - range.start[jid];
  const int blk = (jb & 7) * static_cast<int>(J.prow_pad / kFlipRows / 8) + (jb >> 3);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the row: wave-uniform
  const int64_t i0 = static_cast<int64_t>(blk) * kFlipRows;
  const int64_t i = i0 + wave;
  const bool live = i < d.rows;
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const float kappa = R1 ? d.kappa[0] : 0.f;
  const bool planes = J.planes != 0;
  SMX_GLOBAL float *mrow = live ? d.momentum + i * d.cols : nullptr;
  const bool vec = J.wvec != 0;
  const int n4 = static_cast<int>(d.cols / 4);
  const SMX_GLOBAL float *grow = live && vec ? (const SMX_GLOBAL float *)d.grad + i * d.cols : nullptr;
  const float b = live ? d.inv_row[i] : 0.f;
  // Slice t of chunk c of this lane: float4 c * kFlipChunk / 4 + lane + 64 t.
  float y2 = 0.f, yz = 0.f;
  if (vec) {
    // Two slices' loads in flight at a time: with kMaxSlices at once the
    // 1024-thread block needs more than 64 VGPRs, and a CU then holds one
    // block instead of two.
    constexpr int kB = 2;
    for (int c4 = 0; c4 < n4; c4 += kFlipChunk / 4) {
#pragma unroll
      for (int t0 = 0; t0 < kMaxSlices; t0 += kB) {
      float4 g[kB], m[kB], a[kB], z[kB];
#pragma unroll
      for (int tb = 0; tb < kB; ++tb) {
        const int q = c4 + lane + 64 * (t0 + tb);
        if (t0 + tb < kMaxSlices && q < n4) {
          a[tb] = ld4(d.inv_col, q);
          if constexpr (R1) z[tb] = ld4(d.z, q);
          if (live) {
            g[tb] = ld4(grow, q);
            m[tb] = ld4(mrow, q);
          }
        }
      }
#pragma unroll
      for (int tb = 0; tb < kB; ++tb) {
        const int t = t0 + tb;
        if (t >= kMaxSlices) continue;
        const int q = c4 + lane + 64 * t;
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q < n4 && live) {
          const float4 aa = a[tb], gg = g[tb];
          float4 mm = m[tb];
          mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
          mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
          st4(mrow, q, mm);
          y.x = fmaf(mm.x, beta, gg.x * omb) * aa.x; y.y = fmaf(mm.y, beta, gg.y * omb) * aa.y;
          y.z = fmaf(mm.z, beta, gg.z * omb) * aa.z; y.w = fmaf(mm.w, beta, gg.w * omb) * aa.w;
          y2 = fmaf(y.x, y.x, fmaf(y.y, y.y, fmaf(y.z, y.z, fmaf(y.w, y.w, y2))));
          if constexpr (R1) {
            const float4 zz4 = z[tb];
            yz = fmaf(y.x, zz4.x, fmaf(y.y, zz4.y, fmaf(y.z, zz4.z, fmaf(y.w, zz4.w, yz))));
          }
        }
      }
      }
    }
  } else {
    for (int j = lane; j < d.cols; j += 64) {
      const float a = d.inv_col[j];
      float zj = 0.f;
      if constexpr (R1) zj = d.z[j];
      if (live) {
        const float g = load_grad((const void *)d.grad, d.grad_dtype, i * d.cols + j);
        const float m = fmaf(mrow[j], beta, g * omb);
        mrow[j] = m;
        const float y = fmaf(m, beta, g * omb) * a;
        y2 = fmaf(y, y, y2);
        if constexpr (R1) yz = fmaf(y, zj, yz);
      }
    }
  }
  const double Y2 = wave_sum(y2), YZ = wave_sum(yz);
  double vy = 0.0, vu = 0.0;  // the row's b^2 |S a|^2 and u^2
  float ku = 0.f;
  if (live) {
    const double bd = b;
    const double u = bd * YZ;
    ku = R1 ? kappa * static_cast<float>(u) : 0.f;
    vy = bd * bd * Y2;
    vu = u * u;
    if (lane == 0) J.u[i] = static_cast<float>(u);
  }

  // ---- pass 2, chunk by chunk through LDS.
  const int qq = threadIdx.x & 3;  // 4-row quarter of the K group
  for (int c0 = 0; c0 < J.pcol_pad; c0 += kFlipChunk) {
    const int c4 = c0 / 4;
    {
    float4 g[kMaxSlices], m[kMaxSlices], a[kMaxSlices], z[kMaxSlices];
#pragma unroll
    for (int t = 0; t < kMaxSlices; ++t) {
      const int q = c4 + lane + 64 * t;
      if (vec && live && q < n4) {
        if constexpr (R1) z[t] = ld4(d.z, q);
        g[t] = ld4(grow, q);
        m[t] = ld4(mrow, q);
        a[t] = ld4(d.inv_col, q);
      }
    }
#pragma unroll
    for (int t = 0; t < kMaxSlices; ++t) {
      const int q = c4 + lane + 64 * t;
      const int j = 4 * q;
      float w[4] = {0.f, 0.f, 0.f, 0.f};
      if (live && j < d.cols) {
        if (vec) {
          float4 y;
          y.x = fmaf(m[t].x, beta, g[t].x * omb) * a[t].x; y.y = fmaf(m[t].y, beta, g[t].y * omb) * a[t].y;
          y.z = fmaf(m[t].z, beta, g[t].z * omb) * a[t].z; y.w = fmaf(m[t].w, beta, g[t].w * omb) * a[t].w;
          float4 zz4 = make_float4(0.f, 0.f, 0.f, 0.f);
          if constexpr (R1) zz4 = z[t];
          w[0] = fmaf(ku, zz4.x, b * y.x); w[1] = fmaf(ku, zz4.y, b * y.y);
          w[2] = fmaf(ku, zz4.z, b * y.z); w[3] = fmaf(ku, zz4.w, b * y.w);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (j + e < d.cols) {
              const float gv = load_grad((const void *)d.grad, d.grad_dtype, i * d.cols + j + e);
              float x = b * (fmaf(mrow[j + e], beta, gv * omb) * d.inv_col[j + e]);
              if constexpr (R1) x = fmaf(ku, d.z[j + e], x);
              w[e] = x;
            }
          }
        }
      }
      *reinterpret_cast<float4 *>(&tile[wave][4 * (lane + 64 * t)]) = make_float4(w[0], w[1], w[2], w[3]);
    }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kFlipChunk / 256; ++r) {
      const int jj = (threadIdx.x >> 2) + 256 * r;  // X row in the chunk
      if (c0 + jj < J.pcol_pad) {
        const float w[4] = {tile[4 * qq][jj], tile[4 * qq + 1][jj], tile[4 * qq + 2][jj], tile[4 * qq + 3][jj]};
        // (the 4 lanes of an X row are in it together, so lane pairs are whole)
        put_operand4_paired(J.x, tiled_index(c0 + jj, i0 + 4 * qq, J.prow_pad), w, planes, true);
      }
    }
    __syncthreads();
  }
  if (lane == 0) {
    rp[0][wave] = vy;
    rp[1][wave] = vu;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    double t = 0.0;
    for (int r = 0; r < kFlipRows; ++r) t += rp[threadIdx.x][r];
    J.fro[threadIdx.x * whiten_blocks(J) + blk] = t;
  }
}

// ------------------------------------------------------------ mapback ---
// From the stage-5 row-sum partials: u_i = sum_j Q_ij z_j and ||U_i||^2 in
// closed form, b_i^2 (sum (a Q)^2 + 2 kappa u_i sum (a Q)(a z) + kappa^2
// u_i^2 sum (a z)^2); per-block partials of ||U||^2.  kNormRows rows per
// block, 4 lanes per row (strips p, p + 4, ... of lane p, all loads of a
// lane in flight together for up to 4 kNormUnroll strips per row).
constexpr int kNormRows = kRowThreads / 4;
constexpr int kNormUnroll = 12;

template <bool R1>
__global__ void __launch_bounds__(kRowThreads) mapback_norm_kernel(JobRange range) {
  __shared__ double scratch[16];
  const int jid = find_job(range, blockIdx.x);
  const DevJob J = load_job(range.jobs, jid);
  const DevDesc &d = J.d;
  const int blk = blockIdx.x - range.start[jid];
  const int part = threadIdx.x & 3;
  const int64_t i = static_cast<int64_t>(blk) * kNormRows + (threadIdx.x >> 2);
  const bool live = i < d.rows;
  double su = 0.0, sa = 0.0, sb = 0.0;
  if (live) {
    const SMX_GLOBAL float *p0 = J.mrp + i;
    for (int k0 = part; k0 < J.strips; k0 += 4 * kNormUnroll) {
      float v[kNormUnroll][3];
#pragma unroll
      for (int u = 0; u < kNormUnroll; ++u) {
        const int k = k0 + 4 * u;
        const int64_t o = static_cast<int64_t>(k) * J.prow_pad;
        const bool in = k < J.strips;
        v[u][0] = in ? p0[o] : 0.f;
        v[u][1] = in ? p0[J.mrp_size + o] : 0.f;
        v[u][2] = in ? p0[2 * J.mrp_size + o] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kNormUnroll; ++u) {
        su += v[u][0];
        sa += v[u][1];
        sb += v[u][2];
      }
    }
  }
  // the row's 4 lanes (a DPP quad), fixed order
  su += dpp_mov<0xB1>(su); su += dpp_mov<0x4E>(su);
  sa += dpp_mov<0xB1>(sa); sa += dpp_mov<0x4E>(sa);
  sb += dpp_mov<0xB1>(sb); sb += dpp_mov<0x4E>(sb);
  double row_part = 0.0;
  if (live && part == 0) {
    const double b = d.inv_row[i];
    const double kappa = R1 ? d.kappa[0] : 0.0;
    const double cz = R1 ? J.cst[kCstAZ] : 0.0;
    J.u[i] = static_cast<float>(su);
    row_part = b * b * (sa + 2.0 * kappa * su * sb + kappa * kappa * su * su * cz);
  }
  const double t = block_sum(row_part, scratch);
  if (threadIdx.x == 0) J.mb[blk] = t;
}

// W -= lr * sqrt(rows) / max(||U||_F, FLT_MIN) * U (wpr waves per row).  A
// 16-bit parameter takes W = round(W - lr * round(direction))
// (sandmuon/optimizer.py:315) on the per-element path.
template <bool R1>
__global__ void __launch_bounds__(kRowThreads) mapback_apply_kernel(JobRange range) {
  const int jid = find_job(range, blockIdx.x);
  const DevJob J = load_job(range.jobs, jid);
  const DevDesc &d = J.d;
  const int blk = blockIdx.x - range.start[jid];
  const RowPos p = row_pos(J, blk);
  if (p.i >= d.rows) return;
  const int pdt = d.param_dtype;
  const SMX_GLOBAL float *q = J.q + p.i * J.pcol_pad;
  // ||U||^2 from mapback_norm's per-block partials, added by every wave in
  // the same fixed order (lane l takes partials l, l + 64, ..., then the
  // wave sum), so that every block of the matrix scales by the same value
  // (a separate one-block-per-matrix launch for this sum cost more than
  // these few cached loads).
  double n2 = 0.0;
  {
    const int64_t nb = norm_blocks(J);
    for (int64_t k = threadIdx.x & 63; k < nb; k += 64) n2 += J.mb[k];
    n2 = wave_sum(n2);
  }
  const float norm = static_cast<float>(sqrt(n2));
  // _graft_direction: sqrt(rows) / max(||U||, FLT_MIN); a zero direction
  // gives a zero update.
  const float scale = n2 > 0.0 ? static_cast<float>(sqrt(static_cast<double>(d.rows))) / fmaxf(norm, FLT_MIN) : 0.f;
  const float nlr = static_cast<float>(-d.lr);
  const float b = d.inv_row[p.i];
  const float ku = R1 ? d.kappa[0] * J.u[p.i] : 0.f;
  if (J.mvec) {
    SMX_GLOBAL float *w = (SMX_GLOBAL float *)d.param + p.i * d.cols;
    const int n4 = static_cast<int>(d.cols / 4);
    for (int q0 = p.q0; q0 < n4; q0 += p.span * kMaxSlices) {
      float4 qv[kMaxSlices], av[kMaxSlices], wv[kMaxSlices], zv[kMaxSlices];
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int k = q0 + p.span * t;
        if (k < n4) {
          qv[t] = ld4(q, k);
          wv[t] = ld4(w, k);
          av[t] = ld4(d.inv_col, k);
          if constexpr (R1) zv[t] = ld4(d.z, k);
        }
      }
#pragma unroll
      for (int t = 0; t < kMaxSlices; ++t) {
        const int k = q0 + p.span * t;
        if (k < n4) {
          float4 v = qv[t], ww = wv[t];
          const float4 a = av[t];
          if constexpr (R1) {
            const float4 z = zv[t];
            v.x = fmaf(ku, z.x, v.x); v.y = fmaf(ku, z.y, v.y); v.z = fmaf(ku, z.z, v.z); v.w = fmaf(ku, z.w, v.w);
          }
          ww.x = fmaf(nlr, ((v.x * b) * a.x) * scale, ww.x);
          ww.y = fmaf(nlr, ((v.y * b) * a.y) * scale, ww.y);
          ww.z = fmaf(nlr, ((v.z * b) * a.z) * scale, ww.z);
          ww.w = fmaf(nlr, ((v.w * b) * a.w) * scale, ww.w);
          st4(w, k, ww);
        }
      }
    }
  } else {
    const int64_t row = p.i * d.cols;
    for (int j = p.q0; j < d.cols; j += p.span) {
      float v = q[j];
      if constexpr (R1) v = fmaf(ku, d.z[j], v);
      const float dir = round_to(pdt, ((v * b) * d.inv_col[j]) * scale);
      store_any((void *)d.param, pdt, row + j, round_to(pdt, fmaf(nlr, dir, load_any((const void *)d.param, pdt, row + j))));
    }
  }
}

// --------------------------------------------------------------- host ---
static bool oriented(const smx_matrix_desc &d, int64_t &r, int64_t &c, bool &flip) {
  flip = d.rows > d.cols;
  r = flip ? d.cols : d.rows;
  c = flip ? d.rows : d.cols;
  return true;
}

// Groups of matrices with at most kMaxClasses distinct oriented shapes,
// formed greedily in table order.
static std::vector<std::vector<int32_t>> shape_groups(const int64_t *rows, const int64_t *cols, int32_t n) {
  std::vector<std::vector<int32_t>> groups;
  std::vector<std::pair<int64_t, int64_t>> shapes;
  for (int32_t i = 0; i < n; ++i) {
    const std::pair<int64_t, int64_t> s(std::min(rows[i], cols[i]), std::max(rows[i], cols[i]));
    if (groups.empty() || (std::find(shapes.begin(), shapes.end(), s) == shapes.end() &&
                           static_cast<int>(shapes.size()) == kMaxClasses)) {
      groups.emplace_back();
      shapes.clear();
    }
    if (std::find(shapes.begin(), shapes.end(), s) == shapes.end()) shapes.push_back(s);
    groups.back().push_back(i);
  }
  return groups;
}

// The job table follows the S8 buffers of a group.
static size_t table_bytes(size_t jobs) { return static_cast<size_t>(round_up(jobs * sizeof(MatJob), 256)); }

static size_t group_bytes(const int64_t *rows, const int64_t *cols, const std::vector<int32_t> &g, int mode) {
  const int32_t m = static_cast<int32_t>(g.size());
  std::vector<int64_t> r(m), c(m);
  std::unique_ptr<bool[]> fl(new bool[m]);
  for (int32_t k = 0; k < m; ++k) {
    r[k] = std::min(rows[g[k]], cols[g[k]]);
    c[k] = std::max(rows[g[k]], cols[g[k]]);
    fl[k] = rows[g[k]] > cols[g[k]];
  }
  S8Plan plan;
  std::vector<int32_t> cls(m), slot(m);
  plan_s8(r.data(), c.data(), fl.get(), m, mode, nullptr, plan, cls.data(), slot.data());
  return plan.bytes + table_bytes(m);
}

// Waves per row and float4 per lane for rows of `cols` columns.
static void row_geometry(int64_t cols, int32_t &wpr, int32_t &slices) {
  const int64_t n4 = ceil_div(cols, 4);
  wpr = n4 <= 64 * kMaxSlices ? 1 : n4 <= 128 * kMaxSlices ? 2 : 4;
  slices = static_cast<int32_t>(ceil_div(n4, 64 * wpr));
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Launches `kernel` over table jobs [first, first + n), kLaunchJobs at a time.
template <typename KernelFn>
static int launch_range(const MatJob *host, MatJob *table, int32_t first, int32_t n,
                        int64_t (*blocks_of)(const MatJob &), KernelFn kernel, int threads, const char *what,
                        hipStream_t st) {
  for (int32_t b = first; b < first + n; b += kLaunchJobs) {
    JobRange r{};
    r.jobs = table + b;
    r.n = std::min<int32_t>(kLaunchJobs, first + n - b);
    int64_t total = 0;
    for (int k = 0; k < kLaunchJobs; ++k) r.start[k] = INT32_MAX;
    for (int k = 0; k < r.n; ++k) {
      r.start[k] = static_cast<int32_t>(total);
      total += blocks_of(host[b + k]);
    }
    SMX_REQUIRE(total < INT32_MAX, SMX_ESHAPE, std::string(what) + ": too many blocks for one launch");
    if (total == 0) continue;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total)), dim3(threads), 0, st, r);
    const int rc = check_launch(what);
    if (rc) return rc;
  }
  return SMX_OK;
}

static int matrix_totals(MatJob *table, int32_t m, hipStream_t st) {
  hipLaunchKernelGGL(matrix_total_kernel, dim3(static_cast<unsigned>(m)), dim3(kTotalThreads), 0, st, table);
  return check_launch("matrix_total");
}

}  // namespace smx

using namespace smx;

extern "C" size_t smx_matrix_step_workspace_bytes(const int64_t *rows, const int64_t *cols, int32_t n,
                                                  int mode) {
  if (n <= 0 || !rows || !cols) return 0;
  size_t best = 0;
  for (const auto &g : shape_groups(rows, cols, n)) best = std::max(best, group_bytes(rows, cols, g, mode));
  return best;
}

extern "C" int smx_matrix_step(const smx_matrix_desc *descs, int32_t n, int mode, void *workspace,
                               size_t workspace_bytes, void *stream) {
  SMX_REQUIRE(n >= 0, SMX_EINVAL, "matrix_step: n < 0");
  if (n == 0) return SMX_OK;
  SMX_REQUIRE(descs && workspace, SMX_EINVAL, "matrix_step: null descriptor table or workspace");
  SMX_REQUIRE(mode == SMX_S8_FP32 || mode == SMX_S8_COMP_BF16 || mode == SMX_S8_MIXED, SMX_EINVAL,
              "matrix_step: unknown S8 mode");
  std::vector<int64_t> rows(n), cols(n);
  for (int32_t i = 0; i < n; ++i) {
    const smx_matrix_desc &d = descs[i];
    SMX_REQUIRE(d.param && d.grad && d.momentum && d.inv_row && d.inv_col, SMX_EINVAL,
                "matrix_step: param, grad, momentum, inv_row and inv_col are required");
    SMX_REQUIRE((d.z == nullptr) == (d.kappa == nullptr), SMX_EINVAL,
                "matrix_step: z and kappa must both be set or both NULL");
    SMX_REQUIRE((d.z == nullptr) == (descs[0].z == nullptr), SMX_EINVAL,
                "matrix_step: either every matrix of a call has a rank-one term or none has");
    SMX_REQUIRE(d.rows >= 1 && d.cols >= 1, SMX_ESHAPE, "matrix_step: rows and cols must be >= 1");
    SMX_REQUIRE(d.grad_dtype == SMX_F32 || d.grad_dtype == SMX_BF16 || d.grad_dtype == SMX_F16, SMX_EDTYPE,
                "matrix_step: grad dtype must be f32, bf16 or f16");
    SMX_REQUIRE(d.param_dtype == SMX_F32 || d.param_dtype == SMX_BF16 || d.param_dtype == SMX_F16, SMX_EDTYPE,
                "matrix_step: param dtype must be f32, bf16 or f16");
    rows[i] = d.rows;
    cols[i] = d.cols;
  }
  const size_t need = smx_matrix_step_workspace_bytes(rows.data(), cols.data(), n, mode);
  SMX_REQUIRE(workspace_bytes >= need, SMX_EWORKSPACE, "matrix_step: workspace too small");
  SMX_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SMX_EALIGN,
              "matrix_step: workspace must be 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool r1 = descs[0].z != nullptr;
  for (const auto &g : shape_groups(rows.data(), cols.data(), n)) {
    const int32_t m = static_cast<int32_t>(g.size());
    std::vector<int64_t> r(m), c(m);
    std::unique_ptr<bool[]> fl(new bool[m]);
    for (int32_t k = 0; k < m; ++k) {
      bool f;
      oriented(descs[g[k]], r[k], c[k], f);
      fl[k] = f;
    }
    S8Plan plan;
    std::vector<int32_t> cls(m), slot(m);
    if (!plan_s8(r.data(), c.data(), fl.get(), m, mode, static_cast<char *>(workspace), plan, cls.data(),
                 slot.data()))
      return fail(SMX_EINVAL, "matrix_step: internal shape grouping error");
    MatJob *table = reinterpret_cast<MatJob *>(static_cast<char *>(workspace) + plan.bytes);
    // Table order (one whiten launch each): parameters kept as they are,
    // except those of the next bucket; parameters kept as they are whose
    // wide rows leave y in registers (whiten_rows_kept); transposed ones
    // whose rows fit one LDS chunk with the float4 path; the other
    // transposed ones.  Both mapback launches take the whole table.
    std::vector<MatJob> jobs;
    jobs.reserve(m);
    int32_t n_plain = 0, n_kept = 0;
    auto vec_path = [&](int32_t k) {  // the float4 path of the whiten kernels
      const smx_matrix_desc &d = descs[g[k]];
      return d.cols % 4 == 0 && d.grad_dtype == SMX_F32 && aligned16(d.grad) && aligned16(d.momentum) &&
             aligned16(d.inv_col) && (!r1 || aligned16(d.z));
    };
    auto plain_kept = [&](int32_t k) {  // whiten_rows_kept: y of the padded row fits the registers
      int32_t wpr, slices;
      row_geometry(descs[g[k]].cols, wpr, slices);
      const S8Mat M{plan.layout.cls[cls[k]], slot[k]};
      return vec_path(k) && slices > kMaxSlices && ceil_div(M.pcol_pad() / 4, 64 * wpr) <= kKeptSlices;
    };
    auto bucket = [&](int32_t k) {
      if (!fl[k]) return plain_kept(k) ? 1 : 0;
      return vec_path(k) && descs[g[k]].cols <= kFlipChunk ? 2 : 3;
    };
    int32_t n_wide = 0;
    for (int pass = 0; pass < 4; ++pass) {
      for (int32_t k = 0; k < m; ++k) {
        if (pass != bucket(k)) continue;
        const S8Mat M{plan.layout.cls[cls[k]], slot[k]};
        MatJob j{};
        j.d = descs[g[k]];
        j.x = M.x0();
        j.flip = M.flip();
        j.q = M.result();
        j.u = M.u();
        j.fro = M.fro();
        j.mb = M.mb();
        j.cst = M.cst();
        j.colv = M.colv();
        j.mrp = M.mrp(0);
        j.mrp_size = M.mrp_size();
        j.strips = static_cast<int32_t>(M.strips());
        j.prow_pad = static_cast<int32_t>(M.prow_pad());
        j.pcol_pad = static_cast<int32_t>(M.pcol_pad());
        j.planes = mode != SMX_S8_FP32;  // stage 1 reads X0 compensated in both BF16 modes
        row_geometry(j.d.cols, j.wpr, j.slices);
        j.cvec = j.d.cols % 4 == 0 && aligned16(j.d.inv_col) && (!r1 || aligned16(j.d.z));
        j.wvec = j.cvec && j.d.grad_dtype == SMX_F32 && aligned16(j.d.grad) && aligned16(j.d.momentum);
        j.mvec = j.cvec && j.d.param_dtype == SMX_F32 && aligned16(j.d.param);
        jobs.push_back(j);
        n_plain += pass == 0;
        n_wide += pass <= 1;
        n_kept += pass <= 2;
      }
    }
    for (int32_t b = 0; b < m; b += kPrepBatch) {
      PrepPack pk{};
      pk.n = std::min<int32_t>(kPrepBatch, m - b);
      for (int k = 0; k < pk.n; ++k) pk.j[k] = jobs[b + k];
      pk.table = table + b;
      hipLaunchKernelGGL(matrix_prep_kernel, dim3(pk.n), dim3(64), 0, st, pk);
      const int rc = check_launch("matrix_prep");
      if (rc) return rc;
    }
    // The kernels are specialised on whether the matrices carry a rank-one
    // term (all of a call or none, checked above).
    const MatJob *h = jobs.data();
    int rc = r1 ? launch_range(h, table, 0, n_plain, whiten_blocks, whiten_kernel<true, false>, kRowThreads,
                               "whiten", st)
                : launch_range(h, table, 0, n_plain, whiten_blocks, whiten_kernel<false, false>, kRowThreads,
                               "whiten", st);
    if (!rc && n_wide > n_plain)
      rc = r1 ? launch_range(h, table, n_plain, n_wide - n_plain, whiten_blocks, whiten_kernel<true, true>,
                             kRowThreads, "whiten", st)
              : launch_range(h, table, n_plain, n_wide - n_plain, whiten_blocks, whiten_kernel<false, true>,
                             kRowThreads, "whiten", st);
    if (!rc && n_kept > n_wide)
      rc = r1 ? launch_range(h, table, n_wide, n_kept - n_wide, whiten_blocks, whiten_flip_kept_kernel<true>,
                             kFlipThreads, "whiten", st)
              : launch_range(h, table, n_wide, n_kept - n_wide, whiten_blocks, whiten_flip_kept_kernel<false>,
                             kFlipThreads, "whiten", st);
    if (!rc && m > n_kept)
      rc = r1 ? launch_range(h, table, n_kept, m - n_kept, whiten_blocks, whiten_flip_kernel<true>,
                             kFlipThreads, "whiten", st)
              : launch_range(h, table, n_kept, m - n_kept, whiten_blocks, whiten_flip_kernel<false>,
                             kFlipThreads, "whiten", st);
    if (!rc) rc = matrix_totals(table, m, st);
    plan.layout.rowsums = 1;
    if (!rc) rc = run_s8_stages(plan.layout, st);
    if (!rc)
      rc = r1 ? launch_range(h, table, 0, m, norm_blocks, mapback_norm_kernel<true>, kRowThreads, "mapback_norm", st)
              : launch_range(h, table, 0, m, norm_blocks, mapback_norm_kernel<false>, kRowThreads, "mapback_norm", st);
    if (!rc)
      rc = r1 ? launch_range(h, table, 0, m, mapback_blocks, mapback_apply_kernel<true>, kRowThreads, "mapback_apply",
                             st)
              : launch_range(h, table, 0, m, mapback_blocks, mapback_apply_kernel<false>, kRowThreads,
                             "mapback_apply", st);
    if (rc) return rc;
  }
  return SMX_OK;
}
