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
// and B on rows, whichever orientation the S8 map uses; the whiten kernel
// writes the oriented iterate X (r x c, r <= c).
//
// whiten       two passes per row in one launch: momentum update,
//              u_i = b_i sum_j S_ij a_j z_j and the row's ||V_i||^2 in closed
//              form (||V_i||^2 = b_i^2 sum_j (S_ij a_j)^2 + (2 kappa + kappa^2 |z|^2) u_i^2);
//              then V from (g, m', u) stored to X directly, or transposed
//              through LDS for a transposed parameter.
// mapback_rows u_i = sum_j Q_ij z_j and ||U_i||^2 in closed form.
// mapback_apply W -= lr * scale * U.
#include "s8.h"

#include <algorithm>
#include <climits>
#include <cfloat>
#include <cmath>
#include <memory>
#include <vector>

namespace smx {

struct MatJob {
  smx_matrix_desc d;
  float *pl;         // parameter-layout buffer [prow_pad][pcol_pad]
  float *tl;         // transposed buffer [pcol_pad][prow_pad] (whiten of a transposed parameter)
  float *u;          // [rows] rank-one row coefficients
  double *part;      // [ceil(rows/kPartRows)] partial sums
  double *cst;       // [2]: sum z^2, sum (a z)^2 (matrix_consts_kernel)
  int64_t prow_pad, pcol_pad;
  int32_t blk0;      // first block of this job in the launch
  int32_t planes;    // whiten: write X, X^T as BF16 hi/lo planes (comp mode)
};

constexpr int kMatBatch = 24;
struct MatPack {
  int32_t start[kMatBatch];  // first block of each job; INT32_MAX past the last
  MatJob j[kMatBatch];
  int32_t n;
  int32_t total_blocks;
};
static_assert(sizeof(MatPack) <= 4000, "MatPack is passed by value in the kernel arguments");

// The job of block b: independent compares against the compact start
// table (a few batched scalar loads, no chain of dependent lookups).
__device__ __forceinline__ int find_job(const MatPack &p, int b) {
  int k = 0;
#pragma unroll
  for (int t = 1; t < kMatBatch; ++t) k += b >= p.start[t] ? 1 : 0;
  return k;
}

__device__ __forceinline__ float load_grad(const void *g, int dt, int64_t i) {
  if (dt == SMX_F32) return static_cast<const float *>(g)[i];
  if (dt == SMX_BF16) return load_elem<SMX_BF16>(g, i);
  return load_elem<SMX_F16>(g, i);
}

__device__ __forceinline__ bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
__device__ __forceinline__ float4 ld4(const float *p, int64_t q) { return reinterpret_cast<const float4 *>(p)[q]; }
__device__ __forceinline__ void st4(float *p, int64_t q, float4 v) { reinterpret_cast<float4 *>(p)[q] = v; }

// One block per job: the rank-one constants of the matrix,
// cst = {sum_j z_j^2, sum_j (a_j z_j)^2} (FP64), used by the row kernels.
__global__ void __launch_bounds__(256) matrix_consts_kernel(MatPack pack) {
  __shared__ double scratch[16];
  const MatJob &J = pack.j[blockIdx.x];
  const smx_matrix_desc &d = J.d;
  if (d.z == nullptr) return;
  double zz = 0.0, az = 0.0;
  for (int64_t j = threadIdx.x; j < d.cols; j += blockDim.x) {
    const double z = d.z[j], a = d.inv_col[j];
    zz += z * z;
    az += (a * z) * (a * z);
  }
  zz = block_sum(zz, scratch);
  az = block_sum(az, scratch);
  if (threadIdx.x == 0) {
    J.cst[0] = zz;
    J.cst[1] = az;
  }
}

// The row kernels run one wave per row.  Per-row reductions use FP32 lane
// partials and an FP32 wave sum; rows are accumulated in FP64, one partial
// per kPartRows rows.
constexpr int kRowThreads = 64 * kRowsPerPart;  // the largest block (16 rows)
constexpr int kMapThreads = 64 * kPartRows;     // mapback blocks (4 rows)
constexpr int kRowUnroll = 4;  // float4 columns per lane whose loads are in flight together

// FP64 sum of the NW per-wave row partials, in wave order; the result is
// valid in thread 0.
template <int NW>
__device__ __forceinline__ double sum_wave_parts(double part, double *wave_part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) wave_part[wave] = part;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < NW; ++w) t += wave_part[w];
  return t;
}

// ------------------------------------------------------------- whiten ---
// One wave per row of the padded parameter layout (blocks of 4 rows, or 16
// for a transposed parameter), two passes over the row:
//  1. momentum m' = b m + (1-b) g (in place), u_i = b_i sum_j S_ij a_j z_j
//     and the row's ||V_i||^2 (closed form) for S = b m' + (1-b) g;
//  2. V_ij = b_i S_ij a_j + kappa u_i z_j stored in operand form to the
//     oriented iterate: row i of X directly (pl), or, for a transposed
//     parameter (tl), through LDS in chunks of kWhitenChunk columns, where
//     the block's 16 rows are one 16-element K group of each X row.
// KEEP > 0 (rows of at most KEEP * kWhitenChunk columns, FP32 gradients,
// 16-byte aligned): pass 1 keeps S of the lane's columns in registers and
// pass 2 reads it from there; KEEP = 0: pass 2 reads g and m' again (the
// row was just read, so mostly from cache).  Both give the same bits.
// Rows and columns of the padding are written as zeros.
constexpr int kWhitenChunk = 1024;  // = 4 * 64 * kRowUnroll
// Most column chunks a row keeps in registers: 4 for parameters kept as
// they are (256-thread blocks, up to ~170 VGPRs), 1 for transposed ones
// (1024-thread blocks hold at most 128 VGPRs per lane).
constexpr int kWhitenKeep = 4;
constexpr int kWhitenKeepFlip = 1;

// Rows per block: a transposed parameter needs 16 (one K group of every X
// row); the others take kPartRows, so that more, shorter blocks share a CU.
template <bool FLIP>
constexpr int whiten_rows_per_block() { return FLIP ? kRowsPerPart : kPartRows; }

template <bool R1, bool FLIP, int KEEP>
__global__ void __launch_bounds__(64 * whiten_rows_per_block<FLIP>()) whiten_kernel(MatPack pack) {
  constexpr int RB = whiten_rows_per_block<FLIP>();
  static_assert(kRowsPerPart == 16 && kRowThreads == 1024, "one 16-row K group per transposed block, 4 lanes per X row");
  static_assert(RB % kPartRows == 0, "whole partials per block");
  __shared__ double wave_part[RB];
  __shared__ float tile[FLIP ? kRowsPerPart : 1][FLIP ? kWhitenChunk + 4 : 1];
  const MatJob &J = pack.j[find_job(pack, blockIdx.x)];
  const smx_matrix_desc &d = J.d;
  const int blk = blockIdx.x - J.blk0;
  constexpr bool r1 = R1;
  const double zz = r1 ? J.cst[0] : 0.0;
  const float kappa = r1 ? d.kappa[0] : 0.f;
  const double corr = r1 ? 2.0 * kappa + static_cast<double>(kappa) * kappa * zz : 0.0;
  const float beta = static_cast<float>(d.momentum_beta), omb = static_cast<float>(1.0 - d.momentum_beta);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool vec = d.grad_dtype == SMX_F32 && d.cols % 4 == 0 && aligned16(d.grad) && aligned16(d.momentum) &&
                   aligned16(d.inv_col) && (!r1 || aligned16(d.z));
  const bool planes = J.planes != 0;
  const int64_t i0 = static_cast<int64_t>(blk) * RB;
  const int64_t i = i0 + wave;
  const bool live = i < d.rows;
  float *mrow = live ? d.momentum + i * d.cols : nullptr;
  const float *grow = live && vec ? static_cast<const float *>(d.grad) + i * d.cols : nullptr;
  // S of this lane's columns: chunk k, float4 u covers columns
  // 4 lane + 4 * 64 u + kWhitenChunk k (pass 1's and pass 2's mapping).
  const bool kept = KEEP > 0 && vec && d.cols <= static_cast<int64_t>(KEEP) * kWhitenChunk;
  float4 sk[KEEP > 0 ? KEEP : 1][kRowUnroll];

  // ---- pass 1
  double part = 0.0;
  float b = 0.f, ku = 0.f;
  if (live) {
    float y2 = 0.f, yz = 0.f;
    if (vec) {
      const int64_t n4 = d.cols / 4;
      // One chunk of kRowUnroll float4 per lane; S goes to keep_s.
      auto chunk = [&](int64_t q0, float4 (&keep_s)[kRowUnroll]) {
        // Every load of the chunk is issued before the first store.
        float4 g[kRowUnroll], m[kRowUnroll], a[kRowUnroll], z[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const int64_t q = q0 + 64 * u;
          if (q < n4) {
            g[u] = ld4(grow, q);
            m[u] = ld4(mrow, q);
            a[u] = ld4(d.inv_col, q);
            if constexpr (R1) z[u] = ld4(d.z, q);
          }
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const int64_t q = q0 + 64 * u;
          if (q < n4) {
            float4 mm = m[u];
            const float4 gg = g[u], aa = a[u];
            mm.x = fmaf(mm.x, beta, gg.x * omb); mm.y = fmaf(mm.y, beta, gg.y * omb);
            mm.z = fmaf(mm.z, beta, gg.z * omb); mm.w = fmaf(mm.w, beta, gg.w * omb);
            st4(mrow, q, mm);
            const float s0 = fmaf(mm.x, beta, gg.x * omb), s1 = fmaf(mm.y, beta, gg.y * omb);
            const float s2 = fmaf(mm.z, beta, gg.z * omb), s3 = fmaf(mm.w, beta, gg.w * omb);
            keep_s[u] = make_float4(s0, s1, s2, s3);
            const float y0 = s0 * aa.x, y1 = s1 * aa.y;
            const float y2_ = s2 * aa.z, y3 = s3 * aa.w;
            y2 = fmaf(y0, y0, fmaf(y1, y1, fmaf(y2_, y2_, fmaf(y3, y3, y2))));
            if constexpr (R1) {
              const float4 zz4 = z[u];
              yz = fmaf(y0, zz4.x, fmaf(y1, zz4.y, fmaf(y2_, zz4.z, fmaf(y3, zz4.w, yz))));
            }
          } else {
            keep_s[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      };
      if (kept) {
#pragma unroll
        for (int k = 0; k < (KEEP > 0 ? KEEP : 1); ++k) chunk(lane + 64 * kRowUnroll * k, sk[k]);
      } else {
        for (int64_t q0 = lane; q0 < n4; q0 += 64 * kRowUnroll) chunk(q0, sk[0]);
      }
    } else {
      for (int64_t j = lane; j < d.cols; j += 64) {
        const float g = load_grad(d.grad, d.grad_dtype, i * d.cols + j);
        const float m = fmaf(mrow[j], beta, g * omb);
        mrow[j] = m;
        const float y = fmaf(m, beta, g * omb) * d.inv_col[j];
        y2 = fmaf(y, y, y2);
        if (r1) yz = fmaf(y, d.z[j], yz);
      }
    }
    const double Y2 = wave_sum(y2);
    const double YZ = wave_sum(yz);
    const double bd = d.inv_row[i];
    const double u = bd * YZ;
    b = d.inv_row[i];
    ku = r1 ? kappa * static_cast<float>(u) : 0.f;
    if (lane == 0) {
      J.u[i] = static_cast<float>(u);
      part = bd * bd * Y2 + corr * u * u;
    }
  }
  // ---- pass 2: V of the row, kRowUnroll groups of four consecutive
  // columns at a time, every load of a batch issued before the arithmetic.
  auto batch = [&](int64_t j0, int64_t stride, float (&v)[kRowUnroll][4]) {
    if (live && vec) {
      float4 g[kRowUnroll], m[kRowUnroll], a[kRowUnroll], z[kRowUnroll];
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        const int64_t j = j0 + stride * u;
        if (j < d.cols) {
          g[u] = ld4(grow, j / 4);
          m[u] = ld4(mrow, j / 4);
          a[u] = ld4(d.inv_col, j / 4);
          if constexpr (R1) z[u] = ld4(d.z, j / 4);
        }
      }
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        const int64_t j = j0 + stride * u;
        const float gs[4] = {g[u].x, g[u].y, g[u].z, g[u].w}, ms[4] = {m[u].x, m[u].y, m[u].z, m[u].w};
        const float as[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
        float zs[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (R1) {
          zs[0] = z[u].x; zs[1] = z[u].y; zs[2] = z[u].z; zs[3] = z[u].w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float s = fmaf(ms[e], beta, gs[e] * omb);
          float x = (s * b) * as[e];
          if constexpr (R1) x = fmaf(ku, zs[e], x);
          v[u][e] = j < d.cols ? x : 0.f;
        }
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t j = j0 + stride * u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[u][e] = 0.f;
        if (live && j + e < d.cols) {
          const float g = load_grad(d.grad, d.grad_dtype, i * d.cols + j + e);
          const float s = fmaf(mrow[j + e], beta, g * omb);
          v[u][e] = (s * b) * d.inv_col[j + e];
          if constexpr (R1) v[u][e] = fmaf(ku, d.z[j + e], v[u][e]);
        }
      }
    }
  };
  // The same with S from the registers of pass 1 (chunk k of the lane).
  auto batch_kept = [&](int k, int64_t j0, float (&v)[kRowUnroll][4]) {
    float4 a[kRowUnroll], z[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t j = j0 + 4 * 64 * u;
      if (j < d.cols) {
        a[u] = ld4(d.inv_col, j / 4);
        if constexpr (R1) z[u] = ld4(d.z, j / 4);
      }
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t j = j0 + 4 * 64 * u;
      const float4 sv = sk[KEEP > 0 ? k : 0][u];
      const float ss[4] = {sv.x, sv.y, sv.z, sv.w};
      float as[4] = {0.f, 0.f, 0.f, 0.f}, zs[4] = {0.f, 0.f, 0.f, 0.f};
      if (j < d.cols) {
        as[0] = a[u].x; as[1] = a[u].y; as[2] = a[u].z; as[3] = a[u].w;
        if constexpr (R1) {
          zs[0] = z[u].x; zs[1] = z[u].y; zs[2] = z[u].z; zs[3] = z[u].w;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = (ss[e] * b) * as[e];
        if constexpr (R1) x = fmaf(ku, zs[e], x);
        v[u][e] = live && j < d.cols ? x : 0.f;
      }
    }
  };
  if constexpr (!FLIP) {
    auto store = [&](int64_t j0, const float (&v)[kRowUnroll][4]) {
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        const int64_t j = j0 + 4 * 64 * u;
        if (j < J.pcol_pad) put_operand4(J.pl, i * J.pcol_pad + j, v[u], planes);
      }
    };
    if (kept) {
#pragma unroll
      for (int k = 0; k < (KEEP > 0 ? KEEP : 1); ++k) {
        const int64_t j0 = 4 * lane + static_cast<int64_t>(kWhitenChunk) * k;
        if (j0 < J.pcol_pad) {
          float v[kRowUnroll][4];
          batch_kept(k, j0, v);
          store(j0, v);
        }
      }
    } else {
      for (int64_t j0 = 4 * lane; j0 < J.pcol_pad; j0 += 4 * 64 * kRowUnroll) {
        float v[kRowUnroll][4];
        batch(j0, 4 * 64, v);
        store(j0, v);
      }
    }
  } else {
    static_assert(kWhitenChunk == 4 * 64 * kRowUnroll, "one batch per lane fills a chunk row");
    const int qq = threadIdx.x & 3;  // 4-row quarter of the K group
    // `kept` is uniform per block (one job per block), so the chunk loop and
    // its barriers are too.
    for (int64_t c0 = 0; c0 < J.pcol_pad; c0 += kWhitenChunk) {
      float v[kRowUnroll][4];
      if (kept) {
        const int k = static_cast<int>(c0 / kWhitenChunk);
#pragma unroll
        for (int kk = 0; kk < (KEEP > 0 ? KEEP : 1); ++kk)
          if (kk == k) batch_kept(kk, c0 + 4 * lane, v);
      } else {
        batch(c0 + 4 * lane, 4 * 64, v);
      }
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u)
        *reinterpret_cast<float4 *>(&tile[wave][4 * (lane + 64 * u)]) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
      __syncthreads();
#pragma unroll
      for (int r = 0; r < kWhitenChunk / 256; ++r) {
        const int jj = (threadIdx.x >> 2) + 256 * r;  // X row in the chunk
        if (c0 + jj < J.pcol_pad) {
          const float w[4] = {tile[4 * qq][jj], tile[4 * qq + 1][jj], tile[4 * qq + 2][jj], tile[4 * qq + 3][jj]};
          put_operand4(J.tl, (c0 + jj) * J.prow_pad + i0 + 4 * qq, w, planes);
        }
      }
      __syncthreads();
    }
  }
  // The partials of ||V||^2 (one per kPartRows rows, waves in order), after
  // pass 2 so that no barrier separates the passes.
  if (lane == 0) wave_part[wave] = part;
  __syncthreads();
  if (threadIdx.x < RB / kPartRows) {
    const int p = threadIdx.x;
    const int64_t r0 = i0 + p * kPartRows;
    if (r0 < d.rows) {
      double t = 0.0;
      for (int w = 0; w < kPartRows; ++w) t += wave_part[p * kPartRows + w];
      J.part[r0 / kPartRows] = t;
    }
  }
}

// ------------------------------------------------------------ mapback ---
// u_i = sum_j Q_ij z_j and ||U_i||^2 in closed form:
// b_i^2 (sum (a Q)^2 + 2 kappa u_i sum (a Q)(a z) + kappa^2 u_i^2 sum (a z)^2).
template <bool R1>
__global__ void __launch_bounds__(kMapThreads) mapback_rows_kernel(MatPack pack) {
  __shared__ double wave_part[kPartRows];
  const MatJob &J = pack.j[find_job(pack, blockIdx.x)];
  const smx_matrix_desc &d = J.d;
  const int blk = blockIdx.x - J.blk0;
  constexpr bool r1 = R1;
  const double cz = r1 ? J.cst[1] : 0.0;
  const double kappa = r1 ? d.kappa[0] : 0.0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool vec = d.cols % 4 == 0 && aligned16(d.inv_col) && (!r1 || aligned16(d.z));
  double part = 0.0;
  const int64_t i = static_cast<int64_t>(blk) * kPartRows + wave;
  if (i < d.rows) {
    const float *q = J.pl + i * J.pcol_pad;
    float su = 0.f, sa = 0.f, sb = 0.f;
    if (vec) {
      const int64_t n4 = d.cols / 4;
      for (int64_t k0 = lane; k0 < n4; k0 += 64 * kRowUnroll) {
        float4 qv[kRowUnroll], av[kRowUnroll], zv[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          const int64_t k = k0 + 64 * u;
          if (k < n4) {
            qv[u] = ld4(q, k);
            av[u] = ld4(d.inv_col, k);
            if constexpr (R1) zv[u] = ld4(d.z, k);
          }
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
          if (k0 + 64 * u < n4) {
            const float4 qq = qv[u], a = av[u];
            const float aq0 = a.x * qq.x, aq1 = a.y * qq.y, aq2 = a.z * qq.z, aq3 = a.w * qq.w;
            sa = fmaf(aq0, aq0, fmaf(aq1, aq1, fmaf(aq2, aq2, fmaf(aq3, aq3, sa))));
            if constexpr (R1) {
              const float4 z = zv[u];
              su = fmaf(qq.x, z.x, fmaf(qq.y, z.y, fmaf(qq.z, z.z, fmaf(qq.w, z.w, su))));
              sb = fmaf(aq0, a.x * z.x, fmaf(aq1, a.y * z.y, fmaf(aq2, a.z * z.z, fmaf(aq3, a.w * z.w, sb))));
            }
          }
        }
      }
    } else {
      for (int64_t j = lane; j < d.cols; j += 64) {
        const float a = d.inv_col[j];
        const float aq = a * q[j];
        sa = fmaf(aq, aq, sa);
        if (r1) {
          su = fmaf(q[j], d.z[j], su);
          sb = fmaf(aq, a * d.z[j], sb);
        }
      }
    }
    const double U = wave_sum(su);
    const double A = wave_sum(sa);
    const double B = wave_sum(sb);
    if (lane == 0) {
      const double b = d.inv_row[i];
      J.u[i] = static_cast<float>(U);
      part = b * b * (A + 2.0 * kappa * U * B + kappa * kappa * U * U * cz);
    }
  }
  const double t = sum_wave_parts<kPartRows>(part, wave_part);
  if (threadIdx.x == 0) J.part[blk] = t;
}

// W -= lr * sqrt(rows) / max(||U||_F, FLT_MIN) * U over kPartRows rows
// (one wave per row).  The first chunk of the row is loaded before the
// norm is summed, so the block does not wait on two memory round trips in
// a row.  A 16-bit parameter takes W = round(W - lr * round(direction))
// (sandmuon/optimizer.py:315) on the per-element path.
template <bool R1>
__global__ void __launch_bounds__(kMapThreads) mapback_apply_kernel(MatPack pack) {
  __shared__ double bcast;
  const MatJob &J = pack.j[find_job(pack, blockIdx.x)];
  const smx_matrix_desc &d = J.d;
  const int blk = blockIdx.x - J.blk0;
  constexpr bool r1 = R1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pdt = d.param_dtype;
  const bool vec = pdt == SMX_F32 && d.cols % 4 == 0 && aligned16(d.param) && aligned16(d.inv_col) &&
                   (!r1 || aligned16(d.z));
  const int64_t i = static_cast<int64_t>(blk) * kPartRows + wave;
  const bool live = i < d.rows;
  const float *q = live ? J.pl + i * J.pcol_pad : nullptr;
  float *w = live && pdt == SMX_F32 ? static_cast<float *>(d.param) + i * d.cols : nullptr;
  const int64_t n4 = d.cols / 4;
  float4 qv[kRowUnroll], av[kRowUnroll], wv[kRowUnroll], zv[kRowUnroll];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t k = k0 + 64 * u;
      if (k < n4) {
        qv[u] = ld4(q, k);
        av[u] = ld4(d.inv_col, k);
        wv[u] = ld4(w, k);
        if constexpr (R1) zv[u] = ld4(d.z, k);
      }
    }
  };
  if (live && vec) load(lane);
  if (threadIdx.x < 64) {
    double s = 0.0;
    const int np = static_cast<int>(ceil_div(d.rows, kPartRows));
    for (int k = threadIdx.x; k < np; k += 64) s += J.part[k];
    s = wave_sum(s);
    if (threadIdx.x == 0) bcast = s;
  }
  __syncthreads();
  const double n2 = bcast;
  const float norm = static_cast<float>(sqrt(n2));
  // _graft_direction: sqrt(rows) / max(||U||, FLT_MIN); a zero direction
  // gives a zero update.
  const float scale = n2 > 0.0 ? static_cast<float>(sqrt(static_cast<double>(d.rows))) / fmaxf(norm, FLT_MIN) : 0.f;
  const float nlr = static_cast<float>(-d.lr);
  const float kappa = r1 ? d.kappa[0] : 0.f;
  if (!live) return;
  const float b = d.inv_row[i];
  const float ku = r1 ? kappa * J.u[i] : 0.f;
  if (vec) {
    for (int64_t k0 = lane; k0 < n4; k0 += 64 * kRowUnroll) {
      if (k0 != lane) load(k0);  // the first chunk was loaded above
#pragma unroll
      for (int u = 0; u < kRowUnroll; ++u) {
        const int64_t k = k0 + 64 * u;
        if (k < n4) {
          float4 v = qv[u], ww = wv[u];
          const float4 a = av[u];
          if constexpr (R1) {
            const float4 z = zv[u];
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
    const int64_t row = i * d.cols;
    for (int64_t j = lane; j < d.cols; j += 64) {
      float v = q[j];
      if (r1) v = fmaf(ku, d.z[j], v);
      const float dir = round_to(pdt, ((v * b) * d.inv_col[j]) * scale);
      store_any(d.param, pdt, row + j, round_to(pdt, fmaf(nlr, dir, load_any(d.param, pdt, row + j))));
    }
  }
}

// --------------------------------------------------------------- host ---
struct Planned {
  S8Plan plan;
  std::vector<int32_t> cls, slot;
};

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
  return plan.bytes;
}

template <typename KernelFn>
static int launch_jobs(std::vector<MatJob> &jobs, int64_t (*blocks_of)(const MatJob &), KernelFn kernel,
                       int threads, const char *what, hipStream_t st) {
  for (size_t b = 0; b < jobs.size(); b += kMatBatch) {
    MatPack pack{};
    pack.n = static_cast<int32_t>(std::min<size_t>(kMatBatch, jobs.size() - b));
    int64_t total = 0;
    for (int k = 0; k < kMatBatch; ++k) pack.start[k] = INT32_MAX;
    for (int k = 0; k < pack.n; ++k) {
      pack.j[k] = jobs[b + k];
      pack.j[k].blk0 = static_cast<int32_t>(total);
      pack.start[k] = static_cast<int32_t>(total);
      total += blocks_of(pack.j[k]);
    }
    pack.total_blocks = static_cast<int32_t>(total);
    if (total == 0) continue;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(total)), dim3(threads), 0, st, pack);
    const int rc = check_launch(what);
    if (rc) return rc;
  }
  return SMX_OK;
}

static int64_t one_block(const MatJob &) { return 1; }
static int64_t map_blocks(const MatJob &j) { return ceil_div(j.d.rows, kPartRows); }
template <bool FLIP>
static int64_t whiten_blocks(const MatJob &j) { return j.prow_pad / whiten_rows_per_block<FLIP>(); }

// Whiten launches for the job lists bucketed by kept chunks (index KEEP).
template <int KEEP>
static int launch_whiten_keep(std::vector<MatJob> *keep, std::vector<MatJob> *flip, bool r1, hipStream_t st) {
  constexpr int kKeepThreads = 64 * whiten_rows_per_block<false>();
  int rc = SMX_OK;
  if (!keep[KEEP].empty())
    rc = r1 ? launch_jobs(keep[KEEP], whiten_blocks<false>, whiten_kernel<true, false, KEEP>, kKeepThreads, "whiten", st)
            : launch_jobs(keep[KEEP], whiten_blocks<false>, whiten_kernel<false, false, KEEP>, kKeepThreads, "whiten", st);
  if constexpr (KEEP <= kWhitenKeepFlip) {
    if (!rc && !flip[KEEP].empty())
      rc = r1 ? launch_jobs(flip[KEEP], whiten_blocks<true>, whiten_kernel<true, true, KEEP>, kRowThreads, "whiten", st)
              : launch_jobs(flip[KEEP], whiten_blocks<true>, whiten_kernel<false, true, KEEP>, kRowThreads, "whiten", st);
  }
  if constexpr (KEEP < kWhitenKeep) {
    if (!rc) rc = launch_whiten_keep<KEEP + 1>(keep, flip, r1, st);
  }
  return rc;
}

static int launch_whiten(std::vector<MatJob> *keep, std::vector<MatJob> *flip, bool r1, hipStream_t st) {
  return launch_whiten_keep<0>(keep, flip, r1, st);
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
  SMX_REQUIRE(mode == SMX_S8_FP32 || mode == SMX_S8_COMP_BF16, SMX_EINVAL, "matrix_step: unknown S8 mode");
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
    std::vector<MatJob> ping(m), fin(m);
    for (int32_t k = 0; k < m; ++k) {
      const S8Mat M{plan.layout.cls[cls[k]], slot[k]};
      MatJob j{};
      j.d = descs[g[k]];
      j.u = M.u();
      j.prow_pad = M.prow_pad();
      j.pcol_pad = M.pcol_pad();
      // The oriented iterate x0 is the parameter layout, or its transpose.
      j.pl = M.flip() ? nullptr : M.x0();
      j.tl = M.flip() ? M.x0() : nullptr;
      j.part = M.fro();
      j.cst = M.cst();
      j.planes = mode == SMX_S8_COMP_BF16;
      ping[k] = j;
      j.pl = M.result();
      j.tl = nullptr;
      j.part = M.mb();
      j.planes = 0;
      fin[k] = j;
    }
    // The kernels are specialised on whether the matrices carry a rank-one
    // term (all of a call or none, checked above).
    const bool r1 = descs[0].z != nullptr;
    // The rank-one constants (sum z^2, sum (a z)^2) exist only with a rank-one term.
    int rc = r1 ? launch_jobs(ping, one_block, matrix_consts_kernel, 256, "matrix_consts", st) : SMX_OK;
    // The whiten kernel is specialised on the orientation too: the jobs go
    // to two launches, parameters kept as they are and transposed ones,
    // and on how many kWhitenChunk column chunks of a row pass 1 keeps in
    // registers (rows of at most kWhitenKeep chunks, kWhitenKeepFlip for
    // transposed parameters; wider rows re-read).
    std::vector<MatJob> keep[kWhitenKeep + 1], flip[kWhitenKeep + 1];
    for (const MatJob &j : ping) {
      const int64_t chunks = ceil_div(j.d.cols, kWhitenChunk);
      const int64_t most = j.tl ? kWhitenKeepFlip : kWhitenKeep;
      (j.tl ? flip : keep)[chunks <= most ? chunks : 0].push_back(j);
    }
    if (!rc) rc = launch_whiten(keep, flip, r1, st);
    if (!rc) rc = run_s8_stages(plan.layout, st);
    if (!rc) rc = r1 ? launch_jobs(fin, map_blocks, mapback_rows_kernel<true>, kMapThreads, "mapback_rows", st)
                     : launch_jobs(fin, map_blocks, mapback_rows_kernel<false>, kMapThreads, "mapback_rows", st);
    if (!rc) rc = r1 ? launch_jobs(fin, map_blocks, mapback_apply_kernel<true>, kMapThreads, "mapback_apply", st)
                     : launch_jobs(fin, map_blocks, mapback_apply_kernel<false>, kMapThreads, "mapback_apply", st);
    if (rc) return rc;
  }
  return SMX_OK;
}
