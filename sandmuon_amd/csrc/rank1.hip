// Generic rank-one whitening / mapback on a batch, and the Frobenius graft:
// the module-level helpers rank1_whiten (sandmuon/optimizer.py:38-45),
// rank1_mapback (:48-60) and _graft_direction (:63-66).  The optimizer's
// own step uses the fused one-sided kernels of matrix.hip; these entry
// points serve direct calls of the helpers with both sides non-trivial.
//
// whiten  (order 0): V0 = X * (li x ri); V1 = V0 + lc lz (lz^T V0);
//                    out = V1 + rc (V1 rz) rz^T
// mapback (order 1): V1 = X + lc lz (lz^T X); V2 = V1 + rc (V1 rz) rz^T;
//                    out = V2 * (li x ri)
#include "common.h"

#include <algorithm>
#include <cfloat>
#include <cmath>

namespace smx {

struct Rank1Args {
  const float *x;
  float *out;
  int64_t rows, cols;
  const float *li, *lz, *lc;  // [batch][rows], [batch][rows], [batch]
  const float *ri, *rz, *rc;  // [batch][cols], [batch][cols], [batch]
  float *work;                // [batch][rows + cols]
  int32_t order;
};

// One block (256 threads) per matrix; grid.x = batch.
__global__ void __launch_bounds__(256) rank1_apply_kernel(Rank1Args a) {
  const int64_t b = blockIdx.x;
  const int64_t R = a.rows, C = a.cols;
  const float *x = a.x + b * R * C;
  float *out = a.out + b * R * C;
  const float *li = a.li + b * R, *lz = a.lz + b * R;
  const float *ri = a.ri + b * C, *rz = a.rz + b * C;
  const float lc = a.lc[b], rc = a.rc[b];
  float *t = a.work + b * (R + C);  // [C] column sums lz^T V
  float *u = t + C;                 // [R] row sums V1 rz
  const bool w = a.order == 0;
  auto v0 = [&](int64_t i, int64_t j) { return w ? (x[i * C + j] * li[i]) * ri[j] : x[i * C + j]; };
  for (int64_t j = threadIdx.x; j < C; j += 256) {
    double s = 0.0;
    for (int64_t i = 0; i < R; ++i) s += static_cast<double>(lz[i]) * v0(i, j);
    t[j] = static_cast<float>(s);
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < R; i += 256) {
    double s = 0.0;
    for (int64_t j = 0; j < C; ++j) s += static_cast<double>(v0(i, j) + lc * lz[i] * t[j]) * rz[j];
    u[i] = static_cast<float>(s);
  }
  __syncthreads();
  for (int64_t e = threadIdx.x; e < R * C; e += 256) {
    const int64_t i = e / C, j = e % C;
    float v = v0(i, j) + lc * lz[i] * t[j];
    v = v + rc * u[i] * rz[j];
    out[e] = w ? v : (v * li[i]) * ri[j];
  }
}

// Graft: out = x * sqrt(rows) / max(||x||_F, FLT_MIN) (zero stays zero).
// Pass 1: per-block partial sums of squares; pass 2: scale.
__global__ void __launch_bounds__(256) graft_partial_kernel(const float *x, int64_t n, double *parts) {
  __shared__ double scratch[16];
  double s = 0.0;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n; e += static_cast<int64_t>(gridDim.x) * 256) {
    const double v = x[e];
    s += v * v;
  }
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) parts[blockIdx.x] = s;
}

__global__ void __launch_bounds__(256) graft_scale_kernel(const float *x, float *out, int64_t n, const double *parts,
                                                          int nparts, float sqrt_rows) {
  __shared__ double bcast;
  if (threadIdx.x < 64) {
    double s = 0.0;
    for (int k = threadIdx.x; k < nparts; k += 64) s += parts[k];
    s = wave_sum(s);
    if (threadIdx.x == 0) bcast = s;
  }
  __syncthreads();
  const double n2 = bcast;
  const float scale = n2 > 0.0 ? sqrt_rows / fmaxf(static_cast<float>(sqrt(n2)), FLT_MIN) : 0.f;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n; e += static_cast<int64_t>(gridDim.x) * 256)
    out[e] = x[e] * scale;
}

}  // namespace smx

using namespace smx;

extern "C" int smx_rank1_apply(const float *x, float *out, int64_t batch, int64_t rows, int64_t cols,
                               const float *li, const float *lz, const float *lc, const float *ri, const float *rz,
                               const float *rc, int order, float *work, void *stream) {
  SMX_REQUIRE(x && out && li && lz && lc && ri && rz && rc && work, SMX_EINVAL, "rank1_apply: null pointer");
  SMX_REQUIRE(order == 0 || order == 1, SMX_EINVAL, "rank1_apply: order must be 0 (whiten) or 1 (mapback)");
  SMX_REQUIRE(batch >= 0 && rows >= 1 && cols >= 1 && batch <= 0x7fffffff, SMX_ESHAPE, "rank1_apply: bad shape");
  SMX_REQUIRE(out != x, SMX_EINVAL, "rank1_apply: out must not alias x");
  if (batch == 0) return SMX_OK;
  Rank1Args a{x, out, rows, cols, li, lz, lc, ri, rz, rc, work, order};
  hipLaunchKernelGGL(rank1_apply_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("rank1_apply");
}

extern "C" int smx_graft(const float *x, float *out, int64_t n, int64_t output_rows, double *work, int32_t work_len,
                         void *stream) {
  SMX_REQUIRE(x && out && work, SMX_EINVAL, "graft: null pointer");
  SMX_REQUIRE(n >= 0 && output_rows >= 0 && work_len >= 1, SMX_ESHAPE, "graft: bad size");
  if (n == 0) return SMX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = static_cast<int>(std::min<int64_t>(work_len, std::min<int64_t>(1024, ceil_div(n, 256))));
  hipLaunchKernelGGL(graft_partial_kernel, dim3(nb), dim3(256), 0, st, x, n, work);
  int rc = check_launch("graft partial");
  if (rc) return rc;
  hipLaunchKernelGGL(graft_scale_kernel, dim3(nb), dim3(256), 0, st, x, out, n, work, nb,
                     static_cast<float>(std::sqrt(static_cast<double>(output_rows))));
  return check_launch("graft scale");
}
