// The module-level helpers of sandmuon/optimizer.py, in the dtype of their
// inputs (FP32 or FP64, as the reference computes them):
//   diagonal_inverse_sqrt (:19-24) and rank1_inverse_sqrt (:27-35)
//                         -> smx_inverse_sqrt (one block per vector);
//   rank1_whiten (:38-45) and rank1_mapback (:48-60) -> smx_rank1_apply;
//   _graft_direction (:63-66) -> smx_graft (FP32, as the reference).
// The optimizer's own step uses the fused one-sided kernels of matrix.hip
// and the batched finish of stats.hip; these entry points serve direct
// calls of the helpers.
//
// rank1_apply, with t_j = sum_i lz_i V_ij and u_i = sum_j V_ij rz_j (sums in
// FP64, rounded to T):
//   whiten  (order 0): V0 = (X li) ri;  V1 = V0 + (lc lz_i) t_j;
//                      out = V1 + (rc u_i) rz_j
//   mapback (order 1): V1 = X + (lc lz_i) t_j;  V2 = V1 + (rc u_i) rz_j;
//                      out = (V2 li) ri
// in three launches: column sums (threads over columns, rows walked in
// order: coalesced), row sums (one wave per row), elementwise output.
#include "common.h"

#include <algorithm>
#include <cfloat>
#include <cmath>

namespace smx {

template <typename T>
struct Rank1Args {
  const T *x;
  T *out;
  int64_t rows, cols;
  const T *li, *lz, *lc;  // [batch][rows], [batch][rows], [batch]
  const T *ri, *rz, *rc;  // [batch][cols], [batch][cols], [batch]
  double *t;              // [batch][cols] column sums lz^T V
  double *u;              // [batch][rows] row sums V1 rz
  int32_t order;
};

// The first-stage value V0 (whiten) or X (mapback) of element (i, j).
template <typename T>
__device__ __forceinline__ T r1_v0(const Rank1Args<T> &a, int64_t b, int64_t i, int64_t j) {
  const T x = a.x[(b * a.rows + i) * a.cols + j];
  return a.order == 0 ? (x * a.li[b * a.rows + i]) * a.ri[b * a.cols + j] : x;
}

// V1 of element (i, j): V0 + (lc lz_i) t_j.
template <typename T>
__device__ __forceinline__ T r1_v1(const Rank1Args<T> &a, int64_t b, int64_t i, int64_t j) {
  const T t = static_cast<T>(a.t[b * a.cols + j]);
  return r1_v0(a, b, i, j) + (a.lc[b] * a.lz[b * a.rows + i]) * t;
}

// t[b][j] = sum_i lz_i V0_ij; grid (ceil(cols / 256), batch).
template <typename T>
__global__ void __launch_bounds__(256) rank1_colsum_kernel(Rank1Args<T> a) {
  const int64_t b = blockIdx.y;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (j >= a.cols) return;
  double s = 0.0;
  for (int64_t i = 0; i < a.rows; ++i)
    s += static_cast<double>(a.lz[b * a.rows + i]) * static_cast<double>(r1_v0(a, b, i, j));
  a.t[b * a.cols + j] = s;
}

// u[b][i] = sum_j V1_ij rz_j, one wave per row; grid (ceil(rows / 4), batch).
template <typename T>
__global__ void __launch_bounds__(256) rank1_rowsum_kernel(Rank1Args<T> a) {
  const int64_t b = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= a.rows) return;  // wave-uniform
  double s = 0.0;
  for (int64_t j = lane; j < a.cols; j += 64)
    s += static_cast<double>(r1_v1(a, b, i, j)) * static_cast<double>(a.rz[b * a.cols + j]);
  s = wave_sum(s);
  if (lane == 0) a.u[b * a.rows + i] = s;
}

// Elementwise output; grid (ceil(rows * cols / 256), batch).
template <typename T>
__global__ void __launch_bounds__(256) rank1_out_kernel(Rank1Args<T> a) {
  const int64_t b = blockIdx.y;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= a.rows * a.cols) return;
  const int64_t i = e / a.cols, j = e % a.cols;
  const T u = static_cast<T>(a.u[b * a.rows + i]);
  T v = r1_v1(a, b, i, j) + (a.rc[b] * u) * a.rz[b * a.cols + j];
  if (a.order == 1) v = (v * a.li[b * a.rows + i]) * a.ri[b * a.cols + j];
  a.out[b * a.rows * a.cols + e] = v;
}

template <typename T>
static int launch_rank1(const Rank1Args<T> &a, int64_t batch, hipStream_t st) {
  const unsigned nb = static_cast<unsigned>(batch);
  hipLaunchKernelGGL(rank1_colsum_kernel<T>, dim3(static_cast<unsigned>(ceil_div(a.cols, 256)), nb), dim3(256), 0,
                     st, a);
  int rc = check_launch("rank1_apply column sums");
  if (rc) return rc;
  hipLaunchKernelGGL(rank1_rowsum_kernel<T>, dim3(static_cast<unsigned>(ceil_div(a.rows, 4)), nb), dim3(256), 0, st,
                     a);
  rc = check_launch("rank1_apply row sums");
  if (rc) return rc;
  hipLaunchKernelGGL(rank1_out_kernel<T>, dim3(static_cast<unsigned>(ceil_div(a.rows * a.cols, 256)), nb), dim3(256),
                     0, st, a);
  return check_launch("rank1_apply output");
}

// ---------------------------------------------------- inverse sqrt ---
template <typename T>
__device__ __forceinline__ T rsqrt_t(T v);
template <>
__device__ __forceinline__ float rsqrt_t<float>(float v) { return rsqrtf(v); }
template <>
__device__ __forceinline__ double rsqrt_t<double>(double v) { return 1.0 / sqrt(v); }

template <typename T>
constexpr T tiny_t() { return sizeof(T) == 4 ? static_cast<T>(FLT_MIN) : static_cast<T>(DBL_MIN); }

// One block of 1024 threads per vector.  Means and sum z^2 in FP64,
// rounded to T where the reference holds them in T.
template <typename T>
__global__ void __launch_bounds__(1024) inverse_sqrt_kernel(int kind, const T *second, const T *mean, int64_t n,
                                                             T *inv, T *z, T *kappa) {
  __shared__ double scratch[16];
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < n; c += blockDim.x) s += static_cast<double>(second[c]);
  const T m = static_cast<T>(block_sum(s, scratch) / static_cast<double>(n));
  if (kind == 0) {
    const T floor = m * static_cast<T>(1e-6);
    const T den = m > tiny_t<T>() ? m : tiny_t<T>();
    for (int64_t c = threadIdx.x; c < n; c += blockDim.x) {
      const T v = second[c] > floor ? second[c] : floor;
      const T r = v / den;
      inv[c] = rsqrt_t<T>(r > static_cast<T>(1e-6) ? r : static_cast<T>(1e-6));
    }
    return;
  }
  const T q = m > tiny_t<T>() ? m : tiny_t<T>();
  const T sq = sqrt(q);
  double zpart = 0.0;
  for (int64_t c = threadIdx.x; c < n; c += blockDim.x) {
    const T mc = mean[c];
    T var = second[c] - mc * mc;
    var = var > static_cast<T>(0) ? var : static_cast<T>(0);
    const T r = var / q;
    const T iv = rsqrt_t<T>(r > static_cast<T>(1e-6) ? r : static_cast<T>(1e-6));
    const T zc = iv * (mc / sq);
    inv[c] = iv;
    z[c] = zc;
    zpart += static_cast<double>(zc) * static_cast<double>(zc);
  }
  const T zz = static_cast<T>(block_sum(zpart, scratch));
  if (threadIdx.x == 0) {
    const T rho = sqrt(static_cast<T>(1) + zz);
    kappa[0] = static_cast<T>(-1) / (rho * (rho + static_cast<T>(1)));
  }
}

// ------------------------------------------------------------- graft ---
// out = x * sqrt(rows) / max(||x||_F, FLT_MIN) (zero stays zero).
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

extern "C" int smx_inverse_sqrt(int kind, int dtype, const void *second, const void *mean, int64_t n, void *inv,
                                void *z, void *kappa, void *stream) {
  SMX_REQUIRE(kind == 0 || kind == 1, SMX_EINVAL, "inverse_sqrt: kind must be 0 (diagonal) or 1 (rank-one)");
  SMX_REQUIRE(dtype == SMX_F32 || dtype == SMX_F64, SMX_EDTYPE, "inverse_sqrt: dtype must be f32 or f64");
  SMX_REQUIRE(n >= 1, SMX_ESHAPE, "inverse_sqrt: n must be >= 1");
  SMX_REQUIRE(second && inv, SMX_EINVAL, "inverse_sqrt: null pointer");
  SMX_REQUIRE(kind == 0 || (mean && z && kappa), SMX_EINVAL, "inverse_sqrt: rank-one needs mean, z and kappa");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SMX_F32)
    hipLaunchKernelGGL(inverse_sqrt_kernel<float>, dim3(1), dim3(1024), 0, st, kind,
                       static_cast<const float *>(second), static_cast<const float *>(mean), n,
                       static_cast<float *>(inv), static_cast<float *>(z), static_cast<float *>(kappa));
  else
    hipLaunchKernelGGL(inverse_sqrt_kernel<double>, dim3(1), dim3(1024), 0, st, kind,
                       static_cast<const double *>(second), static_cast<const double *>(mean), n,
                       static_cast<double *>(inv), static_cast<double *>(z), static_cast<double *>(kappa));
  return check_launch("inverse_sqrt");
}

extern "C" int smx_rank1_apply(int dtype, const void *x, void *out, int64_t batch, int64_t rows, int64_t cols,
                               const void *li, const void *lz, const void *lc, const void *ri, const void *rz,
                               const void *rc, int order, double *work, void *stream) {
  SMX_REQUIRE(dtype == SMX_F32 || dtype == SMX_F64, SMX_EDTYPE, "rank1_apply: dtype must be f32 or f64");
  SMX_REQUIRE(x && out && li && lz && lc && ri && rz && rc && work, SMX_EINVAL, "rank1_apply: null pointer");
  SMX_REQUIRE(order == 0 || order == 1, SMX_EINVAL, "rank1_apply: order must be 0 (whiten) or 1 (mapback)");
  SMX_REQUIRE(batch >= 0 && rows >= 1 && cols >= 1 && batch <= 65535, SMX_ESHAPE, "rank1_apply: bad shape");
  SMX_REQUIRE(ceil_div(rows * cols, 256) <= 0x7fffffff, SMX_ESHAPE, "rank1_apply: matrix too large");
  SMX_REQUIRE(out != x, SMX_EINVAL, "rank1_apply: out must not alias x");
  if (batch == 0) return SMX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  double *t = work, *u = work + batch * cols;
  if (dtype == SMX_F32) {
    Rank1Args<float> a{static_cast<const float *>(x), static_cast<float *>(out), rows, cols,
                       static_cast<const float *>(li), static_cast<const float *>(lz), static_cast<const float *>(lc),
                       static_cast<const float *>(ri), static_cast<const float *>(rz), static_cast<const float *>(rc),
                       t, u, order};
    return launch_rank1(a, batch, st);
  }
  Rank1Args<double> a{static_cast<const double *>(x), static_cast<double *>(out), rows, cols,
                      static_cast<const double *>(li), static_cast<const double *>(lz),
                      static_cast<const double *>(lc), static_cast<const double *>(ri),
                      static_cast<const double *>(rz), static_cast<const double *>(rc), t, u, order};
  return launch_rank1(a, batch, st);
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
