// Stand-alone S8 polar map on a strided batch (the module-level _s8_fp32
// helper of sandmuon/optimizer.py:69-93): load -> five stages -> store.
#include "s8.h"

#include <memory>
#include <vector>

namespace smx {

struct S8IoArgs {
  S8Class k;
  const float *x;
  float *out;
  int64_t rows, cols;          // input (= output) shape per matrix
  int64_t sb, sr, sc;          // element strides: batch, row, col
  int32_t planes;              // iterate stored as BF16 planes (comp mode)
};

// Norm pass: the input's sum of squares (FP64) -> the matrix's kCstFro.
// grid = (1, batch), block 256.
__global__ void __launch_bounds__(256) s8_load_norm_kernel(S8IoArgs a) {
  __shared__ double scratch[16];
  const S8Mat M{a.k, static_cast<int32_t>(blockIdx.y)};
  const float *x = a.x + static_cast<int64_t>(blockIdx.y) * a.sb;
  double s = 0.0;
  for (int64_t i = 0; i < a.rows; ++i)
    for (int64_t j = threadIdx.x; j < a.cols; j += 256) {
      const double v = x[i * a.sr + j * a.sc];
      s += v * v;
    }
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) M.cst()[kCstFro] = s;
}

// Tile pass: 64x64 tiles of the padded parameter layout (input layout)
// into the oriented iterate x0 (a tiled operand): directly, or transposed
// through LDS for transposed parameters.  grid = (tiles, batch), block 256.
__global__ void __launch_bounds__(256) s8_load_tiles_kernel(S8IoArgs a) {
  __shared__ float tile[64][65];
  const S8Mat M{a.k, static_cast<int32_t>(blockIdx.y)};
  const float *x = a.x + static_cast<int64_t>(blockIdx.y) * a.sb;
  float *pl = M.flip() ? nullptr : M.x0();
  float *tl = M.flip() ? M.x0() : nullptr;
  const int64_t ppad = M.pcol_pad(), rpad = M.prow_pad();
  const int64_t tiles_c = ppad / 64;
  const int64_t i0 = (blockIdx.x / tiles_c) * 64, j0 = (blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x, lc = (t & 15) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int lr = (t >> 4) + 16 * q;
    const int64_t i = i0 + lr;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t j = j0 + lc + e;
      v[e] = (i < a.rows && j < a.cols) ? x[i * a.sr + j * a.sc] : 0.f;
      tile[lr][lc + e] = v[e];
    }
    if (pl) put_operand4(pl, tiled_index(i, j0 + lc, ppad), v, a.planes != 0);
  }
  if (!tl) return;  // uniform per block
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int lr = (t >> 4) + 16 * q;
    const float v[4] = {tile[lc][lr], tile[lc + 1][lr], tile[lc + 2][lr], tile[lc + 3][lr]};
    put_operand4(tl, tiled_index(j0 + lr, i0 + lc, rpad), v, a.planes != 0);
  }
}

// Store: final iterate (parameter layout) -> out (strided).
// grid = (ceil(rows*cols / 256), batch).
__global__ void __launch_bounds__(256) s8_store_kernel(S8IoArgs a) {
  const S8Mat M{a.k, static_cast<int32_t>(blockIdx.y)};
  const float *q = M.result();
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= a.rows * a.cols) return;
  const int64_t i = e / a.cols, j = e % a.cols;
  a.out[static_cast<int64_t>(blockIdx.y) * a.sb + i * a.sr + j * a.sc] = q[i * M.pcol_pad() + j];
}

}  // namespace smx

using namespace smx;

static bool plan_single(int64_t batch, int64_t rows, int64_t cols, int mode, char *base, S8Plan &plan) {
  const bool flip = rows > cols;
  std::vector<int64_t> r(batch, flip ? cols : rows), c(batch, flip ? rows : cols);
  std::unique_ptr<bool[]> f(new bool[batch]);
  for (int64_t i = 0; i < batch; ++i) f[i] = flip;
  std::vector<int32_t> cls(batch), slot(batch);
  return plan_s8(r.data(), c.data(), f.get(), static_cast<int32_t>(batch), mode, base, plan, cls.data(),
                 slot.data());
}

extern "C" size_t smx_s8_workspace_bytes(int64_t batch, int64_t rows, int64_t cols, int mode) {
  if (batch < 1 || rows < 1 || cols < 1) return 0;
  S8Plan plan;
  plan_single(batch, rows, cols, mode, nullptr, plan);
  return plan.bytes;
}

extern "C" int smx_s8(const float *x, float *out, int64_t batch, int64_t rows, int64_t cols, int64_t batch_stride,
                      int64_t row_stride, int64_t col_stride, int mode, void *workspace, size_t workspace_bytes,
                      void *stream) {
  SMX_REQUIRE(x && out, SMX_EINVAL, "s8: null pointer");
  SMX_REQUIRE(mode == SMX_S8_FP32 || mode == SMX_S8_COMP_BF16 || mode == SMX_S8_MIXED, SMX_EINVAL,
              "s8: unknown mode");
  SMX_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, SMX_ESHAPE, "s8: negative shape");
  SMX_REQUIRE(batch <= 65535, SMX_ESHAPE, "s8: batch must be <= 65535");
  if (batch == 0 || rows == 0 || cols == 0) return SMX_OK;
  SMX_REQUIRE(workspace, SMX_EINVAL, "s8: null workspace");
  SMX_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SMX_EALIGN, "s8: workspace must be 256-byte aligned");
  S8Plan plan;
  plan_single(batch, rows, cols, mode, static_cast<char *>(workspace), plan);
  SMX_REQUIRE(workspace_bytes >= plan.bytes, SMX_EWORKSPACE, "s8: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  S8IoArgs a{};
  a.k = plan.layout.cls[0];
  a.x = x;
  a.out = out;
  a.rows = rows;
  a.cols = cols;
  a.sb = batch_stride;
  a.sr = row_stride;
  a.sc = col_stride;
  a.planes = mode != SMX_S8_FP32;  // stage 1 reads X0 compensated in both BF16 modes
  const S8Mat M0{a.k, 0};
  const unsigned tiles = static_cast<unsigned>((M0.prow_pad() / 64) * (M0.pcol_pad() / 64));
  hipLaunchKernelGGL(s8_load_norm_kernel, dim3(1, batch), dim3(256), 0, st, a);
  int rc = check_launch("s8 load norm");
  if (rc) return rc;
  hipLaunchKernelGGL(s8_load_tiles_kernel, dim3(tiles, batch), dim3(256), 0, st, a);
  rc = check_launch("s8 load tiles");
  if (rc) return rc;
  rc = run_s8_stages(plan.layout, st);
  if (rc) return rc;
  hipLaunchKernelGGL(s8_store_kernel, dim3(static_cast<unsigned>(ceil_div(rows * cols, 256)), batch), dim3(256),
                     0, st, a);
  return check_launch("s8 store");
}
