// AdamW on the auxiliary (non-matrix) parameters, all tensors in one
// flattened launch: sandmuon/optimizer.py:268-281.
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
//   u = (m / bias1) / (sqrt(v / bias2) + eps)
//   p = p (1 - lr wd);  p = p - lr u
#include "common.h"

#include <algorithm>
#include <cmath>

namespace smx {

constexpr int kAdamBatch = 32;
constexpr int kAdamChunk = 2048;  // elements per block

struct AdamPack {
  smx_adamw_desc d[kAdamBatch];
  int32_t n;
  int64_t total;
  float neg_lr, decay, b1, omb1, b2, omb2, eps;
};

__global__ void __launch_bounds__(256) adamw_kernel(AdamPack pk) {
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kAdamChunk;
  const int64_t e1 = min(pk.total, e0 + kAdamChunk);
  // Tensor holding e0 (offsets are ascending).
  int k = 0;
  while (k + 1 < pk.n && pk.d[k + 1].offset <= e0) ++k;
  for (; k < pk.n && pk.d[k].offset < e1; ++k) {
    const smx_adamw_desc &d = pk.d[k];
    const int64_t lo = max(e0, d.offset) - d.offset;
    const int64_t hi = min(e1, d.offset + d.n) - d.offset;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
      float g;
      if (d.grad_dtype == SMX_F32) g = static_cast<const float *>(d.grad)[i];
      else if (d.grad_dtype == SMX_BF16) g = load_elem<SMX_BF16>(d.grad, i);
      else g = load_elem<SMX_F16>(d.grad, i);
      const float m = d.exp_avg[i] * pk.b1 + g * pk.omb1;
      const float v = d.exp_avg_sq[i] * pk.b2 + (g * g) * pk.omb2;
      d.exp_avg[i] = m;
      d.exp_avg_sq[i] = v;
      const float u = (m / d.bias1) / (sqrtf(v / d.bias2) + pk.eps);
      const float p = d.param[i] * pk.decay;
      d.param[i] = p + pk.neg_lr * u;
    }
  }
}

}  // namespace smx

using namespace smx;

extern "C" int smx_adamw(const smx_adamw_desc *descs, int32_t n_desc, int64_t total, double lr, double beta1,
                         double beta2, double eps, double weight_decay, void *stream) {
  SMX_REQUIRE(n_desc >= 0 && (n_desc == 0 || descs), SMX_EINVAL, "adamw: bad descriptor table");
  int64_t sum = 0;
  for (int32_t i = 0; i < n_desc; ++i) {
    const smx_adamw_desc &d = descs[i];
    SMX_REQUIRE(d.param && d.grad && d.exp_avg && d.exp_avg_sq, SMX_EINVAL, "adamw: null pointer");
    SMX_REQUIRE(d.n >= 0 && d.offset == sum, SMX_ESHAPE, "adamw: offsets must be the prefix sums of n");
    SMX_REQUIRE(d.grad_dtype == SMX_F32 || d.grad_dtype == SMX_BF16 || d.grad_dtype == SMX_F16, SMX_EDTYPE,
                "adamw: grad dtype must be f32, bf16 or f16");
    SMX_REQUIRE(d.bias1 > 0.f && d.bias2 > 0.f, SMX_EINVAL, "adamw: bias corrections must be positive");
    sum += d.n;
  }
  SMX_REQUIRE(sum == total, SMX_ESHAPE, "adamw: total != sum of n");
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int32_t b = 0; b < n_desc; b += kAdamBatch) {
    AdamPack pk{};
    pk.n = std::min<int32_t>(kAdamBatch, n_desc - b);
    const int64_t base = descs[b].offset;
    for (int i = 0; i < pk.n; ++i) {
      pk.d[i] = descs[b + i];
      pk.d[i].offset -= base;
    }
    pk.total = pk.d[pk.n - 1].offset + pk.d[pk.n - 1].n;
    // Each FP32 coefficient is rounded from the double the reference
    // computes in Python (1 - lr*wd, 1 - beta, -lr).
    pk.neg_lr = static_cast<float>(-lr);
    pk.decay = static_cast<float>(1.0 - lr * weight_decay);
    pk.b1 = static_cast<float>(beta1);
    pk.omb1 = static_cast<float>(1.0 - beta1);
    pk.b2 = static_cast<float>(beta2);
    pk.omb2 = static_cast<float>(1.0 - beta2);
    pk.eps = static_cast<float>(eps);
    if (pk.total == 0) continue;
    hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(ceil_div(pk.total, kAdamChunk))), dim3(256),
                       0, st, pk);
    const int rc = check_launch("adamw");
    if (rc) return rc;
  }
  return SMX_OK;
}
