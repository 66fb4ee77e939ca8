// AdamW on the auxiliary (non-matrix) parameters, all tensors in one
// flattened launch: sandmuon/optimizer.py:268-281.
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
//   u = (m / bias1) / (sqrt(v / bias2) + eps)
//   p = p (1 - lr wd);  p = p - lr u
// A 16-bit parameter is rounded to its dtype after each of the two
// parameter updates and u before the second, as the reference's in-place
// mul_ and add_(u.to(p.dtype)) on that dtype do (:280-281).
#include "common.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>

namespace smx {

constexpr int kAdamBatch = 56;
constexpr int kAdamMaxChunk = 2048;  // elements per block (large launches)
constexpr int kAdamUnroll = 4;
constexpr int kAdamVec = 2;  // float4 per thread per pass (FP32 tensors)

// The scalars of one launch: its element count and block chunk, and the
// FP32 coefficients.
struct AdamScalars {
  int32_t n;
  int64_t total;
  int64_t chunk;
  float neg_lr, decay, b1, omb1, b2, omb2, eps;
};
struct AdamPack {
  int32_t first_blk[kAdamBatch];  // ceil(offset / chunk); INT32_MAX past the last
  smx_adamw_desc d[kAdamBatch];
  AdamScalars sc;
};
static_assert(sizeof(AdamPack) <= 4000, "AdamPack is passed by value in the kernel arguments");

// Elements per block: short chunks for small launches (the biases and norms
// left after the embeddings), so they spread over more CUs instead of
// queueing behind each other in a few blocks.
static int64_t adam_chunk(int64_t total) {
  return std::min<int64_t>(kAdamMaxChunk, std::max<int64_t>(256, ceil_div(ceil_div(total, 2048), 256) * 256));
}

__device__ __forceinline__ bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The moments and the step of one element, with explicit fused
// multiply-adds so that every code path rounds the same way.
__device__ __forceinline__ float adam_step(const AdamScalars &pk, const smx_adamw_desc &d, float g, float &m, float &v) {
  m = fmaf(m, pk.b1, g * pk.omb1);
  v = fmaf(v, pk.b2, (g * g) * pk.omb2);
  return (m / d.bias1) / (sqrtf(v / d.bias2) + pk.eps);
}

// One element of the FP32 update.
__device__ __forceinline__ void adam_f32(const AdamScalars &pk, const smx_adamw_desc &d, float g, float &m, float &v,
                                         float &p) {
  const float step = adam_step(pk, d, g, m, v);
  p = fmaf(pk.neg_lr, step, p * pk.decay);
}

// The block's elements [e0, e1) of the flattened tensors, from tensor k (the
// last whose offset is <= e0) on; desc(k) gives tensor k's descriptor.
template <class Desc>
__device__ __forceinline__ void adamw_block(const AdamScalars &pk, Desc desc, int k) {
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * pk.chunk;
  const int64_t e1 = min(pk.total, e0 + pk.chunk);
  for (; k < pk.n; ++k) {
    const smx_adamw_desc d = desc(k);
    if (d.offset >= e1) break;
    int64_t lo = max(e0, d.offset) - d.offset;
    const int64_t hi = min(e1, d.offset + d.n) - d.offset;
    // FP32 tensors whose block range starts on a 16-byte boundary: float4
    // loads and stores, kAdamVec per thread in flight; the scalar loop
    // below takes the tail.
    if (d.param_dtype == SMX_F32 && d.grad_dtype == SMX_F32 && (lo & 3) == 0 && aligned16(d.param) &&
        aligned16(d.grad) && aligned16(d.exp_avg) && aligned16(d.exp_avg_sq)) {
      const int64_t lo4 = lo / 4, hi4 = hi / 4;
      const float4 *G = static_cast<const float4 *>(d.grad);
      float4 *P = static_cast<float4 *>(d.param);
      float4 *M = reinterpret_cast<float4 *>(d.exp_avg);
      float4 *V = reinterpret_cast<float4 *>(d.exp_avg_sq);
      for (int64_t q0 = lo4 + threadIdx.x; q0 < hi4; q0 += 256 * kAdamVec) {
        float4 g[kAdamVec], m[kAdamVec], v[kAdamVec], p[kAdamVec];
#pragma unroll
        for (int u = 0; u < kAdamVec; ++u) {
          const int64_t q = q0 + 256 * u;
          if (q < hi4) {
            g[u] = G[q];
            m[u] = M[q];
            v[u] = V[q];
            p[u] = P[q];
          }
        }
#pragma unroll
        for (int u = 0; u < kAdamVec; ++u) {
          const int64_t q = q0 + 256 * u;
          if (q < hi4) {
            adam_f32(pk, d, g[u].x, m[u].x, v[u].x, p[u].x);
            adam_f32(pk, d, g[u].y, m[u].y, v[u].y, p[u].y);
            adam_f32(pk, d, g[u].z, m[u].z, v[u].z, p[u].z);
            adam_f32(pk, d, g[u].w, m[u].w, v[u].w, p[u].w);
            M[q] = m[u];
            V[q] = v[u];
            P[q] = p[u];
          }
        }
      }
      lo = hi4 * 4;
    }
    // kAdamUnroll elements per thread per pass, all loaded before any is
    // updated, so a block over small tensors is not one latency per element.
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 256 * kAdamUnroll) {
      float g[kAdamUnroll], m[kAdamUnroll], v[kAdamUnroll], p[kAdamUnroll];
#pragma unroll
      for (int u = 0; u < kAdamUnroll; ++u) {
        const int64_t i = i0 + u * 256;
        if (i < hi) {
          if (d.grad_dtype == SMX_F32) g[u] = static_cast<const float *>(d.grad)[i];
          else if (d.grad_dtype == SMX_BF16) g[u] = load_elem<SMX_BF16>(d.grad, i);
          else g[u] = load_elem<SMX_F16>(d.grad, i);
          m[u] = d.exp_avg[i];
          v[u] = d.exp_avg_sq[i];
          p[u] = d.param_dtype == SMX_F32 ? static_cast<const float *>(d.param)[i] : load_any(d.param, d.param_dtype, i);
        }
      }
#pragma unroll
      for (int u = 0; u < kAdamUnroll; ++u) {
        const int64_t i = i0 + u * 256;
        if (i < hi) {
          if (d.param_dtype == SMX_F32) {
            adam_f32(pk, d, g[u], m[u], v[u], p[u]);
            d.exp_avg[i] = m[u];
            d.exp_avg_sq[i] = v[u];
            static_cast<float *>(d.param)[i] = p[u];
            continue;
          }
          const float step = adam_step(pk, d, g[u], m[u], v[u]);
          d.exp_avg[i] = m[u];
          d.exp_avg_sq[i] = v[u];
          {
            const int dt = d.param_dtype;
            const float p1 = round_to(dt, p[u] * pk.decay);
            store_any(d.param, dt, i, round_to(dt, fmaf(pk.neg_lr, round_to(dt, step), p1)));
          }
        }
      }
    }
  }
}

__global__ void __launch_bounds__(256) adamw_kernel(AdamPack pk) {
  // Tensor holding the block's first element, the last with offset <= e0
  // (offsets are ascending): independent compares, no chain of dependent
  // descriptor loads.
  int k = 0;
#pragma unroll
  for (int t = 1; t < kAdamBatch; ++t) k += static_cast<int>(blockIdx.x) >= pk.first_blk[t] ? 1 : 0;
  adamw_block(pk.sc, [&](int i) { return pk.d[i]; }, k);
}

// The same over a descriptor table in device memory.  The block's first
// tensor is the last one whose offset is <= its first element (offsets are
// ascending, the first is 0): a binary search over the table, the tensor
// adamw_kernel's compares find.
__global__ void __launch_bounds__(256) adamw_table_kernel(AdamScalars sc, const smx_adamw_desc *__restrict__ table) {
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * sc.chunk;
  int lo = 0, hi = sc.n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    // (the index is block-uniform: the descriptor loads are scalar loads)
    if (table[__builtin_amdgcn_readfirstlane(mid)].offset <= e0) lo = mid;
    else hi = mid - 1;
  }
  adamw_block(sc, [&](int i) { return table[__builtin_amdgcn_readfirstlane(i)]; }, __builtin_amdgcn_readfirstlane(lo));
}

}  // namespace smx

using namespace smx;

static int check_adamw_descs(const smx_adamw_desc *descs, int32_t n_desc, int64_t total) {
  SMX_REQUIRE(n_desc >= 0 && (n_desc == 0 || descs), SMX_EINVAL, "adamw: bad descriptor table");
  int64_t sum = 0;
  for (int32_t i = 0; i < n_desc; ++i) {
    const smx_adamw_desc &d = descs[i];
    SMX_REQUIRE(d.param && d.grad && d.exp_avg && d.exp_avg_sq, SMX_EINVAL, "adamw: null pointer");
    SMX_REQUIRE(d.n >= 0 && d.offset == sum, SMX_ESHAPE, "adamw: offsets must be the prefix sums of n");
    SMX_REQUIRE(d.grad_dtype == SMX_F32 || d.grad_dtype == SMX_BF16 || d.grad_dtype == SMX_F16, SMX_EDTYPE,
                "adamw: grad dtype must be f32, bf16 or f16");
    SMX_REQUIRE(d.param_dtype == SMX_F32 || d.param_dtype == SMX_BF16 || d.param_dtype == SMX_F16, SMX_EDTYPE,
                "adamw: param dtype must be f32, bf16 or f16");
    SMX_REQUIRE(d.bias1 > 0.f && d.bias2 > 0.f, SMX_EINVAL, "adamw: bias corrections must be positive");
    sum += d.n;
  }
  SMX_REQUIRE(sum == total, SMX_ESHAPE, "adamw: total != sum of n");
  return SMX_OK;
}

// Each FP32 coefficient is rounded from the double the reference computes
// in Python (1 - lr*wd, 1 - beta, -lr).
static AdamScalars adam_scalars(int32_t n, int64_t total, double lr, double beta1, double beta2, double eps,
                                double weight_decay) {
  AdamScalars sc{};
  sc.n = n;
  sc.total = total;
  sc.chunk = adam_chunk(total);
  sc.neg_lr = static_cast<float>(-lr);
  sc.decay = static_cast<float>(1.0 - lr * weight_decay);
  sc.b1 = static_cast<float>(beta1);
  sc.omb1 = static_cast<float>(1.0 - beta1);
  sc.b2 = static_cast<float>(beta2);
  sc.omb2 = static_cast<float>(1.0 - beta2);
  sc.eps = static_cast<float>(eps);
  return sc;
}

extern "C" int smx_adamw(const smx_adamw_desc *descs, int32_t n_desc, int64_t total, double lr, double beta1,
                         double beta2, double eps, double weight_decay, void *stream) {
  if (const int rc = check_adamw_descs(descs, n_desc, total)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int32_t b = 0; b < n_desc; b += kAdamBatch) {
    AdamPack pk{};
    const int32_t n = std::min<int32_t>(kAdamBatch, n_desc - b);
    const int64_t base = descs[b].offset;
    for (int i = 0; i < n; ++i) {
      pk.d[i] = descs[b + i];
      pk.d[i].offset -= base;
    }
    pk.sc = adam_scalars(n, pk.d[n - 1].offset + pk.d[n - 1].n, lr, beta1, beta2, eps, weight_decay);
    if (pk.sc.total == 0) continue;
    const int64_t blocks = ceil_div(pk.sc.total, pk.sc.chunk);
    SMX_REQUIRE(blocks < INT32_MAX, SMX_ESHAPE, "adamw: too many elements for one launch");
    for (int i = 0; i < kAdamBatch; ++i)
      pk.first_blk[i] = i < n ? static_cast<int32_t>(ceil_div(pk.d[i].offset, pk.sc.chunk)) : INT32_MAX;
    hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, pk);
    const int rc = check_launch("adamw");
    if (rc) return rc;
  }
  return SMX_OK;
}

// Table of smx_adamw_staged: the descriptors.
static size_t adamw_table_bytes(int32_t n_desc, int64_t total) {
  if (n_desc <= 0 || total <= 0) return 0;
  return static_cast<size_t>(n_desc) * sizeof(smx_adamw_desc);
}

extern "C" size_t smx_adamw_table_bytes(int32_t n_desc, int64_t total) { return adamw_table_bytes(n_desc, total); }

extern "C" int smx_adamw_staged(const smx_adamw_desc *descs, int32_t n_desc, int64_t total, double lr, double beta1,
                                double beta2, double eps, double weight_decay, void *dev_table, size_t table_bytes,
                                void *stream) {
  if (const int rc = check_adamw_descs(descs, n_desc, total)) return rc;
  if (n_desc == 0 || total == 0) return SMX_OK;
  const size_t need = adamw_table_bytes(n_desc, total);
  SMX_REQUIRE(dev_table && table_bytes >= need, SMX_EWORKSPACE,
              "adamw_staged: dev_table needs smx_adamw_table_bytes(n_desc, total) bytes");
  const AdamScalars sc = adam_scalars(n_desc, total, lr, beta1, beta2, eps, weight_decay);
  const int64_t blocks = ceil_div(total, sc.chunk);
  SMX_REQUIRE(blocks < INT32_MAX, SMX_ESHAPE, "adamw: too many elements for one launch");
  hipStream_t st = static_cast<hipStream_t>(stream);
  static_assert(sizeof(smx_adamw_desc) % 4 == 0, "the table is uploaded as 32-bit words");
  if (const int rc = upload_table(dev_table, descs, need, st)) return rc;
  const auto *table = static_cast<const smx_adamw_desc *>(dev_table);
  hipLaunchKernelGGL(adamw_table_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, sc, table);
  return check_launch("adamw_staged");
}
