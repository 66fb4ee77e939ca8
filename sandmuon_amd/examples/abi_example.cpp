// A host program that drives libsandmuon_amd.so through its C ABI alone:
// HIP device memory, one hipStream_t, no Python and no torch.  It is what a
// framework other than torch would write against include/sandmuon_amd.h.
//
//   1. the cotangent statistic of a bf16 [16384, 768] tensor over two hook
//      calls, folded into the running sum (smx_stats_accumulate,
//      smx_stats_fold), against FP64 host sums;
//   2. the fused bias-gradient column sum with the same statistic
//      (smx_stats_colsum), and one batched launch over two inputs
//      (smx_stats_accumulate_batch), which must add exactly what one call
//      per input adds, folded over the slot rows it touched
//      (smx_stats_slot_rows);
//   3. one matrix step of a 256 x 384 parameter with diagonal factors in
//      FP32-MFMA mode (smx_matrix_step): the momentum is exactly
//      (1 - beta) g from a zero start, and the update has ||dW|| / lr =
//      sqrt(rows) (the Frobenius graft of sandmuon/optimizer.py:63-66).
//
// Prints one line per check and exits 0 when all pass, 1 otherwise.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/sandmuon_amd.h"

#define HIP_OK(expr)                                                              \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s: %s\n", #expr, hipGetErrorString(e_));             \
      return 2;                                                                   \
    }                                                                             \
  } while (0)
#define SMX_OK_(expr)                                                             \
  do {                                                                            \
    int r_ = (expr);                                                              \
    if (r_ != SMX_OK) {                                                           \
      std::fprintf(stderr, "%s -> %d: %s\n", #expr, r_, smx_last_error());        \
      return 2;                                                                   \
    }                                                                             \
  } while (0)

static uint32_t lcg(uint64_t &s) {
  s = s * 6364136223846793005ull + 1442695040888963407ull;
  return static_cast<uint32_t>(s >> 33);
}
static float uniform(uint64_t &s) { return (lcg(s) + 0.5f) / 2147483648.0f - 1.0f; }  // (-1, 1)
static uint16_t to_bf16(float f) {  // round to nearest even (finite inputs)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
static float from_bf16(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

static bool report(const char *what, double err, double tol) {
  const bool ok = err <= tol;
  std::printf("%-58s %.3e (gate %.0e) %s\n", what, err, tol, ok ? "ok" : "FAIL");
  return ok;
}

int main() {
  if (smx_abi_version() != SMX_ABI_VERSION) {
    std::fprintf(stderr, "ABI version %d, header %d\n", smx_abi_version(), SMX_ABI_VERSION);
    return 1;
  }
  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  bool ok = true;

  // ---- 1, 2: statistics
  const int64_t rows = 16384, cols = 768;
  const int32_t slots = 128;
  std::vector<uint16_t> x(rows * cols);
  uint64_t seed = 2024;
  for (auto &v : x) v = to_bf16(1e-3f * uniform(seed) + 2e-4f);
  std::vector<double> want_sq(cols, 0.0), want_sum(cols, 0.0), mag(cols, 0.0);
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < cols; ++j) {
      const double v = from_bf16(x[i * cols + j]);
      want_sq[j] += v * v;
      want_sum[j] += v;
      mag[j] += std::fabs(v);
    }
  void *xd;
  float *slot_d, *sum_d, *colsum_d;
  HIP_OK(hipMalloc(&xd, x.size() * 2));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&slot_d), slots * cols * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&sum_d), cols * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&colsum_d), cols * 4));
  HIP_OK(hipMemcpy(xd, x.data(), x.size() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(slot_d, 0, slots * cols * 4));
  HIP_OK(hipMemset(sum_d, 0, cols * 4));
  for (int call = 0; call < 2; ++call)  // two microbatches of the same tensor
    SMX_OK_(smx_stats_accumulate(xd, SMX_BF16, rows, cols, cols, slot_d, nullptr, slots, st));
  SMX_OK_(smx_stats_fold(sum_d, slot_d, nullptr, nullptr, cols, slots, st));
  const int64_t ws_bytes = smx_stats_colsum_workspace_bytes(cols, slots);
  void *ws;
  float *slot2_d;
  HIP_OK(hipMalloc(&ws, ws_bytes));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&slot2_d), slots * cols * 4));
  HIP_OK(hipMemset(slot2_d, 0, slots * cols * 4));
  SMX_OK_(smx_stats_colsum(xd, SMX_BF16, rows, cols, cols, slot2_d, slots, colsum_d, ws, ws_bytes, st));
  HIP_OK(hipStreamSynchronize(st));
  std::vector<float> sum(cols), colsum(cols);
  HIP_OK(hipMemcpy(sum.data(), sum_d, cols * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(colsum.data(), colsum_d, cols * 4, hipMemcpyDeviceToHost));
  double num = 0, den = 0, worst = 0;
  for (int64_t j = 0; j < cols; ++j) {
    num += (sum[j] - 2 * want_sq[j]) * (sum[j] - 2 * want_sq[j]);
    den += 4 * want_sq[j] * want_sq[j];
    worst = std::fmax(worst, std::fabs(colsum[j] - want_sum[j]) / mag[j]);
  }
  ok &= report("stats_accumulate x2 + fold: rel. error of sum x^2", std::sqrt(num / den), 1e-6);
  ok &= report("stats_colsum: max |colsum - sum x| / sum |x|", worst, 1e-6);

  // Batched: the whole tensor and its first 5000 rows (an odd microbatch)
  // into two slot buffers in one launch, against one call each.
  const int64_t part_rows = 5000;
  float *sb_d[4];
  for (auto &p : sb_d) {
    HIP_OK(hipMalloc(reinterpret_cast<void **>(&p), slots * cols * 4));
    HIP_OK(hipMemset(p, 0, slots * cols * 4));
  }
  smx_stats_desc descs[2] = {{xd, sb_d[0], nullptr, rows, cols, cols, SMX_BF16, slots},
                             {xd, sb_d[1], nullptr, part_rows, cols, cols, SMX_BF16, slots}};
  SMX_OK_(smx_stats_accumulate_batch(descs, 2, st));
  SMX_OK_(smx_stats_accumulate(xd, SMX_BF16, rows, cols, cols, sb_d[2], nullptr, slots, st));
  SMX_OK_(smx_stats_accumulate(xd, SMX_BF16, part_rows, cols, cols, sb_d[3], nullptr, slots, st));
  HIP_OK(hipStreamSynchronize(st));
  std::vector<float> sb[4];
  for (int k = 0; k < 4; ++k) {
    sb[k].resize(slots * cols);
    HIP_OK(hipMemcpy(sb[k].data(), sb_d[k], slots * cols * 4, hipMemcpyDeviceToHost));
  }
  const bool same = sb[0] == sb[2] && sb[1] == sb[3];
  std::printf("%-58s %s\n", "stats_accumulate_batch: bit-identical to one call each", same ? "ok" : "FAIL");
  ok &= same;
  // Only the leading slot rows a call touched hold partials.
  const int32_t used = smx_stats_slot_rows(rows, slots);
  bool rest_zero = used >= 1 && used <= slots;
  for (int64_t i = static_cast<int64_t>(used) * cols; i < slots * cols; ++i) rest_zero &= sb[0][i] == 0.f;
  HIP_OK(hipMemset(sum_d, 0, cols * 4));
  SMX_OK_(smx_stats_fold(sum_d, sb_d[0], nullptr, nullptr, cols, used, st));
  HIP_OK(hipMemcpy(sum.data(), sum_d, cols * 4, hipMemcpyDeviceToHost));
  num = den = 0;
  for (int64_t j = 0; j < cols; ++j) {
    num += (sum[j] - want_sq[j]) * (sum[j] - want_sq[j]);
    den += want_sq[j] * want_sq[j];
  }
  std::printf("%-58s %d of %d %s\n", "smx_stats_slot_rows: rows touched, the rest zero", used, slots,
              rest_zero ? "ok" : "FAIL");
  ok &= rest_zero;
  ok &= report("batched stats, fold of the touched rows: rel. error", std::sqrt(num / den), 1e-6);

  // ---- 3: one matrix step, diagonal factors, FP32-MFMA mode
  const int64_t r = 256, c = 384;
  const double lr = 1e-2, beta = 0.8;
  std::vector<float> w(r * c), g(r * c), inv_row(r), inv_col(c);
  for (auto &v : w) v = 0.02f * uniform(seed);
  for (auto &v : g) v = 1e-3f * uniform(seed);
  for (auto &v : inv_row) v = 1.0f + 0.5f * uniform(seed);
  for (auto &v : inv_col) v = 1.0f + 0.5f * uniform(seed);
  float *w_d, *g_d, *m_d, *ir_d, *ic_d;
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&w_d), r * c * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&g_d), r * c * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&m_d), r * c * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&ir_d), r * 4));
  HIP_OK(hipMalloc(reinterpret_cast<void **>(&ic_d), c * 4));
  HIP_OK(hipMemcpy(w_d, w.data(), r * c * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(g_d, g.data(), r * c * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(m_d, 0, r * c * 4));
  HIP_OK(hipMemcpy(ir_d, inv_row.data(), r * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ic_d, inv_col.data(), c * 4, hipMemcpyHostToDevice));
  smx_matrix_desc d{};
  d.param = w_d;
  d.grad = g_d;
  d.momentum = m_d;
  d.inv_row = ir_d;
  d.inv_col = ic_d;
  d.rows = r;
  d.cols = c;
  d.lr = lr;
  d.momentum_beta = beta;
  d.grad_dtype = SMX_F32;
  const size_t need = smx_matrix_step_workspace_bytes(&r, &c, 1, SMX_S8_FP32);
  void *mws;
  HIP_OK(hipMalloc(&mws, need));
  SMX_OK_(smx_matrix_step(&d, 1, SMX_S8_FP32, mws, need, st));
  HIP_OK(hipStreamSynchronize(st));
  std::vector<float> w1(r * c), m1(r * c);
  HIP_OK(hipMemcpy(w1.data(), w_d, r * c * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(m1.data(), m_d, r * c * 4, hipMemcpyDeviceToHost));
  const float omb = static_cast<float>(1.0 - beta), bf = static_cast<float>(beta);
  double mom_err = 0, dw2 = 0;
  for (int64_t i = 0; i < r * c; ++i) {
    const float want = std::fmaf(0.0f, bf, g[i] * omb);  // m' = b m + (1-b) g, m = 0
    mom_err = std::fmax(mom_err, std::fabs(static_cast<double>(m1[i]) - want));
    const double dw = (static_cast<double>(w[i]) - w1[i]) / lr;
    dw2 += dw * dw;
  }
  ok &= report("matrix_step: max |momentum - (1-beta) g| (exact)", mom_err, 0.0);
  ok &= report("matrix_step: | ||dW||/lr - sqrt(rows) | / sqrt(rows)",
               std::fabs(std::sqrt(dw2) - std::sqrt(static_cast<double>(r))) / std::sqrt(static_cast<double>(r)),
               1e-4);

  hipFree(xd); hipFree(slot_d); hipFree(sum_d); hipFree(colsum_d); hipFree(ws); hipFree(slot2_d);
  for (auto p : sb_d) hipFree(p);
  hipFree(w_d); hipFree(g_d); hipFree(m_d); hipFree(ir_d); hipFree(ic_d); hipFree(mws);
  hipStreamDestroy(st);
  std::printf("%s\n", ok ? "all checks passed" : "FAILED");
  return ok ? 0 : 1;
}
