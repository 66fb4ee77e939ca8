// smx_matrix_step_static: the matrix update of smx_matrix_step with its
// workspace in a file-scope device array instead of a caller buffer, for
// callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid allocation).
//
// The array lives in this translation unit's own code object, so it is
// only placed on a GPU (and held there until the process ends) once this
// entry point runs on that GPU.  Host code never uses the array's name as
// a device address: the first call on a device, with that device current,
// resolves the device address with hipGetSymbolAddress and keeps it per
// device; every later call passes that address to the kernels.
//
// The workspace contents on entry are irrelevant to the matrix step, so
// nothing is cleared between calls.  Calls on one GPU share the array:
// calls that overlap on one GPU (two streams, two threads) race.
#include "common.h"

#include <mutex>
#include <string>
#include <vector>

namespace smx {

constexpr size_t kStaticScratchBytes = SMX_MATRIX_STEP_STATIC_BYTES;  // 1 GiB; the 103M-GPT step needs 0.85 GB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

static std::mutex g_scratch_lock;
static void *g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch (resolved once per device).
static int scratch_of_current_device(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SMX_ELAUNCH, "matrix_step_static: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(SMX_ELAUNCH, std::string("matrix_step_static: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SMX_OK;
}

}  // namespace smx

extern "C" int smx_matrix_step_static(const smx_matrix_desc *descs, int32_t n, int mode, void *stream) {
  SMX_REQUIRE(n >= 0, SMX_EINVAL, "matrix_step_static: n < 0");
  if (n == 0) return SMX_OK;
  SMX_REQUIRE(descs, SMX_EINVAL, "matrix_step_static: null descriptor table");
  SMX_REQUIRE(mode == SMX_S8_FP32 || mode == SMX_S8_COMP_BF16 || mode == SMX_S8_MIXED, SMX_EINVAL,
              "matrix_step_static: unknown S8 mode");
  std::vector<int64_t> rows(n), cols(n);
  for (int32_t i = 0; i < n; ++i) {
    SMX_REQUIRE(descs[i].rows >= 1 && descs[i].cols >= 1, SMX_ESHAPE,
                "matrix_step_static: rows and cols must be >= 1");
    rows[i] = descs[i].rows;
    cols[i] = descs[i].cols;
  }
  const size_t need = smx_matrix_step_workspace_bytes(rows.data(), cols.data(), n, mode);
  if (need > smx::kStaticScratchBytes)
    return smx::fail(SMX_EWORKSPACE, "matrix_step_static: these matrices need " + std::to_string(need) +
                                         " bytes of workspace, more than the " +
                                         std::to_string(smx::kStaticScratchBytes) +
                                         "-byte static scratch; use smx_matrix_step with a caller workspace");
  void *ws = nullptr;
  const int rc = smx::scratch_of_current_device(&ws);
  if (rc) return rc;
  return smx_matrix_step(descs, n, mode, ws, smx::kStaticScratchBytes, stream);
}
