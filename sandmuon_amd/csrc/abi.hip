// Library-wide ABI plumbing: version, thread-local error reporting, and the
// in-order upload of host tables through kernel arguments.
#include "common.h"

#include <algorithm>
#include <cstdio>
#include <cstring>

namespace smx {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), "%s: launch failed: %s", what, hipGetErrorString(e));
    g_last_error = buf;
    return SMX_ELAUNCH;
  }
  return SMX_OK;
}

constexpr int kUploadWords = 960;  // 3840 bytes of payload per launch
struct UploadPack {
  uint32_t w[kUploadWords];
  uint32_t *dst;
  int32_t words;
};
static_assert(sizeof(UploadPack) <= 4000, "UploadPack is passed by value in the kernel arguments");

__global__ void __launch_bounds__(256) upload_kernel(UploadPack p) {
  const uint32_t *src = p.w;
  for (int k = threadIdx.x; k < p.words; k += 256) p.dst[k] = src[k];
}

int upload_table(void *dst, const void *src, size_t bytes, hipStream_t st) {
  if (bytes % 4 != 0 || (bytes && (!dst || !src))) return fail(SMX_EINVAL, "upload_table: bad table");
  const auto *s = static_cast<const uint32_t *>(src);
  auto *d = static_cast<uint32_t *>(dst);
  const size_t words = bytes / 4;
  for (size_t o = 0; o < words; o += kUploadWords) {
    UploadPack p{};  // (the unused tail of the payload is zeros, not stale host bytes)
    p.words = static_cast<int32_t>(std::min<size_t>(kUploadWords, words - o));
    std::memcpy(p.w, s + o, static_cast<size_t>(p.words) * 4);
    p.dst = d + o;
    hipLaunchKernelGGL(upload_kernel, dim3(1), dim3(256), 0, st, p);
    const int rc = check_launch("upload_table");
    if (rc) return rc;
  }
  return SMX_OK;
}

}  // namespace smx

extern "C" int smx_abi_version(void) { return SMX_ABI_VERSION; }

extern "C" const char *smx_last_error(void) { return smx::g_last_error.c_str(); }
