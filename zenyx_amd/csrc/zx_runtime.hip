// zx_runtime.hip -- error reporting and device queries shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "zx_common.h"

namespace zx {

static thread_local char g_msg[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_msg[0] = 0; }

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ZX_ERR_HIP, "launch of %s failed: %s", what, hipGetErrorString(e));
  return ZX_OK;
}

int num_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// 2 s at the 100 MHz s_memrealtime clock: far beyond any exchange of a co-resident grid.
constexpr uint64_t kDefaultWaitTicks = 200000000ull;
static std::atomic<uint64_t> g_wait_ticks{kDefaultWaitTicks};

uint64_t wait_bound_ticks() { return g_wait_ticks.load(std::memory_order_relaxed); }

}  // namespace zx

extern "C" int zx_set_wait_bound_us(int64_t us) {
  zx::g_wait_ticks.store(us < 0 ? zx::kDefaultWaitTicks : (uint64_t)us * 100u, std::memory_order_relaxed);
  return ZX_OK;
}

extern "C" const char *zx_last_error(void) { return zx::g_msg; }

extern "C" int zx_abi_version(void) { return 7; }
