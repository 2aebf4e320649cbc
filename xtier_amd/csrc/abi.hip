// Library-wide entry points and host helpers of the C ABI: version, last-error text, launch checks, LDS allowance.
#include "xt_host.h"

#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <utility>

namespace xt {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = 0;
  return XT_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(XT_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

int allow_lds(const void* fn, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return XT_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(XT_ELAUNCH, "%s: no current device", what);
  const std::pair<const void*, int> key{fn, dev};
  // allowances only grow, so what this thread has seen allowed stays allowed: launches after the first take no lock
  thread_local std::map<std::pair<const void*, int>, size_t> seen;
  const auto it = seen.find(key);
  if (it != seen.end() && bytes <= it->second) return XT_OK;
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> allowed;   // (kernel, device) -> bytes allowed so far
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = allowed[key];
  if (bytes > have) {
    const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (err != hipSuccess)
      return fail(XT_ELAUNCH, "%s: could not allow %zu bytes of LDS: %s", what, bytes, hipGetErrorString(err));
    have = bytes;
  }
  seen[key] = have;
  return XT_OK;
}

int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];   // 0: not read yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace xt

extern "C" int xt_version(void) { return 100; }

extern "C" const char* xt_last_error(void) { return xt::g_last_error; }
