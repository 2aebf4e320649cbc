// Host-side helpers of the C ABI: the per-thread last-error text and launch checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/xtier_amd.h"

namespace xt {

// Records the message for xt_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the last error and returns XT_OK.
int ok();
// XT_OK, or XT_ELAUNCH with the HIP error text, after a kernel launch.
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Dynamic LDS above 64 KB must be allowed per kernel and device. Raises kernel `fn`'s allowance on the current device
// to `bytes` when a launch asks for more than any before it; thread-safe. XT_OK or XT_ELAUNCH.
int allow_lds(const void* fn, size_t bytes, const char* what);

// Compute units of the current device (256 on an MI355X), read once per device; 256 if the query fails.
int device_cus();

// Workspaces of the split kernels (fused decode, sparse MLA) begin with a fixed region of arrival counters, one per
// (row, head group) of a call: zero before the first call, left zero by every call. Split partials follow it, so calls
// of any shape, of either kernel, may share one workspace as long as they do not overlap in time.
constexpr int kCounterSlots = 16384;
constexpr size_t kCounterBytes = (size_t)kCounterSlots * 4;

}  // namespace xt
