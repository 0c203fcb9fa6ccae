// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// launch checking and argument validation.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "shrimp_hip.h"

namespace shrimp {

int set_error(int code, const char* fmt, ...);

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SHRIMP_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return SHRIMP_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Largest dynamic LDS allocation one workgroup may request on the current
// device (queried once per device).
int max_lds_per_block();

// The value / moves-left heads of the trunk tail from the head inputs in
// a->workspace ((B, 6C) fp32: [T0 | T1 | pooled | T4 | T5 | pooled]).
int launch_value_heads(const shrimp_tail_args* a, hipStream_t st);
// Compute units of the current device (queried once per device).
int cu_count();

// Conv kernel selection: 0 = automatic (small batches: one 64-row tile per
// workgroup; else big-tile LDS kernel for the 128-channel 7-tap shape, else
// LDS-staged when the position fits, else global gather), 1 = always the
// global-gather kernel, 2 = LDS-staged (no big tiles), 3 = as 0 without the
// small-batch row split.
extern std::atomic<int> g_conv_variant;
// Attention: 0 = automatic (two heads per workgroup when they fit), 1 = one
// head per workgroup, 2 = two heads on four waves, 3 = the chunked kernel
// (keys streamed through LDS; otherwise used only for sequences that do not
// fit one workgroup's LDS).
extern std::atomic<int> g_attn_variant;

}  // namespace shrimp

#define SHRIMP_REQUIRE(cond, ...)                                 \
  do {                                                            \
    if (!(cond)) return ::shrimp::set_error(SHRIMP_EINVAL, __VA_ARGS__); \
  } while (0)
