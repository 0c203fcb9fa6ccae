// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// launch checking and argument validation.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <initializer_list>
#include <string>

#include "shrimp_hip.h"

// Checked builds (SHRIMP_DEBUG=1) compile the kernels' input checks
// (SHRIMP_DCHECK, common.hpp) and synchronise after every launch.
#ifndef SHRIMP_DEBUG
#define SHRIMP_DEBUG 0
#endif

namespace shrimp {

int set_error(int code, const char* fmt, ...);

#if SHRIMP_DEBUG
// Waits for the device, then reads and clears the fault word of the calling
// source file's kernels (defined beside that word in common.hpp).
static int debug_sync(const char* what);
#endif

static inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SHRIMP_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
#if SHRIMP_DEBUG
  return debug_sync(what);
#else
  return SHRIMP_OK;
#endif
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Strides (in elements) that the buffer-extent checks accept: non-negative and
// below 2^31, so an extent (count - 1) * stride + width stays far inside
// int64_t for any int32 count and width (larger strides could not pass the
// 32-bit buffer-offset limit anyway).
inline bool strides_ok(std::initializer_list<int64_t> strides) {
  for (int64_t v : strides)
    if (v < 0 || v >= ((int64_t)1 << 31)) return false;
  return true;
}

// Largest row / sequence count an entry point takes: past it no buffer of the
// shape fits a 32-bit offset, and rounding it up stays inside int.
constexpr int kMaxDim = 1 << 24;

// Product of non-negative factors, INT64_MAX when it overflows (a negative
// factor gives -1): byte counts checked against a limit without signed
// overflow.
inline int64_t mul_sat(std::initializer_list<int64_t> factors) {
  int64_t r = 1;
  for (int64_t v : factors) {
    if (v < 0) return -1;
    if (__builtin_mul_overflow(r, v, &r)) return INT64_MAX;
  }
  return r;
}

// Largest dynamic LDS allocation one workgroup may request on the current
// device (queried once per device).
int max_lds_per_block();

// The value / moves-left heads of the trunk tail from the head inputs in
// a->workspace ((B, 6C) fp32: [T0 | T1 | pooled | T4 | T5 | pooled]).
int launch_value_heads(const shrimp_tail_args* a, hipStream_t st);
// Compute units of the current device (queried once per device).
int cu_count();

// Stamp buffer of the attention kernels in phase builds (attn.hip; the conv
// kernels' is set in hex_conv.hip), cycles != 0 to record the core clock too;
// SHRIMP_EINVAL in other builds.
int attn_phase_set(void* stamps, int cycles);
int fill_tokens_check(const float* tokens, int n_tokens, int C, const void* seq, int64_t seq_sb,
                      const void* tok_lo, int B);

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
