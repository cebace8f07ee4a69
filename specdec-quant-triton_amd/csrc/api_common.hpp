// Host-side helpers shared by the C-ABI translation units: error reporting, argument checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/specq.h"

namespace specq {

void set_error(const char* fmt, ...);
void clear_error();

inline int fail(int code, const char* what) {
  set_error("%s", what);
  return code;
}

#define SPECQ_REQUIRE(cond, code, ...) \
  do {                                 \
    if (!(cond)) {                     \
      ::specq::set_error(__VA_ARGS__); \
      return code;                     \
    }                                  \
  } while (0)

// Flag in the `variant` of a GEMM resource query: the call ran with a plan (tile rules differ).
constexpr int kAttrsPlan = 16;
// Flag in the `variant` of an attention resource query: fp32 K/V scales (else fp16).
constexpr int kAttrsScaleFp32 = 1 << 16;

// Every workspace starts with a fixed counter region (zero between calls), then scratch.
constexpr size_t kCounterBytes = 256 * 1024;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Largest power of two <= 16 dividing every value (pointer addresses and element counts).
inline int common_vec(std::initializer_list<uint64_t> vals) {
  int v = 16;
  for (uint64_t x : vals)
    while (v > 1 && (x % (uint64_t)v) != 0) v >>= 1;
  return v;
}

int launch(const void* fn, int grid, int threads, size_t lds, hipStream_t stream, void* params);

// Kernels using more than 64 KiB of dynamic LDS opt in once per kernel.
int ensure_lds(const void* fn, size_t lds);

// Number of CUs of the current device (cached per device).
int device_cus();

// The measured tile of a launch shape (tuned_tiles.hpp) for M rows: kind 0 = W8A8, 1 = W4A16;
// N is the launch's total width.  Only on a device of the CU count the table was measured on.
bool tuned_tile(int kind, int N, int K, int M, int* block_m, int* block_n, int* split_k);

// Timestamp buffer the kernels of the diagnostics build write (specq_diag_set_timeline);
// null, and never set, in the product build.
void diag_timeline(uint64_t** tl, int* cap);

}  // namespace specq
