// Host-side helpers shared by the C-ABI entry points: status codes, the thread-local error
// message, and argument validation that runs before any HIP call (so CPU-only tests can force
// every error path).
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/iron_hip.h"

namespace iron {

void set_error(const char* fmt, ...);
void clear_error();

inline int fail(int status, const char* fmt, ...) {
  char buf[480];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  set_error("%s", buf);
  return status;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IRON_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return IRON_OK;
}

inline bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }
inline int ilog2(int v) { int l = 0; while ((1 << l) < v) ++l; return l; }
inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Bytes of one row-block of the int8 wire: tile_m rows of K int8, then tile_m*(K/G) bf16 scales.
inline size_t wire_block_bytes(int K, int G, int tile_m) {
  return (size_t)tile_m * (size_t)K + (size_t)tile_m * (size_t)(K / G) * 2u;
}

// Validates the int8 wire geometry shared by every int8 entry point.
int check_wire(const char* fn, const void* wire, int M, int K, int G, int tile_m, int domain);

}  // namespace iron
