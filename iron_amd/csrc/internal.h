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

// Small prologue kernels (api.hip).
int rmsnorm_launch(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows, int cols,
                   float eps, hipStream_t stream);
// y = RMSNorm(cur + a) * w in fp32, written as its three exact bf16 planes (hi, mid, lo):
// planes [3][rows][cols], plane stride rows * cols.
int res_rmsnorm_planes_launch(const uint16_t* cur, const uint16_t* a, const uint16_t* w,
                              uint16_t* planes, int rows, int cols, float eps,
                              hipStream_t stream);

// MFMA batched GEMM (gemm_mfma.hip) for decode batches above the GEMV limit.
// The fused QKV head and MLP run batches up to kGemvMaxBatch on the GEMV kernels and larger ones
// on the MFMA GEMM. The standalone GEMV entry point (iron_gemv_w8a16) also takes batches up to
// kGemvBatchedMax on the exact batched kernel (gemv_batch_kernel); at batch 8 that kernel is bound
// by its fp64 FMAs (one per weight and batch row) and measured 2x the MFMA GEMM's time on the
// Qwen3-1.7B MLP, so the fused blocks keep the MFMA path from batch 5.
constexpr int kGemvMaxBatch = 4;
constexpr int kGemvBatchedMax = 15;
constexpr int kGemmMaxBatch = 16;
// Epilogues: bf16(acc) | silu(acc0) * acc1 in fp32 as three bf16 planes (dual) |
// bf16(f32(r1 + r2) + acc).
enum : int { GEMM_EPI_BF16 = 0, GEMM_EPI_SWIGLU_PLANES = 1, GEMM_EPI_RES_BF16 = 2 };
int gemm_check(const char* fn, int B, int M, int K, int G);
// The split-K arrival counters of the MFMA GEMM: a block at offset 0 of the workspace of every
// entry point that can run that GEMM (whatever B, so one workspace serves every batch size).
// The block is zero before the first call, and every call leaves it zero.
constexpr size_t kGemmCtrBytes = 16384;
// Bytes of fp64 split-K partials a GEMM of M rows needs, over every K.
size_t gemm_workspace_bound(int M, bool dual);
// The MLP's residual RMSNorm folded into the GEMM pair around it (hf = f32((x1 * inv_rms(x1)) *
// w), x1 = f32(cur + a), a = bf16(Wo . cx)). The producer (Wo: bf16 epilogue, split K) also
// writes, for each of its 64-row tiles and each batch row, the fp64 sum of x1^2 over the tile's
// rows (a fixed-order wavefront sum) to ssq [D / 64][16]. The consumer (gate/up, register-streamed
// form) sums a batch row's D / 64 tile sums in a fixed order and stages hf's three bf16 planes
// from cur, a and w chunk by chunk, where it otherwise reads the planes a separate kernel wrote.
struct GemmResNorm {
  double* ssq;
  const uint16_t* cur;  // [B][D]
  const uint16_t* a;    // [B][D]: null for the producer
  const uint16_t* w;    // [D] (consumer)
  int D;
  float eps;
};
// ssq null: no producer; the consumer (gate/up, staged form, at most 4 steps per split, B <= 8)
// sums x1^2 over each whole batch row in every workgroup and stages hf's planes for its K range
// once.
// Whether the fold applies to an MLP of these shapes: the producer splits K (its last split sums
// a tile's outputs) and the consumer runs the register-streamed form.
bool gemm_resnorm_foldable(int D, int QD, int FF);
// Whether the consumer-only fold (no tile sums) applies to the gate/up GEMM of these shapes.
bool gemm_selfnorm_foldable(int B, int D, int FF);
// x: bf16 [B][x_stride], or (x_plane > 0) an fp32 activation as three exact bf16 planes
// [3][B][x_stride] with plane stride x_plane elements. y_plane: the plane stride of the planes
// epilogue's output. rn: the folded RMSNorm's producer or consumer side, or null.
int gemm_w8_launch(const void* w0, const void* w1, int M, int K, int G, int tile_m, int domain,
                   const uint16_t* x, size_t x_plane, int B, int x_stride, int epi, void* y,
                   int y_stride, size_t y_plane, const uint16_t* r1, const uint16_t* r2,
                   int r_stride, unsigned int* ctr, void* part, size_t part_bytes,
                   hipStream_t stream, const char* fn, const GemmResNorm* rn = nullptr);


// The persistent kernel's tagged-word hand-off alone (decode_persistent.hip), for the hand-off
// probe: n words (a multiple of 256, at most kHandoffMaxWords) over n_phases phases.
constexpr int kHandoffMaxWords = 2048;
size_t handoff_tagged_bytes();
int handoff_tagged_launch(void* vec, uint32_t* err, int n, int n_phases, uint32_t base,
                          hipStream_t s);
// The same words exchanged inside each XCD's group of 32 workgroups (l2: through its L2).
int handoff_xcd_launch(bool l2, void* vec, uint32_t* err, int n, int n_phases, uint32_t base,
                       hipStream_t s);

// The raw-QKV stage shared by the QKV head and the fused QKV head + attention (qkv.hip).
size_t qkv_raw_bytes(int B, int D, int M);
// raw (bf16 [B][M]) sits after the GEMM counters at the front of the stage's workspace.
inline uint16_t* qkv_raw_of(void* ws) { return (uint16_t*)((char*)ws + kGemmCtrBytes); }
int qkv_raw_internal(const void* wqkv, const uint16_t* cur, const uint16_t* n_in, void* ws,
                     size_t ws_bytes, int B, int M, int D, int G, int tile_m, int domain,
                     float eps, hipStream_t s, const char* fn);
int gemv_rms_internal(const void* wire, const uint16_t* x, const uint16_t* nw, uint16_t* y,
                      int B, int M, int K, int G, int tile_m, int domain, float eps,
                      hipStream_t stream, const char* fn);

}  // namespace iron
