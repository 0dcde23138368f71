// Library plumbing (error state, version, test hooks) and the small kernels around the decode
// loop: standalone weighted RMSNorm, embedding gather and the on-device next-token step.
//
// Reference: RMSNorm (iron/operators/rms_norm/op.py:21-130, kernel rms_norm.cc:83-147, golden
// rms_norm/reference.py:8-17); the host argmax + embedding lookup of the decode loop
// (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:612-621, check_cosine_int8.py:41-52).
#include <string.h>
#include "common.h"
#include "internal.h"

namespace iron {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

}  // namespace iron

namespace {

// One 256-thread workgroup per row: y = bf16((x * (1 / sqrt(mean(x^2) + eps))) * w), the
// golden's closed form evaluated in fp64 and rounded once. A thread holds up to kRegSlots 8-element
// slices of the row in registers (one vector load each); longer rows reload the rest.
constexpr int kRegSlots = 4;

IRON_DEV void unpack8_f(const uint4 v, float (&f)[8]) {
  f[0] = bf16lo_to_f32(v.x); f[1] = bf16hi_to_f32(v.x);
  f[2] = bf16lo_to_f32(v.y); f[3] = bf16hi_to_f32(v.y);
  f[4] = bf16lo_to_f32(v.z); f[5] = bf16hi_to_f32(v.z);
  f[6] = bf16lo_to_f32(v.w); f[7] = bf16hi_to_f32(v.w);
}

// x (and x2 when given, added in fp32) of slice i, as exact fp32
IRON_DEV void row_slice(const uint4* x, const uint4* x2, int i, float (&f)[8]) {
  unpack8_f(x[i], f);
  if (x2) {
    float g[8];
    unpack8_f(x2[i], g);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = f[j] + g[j];
  }
}

// plane != 0: y = f32((x1 * inv) * w) as three exact bf16 planes at out, out + plane,
// out + 2 plane (the MLP's hf for the MFMA path); else bf16(y) into out.
__device__ void rms_row(const uint16_t* __restrict__ x, const uint16_t* __restrict__ x2,
                        const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                        size_t plane, int cols, float eps, double* red) {
  const int n8 = cols >> 3;
  const uint4* xv = (const uint4*)x;
  const uint4* x2v = (const uint4*)x2;
  const uint4* wv = (const uint4*)w;
  float f[kRegSlots][8];
  uint4 wr[kRegSlots];
  double ss = 0.0;
#pragma unroll
  for (int r = 0; r < kRegSlots; ++r) {
    const int i = threadIdx.x + 256 * r;
    if (i < n8) {
      row_slice(xv, x2v, i, f[r]);
      wr[r] = w ? wv[i] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
#pragma unroll
  for (int r = 0; r < kRegSlots; ++r)
    if (threadIdx.x + 256 * r < n8) {
      double v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = f[r][j];
      ss += sum_sq_tree(v);
    }
  for (int i = threadIdx.x + 256 * kRegSlots; i < n8; i += 256) {
    float g[8];
    row_slice(xv, x2v, i, g);
    double v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = g[j];
    ss += sum_sq_tree(v);
  }
  ss = block_sum_256_d(ss, red);
  const double inv = inv_rms(ss, cols, (double)eps);
  auto emit = [&](int i, const float (&g)[8], const uint4 wq) {
    float wf[8];
    unpack8_f(wq, wf);
    double y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      y[j] = (double)g[j] * inv;
      if (w) y[j] *= (double)wf[j];
    }
    if (plane) {
      uint32_t h[3][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint16_t e0[3], e1[3];
        split3_bf16((float)y[2 * j], e0[0], e0[1], e0[2]);
        split3_bf16((float)y[2 * j + 1], e1[0], e1[1], e1[2]);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) h[pl][j] = (uint32_t)e0[pl] | ((uint32_t)e1[pl] << 16);
      }
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        ((uint4*)(out + pl * plane))[i] = make_uint4(h[pl][0], h[pl][1], h[pl][2], h[pl][3]);
    } else {
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        h[j] = (uint32_t)f64_to_bf16(y[2 * j]) | ((uint32_t)f64_to_bf16(y[2 * j + 1]) << 16);
      ((uint4*)out)[i] = make_uint4(h[0], h[1], h[2], h[3]);
    }
  };
#pragma unroll
  for (int r = 0; r < kRegSlots; ++r) {
    const int i = threadIdx.x + 256 * r;
    if (i < n8) emit(i, f[r], wr[r]);
  }
  for (int i = threadIdx.x + 256 * kRegSlots; i < n8; i += 256) {
    float g[8];
    row_slice(xv, x2v, i, g);
    emit(i, g, w ? wv[i] : make_uint4(0u, 0u, 0u, 0u));
  }
}

// rows with cols % 8 == 0 and 16-byte aligned row starts (validated by the launchers)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      uint16_t* __restrict__ y, int cols,
                                                      float eps) {
  __shared__ double red[4];
  const size_t r = (size_t)blockIdx.x * cols;
  rms_row(x + r, nullptr, w, y + r, 0, cols, eps, red);
}

// Scalar fallback for rows that are not a whole number of 16-byte slices.
__global__ __launch_bounds__(256) void rmsnorm_scalar_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ y, int cols,
                                                             float eps) {
  __shared__ double red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * cols;
  uint16_t* yr = y + (size_t)blockIdx.x * cols;
  double ss = 0.0;
  for (int i = threadIdx.x; i < cols; i += 256) {
    const double v = bf16_to_f32(xr[i]);
    ss = fma(v, v, ss);
  }
  ss = block_sum_256_d(ss, red);
  const double inv = inv_rms(ss, cols, (double)eps);
  for (int i = threadIdx.x; i < cols; i += 256) {
    const double v = (double)bf16_to_f32(xr[i]) * inv;
    yr[i] = f64_to_bf16(w ? v * (double)bf16_to_f32(w[i]) : v);
  }
}

// One 256-thread workgroup per row: x1 = f32(cur + a), y = f32((x1 * inv_rms(x1)) * w), the
// SwiGLU MLP's fp32 hf (swiglu_mlp_dp/reference.py:54-67) for batches on the MFMA path, written as
// three exact bf16 planes [3][rows][cols].
__global__ __launch_bounds__(256) void res_rmsnorm_planes_kernel(const uint16_t* __restrict__ cur,
                                                                 const uint16_t* __restrict__ a,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ planes,
                                                                 int rows, int cols, float eps) {
  __shared__ double red[4];
  const size_t r = (size_t)blockIdx.x * cols;
  rms_row(cur + r, a + r, w, planes + r, (size_t)rows * cols, cols, eps, red);
}

__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tokens,
                                                    const uint16_t* __restrict__ emb,
                                                    uint16_t* __restrict__ x, int D, int vocab) {
  const int b = blockIdx.x;
  int t = tokens[b];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  for (int i = threadIdx.x; i < D; i += 256) x[(size_t)b * D + i] = emb[(size_t)t * D + i];
}

// Single workgroup: decode every argmax key, reset it, gather the embeddings, log the tokens.
__global__ __launch_bounds__(256) void next_token_kernel(unsigned long long* keys,
                                                         int32_t* tokens,
                                                         const uint16_t* __restrict__ emb,
                                                         uint16_t* __restrict__ x,
                                                         int32_t* token_log, int log_stride,
                                                         int log_len, int32_t* step, int B, int D,
                                                         int vocab) {
  __shared__ int32_t s_tok[64];
  __shared__ int32_t s_step;
  if (threadIdx.x < B) {
    const unsigned long long k = keys[threadIdx.x];
    int32_t t = k ? (int32_t)(~(uint32_t)(k & 0xffffffffull)) : 0;
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
    s_tok[threadIdx.x] = t;
    tokens[threadIdx.x] = t;
  }
  if (threadIdx.x == 0) s_step = step ? *step : 0;
  __syncthreads();
  if (threadIdx.x < B) {
    keys[threadIdx.x] = 0ull;
    // the log holds log_len entries per row; steps past it are counted but not logged
    if (token_log && s_step >= 0 && s_step < log_len)
      token_log[(size_t)threadIdx.x * log_stride + s_step] = s_tok[threadIdx.x];
  }
  if (threadIdx.x == 0 && step) *step = s_step + 1;
  if (emb) {
    for (int b = 0; b < B; ++b) {
      const uint16_t* src = emb + (size_t)s_tok[b] * D;
      for (int i = threadIdx.x; i < D; i += 256) x[(size_t)b * D + i] = src[i];
    }
  }
}

// grid (B), 64 threads: pos[b] += delta, ctx[b] = pos[b] + 1, ang_rows[b] = table[pos[b]].
__global__ __launch_bounds__(64) void advance_kernel(int32_t* pos, int32_t* ctx,
                                                     const uint16_t* table, uint16_t* ang_rows,
                                                     int HD, int max_pos, int delta) {
  const int b = blockIdx.x;
  int p = 0;
  if (pos) p = pos[b] + delta;
  else if (ctx) p = ctx[b] - 1 + delta;
  __syncthreads();  // every thread has read the old value before it is replaced
  if (threadIdx.x == 0) {
    if (pos) pos[b] = p;
    if (ctx) ctx[b] = p + 1;
  }
  if (table && p >= 0 && p < max_pos) {
    const uint4* src = (const uint4*)(table + (size_t)p * HD);
    uint4* dst = (uint4*)(ang_rows + (size_t)b * HD);
    for (int i = threadIdx.x; i < HD / 8; i += 64) dst[i] = src[i];
  }
}

// Streaming read (the bandwidth reference of iron_stream_read): workgroup b reads the contiguous
// 16-byte words [b per, (b + 1) per) with sixteen loads in flight per thread. Contiguous chunks
// per workgroup read faster than a grid-stride sweep (6.1 against 5.3 TB/s on a 1 GiB buffer);
// every index stays below n16.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          size_t per, uint32_t* __restrict__ out) {
  constexpr int U = 16;
  uint32_t a = 0;
  const size_t b0 = (size_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
  for (size_t i = b0 + threadIdx.x; i < b1; i += (size_t)U * 256) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t k = i + (size_t)u * 256;
      v[u] = k < b1 ? p[k] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) a ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = a;
}

// Exhaustive check of the hardware bf16 rounding: thread i covers fp32 bit patterns
// [i * per, (i + 1) * per). out[0] counts patterns whose f32_to_bf16 differs from
// f32_to_bf16_rne (NaNs: a result that is not a NaN), out[1] is the smallest such pattern, and
// out[2] is f64_to_bf16(1 + 2^-8 + 2^-40): 0x3f80 when it rounds twice (fp64 -> fp32 -> bf16) as
// required, 0x3f81 if the two roundings were fused into one.
__global__ __launch_bounds__(256) void bf16_round_check_kernel(uint32_t per, uint32_t* out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t bad = 0, first = 0xffffffffu;
  for (uint32_t k = 0; k < per; ++k) {
    const uint32_t u = i * per + k;
    const float f = __uint_as_float(u);
    const uint32_t hw = f32_to_bf16(f), sw = f32_to_bf16_rne(f);
    const bool nan_in = (u & 0x7fffffffu) > 0x7f800000u;
    const bool ok = nan_in ? ((hw & 0x7fffu) > 0x7f80u) : hw == sw;
    if (!ok) {
      ++bad;
      first = u < first ? u : first;
    }
  }
  if (bad) {
    atomicAdd(out, bad);
    atomicMin(out + 1, first);
  }
  if (i == 0) out[2] = f64_to_bf16(1.0 + 0x1p-8 + 0x1p-40);
}

}  // namespace

namespace iron {

int rmsnorm_launch(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows, int cols,
                   float eps, hipStream_t stream) {
  const bool vec = cols % 8 == 0 && aligned(x, 16) && aligned(y, 16) && (!w || aligned(w, 16));
  if (vec) hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream, x, w, y, cols, eps);
  else hipLaunchKernelGGL(rmsnorm_scalar_kernel, dim3(rows), dim3(256), 0, stream, x, w, y, cols,
                          eps);
  return check_launch("rmsnorm");
}

int res_rmsnorm_planes_launch(const uint16_t* cur, const uint16_t* a, const uint16_t* w,
                              uint16_t* planes, int rows, int cols, float eps,
                              hipStream_t stream) {
  hipLaunchKernelGGL(res_rmsnorm_planes_kernel, dim3(rows), dim3(256), 0, stream, cur, a, w,
                     planes, rows, cols, eps);
  return check_launch("res_rmsnorm_planes");
}

}  // namespace iron

extern "C" {

int iron_abi_version(void) { return IRON_ABI_VERSION; }

int iron_advance_positions(int32_t* pos, int32_t* ctx, const uint16_t* table,
                           uint16_t* ang_rows, int HD, int max_pos, int B, int delta,
                           void* stream) {
  iron::clear_error();
  const char* fn = "iron_advance_positions";
  if (!pos && !ctx) return iron::fail(IRON_ERR_NULL, "%s: no buffers", fn);
  if (B <= 0) return iron::fail(IRON_ERR_SHAPE, "%s: B=%d must be positive", fn, B);
  if (table) {
    if (!ang_rows) return iron::fail(IRON_ERR_NULL, "%s: table without ang_rows", fn);
    if (HD <= 0 || HD % 8 || max_pos <= 0)
      return iron::fail(IRON_ERR_SHAPE, "%s: HD=%d max_pos=%d", fn, HD, max_pos);
    if (!iron::aligned(table, 16) || !iron::aligned(ang_rows, 16))
      return iron::fail(IRON_ERR_ALIGN, "%s: table / ang_rows must be 16-byte aligned", fn);
  }
  hipLaunchKernelGGL(advance_kernel, dim3(B), dim3(64), 0, (hipStream_t)stream, pos, ctx, table,
                     ang_rows, HD, max_pos, delta);
  return iron::check_launch(fn);
}

const char* iron_last_error(void) { return iron::g_err; }

uint32_t iron_test_fastdiv(uint32_t n, uint32_t d) {
  if (d == 0) return 0xffffffffu;
  return fastdiv_host(n, make_fastdiv(d));
}

int iron_test_bf16_round(uint32_t* out, void* stream) {
  iron::clear_error();
  if (!out) return iron::fail(IRON_ERR_NULL, "iron_test_bf16_round: null buffer");
  // 2^20 threads x 4096 patterns = every fp32 bit pattern; out[0..2] start as 0, ~0, 0
  hipLaunchKernelGGL(bf16_round_check_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream,
                     4096u, out);
  return iron::check_launch("iron_test_bf16_round");
}

int iron_stream_read(const void* p, size_t bytes, uint32_t* out, int blocks, void* stream) {
  iron::clear_error();
  const char* fn = "iron_stream_read";
  if (!p || !out) return iron::fail(IRON_ERR_NULL, "%s: null buffer", fn);
  if (bytes % 16 || !iron::aligned(p, 16) || blocks <= 0)
    return iron::fail(IRON_ERR_SHAPE, "%s: bytes %zu / blocks %d / alignment", fn, bytes, blocks);
  const size_t n16 = bytes / 16;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)p, n16, (n16 + blocks - 1) / blocks, out);
  return iron::check_launch(fn);
}

int iron_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* y, int rows, int cols, float eps,
                 void* stream) {
  iron::clear_error();
  if (!x || !y) return iron::fail(IRON_ERR_NULL, "iron_rmsnorm: null tensor");
  if (rows <= 0 || cols <= 0)
    return iron::fail(IRON_ERR_SHAPE, "iron_rmsnorm: bad shape rows=%d cols=%d", rows, cols);
  return iron::rmsnorm_launch(x, w, y, rows, cols, eps, (hipStream_t)stream);
}

int iron_embed(const int32_t* tokens, const uint16_t* emb, uint16_t* x, int B, int D, int vocab,
               void* stream) {
  iron::clear_error();
  if (!tokens || !emb || !x) return iron::fail(IRON_ERR_NULL, "iron_embed: null tensor");
  if (B <= 0 || D <= 0 || vocab <= 0)
    return iron::fail(IRON_ERR_SHAPE, "iron_embed: bad shape B=%d D=%d vocab=%d", B, D, vocab);
  hipLaunchKernelGGL(embed_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, tokens, emb, x, D,
                     vocab);
  return iron::check_launch("iron_embed");
}

int iron_next_token(unsigned long long* keys, int32_t* tokens, const uint16_t* emb, uint16_t* x,
                    int32_t* token_log, int log_stride, int log_len, int32_t* step, int B, int D,
                    int vocab, void* stream) {
  iron::clear_error();
  if (!keys || !tokens) return iron::fail(IRON_ERR_NULL, "iron_next_token: null keys/tokens");
  if (B <= 0 || B > 64 || vocab <= 0)
    return iron::fail(IRON_ERR_SHAPE, "iron_next_token: B=%d must be in [1,64]", B);
  if (emb && (!x || D <= 0))
    return iron::fail(IRON_ERR_NULL, "iron_next_token: embedding gather needs x and D > 0");
  if (token_log && !step)
    return iron::fail(IRON_ERR_NULL, "iron_next_token: token_log needs a step counter");
  if (token_log && (log_len <= 0 || (B > 1 && log_stride < log_len)))
    return iron::fail(IRON_ERR_SHAPE, "iron_next_token: log_len=%d (row stride %d)", log_len,
                      log_stride);
  hipLaunchKernelGGL(next_token_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, keys, tokens,
                     emb, x, token_log, log_stride, log_len, step, B, D, vocab);
  return iron::check_launch("iron_next_token");
}

}  // extern "C"
