// Standalone RoPE and the fused decode QK-norm + RoPE + V copy, with the numerics of the fused
// QKV epilogue (qkv.hip): fp64 arithmetic (the exact values of the closed forms for bf16 inputs),
// one bf16 rounding at each of the reference's boundaries.
//
// iron_rope: iron/operators/rope/op.py:19-96 (spec [x (rows, cols), angles (angle_rows, cols),
//   y (rows, cols)], angle row r / (rows / angle_rows) for row r: design.py's consecutive-row
//   reuse); kernel aie_kernels/generic/rope.cc (TWO_HALVES and interleaved methods); golden
//   rope/reference.py:118-154 (TWO_HALVES).
// iron_qk_norm_rope: iron/operators/qk_norm_rope/op.py:20-117; kernels
//   aie_kernels/aie2p/qk_norm_rope.cc:30-108 (per-head RMSNorm rounded to bf16, then rotate_half
//   with the head_dim-long cos and sin tables, V copied) and qk_norm_rope_kv.cc (kv_direct: the
//   K|V slice also lands in the head-major [K_t | V_t] cache at the element offset
//   k_cache_offset, design.py:50-85); golden qk_norm_rope/reference.py:19-40.
#include "common.h"
#include "internal.h"

namespace {

// grid-stride over rows; thread i of a row computes pair i (< cols / 2) and stores both outputs
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ ang,
                                                   uint16_t* __restrict__ y, int rows, int cols,
                                                   int rep, int method) {
  const int half = cols / 2;
  for (int r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint16_t* xr = x + (size_t)r * cols;
    const uint16_t* ar = ang + (size_t)(r / rep) * cols;
    uint16_t* yr = y + (size_t)r * cols;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      const int ia = method == IRON_ROPE_TWO_HALVES ? i : 2 * i;
      const int ib = method == IRON_ROPE_TWO_HALVES ? i + half : 2 * i + 1;
      const double c = bf16_to_f32(ar[2 * i]), s = bf16_to_f32(ar[2 * i + 1]);
      const double a = bf16_to_f32(xr[ia]), b = bf16_to_f32(xr[ib]);
      yr[ia] = f64_to_bf16(a * c - b * s);
      yr[ib] = f64_to_bf16(b * c + a * s);
    }
  }
}

struct QkNormRopeParams {
  const uint16_t* in;
  const uint16_t* gamma;  // [n_qk][hd], then cos [hd], sin [hd]
  uint16_t* out;
  uint16_t* kv;           // null: no cache write
  const int32_t* kv_off;
  int hd, n_qk, n_v, max_seq;
  float eps;
};

// grid (n_qk + n_v), one thread per head dimension (blockDim = hd rounded up to 64).
__global__ __launch_bounds__(1024) void qk_norm_rope_kernel(QkNormRopeParams p) {
  const int head = blockIdx.x, d = threadIdx.x, hd = p.hd, half = hd / 2;
  const bool on = d < hd;
  const int n_q = p.n_qk - p.n_v;
  // every global load is issued before the first reduction
  const uint16_t hx = on ? p.in[(size_t)head * hd + d] : (uint16_t)0;
  const bool is_v = head >= p.n_qk;
  const uint16_t* cs = p.gamma + (size_t)p.n_qk * hd;
  const uint16_t hg = on && !is_v ? p.gamma[(size_t)head * hd + d] : (uint16_t)0;
  const uint16_t hc = on && !is_v ? cs[d] : (uint16_t)0;
  const uint16_t hs = on && !is_v ? cs[hd + d] : (uint16_t)0;
  long long off = -1;
  if (p.kv) {
    const long long o = p.kv_off ? (long long)*p.kv_off : 0;
    if (o >= 0 && o + 2LL * hd <= 2LL * p.max_seq * hd) off = o;
  }
  if (is_v) {  // V head: copied, and (kv_direct) into the V half of its cache row
    if (on) {
      p.out[(size_t)head * hd + d] = hx;
      const int j = head - p.n_qk;
      if (off >= 0) p.kv[(size_t)j * 2 * p.max_seq * hd + off + hd + d] = hx;
    }
    return;
  }
  __shared__ double s_red[16];
  __shared__ double s_y[1024];
  const double x = bf16_to_f32(hx);
  const double w = wave_sum_d(x * x);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = w;
  __syncthreads();
  double ss = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) ss += s_red[i];
  const double inv = inv_rms(ss, hd, (double)p.eps);
  const double y = bf16_to_f32(f64_to_bf16((x * inv) * (double)bf16_to_f32(hg)));
  s_y[d] = y;
  __syncthreads();
  if (!on) return;
  const double c = bf16_to_f32(hc), s = bf16_to_f32(hs);
  const double r = d < half ? y * c - s_y[d + half] * s : y * c + s_y[d - half] * s;
  const uint16_t hr = f64_to_bf16(r);
  p.out[(size_t)head * hd + d] = hr;
  if (off >= 0 && head >= n_q)  // K head: the K half of its cache row
    p.kv[(size_t)(head - n_q) * 2 * p.max_seq * hd + off + d] = hr;
}

}  // namespace

extern "C" {

int iron_rope(const uint16_t* x, const uint16_t* angles, uint16_t* y, int rows, int cols,
              int angle_rows, int method, void* stream) {
  iron::clear_error();
  if (!x || !angles || !y) return iron::fail(IRON_ERR_NULL, "iron_rope: null tensor");
  if (rows <= 0 || cols <= 0 || cols % 2 || angle_rows <= 0 || angle_rows > rows ||
      rows % angle_rows)
    return iron::fail(IRON_ERR_SHAPE,
                      "iron_rope: rows=%d cols=%d angle_rows=%d (cols even, angle_rows dividing "
                      "rows)", rows, cols, angle_rows);
  if (method != IRON_ROPE_TWO_HALVES && method != IRON_ROPE_INTERLEAVED)
    return iron::fail(IRON_ERR_UNSUPPORTED, "iron_rope: unknown method %d", method);
  const int grid = rows < 4096 ? rows : 4096;
  hipLaunchKernelGGL(rope_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, angles, y,
                     rows, cols, rows / angle_rows, method);
  return iron::check_launch("iron_rope");
}

int iron_qk_norm_rope(const uint16_t* qkv_in, const uint16_t* scratch, uint16_t* qkv_out,
                      uint16_t* kv_cache, const int32_t* kv_offset, int head_dim, int n_qk_heads,
                      int n_v_heads, int max_seq, float eps, void* stream) {
  iron::clear_error();
  if (!qkv_in || !scratch || !qkv_out)
    return iron::fail(IRON_ERR_NULL, "iron_qk_norm_rope: null tensor");
  if (head_dim <= 0 || head_dim % 2 || head_dim > 1024 || n_qk_heads <= 0 || n_v_heads < 0 ||
      n_v_heads > n_qk_heads)
    return iron::fail(IRON_ERR_SHAPE,
                      "iron_qk_norm_rope: head_dim=%d (even, <= 1024) n_qk_heads=%d n_v_heads=%d",
                      head_dim, n_qk_heads, n_v_heads);
  if (kv_cache && (!kv_offset || max_seq <= 0))
    return iron::fail(IRON_ERR_SHAPE,
                      "iron_qk_norm_rope: the cache write needs a device offset and max_seq > 0");
  QkNormRopeParams p;
  p.in = qkv_in;
  p.gamma = scratch;
  p.out = qkv_out;
  p.kv = kv_cache;
  p.kv_off = kv_offset;
  p.hd = head_dim;
  p.n_qk = n_qk_heads;
  p.n_v = n_v_heads;
  p.max_seq = max_seq;
  p.eps = eps;
  const int threads = (head_dim + 63) / 64 * 64;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(n_qk_heads + n_v_heads), dim3(threads), 0,
                     (hipStream_t)stream, p);
  return iron::check_launch("iron_qk_norm_rope");
}

}  // extern "C"
