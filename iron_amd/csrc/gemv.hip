// Weight-streaming GEMV kernels for batch-1..4 decode on gfx950.
//
// Reference path: the int8 W8A16 matvec (aie_kernels/aie2p/mv_int8_signed.cc:60-113, biased
// form mv_int8.cc:60-115) behind GEMVInt8 (iron/operators/gemv_int8/op.py:20-178), the fused
// QKV GEMV (qkv_head_dp), the gate/up/down GEMVs of the fused SwiGLU MLP (swiglu_mlp_dp) and the
// LM head (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:242-246).
//
// Weight wire (the reference's own packing, gemv_int8/reference.py:59-80): consecutive
// row-blocks of `tile_m` rows, each block = tile_m*K int8 payload (row-major) followed by
// tile_m*(K/G) bf16 group scales (row-major). The payload domain is signed two's-complement q or
// biased q+128; both feed the same integer q.
//
// Arithmetic (the exact-dequant golden of GEMVInt8.reference, gemv_int8/op.py:173-178):
//     y[b][m] = sum_g s[m][g] * sum_{k in g} q[m][k] * x[b][k]     (fp32), one bf16 rounding.
// Every product q*s*x is exact in fp32 (8 x 8 x 8 significant bits), so this matches the golden
// to fp32 summation order. The inner loop reads the payload as u = q+128 (XOR 0x80 for the
// signed domain, a single v_cvt_f32_ubyteN per weight) and removes the bias per group with the
// lane's precomputed sum of x: sum q*x = sum u*x - 128*sum x.
//
// Mapping: 256-thread workgroups, 4 wavefronts, each wavefront owns R consecutive rows; lane l
// reads 16 consecutive K elements (one 128-bit load) per 1024-wide chunk, so one wavefront load
// instruction covers 1 KiB of one row, fully coalesced. x is staged once per workgroup in LDS
// as fp32 by a prologue that can also fuse RMSNorm / residual adds.
#include "common.h"
#include "internal.h"

namespace {

enum Prologue : int {
  PRO_BF16 = 0,        // xs = x                                   (x bf16)
  PRO_RMS_BF16 = 1,    // xs = bf16(rmsnorm(x) * w)                (fused RMSNorm, bf16 boundary)
  PRO_RES_RMS_F32 = 2, // xs = rmsnorm(x + x2) * w  in fp32        (SwiGLU MLP: x1 = cur + a)
  PRO_F32 = 3,         // xs = x                                   (x fp32)
};

enum Epilogue : int {
  EPI_BF16 = 0,        // y = bf16(acc)
  EPI_F32 = 1,         // y = acc (fp32)
  EPI_RES_BF16 = 2,    // y = bf16((r1 + r2) + acc)                (down GEMV + residual)
  EPI_SWIGLU_F32 = 3,  // y = silu(acc_gate) * acc_up (fp32)       (dual matrix)
  EPI_BF16_ARGMAX = 4, // y = bf16(acc), plus atomic argmax of the bf16 value
};

struct GemvParams {
  const uint8_t* w;     // int8 wire or bf16 row-major weights
  const uint8_t* w2;    // second int8 wire (EPI_SWIGLU_F32)
  int M, K, gshift, tile_m;
  FastDiv tdiv;
  uint32_t blk_bytes;
  uint32_t xor_mask;    // 0x80808080 for the signed domain, 0 for biased
  // prologue
  int pro;
  const void* x;        // [B][x_stride] bf16 or fp32
  const uint16_t* x2;   // [B][x2_stride] bf16 (residual term), may be null
  const uint16_t* nw;   // [K] bf16 RMSNorm weight
  float eps;
  int x_stride, x2_stride;
  // epilogue
  int epi;
  void* y;              // [B][y_stride]
  int y_stride;
  const uint16_t* r1;   // [B][r_stride] residual inputs (bf16)
  const uint16_t* r2;
  int r_stride;
  unsigned long long* argmax;  // [B] packed (ordered bf16 << 32 | ~row)
};

// ------------------------------------------------------------------------------------------
// Prologue: stage B vectors of length K into LDS as fp32.
// ------------------------------------------------------------------------------------------
template <int B>
__device__ void stage_x(const GemvParams& p, float* __restrict__ xs, float* red) {
  const int K = p.K;
  for (int b = 0; b < B; ++b) {
    float* dst = xs + (size_t)b * K;
    if (p.pro == PRO_F32) {
      const float* src = (const float*)p.x + (size_t)b * p.x_stride;
      for (int i = threadIdx.x; i < K; i += blockDim.x) dst[i] = src[i];
    } else if (p.pro == PRO_BF16) {
      const uint16_t* src = (const uint16_t*)p.x + (size_t)b * p.x_stride;
      for (int i = threadIdx.x; i < K; i += blockDim.x) dst[i] = bf16_to_f32(src[i]);
    } else {
      const uint16_t* src = (const uint16_t*)p.x + (size_t)b * p.x_stride;
      const uint16_t* src2 = p.x2 ? p.x2 + (size_t)b * p.x2_stride : nullptr;
      float ss = 0.f;
      for (int i = threadIdx.x; i < K; i += blockDim.x) {
        float v = bf16_to_f32(src[i]);
        if (src2) v += bf16_to_f32(src2[i]);
        dst[i] = v;
        ss = fmaf(v, v, ss);
      }
      ss = block_sum_256(ss, red);
      const float inv = 1.0f / sqrtf(ss / (float)K + p.eps);
      for (int i = threadIdx.x; i < K; i += blockDim.x) {
        float v = dst[i] * inv * bf16_to_f32(p.nw[i]);
        dst[i] = (p.pro == PRO_RMS_BF16) ? round_bf16(v) : v;
      }
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------
// int8 core: R rows x B vectors, full-row dot products (every lane ends with the totals).
// ------------------------------------------------------------------------------------------
template <int B, int R>
__device__ __forceinline__ void w8_rows(const GemvParams& p, const uint8_t* __restrict__ wire,
                                        int row0, const float* __restrict__ xs, int lane,
                                        float (&acc)[R][B]) {
  const int K = p.K;
  const int ng = K >> p.gshift;
  const uint8_t* qrow[R];
  const uint16_t* srow[R];
  bool rv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    rv[r] = row < p.M;
    const uint32_t rr = rv[r] ? (uint32_t)row : 0u;
    const uint32_t blk = fastdiv(rr, p.tdiv);
    const uint32_t in = rr - blk * (uint32_t)p.tile_m;
    const uint8_t* base = wire + (size_t)blk * p.blk_bytes;
    qrow[r] = base + (size_t)in * K;
    srow[r] = (const uint16_t*)(base + (size_t)p.tile_m * K) + (size_t)in * ng;
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = 0.f;
  }

  for (int c0 = 0; c0 < K; c0 += 1024) {
    const int e = c0 + lane * 16;
    const bool ev = e < K;
    uint4 w[R];
    float s[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (ev && rv[r]) {
        w[r] = *(const uint4*)(qrow[r] + e);
        s[r] = bf16_to_f32(srow[r][e >> p.gshift]);
      } else {
        w[r] = make_uint4(0x80808080u ^ p.xor_mask, 0x80808080u ^ p.xor_mask,
                          0x80808080u ^ p.xor_mask, 0x80808080u ^ p.xor_mask);
        s[r] = 0.f;
      }
    }
    float xv[B][16];
    float xsum[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (ev) {
        const float4* src = (const float4*)(xs + (size_t)b * K + e);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4 t = src[j];
          xv[b][4 * j + 0] = t.x;
          xv[b][4 * j + 1] = t.y;
          xv[b][4 * j + 2] = t.z;
          xv[b][4 * j + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) xv[b][j] = 0.f;
      }
      float t0 = 0.f, t1 = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j += 2) {
        t0 += xv[b][j];
        t1 += xv[b][j + 1];
      }
      xsum[b] = t0 + t1;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t d0 = w[r].x ^ p.xor_mask, d1 = w[r].y ^ p.xor_mask;
      const uint32_t d2 = w[r].z ^ p.xor_mask, d3 = w[r].w ^ p.xor_mask;
      const uint32_t dd[4] = {d0, d1, d2, d3};
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float pa = 0.f, pb = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d = dd[j];
          pa = fmaf((float)(d & 0xffu), xv[b][4 * j + 0], pa);
          pb = fmaf((float)((d >> 8) & 0xffu), xv[b][4 * j + 1], pb);
          pa = fmaf((float)((d >> 16) & 0xffu), xv[b][4 * j + 2], pa);
          pb = fmaf((float)(d >> 24), xv[b][4 * j + 3], pb);
        }
        acc[r][b] = fmaf(s[r], (pa + pb) - 128.f * xsum[b], acc[r][b]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = wave_sum(acc[r][b]);
}

// ------------------------------------------------------------------------------------------
// bf16-weight core (row-major [M][K] bf16): lane l reads 8 consecutive K per 512-wide chunk.
// ------------------------------------------------------------------------------------------
template <int B, int R>
__device__ __forceinline__ void w16_rows(const GemvParams& p, int row0,
                                         const float* __restrict__ xs, int lane,
                                         float (&acc)[R][B]) {
  const int K = p.K;
  const uint16_t* W = (const uint16_t*)p.w;
  bool rv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rv[r] = (row0 + r) < p.M;
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = 0.f;
  }
  for (int c0 = 0; c0 < K; c0 += 512) {
    const int e = c0 + lane * 8;
    const bool ev = e < K;
    uint4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      w[r] = (ev && rv[r]) ? *(const uint4*)(W + (size_t)(row0 + r) * K + e)
                           : make_uint4(0u, 0u, 0u, 0u);
    float xv[B][8];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (ev) {
        const float4* src = (const float4*)(xs + (size_t)b * K + e);
        float4 t0 = src[0], t1 = src[1];
        xv[b][0] = t0.x; xv[b][1] = t0.y; xv[b][2] = t0.z; xv[b][3] = t0.w;
        xv[b][4] = t1.x; xv[b][5] = t1.y; xv[b][6] = t1.z; xv[b][7] = t1.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[b][j] = 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
      for (int b = 0; b < B; ++b) {
        float a = acc[r][b];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a = fmaf(bf16lo_to_f32(dd[j]), xv[b][2 * j], a);
          a = fmaf(bf16hi_to_f32(dd[j]), xv[b][2 * j + 1], a);
        }
        acc[r][b] = a;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = wave_sum(acc[r][b]);
}

IRON_DEV uint32_t bf16_order_key(uint16_t h) {
  return (h & 0x8000u) ? (uint32_t)(~h & 0xffffu) : (uint32_t)(h | 0x8000u);
}

template <int B, int R>
__device__ __forceinline__ void store_rows(const GemvParams& p, int row0, int lane,
                                           const float (&acc)[R][B], const float (&acc2)[R][B],
                                           unsigned long long (&best)[B]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    if (row >= p.M) continue;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const float v = acc[r][b];
      const size_t o = (size_t)b * p.y_stride + row;
      if (p.epi == EPI_BF16_ARGMAX) {
        const uint16_t h = f32_to_bf16(v);
        const unsigned long long key =
            ((unsigned long long)bf16_order_key(h) << 32) | (unsigned long long)(~(uint32_t)row);
        best[b] = key > best[b] ? key : best[b];
        if (lane == r * B + b) ((uint16_t*)p.y)[o] = h;
      } else if (lane == r * B + b) {
        if (p.epi == EPI_BF16) {
          ((uint16_t*)p.y)[o] = f32_to_bf16(v);
        } else if (p.epi == EPI_F32) {
          ((float*)p.y)[o] = v;
        } else if (p.epi == EPI_RES_BF16) {
          const size_t ro = (size_t)b * p.r_stride + row;
          float x1 = bf16_to_f32(p.r1[ro]);
          if (p.r2) x1 += bf16_to_f32(p.r2[ro]);
          ((uint16_t*)p.y)[o] = f32_to_bf16(x1 + v);
        } else {  // EPI_SWIGLU_F32
          const float g = v;
          const float sg = g / (1.0f + expf(-g));
          ((float*)p.y)[o] = sg * acc2[r][b];
        }
      }
    }
  }
}

template <int B, int R, bool INT8>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  extern __shared__ float xs[];
  __shared__ float red[8];
  stage_x<B>(p, xs, red);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  unsigned long long best[B];
#pragma unroll
  for (int b = 0; b < B; ++b) best[b] = 0ull;
  const int rows_per_wg = 4 * R;
  for (int grp = blockIdx.x; grp * rows_per_wg < p.M; grp += gridDim.x) {
    const int row0 = grp * rows_per_wg + wave * R;
    if (row0 >= p.M) continue;
    float acc[R][B];
    float acc2[R][B];
    if constexpr (INT8) {
      w8_rows<B, R>(p, p.w, row0, xs, lane, acc);
      if (p.epi == EPI_SWIGLU_F32) {
        w8_rows<B, R>(p, p.w2, row0, xs, lane, acc2);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int b = 0; b < B; ++b) acc2[r][b] = 0.f;
      }
    } else {
      w16_rows<B, R>(p, row0, xs, lane, acc);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc2[r][b] = 0.f;
    }
    store_rows<B, R>(p, row0, lane, acc, acc2, best);
  }
  if (p.epi == EPI_BF16_ARGMAX && lane == 0) {
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (best[b]) atomicMax(p.argmax + b, best[b]);
  }
}

// ------------------------------------------------------------------------------------------
// Bit-exact dequant: w[m][k] = bf16(q[m][k] * s[m][k/G]). q*s is exact in fp32, so the single
// RNE rounding is the only rounding (qwen3_npu_int8.py:350-379, op_ours.py:31-43,515-541).
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ wire,
                                                      uint16_t* __restrict__ out, int M, int K,
                                                      int gshift, int tile_m, FastDiv tdiv,
                                                      uint32_t blk_bytes, uint32_t xor_mask) {
  const int per_row = K >> 4;
  const long long total = (long long)M * per_row;
  const int ng = K >> gshift;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(i / per_row);
    const int e = (int)(i - (long long)row * per_row) * 16;
    const uint32_t blk = fastdiv(row, tdiv);
    const uint32_t in = row - blk * (uint32_t)tile_m;
    const uint8_t* base = wire + (size_t)blk * blk_bytes;
    const uint4 w = *(const uint4*)(base + (size_t)in * K + e);
    const float s = bf16_to_f32(((const uint16_t*)(base + (size_t)tile_m * K))[(size_t)in * ng +
                                                                               (e >> gshift)]);
    const uint32_t dd[4] = {w.x ^ xor_mask, w.y ^ xor_mask, w.z ^ xor_mask, w.w ^ xor_mask};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = dd[j];
      const float q0 = (float)(int)((d & 0xffu)) - 128.f;
      const float q1 = (float)(int)((d >> 8) & 0xffu) - 128.f;
      const float q2 = (float)(int)((d >> 16) & 0xffu) - 128.f;
      const float q3 = (float)(int)(d >> 24) - 128.f;
      o[2 * j] = (uint32_t)f32_to_bf16(q0 * s) | ((uint32_t)f32_to_bf16(q1 * s) << 16);
      o[2 * j + 1] = (uint32_t)f32_to_bf16(q2 * s) | ((uint32_t)f32_to_bf16(q3 * s) << 16);
    }
    uint4* dst = (uint4*)(out + (size_t)row * K + e);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// ------------------------------------------------------------------------------------------
// Host launch helpers
// ------------------------------------------------------------------------------------------
constexpr int kMaxLdsBytes = 131072;

template <bool INT8>
int launch_gemv(const GemvParams& p, int B, hipStream_t stream, const char* fn) {
  const size_t lds = (size_t)B * p.K * sizeof(float);
  if (lds > (size_t)kMaxLdsBytes)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: B*K = %d*%d exceeds the LDS-staged GEMV limit",
                      fn, B, p.K);
  // R = 4 rows per wavefront for small M (more workgroups), 8 for large M (more bytes in flight).
  const bool big = p.M >= 65536;
  const int rows_per_wg = 4 * (big ? 8 : 4);
  long long groups = ((long long)p.M + rows_per_wg - 1) / rows_per_wg;
  const int grid = (int)(groups < 16384 ? groups : 16384);
#define IRON_GEMV_CASE(BB)                                                                     \
  case BB:                                                                                     \
    if (big)                                                                                   \
      hipLaunchKernelGGL((gemv_kernel<BB, 8, INT8>), dim3(grid), dim3(256), lds, stream, p);   \
    else                                                                                       \
      hipLaunchKernelGGL((gemv_kernel<BB, 4, INT8>), dim3(grid), dim3(256), lds, stream, p);   \
    break;
  switch (B) {
    IRON_GEMV_CASE(1)
    IRON_GEMV_CASE(2)
    IRON_GEMV_CASE(3)
    IRON_GEMV_CASE(4)
    default:
      return iron::fail(IRON_ERR_UNSUPPORTED, "%s: batch %d > 4 needs the MFMA path", fn, B);
  }
#undef IRON_GEMV_CASE
  return iron::check_launch(fn);
}

GemvParams wire_params(const void* wire, int M, int K, int G, int tile_m, int domain) {
  GemvParams p = {};
  p.w = (const uint8_t*)wire;
  p.M = M;
  p.K = K;
  p.gshift = iron::ilog2(G);
  p.tile_m = tile_m;
  p.tdiv = make_fastdiv((uint32_t)tile_m);
  p.blk_bytes = (uint32_t)iron::wire_block_bytes(K, G, tile_m);
  p.xor_mask = domain == IRON_DOMAIN_SIGNED ? 0x80808080u : 0u;
  return p;
}

}  // namespace

namespace iron {
int gemv_swiglu_internal(const void* wg, const void* wu, const uint16_t* cur,
                         const uint16_t* a, const uint16_t* n_pf, float* gh, int B, int D,
                         int FF, int G, int tile_m, int domain, float eps, hipStream_t stream) {
  GemvParams p = wire_params(wg, FF, D, G, tile_m, domain);
  p.w2 = (const uint8_t*)wu;
  p.pro = PRO_RES_RMS_F32;
  p.x = cur;
  p.x2 = a;
  p.nw = n_pf;
  p.eps = eps;
  p.x_stride = D;
  p.x2_stride = D;
  p.epi = EPI_SWIGLU_F32;
  p.y = gh;
  p.y_stride = FF;
  return launch_gemv<true>(p, B, stream, "iron_swiglu_mlp(gate/up)");
}

int gemv_down_internal(const void* wd, const float* gh, const uint16_t* cur, const uint16_t* a,
                       uint16_t* nxt, int B, int D, int FF, int G, int tile_m, int domain,
                       hipStream_t stream) {
  GemvParams p = wire_params(wd, D, FF, G, tile_m, domain);
  p.pro = PRO_F32;
  p.x = gh;
  p.x_stride = FF;
  p.epi = EPI_RES_BF16;
  p.y = nxt;
  p.y_stride = D;
  p.r1 = cur;
  p.r2 = a;
  p.r_stride = D;
  return launch_gemv<true>(p, B, stream, "iron_swiglu_mlp(down)");
}

int gemv_rms_internal(const void* wire, const uint16_t* x, const uint16_t* nw, uint16_t* y,
                      int B, int M, int K, int G, int tile_m, int domain, float eps,
                      hipStream_t stream, const char* fn) {
  GemvParams p = wire_params(wire, M, K, G, tile_m, domain);
  p.pro = PRO_RMS_BF16;
  p.x = x;
  p.nw = nw;
  p.eps = eps;
  p.x_stride = K;
  p.epi = EPI_BF16;
  p.y = y;
  p.y_stride = M;
  return launch_gemv<true>(p, B, stream, fn);
}

int check_wire(const char* fn, const void* wire, int M, int K, int G, int tile_m, int domain) {
  if (!wire) return fail(IRON_ERR_NULL, "%s: weight wire is null", fn);
  if (M <= 0 || K <= 0) return fail(IRON_ERR_SHAPE, "%s: M=%d K=%d must be positive", fn, M, K);
  if (!is_pow2(G) || G < 16)
    return fail(IRON_ERR_SHAPE, "%s: group size %d must be a power of two >= 16", fn, G);
  if (K % G != 0) return fail(IRON_ERR_SHAPE, "%s: K=%d is not a multiple of G=%d", fn, K, G);
  if (tile_m <= 0 || M % tile_m != 0)
    return fail(IRON_ERR_SHAPE, "%s: tile_m=%d must divide M=%d", fn, tile_m, M);
  if ((wire_block_bytes(K, G, tile_m) % 16) != 0 || ((size_t)tile_m * K) % 16 != 0)
    return fail(IRON_ERR_ALIGN, "%s: wire block of tile_m=%d rows is not 16-byte aligned", fn,
                tile_m);
  if (!aligned(wire, 16)) return fail(IRON_ERR_ALIGN, "%s: wire pointer not 16-byte aligned", fn);
  if (domain != IRON_DOMAIN_SIGNED && domain != IRON_DOMAIN_BIASED)
    return fail(IRON_ERR_SHAPE, "%s: unknown payload domain %d", fn, domain);
  if ((long long)M >= (1ll << 31)) return fail(IRON_ERR_SHAPE, "%s: M too large", fn);
  return IRON_OK;
}
}  // namespace iron

extern "C" {

int iron_wire_bytes(int M, int K, int G, int tile_m, size_t* out_bytes) {
  iron::clear_error();
  if (!out_bytes) return iron::fail(IRON_ERR_NULL, "iron_wire_bytes: out_bytes is null");
  if (M <= 0 || K <= 0 || G <= 0 || tile_m <= 0 || K % G || M % tile_m)
    return iron::fail(IRON_ERR_SHAPE, "iron_wire_bytes: bad geometry M=%d K=%d G=%d tile_m=%d",
                      M, K, G, tile_m);
  *out_bytes = (size_t)(M / tile_m) * iron::wire_block_bytes(K, G, tile_m);
  return IRON_OK;
}

int iron_dequant_w8(const void* wire, uint16_t* w_out, int M, int K, int G, int tile_m,
                    int domain, void* stream) {
  iron::clear_error();
  int st = iron::check_wire("iron_dequant_w8", wire, M, K, G, tile_m, domain);
  if (st) return st;
  if (!w_out) return iron::fail(IRON_ERR_NULL, "iron_dequant_w8: output is null");
  if (K % 16) return iron::fail(IRON_ERR_SHAPE, "iron_dequant_w8: K=%d must be a multiple of 16", K);
  if (!iron::aligned(w_out, 16))
    return iron::fail(IRON_ERR_ALIGN, "iron_dequant_w8: output not 16-byte aligned");
  const long long work = (long long)M * (K / 16);
  long long blocks = (work + 255) / 256;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
  hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)wire, w_out, M, K, iron::ilog2(G), tile_m,
                     make_fastdiv((uint32_t)tile_m),
                     (uint32_t)iron::wire_block_bytes(K, G, tile_m),
                     domain == IRON_DOMAIN_SIGNED ? 0x80808080u : 0u);
  return iron::check_launch("iron_dequant_w8");
}

int iron_gemv_w8a16(const void* wire, const uint16_t* x, uint16_t* y, int B, int M, int K, int G,
                    int tile_m, int domain, void* stream) {
  iron::clear_error();
  int st = iron::check_wire("iron_gemv_w8a16", wire, M, K, G, tile_m, domain);
  if (st) return st;
  if (!x || !y) return iron::fail(IRON_ERR_NULL, "iron_gemv_w8a16: x or y is null");
  if (B <= 0) return iron::fail(IRON_ERR_SHAPE, "iron_gemv_w8a16: batch %d must be positive", B);
  if (K % 16) return iron::fail(IRON_ERR_SHAPE, "iron_gemv_w8a16: K=%d must be a multiple of 16", K);
  GemvParams p = wire_params(wire, M, K, G, tile_m, domain);
  p.pro = PRO_BF16;
  p.x = x;
  p.x_stride = K;
  p.epi = EPI_BF16;
  p.y = y;
  p.y_stride = M;
  return launch_gemv<true>(p, B, (hipStream_t)stream, "iron_gemv_w8a16");
}

int iron_gemv_bf16(const uint16_t* w, const uint16_t* x, uint16_t* y, int B, int M, int K,
                   void* stream) {
  iron::clear_error();
  if (!w || !x || !y) return iron::fail(IRON_ERR_NULL, "iron_gemv_bf16: null pointer");
  if (B <= 0 || M <= 0 || K <= 0 || K % 8)
    return iron::fail(IRON_ERR_SHAPE, "iron_gemv_bf16: bad shape B=%d M=%d K=%d", B, M, K);
  if (!iron::aligned(w, 16)) return iron::fail(IRON_ERR_ALIGN, "iron_gemv_bf16: W not 16B aligned");
  GemvParams p = {};
  p.w = (const uint8_t*)w;
  p.M = M;
  p.K = K;
  p.pro = PRO_BF16;
  p.x = x;
  p.x_stride = K;
  p.epi = EPI_BF16;
  p.y = y;
  p.y_stride = M;
  return launch_gemv<false>(p, B, (hipStream_t)stream, "iron_gemv_bf16");
}

int iron_lm_head(const void* w, int w_kind, const uint16_t* x, const uint16_t* norm_w, float eps,
                 uint16_t* logits, unsigned long long* argmax_keys, int B, int V, int D, int G,
                 int tile_m, int domain, void* stream) {
  iron::clear_error();
  if (!w || !x || !logits) return iron::fail(IRON_ERR_NULL, "iron_lm_head: null pointer");
  if (B <= 0 || V <= 0 || D <= 0 || D % 16)
    return iron::fail(IRON_ERR_SHAPE, "iron_lm_head: bad shape B=%d V=%d D=%d", B, V, D);
  GemvParams p = {};
  if (w_kind == IRON_WEIGHT_INT8) {
    int st = iron::check_wire("iron_lm_head", w, V, D, G, tile_m, domain);
    if (st) return st;
    p = wire_params(w, V, D, G, tile_m, domain);
  } else if (w_kind == IRON_WEIGHT_BF16) {
    if (!iron::aligned(w, 16)) return iron::fail(IRON_ERR_ALIGN, "iron_lm_head: W not 16B aligned");
    p.w = (const uint8_t*)w;
    p.M = V;
    p.K = D;
  } else {
    return iron::fail(IRON_ERR_SHAPE, "iron_lm_head: unknown weight kind %d", w_kind);
  }
  p.pro = norm_w ? PRO_RMS_BF16 : PRO_BF16;
  p.x = x;
  p.nw = norm_w;
  p.eps = eps;
  p.x_stride = D;
  p.epi = argmax_keys ? EPI_BF16_ARGMAX : EPI_BF16;
  p.y = logits;
  p.y_stride = V;
  p.argmax = argmax_keys;
  if (w_kind == IRON_WEIGHT_INT8) return launch_gemv<true>(p, B, (hipStream_t)stream, "iron_lm_head");
  return launch_gemv<false>(p, B, (hipStream_t)stream, "iron_lm_head");
}

}  // extern "C"
