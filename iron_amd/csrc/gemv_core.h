// Device building blocks of the weight-streaming GEMV, shared by the standalone kernels
// (gemv.hip) and the persistent whole-token decode kernel (decode_persistent.hip).
//
// Reference arithmetic: the int8 W8A16 matvec (aie_kernels/aie2p/mv_int8_signed.cc:60-113) with
// the value of the golden GEMVInt8.reference (iron/operators/gemv_int8/op.py:173-178),
// accumulated in fp64 and rounded once. Weights travel in the row-block wire of
// iron/operators/gemv_int8/reference.py:59-80.
#pragma once
#include "common.h"

namespace iron {
namespace dev {

enum Prologue : int {
  PRO_BF16 = 0,        // xs = x                                   (x bf16)
  PRO_RMS_BF16 = 1,    // xs = bf16(rmsnorm(x) * w)                (fused RMSNorm, bf16 boundary)
  PRO_RES_RMS_F32 = 2, // xs = f32(rmsnorm(f32(x + x2)) * w)       (SwiGLU MLP: x1 = cur + a)
  PRO_F32 = 3,         // xs = x                                   (x fp32)
};

enum Epilogue : int {
  EPI_BF16 = 0,        // y = bf16(acc)
  EPI_F32 = 1,         // y = f32(acc)
  EPI_RES_BF16 = 2,    // y = bf16(f32(r1 + r2) + acc)             (down GEMV + residual)
  EPI_SWIGLU_F32 = 3,  // y = f32(silu(acc_gate) * acc_up)         (dual matrix)
  EPI_BF16_ARGMAX = 4, // y = bf16(acc), plus the argmax key of the bf16 values
};

struct GemvParams {
  const uint8_t* w;     // int8 wire or bf16 row-major weights
  const uint8_t* w2;    // second int8 wire (EPI_SWIGLU_F32)
  int M, K, gshift, tile_m;
  FastDiv tdiv;
  uint32_t blk_bytes;
  uint32_t xor_mask;    // 0x80808080 for the biased domain (turns q+128 into q), 0 for signed
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
  int nb;               // batch rows of the launch (gemv.hip; rows past it are not read or written)
  int n_bgroups;        // batch groups of a multi-group launch (gemv.hip)
};

IRON_DEV void unpack8(const uint4 v, float (&f)[8]) {
  f[0] = bf16lo_to_f32(v.x); f[1] = bf16hi_to_f32(v.x);
  f[2] = bf16lo_to_f32(v.y); f[3] = bf16hi_to_f32(v.y);
  f[4] = bf16lo_to_f32(v.z); f[5] = bf16hi_to_f32(v.z);
  f[6] = bf16lo_to_f32(v.w); f[7] = bf16hi_to_f32(v.w);
}

// x (+ x2) of one slot as exact fp32 values (x1 = cur + a is the one fp32 rounding)
IRON_DEV void slot_values(uint4 xv, uint4 x2v, bool has_x2, float (&f)[8]) {
  unpack8(xv, f);
  if (has_x2) {
    float g[8];
    unpack8(x2v, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = f[j] + g[j];
  }
}

// ------------------------------------------------------------------------------------------
// Weight fetch: lane-resident 16-byte slices of R rows x NCH chunks (+ their group scales).
// ------------------------------------------------------------------------------------------
// Loads go to clamped addresses with no branch and no use of the loaded value, so every load of
// the group is in flight at once (a value read right after its load would make the wavefront
// wait for all earlier loads). Out-of-range slices are masked where they are used: their scale
// counts as 0 and their rows are never stored.
template <int R, int NCH>
IRON_DEV void fetch_w8(const GemvParams& p, const uint8_t* __restrict__ wire, int row0, int lane,
                       uint4 (&w)[R][NCH], uint32_t (&sraw)[R][NCH]) {
  const int K = p.K;
  const int ng = K >> p.gshift;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    const uint32_t rr = row < p.M ? (uint32_t)row : 0u;
    const uint32_t blk = fastdiv(rr, p.tdiv);
    const uint32_t in = rr - blk * (uint32_t)p.tile_m;
    const uint8_t* base = wire + (size_t)blk * p.blk_bytes;
    const uint8_t* qrow = base + (size_t)in * K;
    const uint16_t* srow = (const uint16_t*)(base + (size_t)p.tile_m * K) + (size_t)in * ng;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int e = c * 1024 + lane * 16;
      const int ec = e < K ? e : 0;
      w[r][c] = ld_global((const uint4*)(qrow + ec));
      sraw[r][c] = ld_global(srow + (ec >> p.gshift));
    }
  }
}

// scale of slice (r, c) as used by the dot product: 0 outside the matrix
IRON_DEV double slice_scale(const GemvParams& p, uint32_t sraw, int row, int e) {
  return (row < p.M && e < p.K) ? (double)bf16_to_f32(sraw) : 0.0;
}

IRON_DEV double sbyte(uint32_t d, int j) {
  return (double)(int)(((int32_t)(d << (24 - 8 * j))) >> 24);
}

// ------------------------------------------------------------------------------------------
// Batch-1 path with the activation in registers: lane l of a wavefront multiplies elements
// [c*CH + l*EPL, +EPL) of every chunk c (CH = 1024, EPL = 16 for int8; 512 and 8 for bf16), so
// it loads exactly those x (and norm-weight / residual) elements, and the RMSNorm statistic is a
// wavefront reduction: no LDS staging and no workgroup barrier. Every wavefront of a workgroup
// computes the (identical) statistic itself.
// ------------------------------------------------------------------------------------------
template <int NCH, int EPL>
IRON_DEV void load_x_lane(const GemvParams& p, int lane, uint4 (&xl)[NCH][EPL / 4],
                          uint4 (&x2l)[NCH][EPL / 8], uint4 (&nwl)[NCH][EPL / 8]) {
  const bool rms = p.pro == PRO_RMS_BF16 || p.pro == PRO_RES_RMS_F32;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 64 * EPL + lane * EPL;
#pragma unroll
    for (int u = 0; u < EPL / 4; ++u) xl[c][u] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int u = 0; u < EPL / 8; ++u) {
      x2l[c][u] = make_uint4(0u, 0u, 0u, 0u);
      nwl[c][u] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (e < p.K) {
      if (p.pro == PRO_F32) {
        const uint4* src = (const uint4*)((const float*)p.x + e);
#pragma unroll
        for (int u = 0; u < EPL / 4; ++u) xl[c][u] = src[u];
      } else {
        const uint4* src = (const uint4*)((const uint16_t*)p.x + e);
#pragma unroll
        for (int u = 0; u < EPL / 8; ++u) xl[c][u] = src[u];
        if (p.x2) {
#pragma unroll
          for (int u = 0; u < EPL / 8; ++u) x2l[c][u] = ((const uint4*)(p.x2 + e))[u];
        }
      }
      if (rms) {
#pragma unroll
        for (int u = 0; u < EPL / 8; ++u) nwl[c][u] = ((const uint4*)(p.nw + e))[u];
      }
    }
  }
}

// The prologue of the lane's elements: xf = the (exact fp32) value the dot product multiplies.
template <int NCH, int EPL>
IRON_DEV void prologue_lane(const GemvParams& p, int lane, const uint4 (&xl)[NCH][EPL / 4],
                            const uint4 (&x2l)[NCH][EPL / 8], const uint4 (&nwl)[NCH][EPL / 8],
                            float (&xf)[NCH][EPL]) {
  const bool has_x2 = p.x2 != nullptr;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (p.pro == PRO_F32) {
#pragma unroll
      for (int u = 0; u < EPL / 4; ++u) {
        xf[c][4 * u] = __uint_as_float(xl[c][u].x);
        xf[c][4 * u + 1] = __uint_as_float(xl[c][u].y);
        xf[c][4 * u + 2] = __uint_as_float(xl[c][u].z);
        xf[c][4 * u + 3] = __uint_as_float(xl[c][u].w);
      }
    } else {
#pragma unroll
      for (int u = 0; u < EPL / 8; ++u) {
        float f[8];
        slot_values(xl[c][u], x2l[c][u], has_x2, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) xf[c][8 * u + j] = f[j];
      }
    }
  }
  if (p.pro != PRO_RMS_BF16 && p.pro != PRO_RES_RMS_F32) return;
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    double v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) v[j] = xf[c][j];
    ss += sum_sq_tree(v);
  }
  ss = wave_sum_d(ss);
  const double inv = inv_rms(ss, p.K, (double)p.eps);
  const bool to_bf16 = p.pro == PRO_RMS_BF16;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int u = 0; u < EPL / 8; ++u) {
      float wf[8];
      unpack8(nwl[c][u], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const double y = ((double)xf[c][8 * u + j] * inv) * (double)wf[j];
        xf[c][8 * u + j] = to_bf16 ? round_bf16((float)y) : (float)y;
      }
    }
  }
}

// With REDUCE, acc[r] ends as row r's total in every lane (wave_sum_d); without, as this lane's
// partial, for a caller that reduces several rows together.
template <int R, int NCH, bool REDUCE = true>
IRON_DEV void dot_w8_lane(const GemvParams& p, const uint4 (&w)[R][NCH],
                          const uint32_t (&sc)[R][NCH], const float (&xf)[NCH][16], int row0,
                          int lane, double (&acc)[R][1]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r][0] = 0.0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    double xv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) xv[j] = xf[c][j];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd[4] = {w[r][c].x ^ p.xor_mask, w[r][c].y ^ p.xor_mask,
                              w[r][c].z ^ p.xor_mask, w[r][c].w ^ p.xor_mask};
      double pa = 0.0, pb = 0.0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa = fma(sbyte(dd[j], 0), xv[4 * j + 0], pa);
        pb = fma(sbyte(dd[j], 1), xv[4 * j + 1], pb);
        pa = fma(sbyte(dd[j], 2), xv[4 * j + 2], pa);
        pb = fma(sbyte(dd[j], 3), xv[4 * j + 3], pb);
      }
      acc[r][0] = fma(slice_scale(p, sc[r][c], row0 + r, c * 1024 + lane * 16), pa + pb,
                      acc[r][0]);
    }
  }
  if constexpr (REDUCE) {
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][0] = wave_sum_d(acc[r][0]);
  }
}

// Order-preserving key of a bf16 value (the argmax epilogues pack it above ~row).
IRON_DEV uint32_t bf16_order_key(uint16_t h) {
  return (h & 0x8000u) ? (uint32_t)(~h & 0xffffu) : (uint32_t)(h | 0x8000u);
}

// SiLU(g) * u in fp64 with the golden's numerically stable sigmoid
// (iron/operators/swiglu_mlp_dp/reference.py:28-33).
IRON_DEV double silu_mul(double g, double u) {
  // one exponential of -|g| serves both branches of the stable form (no divergent branch)
  const double e = exp(-fabs(g));
  const double sig = g >= 0.0 ? 1.0 / (1.0 + e) : e / (1.0 + e);
  return (g * sig) * u;
}

}  // namespace dev
}  // namespace iron
