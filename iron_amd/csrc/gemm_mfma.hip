// Batched int8-weight GEMM on MFMA for the fused blocks' decode batches above the GEMV path
// (B = 5..16; the entry point iron_gemm_w8a16 takes any B = 1..16):
//   Y[b][m] = EPI( sum_g s[m][g] * sum_{k in g} q[m][k] * x[b][k] )
//
// Reference: there is no int8 batched GEMM in the reference; its bf16 GEMM operator
// (iron/operators/gemm/op.py:23-80, golden gemm/reference.py:8-19) and the int8 GEMV golden
// (gemv_int8/op.py:173-178: dequantize, matmul, bf16) define the arithmetic. The weights are the
// same row-block wire as the GEMV (gemv_int8/reference.py:59-80).
//
// Arithmetic: q is exact in bf16 (|q| <= 127), so one v_mfma_f32_16x16x32_bf16 per 32-wide k
// step multiplies q by x exactly and sums 32 products in fp32; at the end of each quantization
// group the fp32 partial is scaled by s (in fp64) and added to an fp64 accumulator. fp32 inputs (the MLP's hf and gh) arrive as their three exact bf16 planes (hi +
// mid + lo, written so by their producers), three MFMAs per step. The result is within the fp32
// rounding of the per-group sums of the exact value (the parity bar is the north star's rel/abs
// 1e-2, and every output within one bf16 ulp of exact).
//
// Mapping: a workgroup (8 wavefronts, two per SIMD) owns 64 rows x 16 batch columns over a K range
// (split-K when the row tiles alone do not cover the chip). Per 128-wide K step the workgroup
// stages the weight tile (64 rows x 128 int8 per matrix), its group scales and x (16 x 128, bf16
// planes) in LDS (double buffered: the next step's global loads are in flight while this one
// computes). Wavefront w multiplies rows 16 (w % 4) .. +15 over the step's 64-wide half w / 4:
// lane l reads A = 8 int8 of row l%16 at k = (l/16)*8 and B = 8 bf16 of batch column l%16 at the
// same k; its 4 accumulators are rows (l/16)*4 + i, column l%16 (the gfx950 16x16x32 operand
// layout, checked on the device). The two halves' fp64 sums add through LDS at the end. With one
// wavefront per SIMD every step waited out its own LDS -> convert -> MFMA -> scale chain (about
// 1.6 us a step); the second wavefront per SIMD overlaps them.
#include "common.h"
#include "internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kTM = 64;           // rows per workgroup
constexpr int kKS = 128;          // K per pipeline step
constexpr int kBN = 16;           // batch columns
constexpr int kWRow = kKS + 16;   // LDS bytes per weight row (padded)
constexpr int kXRow = kKS + 8;    // LDS bf16 per x row (padded)

// epilogues (iron::GEMM_EPI_*): bf16(acc) | f32(silu(acc0) * acc1) as three bf16 planes (dual) |
// bf16(f32(r1 + r2) + acc)

struct GemmParams {
  const uint8_t* w0;
  const uint8_t* w1;      // second matrix (dual) or null
  int M, K, gshift, tile_m;
  FastDiv tdiv;
  uint32_t blk_bytes, xor_mask;
  const uint16_t* x;      // [B][x_stride] bf16, or [3][B][x_stride] bf16 planes of fp32 values
  size_t x_plane;         // plane stride (elements) of the planes form, 0 for plain bf16
  int B, x_stride;
  int splits, ksteps;     // split s covers pipeline steps [s*ksteps, (s+1)*ksteps)
  double* part;           // [2][splits][kBN][M] fp64 partials (splits > 1)
  unsigned int* ctr;      // [M / kTM] arrival counts of the splits (splits > 1; zero between calls)
  int epi;
  void* y;
  int y_stride;
  size_t y_plane;         // plane stride of the planes epilogue
  const uint16_t* r1;
  const uint16_t* r2;
  int r_stride;
  // the folded residual RMSNorm (iron::GemmResNorm): the tile sums of squares the producer writes
  // and the consumer reads; for the consumer also the norm weight, D / 64 and eps (cur, a: r1, r2)
  double* ssq;
  const uint16_t* n_w;
  int n_tiles;
  float n_eps;
};

IRON_DEV double silu_mul_d(double g, double u) {
  double sig;
  if (g >= 0.0) {
    sig = 1.0 / (1.0 + exp(-g));
  } else {
    const double e = exp(g);
    sig = e / (1.0 + e);
  }
  return (g * sig) * u;
}

IRON_DEV void store_out(const GemmParams& p, int b, int m, double a0, double a1) {
  const size_t o = (size_t)b * p.y_stride + m;
  switch (p.epi) {
    case iron::GEMM_EPI_BF16: ((uint16_t*)p.y)[o] = f64_to_bf16(a0); break;
    case iron::GEMM_EPI_SWIGLU_PLANES: {
      uint16_t* y = (uint16_t*)p.y;
      split3_bf16((float)silu_mul_d(a0, a1), y[o], y[o + p.y_plane], y[o + 2 * p.y_plane]);
      break;
    }
    default: {
      const size_t ro = (size_t)b * p.r_stride + m;
      float x1 = bf16_to_f32(p.r1[ro]);
      if (p.r2) x1 = x1 + bf16_to_f32(p.r2[ro]);
      ((uint16_t*)p.y)[o] = f64_to_bf16((double)x1 + a0);
    }
  }
}

// 8 int8 weights as biased bytes u = q + 128 (two dwords) -> 8 bf16 of q (exact: |q| <= 128 has
// at most 8 significant bits, so the high half of f32(q) is its bf16). f32(u) is one
// v_cvt_f32_ubyte per byte, f32(u) - 128 = f32(q) exactly, and one v_perm_b32 packs two high
// halves: 20 VALU instructions for 8 weights where a sign extension, convert and shift per byte
// took 28.
IRON_DEV bf16x8 u8_to_bf16q(uint32_t lo, uint32_t hi) {
  auto two = [](uint32_t d, int sh) {
    const float f0 = (float)((d >> sh) & 0xffu) - 128.f;
    const float f1 = (float)((d >> (sh + 8)) & 0xffu) - 128.f;
    return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  };
  const uint4 r = make_uint4(two(lo, 0), two(lo, 16), two(hi, 0), two(hi, 16));
  return __builtin_bit_cast(bf16x8, r);
}

// NORM: x is the residual RMSNorm's hf (iron::GemmResNorm without tile sums). Every workgroup
// sums x1^2 over each whole batch row (2 B x K bf16 from the L2), then writes hf's three planes
// for its split's K range (at most kNormSteps steps) into LDS once, from cur (r1), a (r2) and the
// norm weight (n_w); the step loop then loads and stages weights only. Staging the planes step by
// step instead, between the step's loads and its barrier, measured 2-4 us slower on config 2.
constexpr int kNormSteps = 4;
constexpr int kHRow = kNormSteps * kKS + 8;  // bf16 per plane row of hf (padded like s_x's rows)
template <bool DUAL, bool XPL, bool NORM = false>
__global__ __launch_bounds__(512) void gemm_w8_mfma_kernel(GemmParams p) {
  static_assert(!NORM || (DUAL && XPL), "the residual RMSNorm feeds the dual GEMM's fp32 planes");
  constexpr int NM = DUAL ? 2 : 1;
  constexpr int NX = XPL ? 3 : 1;    // bf16 planes of x (fp32 x: hi, mid, lo)
  __shared__ __align__(16) uint8_t s_w[2][NM][kTM][kWRow];
  __shared__ __align__(16) uint16_t s_s[2][NM][kTM][kKS / 32];
  __shared__ __align__(16) uint16_t s_x[2][NX][kBN][kXRow];
  // NORM: hf's planes [3][B][kHRow] in the launch's dynamic LDS (B rows only: at B <= 8 two
  // workgroups fit on a CU)
  extern __shared__ __align__(16) uint16_t s_hf[];
  __shared__ double s_inv[kBN];
  // the upper half's sums at the end, in the weight tiles' space past the split-K staging (s_part
  // below): 16 KiB less LDS, so two dual workgroups fit on a CU (measured neutral: the kernel is
  // bound by its issue, not its occupancy)
  constexpr size_t kAccOff = (sizeof(double) * NM * kBN * (kTM + 1) + 255) & ~(size_t)255;
  static_assert(kAccOff + sizeof(double) * 4 * NM * 4 * 64 <= sizeof(s_w), "s_acc fits in s_w");
  double (*const s_acc)[NM][4][64] =
      reinterpret_cast<double (*)[NM][4][64]>(&s_w[0][0][0][0] + kAccOff);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int half = wave >> 2;  // the 64-wide half of every step this wavefront multiplies
  const int row0 = blockIdx.x * kTM;
  const int split = blockIdx.y;
  const int step0 = split * p.ksteps;
  const int nsteps = min(p.ksteps, p.K / kKS - step0);  // the last split may be shorter
  const int ng = p.K >> p.gshift;
  const int G = 1 << p.gshift;

  // ---- global -> register staging of one pipeline step
  const int lrow = tid >> 3, lpart = tid & 7;  // weight tile: row, 16-byte eighth
  const uint8_t* wbase[NM];
  const uint16_t* sbase[NM];
  {
    const uint32_t row = (uint32_t)(row0 + lrow);
    const uint32_t blk = fastdiv(row, p.tdiv);
    const uint32_t in = row - blk * (uint32_t)p.tile_m;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      const uint8_t* base = (mi == 0 ? p.w0 : p.w1) + (size_t)blk * p.blk_bytes;
      wbase[mi] = base + (size_t)in * p.K;
      sbase[mi] = (const uint16_t*)(base + (size_t)p.tile_m * p.K) + (size_t)in * ng;
    }
  }
  // x tile: batch row, 8-element chunk (wavefronts 4..7 load the same x as 0..3 and store none)
  const int xb = (tid >> 4) & 15, xk = (tid & 15) * 8;
  // registers of one pipeline step: the weight eighth-rows of matrix 0 (and 1), their
  // scales, and 8 x values of each plane
  uint4 wa0, wb0, rx0, rx1, rx2;
  uint32_t sa, sb;
  const int gpr = kKS / G;  // groups per step (G <= kKS)
  const uint8_t* wsrc0 = wbase[0];
  const uint8_t* wsrc1 = wbase[NM - 1];
  const uint16_t* ssrc0 = sbase[0];
  const uint16_t* ssrc1 = sbase[NM - 1];
  const size_t xrow = (size_t)(xb < p.B ? xb : 0) * p.x_stride;
#define GEMM_GLOAD(step_)                                                                      \
  do {                                                                                         \
    const int k0_ = (step_) * kKS;                                                             \
    const int gi_ = (k0_ >> p.gshift) + (lpart < gpr ? lpart : 0);                             \
    wa0 = *(const uint4*)(wsrc0 + k0_ + lpart * 16);                                           \
    sa = ssrc0[gi_];                                                                           \
    if (DUAL) {                                                                                \
      wb0 = *(const uint4*)(wsrc1 + k0_ + lpart * 16);                                         \
      sb = ssrc1[gi_];                                                                         \
    }                                                                                          \
    if (!NORM) rx0 = *(const uint4*)(p.x + xrow + k0_ + xk);                                   \
    if (XPL && !NORM) {                                                                        \
      rx1 = *(const uint4*)(p.x + p.x_plane + xrow + k0_ + xk);                                \
      rx2 = *(const uint4*)(p.x + 2 * p.x_plane + xrow + k0_ + xk);                            \
    }                                                                                          \
  } while (0)
#define GEMM_LSTORE(buf_)                                                                      \
  do {                                                                                         \
    *(uint4*)&s_w[(buf_)][0][lrow][lpart * 16] = wa0;                                          \
    if (lpart < kKS / 32) s_s[(buf_)][0][lrow][lpart] = (uint16_t)sa;                          \
    if (DUAL) {                                                                                \
      *(uint4*)&s_w[(buf_)][NM - 1][lrow][lpart * 16] = wb0;                                   \
      if (lpart < kKS / 32) s_s[(buf_)][NM - 1][lrow][lpart] = (uint16_t)sb;                   \
    }                                                                                          \
    if (!NORM && tid < 256) {                                                                  \
      *(uint4*)&s_x[(buf_)][0][xb][xk] = xb < p.B ? rx0 : make_uint4(0u, 0u, 0u, 0u);          \
      if (XPL) {                                                                               \
        *(uint4*)&s_x[(buf_)][NX - 2][xb][xk] = xb < p.B ? rx1 : make_uint4(0u, 0u, 0u, 0u);   \
        *(uint4*)&s_x[(buf_)][NX - 1][xb][xk] = xb < p.B ? rx2 : make_uint4(0u, 0u, 0u, 0u);   \
      }                                                                                        \
    }                                                                                          \
  } while (0)

  // ---- compute state
  double acc[NM][4];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mi][i] = 0.0;
  f32x4 c[NM];
#pragma unroll
  for (int mi = 0; mi < NM; ++mi) c[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t to_u = p.xor_mask ^ 0x80808080u;  // stored bytes -> q + 128
  const int wrow = (wave & 3) * 16;              // this wavefront's 16 rows (tile-relative)
  const int arow = wrow + (lane & 15);           // A operand row
  const int kq = (lane >> 4) * 8;                // k offset of this lane in a 32-step
  const int bcol = lane & 15;                    // B operand / C column (batch)
  const int crow = wrow + (lane >> 4) * 4;       // first C row
  // NORM: the plane row of this lane's batch column (columns past B read row 0; their outputs are
  // never stored)
  const int hrow = bcol < p.B ? bcol : 0;

  // NORM: the row sums' inputs of the first 2048 elements of row `wave` and the split's pieces
  // of cur, a and the norm weight are loaded ahead of the first step's weights, so that their
  // wait does not include the weights' (the counts are in order)
  const int n8 = nsteps * (kKS / 8);  // NORM: 8-element pieces per row of the split's K range
  const int kb = step0 * kKS;
  const int bw = __builtin_amdgcn_readfirstlane(wave);
  uint4 hc[2], ha[2], hw[2], rc[4], ra[4];
  auto load_round = [&](int b, int k0, uint4 (&c4)[4], uint4 (&a4)[4]) __attribute__((always_inline)) {
    const uint16_t* cr = p.r1 + (size_t)b * p.x_stride;
    const uint16_t* ar = p.r2 + (size_t)b * p.x_stride;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int k = k0 + 512 * q;
      c4[q] = k < p.K ? *(const uint4*)(cr + k) : make_uint4(0u, 0u, 0u, 0u);
      a4[q] = k < p.K ? *(const uint4*)(ar + k) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  if constexpr (NORM) {
    // the split's pieces (8 elements each, at most two per thread: B x nsteps x 16 <= 1024)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + 512 * u, b = i / n8, c = (i - b * n8) * 8;
      if (i < p.B * n8) {
        const size_t o = (size_t)b * p.x_stride + kb + c;
        hc[u] = *(const uint4*)(p.r1 + o);
        ha[u] = *(const uint4*)(p.r2 + o);
        hw[u] = *(const uint4*)(p.n_w + kb + c);
      }
    }
    if (bw < p.B) load_round(bw, lane * 8, rc, ra);
  }
  GEMM_GLOAD(step0);
  if constexpr (NORM) {
    // 1 / RMS of every batch row over the whole of x1 = f32(cur + a) (K = D elements): wavefront
    // w sums rows w and w + 8, each lane 8 elements of every 512, a round of 2048 elements'
    // loads in flight together. The squares and their fp64 sums are exact (see sum_sq_tree), so
    // this order gives the separate kernel's value.
    for (int b = bw; b < p.B; b += 8) {
      double sq[4] = {0.0, 0.0, 0.0, 0.0};
      auto accum = [&](const uint4 (&c4)[4], const uint4 (&a4)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t cw[4] = {c4[q].x, c4[q].y, c4[q].z, c4[q].w};
          const uint32_t aw[4] = {a4[q].x, a4[q].y, a4[q].z, a4[q].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(cw[e] << 16) + __uint_as_float(aw[e] << 16);
            const float hi = __uint_as_float(cw[e] & 0xffff0000u) +
                             __uint_as_float(aw[e] & 0xffff0000u);
            sq[e] = fma((double)lo, (double)lo, sq[e]);
            sq[e] = fma((double)hi, (double)hi, sq[e]);
          }
        }
      };
      if (b == bw) {
        accum(rc, ra);
      } else {
        uint4 c4[4], a4[4];
        load_round(b, lane * 8, c4, a4);
        accum(c4, a4);
      }
      for (int k0 = lane * 8 + 2048; k0 < p.K; k0 += 2048) {
        uint4 c4[4], a4[4];
        load_round(b, k0, c4, a4);
        accum(c4, a4);
      }
      const double ss = wave_sum_d((sq[0] + sq[1]) + (sq[2] + sq[3]));
      if (lane == 0) s_inv[b] = inv_rms(ss, p.K, (double)p.n_eps);
    }
    __syncthreads();
    // hf = f32((f32(cur + a) * inv) * w), evaluated in fp64 (the separate kernel's roundings),
    // as three exact bf16 planes over the split's K range
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + 512 * u, b = i / n8, c = (i - b * n8) * 8;
      if (i >= p.B * n8) break;
      uint4 pl[3];
      {
        const uint4 c4 = hc[u], a4 = ha[u], w4 = hw[u];
        const double inv = s_inv[b];
        const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w}, aw[4] = {a4.x, a4.y, a4.z, a4.w};
        const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
        uint32_t pw[3][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t h[2][3];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            auto el = [&](uint32_t d) {
              return __uint_as_float(hh ? (d & 0xffff0000u) : (d << 16));
            };
            const float x1 = el(cw[e]) + el(aw[e]);
            const double y = ((double)x1 * inv) * (double)el(ww[e]);
            split3_bf16((float)y, h[hh][0], h[hh][1], h[hh][2]);
          }
#pragma unroll
          for (int xi = 0; xi < 3; ++xi)
            pw[xi][e] = (uint32_t)h[0][xi] | ((uint32_t)h[1][xi] << 16);
        }
#pragma unroll
        for (int xi = 0; xi < 3; ++xi) pl[xi] = make_uint4(pw[xi][0], pw[xi][1], pw[xi][2], pw[xi][3]);
      }
#pragma unroll
      for (int xi = 0; xi < 3; ++xi) *(uint4*)&s_hf[(xi * p.B + b) * kHRow + c] = pl[xi];
    }
  }
  GEMM_LSTORE(0);
  __syncthreads();
  for (int it = 0; it < nsteps; ++it) {
    const int buf = it & 1;
    if (it + 1 < nsteps) GEMM_GLOAD(step0 + it + 1);
    const int k0 = (step0 + it) * kKS;
    // this wavefront's two 32-wide steps: the group sums are flushed at every group end and at the
    // end of the half (a group longer than 64 continues in the other half's wavefront)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * half + jj;
      bf16x8 bx[NX];
#pragma unroll
      for (int xi = 0; xi < NX; ++xi)
        bx[xi] = __builtin_bit_cast(
            bf16x8, NORM ? *(const uint4*)&s_hf[(xi * p.B + hrow) * kHRow + it * kKS + 32 * j + kq]
                         : *(const uint4*)&s_x[buf][xi][bcol][32 * j + kq]);
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        const uint2 qa = *(const uint2*)&s_w[buf][mi][arow][32 * j + kq];
        const bf16x8 a = u8_to_bf16q(qa.x ^ to_u, qa.y ^ to_u);
#pragma unroll
        for (int xi = 0; xi < NX; ++xi)
          c[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bx[xi], c[mi], 0, 0, 0);
      }

      if (jj == 1 || ((k0 + 32 * (j + 1)) & (G - 1)) == 0) {  // end of a group or of the half
        const int gl = (32 * j) >> p.gshift;        // group index within this step
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const double s = bf16_to_f32(s_s[buf][mi][crow + i][gl]);
            acc[mi][i] = fma(s, (double)c[mi][i], acc[mi][i]);
          }
          c[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    if (it + 1 < nsteps) GEMM_LSTORE(buf ^ 1);
    __syncthreads();
  }

#undef GEMM_GLOAD
#undef GEMM_LSTORE
  // ---- the upper half's sums join the lower half's (in that order), then the write
  if (half) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_acc[wave & 3][mi][i][lane] = acc[mi][i];
  }
  __syncthreads();
  if (!half) {
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mi][i] += s_acc[wave][mi][i][lane];
  }
  if (p.splits == 1) {
    if (!half && bcol < p.B) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        store_out(p, bcol, row0 + crow + i, acc[0][i], NM > 1 ? acc[NM - 1][i] : 0.0);
    }
    return;
  }
  // Split K: this split's fp64 partials go to memory (agent-scope stores write through the L2),
  // and the last split of the row tile to arrive (one atomic count per tile) sums them in split
  // order -- the order a separate reduce kernel used -- and applies the epilogue, then clears
  // the count for the next call. Every thread's stores are complete before the count. The
  // partials pass through LDS (the weight tiles' space) so that consecutive threads store
  // consecutive rows: write-through stores are not merged in the L2, so scattered 8-byte stores
  // would each cost a whole memory sector.
  // (rows padded to kTM + 1 doubles: the 16 batch columns a wavefront writes fall in distinct banks)
  double (*const s_part)[kBN][kTM + 1] =
      reinterpret_cast<double (*)[kBN][kTM + 1]>(&s_w[0][0][0][0]);
  static_assert(sizeof(double) * NM * kBN * (kTM + 1) <= sizeof(s_w), "s_part fits in s_w");
  if (!half) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) s_part[mi][bcol][crow + i] = acc[mi][i];
  }
  __syncthreads();
  for (int t = tid; t < NM * p.B * kTM; t += 512) {
    const int mi = t / (p.B * kTM), b = (t / kTM) % p.B, r = t % kTM;
    __hip_atomic_store(p.part + (((size_t)mi * p.splits + split) * kBN + b) * p.M + row0 + r,
                       s_part[mi][b][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  __shared__ unsigned int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.ctr + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == (unsigned int)(p.splits - 1);
  __syncthreads();
  if (!s_last) return;
  // The partials are read past this XCD's L2 (which may hold lines of an earlier call) with
  // device-scope (sc1) buffer loads, eight in flight per thread; the sum runs in split order.
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      p.part, 0, NM * p.splits * kBN * p.M * (int)sizeof(double), kBufferDword3);
  static_assert(kTM == 64, "a wavefront's lanes are one batch row's tile rows");
  for (int t = tid; t < kTM * p.B; t += 512) {  // whole wavefronts: kTM * B is a multiple of 64
    const int b = t / kTM, m = row0 + t % kTM;
    // the folded RMSNorm's residual input, loaded ahead of the partials (in flight with them)
    const uint16_t cur = p.ssq ? p.r1[(size_t)b * p.r_stride + m] : (uint16_t)0;
    double a[2] = {0.0, 0.0};
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
      for (int s0 = 0; s0 < p.splits; s0 += 8) {
        double v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int sp = s0 + j < p.splits ? s0 + j : p.splits - 1;
          v[j] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(
              rs, (((mi * p.splits + sp) * kBN + b) * p.M + m) * (int)sizeof(double), 0, kCpolSc1));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (s0 + j < p.splits) a[mi] += v[j];
      }
    store_out(p, b, m, a[0], a[1]);
    if (p.ssq) {
      // x1 = f32(cur + bf16(y)) of the folded RMSNorm, squared (exact in fp64): a wavefront's 64
      // lanes are the tile's 64 rows of one batch row (kTM = 64, t = 64 w + lane), so the tile's
      // sum is a wavefront sum in wave_sum_d's fixed order
      const float x1 = bf16_to_f32(cur) + bf16_to_f32(f64_to_bf16(a[0]));
      const double ss = wave_sum_d((double)x1 * (double)x1);
      if (lane == 0) p.ssq[(size_t)blockIdx.x * kBN + b] = ss;
    }
  }
  if (tid == 0) __hip_atomic_store(p.ctr + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// Register-streamed form (M a multiple of the tile, K of 256): the weights never pass through LDS
// and the K loop has one barrier per 256-wide chunk. Each of a workgroup's 4 wavefronts owns RB
// 16-row blocks over the workgroup's K range and streams them from memory straight into MFMA
// operands, one 16-byte load per lane per row block and 64-wide k block (lane (q, r) = lane / 16,
// lane % 16: row r, bytes q*16 .. +15 of the block; each instruction reads 64 bytes of 16 rows),
// kRDepth blocks ahead: the ring is a chunk deep. x (every plane) and the tile's group scales
// pass through LDS a chunk at a time, loaded a chunk ahead into registers and written at the
// chunk's end. The activations are the MFMA A operand (lane (q, b): batch row b, k q*8 .. +7 of
// the 32-wide group; rows past B read as zero from a buffer sized to B rows), the weights the B
// operand (lane (q, r): row r, the same k), so C[b][row] sits in lane (q, r) for batch rows
// 4q .. 4q+3 of row r, and each lane scales its own row's group sums.
//
// Why not LDS for the weights too: the staged form keeps one step of loads in flight per
// workgroup. A read probe over a 100 MB matrix (16 rows x 64 bytes per instruction, 4 loads in
// flight per row block, 2 or 4 splits) reads at 4.5-5.2 TB/s; 8-byte loads (16 rows x 32 bytes)
// at 2.8-3.4, and every activation load in the weight loop costs about as much as a weight load.
constexpr int kRChunk = 256;              // k per LDS chunk of x and scales
constexpr int kRBlk = 64;                 // k per 16-byte weight load
constexpr int kRDepth = kRChunk / kRBlk;  // weight loads in flight per row block: one chunk
constexpr int kRXRow = kRChunk + 8;       // LDS bf16 per x row (padded: conflict-free reads)

// The four 16-lane rows of a wavefront hold 16 consecutive k of the same 16 weight rows (bytes
// q*16 .. +15 of a 64-wide block). Two swaps put them in the MFMA operand order of the block's two
// 32-wide groups: afterwards lane (q, r) holds k q*8 .. +7 of group 0 in (x, y) and of group 1
// in (z, w) (permlane16_swap exchanges the odd rows of its first operand with the even rows of
// its second, permlane32_swap the upper half of the first with the lower half of the second).
IRON_DEV iron_u32x4 quarter_transpose(iron_u32x4 v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v.x, v.z, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(v.y, v.w, false, false);
  const auto c = __builtin_amdgcn_permlane32_swap(a[0], a[1], false, false);
  const auto d = __builtin_amdgcn_permlane32_swap(b[0], b[1], false, false);
  return iron_u32x4{c[0], d[0], c[1], d[1]};
}

// 8 int8 weights as biased bytes u = q + 128 (two dwords) -> 8 bf16 of u (exact: u <= 255 has
// at most 8 significant bits): one v_cvt_f32_ubyte per byte and one v_perm_b32 per two, 12 VALU
// instructions where the signed form takes 20; the -128 q offset enters through the group's
// accumulator start value, -128 * (the group's x sum) per batch row.
IRON_DEV bf16x8 u8_to_bf16u(uint32_t lo, uint32_t hi) {
  auto two = [](uint32_t d, int sh) {
    const float f0 = (float)((d >> sh) & 0xffu);
    const float f1 = (float)((d >> (sh + 8)) & 0xffu);
    return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  };
  const uint4 r = make_uint4(two(lo, 0), two(lo, 16), two(hi, 0), two(hi, 16));
  return __builtin_bit_cast(bf16x8, r);
}


// NORM: x is the folded residual RMSNorm's hf (iron::GemmResNorm), staged from cur (r1), a (r2)
// and the norm weight (n_w): the three buffers take the places of the three planes.
template <bool DUAL, bool XPL, int W, int RB, bool G32, bool NORM = false>
__global__ __launch_bounds__(64 * W, 4) void gemm_w8_rs_kernel(GemmParams p) {
  constexpr int NM = DUAL ? 2 : 1;
  constexpr int NX = XPL ? 3 : 1;
  static_assert(!NORM || XPL, "the folded RMSNorm stages fp32 hf as three planes");
  constexpr int NT = 64 * W;                      // threads
  constexpr int TILE = 16 * RB * W;
  constexpr int XP = kBN * kRChunk * 2 / (NT * 16);  // 16-byte x pieces per plane and thread
  constexpr int SB = NM * TILE * 16 / NT;         // scale bytes per thread and chunk
  static_assert(XP >= 1 && (SB == 4 || SB == 8 || SB == 16), "chunk staging per thread");
  static_assert(W % NM == 0, "whole wavefronts stage each matrix's scales");
  __shared__ __align__(16) uint16_t s_x[2][NX][kBN][kRXRow];
  __shared__ __align__(16) uint8_t s_s[2][NM][TILE][16];  // 8 group scales per row and chunk
  __shared__ __align__(16) float s_corr[2][8][kBN];  // -128 * (x sum) per group and batch row
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 15, quarter = lane >> 4;
  const int tile0 = blockIdx.x * TILE, row0 = tile0 + wave * 16 * RB;
  const int gmask = (1 << p.gshift) - 1;
  const int split = blockIdx.y;
  const int cb = split * p.ksteps;                           // first chunk of this split
  const int nc = min(p.ksteps, p.K / kRChunk - cb);          // its chunks (>= 1)
  const int nb = nc * kRDepth;                               // its 64-wide blocks
  const int kbase = cb * kRChunk;
  const int ng = p.K >> p.gshift;
  const uint32_t to_u = p.xor_mask ^ 0x80808080u;  // stored bytes -> q + 128

  // this lane's weight rows row0 + 16 rb + col: bytes quarter*16 of each 64-wide block
  const uint8_t* wp[RB][NM];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint32_t row = (uint32_t)(row0 + 16 * rb + col);
    const uint32_t blk = fastdiv(row, p.tdiv);
    const uint32_t in = row - blk * (uint32_t)p.tile_m;
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
      wp[rb][mi] = (mi == 0 ? p.w0 : p.w1) + (size_t)blk * p.blk_bytes + (size_t)in * p.K + kbase +
                   quarter * 16;
  }
  // staging of a chunk: x (two 16-byte pieces per plane and thread: row idx / 32, k (idx % 32)*8)
  // and SB bytes of the tile's scales (flat byte f = tid * SB of [NM][TILE][16], from the row's
  // scale of the chunk's first group; reads past a row's own groups land in the wire or past its
  // end, where the buffer returns zero, and are never used)
  __amdgpu_buffer_rsrc_t xr[NX];
  if constexpr (NORM) {  // cur, a (rows of x_stride = D elements) and the norm weight
    xr[0] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.r1), 0,
                                              p.B * p.x_stride * 2, kBufferDword3);
    xr[1] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.r2), 0,
                                              p.B * p.x_stride * 2, kBufferDword3);
    xr[2] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.n_w), 0, p.K * 2,
                                              kBufferDword3);
  } else {
#pragma unroll
    for (int xi = 0; xi < NX; ++xi)
      xr[xi] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x + xi * p.x_plane), 0,
                                                 p.B * p.x_stride * 2, kBufferDword3);
  }
  int xvo[XP];
#pragma unroll
  for (int h = 0; h < XP; ++h) {
    const int idx = tid + NT * h;
    xvo[h] = ((idx >> 5) * p.x_stride + (idx & 31) * 8) * 2;
  }
  // NORM: 1 / RMS of every batch row from the producer's D / 64 tile sums (up to 128): lane j of
  // the 32 that serve batch row b = tid / 32 loads tiles j, j + 32, .. (issued first, ahead of the
  // first chunk and the ring), and after the ring is issued the 32 lanes add in a fixed tree
  // order. Rows past B get 0 (their cur and a read as zero).
  __shared__ double s_inv[kBN];
  double nv[4];
  auto norm_issue = [&]() {
    static_assert(NT >= 32 * kBN, "32 lanes per batch row");
    const int b = (tid >> 5) & (kBN - 1), j = tid & 31;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = j + 32 * k;
      nv[k] = tid < 32 * kBN && b < p.B && t < p.n_tiles ? p.ssq[(size_t)t * kBN + b] : 0.0;
    }
  };
  auto norm_finish = [&]() {
    const int b = (tid >> 5) & (kBN - 1), j = tid & 31;
    double ss = (nv[0] + nv[1]) + (nv[2] + nv[3]);
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 32);
    if (tid < 32 * kBN && j == 0) s_inv[b] = b < p.B ? inv_rms(ss, p.K, (double)p.n_eps) : 0.0;
    __syncthreads();
  };
  const int sf = tid * SB;
  // the matrix is the same across a wavefront (W / NM whole wavefronts per matrix): a uniform
  // value keeps the buffer descriptor in scalar registers (else every load loops over lanes)
  const int s_mi = __builtin_amdgcn_readfirstlane(sf / (TILE * 16));
  const int s_row = (sf >> 4) % TILE, s_byte = sf & 15;
  __amdgpu_buffer_rsrc_t sr;
  int svo;
  {
    const uint32_t row = (uint32_t)(tile0 + s_row);
    const uint32_t blk = fastdiv(row, p.tdiv);
    const uint32_t in = row - blk * (uint32_t)p.tile_m;
    const uint32_t nblk = ((uint32_t)p.M + p.tile_m - 1) / (uint32_t)p.tile_m;
    sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(s_mi == 0 ? p.w0 : p.w1), 0,
                                           (int)(nblk * p.blk_bytes), kBufferDword3);
    svo = (int)(blk * p.blk_bytes + (uint32_t)p.tile_m * p.K + (in * ng) * 2 + s_byte);
  }
  iron_u32x4 xs[NX][XP];
  iron_u32x4 ss4;
  iron_u32x2 ss2;
  uint32_t ss1;
  auto xload = [&](int c) {
    const int kc = kbase + c * kRChunk;
#pragma unroll
    for (int xi = 0; xi < NX; ++xi)
#pragma unroll
      for (int h = 0; h < XP; ++h) {
        // NORM's norm weight has no batch rows: element k of the piece's row at every row
        const int vo = NORM && xi == 2 ? ((tid + NT * h) & 31) * 16 : xvo[h];
        xs[xi][h] = __builtin_amdgcn_raw_buffer_load_b128(xr[xi], vo, kc * 2, 0);
      }
    const int so = (kc >> p.gshift) * 2;
    if constexpr (SB == 16) ss4 = __builtin_amdgcn_raw_buffer_load_b128(sr, svo, so, 0);
    else if constexpr (SB == 8) ss2 = __builtin_amdgcn_raw_buffer_load_b64(sr, svo, so, 0);
    else ss1 = __builtin_amdgcn_raw_buffer_load_b32(sr, svo, so, 0);
  };
  auto xstore = [&](int buf) {
#pragma unroll
    for (int h = 0; h < XP; ++h) {
      const int idx = tid + NT * h;
      iron_u32x4 xp[NX];  // the piece's planes
      if constexpr (NORM) {
        // hf = f32((f32(cur + a) * inv) * w), evaluated in fp64 and split into three exact
        // planes: the values and roundings of the separate residual-RMSNorm kernel (api.hip)
        const double inv = s_inv[idx >> 5];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t pl[2][3];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint32_t sh = hh ? 0xffff0000u : 0u;
            auto el = [&](uint32_t d) {
              return __uint_as_float(hh ? (d & sh) : (d << 16));
            };
            const float x1 = el(xs[0][h][e]) + el(xs[1][h][e]);
            const double y = ((double)x1 * inv) * (double)el(xs[2][h][e]);
            split3_bf16((float)y, pl[hh][0], pl[hh][1], pl[hh][2]);
          }
#pragma unroll
          for (int xi = 0; xi < 3; ++xi)
            xp[xi][e] = (uint32_t)pl[0][xi] | ((uint32_t)pl[1][xi] << 16);
        }
      } else {
#pragma unroll
        for (int xi = 0; xi < NX; ++xi) xp[xi] = xs[xi][h];
      }
      double sx = 0.0;  // this piece's x (every plane), then the group's over its 4 G/32 lanes
#pragma unroll
      for (int xi = 0; xi < NX; ++xi) {
        *(iron_u32x4*)&s_x[buf][xi][idx >> 5][(idx & 31) * 8] = xp[xi];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sx += (double)__uint_as_float(xp[xi][e] << 16);
          sx += (double)__uint_as_float(xp[xi][e] & 0xffff0000u);
        }
      }
      sx += dpp_d<0xb1>(sx);  // quad_perm [1,0,3,2]
      sx += dpp_d<0x4e>(sx);  // quad_perm [2,3,0,1]
      if (p.gshift >= 6) sx += dpp_d<0x141>(sx);  // row_half_mirror: the other quad of 8
      if (p.gshift >= 7) sx += dpp_d<0x140>(sx);  // row_mirror: the other 8 of 16
      const int kq = (idx & 31) * 8;
      if ((kq & gmask) == 0) s_corr[buf][kq >> p.gshift][idx >> 5] = (float)(-128.0 * sx);
    }
    if constexpr (SB == 16) *(iron_u32x4*)&s_s[buf][s_mi][s_row][s_byte] = ss4;
    else if constexpr (SB == 8) *(iron_u32x2*)&s_s[buf][s_mi][s_row][s_byte] = ss2;
    else *(uint32_t*)&s_s[buf][s_mi][s_row][s_byte] = ss1;
  };

  iron_u32x4 ring[kRDepth][RB][NM];
  auto wload = [&](iron_u32x4 (&st)[RB][NM], int j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) st[rb][mi] = *(const iron_u32x4*)(wp[rb][mi] + kRBlk * j);
  };

  double acc[RB][NM][4];
  f32x4 c[RB][NM];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mi = 0; mi < NM; ++mi) {
      c[rb][mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[rb][mi][i] = 0.0;
    }

  // Every block issues the same loads (past the split's end they re-read its last block), no load
  // sits in a branch, and scheduling barriers keep the loads in issue order: the wait before a
  // block's MFMAs then counts the later blocks' loads. (A branch around a load, or the scheduler
  // hoisting a later load above an earlier one, drops the compiler's wait to zero and drains the
  // ring every block.)
  if constexpr (NORM) {
    norm_issue();
    __builtin_amdgcn_sched_barrier(0);
  }
  xload(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kRDepth; ++u) {
    wload(ring[u], min(u, nb - 1));
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (NORM) norm_finish();
  xstore(0);
  __builtin_amdgcn_sched_barrier(0);
  xload(min(1, nc - 1));
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  for (int ch = 0; ch < nc; ++ch) {
    const int buf = ch & 1;
#pragma unroll
    for (int u = 0; u < kRDepth; ++u) {
      iron_u32x4 t[RB][NM];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) t[rb][mi] = quarter_transpose(ring[u][rb][mi]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // a 32-wide MFMA group at k kl of the chunk; quantization groups (G >= 32, dividing the
        // chunk) start and end on MFMA group boundaries
        const int kl = kRBlk * u + 32 * h;
        const bool gstart = G32 || (kl & gmask) == 0, gend = G32 || ((kl + 32) & gmask) == 0;
        bf16x8 bx[NX];
#pragma unroll
        for (int xi = 0; xi < NX; ++xi)
          bx[xi] = __builtin_bit_cast(bf16x8, *(const iron_u32x4*)&s_x[buf][xi][col][kl + quarter * 8]);
        f32x4 ci = {0.f, 0.f, 0.f, 0.f};
        if (gstart) ci = *(const f32x4*)&s_corr[buf][kl >> p.gshift][quarter * 4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) {
            const uint32_t lo = h ? t[rb][mi].z : t[rb][mi].x;
            const uint32_t hi = h ? t[rb][mi].w : t[rb][mi].y;
            const bf16x8 bw = u8_to_bf16u(lo ^ to_u, hi ^ to_u);
            if constexpr (G32) {
              c[rb][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bx[0], bw, ci, 0, 0, 0);
            } else {
              if (gstart) c[rb][mi] = ci;
              c[rb][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bx[0], bw, c[rb][mi], 0, 0, 0);
            }
#pragma unroll
            for (int xi = 1; xi < NX; ++xi)
              c[rb][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bx[xi], bw, c[rb][mi], 0, 0, 0);
          }
        if (gend) {  // the quantization group's sums, scaled, into the fp64 accumulators
          const int gl = kl >> p.gshift;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int mi = 0; mi < NM; ++mi) {
              const double sc = bf16_to_f32(
                  *(const uint16_t*)&s_s[buf][mi][wave * 16 * RB + 16 * rb + col][2 * gl]);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                acc[rb][mi][i] = fma(sc, (double)c[rb][mi][i], acc[rb][mi][i]);
                // fold here: left to itself the compiler sinks every group's fold to the end of
                // the chunk and keeps all the groups' sums live (registers spill)
                asm volatile("" : "+v"(acc[rb][mi][i]));
              }
            }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      wload(ring[u], min(ch * kRDepth + u + kRDepth, nb - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next chunk's x and scales into the other buffer (last read a chunk ago, before the
    // previous barrier), then the loads of the chunk after it
    xstore(buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    xload(min(ch + 2, nc - 1));
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  }

  if (p.splits == 1) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = quarter * 4 + i;
        if (b < p.B) store_out(p, b, row0 + 16 * rb + col, acc[rb][0][i], acc[rb][NM - 1][i]);
      }
    return;
  }
  // Split K: the fp64 partials go out write-through (16 consecutive rows per 128 bytes), then the
  // arrival count; the last split of the tile sums the partials in split order.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mi = 0; mi < NM; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = quarter * 4 + i;
        if (b < p.B)
          __hip_atomic_store(
              p.part + (((size_t)mi * p.splits + split) * kBN + b) * p.M + row0 + 16 * rb + col,
              acc[rb][mi][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  __shared__ unsigned int s_last;
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(p.ctr + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == (unsigned int)(p.splits - 1);
  __syncthreads();
  if (!s_last) return;
  // Every thread's outputs (b, m) = (t / TILE, t % TILE) for t = tid + NT o, and SQ splits of
  // each in one round of loads: the merge is a couple of memory round trips, not one per output
  // and eight splits.
  constexpr int PER = TILE * kBN / NT;   // outputs per thread at B = 16
  constexpr int SQ = 32 / (PER * NM);    // splits per round (32 loads in flight)
  static_assert(SQ >= 1, "merge round");
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      p.part, 0, NM * p.splits * kBN * p.M * (int)sizeof(double), kBufferDword3);
  int off[PER];
#pragma unroll
  for (int o = 0; o < PER; ++o) {
    const int t = min(tid + NT * o, TILE * p.B - 1);
    off[o] = ((t / TILE) * p.M + tile0 + t % TILE) * (int)sizeof(double);
  }
  const int sstride = kBN * p.M * (int)sizeof(double);  // one split's partials
  double a[PER][2] = {};
  for (int s0 = 0; s0 < p.splits; s0 += SQ) {
    double v[PER][NM][SQ];
#pragma unroll
    for (int q = 0; q < SQ; ++q) {
      const int spl = s0 + q < p.splits ? s0 + q : p.splits - 1;
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
#pragma unroll
        for (int o = 0; o < PER; ++o)
          v[o][mi][q] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(
              rs, off[o] + (mi * p.splits + spl) * sstride, 0, kCpolSc1));
    }
#pragma unroll
    for (int q = 0; q < SQ; ++q)
      if (s0 + q < p.splits) {
#pragma unroll
        for (int mi = 0; mi < NM; ++mi)
#pragma unroll
          for (int o = 0; o < PER; ++o) a[o][mi] += v[o][mi][q];
      }
  }
#pragma unroll
  for (int o = 0; o < PER; ++o) {
    const int t = tid + NT * o;
    if (t < TILE * p.B) store_out(p, t / TILE, tile0 + t % TILE, a[o][0], a[o][NM - 1]);
  }
  if (tid == 0)
    __hip_atomic_store(p.ctr + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemmPlan {
  bool rs;             // the register-streamed form (else the staged one)
  int splits, ksteps;  // split s covers steps [s*ksteps, (s+1)*ksteps): 128-wide (staged) or
                       // 256-wide chunks (register-streamed)
};

// Split K until at most 512 workgroups cover the chip (two per CU), keeping at least kMinSteps
// pipeline steps per split; the last split takes what is left (splits need not divide the steps).
// Measured per shape at B=16: 6144x4096 20.3 -> 17.0 us and 4096x12288 28.8 -> 24.4 us against
// one workgroup per CU; 2048x6144 (48 steps) best at 8 splits of 6 steps (16 splits of 3: 14.9
// against 13.1 us). Config 2 at B=8 (16- and 48-step GEMMs): 33.6 -> 32.3 us with kMinSteps 4 and
// uneven splits against 6 and even splits; config 5 8.82 -> 8.73 ms. Issuing all the
// loads of a split of at most 4 steps at its start measured slower (config 2 at B=8: 41.6 us; the
// gate/up kernel then needs 131 VGPRs, one workgroup per CU; for the single-matrix GEMMs alone
// 34.1 us).
constexpr int kSplitTarget = 512;
constexpr int kMinSteps = 4;
GemmPlan plan_staged(int M, int K) {
  const int tiles = M / kTM;
  const int steps = K / kKS;
  // at most the target: the 192 row tiles of Qwen3-8B's gate/up took 49.9 us at 2 splits (384
  // workgroups) against 51.4 us at 3 (576: more than two per CU)
  int splits = kSplitTarget / tiles;
  if (splits < 1) splits = 1;
  const int by_steps = steps / kMinSteps > 1 ? steps / kMinSteps : 1;
  if (splits > by_steps) splits = by_steps;
  // never fewer workgroups than one per CU would give (short K: 4096x1024 keeps 4 splits)
  const int per_cu = (256 + tiles - 1) / tiles;
  if (splits < per_cu) splits = per_cu;
  if (splits > steps) splits = steps;
  const int ksteps = (steps + splits - 1) / splits;
  return {false, (steps + ksteps - 1) / ksteps, ksteps};  // no empty split
}

// The register-streamed form: up to two 4-wavefront workgroups per CU (512), at least
// kRMinChunks chunks per split, and never fewer workgroups than CUs while a split can shrink.
constexpr int kRW = 8, kRRB = 1;         // wavefronts per workgroup, 16-row blocks per wavefront
constexpr int kRTile = 16 * kRW * kRRB;  // rows per workgroup
constexpr int kRMinChunks = 2;
GemmPlan plan_rs(int M, int K) {
  const int tiles = M / kRTile;
  const int chunks = K / kRChunk;
  int target = kSplitTarget / tiles;
  if (target < 1) target = 1;
  const int by_chunks = chunks / kRMinChunks > 1 ? chunks / kRMinChunks : 1;
  if (target > by_chunks) target = by_chunks;
  const int per_cu = (256 + tiles - 1) / tiles;
  if (target < per_cu) target = per_cu;
  if (target > chunks) target = chunks;
  int ksteps = (chunks + target - 1) / target;
  while (ksteps > 1 && tiles * ((chunks + ksteps - 1) / ksteps) < 256) --ksteps;
  return {true, (chunks + ksteps - 1) / ksteps, ksteps};
}

// The register-streamed form runs the dual (gate/up) GEMM of K >= 4096 (config 5's gate/up: 43.6
// against 50.1 us, the step 8.43 -> 8.20 ms); everywhere else the staged form measured as fast
// or faster (config 5 at B=16, us: down 28.4 against 25.1, QKV 14.3 against 13.8, Wo 14.3
// against 11.4; config 2 at B=8, whose 2048-deep gate/up splits to single chunks: 45.2 against
// 32.4 for the MLP).
GemmPlan plan_gemm(int M, int K, bool dual) {
  if (dual && K >= 4096 && M % kRTile == 0 && K % kRChunk == 0) return plan_rs(M, K);
  return plan_staged(M, K);
}

}  // namespace

namespace iron {

constexpr int kMaxTiles = (int)(kGemmCtrBytes / sizeof(unsigned int));  // M <= 262144

// Bytes of fp64 split-K partials (none without a split).
size_t gemm_workspace_bytes(int M, int K, bool dual) {
  const GemmPlan pl = plan_gemm(M, K, dual);
  if (pl.splits == 1) return 0;
  return (size_t)(dual ? 2 : 1) * pl.splits * kBN * M * sizeof(double);
}

// An upper bound over every K: the staged form's split count never exceeds
// ceil(kSplitTarget / (M / 64)), the register-streamed form's ceil(kSplitTarget / (M / 128)) or
// ceil(256 / (M / 128)), both at most ceil(2 kSplitTarget / (M / 64)).
size_t gemm_workspace_bound(int M, bool dual) {
  if (M <= 0 || M % kTM) return 0;
  const size_t splits = (2 * kSplitTarget + M / kTM - 1) / (M / kTM);
  return ((size_t)(dual ? 2 : 1) * splits * kBN * M * sizeof(double) + 255) & ~(size_t)255;
}

// Y = EPI(W0 [, W1] . x), B in [1, 16]; validation of M/K/G/B is the caller's (gemm_check).
int gemm_check(const char* fn, int B, int M, int K, int G) {
  if (B < 1 || B > kBN)
    return fail(IRON_ERR_UNSUPPORTED, "%s: MFMA batch %d outside [1, %d]", fn, B, kBN);
  if (M % kTM) return fail(IRON_ERR_UNSUPPORTED, "%s: M=%d not a multiple of %d", fn, M, kTM);
  if (M / kTM > kMaxTiles)
    return fail(IRON_ERR_UNSUPPORTED, "%s: M=%d above %d on the MFMA path", fn, M, kMaxTiles * kTM);
  if (K % kKS) return fail(IRON_ERR_UNSUPPORTED, "%s: K=%d not a multiple of %d", fn, K, kKS);
  if (G < 32 || G > kKS)
    return fail(IRON_ERR_UNSUPPORTED, "%s: group size %d outside [32, %d] on the MFMA path", fn,
                G, kKS);
  return IRON_OK;
}

bool gemm_resnorm_foldable(int D, int QD, int FF) {
  if (D <= 0 || QD <= 0 || FF <= 0 || D % kTM || D / kTM > 32 * 4 || QD % kKS) return false;
  const GemmPlan po = plan_gemm(D, QD, false), pg = plan_gemm(FF, D, true);
  return !po.rs && po.splits > 1 && pg.rs;
}

bool gemm_selfnorm_foldable(int B, int D, int FF) {
  // up to 8 batch rows: the planes' LDS then leaves room for two workgroups per CU (config 2:
  // B = 5 31.6 -> 30.6 us, B = 8 32.4 -> 31.9 us; at B = 16, one workgroup per CU, 37.7 -> 43.5)
  if (B < 1 || B > 8 || D <= 0 || FF <= 0 || D % kKS || FF % kTM) return false;
  const GemmPlan pg = plan_gemm(FF, D, true);
  return !pg.rs && pg.ksteps <= kNormSteps;
}

int gemm_w8_launch(const void* w0, const void* w1, int M, int K, int G, int tile_m, int domain,
                   const uint16_t* x, size_t x_plane, int B, int x_stride, int epi, void* y,
                   int y_stride, size_t y_plane, const uint16_t* r1, const uint16_t* r2,
                   int r_stride, unsigned int* ctr, void* part, size_t part_bytes,
                   hipStream_t stream, const char* fn, const GemmResNorm* rn) {
  int st = gemm_check(fn, B, M, K, G);
  if (st) return st;
  const bool dual = w1 != nullptr;
  const GemmPlan pl = plan_gemm(M, K, dual);
  // the folded residual RMSNorm: the producer (no a) splits K and has the bf16 epilogue; the
  // consumer is the register-streamed dual GEMM over the norm's D
  // consumer; without tile sums, the staged dual GEMM of at most kNormSteps steps per split sums
  // each batch row itself
  const bool rn_self = rn && !rn->ssq;
  const bool rn_prod = rn && rn->ssq && !rn->a, rn_cons = rn && rn->ssq && rn->a;
  if (rn && (!rn->cur || !aligned(rn->ssq, 8) ||
             (rn_prod && (pl.rs || pl.splits < 2 || epi != GEMM_EPI_BF16 || M != rn->D)) ||
             (rn_cons && (!pl.rs || !dual || !rn->w || K != rn->D || rn->D % kTM ||
                          rn->D / kTM > 32 * 4)) ||
             (rn_self && (pl.rs || pl.ksteps > kNormSteps || !dual || !rn->a || !rn->w ||
                          K != rn->D || !aligned(rn->cur, 16) || !aligned(rn->a, 16) ||
                          !aligned(rn->w, 16)))))
    return fail(IRON_ERR_UNSUPPORTED, "%s: the folded RMSNorm does not fit this GEMM plan", fn);
  GemmParams p = {};
  p.w0 = (const uint8_t*)w0;
  p.w1 = (const uint8_t*)w1;
  p.M = M;
  p.K = K;
  p.gshift = ilog2(G);
  p.tile_m = tile_m;
  p.tdiv = make_fastdiv((uint32_t)tile_m);
  p.blk_bytes = (uint32_t)wire_block_bytes(K, G, tile_m);
  p.xor_mask = domain == IRON_DOMAIN_BIASED ? 0x80808080u : 0u;
  p.x = x;
  p.x_plane = x_plane;
  const bool x_f32 = x_plane != 0;
  p.B = B;
  p.x_stride = x_stride;
  p.splits = pl.splits;
  p.ksteps = pl.ksteps;
  p.epi = epi;
  p.y = y;
  p.y_stride = y_stride;
  p.y_plane = y_plane;
  p.r1 = r1;
  p.r2 = r2;
  p.r_stride = r_stride;
  if (rn_prod) {
    p.ssq = rn->ssq;
    p.r1 = rn->cur;
    p.r_stride = rn->D;
  } else if (rn_cons || rn_self) {
    p.ssq = rn->ssq;
    p.r1 = rn->cur;
    p.r2 = rn->a;
    p.x_stride = rn->D;
    p.n_w = rn->w;
    p.n_tiles = rn->D / kTM;
    p.n_eps = rn->eps;
  }
  if (pl.splits > 1) {
    const size_t need = gemm_workspace_bytes(M, K, dual);
    if (!part || !ctr || part_bytes < need)
      return fail(IRON_ERR_WORKSPACE, "%s: MFMA partials %zu < %zu bytes", fn, part_bytes, need);
    if (!aligned(part, 256) || !aligned(ctr, 256))
      return fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
    p.part = (double*)part;
    p.ctr = ctr;
  }
  if (pl.rs) {
    dim3 grid(M / kRTile, pl.splits);
    const dim3 blk(64 * kRW);
    const bool g32 = G == 32;
#define IRON_RS(D_, X_)                                                                      \
  do {                                                                                       \
    if (g32) hipLaunchKernelGGL((gemm_w8_rs_kernel<D_, X_, kRW, kRRB, true>), grid, blk, 0,  \
                                stream, p);                                                  \
    else hipLaunchKernelGGL((gemm_w8_rs_kernel<D_, X_, kRW, kRRB, false>), grid, blk, 0,     \
                            stream, p);                                                      \
  } while (0)
    if (rn_cons) {
      if (g32) hipLaunchKernelGGL((gemm_w8_rs_kernel<true, true, kRW, kRRB, true, true>), grid,
                                  blk, 0, stream, p);
      else hipLaunchKernelGGL((gemm_w8_rs_kernel<true, true, kRW, kRRB, false, true>), grid, blk,
                              0, stream, p);
    } else if (dual) {
      if (x_f32) IRON_RS(true, true);
      else IRON_RS(true, false);
    } else {
      if (x_f32) IRON_RS(false, true);
      else IRON_RS(false, false);
    }
#undef IRON_RS
    return check_launch(fn);
  }
  dim3 grid(M / kTM, pl.splits);
  if (rn_self) {
    hipLaunchKernelGGL((gemm_w8_mfma_kernel<true, true, true>), grid, dim3(512),
                       (size_t)3 * B * kHRow * sizeof(uint16_t), stream, p);
  } else if (dual) {
    if (x_f32) hipLaunchKernelGGL((gemm_w8_mfma_kernel<true, true>), grid, dim3(512), 0, stream, p);
    else hipLaunchKernelGGL((gemm_w8_mfma_kernel<true, false>), grid, dim3(512), 0, stream, p);
  } else {
    if (x_f32) hipLaunchKernelGGL((gemm_w8_mfma_kernel<false, true>), grid, dim3(512), 0, stream, p);
    else hipLaunchKernelGGL((gemm_w8_mfma_kernel<false, false>), grid, dim3(512), 0, stream, p);
  }
  return check_launch(fn);
}

}  // namespace iron

extern "C" {

size_t iron_gemm_w8a16_workspace(int B, int M, int K, int G) {
  (void)B;
  (void)G;
  if (M <= 0 || K <= 0 || M % kTM || K % kKS) return 0;
  const size_t n = iron::gemm_workspace_bytes(M, K, false);
  return n ? iron::kGemmCtrBytes + n : 256;
}

int iron_gemm_w8a16(const void* wire, const uint16_t* x, uint16_t* y, int B, int M, int K, int G,
                    int tile_m, int domain, void* workspace, size_t workspace_bytes,
                    void* stream) {
  iron::clear_error();
  const char* fn = "iron_gemm_w8a16";
  if (!x || !y) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  int st = iron::check_wire(fn, wire, M, K, G, tile_m, domain);
  if (st) return st;
  if (!iron::aligned(x, 16)) return iron::fail(IRON_ERR_ALIGN, "%s: x not 16-byte aligned", fn);
  const size_t ctr = workspace_bytes >= iron::kGemmCtrBytes ? iron::kGemmCtrBytes : 0;
  return iron::gemm_w8_launch(wire, nullptr, M, K, G, tile_m, domain, x, 0, B, K,
                              iron::GEMM_EPI_BF16, y, M, 0, nullptr, nullptr, 0,
                              (unsigned int*)workspace, workspace ? (char*)workspace + ctr : nullptr,
                              workspace_bytes - ctr, (hipStream_t)stream, fn);
}

}  // extern "C"
