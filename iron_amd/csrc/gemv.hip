// Weight-streaming GEMV kernels for batch-1..15 decode on gfx950 (the fused QKV head and MLP use
// batches 1..4; 5..15 reach the batched kernel through iron_gemv_w8a16).
//
// Reference path: the int8 W8A16 matvec (aie_kernels/aie2p/mv_int8_signed.cc:60-113, biased
// form mv_int8.cc:60-115) behind GEMVInt8 (iron/operators/gemv_int8/op.py:20-178), the fused
// QKV GEMV (qkv_head_dp), the gate/up/down GEMVs of the fused SwiGLU MLP (swiglu_mlp_dp) and the
// LM head (iron/applications/qwen3_0.6b/qwen3_npu_int8.py:242-246).
//
// Weight wire (the reference's own packing, gemv_int8/reference.py:59-80): consecutive
// row-blocks of `tile_m` rows, each block = tile_m*K int8 payload (row-major) followed by
// tile_m*(K/G) bf16 group scales (row-major). The payload domain is signed two's-complement q or
// biased q+128; both carry the same integer q.
//
// Arithmetic: the exact value of the reference golden GEMVInt8.reference (gemv_int8/op.py:
// 173-178), y[b][m] = sum_g s[m][g] * sum_{k in g} q[m][k] * x[b][k], accumulated in fp64 (every
// product q*x is exact in fp64 and so is the accumulation to within 2^-53), then one rounding to
// the output type. Non-packed fp64 FMA issues at the fp32 FMA rate on CDNA4, so exactness costs
// one extra convert per weight, and it makes the device result equal the correctly rounded
// value the fp64 oracle computes, not merely close to it.
//
// Mapping: 256-thread workgroups (4 wavefronts); each wavefront owns R consecutive rows and each
// lane one 16-byte slice of every 1024-wide (int8) or 512-wide (bf16) chunk of those rows, so a
// wavefront load instruction reads 1 KiB of one row. A workgroup owns one group of 4*R rows: it
// first issues every weight/scale load of the group (R*NCH 128-bit loads per lane, all in
// flight) behind the activation loads, then stages x into LDS (the prologue, overlapping the
// weight latency), then reduces. A batch whose rows do not all fit in LDS at once (long rows)
// runs as batch groups, one workgroup per row group and batch group (gemv_kernel, MULTI).
#include <type_traits>

#include "common.h"
#include "gemv_core.h"
#include "internal.h"

namespace {

using namespace iron::dev;

// ------------------------------------------------------------------------------------------
// Prologue: stage B vectors of length K into LDS as fp32 (K % 8 == 0, 16-byte aligned rows).
// Every staged value is an exact fp32: a bf16 activation, an fp32 one, or the fp32 (or bf16)
// rounding of the RMSNorm output, so the dot products see the same numbers as from fp64 staging
// in half the LDS (a 4 x 6144 batch fits).
//
// LDS layout: lane-contiguous quads. A lane of the dot product consumes J consecutive quads
// x[4Q .. 4Q+3] per chunk (J = 4 for int8 chunks of 1024, 2 for bf16 chunks of 512); quad Q
// lives at slot (c*J + j)*64 + lane with c = Q / (64*J), lane = (Q % (64*J)) / J, j = Q % J, so
// one ds_read_b128 of a wavefront reads 64 consecutive 16-byte slots (no bank conflicts). A
// vector occupies ceil(K / chunk) * chunk floats.
// ------------------------------------------------------------------------------------------
template <bool INT8>
IRON_DEV int quad_slot(int Q) {
  constexpr int J = INT8 ? 4 : 2;
  constexpr int QC = 64 * J;  // quads per chunk
  const int c = Q / QC, rem = Q % QC;
  return (c * J + (rem % J)) * 64 + rem / J;
}

template <bool INT8>
IRON_DEV int padded_k(int K) {
  constexpr int chunk = INT8 ? 1024 : 512;
  return (K + chunk - 1) / chunk * chunk;
}

// thread t's 8 elements x[8t..8t+7] are quads 2t, 2t+1
template <bool INT8>
IRON_DEV void put8(float4* dst, int i, const float (&v)[8]) {
  dst[quad_slot<INT8>(2 * i)] = make_float4(v[0], v[1], v[2], v[3]);
  dst[quad_slot<INT8>(2 * i + 1)] = make_float4(v[4], v[5], v[6], v[7]);
}

// The activation side is loaded into registers before the weight loads are issued: loads
// complete in issue order, so the prologue (and its block reduction) then runs while the weight
// stream is still in flight. Each thread owns up to S 8-element slots per batch row
// (i = threadIdx.x + 256*r); slots beyond S (K > 2048*S) are loaded in the compute pass.
//   xa: bf16 x, or the low half of fp32 x;  xb: the high half of fp32 x (PRO_F32) or the
//   residual term x2 (PRO_RES_RMS_F32);  xn: the RMSNorm weight.
template <int B>
constexpr int x_slots() { return B == 1 ? 4 : (B == 2 ? 2 : 1); }

template <int B, int S>
IRON_DEV void load_x(const GemvParams& p, uint4 (&xa)[B][S], uint4 (&xb)[B][S], uint4 (&xn)[S]) {
  const int n8 = p.K >> 3;
  const bool rms = p.pro == PRO_RMS_BF16 || p.pro == PRO_RES_RMS_F32;
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int r = 0; r < S; ++r) {
      const int i = threadIdx.x + 256 * r;
      xa[b][r] = make_uint4(0u, 0u, 0u, 0u);
      xb[b][r] = make_uint4(0u, 0u, 0u, 0u);
      if (i < n8 && b < p.nb) {
        if (p.pro == PRO_F32) {
          const uint4* src = (const uint4*)((const float*)p.x + (size_t)b * p.x_stride);
          xa[b][r] = src[2 * i];
          xb[b][r] = src[2 * i + 1];
        } else {
          xa[b][r] = ((const uint4*)((const uint16_t*)p.x + (size_t)b * p.x_stride))[i];
          if (p.x2) xb[b][r] = ((const uint4*)(p.x2 + (size_t)b * p.x2_stride))[i];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < S; ++r) {
    const int i = threadIdx.x + 256 * r;
    xn[r] = make_uint4(0u, 0u, 0u, 0u);
    if (rms && i < n8) xn[r] = ((const uint4*)p.nw)[i];
  }
}

// Rows b >= p.nb are not staged (their LDS rows keep older values; their results are not stored).
template <int B, int S, bool INT8>
IRON_DEV void stage_x(const GemvParams& p, const uint4 (&xa)[B][S], const uint4 (&xb)[B][S],
                      const uint4 (&xn)[S], float* __restrict__ xs, double* red) {
  const int K = p.K;
  const int n8 = K >> 3;
  const int KP = padded_k<INT8>(K);
  const int tid = threadIdx.x;
#pragma unroll
  for (int b = 0; b < B; ++b) {
    if (b >= p.nb) break;  // workgroup-uniform
    float4* dst = (float4*)(xs + (size_t)b * KP);
    if (p.pro == PRO_F32) {
      const uint4* src = (const uint4*)((const float*)p.x + (size_t)b * p.x_stride);
#pragma unroll
      for (int r = 0; r < S; ++r) {
        const int i = tid + 256 * r;
        if (i < n8) {
          const uint4 lo = xa[b][r], hi = xb[b][r];
          const float v[8] = {__uint_as_float(lo.x), __uint_as_float(lo.y), __uint_as_float(lo.z),
                              __uint_as_float(lo.w), __uint_as_float(hi.x), __uint_as_float(hi.y),
                              __uint_as_float(hi.z), __uint_as_float(hi.w)};
          put8<INT8>(dst, i, v);
        }
      }
      for (int i = tid + 256 * S; i < n8; i += 256) {
        const uint4 lo = src[2 * i], hi = src[2 * i + 1];
        const float v[8] = {__uint_as_float(lo.x), __uint_as_float(lo.y), __uint_as_float(lo.z),
                            __uint_as_float(lo.w), __uint_as_float(hi.x), __uint_as_float(hi.y),
                            __uint_as_float(hi.z), __uint_as_float(hi.w)};
        put8<INT8>(dst, i, v);
      }
      continue;
    }
    const uint4* src = (const uint4*)((const uint16_t*)p.x + (size_t)b * p.x_stride);
    if (p.pro == PRO_BF16) {
#pragma unroll
      for (int r = 0; r < S; ++r) {
        const int i = tid + 256 * r;
        if (i < n8) {
          float f[8];
          unpack8(xa[b][r], f);
          put8<INT8>(dst, i, f);
        }
      }
      for (int i = tid + 256 * S; i < n8; i += 256) {
        float f[8];
        unpack8(src[i], f);
        put8<INT8>(dst, i, f);
      }
      continue;
    }
    // RMS prologues
    const bool has_x2 = p.x2 != nullptr;
    const uint4* src2 = (const uint4*)(p.x2 + (size_t)b * p.x2_stride);
    const uint4* wsrc = (const uint4*)p.nw;
    double ss = 0.0;
#pragma unroll
    for (int r = 0; r < S; ++r) {
      if (tid + 256 * r < n8) {
        float f[8];
        slot_values(xa[b][r], xb[b][r], has_x2, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
      }
    }
    for (int i = tid + 256 * S; i < n8; i += 256) {
      float f[8];
      slot_values(src[i], has_x2 ? src2[i] : make_uint4(0u, 0u, 0u, 0u), has_x2, f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
    }
    ss = block_sum_256_d(ss, red);
    const double inv = inv_rms(ss, K, (double)p.eps);
    const bool to_bf16 = p.pro == PRO_RMS_BF16;
#pragma unroll
    for (int r = 0; r < S + 1; ++r) {
      // r < S: register slots; r == S: the remaining slots, loaded here
      for (int i = tid + 256 * r; i < n8; i += (r < S ? n8 : 256)) {
        float f[8], wf[8];
        if (r < S) {
          slot_values(xa[b][r], xb[b][r], has_x2, f);
          unpack8(xn[r], wf);
        } else {
          slot_values(src[i], has_x2 ? src2[i] : make_uint4(0u, 0u, 0u, 0u), has_x2, f);
          unpack8(wsrc[i], wf);
        }
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const double y = ((double)f[j] * inv) * (double)wf[j];
          v[j] = to_bf16 ? round_bf16((float)y) : (float)y;
        }
        put8<INT8>(dst, i, v);
      }
    }
  }
  __syncthreads();
}

template <int B, int R, int NCH>
IRON_DEV void dot_w8(const GemvParams& p, const uint4 (&w)[R][NCH], const uint32_t (&sc)[R][NCH],
                     const float* __restrict__ xs, int row0, int lane, double (&acc)[R][B]) {
  const int K = p.K;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = 0.0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 1024 + lane * 16;
    if (c * 1024 >= K) break;
    double xv[B][16];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (e < K) {
        // quads (c*4 + j)*64 + lane, j = 0..3 (the lane-contiguous staging layout)
        const float4* src = (const float4*)(xs + (size_t)b * padded_k<true>(K)) + c * 256 + lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 t = src[j * 64];
          xv[b][4 * j] = t.x;
          xv[b][4 * j + 1] = t.y;
          xv[b][4 * j + 2] = t.z;
          xv[b][4 * j + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) xv[b][j] = 0.0;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd[4] = {w[r][c].x ^ p.xor_mask, w[r][c].y ^ p.xor_mask,
                              w[r][c].z ^ p.xor_mask, w[r][c].w ^ p.xor_mask};
      const double s = slice_scale(p, sc[r][c], row0 + r, e);
#pragma unroll
      for (int b = 0; b < B; ++b) {
        double pa = 0.0, pb = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pa = fma(sbyte(dd[j], 0), xv[b][4 * j + 0], pa);
          pb = fma(sbyte(dd[j], 1), xv[b][4 * j + 1], pb);
          pa = fma(sbyte(dd[j], 2), xv[b][4 * j + 2], pa);
          pb = fma(sbyte(dd[j], 3), xv[b][4 * j + 3], pb);
        }
        acc[r][b] = fma(s, pa + pb, acc[r][b]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = wave_sum_d(acc[r][b]);
}

// bf16 row-major weights: lane slices of 8 bf16 per 512-wide chunk.
template <int R, int NCH>
IRON_DEV void fetch_w16(const GemvParams& p, int row0, int lane, uint4 (&w)[R][NCH]) {
  const uint16_t* W = (const uint16_t*)p.w;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int e = c * 512 + lane * 8;
      // clamped address; an out-of-range row is never stored and x is 0 past K
      w[r][c] = *(const uint4*)(W + (size_t)(row < p.M ? row : 0) * p.K + (e < p.K ? e : 0));
    }
  }
}

template <int B, int R, int NCH>
IRON_DEV void dot_w16(const GemvParams& p, const uint4 (&w)[R][NCH],
                      const float* __restrict__ xs, int lane, double (&acc)[R][B]) {
  const int K = p.K;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = 0.0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = c * 512 + lane * 8;
    if (c * 512 >= K) break;
    double xv[B][8];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (e < K) {
        // quads (c*2 + j)*64 + lane, j = 0..1
        const float4* src = (const float4*)(xs + (size_t)b * padded_k<false>(K)) + c * 128 + lane;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float4 t = src[j * 64];
          xv[b][4 * j] = t.x;
          xv[b][4 * j + 1] = t.y;
          xv[b][4 * j + 2] = t.z;
          xv[b][4 * j + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[b][j] = 0.0;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd[4] = {w[r][c].x, w[r][c].y, w[r][c].z, w[r][c].w};
#pragma unroll
      for (int b = 0; b < B; ++b) {
        double pa = 0.0, pb = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pa = fma((double)bf16lo_to_f32(dd[j]), xv[b][2 * j], pa);
          pb = fma((double)bf16hi_to_f32(dd[j]), xv[b][2 * j + 1], pb);
        }
        acc[r][b] += pa + pb;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[r][b] = wave_sum_d(acc[r][b]);
}

template <int R, int NCH>
IRON_DEV void dot_w16_lane(const uint4 (&w)[R][NCH], const float (&xf)[NCH][8],
                           double (&acc)[R][1]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r][0] = 0.0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    double xv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = xf[c][j];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd[4] = {w[r][c].x, w[r][c].y, w[r][c].z, w[r][c].w};
      double pa = 0.0, pb = 0.0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa = fma((double)bf16lo_to_f32(dd[j]), xv[2 * j], pa);
        pb = fma((double)bf16hi_to_f32(dd[j]), xv[2 * j + 1], pb);
      }
      acc[r][0] += pa + pb;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r][0] = wave_sum_d(acc[r][0]);
}

template <int B, int R>
IRON_DEV void store_rows(const GemvParams& p, int row0, int lane, const double (&acc)[R][B],
                         const double (&acc2)[R][B], unsigned long long (&best)[B]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    if (row >= p.M) continue;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (b >= p.nb) break;  // rows past the batch (a partial group)
      const double v = acc[r][b];
      const size_t o = (size_t)b * p.y_stride + row;
      if (p.epi == EPI_BF16_ARGMAX) {
        const uint16_t h = f64_to_bf16(v);
        const unsigned long long key =
            ((unsigned long long)bf16_order_key(h) << 32) | (unsigned long long)(~(uint32_t)row);
        best[b] = key > best[b] ? key : best[b];
        if (lane == r * B + b) ((uint16_t*)p.y)[o] = h;
      } else if (lane == r * B + b) {
        if (p.epi == EPI_BF16) {
          ((uint16_t*)p.y)[o] = f64_to_bf16(v);
        } else if (p.epi == EPI_F32) {
          ((float*)p.y)[o] = (float)v;
        } else if (p.epi == EPI_RES_BF16) {
          const size_t ro = (size_t)b * p.r_stride + row;
          float x1 = bf16_to_f32(p.r1[ro]);
          if (p.r2) x1 = x1 + bf16_to_f32(p.r2[ro]);
          ((uint16_t*)p.y)[o] = f64_to_bf16((double)x1 + v);
        } else {  // EPI_SWIGLU_F32
          ((float*)p.y)[o] = (float)silu_mul(v, acc2[r][b]);
        }
      }
    }
  }
}

// Batch 1 with at most two chunks per lane keeps the activation in registers (longer rows
// stage it once per workgroup in LDS: every wavefront loading the whole vector costs more).
constexpr bool xreg_path(int B, int NCH) { return B == 1 && NCH <= 2; }

// The parameters of batch rows [b0, b0 + B) of a launch over p.nb rows: operands advanced by b0
// rows, nb the rows of the group that exist.
template <int B>
IRON_DEV GemvParams batch_group(const GemvParams& p, int b0) {
  GemvParams q = p;
  if (b0 == 0) {
    q.nb = p.nb < B ? p.nb : B;
    return q;
  }
  q.nb = p.nb - b0 < B ? p.nb - b0 : B;
  if (p.pro == PRO_F32) q.x = (const float*)p.x + (size_t)b0 * p.x_stride;
  else q.x = (const uint16_t*)p.x + (size_t)b0 * p.x_stride;
  if (p.x2) q.x2 = p.x2 + (size_t)b0 * p.x2_stride;
  if (p.epi == EPI_F32 || p.epi == EPI_SWIGLU_F32) q.y = (float*)p.y + (size_t)b0 * p.y_stride;
  else q.y = (uint16_t*)p.y + (size_t)b0 * p.y_stride;
  if (p.r1) q.r1 = p.r1 + (size_t)b0 * p.r_stride;
  if (p.r2) q.r2 = p.r2 + (size_t)b0 * p.r_stride;
  if (p.argmax) q.argmax = p.argmax + b0;
  return q;
}

// One candidate per workgroup and batch row; an atomic only when it beats the value already
// published (a stale read costs at most a redundant atomicMax, never a wrong result). Resets best.
template <int B>
IRON_DEV void publish_argmax(const GemvParams& p, int wave, int lane,
                             unsigned long long (&best)[B], unsigned long long (*s_best)[4]) {
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < B; ++b) s_best[wave][b] = best[b];
  }
  __syncthreads();
  if (threadIdx.x < B && (int)threadIdx.x < p.nb) {
    const int b = threadIdx.x;
    unsigned long long k = s_best[0][b];
    for (int i = 1; i < 4; ++i) k = s_best[i][b] > k ? s_best[i][b] : k;
    const unsigned long long cur =
        __hip_atomic_load(p.argmax + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k > cur) atomicMax(p.argmax + b, k);
  }
  __syncthreads();  // s_best is read before a later group rewrites it
#pragma unroll
  for (int b = 0; b < B; ++b) best[b] = 0ull;
}

// IT: row blocks per workgroup (register-activation path only). A workgroup then streams IT
// consecutive blocks of 4R rows: fewer, longer workgroups read HBM faster (a 311 MB bf16 LM head:
// 5.7 TB/s with one block, 6.3 TB/s with four, measured with the same access pattern).
// p.nb batch rows: at most B, or with MULTI p.n_bgroups groups of B rows, one workgroup per
// (row group, batch group). The workgroups of one octet of row groups and one batch group are 8
// consecutive workgroups, the octet's batch groups follow each other: a workgroup w sits on XCD
// w % 8 (the dispatcher's round robin), so the batch groups of a row group run on one XCD at the
// same time and their reads of its weights meet in that XCD's L2 (HBM streams each weight once).
template <int B, int R, int NCH, bool INT8, bool DUAL, int IT = 1, bool MULTI = false>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
  extern __shared__ float xs[];
  __shared__ double red[4];
  __shared__ unsigned long long s_best[4][4];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  static_assert(IT == 1 || xreg_path(B, NCH), "row-block loop on the register path only");
  static_assert(!MULTI || !xreg_path(B, NCH), "batch groups on the LDS path only");
  int blk = blockIdx.x;
  if constexpr (MULTI) {
    const int ng = p.n_bgroups;
    const int bg = (blk / 8) % ng;
    blk = (blk / (8 * ng)) * 8 + blk % 8;
    if (blk * 4 * R >= p.M) return;  // the last octet's padding (workgroup-uniform)
    p = batch_group<B>(p, bg * B);
  }
  int row0 = (blk * IT * 4 + wave) * R;

  uint4 w[R][NCH];
  uint32_t sc[R][NCH];
  uint4 w2[DUAL ? R : 1][DUAL ? NCH : 1];
  uint32_t sc2[DUAL ? R : 1][DUAL ? NCH : 1];
  auto fetch_weights = [&]() {
    if constexpr (INT8) {
      fetch_w8<R, NCH>(p, p.w, row0, lane, w, sc);
      if constexpr (DUAL) fetch_w8<R, NCH>(p, p.w2, row0, lane, w2, sc2);
    } else {
      fetch_w16<R, NCH>(p, row0, lane, w);
    }
  };
  double acc[R][B], acc2[R][B];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < B; ++b) acc2[r][b] = 0.0;
  unsigned long long best[B];
#pragma unroll
  for (int b = 0; b < B; ++b) best[b] = 0ull;

  if constexpr (xreg_path(B, NCH)) {
    // 1. this lane's activation elements, then the weights; 2. the prologue in registers
    constexpr int EPL = INT8 ? 16 : 8;
    uint4 xl[NCH][EPL / 4], x2l[NCH][EPL / 8], nwl[NCH][EPL / 8];
    load_x_lane<NCH, EPL>(p, lane, xl, x2l, nwl);
    fetch_weights();
    float xf[NCH][EPL];
    prologue_lane<NCH, EPL>(p, lane, xl, x2l, nwl, xf);
    for (int it = 0; it < IT; ++it) {
      // 3. reduce
      if constexpr (INT8) {
        dot_w8_lane<R, NCH>(p, w, sc, xf, row0, lane, acc);
        if constexpr (DUAL) dot_w8_lane<R, NCH>(p, w2, sc2, xf, row0, lane, acc2);
      } else {
        dot_w16_lane<R, NCH>(w, xf, acc);
      }
      if (row0 < p.M) store_rows<B, R>(p, row0, lane, acc, acc2, best);
      if (it + 1 < IT) {
        row0 += 4 * R;
        fetch_weights();
      }
    }
    if (p.epi == EPI_BF16_ARGMAX) publish_argmax<B>(p, wave, lane, best, s_best);
  } else {
    // 1. the activation side first, then every weight load of this wavefront's rows
    constexpr int S = x_slots<B>();
    uint4 xa[B][S], xb[B][S], xn[S];
    load_x<B, S>(p, xa, xb, xn);
    fetch_weights();
    // 2. the prologue runs while the weights are in flight
    stage_x<B, S, INT8>(p, xa, xb, xn, xs, red);
    // 3. reduce
    if constexpr (INT8) {
      dot_w8<B, R, NCH>(p, w, sc, xs, row0, lane, acc);
      if constexpr (DUAL) dot_w8<B, R, NCH>(p, w2, sc2, xs, row0, lane, acc2);
    } else {
      dot_w16<B, R, NCH>(p, w, xs, lane, acc);
    }
    if (row0 < p.M) store_rows<B, R>(p, row0, lane, acc, acc2, best);
    if (p.epi == EPI_BF16_ARGMAX) publish_argmax<B>(p, wave, lane, best, s_best);
  }
}

// ------------------------------------------------------------------------------------------
// Batched GEMV (batches 5..15, int8 weights): the weights are streamed and converted once per
// workgroup and multiplied with every batch row, where the batch-group form re-reads and
// re-converts them per group of four rows.
//
// Mapping: wavefront w of workgroup blk owns rows (4 blk + w) R ..; K runs in chunks of kBKC = 512
// elements, lane l taking elements [c + 8 l, +8) of every row (one 8-byte load per row and chunk,
// eight weights inside one scale group since G >= 16). Every weight load of the wavefront's rows
// is issued at the start (all chunks in flight at once: with one chunk ahead the kernel ran at a
// tenth of the bandwidth). Per chunk the workgroup stages the nb activation rows of the chunk in
// LDS as fp64 (exact: bf16 / fp32 values, or the fp32 / bf16 rounding of the RMSNorm prologue),
// loaded one chunk ahead; each lane converts its weights once, q s (exact in fp64: an 8-bit by
// 8-bit significand product), and runs nb fp64 FMA chains over them. The per-lane partial sums of
// every (row, batch) output are added over the 64 lanes through LDS at the end.
//
// Arithmetic: sum_k (q_k s_g) x_k in fp64 -- every term exact, the accumulation within 2^-53 --
// then the output rounding of the single-row kernels (the same correctly rounded values).
// ------------------------------------------------------------------------------------------
constexpr int kBKC = 512;   // K elements per chunk
constexpr int kRedRow = 66;  // doubles between the LDS rows of the final lane reduction

// Rows per wavefront for NB batch rows and NCK chunks held in registers: 2 or 1, whichever keeps
// the weight registers (two per 8-byte slice, one per scale) within 96 and the fp64 accumulators
// within 64 registers; 0 when neither does or the variant spilled to scratch when compiled (NB = 16
// beyond 8 chunks): the batch-group kernel runs instead.
template <int NB, bool DUAL, int NCK>
constexpr int batch_rows() {
  constexpr int m = DUAL ? 2 : 1;
  if (NCK > (NB == 16 ? 8 : 16)) return 0;
  return (NCK * 2 * m * 3 <= 96 && 2 * NB * m * 2 <= 64) ? 2
         : (NCK * m * 3 <= 96 && NB * m * 2 <= 64)     ? 1
                                                        : 0;
}

template <int NB, bool DUAL, int NCK>
constexpr int batch_lds_doubles() {
  constexpr int R = batch_rows<NB, DUAL, NCK>();
  constexpr int xs = NB * kBKC, red = 4 * R * NB * kRedRow;
  return xs > red ? xs : red;
}

// inv[b] = 1 / RMS of batch row b's prologue input (x, or f32(x + x2)), for the RMS prologues:
// wavefront w reduces rows b = w, w + 4, ... over all of K.
IRON_DEV void batch_inv_rms(const GemvParams& p, double* s_inv) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n8 = p.K >> 3;
  for (int b = wave; b < p.nb; b += 4) {
    const uint4* src = (const uint4*)((const uint16_t*)p.x + (size_t)b * p.x_stride);
    const uint4* src2 = p.x2 ? (const uint4*)(p.x2 + (size_t)b * p.x2_stride) : nullptr;
    double ss = 0.0;
    for (int i = lane; i < n8; i += 64) {
      float f[8];
      slot_values(src[i], src2 ? src2[i] : make_uint4(0u, 0u, 0u, 0u), src2 != nullptr, f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fma((double)f[j], (double)f[j], ss);
    }
    ss = wave_sum_d(ss);
    if (lane == 0) s_inv[b] = inv_rms(ss, p.K, (double)p.eps);
  }
}

// The activation slots of one chunk that thread t stages: slot t + 256 k (k < NB / 4) is row
// b = slot / 64, elements [c0 + 8 (slot % 64), +8). Loaded a chunk ahead (batch_load), widened
// and normalised into LDS when the chunk starts (batch_store)
// (native vector types: a struct of HIP uint4 arrays is not split into registers, and lands in
// scratch memory)
template <int NB>
struct XSlots {
  iron_u32x4 a[NB / 4], b[NB / 4], n[NB / 4];  // x (bf16, or fp32 low half), x2 / fp32 high half, w
};

IRON_DEV iron_u32x4 ld16(const void* p) { return *(const iron_u32x4*)p; }
IRON_DEV uint4 as_uint4(iron_u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

template <int NB>
IRON_DEV void batch_load(const GemvParams& p, int c0, XSlots<NB>& xr) {
  constexpr int P8 = kBKC / 8;  // 8-element slots per row and chunk
  const bool rms = p.pro == PRO_RMS_BF16 || p.pro == PRO_RES_RMS_F32;
  const iron_u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < NB / 4; ++k) {
    const int t = threadIdx.x + 256 * k, b = t / P8, e = c0 + 8 * (t % P8);
    iron_u32x4 va = zero, vb = zero, vn = zero;
    if (b < p.nb && e < p.K) {
      if (p.pro == PRO_F32) {
        const float* src = (const float*)p.x + (size_t)b * p.x_stride + e;
        va = ld16(src);
        vb = ld16(src + 4);
      } else {
        va = ld16((const uint16_t*)p.x + (size_t)b * p.x_stride + e);
        if (p.x2) vb = ld16(p.x2 + (size_t)b * p.x2_stride + e);
        if (rms) vn = ld16(p.nw + e);
      }
    }
    xr.a[k] = va;
    xr.b[k] = vb;
    xr.n[k] = vn;
  }
}

// xs[b][e] (fp64) for the chunk's slots: the values stage_x puts in LDS, widened; zeros at or
// past K. Rows past nb are not written (never read).
template <int NB>
IRON_DEV void batch_store(const GemvParams& p, const XSlots<NB>& xr, const double* s_inv,
                          double* xs) {
  constexpr int P8 = kBKC / 8;
  const bool rms = p.pro == PRO_RMS_BF16 || p.pro == PRO_RES_RMS_F32;
#pragma unroll
  for (int k = 0; k < NB / 4; ++k) {
    const int t = threadIdx.x + 256 * k, b = t / P8, i = t % P8;
    if (b < p.nb) {
      double v[8];
      if (p.pro == PRO_F32) {
        const uint32_t u[8] = {xr.a[k].x, xr.a[k].y, xr.a[k].z, xr.a[k].w,
                               xr.b[k].x, xr.b[k].y, xr.b[k].z, xr.b[k].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(u[j]);
      } else {
        float f[8];
        slot_values(as_uint4(xr.a[k]), as_uint4(xr.b[k]), p.x2 != nullptr, f);
        if (rms) {
          float wf[8];
          unpack8(as_uint4(xr.n[k]), wf);
          const double inv = s_inv[b];
          const bool to_bf16 = p.pro == PRO_RMS_BF16;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const double y = ((double)f[j] * inv) * (double)wf[j];
            v[j] = to_bf16 ? round_bf16((float)y) : (float)y;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = f[j];
        }
      }
      // piece j of slot i (elements 8 i + 2 j, +1) at double2 j * 64 + i: a wavefront's access
      // to piece j covers 64 consecutive 16-byte slots (no bank conflicts; contiguous slots per
      // lane measured 14.7 M conflict cycles per launch of the Qwen3-1.7B gate/up at batch 8)
      double2* d = (double2*)(xs + (size_t)b * kBKC);
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j * 64 + i] = make_double2(v[2 * j], v[2 * j + 1]);
    }
  }
}

// Row r's 8-byte weight slice at element e of a chunk and its group scale (clamped addresses;
// rows past M and elements past K are masked through a zero scale).
template <int R>
IRON_DEV void batch_fetch(const GemvParams& p, const uint8_t* __restrict__ wire, int row0, int e,
                          uint2 (&w)[R], uint32_t (&sc)[R]) {
  const int K = p.K, ng = K >> p.gshift;
  const int ec = e < K ? e : 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    const uint32_t rr = row < p.M ? (uint32_t)row : 0u;
    const uint32_t blk = fastdiv(rr, p.tdiv);
    const uint32_t in = rr - blk * (uint32_t)p.tile_m;
    const uint8_t* base = wire + (size_t)blk * p.blk_bytes;
    w[r] = ld_global((const uint2*)(base + (size_t)in * K + ec));
    sc[r] = ld_global((const uint16_t*)(base + (size_t)p.tile_m * K) + (size_t)in * ng +
                      (ec >> p.gshift));
  }
}

// acc[r][b] += sum_j (q_j s) x[b][e + j] over this lane's 8 elements of the staged chunk, for the
// M matrices of the call (two for gate/up, which then read each activation slice once).
template <int NB, int R, int M>
IRON_DEV void batch_fma(const GemvParams& p, const uint2 (&w)[M][R], const uint32_t (&sc)[M][R],
                        int row0, int e, const double* xs, int lane, double (&acc)[M][R][NB]) {
  double wf[M][R][8];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const double s = slice_scale(p, sc[m][r], row0 + r, e);
    const uint32_t d[2] = {w[m][r].x ^ p.xor_mask, w[m][r].y ^ p.xor_mask};
#pragma unroll
    for (int j = 0; j < 8; ++j) wf[m][r][j] = sbyte(d[j >> 2], j & 3) * s;
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b < p.nb) {  // workgroup-uniform; a guarded body keeps acc[r][b] statically indexed
      const double2* x2 = (const double2*)(xs + (size_t)b * kBKC);
      double xv[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double2 t = x2[j * 64 + lane];
        xv[2 * j] = t.x;
        xv[2 * j + 1] = t.y;
      }
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[m][r][b] = fma(wf[m][r][j], xv[j], acc[m][r][b]);
    }
  }
}

// The 64-lane totals of this wavefront's R x NB partial sums: lanes 2o and 2o + 1 of output
// o = r NB + b each add 32 of its 64 partials (through this wavefront's LDS rows), then the pair.
// Returns output (lane / 2)'s total in lanes 2o, 2o + 1 (garbage in lanes past 2 R NB). Rows are
// kRedRow doubles apart (16 bytes past a multiple of the 256-byte bank cycle, so the rows the
// lanes read at one offset fall on different banks) and lane h of a pair reads the odd or even
// 16-byte pieces of its row.

template <int NB, int R>
IRON_DEV double batch_reduce(const double (&acc)[R][NB], double* red) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) red[(r * NB + b) * kRedRow + lane] = acc[r][b];
  // one wavefront's LDS accesses complete in order: its reads below see its writes
  const int o = lane >> 1, h = lane & 1;
  double t = 0.0;
  if (o < R * NB) {
    const double2* q = (const double2*)(red + o * kRedRow);
    double v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double2 d = q[2 * i + h];
      v[i] = d.x + d.y;
    }
#pragma unroll
    for (int wdt = 8; wdt >= 1; wdt >>= 1)
#pragma unroll
      for (int i = 0; i < wdt; ++i) v[i] += v[i + wdt];
    t = v[0];
  }
  return t + dpp_d<0xb1>(t);  // quad_perm [1,0,3,2]: lanes 2o and 2o + 1
}

template <int NB, bool DUAL, int NCK>
__global__ __launch_bounds__(256) void gemv_batch_kernel(GemvParams p) {
  constexpr int R = batch_rows<NB, DUAL, NCK>();
  static_assert(R > 0, "no register budget for this batch and K");
  __shared__ __align__(16) double s_buf[batch_lds_doubles<NB, DUAL, NCK>()];
  __shared__ double s_inv[NB];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const bool rms = p.pro == PRO_RMS_BF16 || p.pro == PRO_RES_RMS_F32;
  constexpr int M = DUAL ? 2 : 1;  // matrices (gate, up)
  uint2 w[NCK][M][R];
  uint32_t sc[NCK][M][R];
  XSlots<NB> xr;
  const int nch = (p.K + kBKC - 1) / kBKC;  // <= NCK
  // the first chunk's activations, then every weight load of this wavefront's rows, then the
  // activation statistics while they are in flight
  batch_load<NB>(p, 0, xr);
#pragma unroll
  for (int c = 0; c < NCK; ++c) {
    if (c < nch) {
      batch_fetch<R>(p, p.w, row0, c * kBKC + lane * 8, w[c][0], sc[c][0]);
      if constexpr (DUAL) batch_fetch<R>(p, p.w2, row0, c * kBKC + lane * 8, w[c][M - 1],
                                         sc[c][M - 1]);
    }
  }
  if (rms) batch_inv_rms(p, s_inv);
  double acc[M][R][NB];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0;
#pragma unroll
  for (int c = 0; c < NCK; ++c) {
    if (c < nch) {  // workgroup-uniform
      const int e = c * kBKC + lane * 8;
      __syncthreads();  // the previous chunk's LDS reads (and the statistics) are done
      batch_store<NB>(p, xr, s_inv, s_buf);
      if (c + 1 < nch) batch_load<NB>(p, (c + 1) * kBKC, xr);  // streams during this chunk
      __syncthreads();
      batch_fma<NB, R, M>(p, w[c], sc[c], row0, e, s_buf, lane, acc);
    }
  }
  __syncthreads();  // the staged activations are no longer read: s_buf becomes the reduction
  double* red = s_buf + (size_t)wave * R * NB * kRedRow;
  const double v = batch_reduce<NB, R>(acc[0], red);
  double v2 = 0.0;
  if constexpr (DUAL) v2 = batch_reduce<NB, R>(acc[M - 1], red);
  const int o = lane >> 1, r = o / NB, b = o % NB, row = row0 + r;
  if ((lane & 1) || o >= R * NB || b >= p.nb || row >= p.M) return;
  const size_t out = (size_t)b * p.y_stride + row;
  if (p.epi == EPI_BF16) {
    ((uint16_t*)p.y)[out] = f64_to_bf16(v);
  } else if (p.epi == EPI_F32) {
    ((float*)p.y)[out] = (float)v;
  } else if (p.epi == EPI_RES_BF16) {
    const size_t ro = (size_t)b * p.r_stride + row;
    float x1 = bf16_to_f32(p.r1[ro]);
    if (p.r2) x1 = x1 + bf16_to_f32(p.r2[ro]);
    ((uint16_t*)p.y)[out] = f64_to_bf16((double)x1 + v);
  } else if (p.epi == EPI_SWIGLU_F32) {
    ((float*)p.y)[out] = (float)silu_mul(v, v2);
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
      const float q0 = (float)(int)(((int32_t)(d << 24)) >> 24);
      const float q1 = (float)(int)(((int32_t)(d << 16)) >> 24);
      const float q2 = (float)(int)(((int32_t)(d << 8)) >> 24);
      const float q3 = (float)(int)(((int32_t)d) >> 24);
      o[2 * j] = (uint32_t)f32_to_bf16(q0 * s) | ((uint32_t)f32_to_bf16(q1 * s) << 16);
      o[2 * j + 1] = (uint32_t)f32_to_bf16(q2 * s) | ((uint32_t)f32_to_bf16(q3 * s) << 16);
    }
    uint4* dst = (uint4*)(out + (size_t)row * K + e);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// ------------------------------------------------------------------------------------------
// Host launch: choose (R, NCH) so that every lane keeps at most 16 weight slices in flight and
// the grid has enough workgroups to cover the chip.
// ------------------------------------------------------------------------------------------
constexpr int kMaxLdsBytes = 147456;
constexpr int kMaxSlices = 16;

int round_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Long batch-1 GEMVs (the LM head: >= 4096 blocks of 4R = 32 rows) stream four row blocks per
// workgroup.
constexpr long long kLongGroups = 4096;

template <bool INT8, bool DUAL, int B, int R, int NCH>
void launch_one(const GemvParams& p, int grid, size_t lds, hipStream_t s) {
  if constexpr (!xreg_path(B, NCH) && (B == 4 || B == 3 || B == 2)) {
    if (p.nb > B) {  // batches above the staged rows: a workgroup per row group and batch group
      const long long octets = (grid + 7) / 8;
      hipLaunchKernelGGL((gemv_kernel<B, R, NCH, INT8, DUAL, 1, true>),
                         dim3((unsigned)(octets * 8 * p.n_bgroups)), dim3(256), lds, s, p);
      return;
    }
  }
  if constexpr (B == 1 && !DUAL && R == 8 && xreg_path(B, NCH)) {
    if (grid >= kLongGroups) {
      hipLaunchKernelGGL((gemv_kernel<B, R, NCH, INT8, DUAL, 4>), dim3((grid + 3) / 4),
                         dim3(256), lds, s, p);
      return;
    }
  }
  hipLaunchKernelGGL((gemv_kernel<B, R, NCH, INT8, DUAL>), dim3(grid), dim3(256), lds, s, p);
}

template <bool INT8, bool DUAL, int B, int NCH>
bool launch_r(const GemvParams& p, int R, int grid, size_t lds, hipStream_t s) {
  constexpr int slices = DUAL ? 2 * NCH : NCH;
  switch (R) {
    case 1: launch_one<INT8, DUAL, B, 1, NCH>(p, grid, lds, s); return true;
    case 2: if constexpr (2 * slices <= kMaxSlices) { launch_one<INT8, DUAL, B, 2, NCH>(p, grid, lds, s); return true; } break;
    case 4: if constexpr (4 * slices <= kMaxSlices) { launch_one<INT8, DUAL, B, 4, NCH>(p, grid, lds, s); return true; } break;
    case 8: if constexpr (8 * slices <= kMaxSlices) { launch_one<INT8, DUAL, B, 8, NCH>(p, grid, lds, s); return true; } break;
  }
  return false;
}

template <bool INT8, bool DUAL, int B>
bool launch_nch(const GemvParams& p, int NCH, int R, int grid, size_t lds, hipStream_t s) {
  switch (NCH) {
    case 1: return launch_r<INT8, DUAL, B, 1>(p, R, grid, lds, s);
    case 2: return launch_r<INT8, DUAL, B, 2>(p, R, grid, lds, s);
    case 4: return launch_r<INT8, DUAL, B, 4>(p, R, grid, lds, s);
    case 8: return launch_r<INT8, DUAL, B, 8>(p, R, grid, lds, s);
    case 16: if constexpr (!DUAL) return launch_r<INT8, DUAL, B, 16>(p, R, grid, lds, s);
  }
  return false;
}

// gemv_batch_kernel for batches 5..15 when its registers hold every chunk of K (false: use the
// batch-group kernel).
template <int NB, bool DUAL, int NCK>
bool launch_batch_nck(const GemvParams& p, hipStream_t stream) {
  constexpr int R = batch_rows<NB, DUAL, NCK>();
  if constexpr (R == 0) {
    return false;
  } else {
    const long long groups = ((long long)p.M + 4 * R - 1) / (4 * R);
    if (groups > (1ll << 30)) return false;
    hipLaunchKernelGGL((gemv_batch_kernel<NB, DUAL, NCK>), dim3((unsigned)groups), dim3(256), 0,
                       stream, p);
    return true;
  }
}

template <int NB, bool DUAL>
bool launch_batch_nb(const GemvParams& p, hipStream_t stream) {
  const int nch = (p.K + kBKC - 1) / kBKC;
  if (nch <= 4) return launch_batch_nck<NB, DUAL, 4>(p, stream);
  if (nch <= 8) return launch_batch_nck<NB, DUAL, 8>(p, stream);
  if (nch <= 16) return launch_batch_nck<NB, DUAL, 16>(p, stream);
  return false;
}

template <bool DUAL>
bool launch_batch(const GemvParams& p, int B, hipStream_t stream) {
  return B <= 8 ? launch_batch_nb<8, DUAL>(p, stream) : launch_batch_nb<16, DUAL>(p, stream);
}

template <bool INT8, bool DUAL>
int launch_gemv(GemvParams p, int B, hipStream_t stream, const char* fn) {
  if (B < 1 || B > iron::kGemvBatchedMax)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: batch %d outside the GEMV path's 1..%d", fn, B,
                      iron::kGemvBatchedMax);
  p.nb = B;
  if constexpr (INT8) {
    if (B > 4 && p.epi != EPI_BF16_ARGMAX && launch_batch<DUAL>(p, B, stream))
      return iron::check_launch(fn);
  }
  const int chunk = INT8 ? 1024 : 512;
  const size_t row_bytes = (size_t)((p.K + chunk - 1) / chunk * chunk) * sizeof(float);
  // kernel batch: the rows staged in LDS at once (at most 4, fewer for long rows); larger
  // batches run in groups of BK rows over the same weight registers
  int BK = B < 4 ? B : 4;
  while (BK > 1 && (size_t)BK * row_bytes > (size_t)kMaxLdsBytes) --BK;
  p.n_bgroups = (B + BK - 1) / BK;
  size_t lds = (size_t)BK * row_bytes;
  if (lds > (size_t)kMaxLdsBytes)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: K=%d exceeds the LDS-staged GEMV limit", fn,
                      p.K);
  const int NCH = round_pow2((p.K + chunk - 1) / chunk);
  if (xreg_path(BK, NCH)) {
    if (B > 1)  // the register path holds one row (only short rows take it, and they fit 4)
      return iron::fail(IRON_ERR_UNSUPPORTED, "%s: batch %d with K=%d", fn, B, p.K);
    lds = 0;  // the activation stays in registers
  }
  const int slices = (DUAL ? 2 : 1) * NCH;
  if (slices > kMaxSlices)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: K=%d too long for the resident-slice GEMV", fn,
                      p.K);
  // rows per wavefront: as many as the slice budget allows while the grid stays >= 2 waves of
  // workgroups over the 256 CUs
  int R = 1;
  while (R < 8 && 2 * R * slices <= kMaxSlices &&
         (long long)p.M >= (long long)4 * (2 * R) * 512)
    R *= 2;
  const long long groups = ((long long)p.M + 4 * R - 1) / (4 * R);
  if (groups > (1ll << 30)) return iron::fail(IRON_ERR_SHAPE, "%s: M too large", fn);
  const int grid = (int)groups;
  bool ok = false;
  if (p.n_bgroups > 1 && BK == 1)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: batch %d with K=%d", fn, B, p.K);
  if ((long long)grid * p.n_bgroups + 8ll * p.n_bgroups > (1ll << 30))
    return iron::fail(IRON_ERR_SHAPE, "%s: M too large", fn);
  switch (BK) {
    case 1: ok = launch_nch<INT8, DUAL, 1>(p, NCH, R, grid, lds, stream); break;
    case 2: ok = launch_nch<INT8, DUAL, 2>(p, NCH, R, grid, lds, stream); break;
    case 3: ok = launch_nch<INT8, DUAL, 3>(p, NCH, R, grid, lds, stream); break;
    default: ok = launch_nch<INT8, DUAL, 4>(p, NCH, R, grid, lds, stream); break;
  }
  if (!ok) return iron::fail(IRON_ERR_UNSUPPORTED, "%s: no kernel for K=%d R=%d", fn, p.K, R);
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
  p.xor_mask = domain == IRON_DOMAIN_BIASED ? 0x80808080u : 0u;
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
  return launch_gemv<true, true>(p, B, stream, "iron_swiglu_mlp(gate/up)");
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
  return launch_gemv<true, false>(p, B, stream, "iron_swiglu_mlp(down)");
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
  return launch_gemv<true, false>(p, B, stream, fn);
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
                     domain == IRON_DOMAIN_BIASED ? 0x80808080u : 0u);
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
  if (!iron::aligned(x, 16))
    return iron::fail(IRON_ERR_ALIGN, "iron_gemv_w8a16: x not 16-byte aligned");
  GemvParams p = wire_params(wire, M, K, G, tile_m, domain);
  p.pro = PRO_BF16;
  p.x = x;
  p.x_stride = K;
  p.epi = EPI_BF16;
  p.y = y;
  p.y_stride = M;
  return launch_gemv<true, false>(p, B, (hipStream_t)stream, "iron_gemv_w8a16");
}

int iron_gemv_bf16(const uint16_t* w, const uint16_t* x, uint16_t* y, int B, int M, int K,
                   void* stream) {
  iron::clear_error();
  if (!w || !x || !y) return iron::fail(IRON_ERR_NULL, "iron_gemv_bf16: null pointer");
  if (B <= 0 || M <= 0 || K <= 0 || K % 8)
    return iron::fail(IRON_ERR_SHAPE, "iron_gemv_bf16: bad shape B=%d M=%d K=%d", B, M, K);
  if (!iron::aligned(w, 16) || !iron::aligned(x, 16))
    return iron::fail(IRON_ERR_ALIGN, "iron_gemv_bf16: W or x not 16B aligned");
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
  return launch_gemv<false, false>(p, B, (hipStream_t)stream, "iron_gemv_bf16");
}

int iron_lm_head(const void* w, int w_kind, const uint16_t* x, const uint16_t* norm_w, float eps,
                 uint16_t* logits, unsigned long long* argmax_keys, int B, int V, int D, int G,
                 int tile_m, int domain, void* stream) {
  iron::clear_error();
  if (!w || !x || !logits) return iron::fail(IRON_ERR_NULL, "iron_lm_head: null pointer");
  if (B <= 0 || V <= 0 || D <= 0 || D % 16)
    return iron::fail(IRON_ERR_SHAPE, "iron_lm_head: bad shape B=%d V=%d D=%d", B, V, D);
  if (!iron::aligned(x, 16) || (norm_w && !iron::aligned(norm_w, 16)))
    return iron::fail(IRON_ERR_ALIGN, "iron_lm_head: x / norm weight not 16B aligned");
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
  if (w_kind == IRON_WEIGHT_INT8)
    return launch_gemv<true, false>(p, B, (hipStream_t)stream, "iron_lm_head");
  return launch_gemv<false, false>(p, B, (hipStream_t)stream, "iron_lm_head");
}

}  // extern "C"
