// Device building blocks of the exact (fp64) GQA decode-attention core, shared by the split-K
// kernels (attention.hip) and the persistent whole-token decode kernel (decode_persistent.hip).
//
// Reference: DecodeAttention (iron/operators/decode_attn/op.py:20-181), kernels
// aie_kernels/aie2p/decode_attn.cc:117-311, golden iron/operators/decode_attn/reference.py:26-38;
// the per-head QKV epilogue follows qkv_head_dp/reference.py:13-33.
//
// A workgroup is 256 threads (4 wavefronts). Lane l of wavefront w works on token rows
// 16u + 4w + l/16 (u = 0..3) of a 64-token tile and on head dims [8 (l % 16), +8), so one
// 128-bit load per lane reads 4 consecutive K (or V) rows per wavefront instruction, and the HB
// query heads of a GQA group share every K/V load.
#pragma once
#include <utility>

#include "common.h"

namespace iron {
namespace dev {

constexpr int kAttnD = 128;   // head dim
constexpr int kAttnTile = 64; // tokens per tile

template <int N>
IRON_DEV double row_share_d(double v) {
  // every lane of a 16-lane row receives lane N of that row (row_newbcast)
  return dpp_d<0x150 + N>(v);
}

template <int N, int HB, int U>
IRON_DEV void share_one(double ev, double (&pe)[U][HB]) {
  if constexpr (N < U * HB) pe[N / HB][N % HB] = row_share_d<N>(ev);
}

template <int HB, int U, int... Ns>
IRON_DEV void share_all(double ev, double (&pe)[U][HB], std::integer_sequence<int, Ns...>) {
  (share_one<Ns, HB, U>(ev, pe), ...);
}

// Sum of a tile's U exponentials of head h, as a balanced pairwise tree ((0+1)+(2+3) for U = 4).
template <int U, int HB>
IRON_DEV double tile_sum(const double (&pe)[U][HB], int h) {
  if constexpr (U == 4) {
    return (pe[0][h] + pe[1][h]) + (pe[2][h] + pe[3][h]);
  } else {
    double t = (pe[0][h] + pe[1][h]) + (pe[2][h] + pe[3][h]);
#pragma unroll
    for (int u = 4; u < U; ++u) t += pe[u][h];
    return t;
  }
}

IRON_DEV void unpack8d(const uint4 v, double (&f)[8]) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = bf16lo_to_f32(d[j]);
    f[2 * j + 1] = bf16hi_to_f32(d[j]);
  }
}

IRON_DEV uint4 pack8_bf16(const double (&f)[8]) {
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = (uint32_t)f64_to_bf16(f[2 * j]) | ((uint32_t)f64_to_bf16(f[2 * j + 1]) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// The QKV head epilogue for one head held by a 16-lane row (lane dl owns dims 8*dl..8*dl+7):
//   y = bf16(RMSNorm(x) * w), r = bf16(RoPE(y)) with the two-halves rotation
//   r[i] = y[i] cos_i - y[i+64] sin_i, r[i+64] = y[i+64] cos_i + y[i] sin_i (i < 64).
// a0/a1: this lane's 8 (cos, sin) bf16 pairs of the interleaved angle row (indices (dl%8)*8..+8).
// The same operations and roundings as the standalone epilogue kernel (qkv.hip).
IRON_DEV void norm_rope8(const uint4 xr, const uint4 wr, const uint4 a0, const uint4 a1, int dl,
                         double eps, double (&out)[8]) {
  double x[8], w[8];
  unpack8d(xr, x);
  unpack8d(wr, w);
  const double ss = row16_sum_d(sum_sq_tree(x));
  const double inv = inv_rms(ss, kAttnD, eps);
  float y[8], yp[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = bf16_to_f32(f64_to_bf16((x[j] * inv) * w[j]));
  // the partner dims (+-64) live in lane dl ^ 8 of the same row (row_ror:8)
#pragma unroll
  for (int j = 0; j < 8; ++j) yp[j] = dpp_f<0x128>(y[j]);
  const uint32_t ad[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const double c = bf16lo_to_f32(ad[j]), s = bf16hi_to_f32(ad[j]);
    const double r = dl < 8 ? (double)y[j] * c - (double)yp[j] * s
                            : (double)y[j] * c + (double)yp[j] * s;
    out[j] = bf16_to_f32(f64_to_bf16(r));
  }
}

// Row transpose-sum: v[0..N) in every lane of a 16-lane row (N = 4, 8 or 16); afterwards lane dl
// holds the sum over the row's 16 lanes of v[dl % N]. log2(N) exchange steps each halve the values
// a lane keeps (it keeps one half of its current set, sends the other to its partner and adds
// what the partner sends: partners differ in bit 3 (row_ror:8), bit 2 (row_half_mirror, lane
// 7 - l within each half), bit 1 (quad_perm [2,3,0,1]) and bit 0 (quad_perm [1,0,3,2]), taken
// from bit log2(N) - 1 down), then plain sums over the remaining high bits (rotations by 4 and 8,
// which pair lanes with the same low bits). 15 exchanged values
// for N = 16, against 16 four-step row sums. The order of the additions differs from a row sum
// per value; the q.k sums it serves are exact in fp64 (bf16 products), so the totals do not.
template <int STEP_CTRL, int N>
IRON_DEV void tsum_step(const double (&in)[N], double (&out)[N / 2], bool upper) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const double keep = upper ? in[N / 2 + i] : in[i];
    const double send = upper ? in[i] : in[N / 2 + i];
    out[i] = keep + dpp_d<STEP_CTRL>(send);
  }
}

template <int N>
IRON_DEV double row16_transpose_sum(const double (&v)[N], int dl) {
  static_assert(N == 4 || N == 8 || N == 16, "4, 8 or 16 values");
  double r;
  if constexpr (N == 16) {
    double a[8], b[4], c[2];
    tsum_step<0x128, 16>(v, a, (dl & 8) != 0);
    tsum_step<0x141, 8>(a, b, (dl & 4) != 0);
    tsum_step<0x4e, 4>(b, c, (dl & 2) != 0);
    double d[1];
    tsum_step<0xb1, 2>(c, d, (dl & 1) != 0);
    r = d[0];
  } else if constexpr (N == 8) {
    double b[4], c[2], d[1];
    tsum_step<0x141, 8>(v, b, (dl & 4) != 0);
    tsum_step<0x4e, 4>(b, c, (dl & 2) != 0);
    tsum_step<0xb1, 2>(c, d, (dl & 1) != 0);
    r = d[0];
    r += dpp_d<0x128>(r);
  } else {
    double c[2], d[1];
    tsum_step<0x4e, 4>(v, c, (dl & 2) != 0);
    tsum_step<0xb1, 2>(c, d, (dl & 1) != 0);
    r = d[0];
    r += dpp_d<0x124>(r);  // row_ror:4, then row_ror:8: the four lanes with this dl % 4
    r += dpp_d<0x128>(r);
  }
  return r;
}

// One 64-token tile of the exact (fp64) core. Lane (wave, row, dl) holds the K/V rows
// t0 + 16u + 4 wave + row (u = 0..3), head dims 8 dl..+8; rows at or past t_end are masked and,
// with FUSED and has_new, the row at `pos` is replaced by the current token's rows (s_new).
// Updates the running maximum m, sum l and unnormalised output o of the HB heads; `it` is the
// tile's index within this workgroup's sequence (0 = the first tile, which starts from zero).
// s_mx is the workgroup's tile-maximum exchange; the function ends past its one barrier.
// Score (u, h) of a row is reduced into lane dl = u HB + h (row16_transpose_sum), which also
// evaluates its exponential; lane h evaluates head h's rescale factor; both are broadcast over
// the row (row_newbcast).
template <int HB, bool FUSED, int U = 4>
IRON_DEV void attn_tile_f64(uint4 (&kr)[U], uint4 (&vr)[U], int t0, int t_end, bool has_new,
                            int pos, const uint4 (&s_new)[2][16], const double (&qf)[HB][8],
                            double scale, int it, double (&m)[HB], double (&l)[HB],
                            double (&o)[HB][8], double (&s_mx)[2][4][HB], int wave, int lane,
                            int row, int dl) {
  constexpr int N = U * HB;
  static_assert(N == 4 || N == 8 || N == 16, "one score per lane of a 16-lane row");
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = t0 + u * 16 + wave * 4 + row;
    if constexpr (FUSED) {
      if (has_new && t == pos) {
        kr[u] = s_new[0][dl];
        vr[u] = s_new[1][dl];
      }
    }
    if (t >= t_end) vr[u] = make_uint4(0u, 0u, 0u, 0u);  // rows past the context may hold NaNs
  }
  // Two workgroups share each CU, so two wavefronts each SIMD. A wavefront raises its priority
  // from the q.k dot products through the tile's dependent chain (the transpose sum, the maximum
  // and its barrier, the exponentials and their broadcast) and drops it for P.V, so the SIMD's
  // other wavefront fills the chain's latency with its own P.V FMAs (config 5: 7.84 -> 7.68 ms
  // per step; config 3 B=8: 22.3 -> 21.3 us).
  __builtin_amdgcn_s_setprio(1);
  // this lane's 8-dim partials of every (u, h), then the row sums, score (u, h) in lane u HB + h
  double part[N];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double kf[8];
    unpack8d(kr[u], kf);
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      double a = 0.0;
#pragma unroll
      for (int j = 0; j < 8; ++j) a = fma(qf[h][j], kf[j], a);
      part[u * HB + h] = a;
    }
  }
  const int si = dl % N, sh = si % HB;
  const bool sv = t0 + (si / HB) * 16 + wave * 4 + row < t_end;
  double tot = row16_transpose_sum<N>(part, dl);
  // The exchange must run with every lane of the row active: its DPP moves read partner lanes,
  // and the compiler would otherwise sink it into the branch on sv below (sv differs between the
  // lanes of a row), where the masked lanes' values would be read stale.
  __asm__ volatile("" : "+v"(tot));
  const double sc = sv ? tot * scale : -INFINITY;
  // workgroup-wide tile maximum per head: over the U lanes of head sh in the row (lanes sh + k HB,
  // k < U: rotations by HB, 2 HB, ... within the 16-lane row), the wavefront's rows, the waves
  double v = sc;
  if constexpr (HB * U >= 2 && HB < 16) {
#pragma unroll
    for (int k = HB; k < 16; k *= 2) {
      if (k == 1) v = fmax(v, dpp_d<0x121>(v));
      else if (k == 2) v = fmax(v, dpp_d<0x122>(v));
      else if (k == 4) v = fmax(v, dpp_d<0x124>(v));
      else v = fmax(v, dpp_d<0x128>(v));
    }
  }
  v = fmax(v, __shfl_xor(v, 16));
  v = fmax(v, __shfl_xor(v, 32));
  if (lane < HB) s_mx[it & 1][wave][lane] = v;  // lane h < HB holds head h's maximum
  __syncthreads();
  double mn[HB];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    const double t = fmax(fmax(s_mx[it & 1][0][h], s_mx[it & 1][1][h]),
                          fmax(s_mx[it & 1][2][h], s_mx[it & 1][3][h]));
    mn[h] = fmax(m[h], t);
  }
  // every tile of the loop holds at least one valid token, so mn is finite here
  double mn_s = mn[0], m_s = m[0];
#pragma unroll
  for (int h = 1; h < HB; ++h)
    if (sh == h) {
      mn_s = mn[h];
      m_s = m[h];
    }
  const double ev = sc == -INFINITY ? 0.0 : exp(sc - mn_s);
  double pe[U][HB];
  share_all<HB, U>(ev, pe, std::make_integer_sequence<int, 16>{});
  __builtin_amdgcn_s_setprio(0);
  // rescale the running sums (the first tile starts from zero): lane h has head h's factor.
  // Skipped when no maximum moved (every factor would be e^0 = 1 exactly); workgroup-uniform.
  bool moved = false;
#pragma unroll
  for (int h = 0; h < HB; ++h) moved = moved || mn[h] != m[h];
  if (it > 0 && moved) {
    const double cf = m_s == -INFINITY ? 0.0 : exp(m_s - mn_s);
    double c[HB];
    if constexpr (HB == 1) c[0] = row_share_d<0>(cf);
    else if constexpr (HB == 2) { c[0] = row_share_d<0>(cf); c[1] = row_share_d<1>(cf); }
    else {
      c[0] = row_share_d<0>(cf); c[1] = row_share_d<1>(cf);
      c[2] = row_share_d<2>(cf); c[3] = row_share_d<3>(cf);
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      l[h] *= c[h];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= c[h];
    }
  }
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    l[h] += tile_sum<U>(pe, h);
    m[h] = mn[h];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double vf[8];
    unpack8d(vr[u], vf);
#pragma unroll
    for (int h = 0; h < HB; ++h)
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] = fma(pe[u][h], vf[j], o[h][j]);
  }
}

// The end of the exact core: the 16 token rows of a workgroup (4 per wavefront) hold partial sums
// under the same offsets m, so they add. For every (head oh, dim od) of the HB heads the
// workgroup's unnormalised output O, its sum L and maximum M go to emit(oh, od, O, L, M), called
// once per pair by one thread. s_o is the caller's LDS (16 x HB x kAttnD doubles), free on entry.
template <int HB, class Emit>
IRON_DEV void attn_finish_f64(const double (&m)[HB], const double (&l)[HB],
                              const double (&o)[HB][8], int wave, int row, int dl,
                              double (*s_o)[HB][kAttnD], Emit emit) {
  __shared__ double s_l[16][HB];
  __shared__ double s_mm[HB];  // m is the workgroup's (s_mx): thread 0's copy, read by index
  const int rr = wave * 4 + row;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
#pragma unroll
    for (int j = 0; j < 8; j += 2)
      *(double2*)&s_o[rr][h][dl * 8 + j] = make_double2(o[h][j], o[h][j + 1]);
    if (dl == 0) s_l[rr][h] = l[h];
    if (threadIdx.x == 0) s_mm[h] = m[h];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < HB * kAttnD; t += 256) {
    const int oh = t / kAttnD, od = t % kAttnD;
    double so[16], sl[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      so[r] = s_o[r][oh][od];
      sl[r] = s_l[r][oh];
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int r = 0; r < w; ++r) {
        so[r] += so[r + w];
        sl[r] += sl[r + w];
      }
    emit(oh, od, so[0], sl[0], s_mm[oh]);
  }
}

}  // namespace dev
}  // namespace iron
