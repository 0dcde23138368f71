// GQA decode attention (one query token per sequence) over a bf16 KV cache: split-K across
// workgroups (flash-decoding), then a merge kernel.
//
// Reference: DecodeAttention (iron/operators/decode_attn/op.py:20-181), kernels
// aie_kernels/aie2p/decode_attn.cc:117-311 (scores with scale log2(e)/sqrt(D), online softmax over
// KV blocks, finalize out/l with l == 0 -> 0), golden iron/operators/decode_attn/reference.py:
// 26-38 (kv = h*KV//H).
//
// Arithmetic: the exact value of the golden, o = sum_j e^(s_j - m) v_j / sum_j e^(s_j - m) with
// s_j = (q . k_j) / sqrt(D), evaluated in fp64 (scores, exponentials, sums, accumulation) and
// rounded once to bf16. The exp2/log2(e) form of the reference is the same function.
//
// Mapping: grid (split, kv * head_groups, b), 256 threads = 4 wavefronts. Lane l works on token
// row l/16 of a 4-token group and on head dims [8*(l%16), +8): one 128-bit load per lane reads 4
// consecutive K (or V) rows = 1 KiB per wavefront instruction. HB query heads of the GQA group
// share every K/V load. Per 16 tokens (4 rows x 4 unrolled groups) a row keeps one online-softmax
// state per head; the row's lanes split the block's exponentials between them (one exp per
// (token, head) instead of sixteen) and share the results with DPP row broadcasts. Rows and
// wavefronts merge through shuffles and LDS; splits merge in a second kernel.
#include <utility>

#include "common.h"
#include "internal.h"

namespace {

constexpr int kD = 128;
constexpr int kTokensPerIter = 64;  // 4 waves x 4 rows x 4 unrolled groups

struct AttnParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  long long sb, sh, st;
  const int32_t* ctx_len;
  int ctx_const;
  int max_ctx;
  uint16_t* out;
  int H, KV, HG, HB;   // heads, kv heads, GQA group, heads per workgroup
  int chunk, nsplit;
  double scale;
  double* part;        // [B][H][nsplit][D + 2]: o (unnormalised), m, l
};

template <int N>
IRON_DEV double row_share_d(double v) {
  // every lane of a 16-lane row receives lane N of that row
  return dpp_d<0x150 + N>(v);
}

// Lane N of each row evaluated exponential N; every lane of the row receives it.
template <int N, int HB>
IRON_DEV void share_one(double ev, double (&pe)[4][HB], double (&corr)[HB]) {
  if constexpr (N < 4 * HB) {
    pe[N / HB][N % HB] = row_share_d<N>(ev);
  } else if constexpr (N < 5 * HB) {
    corr[N - 4 * HB] = row_share_d<N>(ev);
  }
}

template <int HB, int... Ns>
IRON_DEV void share_all(double ev, double (&pe)[4][HB], double (&corr)[HB],
                        std::integer_sequence<int, Ns...>) {
  (share_one<Ns, HB>(ev, pe, corr), ...);
}

IRON_DEV double pick(const double* vals, int idx, int n) {
  double r = vals[0];
#pragma unroll
  for (int i = 1; i < 16; ++i)
    if (i < n && idx == i) r = vals[i];
  return r;
}

template <int HB>
__global__ __launch_bounds__(256) void decode_attn_kernel(AttnParams p) {
  const int split = blockIdx.x, b = blockIdx.z;
  const int groups = p.HG / HB;
  const int kv = blockIdx.y / groups, hg = blockIdx.y % groups;
  const int h0 = kv * p.HG + hg * HB;  // first query head of this workgroup
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane >> 4, dl = lane & 15;

  int ctx = p.ctx_len ? p.ctx_len[b] : p.ctx_const;
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int t_begin = split * p.chunk;
  const int t_end = min(ctx, t_begin + p.chunk);

  double qf[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    const uint4 qq = *(const uint4*)(p.q + ((size_t)b * p.H + h0 + h) * kD + dl * 8);
    const uint32_t qd[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qf[h][2 * j] = bf16lo_to_f32(qd[j]);
      qf[h][2 * j + 1] = bf16hi_to_f32(qd[j]);
    }
  }

  double m[HB], l[HB], o[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.0;
  }

  const uint16_t* kbase = p.k + (size_t)b * p.sb + (size_t)kv * p.sh + dl * 8;
  const uint16_t* vbase = p.v + (size_t)b * p.sb + (size_t)kv * p.sh + dl * 8;

  for (int t0 = t_begin; t0 < t_end; t0 += kTokensPerIter) {
    uint4 kr[4], vr[4];
    bool tv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * 16 + wave * 4 + row;
      tv[u] = t < t_end;
      if (tv[u]) {
        kr[u] = *(const uint4*)(kbase + (size_t)t * p.st);
        vr[u] = *(const uint4*)(vbase + (size_t)t * p.st);
      } else {
        kr[u] = make_uint4(0u, 0u, 0u, 0u);
        vr[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    // scores s[u][h], identical in every lane of the row
    double s[4][HB];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t kd[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
      double kf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kf[2 * j] = bf16lo_to_f32(kd[j]);
        kf[2 * j + 1] = bf16hi_to_f32(kd[j]);
      }
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        double a = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fma(qf[h][j], kf[j], a);
        a = row16_sum_d(a) * p.scale;
        s[u][h] = tv[u] ? a : -INFINITY;
      }
    }
    // new running max per head (row-uniform)
    double mn[HB];
    bool any = false;
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const double mb = fmax(fmax(s[0][h], s[1][h]), fmax(s[2][h], s[3][h]));
      mn[h] = fmax(m[h], mb);
      any |= mn[h] != -INFINITY;
    }
    if (!any) continue;  // row-uniform: no valid token in this row yet
    // lane dl evaluates one exponential: (u, h) = (dl / HB, dl % HB) for dl < 4*HB, the
    // correction e^(m_old - m_new) of head dl - 4*HB for 4*HB <= dl < 5*HB
    double arg = -INFINITY;
    {
      double vals[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) vals[i] = -INFINITY;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < HB; ++h) vals[u * HB + h] = s[u][h] - mn[h];
#pragma unroll
      for (int h = 0; h < HB; ++h)
        if (4 * HB + h < 16) vals[4 * HB + h] = (m[h] == -INFINITY) ? -INFINITY : m[h] - mn[h];
      arg = pick(vals, dl, 5 * HB);
    }
    // exp(-inf) = 0 covers invalid tokens and heads with no valid token (mn == -inf makes the
    // argument NaN only when both sides are -inf, which the guard above excludes for m)
    const double ev = (arg == -INFINITY || arg != arg) ? 0.0 : exp(arg);
    double pe[4][HB], corr[HB];
    share_all<HB>(ev, pe, corr, std::make_integer_sequence<int, 16>{});
    if constexpr (HB >= 4) {
      // 5*HB = 20 > 16 lanes: the last four corrections are computed directly
#pragma unroll
      for (int h = 0; h < HB; ++h)
        if (4 * HB + h >= 16) corr[h] = (m[h] == -INFINITY) ? 0.0 : exp(m[h] - mn[h]);
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      if (mn[h] == -INFINITY) continue;
      const double c = (m[h] == -INFINITY) ? 0.0 : corr[h];
      l[h] = l[h] * c + ((pe[0][h] + pe[1][h]) + (pe[2][h] + pe[3][h]));
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= c;
      m[h] = mn[h];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t vd[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
      double vf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vf[2 * j] = bf16lo_to_f32(vd[j]);
        vf[2 * j + 1] = bf16hi_to_f32(vd[j]);
      }
#pragma unroll
      for (int h = 0; h < HB; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) o[h][j] = fma(pe[u][h], vf[j], o[h][j]);
    }
  }

  // merge the 4 token rows of this wavefront (lanes l, l^16, l^32, l^48 share head dims)
#pragma unroll
  for (int step = 16; step <= 32; step <<= 1) {
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const double mo = __shfl_xor(m[h], step);
      const double lo = __shfl_xor(l[h], step);
      double oo[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) oo[j] = __shfl_xor(o[h][j], step);
      const double mm = fmax(m[h], mo);
      if (mm != -INFINITY) {
        const double c1 = m[h] == -INFINITY ? 0.0 : exp(m[h] - mm);
        const double c2 = mo == -INFINITY ? 0.0 : exp(mo - mm);
        l[h] = l[h] * c1 + lo * c2;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[h][j] = o[h][j] * c1 + oo[j] * c2;
        m[h] = mm;
      }
    }
  }

  // merge the 4 wavefronts through LDS
  __shared__ double s_o[4][HB][kD];
  __shared__ double s_m[4][HB], s_l[4][HB];
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < HB; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s_o[wave][h][dl * 8 + j] = o[h][j];
      if (dl == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < HB * kD; t += 256) {
    const int oh = t / kD, od = t % kD;
    double M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmax(M, s_m[w][oh]);
    double L = 0.0, O = 0.0;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const double f = s_m[w][oh] == -INFINITY ? 0.0 : exp(s_m[w][oh] - M);
        L += f * s_l[w][oh];
        O += f * s_o[w][oh][od];
      }
    }
    const int hq = h0 + oh;
    if (p.nsplit == 1) {
      p.out[((size_t)b * p.H + hq) * kD + od] = f64_to_bf16(L > 0.0 ? O / L : 0.0);
    } else {
      double* part = p.part + (((size_t)b * p.H + hq) * p.nsplit + split) * (kD + 2);
      part[od] = O;
      if (od == 0) {
        part[kD] = M;
        part[kD + 1] = L;
      }
    }
  }
}

// grid (H, B), 128 threads: o = sum_s f_s O_s / sum_s f_s L_s, f_s = e^(m_s - max m).
__global__ __launch_bounds__(128) void attn_merge_kernel(AttnParams p) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int ns = p.nsplit;
  const double* base = p.part + ((size_t)b * p.H + h) * ns * (kD + 2);
  __shared__ double s_f[256];
  __shared__ double s_red[2];
  double mloc = -INFINITY;
  for (int s = d; s < ns; s += 128) mloc = fmax(mloc, base[(size_t)s * (kD + 2) + kD]);
  // block max over 2 wavefronts
  mloc = fmax(mloc, __shfl_xor(mloc, 1));
  mloc = fmax(mloc, __shfl_xor(mloc, 2));
  mloc = fmax(mloc, __shfl_xor(mloc, 4));
  mloc = fmax(mloc, __shfl_xor(mloc, 8));
  mloc = fmax(mloc, __shfl_xor(mloc, 16));
  mloc = fmax(mloc, __shfl_xor(mloc, 32));
  if ((d & 63) == 0) s_red[d >> 6] = mloc;
  __syncthreads();
  const double M = fmax(s_red[0], s_red[1]);
  __syncthreads();
  double lloc = 0.0;
  for (int s = d; s < ns; s += 128) {
    const double ms = base[(size_t)s * (kD + 2) + kD];
    const double f = (M == -INFINITY || ms == -INFINITY) ? 0.0 : exp(ms - M);
    s_f[s] = f;
    lloc += f * base[(size_t)s * (kD + 2) + kD + 1];
  }
  lloc = wave_sum_d(lloc);
  if ((d & 63) == 0) s_red[d >> 6] = lloc;
  __syncthreads();
  const double L = s_red[0] + s_red[1];
  double O0 = 0.0, O1 = 0.0;
  int s = 0;
  for (; s + 2 <= ns; s += 2) {
    O0 = fma(s_f[s], base[(size_t)s * (kD + 2) + d], O0);
    O1 = fma(s_f[s + 1], base[(size_t)(s + 1) * (kD + 2) + d], O1);
  }
  if (s < ns) O0 = fma(s_f[s], base[(size_t)s * (kD + 2) + d], O0);
  const double O = O0 + O1;
  p.out[((size_t)b * p.H + h) * kD + d] = f64_to_bf16(L > 0.0 ? O / L : 0.0);
}

struct SplitPlan {
  int nsplit, chunk, hb;
};

SplitPlan plan_split(int B, int H, int KV, int max_ctx) {
  SplitPlan sp;
  const int HG = H / KV;
  sp.hb = HG >= 4 ? 4 : HG;
  const int wg_per_split = B * KV * (HG / sp.hb);
  const int target_wgs = 512;
  int ns = (target_wgs + wg_per_split - 1) / wg_per_split;
  const int max_ns = (max_ctx + kTokensPerIter - 1) / kTokensPerIter;
  if (ns > max_ns) ns = max_ns;
  if (ns > 256) ns = 256;
  if (ns < 1) ns = 1;
  int chunk = (max_ctx + ns - 1) / ns;
  chunk = ((chunk + kTokensPerIter - 1) / kTokensPerIter) * kTokensPerIter;
  ns = (max_ctx + chunk - 1) / chunk;
  if (ns < 1) ns = 1;
  sp.nsplit = ns;
  sp.chunk = chunk;
  return sp;
}

size_t attn_ws_bytes(int B, int H, int KV, int max_ctx) {
  const SplitPlan sp = plan_split(B, H, KV, max_ctx);
  if (sp.nsplit == 1) return 0;
  return (((size_t)B * H * sp.nsplit * (kD + 2) * sizeof(double)) + 255) & ~(size_t)255;
}

}  // namespace

extern "C" {

size_t iron_decode_attn_workspace(int B, int H, int KV, int D, int max_ctx) {
  if (B <= 0 || H <= 0 || KV <= 0 || D != kD || H % KV || max_ctx <= 0) return 0;
  const size_t n = attn_ws_bytes(B, H, KV, max_ctx);
  return n ? n : 256;
}

int iron_decode_attn(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                     long long kv_sb, long long kv_sh, long long kv_st, const int32_t* ctx_len,
                     int ctx_const, uint16_t* out, int B, int H, int KV, int D, int max_ctx,
                     float scale, void* workspace, size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_decode_attn";
  if (!q || !k_cache || !v_cache || !out) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  if (B <= 0 || H <= 0 || KV <= 0 || max_ctx <= 0)
    return iron::fail(IRON_ERR_SHAPE, "%s: bad shape B=%d H=%d KV=%d max_ctx=%d", fn, B, H, KV,
                      max_ctx);
  if (D != kD) return iron::fail(IRON_ERR_UNSUPPORTED, "%s: head_dim %d (only 128)", fn, D);
  if (H % KV) return iron::fail(IRON_ERR_SHAPE, "%s: H=%d not a multiple of KV=%d", fn, H, KV);
  const int HG = H / KV;
  if (HG != 1 && HG != 2 && HG % 4 != 0)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: GQA group %d not 1, 2 or a multiple of 4", fn,
                      HG);
  if (kv_st % 8 || kv_sh % 8 || kv_sb % 8 || !iron::aligned(k_cache, 16) ||
      !iron::aligned(v_cache, 16) || !iron::aligned(q, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: K/V/Q rows must be 16-byte aligned", fn);
  if (!ctx_len && (ctx_const < 0 || ctx_const > max_ctx))
    return iron::fail(IRON_ERR_SHAPE, "%s: ctx_const=%d outside [0, %d]", fn, ctx_const, max_ctx);
  const SplitPlan sp = plan_split(B, H, KV, max_ctx);
  AttnParams p = {};
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.sb = kv_sb;
  p.sh = kv_sh;
  p.st = kv_st;
  p.ctx_len = ctx_len;
  p.ctx_const = ctx_const;
  p.max_ctx = max_ctx;
  p.out = out;
  p.H = H;
  p.KV = KV;
  p.HG = HG;
  p.HB = sp.hb;
  p.chunk = sp.chunk;
  p.nsplit = sp.nsplit;
  p.scale = (double)scale;
  if (sp.nsplit > 1) {
    const size_t need = attn_ws_bytes(B, H, KV, max_ctx);
    if (!workspace || workspace_bytes < need)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                        need);
    if (!iron::aligned(workspace, 256))
      return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
    p.part = (double*)workspace;
  }
  dim3 grid(sp.nsplit, KV * (HG / sp.hb), B);
  hipStream_t s = (hipStream_t)stream;
  switch (sp.hb) {
    case 1: hipLaunchKernelGGL(decode_attn_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(decode_attn_kernel<2>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(decode_attn_kernel<4>, grid, dim3(256), 0, s, p); break;
  }
  int st = iron::check_launch(fn);
  if (st || sp.nsplit == 1) return st;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(H, B), dim3(128), 0, s, p);
  return iron::check_launch(fn);
}

}  // extern "C"
