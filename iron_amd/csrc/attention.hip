// GQA decode attention (one query token per sequence) over a bf16 KV cache, split-K across
// workgroups (flash-decoding) with an in-kernel merge by the last workgroup of each (b, kv head).
//
// Reference: DecodeAttention (iron/operators/decode_attn/op.py:20-181), kernels
// aie_kernels/aie2p/decode_attn.cc:117-311 (scores with scale log2(e)/sqrt(D), exp2 online
// softmax over KV blocks, finalize out/l with l == 0 -> 0), golden
// iron/operators/decode_attn/reference.py:26-38 (fp32, exp2 form, kv = h*KV//H).
// Numerics here: fp32 scores, fp32 probabilities (no bf16 rounding of p), fp32 accumulation,
// one bf16 rounding of the output.
//
// Mapping: grid (split, kv, b), 256 threads = 4 wavefronts. Lane l works on token row l/16 of a
// 4-token group and on head dims [8*(l%16), +8): one 128-bit load per lane reads 4 consecutive
// K (or V) rows = 1 KiB per wavefront instruction. The HG = H/KV query heads of the GQA group
// share every K/V load. Each 16-lane row keeps its own online-softmax state; rows, wavefronts
// and finally splits are merged with the standard (m, l, o) rescaling.
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
  int H, KV;
  int chunk, nsplit;
  float scale_log2;
  float* part;         // [B][KV][nsplit][HG*(D+2)]
  unsigned int* cnt;   // [B][KV]
};

IRON_DEV float safe_exp2_diff(float a, float m) {
  // exp2(a - m) with a == -inf -> 0 (m is finite whenever this is called)
  return exp2f(a - m);
}

template <int HG>
__global__ __launch_bounds__(256) void decode_attn_kernel(AttnParams p) {
  const int split = blockIdx.x, kv = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane >> 4, dl = lane & 15;

  int ctx = p.ctx_len ? p.ctx_len[b] : p.ctx_const;
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int t_begin = split * p.chunk;
  const int t_end = min(ctx, t_begin + p.chunk);

  float qf[HG][8];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    const uint4 qq = *(const uint4*)(p.q + ((size_t)b * p.H + (size_t)kv * HG + h) * kD + dl * 8);
    const uint32_t qd[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qf[h][2 * j] = bf16lo_to_f32(qd[j]) * p.scale_log2;
      qf[h][2 * j + 1] = bf16hi_to_f32(qd[j]) * p.scale_log2;
    }
  }

  float m[HG], l[HG], o[HG][8];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.f;
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
    float s[4][HG];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t kd[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
      float kf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kf[2 * j] = bf16lo_to_f32(kd[j]);
        kf[2 * j + 1] = bf16hi_to_f32(kd[j]);
      }
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fmaf(qf[h][j], kf[j], a);
        a = row16_sum(a);
        s[u][h] = tv[u] ? a : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float mb = fmaxf(fmaxf(s[0][h], s[1][h]), fmaxf(s[2][h], s[3][h]));
      const float mn = fmaxf(m[h], mb);
      if (mn == -INFINITY) continue;  // row-uniform: no valid token yet
      const float c = safe_exp2_diff(m[h], mn);
      l[h] *= c;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= c;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float pu = safe_exp2_diff(s[u][h], mn);
        l[h] += pu;
        const uint32_t vd[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[h][2 * j] = fmaf(pu, bf16lo_to_f32(vd[j]), o[h][2 * j]);
          o[h][2 * j + 1] = fmaf(pu, bf16hi_to_f32(vd[j]), o[h][2 * j + 1]);
        }
      }
      m[h] = mn;
    }
  }

  // Merge the 4 token rows of this wavefront (lanes l, l^16, l^32, l^48 share head dims).
#pragma unroll
  for (int step = 16; step <= 32; step <<= 1) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
      const float mo = __shfl_xor(m[h], step);
      const float lo = __shfl_xor(l[h], step);
      float oo[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) oo[j] = __shfl_xor(o[h][j], step);
      const float mn = fmaxf(m[h], mo);
      if (mn != -INFINITY) {
        const float c1 = safe_exp2_diff(m[h], mn), c2 = safe_exp2_diff(mo, mn);
        l[h] = l[h] * c1 + lo * c2;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[h][j] = o[h][j] * c1 + oo[j] * c2;
        m[h] = mn;
      }
    }
  }

  // Merge the 4 wavefronts through LDS.
  __shared__ float s_o[4][HG][kD];
  __shared__ float s_m[4][HG], s_l[4][HG];
  __shared__ float s_f[64][HG];  // split weights for the final merge
  __shared__ float s_L[HG];
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < HG; ++h) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s_o[wave][h][dl * 8 + j] = o[h][j];
      if (dl == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();

  const int HGD = HG * kD;
  // Each thread owns HGD/256 outputs (one for HG <= 2).
  for (int t = threadIdx.x; t < HGD; t += 256) {
    const int oh = t / kD;
    const int od = t % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][oh]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = safe_exp2_diff(s_m[w][oh], M);
        L += f * s_l[w][oh];
        O += f * s_o[w][oh][od];
      }
    }
    if (p.nsplit == 1) {
      const float r = L > 0.f ? O / L : 0.f;
      p.out[((size_t)b * p.H + (size_t)kv * HG + oh) * kD + od] = f32_to_bf16(r);
    } else {
      float* part = p.part + (((size_t)b * p.KV + kv) * p.nsplit + split) * (HG * (kD + 2));
      part[oh * kD + od] = O;
      if (od == 0) {
        part[HGD + oh] = M;
        part[HGD + HG + oh] = L;
      }
    }
  }
  if (p.nsplit == 1) return;

  if (!arrive_is_last(p.cnt + (size_t)b * p.KV + kv, (unsigned)p.nsplit)) return;

  // Last workgroup of this (b, kv): merge the nsplit partials.
  const float* base = p.part + ((size_t)b * p.KV + kv) * p.nsplit * (HG * (kD + 2));
  const int ns = p.nsplit;
  __shared__ float s_red[4];
  for (int h = 0; h < HG; ++h) {
    // split weights f_s = exp2(m_s - M), L = sum f_s l_s
    float mloc = -INFINITY;
    for (int sidx = threadIdx.x; sidx < ns; sidx += 256)
      mloc = fmaxf(mloc, base[(size_t)sidx * (HG * (kD + 2)) + HGD + h]);
    mloc = wave_max(mloc);
    if (lane == 0) s_red[wave] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    float lloc = 0.f;
    for (int sidx = threadIdx.x; sidx < ns; sidx += 256) {
      const float* ps = base + (size_t)sidx * (HG * (kD + 2));
      const float ms = ps[HGD + h];
      const float f = (M == -INFINITY || ms == -INFINITY) ? 0.f : exp2f(ms - M);
      s_f[sidx][h] = f;
      lloc += f * ps[HGD + HG + h];
    }
    lloc = block_sum_256(lloc, s_red);
    if (threadIdx.x == 0) s_L[h] = lloc;
    __syncthreads();
  }
  for (int t = threadIdx.x; t < HGD; t += 256) {
    const int h = t / kD, d = t % kD;
    float O0 = 0.f, O1 = 0.f, O2 = 0.f, O3 = 0.f;
    int sidx = 0;
    for (; sidx + 4 <= ns; sidx += 4) {
      const float* ps = base + (size_t)sidx * (HG * (kD + 2)) + h * kD + d;
      const size_t S = HG * (kD + 2);
      O0 = fmaf(s_f[sidx][h], ps[0], O0);
      O1 = fmaf(s_f[sidx + 1][h], ps[S], O1);
      O2 = fmaf(s_f[sidx + 2][h], ps[2 * S], O2);
      O3 = fmaf(s_f[sidx + 3][h], ps[3 * S], O3);
    }
    for (; sidx < ns; ++sidx)
      O0 = fmaf(s_f[sidx][h], base[(size_t)sidx * (HG * (kD + 2)) + h * kD + d], O0);
    const float L = s_L[h];
    const float O = (O0 + O1) + (O2 + O3);
    const float r = L > 0.f ? O / L : 0.f;
    p.out[((size_t)b * p.H + (size_t)kv * HG + h) * kD + d] = f32_to_bf16(r);
  }
}

struct SplitPlan {
  int nsplit, chunk;
};

SplitPlan plan_split(int B, int KV, int max_ctx) {
  SplitPlan sp;
  const int target_wgs = 256;
  int ns = (target_wgs + B * KV - 1) / (B * KV);
  const int max_ns = (max_ctx + 63) / 64;
  if (ns > max_ns) ns = max_ns;
  if (ns > 64) ns = 64;
  if (ns < 1) ns = 1;
  int chunk = (max_ctx + ns - 1) / ns;
  chunk = ((chunk + 63) / 64) * 64;
  if (chunk < 64) chunk = 64;
  ns = (max_ctx + chunk - 1) / chunk;
  if (ns < 1) ns = 1;
  sp.nsplit = ns;
  sp.chunk = chunk;
  return sp;
}

size_t attn_ws_bytes(int B, int H, int KV, int max_ctx) {
  const SplitPlan sp = plan_split(B, KV, max_ctx);
  const int HG = H / KV;
  size_t part = (size_t)B * KV * sp.nsplit * HG * (kD + 2) * sizeof(float);
  part = (part + 255) & ~(size_t)255;
  return part + (size_t)B * KV * sizeof(unsigned int) + 256;
}

}  // namespace

extern "C" {

size_t iron_decode_attn_workspace(int B, int H, int KV, int D, int max_ctx) {
  if (B <= 0 || H <= 0 || KV <= 0 || D != kD || H % KV || max_ctx <= 0) return 0;
  return attn_ws_bytes(B, H, KV, max_ctx);
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
  if (HG != 1 && HG != 2 && HG != 4 && HG != 8)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: GQA group %d not in {1,2,4,8}", fn, HG);
  if (kv_st % 8 || kv_sh % 8 || kv_sb % 8 || !iron::aligned(k_cache, 16) ||
      !iron::aligned(v_cache, 16) || !iron::aligned(q, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: K/V/Q rows must be 16-byte aligned", fn);
  if (!ctx_len && (ctx_const < 0 || ctx_const > max_ctx))
    return iron::fail(IRON_ERR_SHAPE, "%s: ctx_const=%d outside [0, %d]", fn, ctx_const, max_ctx);
  const SplitPlan sp = plan_split(B, KV, max_ctx);
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
  p.chunk = sp.chunk;
  p.nsplit = sp.nsplit;
  p.scale_log2 = scale * 1.4426950408889634f;
  if (sp.nsplit > 1) {
    const size_t need = attn_ws_bytes(B, H, KV, max_ctx);
    if (!workspace || workspace_bytes < need)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                        need);
    if (!iron::aligned(workspace, 256))
      return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
    size_t part = (size_t)B * KV * sp.nsplit * HG * (kD + 2) * sizeof(float);
    part = (part + 255) & ~(size_t)255;
    p.part = (float*)workspace;
    p.cnt = (unsigned int*)((char*)workspace + part);
  }
  dim3 grid(sp.nsplit, KV, B);
  hipStream_t s = (hipStream_t)stream;
  switch (HG) {
    case 1: hipLaunchKernelGGL(decode_attn_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(decode_attn_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL(decode_attn_kernel<4>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(decode_attn_kernel<8>, grid, dim3(256), 0, s, p); break;
  }
  return iron::check_launch(fn);
}

}  // extern "C"
