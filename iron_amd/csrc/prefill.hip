// Causal prefill multi-head attention (GQA) on MFMA: O = softmax(Q K^T * scale, causal) V.
//
// Reference: MHA (iron/operators/mha/op.py:20-153; golden iron/operators/mha/reference.py:27-94,
// torch SDPA with is_causal=True, scale 1/sqrt(d), K/V heads shared by H/KV query heads via
// repeat_interleave). The reference kernel supports d = 64; this one d = 64 and 128 (Qwen3-8B).
//
// Arithmetic (flash-attention forward): scores in fp32 from bf16 MFMAs, an online softmax with
// exp2 in fp32, probabilities rounded to bf16 for the P V product (as the reference's AIE kernels
// do), fp32 accumulation, one division by the row sum and one bf16 rounding of the output.
//
// Mapping: a wavefront owns 16 query rows of one head; a workgroup (4 wavefronts) owns 4 heads of
// one GQA group for the same 16 rows (or, for groups smaller than 4, more query blocks), so the
// 32-key K/V blocks it stages in LDS (double buffered) serve every wavefront. Per key block a
// wavefront computes S^T = K Q^T (two 16-key tiles, D/32 v_mfma_f32_16x16x32_bf16 each): lane l
// then holds the scores of query l%16 for keys (l/16)*4 + i of each tile, which is exactly the
// A-operand layout of P for the P V product when its 32 k-slots take the keys in the order
// (tile 0: 4 keys, tile 1: 4 keys) per lane quarter; V is staged transposed so the B operand
// reads those keys with two 8-byte LDS reads. Row statistics of query q live in the lanes with
// l%16 == q; the output tiles (rows (l/16)*4 + i) fetch them with cross-lane shuffles.
#include "common.h"
#include "internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kQB = 16;   // query rows per wavefront
constexpr int kKB = 32;   // keys per block

struct PrefillParams {
  const uint16_t* q;   // [B][H][S][D]
  const uint16_t* k;   // [B][KV][S][D]
  const uint16_t* v;
  uint16_t* o;         // [B][H][S][D]
  int H, KV, S;
  float scale_log2;    // scale * log2(e)
};

IRON_DEV bf16x8 as_bf16x8(const uint4 u) { return __builtin_bit_cast(bf16x8, u); }

IRON_DEV uint16_t f32_to_bf16_rne(float f) { return f32_to_bf16(f); }

// HW = query heads per workgroup (min(group, 4)); the 4 wavefronts are HW heads x (4 / HW) query
// blocks.
template <int D, int HW>
__global__ __launch_bounds__(256) void prefill_attn_kernel(PrefillParams p) {
  constexpr int QBW = 4 / HW;          // query blocks per workgroup
  constexpr int QT = kQB * QBW;        // query rows per workgroup
  constexpr int KROW = D + 8;          // padded LDS row of K (bf16)
  constexpr int VROW = kKB + 8;        // padded LDS row of V^T (bf16)
  constexpr int ND = D / 16;           // output d tiles
  __shared__ __align__(16) uint16_t s_k[2][kKB][KROW];
  __shared__ __align__(16) uint16_t s_vt[2][D][VROW];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int HG = p.H / p.KV;
  const int kv = blockIdx.y;
  const int b = blockIdx.z / (HG / HW), hsub = blockIdx.z % (HG / HW);
  const int head = kv * HG + hsub * HW + wave % HW;
  const int qw0 = blockIdx.x * QT + (wave / HW) * kQB;  // this wavefront's first query row
  const int q_last = blockIdx.x * QT + QT - 1;          // the workgroup's last query row
  const int nkb = q_last / kKB + 1;                     // key blocks the workgroup needs
  const int S = p.S;

  const uint16_t* kbase = p.k + ((size_t)b * p.KV + kv) * S * D;
  const uint16_t* vbase = p.v + ((size_t)b * p.KV + kv) * S * D;

  // Q^T operand: lane l holds q row qw0 + l%16, d = 32j + (l/16)*8 .. +8
  uint4 qf[D / 32];
  {
    const uint16_t* qrow = p.q + (((size_t)b * p.H + head) * S + qw0 + (lane & 15)) * D;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) qf[j] = *(const uint4*)(qrow + 32 * j + (lane >> 4) * 8);
  }

  // staging of one key block: thread -> key tid / (256/32), D/8 columns split over the rest
  constexpr int TPK = 256 / kKB;        // threads per key row (8)
  constexpr int EPT = D / TPK;          // elements per thread (16 for D=128, 8 for D=64)
  const int skey = tid / TPK, scol = (tid % TPK) * EPT;
  static_assert(EPT == 8 || EPT == 16, "one or two 16-byte chunks per thread");
  uint4 rk0, rk1, rv0, rv1;
  const size_t soff = (size_t)skey * D + scol;
#define PREFILL_GLOAD(kb_)                                                                     \
  do {                                                                                         \
    const size_t o_ = (size_t)(kb_) * kKB * D + soff;                                          \
    rk0 = *(const uint4*)(kbase + o_);                                                         \
    rv0 = *(const uint4*)(vbase + o_);                                                         \
    if (EPT == 16) {                                                                           \
      rk1 = *(const uint4*)(kbase + o_ + 8);                                                   \
      rv1 = *(const uint4*)(vbase + o_ + 8);                                                   \
    }                                                                                          \
  } while (0)
#define PREFILL_VT(buf_, c_, u_)                                                               \
  do {                                                                                         \
    const uint32_t w_[4] = {(u_).x, (u_).y, (u_).z, (u_).w};                                   \
    _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_) {                                         \
      s_vt[(buf_)][(c_) + 2 * j_][skey] = (uint16_t)(w_[j_] & 0xffffu);                        \
      s_vt[(buf_)][(c_) + 2 * j_ + 1][skey] = (uint16_t)(w_[j_] >> 16);                        \
    }                                                                                          \
  } while (0)
#define PREFILL_LSTORE(buf_)                                                                   \
  do {                                                                                         \
    *(uint4*)&s_k[(buf_)][skey][scol] = rk0;                                                   \
    PREFILL_VT(buf_, scol, rv0);                                                               \
    if (EPT == 16) {                                                                           \
      *(uint4*)&s_k[(buf_)][skey][scol + 8] = rk1;                                             \
      PREFILL_VT(buf_, scol + 8, rv1);                                                         \
    }                                                                                          \
  } while (0)

  f32x4 o[ND];
#pragma unroll
  for (int t = 0; t < ND; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;  // statistics of query qw0 + lane%16 (this lane's share)
  const int qi = qw0 + (lane & 15);

  PREFILL_GLOAD(0);
  PREFILL_LSTORE(0);
  __syncthreads();
  for (int kbi = 0; kbi < nkb; ++kbi) {
    const int buf = kbi & 1;
    if (kbi + 1 < nkb) PREFILL_GLOAD(kbi + 1);
    const int kb0 = kbi * kKB;
    if (kb0 <= qw0 + kQB - 1) {  // this wavefront has unmasked keys in the block
      // S^T tiles: rows = keys kb0 + 16t + l%16 (A operand from LDS), columns = queries
      f32x4 st[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
          const bf16x8 a =
              as_bf16x8(*(const uint4*)&s_k[buf][16 * t + (lane & 15)][32 * j + (lane >> 4) * 8]);
          st[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(qf[j]), st[t], 0, 0, 0);
        }
      }
      // scale (log2 domain), causal mask, block maximum of query qi across the lane quarters
      float sv[2][4];
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb0 + 16 * t + (lane >> 4) * 4 + i;
          const float v = key <= qi ? st[t][i] * p.scale_log2 : -INFINITY;
          sv[t][i] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m, mx);  // finite: key kb0 <= qw0 <= qi is always valid
      const float corr = exp2f(m - mn);  // m = -inf on the first block -> 0
      m = mn;
      float ps = 0.f;
      bf16x8 pa;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = exp2f(sv[t][i] - mn);
          ps += e;
          pa[4 * t + i] = __builtin_bit_cast(__bf16, f32_to_bf16_rne(e));
        }
      lsum = lsum * corr + ps;
      // rescale the output rows (l/16)*4 + i with their queries' corrections
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c = __shfl(corr, (lane >> 4) * 4 + i);
#pragma unroll
        for (int t = 0; t < ND; ++t) o[t][i] *= c;
      }
      // O += P V: B operand = V^T[d][keys (l/16)*4 .. +4 of each tile]
#pragma unroll
      for (int t = 0; t < ND; ++t) {
        const uint16_t* vr = &s_vt[buf][16 * t + (lane & 15)][(lane >> 4) * 4];
        const uint2 v0 = *(const uint2*)vr;
        const uint2 v1 = *(const uint2*)(vr + 16);
        const bf16x8 bv = as_bf16x8(make_uint4(v0.x, v0.y, v1.x, v1.y));
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, bv, o[t], 0, 0, 0);
      }
    }
    if (kbi + 1 < nkb) PREFILL_LSTORE(buf ^ 1);
    __syncthreads();
  }

#undef PREFILL_GLOAD
#undef PREFILL_VT
#undef PREFILL_LSTORE
  // row sums: every lane quarter holds part of query qi's sum
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  uint16_t* obase = p.o + (((size_t)b * p.H + head) * S + qw0) * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (lane >> 4) * 4 + i;
    const float inv = 1.f / __shfl(lsum, r);
#pragma unroll
    for (int t = 0; t < ND; ++t)
      obase[(size_t)r * D + 16 * t + (lane & 15)] = f32_to_bf16_rne(o[t][i] * inv);
  }
}

template <int D>
void launch_d(const PrefillParams& p, int B, int HG, hipStream_t s) {
  const int HW = HG >= 4 ? 4 : HG;
  const int QT = kQB * (4 / HW);
  dim3 grid(p.S / QT, p.KV, B * (HG / HW));
  switch (HW) {
    case 1: hipLaunchKernelGGL((prefill_attn_kernel<D, 1>), grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL((prefill_attn_kernel<D, 2>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((prefill_attn_kernel<D, 4>), grid, dim3(256), 0, s, p); break;
  }
}

}  // namespace

extern "C" {

int iron_prefill_attn(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int B,
                      int H, int KV, int S, int D, float scale, void* stream) {
  iron::clear_error();
  const char* fn = "iron_prefill_attn";
  if (!q || !k || !v || !o) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  if (B <= 0 || H <= 0 || KV <= 0 || S <= 0 || H % KV)
    return iron::fail(IRON_ERR_SHAPE, "%s: bad shape B=%d H=%d KV=%d S=%d", fn, B, H, KV, S);
  if (D != 64 && D != 128)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: head_dim %d (64 or 128)", fn, D);
  if (S % 64) return iron::fail(IRON_ERR_SHAPE, "%s: S=%d must be padded to 64", fn, S);
  const int HG = H / KV;
  if (HG != 1 && HG != 2 && HG % 4)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: GQA group %d not 1, 2 or a multiple of 4", fn,
                      HG);
  if (!iron::aligned(q, 16) || !iron::aligned(k, 16) || !iron::aligned(v, 16) ||
      !iron::aligned(o, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: tensors must be 16-byte aligned", fn);
  PrefillParams p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.H = H;
  p.KV = KV;
  p.S = S;
  p.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = (hipStream_t)stream;
  if (D == 128) launch_d<128>(p, B, HG, s);
  else launch_d<64>(p, B, HG, s);
  return iron::check_launch(fn);
}

}  // extern "C"
