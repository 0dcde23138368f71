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
// Mapping: a wavefront owns 32 query rows (two 16-row tiles) of one head; a workgroup (4
// wavefronts) owns 4 heads of one GQA group for the same rows (or, for groups smaller than 4,
// more query blocks), so the K/V blocks it stages in LDS (16 KiB each: 64 keys at d = 128, 128 at
// d = 64; double buffered, V transposed) serve every wavefront. Per key block a wavefront computes
// S^T = K Q^T per 16-key tile (each K operand read serves both query tiles): lane l then holds the
// scores of query l%16 for keys (l/16)*4 + i of the tile, which is exactly the B-operand layout of
// P^T for O^T = V^T P^T when a 32-key step takes its keys in the order (tile 2s: 4 keys, tile
// 2s+1: 4 keys) per lane quarter; the V^T operand reads those keys with two 8-byte LDS reads. In
// O^T's layout lane l also owns query l%16, so the softmax correction and the final division need
// no cross-lane exchange. Query blocks run latest (longest) first.
#include "common.h"
#include "internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;


struct PrefillParams {
  const uint16_t* q;   // [B][H][S][D]
  const uint16_t* k;   // [B][KV][S][D]
  const uint16_t* v;
  uint16_t* o;         // [B][H][S][D]
  int B, H, KV, S;
  float scale_log2;    // scale * log2(e)
};

IRON_DEV bf16x8 as_bf16x8(const uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Staging of one key block (keys clamped to the sequence). K rows go to LDS as they are; V goes
// transposed, the 4 keys of one dim in one 8-byte write.
// The staging registers of one key block (four K and four V slices of 8 dims), as native vectors
// so that they stay in registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
struct KVRegs {
  u32x4 k0, k1, k2, k3, v0, v1, v2, v3;
};

// Staging coordinates: K is copied by thread -> (keys 4 kg .. +4, dims kd .. +8) with the dims
// fastest across lanes (whole rows per 16 lanes: conflict-free row writes); V by thread -> (keys
// 4 vg .. +4, dims vd .. +8) with the key groups fastest across lanes, so that the 8-byte V^T
// writes of a wavefront spread over the LDS banks.
struct StageIdx {
  int kg, kd, vg, vd;
};

template <int D, int KB>
IRON_DEV StageIdx stage_idx(int tid) {
  constexpr int TPG = D / 8;   // threads per key row
  constexpr int NG = KB / 4;   // key groups per block
  return StageIdx{tid / TPG, (tid % TPG) * 8, tid % NG, (tid / NG) * 8};
}

// The K and V of one (sequence, KV head) as raw buffers of S rows: a block's loads take its byte
// offset as the scalar operand and each thread's fixed offset (rows 4 g .. +3 of the block,
// dims d .. +8; the row steps are immediates), so a block costs no address arithmetic. Keys past
// S (the last block at D = 64 when S is not a multiple of 128) read as zero: they lie past every
// query, so the causal mask drops their scores and their probabilities are zero.
struct KVSrc {
  __amdgpu_buffer_rsrc_t k, v;
  int koff, voff;  // this thread's byte offsets within a block
};

template <int D, int KB>
IRON_DEV void pf_gload(const KVSrc& src, int kb, KVRegs& r) {
  const int sb = kb * KB * D * 2;
  r.k0 = __builtin_amdgcn_raw_buffer_load_b128(src.k, src.koff, sb, 0);
  r.k1 = __builtin_amdgcn_raw_buffer_load_b128(src.k, src.koff + D * 2, sb, 0);
  r.k2 = __builtin_amdgcn_raw_buffer_load_b128(src.k, src.koff + 2 * D * 2, sb, 0);
  r.k3 = __builtin_amdgcn_raw_buffer_load_b128(src.k, src.koff + 3 * D * 2, sb, 0);
  r.v0 = __builtin_amdgcn_raw_buffer_load_b128(src.v, src.voff, sb, 0);
  r.v1 = __builtin_amdgcn_raw_buffer_load_b128(src.v, src.voff + D * 2, sb, 0);
  r.v2 = __builtin_amdgcn_raw_buffer_load_b128(src.v, src.voff + 2 * D * 2, sb, 0);
  r.v3 = __builtin_amdgcn_raw_buffer_load_b128(src.v, src.voff + 3 * D * 2, sb, 0);
}

// dims dc + 2w (low halves) and dc + 2w + 1 (high halves) of the 4 keys, one 8-byte write each
IRON_DEV void pf_vt_pair(uint16_t* lo_row, uint16_t* hi_row, uint32_t a0, uint32_t a1, uint32_t a2,
                         uint32_t a3) {
  *(uint2*)lo_row = make_uint2((a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16));
  *(uint2*)hi_row = make_uint2((a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u));
}

template <int D, int KB>
IRON_DEV void pf_lstore(uint16_t (*s_k)[D + 8], uint16_t (*s_vt)[KB + 4], const StageIdx& x,
                        const KVRegs& r) {
  *(u32x4*)&s_k[4 * x.kg][x.kd] = r.k0;
  *(u32x4*)&s_k[4 * x.kg + 1][x.kd] = r.k1;
  *(u32x4*)&s_k[4 * x.kg + 2][x.kd] = r.k2;
  *(u32x4*)&s_k[4 * x.kg + 3][x.kd] = r.k3;
  const int c = 4 * x.vg, dc = x.vd;
  pf_vt_pair(&s_vt[dc][c], &s_vt[dc + 1][c], r.v0.x, r.v1.x, r.v2.x, r.v3.x);
  pf_vt_pair(&s_vt[dc + 2][c], &s_vt[dc + 3][c], r.v0.y, r.v1.y, r.v2.y, r.v3.y);
  pf_vt_pair(&s_vt[dc + 4][c], &s_vt[dc + 5][c], r.v0.z, r.v1.z, r.v2.z, r.v3.z);
  pf_vt_pair(&s_vt[dc + 6][c], &s_vt[dc + 7][c], r.v0.w, r.v1.w, r.v2.w, r.v3.w);
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

// Round-to-nearest-even of two fp32 values to packed bf16 (v_cvt_pk_bf16_f32).
IRON_DEV uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}

// HW = query heads per workgroup (min(group, 4)); the 4 wavefronts are HW heads x (4 / HW) query
// tile pairs. Query tiles are 16 rows; pair i is tiles i and NT - 1 - i (NT = S / 16), so every
// pair costs the same number of key blocks and the workgroups stay balanced under the causal mask.
template <int D, int HW>
__global__ __launch_bounds__(256, 2) void prefill_attn_kernel(PrefillParams p) {
  constexpr int KB = 8192 / D;         // keys per block (16 KiB of K)
  constexpr int NKT = KB / 16;         // 16-key tiles per block
  constexpr int NKS = KB / 32;         // 32-key P.V steps per block
  constexpr int NJ = D / 32;           // 32-wide head-dim steps of Q K^T
  constexpr int ND = D / 16;           // 16-wide head-dim tiles of O
  constexpr int PW = 4 / HW;           // tile pairs per workgroup
  __shared__ __align__(16) uint16_t s_k[2][KB][D + 8];
  // V^T rows of KB + 4 elements (34 dwords at D = 128): the 8-byte reads of 16 consecutive rows
  // hit distinct banks (at KB + 8 rows r and r + 8 shared them: 3x the bank-conflict cycles)
  __shared__ __align__(16) uint16_t s_vt[2][D][KB + 4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int quarter = lane >> 4, col = lane & 15;
  const int HG = p.H / p.KV;
  // 1-D grid, head groups fastest: consecutive workgroups go to consecutive XCDs, so with a
  // multiple of 8 groups every workgroup of one (sequence, KV head) runs on the same XCD and its
  // K/V blocks stay in that XCD's L2
  const int ngroups = p.B * p.KV * (HG / HW);
  const int grp = blockIdx.x % ngroups, pblk = blockIdx.x / ngroups;
  const int kv = grp % p.KV;
  const int bh = grp / p.KV;
  const int b = bh / (HG / HW), hsub = bh % (HG / HW);
  const int head = kv * HG + hsub * HW + wave % HW;
  const int S = p.S;
  const int NT = S / 16, npairs = (NT + 1) / 2;
  const int pair = pblk * PW + wave / HW;                // this wavefront's tile pair
  const bool live = pair < npairs;
  // tile t's first row (t = 0 light, t = 1 heavy; with an odd tile count the middle tile pairs
  // with itself and the copy is skipped)
  const int r0[2] = {16 * pair, 16 * (NT - 1 - pair)};
  const bool twin = live && r0[0] == r0[1];
  // key blocks the workgroup needs: up to the heavy tile of its lightest pair
  const int pmin = pblk * PW;
  const int nkb = (16 * (NT - 1 - pmin) + 15) / KB + 1;

  const size_t kvo = ((size_t)b * p.KV + kv) * S * D;

  // Q^T operands: lane l holds query row r0[t] + l%16 (clamped), d = 32 j + (l/16)*8 .. +8
  uint4 qf[2][NJ];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int qr = max(0, min(r0[t] + col, S - 1));  // pairs past the last one read row 0
    const uint16_t* qrow = p.q + (((size_t)b * p.H + head) * S + qr) * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) qf[t][j] = *(const uint4*)(qrow + 32 * j + quarter * 8);
  }

  const StageIdx sx = stage_idx<D, KB>(tid);
  KVSrc src;
  src.k = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.k + kvo), 0, S * D * 2,
                                            kBufferDword3);
  src.v = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.v + kvo), 0, S * D * 2,
                                            kBufferDword3);
  src.koff = (4 * sx.kg * D + sx.kd) * 2;
  src.voff = (4 * sx.vg * D + sx.vd) * 2;
  KVRegs ra, rb;  // two register sets: block i + 2 is fetched while block i + 1 waits

  // O^T accumulators: tile (t, dt) is 16 dims x 16 queries; lane l holds query r0[t] + l%16,
  // dims 16 dt + (l/16)*4 + i
  f32x4 o[2][ND];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f};  // this lane's share of query stats
  const float c = p.scale_log2;

  pf_gload<D, KB>(src, 0, ra);
  if (nkb > 1) pf_gload<D, KB>(src, 1, rb);
  pf_lstore<D, KB>(s_k[0], s_vt[0], sx, ra);
  __syncthreads();
  // iteration kbi: fetch block kbi + 2 into the set that held block kbi, compute block kbi, then
  // stage block kbi + 1 (fetched an iteration earlier) into the other LDS buffer
  auto iteration = [&](int kbi, KVRegs& fetch, KVRegs& stage) {
    const int buf = kbi & 1;
    const int kb0 = kbi * KB;
    // unconditional (past the last block it re-reads it): a load in a branch would make the
    // compiler's wait before the staging below count it as the youngest load, draining the fetch
    pf_gload<D, KB>(src, min(kbi + 2, nkb - 1), fetch);
    // tile t takes part while the block starts at or before its last row (wave-uniform)
    const bool act[2] = {live && !twin && kb0 <= r0[0] + 15, live && kb0 <= r0[1] + 15};
    f32x4 st[2][NKT];
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const bf16x8 a = as_bf16x8(*(const uint4*)&s_k[buf][16 * kt + col][32 * j + quarter * 8]);
        if (act[0])
          st[0][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(qf[0][j]),
                                                              j ? st[0][kt] : zero, 0, 0, 0);
        if (act[1])
          st[1][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(qf[1][j]),
                                                              j ? st[1][kt] : zero, 0, 0, 0);
      }
    }
    bf16x8 pb[2][NKS];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (!act[t]) continue;
      const int qi = r0[t] + col;
      const bool diag = kb0 + KB - 1 > r0[t];  // some key may lie past some query: mask
      if (diag) {  // wave-uniform: only the blocks that reach past a query need the mask
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kb0 + 16 * kt + quarter * 4 + i > qi) st[t][kt][i] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[t][kt][i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // running maximum in the exp2 domain (scale > 0, so the raw maximum maps to it)
      const float mn = fmaxf(m[t], mx * c);  // finite: every query has a key in block 0
      const float corr = __builtin_amdgcn_exp2f(m[t] - mn);  // m = -inf on the first block
      m[t] = mn;
      float ps = 0.f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float e[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            e[i] = __builtin_amdgcn_exp2f(fmaf(st[t][2 * ks + h][i], c, -mn));
            ps += e[i];
          }
          w[2 * h] = pack_bf16(e[0], e[1]);
          w[2 * h + 1] = pack_bf16(e[2], e[3]);
        }
        pb[t][ks] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
      }
      lsum[t] = lsum[t] * corr + ps;
      if (__ballot(corr != 1.f)) {  // no lane's maximum moved: every factor is exactly 1
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[t][dt][i] *= corr;
      }
    }
    // O^T += V^T P^T; each V^T operand serves both query tiles
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const uint16_t* vr = &s_vt[buf][16 * dt + col][32 * ks + quarter * 4];
        const uint2 v0 = *(const uint2*)vr;
        const uint2 v1 = *(const uint2*)(vr + 16);
        const bf16x8 a = as_bf16x8(make_uint4(v0.x, v0.y, v1.x, v1.y));
        if (act[0]) o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[0][ks], o[0][dt], 0, 0, 0);
        if (act[1]) o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[1][ks], o[1][dt], 0, 0, 0);
      }
    if (kbi + 1 < nkb) pf_lstore<D, KB>(s_k[buf ^ 1], s_vt[buf ^ 1], sx, stage);
    __syncthreads();
  };
  int kbi = 0;
  for (; kbi + 1 < nkb; kbi += 2) {  // no branch around an iteration's loads inside the loop
    iteration(kbi, ra, rb);
    iteration(kbi + 1, rb, ra);
  }
  if (kbi < nkb) iteration(kbi, ra, rb);

  // row sums: the four lane quarters hold disjoint keys of the same query
  if (!live) return;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t == 0 && twin) continue;
    float l = lsum[t];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.f / l;
    uint16_t* orow = p.o + (((size_t)b * p.H + head) * S + r0[t] + col) * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
      *(uint2*)(orow + 16 * dt + quarter * 4) =
          make_uint2(pack_bf16(o[t][dt][0] * inv, o[t][dt][1] * inv),
                     pack_bf16(o[t][dt][2] * inv, o[t][dt][3] * inv));
  }
}

template <int D>
void launch_d(const PrefillParams& p, int B, int HG, hipStream_t s) {
  const int HW = HG >= 4 ? 4 : HG;
  const int PW = 4 / HW;
  const int npairs = (p.S / 16 + 1) / 2;
  dim3 grid((unsigned)((npairs + PW - 1) / PW) * B * p.KV * (HG / HW));
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
  p.B = B;
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
