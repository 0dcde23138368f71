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
// d = 64) serve every wavefront. Per key block a wavefront computes S^T = K Q^T per 16-key tile
// (each K operand read serves both query tiles): lane l then holds the scores of query l%16 for
// keys (l/16)*4 + i of the tile, which is exactly the B-operand layout of P^T for O^T = V^T P^T
// when a 32-key step takes its keys in the order (tile 2s: 4 keys, tile 2s+1: 4 keys) per lane
// quarter. In O^T's layout lane l also owns query l%16, so the softmax correction and the final
// division need no cross-lane exchange. Query blocks run latest (longest) first.
//
// Staging: K and V blocks go from memory straight into LDS (global_load_lds_dwordx4, no staging
// registers), both in their natural row-major layout with the 16-byte chunks of each row
// XOR-swizzled by row (conflict-free operand reads). The V^T operand is read with gfx950's
// transposing LDS load (ds_read_tr16_b64: within each 16 lanes, lane j receives element j & 3 of
// the 8 bytes that lanes 4k + j / 4 address, k = 0..3). Block i + 1 is loaded while block i is
// computed (two LDS halves each for K and V). Which of a wavefront's two tiles take part in a
// block is decided once per block (a wave-uniform branch between a two-tile and a one-tile copy
// of the block's code), not per MFMA: per-MFMA branches split the block into basic blocks the
// scheduler cannot interleave, and the values live across them spill.
//
// Two wavefronts share each SIMD (two workgroups per CU). A wavefront raises its priority
// (s_setprio 1) while it issues its P.V MFMAs, so the SIMD's other wavefront fills the MFMA's
// cycles with its softmax VALU work instead of both contending for the same phase.
#include <type_traits>

#include "common.h"
#include "internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef short s16x4 __attribute__((ext_vector_type(4)));

struct PrefillParams {
  const uint16_t* q;   // [B][H][S][D]
  const uint16_t* k;   // [B][KV][S][D]
  const uint16_t* v;
  uint16_t* o;         // [B][H][S][D]
  int B, H, KV, S;
  float scale_log2;    // scale * log2(e)
};

IRON_DEV bf16x8 as_bf16x8(const uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// One lane's 16 bytes from global memory (base + off bytes) into LDS at m0 + 16 * lane
// (global_load_lds_dwordx4; lds wave-uniform). Inline asm: seeing an LDS-DMA store, the compiler
// would wait for every one outstanding (vmcnt(0)) before any LDS read; the kernel orders the
// staging itself (s_waitcnt vmcnt(0) and a barrier once per block).
IRON_DEV void pf_dma16(const void* base, uint32_t off, uint32_t lds) {
  __asm__ volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(off), "s"(base), "s"(lds)
                   : "memory");
}

// The 16-byte chunk c of row r of a staged block lives at chunk c ^ swz(r) (NCH chunks a row):
// K rows by r (the 16 rows of an operand read hit 16 distinct chunks), V rows by 2r (the
// transposing read takes a chunk pair of 16 consecutive rows: pairs stay adjacent).
template <int NCH> IRON_DEV int swz_k(int r) { return r & (NCH - 1); }
template <int NCH> IRON_DEV int swz_v(int r) { return (2 * r) & (NCH - 1); }

// One block of KB keys (K or V) from rows kb0.. of a [S][D] slab into LDS: four instructions per
// thread; instruction i of wavefront w fills bytes i*4096 + w*1024 .. +1024 of the block, lane l
// its 16-byte chunk position (that offset + 16 l) % (2 D) of row (that offset + 16 l) / (2 D),
// loading the global chunk the swizzle maps there. Rows past S repeat row S - 1 (they lie past
// every query: the causal mask drops them).
template <int D, bool IS_V>
IRON_DEV void pf_dma_block(const uint16_t* slab, int kb0, int S, uint32_t lds_block, int wave,
                           int lane) {
  constexpr int NCH = D / 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int byte = i * 4096 + wave * 1024 + lane * 16;
    const int r = byte / (2 * D), p = (byte % (2 * D)) / 16;
    const int g = p ^ (IS_V ? swz_v<NCH>(r) : swz_k<NCH>(r));
    const int row = min(kb0 + r, S - 1);
    pf_dma16(slab, (uint32_t)(row * D + g * 8) * 2u,
             (uint32_t)__builtin_amdgcn_readfirstlane(lds_block + i * 4096 + wave * 1024));
  }
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
  constexpr int NCH = D / 8;           // 16-byte chunks per row
  constexpr int NKT = KB / 16;         // 16-key tiles per block
  constexpr int NKS = KB / 32;         // 32-key P.V steps per block
  constexpr int NJ = D / 32;           // 32-wide head-dim steps of Q K^T
  constexpr int ND = D / 16;           // 16-wide head-dim tiles of O
  constexpr int PW = 4 / HW;           // tile pairs per workgroup
  constexpr float kLazy = 8.f;         // how far the softmax reference may trail the maximum
  __shared__ __align__(16) uint16_t s_k[2][KB * D];
  __shared__ __align__(16) uint16_t s_v[2][KB * D];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
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
  const uint16_t* kslab = p.k + kvo;
  const uint16_t* vslab = p.v + kvo;

  // Q^T operands: lane l holds query row r0[t] + l%16 (clamped), d = 32 j + (l/16)*8 .. +8
  uint4 qf[2][NJ];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int qr = max(0, min(r0[t] + col, S - 1));  // pairs past the last one read row 0
    const uint16_t* qrow = p.q + (((size_t)b * p.H + head) * S + qr) * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) qf[t][j] = *(const uint4*)(qrow + 32 * j + quarter * 8);
  }

  // O^T accumulators: tile (t, dt) is 16 dims x 16 queries; lane l holds query r0[t] + l%16,
  // dims 16 dt + (l/16)*4 + i
  f32x4 o[2][ND];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f};  // this lane's share of query stats
  const float c = p.scale_log2;
  // tile t takes part in block kbi while the block starts at or before its last row
  auto active = [&](int kbi, int t) {
    return live && !(t == 0 && twin) && kbi * KB <= r0[t] + 15;
  };
  const uint32_t kbase = (uint32_t)(uintptr_t)&s_k[0][0], vbase = (uint32_t)(uintptr_t)&s_v[0][0];
  auto k_block = [&](int kbi) { return kbase + (uint32_t)((kbi & 1) * KB * D * 2); };
  auto v_block = [&](int kbi) { return vbase + (uint32_t)((kbi & 1) * KB * D * 2); };

  // S^T of block kbi for tiles T0..1 (K from its LDS half)
  auto qk = [&](auto t0c, int kbi, f32x4 (&st)[2][NKT]) {
    constexpr int T0 = decltype(t0c)::value;
    const uint16_t* kb = &s_k[kbi & 1][0];
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      const int r = 16 * kt + col;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int ch = (4 * j + quarter) ^ swz_k<NCH>(r);
        const bf16x8 a = as_bf16x8(*(const uint4*)&kb[r * D + ch * 8]);
#pragma unroll
        for (int t = T0; t < 2; ++t)
          st[t][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(qf[t][j]),
                                                              j ? st[t][kt] : zero, 0, 0, 0);
      }
    }
  };
  // The V^T operand of (32-key step ks, dim tile dt): lane (q, j) gets dims 16 dt + j of keys
  // 32 ks + 4 q + 0..3 and 32 ks + 16 + 4 q + 0..3, by two transposing reads in which lane s
  // addresses the 4 dims 16 dt + 4 (s & 3) .. +3 of key 32 ks + 4 q + s / 4 (+ 16).
  auto vt_operand = [&](const uint16_t* vb, int ks, int dt) {
    const int s = col;
    const int dcol = 16 * dt + 4 * (s & 3);
    bf16x4 h[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int r = 32 * ks + 16 * hh + 4 * quarter + (s >> 2);
      const int ch = (dcol >> 3) ^ swz_v<NCH>(r);
      const uint16_t* a = &vb[r * D + ch * 8 + (dcol & 7)];
      h[hh] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(const_cast<uint16_t*>(a))));
    }
    return __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // max over the four lane quarters (lanes l, l ^ 16, l ^ 32, l ^ 48) by two lane swaps:
  // v_permlane16_swap exchanges the odd 16-lane rows of its first operand with the even rows of
  // its second, v_permlane32_swap the upper half of the first with the lower half of the second
  auto quarter_max = [](float x) __attribute__((always_inline)) {
    const uint32_t u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t w = __float_as_uint(x);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
  };
  // the online softmax of block kbi's scores for tiles T0..1, then O^T += V^T P^T (V from its
  // LDS half)
  auto softmax_pv = [&](auto t0c, int kbi, f32x4 (&st)[2][NKT]) {
    constexpr int T0 = decltype(t0c)::value;
    const uint16_t* vb = &s_v[kbi & 1][0];
    const int kb0 = kbi * KB;
    bf16x8 pb[2][NKS];
    float mx[2];
#pragma unroll
    for (int t = T0; t < 2; ++t) {
      const bool diag = kb0 + KB - 1 > r0[t];  // some key may lie past some query: mask
      if (diag) {  // wave-uniform: only the blocks that reach past a query need the mask
        // key kb0 + 16 kt + 4 quarter + i lies past query r0[t] + col
        const int lim = r0[t] + col - kb0 - 4 * quarter;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * kt + i > lim) st[t][kt][i] = -INFINITY;
      }
      float x = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) x = fmaxf(x, st[t][kt][i]);
      mx[t] = quarter_max(x) * c;  // the block's maximum in the exp2 domain (scale > 0)
    }
    // The probabilities are taken against a reference m[t] that may trail the running maximum
    // by up to kLazy (so they reach 2^kLazy at most: no overflow in fp32 or bf16, and the final
    // division by the row sum cancels the reference). The reference moves, and O and the row sums
    // are rescaled, only when some lane's maximum passes it by more: after the first blocks that
    // is rare (the rescale costs 32 multiplies per tile, twice the block's 16 scores per lane).
    // m = -inf before block 0, and every query has a key in block 0, so the first block always
    // sets it.
    bool grow = false;
#pragma unroll
    for (int t = T0; t < 2; ++t) grow |= mx[t] > m[t] + kLazy;
    if (__ballot(grow)) {
#pragma unroll
      for (int t = T0; t < 2; ++t) {
        const float mn = fmaxf(m[t], mx[t]);
        const float corr = __builtin_amdgcn_exp2f(m[t] - mn);  // 0 on the first block
        m[t] = mn;
        lsum[t] *= corr;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[t][dt][i] *= corr;
      }
    }
#pragma unroll
    for (int t = T0; t < 2; ++t) {
      const float mn = m[t];
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
      lsum[t] += ps;
    }
    // O^T += V^T P^T; each V^T operand serves both query tiles
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const bf16x8 a = vt_operand(vb, ks, dt);
#pragma unroll
        for (int t = T0; t < 2; ++t)
          o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[t][ks], o[t][dt], 0, 0, 0);
      }
    __builtin_amdgcn_s_setprio(0);
  };
  // start of iteration kbi (after the previous barrier): block kbi + 1 into the halves block
  // kbi - 1 was read from
  auto fetch = [&](int kbi) {
    if (kbi + 1 < nkb) {
      pf_dma_block<D, false>(kslab, (kbi + 1) * KB, S, k_block(kbi + 1), wave, lane);
      pf_dma_block<D, true>(vslab, (kbi + 1) * KB, S, v_block(kbi + 1), wave, lane);
    }
  };
  // end of iteration: this thread's block loads have landed, then every thread's have
  auto land = [&]() {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  pf_dma_block<D, false>(kslab, 0, S, k_block(0), wave, lane);
  pf_dma_block<D, true>(vslab, 0, S, v_block(0), wave, lane);
  land();
  for (int kbi = 0; kbi < nkb; ++kbi) {
    f32x4 st[2][NKT];
    fetch(kbi);
    // tile 0 active implies tile 1 active (its rows come later): one branch per block
    if (active(kbi, 0)) {
      qk(std::integral_constant<int, 0>(), kbi, st);
      softmax_pv(std::integral_constant<int, 0>(), kbi, st);
    } else if (active(kbi, 1)) {
      qk(std::integral_constant<int, 1>(), kbi, st);
      softmax_pv(std::integral_constant<int, 1>(), kbi, st);
    }
    land();
  }

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
