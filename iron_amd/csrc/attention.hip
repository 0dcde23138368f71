// GQA decode attention (one query token per sequence) over a bf16 KV cache: split-K across
// workgroups (flash-decoding), the last split of each (sequence, head group) to finish merging
// the group's partials in the same launch (arrival counters in the workspace). A fused variant also performs the QKV head's
// per-head epilogue (QK RMSNorm, RoPE, KV-cache append) so that the QKV GEMV output feeds
// attention directly.
//
// Reference: DecodeAttention (iron/operators/decode_attn/op.py:20-181), kernels
// aie_kernels/aie2p/decode_attn.cc:117-311 (scores with scale log2(e)/sqrt(D), online softmax over
// KV blocks, finalize out/l with l == 0 -> 0), golden iron/operators/decode_attn/reference.py:
// 26-38 (kv = h*KV//H). Fused epilogue: QKVHeadDataParallelOurs (qkv_head_dp/op_ours.py:31-262),
// golden qkv_head_dp/reference.py:13-33 (rms_norm/reference.py:8-17, rope/reference.py:118-154).
//
// Arithmetic: the exact value of the golden, o = sum_j e^(s_j - m) v_j / sum_j e^(s_j - m) with
// s_j = (q . k_j) / sqrt(D), evaluated in fp64 (scores, exponentials, sums, accumulation) and
// rounded once to bf16. The exp2/log2(e) form of the reference is the same function.
//
// Mapping: grid (split, kv * head_groups, b), 256 threads = 4 wavefronts. A tile is 64 tokens:
// lane l of wavefront w works on tokens t0 + 16u + 4w + l/16 (u = 0..3) and on head dims
// [8*(l%16), +8), so one 128-bit load per lane reads 4 consecutive K (or V) rows = 1 KiB per
// wavefront instruction, and HB query heads of the GQA group share every K/V load. The softmax
// offset of a tile is the workgroup-wide maximum (one LDS exchange), so the token rows and the
// wavefronts hold partial sums under the same offset and combine by plain addition. A row's lanes
// split the tile's exponentials between them (one exp per (token, head)) and share them with DPP
// row broadcasts. The last split to finish merges (merge_last).
//
// With one sequence (B == 1) the first tile's K/V loads are issued before the context length is
// known (bounded by max_ctx, masked afterwards), which takes the length's load off the critical
// path; with several sequences the length is read first so that short sequences read nothing
// beyond their context.
#include <mutex>
#include <type_traits>
#include <utility>

#include "attn_core.h"
#include "common.h"
#include "internal.h"

namespace {

using namespace iron::dev;

constexpr int kD = 128;
constexpr int kTile = 64;  // 4 waves x 4 rows x 4 unrolled groups
constexpr int kMaxSplit = 256;  // the merge kernels hold one split weight per thread pair
// Arrival counters of the in-kernel merge at the front of a split workspace: one per (sequence,
// KV head, head group). Zero before the first call; the last split to arrive resets its counter,
// so every call leaves the block zero.
// Each counter has a 128-byte line of its own: the splits of different groups arrive at about the
// same time, and device-scope atomics on one line serialise.
constexpr size_t kAttnCtrBytes = 16384;
constexpr int kAttnCtrStride = 32;  // words
constexpr int kAttnCtrs = (int)(kAttnCtrBytes / sizeof(unsigned int)) / kAttnCtrStride;

struct AttnParams {
  const uint16_t* q;       // [B][H][D] (plain mode)
  // fused mode: q and the current token's K/V come from the raw QKV GEMV output
  const uint16_t* raw;     // [B][(H + 2 KV) * D]
  const uint16_t* n_qn;
  const uint16_t* n_kn;
  const uint16_t* ang;     // [B][D] angle rows (fused mode)
  const int32_t* pos;      // [B]
  double eps;
  uint16_t* k;
  uint16_t* v;
  long long sb, sh, st;
  const int32_t* ctx_len;  // plain mode
  int ctx_const;
  int max_ctx;
  int spec;                // issue the first tile before the context length is known
  uint16_t* out;
  int H, KV, HG, HB;       // heads, kv heads, GQA group, heads per workgroup
  int chunk, nsplit;
  double scale;
  float scale2;            // scale * log2(e) (fp32 kernels: scores in the exp2 domain)
  void* part;              // split partials, rows of D + 2 fp64 (or fp32): o (unnormalised), m, l
  unsigned int* ctr;       // the in-kernel merge's arrival counters, or null (merge kernel)
  int bal;                 // balanced split assignment (balanced_slot)
  int nslot;               // nsplit * B: the workgroups of one head group
};

// Workgroup coordinates: grid (split, kv * head_groups, b), 256 threads.
struct AttnCoords {
  int b, kv, hg, h0, wave, row, dl, t_begin, t_lim;
};

template <int HB>
IRON_DEV AttnCoords attn_coords(const AttnParams& p) {
  AttnCoords c;
  const int groups = p.HG / HB;
  c.b = blockIdx.z;
  c.kv = blockIdx.y / groups;
  c.hg = blockIdx.y % groups;
  c.h0 = c.kv * p.HG + c.hg * HB;  // first query head of this workgroup
  c.wave = threadIdx.x >> 6;
  c.row = (threadIdx.x & 63) >> 4;
  c.dl = threadIdx.x & 15;
  c.t_begin = blockIdx.x * p.chunk;
  c.t_lim = min(p.max_ctx, c.t_begin + p.chunk);
  return c;
}

IRON_DEV int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

IRON_DEV int wave_scan_int(int v) {  // inclusive prefix sum over the lanes
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

// Balanced split assignment (B > 1 with per-sequence lengths and the in-kernel merge). The
// nslot = nsplit * B workgroups of a head group are dealt to the sequences in proportion to their
// 64-token tiles instead of nsplit each: with T tiles in all, sequence b gets
//   n_b = min(1 + floor((nslot - B) tiles_b / T), tiles_b, kMaxSplit)
// slots (one for an empty sequence), consecutive from slot0_b = sum of the earlier n_b', and its
// tiles are cut into runs of ceil(tiles_b / n_b) tiles -- n_b' <= n_b runs, the last shorter. The
// longest sequence of a ragged batch then spans about its share of the chip instead of nsplit
// workgroups. Every wavefront computes the same assignment from the lengths (B <= 128: two per
// lane); a slot past the last run returns false (no work, no arrival).
static_assert(kAttnCtrs <= 128, "balanced_slot holds two sequences per lane");
struct BalancedSlot {
  int b, j, n, slot0, t_begin, t_lim;  // sequence, run, runs of the sequence, its first slot
};

template <bool FUSED>
IRON_DEV bool balanced_slot(const AttnParams& p, int slot, BalancedSlot& a) {
  const int B = gridDim.z, lane = threadIdx.x & 63;
  int tl[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int b = lane + 64 * k;
    int len = 0;
    if (b < B) len = FUSED ? p.pos[b] + 1 : p.ctx_len[b];
    len = len < 0 ? 0 : (len > p.max_ctx ? p.max_ctx : len);
    tl[k] = (len + kTile - 1) / kTile;
  }
  const int T = wave_sum_int(tl[0] + tl[1]);
  const int extra = p.nslot - B;
  int start = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int t = tl[k];
    const bool valid = lane + 64 * k < B;
    int n = 1 + (T > 0 ? (int)((long long)extra * t / T) : 0);
    n = min(min(n, max(t, 1)), kMaxSplit);
    const int ch = t > 0 ? (t + n - 1) / n : 0;  // tiles per run
    const int nr = valid ? (t > 0 ? (t + ch - 1) / ch : 1) : 0;
    const int incl = wave_scan_int(nr);
    const int first = start + incl - nr;
    const unsigned long long mine = __ballot(valid && slot >= first && slot < first + nr);
    if (mine) {
      const int L = __ffsll((long long)mine) - 1;
      a.b = 64 * k + L;
      a.slot0 = __builtin_amdgcn_readlane(first, L);
      a.n = __builtin_amdgcn_readlane(nr, L);
      a.j = slot - a.slot0;
      const int chL = __builtin_amdgcn_readlane(ch, L);
      a.t_begin = a.j * chL * kTile;
      a.t_lim = min(p.max_ctx, a.t_begin + chL * kTile);
      return true;
    }
    start += __builtin_amdgcn_readlane(incl, 63);
  }
  return false;
}

// One 64-token K/V tile: lane (wave, row, dl) loads rows t0 + 16u + 4 wave + row, dims 8 dl..+8.
// Rows past `bound` (> t0) are clamped to bound - 1: every load is issued unconditionally, so
// the compiler's wait counts stay exact; those rows are masked where they are used.
IRON_DEV void load_kv_tile(const AttnParams& p, const AttnCoords& c, int t0, int bound,
                           uint4 (&kr)[4], uint4 (&vr)[4]) {
  const size_t base = (size_t)c.b * p.sb + (size_t)c.kv * p.sh + c.dl * 8;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    int t = t0 + u * 16 + c.wave * 4 + c.row;
    t = t < bound ? t : bound - 1;
    kr[u] = *(const uint4*)(p.k + base + (size_t)t * p.st);
    vr[u] = *(const uint4*)(p.v + base + (size_t)t * p.st);
  }
}

// One lane's 16 bytes from global memory into LDS at m0 + 16 * lane (global_load_lds_dwordx4;
// lds is wave-uniform), and one 16-byte LDS read. Inline asm so that the compiler, which would
// otherwise wait for every outstanding LDS-DMA before any LDS read, leaves the waits to the caller:
// a ring slot is read after s_waitcnt vmcnt(N) for the N loads issued after its own, and the
// read's result is used after s_waitcnt lgkmcnt(0).
IRON_DEV void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  __asm__ volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(off), "s"(base), "s"(lds)
                   : "memory");
}

IRON_DEV iron_u32x4 lds_read16(uint32_t addr) {
  iron_u32x4 v;
  __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// The query-side loads, issued before any K/V tile. Fused mode: the raw q row this wave rotates
// (xq[0]), the current token's raw K and V rows, the two norm weights and the angle
// row (e = {n_qn, n_kn, raw k, raw v, angles lo, angles hi}); plain mode: the q rows. Returns the
// (unclamped) context length; `pos` is the current token's position (fused) or -1.
template <int HB, bool FUSED>
IRON_DEV int load_query_side(const AttnParams& p, const AttnCoords& c, uint4 (&xq)[HB],
                             uint4 (&e)[6], int& pos) {
  const int dl = c.dl;
  if constexpr (FUSED) {
    pos = p.pos[c.b];
    const uint16_t* rawb = p.raw + (size_t)c.b * (p.H + 2 * p.KV) * kD;
    // wave h < HB rotates query head h0 + h: each wave loads only that row (into xq[0])
    const int hw = c.wave < HB ? c.wave : HB - 1;
    xq[0] = *(const uint4*)(rawb + (size_t)(c.h0 + hw) * kD + dl * 8);
    e[2] = *(const uint4*)(rawb + (size_t)(p.H + c.kv) * kD + dl * 8);
    e[3] = *(const uint4*)(rawb + (size_t)(p.H + p.KV + c.kv) * kD + dl * 8);
    e[0] = *(const uint4*)(p.n_qn + dl * 8);
    e[1] = *(const uint4*)(p.n_kn + dl * 8);
    const uint16_t* arow = p.ang + (size_t)c.b * kD + 16 * (dl & 7);
    e[4] = *(const uint4*)arow;
    e[5] = *(const uint4*)(arow + 8);
    return pos + 1;
  } else {
#pragma unroll
    for (int h = 0; h < HB; ++h)
      xq[h] = *(const uint4*)(p.q + ((size_t)c.b * p.H + c.h0 + h) * kD + dl * 8);
    pos = -1;
    return p.ctx_len ? p.ctx_len[c.b] : p.ctx_const;
  }
}

// Fused mode: the per-head epilogues run in parallel -- wave h < HB rotates query head h into
// s_q[h], wave HB % 4 (wave 0 when HB == 4, after its query head) builds the current token's K
// row into s_new (with its V row) and, in one workgroup per (b, kv head), into the caches. Ends
// with a barrier. Returns whether the current token lies in this workgroup's split
// (workgroup-uniform).
template <int HB>
IRON_DEV bool rotate_query_side(const AttnParams& p, const AttnCoords& c, const uint4 (&xq)[HB],
                                const uint4 (&e)[6], int pos, uint4 (&s_q)[HB][16],
                                uint4 (&s_new)[2][16]) {
  const bool pos_ok = pos >= 0 && pos < p.max_ctx;
  const bool has_new = pos_ok && pos >= c.t_begin && pos < c.t_lim;
  if (c.wave < HB) {
    double qn[8];
    norm_rope8(xq[0], e[0], e[4], e[5], c.dl, p.eps, qn);
    if (c.row == 0) s_q[c.wave][c.dl] = pack8_bf16(qn);
  }
  if (has_new && c.wave == HB % 4) {
    double kn[8];
    norm_rope8(e[2], e[1], e[4], e[5], c.dl, p.eps, kn);
    const uint4 kp = pack8_bf16(kn);
    if (c.row == 0) {
      s_new[0][c.dl] = kp;
      s_new[1][c.dl] = e[3];
      if (c.hg == 0) {  // one writer per (b, kv head)
        const size_t at = (size_t)c.b * p.sb + (size_t)c.kv * p.sh + (size_t)pos * p.st + c.dl * 8;
        *(uint4*)(p.k + at) = kp;
        *(uint4*)(p.v + at) = e[3];
      }
    }
  }
  __syncthreads();
  return has_new;
}

IRON_DEV float exp2_f(float x) { return __builtin_amdgcn_exp2f(x); }

// The split merge of one workgroup's HB query heads, run by the last split to finish (p.ctr): the
// arithmetic of attn_merge_kernel --
//   o = sum_s f_s O_s / sum_s f_s L_s,  f_s = e^(m_s - max m)  (exp2 in the fp32 mode)
// -- with 4 / HB wavefronts per head: every wavefront computes its head's statistics over all
// splits (lane l holds splits l, l + 64, ...) and sums the O partials of its share of the splits
// for dims 2l, 2l + 1 (weights broadcast from LDS); the shares add in LDS in a fixed order. The
// partials were stored write-through (st_agent) and are read with sc1 loads: the statistics, then
// batches of kMergeW O rows per wavefront (16 at HB = 4, whose attention loop leaves fewer
// registers), a batch's loads all in flight before the first wait. The code is branch-free and
// short: only the last split of each group runs it, after every other workgroup has left, so each
// instruction line it fetches is a cache miss on its critical path.
// The group's ns split rows of query head h start at row r0 + h hs of p.part.
template <bool F32, int HB>
IRON_DEV void merge_last(const AttnParams& p, int b, int h0, int ns, size_t r0, size_t hs) {
  constexpr int kMergeW = HB == 4 ? 16 : 32;
  using T = typename std::conditional<F32, float, double>::type;
  using T2 = typename std::conditional<F32, float2, double2>::type;
  constexpr int WPH = 4 / HB;  // wavefronts per head
  constexpr int kRow = (kD + 2) * (int)sizeof(T);  // bytes per split row
  // wave-uniform in a scalar register, so the buffer descriptor below is scalar too
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const int oh = wave / WPH, qi = wave % WPH, h = h0 + oh;
  const int per = (ns + WPH - 1) / WPH;
  const int s0 = qi * per, s1 = min(ns, s0 + per);
  const T* base = (const T*)p.part + (r0 + (size_t)h * hs) * (kD + 2);
  const __amdgpu_buffer_rsrc_t rs = agent_rsrc(base, (size_t)ns * kRow);
  // this wavefront's share of the O rows; the buffer's range ends with it, so the loads of a batch
  // past its end return zero (and add +0 below)
  const __amdgpu_buffer_rsrc_t ro =
      agent_rsrc(base + (size_t)s0 * (kD + 2), (size_t)max(s1 - s0, 0) * kRow);
  auto ld_pair = [&](__amdgpu_buffer_rsrc_t r, int off) -> T2 {  // two T at byte offset off
    if constexpr (F32) {
      const iron_u32x2 v = ld_agent_b64(r, off);
      return T2{__uint_as_float(v.x), __uint_as_float(v.y)};
    } else {
      const iron_u32x4 v = ld_agent_b128(r, off);
      return T2{__hiloint2double((int)v.y, (int)v.x), __hiloint2double((int)v.w, (int)v.z)};
    }
  };
  T ms[kMaxSplit / 64], ls[kMaxSplit / 64];
#pragma unroll
  for (int i = 0; i < kMaxSplit / 64; ++i) {
    const int sp = l + 64 * i;
    const T2 ml = ld_pair(rs, (sp < ns ? sp : 0) * kRow + kD * (int)sizeof(T));  // (m, l)
    ms[i] = sp < ns ? ml.x : (T)-INFINITY;
    ls[i] = sp < ns ? ml.y : (T)0;
  }
  auto issue = [&](int sb, T2 (&v)[kMergeW]) {
#pragma unroll
    for (int u = 0; u < kMergeW; ++u) v[u] = ld_pair(ro, (sb + u) * kRow + 2 * l * (int)sizeof(T));
  };
  T2 v[kMergeW];
  issue(0, v);  // the first batch, in flight while the statistics are reduced
  T mloc = ms[0];
#pragma unroll
  for (int i = 1; i < kMaxSplit / 64; ++i) mloc = F32 ? fmaxf(mloc, ms[i]) : fmax(mloc, ms[i]);
  T M;
  if constexpr (F32) {
    M = row16_max(mloc);
    M = fmaxf(M, __shfl_xor(M, 16));
    M = fmaxf(M, __shfl_xor(M, 32));
  } else {
    M = row16_max_d(mloc);
    M = fmax(M, __shfl_xor(M, 16));
    M = fmax(M, __shfl_xor(M, 32));
  }
  // the split weights f_s (zero from split ns on), published in LDS for this wavefront's broadcast
  // reads (a wavefront's LDS accesses complete in order, so its own writes need no barrier)
  __shared__ T s_f[4][kMaxSplit + kMergeW];
  T lloc = 0;
#pragma unroll
  for (int i = 0; i < kMaxSplit / 64; ++i) {
    T f = 0;
    if (64 * i < ns) {
      if constexpr (F32) f = (M == -INFINITY || ms[i] == -INFINITY) ? 0.f : exp2_f(ms[i] - M);
      else f = (M == -INFINITY || ms[i] == -INFINITY) ? 0.0 : exp(ms[i] - M);
      lloc += f * ls[i];
    }
    s_f[wave][l + 64 * i] = f;
  }
  if (l < kMergeW) s_f[wave][kMaxSplit + l] = 0;
  __builtin_amdgcn_wave_barrier();
  const T L = F32 ? (T)wave_sum((float)lloc) : (T)wave_sum_d((double)lloc);
  T a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
  auto accumulate = [&](int sb, const T2 (&v)[kMergeW]) {
#pragma unroll
    for (int u = 0; u < kMergeW; ++u) {
      const T w = s_f[wave][s0 + sb + u];
      a0[u & 3] = F32 ? fmaf(w, v[u].x, a0[u & 3]) : fma(w, v[u].x, a0[u & 3]);
      a1[u & 3] = F32 ? fmaf(w, v[u].y, a1[u & 3]) : fma(w, v[u].y, a1[u & 3]);
    }
  };
  accumulate(0, v);
  for (int sb = kMergeW; sb < s1 - s0; sb += kMergeW) {  // shares longer than one batch
    T2 vb[kMergeW];
    issue(sb, vb);
    accumulate(sb, vb);
  }
  __shared__ T2 s_m[4][64];
  s_m[wave][l] = T2{(a0[0] + a0[2]) + (a0[1] + a0[3]), (a1[0] + a1[2]) + (a1[1] + a1[3])};
  __syncthreads();
  if (qi != 0) return;
  T o0 = 0, o1 = 0;
#pragma unroll
  for (int q = 0; q < WPH; ++q) {
    o0 += s_m[wave + q][l].x;
    o1 += s_m[wave + q][l].y;
  }
  uint16_t e0, e1;
  if constexpr (F32) {
    e0 = f32_to_bf16(L > 0.f ? o0 / L : 0.f);
    e1 = f32_to_bf16(L > 0.f ? o1 / L : 0.f);
  } else {
    e0 = f64_to_bf16(L > 0.0 ? o0 / L : 0.0);
    e1 = f64_to_bf16(L > 0.0 ? o1 / L : 0.0);
  }
  *(uint32_t*)(p.out + ((size_t)b * p.H + h) * kD + 2 * l) = (uint32_t)e0 | ((uint32_t)e1 << 16);
}

// After this workgroup's partials are stored (write-through): count its arrival on its (sequence,
// head group) counter; the last of the ns splits merges the group's heads (merge_last).
template <bool F32, int HB>
IRON_DEV void merge_if_last(const AttnParams& p, int b, int h0, int ns, size_t r0, size_t hs) {
  if (!p.ctr) return;
  const unsigned idx = (unsigned)(b * gridDim.y + blockIdx.y);
  if (arrive_is_last_wt(p.ctr + idx * kAttnCtrStride, (unsigned)ns))
    merge_last<F32, HB>(p, b, h0, ns, r0, hs);
}

// This workgroup's place in the split partials: its split, the splits of its sequence and the
// rows (merge_last's r0, hs) -- [B][H][nsplit] rows, or in balanced mode [H][nslot] rows with a
// sequence's runs in consecutive slots. Applies the balanced assignment to c; false: no work.
struct SplitSlot {
  int split, ns;
  size_t r0, hs;
};

template <bool FUSED>
IRON_DEV bool split_slot(const AttnParams& p, AttnCoords& c, SplitSlot& q) {
  q.split = blockIdx.x;
  q.ns = p.nsplit;
  q.r0 = (size_t)c.b * p.H * p.nsplit;
  q.hs = p.nsplit;
  if (!p.bal) return true;
  BalancedSlot a;
  if (!balanced_slot<FUSED>(p, blockIdx.z * p.nsplit + blockIdx.x, a)) return false;
  c.b = a.b;
  c.t_begin = a.t_begin;
  c.t_lim = a.t_lim;
  q.split = a.j;
  q.ns = a.n;
  q.r0 = a.slot0;
  q.hs = p.nslot;
  return true;
}

template <int HB, bool FUSED>
__global__ __launch_bounds__(256, 2) void decode_attn_kernel(AttnParams p) {
  AttnCoords c = attn_coords<HB>(p);
  SplitSlot q;
  if (!split_slot<FUSED>(p, c, q)) return;
  const int split = q.split, b = c.b, h0 = c.h0;
  const int wave = c.wave, lane = threadIdx.x & 63, row = c.row, dl = c.dl;
  const int t_begin = c.t_begin, t_lim = c.t_lim;

  uint4 kr[4], vr[4];
  // Issue order: the position / context length and the query-side rows, then (B == 1) the
  // first K/V tile. Loads complete in issue order, so the query-side work below waits only for
  // the first group while the tile is still in flight.
  uint4 xq[HB], e[6];
  int pos;
  int ctx = load_query_side<HB, FUSED>(p, c, xq, e, pos);
  if (p.spec) load_kv_tile(p, c, t_begin, t_lim, kr, vr);
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int t_end = min(ctx, t_lim);

  double qf[HB][8];
  __shared__ uint4 s_new[2][16];   // the current token's K and V rows (fused mode)
  __shared__ uint4 s_q[HB][16];    // the rotated query rows (fused mode)
  bool has_new = false;
  if constexpr (FUSED) {
    has_new = rotate_query_side<HB>(p, c, xq, e, pos, s_q, s_new);
#pragma unroll
    for (int h = 0; h < HB; ++h) unpack8d(s_q[h][dl], qf[h]);
  } else {
#pragma unroll
    for (int h = 0; h < HB; ++h) unpack8d(xq[h], qf[h]);
  }

  double m[HB], l[HB], o[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.0;
  }

  __shared__ double s_mx[2][4][HB];
  // the end-of-kernel sums' staging (attn_finish_f64); with four query heads also the K/V ring
  __shared__ __align__(16) double s_ro[16][HB][kAttnD];
  if constexpr (HB >= 4) {
    // Four query heads hold 128 fp64 values per lane (q and the outputs): one register set of
    // K/V rows keeps the kernel within half the register file (two workgroups per CU). The
    // tiles after it come through LDS instead: each lane's 16-byte K and V rows of a tile go by
    // global_load_lds into the lane's own slots of a two-tile ring (32 KiB a tile, in s_ro's
    // 64 KiB), so while a tile is processed from registers the next two are in flight. A lane
    // reads back only what it loaded, so its own load count orders the ring (no barrier): the
    // loads and the reads are inline asm, which the compiler does not see as an LDS store (it
    // would otherwise wait for every such load before any LDS read) and the waits are explicit.
    if (p.spec || t_begin >= t_end) {  // B = 1: the first tile already went out with the query
      if (!p.spec && t_begin < t_end) load_kv_tile(p, c, t_begin, t_lim, kr, vr);
      int it = 0;
      for (int t0 = t_begin; t0 < t_end; t0 += kTile, ++it) {
        if (t0 > t_begin) load_kv_tile(p, c, t0, t_lim, kr, vr);
        attn_tile_f64<HB, FUSED>(kr, vr, t0, t_end, has_new, pos, s_new, qf, p.scale, it, m, l,
                                 o, s_mx, wave, lane, row, dl);
      }
    } else {
      static_assert(sizeof(s_ro) >= 2 * 4 * 8 * 1024, "the ring fits in the sums' staging");
      const uint32_t ring = (uint32_t)(uintptr_t)&s_ro[0][0][0];
      auto slot = [&](int s, int j) {  // wave-uniform: slot of row j (K 2u, V 2u + 1), ring half s
        return (uint32_t)__builtin_amdgcn_readfirstlane(ring + ((s * 4 + wave) * 8 + j) * 1024);
      };
      // byte offsets from the K and V bases (one 32-bit offset serves both: the same strides)
      const uint16_t* kb = p.k + (size_t)b * p.sb + (size_t)c.kv * p.sh;
      const uint16_t* vb = p.v + (size_t)b * p.sb + (size_t)c.kv * p.sh;
      auto dma_tile = [&](int t0, int s) {  // rows clamped below t_lim, as load_kv_tile's
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          int t = t0 + u * 16 + wave * 4 + row;
          t = t < t_lim ? t : t_lim - 1;
          const uint32_t off = (uint32_t)(t * p.st + dl * 8) * 2u;
          lds_dma16(kb, off, slot(s, 2 * u));
          lds_dma16(vb, off, slot(s, 2 * u + 1));
        }
      };
      auto read_tile = [&](int s) {  // the older of the two tiles in flight (8 loads each)
        __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
        iron_u32x4* const k4 = reinterpret_cast<iron_u32x4*>(kr);
        iron_u32x4* const v4 = reinterpret_cast<iron_u32x4*>(vr);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          k4[u] = lds_read16(slot(s, 2 * u) + lane * 16);
          v4[u] = lds_read16(slot(s, 2 * u + 1) + lane * 16);
        }
        __asm__ volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(k4[0]), "+v"(k4[1]), "+v"(k4[2]), "+v"(k4[3]), "+v"(v4[0]),
                           "+v"(v4[1]), "+v"(v4[2]), "+v"(v4[3])
                         :
                         : "memory");
      };
      dma_tile(t_begin, 0);
      dma_tile(t_begin + kTile, 1);
      int it = 0;
      for (int t0 = t_begin; t0 < t_end; t0 += kTile, ++it) {
        read_tile(it & 1);                        // tile it (tile it + 1 may be in flight)
        dma_tile(t0 + 2 * kTile, it & 1);         // tile it + 2 into the half just read
        attn_tile_f64<HB, FUSED>(kr, vr, t0, t_end, has_new, pos, s_new, qf, p.scale, it, m, l,
                                 o, s_mx, wave, lane, row, dl);
      }
      // every lane's ring loads have landed before s_ro is rewritten
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  } else {
    // Tiles alternate between two register sets, the next tile's rows in flight while one is
    // processed (separate named sets: a copy between them would wait for the loads). Every load
    // is issued, rows clamped below t_lim (rows at or past t_end are masked where they are used).
    uint4 kr2[4], vr2[4];
    if (!p.spec && t_begin < t_end) load_kv_tile(p, c, t_begin, t_lim, kr, vr);
    int it = 0;
    for (int t0 = t_begin; t0 < t_end; t0 += 2 * kTile, it += 2) {
      load_kv_tile(p, c, t0 + kTile, t_lim, kr2, vr2);
      attn_tile_f64<HB, FUSED>(kr, vr, t0, t_end, has_new, pos, s_new, qf, p.scale, it, m, l, o,
                               s_mx, wave, lane, row, dl);
      if (t0 + kTile >= t_end) break;
      load_kv_tile(p, c, t0 + 2 * kTile, t_lim, kr, vr);
      attn_tile_f64<HB, FUSED>(kr2, vr2, t0 + kTile, t_end, has_new, pos, s_new, qf, p.scale,
                               it + 1, m, l, o, s_mx, wave, lane, row, dl);
    }
  }

  attn_finish_f64<HB>(m, l, o, wave, row, dl, s_ro, [&](int oh, int od, double O, double L, double M) {
    const int hq = h0 + oh;
    if (q.ns == 1) {
      p.out[((size_t)b * p.H + hq) * kD + od] = f64_to_bf16(L > 0.0 ? O / L : 0.0);
    } else {
      double* part = (double*)p.part + (q.r0 + hq * q.hs + split) * (kD + 2);
      st_agent(part + od, O);
      if (od == 0) {
        st_agent(part + kD, M);
        st_agent(part + kD + 1, L);
      }
    }
  });
  if (q.ns > 1) merge_if_last<false, HB>(p, b, h0, q.ns, q.r0, q.hs);
}

// ---------------------------------------------------------------------------------------------
// fp32-accumulation variant: the arithmetic the reference kernel specifies (bf16 inputs, fp32
// scores / softmax / accumulation, decode_attn.cc:117-311) rather than the exact value.
//   * q . k_j: v_dot2_f32_bf16 on packed bf16 pairs (the products are exact in fp32), summed over
//     the 16 lanes of a row with DPP; s_j = (q . k_j) * scale * log2(e), probabilities exp2(s - m)
//     (v_exp_f32), o accumulated with fp32 FMAs, one rounding of o / l to bf16.
//   * each wavefront keeps its own running maximum (no workgroup barrier per tile); the four
//     wavefronts' sums are rescaled to the common maximum once, at the end.
//   * the next tile's K/V rows are loaded while the current tile is processed.
// The fused query-side epilogue (QK RMSNorm, RoPE, cache append) is the exact one above, so the
// KV cache holds the same rows in both variants.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

IRON_DEV float dot8_bf16(const uint4 a, const uint4 b) {
  float s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x),
                                            __builtin_bit_cast(bf16x2_t, b.x), 0.0f, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y),
                                      __builtin_bit_cast(bf16x2_t, b.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z),
                                      __builtin_bit_cast(bf16x2_t, b.z), s, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w),
                                         __builtin_bit_cast(bf16x2_t, b.w), s, false);
}

template <int N, int HB>
IRON_DEV void share_one_f(float ev, float (&pe)[4][HB]) {
  if constexpr (N < 4 * HB) pe[N / HB][N % HB] = dpp_f<0x150 + N>(ev);  // row_newbcast:N
}

template <int HB, int... Ns>
IRON_DEV void share_all_f(float ev, float (&pe)[4][HB], std::integer_sequence<int, Ns...>) {
  (share_one_f<Ns, HB>(ev, pe), ...);
}


template <int HB, bool FUSED>
__global__ __launch_bounds__(256) void decode_attn_f32_kernel(AttnParams p) {
  AttnCoords c = attn_coords<HB>(p);
  SplitSlot q;
  if (!split_slot<FUSED>(p, c, q)) return;
  const int split = q.split, b = c.b;
  const int wave = c.wave, lane = threadIdx.x & 63, row = c.row, dl = c.dl;
  const int t_begin = c.t_begin, t_lim = c.t_lim;

  uint4 kr[4], vr[4];
  uint4 xq[HB], e[6];
  int pos;
  int ctx = load_query_side<HB, FUSED>(p, c, xq, e, pos);
  if (p.spec) load_kv_tile(p, c, t_begin, t_lim, kr, vr);
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int t_end = min(ctx, t_lim);
  if (!p.spec && t_begin < t_end) load_kv_tile(p, c, t_begin, t_end, kr, vr);

  uint4 qp[HB];                    // packed bf16 query rows (dims 8 dl..+8)
  __shared__ uint4 s_new[2][16];
  __shared__ uint4 s_q[HB][16];
  bool has_new = false;
  if constexpr (FUSED) {
    has_new = rotate_query_side<HB>(p, c, xq, e, pos, s_q, s_new);
#pragma unroll
    for (int h = 0; h < HB; ++h) qp[h] = s_q[h][dl];
  } else {
#pragma unroll
    for (int h = 0; h < HB; ++h) qp[h] = xq[h];
  }

  float m[HB], l[HB], o[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.0f;
  }

  for (int t0 = t_begin; t0 < t_end; t0 += kTile) {
    // prefetch the next tile (past the context every row clamps to the last valid row, which
    // the current tile has just brought into the cache)
    uint4 kn[4], vn[4];
    load_kv_tile(p, c, t0 + kTile, t_end, kn, vn);
    bool tv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u * 16 + wave * 4 + row;
      tv[u] = t < t_end;
      if constexpr (FUSED) {
        if (has_new && t == pos) {
          kr[u] = s_new[0][dl];
          vr[u] = s_new[1][dl];
        }
      }
      if (!tv[u]) vr[u] = make_uint4(0u, 0u, 0u, 0u);  // rows past the context may hold NaNs
    }
    // Raised wave priority from the scores through the exponentials' broadcast (two workgroups
    // per CU: the SIMD's other wavefront fills this chain's latency with its P.V FMAs; config 3
    // B=8 19.6 -> 19.1 us, config 5 7.44 -> 7.34 ms per step)
    __builtin_amdgcn_s_setprio(1);
    // scores in the exp2 domain, identical in every lane of the row
    float s[4][HB];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        const float a = row16_sum(dot8_bf16(qp[h], kr[u])) * p.scale2;
        s[u][h] = tv[u] ? a : -INFINITY;
      }
    // wavefront running maximum per head
    float mn[HB];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      float v = fmaxf(fmaxf(s[0][h], s[1][h]), fmaxf(s[2][h], s[3][h]));
      v = fmaxf(v, __shfl_xor(v, 16));
      v = fmaxf(v, __shfl_xor(v, 32));
      mn[h] = fmaxf(m[h], v);
    }
    // lane dl < 4*HB evaluates exponential (u, h) = (dl / HB, dl % HB); a masked token (or a
    // wavefront with no valid token yet) contributes 0
    float sv = -INFINITY, mv = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int h = 0; h < HB; ++h)
        if (dl == u * HB + h) {
          sv = s[u][h];
          mv = mn[h];
        }
    const float ev = sv == -INFINITY ? 0.0f : exp2_f(sv - mv);
    float pe[4][HB];
    share_all_f<HB>(ev, pe, std::make_integer_sequence<int, 16>{});
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const float cf = m[h] == mn[h] ? 1.0f : exp2_f(m[h] - mn[h]);
      l[h] = l[h] * cf + ((pe[0][h] + pe[1][h]) + (pe[2][h] + pe[3][h]));
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= cf;
      m[h] = mn[h];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t d[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float v0 = bf16lo_to_f32(d[jj]), v1 = bf16hi_to_f32(d[jj]);
#pragma unroll
        for (int h = 0; h < HB; ++h) {
          o[h][2 * jj] = fmaf(pe[u][h], v0, o[h][2 * jj]);
          o[h][2 * jj + 1] = fmaf(pe[u][h], v1, o[h][2 * jj + 1]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kr[u] = kn[u];
      vr[u] = vn[u];
    }
  }

  // 16 token rows: the 4 rows of a wavefront share its maximum; wavefronts rescale to the common
  // maximum M with f_w = exp2(m_w - M)
  __shared__ float s_o[16][HB][kD];
  __shared__ float s_l[16][HB];
  __shared__ float s_m[4][HB];
  const int rr = wave * 4 + row;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    *(float4*)&s_o[rr][h][dl * 8] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
    *(float4*)&s_o[rr][h][dl * 8 + 4] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    if (dl == 0) s_l[rr][h] = l[h];
    if (lane == 0) s_m[wave][h] = m[h];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < HB * kD; t += 256) {
    const int oh = t / kD, od = t % kD;
    float mw[4], f[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) mw[w] = s_m[w][oh];
    const float M = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
#pragma unroll
    for (int w = 0; w < 4; ++w) f[w] = mw[w] == -INFINITY ? 0.0f : exp2_f(mw[w] - M);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float ow = (s_o[4 * w][oh][od] + s_o[4 * w + 1][oh][od]) +
                       (s_o[4 * w + 2][oh][od] + s_o[4 * w + 3][oh][od]);
      const float lw = (s_l[4 * w][oh] + s_l[4 * w + 1][oh]) +
                       (s_l[4 * w + 2][oh] + s_l[4 * w + 3][oh]);
      O = fmaf(f[w], ow, O);
      L = fmaf(f[w], lw, L);
    }
    const int hq = c.h0 + oh;
    if (q.ns == 1) {
      p.out[((size_t)b * p.H + hq) * kD + od] = f32_to_bf16(L > 0.0f ? O / L : 0.0f);
    } else {
      float* part = (float*)p.part + (q.r0 + hq * q.hs + split) * (kD + 2);
      st_agent(part + od, O);
      if (od == 0) {
        st_agent(part + kD, M);
        st_agent(part + kD + 1, L);
      }
    }
  }
  if (q.ns > 1) merge_if_last<true, HB>(p, b, c.h0, q.ns, q.r0, q.hs);
}


// Split merge, grid (H, B), 4 wavefronts per (head, sequence):
//   o = sum_s f_s O_s / sum_s f_s L_s,  f_s = e^(m_s - max m)  (exp2 in the fp32 mode, whose
//   maxima are in the log2 domain)
// Every wavefront computes the statistics of all splits (lane l holds splits l, l+64, ...), then
// sums the O partials of its quarter of the splits for head dims 2l, 2l+1, taking the weights by
// readlane; the four quarter sums add in LDS in a fixed order. All O loads of a quarter (up to
// kRegW splits) are issued before the first reduction.
constexpr int kRegW = 16;

template <bool F32>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p) {
  using T = typename std::conditional<F32, float, double>::type;
  using T2 = typename std::conditional<F32, float2, double2>::type;
  const int h = blockIdx.x, b = blockIdx.y;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int ns = p.nsplit;
  const int per = (ns + 3) >> 2;                // splits per wavefront
  const int s0 = wave * per, s1 = min(ns, s0 + per);
  const T* base = (const T*)p.part + ((size_t)b * p.H + h) * ns * (kD + 2);
  T2 ov[kRegW];
#pragma unroll
  for (int i = 0; i < kRegW; ++i) {
    const int sp = s0 + i;
    const int sc = sp < s1 ? sp : 0;  // clamped: every load is issued
    ov[i] = *(const T2*)(base + (size_t)sc * (kD + 2) + 2 * l);
  }
  T ms[kMaxSplit / 64], ls[kMaxSplit / 64];
#pragma unroll
  for (int i = 0; i < kMaxSplit / 64; ++i) {
    const int sp = l + 64 * i;
    const int sc = sp < ns ? sp : 0;
    ms[i] = base[(size_t)sc * (kD + 2) + kD];
    ls[i] = base[(size_t)sc * (kD + 2) + kD + 1];
    if (sp >= ns) {
      ms[i] = -INFINITY;
      ls[i] = 0;
    }
  }
  T mloc = ms[0];
#pragma unroll
  for (int i = 1; i < kMaxSplit / 64; ++i) mloc = F32 ? fmaxf(mloc, ms[i]) : fmax(mloc, ms[i]);
  T M;
  if constexpr (F32) {
    M = row16_max(mloc);
    M = fmaxf(M, __shfl_xor(M, 16));
    M = fmaxf(M, __shfl_xor(M, 32));
  } else {
    M = row16_max_d(mloc);
    M = fmax(M, __shfl_xor(M, 16));
    M = fmax(M, __shfl_xor(M, 32));
  }
  T f[kMaxSplit / 64];
  T lloc = 0;
#pragma unroll
  for (int i = 0; i < kMaxSplit / 64; ++i) {
    if constexpr (F32) f[i] = (M == -INFINITY || ms[i] == -INFINITY) ? 0.f : exp2_f(ms[i] - M);
    else f[i] = (M == -INFINITY || ms[i] == -INFINITY) ? 0.0 : exp(ms[i] - M);
    lloc += f[i] * ls[i];
  }
  const T L = F32 ? (T)wave_sum((float)lloc) : (T)wave_sum_d((double)lloc);
  auto weight = [&](int sp) -> T {  // f of split sp, wave-uniform
    const int i = sp >> 6, lane = sp & 63;
    const T v = i == 0 ? f[0] : (i == 1 ? f[1] : (i == 2 ? f[2] : f[3]));
    if constexpr (F32) {
      return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
    } else {
      const int lo = __builtin_amdgcn_readlane(__double2loint(v), lane);
      const int hi = __builtin_amdgcn_readlane(__double2hiint(v), lane);
      return __hiloint2double(hi, lo);
    }
  };
  T a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kRegW; ++i)
    if (s0 + i < s1) {
      const T w = weight(s0 + i);
      a0[i & 3] = F32 ? fmaf(w, ov[i].x, a0[i & 3]) : fma(w, ov[i].x, a0[i & 3]);
      a1[i & 3] = F32 ? fmaf(w, ov[i].y, a1[i & 3]) : fma(w, ov[i].y, a1[i & 3]);
    }
  for (int sp = s0 + kRegW; sp < s1; ++sp) {
    const T w = weight(sp);
    const T2 v = *(const T2*)(base + (size_t)sp * (kD + 2) + 2 * l);
    a0[0] = F32 ? fmaf(w, v.x, a0[0]) : fma(w, v.x, a0[0]);
    a1[0] = F32 ? fmaf(w, v.y, a1[0]) : fma(w, v.y, a1[0]);
  }
  __shared__ T2 s_q[4][64];
  s_q[wave][l] = T2{(a0[0] + a0[2]) + (a0[1] + a0[3]), (a1[0] + a1[2]) + (a1[1] + a1[3])};
  __syncthreads();
  if (wave != 0) return;
  const T2 q0 = s_q[0][l], q1 = s_q[1][l], q2 = s_q[2][l], q3 = s_q[3][l];
  const T o0 = (q0.x + q1.x) + (q2.x + q3.x);
  const T o1 = (q0.y + q1.y) + (q2.y + q3.y);
  uint16_t r0, r1;
  if constexpr (F32) {
    r0 = f32_to_bf16(L > 0.f ? o0 / L : 0.f);
    r1 = f32_to_bf16(L > 0.f ? o1 / L : 0.f);
  } else {
    r0 = f64_to_bf16(L > 0.0 ? o0 / L : 0.0);
    r1 = f64_to_bf16(L > 0.0 ? o1 / L : 0.0);
  }
  *(uint32_t*)(p.out + ((size_t)b * p.H + h) * kD + 2 * l) = (uint32_t)r0 | ((uint32_t)r1 << 16);
}

struct SplitPlan {
  int nsplit, chunk, hb;
};

SplitPlan plan_split(int B, int H, int KV, int max_ctx, bool f32) {
  SplitPlan sp;
  const int HG = H / KV;
  sp.hb = HG >= 4 ? 4 : HG;
  const int wg_per_split = B * KV * (HG / sp.hb);
  // About 512 workgroups; with the fp64 core, 256 where 512 would take more than 32 splits (B=1):
  // the last split's merge of 64 partials then costs more than the longer tiles of 32 splits
  // (config 3 at B=1: 12.5 -> 10.5 us; B=8 ragged at a 256 target: 22.6 -> 23.0 us). The fp32
  // core keeps 64 splits (9.9 -> 9.0 us at 32): its result depends on the split boundaries, and
  // 32 splits moved enough logits of the 128-step Qwen3-0.6B greedy run to flip 7 of its 124
  // decided tokens against the exact chain, where 64 splits agree on all of them.
  const int target_wgs = !f32 && 512 / wg_per_split > 32 ? 256 : 512;
  const int max_ns = (max_ctx + kTile - 1) / kTile;
  int ns = (target_wgs + wg_per_split - 1) / wg_per_split;
  if (ns > max_ns) ns = max_ns;
  if (ns > kMaxSplit) ns = kMaxSplit;
  if (ns < 1) ns = 1;
  int chunk = (max_ctx + ns - 1) / ns;
  chunk = ((chunk + kTile - 1) / kTile) * kTile;
  ns = (max_ctx + chunk - 1) / chunk;
  if (ns < 1) ns = 1;
  sp.nsplit = ns;
  sp.chunk = chunk;
  return sp;
}

// The split workspace: the merge's arrival counters (kAttnCtrBytes, zero before the first call
// and after every call), then the partials.
size_t attn_ws_bytes(int B, int H, int KV, int max_ctx) {
  const SplitPlan sp = plan_split(B, H, KV, max_ctx, true);  // the larger of the two plans
  if (sp.nsplit == 1) return 0;
  return kAttnCtrBytes +
         ((((size_t)B * H * sp.nsplit * (kD + 2) * sizeof(double)) + 255) & ~(size_t)255);
}

int check_attn_shape(const char* fn, int B, int H, int KV, int D, int max_ctx) {
  if (B <= 0 || H <= 0 || KV <= 0 || max_ctx <= 0)
    return iron::fail(IRON_ERR_SHAPE, "%s: bad shape B=%d H=%d KV=%d max_ctx=%d", fn, B, H, KV,
                      max_ctx);
  if (D != kD) return iron::fail(IRON_ERR_UNSUPPORTED, "%s: head_dim %d (only 128)", fn, D);
  if (H % KV) return iron::fail(IRON_ERR_SHAPE, "%s: H=%d not a multiple of KV=%d", fn, H, KV);
  const int HG = H / KV;
  if (HG != 1 && HG != 2 && HG % 4 != 0)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: GQA group %d not 1, 2 or a multiple of 4", fn,
                      HG);
  return IRON_OK;
}

// Launches the split kernel (and the merge when the context is split). `p` carries the inputs;
// the split plan, partial buffer and head blocking are filled in here.
int launch_attention(AttnParams p, bool fused, int acc, int B, void* part_ws, size_t part_bytes,
                     hipStream_t s, const char* fn) {
  if (acc != IRON_ACCUM_F64 && acc != IRON_ACCUM_F32)
    return iron::fail(IRON_ERR_SHAPE, "%s: unknown accumulation mode %d", fn, acc);
  const bool f32 = acc == IRON_ACCUM_F32;
  p.scale2 = (float)(p.scale * 1.4426950408889634);
  const SplitPlan sp = plan_split(B, p.H, p.KV, p.max_ctx, f32);
  p.HG = p.H / p.KV;
  p.HB = sp.hb;
  p.ctr = nullptr;
  p.bal = 0;
  p.chunk = sp.chunk;
  p.nsplit = sp.nsplit;
  p.spec = B == 1 ? 1 : 0;
  if (sp.nsplit > 1) {
    const size_t need = attn_ws_bytes(B, p.H, p.KV, p.max_ctx);
    if (!part_ws || part_bytes < need)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, part_bytes, need);
    if (!iron::aligned(part_ws, 256))
      return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
    p.part = (char*)part_ws + kAttnCtrBytes;
    // the last split of each (sequence, head group) merges in the kernel: one launch; with more
    // groups than counters the merge kernel runs instead
    const long long groups = (long long)B * p.KV * (p.HG / sp.hb);
    p.ctr = groups <= kAttnCtrs ? (unsigned int*)part_ws : nullptr;
    // per-sequence lengths at B > 1: deal the splits by length (B <= kAttnCtrs here)
    p.bal = p.ctr && B > 1 && (fused || p.ctx_len) ? 1 : 0;
  }
  p.nslot = sp.nsplit * B;
  dim3 grid(sp.nsplit, p.KV * (p.HG / sp.hb), B);
#define IRON_ATTN_LAUNCH(HBV)                                                                  \
  do {                                                                                         \
    if (f32 && fused)                                                                          \
      hipLaunchKernelGGL((decode_attn_f32_kernel<HBV, true>), grid, dim3(256), 0, s, p);       \
    else if (f32)                                                                              \
      hipLaunchKernelGGL((decode_attn_f32_kernel<HBV, false>), grid, dim3(256), 0, s, p);      \
    else if (fused)                                                                            \
      hipLaunchKernelGGL((decode_attn_kernel<HBV, true>), grid, dim3(256), 0, s, p);           \
    else                                                                                       \
      hipLaunchKernelGGL((decode_attn_kernel<HBV, false>), grid, dim3(256), 0, s, p);          \
  } while (0)
  switch (sp.hb) {
    case 1: IRON_ATTN_LAUNCH(1); break;
    case 2: IRON_ATTN_LAUNCH(2); break;
    default: IRON_ATTN_LAUNCH(4); break;
  }
#undef IRON_ATTN_LAUNCH
  int st = iron::check_launch(fn);
  if (st || sp.nsplit == 1 || p.ctr) return st;
  if (f32)
    hipLaunchKernelGGL(attn_merge_kernel<true>, dim3(p.H, B), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(attn_merge_kernel<false>, dim3(p.H, B), dim3(256), 0, s, p);
  return iron::check_launch(fn);
}

// ---------------------------------------------------------------------------------------------
// Batch / verify mode (speculative-decode verify): n new tokens at positions base..base+n-1 each
// query one shared KV cache; token t attends keys [0, min(base + t + 1, S)) when causal, all S
// keys otherwise (iron/operators/decode_attn/op.py:40-48, design.py:243-276). The reference
// streams the cache once per group of M queries; here a workgroup stages each 64-key K/V block in
// LDS once and applies it to up to 64 query rows (4 wavefronts x 16 rows, row = t * HG + g for
// query head kv * HG + g), so the cache is read once per 64 / HG tokens.
//
// Arithmetic: the reference kernel's (decode_attn.cc:117-311): bf16 operands, fp32 scores
// (v_mfma_f32_16x16x32_bf16), exp2-domain online softmax in fp32, probabilities rounded to bf16
// for the P.V product, fp32 accumulation, one division and bf16 rounding of the output. Splits
// of the key range merge in the fp32 merge kernel above (maxima in the exp2 domain).
//
// MFMA layouts (checked on the device for the prefill kernel, prefill.hip): S^T = K Q^T per 16-key
// tile leaves lane l with query l % 16 and keys 4 (l / 16) + i; a 32-key P.V step takes tiles 2s
// and 2s + 1 in that order, which is the B-operand layout of P^T for O^T = V^T P^T when V^T reads
// the same key permutation.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 vbf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float vf32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float vf32x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 vbf16x2;

constexpr int kVB = 64;  // keys per staged block

struct VerifyParams {
  const uint16_t* q;         // [n][H][D] token-major
  const uint16_t* k;
  const uint16_t* v;
  long long sh, st;          // head and token strides of the caches (elements)
  const int32_t* base_ptr;   // device S_kv_base, or null (base_const)
  int base_const;
  int causal, n, H, KV, HG, S, rows;  // rows = n * HG query rows per KV head
  int chunk, nsplit, qgroups;
  float c;                   // scale * log2(e)
  float* part;               // [n][H][nsplit][D + 2]: o (unnormalised), m (exp2 domain), l
  uint16_t* out;             // [n][H][D]
};

IRON_DEV vbf16x8 as_vbf16x8(const uint4 u) { return __builtin_bit_cast(vbf16x8, u); }

IRON_DEV uint32_t pack2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((vf32x2{lo, hi}), vbf16x2));
}

__global__ __launch_bounds__(256) void verify_attn_kernel(VerifyParams p) {
  __shared__ __align__(16) uint16_t s_k[kVB][kD + 8];
  __shared__ __align__(16) uint16_t s_vt[kD][kVB + 8];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int quarter = lane >> 4, col = lane & 15;
  const int split = blockIdx.x;
  const int kv = blockIdx.y / p.qgroups, qg = blockIdx.y % p.qgroups;
  const int tile = qg * 4 + wave;              // this wavefront's 16 query rows
  const bool live = tile * 16 < p.rows;         // wavefront-uniform
  const int r = tile * 16 + col;               // this lane's query row
  const bool rv = r < p.rows;
  const int rc = rv ? r : 0;                   // rows past the end read row 0, never stored
  const int t = rc / p.HG, h = kv * p.HG + rc % p.HG;
  int base = p.base_ptr ? *p.base_ptr : p.base_const;
  base = base < 0 ? 0 : base;
  const int s_eff = p.causal ? min(base + p.n, p.S) : p.S;  // keys some query attends
  const int bound = p.causal ? min(base + t + 1, p.S) : p.S;
  const int k0 = split * p.chunk, k1 = min(k0 + p.chunk, s_eff);
  const int lim = min(bound, k1);              // this lane's valid keys in the split: [k0, lim)

  uint4 qf[kD / 32];                           // Q^T operand: dims 32 j + 8 quarter .. +8
  const uint16_t* qrow = p.q + ((size_t)t * p.H + h) * kD;
#pragma unroll
  for (int j = 0; j < kD / 32; ++j) qf[j] = *(const uint4*)(qrow + 32 * j + quarter * 8);

  const uint16_t* kb = p.k + (size_t)kv * p.sh;
  const uint16_t* vb = p.v + (size_t)kv * p.sh;
  // staging: K keys 4 (tid / 16) + i, dims 8 (tid % 16); V keys 4 (tid % 16) + i, dims
  // 8 (tid / 16) (key groups fastest across lanes: the transposed writes spread over banks)
  const int kg = tid >> 4, kd = (tid & 15) * 8, vg = tid & 15, vd = (tid >> 4) * 8;
  uint4 kreg[4], vreg[4];
  auto gload = [&](int kb0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jk = min(kb0 + 4 * kg + i, k1 - 1), jv = min(kb0 + 4 * vg + i, k1 - 1);
      kreg[i] = *(const uint4*)(kb + (size_t)jk * p.st + kd);
      vreg[i] = *(const uint4*)(vb + (size_t)jv * p.st + vd);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) *(uint4*)&s_k[4 * kg + i][kd] = kreg[i];
    const uint32_t a[4][4] = {{vreg[0].x, vreg[0].y, vreg[0].z, vreg[0].w},
                              {vreg[1].x, vreg[1].y, vreg[1].z, vreg[1].w},
                              {vreg[2].x, vreg[2].y, vreg[2].z, vreg[2].w},
                              {vreg[3].x, vreg[3].y, vreg[3].z, vreg[3].w}};
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // dims vd + 2w (low halves) and vd + 2w + 1 (high halves)
      *(uint2*)&s_vt[vd + 2 * w][4 * vg] =
          make_uint2((a[0][w] & 0xffffu) | (a[1][w] << 16), (a[2][w] & 0xffffu) | (a[3][w] << 16));
      *(uint2*)&s_vt[vd + 2 * w + 1][4 * vg] =
          make_uint2((a[0][w] >> 16) | (a[1][w] & 0xffff0000u),
                     (a[2][w] >> 16) | (a[3][w] & 0xffff0000u));
    }
  };

  vf32x4 o[kD / 16];
#pragma unroll
  for (int dt = 0; dt < kD / 16; ++dt) o[dt] = vf32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;                // this lane's share of its query's statistics

  if (k0 < k1) gload(k0);
  for (int kb0 = k0; kb0 < k1; kb0 += kVB) {
    __syncthreads();                           // the previous block's LDS reads are done
    lstore();
    __syncthreads();
    if (kb0 + kVB < k1) gload(kb0 + kVB);      // in flight during this block's products
    if (!live) continue;
    vf32x4 sc[kVB / 16];
#pragma unroll
    for (int kt = 0; kt < kVB / 16; ++kt) {
      sc[kt] = vf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kD / 32; ++j) {
        const uint4 a = *(const uint4*)&s_k[16 * kt + col][32 * j + quarter * 8];
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_vbf16x8(a), as_vbf16x8(qf[j]),
                                                         sc[kt], 0, 0, 0);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < kVB / 16; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int jk = kb0 + 16 * kt + quarter * 4 + i;
        if (jk >= lim) sc[kt][i] = -INFINITY;
        mx = fmaxf(mx, sc[kt][i]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m, mx * p.c);       // the scale is positive: max maps to max
    const bool none = mn == -INFINITY;         // no valid key of this query yet
    const float corr = none ? 1.f : exp2_f(m - mn);
    m = mn;
    float ps = 0.f;
    vbf16x8 pb[kVB / 32];
#pragma unroll
    for (int ks = 0; ks < kVB / 32; ++ks) {
      uint32_t w[4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e[i] = none ? 0.f : exp2_f(fmaf(sc[2 * ks + hh][i], p.c, -mn));
          ps += e[i];
        }
        w[2 * hh] = pack2_bf16(e[0], e[1]);
        w[2 * hh + 1] = pack2_bf16(e[2], e[3]);
      }
      pb[ks] = as_vbf16x8(make_uint4(w[0], w[1], w[2], w[3]));
    }
    l = l * corr + ps;
#pragma unroll
    for (int dt = 0; dt < kD / 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= corr;
#pragma unroll
    for (int ks = 0; ks < kVB / 32; ++ks)
#pragma unroll
      for (int dt = 0; dt < kD / 16; ++dt) {
        const uint16_t* vr = &s_vt[16 * dt + col][32 * ks + quarter * 4];
        const uint2 v0 = *(const uint2*)vr;
        const uint2 v1 = *(const uint2*)(vr + 16);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_vbf16x8(make_uint4(v0.x, v0.y, v1.x, v1.y)), pb[ks], o[dt], 0, 0, 0);
      }
  }
  // the four lane quarters of a query hold disjoint keys under the same maximum
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (!rv) return;
  const size_t row = (size_t)t * p.H + h;
  if (p.nsplit == 1) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = p.out + row * kD;
#pragma unroll
    for (int dt = 0; dt < kD / 16; ++dt)
      *(uint2*)(orow + 16 * dt + quarter * 4) =
          make_uint2(pack2_bf16(o[dt][0] * inv, o[dt][1] * inv),
                     pack2_bf16(o[dt][2] * inv, o[dt][3] * inv));
    return;
  }
  float* part = p.part + (row * p.nsplit + split) * (kD + 2);
#pragma unroll
  for (int dt = 0; dt < kD / 16; ++dt)
    *(float4*)(part + 16 * dt + quarter * 4) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
  if (quarter == 0) {
    part[kD] = m;
    part[kD + 1] = l;
  }
}

struct VerifyPlan {
  int nsplit, chunk, qgroups;
};

VerifyPlan plan_verify(int n, int H, int KV, int max_ctx) {
  VerifyPlan vp;
  const int rows = n * (H / KV);
  vp.qgroups = (rows + 63) / 64;
  const int per_split = KV * vp.qgroups;
  const int max_ns = (max_ctx + kVB - 1) / kVB;
  int ns = (512 + per_split - 1) / per_split;
  ns = ns > max_ns ? max_ns : ns;
  ns = ns > kMaxSplit ? kMaxSplit : (ns < 1 ? 1 : ns);
  int chunk = (max_ctx + ns - 1) / ns;
  chunk = (chunk + kVB - 1) / kVB * kVB;
  vp.chunk = chunk;
  vp.nsplit = (max_ctx + chunk - 1) / chunk;
  return vp;
}

size_t verify_ws_bytes(int n, int H, int KV, int max_ctx) {
  const VerifyPlan vp = plan_verify(n, H, KV, max_ctx);
  if (vp.nsplit == 1) return 0;
  return (((size_t)n * H * vp.nsplit * (kD + 2) * sizeof(float)) + 255) & ~(size_t)255;
}

constexpr int kVerifyMaxTokens = 4096;

// ---------------------------------------------------------------------------------------------
// Library-owned scratch for iron_decode_attn_noalloc: the split-K partials of callers that cannot
// allocate. Each GPU the library runs on holds its own copy of this array (at its own address)
// until the process ends. Host code never passes the array's name to a kernel: in host code it is
// a stand-in, not a device address. The device address comes from hipGetSymbolAddress, looked up
// once per device with that device current, and is the only handle used afterwards.
// ---------------------------------------------------------------------------------------------
constexpr size_t kNoallocScratchBytes = IRON_ATTN_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_of_current_device(void** out, const char* fn);

}  // namespace

static __device__ __align__(256) unsigned char scratch[IRON_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {

int scratch_of_current_device(void** out, const char* fn) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return iron::fail(IRON_ERR_HIP, "%s: no current HIP device", fn);
  if (dev < 0 || dev >= kMaxDevices)
    return iron::fail(IRON_ERR_UNSUPPORTED, "%s: device %d (at most %d devices)", fn, dev,
                      kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return iron::fail(IRON_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn,
                        dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return IRON_OK;
}

// Validation and launch shared by iron_decode_attn and iron_decode_attn_noalloc.
int decode_attn_entry(const char* fn, const uint16_t* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, long long kv_sb, long long kv_sh, long long kv_st,
                      const int32_t* ctx_len, int ctx_const, uint16_t* out, int B, int H, int KV,
                      int D, int max_ctx, float scale, int acc, void* workspace,
                      size_t workspace_bytes, bool noalloc, void* stream) {
  if (!q || !k_cache || !v_cache || !out) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  int st = check_attn_shape(fn, B, H, KV, D, max_ctx);
  if (st) return st;
  if (kv_st % 8 || kv_sh % 8 || kv_sb % 8 || !iron::aligned(k_cache, 16) ||
      !iron::aligned(v_cache, 16) || !iron::aligned(q, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: K/V/Q rows must be 16-byte aligned", fn);
  if (!ctx_len && (ctx_const < 0 || ctx_const > max_ctx))
    return iron::fail(IRON_ERR_SHAPE, "%s: ctx_const=%d outside [0, %d]", fn, ctx_const, max_ctx);
  if (acc != IRON_ACCUM_F64 && acc != IRON_ACCUM_F32)
    return iron::fail(IRON_ERR_SHAPE, "%s: unknown accumulation mode %d", fn, acc);
  if (noalloc) {
    const size_t need = attn_ws_bytes(B, H, KV, max_ctx);
    if (need > kNoallocScratchBytes)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: the split partials of B=%d H=%d max_ctx=%d need "
                        "%zu bytes, more than the %zu-byte scratch (use iron_decode_attn with a "
                        "workspace)", fn, B, H, max_ctx, need, kNoallocScratchBytes);
    workspace_bytes = kNoallocScratchBytes;
    if ((st = scratch_of_current_device(&workspace, fn))) return st;
  }
  AttnParams p = {};
  p.q = q;
  p.k = const_cast<uint16_t*>(k_cache);
  p.v = const_cast<uint16_t*>(v_cache);
  p.sb = kv_sb;
  p.sh = kv_sh;
  p.st = kv_st;
  p.ctx_len = ctx_len;
  p.ctx_const = ctx_const;
  p.max_ctx = max_ctx;
  p.out = out;
  p.H = H;
  p.KV = KV;
  p.scale = (double)scale;
  return launch_attention(p, false, acc, B, workspace, workspace_bytes, (hipStream_t)stream,
                          fn);
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
                     float scale, int acc, void* workspace, size_t workspace_bytes,
                     void* stream) {
  iron::clear_error();
  return decode_attn_entry("iron_decode_attn", q, k_cache, v_cache, kv_sb, kv_sh, kv_st, ctx_len,
                           ctx_const, out, B, H, KV, D, max_ctx, scale, acc, workspace,
                           workspace_bytes, false, stream);
}

int iron_decode_attn_noalloc(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                             long long kv_sb, long long kv_sh, long long kv_st,
                             const int32_t* ctx_len, int ctx_const, uint16_t* out, int B, int H,
                             int KV, int D, int max_ctx, float scale, int acc, void* stream) {
  iron::clear_error();
  return decode_attn_entry("iron_decode_attn_noalloc", q, k_cache, v_cache, kv_sb, kv_sh, kv_st,
                           ctx_len, ctx_const, out, B, H, KV, D, max_ctx, scale, acc, nullptr, 0,
                           true, stream);
}

size_t iron_qkv_attn_workspace(int B, int D, int Hq, int Hkv, int HD, int max_seq) {
  if (B <= 0 || D <= 0 || Hq <= 0 || Hkv <= 0 || HD != kD || Hq % Hkv || max_seq <= 0) return 0;
  return iron::qkv_raw_bytes(B, D, (Hq + 2 * Hkv) * HD) + attn_ws_bytes(B, Hq, Hkv, max_seq) +
         256;
}

int iron_qkv_attn(const uint16_t* cur, const uint16_t* n_in, const void* wqkv,
                  const uint16_t* n_qn, const uint16_t* n_kn, const uint16_t* ang,
                  uint16_t* k_cache, uint16_t* v_cache, long long kv_sb, long long kv_sh,
                  long long kv_st, const int32_t* pos, uint16_t* out, int B, int D, int HD, int Hq,
                  int Hkv, int max_seq, int G, int tile_m, int domain, float eps, float scale,
                  int acc, void* workspace, size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_qkv_attn";
  if (!cur || !n_in || !n_qn || !n_kn || !ang || !k_cache || !v_cache || !pos || !out)
    return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  int st = check_attn_shape(fn, B, Hq, Hkv, HD, max_seq);
  if (st) return st;
  if (D <= 0 || D % 16) return iron::fail(IRON_ERR_SHAPE, "%s: bad hidden size D=%d", fn, D);
  if (kv_st % 8 || kv_sh % 8 || kv_sb % 8 || !iron::aligned(k_cache, 16) ||
      !iron::aligned(v_cache, 16) || !iron::aligned(ang, 16) || !iron::aligned(n_qn, 16) ||
      !iron::aligned(n_kn, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: K/V rows, angles and norm weights must be 16-byte "
                      "aligned", fn);
  const int M = (Hq + 2 * Hkv) * HD;
  st = iron::check_wire(fn, wqkv, M, D, G, tile_m, domain);
  if (st) return st;
  const size_t need = iron_qkv_attn_workspace(B, D, Hq, Hkv, HD, max_seq);
  if (!workspace || workspace_bytes < need)
    return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                      need);
  if (!iron::aligned(workspace, 256))
    return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
  hipStream_t s = (hipStream_t)stream;
  uint16_t* raw = iron::qkv_raw_of(workspace);
  const size_t raw_bytes = iron::qkv_raw_bytes(B, D, M);
  st = iron::qkv_raw_internal(wqkv, cur, n_in, workspace, raw_bytes, B, M, D, G, tile_m, domain,
                              eps, s, fn);
  if (st) return st;
  AttnParams p = {};
  p.raw = raw;
  p.n_qn = n_qn;
  p.n_kn = n_kn;
  p.ang = ang;
  p.pos = pos;
  p.eps = (double)eps;
  p.k = k_cache;
  p.v = v_cache;
  p.sb = kv_sb;
  p.sh = kv_sh;
  p.st = kv_st;
  p.max_ctx = max_seq;
  p.out = out;
  p.H = Hq;
  p.KV = Hkv;
  p.scale = (double)scale;
  return launch_attention(p, true, acc, B, (char*)workspace + raw_bytes,
                          workspace_bytes - raw_bytes, s, fn);
}


size_t iron_decode_attn_verify_workspace(int n_new, int H, int KV, int D, int max_ctx) {
  if (n_new <= 0 || n_new > kVerifyMaxTokens || H <= 0 || KV <= 0 || D != kD || H % KV ||
      max_ctx <= 0)
    return 0;
  const size_t n = verify_ws_bytes(n_new, H, KV, max_ctx);
  return n ? n : 256;
}

int iron_decode_attn_verify(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            long long kv_sh, long long kv_st, const int32_t* base,
                            int base_const, int causal, uint16_t* out, int n_new, int H, int KV,
                            int D, int max_ctx, float scale, void* workspace,
                            size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_decode_attn_verify";
  if (!q || !k_cache || !v_cache || !out) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  int st = check_attn_shape(fn, 1, H, KV, D, max_ctx);
  if (st) return st;
  if (n_new <= 0 || n_new > kVerifyMaxTokens)
    return iron::fail(IRON_ERR_SHAPE, "%s: n_new=%d outside [1, %d]", fn, n_new,
                      kVerifyMaxTokens);
  if (kv_st % 8 || kv_sh % 8 || kv_st < kD || !iron::aligned(k_cache, 16) ||
      !iron::aligned(v_cache, 16) || !iron::aligned(q, 16) || !iron::aligned(out, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: Q/O/K/V rows must be 16-byte aligned", fn);
  if (!base && (base_const < 0 || base_const > max_ctx))
    return iron::fail(IRON_ERR_SHAPE, "%s: base_const=%d outside [0, %d]", fn, base_const,
                      max_ctx);
  if (!(scale > 0.f)) return iron::fail(IRON_ERR_SHAPE, "%s: scale must be positive", fn);
  const VerifyPlan vp = plan_verify(n_new, H, KV, max_ctx);
  VerifyParams p = {};
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.sh = kv_sh;
  p.st = kv_st;
  p.base_ptr = base;
  p.base_const = base_const;
  p.causal = causal ? 1 : 0;
  p.n = n_new;
  p.H = H;
  p.KV = KV;
  p.HG = H / KV;
  p.S = max_ctx;
  p.rows = n_new * p.HG;
  p.chunk = vp.chunk;
  p.nsplit = vp.nsplit;
  p.qgroups = vp.qgroups;
  p.c = scale * 1.4426950408889634f;
  p.out = out;
  if (vp.nsplit > 1) {
    const size_t need = verify_ws_bytes(n_new, H, KV, max_ctx);
    if (!workspace || workspace_bytes < need)
      return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                        need);
    if (!iron::aligned(workspace, 256))
      return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
    p.part = (float*)workspace;
  }
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(verify_attn_kernel, dim3(vp.nsplit, KV * vp.qgroups), dim3(256), 0, s, p);
  st = iron::check_launch(fn);
  if (st || vp.nsplit == 1) return st;
  AttnParams mp = {};
  mp.part = p.part;
  mp.nsplit = vp.nsplit;
  mp.H = H;
  mp.out = out;
  hipLaunchKernelGGL(attn_merge_kernel<true>, dim3(H, n_new), dim3(256), 0, s, mp);
  return iron::check_launch(fn);
}

}  // extern "C"
