// Fused decode QKV head: RMSNorm prologue + concatenated int8 QKV GEMV, then a per-head
// epilogue (QK RMSNorm, two-halves RoPE, KV-cache append).
//
// Reference: QKVHeadDataParallelOurs (iron/operators/qkv_head_dp/op_ours.py:31-262, op.py:20-231,
// design_ours_kvlayout.py:399-447 core, :640-692 KV drains); golden
// iron/operators/qkv_head_dp/reference.py:13-33, composed of rms_norm/reference.py:8-17 and
// rope/reference.py:118-154 (method_type 0, TWO_HALVES, interleaved [cos, sin] angle row).
// Kernel numerics followed: rms_norm.cc:83-147 (fp32, one bf16 rounding), generic/rope.cc:42-83.
#include "common.h"
#include "internal.h"

namespace {

constexpr int kHD = 128;

struct QkvEpiParams {
  const uint16_t* raw;   // [B][(Hq + 2 Hkv) * HD] bf16
  const uint16_t* n_qn;
  const uint16_t* n_kn;
  const uint16_t* ang;
  int ang_by_pos;
  uint16_t* q_out;       // [B][Hq*HD]
  uint16_t* k_cache;
  uint16_t* v_cache;
  long long sb, sh, st;
  const int32_t* pos;    // [B]
  int Hq, Hkv, max_seq;
  float eps;
};

// grid (Hq + 2*Hkv, B), 128 threads: one thread per head dimension. fp64 math (the exact value
// of the golden's closed forms), bf16 at the reference's boundaries: the normalised head and the
// rotated head are each rounded once (qkv_head_dp/reference.py:27-32).
__global__ __launch_bounds__(128) void qkv_epilogue_kernel(QkvEpiParams p) {
  const int head = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int nheads = p.Hq + 2 * p.Hkv;
  // every global load is issued before the first reduction
  const uint16_t hraw = p.raw[((size_t)b * nheads + head) * kHD + d];
  const int pos = p.pos ? p.pos[b] : 0;
  const bool pos_ok = pos >= 0 && pos < p.max_seq;
  const bool is_v = head >= p.Hq + p.Hkv;
  const uint16_t* nw = head < p.Hq ? p.n_qn : p.n_kn;
  const uint16_t hw = is_v ? (uint16_t)0 : nw[d];
  const int i = d & (kHD / 2 - 1);
  const uint16_t* arow = p.ang + (size_t)(p.ang_by_pos ? (pos_ok ? pos : 0) : b) * kHD;
  const uint16_t hc = is_v ? (uint16_t)0 : arow[2 * i];
  const uint16_t hs = is_v ? (uint16_t)0 : arow[2 * i + 1];
  if (is_v) {  // v head: the raw bf16 value goes to the cache unchanged
    const int hv = head - p.Hq - p.Hkv;
    if (pos_ok) p.v_cache[(size_t)b * p.sb + (size_t)hv * p.sh + (size_t)pos * p.st + d] = hraw;
    return;
  }
  __shared__ double s_red[2];
  __shared__ double s_y[kHD];
  const double x = bf16_to_f32(hraw);
  double ss = wave_sum_d(x * x);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = s_red[0] + s_red[1];
  const double inv = inv_rms(ss, kHD, (double)p.eps);
  const double y = bf16_to_f32(f64_to_bf16((x * inv) * (double)bf16_to_f32(hw)));
  s_y[d] = y;
  __syncthreads();
  const double c = bf16_to_f32(hc), s = bf16_to_f32(hs);
  double r;
  if (d < kHD / 2) {
    r = y * c - s_y[d + kHD / 2] * s;   // y1*cos - y2*sin  (exact in fp64)
  } else {
    r = y * c + s_y[d - kHD / 2] * s;   // y2*cos + y1*sin
  }
  const uint16_t hr = f64_to_bf16(r);
  if (head < p.Hq) {
    p.q_out[((size_t)b * p.Hq + head) * kHD + d] = hr;
  } else if (pos_ok) {
    const int hk = head - p.Hq;
    p.k_cache[(size_t)b * p.sb + (size_t)hk * p.sh + (size_t)pos * p.st + d] = hr;
  }
}

}  // namespace

namespace iron {

static size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// Bytes of the raw-QKV stage: the GEMM's split-K counters (kGemmCtrBytes, for every B), raw
// (bf16 [B][M]), and for B > 4 (MFMA) the normalised input (bf16 [B][D]) and the split-K partials.
size_t qkv_raw_bytes(int B, int D, int M) {
  size_t n = kGemmCtrBytes + round256((size_t)B * M * 2);
  if (B > kGemvMaxBatch) n += round256((size_t)B * D * 2) + gemm_workspace_bound(M, false);
  return n;
}

// raw = bf16(Wqkv . bf16(RMSNorm(cur) * n_in)): the fused-prologue GEMV for B <= 4; for larger
// batches the normalisation runs once per row and the product on MFMA.
int qkv_raw_internal(const void* wqkv, const uint16_t* cur, const uint16_t* n_in, void* ws,
                     size_t ws_bytes, int B, int M, int D, int G, int tile_m, int domain,
                     float eps, hipStream_t s, const char* fn) {
  uint16_t* raw = qkv_raw_of(ws);
  if (B <= kGemvMaxBatch)
    return gemv_rms_internal(wqkv, cur, n_in, raw, B, M, D, G, tile_m, domain, eps, s, fn);
  int st = gemm_check(fn, B, M, D, G);
  if (st) return st;
  uint16_t* hn = (uint16_t*)((char*)raw + round256((size_t)B * M * 2));
  char* part = (char*)hn + round256((size_t)B * D * 2);
  st = rmsnorm_launch(cur, n_in, hn, B, D, eps, s);
  if (st) return st;
  return gemm_w8_launch(wqkv, nullptr, M, D, G, tile_m, domain, hn, 0, B, D, GEMM_EPI_BF16,
                        raw, M, 0, nullptr, nullptr, 0, (unsigned int*)ws, part,
                        ws_bytes - (size_t)(part - (char*)ws), s, fn);
}

}  // namespace iron

extern "C" {

size_t iron_qkv_head_workspace(int B, int D, int Hq, int Hkv, int HD) {
  if (B <= 0 || D <= 0 || Hq <= 0 || Hkv <= 0 || HD <= 0) return 0;
  return iron::qkv_raw_bytes(B, D, (Hq + 2 * Hkv) * HD);
}

int iron_qkv_head(const uint16_t* cur, const uint16_t* n_in, const void* wqkv,
                  const uint16_t* n_qn, const uint16_t* n_kn, const uint16_t* ang, int ang_by_pos,
                  uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, long long kv_sb,
                  long long kv_sh, long long kv_st, const int32_t* pos, int B, int D, int HD,
                  int Hq, int Hkv, int max_seq, int G, int tile_m, int domain, float eps,
                  void* workspace, size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_qkv_head";
  if (!cur || !n_in || !n_qn || !n_kn || !ang || !q_out || !k_cache || !v_cache || !pos)
    return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  if (HD != kHD) return iron::fail(IRON_ERR_UNSUPPORTED, "%s: head_dim %d (only 128)", fn, HD);
  if (B <= 0 || D <= 0 || Hq <= 0 || Hkv <= 0 || max_seq <= 0 || D % 16)
    return iron::fail(IRON_ERR_SHAPE, "%s: bad shape B=%d D=%d Hq=%d Hkv=%d S=%d", fn, B, D, Hq,
                      Hkv, max_seq);
  const int M = (Hq + 2 * Hkv) * HD;
  int st = iron::check_wire(fn, wqkv, M, D, G, tile_m, domain);
  if (st) return st;
  const size_t need = iron_qkv_head_workspace(B, D, Hq, Hkv, HD);
  if (!workspace || workspace_bytes < need)
    return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                      need);
  if (!iron::aligned(workspace, 256))
    return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
  hipStream_t s = (hipStream_t)stream;
  uint16_t* raw = iron::qkv_raw_of(workspace);
  st = iron::qkv_raw_internal(wqkv, cur, n_in, workspace, workspace_bytes, B, M, D, G, tile_m,
                              domain, eps, s, fn);
  if (st) return st;
  QkvEpiParams p = {};
  p.raw = raw;
  p.n_qn = n_qn;
  p.n_kn = n_kn;
  p.ang = ang;
  p.ang_by_pos = ang_by_pos;
  p.q_out = q_out;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.sb = kv_sb;
  p.sh = kv_sh;
  p.st = kv_st;
  p.pos = pos;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.max_seq = max_seq;
  p.eps = eps;
  hipLaunchKernelGGL(qkv_epilogue_kernel, dim3(Hq + 2 * Hkv, B), dim3(kHD), 0, s, p);
  return iron::check_launch(fn);
}

}  // extern "C"
