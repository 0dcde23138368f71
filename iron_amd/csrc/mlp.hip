// Fused decode SwiGLU MLP block (optionally with the attention output projection, fuse_o).
//
// Reference: SwiGLUMLPDataParallelOurs (iron/operators/swiglu_mlp_dp/op_ours.py:46-582, base
// op.py:22-227, design core design_ours_int8.py:753-975); golden
// iron/operators/swiglu_mlp_dp/reference.py:8-67 (fp32 x1/hf/g/u/gh, exact sigmoid,
// a = bf16(Wo @ cx) under fuse_o) with the exact fp32 dequant of op_ours.py:515-582.
//
// Three stream-ordered launches, each a weight-streaming GEMV of gemv.hip:
//   1. (fuse_o) a = bf16(Wo . cx)                          [D x QD]
//   2. hf = RMSNorm(cur + a) * n_pf in LDS, g/u rows of Wg/Wu, gh = silu(g)*u (fp32)   [FF x D]
//   3. nxt = bf16((cur + a) + Wd . gh)                     [D x FF]
// The kernel boundaries are the device-wide all-gathers the reference performs through its
// a_scratch / gh_scratch DRAM round trips (design_ours_int8.py:1122-1135, 1179-1206).
#include "common.h"
#include "internal.h"

namespace iron {
int gemv_swiglu_internal(const void* wg, const void* wu, const uint16_t* cur,
                         const uint16_t* a, const uint16_t* n_pf, float* gh, int B, int D,
                         int FF, int G, int tile_m, int domain, float eps, hipStream_t stream);
int gemv_down_internal(const void* wd, const float* gh, const uint16_t* cur, const uint16_t* a,
                       uint16_t* nxt, int B, int D, int FF, int G, int tile_m, int domain,
                       hipStream_t stream);
}

extern "C" {

static size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// Layout: the GEMM's split-K counters (kGemmCtrBytes, for every B), then for B <= 4 (GEMV):
// gh (fp32 [B][FF]) | a (bf16 [B][D]); for B > 4 (MFMA): gh (three bf16 planes [3][B][FF] of
// the fp32 values) | a (bf16 [B][D]) | hf (planes [3][B][D]; with the folded RMSNorm, the
// producer's tile sums of squares [D / 64][16] fp64 instead) | the split-K partials (shared by
// the GEMMs, which run in sequence).
size_t iron_swiglu_mlp_workspace(int B, int D, int FF) {
  if (B <= 0 || D <= 0 || FF <= 0) return 0;
  if (B <= iron::kGemvMaxBatch)
    return iron::kGemmCtrBytes + round256((size_t)B * FF * sizeof(float)) +
           round256((size_t)B * D * 2);
  size_t part = iron::gemm_workspace_bound(FF, true);
  const size_t pd = iron::gemm_workspace_bound(D, false);
  part = part > pd ? part : pd;
  return iron::kGemmCtrBytes + round256((size_t)3 * B * FF * 2) + round256((size_t)B * D * 2) +
         round256((size_t)3 * B * D * 2) + part;
}

int iron_swiglu_mlp(const uint16_t* cur, const uint16_t* cx_or_a, const uint16_t* n_pf,
                    const void* wo, const void* wg, const void* wu, const void* wd,
                    uint16_t* nxt, uint16_t* a_out, int B, int D, int FF, int QD, int G,
                    int tile_m_o, int tile_m_gu, int tile_m_d, int domain, float eps,
                    void* workspace, size_t workspace_bytes, void* stream) {
  iron::clear_error();
  const char* fn = "iron_swiglu_mlp";
  if (!cur || !cx_or_a || !n_pf || !nxt) return iron::fail(IRON_ERR_NULL, "%s: null tensor", fn);
  if (B <= 0 || D <= 0 || FF <= 0 || D % 16 || FF % 16)
    return iron::fail(IRON_ERR_SHAPE, "%s: bad shape B=%d D=%d FF=%d", fn, B, D, FF);
  if (!iron::aligned(cur, 16) || !iron::aligned(cx_or_a, 16) || !iron::aligned(n_pf, 16) ||
      !iron::aligned(nxt, 16))
    return iron::fail(IRON_ERR_ALIGN, "%s: activations and norm weight must be 16-byte aligned",
                      fn);
  int st = iron::check_wire(fn, wg, FF, D, G, tile_m_gu, domain);
  if (st) return st;
  st = iron::check_wire(fn, wu, FF, D, G, tile_m_gu, domain);
  if (st) return st;
  st = iron::check_wire(fn, wd, D, FF, G, tile_m_d, domain);
  if (st) return st;
  if (wo) {
    if (QD <= 0 || QD % 16) return iron::fail(IRON_ERR_SHAPE, "%s: fuse_o needs QD > 0", fn);
    st = iron::check_wire(fn, wo, D, QD, G, tile_m_o, domain);
    if (st) return st;
  }
  const size_t need = iron_swiglu_mlp_workspace(B, D, FF);
  if (!workspace || workspace_bytes < need)
    return iron::fail(IRON_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", fn, workspace_bytes,
                      need);
  if (!iron::aligned(workspace, 256))
    return iron::fail(IRON_ERR_ALIGN, "%s: workspace not 256-byte aligned", fn);
  hipStream_t s = (hipStream_t)stream;
  unsigned int* ctr = (unsigned int*)workspace;
  char* const base = (char*)workspace + iron::kGemmCtrBytes;
  workspace_bytes -= iron::kGemmCtrBytes;
  if (B > iron::kGemvMaxBatch) {
    // MFMA path: the prologue (x1 = cur + a, hf = RMSNorm(x1) * n_pf in fp32) folds into Wo's
    // epilogue and the gate/up GEMM's staging (with Wo, when the plans allow), or into the
    // staged gate/up GEMM alone, or runs once per row in its own kernel; then the GEMMs with the
    // SwiGLU / residual epilogues
    if ((st = iron::gemm_check(fn, B, FF, D, G)) || (st = iron::gemm_check(fn, B, D, FF, G)))
      return st;
    if (wo && (st = iron::gemm_check(fn, B, D, QD, G))) return st;
    uint16_t* gh = (uint16_t*)base;
    uint16_t* a_buf = (uint16_t*)(base + round256((size_t)3 * B * FF * 2));
    uint16_t* hf = (uint16_t*)((char*)a_buf + round256((size_t)B * D * 2));
    char* part = (char*)hf + round256((size_t)3 * B * D * 2);
    const size_t part_bytes = workspace_bytes - (size_t)(part - base);
    const uint16_t* a = cx_or_a;
    // with the output projection, the residual RMSNorm folds into it and the gate/up GEMM when
    // their plans allow (iron::GemmResNorm; its tile sums take hf's place in the workspace)
    const bool fold = wo && iron::gemm_resnorm_foldable(D, QD, FF);
    iron::GemmResNorm rn = {(double*)hf, cur, nullptr, n_pf, D, eps};
    if (wo) {
      uint16_t* dst = a_out ? a_out : a_buf;
      st = iron::gemm_w8_launch(wo, nullptr, D, QD, G, tile_m_o, domain, cx_or_a, 0, B, QD,
                                iron::GEMM_EPI_BF16, dst, D, 0, nullptr, nullptr, 0, ctr, part,
                                part_bytes, s, fn, fold ? &rn : nullptr);
      if (st) return st;
      a = dst;
    }
    if (fold) {
      rn.a = a;
      st = iron::gemm_w8_launch(wg, wu, FF, D, G, tile_m_gu, domain, nullptr, 0, B, D,
                                iron::GEMM_EPI_SWIGLU_PLANES, gh, FF, (size_t)B * FF, nullptr,
                                nullptr, 0, ctr, part, part_bytes, s, fn, &rn);
    } else if (iron::gemm_selfnorm_foldable(B, D, FF)) {
      // no producer to fold into: the gate/up GEMM sums each row's squares itself
      const iron::GemmResNorm rs = {nullptr, cur, a, n_pf, D, eps};
      st = iron::gemm_w8_launch(wg, wu, FF, D, G, tile_m_gu, domain, nullptr, 0, B, D,
                                iron::GEMM_EPI_SWIGLU_PLANES, gh, FF, (size_t)B * FF, nullptr,
                                nullptr, 0, ctr, part, part_bytes, s, fn, &rs);
    } else {
      st = iron::res_rmsnorm_planes_launch(cur, a, n_pf, hf, B, D, eps, s);
      if (st) return st;
      st = iron::gemm_w8_launch(wg, wu, FF, D, G, tile_m_gu, domain, hf, (size_t)B * D, B, D,
                                iron::GEMM_EPI_SWIGLU_PLANES, gh, FF, (size_t)B * FF, nullptr,
                                nullptr, 0, ctr, part, part_bytes, s, fn);
    }
    if (st) return st;
    return iron::gemm_w8_launch(wd, nullptr, D, FF, G, tile_m_d, domain, gh, (size_t)B * FF, B,
                                FF, iron::GEMM_EPI_RES_BF16, nxt, D, 0, cur, a, D, ctr, part,
                                part_bytes, s, fn);
  }
  float* gh = (float*)base;
  const size_t gh_bytes = round256((size_t)B * FF * sizeof(float));
  const uint16_t* a = cx_or_a;
  if (wo) {
    uint16_t* a_buf = a_out ? a_out : (uint16_t*)(base + gh_bytes);
    st = iron_gemv_w8a16(wo, cx_or_a, a_buf, B, D, QD, G, tile_m_o, domain, stream);
    if (st) return st;
    a = a_buf;
  }
  st = iron::gemv_swiglu_internal(wg, wu, cur, a, n_pf, gh, B, D, FF, G, tile_m_gu, domain, eps,
                                  s);
  if (st) return st;
  return iron::gemv_down_internal(wd, gh, cur, a, nxt, B, D, FF, G, tile_m_d, domain, s);
}

}  // extern "C"
