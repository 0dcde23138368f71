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

size_t iron_swiglu_mlp_workspace(int B, int D, int FF) {
  if (B <= 0 || D <= 0 || FF <= 0) return 0;
  size_t gh = ((size_t)B * FF * sizeof(float) + 255) & ~(size_t)255;
  size_t a = ((size_t)B * D * 2 + 255) & ~(size_t)255;
  return gh + a;
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
  float* gh = (float*)workspace;
  const size_t gh_bytes = ((size_t)B * FF * sizeof(float) + 255) & ~(size_t)255;
  const uint16_t* a = cx_or_a;
  if (wo) {
    uint16_t* a_buf = a_out ? a_out : (uint16_t*)((char*)workspace + gh_bytes);
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
