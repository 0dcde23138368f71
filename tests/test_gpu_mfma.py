"""GPU parity of the MFMA batched-decode path against the CPU oracle: the fused QKV head and MLP
route batches 5..16 there (GEMVInt8 runs 5..15 on the exact batched GEMV, bit-exact in
test_gpu_ops.py), and the GEMM entry point iron_gemm_w8a16 itself takes any batch 1..16, which
test_gemm_mfma covers directly.

The MFMA path sums each 32-wide group of exact q*x products in fp32 (v_mfma_f32_16x16x32_bf16)
and applies the group scales in fp64, so its results are within the fp32 rounding of the exact
value rather than correctly rounded. Two bars per case, both written here:
  * the north-star tolerance rel 1e-2 / abs 1e-2 against the exact oracle and the literal golden;
  * every bf16 output within one bf16 ulp of the exact oracle's (the fp32 group sums can move a
    value across a bf16 rounding boundary, never further), with the count of bit-exact outputs
    printed.
"""

import numpy as np
import pytest
import torch

from iron_amd.common.test_utils import verify_buffer
from iron_amd.operators import MHA, QKVHeadAttention, SwiGLUMLPDataParallelOurs
from iron_amd.operators.wire import pack_wire
from oracle import attention as oatt
from oracle import blocks as oblk
from oracle import gemv as ogemv
from oracle import norms as onorm
from oracle.numerics import LITERAL

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def assert_within_one_ulp(got: torch.Tensor, want: torch.Tensor, what: str):
    g = got.cpu().float().reshape(-1)
    w = want.cpu().float().reshape(-1)
    exact = int((g == w).sum())
    # one bf16 ulp of the larger magnitude (8 significant bits)
    mag = torch.maximum(g.abs(), w.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    bad = int(((g - w).abs() > ulp).sum())
    print(f"{what}: {exact}/{w.numel()} bit-exact, {bad} beyond one ulp", flush=True)
    assert bad == 0, f"{what}: {bad} of {w.numel()} outputs differ by more than one bf16 ulp"


def assert_within_mlp_bound(got, want, cur, a, n_pf, wg, wu, wd, eps, what):
    """nxt of the MFMA MLP against the exact oracle: within one bf16 ulp, or within 2^-17 of the
    magnitude sum_k |Wd[r, k] gh[k]| that the down GEMM's fp32 group sums round against. The fp32
    group sums of gate/up and down each carry a relative error of a few 2^-24 of that magnitude;
    where the residual cancels (x1 + d small), that is more than one ulp of nxt."""
    from oracle.blocks import _sigmoid_stable
    from oracle.gemv import dequant_f, gemv
    from oracle.norms import rms_norm
    x1 = cur.reshape(-1, cur.shape[-1]).float() + a.reshape(-1, cur.shape[-1]).float()
    hf = rms_norm(x1, n_pf, eps, out_bf16=False)
    g, u = gemv(dequant_f(*wg), hf), gemv(dequant_f(*wu), hf)
    gh = ((g * _sigmoid_stable(g)) * u).float().double()
    mag = gh.abs() @ dequant_f(*wd).double().abs().T
    g_ = got.cpu().double().reshape(mag.shape)
    w_ = want.cpu().double().reshape(mag.shape)
    m_ = torch.maximum(g_.abs(), w_.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(m_)) - 7)
    err = (g_ - w_).abs()
    bad = int((err > torch.maximum(ulp, mag * 2.0 ** -17)).sum())
    print(f"{what}: {int((err == 0).sum())}/{err.numel()} bit-exact, {int((err > ulp).sum())} "
          f"beyond one ulp, worst error / magnitude {float((err / mag.clamp_min(1e-30)).max()):.3g}",
          flush=True)
    assert bad == 0, f"{what}: {bad} outputs beyond both bounds"


def _weights(M, K, G, gen):
    q = torch.randint(-127, 128, (M, K), generator=gen, dtype=torch.int16)
    s = (torch.randn(M, K // G, generator=gen) * 0.02).abs().to(torch.bfloat16)
    return q, s


@pytest.mark.parametrize("M,K,G,tile_m,B,domain", [
    (6144, 4096, 32, 4, 16, "signed"),    # Qwen3-8B fused QKV, BASELINE config 5 batch
    (4096, 12288, 32, 4, 16, "signed"),   # Qwen3-8B down projection
    (6144, 2048, 32, 12, 8, "signed"),    # Qwen3-1.7B gate/up at batch 8 (the GEMM entry point)
    (256, 512, 64, 16, 5, "biased"),
    (64, 128, 128, 8, 11, "signed"),
])
def test_gemm_mfma(M, K, G, tile_m, B, domain):
    _say(f"gemm_mfma M={M} K={K} G={G} tile_m={tile_m} B={B} {domain}")
    import ctypes  # noqa: F401
    from iron_amd import _lib
    lib = _lib.load()
    gen = torch.Generator().manual_seed(M + K + B)
    q, s = _weights(M, K, G, gen)
    x = torch.randn(B, K, generator=gen).to(torch.bfloat16)
    wire = pack_wire(q, s, tile_m, domain).to(DEV)
    ws = torch.zeros(lib.iron_gemm_w8a16_workspace(B, M, K, G), dtype=torch.uint8, device=DEV)
    y = torch.zeros(B, M, dtype=torch.bfloat16, device=DEV)
    dom = _lib.IRON_DOMAIN_SIGNED if domain == "signed" else _lib.IRON_DOMAIN_BIASED
    xd = x.to(DEV)

    def fn(w_, x_, y_):
        _lib.check(lib.iron_gemm_w8a16(w_.data_ptr(), x_.data_ptr(), y_.data_ptr(), B, M, K, G,
                                       tile_m, dom, ws.data_ptr(), ws.numel(),
                                       _lib.stream_handle()), "iron_gemm_w8a16")

    fn(wire, xd, y)
    torch.cuda.synchronize()
    exact = ogemv.gemv_exact(q, s, x).float().to(torch.bfloat16)
    assert not verify_buffer(y.cpu(), "y", exact, rel_tol=RTOL, abs_tol=ATOL)
    literal = ogemv.gemv_exact(q, s, x, dt=LITERAL).to(torch.bfloat16)
    assert not verify_buffer(y.cpu(), "y", literal, rel_tol=RTOL, abs_tol=ATOL)
    assert_within_one_ulp(y, exact, "gemm")
    y2 = torch.zeros_like(y)                  # deterministic: a second call gives the same bits
    fn(wire, xd, y2)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu().view(torch.int16), y2.cpu().view(torch.int16))


@pytest.mark.parametrize("D,FF,QD,fuse_o,G,B", [
    (2048, 6144, 0, False, 32, 8),      # BASELINE config 2, batch 8 (Qwen3-1.7B MLP)
    (1024, 3072, 2048, True, 32, 5),    # Qwen3-0.6B chain arm, the smallest MFMA batch
    (2048, 6144, 0, False, 32, 16),     # Qwen3-1.7B MLP at batch 16
    (1024, 3072, 2048, True, 32, 16),   # Qwen3-0.6B chain arm at batch 16
    (4096, 12288, 4096, True, 32, 16),  # Qwen3-8B layer MLP at BASELINE config 5 (B=16)
    (2560, 9728, 4096, True, 32, 16),   # Qwen3-4B: FF % D != 0 (the chunked-down arm)
    # gate/up on the register-streamed form (dual, K = D >= 4096) at the other group sizes and
    # a batch below 16 (rows past B read as zero)
    (4096, 1024, 0, False, 64, 5),
    (4096, 2048, 0, False, 128, 16),
    (4096, 1024, 0, False, 32, 8),
    # the residual RMSNorm folded into Wo (tile sums of squares) and the register-streamed gate/up
    # (hf staged from cur, a and the norm weight), at other group sizes and batches below 16
    (4096, 1024, 2048, True, 64, 5),
    (4096, 2048, 4096, True, 128, 9),
])
def test_swiglu_mlp_mfma(D, FF, QD, fuse_o, G, B):
    _say(f"swiglu mfma D={D} FF={FF} QD={QD} fuse_o={fuse_o} G={G} B={B}")
    gen = torch.Generator().manual_seed(D + FF + B)
    op = SwiGLUMLPDataParallelOurs(D=D, FF=FF, QD=QD or None, fuse_o=fuse_o, group_size=G,
                                   epsilon=1e-6, batch=B, kernel_source="mv_int8_signed.cc")

    def lin(M, K, std):
        return ogemv.rtn_quantize(torch.randn(M, K, generator=gen) * std, G)

    wg, wu, wd = lin(FF, D, 0.05), lin(FF, D, 0.05), lin(D, FF, 0.05)
    cur = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    n_pf = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16)
    wo = lin(D, QD, 0.05) if fuse_o else None
    cx = torch.randn(B, QD if fuse_o else D, generator=gen).to(torch.bfloat16)
    wires = {}
    if fuse_o:
        wires["Wo"] = pack_wire(*wo, op.tile_rows_o, "signed")
    wires["Wg"] = pack_wire(*wg, op.tile_rows_gu, "signed")
    wires["Wu"] = pack_wire(*wu, op.tile_rows_gu, "signed")
    wires["Wd"] = pack_wire(*wd, op.tile_rows_d, "signed")
    ws = torch.zeros(op.workspace_bytes(), dtype=torch.uint8, device=DEV)
    nxt = torch.zeros(B * D, dtype=torch.bfloat16, device=DEV)
    args = [cur.reshape(-1).to(DEV), cx.reshape(-1).to(DEV), n_pf.to(DEV)]
    args += [wires[k].view(torch.bfloat16).to(DEV) for k in ("Wo", "Wg", "Wu", "Wd") if k in wires]
    args.append(ws)
    a_s = torch.zeros(B * D, dtype=torch.bfloat16, device=DEV)
    if fuse_o:
        args.append(a_s)
    args.append(nxt)
    op.get_callable()(*args)
    torch.cuda.synchronize()
    # deterministic: a second call (split-K merge, folded RMSNorm sums) gives the same bits
    first = nxt.clone()
    op.get_callable()(*args)
    torch.cuda.synchronize()
    assert torch.equal(first.cpu().view(torch.int16), nxt.cpu().view(torch.int16))
    want, want_a = oblk.swiglu_mlp(cur, cx, n_pf, wg, wu, wd, 1e-6, wo=wo)
    assert not verify_buffer(nxt.cpu(), "nxt", want, RTOL, ATOL)
    if fuse_o:
        # a = bf16(Wo . cx) is within one ulp of exact; a one-ulp step of a moves nxt by the same
        # amount through the residual x1 = cur + a, which is many ulps of a small (cancelled) nxt,
        # so the rest of the block is checked from the device's own a, stage by stage
        assert_within_one_ulp(a_s, want_a, "mlp a")
        a_dev = a_s.cpu().reshape(B, D)
        want, _ = oblk.swiglu_mlp(cur, a_dev, n_pf, wg, wu, wd, 1e-6)
        lit, _ = oblk.swiglu_mlp(cur, a_dev, n_pf, wg, wu, wd, 1e-6, dt=LITERAL)
    else:
        a_dev = cx
        lit, _ = oblk.swiglu_mlp(cur, cx, n_pf, wg, wu, wd, 1e-6, wo=wo, dt=LITERAL)
    assert not verify_buffer(nxt.cpu(), "nxt", lit, RTOL, ATOL)
    assert_within_mlp_bound(nxt, want, cur, a_dev, n_pf, wg, wu, wd, 1e-6, "mlp nxt")


def test_mlp_workspace_reused_across_batches(lib):
    """One workspace serves the MLP entry at every batch size: an MFMA call (B=16, split-K with
    in-kernel reduction), a GEMV call (B=3) on the same memory, then the MFMA call again. The
    split-K arrival counters sit in the first 16 KiB for every B, so the repeat gives the first
    call's bits, the GEMV call gives a fresh workspace's bits, and the counters end at zero."""
    import ctypes
    from iron_amd import _lib

    D, FF, G = 2048, 6144, 32
    _say(f"mlp workspace reuse D={D} FF={FF} B=16,3,16")
    gen = torch.Generator().manual_seed(77)

    qs = [ogemv.rtn_quantize(torch.randn(M, K, generator=gen) * 0.05, G)
          for M, K in ((FF, D), (FF, D), (D, FF))]
    wg, wu, wd = [pack_wire(*w, tm, "signed").to(DEV) for w, tm in zip(qs, (12, 12, 4))]
    nw = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16).to(DEV)
    cur = torch.randn(16, D, generator=gen).to(torch.bfloat16).to(DEV)
    a = torch.randn(16, D, generator=gen).to(torch.bfloat16).to(DEV)
    size = max(lib.iron_swiglu_mlp_workspace(16, D, FF), lib.iron_swiglu_mlp_workspace(3, D, FF))
    ws = torch.zeros(size, dtype=torch.uint8, device=DEV)

    def run(B, work):
        out = torch.zeros(B, D, dtype=torch.bfloat16, device=DEV)
        _lib.check(lib.iron_swiglu_mlp(cur.data_ptr(), a.data_ptr(), nw.data_ptr(), None,
                                       wg.data_ptr(), wu.data_ptr(), wd.data_ptr(),
                                       out.data_ptr(), None, B, D, FF, 0, G, 4, 12, 4, 0,
                                       ctypes.c_float(1e-6), work.data_ptr(), work.numel(),
                                       _lib.stream_handle()))
        torch.cuda.synchronize()
        return out.cpu()

    first = run(16, ws)
    small = run(3, ws)
    again = run(16, ws)
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))
    fresh = run(3, torch.zeros(size, dtype=torch.uint8, device=DEV))
    assert torch.equal(small.view(torch.int16), fresh.view(torch.int16))
    assert int(ws[:16384].count_nonzero()) == 0, "split-K counters not left at zero"
    want, _ = oblk.swiglu_mlp(cur.cpu(), a.cpu(), nw.cpu(), *qs, 1e-6)
    assert_within_mlp_bound(first, want, cur.cpu(), a.cpu(), nw.cpu(), *qs, 1e-6, "mlp B=16")


def test_qkv_attention_mfma_batch16():
    """Qwen3-8B heads (32 Q / 8 KV x 128, D = 4096) at batch 16: the raw QKV on MFMA, then the
    fused epilogue + attention; ragged positions."""
    D, Hq, Hkv, HD, S, G, tm, B = 4096, 32, 8, 128, 512, 32, 16, 16
    _say(f"qkv_attn mfma D={D} Hq={Hq} Hkv={Hkv} S={S} B={B}")
    gen = torch.Generator().manual_seed(4242)
    M = (Hq + 2 * Hkv) * HD
    q8, s = ogemv.rtn_quantize(torch.randn(M, D, generator=gen) * 0.05, G)
    cur = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    n_in = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16)
    n_qn = (torch.rand(HD, generator=gen) + 0.5).to(torch.bfloat16)
    n_kn = (torch.rand(HD, generator=gen) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, S, (B,), generator=gen)
    table = onorm.rope_angle_table(S, HD, 1e6)
    k0 = torch.randn(B, Hkv, S, HD, generator=gen).to(torch.bfloat16)
    v0 = torch.randn(B, Hkv, S, HD, generator=gen).to(torch.bfloat16)
    op = QKVHeadAttention(D=D, HD=HD, Hq=Hq, Hkv=Hkv, max_seq=S, group_size=G,
                          tile_size_input=tm, kv_layout="separate", batch=B, num_aie_columns=1,
                          kernel_source="mv_int8_signed.cc")
    fn = op.get_callable()
    fn.params.write(op.kv_offset_parameter, (pos * HD).numpy())
    kc, vc = k0.clone().to(DEV), v0.clone().to(DEV)
    out = torch.zeros(B * Hq * HD, dtype=torch.bfloat16, device=DEV)
    fn(cur.reshape(-1).to(DEV), n_in.to(DEV),
       pack_wire(q8, s, tm, "signed").view(torch.bfloat16).to(DEV), n_qn.to(DEV), n_kn.to(DEV),
       table[pos].reshape(-1).to(DEV), kc.reshape(-1), vc.reshape(-1), out)
    torch.cuda.synchronize()
    wq, wk, wv = oblk.qkv_head(cur, n_in, q8, s, n_qn, n_kn, table[pos], Hq, Hkv, HD, 1e-6)
    kk, vv = k0.clone(), v0.clone()
    for b in range(B):
        kk[b, :, int(pos[b])] = wk[b].reshape(Hkv, HD)
        vv[b, :, int(pos[b])] = wv[b].reshape(Hkv, HD)
    want = oatt.decode_attention(wq.reshape(B, Hq, HD), kk, vv, (pos + 1).tolist())
    assert not verify_buffer(out.cpu(), "attn", want.reshape(-1), RTOL, ATOL)
    # the cache rows written at each position hold the oracle's k and v (to one ulp: raw QKV
    # comes from the MFMA sums)
    for b in range(B):
        p = int(pos[b])
        assert_within_one_ulp(kc[b, :, p].cpu(), wk[b].reshape(Hkv, HD), f"k@{b}")


def test_qwen3_8b_layer_b16_context_8192():
    """One Qwen3-8B layer exactly as BASELINE config 5's decode step runs it (the bench's
    c5_decode_b16): B = 16 rows at positions near 8192, the fused QKV head + attention with the
    exact fp64 core (a split plan of several splits, each several tiles), then the MLP with the
    output projection folded in (Wo 4096 x 4096, gate/up 12288 x 4096 with the SwiGLU-planes
    epilogue, down 4096 x 12288) on MFMA. Attention within rel/abs 1e-2 of the oracle (its raw
    QKV comes from MFMA sums, one ulp from exact); the MLP, fed the device's attention output,
    within one bf16 ulp of the exact oracle."""
    D, Hq, Hkv, HD, S, G, FF, B = 4096, 32, 8, 128, 8192, 32, 12288, 16
    QD, M = Hq * HD, (Hq + 2 * Hkv) * HD
    _say(f"qwen3-8b layer B={B} context ~{S}")
    gen = torch.Generator().manual_seed(88)

    def lin(Mr, K, std=0.02):
        return ogemv.rtn_quantize(torch.randn(Mr, K, generator=gen) * std, G)

    wqkv, wo, wg, wu, wd = lin(M, D), lin(D, QD), lin(FF, D), lin(FF, D), lin(D, FF)
    cur = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    n_in, n_pf = [(torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16) for _ in range(2)]
    n_qn, n_kn = [(torch.rand(HD, generator=gen) + 0.5).to(torch.bfloat16) for _ in range(2)]
    pos = torch.randint(S - 200, S, (B,), generator=gen)
    table = onorm.rope_angle_table(S, HD, 1e6)
    k0 = torch.randn(B, Hkv, S, HD, generator=gen).to(torch.bfloat16)
    v0 = torch.randn(B, Hkv, S, HD, generator=gen).to(torch.bfloat16)
    qa = QKVHeadAttention(D=D, HD=HD, Hq=Hq, Hkv=Hkv, max_seq=S, group_size=G, tile_size_input=16,
                          kv_layout="separate", batch=B, num_aie_columns=1, accumulate="f64",
                          kernel_source="mv_int8_signed.cc")
    fa = qa.get_callable()
    fa.params.write(qa.kv_offset_parameter, (pos * HD).numpy())
    kc, vc = k0.to(DEV), v0.to(DEV)
    attn = torch.zeros(B * QD, dtype=torch.bfloat16, device=DEV)
    fa(cur.reshape(-1).to(DEV), n_in.to(DEV),
       pack_wire(*wqkv, 16, "signed").view(torch.bfloat16).to(DEV), n_qn.to(DEV), n_kn.to(DEV),
       table[pos].reshape(-1).to(DEV), kc.reshape(-1), vc.reshape(-1), attn)
    mlp = SwiGLUMLPDataParallelOurs(D=D, FF=FF, QD=QD, fuse_o=True, group_size=G, epsilon=1e-6,
                                    batch=B, kernel_source="mv_int8_signed.cc")
    ws = torch.zeros(mlp.workspace_bytes(), dtype=torch.uint8, device=DEV)
    a_s = torch.zeros(B * D, dtype=torch.bfloat16, device=DEV)
    nxt = torch.zeros(B * D, dtype=torch.bfloat16, device=DEV)
    wires = [pack_wire(*wo, mlp.tile_rows_o, "signed"), pack_wire(*wg, mlp.tile_rows_gu, "signed"),
             pack_wire(*wu, mlp.tile_rows_gu, "signed"), pack_wire(*wd, mlp.tile_rows_d, "signed")]
    mlp.get_callable()(cur.reshape(-1).to(DEV), attn, n_pf.to(DEV),
                       *[w.view(torch.bfloat16).to(DEV) for w in wires], ws, a_s, nxt)
    torch.cuda.synchronize()
    wq, wk, wv = oblk.qkv_head(cur, n_in, *wqkv, n_qn, n_kn, table[pos], Hq, Hkv, HD, 1e-6)
    kk, vv = k0.clone(), v0.clone()
    for b in range(B):
        kk[b, :, int(pos[b])] = wk[b].reshape(Hkv, HD)
        vv[b, :, int(pos[b])] = wv[b].reshape(Hkv, HD)
    want_att = oatt.decode_attention(wq.reshape(B, Hq, HD), kk, vv, (pos + 1).tolist())
    assert not verify_buffer(attn.cpu(), "attn", want_att.reshape(-1), RTOL, ATOL)
    got_att = attn.cpu().reshape(B, QD)
    want, want_a = oblk.swiglu_mlp(cur, got_att, n_pf, wg, wu, wd, 1e-6, wo=wo)
    assert_within_one_ulp(a_s, want_a, "8b layer a")
    assert_within_one_ulp(nxt, want, "8b layer nxt")
    lit, _ = oblk.swiglu_mlp(cur, got_att, n_pf, wg, wu, wd, 1e-6, wo=wo, dt=LITERAL)
    assert not verify_buffer(nxt.cpu(), "nxt", lit, RTOL, ATOL)


@pytest.mark.parametrize("H,KV,S,D,dist", [
    (32, 8, 2048, 128, "normal"),   # BASELINE config 5 prefill: Qwen3-8B heads, S = 2048
    (4, 2, 256, 64, "rand4"),       # the reference golden's input distribution, d = 64
    (8, 8, 128, 128, "normal"),     # plain MHA
    (16, 8, 512, 64, "normal"),     # GQA 2
    (4, 1, 192, 128, "normal"),     # S padded from 150 (the reference's 64-padding)
    (8, 2, 512, 128, "ramp"),       # scores rising by ~20 (log2) a block: every block rescales
])
def test_prefill_attention(H, KV, S, D, dist, oracle_provider):
    _say(f"prefill H={H} KV={KV} S={S} D={D} {dist}")
    gen = torch.Generator().manual_seed(H * S + D)
    seq = 150 if S == 192 else S
    op = MHA(num_heads=H, seq_len=seq, d=D, num_KV_heads=KV)
    Sp = op.seq_padded
    assert Sp == S

    def draw(*shape):
        if dist == "rand4":
            return (torch.rand(*shape, generator=gen) * 4).to(torch.bfloat16)
        return torch.randn(*shape, generator=gen).to(torch.bfloat16)

    q, k, v = draw(H, Sp, D), draw(KV, Sp, D), draw(KV, Sp, D)
    if dist == "ramp":  # key j's scores grow with j: each block's maximum passes the last one's
        q = q.float().abs().to(torch.bfloat16)
        k = (k.float().abs() * (torch.arange(Sp).float() / 32).reshape(1, Sp, 1)).to(torch.bfloat16)
    o = torch.zeros(H * Sp * D, dtype=torch.bfloat16, device=DEV)
    op.get_callable()(q.reshape(-1).to(DEV), k.reshape(-1).to(DEV), v.reshape(-1).to(DEV), o)
    torch.cuda.synchronize()
    want = op.reference(q.reshape(-1), k.reshape(-1), v.reshape(-1)).reshape(H, Sp, D)
    got = o.cpu().reshape(H, Sp, D)
    err = (got.float() - want.float()).abs()
    print(f"prefill max abs err {float(err.max()):.3g} (rows < seq_len)", flush=True)
    # rows past seq_len are padding (their outputs are defined but unused, as in the reference)
    assert not verify_buffer(got[:, :seq].contiguous(), "o", want[:, :seq].contiguous(), RTOL,
                             ATOL)
