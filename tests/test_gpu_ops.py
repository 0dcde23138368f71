"""GPU parity of every hot-path operator against the CPU oracle, through the operator API.

Two bars per case, both written in the test:
  * bit-exact against the exact oracle (the reference golden evaluated in fp64 and rounded at the
    reference's boundaries) -- the device kernels evaluate the same closed forms in fp64, so
    their bf16 outputs are the correctly rounded values too;
  * rel 1e-2 / abs 1e-2 against the literal fp32 golden, the reference
    golden as written.
Dequant is bit-exact by construction. Every case prints its name and shape before the GPU call.
"""

import numpy as np
import pytest
import torch

from iron_amd.common.test_utils import verify_buffer
from iron_amd.operators import (DecodeAttention, GEMVInt8, QKVHeadAttention,
                                QKVHeadDataParallelOurs, RMSNorm, SwiGLUMLPDataParallelOurs)
from iron_amd.operators.wire import pack_wire
from oracle import attention as oatt
from oracle import blocks as oblk
from oracle import cref
from oracle import gemv as ogemv
from oracle import norms as onorm
from oracle.numerics import LITERAL, bf16_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 1e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)


def assert_bit_exact(got: torch.Tensor, want: torch.Tensor, what: str):
    g = bf16_bits(got.cpu().reshape(-1))
    w = bf16_bits(want.cpu().reshape(-1))
    bad = int((g != w).sum())
    assert bad == 0, f"{what}: {bad} of {w.numel()} bf16 values differ from the exact oracle"


def _baseline_weights(M, K, G, gen):
    """BASELINE-config weights: q ~ U{-127..127}, s = bf16(|N(0, 0.02)|) per group."""
    q = torch.randint(-127, 128, (M, K), generator=gen, dtype=torch.int16)
    s = (torch.randn(M, K // G, generator=gen) * 0.02).abs().to(torch.bfloat16)
    return q, s


def _src(domain):
    return "mv_int8_signed.cc" if domain == "signed" else None


@pytest.mark.parametrize("M,K,G,tile_m,domain", [
    (4096, 1024, 32, 4, "signed"),
    (4096, 1024, 128, 4, "biased"),
    (96, 256, 32, 12, "signed"),
    (128, 2048, 64, 1, "biased"),
])
def test_dequant_bit_exact(M, K, G, tile_m, domain):
    _say(f"dequant M={M} K={K} G={G} tile_m={tile_m} {domain}")
    gen = torch.Generator().manual_seed(M + K + G)
    q, s = _baseline_weights(M, K, G, gen)
    op = GEMVInt8(M=M, K=K, tile_size_input=tile_m, group_size=G, kernel_vector_size=min(128, K),
                  kernel_source=_src(domain))
    wire = pack_wire(q, s, tile_m, domain).to(DEV)
    got = op.dequantize(wire).cpu()
    want = ogemv.dequant(q, s)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(want.view(torch.int16), cref.dequant(q, s).view(torch.int16))


@pytest.mark.parametrize("M,K,G,tile_m,B,domain", [
    (4096, 1024, 32, 4, 1, "signed"),
    (4096, 1024, 128, 4, 1, "biased"),    # reference group
    (6144, 2048, 32, 12, 1, "signed"),    # 1.7B gate/up shape
    (2048, 6144, 32, 4, 1, "signed"),     # 1.7B down shape
    (1024, 3072, 32, 4, 2, "signed"),
    (512, 4096, 32, 4, 3, "biased"),
    (640, 1024, 32, 16, 4, "signed"),
    (64, 128, 32, 2, 1, "signed"),
    (200, 1040, 16, 8, 1, "signed"),       # K not a multiple of 1024, odd row count per grid
    (4096, 12288, 32, 4, 1, "signed"),     # Qwen3-8B down shape (16 resident slices)
    (2048, 6144, 32, 4, 4, "signed"),      # 1.7B down at batch 4 (4 x 6144 staged rows)
    (4096, 12288, 32, 4, 4, "biased"),     # Qwen3-8B down at batch 4: two workgroups of 3 + 1 rows
    (4096, 12288, 32, 4, 2, "signed"),
    # batches 5..15 on the exact batched kernel (every weight converted once, all rows per pass)
    (4096, 1024, 32, 4, 5, "signed"),      # Qwen3-0.6B fused QKV at batch 5
    (6144, 2048, 32, 12, 8, "biased"),     # 1.7B gate/up shape at BASELINE config 2's batch 8
    (2048, 6144, 32, 4, 8, "signed"),      # 1.7B down at batch 8
    (1024, 3072, 128, 4, 15, "signed"),    # the largest GEMV batch, reference group size
    (200, 1040, 16, 8, 13, "signed"),      # ragged K and rows, a partial last batch group
])
def test_gemv_int8(M, K, G, tile_m, B, domain):
    _say(f"gemv M={M} K={K} G={G} tile_m={tile_m} B={B} {domain}")
    gen = torch.Generator().manual_seed(7 * M + K + B)
    q, s = _baseline_weights(M, K, G, gen)
    x = torch.randn(B, K, generator=gen).to(torch.bfloat16)
    op = GEMVInt8(M=M, K=K, tile_size_input=tile_m, group_size=G, batch_size=B,
                  kernel_vector_size=16, kernel_source=_src(domain))
    op.compile()
    fn = op.get_callable()
    wire = pack_wire(q, s, tile_m, domain).view(torch.bfloat16).to(DEV)
    xd = x.reshape(op.get_arg_spec()[1].shape).to(DEV)
    y = torch.zeros(op.get_arg_spec()[2].shape, dtype=torch.bfloat16, device=DEV)
    fn(wire, xd, y)
    torch.cuda.synchronize()
    exact = ogemv.gemv_exact(q, s, x).float().to(torch.bfloat16)
    assert_bit_exact(y, exact, "gemv")
    literal = ogemv.gemv_exact(q, s, x, dt=LITERAL).to(torch.bfloat16)
    assert not verify_buffer(y.cpu(), "y", literal, rel_tol=RTOL, abs_tol=ATOL)
    # the independent C witness (fp64, no rounding)
    assert not verify_buffer(y.cpu().float().reshape(B, M), "y64", cref.gemv_f64(q, s, x),
                             rel_tol=2 ** -8, abs_tol=1e-6)


def test_gemv_num_batches():
    _say("gemv num_batches=3")
    M, K, G, tm = 256, 512, 32, 4
    gen = torch.Generator().manual_seed(3)
    ws, xs, ys = [], [], []
    for _ in range(3):
        q, s = _baseline_weights(M, K, G, gen)
        x = torch.randn(K, generator=gen).to(torch.bfloat16)
        ws.append(pack_wire(q, s, tm, "signed"))
        xs.append(x)
        ys.append(ogemv.gemv_exact(q, s, x).float().to(torch.bfloat16))
    op = GEMVInt8(M=M, K=K, tile_size_input=tm, group_size=G, num_batches=3,
                  kernel_source="mv_int8_signed.cc")
    y = torch.zeros(3, M, dtype=torch.bfloat16, device=DEV)
    op.get_callable()(torch.cat(ws).view(torch.bfloat16).to(DEV), torch.stack(xs).to(DEV), y)
    torch.cuda.synchronize()
    assert_bit_exact(y, torch.stack(ys), "gemv num_batches")


@pytest.mark.parametrize("rows,cols", [(1, 1024), (4, 2048), (16, 128), (3, 1000)])
def test_rmsnorm(rows, cols):
    _say(f"rmsnorm rows={rows} cols={cols}")
    gen = torch.Generator().manual_seed(rows * cols)
    x = (torch.randn(rows, cols, generator=gen) * 3).to(torch.bfloat16)
    w = (torch.rand(cols, generator=gen) + 0.5).to(torch.bfloat16)
    op = RMSNorm(size=rows * cols, num_aie_columns=1, num_channels=1, tile_size=cols,
                 weighted=True, epsilon=1e-6)
    y = torch.zeros(rows, cols, dtype=torch.bfloat16, device=DEV)
    op.get_callable()(x.to(DEV), w.to(DEV), y)
    torch.cuda.synchronize()
    assert_bit_exact(y, onorm.rms_norm(x, w, 1e-6), "rmsnorm")
    assert not verify_buffer(y.cpu(), "y", onorm.rms_norm(x, w, 1e-6, dt=LITERAL), RTOL, ATOL)


def _kv(B, KV, L, D, gen, scale=1.0):
    k = (torch.randn(B, KV, L, D, generator=gen) * scale).to(torch.bfloat16)
    v = (torch.randn(B, KV, L, D, generator=gen) * scale).to(torch.bfloat16)
    return k, v


@pytest.mark.parametrize("B,H,KV,L,ctx", [
    (1, 16, 8, 4096, [4096]),                 # BASELINE config 3, B=1
    (8, 16, 8, 4096, "ragged"),               # BASELINE config 3, B=8 ragged
    (1, 32, 8, 512, [300]),                   # GQA 4 (Qwen3-8B heads)
    (2, 8, 8, 256, [1, 65]),                  # MHA, tiny contexts
    (3, 16, 2, 128, [0, 63, 64]),             # GQA 8, empty sequence
    (1, 16, 16, 8192, [8191]),                # long context, GQA 1
    (2, 32, 8, 8192, [8192, 5000]),           # Qwen3-8B attention shape, full context
    (100, 4, 1, 512, "ragged0"),              # B > 64 (two sequences a lane in the split deal), empties
    (70, 8, 2, 1024, "ragged0"),              # more (sequence, group) pairs than merge counters
])
def test_decode_attention(B, H, KV, L, ctx):
    gen = torch.Generator().manual_seed(B * 100 + L)
    if ctx == "ragged":
        ctx = torch.randint(512, 4097, (B,), generator=gen).tolist()
    elif ctx == "ragged0":                    # lengths 0..L, every seventh empty
        ctx = torch.randint(0, L + 1, (B,), generator=gen)
        ctx[::7] = 0
        ctx = ctx.tolist()
    _say(f"decode_attn B={B} H={H} KV={KV} L={L} ctx={ctx}")
    D = 128
    q = torch.randn(B, H, D, generator=gen).to(torch.bfloat16)
    k, v = _kv(B, KV, L, D, gen)
    op = DecodeAttention(num_heads=H, num_kv_heads=KV, head_dim=D, seq_len_kv=L,
                         use_runtime_seq_len=True, kv_layout="separate", batch=B)
    fn = op.get_callable()
    fn.params.write("S_kv_eff", ctx)
    o = torch.zeros(B * H, D, dtype=torch.bfloat16, device=DEV)
    qd = q.reshape(B * H, D).to(DEV)
    kd, vd = k.reshape(B * KV, L * D).to(DEV), v.reshape(B * KV, L * D).to(DEV)
    fn(qd, kd, vd, o)
    torch.cuda.synchronize()
    assert_bit_exact(o, oatt.decode_attention(q, k, v, ctx).reshape(B * H, D), "attention")
    literal = oatt.decode_attention(q, k, v, ctx, dt=LITERAL).reshape(B * H, D)
    assert not verify_buffer(o.cpu(), "o", literal, RTOL, ATOL)
    o2 = torch.zeros_like(o)            # a second call gives the same bits
    fn(qd, kd, vd, o2)
    torch.cuda.synchronize()
    assert torch.equal(o.cpu(), o2.cpu())


@pytest.mark.parametrize("interleaved", [True, False])
def test_decode_attention_combined_layouts(interleaved, oracle_provider):
    _say(f"decode_attn combined interleaved={interleaved}")
    H, KV, D, S = 16, 8, 128, 512
    gen = torch.Generator().manual_seed(11)
    q = torch.randn(H, D, generator=gen).to(torch.bfloat16)
    kv = (torch.randn(KV, 2 * S * D, generator=gen) * 0.3).to(torch.bfloat16)
    op = DecodeAttention(num_heads=H, num_kv_heads=KV, head_dim=D, seq_len_kv=S,
                         kv_token_interleaved=interleaved)
    o = torch.zeros(H, D, dtype=torch.bfloat16, device=DEV)
    op.get_callable()(q.to(DEV), kv.to(DEV), o)
    torch.cuda.synchronize()
    assert_bit_exact(o, op.reference(q, kv), "attention combined")


@pytest.mark.parametrize("H,KV,S,n,M,base,layout", [
    (16, 8, 256, 16, 8, 192, "interleaved"),   # the reference's batch test (test_batch.py)
    (32, 8, 512, 16, 8, 480, "interleaved"),   # its Qwen3-4B heads case (test_batch_4b.py)
    (16, 8, 4096, 16, 8, 4000, "separate"),    # long cache: several splits, then the merge
    (16, 8, 256, 1, 1, 100, "separate"),       # M = 1: a plain decode step
    (16, 2, 1024, 5, 5, 1019, "blocked"),      # GQA 8, odd n, bounds clamped at S
])
@pytest.mark.parametrize("causal", [True, False])
def test_decode_attention_verify(H, KV, S, n, M, base, layout, causal, oracle_provider):
    """Batch / verify mode (decode_attn/op.py:40-48, design.py:243-276): every new token's
    output against the exact oracle and the torch.softmax form at rel/abs 1e-2 (the reference's
    own batch tests use cosine > 0.99); pad rows of a taller O stay untouched."""
    _say(f"decode_attn verify H={H} KV={KV} S={S} n={n} M={M} base={base} {layout} "
         f"causal={causal}")
    D = 128
    gen = torch.Generator().manual_seed(S + n + base)
    q = (torch.randn(n, H, D, generator=gen) * 0.5).to(torch.bfloat16)
    k = (torch.randn(KV, S, D, generator=gen) * 0.3).to(torch.bfloat16)
    v = (torch.randn(KV, S, D, generator=gen) * 0.3).to(torch.bfloat16)
    pad = 3
    op = DecodeAttention(num_heads=H, num_kv_heads=KV, head_dim=D, seq_len_kv=S,
                         use_runtime_seq_len=True, batch_queries=M, num_new_tokens=n,
                         causal=causal, out_buffer_tokens=n + pad,
                         kv_layout="separate" if layout == "separate" else "combined",
                         kv_token_interleaved=layout == "interleaved")
    fn = op.get_callable()
    fn.params.write("S_kv_base", base)
    o = torch.full(((n + pad) * H, D), 7.0, dtype=torch.bfloat16, device=DEV)
    if layout == "separate":
        args = [k.reshape(KV, S * D).to(DEV), v.reshape(KV, S * D).to(DEV)]
    elif layout == "interleaved":
        args = [torch.stack([k, v], dim=2).reshape(KV, 2 * S * D).to(DEV)]
    else:
        args = [torch.cat([k.reshape(KV, S * D), v.reshape(KV, S * D)], dim=1).to(DEV)]
    fn(q.reshape(n * H, D).to(DEV), *args, o)
    torch.cuda.synchronize()
    got = o.cpu()[: n * H].reshape(n, H, D)
    assert torch.all(o.cpu()[n * H:].float() == 7.0), "rows past the new tokens were written"
    want = oatt.decode_attention_verify(q, k, v, base, causal)
    assert not verify_buffer(got, "verify o", want, RTOL, ATOL)
    bounds = oatt.verify_bounds(n, base, S, causal)
    sm = torch.zeros(n, H, D)
    for t in range(n):
        sm[t] = oatt.decode_attention_softmax(q[t:t + 1], k[None], v[None], bounds[t])[0].float()
    assert not verify_buffer(got, "verify o (softmax form)", sm, RTOL, ATOL)
    cos = torch.nn.functional.cosine_similarity(got.float().reshape(-1), want.float().reshape(-1),
                                                dim=0)
    assert cos > 0.999
    # the golden through the operator's reference() on the same inputs (S_kv_base from params)
    ref = op.reference(q.reshape(n * H, D), *[a.cpu() for a in args],
                       params=fn.params.snapshot())
    assert torch.equal(bf16_bits(ref.reshape(-1)), bf16_bits(want.reshape(-1)))


def _qkv_case(D, Hq, Hkv, S, G, B, seed):
    HD = 128
    gen = torch.Generator().manual_seed(seed)
    M = (Hq + 2 * Hkv) * HD
    w = torch.randn(M, D, generator=gen) * 0.05
    q8, s = ogemv.rtn_quantize(w, G)
    cur = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    n_in = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16)
    n_qn = (torch.rand(HD, generator=gen) + 0.5).to(torch.bfloat16)
    n_kn = (torch.rand(HD, generator=gen) + 0.5).to(torch.bfloat16)
    table = onorm.rope_angle_table(S, HD, 1e6)
    pos = torch.randint(0, S, (B,), generator=gen)
    return dict(HD=HD, M=M, q8=q8, s=s, cur=cur, n_in=n_in, n_qn=n_qn, n_kn=n_kn,
                ang=table[pos], pos=pos)


@pytest.mark.parametrize("D,Hq,Hkv,S,G,tm,layout,B", [
    (1024, 16, 8, 512, 32, 4, "interleaved", 1),    # Qwen3-0.6B, reference cache layout
    (1024, 16, 8, 2048, 128, 4, "separate", 1),
    (4096, 32, 8, 256, 32, 16, "separate", 2),      # Qwen3-8B head shape, batch 2
    (256, 2, 1, 64, 32, 4, "separate", 4),
    (4096, 32, 8, 256, 32, 16, "separate", 4),      # Qwen3-8B head shape, batch 4
])
def test_qkv_head(D, Hq, Hkv, S, G, tm, layout, B):
    _say(f"qkv_head D={D} Hq={Hq} Hkv={Hkv} S={S} G={G} layout={layout} B={B}")
    c = _qkv_case(D, Hq, Hkv, S, G, B, seed=D + S + B)
    HD = c["HD"]
    op = QKVHeadDataParallelOurs(D=D, HD=HD, Hq=Hq, Hkv=Hkv, max_seq=S, group_size=G,
                                 tile_size_input=tm, kv_layout=layout, batch=B,
                                 num_aie_columns=1, kernel_source="mv_int8_signed.cc")
    fn = op.get_callable()
    per_tok = HD if layout == "separate" else 2 * HD
    fn.params.write(op.kv_offset_parameter, (c["pos"] * per_tok).numpy())
    wire = pack_wire(c["q8"], c["s"], tm, "signed").view(torch.bfloat16).to(DEV)
    qo = torch.zeros(B * Hq * HD, dtype=torch.bfloat16, device=DEV)
    if layout == "separate":
        kc = torch.zeros(B, Hkv, S, HD, dtype=torch.bfloat16, device=DEV)
        vc = torch.zeros_like(kc)
        caches = (kc.reshape(-1), vc.reshape(-1))
    else:
        kvc = torch.zeros(B, Hkv, S, 2, HD, dtype=torch.bfloat16, device=DEV)
        caches = (kvc.reshape(-1),)
    fn(c["cur"].reshape(-1).to(DEV), c["n_in"].to(DEV), wire, c["n_qn"].to(DEV),
       c["n_kn"].to(DEV), c["ang"].reshape(-1).to(DEV), qo, *caches)
    torch.cuda.synchronize()
    args = (c["cur"], c["n_in"], c["q8"], c["s"], c["n_qn"], c["n_kn"], c["ang"], Hq, Hkv, HD,
            1e-6)
    wq, wk, wv = oblk.qkv_head(*args)
    lq, _, _ = oblk.qkv_head(*args, dt=LITERAL)
    assert_bit_exact(qo, wq, "q")
    assert not verify_buffer(qo.cpu(), "q", lq, RTOL, ATOL)
    if layout == "separate":
        kcc, vcc = kc.cpu(), vc.cpu()
    else:
        kcc, vcc = kvc.cpu()[:, :, :, 0], kvc.cpu()[:, :, :, 1]
    for b in range(B):
        p = int(c["pos"][b])
        assert_bit_exact(kcc[b, :, p], wk[b], "k")
        assert_bit_exact(vcc[b, :, p], wv[b], "v")
        mask = torch.ones(S, dtype=torch.bool)          # nothing else in the cache was touched
        mask[p] = False
        assert kcc[b][:, mask].abs().sum() == 0 and vcc[b][:, mask].abs().sum() == 0


@pytest.mark.parametrize("D,Hq,Hkv,S,G,tm,layout,pos", [
    (1024, 16, 8, 2240, 32, 4, "separate", [2048]),      # the bench step (B=1, speculative)
    (1024, 16, 8, 512, 32, 4, "interleaved", [0]),       # first position, reference cache layout
    (1024, 16, 8, 512, 32, 4, "separate", [64]),         # first token of a tile
    (4096, 32, 8, 1024, 32, 16, "separate", [1000, 63]), # Qwen3-8B heads (4 per workgroup), B=2
    (256, 2, 1, 128, 32, 4, "separate", [127, 5, 64]),   # GQA 2, B=3, last position
])
def test_qkv_attention_fused(D, Hq, Hkv, S, G, tm, layout, pos):
    """QKVHeadAttention == QKVHeadDataParallelOurs -> DecodeAttention(S_kv_eff = pos + 1), bit for
    bit (output and caches), and == the exact oracle. Cache rows past each position hold NaN/inf
    bit patterns: they are read by the speculative first tile and must not leak into the result."""
    B = len(pos)
    _say(f"qkv_attn D={D} Hq={Hq} Hkv={Hkv} S={S} G={G} layout={layout} pos={pos}")
    c = _qkv_case(D, Hq, Hkv, S, G, B, seed=D + S + 7 * B)
    HD = c["HD"]
    gen = torch.Generator().manual_seed(S + B)
    k0, v0 = _kv(B, Hkv, S, HD, gen)
    for b, p in enumerate(pos):                     # garbage past the context
        k0[b, :, p:] = torch.tensor([0x7FC0, 0x7F80, -0x80, 0x7FFF], dtype=torch.int16).view(
            torch.bfloat16).repeat(HD // 4)
        v0[b, :, p:] = k0[b, :, p:]
    table = onorm.rope_angle_table(S, HD, 1e6)
    common = dict(D=D, HD=HD, Hq=Hq, Hkv=Hkv, max_seq=S, group_size=G, tile_size_input=tm,
                  kv_layout=layout, batch=B, num_aie_columns=1, kernel_source="mv_int8_signed.cc")
    fused = QKVHeadAttention(**common)                           # one angle row per batch row
    qkv = QKVHeadDataParallelOurs(**common, angles_from_table=True)  # the whole table
    attn = DecodeAttention(num_heads=Hq, num_kv_heads=Hkv, head_dim=HD, seq_len_kv=S,
                           use_runtime_seq_len=True, batch=B,
                           kv_layout="separate" if layout == "separate" else "combined")
    per_tok = HD if layout == "separate" else 2 * HD
    offs = np.asarray(pos) * per_tok
    wire = pack_wire(c["q8"], c["s"], tm, "signed").view(torch.bfloat16).to(DEV)
    ins = (c["cur"].reshape(-1).to(DEV), c["n_in"].to(DEV), wire, c["n_qn"].to(DEV),
           c["n_kn"].to(DEV))
    rows = table[torch.tensor(pos)].reshape(-1).to(DEV)

    def caches():
        if layout == "separate":
            return [k0.clone().reshape(-1).to(DEV), v0.clone().reshape(-1).to(DEV)]
        return [torch.stack([k0, v0], dim=3).reshape(-1).to(DEV)]

    ca, cb = caches(), caches()
    fa = fused.get_callable()
    fa.params.write(fused.kv_offset_parameter, offs)
    out_a = torch.zeros(B * Hq * HD, dtype=torch.bfloat16, device=DEV)
    fa(*ins, rows, *ca, out_a)
    fq = qkv.get_callable()
    fq.params.write(qkv.kv_offset_parameter, offs)
    fattn = attn.get_callable()
    fattn.params.write("S_kv_eff", [p + 1 for p in pos])
    qo = torch.zeros(B * Hq * HD, dtype=torch.bfloat16, device=DEV)
    out_b = torch.zeros_like(out_a)
    fq(*ins, table.reshape(-1).to(DEV), qo, *cb)
    fattn(qo.reshape(B * Hq, HD), *[t.reshape(B * Hkv, -1) for t in cb], out_b.reshape(B * Hq, HD))
    torch.cuda.synchronize()
    assert torch.equal(out_a.cpu().view(torch.int16), out_b.cpu().view(torch.int16)), "output"
    for x, y in zip(ca, cb):
        assert torch.equal(x.cpu().view(torch.int16), y.cpu().view(torch.int16)), "caches"
    # exact oracle: QKV head, append, attention over 0..pos
    wq, wk, wv = oblk.qkv_head(c["cur"], c["n_in"], c["q8"], c["s"], c["n_qn"], c["n_kn"],
                               table[torch.tensor(pos)], Hq, Hkv, HD, 1e-6)
    kk, vv = k0.clone(), v0.clone()
    for b, p in enumerate(pos):
        kk[b, :, p] = wk[b].reshape(Hkv, HD)
        vv[b, :, p] = wv[b].reshape(Hkv, HD)
    want = oatt.decode_attention(wq.reshape(B, Hq, HD), kk, vv, [p + 1 for p in pos])
    assert_bit_exact(out_a, want, "fused attention")


@pytest.mark.parametrize("D,FF,QD,fuse_o,G,B", [
    (1024, 3072, 2048, True, 32, 1),    # Qwen3-0.6B chain arm
    (2048, 6144, 0, False, 32, 1),      # BASELINE config 2, B=1
    (2048, 6144, 0, False, 32, 2),
    (1024, 3072, 2048, True, 128, 2),   # reference group size
    (2560, 9728, 4096, True, 32, 1),    # Qwen3-4B: FF % D != 0 (the chunked-down arm)
    (2560, 9728, 4096, True, 128, 1),
    (2048, 6144, 0, False, 32, 4),      # BASELINE config 2 shape at batch 4
    (2560, 9728, 4096, True, 32, 3),    # Qwen3-4B at batch 3
    (4096, 12288, 4096, True, 32, 4),   # Qwen3-8B layer MLP at batch 4 (down in groups of 3 + 1)
])
def test_swiglu_mlp(D, FF, QD, fuse_o, G, B):
    _say(f"swiglu D={D} FF={FF} QD={QD} fuse_o={fuse_o} G={G} B={B}")
    gen = torch.Generator().manual_seed(D + FF + B)
    op = SwiGLUMLPDataParallelOurs(D=D, FF=FF, QD=QD or None, fuse_o=fuse_o, group_size=G,
                                   epsilon=1e-6, batch=B, kernel_source="mv_int8_signed.cc")

    def lin(M, K, std):
        return ogemv.rtn_quantize(torch.randn(M, K, generator=gen) * std, G)

    wg, wu, wd = lin(FF, D, 0.05), lin(FF, D, 0.05), lin(D, FF, 0.05)
    cur = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    n_pf = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16)
    if fuse_o:
        wo = lin(D, QD, 0.05)
        cx = torch.randn(B, QD, generator=gen).to(torch.bfloat16)
    else:
        wo = None
        cx = torch.randn(B, D, generator=gen).to(torch.bfloat16)
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
    want, want_a = oblk.swiglu_mlp(cur, cx, n_pf, wg, wu, wd, 1e-6, wo=wo)
    assert_bit_exact(nxt, want, "nxt")
    if fuse_o:
        assert_bit_exact(a_s, want_a, "a")
        # the literal fp32 golden's own a can sit a bf16 ulp from the exact one (Qwen3-8B widths),
        # which the residual x1 = cur + a carries into many ulps of nxt: the rest of the block is
        # checked against the literal golden from the exact a
        lit, _ = oblk.swiglu_mlp(cur, a_s.cpu().reshape(B, D), n_pf, wg, wu, wd, 1e-6,
                                 dt=LITERAL)
    else:
        lit, _ = oblk.swiglu_mlp(cur, cx, n_pf, wg, wu, wd, 1e-6, dt=LITERAL)
    assert not verify_buffer(nxt.cpu(), "nxt", lit, RTOL, ATOL)


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_lm_head_argmax(kind, lib):
    from iron_amd import _lib

    V, D, G, tm = 151936, 1024, 32, 4
    _say(f"lm_head {kind} V={V} D={D}")
    gen = torch.Generator().manual_seed(5)
    emb = (torch.randn(V, D, generator=gen) * 0.1).to(torch.bfloat16)
    x = torch.randn(1, D, generator=gen).to(torch.bfloat16)
    nw = (torch.rand(D, generator=gen) + 0.5).to(torch.bfloat16)
    xn = onorm.rms_norm(x, nw, 1e-6)
    if kind == "bf16":
        w = emb.to(DEV)
        wk = _lib.IRON_WEIGHT_BF16
        want = ogemv.gemv(emb, xn.reshape(-1)).float().to(torch.bfloat16)
    else:
        q8, s = ogemv.rtn_quantize(emb, G)
        w = pack_wire(q8, s, tm, "signed").to(DEV)
        wk = _lib.IRON_WEIGHT_INT8
        want = ogemv.gemv_exact(q8, s, xn.reshape(-1)).float().to(torch.bfloat16)
    logits = torch.zeros(V, dtype=torch.bfloat16, device=DEV)
    keys = torch.zeros(1, dtype=torch.int64, device=DEV)
    xd, nwd = x.to(DEV), nw.to(DEV)  # keep the device copies alive across the async launch
    _lib.call("iron_lm_head", w.data_ptr(), wk, xd.data_ptr(), nwd.data_ptr(),
              1e-6, logits.data_ptr(), keys.data_ptr(), 1, V, D, G, tm, 0,
              torch.cuda.current_stream().cuda_stream)
    tokens = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.call("iron_next_token", keys.data_ptr(), tokens.data_ptr(), None, None, None, 0, 0,
              None, 1, D, V, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = logits.cpu()
    assert_bit_exact(got, want, "logits")
    # device argmax == first index of the max of the bf16 logits
    assert int(tokens.item()) == int(torch.argmax(got.float()))
    assert int(keys.item()) == 0  # consumed and reset


def test_bf16_rounding_exhaustive(lib):
    """Every kernel rounds fp32 -> bf16 with the gfx950 conversion instruction: it must equal the
    integer round-to-nearest-even (the oracle's f32_to_bf16_rne) on all 2^32 fp32 bit patterns, and
    fp64 values must round twice (fp64 -> fp32 -> bf16, as torch and the oracle do)."""
    from iron_amd import _lib

    _say("bf16 rounding: all 2^32 fp32 patterns")
    out = torch.tensor([0, -1, 0], dtype=torch.int32, device=DEV)
    _lib.call("iron_test_bf16_round", out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    bad, first, dbl = (int(v) & 0xFFFFFFFF for v in out.cpu().tolist())
    assert bad == 0, f"{bad} fp32 patterns round differently, first {first:#010x}"
    # 1 + 2^-8 + 2^-40: fp32 drops 2^-40, the bf16 tie then goes to even (1.0); one rounding from
    # fp64 would go up to 1 + 2^-7
    x = torch.tensor([1.0 + 2.0 ** -8 + 2.0 ** -40], dtype=torch.float64)
    want = int(x.float().to(torch.bfloat16).view(torch.int16).item()) & 0xFFFF
    assert want == 0x3F80 and dbl == want
