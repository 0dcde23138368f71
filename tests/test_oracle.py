"""Pins of the CPU oracle (no GPU). The reference ships no golden vectors or fixtures, so every
oracle function is checked against what the mathematics fixes -- exhaustive enumeration, fp64
brute force with explicit loops, closed forms, invariants -- and against the independent C
restatement (oracle/c/oracle.c), chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one check."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import blocks as oblk
from oracle import cref
from oracle import gemv as og
from oracle import norms as on
from oracle.numerics import bf16_bits

# ----------------------------------------------------------------------------------- dequant


def test_dequant_exhaustive_bit_exact():
    """All 256 int8 codes x a spread of bf16 scales: bf16(q*s) with q*s exact in fp32."""
    q = torch.arange(-128, 128, dtype=torch.int16).repeat(64, 1)             # (64, 256)
    exps = torch.linspace(-30, 10, 64)
    s = (torch.rand(64) + 1.0) * torch.pow(2.0, exps)
    s = s.to(torch.bfloat16)[:, None]                                        # one group per row
    got = og.dequant(q, s)
    prod64 = q.double() * s.double()
    assert torch.equal(prod64.float().double(), prod64)                      # exact in fp32
    want = prod64.float().to(torch.bfloat16)
    assert torch.equal(bf16_bits(got), bf16_bits(want))
    assert torch.equal(bf16_bits(got), bf16_bits(cref.dequant(q, s)))


def test_dequant_group_indexing():
    """Scale g applies to columns [g*G, (g+1)*G) only (a wrong group index fails)."""
    M, K, G = 3, 96, 32
    q = torch.ones(M, K, dtype=torch.int16)
    s = torch.tensor([[1.0, 2.0, 4.0]] * M).to(torch.bfloat16)
    w = og.dequant(q, s).float()
    assert torch.equal(w[:, :32], torch.ones(M, 32))
    assert torch.equal(w[:, 32:64], 2 * torch.ones(M, 32))
    assert torch.equal(w[:, 64:], 4 * torch.ones(M, 32))


# ----------------------------------------------------------------------------------- GEMV


def _rand_wq(M, K, G, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int16)
    s = (torch.randn(M, K // G, generator=g) * 0.02).abs().to(torch.bfloat16)
    x = torch.randn(K, generator=g).to(torch.bfloat16)
    return q, s, x


def test_gemv_exact_vs_fp64_loops():
    M, K, G = 7, 64, 32
    q, s, x = _rand_wq(M, K, G, 1)
    y = og.gemv_exact(q, s, x)
    for m in range(M):
        acc = 0.0
        for k in range(K):
            acc += float(q[m, k]) * float(s[m, k // G].float()) * float(x[k].float())
        assert abs(float(y[m]) - acc) <= 1e-5 * (1 + abs(acc))


def test_gemv_exact_vs_c_restatement_and_batch():
    q, s, _ = _rand_wq(128, 512, 32, 2)
    X = torch.randn(3, 512, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    y = og.gemv_exact(q, s, X)                                    # exact (fp64)
    y64 = cref.gemv_f64(q, s, X)
    assert torch.allclose(y, y64, rtol=1e-12, atol=1e-12)
    lit = og.gemv_exact(q, s, X, dt=torch.float32)                 # literal fp32 golden
    assert torch.allclose(lit.double(), y64, rtol=1e-5, atol=1e-5)


def test_gemv_closed_forms():
    q, s, _ = _rand_wq(16, 128, 32, 3)
    k = 77
    x = torch.zeros(128, dtype=torch.bfloat16)
    x[k] = 1.0
    y = og.gemv_exact(q, s, x)                                   # one-hot x -> column k
    assert torch.equal(y, q[:, k].double() * s[:, k // 32].double())
    assert torch.equal(og.gemv_exact(q, torch.zeros_like(s), x), torch.zeros(16, dtype=torch.float64))
    # non-square: a transposed operand would not even multiply
    with pytest.raises(RuntimeError):
        og.dequant_f32(q, s).t() @ torch.randn(128)


def test_gemv_premul_relation():
    """The kernel-form golden (x*s rounded to bf16, summed in fp32) equals the exact form up to
    fp32 summation error when x*s is exact, and stays within its rounding bound otherwise."""
    q, s, x = _rand_wq(32, 256, 32, 4)
    g = torch.Generator().manual_seed(9)
    s2 = torch.pow(2.0, torch.randint(-12, -4, s.shape, generator=g).float()).to(torch.bfloat16)
    # power-of-two scales: every product q * bf16(x * s) is exact in fp32, so only the fp32 sum
    # of K terms rounds (recursive-summation bound K * 2^-24 * sum |terms|)
    d1 = (og.gemv_premul(q, s2, x).double() - og.gemv_exact(q, s2, x)).abs()
    mag = (q.abs().double() * (x.double()[None] * s2.double().repeat_interleave(32, 1)).abs()).sum(1)
    assert torch.all(d1 <= 256 * 2.0 ** -24 * mag)
    d = (og.gemv_premul(q, s, x).double() - og.gemv_exact(q, s, x)).abs().float()
    bound = (q.abs().float() * (x.float()[None] * s.float().repeat_interleave(32, 1)).abs()
             ).sum(1) * 2 ** -8
    assert torch.all(d <= bound + 1e-6)


# ----------------------------------------------------------------------------------- wires


def test_wire_literal_bytes():
    """Tiny wire spelled out by hand: tile_m=2, K=32, G=16, signed and biased."""
    q = torch.tensor([[i - 16 for i in range(32)], [15 - i for i in range(32)],
                      [1] * 32, [-1] * 32], dtype=torch.int16)
    s = torch.tensor([[1.0, 2.0], [0.5, 0.25], [1.0, 1.0], [4.0, 8.0]]).to(torch.bfloat16)
    w = og.pack_wire(q, s, 2, "signed")
    assert w.size == 2 * (2 * 32 + 2 * 2 * 2)
    assert list(w[:4]) == [0xF0, 0xF1, 0xF2, 0xF3]                 # -16..-13 as int8
    sb = w[64:72].view(np.uint16)
    assert list(sb) == [0x3F80, 0x4000, 0x3F00, 0x3E80]             # 1, 2, 0.5, 0.25 in bf16
    assert list(w[72:74]) == [1, 1]                                 # block 2 payload starts
    wb = og.pack_wire(q, s, 2, "biased")
    assert list(wb[:2]) == [112, 113]                               # q + 128
    assert np.array_equal(wb[64:72], w[64:72])                      # scales identical


@pytest.mark.parametrize("tile_m,domain", [(1, "signed"), (4, "biased"), (12, "signed")])
def test_wire_roundtrip_torch_and_c(tile_m, domain):
    q, s, _ = _rand_wq(48, 256, 64, tile_m)
    w = og.pack_wire(q, s, tile_m, domain)
    q2, s2 = og.unpack_wire(w, 48, 256, 64, tile_m, domain)
    q3, s3 = cref.wire_unpack(w, 48, 256, 64, tile_m, domain)
    assert torch.equal(q2, q) and torch.equal(q3, q)
    assert torch.equal(bf16_bits(s2), bf16_bits(s)) and torch.equal(bf16_bits(s3), bf16_bits(s))


def test_rtn_quantizer_bounds():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(64, 256, generator=g) * 0.05
    w[3, :32] = 0.0                                                   # an all-zero group
    q, s = og.rtn_quantize(w, 32)
    assert q.abs().max() <= 127
    assert float(s[3, 0]) == 1.0 and torch.all(q[3, :32] == 0)
    deq = og.dequant_f32(q, s)
    sx = s.float().repeat_interleave(32, 1)
    assert torch.all((w - deq).abs() <= sx * 0.5 + 1e-7)
    peak = q.reshape(64, 8, 32).abs().amax(-1)
    assert torch.all(peak[torch.arange(64) != 3] >= 126)              # the peak maps to +-127


def test_gptq_unpack_known_pattern():
    """Pack known q (zero-point 128, 4 u8 per int32 little-endian along K) and unpack."""
    M, K, G = 8, 32, 16
    g = torch.Generator().manual_seed(6)
    q = torch.randint(-128, 128, (M, K), generator=g)
    u = (q + 128).to(torch.int64).t().reshape(K // 4, 4, M)          # (K/4, 4, M)
    words = (u[:, 0] | (u[:, 1] << 8) | (u[:, 2] << 16) | (u[:, 3] << 24))
    qweight = torch.from_numpy(words.numpy().astype(np.uint32).view(np.int32))
    scales = torch.rand(K // G, M).to(torch.float16)
    q2, s2 = og.gptq_unpack(qweight, scales)
    assert torch.equal(q2.to(torch.int64), q)
    assert torch.equal(s2.float(), scales.float().to(torch.bfloat16).float().t())


# ----------------------------------------------------------------------------------- norms


def test_rms_norm_closed_form_and_invariance():
    x = torch.tensor([[3.0, 4.0, 0.0, 0.0]])
    y = on.rms_norm(x, None, 0.0, out_bf16=False)
    r = math.sqrt((9 + 16) / 4)
    assert torch.allclose(y, torch.tensor([[3 / r, 4 / r, 0.0, 0.0]]))
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, 128, generator=g)
    w = torch.rand(128, generator=g) + 0.5
    a = on.rms_norm(x, w, 1e-12, out_bf16=False)
    b = on.rms_norm(x * 8.0, w, 1e-12, out_bf16=False)                # scale invariance
    assert torch.allclose(a, b, rtol=1e-6, atol=1e-6)
    x64 = x.double()
    ref = x64 / torch.sqrt((x64 ** 2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(on.rms_norm(x, w, 1e-6, out_bf16=False).double(), ref, rtol=1e-6)
    assert torch.equal(on.rms_norm(x, w, 1e-6), ref.float().to(torch.bfloat16)) or \
        (on.rms_norm(x, w, 1e-6).float() - ref).abs().max() <= 2 ** -7 * ref.abs().max()


def test_rope_identity_norm_and_complex_form():
    HD = 128
    g = torch.Generator().manual_seed(8)
    x = torch.randn(5, HD, generator=g).to(torch.bfloat16)
    table = on.rope_angle_table(4096, HD, 1e6)
    assert torch.equal(on.rope(x, table[0]), x)                       # angle 0 is the identity
    y = on.rope(x, table[1234]).float()
    xf = x.float()
    n_in = xf[:, :64] ** 2 + xf[:, 64:] ** 2
    n_out = y[:, :64] ** 2 + y[:, 64:] ** 2                           # pair (i, i+64) norms
    assert torch.allclose(n_in, n_out, rtol=2e-2, atol=1e-2)
    c, s = table[1234][0::2].float(), table[1234][1::2].float()
    z = torch.complex(xf[:, :64], xf[:, 64:]) * torch.complex(c, s)   # rotate_half == complex mul
    assert torch.allclose(y[:, :64], z.real, rtol=1e-2, atol=1e-2)
    assert torch.allclose(y[:, 64:], z.imag, rtol=1e-2, atol=1e-2)


def test_rope_block_major_angle_rows():
    """Reference convention (iron/tests/operators/rope_reference_convention.py:21-64): row r
    uses angle row r // (rows // angle_rows)."""
    g = torch.Generator().manual_seed(9)
    for rows, arows in [(6, 3), (8, 2), (12, 4), (4, 4)]:
        x = torch.randn(rows, 4, generator=g).to(torch.bfloat16)
        ang = torch.rand(arows, 4, generator=g).to(torch.bfloat16)
        got = on.rope(x, ang)
        for r in range(rows):
            a = r // (rows // arows)
            want = on.rope(x[r:r + 1], ang[a:a + 1])
            assert torch.equal(got[r:r + 1], want)


def test_rope_angle_table_closed_form():
    t = on.rope_angle_table(2048, 128, 1e6)
    assert torch.equal(t[0, 0::2].float(), torch.ones(64))
    assert torch.equal(t[0, 1::2].float(), torch.zeros(64))
    pos, i = 1000, 5
    ang = pos * 1e6 ** (-i / 64)
    assert abs(float(t[pos, 2 * i]) - math.cos(ang)) <= 2 ** -8 * 2
    assert abs(float(t[pos, 2 * i + 1]) - math.sin(ang)) <= 2 ** -8 * 2


def test_rope_halves_pins():
    """With duplicated halves it is ``rope`` (pinned above) bit for bit; closed forms at 0 and
    90 degrees; with distinct halves the second half uses its own entries (a restatement that
    reused cos[:m] / sin[:m] for both halves fails the last check)."""
    HD, m = 128, 64
    g = torch.Generator().manual_seed(10)
    x = torch.randn(5, HD, generator=g).to(torch.bfloat16)
    table = on.rope_angle_table(4096, HD, 1e6)
    for pos in (0, 1, 777, 4095):
        c, s = table[pos][0::2], table[pos][1::2]
        got = on.rope_halves(x, torch.cat([c, c]), torch.cat([s, s]))
        assert torch.equal(got, on.rope(x, table[pos]))
    one, zero = torch.ones(HD, dtype=torch.bfloat16), torch.zeros(HD, dtype=torch.bfloat16)
    assert torch.equal(on.rope_halves(x, one, zero), x)
    assert torch.equal(on.rope_halves(x, zero, one), torch.cat([-x[:, m:], x[:, :m]], dim=-1))
    cos = torch.cat([one[:m], zero[:m]])
    sin = torch.cat([zero[:m], one[:m]])
    want = torch.cat([x[:, :m], x[:, :m]], dim=-1)        # y1 = x1; y2 = x2*0 + x1*1
    assert torch.equal(on.rope_halves(x, cos, sin), want)
    reused = torch.cat([x[:, :m] * cos[:m] - x[:, m:] * sin[:m],
                        x[:, m:] * cos[:m] + x[:, :m] * sin[:m]], dim=-1)
    assert not torch.equal(reused, want)                   # the check tells the two apart


def test_rope_interleaved_is_the_two_halves_form_on_permuted_dims():
    """Gathering the even dims then the odd ones turns pairs (2i, 2i+1) into (i, i + m): the
    interleaved method is ``rope`` (pinned above) conjugated by that permutation, also with
    block-shared angle rows; plus the 90-degree closed form."""
    HD, m = 128, 64
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, HD, generator=g).to(torch.bfloat16)
    ang = on.rope_angle_table(512, HD, 1e4)[torch.tensor([5, 300, 511])]
    perm = torch.cat([x[:, 0::2], x[:, 1::2]], dim=-1)
    two = on.rope(perm, ang)
    want = torch.empty_like(x)
    want[:, 0::2], want[:, 1::2] = two[:, :m], two[:, m:]
    assert torch.equal(on.rope_interleaved(x, ang), want)
    quarter = torch.zeros(1, HD, dtype=torch.bfloat16)
    quarter[0, 1::2] = 1.0                                    # cos 0, sin 1
    y = on.rope_interleaved(x, quarter)
    assert torch.equal(y[:, 0::2], -x[:, 1::2]) and torch.equal(y[:, 1::2], x[:, 0::2])


def test_qk_norm_rope_pins():
    """V is copied; at angle 0 each Q/K head is its RMSNorm with its own gamma row (pinned
    above); a head's output depends on that head only (scaling one head's input by 4 leaves
    every output but that head's unchanged, and that head's within one bf16 ulp); the golden's
    single rounding stays within the reference test's tolerance of the kernel's two."""
    n_q, n_v, HD = 4, 2, 128
    n_qk = n_q + n_v
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn((n_qk + n_v) * HD, generator=g).to(torch.bfloat16)
    gamma = (torch.randn(n_qk * HD, generator=g) * 0.2 + 1.0).to(torch.bfloat16)
    one, zero = torch.ones(HD, dtype=torch.bfloat16), torch.zeros(HD, dtype=torch.bfloat16)
    out = on.qk_norm_rope(qkv, torch.cat([gamma, one, zero]), n_qk, n_v, HD, 1e-6)
    assert torch.equal(out[n_qk * HD:], qkv[n_qk * HD:])
    heads = qkv[: n_qk * HD].reshape(n_qk, HD)
    want = on.rms_norm(heads, gamma.reshape(n_qk, HD), 1e-6)
    assert torch.equal(out[: n_qk * HD].reshape(n_qk, HD), want)
    table = on.rope_angle_table(1024, HD, 1e6)
    c, s = table[321][0::2], table[321][1::2]
    sc = torch.cat([gamma, c, c, s, s])
    a = on.qk_norm_rope(qkv, sc, n_qk, n_v, HD, 1e-6)
    scaled = qkv.clone()
    scaled[2 * HD: 3 * HD] = (scaled[2 * HD: 3 * HD].float() * 4).to(torch.bfloat16)
    b = on.qk_norm_rope(scaled, sc, n_qk, n_v, HD, 1e-6)
    rest = torch.ones(a.numel(), dtype=torch.bool)
    rest[2 * HD: 3 * HD] = False
    assert torch.equal(a[rest], b[rest])
    d = (a[2 * HD: 3 * HD].float() - b[2 * HD: 3 * HD].float()).abs()
    assert (d <= a[2 * HD: 3 * HD].float().abs() * 2 ** -7 + 1e-30).all()
    gold = on.qk_norm_rope(qkv, sc, n_qk, n_v, HD, 1e-6, round_norm=False)
    err = (a.float() - gold.float()).abs()
    assert (err <= 0.02 + 0.05 * gold.float().abs()).all()


# ----------------------------------------------------------------------------------- attention


def _qkv(B, H, KV, L, D, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    k = (torch.randn(B, KV, L, D, generator=g) * scale).to(torch.bfloat16)
    v = (torch.randn(B, KV, L, D, generator=g) * scale).to(torch.bfloat16)
    return q, k, v


def test_attention_single_key_and_constant_keys():
    q, k, v = _qkv(1, 4, 2, 16, 128, 10)
    o = oatt.decode_attention(q, k, v, 1)
    for h in range(4):
        assert torch.equal(o[0, h], v[0, h * 2 // 4, 0])             # L=1 -> v0
    k2 = k.clone()
    k2[:] = k[:, :, :1]                                               # all keys equal -> mean V
    o2 = oatt.decode_attention(q, k2, v, 16).float()
    want = v[:, :, :16].float().mean(2)
    for h in range(4):
        assert torch.allclose(o2[0, h], want[0, h * 2 // 4], atol=1e-2)


def test_attention_vs_fp64_and_c_and_softmax():
    q, k, v = _qkv(2, 8, 2, 200, 128, 11)
    ctx = [200, 37]
    o = oatt.decode_attention(q, k, v, ctx).double()
    o64 = oatt.decode_attention_f64(q, k, v, ctx)
    oc = cref.decode_attn_f64(q, k, v, ctx, 1 / math.sqrt(128))
    assert torch.allclose(o64, oc, atol=1e-10)
    assert torch.allclose(o, o64, rtol=1e-2, atol=4e-3)
    assert torch.allclose(oatt.decode_attention_softmax(q, k, v, ctx).double(), o, atol=4e-3)


def test_attention_invariants():
    q, k, v = _qkv(1, 4, 4, 64, 128, 12)
    o = oatt.decode_attention(q, k, v, 64).float()
    assert torch.allclose(oatt.decode_attention_f64(q, k, v, 64), o.double(), atol=4e-3)
    # adding the same vector to every key shifts all scores of a head equally: output
    # unchanged. Integer-valued keys keep k + c exact in bf16.
    g = torch.Generator().manual_seed(21)
    ki = torch.randint(-4, 5, (1, 4, 64, 128), generator=g).to(torch.bfloat16)
    c = torch.randint(-3, 4, (128,), generator=g).to(torch.bfloat16)
    ks = (ki.float() + c.float()).to(torch.bfloat16)
    qs = (q.float() / 8).to(torch.bfloat16)
    assert torch.allclose(oatt.decode_attention_f64(qs, ks, v, 64),
                          oatt.decode_attention_f64(qs, ki, v, 64), atol=1e-9)
    assert torch.allclose(oatt.decode_attention(qs, ks, v, 64).float(),
                          oatt.decode_attention(qs, ki, v, 64).float(), atol=4e-3)
    # GQA map h -> h*KV//H: permuting KV heads permutes the outputs of their query groups
    q2, k2, v2 = _qkv(1, 8, 2, 32, 128, 13)
    a = oatt.decode_attention(q2, k2, v2, 32)
    b = oatt.decode_attention(q2[:, [4, 5, 6, 7, 0, 1, 2, 3]], k2[:, [1, 0]], v2[:, [1, 0]], 32)
    assert torch.equal(a[:, [4, 5, 6, 7, 0, 1, 2, 3]], b)
    # ctx 0 -> zeros; ragged batch == per-sequence calls
    assert torch.all(oatt.decode_attention(q, k, v, 0) == 0)
    q3, k3, v3 = _qkv(3, 4, 2, 48, 128, 14)
    r = oatt.decode_attention(q3, k3, v3, [48, 1, 20])
    for b_, n in enumerate([48, 1, 20]):
        assert torch.equal(r[b_:b_ + 1], oatt.decode_attention(q3[b_:b_ + 1], k3[b_:b_ + 1],
                                                               v3[b_:b_ + 1], n))


def test_verify_attention_pins():
    """Batch/verify decode attention (decode_attn/design.py:243-276): token t of a causal block
    is a single-query decode at context base + t + 1, the non-causal block attends the whole
    cache, n = 1 reduces to the decode step, bounds clamp at the cache length, and the
    torch.softmax form of the reference's own batch test (test_batch.py:31-45) agrees."""
    g = torch.Generator().manual_seed(11)
    H, KV, D, S, n, base = 4, 2, 128, 96, 6, 40
    q = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    k = (torch.randn(KV, S, D, generator=g) * 0.5).to(torch.bfloat16)
    v = torch.randn(KV, S, D, generator=g).to(torch.bfloat16)
    got = oatt.decode_attention_verify(q, k, v, base, causal=True)
    for t in range(n):
        one = oatt.decode_attention(q[t:t + 1], k[None], v[None], base + t + 1)
        assert torch.equal(bf16_bits(got[t]), bf16_bits(one[0]))
    full = oatt.decode_attention_verify(q, k, v, base, causal=False)
    for t in range(n):
        one = oatt.decode_attention(q[t:t + 1], k[None], v[None], S)
        assert torch.equal(bf16_bits(full[t]), bf16_bits(one[0]))
    assert not torch.equal(bf16_bits(got), bf16_bits(full))       # the mask matters
    assert oatt.verify_bounds(4, 94, S, True) == [95, 96, 96, 96]   # clamped at S
    assert oatt.verify_bounds(3, 5, S, False) == [S, S, S]
    # the reference test's closed form, restated with torch.softmax in fp32
    sm = torch.zeros(n, H, D)
    for t in range(n):
        nk = base + t + 1
        for h in range(H):
            kv = h // (H // KV)
            sc = q[t, h].float() @ k[kv, :nk].float().t() / math.sqrt(D)
            sm[t, h] = torch.softmax(sc, 0) @ v[kv, :nk].float()
    assert torch.allclose(got.float(), sm, rtol=1e-2, atol=1e-2)
    # a wrong GQA map (h // 2 -> h % 2) changes the result
    bad = oatt.decode_attention(q[:1, [0, 2, 1, 3]], k[None], v[None], base + 1)
    assert not torch.equal(bf16_bits(bad[0][[0, 2, 1, 3]]), bf16_bits(got[0]))


def test_causal_prefill_first_row_and_bruteforce():
    g = torch.Generator().manual_seed(15)
    q = torch.randn(4, 9, 128, generator=g)
    k = torch.randn(2, 9, 128, generator=g)
    v = torch.randn(2, 9, 128, generator=g)
    o = oatt.causal_prefill_attention(q, k, v)
    assert torch.allclose(o[0, 0], v[0, 0]) and torch.allclose(o[3, 0], v[1, 0])
    for h in range(4):
        for t in range(9):
            s = torch.tensor([float(q[h, t] @ k[h // 2, j]) for j in range(t + 1)]) / math.sqrt(128)
            w = torch.softmax(s.double(), 0)
            want = (w[:, None] * v[h // 2, : t + 1].double()).sum(0)
            assert torch.allclose(o[h, t].double(), want, atol=1e-5)


# ----------------------------------------------------------------------------------- blocks


def test_qkv_head_composition():
    g = torch.Generator().manual_seed(16)
    D, Hq, Hkv, HD, G = 256, 2, 1, 128, 32
    M = (Hq + 2 * Hkv) * HD
    q8, s = og.rtn_quantize(torch.randn(M, D, generator=g) * 0.05, G)
    cur = torch.randn(1, D, generator=g).to(torch.bfloat16)
    n_in = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    n_qn = (torch.rand(HD, generator=g) + 0.5).to(torch.bfloat16)
    n_kn = (torch.rand(HD, generator=g) + 0.5).to(torch.bfloat16)
    table = on.rope_angle_table(64, HD, 1e6)
    qq, kk, vv = oblk.qkv_head(cur, n_in, q8, s, n_qn, n_kn, table[0], Hq, Hkv, HD, 1e-6)
    hn = on.rms_norm(cur, n_in, 1e-6)
    raw = og.gemv(og.dequant_f(q8, s), hn.reshape(-1)).float().to(torch.bfloat16)
    assert torch.equal(vv.reshape(-1), raw[(Hq + Hkv) * HD:])         # v = raw, unnormalised
    # angle 0: RoPE is the identity, q = RMSNorm_w(raw_q) per head
    assert torch.equal(qq.reshape(Hq, HD), on.rms_norm(raw[: Hq * HD].reshape(Hq, HD), n_qn, 1e-6))
    assert torch.equal(kk.reshape(Hkv, HD),
                       on.rms_norm(raw[Hq * HD:(Hq + Hkv) * HD].reshape(Hkv, HD), n_kn, 1e-6))
    q7, _, _ = oblk.qkv_head(cur, n_in, q8, s, n_qn, n_kn, table[7], Hq, Hkv, HD, 1e-6)
    assert torch.equal(q7.reshape(Hq, HD), on.rope(qq.reshape(Hq, HD), table[7]))


def test_swiglu_closed_forms():
    g = torch.Generator().manual_seed(17)
    D, FF, G = 64, 192, 32
    lin = lambda M, K: og.rtn_quantize(torch.randn(M, K, generator=g) * 0.1, G)  # noqa: E731
    wg, wu, wd = lin(FF, D), lin(FF, D), lin(D, FF)
    cur = torch.randn(2, D, generator=g).to(torch.bfloat16)
    a = torch.randn(2, D, generator=g).to(torch.bfloat16)
    n = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    zero_d = (torch.zeros_like(wd[0]), wd[1])
    nxt, _ = oblk.swiglu_mlp(cur, a, n, wg, wu, zero_d, 1e-6)
    assert torch.equal(nxt, (cur.float() + a.float()).to(torch.bfloat16))   # Wd = 0 -> x1
    nxt, _ = oblk.swiglu_mlp(cur, a, n, wg, wu, wd, 1e-6)
    x1 = cur.double() + a.double()
    hf = x1 / torch.sqrt((x1 ** 2).mean(-1, keepdim=True) + 1e-6) * n.double()
    Wg, Wu, Wd = (og.dequant_f32(*w).double() for w in (wg, wu, wd))
    gg = hf @ Wg.t()
    want = x1 + (gg / (1 + torch.exp(-gg)) * (hf @ Wu.t())) @ Wd.t()
    assert torch.allclose(nxt.double(), want, rtol=1e-2, atol=1e-2)
    # fuse_o: a = bf16(Wo @ cx)
    wo = lin(D, 128)
    cx = torch.randn(2, 128, generator=g).to(torch.bfloat16)
    nxt_o, a_o = oblk.swiglu_mlp(cur, cx, n, wg, wu, wd, 1e-6, wo=wo)
    assert torch.equal(a_o, (cx.double() @ og.dequant_f(*wo).t()).float().to(torch.bfloat16))
    assert torch.equal(nxt_o, oblk.swiglu_mlp(cur, a_o, n, wg, wu, wd, 1e-6)[0])
    # the literal fp32 golden stays within the north-star tolerance of the exact one
    lit, _ = oblk.swiglu_mlp(cur, cx, n, wg, wu, wd, 1e-6, wo=wo, dt=torch.float32)
    assert torch.allclose(lit.float(), nxt_o.float(), rtol=1e-2, atol=1e-2)


def test_exact_and_literal_chains_tiny_model():
    """The fp64 (parity) and fp32 (baseline) chains agree within tolerance on a tiny model, and
    one chain step reproduces the block goldens composed by hand."""
    from iron_amd.applications.qwen3_0_6b.weights import Qwen3Config, random_qwen3_weights
    from oracle.qwen3 import Qwen3CpuChain

    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=3)
    ex = Qwen3CpuChain(cfg, w, 64)
    li = Qwen3CpuChain(cfg, w, 64, dt=torch.float32)
    tok = 9
    for pos in range(4):
        le, ll = ex.step(tok, pos), li.step(tok, pos)
        assert torch.allclose(le.float(), ll.float(), rtol=1e-2, atol=5e-2)
        tok = Qwen3CpuChain.argmax(le)
    # hand composition of layer 0 at position 4 against the chain's cache append
    L = w["layers"][0]
    x = w["embed"][tok].reshape(1, -1)
    table = on.rope_angle_table(64, cfg.head_dim, cfg.rope_theta)
    q, k, v = oblk.qkv_head(x, L["input_norm"], *L["qkv"], L["q_norm"], L["k_norm"], table[4],
                            cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.eps)
    ex.step(tok, 4)
    assert torch.equal(ex.k_cache[0, :, 4].reshape(-1), k.reshape(-1))
    assert torch.equal(ex.v_cache[0, :, 4].reshape(-1), v.reshape(-1))
