"""GPU parity of the RoPE and QKNormRoPE drop-ins against the CPU oracle (oracle/norms.py),
through the operator API.

Bars, written in each test: bit-exact against the exact oracle (each rotated value and each
normalised head evaluated exactly and rounded once to bf16, as the device does in fp64); and the
reference test's own tolerance (rel 0.05 / abs 0.02, iron/operators/qk_norm_rope/test.py) against
the reference golden's single final rounding (round_norm=False). Shapes follow the reference
tests (rope/test.py get_params, qk_norm_rope/test.py: Qwen3-0.6B 16/8 and Qwen3-4B 32/8 heads),
plus edge cases: one angle row for all rows, interleaved pairs, head_dim not a multiple of 64,
distinct cos/sin halves, and the kv_direct cache write at the first, a middle and the last
position and at an offset past the cache (no write).
"""

import pytest
import torch

from iron_amd.operators import QKNormRoPE, RoPE
from oracle import norms as onorm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _bits_equal(got, want, what):
    g = got.cpu().reshape(-1).view(torch.int16)
    w = want.cpu().reshape(-1).view(torch.int16)
    bad = int((g != w).sum())
    assert bad == 0, f"{what}: {bad} of {w.numel()} bf16 values differ from the exact oracle"


@pytest.mark.parametrize("rows,cols,angle_rows,method", [
    (32, 512, 8, 0), (32, 512, 32, 0),          # the reference's regular cases
    (64, 128, 16, 0), (32, 128, 8, 1), (64, 128, 32, 1),
    (4096, 64, 4096, 0),                       # rope/reference.py generator defaults
    (24, 128, 1, 0),                           # one angle row for all rows (a decode step)
    (8, 32, 2, 1),
])
def test_rope(rows, cols, angle_rows, method):
    _say(f"rope rows={rows} cols={cols} angle_rows={angle_rows} method={method}")
    gen = torch.Generator().manual_seed(rows * 7 + cols + angle_rows + method)
    x = torch.randn(rows, cols, generator=gen).to(torch.bfloat16)
    table = onorm.rope_angle_table(8192, cols, 1e4)
    ang = table[torch.randint(0, 8192, (angle_rows,), generator=gen)]
    op = RoPE(rows=rows, cols=cols, angle_rows=angle_rows, method_type=method)
    fn = op.get_callable()
    y = torch.zeros(rows, cols, dtype=torch.bfloat16, device=DEV)
    fn(x.to(DEV), ang.to(DEV), y)
    torch.cuda.synchronize()
    want = (onorm.rope if method == 0 else onorm.rope_interleaved)(x, ang)
    _bits_equal(y, want, "rope")


def _qk_case(n_q, n_v, HD, seed, halves="dup"):
    """The reference golden's generator, restated (qk_norm_rope/reference.py:43-57): N(0,1) qkv,
    gamma = N(0,1) * 0.2 + 1 per head, cos / sin of uniform angles with duplicated halves; or
    independent halves ("split")."""
    gen = torch.Generator().manual_seed(seed)
    n_qk = n_q + n_v
    qkv = torch.randn((n_qk + n_v) * HD, generator=gen).to(torch.bfloat16)
    gamma = (torch.randn(n_qk * HD, generator=gen) * 0.2 + 1.0).to(torch.bfloat16)
    ang = torch.rand(HD // 2, generator=gen) * 2 * torch.pi
    if halves == "dup":
        cos, sin = torch.cat([ang.cos(), ang.cos()]), torch.cat([ang.sin(), ang.sin()])
    else:
        ang2 = torch.rand(HD // 2, generator=gen) * 2 * torch.pi
        cos, sin = torch.cat([ang.cos(), ang2.cos()]), torch.cat([ang.sin(), ang2.sin()])
    scratch = torch.cat([gamma, cos.to(torch.bfloat16), sin.to(torch.bfloat16)])
    return qkv, scratch


@pytest.mark.parametrize("n_q,n_v,HD,halves", [
    (16, 8, 128, "dup"),      # Qwen3-0.6B (reference test id qwen3-0.6b)
    (32, 8, 128, "dup"),      # Qwen3-4B (qwen3-4b)
    (16, 8, 128, "split"),    # distinct cos / sin halves
    (4, 2, 96, "dup"),        # head_dim below / not a multiple of 64
    (2, 1, 256, "split"),
])
def test_qk_norm_rope(n_q, n_v, HD, halves):
    _say(f"qk_norm_rope n_q={n_q} n_v={n_v} HD={HD} halves={halves}")
    n_qk = n_q + n_v
    qkv, scratch = _qk_case(n_q, n_v, HD, seed=n_q * 100 + HD, halves=halves)
    op = QKNormRoPE(qkv_dim=(n_qk + n_v) * HD, head_dim=HD, n_qk_heads=n_qk, n_v_heads=n_v,
                    epsilon=1e-6)
    fn = op.get_callable()
    out = torch.zeros_like(qkv, device=DEV)
    fn(qkv.to(DEV), out, scratch.to(DEV))
    torch.cuda.synchronize()
    _bits_equal(out, onorm.qk_norm_rope(qkv, scratch, n_qk, n_v, HD, 1e-6), "qk_norm_rope")
    gold = onorm.qk_norm_rope(qkv, scratch, n_qk, n_v, HD, 1e-6, round_norm=False).float()
    err = (out.cpu().float() - gold).abs()
    assert (err <= 0.02 + 0.05 * gold.abs()).all()


@pytest.mark.parametrize("pos", [0, 300, 511, 512])
def test_qk_norm_rope_kv_direct(oracle_provider, pos):
    """kv_direct: the rotated K heads and the V heads land in the head-major [K_t | V_t] cache
    at the element offset pos * 2 * head_dim; pos 512 is past the 512-token cache (no write).
    Every other cache element keeps its value."""
    n_q, n_v, HD, S = 16, 8, 128, 512
    n_qk = n_q + n_v
    _say(f"qk_norm_rope kv_direct pos={pos}")
    qkv, scratch = _qk_case(n_q, n_v, HD, seed=pos + 5)
    op = QKNormRoPE(qkv_dim=(n_qk + n_v) * HD, head_dim=HD, n_qk_heads=n_qk, n_v_heads=n_v,
                    kv_direct=True, max_seq_len=S)
    fn = op.get_callable()
    fn.params.write(op.kv_offset_parameter, pos * 2 * HD)
    cache0 = torch.randn(op.kv_cache_elems, generator=torch.Generator().manual_seed(1)).to(
        torch.bfloat16)
    cache = cache0.to(DEV)
    out = torch.zeros_like(qkv, device=DEV)
    fn(qkv.to(DEV), out, scratch.to(DEV), cache)
    torch.cuda.synchronize()
    out_want = torch.zeros_like(qkv)
    cache_want = op.reference(qkv, out_want, scratch, cache0,
                              params={op.kv_offset_parameter: pos * 2 * HD}, last=cache0)
    _bits_equal(out, out_want, "qkv_out")
    _bits_equal(cache, cache_want, "kv cache")
    if pos >= S:
        assert torch.equal(cache.cpu(), cache0)
