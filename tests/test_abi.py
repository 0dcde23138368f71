"""CPU checks of the C ABI: the library loads, exports every declared symbol, and rejects bad
arguments with the documented status before touching the GPU (the reference raises ValueError
for shape constraints, iron/operators/gemv_int8/op.py:74-84)."""

import ctypes
import re
from pathlib import Path

import pytest

from iron_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "iron_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:[\w\*\s]+?)\b(iron_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared()
    assert "iron_gemv_w8a16" in names and "iron_decode_attn" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in iron_hip.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) <= set(names)


def test_abi_version(lib):
    assert lib.iron_abi_version() == _lib.ABI_VERSION == 11


def test_wire_bytes(lib):
    out = ctypes.c_size_t()
    assert lib.iron_wire_bytes(4096, 1024, 32, 4, ctypes.byref(out)) == 0
    assert out.value == 1024 * (4 * 1024 + 4 * 32 * 2)
    assert lib.iron_wire_bytes(4096, 1000, 32, 4, ctypes.byref(out)) == _lib.IRON_ERR_SHAPE
    assert b"bad geometry" in lib.iron_last_error()


@pytest.mark.parametrize("d", [1, 2, 3, 4, 12, 16, 37, 1000, 65535])
def test_fastdiv_matches_integer_division(lib, d):
    for n in list(range(0, 5000, 7)) + [2**20 - 1, 2**24 + 5, 2**31 - 1, 151936]:
        assert lib.iron_test_fastdiv(n, d) == n // d


def test_gemv_rejects_bad_arguments(lib):
    f = lib.iron_gemv_w8a16
    # null wire
    assert f(None, 16, 16, 1, 64, 128, 32, 4, 0, None) == _lib.IRON_ERR_NULL
    fake = 1 << 20  # an aligned non-null address; validation fails before any use
    # K not a multiple of G
    assert f(fake, fake, fake, 1, 64, 100, 32, 4, 0, None) == _lib.IRON_ERR_SHAPE
    # tile_m does not divide M
    assert f(fake, fake, fake, 1, 66, 128, 32, 4, 0, None) == _lib.IRON_ERR_SHAPE
    # non power-of-two group
    assert f(fake, fake, fake, 1, 64, 144, 48, 4, 0, None) == _lib.IRON_ERR_SHAPE
    # misaligned wire
    assert f(fake + 2, fake, fake, 1, 64, 128, 32, 4, 0, None) == _lib.IRON_ERR_ALIGN
    # batch 16 -> unsupported on the GEMV path (MFMA GEMM)
    assert f(fake, fake, fake, 16, 64, 128, 32, 4, 0, None) == _lib.IRON_ERR_UNSUPPORTED
    # unknown domain
    assert f(fake, fake, fake, 1, 64, 128, 32, 4, 7, None) == _lib.IRON_ERR_SHAPE


def test_attention_rejects_bad_arguments(lib):
    f = lib.iron_decode_attn
    fake = 1 << 20
    args = lambda **kw: dict(dict(q=fake, k=fake, v=fake, sb=0, sh=0, st=128, ctx=None, cc=1,  # noqa
                                  o=fake, B=1, H=16, KV=8, D=128, L=64, scale=0.1, acc=0,
                                  ws=None, wsb=0), **kw)

    def call(**kw):
        a = args(**kw)
        return f(a["q"], a["k"], a["v"], a["sb"], a["sh"], a["st"], a["ctx"], a["cc"], a["o"],
                 a["B"], a["H"], a["KV"], a["D"], a["L"], a["scale"], a["acc"], a["ws"], a["wsb"],
                 None)

    assert call(q=None) == _lib.IRON_ERR_NULL
    assert call(D=64) == _lib.IRON_ERR_UNSUPPORTED
    assert call(H=12, KV=8) == _lib.IRON_ERR_SHAPE
    assert call(cc=65) == _lib.IRON_ERR_SHAPE
    assert call(st=100) == _lib.IRON_ERR_ALIGN
    assert call(acc=7) == _lib.IRON_ERR_SHAPE           # unknown accumulation mode
    # a long context needs split-K scratch: missing workspace is reported, not ignored
    assert call(L=4096, cc=4096) == _lib.IRON_ERR_WORKSPACE
    assert lib.iron_decode_attn_workspace(1, 16, 8, 128, 4096) > 0
    assert lib.iron_decode_attn_workspace(1, 16, 8, 64, 4096) == 0


def test_rope_and_qk_norm_rope_reject_bad_arguments(lib):
    fake = 1 << 20
    r = lib.iron_rope
    assert r(None, fake, fake, 4, 128, 4, 0, None) == _lib.IRON_ERR_NULL
    assert r(fake, fake, fake, 4, 127, 4, 0, None) == _lib.IRON_ERR_SHAPE      # odd cols
    assert r(fake, fake, fake, 6, 128, 4, 0, None) == _lib.IRON_ERR_SHAPE      # 4 does not divide 6
    assert r(fake, fake, fake, 4, 128, 8, 0, None) == _lib.IRON_ERR_SHAPE      # more angle rows
    assert r(fake, fake, fake, 4, 128, 0, 0, None) == _lib.IRON_ERR_SHAPE
    assert r(fake, fake, fake, 4, 128, 4, 2, None) == _lib.IRON_ERR_UNSUPPORTED
    assert b"method" in lib.iron_last_error()
    q = lib.iron_qk_norm_rope
    assert q(fake, None, fake, None, None, 128, 24, 8, 0, 1e-6, None) == _lib.IRON_ERR_NULL
    assert q(fake, fake, fake, None, None, 127, 24, 8, 0, 1e-6, None) == _lib.IRON_ERR_SHAPE
    assert q(fake, fake, fake, None, None, 2048, 24, 8, 0, 1e-6, None) == _lib.IRON_ERR_SHAPE
    assert q(fake, fake, fake, None, None, 128, 8, 9, 0, 1e-6, None) == _lib.IRON_ERR_SHAPE
    # the cache write needs the device offset and the cache length
    assert q(fake, fake, fake, fake, None, 128, 24, 8, 512, 1e-6, None) == _lib.IRON_ERR_SHAPE
    assert q(fake, fake, fake, fake, fake, 128, 24, 8, 0, 1e-6, None) == _lib.IRON_ERR_SHAPE


def test_rope_operators_reject_invalid_shapes():
    """The reference operators' constraints (rope/op.py:37-52) and the QKV layout."""
    from iron_amd.operators import QKNormRoPE, RoPE
    for kw in (dict(rows=32, cols=48), dict(rows=32, cols=64, angle_rows=12),
               dict(rows=32, cols=64, angle_rows=64), dict(rows=32, cols=64, method_type=2),
               dict(rows=6, cols=64, num_aie_columns=4)):
        with pytest.raises(ValueError):
            RoPE(**kw)
    with pytest.raises(ValueError):
        QKNormRoPE(qkv_dim=4000, head_dim=128, n_qk_heads=24, n_v_heads=8)
    with pytest.raises(ValueError):
        QKNormRoPE(qkv_dim=1280, head_dim=128, n_qk_heads=2, n_v_heads=8)
    op = QKNormRoPE(qkv_dim=4096, head_dim=128, n_qk_heads=24, n_v_heads=8, kv_direct=True)
    assert op.kv_cache_elems == 8 * 2 * 512 * 128
    assert [s.shape for s in op.get_arg_spec()] == [(4096,), (4096,), (3328,), (1048576,)]


def test_status_to_exception(lib):
    lib.iron_wire_bytes(1, 1, 3, 4, ctypes.byref(ctypes.c_size_t()))
    with pytest.raises(ValueError, match="bad geometry"):
        _lib.check(_lib.IRON_ERR_SHAPE, "iron_wire_bytes")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.IRON_ERR_HIP, "x")


def test_mlp_and_qkv_reject_bad_arguments(lib):
    fake = 1 << 20
    # MLP: FF not divisible by tile_m_gu
    rc = lib.iron_swiglu_mlp(fake, fake, fake, None, fake, fake, fake, fake, None, 1, 1024, 3000,
                             0, 32, 4, 12, 4, 0, 1e-6, fake, 1 << 20, None)
    assert rc == _lib.IRON_ERR_SHAPE
    # QKV: head_dim 64 unsupported
    rc = lib.iron_qkv_head(fake, fake, fake, fake, fake, fake, 0, fake, fake, fake, 0, 0, 0,
                           fake, 1, 1024, 64, 16, 8, 512, 32, 4, 0, 1e-6, fake, 1 << 20, None)
    assert rc == _lib.IRON_ERR_UNSUPPORTED
    # QKV: workspace too small
    rc = lib.iron_qkv_head(fake, fake, fake, fake, fake, fake, 0, fake, fake, fake, 0, 0, 0,
                           fake, 1, 1024, 128, 16, 8, 512, 32, 4, 0, 1e-6, fake, 16, None)
    assert rc == _lib.IRON_ERR_WORKSPACE


def test_persistent_decode_rejects_bad_arguments(lib):
    """Validation of iron_decode_persistent runs before any HIP call."""
    f = lib.iron_decode_persistent
    fake = 1 << 20
    ws = lib.iron_decode_persistent_workspace(1024, 3072, 16, 8, 128)
    assert ws > 0 and ws % 256 == 0
    assert lib.iron_decode_persistent_workspace(1024, 3072, 16, 8, 64) == 0
    assert lib.iron_decode_persistent_workspace(2048, 6144, 16, 8, 128) == 0

    def call(**kw):
        a = dict(layers=fake, n=28, D=1024, FF=3072, Hq=16, Hkv=8, HD=128, S=4096,
                 sh=4096 * 128, st=128, G=32, tq=4, to=4, tgu=12, td=4, dom=0, x=fake, xo=fake,
                 pos=fake, ang=fake, ws=fake, wsb=ws)
        a.update(kw)
        return f(a["layers"], a["n"], a["D"], a["FF"], a["Hq"], a["Hkv"], a["HD"], a["S"],
                 a["sh"], a["st"], a["G"], a["tq"], a["to"], a["tgu"], a["td"], a["dom"], a["x"],
                 a["xo"], a["pos"], a["ang"], 1e-6, 0.088, a["ws"], a["wsb"], None)

    assert call(layers=None) == _lib.IRON_ERR_NULL
    assert call(FF=4096) == _lib.IRON_ERR_UNSUPPORTED       # no kernel for that shape
    assert b"no persistent kernel" in lib.iron_last_error()
    assert call(n=0) == _lib.IRON_ERR_SHAPE
    assert call(st=100) == _lib.IRON_ERR_SHAPE              # token stride not 16-byte rows
    assert call(G=48) == _lib.IRON_ERR_SHAPE
    assert call(tgu=7) == _lib.IRON_ERR_SHAPE               # row blocks must divide FF
    assert call(dom=5) == _lib.IRON_ERR_SHAPE
    assert call(ang=fake + 2) == _lib.IRON_ERR_ALIGN
    assert call(wsb=ws - 8) == _lib.IRON_ERR_WORKSPACE
    assert call(ws=fake + 64) == _lib.IRON_ERR_ALIGN


def test_persistent_gen_validation(lib):
    """The greedy-loop variant's own argument checks (host-only; nothing is launched)."""
    f = lib.iron_decode_persistent_gen
    fake = 1 << 20
    ws = lib.iron_decode_persistent_workspace(1024, 3072, 16, 8, 128)

    def call(gen, **kw):
        a = dict(ang=fake, wsb=ws)
        a.update(kw)
        g = ctypes.byref(gen) if gen is not None else None
        return f(fake, 28, 1024, 3072, 16, 8, 128, 4096, 4096 * 128, 128, 32, 4, 4, 12, 4, 0, g,
                 fake, fake, a["ang"], 1e-6, 0.088, fake, a["wsb"], None)

    def gen(**kw):
        a = dict(keys=fake, emb=fake, tokens=fake, token_log=fake, step=fake, ctx=fake,
                 rope_table=fake, vocab=151936, log_len=4097)
        a.update(kw)
        return _lib.DecodeGen(**a)

    assert call(None) == _lib.IRON_ERR_NULL
    assert b"null gen" in lib.iron_last_error()
    assert call(gen(keys=None)) == _lib.IRON_ERR_NULL
    assert call(gen(emb=None)) == _lib.IRON_ERR_NULL
    assert call(gen(vocab=0)) == _lib.IRON_ERR_SHAPE
    assert call(gen(step=None)) == _lib.IRON_ERR_NULL      # a log needs a step counter
    assert call(gen(log_len=0)) == _lib.IRON_ERR_NULL
    assert call(gen(emb=fake + 2)) == _lib.IRON_ERR_ALIGN
    assert call(gen(rope_table=fake + 2)) == _lib.IRON_ERR_ALIGN
    assert call(gen(), ang=fake + 2) == _lib.IRON_ERR_ALIGN
    assert call(gen(), wsb=ws - 8) == _lib.IRON_ERR_WORKSPACE


def test_persistent_layer_check(lib):
    fake = 1 << 20
    d = _lib.LayerDesc(*([fake] * 11))
    args = (1024, 3072, 16, 8, 128, 32, 4, 4, 12, 4, 0)
    assert lib.iron_decode_persistent_check_layer(ctypes.byref(d), *args) == _lib.IRON_OK
    d.wd = fake + 8
    assert lib.iron_decode_persistent_check_layer(ctypes.byref(d), *args) == _lib.IRON_ERR_ALIGN
    d.wd = fake
    d.n_kn = None
    assert lib.iron_decode_persistent_check_layer(ctypes.byref(d), *args) == _lib.IRON_ERR_NULL
    assert lib.iron_decode_persistent_check_layer(None, *args) == _lib.IRON_ERR_NULL


def test_next_token_validation(lib):
    """The token log is bounded: a log needs a positive length (and a row stride that holds it
    when B > 1); these checks fail before anything is launched."""
    f = lib.iron_next_token
    fake = 1 << 20
    # keys, tokens, emb, x, token_log, log_stride, log_len, step, B, D, vocab, stream
    assert f(None, fake, None, None, None, 0, 0, None, 1, 1024, 100, None) == _lib.IRON_ERR_NULL
    assert f(fake, fake, None, None, fake, 0, 8, None, 1, 1024, 100, None) == _lib.IRON_ERR_NULL
    assert f(fake, fake, None, None, fake, 0, 0, fake, 1, 1024, 100, None) == _lib.IRON_ERR_SHAPE
    assert b"log_len" in lib.iron_last_error()
    assert f(fake, fake, None, None, fake, 4, 8, fake, 2, 1024, 100, None) == _lib.IRON_ERR_SHAPE
    assert f(fake, fake, None, None, None, 0, 0, None, 65, 1024, 100, None) == _lib.IRON_ERR_SHAPE


def test_handoff_probe_validation(lib):
    """The hand-off probe's arguments are checked before the device is queried or anything is
    launched."""
    q = lib.iron_handoff_probe_workspace
    assert q(1024) == q(256) == 2 * 8 * 4096 * 8 + 4096  # the tagged mode's 8 copies, twice
    assert q(0) == 0 and q(1000) == 0 and q(2048 + 256) == 0
    assert q(640) == q(256)  # the XCD modes take multiples of 32
    f = lib.iron_handoff_probe
    ws, fake = q(1024), 1 << 20
    assert f(5, 1024, 10, 0, fake, ws, None) == _lib.IRON_ERR_SHAPE
    assert b"unknown mode" in lib.iron_last_error()
    assert f(_lib.IRON_HANDOFF_TAGGED, 1000, 10, 0, fake, ws, None) == _lib.IRON_ERR_SHAPE
    assert f(_lib.IRON_HANDOFF_TAGGED, 640, 10, 0, fake, ws, None) == _lib.IRON_ERR_SHAPE
    assert f(_lib.IRON_HANDOFF_XCD_L2, 650, 10, 0, fake, ws, None) == _lib.IRON_ERR_SHAPE
    assert f(_lib.IRON_HANDOFF_TAGGED, 1024, 0, 0, fake, ws, None) == _lib.IRON_ERR_SHAPE
    assert f(_lib.IRON_HANDOFF_FLAGS, 1024, 10, 0, None, ws, None) == _lib.IRON_ERR_WORKSPACE
    assert f(_lib.IRON_HANDOFF_FLAGS, 1024, 10, 0, fake, ws - 8, None) == _lib.IRON_ERR_WORKSPACE
    assert f(_lib.IRON_HANDOFF_COUNTER, 1024, 10, 0, fake + 8, ws, None) == _lib.IRON_ERR_ALIGN


def test_persistent_trace_setter(lib):
    """The phase-stamp setter checks alignment and is cleared with NULL (no device access)."""
    f = lib.iron_decode_persistent_set_trace
    assert f((1 << 20) + 4, 4096) == _lib.IRON_ERR_ALIGN
    assert f(1 << 20, 4096) == _lib.IRON_OK
    assert f(None, 0) == _lib.IRON_OK
