"""ctypes binding of ``libiron_hip.so`` (declared in ``include/iron_hip.h``).

The library is the only compute path: loading fails loudly when it has not been built, and every
entry point's status is turned into the reference's exception classes -- ``ValueError`` for
shape/null/alignment problems (the reference raises ValueError for shape constraints,
iron/operators/gemv_int8/op.py:74-84) and ``RuntimeError`` for HIP failures (the reference raises
RuntimeError on kernel failure, iron/common/sequence.py:858-862).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libiron_hip.so"

ABI_VERSION = 11         # IRON_ABI_VERSION of include/iron_hip.h
IRON_OK = 0
IRON_ERR_NULL = -1
IRON_ERR_SHAPE = -2
IRON_ERR_ALIGN = -3
IRON_ERR_WORKSPACE = -4
IRON_ERR_HIP = -5
IRON_ERR_UNSUPPORTED = -6

IRON_DOMAIN_SIGNED = 0
IRON_DOMAIN_BIASED = 1
IRON_WEIGHT_INT8 = 0
IRON_WEIGHT_BF16 = 1
IRON_ACCUM_F64 = 0
IRON_ACCUM_F32 = 1
ACCUM = {"f64": IRON_ACCUM_F64, "f32": IRON_ACCUM_F32}
IRON_ROPE_TWO_HALVES = 0
IRON_ROPE_INTERLEAVED = 1
IRON_HANDOFF_TAGGED = 0
IRON_HANDOFF_COUNTER = 1
IRON_HANDOFF_FLAGS = 2
IRON_HANDOFF_XCD_L2 = 3
IRON_HANDOFF_XCD_AGENT = 4


def accum_mode(name: str) -> int:
    """Attention accumulation mode (enum iron_accum) from its name, "f64" or "f32"."""
    if name not in ACCUM:
        raise ValueError(f"accumulate must be one of {sorted(ACCUM)}, got {name!r}")
    return ACCUM[name]

_VALUE_ERRORS = {IRON_ERR_NULL, IRON_ERR_SHAPE, IRON_ERR_ALIGN, IRON_ERR_WORKSPACE}

_c_int, _c_ll, _c_f, _c_sz, _c_vp = (ctypes.c_int, ctypes.c_longlong, ctypes.c_float,
                                     ctypes.c_size_t, ctypes.c_void_p)


class LayerDesc(ctypes.Structure):
    """``iron_layer_desc``: one decoder layer's device pointers (include/iron_hip.h)."""

    _fields_ = [(name, _c_vp) for name in ("wqkv", "wo", "wg", "wu", "wd", "n_in", "n_post",
                                           "n_qn", "n_kn", "k_cache", "v_cache")]


class DecodeGen(ctypes.Structure):
    """``iron_decode_gen``: device state of the greedy loop (include/iron_hip.h)."""

    _fields_ = [(name, _c_vp) for name in ("keys", "emb", "tokens", "token_log", "step", "ctx",
                                           "rope_table")] + [("vocab", _c_int),
                                                             ("log_len", _c_int)] + \
        [(name, _c_vp) for name in ("lm_head", "lm_norm", "logits")]


# name -> (restype, argtypes). Kept in the order of include/iron_hip.h.
SIGNATURES = {
    "iron_abi_version": (_c_int, []),
    "iron_last_error": (ctypes.c_char_p, []),
    "iron_wire_bytes": (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_sz)]),
    "iron_dequant_w8": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "iron_gemv_w8a16": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _c_int, _c_vp]),
    "iron_gemv_bf16": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp]),
    "iron_gemm_w8a16_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int]),
    "iron_gemm_w8a16": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _c_int, _c_vp, _c_sz, _c_vp]),
    "iron_rmsnorm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_f, _c_vp]),
    "iron_rope": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "iron_qk_norm_rope": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int,
                                   _c_int, _c_f, _c_vp]),
    "iron_lm_head": (_c_int, [_c_vp, _c_int, _c_vp, _c_vp, _c_f, _c_vp, _c_vp, _c_int, _c_int,
                              _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "iron_next_token": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp,
                                 _c_int, _c_int, _c_int, _c_vp]),
    "iron_embed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp]),
    "iron_advance_positions": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int,
                                        _c_int, _c_vp]),
    "iron_qkv_head_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_qkv_head": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp,
                               _c_vp, _c_ll, _c_ll, _c_ll, _c_vp, _c_int, _c_int, _c_int, _c_int,
                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_vp, _c_sz,
                               _c_vp]),
    "iron_decode_attn_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_decode_attn": (_c_int, [_c_vp, _c_vp, _c_vp, _c_ll, _c_ll, _c_ll, _c_vp, _c_int,
                                  _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_int,
                                  _c_vp, _c_sz, _c_vp]),
    "iron_decode_attn_noalloc": (_c_int, [_c_vp, _c_vp, _c_vp, _c_ll, _c_ll, _c_ll, _c_vp,
                                          _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _c_f, _c_int, _c_vp]),
    "iron_decode_attn_verify_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_decode_attn_verify": (_c_int, [_c_vp, _c_vp, _c_vp, _c_ll, _c_ll, _c_vp, _c_int,
                                         _c_int, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _c_f, _c_vp, _c_sz, _c_vp]),
    "iron_qkv_attn_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_qkv_attn": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                               _c_ll, _c_ll, _c_ll, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _c_f, _c_int, _c_vp,
                               _c_sz, _c_vp]),
    "iron_prefill_attn": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                   _c_int, _c_f, _c_vp]),
    "iron_swiglu_mlp_workspace": (_c_sz, [_c_int, _c_int, _c_int]),
    "iron_swiglu_mlp": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                 _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                 _c_int, _c_f, _c_vp, _c_sz, _c_vp]),
    "iron_decode_persistent_workspace": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_decode_persistent_supported": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "iron_decode_persistent_check_layer": (_c_int, [ctypes.POINTER(LayerDesc), _c_int, _c_int,
                                                    _c_int, _c_int, _c_int, _c_int, _c_int,
                                                    _c_int, _c_int, _c_int, _c_int]),
    "iron_decode_persistent": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _c_ll, _c_ll, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_f, _c_f,
                                        _c_vp, _c_sz, _c_vp]),
    "iron_decode_persistent_gen": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                            _c_int, _c_int, _c_ll, _c_ll, _c_int, _c_int, _c_int,
                                            _c_int, _c_int, _c_int, ctypes.POINTER(DecodeGen),
                                            _c_vp, _c_vp, _c_vp, _c_f, _c_f, _c_vp, _c_sz,
                                            _c_vp]),
    "iron_test_fastdiv": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32]),
    "iron_test_bf16_round": (_c_int, [_c_vp, _c_vp]),
    "iron_stream_read": (_c_int, [_c_vp, _c_sz, _c_vp, _c_int, _c_vp]),
    "iron_decode_persistent_set_trace": (_c_int, [_c_vp, _c_sz]),
    "iron_handoff_probe_workspace": (_c_sz, [_c_int]),
    "iron_handoff_probe": (_c_int, [_c_int, _c_int, _c_int, ctypes.c_uint, _c_vp, _c_sz, _c_vp]),
}

_lock = threading.Lock()
_lib = None


class IronLibraryMissing(RuntimeError):
    """The HIP library has not been built; there is no other compute path."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library with every signature declared."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        # torch first: its bundled HIP runtime then satisfies the library's libamdhip64
        # dependency by SONAME, so torch streams and our launches share one runtime.
        import torch  # noqa: F401

        path = Path(os.environ.get("IRON_HIP_LIB", LIB_PATH))
        if not path.exists():
            raise IronLibraryMissing(
                f"{path} is not built; run `python -m iron_amd.build` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.iron_abi_version() != ABI_VERSION:
            raise IronLibraryMissing(f"{path}: ABI version {lib.iron_abi_version()} != "
                                     f"{ABI_VERSION} (rebuild the library)")
        _lib = lib
        return lib


def check(status: int, what: str = "") -> None:
    """Raise the reference's exception class for a non-zero status."""
    if status == IRON_OK:
        return
    msg = load().iron_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if status in _VALUE_ERRORS:
        raise ValueError(text)
    raise RuntimeError(text)


def call(name: str, *args) -> None:
    """Invoke an int-returning entry point and raise on failure."""
    check(getattr(load(), name)(*args), name)


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None passes through as NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(stream=None) -> int | None:
    """hipStream_t of the given torch stream (default: torch's current stream)."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
