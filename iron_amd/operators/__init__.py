"""The operator library (lazy re-exports, as iron/operators/__init__.py:13-55 does).

    from iron_amd.operators import GEMVInt8   # imports iron_amd.operators.gemv_int8.op only
"""

import importlib

_OPERATOR_MODULES = {
    "DecodeAttention": "decode_attn",
    "GEMV": "gemv",
    "GEMVInt8": "gemv_int8",
    "MHA": "mha",
    "QKNormRoPE": "qk_norm_rope",
    "QKVHeadAttention": "qkv_attn",
    "QKVHeadDataParallel": "qkv_head_dp",
    "QKVHeadDataParallelOurs": "qkv_head_dp:op_ours",
    "RMSNorm": "rms_norm",
    "RoPE": "rope",
    "SwiGLUMLPDataParallel": "swiglu_mlp_dp",
    "SwiGLUMLPDataParallelOurs": "swiglu_mlp_dp:op_ours",
}

__all__ = sorted(_OPERATOR_MODULES)


def __getattr__(name):
    module = _OPERATOR_MODULES.get(name)
    if module is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    module, _, attr = module.partition(":")
    if attr:
        return getattr(importlib.import_module(f".{module}.{attr}", __name__), name)
    return getattr(importlib.import_module(f".{module}.op", __name__), name)


def __dir__():
    return sorted(set(globals()) | set(_OPERATOR_MODULES))
