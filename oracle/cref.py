"""ctypes binding of the C restatement ``oracle/liboracle.so`` (test infrastructure only)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import torch

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        vp, ci = ctypes.c_void_p, ctypes.c_int
        lib.oracle_wire_unpack.argtypes = [vp, ci, ci, ci, ci, ci, vp, vp]
        lib.oracle_wire_unpack.restype = ci
        lib.oracle_dequant.argtypes = [vp, vp, vp, ci, ci, ci]
        lib.oracle_gemv_f64.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci]
        lib.oracle_decode_attn_f64.argtypes = [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci,
                                               ctypes.c_double]
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _bits(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.to(torch.bfloat16).contiguous().view(torch.int16).numpy()
                                ).view(np.uint16)


def wire_unpack(wire: np.ndarray, M, K, G, tile_m, domain: str):
    w = np.ascontiguousarray(np.asarray(wire).view(np.uint8))
    q = np.empty((M, K), np.int16)
    s = np.empty((M, K // G), np.uint16)
    rc = load().oracle_wire_unpack(_p(w), M, K, G, tile_m, 1 if domain == "biased" else 0,
                                   _p(q), _p(s))
    if rc:
        raise ValueError("bad wire geometry")
    return torch.from_numpy(q), torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)


def dequant(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    M, K = q.shape
    qn = np.ascontiguousarray(q.to(torch.int16).numpy())
    sn = _bits(s)
    out = np.empty((M, K), np.uint16)
    load().oracle_dequant(_p(qn), _p(sn), _p(out), M, K, K // s.shape[1])
    return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)


def gemv_f64(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    M, K = q.shape
    xb = _bits(x.reshape(-1, K))
    B = xb.shape[0]
    qn = np.ascontiguousarray(q.to(torch.int16).numpy())
    y = np.empty((B, M), np.float64)
    load().oracle_gemv_f64(_p(qn), _p(_bits(s)), _p(xb), _p(y), B, M, K, K // s.shape[1])
    return torch.from_numpy(y)


def decode_attn_f64(q, k, v, ctx, scale: float) -> torch.Tensor:
    B, H, D = q.shape
    KV, L = k.shape[1], k.shape[2]
    c = np.ascontiguousarray(np.asarray(ctx, dtype=np.int32).reshape(B))
    out = np.empty((B, H, D), np.float64)
    load().oracle_decode_attn_f64(_p(_bits(q)), _p(_bits(k)), _p(_bits(v)), _p(c), _p(out), B,
                                  H, KV, L, D, float(scale))
    return torch.from_numpy(out)
