"""Helpers shared by the operator classes: payload-domain codes, runtime parameters and
workspace ownership."""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib


def domain_code(domain: str) -> int:
    if domain == "signed":
        return _lib.IRON_DOMAIN_SIGNED
    if domain == "biased":
        return _lib.IRON_DOMAIN_BIASED
    raise ValueError(f"unknown payload domain: {domain}")


def stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


class RuntimeParams:
    """Named int32 runtime parameters living in device memory.

    The reference writes per-dispatch scalars (``k_cache_offset``, ``S_kv_eff``) into an NPU
    scratchpad (iron/common/sequence.py:683-711; qwen3_npu_int8.py:608-610). Here each parameter
    is a small device int32 tensor that kernels read, so a captured HIP graph replays with new
    values without re-capture. ``write`` stages the value and ``sync`` copies it to the device
    (``write`` alone also copies, so ``sync`` is only needed for the reference's call shape).
    """

    def __init__(self, device=None):
        self._device = device or torch.device("cuda", 0)
        self._tensors: dict[str, torch.Tensor] = {}
        self._convert: dict[str, object] = {}

    def define(self, name: str, n: int = 1, convert=None) -> torch.Tensor:
        """Declare a parameter of ``n`` entries; ``convert`` maps written values to stored ones."""
        if convert is not None:
            self._convert[name] = convert
        return self.tensor(name, n)

    def tensor(self, name: str, n: int = 1) -> torch.Tensor:
        t = self._tensors.get(name)
        if t is None or t.numel() < n:
            old = t
            t = torch.zeros(n, dtype=torch.int32, device=self._device)
            if old is not None:
                t[: old.numel()].copy_(old)
            self._tensors[name] = t
        return t

    def write(self, name: str, value) -> None:
        conv = self._convert.get(name)
        if conv is not None:
            value = conv(value)
        vals = np.atleast_1d(np.asarray(value, dtype=np.int32))
        t = self.tensor(name, vals.size)
        t[: vals.size].copy_(torch.from_numpy(vals), non_blocking=False)

    def read(self, name: str) -> np.ndarray:
        return self._tensors[name].cpu().numpy()

    def snapshot(self) -> dict:
        """Current values of every parameter (host copies), for the CPU goldens."""
        return {n: t.cpu().numpy() for n, t in self._tensors.items()}

    def sync(self) -> None:
        pass

    def __contains__(self, name: str) -> bool:
        return name in self._tensors


class Workspace:
    """Zero-initialised device scratch owned by an operator callable (reused across calls)."""

    def __init__(self, nbytes: int, device=None):
        self.nbytes = max(int(nbytes), 256)
        self.tensor = torch.zeros(self.nbytes, dtype=torch.uint8,
                                  device=device or torch.device("cuda", 0))

    @property
    def ptr(self) -> int:
        return self.tensor.data_ptr()
