"""Operator context (the reference's AIEContext, iron/common/context.py:13-74).

Holds what the reference's context holds that still has meaning on the GPU: a build directory
(the in-tree HIP library lives next to the package), the device, and the default stream used by
operator callables. The NPU compiler choice becomes the single HIP toolchain.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import ClassVar


@dataclass
class AIEContext:
    base_dir: ClassVar[Path] = Path(__file__).resolve().parent.parent.parent

    build_dir: Path = field(default_factory=lambda: Path(os.getcwd()) / "build")
    mlir_verbose: bool = False
    compiler: str = "hipcc"
    device_index: int = 0

    def __post_init__(self) -> None:
        self.build_dir = Path(self.build_dir)
        if self.compiler != "hipcc":
            raise ValueError(f"compiler must be 'hipcc' on MI355X, got {self.compiler!r}")

    @property
    def device(self):
        import torch

        return torch.device("cuda", self.device_index)

    @property
    def kernels_dir(self) -> Path:
        return self.base_dir / "iron_amd" / "csrc"

    def stream(self):
        import torch

        return torch.cuda.current_stream(self.device)
