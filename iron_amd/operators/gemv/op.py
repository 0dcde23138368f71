"""GEMV: bf16-weight matrix-vector product on gfx950 (used for the bf16 LM head).

Drop-in for iron/operators/gemv/op.py (fields, the kernel_vector_size narrowing rule, the
``[matrix (M, K), vector (K,), output (M,)]`` spec). ``epilogue`` keeps the reference's
``"none"`` and adds ``"argmax"``: the spec then gains a trailing ``(1,)`` int64 output that must
be zero before the call and receives the packed argmax key of the bf16 outputs (decoded on the
device by ``iron_next_token``), which replaces the host argmax of the decode loop
(qwen3_npu_int8.py:612-621). The reference's ``"gelu"`` epilogue is not on this path.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import stream_ptr


@dataclass
class GEMV(MLIROperator):
    M: int
    K: int
    num_aie_columns: int = 1
    tile_size_input: int = 2
    tile_size_output: int | None = None
    num_batches: int = 1
    kernel_vector_size: int = field(default=64, repr=False)
    epilogue: str = field(default="none", repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "num_aie_columns": "col",
        "tile_size_input": "tsi",
        "tile_size_output": "tso",
        "num_batches": "batch",
    }

    def __post_init__(self):
        if self.tile_size_output is None:
            self.tile_size_output = self.tile_size_input
        if not (self.tile_size_output % self.tile_size_input == 0
                and self.tile_size_output >= self.tile_size_input):
            raise ValueError("tile_size_output must be a multiple of tile_size_input")
        while self.kernel_vector_size > 16 and self.K < 2 * self.kernel_vector_size:
            self.kernel_vector_size //= 2
        if self.K % self.kernel_vector_size or self.K < 2 * self.kernel_vector_size:
            raise ValueError(f"K ({self.K}) must be a multiple of kernel_vector_size "
                             f"({self.kernel_vector_size}) and at least twice as large")
        if self.epilogue not in ("none", "argmax"):
            raise ValueError(f"unknown epilogue {self.epilogue!r} (expected 'none' or 'argmax')")
        if self.K % 8:
            raise ValueError("K must be a multiple of 8")
        MLIROperator.__init__(self, context=self.context)

    @property
    def name(self) -> str:
        base = super().name
        return base if self.epilogue == "none" else f"{base}_epi{self.epilogue}"

    def get_arg_spec(self):
        batch_dim = (self.num_batches,) if self.num_batches > 1 else ()
        spec = [
            AIERuntimeArgSpec("in", batch_dim + (self.M, self.K)),   # matrix
            AIERuntimeArgSpec("in", batch_dim + (self.K,)),          # vector
            AIERuntimeArgSpec("out", batch_dim + (self.M,)),         # output
        ]
        if self.epilogue == "argmax":
            spec.append(AIERuntimeArgSpec("inout", (max(self.num_batches, 1),),
                                          dtype=torch.int64))
        return spec

    def get_callable(self):
        lib = _lib.load()
        M, K = self.M, self.K

        def call(*args):
            args = check_args(self, args)
            a, x, y = args[:3]
            keys = args[3] if self.epilogue == "argmax" else None
            s = stream_ptr()
            for nb in range(self.num_batches):
                kp = keys.data_ptr() + nb * 8 if keys is not None else None
                _lib.check(lib.iron_lm_head(
                    a.data_ptr() + nb * M * K * 2, _lib.IRON_WEIGHT_BF16,
                    x.data_ptr() + nb * K * 2, None, 0.0, y.data_ptr() + nb * M * 2, kp, 1, M, K,
                    16, 1, 0, s), "GEMV")

        return call
