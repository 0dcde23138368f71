"""RoPE: rotary position embedding of bf16 rows on gfx950.

Drop-in for iron/operators/rope/op.py:19-96: the fields (rows, cols, angle_rows,
num_aie_columns, method_type), their constraints, and the spec ``[x (rows, cols), angles
(angle_rows, cols), y (rows, cols)]``. ``angles`` rows hold interleaved [cos_i, sin_i] pairs and
each serves ``rows / angle_rows`` consecutive rows (the design's row reuse). method_type 0 pairs
dims (i, i + cols/2) (two halves, Hugging Face), 1 pairs (2i, 2i + 1) (interleaved). Every output
is the exact rotated value rounded once to bf16 (iron_rope), which for bf16 inputs is what
aie_kernels/generic/rope.cc's fp32 accumulation gives.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import stream_ptr


@dataclass
class RoPE(MLIROperator):
    rows: int
    cols: int
    angle_rows: int | None = None
    num_aie_columns: int = 1
    method_type: int = 0
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "num_aie_columns": "col",
        "angle_rows": "arows",
        "method_type": "m",
    }

    def __post_init__(self):
        if self.angle_rows is None:
            self.angle_rows = self.rows
        if self.cols < 32 or self.cols % 32:
            raise ValueError(f"RoPE: cols={self.cols} must be a positive multiple of 32")
        if self.rows % self.num_aie_columns:
            raise ValueError(
                f"RoPE: rows={self.rows} not divisible by num_aie_columns={self.num_aie_columns}")
        if self.angle_rows > self.rows or self.rows % self.angle_rows:
            raise ValueError(f"RoPE: angle_rows={self.angle_rows} must divide rows={self.rows}")
        if self.angle_rows < self.num_aie_columns or self.angle_rows % self.num_aie_columns:
            raise ValueError(f"RoPE: angle_rows={self.angle_rows} not divisible by "
                             f"num_aie_columns={self.num_aie_columns}")
        if self.method_type not in (0, 1):
            raise ValueError(f"RoPE: method_type {self.method_type} is neither 0 (two halves) "
                             "nor 1 (interleaved)")
        MLIROperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        return [
            AIERuntimeArgSpec("in", (self.rows, self.cols)),         # x
            AIERuntimeArgSpec("in", (self.angle_rows, self.cols)),   # angles
            AIERuntimeArgSpec("out", (self.rows, self.cols)),        # y
        ]

    def get_callable(self):
        lib = _lib.load()
        method = _lib.IRON_ROPE_TWO_HALVES if self.method_type == 0 else _lib.IRON_ROPE_INTERLEAVED

        def call(*args):
            x, ang, y = check_args(self, args)
            _lib.check(lib.iron_rope(x.data_ptr(), ang.data_ptr(), y.data_ptr(), self.rows,
                                     self.cols, self.angle_rows, method, stream_ptr()), "RoPE")

        return call
