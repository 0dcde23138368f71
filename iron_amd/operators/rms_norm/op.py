"""RMSNorm: row-wise (optionally weighted) RMS normalisation on gfx950.

Drop-in for iron/operators/rms_norm/op.py:21-130 (fields, the divisibility check, and the
``[x (rows, tile), w (tile,), y (rows, tile)]`` spec). Semantics follow the kernel
(aie_kernels/aie2p/rms_norm.cc:83-147): fp32 mean of squares over each ``tile_size`` row,
``x * rsqrt(mean + eps) * w`` in fp32, one bf16 rounding.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import stream_ptr


@dataclass
class RMSNorm(MLIROperator):
    size: int
    num_aie_columns: int
    num_channels: int
    tile_size: int
    weighted: bool = False
    epsilon: float = 1e-5
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "weighted": "w",
        "epsilon": "eps",
    }

    def __post_init__(self):
        max_multiple = self.num_aie_columns * self.num_channels * self.tile_size
        if self.size % max_multiple != 0:
            raise ValueError(
                f"size ({self.size}) must be a multiple of "
                f"num_aie_columns * num_channels * tile_size ({max_multiple})"
            )
        MLIROperator.__init__(self, context=self.context)

    def get_arg_spec(self):
        specs = [AIERuntimeArgSpec("in", (self.size // self.tile_size, self.tile_size))]
        if self.weighted:
            specs.append(AIERuntimeArgSpec("in", (self.tile_size,)))
        specs.append(AIERuntimeArgSpec("out", (self.size // self.tile_size, self.tile_size)))
        return specs

    def get_callable(self):
        lib = _lib.load()
        rows, cols = self.size // self.tile_size, self.tile_size

        def call(*args):
            args = check_args(self, args)
            x, y = args[0], args[-1]
            w = args[1] if self.weighted else None
            _lib.check(lib.iron_rmsnorm(x.data_ptr(), _lib.ptr(w), y.data_ptr(), rows, cols,
                                        float(self.epsilon), stream_ptr()), "RMSNorm")

        return call
