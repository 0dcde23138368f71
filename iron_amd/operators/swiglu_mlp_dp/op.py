"""SwiGLUMLPDataParallel: fused decode SwiGLU MLP block on gfx950.

Drop-in for iron/operators/swiglu_mlp_dp/op.py:22-227 (fields, validation, spec order):

    x1  = cur + a                      (or a = bf16(Wo @ cx) first, with ``fuse_o``)
    hf  = RMSNorm_weighted(x1, n_pf)
    nxt = x1 + Wd @ (silu(Wg @ hf) * (Wu @ hf))

The parent class carries the reference's bf16-weight arm, which is not on the int8 hot path and
is not implemented here (construction raises); the int8 arm is ``SwiGLUMLPDataParallelOurs``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ...common.base import MLIROperator


@dataclass
class SwiGLUMLPDataParallel(MLIROperator):
    D: int
    FF: int
    num_aie_columns: int = 8
    num_aie_rows: int = 1
    epsilon: float = 1e-5
    QD: int = None
    fuse_o: bool = False
    weight_dtype: str = field(default="bf16", repr=False)
    group_size: int = field(default=0, repr=False)
    weight_depth: int = field(default=2, repr=False)
    tile_rows_gu: int = field(default=0, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "epsilon": "eps",
        "num_aie_columns": "cols",
        "num_aie_rows": "rows",
        "fuse_o": "fo",
        "weight_dtype": "wdt",
        "group_size": "g",
        "weight_depth": "wd",
        "tile_rows_gu": "tr",
    }

    def __post_init__(self):
        if self.D <= 0 or self.FF <= 0:
            raise ValueError(f"D ({self.D}) and FF ({self.FF}) must be positive")
        if self.fuse_o and (not self.QD or self.QD <= 0):
            raise ValueError("fuse_o requires QD (the attention context width)")
        if type(self) is SwiGLUMLPDataParallel:
            raise NotImplementedError(
                "the bf16-weight MLP arm is not on the int8 decode path; use "
                "SwiGLUMLPDataParallelOurs")
        MLIROperator.__init__(self, context=self.context)

    def get_arg_spec(self):  # pragma: no cover - the bf16 arm is never constructed
        raise NotImplementedError

    def get_callable(self):  # pragma: no cover
        raise NotImplementedError
