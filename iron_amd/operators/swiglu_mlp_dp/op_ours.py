"""SwiGLUMLPDataParallelOurs: the int8-weight fused decode MLP (optionally with fuse_o).

Drop-in for iron/operators/swiglu_mlp_dp/op_ours.py:46-582. Spec order as in the reference:

    fuse_o:  cur, cx, n_pf, Wo, Wg, Wu, Wd, gh_scratch, a_scratch, nxt
    else:    cur, a,  n_pf,     Wg, Wu, Wd, gh_scratch,            nxt

Wires are the row-block int8 wire (iron_amd/operators/wire.py); Wg/Wu use ``tile_rows_gu`` rows
per block and Wd ``tile_rows_gu // (FF // D)`` (the reference's shared-tile identity,
qwen3_npu_int8.py:525-530), or 4-row blocks for both when FF is not a multiple of D (the
reference's Qwen3-4B chunked-down arm, op_ours.py:91-117, without its zero padding of FF). Wo uses a plain ``tile_rows_o``-row wire instead of the reference's
NPU per-core overlap windows (op_ours.py:357-369) -- those duplicated pad rows only exist to
feed eight AIE columns. ``gh_scratch`` is the operator's device workspace (fp32 gh, which the
golden keeps unrounded) sized by ``iron_swiglu_mlp_workspace``; ``a_scratch`` receives
``a = bf16(Wo @ cx)`` under fuse_o. ``batch`` (new) runs up to 16 rows with one weight pass (1-4 on the fused GEMV kernels, 5-16
on the MFMA GEMMs).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import torch

from ... import _lib
from ...common.base import AIERuntimeArgSpec, check_args
from .._common import domain_code, stream_ptr
from ..wire import domain_of, wire_nbytes
from .op import SwiGLUMLPDataParallel


@dataclass
class SwiGLUMLPDataParallelOurs(SwiGLUMLPDataParallel):
    tile_rows_gu: int = field(default=12, repr=False)
    weight_depth: int = field(default=1, repr=False)
    weight_memtile: bool = field(default=False)
    weight_stage_depth: int = field(default=16)
    kernel_source: str | None = field(default=None, repr=False)
    acc_kernel_source: str | None = field(default=None, repr=False)
    tile_rows_o: int = 4
    batch: int = 1

    _name_aliases: ClassVar[Dict[str, str]] = {
        **SwiGLUMLPDataParallel._name_aliases,
        "weight_memtile": "wmm",
        "weight_stage_depth": "wsd",
        "tile_rows_o": "tro",
    }

    def __post_init__(self):
        self.weight_dtype = "int8"
        if not self.group_size:
            self.group_size = 128
        super().__post_init__()
        if self.FF % self.D:
            # The reference's chunked-down arm (Qwen3-4B: D=2560, FF=9728; op_ours.py:91-117)
            # pads FF with zero rows to a multiple of D only to give its eight AIE columns equal
            # work, and uses 4-row tiles for gate/up and down alike. The GEMV and MFMA kernels
            # here take any FF (a multiple of the group), so the wires keep FF rows: the same
            # products without the 5% of zero padding.
            self.tile_rows_gu = 4
            if self.FF % self.tile_rows_gu or self.D % self.tile_rows_gu:
                raise ValueError(f"FF={self.FF} and D={self.D} must be multiples of 4")
        else:
            R = self.FF // self.D
            if self.tile_rows_gu % R:
                raise ValueError(f"tile_rows_gu={self.tile_rows_gu} must be a multiple of "
                                 f"FF/D={R}")
        for what, K in (("D", self.D), ("FF", self.FF)) + ((("QD", self.QD),) if self.fuse_o else ()):
            if K % self.group_size:
                raise ValueError(f"{what}={K} not a multiple of group_size={self.group_size}")
        if not 1 <= self.batch <= 16:
            raise ValueError("batch must be in [1, 16]")
        self.ff_pad = self.FF

    @property
    def domain(self) -> str:
        return domain_of(self.kernel_source)

    @property
    def tile_rows_d(self) -> int:
        """Row-block height of the Wd wire: tile_rows_gu / (FF/D) (the reference's shared-tile
        identity, qwen3_npu_int8.py:525-530), or tile_rows_gu itself when FF % D != 0 (its
        chunked-down arm sets TSI_D == TSI_GU, op_ours.py:110-117)."""
        if self.FF % self.D:
            return self.tile_rows_gu
        return self.tile_rows_gu // (self.FF // self.D)

    def wire_bytes(self, which: str) -> int:
        G = self.group_size
        if which in ("Wg", "Wu"):
            return wire_nbytes(self.FF, self.D, G, self.tile_rows_gu)
        if which == "Wd":
            return wire_nbytes(self.D, self.FF, G, self.tile_rows_d)
        if which == "Wo":
            return wire_nbytes(self.D, self.QD, G, self.tile_rows_o)
        raise KeyError(which)

    def workspace_bytes(self) -> int:
        return int(_lib.load().iron_swiglu_mlp_workspace(self.batch, self.D, self.FF))

    def get_arg_spec(self):
        B, D = self.batch, self.D
        u8 = torch.uint8
        w = lambda n: AIERuntimeArgSpec("in", (self.wire_bytes(n) // 2,))  # noqa: E731
        ws = AIERuntimeArgSpec("inout", (self.workspace_bytes(),), dtype=u8)
        if self.fuse_o:
            return [
                AIERuntimeArgSpec("in", (B * D,)),            # cur
                AIERuntimeArgSpec("in", (B * self.QD,)),      # cx (attention context)
                AIERuntimeArgSpec("in", (D,)),                # n_pf
                w("Wo"), w("Wg"), w("Wu"), w("Wd"),
                ws,                                           # gh_scratch (workspace)
                AIERuntimeArgSpec("inout", (B * D,)),         # a_scratch (receives a)
                AIERuntimeArgSpec("out", (B * D,)),           # nxt
            ]
        return [
            AIERuntimeArgSpec("in", (B * D,)),                # cur
            AIERuntimeArgSpec("in", (B * D,)),                # a
            AIERuntimeArgSpec("in", (D,)),                    # n_pf
            w("Wg"), w("Wu"), w("Wd"),
            ws,                                               # gh_scratch (workspace)
            AIERuntimeArgSpec("out", (B * D,)),               # nxt
        ]

    def get_callable(self):
        lib = _lib.load()
        dom = domain_code(self.domain)
        G, B = self.group_size, self.batch

        def call(*args):
            args = check_args(self, args)
            if self.fuse_o:
                cur, cx, n_pf, wo, wg, wu, wd, ws, a_s, nxt = args
                wo_p, a_p, QD = wo.data_ptr(), a_s.data_ptr(), self.QD
            else:
                cur, cx, n_pf, wg, wu, wd, ws, nxt = args
                wo_p, a_p, QD = None, None, 0
            _lib.check(lib.iron_swiglu_mlp(
                cur.data_ptr(), cx.data_ptr(), n_pf.data_ptr(), wo_p, wg.data_ptr(),
                wu.data_ptr(), wd.data_ptr(), nxt.data_ptr(), a_p, B, self.D, self.FF, QD, G,
                self.tile_rows_o, self.tile_rows_gu, self.tile_rows_d, dom, float(self.epsilon),
                ws.data_ptr(), ws.numel() * ws.element_size(), stream_ptr()),
                "SwiGLUMLPDataParallelOurs")

        return call
