"""QKVHeadDataParallel: fused decode QKV head on gfx950.

Drop-in for iron/operators/qkv_head_dp/op.py:20-231: weighted RMSNorm(cur) -> concatenated
``[Hq*HD | Hkv*HD | Hkv*HD] x D`` int8 QKV GEMV -> per-head QK RMSNorm -> two-halves RoPE of q
and k -> k, v appended to the cache at the runtime offset. The spec keeps the reference order
``cur, n_in, Wqkv, n_qn, n_kn, ang, q, kv_cache`` (one merged, head-major, token-interleaved
cache: head h owns ``[h*2*S*HD, +2*S*HD)``, token t's K at ``t*2*HD`` and V at ``t*2*HD + HD``).
The runtime parameter named by ``kv_offset_parameter`` carries the reference's element offset
(``seq_pos * 2 * HD``; qwen3_npu_int8.py:598-609); it is converted to a position on write.

New fields: ``group_size`` (wire group, default 128 as in the reference), ``kv_layout``
(``"interleaved"`` as above, or ``"separate"`` for two ``[Hkv, S, HD]`` caches -- spec
``..., q, k_cache, v_cache``; offsets are then ``seq_pos * HD``), ``batch`` (rows per call; every
row has its own angle row and its own position entry), ``angles_from_table`` (the ``ang`` argument
is then a whole ``(max_seq, HD)`` angle table indexed on the device by each row's position, so a
captured per-token graph needs no host write of the angle row) and ``kernel_source`` selects the
payload domain as in the reference. NPU placement knobs are accepted and ignored.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

import numpy as np

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import RuntimeParams, Workspace, domain_code, stream_ptr
from ..wire import domain_of, wire_nbytes


@dataclass
class QKVHeadDataParallel(MLIROperator):
    D: int
    HD: int
    Hq: int
    Hkv: int
    max_seq: int
    num_aie_columns: int = 8
    epsilon: float = 1e-6
    tile_size_input: int = 4
    stack_size: int = 0xD00
    kv_offset_parameter: str | None = "kv_off"
    group_size: int = 128
    kv_layout: str = "interleaved"
    batch: int = 1
    angles_from_table: bool = False
    weight_depth: int = field(default=2, repr=False)
    misc_chunked: bool = field(default=True, repr=False)
    misc_obj_elems: int | None = field(default=None, repr=False)
    runtime_tile_loop: bool = field(default=False, repr=False)
    kernel_source: str | None = field(default=None, repr=False)
    merge_drains: bool = field(default=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "num_aie_columns": "col",
        "epsilon": "eps",
        "tile_size_input": "tsi",
        "stack_size": "ss",
        "max_seq": "S",
        "kv_offset_parameter": "kvpar",
        "group_size": "g",
        "kv_layout": "kvl",
        "merge_drains": "md",
        "angles_from_table": "aft",
    }

    def __post_init__(self):
        heads = self.Hq + 2 * self.Hkv
        if heads % self.num_aie_columns:
            raise ValueError(
                f"Hq + 2*Hkv ({heads}) must be divisible by num_aie_columns "
                f"({self.num_aie_columns}) -- every core owns a whole number of heads")
        if self.HD % self.tile_size_input:
            raise ValueError(f"head_dim ({self.HD}) must be divisible by tile_size_input "
                             f"({self.tile_size_input})")
        if self.D % self.HD:
            raise ValueError(f"d_model ({self.D}) must be a whole number of head_dim "
                             f"({self.HD}) chunks")
        if self.HD != 128:
            raise NotImplementedError("head_dim 128 only")
        if self.kv_layout not in ("interleaved", "separate"):
            raise ValueError(f"unknown kv_layout {self.kv_layout!r}")
        if self.D % self.group_size:
            raise ValueError(f"D={self.D} not a multiple of group_size={self.group_size}")
        MLIROperator.__init__(self, context=self.context)

    @property
    def M(self) -> int:
        return (self.Hq + 2 * self.Hkv) * self.HD

    @property
    def domain(self) -> str:
        return domain_of(self.kernel_source)

    @property
    def wire_bytes(self) -> int:
        return wire_nbytes(self.M, self.D, self.group_size, self.tile_size_input)

    def kv_strides(self) -> tuple[int, int, int, int]:
        """(v_offset, batch stride, head stride, token stride) in elements, per cache arg."""
        S, HD, KV = self.max_seq, self.HD, self.Hkv
        if self.kv_layout == "separate":
            return 0, KV * S * HD, S * HD, HD
        return HD, KV * 2 * S * HD, 2 * S * HD, 2 * HD

    def offset_to_position(self, off) -> np.ndarray:
        per_token = self.HD if self.kv_layout == "separate" else 2 * self.HD
        return np.atleast_1d(np.asarray(off, dtype=np.int64)) // per_token

    def get_arg_spec(self):
        B, QD, KVD, S = self.batch, self.Hq * self.HD, self.Hkv * self.HD, self.max_seq
        head = [
            AIERuntimeArgSpec("in", (B * self.D,)),                 # cur
            AIERuntimeArgSpec("in", (self.D,)),                     # n_in
            AIERuntimeArgSpec("in", (self.wire_bytes // 2,)),       # Wqkv int8 wire (bf16 view)
            AIERuntimeArgSpec("in", (self.HD,)),                    # n_qn
            AIERuntimeArgSpec("in", (self.HD,)),                    # n_kn
            AIERuntimeArgSpec("in", ((self.max_seq if self.angles_from_table else B)
                                     * self.HD,)),                  # ang rows (or table)
            AIERuntimeArgSpec("out", (B * QD,)),                    # q
        ]
        if self.kv_layout == "separate":
            return head + [AIERuntimeArgSpec("inout", (B * KVD * S,)),   # k cache
                           AIERuntimeArgSpec("inout", (B * KVD * S,))]   # v cache
        return head + [AIERuntimeArgSpec("inout", (B * 2 * KVD * S,))]  # merged kv cache

    def get_callable(self, params: RuntimeParams | None = None):
        """``params``: a shared runtime-parameter store (the sequence's); one is created if None.

        The KV offset parameter is declared with a converter, so writes keep the reference's
        element-offset semantics while the kernel reads positions."""
        lib = _lib.load()
        B = self.batch
        ws = Workspace(lib.iron_qkv_head_workspace(B, self.D, self.Hq, self.Hkv, self.HD),
                       self.context.device)
        dom = domain_code(self.domain)
        voff, sb, sh, st = self.kv_strides()
        params = params if params is not None else RuntimeParams(self.context.device)
        pname = self.kv_offset_parameter or "kv_off"
        params.define(pname, B, convert=self.offset_to_position)

        def call(*args):
            args = check_args(self, args)
            cur, n_in, w, n_qn, n_kn, ang, q = args[:7]
            if self.kv_layout == "separate":
                kp, vp = args[7].data_ptr(), args[8].data_ptr()
            else:
                kp = args[7].data_ptr()
                vp = kp + 2 * voff
            _lib.check(lib.iron_qkv_head(
                cur.data_ptr(), n_in.data_ptr(), w.data_ptr(), n_qn.data_ptr(), n_kn.data_ptr(),
                ang.data_ptr(), int(self.angles_from_table), q.data_ptr(), kp, vp, sb, sh, st,
                params.tensor(pname, B).data_ptr(), B, self.D, self.HD, self.Hq, self.Hkv,
                self.max_seq, self.group_size, self.tile_size_input, dom, float(self.epsilon),
                ws.ptr, ws.nbytes, stream_ptr()), type(self).__name__)

        call.params = params
        call.workspace = ws
        return call
