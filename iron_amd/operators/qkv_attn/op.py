"""QKVHeadAttention: the decode runlist's QKV head and decode attention as one operator.

The reference runs ``QKVHeadDataParallelOurs`` (writes the rotated q and appends k, v to the KV
cache; iron/operators/qkv_head_dp/op_ours.py:31-262) and then ``DecodeAttention`` over positions
``0..seq_pos`` (iron/operators/decode_attn/op.py:20-181) as two runlist entries
(iron/applications/qwen3_0.6b/qwen3_npu_int8.py:249-281). On gfx950 the per-head epilogue (QK
RMSNorm, RoPE, KV append) runs inside the attention kernel, so q never goes through memory and the
step is the QKV GEMV, the attention split kernel and the split merge.

Fields are those of ``QKVHeadDataParallel`` plus ``scale`` (softmax scale, default 1/sqrt(HD)) and
``accumulate`` (the attention core's arithmetic, "f64" exact or "f32" as DecodeAttention).
The spec is the QKV head's inputs and caches followed by the attention output:
``cur, n_in, Wqkv, n_qn, n_kn, ang, k_cache, v_cache, out`` (``kv_layout="separate"``) or
``cur, n_in, Wqkv, n_qn, n_kn, ang, kv_cache, out`` (merged token-interleaved cache). The context
of row b is ``pos[b] + 1`` where ``pos`` is the position carried by the KV offset parameter. The
result equals the two-operator composition bit for bit (same kernels' arithmetic and roundings,
for either accumulation mode).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, check_args
from .._common import RuntimeParams, Workspace, domain_code, stream_ptr
from ..qkv_head_dp.op import QKVHeadDataParallel


@dataclass
class QKVHeadAttention(QKVHeadDataParallel):
    scale: float | None = None
    accumulate: str = "f64"

    _name_aliases: ClassVar[Dict[str, str]] = {**QKVHeadDataParallel._name_aliases, "scale": "sc",
                                               "accumulate": "acc"}

    @property
    def softmax_scale(self) -> float:
        return self.scale if self.scale is not None else 1.0 / math.sqrt(self.HD)

    def get_arg_spec(self):
        spec = super().get_arg_spec()
        head, caches = spec[:6], spec[7:]          # drop the q output of the QKV head
        return head + caches + [AIERuntimeArgSpec("out", (self.batch * self.Hq * self.HD,))]

    def __post_init__(self):
        if self.angles_from_table:
            raise ValueError("QKVHeadAttention takes the position's angle row per batch row "
                             "(angles_from_table=False)")
        _lib.accum_mode(self.accumulate)
        super().__post_init__()

    def get_callable(self, params: RuntimeParams | None = None):
        lib = _lib.load()
        B = self.batch
        ws = Workspace(lib.iron_qkv_attn_workspace(B, self.D, self.Hq, self.Hkv, self.HD,
                                                   self.max_seq),
                       self.context.device)
        dom = domain_code(self.domain)
        acc = _lib.accum_mode(self.accumulate)
        voff, sb, sh, st = self.kv_strides()
        params = params if params is not None else RuntimeParams(self.context.device)
        pname = self.kv_offset_parameter or "kv_off"
        params.define(pname, B, convert=self.offset_to_position)

        def call(*args):
            args = check_args(self, args)
            cur, n_in, w, n_qn, n_kn, ang = args[:6]
            if self.kv_layout == "separate":
                kp, vp, out = args[6].data_ptr(), args[7].data_ptr(), args[8]
            else:
                kp = args[6].data_ptr()
                vp, out = kp + 2 * voff, args[7]
            _lib.check(lib.iron_qkv_attn(
                cur.data_ptr(), n_in.data_ptr(), w.data_ptr(), n_qn.data_ptr(), n_kn.data_ptr(),
                ang.data_ptr(), kp, vp, sb, sh, st,
                params.tensor(pname, B).data_ptr(), out.data_ptr(), B, self.D, self.HD, self.Hq,
                self.Hkv, self.max_seq, self.group_size, self.tile_size_input, dom,
                float(self.epsilon), float(self.softmax_scale), acc, ws.ptr, ws.nbytes,
                stream_ptr()),
                type(self).__name__)

        call.params = params
        call.workspace = ws
        return call
