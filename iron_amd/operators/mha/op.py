"""MHA: causal prefill multi-head attention (GQA) on MFMA.

Drop-in for iron/operators/mha/op.py:20-153: the same fields (``num_heads``, ``seq_len``, ``d``,
``num_KV_heads`` with 0 meaning plain MHA, ``num_of_pipelines``) and the same spec, Q and O as
``(heads, S_pad, d)`` and K, V as ``(kv_heads, S_pad, d)`` flattened, with S padded to a multiple
of 64 exactly as the reference pads (``_calculate_seq_padding``). The golden is causal SDPA with
scale 1/sqrt(d) (mha/reference.py:73-81). The reference kernel is limited to d = 64; this one
takes d = 64 or 128 (the Qwen3 head size). ``num_of_pipelines`` only affects the padding, as in
the reference.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import stream_ptr


@dataclass
class MHA(MLIROperator):
    num_heads: int
    seq_len: int
    d: int
    num_KV_heads: int
    num_of_pipelines: int = field(default=1, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "num_heads": "h",
        "num_KV_heads": "kv",
        "seq_len": "s",
    }

    def __post_init__(self):
        self.B_q = 64
        self.B_kv = 64
        if self.d not in (64, 128):
            raise ValueError(f"d must be 64 or 128, got d={self.d}")
        kv = self.kv_heads
        if self.num_heads % kv:
            raise ValueError("num_heads must be a multiple of num_KV_heads")
        MLIROperator.__init__(self, context=self.context)

    @property
    def kv_heads(self) -> int:
        return self.num_KV_heads if self.num_KV_heads else self.num_heads

    @property
    def seq_padded(self) -> int:
        n = self.num_of_pipelines
        return ((self.seq_len + 63 * n) // (64 * n)) * (64 * n)

    def get_arg_spec(self):
        S = self.seq_padded
        q_size = self.num_heads * self.d * S
        kv_size = self.kv_heads * self.d * S
        return [
            AIERuntimeArgSpec("in", (q_size,)),   # Q
            AIERuntimeArgSpec("in", (kv_size,)),  # K
            AIERuntimeArgSpec("in", (kv_size,)),  # V
            AIERuntimeArgSpec("out", (q_size,)),  # O
        ]

    def get_callable(self):
        lib = _lib.load()
        H, KV, D, S = self.num_heads, self.kv_heads, self.d, self.seq_padded
        scale = 1.0 / math.sqrt(D)

        def call(*args):
            q, k, v, o = check_args(self, args)
            _lib.check(lib.iron_prefill_attn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                             1, H, KV, S, D, float(scale), stream_ptr()), "MHA")

        return call
