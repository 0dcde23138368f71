"""QKNormRoPE: fused decode QK RMSNorm + RoPE + V copy on gfx950.

Drop-in for iron/operators/qk_norm_rope/op.py:20-117: the fields, ``kv_cache_elems`` and the
spec ``[qkv_in (qkv_dim,), qkv_out (qkv_dim,), scratch (n_qk_heads*head_dim + 2*head_dim,)]``
plus, with ``kv_direct``, the layer's whole KV cache (``inout``). qkv is [Q | K | V] heads of
``head_dim``; scratch is [gamma (one row per Q/K head) | cos (head_dim) | sin (head_dim)]. Each
Q/K head is RMS-normalised with its gamma row, rounded to bf16 and rotated (rotate_half with the
two head_dim-long tables), then rounded again; V is copied (kernel qk_norm_rope.cc:42-108).
With ``kv_direct`` the rotated K heads and the V heads are also written to the head-major
``[n_v_heads][max_seq_len][K_t | V_t]`` cache at the element offset in the runtime parameter
``kv_offset_parameter`` (``t * 2 * head_dim``, design.py:50-85); an offset outside the cache
writes nothing there. The K heads are the last ``n_v_heads`` of the ``n_qk_heads``
(qk_norm_rope_kv.cc:36-37, 66).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import RuntimeParams, stream_ptr


@dataclass
class QKNormRoPE(MLIROperator):
    qkv_dim: int
    head_dim: int
    n_qk_heads: int
    n_v_heads: int
    epsilon: float = 1e-6
    num_aie_columns: int = 1
    kv_direct: bool = False
    max_seq_len: int = 512
    kv_offset_parameter: str = field(default="k_cache_offset", repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **MLIROperator._name_aliases,
        "num_aie_columns": "col",
        "epsilon": "eps",
        "kv_direct": "kvdir",
        "max_seq_len": "seq",
    }

    def __post_init__(self):
        if self.qkv_dim != (self.n_qk_heads + self.n_v_heads) * self.head_dim:
            raise ValueError(
                f"QKNormRoPE: qkv_dim={self.qkv_dim} is not (n_qk_heads + n_v_heads) * head_dim "
                f"= {(self.n_qk_heads + self.n_v_heads) * self.head_dim}")
        if self.n_v_heads > self.n_qk_heads:
            raise ValueError("QKNormRoPE: the K heads (the last n_v_heads of the n_qk_heads) "
                             f"need n_v_heads <= n_qk_heads, got {self.n_v_heads} > "
                             f"{self.n_qk_heads}")
        if self.kv_direct and self.max_seq_len <= 0:
            raise ValueError("QKNormRoPE: kv_direct needs the cache's max_seq_len")
        MLIROperator.__init__(self, context=self.context)

    @property
    def kv_cache_elems(self) -> int:
        """Elements of one layer's KV cache: head-major, per token [K_t | V_t]."""
        return self.n_v_heads * 2 * self.max_seq_len * self.head_dim

    @property
    def scratch_elems(self) -> int:
        return self.n_qk_heads * self.head_dim + 2 * self.head_dim

    def get_arg_spec(self):
        spec = [
            AIERuntimeArgSpec("in", (self.qkv_dim,)),          # qkv_in
            AIERuntimeArgSpec("out", (self.qkv_dim,)),         # qkv_out
            AIERuntimeArgSpec("in", (self.scratch_elems,)),    # gamma | cos | sin
        ]
        if self.kv_direct:
            spec.append(AIERuntimeArgSpec("inout", (self.kv_cache_elems,)))
        return spec

    def get_callable(self, params: RuntimeParams | None = None):
        """``params``: a shared runtime-parameter store; one is created if None. With
        ``kv_direct``, write the element offset ``t * 2 * head_dim`` of the current token to
        ``params`` under ``kv_offset_parameter`` before the call."""
        lib = _lib.load()
        params = params if params is not None else RuntimeParams(self.context.device)
        if self.kv_direct:
            params.define(self.kv_offset_parameter, 1)

        def call(*args):
            args = check_args(self, args)
            qkv_in, qkv_out, scratch = args[:3]
            kv = args[3].data_ptr() if self.kv_direct else None
            off = params.tensor(self.kv_offset_parameter, 1).data_ptr() if self.kv_direct \
                else None
            _lib.check(lib.iron_qk_norm_rope(
                qkv_in.data_ptr(), scratch.data_ptr(), qkv_out.data_ptr(), kv, off,
                self.head_dim, self.n_qk_heads, self.n_v_heads,
                self.max_seq_len if self.kv_direct else 0, float(self.epsilon), stream_ptr()),
                type(self).__name__)

        call.params = params
        return call
