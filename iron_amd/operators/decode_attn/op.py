"""DecodeAttention: single-query GQA attention over a bf16 KV cache on gfx950.

Drop-in for iron/operators/decode_attn/op.py:20-181: same fields and validation, the same arg
specs for both KV layouts, and the runtime causal bound ``S_kv_eff`` (the number of valid cached
tokens, written per dispatch) when ``use_runtime_seq_len`` is set; the static arm uses every
cached position, as the reference's does.

KV layouts (all head-major, addressed by strides in one kernel):
  * ``kv_layout="separate"``: K and V args of (KV, S*D) each -- the reference's separate arm and
    BASELINE's contiguous ``[B, KV, L, D]`` caches.
  * ``kv_layout="combined"``, ``kv_token_interleaved=True``: one (KV, 2*S*D) arg with token t's K
    at 2*t*D and V at 2*t*D + D (the shipped chain's layout).
  * ``kv_layout="combined"``, ``kv_token_interleaved=False``: one (KV, 2*S*D) arg with a K half
    then a V half per head -- the layout of the reference golden (decode_attn/reference.py:41-60).
New fields: ``batch`` (sequences per call; Q/O become (batch*H, D), K/V (batch*KV, ...), and
``S_kv_eff`` holds one count per sequence, so ragged batches are one call), ``scale``
(default 1/sqrt(D)) and ``accumulate``: "f64" evaluates the golden exactly (fp64, one rounding to
bf16), "f32" uses the reference kernel's own arithmetic (fp32 dot products, exp2 softmax and
accumulation; decode_attn.cc:117-311).

Batch / verify mode (``batch_queries`` > 0, the reference's speculative-decode verify path,
op.py:40-48 and design.py:243-276): ``num_new_tokens`` new tokens at positions
``S_kv_base .. S_kv_base + num_new_tokens - 1`` query one cache; Q and O are
``(num_new_tokens * H, D)`` token-major (O may be taller, ``out_buffer_tokens``; only the
new tokens' rows are written); the runtime parameter is ``S_kv_base`` (the cached-token count
before the new block). Token t attends keys ``[0, S_kv_base + t]`` when ``causal``, the whole
cache otherwise. The kernel (``iron_decode_attn_verify``) stages every 64-key K/V block once for
up to 64 query rows; ``batch_queries`` (the reference's group size M) is validated and recorded,
the grouping not changing the result. Its arithmetic is the reference kernel's fp32 form.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common.base import AIERuntimeArgSpec, MLIROperator, check_args
from .._common import RuntimeParams, Workspace, stream_ptr


@dataclass
class DecodeAttention(MLIROperator):
    num_heads: int
    num_kv_heads: int
    head_dim: int
    seq_len_kv: int
    num_aie_columns: int = 8
    block_kv: int = 64
    use_runtime_seq_len: bool = field(default=False, repr=False)
    batch_queries: int = 0
    num_new_tokens: int = 0
    causal: bool = True
    kv_token_interleaved: bool = True
    out_buffer_tokens: int = 0
    kv_layout: str = "combined"
    batch: int = 1
    scale: float | None = None
    accumulate: str = "f64"
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        "num_heads": "h",
        "num_kv_heads": "kv",
        "head_dim": "d",
        "seq_len_kv": "skv",
        "num_aie_columns": "col",
        "block_kv": "bkv",
        "batch_queries": "m",
        "num_new_tokens": "new",
        "kv_layout": "kvl",
    }

    def __post_init__(self):
        if self.seq_len_kv % 64 != 0:
            raise ValueError("seq_len_kv must be a multiple of 64")
        if self.block_kv % 16 != 0:
            raise ValueError("block_kv must be a multiple of 16")
        if self.batch_queries > 0:
            if self.num_new_tokens <= 0 or self.num_new_tokens % self.batch_queries:
                raise ValueError(f"num_new_tokens ({self.num_new_tokens}) must be a positive "
                                 f"multiple of batch_queries ({self.batch_queries})")
            if not self.use_runtime_seq_len:
                raise ValueError("the batch (verify) mode reads S_kv_base: it needs "
                                 "use_runtime_seq_len")
            if self.batch != 1:
                raise ValueError("the batch (verify) mode queries one cache (batch=1)")
        if self.kv_layout not in ("combined", "separate"):
            raise ValueError(f"unknown kv_layout {self.kv_layout!r}")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if self.batch < 1:
            raise ValueError("batch must be >= 1")
        _lib.accum_mode(self.accumulate)
        MLIROperator.__init__(self, context=self.context)

    @property
    def softmax_scale(self) -> float:
        return self.scale if self.scale is not None else 1.0 / math.sqrt(self.head_dim)

    def kv_strides(self) -> tuple[int, int, int, int]:
        """(v_offset, batch stride, head stride, token stride) in elements."""
        S, D, KV = self.seq_len_kv, self.head_dim, self.num_kv_heads
        if self.kv_layout == "separate":
            return 0, KV * S * D, S * D, D
        if self.kv_token_interleaved:
            return D, KV * 2 * S * D, 2 * S * D, 2 * D
        return S * D, KV * 2 * S * D, 2 * S * D, D

    @property
    def verify(self) -> bool:
        return self.batch_queries > 0

    def get_arg_spec(self):
        H, KV, D, S, B = self.num_heads, self.num_kv_heads, self.head_dim, self.seq_len_kv, self.batch
        q_rows = self.num_new_tokens * H if self.verify else B * H
        o_rows = (max(self.out_buffer_tokens, self.num_new_tokens) * H if self.verify
                  else B * H)
        if self.kv_layout == "separate":
            return [
                AIERuntimeArgSpec("in", (q_rows, D)),        # Q
                AIERuntimeArgSpec("in", (B * KV, S * D)),    # K cache (head-major)
                AIERuntimeArgSpec("in", (B * KV, S * D)),    # V cache (head-major)
                AIERuntimeArgSpec("out", (o_rows, D)),       # O
            ]
        return [
            AIERuntimeArgSpec("in", (q_rows, D)),            # Q
            AIERuntimeArgSpec("in", (B * KV, 2 * S * D)),    # KV combined
            AIERuntimeArgSpec("out", (o_rows, D)),           # O
        ]

    def get_callable(self, params: RuntimeParams | None = None):
        """``params``: a shared runtime-parameter store holding ``S_kv_eff`` (one is created if
        None and ``use_runtime_seq_len`` is set)."""
        lib = _lib.load()
        H, KV, D, S, B = self.num_heads, self.num_kv_heads, self.head_dim, self.seq_len_kv, self.batch
        if self.verify:
            return self._verify_callable(lib, params)
        ws = Workspace(lib.iron_decode_attn_workspace(B, H, KV, D, S), self.context.device)
        voff, sb, sh, st = self.kv_strides()
        acc = _lib.accum_mode(self.accumulate)
        params = params if params is not None else RuntimeParams(self.context.device)
        if self.use_runtime_seq_len and "S_kv_eff" not in params:
            params.define("S_kv_eff", B)
            params.write("S_kv_eff", [S] * B)

        def call(*args):
            args = check_args(self, args)
            if self.kv_layout == "separate":
                q, k, v, o = args
                kp, vp = k.data_ptr(), v.data_ptr()
            else:
                q, kv, o = args
                kp, vp = kv.data_ptr(), kv.data_ptr() + 2 * voff
            ctx = params.tensor("S_kv_eff", B) if self.use_runtime_seq_len else None
            _lib.check(lib.iron_decode_attn(
                q.data_ptr(), kp, vp, sb, sh, st, _lib.ptr(ctx), S, o.data_ptr(), B, H, KV, D, S,
                float(self.softmax_scale), acc, ws.ptr, ws.nbytes, stream_ptr()), "DecodeAttention")

        call.params = params
        call.workspace = ws
        return call

    def _verify_callable(self, lib, params):
        H, KV, D, S, n = (self.num_heads, self.num_kv_heads, self.head_dim, self.seq_len_kv,
                          self.num_new_tokens)
        ws = Workspace(lib.iron_decode_attn_verify_workspace(n, H, KV, D, S), self.context.device)
        voff, _, sh, st = self.kv_strides()
        params = params if params is not None else RuntimeParams(self.context.device)
        if "S_kv_base" not in params:
            params.define("S_kv_base", 1)

        def call(*args):
            args = check_args(self, args)
            if self.kv_layout == "separate":
                q, k, v, o = args
                kp, vp = k.data_ptr(), v.data_ptr()
            else:
                q, kv, o = args
                kp, vp = kv.data_ptr(), kv.data_ptr() + 2 * voff
            _lib.check(lib.iron_decode_attn_verify(
                q.data_ptr(), kp, vp, sh, st, params.tensor("S_kv_base", 1).data_ptr(), 0,
                int(bool(self.causal)), o.data_ptr(), n, H, KV, D, S,
                float(self.softmax_scale), ws.ptr, ws.nbytes, stream_ptr()), "DecodeAttention")

        call.params = params
        call.workspace = ws
        return call
