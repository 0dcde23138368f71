"""QKVHeadDataParallelOurs: the chain's QKV head arm (merged token-interleaved KV cache).

Drop-in for iron/operators/qkv_head_dp/op_ours.py:31-262. In the reference this arm differs
from its parent only in the KV drain layout (one interleaved per-token cache); the parent here
already implements that layout (``kv_layout="interleaved"``) with the same spec, so the arm is a
named subclass. The M1/M2 probe arms (``with_attn``, ``attn_row3``, ``mlp_row4``) are NPU
placement experiments and are rejected loudly, as the reference rejects them for this design.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict

from .op import QKVHeadDataParallel


@dataclass
class QKVHeadDataParallelOurs(QKVHeadDataParallel):
    attn_colmajor: bool = field(default=False)
    with_attn: bool = field(default=False)
    attn_row3: bool = field(default=False)
    mlp_row4: bool = field(default=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **QKVHeadDataParallel._name_aliases,
        "attn_colmajor": "acm",
        "with_attn": "wa",
        "attn_row3": "ar3",
        "mlp_row4": "mr4",
    }

    def __post_init__(self):
        if self.with_attn or self.attn_row3 or self.mlp_row4 or self.attn_colmajor:
            raise ValueError("with_attn/attn_row3/mlp_row4/attn_colmajor are NPU placement arms "
                             "with no gfx950 counterpart")
        super().__post_init__()
