"""Whole-model Qwen3 decode on the CPU (test infrastructure and the timed CPU baseline).

Composes the per-operator goldens exactly as the reference's CPU sequence mode does
(``SequenceReferenceCallable``, iron/common/sequence.py:972-999): every operator output is
rounded to bf16 at its boundary. Per layer the chain is the one Qwen3NPU builds
(iron/applications/qwen3_0.6b/qwen3_npu_int8.py:249-281): fused QKV head (with the K/V append
at ``seq_pos``), decode attention over ``seq_pos + 1`` keys, fused MLP with the output
projection folded in (fuse_o); then the final RMSNorm, the LM head and a host argmax
(qwen3_npu_int8.py:612-621; first maximal index on ties, as numpy/torch argmax).

``dt`` selects EXACT (fp64, the parity oracle) or LITERAL (fp32, the reference goldens as
written -- the timed CPU baseline); both round at the same boundaries. Weights arrive as plain
tensors (see ``Qwen3CpuChain``) and linear weights are dequantized once, outside any timed
region, as the reference's CPU goldens do (swiglu_mlp_dp/op_ours.py:543-582).
"""

from __future__ import annotations

import torch

from .attention import decode_attention
from .blocks import qkv_head, swiglu_mlp
from .gemv import dequant_f, gemv
from .norms import rms_norm, rope_angle_table
from .numerics import EXACT


def _to_cpu(t):
    """Everything the chain computes with is a CPU tensor (it is the CPU path by definition)."""
    return tuple(x.cpu() for x in t) if isinstance(t, tuple) else t.cpu()


class Qwen3CpuChain:
    """B=1 decode chain. ``weights`` layout:

    ``{"embed": (V,D) bf16, "final_norm": (D,) bf16, "lm_head": (V,D) bf16 or (q, s),
       "layers": [{"input_norm", "post_norm": (D,) bf16, "q_norm", "k_norm": (HD,) bf16,
                   "qkv", "o", "gate", "up", "down": (q int8 (M,K), s bf16 (M,K/G))}, ...]}``
    """

    def __init__(self, cfg, weights: dict, max_seq: int, kv_init=None, dt=EXACT):
        self.cfg = cfg
        self.max_seq = max_seq
        self.dt = dt
        cpu = _to_cpu
        self.embed = cpu(weights["embed"])
        self.final_norm = cpu(weights["final_norm"])
        lm = cpu(weights["lm_head"])
        self.lm = dequant_f(*lm, dt) if isinstance(lm, tuple) else lm.to(dt)
        self.layers = []
        for L in weights["layers"]:
            L = {k: cpu(v) for k, v in L.items()}
            self.layers.append({
                "input_norm": L["input_norm"], "post_norm": L["post_norm"],
                "q_norm": L["q_norm"], "k_norm": L["k_norm"],
                "qkv": dequant_f(*L["qkv"], dt),
                "Wf": {"o": dequant_f(*L["o"], dt), "g": dequant_f(*L["gate"], dt),
                       "u": dequant_f(*L["up"], dt), "d": dequant_f(*L["down"], dt)},
            })
        n, Hkv, HD = cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
        self.k_cache = torch.zeros(n, Hkv, max_seq, HD, dtype=torch.bfloat16)
        self.v_cache = torch.zeros(n, Hkv, max_seq, HD, dtype=torch.bfloat16)
        if kv_init is not None:
            k0, v0 = (t.cpu() for t in kv_init)              # (n, Hkv, P, HD) each
            P = k0.shape[2]
            self.k_cache[:, :, :P] = k0
            self.v_cache[:, :, :P] = v0
        self.table = rope_angle_table(max_seq, HD, cfg.rope_theta)

    def step_x(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """One decode step from a bf16 hidden state x (D,); returns bf16 logits (V,)."""
        cfg, dt = self.cfg, self.dt
        Hq, Hkv, HD, eps = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.eps
        x = x.reshape(1, -1).to(torch.bfloat16)
        ang = self.table[pos]
        for i, L in enumerate(self.layers):
            q, k, v = qkv_head(x, L["input_norm"], None, None, L["q_norm"], L["k_norm"], ang,
                               Hq, Hkv, HD, eps, W=L["qkv"], dt=dt)
            self.k_cache[i, :, pos] = k.reshape(Hkv, HD)
            self.v_cache[i, :, pos] = v.reshape(Hkv, HD)
            o = decode_attention(q.reshape(1, Hq, HD), self.k_cache[i:i + 1],
                                 self.v_cache[i:i + 1], pos + 1, dt=dt)
            x, _ = swiglu_mlp(x, o.reshape(1, -1), L["post_norm"], None, None, None, eps,
                              Wf=L["Wf"], dt=dt)
        xf = rms_norm(x, self.final_norm, eps, dt=dt)
        return gemv(self.lm, xf, dt).float().to(torch.bfloat16).reshape(-1)

    def step(self, token: int, pos: int) -> torch.Tensor:
        return self.step_x(self.embed[int(token)], pos)

    @staticmethod
    def argmax(logits: torch.Tensor) -> int:
        return int(torch.argmax(logits.float()).item())
