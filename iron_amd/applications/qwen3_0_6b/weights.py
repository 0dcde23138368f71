"""Qwen3 model configurations, seeded random-init weights, and the GPTQ checkpoint loader.

Weights travel between the runtime and its checkers as plain tensors in one neutral layout:

    {"embed": (V, D) bf16, "final_norm": (D,) bf16, "lm_head": (V, D) bf16 or (q, s),
     "layers": [{"input_norm", "post_norm": (D,) bf16, "q_norm", "k_norm": (HD,) bf16,
                 "qkv", "o", "gate", "up", "down": (q int8 (M, K), s bf16 (M, K/G))}, ...]}

``qkv`` is the row concatenation [q_proj; k_proj; v_proj] the fused QKV head consumes
(qwen3_npu_int8.py:499-512).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch

from ...operators.wire import gptq_unpack, rtn_quantize


@dataclass(frozen=True)
class Qwen3Config:
    emb_dim: int = 1024          # D
    hidden_dim: int = 3072       # FF
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    n_layers: int = 28
    rope_theta: float = 1e6
    eps: float = 1e-6
    group_size: int = 32

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    @classmethod
    def qwen3_0_6b(cls, group_size: int = 32) -> "Qwen3Config":
        """The chain's model (qwen3_npu_int8.py:99-110)."""
        return cls(group_size=group_size)

    @classmethod
    def qwen3_1_7b(cls, group_size: int = 32) -> "Qwen3Config":
        return cls(emb_dim=2048, hidden_dim=6144, n_heads=16, n_kv_heads=8, n_layers=28,
                   group_size=group_size)

    @classmethod
    def qwen3_8b(cls, group_size: int = 32) -> "Qwen3Config":
        return cls(emb_dim=4096, hidden_dim=12288, n_heads=32, n_kv_heads=8, n_layers=36,
                   vocab_size=151936, group_size=group_size)

    @classmethod
    def tiny(cls) -> "Qwen3Config":
        """A 2-layer model with the 0.6B head geometry, for smoke tests."""
        return cls(emb_dim=256, hidden_dim=768, n_heads=4, n_kv_heads=2, n_layers=2,
                   vocab_size=4096, group_size=32)

    def weight_bytes_per_token(self, lm_head: str = "bf16") -> dict:
        """Algorithmic bytes every decode step reads (excluding the KV cache)."""
        D, FF, G, QD, QKV = self.emb_dim, self.hidden_dim, self.group_size, self.q_dim, self.qkv_dim

        def w8(M, K):
            return M * K + M * (K // G) * 2

        per_layer = w8(QKV, D) + w8(D, QD) + 2 * w8(FF, D) + w8(D, FF) + 2 * D * 2 + \
            2 * self.head_dim * 2
        lm = self.vocab_size * D * 2 if lm_head == "bf16" else w8(self.vocab_size, D)
        return {"per_layer": per_layer, "layers": per_layer * self.n_layers, "lm_head": lm,
                "final_norm": D * 2}


def random_qwen3_weights(cfg: Qwen3Config, seed: int = 0, lin_std: float = 0.02,
                         emb_std: float = 0.1, lm_head: str = "bf16", device=None) -> dict:
    """Seeded random-init weights of the given architecture (no checkpoint needed).

    Linear weights are drawn N(0, lin_std) and RTN-quantized to int8 per-group (the
    reference's own quantizer, qwen3_npu_int8.py:457-491); norms are U[0.8, 1.2]; the
    embedding is N(0, emb_std) and the LM head is tied to it (Qwen3-0.6B ties them), either as
    bf16 or RTN int8. ``emb_std`` sets the logit spread; 0.1 gives logit std ~3 at D=1024.
    ``device`` selects where the numbers are drawn (a GPU generator is much faster at full
    size); the values are deterministic per (seed, device type).
    """
    dev = torch.device(device) if device is not None else torch.device("cpu")
    gen = torch.Generator(device=dev).manual_seed(seed)
    D, FF, HD, G = cfg.emb_dim, cfg.hidden_dim, cfg.head_dim, cfg.group_size

    def lin(M, K):
        return rtn_quantize(torch.randn(M, K, generator=gen, device=dev) * lin_std, G)

    def norm(n):
        return (0.8 + 0.4 * torch.rand(n, generator=gen, device=dev)).to(torch.bfloat16)

    layers = []
    for _ in range(cfg.n_layers):
        layers.append({
            "input_norm": norm(D), "post_norm": norm(D), "q_norm": norm(HD), "k_norm": norm(HD),
            "qkv": lin(cfg.qkv_dim, D), "o": lin(D, cfg.q_dim),
            "gate": lin(FF, D), "up": lin(FF, D), "down": lin(D, FF),
        })
    embed = (torch.randn(cfg.vocab_size, D, generator=gen, device=dev) * emb_std).to(torch.bfloat16)
    head = embed if lm_head == "bf16" else rtn_quantize(embed, G)
    return {"embed": embed, "final_norm": norm(D), "lm_head": head, "layers": layers}


def weights_to(w: dict, device) -> dict:
    """Copy of a neutral weight dict on ``device`` (tied embedding/head stay tied)."""
    def mv(t):
        return tuple(x.to(device) for x in t) if isinstance(t, tuple) else t.to(device)

    out = {"embed": mv(w["embed"]), "final_norm": mv(w["final_norm"]),
           "layers": [{k: mv(v) for k, v in L.items()} for L in w["layers"]]}
    out["lm_head"] = out["embed"] if w["lm_head"] is w["embed"] else mv(w["lm_head"])
    return out


def load_gptq_checkpoint(path, cfg: Qwen3Config, lm_head: str = "bf16") -> dict:
    """Qwen3 GPTQ-int8 safetensors -> neutral weights (qwen3_npu_int8.py:144-181, 350-379).

    The checkpoint's group size (128 for Qwen3-0.6B-GPTQ-Int8) must match ``cfg.group_size``.
    """
    from safetensors import safe_open

    f = safe_open(str(Path(path)), framework="pt")
    get = f.get_tensor
    layers = []
    for i in range(cfg.n_layers):
        L = f"model.layers.{i}"

        def q(name):
            qq, ss = gptq_unpack(get(f"{L}.{name}.qweight"), get(f"{L}.{name}.scales"))
            if qq.shape[1] // ss.shape[1] != cfg.group_size:
                raise ValueError(f"{name}: checkpoint group {qq.shape[1] // ss.shape[1]} != "
                                 f"config group {cfg.group_size}")
            return qq, ss

        qs = [q(f"self_attn.{p}_proj") for p in ("q", "k", "v")]
        layers.append({
            "input_norm": get(f"{L}.input_layernorm.weight").to(torch.bfloat16),
            "post_norm": get(f"{L}.post_attention_layernorm.weight").to(torch.bfloat16),
            "q_norm": get(f"{L}.self_attn.q_norm.weight").to(torch.bfloat16),
            "k_norm": get(f"{L}.self_attn.k_norm.weight").to(torch.bfloat16),
            "qkv": (torch.cat([a for a, _ in qs]), torch.cat([b for _, b in qs])),
            "o": q("self_attn.o_proj"), "gate": q("mlp.gate_proj"), "up": q("mlp.up_proj"),
            "down": q("mlp.down_proj"),
        })
    embed = get("model.embed_tokens.weight").to(torch.bfloat16)
    head = embed if lm_head == "bf16" else rtn_quantize(embed, cfg.group_size)
    return {"embed": embed, "final_norm": get("model.norm.weight").to(torch.bfloat16),
            "lm_head": head, "layers": layers}


def synthetic_kv(cfg: Qwen3Config, n_positions: int, seed: int = 0, scale: float = 1.0):
    """Seeded bf16 K/V for positions [0, n_positions) of every layer: (n_layers, Hkv, P, HD)."""
    gen = torch.Generator().manual_seed(seed)
    shape = (cfg.n_layers, cfg.n_kv_heads, n_positions, cfg.head_dim)
    k = (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)
    v = (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)
    return k, v
