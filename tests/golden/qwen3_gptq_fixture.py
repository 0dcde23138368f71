"""A tiny Qwen3 GPTQ-int8 checkpoint and its Hugging Face reference logits (test data).

``make_checkpoint(path)`` writes a seeded random-init Qwen3-architecture model in the layout of
the Qwen3-0.6B-GPTQ-Int8 safetensors the reference loads (qwen3_npu_int8.py:144-181, 350-379):
per linear layer ``qweight`` (K/4, M) int32 holding four little-endian bytes q + 128 along K
(zero point 128) and ``scales`` (K/G, M) fp16; bf16 embedding (tied LM head) and norm weights.
Its group size is 128, the checkpoint's.

``hf_logits(path)`` loads the same checkpoint's dequantized weights (q * fp16 scale, in fp32)
into a random-init ``transformers`` ``Qwen3ForCausalLM`` built from an explicit config (no
download) and prefills ``PROMPT`` in one forward: the fp32 reference of the reference's own
logit gate (check_cosine_int8.py:29-70: cosine > 0.99 and an argmax match). The fixture file
``qwen3_tiny_hf_logits.safetensors`` holds those logits; ``make_hf_fixtures.py`` writes it.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "qwen3_tiny_hf_logits.safetensors"

D, FF, HQ, HKV, HD, LAYERS, VOCAB, G = 256, 768, 4, 2, 128, 2, 1024, 128
EPS, THETA = 1e-6, 1e6
SEED = 4242
# weight scales: large enough that the layers, not the tied embedding's self-similarity, decide
# each position's argmax (no argmax equals its input token; top-1/top-2 margins >= 0.19)
LIN_STD, EMB_STD = 0.3, 0.1
PROMPT = [17, 301, 5, 988, 42, 613, 77, 250, 1001, 3, 512, 64]


def config():
    """The iron_amd config of the fixture model."""
    from iron_amd.applications.qwen3_0_6b.weights import Qwen3Config

    return Qwen3Config(emb_dim=D, hidden_dim=FF, n_heads=HQ, n_kv_heads=HKV, head_dim=HD,
                       vocab_size=VOCAB, n_layers=LAYERS, rope_theta=THETA, eps=EPS,
                       group_size=G)


def _gptq(w: torch.Tensor):
    """fp32 (M, K) -> (qweight (K/4, M) int32, scales (K/G, M) fp16), symmetric int8 with the
    stored byte q + 128."""
    M, K = w.shape
    wg = w.reshape(M, K // G, G)
    s = (wg.abs().amax(-1) / 127.0).clamp_min(1e-8).to(torch.float16)         # (M, K/G)
    q = torch.round(wg / s.float()[..., None]).clamp(-128, 127).to(torch.int64).reshape(M, K)
    u = (q + 128).t().contiguous()                                            # (K, M) bytes
    u = u.reshape(K // 4, 4, M)
    packed = u[:, 0] | (u[:, 1] << 8) | (u[:, 2] << 16) | (u[:, 3] << 24)
    qweight = torch.where(packed >= 2**31, packed - 2**32, packed).to(torch.int32)
    return qweight, s.t().contiguous()


def _dequant(qweight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """(K/4, M) int32 + (K/G, M) fp16 -> (M, K) fp32 = (byte - 128) * scale."""
    qw = qweight.to(torch.int64) & 0xFFFFFFFF
    K4, M = qw.shape
    u = torch.stack([(qw >> (8 * i)) & 0xFF for i in range(4)], dim=1).reshape(K4 * 4, M)
    q = (u - 128).float().t()                                                 # (M, K)
    return q * scales.float().t().repeat_interleave(G, dim=1)


def tensors() -> dict:
    """The checkpoint's tensors (seeded)."""
    gen = torch.Generator().manual_seed(SEED)
    out = {}

    def lin(name, M, K):
        qw, s = _gptq(torch.randn(M, K, generator=gen) * LIN_STD)
        out[f"{name}.qweight"] = qw
        out[f"{name}.scales"] = s

    def norm(name, n):
        out[name] = (0.8 + 0.4 * torch.rand(n, generator=gen)).to(torch.bfloat16)

    for i in range(LAYERS):
        L = f"model.layers.{i}"
        norm(f"{L}.input_layernorm.weight", D)
        norm(f"{L}.post_attention_layernorm.weight", D)
        norm(f"{L}.self_attn.q_norm.weight", HD)
        norm(f"{L}.self_attn.k_norm.weight", HD)
        lin(f"{L}.self_attn.q_proj", HQ * HD, D)
        lin(f"{L}.self_attn.k_proj", HKV * HD, D)
        lin(f"{L}.self_attn.v_proj", HKV * HD, D)
        lin(f"{L}.self_attn.o_proj", D, HQ * HD)
        lin(f"{L}.mlp.gate_proj", FF, D)
        lin(f"{L}.mlp.up_proj", FF, D)
        lin(f"{L}.mlp.down_proj", D, FF)
    out["model.embed_tokens.weight"] = (torch.randn(VOCAB, D, generator=gen) * EMB_STD).to(
        torch.bfloat16)
    norm("model.norm.weight", D)
    return out


def digest(t: dict) -> str:
    """SHA-256 over the tensors' names and bytes (ties a fixture to the weights it came from)."""
    h = hashlib.sha256()
    for k in sorted(t):
        h.update(k.encode())
        h.update(t[k].contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def make_checkpoint(path) -> str:
    """Write the checkpoint to ``path``; returns its digest."""
    from safetensors.torch import save_file

    t = tensors()
    save_file(t, str(path))
    return digest(t)


def hf_logits(t: dict | None = None) -> torch.Tensor:
    """fp32 logits (len(PROMPT), VOCAB) of a transformers Qwen3ForCausalLM holding the
    checkpoint's dequantized weights, prefilling PROMPT in one forward."""
    from transformers import Qwen3Config, Qwen3ForCausalLM

    t = t or tensors()
    cfg = Qwen3Config(vocab_size=VOCAB, hidden_size=D, intermediate_size=FF,
                      num_hidden_layers=LAYERS, num_attention_heads=HQ,
                      num_key_value_heads=HKV, head_dim=HD, max_position_embeddings=256,
                      rms_norm_eps=EPS, rope_parameters={"rope_theta": THETA,
                                                         "rope_type": "default"},
                      tie_word_embeddings=True, attention_bias=False, hidden_act="silu")
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).float().eval()
    sd = {}
    for k, v in t.items():
        if k.endswith(".qweight"):
            base = k[: -len(".qweight")]
            sd[base + ".weight"] = _dequant(v, t[base + ".scales"])
        elif not k.endswith(".scales"):
            sd[k] = v.float()
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m for m in missing), missing
    with torch.no_grad():
        return model(torch.tensor([PROMPT])).logits[0].float()


def load_fixture() -> tuple[torch.Tensor, str]:
    """(HF logits (len(PROMPT), VOCAB) fp32, the weights digest they belong to)."""
    from safetensors import safe_open

    with safe_open(str(FIXTURE), framework="pt") as f:
        logits = f.get_tensor("logits")
        meta = f.metadata()
    return logits, meta["weights_sha256"]
