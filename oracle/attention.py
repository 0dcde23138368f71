"""Attention goldens (test infrastructure only).

Follows:
  * decode attention -- iron/operators/decode_attn/reference.py:26-38: scores q.K^T scaled,
    causal mask j <= seq_pos, p = exp2(s*log2(e)/sqrt(D) - max), o = (p @ V) / sum(p), bf16
    output; GQA kv = h * KV // H. A sequence with no valid key gives zeros (the kernel's
    finalize, aie_kernels/aie2p/decode_attn.cc:300-311). exp2(log2(e) * t) is exp(t); the form
    used here is the natural exponential of the scaled score, evaluated in ``dt``;
  * the torch.softmax form of the decode-attention scripts (decode_attn/test_seqpos_runtime.py:
    26-34) -- identical in exact arithmetic, used as an independent check;
  * causal prefill MHA -- iron/operators/mha/reference.py:73-81 (SDPA, is_causal, GQA by
    repeat_interleave of K/V heads).
"""

import math

import torch

from .numerics import EXACT, f32


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ctx_len,
                     scale: float | None = None, dt=EXACT) -> torch.Tensor:
    """q (B,H,D); k,v (B,KV,L,D); ctx_len: int or sequence of B ints -> (B,H,D) bf16."""
    B, H, D = q.shape
    KV = k.shape[1]
    if isinstance(ctx_len, int):
        ctx_len = [ctx_len] * B
    sc = f32(scale if scale is not None else 1.0 / math.sqrt(D))
    out = torch.zeros(B, H, D, dtype=dt)
    for b in range(B):
        n = int(ctx_len[b])
        if n <= 0:
            continue
        for h in range(H):
            kv = h * KV // H
            s = (k[b, kv, :n].to(dt) @ q[b, h].to(dt)) * sc
            p = torch.exp(s - s.max())
            out[b, h] = (p @ v[b, kv, :n].to(dt)) / p.sum()
    return out.float().to(torch.bfloat16)


def decode_attention_softmax(q, k, v, ctx_len, scale=None) -> torch.Tensor:
    """Same contract, via torch.softmax in fp32 (the scripts' golden form)."""
    B, H, D = q.shape
    KV = k.shape[1]
    if isinstance(ctx_len, int):
        ctx_len = [ctx_len] * B
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    out = torch.zeros(B, H, D, dtype=torch.float32)
    for b in range(B):
        n = int(ctx_len[b])
        if n <= 0:
            continue
        g = H // KV
        kk = k[b, :, :n].float().repeat_interleave(g, dim=0)
        vv = v[b, :, :n].float().repeat_interleave(g, dim=0)
        att = torch.softmax((q[b].float()[:, None, :] @ kk.transpose(1, 2)) * sc, dim=-1)
        out[b] = (att @ vv)[:, 0]
    return out.to(torch.bfloat16)


def decode_attention_f64(q, k, v, ctx_len, scale=None) -> torch.Tensor:
    """fp64 brute force with explicit loops over heads (no rounding of the result)."""
    B, H, D = q.shape
    KV = k.shape[1]
    if isinstance(ctx_len, int):
        ctx_len = [ctx_len] * B
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    out = torch.zeros(B, H, D, dtype=torch.float64)
    for b in range(B):
        n = int(ctx_len[b])
        for h in range(H):
            kv = h * KV // H
            if n <= 0:
                continue
            s = (k[b, kv, :n].double() @ q[b, h].double()) * sc
            m = float(s.max())
            w = torch.exp(s - m)
            out[b, h] = (w[:, None] * v[b, kv, :n].double()).sum(0) / w.sum()
    return out


def causal_prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             scale: float | None = None, dt=torch.float32) -> torch.Tensor:
    """q (H,S,D), k/v (KV,S,D) -> (H,S,D) in ``dt``, causal, GQA (mha/reference.py:73-81)."""
    H, S, D = q.shape
    KV = k.shape[0]
    g = H // KV
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    kk = k.to(dt).repeat_interleave(g, dim=0)
    vv = v.to(dt).repeat_interleave(g, dim=0)
    s = (q.to(dt) @ kk.transpose(1, 2)) * sc
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    s = s.masked_fill(~mask, float("-inf"))
    return torch.softmax(s, dim=-1) @ vv
