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
    repeat_interleave of K/V heads);
  * batch / verify decode attention -- the DecodeAttention batch mode
    (iron/operators/decode_attn/op.py:40-48, design.py:243-276; the CPU reference of its test,
    decode_attn/test_batch.py:31-45): n new tokens at positions base..base+n-1, token t attends
    keys [0, base + t] when causal and the whole cache [0, S) otherwise.
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


def verify_bounds(n_new: int, base: int, S: int, causal: bool) -> list[int]:
    """Keys each new token attends (decode_attn/design.py:255-262): base + t + 1 when causal
    (the per-query boundary S_kv_base + g*M + m + 1 with t = g*M + m), S otherwise; at most S."""
    return [min(base + t + 1, S) if causal else S for t in range(n_new)]


def decode_attention_verify(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, base: int,
                            causal: bool = True, scale: float | None = None,
                            dt=EXACT) -> torch.Tensor:
    """q (n, H, D) token-major; k, v (KV, S, D) one cache -> (n, H, D) bf16.

    Token t is a decode query over its own bound (``verify_bounds``); the grouping of queries
    (batch_queries) only changes how the cache is streamed, not the result."""
    n, H, D = q.shape
    KV, S = k.shape[0], k.shape[1]
    bounds = verify_bounds(n, base, S, causal)
    kk = k.unsqueeze(0).expand(n, KV, S, D)
    vv = v.unsqueeze(0).expand(n, KV, S, D)
    return decode_attention(q, kk, vv, bounds, scale, dt)
