"""``op.reference()`` provider for iron_amd operators (test infrastructure only).

Tests install it with ``iron_amd.common.base.register_reference_provider(oracle.provider.
reference)``; the operator classes themselves carry no CPU path. Each branch mirrors the
reference operator's own ``reference()`` method:
  GEMVInt8                    -- gemv_int8/op.py:173-178 (dequant, matvec, bf16)
  RMSNorm                     -- rms_norm/op.py:125-130
  DecodeAttention             -- decode_attn/reference.py:26-38 (static arm: every key valid)
  QKVHeadDataParallel(Ours)   -- qkv_head_dp/op.py:225-231 (concatenated [q | k | v])
  SwiGLUMLPDataParallelOurs   -- swiglu_mlp_dp/op_ours.py:543-582
  MHA                         -- mha/reference.py:73-81 (causal SDPA, scale 1/sqrt(d))
Operators are recognised by class name and read only their public fields.
"""

from __future__ import annotations

import torch

from .attention import causal_prefill_attention, decode_attention
from .blocks import qkv_head, swiglu_mlp
from .gemv import gemv_exact, unpack_wire
from .norms import rms_norm


def _domain(op) -> str:
    src = getattr(op, "kernel_source", None)
    return "signed" if (src and "signed" in src) else "biased"


def _unpack(w, M, K, G, tile_m, domain):
    return unpack_wire(w.contiguous().view(torch.uint8).cpu().numpy(), M, K, G, tile_m, domain)


def reference(op, *inputs):
    name = type(op).__name__
    inputs = [t.cpu() if isinstance(t, torch.Tensor) else t for t in inputs]
    if name == "GEMVInt8":
        w, x = inputs
        q, s = _unpack(w, op.M, op.K, op.group_size, op.tile_size_input, _domain(op))
        return gemv_exact(q, s, x.reshape(-1, op.K)).float().to(torch.bfloat16).reshape(-1)
    if name == "RMSNorm":
        x = inputs[0]
        w = inputs[1] if op.weighted else None
        return rms_norm(x, w, op.epsilon)
    if name == "DecodeAttention":
        H, KV, D, S, B = op.num_heads, op.num_kv_heads, op.head_dim, op.seq_len_kv, op.batch
        q = inputs[0].reshape(B, H, D)
        if op.kv_layout == "separate":
            k = inputs[1].reshape(B, KV, S, D)
            v = inputs[2].reshape(B, KV, S, D)
        else:
            kv = inputs[1].reshape(B, KV, 2 * S * D)
            if op.kv_token_interleaved:
                t = kv.reshape(B, KV, S, 2, D)
                k, v = t[:, :, :, 0], t[:, :, :, 1]
            else:
                k = kv[:, :, : S * D].reshape(B, KV, S, D)
                v = kv[:, :, S * D:].reshape(B, KV, S, D)
        return decode_attention(q, k, v, S, op.softmax_scale).reshape(B * H, D)
    if name in ("QKVHeadDataParallel", "QKVHeadDataParallelOurs"):
        cur, n_in, w, n_qn, n_kn, ang = inputs[:6]
        q8, s = _unpack(w, op.M, op.D, op.group_size, op.tile_size_input, _domain(op))
        q, k, v = qkv_head(cur.reshape(op.batch, op.D), n_in, q8, s, n_qn, n_kn,
                           ang.reshape(op.batch, op.HD), op.Hq, op.Hkv, op.HD, op.epsilon)
        return torch.cat([q, k, v], dim=1).reshape(-1)
    if name == "SwiGLUMLPDataParallelOurs":
        dom, G = _domain(op), op.group_size
        cur, cx, n_pf = inputs[:3]
        rest = inputs[3:]
        wo = None
        if op.fuse_o:
            wo = _unpack(rest[0], op.D, op.QD, G, op.tile_rows_o, dom)
            rest = rest[1:]
        wg = _unpack(rest[0], op.FF, op.D, G, op.tile_rows_gu, dom)
        wu = _unpack(rest[1], op.FF, op.D, G, op.tile_rows_gu, dom)
        wd = _unpack(rest[2], op.D, op.FF, G, op.tile_rows_d, dom)
        nxt, _ = swiglu_mlp(cur.reshape(op.batch, op.D), cx, n_pf, wg, wu, wd, op.epsilon,
                            wo=wo)
        return nxt.reshape(-1)
    if name == "MHA":
        H, KV, D, S = op.num_heads, op.kv_heads, op.d, op.seq_padded
        q = inputs[0].reshape(H, S, D)
        k = inputs[1].reshape(KV, S, D)
        v = inputs[2].reshape(KV, S, D)
        return causal_prefill_attention(q, k, v).to(torch.bfloat16).reshape(-1)
    if name == "QKVHeadAttention":
        # The fused operator has no reference counterpart (the reference runs the QKV head and
        # DecodeAttention as two entries); its result is checked against that composition.
        raise NotImplementedError("QKVHeadAttention: compare against the QKV head -> "
                                  "DecodeAttention composition")
    raise NotImplementedError(f"no golden for {name}")
