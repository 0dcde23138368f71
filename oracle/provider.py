"""``op.reference()`` provider for iron_amd operators (test infrastructure only).

Tests install it with ``iron_amd.common.base.register_reference_provider(oracle.provider.
reference)``; the operator classes themselves carry no CPU path. Each branch mirrors the
reference operator's own ``reference()`` method:
  GEMVInt8 / GEMV             -- gemv_int8/op.py:173-178 (dequant, matvec, bf16); with the argmax
                                 epilogue the logits are written into their argument and the
                                 packed argmax key is returned (the host argmax of
                                 qwen3_npu_int8.py:612-621)
  RMSNorm                     -- rms_norm/op.py:125-130
  RoPE                        -- rope/op.py:84-96 (two halves; the interleaved method as
                                 rope/reference.py:94-112)
  QKNormRoPE                  -- qk_norm_rope/reference.py:19-40 with the kernel's bf16 normalised
                                 head (qk_norm_rope.cc:42-108); with kv_direct (``params`` holding
                                 the element offset) the K|V slice written into ``last``, the
                                 cache returned after qkv_out is written into its argument
  DecodeAttention             -- decode_attn/reference.py:26-38; the runtime bound S_kv_eff when
                                 use_runtime_seq_len (else every key is valid); batch/verify mode
                                 (batch_queries > 0) with the per-query bound of
                                 decode_attn/design.py:243-276
  QKVHeadDataParallel(Ours)   -- qkv_head_dp/op.py:225-231 (concatenated [q | k | v]); inside a
                                 sequence (``params`` given) the step's effect instead: q written
                                 into its argument, k and v appended to the cache at the runtime
                                 position, the cache returned
  QKVHeadAttention            -- the composition the fused operator replaces: the QKV head above
                                 (cache append included), then decode attention over 0..pos
  SwiGLUMLPDataParallelOurs   -- swiglu_mlp_dp/op_ours.py:543-582
  MHA                         -- mha/reference.py:73-81 (causal SDPA, scale 1/sqrt(d))
Operators are recognised by class name and read only their public fields. ``params`` maps a
runtime-parameter name to the int values the kernels read (positions, context lengths);
``last`` is the pre-step value of the step's last argument when that argument is ``inout``.
"""

from __future__ import annotations

import numpy as np
import torch

from .attention import causal_prefill_attention, decode_attention, decode_attention_verify
from .blocks import qkv_head, swiglu_mlp
from .gemv import gemv_exact, unpack_wire
from .norms import qk_norm_rope, rms_norm, rope, rope_interleaved


def _domain(op) -> str:
    src = getattr(op, "kernel_source", None)
    return "signed" if (src and "signed" in src) else "biased"


def _unpack(w, M, K, G, tile_m, domain):
    return unpack_wire(w.contiguous().view(torch.uint8).cpu().numpy(), M, K, G, tile_m, domain)


def _param(params, name, n):
    if params is None or name not in params:
        raise KeyError(f"runtime parameter {name!r} is needed by this golden")
    vals = np.atleast_1d(np.asarray(params[name])).astype(np.int64)
    return [int(v) for v in vals[:n]]


def argmax_key(y: torch.Tensor) -> int:
    """The packed key of the first maximal bf16 value (the LM head's argmax epilogue):
    (order-preserving bf16 bits << 32) | ~index."""
    bits = y.to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
    order = torch.where(bits & 0x8000 != 0, (~bits) & 0xFFFF, bits | 0x8000)
    best = int(order.max())
    idx = int(torch.nonzero(order == best)[0, 0])
    return (best << 32) | ((~idx) & 0xFFFFFFFF)


def _kv_views(op, caches, B):
    """(k, v) views (B, Hkv, S, HD) of a QKV operator's cache argument(s)."""
    S, HD, KV = op.max_seq, op.HD, op.Hkv
    if op.kv_layout == "separate":
        return caches[0].reshape(B, KV, S, HD), caches[1].reshape(B, KV, S, HD)
    t = caches[0].reshape(B, KV, S, 2, HD)
    return t[:, :, :, 0], t[:, :, :, 1]


def _qkv_step(op, inputs, params):
    """The QKV head of a decode step: (q (B, Hq*HD), pos list); k, v appended in place."""
    B = op.batch
    cur, n_in, w, n_qn, n_kn, ang = inputs[:6]
    q8, s = _unpack(w, op.M, op.D, op.group_size, op.tile_size_input, _domain(op))
    pname = op.kv_offset_parameter or "kv_off"
    pos = _param(params, pname, B)
    if op.angles_from_table:
        table = ang.reshape(op.max_seq, op.HD)
        ang_rows = torch.stack([table[p] for p in pos])
    else:
        ang_rows = ang.reshape(B, op.HD)
    q, k, v = qkv_head(cur.reshape(B, op.D), n_in, q8, s, n_qn, n_kn, ang_rows, op.Hq, op.Hkv,
                       op.HD, op.epsilon)
    return q, k, v, pos


def reference(op, *inputs, params=None, last=None):
    name = type(op).__name__
    inputs = [t.cpu() if isinstance(t, torch.Tensor) else t for t in inputs]
    if name == "GEMVInt8":
        w, x = inputs[:2]
        q, s = _unpack(w, op.M, op.K, op.group_size, op.tile_size_input, _domain(op))
        y = gemv_exact(q, s, x.reshape(-1, op.K)).float().to(torch.bfloat16).reshape(-1)
        if getattr(op, "epilogue", "none") == "argmax":
            inputs[2].reshape(-1)[: y.numel()].copy_(y)
            return torch.tensor([argmax_key(y[: op.M])], dtype=torch.int64)
        return y
    if name == "GEMV":
        a, x = inputs[:2]
        y = (a.reshape(op.M, op.K).double() @ x.reshape(op.K).double()).float().to(
            torch.bfloat16)
        if op.epilogue == "argmax":
            inputs[2].reshape(-1)[: op.M].copy_(y)
            return torch.tensor([argmax_key(y)], dtype=torch.int64)
        return y
    if name == "RMSNorm":
        x = inputs[0]
        w = inputs[1] if op.weighted else None
        return rms_norm(x, w, op.epsilon)
    if name == "RoPE":
        x, ang = inputs[0].reshape(op.rows, op.cols), inputs[1].reshape(op.angle_rows, op.cols)
        return (rope if op.method_type == 0 else rope_interleaved)(x, ang)
    if name == "QKNormRoPE":
        qkv, scratch = inputs[0].reshape(-1), inputs[2].reshape(-1)
        out = qk_norm_rope(qkv, scratch, op.n_qk_heads, op.n_v_heads, op.head_dim, op.epsilon)
        if not op.kv_direct:
            return out
        if last is None:
            raise ValueError("the kv_direct golden needs the pre-step cache (last=)")
        inputs[1].reshape(-1)[: out.numel()].copy_(out)
        HD, S, nv, nq = op.head_dim, op.max_seq_len, op.n_v_heads, op.n_qk_heads - op.n_v_heads
        off = _param(params, op.kv_offset_parameter, 1)[0]
        cache = last.cpu().clone().reshape(-1)
        if 0 <= off and off + 2 * HD <= 2 * S * HD:
            for j in range(nv):
                base = j * 2 * S * HD + off
                cache[base: base + HD] = out[(nq + j) * HD: (nq + j + 1) * HD]
                cache[base + HD: base + 2 * HD] = out[(nq + nv + j) * HD: (nq + nv + j + 1) * HD]
        return cache
    if name == "DecodeAttention":
        H, KV, D, S, B = op.num_heads, op.num_kv_heads, op.head_dim, op.seq_len_kv, op.batch
        verify = op.batch_queries > 0
        nq = op.num_new_tokens if verify else B
        q = inputs[0].reshape(nq, H, D)
        bk = 1 if verify else B
        if op.kv_layout == "separate":
            k = inputs[1].reshape(bk, KV, S, D)
            v = inputs[2].reshape(bk, KV, S, D)
        else:
            kv = inputs[1].reshape(bk, KV, 2 * S * D)
            if op.kv_token_interleaved:
                t = kv.reshape(bk, KV, S, 2, D)
                k, v = t[:, :, :, 0], t[:, :, :, 1]
            else:
                k = kv[:, :, : S * D].reshape(bk, KV, S, D)
                v = kv[:, :, S * D:].reshape(bk, KV, S, D)
        if verify:
            base = _param(params, "S_kv_base", 1)[0]
            return decode_attention_verify(q, k[0], v[0], base, op.causal,
                                           op.softmax_scale).reshape(nq * H, D)
        ctx = _param(params, "S_kv_eff", B) if (op.use_runtime_seq_len and params) else S
        return decode_attention(q, k, v, ctx, op.softmax_scale).reshape(B * H, D)
    if name in ("QKVHeadDataParallel", "QKVHeadDataParallelOurs"):
        if params is None:
            cur, n_in, w, n_qn, n_kn, ang = inputs[:6]
            q8, s = _unpack(w, op.M, op.D, op.group_size, op.tile_size_input, _domain(op))
            q, k, v = qkv_head(cur.reshape(op.batch, op.D), n_in, q8, s, n_qn, n_kn,
                               ang.reshape(op.batch, op.HD), op.Hq, op.Hkv, op.HD, op.epsilon)
            return torch.cat([q, k, v], dim=1).reshape(-1)
        # a sequence step: q goes into its argument, k and v into the cache at the runtime
        # position; the cache argument that ends the spec (``last``, its pre-step value) is the
        # returned output
        if last is None:
            raise ValueError("the QKV head's cache golden needs the pre-step cache (last=)")
        q, k, v, pos = _qkv_step(op, inputs, params)
        inputs[6].reshape(-1)[: q.numel()].copy_(q.reshape(-1))
        out = last.cpu().clone()
        caches = list(inputs[7:]) + [out]
        kc, vc = _kv_views(op, caches, op.batch)
        for b in range(op.batch):
            kc[b, :, pos[b]] = k[b].reshape(op.Hkv, op.HD)
            vc[b, :, pos[b]] = v[b].reshape(op.Hkv, op.HD)
        return out.reshape(-1)
    if name == "QKVHeadAttention":
        q, k, v, pos = _qkv_step(op, inputs, params)
        B = op.batch
        caches = list(inputs[6:])
        kc, vc = _kv_views(op, caches, B)
        for b in range(B):
            kc[b, :, pos[b]] = k[b].reshape(op.Hkv, op.HD)
            vc[b, :, pos[b]] = v[b].reshape(op.Hkv, op.HD)
        return decode_attention(q.reshape(B, op.Hq, op.HD), kc, vc, [p + 1 for p in pos],
                                op.softmax_scale).reshape(-1)
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
        nxt, a = swiglu_mlp(cur.reshape(op.batch, op.D), cx, n_pf, wg, wu, wd, op.epsilon,
                            wo=wo)
        if op.fuse_o and len(rest) > 4:  # a_scratch (inout) receives a
            rest[4].reshape(-1)[: a.numel()].copy_(a.reshape(-1))
        return nxt.reshape(-1)
    if name == "MHA":
        H, KV, D, S = op.num_heads, op.kv_heads, op.d, op.seq_padded
        q = inputs[0].reshape(H, S, D)
        k = inputs[1].reshape(KV, S, D)
        v = inputs[2].reshape(KV, S, D)
        return causal_prefill_attention(q, k, v).to(torch.bfloat16).reshape(-1)
    raise NotImplementedError(f"no golden for {name}")

