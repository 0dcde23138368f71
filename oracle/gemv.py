"""int8 wire, dequant and GEMV goldens (test infrastructure only).

Follows:
  * wire layout -- iron/operators/gemv_int8/reference.py:59-80 (``pack_payload``) and
    iron/applications/qwen3_0.6b/qwen3_npu_int8.py:381-405 (``_pack_int8``): per row-block of
    ``tile_m`` rows, ``tile_m*K`` payload bytes then ``tile_m*(K/G)`` bf16 scales; payload byte =
    q + 128 (biased) or q as int8 (signed);
  * dequant -- op_ours.py:31-43 (``_payload_to_q``) and :515-541 (``_dequant_tiles``):
    w = q * s, exact in fp32; one RNE rounding gives the bit-exact bf16 weight;
  * exact GEMV golden -- GEMVInt8.reference, iron/operators/gemv_int8/op.py:173-178
    (dequantize, then matvec), evaluated in ``dt``;
  * premul GEMV golden -- iron/operators/gemv_int8/reference.py:25-40 (x*s rounded to bf16);
  * RTN quantizer -- qwen3_npu_int8.py:457-491; GPTQ unpack -- qwen3_npu_int8.py:350-379.
The wire pack/unpack here is written with explicit per-block loops on purpose, independent of
the product's vectorized packer.
"""

import numpy as np
import torch

from .numerics import EXACT


def pack_wire(q: torch.Tensor, s: torch.Tensor, tile_m: int, domain: str = "signed") -> np.ndarray:
    """(M,K) integer q + (M,K/G) bf16 scales -> flat uint8 wire (reference.py:59-80)."""
    q = np.asarray(q.to(torch.int16).numpy(), dtype=np.int16)
    M, K = q.shape
    if domain == "biased":
        w_bytes = (q + 128).astype(np.uint8)
    elif domain == "signed":
        w_bytes = q.astype(np.int8).view(np.uint8)
    else:
        raise ValueError(f"unknown payload domain: {domain}")
    s_bytes = s.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint8)
    s_bytes = s_bytes.reshape(M, -1)
    chunks = []
    for r0 in range(0, M, tile_m):
        chunks.append(w_bytes[r0:r0 + tile_m].reshape(-1))
        chunks.append(s_bytes[r0:r0 + tile_m].reshape(-1))
    return np.concatenate(chunks)


def unpack_wire(wire, M: int, K: int, G: int, tile_m: int, domain: str = "signed"):
    """Flat wire bytes -> ((M,K) int16 q, (M,K/G) bf16 s)."""
    b = np.asarray(wire).view(np.uint8).reshape(-1)
    ng = K // G
    blk = tile_m * K + tile_m * ng * 2
    q = np.empty((M, K), np.int16)
    sb = np.empty((M, ng * 2), np.uint8)
    for i, r0 in enumerate(range(0, M, tile_m)):
        o = i * blk
        pay = b[o:o + tile_m * K].reshape(tile_m, K)
        q[r0:r0 + tile_m] = pay.astype(np.int16) - 128 if domain == "biased" else pay.view(np.int8)
        sb[r0:r0 + tile_m] = b[o + tile_m * K:o + blk].reshape(tile_m, ng * 2)
    s = torch.from_numpy(sb.copy().view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(q), s


def dequant(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """Bit-exact bf16 dequant: bf16(f32(q) * f32(s)), s broadcast over each group of K."""
    G = q.shape[1] // s.shape[1]
    return (q.float() * s.float().repeat_interleave(G, dim=1)).to(torch.bfloat16)


def dequant_f(q: torch.Tensor, s: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """q * s in ``dt`` (exact in fp32 already: 8-bit x 8-bit significands)."""
    G = q.shape[1] // s.shape[1]
    return q.to(dt) * s.to(dt).repeat_interleave(G, dim=1)


def dequant_f32(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    return dequant_f(q, s, torch.float32)


def gemv(W: torch.Tensor, x: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """Dequantized (M,K) weight times x (K,) or (B,K), in ``dt`` (no rounding)."""
    W = W.to(dt)
    return x.to(dt) @ W.t() if x.dim() == 2 else W @ x.to(dt)


def gemv_exact(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """GEMVInt8.reference (op.py:173-178): (q*s) @ x in ``dt``. x: (K,) or (B,K)."""
    return gemv(dequant_f(q, s, dt), x, dt)


def gemv_premul(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """Kernel-form golden (gemv_int8/reference.py:25-40): sum q * bf16(x * s), fp32."""
    M, K = q.shape
    s_exp = s.float().repeat_interleave(K // s.shape[1], dim=1)
    xs = (x.float()[None, :] * s_exp).to(torch.bfloat16).float()
    return (q.float() * xs).sum(dim=1)


def rtn_quantize(w: torch.Tensor, G: int):
    """Symmetric per-group int8 RTN (qwen3_npu_int8.py:457-491) -> (int8 q, bf16 s)."""
    M, K = w.shape
    blk = w.float().reshape(M, K // G, G)
    s = blk.abs().amax(dim=2) / 127.0
    s = torch.where(s > 0, s, torch.ones_like(s)).to(torch.bfloat16)
    q = torch.round(blk / s.float()[:, :, None]).clamp(-127, 127).to(torch.int8)
    return q.reshape(M, K), s


def gptq_unpack(qweight: torch.Tensor, scales: torch.Tensor):
    """GPTQ (K/4,M) int32 + (G,M) fp16 -> ((M,K) int8 q, (M,G) bf16 s); zero-point 128."""
    qw = qweight.numpy().astype(np.uint32)
    K4, M = qw.shape
    out = np.empty((M, K4 * 4), np.int16)
    for j in range(4):
        out[:, j::4] = (((qw >> np.uint32(8 * j)) & np.uint32(0xFF)).astype(np.int16) - 128).T
    s = torch.from_numpy(scales.numpy().astype(np.float32)).to(torch.bfloat16).t().contiguous()
    return torch.from_numpy(out.astype(np.int8)), s
