"""int8 weight wires: packing, unpacking and the two quantizers the decode chain uses.

Wire format (the reference's, iron/operators/gemv_int8/reference.py:59-80 and
iron/applications/qwen3_0.6b/qwen3_npu_int8.py:381-405): consecutive row-blocks of ``tile_m``
rows; block ``i`` holds rows ``[i*tile_m, (i+1)*tile_m)`` as ``tile_m*K`` payload bytes
(row-major) followed by ``tile_m*(K/G)`` bf16 scale bit patterns (row-major). The reference's
per-column split (``cols``) does not change the byte order -- column ``c`` owns a contiguous run
of whole blocks -- so it is not a parameter here. Payload domains: ``"signed"`` stores q as
two's complement, ``"biased"`` stores q + 128; both encode the same integer q.

All functions are vectorized torch code (host or device tensors alike); none is on the per-token
path.
"""

from __future__ import annotations

import torch

DOMAINS = ("signed", "biased")


def wire_nbytes(M: int, K: int, G: int, tile_m: int) -> int:
    if K % G or M % tile_m:
        raise ValueError(f"bad wire geometry M={M} K={K} G={G} tile_m={tile_m}")
    return (M // tile_m) * (tile_m * K + tile_m * (K // G) * 2)


def domain_of(kernel_source: str | None) -> str:
    """Payload domain selected by a reference ``kernel_source`` name (None = biased default)."""
    if kernel_source is None or "signed" not in kernel_source:
        return "biased"
    return "signed"


def pack_wire(q: torch.Tensor, scales: torch.Tensor, tile_m: int, domain: str = "signed"
              ) -> torch.Tensor:
    """(M, K) integer q in [-128, 127] + (M, K/G) bf16 scales -> flat uint8 wire."""
    if domain not in DOMAINS:
        raise ValueError(f"unknown payload domain: {domain}")
    M, K = q.shape
    ng = scales.shape[1]
    if scales.shape[0] != M or K % ng:
        raise ValueError(f"scales {tuple(scales.shape)} do not match q {tuple(q.shape)}")
    if M % tile_m:
        raise ValueError(f"tile_m={tile_m} must divide M={M}")
    qi = q.to(torch.int16)
    if domain == "biased":
        payload = (qi + 128).to(torch.uint8)
    else:
        payload = qi.to(torch.int8).view(torch.uint8)
    sb = scales.to(torch.bfloat16).contiguous().view(torch.uint8).reshape(M, ng * 2)
    nblk = M // tile_m
    blocks = torch.cat([payload.reshape(nblk, tile_m * K), sb.reshape(nblk, tile_m * ng * 2)],
                       dim=1)
    return blocks.reshape(-1).contiguous()


def unpack_wire(wire: torch.Tensor, M: int, K: int, G: int, tile_m: int, domain: str = "signed"
                ) -> tuple[torch.Tensor, torch.Tensor]:
    """Flat wire (any dtype view of the bytes) -> ((M, K) int16 q, (M, K/G) bf16 scales)."""
    if domain not in DOMAINS:
        raise ValueError(f"unknown payload domain: {domain}")
    b = wire.contiguous().view(torch.uint8).reshape(-1)
    n = wire_nbytes(M, K, G, tile_m)
    if b.numel() < n:
        raise ValueError(f"wire holds {b.numel()} bytes, geometry needs {n}")
    ng = K // G
    nblk = M // tile_m
    blocks = b[:n].reshape(nblk, tile_m * K + tile_m * ng * 2)
    payload = blocks[:, : tile_m * K].reshape(M, K)
    sb = blocks[:, tile_m * K:].reshape(M, ng * 2).contiguous()
    if domain == "biased":
        q = payload.to(torch.int16) - 128
    else:
        q = payload.contiguous().view(torch.int8).to(torch.int16)
    return q, sb.view(torch.bfloat16)


def rtn_quantize(w: torch.Tensor, G: int, chunk_rows: int = 16384
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-(row, group) round-to-nearest int8 quantizer.

    Follows ``Qwen3NPU._set_int8_rtn`` (qwen3_npu_int8.py:457-491): ``s = bf16(max|w| / 127)``
    per group (1.0 for an all-zero group), ``q = clamp(round(w / s), -127, 127)`` rounded against
    the bf16 scale the wire carries. Returns ((M, K) int8, (M, K/G) bf16).
    """
    M, K = w.shape
    if K % G:
        raise ValueError(f"K={K} not a multiple of G={G}")
    ng = K // G
    q = torch.empty((M, K), dtype=torch.int8, device=w.device)
    s = torch.empty((M, ng), dtype=torch.bfloat16, device=w.device)
    for r0 in range(0, M, chunk_rows):
        blk = w[r0:r0 + chunk_rows].float().reshape(-1, ng, G)
        s_ = blk.abs().amax(dim=2) / 127.0
        s_ = torch.where(s_ > 0, s_, torch.ones_like(s_))
        s_wire = s_.to(torch.bfloat16)
        qq = torch.round(blk / s_wire.float()[:, :, None]).clamp_(-127, 127)
        q[r0:r0 + chunk_rows] = qq.to(torch.int8).reshape(-1, K)
        s[r0:r0 + chunk_rows] = s_wire
    return q, s


def gptq_unpack(qweight: torch.Tensor, scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """GPTQ sym-int8 checkpoint tensors -> ((M, K) int8 q, (M, n_groups) bf16 scales).

    Follows ``Qwen3NPU._gptq_rows`` (qwen3_npu_int8.py:350-379): ``qweight`` is (K/4, M) int32
    with four little-endian u8 per word along K, the stored byte is q + 128 (zero-point 128), and
    ``scales`` is (n_groups, M) fp16.
    """
    qw = qweight.to(torch.int64) & 0xFFFFFFFF
    K4, M = qw.shape
    shifts = torch.tensor([0, 8, 16, 24], dtype=torch.int64)
    u = (qw[:, :, None] >> shifts) & 0xFF                      # (K/4, M, 4)
    u = u.permute(0, 2, 1).reshape(K4 * 4, M)                  # (K, M)
    q = (u - 128).to(torch.int8).t().contiguous()              # (M, K)
    s = scales.float().to(torch.bfloat16).t().contiguous()     # (M, n_groups)
    return q, s
