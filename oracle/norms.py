"""RMSNorm and RoPE goldens (test infrastructure only).

Follows:
  * weighted RMSNorm -- closed form of iron/operators/rms_norm/reference.py:8-17,
    ``x / sqrt(mean(x^2) + eps) * w``, in the kernel's operation order
    (aie_kernels/aie2p/rms_norm.cc:83-147: inv = 1/sqrt(mean + eps), x * inv, then * w), one
    rounding at the output;
  * RoPE (TWO_HALVES) -- iron/operators/rope/reference.py:118-154: interleaved [cos_i, sin_i]
    angle row, y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin, bf16 result; one angle row per block of
    consecutive rows (rope_reference_convention.py:21-64);
  * angle table -- iron/applications/qwen3_0.6b/qwen3_npu_int8.py:580-591.
"""

import torch

from .numerics import EXACT, f32


def rms_norm(x: torch.Tensor, w: torch.Tensor | None, eps: float, out_bf16: bool = True,
             dt=EXACT):
    """Row-wise weighted RMSNorm over the last dim in ``dt``; output bf16 or fp32."""
    xd = x.to(dt)
    inv = 1.0 / torch.sqrt((xd * xd).mean(dim=-1, keepdim=True) + f32(eps))
    y = xd * inv
    if w is not None:
        y = y * w.to(dt)
    return y.float().to(torch.bfloat16) if out_bf16 else y.float()


def rope(x: torch.Tensor, angles: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """Two-halves RoPE of rows of ``x`` (..., HD) with interleaved angle rows (A, HD).

    Row r of the flattened x uses angle row r // (rows / A) (the device's block-major
    convention); A == 1 applies one row to all. With bf16 inputs every product and sum is exact
    in fp32 already, so ``dt`` only matters for wider inputs."""
    HD = x.shape[-1]
    half = HD // 2
    xf = x.reshape(-1, HD).to(dt)
    rows = xf.shape[0]
    ang = angles.reshape(-1, HD)
    cos = ang[:, 0::2].to(dt)
    sin = ang[:, 1::2].to(dt)
    if cos.shape[0] != rows:
        rep = rows // cos.shape[0]
        cos = cos.repeat_interleave(rep, dim=0)
        sin = sin.repeat_interleave(rep, dim=0)
    x1, x2 = xf[:, :half], xf[:, half:]
    y = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
    return y.float().to(torch.bfloat16).reshape(x.shape)


def rope_angle_table(max_pos: int, head_dim: int, theta: float) -> torch.Tensor:
    """(max_pos, head_dim) bf16 rows of interleaved [cos_i, sin_i], i < head_dim/2."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos = emb.cos().to(torch.bfloat16)[:, :half]
    sin = emb.sin().to(torch.bfloat16)[:, :half]
    return torch.stack([cos, sin], dim=-1).reshape(max_pos, head_dim)
