"""RMSNorm and RoPE goldens (test infrastructure only).

Follows:
  * weighted RMSNorm -- closed form of iron/operators/rms_norm/reference.py:8-17,
    ``x / sqrt(mean(x^2) + eps) * w``, in the kernel's operation order
    (aie_kernels/aie2p/rms_norm.cc:83-147: inv = 1/sqrt(mean + eps), x * inv, then * w), one
    rounding at the output;
  * RoPE (TWO_HALVES) -- iron/operators/rope/reference.py:118-154: interleaved [cos_i, sin_i]
    angle row, y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin, bf16 result; one angle row per block of
    consecutive rows (rope_reference_convention.py:21-64);
  * angle table -- iron/applications/qwen3_0.6b/qwen3_npu_int8.py:580-591;
  * RoPE with head_dim-long cos / sin tables -- iron/operators/qk_norm_rope/reference.py:26-33
    (rotate_half; the second half uses its own table entries);
  * RoPE, interleaved pairs -- iron/operators/rope/reference.py:94-112 (method_type 1) and
    aie_kernels/generic/rope.cc (pairs (2i, 2i + 1));
  * fused QK-norm + RoPE + V copy -- aie_kernels/aie2p/qk_norm_rope.cc:42-108 (the normalised
    head is stored as bf16 before the rotation) and iron/operators/qk_norm_rope/reference.py:19-40
    (which rounds once, at the end).
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


def rope_halves(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """rotate_half RoPE of rows of ``x`` (..., HD) with HD-long ``cos`` / ``sin`` tables: for
    d < m = HD/2, y_d = x_d cos_d - x_{d+m} sin_d; for d >= m, y_d = x_d cos_d + x_{d-m} sin_d.
    Under the duplicated-half convention (cos_{d+m} == cos_d) this is ``rope`` with the angle row
    interleave(cos[:m], sin[:m]). bf16 result."""
    HD = x.shape[-1]
    m = HD // 2
    xf = x.to(dt)
    c, s = cos.to(dt), sin.to(dt)
    x1, x2 = xf[..., :m], xf[..., m:]
    y = torch.cat([x1 * c[:m] - x2 * s[:m], x2 * c[m:] + x1 * s[m:]], dim=-1)
    return y.float().to(torch.bfloat16)


def rope_interleaved(x: torch.Tensor, angles: torch.Tensor, dt=EXACT) -> torch.Tensor:
    """Interleaved-pair RoPE of rows of ``x`` (..., HD) with interleaved [cos_i, sin_i] angle
    rows (A, HD), rows sharing angle rows as in ``rope``: y_{2i} = x_{2i} cos_i - x_{2i+1} sin_i,
    y_{2i+1} = x_{2i} sin_i + x_{2i+1} cos_i. bf16 result."""
    HD = x.shape[-1]
    xf = x.reshape(-1, HD).to(dt)
    rows = xf.shape[0]
    ang = angles.reshape(-1, HD)
    cos = ang[:, 0::2].to(dt)
    sin = ang[:, 1::2].to(dt)
    if cos.shape[0] != rows:
        rep = rows // cos.shape[0]
        cos = cos.repeat_interleave(rep, dim=0)
        sin = sin.repeat_interleave(rep, dim=0)
    xe, xo = xf[:, 0::2], xf[:, 1::2]
    y = torch.empty_like(xf)
    y[:, 0::2] = xe * cos - xo * sin
    y[:, 1::2] = xe * sin + xo * cos
    return y.float().to(torch.bfloat16).reshape(x.shape)


def qk_norm_rope(qkv: torch.Tensor, scratch: torch.Tensor, n_qk_heads: int, n_v_heads: int,
                 head_dim: int, eps: float, round_norm: bool = True, dt=EXACT) -> torch.Tensor:
    """Fused decode QK-norm + RoPE + V copy of one flat QKV vector [Q | K | V] (bf16) with
    scratch = [gamma (n_qk_heads x head_dim) | cos (head_dim) | sin (head_dim)]: each of the
    n_qk_heads Q/K heads is RMS-normalised with its own gamma row and rotated (``rope_halves``),
    the n_v_heads V heads are copied. ``round_norm``: the normalised head is rounded to bf16
    before the rotation (the kernel); False keeps it exact (the reference's golden)."""
    HD = head_dim
    qk = qkv[: n_qk_heads * HD].reshape(n_qk_heads, HD)
    v = qkv[n_qk_heads * HD: (n_qk_heads + n_v_heads) * HD]
    gamma = scratch[: n_qk_heads * HD].reshape(n_qk_heads, HD)
    cos = scratch[n_qk_heads * HD: n_qk_heads * HD + HD]
    sin = scratch[n_qk_heads * HD + HD: n_qk_heads * HD + 2 * HD]
    y = rms_norm(qk, gamma, eps, out_bf16=round_norm, dt=dt)
    if not round_norm:
        y = y.to(dt)
    return torch.cat([rope_halves(y, cos, sin, dt=dt).reshape(-1), v.to(torch.bfloat16)])
