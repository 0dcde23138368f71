"""Fused-block goldens: the decode QKV head and the SwiGLU MLP (test infrastructure only).

Follows:
  * QKV head -- iron/operators/qkv_head_dp/reference.py:13-33: hn = RMSNorm_w(cur, n_in) (bf16);
    raw = bf16(W @ hn); q/k heads: RoPE(bf16(RMSNorm_w(head, n_qn|n_kn))); v = raw (bf16), with
    the int8 weight dequantized exactly (op_ours.py:515-541);
  * SwiGLU MLP -- iron/operators/swiglu_mlp_dp/reference.py:8-67 with the exact dequant of
    op_ours.py:543-582: fuse_o a = bf16(Wo @ cx); x1 = cur + a (fp32); hf = RMSNorm_w(x1) (fp32);
    g, u GEMVs; stable sigmoid; gh = silu(g) * u (fp32); nxt = bf16(x1 + Wd @ gh). The fp32
    values x1, hf and gh are where the golden holds fp32 tensors; those are its boundaries.
Every function evaluates in ``dt`` (EXACT = fp64 or LITERAL = fp32) between those boundaries.
"""

import torch

from .gemv import dequant_f, gemv
from .norms import rms_norm, rope
from .numerics import EXACT


def qkv_head(cur, n_in, q8, s, n_qn, n_kn, ang, Hq: int, Hkv: int, HD: int, eps: float,
             W=None, dt=EXACT):
    """cur (B,D) bf16 -> (q (B,Hq*HD), k (B,Hkv*HD), v (B,Hkv*HD)) bf16. ang: (B,HD) or (HD,).

    ``W`` optionally supplies the dequantized weight (any float dtype) instead of (q8, s)."""
    cur = cur.reshape(-1, cur.shape[-1])
    B = cur.shape[0]
    QD, KVD = Hq * HD, Hkv * HD
    hn = rms_norm(cur, n_in, eps, dt=dt)                             # (B, D) bf16
    Wd = dequant_f(q8, s, dt) if W is None else W
    raw = gemv(Wd, hn, dt).float().to(torch.bfloat16)                # (B, QD + 2 KVD)
    ang = ang.reshape(-1, HD)
    if ang.shape[0] == 1 and B > 1:
        ang = ang.expand(B, HD)
    qs, ks = [], []
    for b in range(B):
        qn = rms_norm(raw[b, :QD].reshape(Hq, HD), n_qn, eps, dt=dt)
        kn = rms_norm(raw[b, QD:QD + KVD].reshape(Hkv, HD), n_kn, eps, dt=dt)
        qs.append(rope(qn, ang[b:b + 1], dt=dt).reshape(QD))
        ks.append(rope(kn, ang[b:b + 1], dt=dt).reshape(KVD))
    return torch.stack(qs), torch.stack(ks), raw[:, QD + KVD:].clone()


def _sigmoid_stable(g: torch.Tensor) -> torch.Tensor:
    pos = g >= 0
    e = torch.exp(torch.where(pos, -g, g))
    return torch.where(pos, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu_mlp(cur, a_or_cx, n_pf, wg, wu, wd, eps: float, wo=None, Wf=None, dt=EXACT):
    """One or more rows. wg/wu/wd/wo: (q, s) tuples, or Wf={'g','u','d','o'} dequantized.

    Returns (nxt bf16 (B,D), a bf16 (B,D))."""
    cur = cur.reshape(-1, cur.shape[-1])
    Wf = Wf or {}
    Wg = Wf["g"] if "g" in Wf else dequant_f(*wg, dt)
    Wu = Wf["u"] if "u" in Wf else dequant_f(*wu, dt)
    Wd = Wf["d"] if "d" in Wf else dequant_f(*wd, dt)
    x_in = a_or_cx.reshape(cur.shape[0], -1)
    if wo is not None or "o" in Wf:
        Wo = Wf["o"] if "o" in Wf else dequant_f(*wo, dt)
        a = gemv(Wo, x_in, dt).float().to(torch.bfloat16)
    else:
        a = x_in.to(torch.bfloat16)
    x1 = cur.float() + a.float()                                     # fp32, as in the golden
    hf = rms_norm(x1, n_pf, eps, out_bf16=False, dt=dt)              # fp32
    g = gemv(Wg, hf, dt)
    u = gemv(Wu, hf, dt)
    gh = ((g * _sigmoid_stable(g)) * u).float()                      # fp32
    d = gemv(Wd, gh, dt)
    nxt = (x1.to(dt) + d).float().to(torch.bfloat16)
    return nxt, a
