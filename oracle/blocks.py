"""Fused-block goldens: the decode QKV head and the SwiGLU MLP (test infrastructure only).

Follows:
  * QKV head -- iron/operators/qkv_head_dp/reference.py:13-33: hn = RMSNorm_w(cur, n_in);
    raw = bf16(W @ hn); q/k heads: RoPE(RMSNorm_w(head, n_qn|n_kn)); v = raw (bf16), with the
    int8 weight dequantized exactly in fp32 (op_ours.py:515-541) and the norm/RoPE numerics of
    oracle.norms;
  * SwiGLU MLP -- iron/operators/swiglu_mlp_dp/reference.py:8-67 (fp32 x1 = cur + a,
    hf = RMSNorm_w(x1), g/u GEMVs, stable sigmoid, gh = silu(g) * u, nxt = bf16(x1 + Wd @ gh);
    fuse_o: a = bf16(Wo @ cx) first) with exact fp32 dequant (op_ours.py:543-582).
"""

import torch

from .gemv import dequant_f32
from .norms import rms_norm, rope


def qkv_head(cur, n_in, q8, s, n_qn, n_kn, ang, Hq: int, Hkv: int, HD: int, eps: float,
             W32: torch.Tensor | None = None):
    """cur (B,D) bf16 -> (q (B,Hq*HD), k (B,Hkv*HD), v (B,Hkv*HD)) bf16. ang: (B,HD) or (HD,)."""
    cur = cur.reshape(-1, cur.shape[-1])
    B = cur.shape[0]
    QD, KVD = Hq * HD, Hkv * HD
    hn = rms_norm(cur, n_in, eps)                                    # (B, D) bf16
    W = dequant_f32(q8, s) if W32 is None else W32
    raw = (hn.float() @ W.t()).to(torch.bfloat16)                    # (B, QD + 2 KVD)
    ang = ang.reshape(-1, HD)
    if ang.shape[0] == 1 and B > 1:
        ang = ang.expand(B, HD)
    qs, ks = [], []
    for b in range(B):
        qn = rms_norm(raw[b, :QD].reshape(Hq, HD), n_qn, eps)
        kn = rms_norm(raw[b, QD:QD + KVD].reshape(Hkv, HD), n_kn, eps)
        qs.append(rope(qn, ang[b:b + 1]).reshape(QD))
        ks.append(rope(kn, ang[b:b + 1]).reshape(KVD))
    return torch.stack(qs), torch.stack(ks), raw[:, QD + KVD:].clone()


def _sigmoid_stable(g: torch.Tensor) -> torch.Tensor:
    pos = g >= 0
    e = torch.exp(torch.where(pos, -g, g))
    return torch.where(pos, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu_mlp(cur, a_or_cx, n_pf, wg, wu, wd, eps: float, wo=None, Wf=None):
    """One or more rows. wg/wu/wd/wo: (q, s) tuples (or use Wf={'g','u','d','o'} fp32).

    Returns (nxt bf16 (B,D), a bf16 (B,D))."""
    cur = cur.reshape(-1, cur.shape[-1]).float()
    Wf = Wf or {}
    Wg = Wf.get("g") if "g" in Wf else dequant_f32(*wg)
    Wu = Wf.get("u") if "u" in Wf else dequant_f32(*wu)
    Wd = Wf.get("d") if "d" in Wf else dequant_f32(*wd)
    x_in = a_or_cx.reshape(cur.shape[0], -1)
    if wo is not None or "o" in Wf:
        Wo = Wf.get("o") if "o" in Wf else dequant_f32(*wo)
        a = (x_in.float() @ Wo.t()).to(torch.bfloat16)
    else:
        a = x_in.to(torch.bfloat16)
    x1 = cur + a.float()
    hf = rms_norm(x1, n_pf, eps, out_bf16=False)
    g = hf @ Wg.t()
    u = hf @ Wu.t()
    gh = g * _sigmoid_stable(g) * u
    nxt = (x1 + gh @ Wd.t()).to(torch.bfloat16)
    return nxt, a
