"""bf16 helpers of the oracle (test infrastructure only).

torch's fp32 -> bf16 conversion is round-to-nearest-even, the rounding the reference applies at
every operator boundary (iron/common/sequence.py:997-999) and in its kernels (conv_even,
aie_kernels/aie2p/mv_int8_signed.cc:66).
"""

import torch


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and return the bf16 tensor."""
    return x.to(torch.bfloat16)


def rbf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and return it as fp32 (the value a bf16 store then reload gives)."""
    return x.float().to(torch.bfloat16).float()


def bf16_bits(x: torch.Tensor) -> torch.Tensor:
    """bf16 tensor -> its int16 bit patterns (for bit-exact comparisons)."""
    return x.to(torch.bfloat16).contiguous().view(torch.int16)


def bf16_from_bits(bits: torch.Tensor) -> torch.Tensor:
    return bits.to(torch.int16).contiguous().view(torch.bfloat16)
