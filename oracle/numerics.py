"""Numeric conventions of the oracle (test infrastructure only).

* Rounding: fp32 -> bf16 is round-to-nearest-even, the rounding the reference applies at every
  operator boundary (iron/common/sequence.py:997-999) and in its kernels (conv_even,
  aie_kernels/aie2p/mv_int8_signed.cc:66). A wider value goes to bf16 through fp32, as torch's
  float64 -> bfloat16 cast does; the device kernels round the same way.
* Compute precision: every golden takes ``dt`` -- ``EXACT`` (float64) evaluates the reference's
  closed forms to within 2^-53, so the value rounded at a boundary is the correctly rounded one
  except with probability ~1e-9 per value; ``LITERAL`` (float32) is the reference golden as
  written in torch fp32 (used for the timed CPU baseline). Both round at the same boundaries.
* Scalars that the device receives as fp32 (eps, softmax scale) are used as their fp32 values.
"""

import numpy as np
import torch

EXACT = torch.float64
LITERAL = torch.float32


def f32(v: float) -> float:
    """The fp32 value of a Python float (what a float kernel parameter holds)."""
    return float(np.float32(v))


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE, through fp32) and return the bf16 tensor."""
    return x.float().to(torch.bfloat16)


def rbf(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 and return it as fp32 (a bf16 store then reload)."""
    return x.float().to(torch.bfloat16).float()


def bf16_bits(x: torch.Tensor) -> torch.Tensor:
    """bf16 tensor -> its int16 bit patterns (for bit-exact comparisons)."""
    return x.to(torch.bfloat16).contiguous().view(torch.int16)


def bf16_from_bits(bits: torch.Tensor) -> torch.Tensor:
    return bits.to(torch.int16).contiguous().view(torch.bfloat16)
