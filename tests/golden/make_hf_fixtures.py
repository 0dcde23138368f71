#!/usr/bin/env python3
"""Write tests/golden/qwen3_tiny_hf_logits.safetensors: the Hugging Face fp32 logits of the tiny
seeded Qwen3 GPTQ checkpoint (tests/golden/qwen3_gptq_fixture.py) over its prompt, with the
SHA-256 of the weights they belong to. Needs transformers (random-init model from an explicit
config; nothing is downloaded). Run from the repository root:
    python tests/golden/make_hf_fixtures.py
"""

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE))

import torch  # noqa: E402
from safetensors.torch import save_file  # noqa: E402

import qwen3_gptq_fixture as fx  # noqa: E402


def main():
    t = fx.tensors()
    logits = fx.hf_logits(t)
    save_file({"logits": logits.contiguous(), "prompt": torch.tensor(fx.PROMPT)},
              str(fx.FIXTURE), metadata={"weights_sha256": fx.digest(t),
                                         "source": "transformers Qwen3ForCausalLM, fp32, eager"})
    print(f"wrote {fx.FIXTURE} ({logits.shape[0]} x {logits.shape[1]} logits)")


if __name__ == "__main__":
    main()
