"""The GPTQ checkpoint path (qwen3_npu_int8.py:144-181, 350-379) and the Hugging Face logit gate
(check_cosine_int8.py:29-70), on a tiny seeded checkpoint (tests/golden/qwen3_gptq_fixture.py):

* CPU: the loader unpacks the checkpoint exactly (zero point 128, fp16 -> bf16 scales, the
  [q; k; v] row order of the fused QKV wire); the CPU oracle chain over the loaded weights passes
  the reference's gate (cosine > 0.99, argmax match) against the committed transformers logits
  at every prompt position -- an independent, third-party pin of the whole oracle chain;
* GPU: Qwen3NPU(weights_path=...) -- persistent kernel and runlist -- passes the same gate and
  equals the exact oracle chain bit for bit.
"""

import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

import qwen3_gptq_fixture as fx  # noqa: E402

from iron_amd.applications.qwen3_0_6b.weights import load_gptq_checkpoint  # noqa: E402
from oracle.qwen3 import Qwen3CpuChain  # noqa: E402


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    path = tmp_path_factory.mktemp("gptq") / "model.safetensors"
    digest = fx.make_checkpoint(path)
    logits, want = fx.load_fixture()
    assert digest == want, "the seeded checkpoint no longer matches the committed HF logits"
    return path, logits


def gate(logits: torch.Tensor, hf: torch.Tensor, what: str):
    """The reference's check (check_cosine_int8.py:61-70): cosine > 0.99, same argmax."""
    cos = torch.nn.functional.cosine_similarity(logits.float(), hf.float(), dim=0).item()
    assert cos > 0.99, f"{what}: cosine {cos:.6f}"
    assert int(logits.float().argmax()) == int(hf.argmax()), f"{what}: argmax differs"
    return cos


def test_loader_unpacks_exactly(ckpt):
    path, _ = ckpt
    t = fx.tensors()
    w = load_gptq_checkpoint(path, fx.config(), "bf16")
    for i, L in enumerate(w["layers"]):
        pre = f"model.layers.{i}"
        for name, key in (("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"),
                          ("up", "mlp.up_proj"), ("down", "mlp.down_proj")):
            q, s = L[name]
            qw, sc = t[f"{pre}.{key}.qweight"], t[f"{pre}.{key}.scales"]
            want = fx._dequant(qw, sc.float().to(torch.bfloat16).float().to(torch.float16))
            got = q.float() * s.float().repeat_interleave(fx.G, dim=1)
            assert torch.equal(got, want), f"layer {i} {name}"
            assert torch.equal(s, sc.float().to(torch.bfloat16).t())
        q, s = L["qkv"]
        rows = [fx._dequant(t[f"{pre}.self_attn.{p}_proj.qweight"],
                            t[f"{pre}.self_attn.{p}_proj.scales"]) for p in "qkv"]
        assert q.shape == (fx.HQ * fx.HD + 2 * fx.HKV * fx.HD, fx.D)
        # q * s is within one fp16->bf16 scale rounding of the checkpoint's own dequant
        got = q.float() * s.float().repeat_interleave(fx.G, dim=1)
        assert torch.allclose(got, torch.cat(rows), rtol=2 ** -8, atol=0)
    with pytest.raises(ValueError, match="group"):
        load_gptq_checkpoint(path, fx.config().__class__(**{**fx.config().__dict__,
                                                            "group_size": 32}), "bf16")


def test_oracle_chain_passes_the_hf_gate(ckpt):
    path, hf = ckpt
    cfg = fx.config()
    chain = Qwen3CpuChain(cfg, load_gptq_checkpoint(path, cfg, "bf16"), 64)
    for pos, tok in enumerate(fx.PROMPT):
        gate(chain.step(tok, pos), hf[pos], f"oracle chain pos {pos}")


@pytest.mark.gpu
@pytest.mark.parametrize("persistent", [None, False])
def test_qwen3npu_from_checkpoint_passes_the_hf_gate(ckpt, persistent):
    from iron_amd.applications.qwen3_0_6b.qwen3_npu_int8 import Qwen3NPU

    path, hf = ckpt
    cfg = fx.config()
    print(f"[case] Qwen3NPU(weights_path) persistent={persistent}", flush=True)
    model = Qwen3NPU(path, config=cfg, max_seq_len=64, persistent=persistent)
    if persistent is None:
        assert model.persistent, "the tiny geometry has a persistent kernel"
    chain = Qwen3CpuChain(cfg, load_gptq_checkpoint(path, cfg, "bf16"), 64)
    for pos, tok in enumerate(fx.PROMPT):
        got = model.step_token(tok, pos)
        lg = model.logits()
        cos = gate(lg, hf[pos], f"device pos {pos}")
        want = chain.step(tok, pos)
        assert torch.equal(lg.view(torch.int16), want.view(torch.int16)), f"pos {pos}"
        assert got == int(hf[pos].argmax())
    print(f"last position cosine vs HF fp32: {cos:.6f}", flush=True)
