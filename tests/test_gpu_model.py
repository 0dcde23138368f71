"""Whole-model GPU parity: the Qwen3 decode chain (HIP) against the CPU oracle chain.

* tiny model: logits within tolerance of the CPU chain at every step, same argmax;
* dispatch modes: the graph-replayed ("fused") and eager ("separate") sequences give
  bit-identical logits (the reference checks the same across its dispatch modes,
  iron/tests/infrastructure/sequence.py:183-203);
* the device-resident greedy loop reproduces the host-driven loop token for token;
* compare mode raises on a planted wrong reference (sequence.py:284-324 in the reference tests);
* Qwen3-0.6B architecture, int8 G=32, bf16 LM head, KV prefilled to 2048 positions, 128 greedy
  steps: greedy-token agreement with the CPU chain >= 99% under teacher forcing, and at full size
  the persistent kernel's last-step logits and the K/V rows it appended are bit-identical to the
  exact (fp64) chain fed the same tokens; the same at a context past 2560 (every attention split
  walks two tiles) and at the checkpoint's group size 128 (check_cosine_int8.py:61-70 is the
  reference's own gate on the same chain).
"""

import pytest
import torch

from iron_amd.applications.qwen3_0_6b.qwen3_npu_int8 import Qwen3NPU
from iron_amd.applications.qwen3_0_6b.weights import (Qwen3Config, random_qwen3_weights,
                                                       synthetic_kv)
from iron_amd.common.test_utils import verify_buffer
from oracle.qwen3 import Qwen3CpuChain

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def tiny():
    cfg = Qwen3Config.tiny()
    return cfg, random_qwen3_weights(cfg, seed=99)


@pytest.mark.parametrize("kv_layout,lm_head", [("separate", "bf16"), ("interleaved", "int8")])
def test_tiny_model_matches_cpu_chain(kv_layout, lm_head):
    _say(f"tiny model kv_layout={kv_layout} lm_head={lm_head}")
    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=5, lm_head=lm_head)
    S = 128
    model = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, kv_layout=kv_layout, persistent=False)
    chain = Qwen3CpuChain(cfg, w, S)                       # exact (fp64) oracle
    literal = Qwen3CpuChain(cfg, w, S, dt=torch.float32)   # the golden as written (fp32)
    tok = 3
    for pos in range(8):
        g = model.step_token(tok, pos)
        lg = model.logits()
        lc = chain.step(tok, pos)
        ll = literal.step(tok, pos)
        # every op boundary is the correctly rounded value on both sides: identical logits
        assert torch.equal(lg.view(torch.int16), lc.view(torch.int16)), f"logits differ @{pos}"
        assert not verify_buffer(lg, f"logits@{pos}", ll, rel_tol=1e-2, abs_tol=5e-2)
        assert g == int(torch.argmax(lg.float())), "device argmax != argmax of device logits"
        assert g == Qwen3CpuChain.argmax(lc)
        tok = g


def test_dispatch_modes_bit_identical(tiny):
    _say("fused vs separate dispatch")
    cfg, w = tiny
    outs = []
    for dispatch in ("fused", "separate"):
        m = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, dispatch=dispatch, persistent=False)
        toks, logits = [], []
        tok = 11
        for pos in range(5):
            tok = m.step_token(tok, pos)
            toks.append(tok)
            logits.append(m.logits())
        outs.append((toks, torch.stack(logits)))
    assert outs[0][0] == outs[1][0]
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))


@pytest.mark.parametrize("persistent", [False, True])
def test_device_generate_matches_host_loop(tiny, persistent):
    _say(f"device generate vs host loop (persistent={persistent})")
    cfg, w = tiny
    prompt = [7, 19, 23, 5]
    n_new = 20
    a = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, persistent=persistent)
    dev_tokens = a.generate(prompt, n_new)
    # the loop's state advanced once per step: position, context length, RoPE row
    end, HD = len(prompt) - 1 + n_new, cfg.head_dim
    assert int(a.fc.params.tensor("k_cache_offset")[0]) == end
    assert int(a.fc.params.tensor("S_kv_eff")[0]) == end + 1
    row = a.fc.get_buffer("rope_row").torch_view(torch.bfloat16)[:HD]
    assert torch.equal(row.view(torch.int16), a.rope_table[end * HD:(end + 1) * HD].view(torch.int16))
    b = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, persistent=persistent)
    pos = 0
    for t in prompt[:-1]:
        b.step_token(t, pos)
        pos += 1
    host = []
    tok = prompt[-1]
    for _ in range(n_new):
        tok = b.step_token(tok, pos)
        pos += 1
        host.append(tok)
    assert dev_tokens == host
    # replaying again from a re-armed state gives the same tokens (graph replay is repeatable)
    a2 = a.generate(prompt, n_new)
    assert a2 == dev_tokens


def test_compare_mode_raises_on_wrong_reference(tiny, oracle_provider):
    """Plant a mistake in the oracle (CPU side): compare dispatch must raise."""
    from iron_amd.common.base import register_reference_provider
    from iron_amd.common.sequence import CompareDispatch, OperatorSequence
    from iron_amd.operators import RMSNorm

    _say("compare mode")
    op = RMSNorm(size=256, num_aie_columns=1, num_channels=1, tile_size=256, weighted=True,
                 epsilon=1e-6)
    seq = OperatorSequence("cmp", [(op, "x", "w", "y")], input_args=["x", "w"],
                           output_args=["y"], dispatch=CompareDispatch(1e-2, 1e-2))
    fc = seq.get_callable()
    fc.get_buffer("x").torch_view()[:256].copy_(torch.randn(256).to(torch.bfloat16))
    fc.get_buffer("w").torch_view()[:256].fill_(1.0)
    fc()  # correct reference: passes
    assert not any(s["mismatch"] for s in fc.last_step_stats)

    def wrong(op_, *inputs, **kw):
        return oracle_provider(op_, *inputs, **kw) * 1.5

    register_reference_provider(wrong)
    try:
        with pytest.raises(RuntimeError, match="deviates"):
            fc()
    finally:
        register_reference_provider(oracle_provider)


def test_reference_dispatch_matches_hip(tiny, oracle_provider):
    _say("reference dispatch vs hip on one layer step")
    from iron_amd.common.sequence import OperatorSequence
    from iron_amd.operators import GEMVInt8
    from iron_amd.operators.wire import pack_wire
    from oracle.gemv import rtn_quantize

    M, K = 512, 256
    op = GEMVInt8(M=M, K=K, tile_size_input=4, group_size=32, kernel_source="mv_int8_signed.cc")
    q, s = rtn_quantize(torch.randn(M, K) * 0.05, 32)
    wire = pack_wire(q, s, 4, "signed")
    x = torch.randn(K).to(torch.bfloat16)
    ys = []
    for dispatch in ("fused", "reference"):
        seq = OperatorSequence("g", [(op, "w", "x", "y")], input_args=["w", "x"],
                               output_args=["y"], dispatch=dispatch)
        fc = seq.get_callable()
        fc.get_buffer("w").torch_view(torch.uint8)[: wire.numel()].copy_(wire)
        fc.get_buffer("x").torch_view()[:K].copy_(x)
        fc()
        ys.append(fc.get_buffer("y").torch_view()[:M].cpu())
    assert not verify_buffer(ys[0], "y", ys[1], rel_tol=1e-2, abs_tol=1e-2)


@pytest.mark.parametrize("fuse_attention,kv_layout", [(True, "separate"), (False, "separate"),
                                                       (True, "interleaved")])
def test_compare_dispatch_runs_the_default_runlist(tiny, oracle_provider, fuse_attention,
                                                   kv_layout):
    """Qwen3NPU(dispatch=compare): every runlist entry of a decode step (QKV head + attention,
    or the fused QKVHeadAttention; the MLP; the final norm; the LM head's argmax) is checked
    against its CPU golden on the same inputs, with zero tolerance (exact arithmetic on both
    sides), over several positions (sequence.py:1002-1085 in the reference)."""
    from iron_amd.common.sequence import CompareDispatch

    _say(f"compare dispatch, fuse_attention={fuse_attention} kv_layout={kv_layout}")
    cfg, w = tiny
    m = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, kv_layout=kv_layout,
                 fuse_attention=fuse_attention, dispatch=CompareDispatch(0.0, 0.0))
    assert not m.persistent
    ref = Qwen3CpuChain(cfg, w, 64)
    tok = 13
    for pos in range(4):
        got = m.step_token(tok, pos)
        stats = m.fc.last_step_stats
        assert len(stats) == len(m.seq.runlist)
        assert not any(st["mismatch"] for st in stats), stats
        want = Qwen3CpuChain.argmax(ref.step(tok, pos))
        assert got == want
        tok = got


def test_compare_dispatch_catches_a_planted_attention_error(tiny, oracle_provider):
    """A mistake planted in the oracle's fused QKV-head + attention golden (CPU side) must make
    compare dispatch raise at that entry."""
    from iron_amd.common.base import register_reference_provider
    from iron_amd.common.sequence import CompareDispatch

    _say("compare dispatch, planted attention error")
    cfg, w = tiny
    m = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, dispatch=CompareDispatch(1e-2, 1e-2))

    def planted(op_, *inputs, **kw):
        out = oracle_provider(op_, *inputs, **kw)
        if type(op_).__name__ == "QKVHeadAttention":
            out = out.clone()
            out[5] = out[5].float() + 1.0          # one output element off by 1.0
        return out

    register_reference_provider(planted)
    try:
        with pytest.raises(RuntimeError, match="QKVHeadAttention"):
            m.step_token(3, 0)
    finally:
        register_reference_provider(oracle_provider)


def test_reference_dispatch_model_matches_hip(tiny, oracle_provider):
    """Qwen3NPU(dispatch=reference) runs the whole runlist through the CPU goldens (KV appends
    included, positions from the runtime parameters); its tokens and logits equal the HIP
    path's bit for bit."""
    _say("reference dispatch, whole model")
    cfg, w = tiny
    hip = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, persistent=False)
    cpu = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, dispatch="reference")
    assert not cpu.persistent
    a = b = 21
    for pos in range(5):
        a = hip.step_token(a, pos)
        b = cpu.step_token(b, pos)
        assert a == b, f"tokens differ at {pos}"
        assert torch.equal(hip.logits().view(torch.int16), cpu.logits().view(torch.int16))
    with pytest.raises(ValueError):
        Qwen3NPU(config=cfg, weights=w, max_seq_len=64, dispatch="reference", persistent=True)


def _bits(t):
    return t.contiguous().view(torch.int16)


def _teacher_forced_chain(cfg, w, S, kv_init, prompt, toks, start_pos):
    """The exact CPU chain run over the prompt and then fed the GPU's tokens: returns the chain,
    the number of steps whose argmax equals the GPU's token, the top1-top2 margins and the last
    step's logits (the ones the GPU's last launch computed)."""
    chain = Qwen3CpuChain(cfg, w, S, kv_init=kv_init)
    pos = start_pos
    for t in prompt[:-1]:
        chain.step(t, pos)
        pos += 1
    agree, margins, lc = 0, [], None
    tok = prompt[-1]
    for i in range(len(toks)):
        lc = chain.step(tok, pos)
        top = torch.topk(lc.float(), 2).values
        margins.append(float(top[0] - top[1]))
        agree += int(Qwen3CpuChain.argmax(lc) == toks[i])
        tok = toks[i]
        pos += 1
    return chain, agree, margins, lc


def _assert_full_size_bits(model, chain, lc, start_pos, end, layers=(0, 13, 27)):
    """The GPU's last logits and its appended K/V rows [start_pos, end) of a few layers equal the
    exact chain's bit for bit."""
    assert torch.equal(_bits(model.logits()), _bits(lc)), "last-step logits differ from the oracle"
    for i in layers:
        kg, vg = (c[:, start_pos:end].cpu() for c in model.kv_caches(i))
        assert torch.equal(_bits(kg), _bits(chain.k_cache[i, :, start_pos:end])), f"K rows, layer {i}"
        assert torch.equal(_bits(vg), _bits(chain.v_cache[i, :, start_pos:end])), f"V rows, layer {i}"


@pytest.mark.slow
def test_qwen3_0_6b_greedy_agreement():
    """BASELINE config 4 shape at full size; agreement measured under teacher forcing."""
    cfg = Qwen3Config.qwen3_0_6b()
    P0, n_prompt, n_new = 1984, 64, 128
    S = P0 + n_prompt + n_new
    _say(f"qwen3-0.6b: weights G={cfg.group_size}, KV prefill {P0}+{n_prompt}, {n_new} steps")
    w = random_qwen3_weights(cfg, seed=2024, device="cuda")
    k0, v0 = synthetic_kv(cfg, P0, seed=7)
    model = Qwen3NPU(config=cfg, weights=w, max_seq_len=S)
    model.load_kv(k0, v0)
    gen = torch.Generator().manual_seed(64)
    prompt = torch.randint(0, cfg.vocab_size, (n_prompt,), generator=gen).tolist()
    toks = model.generate(prompt, n_new, start_pos=P0)
    assert len(toks) == n_new
    assert model.persistent and model.fold_lm_head, "config 4 runs the one-launch token"
    _say("qwen3-0.6b: exact CPU chain (teacher forced)")
    chain, agree, margins, lc = _teacher_forced_chain(cfg, w, S, (k0, v0), prompt, toks, P0)
    rate = agree / n_new
    print(f"greedy agreement {agree}/{n_new} = {rate:.4f}; top1-top2 margin min "
          f"{min(margins):.4g} median {sorted(margins)[len(margins) // 2]:.4g}", flush=True)
    assert rate >= 0.99
    _assert_full_size_bits(model, chain, lc, P0, P0 + n_prompt + n_new - 1)


@pytest.mark.slow
@pytest.mark.parametrize("group_size,P0,n_prompt,n_new", [
    (32, 2700, 4, 20),    # past 80 * 32 = 2560 positions: every attention split walks two tiles
    (128, 600, 4, 20),    # the checkpoint's group (qwen3_npu_int8.py:391)
])
def test_qwen3_0_6b_persistent_bit_exact(group_size, P0, n_prompt, n_new):
    """Full Qwen3-0.6B shape through the one-launch token (persistent kernel with the folded
    bf16 LM head; 20 steps = one 16-launch graph replay + four single replays): every greedy token
    is the exact chain's argmax, and the last logits and the appended K/V rows are bit-identical."""
    cfg = Qwen3Config.qwen3_0_6b(group_size=group_size)
    S = (P0 + n_prompt + n_new + 63) // 64 * 64
    _say(f"qwen3-0.6b persistent vs oracle: G={group_size}, KV {P0}, prompt {n_prompt}, "
         f"{n_new} tokens")
    w = random_qwen3_weights(cfg, seed=2024 + group_size, device="cuda")
    k0, v0 = synthetic_kv(cfg, P0, seed=7)
    model = Qwen3NPU(config=cfg, weights=w, max_seq_len=S)
    assert model.persistent and model.fold_lm_head
    model.load_kv(k0, v0)
    prompt = torch.randint(0, cfg.vocab_size, (n_prompt,),
                           generator=torch.Generator().manual_seed(65)).tolist()
    toks = model.generate(prompt, n_new, start_pos=P0)
    _say(f"qwen3-0.6b G={group_size}: exact CPU chain (teacher forced)")
    chain, agree, margins, lc = _teacher_forced_chain(cfg, w, S, (k0, v0), prompt, toks, P0)
    print(f"G={group_size}: argmax agreement {agree}/{n_new}; margin min {min(margins):.4g}",
          flush=True)
    assert agree == n_new
    _assert_full_size_bits(model, chain, lc, P0, P0 + n_prompt + n_new - 1)
