"""The persistent whole-token decode kernel (iron_decode_persistent) on the GPU.

The kernel runs every layer of a token with the arithmetic of the per-operator entry points
(iron_qkv_attn + iron_swiglu_mlp, exact fp64 accumulation), so its results must be identical:

* tiny model: logits bit-identical to the exact CPU oracle chain (oracle/qwen3.py) at every step,
  for the separate and the reference's interleaved KV layouts, bf16 and int8 LM heads;
* the same model through the runlist (one HIP graph of per-operator kernels) and through the
  persistent kernel: identical logits, tokens and KV-cache rows;
* contexts past one attention tile per split (a split covers ceil(ctx / NS) positions and a tile
  80, so one tile holds up to 80 * NS: 10240 for the tiny shape, NS = 128, and 2560 for Qwen3-0.6B,
  NS = 32): the tiny model at context ~11000 against the exact CPU chain and the runlist, and the
  Qwen3-0.6B architecture with the KV cache prefilled to 2700 positions, whose device greedy loop
  (graph-captured persistent launches) gives the same tokens and caches as the runlist path;
* the generation entry point (iron_decode_persistent_gen) keeps its token log within its length
  while the step counter, position and context length advance every token.
"""

import pytest
import torch

from iron_amd.applications.qwen3_0_6b.qwen3_npu_int8 import Qwen3NPU
from iron_amd.applications.qwen3_0_6b.weights import (Qwen3Config, random_qwen3_weights,
                                                       synthetic_kv)
from oracle.qwen3 import Qwen3CpuChain

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("kv_layout,lm_head", [("separate", "bf16"), ("interleaved", "int8")])
def test_persistent_tiny_matches_cpu_chain(kv_layout, lm_head):
    _say(f"persistent tiny kv_layout={kv_layout} lm_head={lm_head}")
    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=5, lm_head=lm_head)
    S = 128
    model = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, kv_layout=kv_layout, persistent=True)
    assert model.persistent
    chain = Qwen3CpuChain(cfg, w, S)
    tok = 3
    for pos in range(8):
        g = model.step_token(tok, pos)
        lg = model.logits()
        lc = chain.step(tok, pos)
        assert torch.equal(_bits(lg), _bits(lc)), f"logits differ from the oracle @{pos}"
        assert g == Qwen3CpuChain.argmax(lc)
        tok = g
    assert model.persistent_errors() == 0


def test_persistent_gen_short_log():
    """iron_decode_persistent_gen called step by step: a token log shorter than the run keeps its
    first entries and is never written past its length, the step counter and the position still
    advance every token, and the tokens equal the device greedy loop's."""
    _say("persistent generation entry point, 6 steps into a 3-entry token log")
    from iron_amd.applications.qwen3_0_6b.qwen3_npu_int8 import _decode_key

    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=5)
    S, n = 64, 6
    want = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=True).generate([3], n)
    # the two-launch form (layers kernel, then iron_lm_head), driven by hand
    m = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=True, fold_lm_head=False)
    m.start_generation(3, 0)
    gs = m._gen_state()
    log = torch.full((8,), -7, dtype=torch.int32, device="cuda")
    keys = m.fc.get_buffer("argmax_key").torch_view(torch.int64)
    short = {"tokens": gs["tokens"], "log": log[:3], "step": gs["step"]}
    for _ in range(n):
        m.persistent_gen_launch(keys, short)
        m.lm_head_launch()
    torch.cuda.synchronize()
    assert m.persistent_errors() == 0
    assert int(gs["step"].item()) == n
    # step s logs the token it consumed: the armed 3, then the generated ones
    assert log.cpu().tolist() == [3] + want[:2] + [-7] * 5
    assert int(gs["tokens"].item()) == want[n - 2]
    assert _decode_key(int(keys[0].item())) == want[n - 1]
    assert int(m.fc.params.tensor("k_cache_offset")[0]) == n
    assert int(m.fc.params.tensor("S_kv_eff")[0]) == n + 1


def test_persistent_matches_runlist_tiny_prefilled():
    """Prefilled context (several tiles, several splits) through both execution paths."""
    _say("persistent vs runlist, tiny, prefilled KV")
    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=17)
    S, P0 = 512, 300
    k0, v0 = synthetic_kv(cfg, P0, seed=3)
    runs = []
    for persistent in (False, True):
        m = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=persistent)
        m.load_kv(k0, v0)
        toks, logits = [], []
        tok = 41
        for pos in range(P0, P0 + 6):
            tok = m.step_token(tok, pos)
            toks.append(tok)
            logits.append(m.logits())
        caches = [tuple(c[:, : P0 + 6].cpu() for c in m.kv_caches(i)) for i in range(cfg.n_layers)]
        runs.append((toks, torch.stack(logits), caches))
    (ta, la, ca), (tb, lb, cb) = runs
    assert ta == tb
    assert torch.equal(_bits(la), _bits(lb))
    for i in range(cfg.n_layers):
        assert torch.equal(_bits(ca[i][0]), _bits(cb[i][0])), f"K cache of layer {i} differs"
        assert torch.equal(_bits(ca[i][1]), _bits(cb[i][1])), f"V cache of layer {i} differs"


def test_persistent_multi_tile_context_tiny():
    """Context 11000 > 80 * NS = 10240: every split walks two tiles (the in-loop K/V loads and
    the rescale of the running maximum, sum and output); logits equal the exact CPU chain and
    the runlist path, and the appended K/V rows equal the runlist's."""
    cfg = Qwen3Config.tiny()
    P0, n = 11000, 3
    S = 11072
    _say(f"persistent multi-tile: tiny, KV prefilled to {P0}, {n} steps")
    w = random_qwen3_weights(cfg, seed=23)
    k0, v0 = synthetic_kv(cfg, P0, seed=9)
    chain = Qwen3CpuChain(cfg, w, S, kv_init=(k0, v0))
    runs = []
    for persistent in (True, False):
        m = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=persistent)
        assert m.persistent == persistent
        m.load_kv(k0, v0)
        toks, logits = [], []
        tok = 77
        for pos in range(P0, P0 + n):
            tok = m.step_token(tok, pos)
            toks.append(tok)
            logits.append(m.logits())
        caches = [tuple(c[:, P0:P0 + n].cpu() for c in m.kv_caches(i)) for i in range(cfg.n_layers)]
        runs.append((toks, logits, caches))
        if persistent:
            assert m.persistent_errors() == 0
    (ta, la, ca), (tb, lb, cb) = runs
    tok = 77
    for i, pos in enumerate(range(P0, P0 + n)):
        lc = chain.step(tok, pos)
        assert torch.equal(_bits(la[i]), _bits(lc)), f"persistent logits differ from the oracle @{pos}"
        tok = ta[i]
    assert ta == tb
    for i in range(cfg.n_layers):
        assert torch.equal(_bits(ca[i][0]), _bits(cb[i][0])) and torch.equal(_bits(ca[i][1]),
                                                                             _bits(cb[i][1]))


@pytest.mark.parametrize("kv_layout", ["separate", "interleaved"])
def test_folded_lm_head_generation(kv_layout):
    """The whole greedy step in one launch (layers + final norm + bf16 LM head + argmax,
    iron_decode_persistent_gen with lm_head): the same tokens and bit-identical final logits as
    the two-launch loop (layers, then iron_lm_head) and as the exact CPU chain fed those tokens;
    the key slots alternate by epoch across re-armed runs."""
    _say(f"folded LM head, tiny, {kv_layout}")
    cfg = Qwen3Config.tiny()
    w = random_qwen3_weights(cfg, seed=31)
    # 20 steps: one replay of the 16-launch graph, then four single-launch replays
    prompt, n_new = [9, 4, 33], 20
    runs = []
    for fold in (True, False):
        m = Qwen3NPU(config=cfg, weights=w, max_seq_len=64, kv_layout=kv_layout,
                     persistent=True, fold_lm_head=fold)
        assert m.fold_lm_head == fold
        toks = m.generate(prompt, n_new)
        runs.append((toks, m.logits()))
        again = m.generate(prompt, n_new)          # re-armed at a later epoch: same tokens
        assert again == toks
        assert m.persistent_errors() == 0
    (ta, la), (tb, lb) = runs
    assert ta == tb
    assert torch.equal(_bits(la), _bits(lb))
    chain = Qwen3CpuChain(cfg, w, 64)
    pos = 0
    for t in prompt[:-1]:
        chain.step(t, pos)
        pos += 1
    tok = prompt[-1]
    for i in range(n_new):
        lc = chain.step(tok, pos)
        assert Qwen3CpuChain.argmax(lc) == ta[i], f"step {i}"
        tok, pos = ta[i], pos + 1
    # the last launch consumed ta[-2]; its logits are the chain's at that step
    assert torch.equal(_bits(la), _bits(lc))


def test_persistent_epoch_advances_per_token():
    _say("persistent epoch / error words")
    cfg = Qwen3Config.tiny()
    m = Qwen3NPU(config=cfg, weights=random_qwen3_weights(cfg, seed=8), max_seq_len=64,
                 persistent=True)
    ctrl = lambda: m._p_ws[:8].view(torch.int32).cpu().tolist()  # noqa: E731
    e0, err0 = ctrl()
    tok = 1
    for pos in range(3):
        tok = m.step_token(tok, pos)
    e1, err1 = ctrl()
    assert e1 == e0 + 3 and err0 == 0 and err1 == 0


@pytest.mark.slow
def test_persistent_qwen3_0_6b_matches_runlist():
    cfg = Qwen3Config.qwen3_0_6b()
    P0, n_prompt, n_new = 2700, 8, 24   # past 80 * 32 = 2560: every split walks two tiles
    S = (P0 + n_prompt + n_new + 63) // 64 * 64
    _say(f"qwen3-0.6b persistent vs runlist: KV {P0}, prompt {n_prompt}, {n_new} tokens")
    w = random_qwen3_weights(cfg, seed=2024, device="cuda")
    k0, v0 = synthetic_kv(cfg, P0, seed=7)
    prompt = torch.randint(0, cfg.vocab_size, (n_prompt,),
                           generator=torch.Generator().manual_seed(64)).tolist()
    runs = []
    for persistent in (False, True):
        _say(f"qwen3-0.6b persistent={persistent}")
        m = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=persistent)
        assert m.persistent == persistent
        m.load_kv(k0, v0)
        toks = m.generate(prompt, n_new, start_pos=P0)
        end = P0 + n_prompt + n_new - 1
        caches = [tuple(c[:, P0:end].cpu() for c in m.kv_caches(i)) for i in (0, 13, 27)]
        runs.append((toks, m.logits(), caches))
        del m
        torch.cuda.empty_cache()
    (ta, la, ca), (tb, lb, cb) = runs
    assert ta == tb, "greedy tokens differ between the runlist and the persistent kernel"
    assert torch.equal(_bits(la), _bits(lb))
    for a, b in zip(ca, cb):
        assert torch.equal(_bits(a[0]), _bits(b[0])) and torch.equal(_bits(a[1]), _bits(b[1]))


def test_phase_trace_0_6b_keeps_results():
    """The traced copy of the Qwen3-0.6B kernel (iron_decode_persistent_set_trace) gives the
    untraced kernel's logits bit for bit, and every workgroup's 16 stamps of every layer are set
    and in program order."""
    from iron_amd import _lib
    cfg = Qwen3Config.qwen3_0_6b()
    P0 = 300
    _say(f"phase trace: qwen3-0.6b, KV {P0}")
    w = random_qwen3_weights(cfg, seed=11, device="cuda")
    k0, v0 = synthetic_kv(cfg, P0, seed=5)
    m = Qwen3NPU(config=cfg, weights=w, max_seq_len=384, persistent=True)
    m.load_kv(k0, v0)
    lib = _lib.load()
    t0 = m.step_token(17, P0)
    ref = m.logits().clone()
    st = torch.zeros(cfg.n_layers * 256 * 16, dtype=torch.int64, device="cuda")
    _lib.check(lib.iron_decode_persistent_set_trace(st.data_ptr(), st.numel() * 8))
    try:
        t1 = m.step_token(17, P0)  # the same position again: the same KV row is rewritten
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.iron_decode_persistent_set_trace(None, 0))
    assert t1 == t0 and torch.equal(_bits(m.logits()), _bits(ref))
    order = [0, 1, 2, 3, 4, 15, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14]
    s_ = st.view(cfg.n_layers, 256, 16)[:, :, order].cpu()
    assert bool((s_ > 0).all()), "a stamp was not written"
    assert bool((s_[:, :, 1:] >= s_[:, :, :-1]).all()), "stamps out of program order"
    assert bool((s_[1:, :, 0] >= s_[:-1, :, -1]).all()), "layers out of order"
