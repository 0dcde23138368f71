#!/usr/bin/env python3
"""Decode throughput of the Qwen3 int8 hot path on one MI355X.

Workload: Qwen3-0.6B architecture (28 layers, D=1024, 16Q/8KV x 128, FF=3072, vocab 151936),
random-init weights, every linear layer int8 with per-group-32 bf16 scales, bf16 embedding /
tied LM head / norms; the KV cache is prefilled to 2048 positions (1984 seeded synthetic
positions + a 64-token seeded prompt run through the decode path), then greedy decoding at B=1.
A step is one decode token: one launch of the token kernel that consumes the previous argmax on
the device, runs the 28 layers (by default as one persistent kernel, ``--decode runlist`` for the
per-operator graph), the final norm and the LM head (argmax fused). The steps run as HIP-graph
replays with no host synchronisation, 16 token launches per replay on the persistent path
(Qwen3NPU.decode_steps) and one token per replay on the runlist path. ``--warmup`` steps run first,
then the position is rewound and ``--steps`` steps are timed between two device
synchronisations (positions 2048 .. 2048+steps-1).

The JSON line also carries:
  roofline      -- the step's dominant launch (the persistent layers kernel; the LM head on the
                   runlist path) timed with HIP events on the stream it runs on, against the
                   8 TB/s HBM peak, with its measured HBM traffic; ``lm_head`` the same for the
                   311 MB bf16 head; the whole-step algorithmic bytes / step time in
                   ``step_roofline``;
  cpu_baseline  -- the CPU oracle chain (the reference's per-op goldens composed with bf16 op
                   boundaries, oracle/qwen3.py) on the host cores, teacher-forced on the GPU's
                   tokens for a bounded sample, with the greedy agreement on that sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the bf16 LM-head GEMV from two rocprofv3 --pmc passes over this bench:
# FETCH_SIZE 152067.06 KiB x 2.0 + WRITE_SIZE 361.44 KiB x 1.0, the factors being what the same
# counters read for a plain 256 MiB device copy (131083.5 KiB fetched, 262144 KiB written).
LM_HEAD_BF16_TRAFFIC = 311_776_133
# HBM bytes per launch of the persistent layers kernel (all 28 layers, LM head separate), same
# method: FETCH_SIZE 350383.56 KiB x 2.0 + WRITE_SIZE 41012.19 KiB x 1.0 at context 1985..2047.
PERSISTENT_TRAFFIC = 759_582_016
# HBM bytes per launch of the one-launch token (layers + final norm + LM head + argmax): a profiled
# constant, not measured in the run. Same method, over this bench's default run (128 steps): the
# median of the 24 event-timed launches at context 2177, FETCH_SIZE 512911.72 KiB x 2.0 +
# WRITE_SIZE 41840.75 KiB x 1.0. At another context the KV read term moves it by the cache bytes
# per position.
PERSISTENT_TOKEN_TRAFFIC = 1_093_288_128
PERSISTENT_TOKEN_TRAFFIC_CTX = 2177
TRAFFIC_SOURCE = ("profiled constant: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over this "
                  "bench's default run (profiles/decode_qwen3_0_6b_hbm_traffic.md)")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-sample-steps", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the standalone measurements of BASELINE configs 1, 2, 3 and 5")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--lm-head", default="bf16", choices=["bf16", "int8"])
    ap.add_argument("--decode", default="auto", choices=["auto", "persistent", "runlist"],
                    help="auto: the persistent whole-token kernel where available, else the "
                         "per-operator runlist graph")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the single-GPU decode path); "
              "--gpus above 1 is not supported", file=sys.stderr)
        sys.exit(2)
    import torch

    from iron_amd.applications.qwen3_0_6b.qwen3_npu_int8 import Qwen3NPU
    from iron_amd.applications.qwen3_0_6b.weights import (Qwen3Config, random_qwen3_weights,
                                                           synthetic_kv, weights_to)

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    cfg = Qwen3Config.qwen3_0_6b(group_size=32)
    P0, n_prompt = 1984, 64
    start = P0 + n_prompt                       # first decoded position: 2048
    S = start + max(args.steps, args.warmup) + 64
    S = (S + 63) // 64 * 64
    t0 = time.time()
    w = random_qwen3_weights(cfg, seed=args.seed, lm_head=args.lm_head, device="cuda")
    w_cpu = None if args.no_cpu_baseline else weights_to(w, "cpu")
    k0, v0 = synthetic_kv(cfg, P0, seed=7)
    print(f"[bench] weights ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    persistent = {"auto": None, "persistent": True, "runlist": False}[args.decode]
    model = Qwen3NPU(config=cfg, weights=w, max_seq_len=S, persistent=persistent)
    print(f"[bench] decode path: {'persistent kernel' if model.persistent else 'runlist graph'}",
          file=sys.stderr, flush=True)
    model.load_kv(k0, v0)
    gen = torch.Generator().manual_seed(64)
    prompt = torch.randint(0, cfg.vocab_size, (n_prompt,), generator=gen).tolist()
    pos = P0
    for t in prompt[:-1]:
        model.step_token(t, pos)
        pos += 1
    assert pos == start - 1
    last = prompt[-1]
    # The armed token is consumed at position start-1; the generated tokens are 2048.. onwards.
    print(f"[bench] prefill done at pos {pos}", file=sys.stderr, flush=True)

    # warm-up, then rewind and time
    model.start_generation(last, pos)
    model.decode_steps(args.warmup + 1)
    torch.cuda.synchronize()
    model.start_generation(last, pos)
    model.decode_steps(1)              # consumes the prompt's last token at pos 2047
    torch.cuda.synchronize()
    t_begin = time.perf_counter()
    model.decode_steps(args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_begin
    tokens = model.finish_generation()
    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = args.steps / elapsed
    print(f"[bench] {args.steps} steps in {elapsed * 1e3:.2f} ms ({ms_per_step * 1e3:.1f} us/step)",
          file=sys.stderr, flush=True)

    # ---- algorithmic bytes per step (weights once + KV read at the step's context + KV append)
    wb = cfg.weight_bytes_per_token(args.lm_head)
    kv_per_pos = cfg.n_layers * cfg.n_kv_heads * cfg.head_dim * 2 * 2
    mean_ctx = start + 1 + (args.steps - 1) / 2.0
    step_bytes = wb["layers"] + wb["lm_head"] + wb["final_norm"] + kv_per_pos * mean_ctx + \
        kv_per_pos + cfg.vocab_size * 2
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    lm_bytes = wb["lm_head"] + cfg.emb_dim * 2 + cfg.vocab_size * 2
    lm_roofline = None
    if model.persistent and model.fold_lm_head:
        token_us = time_folded_token(model)
        layers_us = lm_us = None
    else:
        token_us = None
        if model.persistent:
            layers_us, lm_us = time_persistent(model)
        else:
            layers_us, lm_us = None, time_runlist_lm_head(model)
        lm_gbs = lm_bytes / (lm_us * 1e-6) / 1e9
        lm_roofline = {
            "bound": "hbm",
            "kernel": "lm_head GEMV (bf16 [151936x1024], RMSNorm prologue, argmax epilogue)"
            if args.lm_head == "bf16" else "lm_head GEMV (int8 G=32, argmax epilogue)",
            "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(lm_gbs / HBM_PEAK_GBS, 4),
            "traffic": LM_HEAD_BF16_TRAFFIC if args.lm_head == "bf16" else None,
            "bytes_per_launch": lm_bytes, "avg_launch_us": round(lm_us, 2)}
    if token_us is not None:
        # one launch per token: the 28 layers, the final norm, the bf16 LM head and its argmax;
        # algorithmic bytes: every layer's weights once, the KV read at the timed context and the
        # rows appended, the embedding row in, the LM head and final norm, the logits out
        ctx = start + args.steps + 1
        tok_bytes = (wb["layers"] + kv_per_pos * ctx + kv_per_pos + cfg.emb_dim * 2 +
                     lm_bytes + wb["final_norm"])
        tok_gbs = tok_bytes / (token_us * 1e-6) / 1e9
        tok_traffic = int(PERSISTENT_TOKEN_TRAFFIC +
                          kv_per_pos * (ctx - PERSISTENT_TOKEN_TRAFFIC_CTX))
        roofline = {"bound": "hbm", "kernel": "decode_persistent_kernel (28 layers: QKV, "
                                              "attention, merge, Wo, gate/up, down; final "
                                              "RMSNorm, bf16 LM head, argmax)",
                    "achieved": round(tok_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(tok_gbs / HBM_PEAK_GBS, 4),
                    "traffic": tok_traffic,
                    "traffic_ratio": round(tok_traffic / tok_bytes, 3),
                    "traffic_source": TRAFFIC_SOURCE,
                    "bytes_per_launch": int(tok_bytes), "avg_launch_us": round(token_us, 2),
                    "context": ctx}
    elif model.persistent:
        # the persistent kernel is the step's dominant launch (all 28 layers); its algorithmic
        # bytes: every layer's weights once, the KV cache read at the timed context, the K/V
        # rows appended, the embedding row in and the hidden state out
        ctx = start + 1
        layer_bytes = wb["layers"] + kv_per_pos * ctx + kv_per_pos + 2 * cfg.emb_dim * 2
        layer_gbs = layer_bytes / (layers_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "kernel": "decode_persistent_kernel (28 layers: QKV, "
                                              "attention, merge, Wo, gate/up, down)",
                    "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                    "traffic": PERSISTENT_TRAFFIC,
                    "bytes_per_launch": int(layer_bytes), "avg_launch_us": round(layers_us, 2),
                    "context": ctx}
    else:
        roofline = lm_roofline

    result = {
        "metric": "decode tokens/s (Qwen3 int8 shapes); achieved HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x bf16 -> f64 accumulate (bf16/fp32 operator boundaries)",
        "data": "synthetic (seeded random-init weights, synthetic KV prefill, seeded prompt)",
        "config": {"workload": "BASELINE config 4: Qwen3-0.6B-architecture int8 (G=32) decode, "
                               f"B=1, {args.lm_head} LM head, context {start + 1}.."
                               f"{start + args.steps}",
                   "global_batch": 1, "seq_len": start + args.steps, "parallelism": "none",
                   "layers": cfg.n_layers, "group_size": cfg.group_size},
        "decode_path": "persistent" if model.persistent else "runlist",
        "roofline": roofline,
        "lm_head": lm_roofline if lm_roofline is not None else "folded into the token launch",
        "step_roofline": {"bytes_per_step": int(step_bytes), "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
    }

    if not args.no_configs:
        # the achievable streaming-read rate on this device, the practical ceiling beside the
        # 8 TB/s nominal peak
        from iron_amd import benchmarks
        rc = benchmarks.read_probe()
        for r in (result["roofline"], result["lm_head"]):
            if isinstance(r, dict):
                r["achievable_read_GB_s"] = rc["GB_s"]
                r["frac_of_achievable"] = round(r["achieved"] / rc["GB_s"], 4)
        # the other BASELINE configurations, each timed standalone over >= 512 MiB of rotating
        # operands (iron_amd/benchmarks.py); config 5 includes the 36-layer Qwen3-8B B=16 stack
        del model, w
        torch.cuda.empty_cache()
        from iron_amd import benchmarks
        print("[bench] configs 1, 2, 3, 5", file=sys.stderr, flush=True)
        result["configs"] = benchmarks.run_all(read_ceiling=rc)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, w_cpu, (k0, v0), prompt, tokens, start, S,
                                              args.cpu_sample_steps)
    print(json.dumps(result), flush=True)


def time_persistent(model, n_rep: int = 24):
    """Average duration of the persistent layers kernel and of the LM head, from HIP events on the
    stream both run on. The events bracket each launch alone; consecutive repetitions recompute
    the same position (the KV row is rewritten with the same values). The 468 MB of layer weights
    exceed the 256 MB last-level cache, so every launch streams them from HBM."""
    import torch

    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n_rep)]
    model.persistent_layers_launch()
    model.lm_head_launch()
    for e0, e1, e2 in ev:
        e0.record(stream)
        model.persistent_layers_launch()
        e1.record(stream)
        model.lm_head_launch()
        e2.record(stream)
    torch.cuda.synchronize()
    if model.persistent_errors():
        raise RuntimeError("persistent kernel reported a hand-off timeout while timing")
    layers_us = sum(e0.elapsed_time(e1) for e0, e1, _ in ev) * 1e3 / n_rep
    lm_us = sum(e1.elapsed_time(e2) for _, e1, e2 in ev) * 1e3 / n_rep
    return layers_us, lm_us


def time_folded_token(model, n_rep: int = 24):
    """Average duration of the one-launch greedy step (layers + final norm + LM head + argmax),
    from HIP events on the stream it runs on; each launch decodes the next position."""
    import torch

    stream = torch.cuda.current_stream()
    gs = model._gen_state()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n_rep)]
    model.persistent_gen_launch(model._p_keys, gs)
    for e0, e1 in ev:
        e0.record(stream)
        model.persistent_gen_launch(model._p_keys, gs)
        e1.record(stream)
    torch.cuda.synchronize()
    if model.persistent_errors():
        raise RuntimeError("persistent kernel reported a hand-off timeout while timing")
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) * 1e3 / n_rep


def time_runlist_lm_head(model, n_rep: int = 32):
    """The runlist path's LM head, timed inside whole decode steps with HIP events on its stream.

    The rest of the step is one graph replay before each launch (the 28 layers stream ~700 MB
    through HBM first, as in the step graph); back-to-back launches alone would find part of the
    311 MB head still in the 256 MB last-level cache and overstate the rate."""
    import torch

    lm_fn = model.fc._fns[id(model.lmhead)]
    lm_views = [v for f, v in model.fc._plan if f is lm_fn][0]
    stream = torch.cuda.current_stream()
    body = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.graph(body, stream=side):
        for fn, views in model.fc._plan:
            if fn is not lm_fn:
                fn(*views)
    stream.wait_stream(side)
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(n_rep)]
    for e0, e1 in pairs:
        body.replay()
        e0.record(stream)
        lm_fn(*lm_views)
        e1.record(stream)
    torch.cuda.synchronize()
    del body
    return sum(e0.elapsed_time(e1) for e0, e1 in pairs) * 1e3 / n_rep


def cpu_baseline(cfg, w, kv0, prompt, gpu_tokens, start, S, n_sample):
    """Time the CPU oracle chain on this host's cores (bounded sample, teacher forced)."""
    import torch

    from oracle.qwen3 import Qwen3CpuChain

    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)
    # the reference goldens as written (fp32 torch); dequant once, outside the timing
    chain = Qwen3CpuChain(cfg, w, S, kv_init=kv0, dt=torch.float32)
    pos = start - len(prompt)
    for t in prompt[:-1]:
        chain.step(t, pos)
        pos += 1
    lg = chain.step(prompt[-1], pos)                      # the armed token at start-1
    pos += 1
    # greedy agreement: the chain's argmax at each step against the token the GPU chose there
    agree = int(Qwen3CpuChain.argmax(lg) == gpu_tokens[0])
    tok = gpu_tokens[0]
    t0 = time.perf_counter()
    for i in range(n_sample):
        lg = chain.step(tok, pos)
        tok = gpu_tokens[i + 1]
        agree += int(Qwen3CpuChain.argmax(lg) == tok)
        pos += 1
    dt = time.perf_counter() - t0
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(n_sample / dt, 3), "unit": "tokens/s", "cores": cores,
            "kind": "port", "greedy_agreement": f"{agree}/{n_sample + 1}",
            "sample": f"{n_sample} decode steps at context {start + 2}..{start + 1 + n_sample} "
                      "fed the GPU's tokens (after the same 1984-position KV prefill and 64-token "
                      f"prompt); the reference goldens composed in torch fp32 on {cpu_model}"}


if __name__ == "__main__":
    main()
