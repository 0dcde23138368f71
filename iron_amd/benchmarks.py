"""Standalone measurements of the hot-path kernels at the BASELINE configurations (1, 2, 3, 5).

    python -m iron_amd.benchmarks            # prints one JSON object

Every measurement replays a captured HIP graph of back-to-back launches that cycle over distinct
copies of the streamed operands (at least 512 MiB in total, twice the 256 MiB Infinity Cache), so
the bytes come from HBM; the per-launch time is the graph time divided by the launches, and the
figure reported is the median (with p10/p90) over the replays. Algorithmic bytes are the
operands each launch must read plus what it writes; ``frac`` is against the 8 TB/s HBM peak, or
against the 2.5 PFLOP/s dense bf16 MFMA peak for the prefill attention.
"""

from __future__ import annotations

import ctypes
import json
import math
import statistics

import torch

from . import _lib

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
# MFMA busy fraction per kernel (SQ_VALU_MFMA_BUSY_CYCLES over the 1024 SIMDs / (GRBM_GUI_ACTIVE / 8
# XCDs x 1024)), measured with rocprofv3 --pmc over `--only c5_prefill` and `--only c5_decode`;
# a counter run, so quoted here rather than measured in the timed run.
MFMA_BUSY = {"prefill_attn_kernel": 0.252,
             "gemm_w8_rs_kernel (gate/up, SwiGLU, 3 activation planes)": 0.077,
             "gemm_w8_mfma_kernel (down, 3 activation planes)": 0.060,
             "gemm_w8_mfma_kernel (QKV)": 0.015, "gemm_w8_mfma_kernel (Wo)": 0.011}
ROTATE_BYTES = 512 << 20
DEV = "cuda"


def _wire(lib, M, K, G, tm, n, seed=0):
    """n device copies of one signed int8 wire drawn as BASELINE specifies: q uniform on
    {-127..127}, per-group-G scales bf16(|N(0, 0.02)|), packed in the row-block wire. The copies
    hold the same bytes at distinct addresses (the rotation only has to defeat the caches)."""
    from .operators.wire import pack_wire

    sz = ctypes.c_size_t()
    _lib.check(lib.iron_wire_bytes(M, K, G, tm, ctypes.byref(sz)))
    key = (M, K, G, tm, seed)
    one = _WIRES.get(key)
    if one is None:
        gen = torch.Generator().manual_seed(seed)
        q = torch.randint(-127, 128, (M, K), generator=gen, dtype=torch.int16)
        s = (torch.randn(M, K // G, generator=gen) * 0.02).abs().to(torch.bfloat16)
        one = _WIRES[key] = pack_wire(q, s, tm, "signed").to(DEV)
    assert one.numel() == sz.value
    return [one.clone() for _ in range(n)], sz.value


_WIRES: dict = {}   # one packed wire per geometry; every use takes device copies of it


def _time_graph(fn, launches: int, replays: int = 40):
    """fn() issues `launches` launches; returns (median, p10, p90) microseconds per launch."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / launches)
    ts.sort()
    return statistics.median(ts), ts[len(ts) // 10], ts[(9 * len(ts)) // 10]


def _result(us, nbytes, extra=None):
    med, p10, p90 = us
    gbs = nbytes / (med * 1e-6) / 1e9
    r = {"us_median": round(med, 3), "us_p10": round(p10, 3), "us_p90": round(p90, 3),
         "bytes": int(nbytes), "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    if extra:
        r.update(extra)
    return r


def _st():
    return torch.cuda.current_stream().cuda_stream


def config1(lib):
    """QKV GEMV, int8 G=32, B=1: x [1,1024], W [4096,1024] -> y [1,4096]."""
    M, K, G, tm = 4096, 1024, 32, 4
    n = math.ceil(ROTATE_BYTES / (M * K))
    ws, wbytes = _wire(lib, M, K, G, tm, n)
    x = torch.randn(K, device=DEV).to(torch.bfloat16)
    y = torch.empty(M, dtype=torch.bfloat16, device=DEV)

    def run():
        for w in ws:
            _lib.check(lib.iron_gemv_w8a16(w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, M, K, G,
                                           tm, 0, _st()))

    return _result(_time_graph(run, n), wbytes + 2 * K + 2 * M,
                   {"shape": "M=4096 K=1024 G=32 B=1", "copies": n})


def config2(lib, B):
    """SwiGLU MLP at Qwen3-1.7B shape (D=2048, FF=6144), B rows."""
    D, FF, G = 2048, 6144, 32
    per = 3 * FF * D
    n = max(2, math.ceil(ROTATE_BYTES / per))
    gate, gb = _wire(lib, FF, D, G, 12, n)
    up, _ = _wire(lib, FF, D, G, 12, n)
    down, db = _wire(lib, D, FF, G, 4, n)
    cur = torch.randn(B, D, device=DEV).to(torch.bfloat16)
    a = torch.randn(B, D, device=DEV).to(torch.bfloat16)
    nw = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    nxt = torch.empty(B, D, dtype=torch.bfloat16, device=DEV)
    wsz = lib.iron_swiglu_mlp_workspace(B, D, FF)
    ws = torch.zeros(wsz, dtype=torch.uint8, device=DEV)

    def run():
        for i in range(n):
            _lib.check(lib.iron_swiglu_mlp(cur.data_ptr(), a.data_ptr(), nw.data_ptr(), None,
                                           gate[i].data_ptr(), up[i].data_ptr(),
                                           down[i].data_ptr(), nxt.data_ptr(), None, B, D, FF, 0,
                                           G, 4, 12, 4, 0, ctypes.c_float(1e-6), ws.data_ptr(),
                                           wsz, _st()))

    return _result(_time_graph(run, n), 2 * gb + db + B * (3 * 2 * D),
                   {"shape": f"D=2048 FF=6144 G=32 B={B}", "copies": n,
                    "path": "GEMV" if B <= 4 else "MFMA"})


def config3(lib, B, ragged, acc="f64"):
    """GQA decode attention, 16 Q / 8 KV x 128, contiguous [B, 8, L, 128] caches; ``acc`` is the
    accumulation mode ("f64" exact, "f32" the reference kernel's arithmetic)."""
    H, KV, D, L = 16, 8, 128, 4096
    g = torch.Generator().manual_seed(3)
    ctx = (torch.randint(512, L + 1, (B,), generator=g) if ragged
           else torch.full((B,), L, dtype=torch.int64))
    per = B * KV * L * D * 2 * 2
    n = max(2, math.ceil(ROTATE_BYTES / per))
    ks = [torch.randn(B * KV * L * D, device=DEV).to(torch.bfloat16) for _ in range(n)]
    vs = [torch.randn(B * KV * L * D, device=DEV).to(torch.bfloat16) for _ in range(n)]
    q = torch.randn(B * H * D, device=DEV).to(torch.bfloat16)
    o = torch.empty(B * H * D, dtype=torch.bfloat16, device=DEV)
    c = ctx.to(torch.int32).to(DEV)
    wsz = lib.iron_decode_attn_workspace(B, H, KV, D, L)
    ws = torch.zeros(wsz, dtype=torch.uint8, device=DEV)
    scale = ctypes.c_float(D ** -0.5)

    def run():
        for i in range(n):
            _lib.check(lib.iron_decode_attn(q.data_ptr(), ks[i].data_ptr(), vs[i].data_ptr(),
                                            KV * L * D, L * D, D, c.data_ptr(), 0, o.data_ptr(), B,
                                            H, KV, D, L, scale, _lib.accum_mode(acc),
                                            ws.data_ptr(), wsz, _st()))

    nbytes = KV * D * 2 * 2 * int(ctx.sum()) + 2 * 2 * B * H * D
    return _result(_time_graph(run, n), nbytes,
                   {"shape": f"B={B} L={'U[512,4096]' if ragged else L}", "copies": n,
                    "context_sum": int(ctx.sum()), "accumulate": acc})


def config5_decode(lib, steps: int = 3, acc: str = "f64"):
    """Qwen3-8B layer stack (36 layers, D=4096, 32 Q / 8 KV x 128, FF=12288, int8 G=32) decode
    at B=16 with every sequence at context 8192: per step, each layer runs the fused QKV head +
    attention (raw QKV on MFMA) and the MLP with the output projection (three MFMA GEMMs)."""
    NL, D, Hq, Hkv, HD, FF, G, B, L = 36, 4096, 32, 8, 128, 12288, 32, 16, 8192
    QD, M = Hq * HD, (Hq + 2 * Hkv) * HD
    layers = []
    for _ in range(NL):
        layers.append({
            "qkv": _wire(lib, M, D, G, 16, 1)[0][0], "o": _wire(lib, D, QD, G, 4, 1)[0][0],
            "g": _wire(lib, FF, D, G, 12, 1)[0][0], "u": _wire(lib, FF, D, G, 12, 1)[0][0],
            "d": _wire(lib, D, FF, G, 4, 1)[0][0],
            "k": torch.randn(B * Hkv * L * HD, device=DEV).to(torch.bfloat16),
            "v": torch.randn(B * Hkv * L * HD, device=DEV).to(torch.bfloat16),
        })
    x = torch.randn(B, D, device=DEV).to(torch.bfloat16)
    nw = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    nh = torch.ones(HD, dtype=torch.bfloat16, device=DEV)
    ang = torch.randn(B * HD, device=DEV).to(torch.bfloat16)
    pos = torch.full((B,), L - 1, dtype=torch.int32, device=DEV)
    attn = torch.empty(B, QD, dtype=torch.bfloat16, device=DEV)
    wq = lib.iron_qkv_attn_workspace(B, D, Hq, Hkv, HD, L)
    wsq = torch.zeros(wq, dtype=torch.uint8, device=DEV)
    wm = lib.iron_swiglu_mlp_workspace(B, D, FF)
    wsm = torch.zeros(wm, dtype=torch.uint8, device=DEV)
    eps, scale = ctypes.c_float(1e-6), ctypes.c_float(HD ** -0.5)
    mode = _lib.accum_mode(acc)

    def step():
        for ly in layers:
            _lib.check(lib.iron_qkv_attn(x.data_ptr(), nw.data_ptr(), ly["qkv"].data_ptr(),
                                         nh.data_ptr(), nh.data_ptr(), ang.data_ptr(),
                                         ly["k"].data_ptr(), ly["v"].data_ptr(), Hkv * L * HD,
                                         L * HD, HD, pos.data_ptr(), attn.data_ptr(), B, D, HD,
                                         Hq, Hkv, L, G, 16, 0, eps, scale, mode, wsq.data_ptr(),
                                         wq, _st()))
            _lib.check(lib.iron_swiglu_mlp(x.data_ptr(), attn.data_ptr(), nw.data_ptr(),
                                           ly["o"].data_ptr(), ly["g"].data_ptr(),
                                           ly["u"].data_ptr(), ly["d"].data_ptr(), x.data_ptr(),
                                           None, B, D, FF, QD, G, 4, 12, 4, 0, eps,
                                           wsm.data_ptr(), wm, _st()))

    med, p10, p90 = _time_graph(step, 1, replays=steps + 2)
    wbytes = sum(t.numel() for ly in layers for key, t in ly.items() if key not in ("k", "v"))
    kvbytes = NL * B * Hkv * L * HD * 2 * 2
    nbytes = wbytes + kvbytes
    gbs = nbytes / (med * 1e-6) / 1e9
    return {"ms_per_step": round(med / 1e3, 3), "tokens_per_s": round(B / (med * 1e-6), 1),
            "bytes_per_step": int(nbytes), "GB_s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "shape": "Qwen3-8B int8 G=32, 36 layers, B=16, context 8192", "accumulate": acc,
            "gemm_mfma_busy": {k: v for k, v in MFMA_BUSY.items() if k.startswith("gemm")}}


def config5_prefill(lib):
    """Causal bf16 prefill attention, Qwen3-8B heads (32 Q / 8 KV x 128), S = 2048, B = 1."""
    H, KV, S, D = 32, 8, 2048, 128
    q = torch.randn(H * S * D, device=DEV).to(torch.bfloat16)
    k = torch.randn(KV * S * D, device=DEV).to(torch.bfloat16)
    v = torch.randn(KV * S * D, device=DEV).to(torch.bfloat16)
    o = torch.empty_like(q)
    reps = 20

    def run():
        for _ in range(reps):
            _lib.check(lib.iron_prefill_attn(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             o.data_ptr(), 1, H, KV, S, D,
                                             ctypes.c_float(D ** -0.5), _st()))

    med, p10, p90 = _time_graph(run, reps, replays=10)
    flops = 4 * D * H * (S * (S + 1) // 2)
    tf = flops / (med * 1e-6) / 1e12
    return {"us_median": round(med, 2), "us_p10": round(p10, 2), "us_p90": round(p90, 2),
            "flops": flops, "TFLOP_s": round(tf, 1), "frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
            "shape": "H=32 KV=8 S=2048 D=128 causal",
            "mfma_busy": MFMA_BUSY["prefill_attn_kernel"]}


def run_all(include_c5: bool = True, read_ceiling: dict | None = None) -> dict:
    """Every configuration; ``read_ceiling``: a read-probe result to report instead of probing
    again (one ceiling per bench line)."""
    _WIRES.clear()
    lib = _lib.load()
    out = {"read_ceiling": read_ceiling if read_ceiling is not None else read_probe(),
           "c1_qkv_gemv": config1(lib),
           "c2_mlp_b1": config2(lib, 1), "c2_mlp_b8": config2(lib, 8),
           "c3_attn_b1": config3(lib, 1, False), "c3_attn_b8_ragged": config3(lib, 8, True),
           "c3_attn_b1_f32": config3(lib, 1, False, "f32"),
           "c3_attn_b8_ragged_f32": config3(lib, 8, True, "f32")}
    _WIRES.clear()
    torch.cuda.empty_cache()
    if include_c5:
        out["c5_prefill_mha"] = config5_prefill(lib)
        out["c5_decode_b16"] = config5_decode(lib)
        out["c5_decode_b16_f32"] = config5_decode(lib, acc="f32")
        torch.cuda.empty_cache()
    return out


def read_probe(gib: int = 1, reps: int = 5) -> dict:
    """The achievable HBM read rate: iron_stream_read over a buffer far larger than the caches
    (grid sizes swept; the best is the ceiling the decode kernels are read against)."""
    lib = _lib.load()
    nbytes = gib << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=DEV)
    out = torch.empty(16384 * 256, dtype=torch.int32, device=DEV)
    best = 0.0
    for blocks in (1024, 2048, 4096, 8192):
        _lib.check(lib.iron_stream_read(buf.data_ptr(), nbytes, out.data_ptr(), blocks, _st()))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            _lib.check(lib.iron_stream_read(buf.data_ptr(), nbytes, out.data_ptr(), blocks, _st()))
        e1.record()
        e1.synchronize()
        gbs = reps * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9
        best = max(best, gbs)
    return {"GB_s": round(best, 1), "frac": round(best / HBM_PEAK_GBS, 4),
            "bytes": nbytes, "kernel": "iron_stream_read (16-byte loads, a contiguous chunk per workgroup)"}


HANDOFF_MODES = {"tagged": _lib.IRON_HANDOFF_TAGGED, "counter": _lib.IRON_HANDOFF_COUNTER,
                 "flags": _lib.IRON_HANDOFF_FLAGS, "xcd_l2": _lib.IRON_HANDOFF_XCD_L2,
                 "xcd_agent": _lib.IRON_HANDOFF_XCD_AGENT}


def handoff_probe(phases: int = 2000, reps: int = 3) -> dict:
    """Microseconds per grid-wide hand-off phase (iron_handoff_probe: 256 workgroups, one per CU):
    the tagged-word exchange at several vector sizes (words every workgroup polls), an atomic
    counter barrier, flags with device-scope fences, and the exchange inside each XCD's 32
    workgroups through its L2 or with device-scope words. Best of `reps` launches of `phases`."""
    lib = _lib.load()
    # xcd_*: 32-workgroup groups (one XCD each); 256 and 640 words are the decode kernel's raw
    # q/k/v and split-partial gathers
    cases = [("tagged", n) for n in (256, 512, 1024, 2048)] + [("counter", 256),
                                                                ("flags", 1024)] + \
        [(m, n) for m in ("xcd_agent", "xcd_l2") for n in (256, 640)]
    out, base = {}, 0
    for name, n in cases:
        nbytes = lib.iron_handoff_probe_workspace(n)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        best = None
        for _ in range(reps):
            ws.zero_()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            _lib.check(lib.iron_handoff_probe(HANDOFF_MODES[name], n, phases, base, ws.data_ptr(),
                                              nbytes, _st()))
            e1.record()
            e1.synchronize()
            base += phases + 1
            err = int(ws[nbytes - 4096 + 256: nbytes - 4096 + 260].view(torch.int32).item())
            if err:
                raise RuntimeError(f"iron_handoff_probe {name} n={n}: a wait gave up")
            us = e0.elapsed_time(e1) * 1e3 / phases
            best = us if best is None else min(best, us)
        out[f"{name}_{n}"] = round(best, 3)
    return {"us_per_phase": out, "phases": phases,
            "kernel": "iron_handoff_probe (256 workgroups x 256 threads, one per CU)"}


STAMP_ORDER = (0, 1, 2, 3, 4, 15, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14)  # marks in program order


def phase_trace(tokens: int = 6, ctx: int = 2048, first_layer: int = 4) -> dict:
    """Per-phase timings of the persistent decode kernel (Qwen3-0.6B shape, B=1, random-init
    weights, KV prefilled to `ctx`) from its phase stamps (iron_decode_persistent_set_trace), for
    layers first_layer..27 of the last of `tokens` decode steps, medians over layers of:
    compute -- the median workgroup's time from its input gathered to its output stored;
    wait    -- the median workgroup's input-gathered time minus the last producer's store (the
               attention and merge phases count only their own XCD's producers, the only ones
               they poll);
    spread  -- the last workgroup's store minus the median workgroup's;
    and the layer period (QKV entry to QKV entry). Stamps read the 100 MHz constant clock."""
    import numpy as np

    from .applications.qwen3_0_6b.qwen3_npu_int8 import Qwen3NPU
    from .applications.qwen3_0_6b.weights import Qwen3Config, random_qwen3_weights, synthetic_kv

    lib = _lib.load()
    cfg = Qwen3Config.qwen3_0_6b(group_size=32)
    w = random_qwen3_weights(cfg, seed=2024, device=DEV)
    k0, v0 = synthetic_kv(cfg, ctx, seed=7)
    m = Qwen3NPU(config=cfg, weights=w, max_seq_len=(ctx + tokens + 63) // 64 * 64,
                 persistent=True)
    m.load_kv(k0, v0)
    L, NT = cfg.n_layers, 256
    st = torch.zeros(L * NT * 16, dtype=torch.int64, device=DEV)
    _lib.check(lib.iron_decode_persistent_set_trace(st.data_ptr(), st.numel() * 8),
               "iron_decode_persistent_set_trace")
    try:
        tok = 17
        for i in range(tokens):
            tok = m.step_token(tok, ctx + i)
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.iron_decode_persistent_set_trace(None, 0), "iron_decode_persistent_set_trace")
    t = st.view(L, NT, 16).cpu().numpy().astype(np.float64) * 0.01  # microseconds
    grp = np.arange(NT) % 8
    phases = {"A_qkv": (1, 2), "B_attention": (3, 5), "C_merge": (6, 7), "D_wo": (8, 9),
              "E_gateup": (10, 12), "F_down": (13, 14)}
    prev = {"A_qkv": (14, -1, False), "B_attention": (2, 0, True), "C_merge": (5, 0, True),
            "D_wo": (7, 0, False), "E_gateup": (9, 0, False), "F_down": (12, 0, False)}
    out = {}
    for name, (got, end) in phases.items():
        pm, dl, local = prev[name]
        waits, comps, spreads = [], [], []
        for l in range(first_layer, L):
            pe = t[l + dl, :, pm]
            last = np.array([pe[grp == g].max() for g in grp]) if local else pe.max()
            waits.append(np.median(t[l, :, got] - last))
            comps.append(np.median(t[l, :, end] - t[l, :, got]))
            spreads.append(t[l, :, end].max() - np.median(t[l, :, end]))
        out[name] = {"wait_us": round(float(np.median(waits)), 2),
                     "compute_us": round(float(np.median(comps)), 2),
                     "spread_us": round(float(np.median(spreads)), 2)}
    per = [np.median(t[l + 1, :, 0] - t[l, :, 0]) for l in range(first_layer, L - 1)]
    sub = lambda a, b: round(float(np.median([np.median(t[l, :, a] - t[l, :, b])
                                              for l in range(first_layer, L)])), 2)
    return {"phases": out, "layer_period_us": round(float(np.median(per)), 2),
            "attention_norm_rope_us": sub(4, 3), "attention_tiles_us": sub(15, 4),
            "attention_partials_us": sub(5, 15), "gateup_prologue_us": sub(11, 10),
            "context": ctx, "layers": f"{first_layer}..{L - 1}",
            "kernel": "decode_persistent_kernel<Traced<Shape<1024, 3072, 16, 8>>>"}


def copy_probe(mib: int = 256, reps: int = 4) -> dict:
    """A plain device copy of a known size: the calibration run for the HBM byte counters
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE read this kernel as mib MiB fetched / written)."""
    src = torch.randn(mib << 18, device=DEV)   # mib MiB of fp32
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes": mib << 20, "reps": reps}


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="standalone timings of the BASELINE configurations")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run only the byte-counter calibration copy")
    ap.add_argument("--read-probe", action="store_true",
                    help="run only the achievable-read-bandwidth probe")
    ap.add_argument("--handoff-probe", action="store_true",
                    help="run only the grid-wide hand-off probe (us per phase per mechanism)")
    ap.add_argument("--phase-trace", action="store_true",
                    help="run only the persistent decode kernel's per-phase timing (stamps)")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c5_prefill", "c5_decode"],
                    help="run one configuration (for profiling)")
    ap.add_argument("--acc", choices=["f64", "f32"], default="f64",
                    help="attention accumulation for --only c3 / c5_decode")
    ap.add_argument("--batch", type=int, default=None,
                    help="batch for --only c2 (default 1) / c3 (default 8, ragged when > 1)")
    a = ap.parse_args()
    if a.copy_probe:
        print(json.dumps(copy_probe()), flush=True)
    elif a.read_probe:
        print(json.dumps(read_probe()), flush=True)
    elif a.handoff_probe:
        print(json.dumps(handoff_probe()), flush=True)
    elif a.phase_trace:
        print(json.dumps(phase_trace()), flush=True)
    elif a.only:
        lib = _lib.load()
        b2, b3 = a.batch or 1, a.batch or 8
        one = {"c1": lambda: config1(lib), "c2": lambda: config2(lib, b2),
               "c3": lambda: config3(lib, b3, b3 > 1, a.acc),
               "c5_prefill": lambda: config5_prefill(lib),
               "c5_decode": lambda: config5_decode(lib, acc=a.acc)}[a.only]
        print(json.dumps(one()), flush=True)
    else:
        print(json.dumps(run_all()), flush=True)
