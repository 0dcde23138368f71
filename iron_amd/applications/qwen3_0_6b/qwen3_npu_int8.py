"""Qwen3 int8 (W8A16, in-kernel dequant) decode on one MI355X -- the reference's ``Qwen3NPU``.

Drop-in for iron/applications/qwen3_0.6b/qwen3_npu_int8.py:129-621: the same operator set and
runlist -- per layer the fused QKV head (RMSNorm + QKV GEMV + QK-norm + RoPE + KV append), decode
attention, and the fused MLP with the output projection folded in (fuse_o); then the final
RMSNorm and the LM head -- run as one ``OperatorSequence`` whose callable replays a HIP graph
(one dispatch per token, as the reference's single full-ELF dispatch). ``model(x, seq_pos)``
keeps the reference call: bf16 hidden state in, argmax token out.

Differences from the reference, all deliberate:
  * the constructor takes a checkpoint path (GPTQ safetensors), explicit weights, or a config +
    seed for random-init weights (no checkpoint is available offline);
  * the KV caches are separate contiguous ``[B, Hkv, max_seq, HD]`` K and V (BASELINE's layout;
    ``kv_layout="interleaved"`` gives the reference's merged cache);
  * by default (``fuse_attention=True``) the QKV head and decode attention run as one operator
    (``QKVHeadAttention``) whose attention kernel performs the QK-norm/RoPE/KV-append epilogue;
    ``fuse_attention=False`` keeps the reference's two runlist entries (identical results);
  * ``attn_accumulate`` selects the attention core's arithmetic: "f64" evaluates it exactly (the
    whole step is then bit-identical to the fp64 oracle chain), "f32" uses the reference
    kernel's fp32 arithmetic (decode_attn.cc:117-311);
  * the LM head carries an argmax epilogue, so the token is chosen on the device (the reference
    copies the logits out and runs numpy argmax, qwen3_npu_int8.py:612-621);
  * ``generate()`` runs greedy decoding entirely on the device: each step replays one graph that
    consumes the previous argmax, gathers its embedding, runs the layers and advances the
    positions, with no host synchronisation between tokens;
  * ``persistent`` runs all layers of a token in ONE kernel (``iron_decode_persistent``) with the
    same arithmetic as the runlist's operators, followed by the LM head with the final RMSNorm
    fused into its prologue: the counterpart of the reference's single dispatch per token
    (sequence.py:270-559). ``None`` (the default) uses it wherever it is available: batch 1, the
    exact attention core, a shape the kernel is built for, and a device that holds its grid.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from ... import _lib
from ...common.context import AIEContext
from ...common.sequence import OperatorSequence
from ...operators import (GEMV, DecodeAttention, GEMVInt8, QKVHeadAttention,
                          QKVHeadDataParallelOurs, RMSNorm, SwiGLUMLPDataParallelOurs)
from ...operators.wire import pack_wire
from .weights import Qwen3Config, load_gptq_checkpoint, random_qwen3_weights

SIGNED_GEMV_KERNEL = "mv_int8_signed.cc"
QKV_TSI = 4
LMHEAD_TSI = 4


def rope_angle_table(max_pos: int, head_dim: int, theta: float) -> torch.Tensor:
    """(max_pos, head_dim) bf16 rows [cos_0, sin_0, cos_1, sin_1, ...] (qwen3_npu_int8.py:580-591)."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv_freq)
    emb = torch.cat([freqs, freqs], dim=-1)
    cos = emb.cos().to(torch.bfloat16)[:, :half]
    sin = emb.sin().to(torch.bfloat16)[:, :half]
    return torch.stack([cos, sin], dim=-1).reshape(max_pos, head_dim)


def _decode_key(key: int) -> int:
    return (~key) & 0xFFFFFFFF


def _encode_token(tok: int) -> int:
    return (1 << 32) | ((~int(tok)) & 0xFFFFFFFF)


class Qwen3NPU:
    def __init__(self, weights_path=None, *, config: Qwen3Config | None = None,
                 weights: dict | None = None, seed: int = 0, max_seq_len: int = 512,
                 kv_layout: str = "separate", lm_head: str | None = None,
                 dispatch: str = "auto", context: AIEContext | None = None,
                 fuse_attention: bool = True, attn_accumulate: str = "f64",
                 persistent: bool | None = None, fold_lm_head: bool = True):
        self.cfg = cfg = config or Qwen3Config.qwen3_0_6b()
        self.max_seq_len = max_seq_len
        self.kv_layout = kv_layout
        self.fuse_attention = fuse_attention
        self.attn_accumulate = attn_accumulate
        self.context = context or AIEContext()
        self.device = self.context.device
        if weights is None:
            if weights_path is not None:
                weights = load_gptq_checkpoint(weights_path, cfg, lm_head or "bf16")
            else:
                weights = random_qwen3_weights(cfg, seed, lm_head=lm_head or "bf16")
        self.lm_head_kind = "int8" if isinstance(weights["lm_head"], tuple) else "bf16"
        self._build_operators()
        self._build_sequence(dispatch)
        self._load_weights(weights)
        self._gen_graph = None
        self._gen_graph_batch = None   # GEN_BATCH token steps in one graph (persistent path)
        self._gen_pos = None
        if self._dispatch_name(dispatch) in ("reference", "compare"):
            # per-step goldens run over the runlist entries (reference: on CPU buffers), so the
            # whole-token kernel, which bypasses the runlist, is not used
            if persistent:
                raise ValueError(f"persistent decode runs no per-step goldens (dispatch="
                                 f"{self._dispatch_name(dispatch)!r})")
            persistent = False
        self.persistent = self._setup_persistent(persistent)
        # the device greedy loop folds the final norm, bf16 LM head and argmax into the
        # persistent launch (one launch per token); an int8 head keeps its own launch
        self.fold_lm_head = bool(fold_lm_head and self.persistent and self.lm_head_kind == "bf16")

    @staticmethod
    def _dispatch_name(dispatch) -> str:
        return dispatch if isinstance(dispatch, str) else getattr(dispatch, "name", "")

    # ---------------- operators ----------------
    def _build_operators(self):
        cfg, c, S = self.cfg, self.context, self.max_seq_len
        self.rms = RMSNorm(size=cfg.emb_dim, num_aie_columns=1, num_channels=1,
                           tile_size=cfg.emb_dim, weighted=True, epsilon=cfg.eps, context=c)
        self.decode_attn = DecodeAttention(
            num_heads=cfg.n_heads, num_kv_heads=cfg.n_kv_heads, head_dim=cfg.head_dim,
            seq_len_kv=S, use_runtime_seq_len=True,
            kv_layout="separate" if self.kv_layout == "separate" else "combined",
            kv_token_interleaved=True, accumulate=self.attn_accumulate, context=c)
        self.mlp_xdna = SwiGLUMLPDataParallelOurs(
            D=cfg.emb_dim, FF=cfg.hidden_dim, group_size=cfg.group_size, epsilon=cfg.eps,
            fuse_o=True, QD=cfg.q_dim, kernel_source=SIGNED_GEMV_KERNEL, context=c)
        self.qkv_dp = QKVHeadDataParallelOurs(
            D=cfg.emb_dim, HD=cfg.head_dim, Hq=cfg.n_heads, Hkv=cfg.n_kv_heads, max_seq=S,
            num_aie_columns=1, tile_size_input=QKV_TSI, epsilon=cfg.eps,
            group_size=cfg.group_size, kv_layout=self.kv_layout,
            kernel_source=SIGNED_GEMV_KERNEL, kv_offset_parameter="k_cache_offset", context=c)
        self.qkv_attn = QKVHeadAttention(
            D=cfg.emb_dim, HD=cfg.head_dim, Hq=cfg.n_heads, Hkv=cfg.n_kv_heads, max_seq=S,
            num_aie_columns=1, tile_size_input=QKV_TSI, epsilon=cfg.eps,
            group_size=cfg.group_size, kv_layout=self.kv_layout,
            kernel_source=SIGNED_GEMV_KERNEL, kv_offset_parameter="k_cache_offset",
            accumulate=self.attn_accumulate, context=c)
        if self.lm_head_kind == "bf16":
            self.lmhead = GEMV(M=cfg.vocab_size, K=cfg.emb_dim, epilogue="argmax", context=c)
        else:
            self.lmhead = GEMVInt8(M=cfg.vocab_size, K=cfg.emb_dim, tile_size_input=LMHEAD_TSI,
                                   group_size=cfg.group_size, kernel_vector_size=16,
                                   kernel_source=SIGNED_GEMV_KERNEL, epilogue="argmax",
                                   context=c)

    # ---------------- sequence ----------------
    def _build_sequence(self, dispatch):
        cfg = self.cfg
        runlist = []
        for i in range(cfg.n_layers):
            caches = ([f"k_cache_{i}", f"v_cache_{i}"] if self.kv_layout == "separate"
                      else [f"kv_cache_{i}"])
            if self.fuse_attention:
                runlist.append((self.qkv_attn, "x", f"W_norm1_{i}", f"W_qkv_{i}", f"W_qn_{i}",
                                f"W_kn_{i}", "rope_row", *caches, "context"))
            else:
                runlist.append((self.qkv_dp, "x", f"W_norm1_{i}", f"W_qkv_{i}", f"W_qn_{i}",
                                f"W_kn_{i}", "rope_row", "rope_q", *caches))
                runlist.append((self.decode_attn, "rope_q", *caches, "context"))
            runlist.append((self.mlp_xdna, "x", "context", f"W_norm2_{i}", f"Wo_{i}", f"Wg_{i}",
                            f"Wu_{i}", f"Wd_{i}", "gh_scratch", "a_scratch", "x"))
        runlist += [
            (self.rms, "x", "W_final_norm", "x_final"),
            (self.lmhead, "W_out_head", "x_final", "logits", "argmax_key"),
        ]
        indep = ["W_out_head"] + [n for entry in runlist for n in entry[1:]
                                  if n.startswith(("W_qkv_", "Wo_", "Wg_", "Wu_", "Wd_",
                                                   "k_cache_", "v_cache_", "kv_cache_"))]
        indep = list(dict.fromkeys(indep))
        self.seq = OperatorSequence("qwen3_decode", runlist, input_args=["x"],
                                    output_args=["logits", "argmax_key"],
                                    independent_buffer_args=indep, dispatch=dispatch,
                                    context=self.context)
        self.seq.compile()
        self.fc = self.seq.get_callable()

    # ---------------- weights ----------------
    def _set(self, name, t):
        b = self.fc.get_buffer(name).torch_view(t.dtype if t.dtype != torch.uint8 else torch.uint8)
        flat = t.reshape(-1)
        b[: flat.numel()].copy_(flat.to(self.device))

    def _set_wire(self, name, qs, tile_m):
        w = pack_wire(qs[0], qs[1], tile_m, "signed")
        self._set(name, w)

    def _load_weights(self, w: dict):
        cfg = self.cfg
        mlp = self.mlp_xdna
        for i, L in enumerate(w["layers"]):
            self._set(f"W_norm1_{i}", L["input_norm"])
            self._set_wire(f"W_qkv_{i}", L["qkv"], QKV_TSI)
            self._set(f"W_qn_{i}", L["q_norm"])
            self._set(f"W_kn_{i}", L["k_norm"])
            self._set(f"W_norm2_{i}", L["post_norm"])
            self._set_wire(f"Wo_{i}", L["o"], mlp.tile_rows_o)
            self._set_wire(f"Wg_{i}", L["gate"], mlp.tile_rows_gu)
            self._set_wire(f"Wu_{i}", L["up"], mlp.tile_rows_gu)
            self._set_wire(f"Wd_{i}", L["down"], mlp.tile_rows_d)
        self._set("W_final_norm", w["final_norm"])
        if self.lm_head_kind == "bf16":
            self._set("W_out_head", w["lm_head"])
            self.embed = self.fc.get_buffer("W_out_head").torch_view(torch.bfloat16)[
                : cfg.vocab_size * cfg.emb_dim]
            if w["embed"] is not w["lm_head"]:
                self.embed = w["embed"].to(self.device).reshape(-1)
        else:
            self._set_wire("W_out_head", w["lm_head"], LMHEAD_TSI)
            self.embed = w["embed"].to(self.device).reshape(-1)
        # the RoPE table stays on the device; the runlist reads the current position's row
        # ("rope_row"), written per token like the reference's angle input
        self.rope_table = rope_angle_table(self.max_seq_len, cfg.head_dim,
                                           cfg.rope_theta).to(self.device).reshape(-1)
        torch.cuda.synchronize(self.device)

    # ---------------- persistent whole-token kernel ----------------
    def persistent_unavailable_reason(self) -> str | None:
        """Why ``iron_decode_persistent`` cannot run this model (None when it can)."""
        cfg = self.cfg
        if self.attn_accumulate != "f64":
            return "the persistent kernel implements the exact (f64) attention core only"
        lib = _lib.load()
        if lib.iron_decode_persistent_supported(cfg.emb_dim, cfg.hidden_dim, cfg.n_heads,
                                                cfg.n_kv_heads, cfg.head_dim) != _lib.IRON_OK:
            return lib.iron_last_error().decode(errors="replace")
        return None

    def _cache_ptrs(self, layer: int):
        if self.kv_layout == "separate":
            return (self.fc.get_buffer(f"k_cache_{layer}").torch_view(torch.bfloat16).data_ptr(),
                    self.fc.get_buffer(f"v_cache_{layer}").torch_view(torch.bfloat16).data_ptr())
        kv = self.fc.get_buffer(f"kv_cache_{layer}").torch_view(torch.bfloat16).data_ptr()
        return kv, kv + 2 * self.cfg.head_dim

    def _kv_strides(self):
        """(head stride, token stride) of a layer's cache in elements (batch 1)."""
        HD, S = self.cfg.head_dim, self.max_seq_len
        per_tok = HD * (1 if self.kv_layout == "separate" else 2)
        return S * per_tok, per_tok

    def _setup_persistent(self, want: bool | None) -> bool:
        if want is False:
            return False
        reason = self.persistent_unavailable_reason()
        if reason is not None:
            if want:
                raise ValueError(f"persistent decode unavailable: {reason}")
            return False
        cfg, lib, mlp = self.cfg, _lib.load(), self.mlp_xdna
        buf = lambda name: self.fc.get_buffer(name).torch_view(torch.uint8).data_ptr()  # noqa: E731
        descs = (_lib.LayerDesc * cfg.n_layers)()
        for i in range(cfg.n_layers):
            k, v = self._cache_ptrs(i)
            d = descs[i]
            d.wqkv, d.wo, d.wg, d.wu, d.wd = (buf(f"W_qkv_{i}"), buf(f"Wo_{i}"), buf(f"Wg_{i}"),
                                              buf(f"Wu_{i}"), buf(f"Wd_{i}"))
            d.n_in, d.n_post = buf(f"W_norm1_{i}"), buf(f"W_norm2_{i}")
            d.n_qn, d.n_kn = buf(f"W_qn_{i}"), buf(f"W_kn_{i}")
            d.k_cache, d.v_cache = k, v
            _lib.check(lib.iron_decode_persistent_check_layer(
                ctypes.byref(d), cfg.emb_dim, cfg.hidden_dim, cfg.n_heads, cfg.n_kv_heads,
                cfg.head_dim, cfg.group_size, QKV_TSI, mlp.tile_rows_o, mlp.tile_rows_gu,
                mlp.tile_rows_d, _lib.IRON_DOMAIN_SIGNED), f"layer {i}")
        self._p_layers = torch.frombuffer(bytearray(descs), dtype=torch.uint8).to(self.device)
        nbytes = lib.iron_decode_persistent_workspace(cfg.emb_dim, cfg.hidden_dim, cfg.n_heads,
                                                      cfg.n_kv_heads, cfg.head_dim)
        self._p_ws = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        self._p_xout = torch.zeros(cfg.emb_dim, dtype=torch.bfloat16, device=self.device)
        # the folded head's two argmax slots (launches alternate between them by epoch)
        self._p_keys = torch.zeros(2, dtype=torch.int64, device=self.device)
        torch.cuda.synchronize(self.device)
        return True

    def _persistent_launches(self):
        """The token's layers in one kernel, then the LM head with the final RMSNorm fused."""
        self.persistent_layers_launch()
        self.lm_head_launch()

    def persistent_layers_launch(self):
        """Launch iron_decode_persistent for the current position on the current stream."""
        cfg, lib, mlp = self.cfg, _lib.load(), self.mlp_xdna
        stream = torch.cuda.current_stream(self.device).cuda_stream
        view = lambda name, dt: self.fc.get_buffer(name).torch_view(dt)  # noqa: E731
        sh, st = self._kv_strides()
        _lib.check(lib.iron_decode_persistent(
            self._p_layers.data_ptr(), cfg.n_layers, cfg.emb_dim, cfg.hidden_dim, cfg.n_heads,
            cfg.n_kv_heads, cfg.head_dim, self.max_seq_len, sh, st, cfg.group_size, QKV_TSI,
            mlp.tile_rows_o, mlp.tile_rows_gu, mlp.tile_rows_d, _lib.IRON_DOMAIN_SIGNED,
            view("x", torch.bfloat16).data_ptr(), self._p_xout.data_ptr(),
            self.fc.params.tensor("k_cache_offset").data_ptr(),
            view("rope_row", torch.bfloat16).data_ptr(), float(cfg.eps),
            1.0 / math.sqrt(cfg.head_dim), self._p_ws.data_ptr(), self._p_ws.numel(), stream),
            "iron_decode_persistent")

    def persistent_gen_launch(self, keys, gs):
        """Launch iron_decode_persistent_gen: one greedy step's layers plus its token decode,
        embedding gather, token log and position advance; with ``keys`` the model's two folded
        argmax slots (``self._p_keys``), also the final norm, the LM head and its argmax."""
        cfg, lib, mlp = self.cfg, _lib.load(), self.mlp_xdna
        stream = torch.cuda.current_stream(self.device).cuda_stream
        view = lambda name, dt: self.fc.get_buffer(name).torch_view(dt)  # noqa: E731
        sh, st = self._kv_strides()
        gen = _lib.DecodeGen(keys=keys.data_ptr(), emb=self.embed.data_ptr(),
                             tokens=gs["tokens"].data_ptr(), token_log=gs["log"].data_ptr(),
                             step=gs["step"].data_ptr(),
                             ctx=self.fc.params.tensor("S_kv_eff").data_ptr(),
                             rope_table=self.rope_table.data_ptr(), vocab=cfg.vocab_size,
                             log_len=gs["log"].numel())
        if self.fold_lm_head and keys is self._p_keys:
            gen.lm_head = view("W_out_head", torch.uint8).data_ptr()
            gen.lm_norm = view("W_final_norm", torch.bfloat16).data_ptr()
            gen.logits = view("logits", torch.bfloat16).data_ptr()
        _lib.check(lib.iron_decode_persistent_gen(
            self._p_layers.data_ptr(), cfg.n_layers, cfg.emb_dim, cfg.hidden_dim, cfg.n_heads,
            cfg.n_kv_heads, cfg.head_dim, self.max_seq_len, sh, st, cfg.group_size, QKV_TSI,
            mlp.tile_rows_o, mlp.tile_rows_gu, mlp.tile_rows_d, _lib.IRON_DOMAIN_SIGNED,
            ctypes.byref(gen), self._p_xout.data_ptr(),
            self.fc.params.tensor("k_cache_offset").data_ptr(),
            view("rope_row", torch.bfloat16).data_ptr(), float(cfg.eps),
            1.0 / math.sqrt(cfg.head_dim), self._p_ws.data_ptr(), self._p_ws.numel(), stream),
            "iron_decode_persistent_gen")

    def lm_head_launch(self):
        """Final RMSNorm + LM head + argmax key over the persistent kernel's output."""
        cfg, lib = self.cfg, _lib.load()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        view = lambda name, dt: self.fc.get_buffer(name).torch_view(dt)  # noqa: E731
        head = view("W_out_head", torch.uint8).data_ptr()
        kind, G, tile = ((_lib.IRON_WEIGHT_BF16, 16, 1) if self.lm_head_kind == "bf16"
                         else (_lib.IRON_WEIGHT_INT8, cfg.group_size, LMHEAD_TSI))
        _lib.check(lib.iron_lm_head(
            head, kind, self._p_xout.data_ptr(), view("W_final_norm", torch.bfloat16).data_ptr(),
            float(cfg.eps), view("logits", torch.bfloat16).data_ptr(),
            view("argmax_key", torch.int64).data_ptr(), 1, cfg.vocab_size, cfg.emb_dim, G, tile,
            _lib.IRON_DOMAIN_SIGNED, stream), "iron_lm_head")

    def persistent_errors(self, clear: bool = True) -> int:
        """The persistent kernel's error word: bit 0, a hand-off wait timed out; bit 1, the
        workgroups with equal index mod 8 did not share an XCD, which the XCD-local hand-offs
        of the Qwen3-0.6B shape assume."""
        if not self.persistent:
            return 0
        word = self._p_ws[4:8].view(torch.int32)
        err = int(word.item())
        if err and clear:
            word.zero_()
        return err

    def _persistent_check(self):
        err = self.persistent_errors()
        if err:
            what = "a hand-off wait timed out" if err & 1 else ""
            if err & 2:
                what += ("; " if what else "") + "workgroups with equal index mod 8 ran on " \
                        "different XCDs"
            raise RuntimeError(f"iron_decode_persistent: {what} (flags {err:#x}); the token's "
                               "outputs are invalid")

    # ---------------- state helpers ----------------
    def kv_caches(self, layer: int):
        """(K, V) device views of one layer's cache, each (Hkv, max_seq, HD)."""
        cfg, S = self.cfg, self.max_seq_len
        if self.kv_layout == "separate":
            k = self.fc.get_buffer(f"k_cache_{layer}").torch_view(torch.bfloat16)
            v = self.fc.get_buffer(f"v_cache_{layer}").torch_view(torch.bfloat16)
            shape = (cfg.n_kv_heads, S, cfg.head_dim)
            return k[: np.prod(shape)].reshape(shape), v[: np.prod(shape)].reshape(shape)
        kv = self.fc.get_buffer(f"kv_cache_{layer}").torch_view(torch.bfloat16)
        t = kv[: cfg.n_kv_heads * S * 2 * cfg.head_dim].reshape(cfg.n_kv_heads, S, 2, cfg.head_dim)
        return t[:, :, 0], t[:, :, 1]

    def load_kv(self, k: torch.Tensor, v: torch.Tensor):
        """Write (n_layers, Hkv, P, HD) K/V into positions [0, P) of every layer's cache."""
        P = k.shape[2]
        for i in range(self.cfg.n_layers):
            kc, vc = self.kv_caches(i)
            kc[:, :P].copy_(k[i].to(self.device))
            vc[:, :P].copy_(v[i].to(self.device))
        torch.cuda.synchronize(self.device)

    def _per_token_offset(self) -> int:
        return self.cfg.head_dim * (1 if self.kv_layout == "separate" else 2)

    def _set_position(self, seq_pos: int):
        HD = self.cfg.head_dim
        self.fc.get_buffer("rope_row").torch_view(torch.bfloat16)[:HD].copy_(
            self.rope_table[seq_pos * HD:(seq_pos + 1) * HD])
        self.fc.params.write("k_cache_offset", seq_pos * self._per_token_offset())
        self.fc.params.write("S_kv_eff", seq_pos + 1)
        self.fc.params.sync()

    def logits(self) -> torch.Tensor:
        return self.fc.get_buffer("logits").torch_view(torch.bfloat16)[: self.cfg.vocab_size].cpu()

    # ---------------- forward (single token) ----------------
    def __call__(self, x, seq_pos: int) -> int:
        """x: (emb_dim,) bf16 hidden state of the new token; returns the argmax token id."""
        if seq_pos >= self.max_seq_len:
            raise ValueError(f"seq_pos {seq_pos} >= max_seq_len {self.max_seq_len}")
        self.fc.get_buffer("x").torch_view(torch.bfloat16)[: self.cfg.emb_dim].copy_(
            torch.as_tensor(x).reshape(-1).to(self.device, torch.bfloat16))
        self.fc.get_buffer("argmax_key").torch_view(torch.int64).zero_()
        self._set_position(seq_pos)
        if self.persistent:
            self._persistent_launches()
            torch.cuda.synchronize(self.device)
            self._persistent_check()
        else:
            self.fc()
        key = int(self.fc.get_buffer("argmax_key").torch_view(torch.int64)[0].item())
        return _decode_key(key)

    def step_token(self, token: int, seq_pos: int) -> int:
        """Embedding lookup + one decode step."""
        D = self.cfg.emb_dim
        return self(self.embed[int(token) * D:(int(token) + 1) * D], seq_pos)

    # ---------------- device-resident greedy decoding ----------------
    def _gen_state(self):
        if getattr(self, "_gs", None) is None:
            dev = self.device
            self._gs = {"tokens": torch.zeros(1, dtype=torch.int32, device=dev),
                        "step": torch.zeros(1, dtype=torch.int32, device=dev),
                        "log": torch.zeros(self.max_seq_len + 1, dtype=torch.int32, device=dev)}
        return self._gs

    def _gen_step_launches(self):
        cfg, gs = self.cfg, self._gen_state()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        keys = self.fc.get_buffer("argmax_key").torch_view(torch.int64)
        if self.persistent:
            # token decode, embedding, log and position advance inside the layers' kernel, and
            # with the folded head the LM head as well: one launch per token
            if self.fold_lm_head:
                self.persistent_gen_launch(self._p_keys, gs)
                return
            self.persistent_gen_launch(keys, gs)
            self.lm_head_launch()
            return
        x = self.fc.get_buffer("x").torch_view(torch.bfloat16)
        _lib.call("iron_next_token", keys.data_ptr(), gs["tokens"].data_ptr(),
                  self.embed.data_ptr(), x.data_ptr(), gs["log"].data_ptr(), 0,
                  gs["log"].numel(), gs["step"].data_ptr(), 1, cfg.emb_dim, cfg.vocab_size,
                  stream)
        self.fc.run_steps()
        _lib.call("iron_advance_positions", self.fc.params.tensor("k_cache_offset").data_ptr(),
                  self.fc.params.tensor("S_kv_eff").data_ptr(), self.rope_table.data_ptr(),
                  self.fc.get_buffer("rope_row").torch_view(torch.bfloat16).data_ptr(),
                  cfg.head_dim, self.max_seq_len, 1, 1, stream)

    # Token steps per replay of the batched generation graph. Every step's state (the argmax key,
    # the position, the epoch) advances on the device, so a graph of several launches runs the
    # same greedy chain; one replay per 16 tokens instead of one per token measured 503 -> 498 us
    # per token (the gap between consecutive graph launches).
    GEN_BATCH = 16

    def _capture_gen_graph(self):
        # State tensors must exist before capture: a tensor created inside the capture would
        # come from the graph's pool and its zero-fill would be recorded into every replay.
        self._gen_state()

        def capture(steps: int):
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream(self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.graph(g, stream=s):
                for _ in range(steps):
                    self._gen_step_launches()
            torch.cuda.current_stream(self.device).wait_stream(s)
            return g

        self._gen_graph = capture(1)
        # the runlist path's token is ~100 launches: it keeps one graph per token
        self._gen_graph_batch = capture(self.GEN_BATCH) if self.persistent else None

    def start_generation(self, first_token: int, start_pos: int):
        """Arm the device loop: the next step consumes ``first_token`` at ``start_pos``."""
        if self._gen_graph is None:
            self._capture_gen_graph()
        gs = self._gen_state()
        if not 0 <= start_pos < self.max_seq_len:
            raise ValueError(f"start position {start_pos} outside [0, {self.max_seq_len})")
        gs["step"].zero_()
        self._gen_pos = start_pos
        self._set_position(start_pos)
        if self.fold_lm_head:
            # the next launch (epoch e) reads keys[e & 1] and clears keys[(e + 1) & 1]
            e = self._epoch()
            self._p_keys[e & 1].fill_(_encode_token(first_token))
            self._p_keys[(e + 1) & 1].zero_()
        else:
            self.fc.get_buffer("argmax_key").torch_view(torch.int64)[:1].fill_(
                _encode_token(first_token))
        torch.cuda.synchronize(self.device)

    def _epoch(self) -> int:
        """The persistent workspace's epoch (control word 0): the next launch's."""
        return int(self._p_ws[:4].view(torch.int32).item()) & 0xFFFFFFFF

    def decode_steps(self, n: int):
        """Run n token steps by graph replays (no host synchronisation): on the persistent path
        n // GEN_BATCH replays of the batched graph, then single-token replays.

        Step i consumes the token at position start_pos + i, so every step's position must stay
        below max_seq_len (the KV caches and the token log are sized by it)."""
        if self._gen_graph is None or self._gen_pos is None:
            raise RuntimeError("decode_steps() before start_generation()")
        if self._gen_pos + n > self.max_seq_len:
            raise ValueError(f"{n} steps from position {self._gen_pos} pass max_seq_len "
                             f"{self.max_seq_len}")
        rest = n
        if self._gen_graph_batch is not None:
            for _ in range(n // self.GEN_BATCH):
                self._gen_graph_batch.replay()
            rest = n % self.GEN_BATCH
        for _ in range(rest):
            self._gen_graph.replay()
        self._gen_pos += n

    def finish_generation(self) -> list[int]:
        """Tokens produced since start_generation (the last one decoded from the final key)."""
        cfg, gs = self.cfg, self._gen_state()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        keys = self.fc.get_buffer("argmax_key").torch_view(torch.int64)
        if self.fold_lm_head:
            torch.cuda.synchronize(self.device)
            keys = self._p_keys[self._epoch() & 1:]   # the last launch's argmax slot
        _lib.call("iron_next_token", keys.data_ptr(), gs["tokens"].data_ptr(), None, None,
                  gs["log"].data_ptr(), 0, gs["log"].numel(), gs["step"].data_ptr(), 1,
                  cfg.emb_dim, cfg.vocab_size, stream)
        torch.cuda.synchronize(self.device)
        self._persistent_check()
        n = int(gs["step"].item())
        # log[0] is the armed first token; log[1..n-1] are the generated ones
        return gs["log"][1:n].cpu().tolist()

    def generate(self, prompt_ids, n_new: int, start_pos: int = 0) -> list[int]:
        """Greedy decode: prefill ``prompt_ids`` token by token from ``start_pos``, then produce
        ``n_new`` tokens on the device. Returns the generated token ids."""
        prompt_ids = list(prompt_ids)
        if not prompt_ids:
            raise ValueError("generate() needs at least one prompt token")
        last = start_pos + len(prompt_ids) - 1 + n_new
        if start_pos < 0 or last > self.max_seq_len:
            raise ValueError(f"{len(prompt_ids)} prompt + {n_new} new tokens from position "
                             f"{start_pos} need max_seq_len >= {last} (it is {self.max_seq_len})")
        pos = start_pos
        for tok in prompt_ids[:-1]:
            self.step_token(tok, pos)
            pos += 1
        self.start_generation(prompt_ids[-1], pos)
        self.decode_steps(n_new)
        return self.finish_generation()
