"""OperatorSequence: a runlist of operators over named device buffers, run as one dispatch.

Mirrors the reference's sequence API (iron/common/sequence.py:270-559 for the operator,
:578-1085 for the callables): ``OperatorSequence(name, runlist, input_args, output_args,
buffer_sizes, dispatch, ...)`` where ``runlist`` is ``[(op, *buffer_names), ...]``; the callable
exposes ``get_buffer(name).torch_view()``, ``params.write(name, value)`` / ``params.sync()``,
``__call__()`` and ``sync_independent_buffers()``.

gfx950 mapping of the dispatch modes:
  * ``"fused"`` (what ``"auto"`` resolves to) -- the whole runlist is captured once into a HIP
    graph and each call replays it: one dispatch per call, the analogue of the reference's
    single full-ELF dispatch (sequence.py:858-862). Runtime parameters are device int32 tensors,
    so replays see new values without re-capture.
  * ``"separate"`` -- every step launches eagerly on the current stream (no graph).
  * ``"reference"`` -- CPU buffers, each step's ``op.reference()`` (needs a registered golden
    provider; there is no built-in CPU path), bf16 cast per output (sequence.py:972-999).
  * ``"compare"`` -- eager HIP steps; after each one the step's reference output on the same
    inputs is compared and a mismatch logged or raised (sequence.py:1002-1085).

Buffers live in device arenas laid out like the reference's (``input`` / ``output`` /
``scratch`` plus one per independent buffer, 64-byte aligned offsets); slices
``"name[start:end]"`` are byte ranges of an explicitly sized parent.
"""

from __future__ import annotations

import logging
import time

import numpy as np
import torch

from .base import AIEOperatorBase, AIERuntimeArgSpec, MLIROperator

logger = logging.getLogger(__name__)


class SequenceDispatch:
    name = None

    def resolve(self):
        return self

    def make_callable(self, seq):
        raise NotImplementedError


class FusedDispatch(SequenceDispatch):
    name = "fused"

    def make_callable(self, seq):
        return SequenceHipCallable(seq, use_graph=True)


class AutoDispatch(SequenceDispatch):
    name = "auto"

    def resolve(self):
        return FusedDispatch()


class SeparateDispatch(SequenceDispatch):
    name = "separate"

    def make_callable(self, seq):
        return SequenceHipCallable(seq, use_graph=False)


class ReferenceDispatch(SequenceDispatch):
    name = "reference"

    def make_callable(self, seq):
        return SequenceReferenceCallable(seq)


class CompareDispatch(SequenceDispatch):
    name = "compare"

    def __init__(self, rel_tol=0.05, abs_tol=0.05, raise_on_mismatch=True):
        self.rel_tol = rel_tol
        self.abs_tol = abs_tol
        self.raise_on_mismatch = raise_on_mismatch

    def make_callable(self, seq):
        return SequenceCompareCallable(seq, self)


_DISPATCH_ALIASES = {
    "auto": AutoDispatch,
    "fused": FusedDispatch,
    "separate": SeparateDispatch,
    "compare": CompareDispatch,
    "reference": ReferenceDispatch,
}


def _align(n: int, a: int = 64) -> int:
    return (n + a - 1) & ~(a - 1)


class OperatorSequence(AIEOperatorBase):
    def __init__(self, name, runlist, input_args, output_args, buffer_sizes=None,
                 dispatch="auto", extra_flags=None, share_designs=False,
                 independent_buffer_args=None, independent_buffer_groups=None, context=None):
        dispatch = self._coerce_dispatch(dispatch)
        if not all(isinstance(op, MLIROperator) and all(isinstance(b, str) for b in bufs)
                   for op, *bufs in runlist):
            raise TypeError("OperatorSequence: every runlist entry is an operator (an "
                            "MLIROperator) followed by its buffer names (strings)")
        super().__init__(context)
        self.runlist = runlist
        self.name = name + "_shared" if share_designs else name
        self.input_args = list(input_args)
        self.output_args = list(output_args)
        self.explicit_buffer_sizes = dict(buffer_sizes or {})
        self.independent_buffer_args = list(independent_buffer_args or [])
        self.independent_buffer_groups = dict(independent_buffer_groups or {})
        self.extra_flags = extra_flags or []
        self.share_designs = share_designs
        self._dispatch = dispatch
        self.subbuffer_layout = None

    @staticmethod
    def _coerce_dispatch(dispatch):
        if isinstance(dispatch, SequenceDispatch):
            return dispatch
        if isinstance(dispatch, str) and dispatch in _DISPATCH_ALIASES:
            return _DISPATCH_ALIASES[dispatch]()
        raise TypeError(f"OperatorSequence: unknown dispatch {dispatch!r} (one of "
                        f"{sorted(_DISPATCH_ALIASES)} or a SequenceDispatch)")

    def unique_operators(self):
        seen = {}
        for op, *_ in self.runlist:
            seen.setdefault(id(op), op)
        return list(seen.values())

    def calculate_buffer_layout(self):
        """(subbuffer_layout, buffer_sizes, slice_info, independent_order, independent_sizes)
        with the reference's conventions (sequence.py:384-516); specs carry their dtype."""
        args: dict[str, AIERuntimeArgSpec] = {}
        sliced: dict[str, tuple] = {}
        for op, *bufs in self.runlist:
            specs = op.get_arg_spec()
            if len(specs) != len(bufs):
                raise ValueError(f"{op!r} declares {len(specs)} arguments but its runlist "
                                 f"entry names {len(bufs)} buffers")
            for buf, spec in zip(bufs, specs):
                if "[" in buf and buf.endswith("]"):
                    base = buf[: buf.index("[")]
                    start, end = map(int, buf[buf.index("[") + 1: -1].split(":"))
                    if base not in args and base not in self.explicit_buffer_sizes:
                        raise ValueError(f"slice {buf!r}: its parent {base!r} needs a size in "
                                         "buffer_sizes")
                    sliced[buf] = (base, start, end, spec)
                elif buf not in args:
                    args[buf] = spec
                elif args[buf].nbytes != spec.nbytes:
                    raise ValueError(f"buffer {buf!r} is declared with two sizes "
                                     f"({args[buf].shape} and {spec.shape}) by different steps")
        names = set(args) | set(sliced)
        for a in self.input_args:
            if a not in names and a not in self.explicit_buffer_sizes:
                raise ValueError(f"input_args names {a!r}, which no runlist step uses")
        for a in self.output_args:
            if a not in names and a not in self.explicit_buffer_sizes:
                raise ValueError(f"output_args names {a!r}, which no runlist step uses")
        layout, slice_info = {}, {}
        self._specs = args

        def add(btype, names_):
            off = 0
            for a in names_:
                if a in self.explicit_buffer_sizes:
                    length = int(self.explicit_buffer_sizes[a])
                elif a in args:
                    length = args[a].nbytes
                else:
                    continue
                layout[a] = (btype, off, length)
                off += _align(length)
            return off

        for buf, (base, start, end, _) in sliced.items():
            slice_info[buf] = (base, start, end)
        indep = set(self.independent_buffer_args)
        in_size = add("input", [a for a in self.input_args if a not in indep])
        out_size = add("output", self.output_args)
        scratch = [a for a in args if a not in self.input_args and a not in self.output_args
                   and a not in indep]
        scratch += [a for a in self.explicit_buffer_sizes if a not in self.input_args
                    and a not in self.output_args and a not in scratch and a not in indep]
        scratch_size = add("scratch", scratch)
        indep_order = list(self.independent_buffer_args)
        indep_sizes = [add(n, [n]) for n in indep_order]
        return layout, (in_size, out_size, scratch_size), slice_info, indep_order, indep_sizes

    def set_up_artifacts(self):
        (self.subbuffer_layout, self.buffer_sizes, self.slice_info, self.independent_order,
         self.independent_sizes) = self.calculate_buffer_layout()
        self._dispatch = self._dispatch.resolve()

    def compile(self, dry_run: bool = False):
        self.set_up_artifacts()
        return super().compile(dry_run)

    def get_arg_spec(self):
        raise NotImplementedError("a sequence has per-buffer layouts, not one argument list: "
                                  "see get_layout_for_buffer()")

    def get_callable(self):
        if self.subbuffer_layout is None:
            self.compile()
        return self._dispatch.make_callable(self)

    def get_layout_for_buffer(self, buffer_name):
        if buffer_name in self.slice_info:
            base, start, end = self.slice_info[buffer_name]
            btype, pstart, _ = self.get_layout_for_buffer(base)
            return btype, pstart + start, pstart + end
        return self.subbuffer_layout[buffer_name]

    def buffer_dtype(self, buffer_name) -> torch.dtype:
        base = buffer_name[: buffer_name.index("[")] if "[" in buffer_name else buffer_name
        spec = self._specs.get(base)
        return spec.dtype if spec is not None else torch.bfloat16


class DeviceBuffer:
    """A named buffer: a typed view into its arena (the reference's XRTSubBuffer role)."""

    def __init__(self, arena: torch.Tensor, offset: int, length: int, dtype: torch.dtype):
        self._bytes = arena[offset: offset + length]
        self.dtype = dtype

    def torch_view(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        dt = dtype or self.dtype
        es = torch.empty((), dtype=dt).element_size()
        n = self._bytes.numel() // es
        return self._bytes[: n * es].view(dt)

    @property
    def data(self):
        return self.torch_view()

    def to(self, _where):
        return self


class SequenceCallable:
    """Shared step iteration / timing for the runtime callables."""

    def __init__(self, op: OperatorSequence):
        self.op = op
        self.last_elapsed = 0.0
        self._buffer_cache = {}
        self._allocate_buffers()

    def _iter_steps(self):
        for step_op, *names in self.op.runlist:
            specs = step_op.get_arg_spec()
            if len(specs) != len(names):
                raise ValueError(f"{step_op!r} declares {len(specs)} arguments but its runlist "
                                 f"entry names {len(names)} buffers")
            yield step_op, names, specs

    def __call__(self):
        t0 = time.perf_counter()
        self._run()
        self.last_elapsed = time.perf_counter() - t0


class SequenceHipCallable(SequenceCallable):
    """Device-arena buffers; eager launches or one captured HIP graph per call."""

    def __init__(self, op: OperatorSequence, use_graph: bool = True):
        from ..operators._common import RuntimeParams

        self.device = op.context.device
        self.params = RuntimeParams(self.device)
        self.use_graph = use_graph
        self._graph = None
        super().__init__(op)
        self._fns = {}
        for step_op in op.unique_operators():
            try:
                fn = step_op.get_callable(params=self.params)
            except TypeError:
                fn = step_op.get_callable()
            self._fns[id(step_op)] = fn
        self._plan = []
        for step_op, names, specs in self._iter_steps():
            views = [self._typed(self.get_buffer(n), s) for n, s in zip(names, specs)]
            self._plan.append((self._fns[id(step_op)], views))

    @staticmethod
    def _typed(buf: DeviceBuffer, spec: AIERuntimeArgSpec) -> torch.Tensor:
        t = buf.torch_view(spec.dtype)
        return t[: spec.numel]

    def _allocate_buffers(self):
        in_sz, out_sz, scratch_sz = self.op.buffer_sizes
        mk = lambda n: torch.zeros(max(_align(n, 256), 256), dtype=torch.uint8,  # noqa: E731
                                   device=self.device)
        self.input_buffer, self.output_buffer, self.scratch_buffer = mk(in_sz), mk(out_sz), mk(
            scratch_sz)
        self.independent_buffers = {n: mk(sz) for n, sz in
                                    zip(self.op.independent_order, self.op.independent_sizes)}

    def get_buffer(self, buffer_name) -> DeviceBuffer:
        if buffer_name in self._buffer_cache:
            return self._buffer_cache[buffer_name]
        btype, off, length = self.op.get_layout_for_buffer(buffer_name)
        if btype in self.independent_buffers:
            arena = self.independent_buffers[btype]
        else:
            arena = {"input": self.input_buffer, "output": self.output_buffer,
                     "scratch": self.scratch_buffer}[btype]
        buf = DeviceBuffer(arena, off, length, self.op.buffer_dtype(buffer_name))
        self._buffer_cache[buffer_name] = buf
        return buf

    def sync_independent_buffers(self):
        """Buffers are device-resident; kept for the reference's call shape."""

    def run_steps(self):
        """Launch every step on the current stream (also what a graph capture records)."""
        for fn, views in self._plan:
            fn(*views)

    def _capture(self):
        # No warm-up run: steps mutate state in place (the residual, the KV cache), and every
        # workspace already exists, so the capture itself allocates nothing.
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.graph(g, stream=stream):
            self.run_steps()
        torch.cuda.current_stream(self.device).wait_stream(stream)
        self._graph = g

    def _run(self):
        if not self.use_graph:
            self.run_steps()
        else:
            if self._graph is None:
                self._capture()
            self._graph.replay()
        torch.cuda.current_stream(self.device).synchronize()


class SequenceReferenceCallable(SequenceCallable):
    """CPU evaluation through each operator's ``reference()`` (needs a golden provider).

    A step's inputs are copies of its buffers; its ``out`` / ``inout`` arguments other than the
    last are passed as the buffers themselves, so a golden that updates them (a KV-cache append,
    the logits beside an argmax key) leaves its effect for later steps. The runtime parameters
    (positions, context lengths, converted as the device callables convert them) go to the golden
    as ``params``, and an ``inout`` last argument's pre-step value as ``last``."""

    def _allocate_buffers(self):
        in_sz, out_sz, scratch_sz = self.op.buffer_sizes
        self._arenas = {"input": torch.zeros(max(in_sz, 2), dtype=torch.uint8),
                        "output": torch.zeros(max(out_sz, 2), dtype=torch.uint8),
                        "scratch": torch.zeros(max(scratch_sz, 2), dtype=torch.uint8)}
        for n, sz in zip(self.op.independent_order, self.op.independent_sizes):
            self._arenas[n] = torch.zeros(max(sz, 2), dtype=torch.uint8)
        self.params = _HostParams()
        for step_op in self.op.unique_operators():
            pname = getattr(step_op, "kv_offset_parameter", None)
            conv = getattr(step_op, "offset_to_position", None)
            if pname and conv is not None:
                self.params.define(pname, convert=conv)

    def get_buffer(self, buffer_name) -> DeviceBuffer:
        if buffer_name not in self._buffer_cache:
            btype, off, length = self.op.get_layout_for_buffer(buffer_name)
            self._buffer_cache[buffer_name] = DeviceBuffer(self._arenas[btype], off, length,
                                                           self.op.buffer_dtype(buffer_name))
        return self._buffer_cache[buffer_name]

    def sync_independent_buffers(self):
        pass

    def _view(self, name, spec):
        return self.get_buffer(name).torch_view(spec.dtype)[: spec.numel].reshape(spec.shape)

    def _run(self):
        for step_op, names, specs in self._iter_steps():
            *in_names, out_name = names
            *in_specs, out_spec = specs
            inputs = [self._view(n, s) if s.direction in ("out", "inout")
                      else self._view(n, s).clone() for n, s in zip(in_names, in_specs)]
            kw = {"params": self.params.snapshot()}
            if out_spec.direction == "inout":
                kw["last"] = self._view(out_name, out_spec).clone()
            out = step_op.reference(*inputs, **kw)
            dst = self.get_buffer(out_name).torch_view(out_spec.dtype)
            flat = out.reshape(-1).to(out_spec.dtype)
            dst[: flat.numel()].copy_(flat)


class _HostParams:
    """Runtime parameters of the reference dispatch (host values, same conversions)."""

    def __init__(self):
        self.values = {}
        self._convert = {}

    def define(self, name, n=1, convert=None):
        if convert is not None:
            self._convert[name] = convert

    def write(self, name, value):
        conv = self._convert.get(name)
        if conv is not None:
            value = conv(value)
        self.values[name] = np.atleast_1d(np.asarray(value, dtype=np.int64))

    def read(self, name):
        return self.values[name]

    def snapshot(self) -> dict:
        return dict(self.values)

    def sync(self):
        pass

    def __contains__(self, name):
        return name in self.values


class SequenceCompareCallable(SequenceHipCallable):
    """Eager HIP steps, each checked against its reference on the same device inputs."""

    def __init__(self, op: OperatorSequence, dispatch: CompareDispatch):
        self.rel_tol = dispatch.rel_tol
        self.abs_tol = dispatch.abs_tol
        self.raise_on_mismatch = dispatch.raise_on_mismatch
        self.last_step_stats = []
        super().__init__(op, use_graph=False)

    def _run(self):
        self.last_step_stats = []
        for idx, ((fn, views), (step_op, names, specs)) in enumerate(
                zip(self._plan, self._iter_steps())):
            cpu_inputs = [v.reshape(s.shape).cpu().clone() for v, s in zip(views[:-1], specs[:-1])]
            kw = {"params": self.params.snapshot()}
            if specs[-1].direction == "inout":
                kw["last"] = views[-1].reshape(specs[-1].shape).cpu().clone()
            fn(*views)
            torch.cuda.synchronize(self.device)
            ref = step_op.reference(*cpu_inputs, **kw).reshape(-1)
            if specs[-1].dtype.is_floating_point:
                dev_out = views[-1].reshape(-1).float().cpu()
                ref = ref.float()
                n = min(ref.numel(), dev_out.numel())
                diff = (dev_out[:n] - ref[:n]).abs()
                max_abs = float(diff.max()) if n else 0.0
                max_rel = float((diff / (ref[:n].abs() + 1e-6)).max()) if n else 0.0
                fail = (max_abs > self.abs_tol) and (max_rel > self.rel_tol)
            else:
                # integer outputs (argmax keys) must match exactly
                dev_out = views[-1].reshape(-1).cpu().to(torch.int64)
                ref = ref.to(torch.int64)
                n = min(ref.numel(), dev_out.numel())
                fail = not torch.equal(dev_out[:n], ref[:n])
                max_abs = max_rel = float(fail)
            stats = {"step": idx, "op": type(step_op).__name__, "output": names[-1],
                     "max_abs": max_abs, "max_rel": max_rel, "mismatch": fail}
            logger.log(logging.ERROR if fail else logging.INFO,
                       "[compare step %d] %s -> %s: max_abs=%.4g max_rel=%.4g%s", idx,
                       stats["op"], names[-1], max_abs, max_rel, "  MISMATCH" if fail else "")
            self.last_step_stats.append(stats)
            if fail and self.raise_on_mismatch:
                raise RuntimeError(
                    f"[compare step {idx}] {stats['op']} -> {names[-1]}: device output deviates "
                    f"from reference (max_abs={max_abs:.4g}, max_rel={max_rel:.4g}; "
                    f"tolerances abs_tol={self.abs_tol}, rel_tol={self.rel_tol})")
