"""Buffer comparison and the single-operator test harness.

``verify_buffer`` keeps the reference's tolerance semantics exactly (iron/common/test_utils.py:
51-126): an element fails when ``|out - ref| > max(abs_tol, rel_tol * (|out| + |ref|))`` -- a
strict ``>`` so that ``rel_tol = abs_tol = 0`` means exact equality. ``run_test`` mirrors the
reference harness (test_utils.py:140-246): it allocates device buffers from the operator's arg
spec, runs warm-up and timed iterations (HIP events on the operator's stream), and verifies the
outputs.
"""

from __future__ import annotations

import numpy as np
import torch

from .base import AIEOperatorBase

torch_dtype_map = {
    "bf16": torch.bfloat16,
    "f32": torch.float32,
    "i8": torch.int8,
    "ui8": torch.uint8,
    "i16": torch.int16,
    "i32": torch.int32,
}


def _to_f64(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().to("cpu").to(torch.float64).contiguous().numpy().reshape(-1)
    return np.asarray(x, dtype=np.float64).reshape(-1)


def verify_buffer(output, buf_name: str, reference, rel_tol: float = 0.04, abs_tol: float = 1e-6,
                  max_error_rate: float = 0.0) -> list[int]:
    expected = _to_f64(reference)
    out = _to_f64(output)
    errors: list[int] = []
    if len(out) < len(expected):
        print(f"Buffer size mismatch for {buf_name}: expected {len(expected)}, got {len(out)}")
        errors.extend(range(len(expected) - len(out)))
    n = min(len(out), len(expected))
    diff = np.abs(out[:n] - expected[:n])
    norm = np.minimum(np.abs(out[:n]) + np.abs(expected[:n]), np.finfo(np.float32).max)
    with np.errstate(invalid="ignore"):
        mask = ~(diff <= np.maximum(abs_tol, rel_tol * norm))  # NaN counts as a mismatch
    idx = np.where(mask)[0].tolist()
    for i in idx[:10]:
        print(f"Mismatch in {buf_name}[{i}]: expected {expected[i]:.6f}, got {out[i]:.6f}")
    errors.extend(idx)
    if max_error_rate > 0.0 and errors:
        allowed = int(n * max_error_rate)
        if len(errors) <= allowed:
            print(f"{buf_name}: {len(errors)} errors within allowed rate {max_error_rate:.2%}")
            return []
        print(f"{buf_name}: {len(errors)} errors exceed allowed rate {max_error_rate:.2%}")
    return errors


def run_test(operator: AIEOperatorBase, input_buffers: dict, output_buffers: dict,
             rel_tol: float = 0.04, abs_tol: float = 1e-6, max_error_rate: float = 0.0,
             warmup_iters: int = 1, timed_iters: int = 1):
    """Run ``operator`` on device copies of ``input_buffers``; verify ``output_buffers``.

    Returns ``(errors, latency_us, bandwidth_gbps)`` like the reference harness, where the
    bandwidth counts every argument's bytes once per call.
    """
    if not isinstance(operator, AIEOperatorBase):
        raise ValueError("run_test only supports AIEOperatorBase subclasses")
    operator.compile()
    fn = operator.get_callable()
    dev = operator.context.device
    args, outputs, total_bytes = [], {}, 0
    in_iter, out_iter = iter(input_buffers.items()), iter(output_buffers.items())
    for spec in operator.get_arg_spec():
        if spec.direction in ("in", "inout"):
            try:
                name, data = next(in_iter)
            except StopIteration:
                raise ValueError("Not enough input buffers provided for arg spec") from None
            t = data.to(dev).contiguous().clone()
            if spec.direction == "inout":
                outputs[name] = t
        else:
            try:
                name, _ = next(out_iter)
            except StopIteration:
                raise ValueError("Not enough output buffers provided for arg spec") from None
            t = torch.zeros(spec.shape, dtype=spec.dtype, device=dev)
            outputs[name] = t
        args.append(t)
        total_bytes += t.numel() * t.element_size()
    for _ in range(warmup_iters):
        fn(*args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(timed_iters):
        fn(*args)
    end.record()
    end.synchronize()
    latency_us = start.elapsed_time(end) * 1e3 / max(timed_iters, 1)
    errors = {}
    for name, expected in output_buffers.items():
        if expected is None:
            continue
        if name not in outputs:
            print(f"Warning: Output buffer {name} not found in operator arguments")
            continue
        e = verify_buffer(outputs[name], name, expected, rel_tol, abs_tol, max_error_rate)
        if e:
            errors[name] = e
    bandwidth_gbps = total_bytes / (latency_us * 1e-6) / 1e9 if latency_us > 0 else 0.0
    return errors, latency_us, bandwidth_gbps
