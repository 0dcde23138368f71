"""Operator base classes and the runtime argument-spec contract.

Mirrors the reference's operator API (iron/common/base.py:31-216): ``AIEOperatorBase`` with
``compile()`` / ``get_arg_spec()`` / ``get_callable()``, ``MLIROperator.name`` derived from the
dataclass fields and ``_name_aliases``, and ``AIERuntimeArgSpec(direction, shape, dtype)``. The
class names are kept so reference callers switch by changing the import; the NPU artifact graph
(MLIR generation, Peano, aiecc) has no counterpart here -- ``compile()`` loads the prebuilt HIP
library instead.

``reference()`` goldens are not part of the product: a test harness registers a provider with
:func:`register_reference_provider` (the repository's ``oracle`` package does), and an operator
without one raises instead of silently falling back to a CPU path.
"""

from __future__ import annotations

import dataclasses
from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any, Callable, ClassVar

import torch

from .context import AIEContext

DEVICE_NAME = "gfx950"

_REFERENCE_PROVIDER: Callable[..., Any] | None = None


def register_reference_provider(provider: Callable[..., Any] | None) -> None:
    """Install ``provider(op, *inputs, **context) -> output`` as the source of
    ``op.reference()`` (``context``: ``params`` and ``last`` inside a sequence)."""
    global _REFERENCE_PROVIDER
    _REFERENCE_PROVIDER = provider


def reference_provider() -> Callable[..., Any] | None:
    return _REFERENCE_PROVIDER


@dataclass(frozen=True)
class AIERuntimeArgSpec:
    """One runtime argument of an operator (iron/common/base.py:203-216).

    ``dtype`` is a torch dtype (bf16 by default, as in the reference); weight wires are declared
    as the reference declares them, i.e. as a bf16 view of the packed bytes.
    """

    direction: str
    shape: tuple[int, ...]
    dtype: torch.dtype = torch.bfloat16

    def __post_init__(self) -> None:
        if self.direction not in {"in", "out", "inout"}:
            raise ValueError(
                f"argument direction {self.direction!r} is not 'in', 'out' or 'inout'"
            )

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    @property
    def nbytes(self) -> int:
        return self.numel * torch.empty((), dtype=self.dtype).element_size()


class AIEOperatorBase(ABC):
    """Base class of every operator (iron/common/base.py:31-88)."""

    _default_context: ClassVar[AIEContext | None] = None

    def __init__(self, context: AIEContext | None = None) -> None:
        if context is None:
            context = self.get_default_context()
        self.context = context

    @classmethod
    def get_default_context(cls) -> AIEContext:
        """Process-wide default context, created on first use (lazy singleton)."""
        if AIEOperatorBase._default_context is None:
            AIEOperatorBase._default_context = AIEContext()
        return AIEOperatorBase._default_context

    def set_up_artifacts(self) -> None:
        """No artifact graph: the kernels are prebuilt into libiron_hip.so."""

    def compile(self, dry_run: bool = False) -> "AIEOperatorBase":
        """Check the operator against the HIP library (loads it unless ``dry_run``)."""
        if not dry_run:
            from .. import _lib

            _lib.load()
        return self

    @abstractmethod
    def get_arg_spec(self) -> list[AIERuntimeArgSpec]:
        ...

    @abstractmethod
    def get_callable(self) -> Callable[..., Any]:
        ...


def _serialize_param(v: object) -> str:
    if isinstance(v, bool):
        return str(int(v))
    if isinstance(v, float):
        return f"{v:g}".replace(".", "p").replace("-", "m")
    if isinstance(v, (list, tuple)):
        return "x".join(str(x) for x in v)
    return str(v)


class MLIROperator(AIEOperatorBase):
    """Dataclass-driven operator (the reference's MLIROperator, iron/common/base.py:91-193).

    The class keeps its reference name so code written against the reference's operator classes
    resolves unchanged; here it describes a set of HIP kernels, not an MLIR design.
    """

    _name_aliases: ClassVar[dict[str, str]] = {
        "num_aie_columns": "c",
        "num_channels": "ch",
        "tile_size": "t",
        "size": "sz",
        "scalar_factor": "sf",
        "rows": "r",
        "cols": "n",
    }

    @property
    def name(self) -> str:
        if not dataclasses.is_dataclass(self):
            raise NotImplementedError(
                f"{type(self).__name__}: the operator name is built from dataclass fields; "
                "declare the class with @dataclass or define its own name"
            )
        aliases = type(self)._name_aliases
        parts = (
            f"{aliases.get(f.name, f.name)}{_serialize_param(getattr(self, f.name))}"
            for f in dataclasses.fields(self)
            if f.repr and getattr(self, f.name) is not None
        )
        return type(self).__name__ + "_" + "_".join(parts) + f"_{DEVICE_NAME}"

    def design_key(self) -> str | None:
        return None

    def reference(self, *inputs, **context):
        """Golden output for ``inputs`` from the registered reference provider. A sequence adds
        ``params`` (runtime-parameter values) and, for an ``inout`` last argument, ``last``."""
        provider = reference_provider()
        if provider is None:
            raise RuntimeError(
                f"{type(self).__name__}.reference(): no reference provider registered; the CPU "
                "goldens live in the test oracle (register_reference_provider)"
            )
        return provider(self, *inputs, **context)


class CompositeOperator(AIEOperatorBase):
    """Base class of operators that chain sub-operators."""


def check_args(op: AIEOperatorBase, args) -> list[torch.Tensor]:
    """Validate call arguments against ``op.get_arg_spec()``: count, device, dtype, size."""
    specs = op.get_arg_spec()
    if len(args) != len(specs):
        raise ValueError(f"{type(op).__name__}: expected {len(specs)} arguments, got {len(args)}")
    out = []
    for i, (a, s) in enumerate(zip(args, specs)):
        if not isinstance(a, torch.Tensor):
            raise TypeError(f"{type(op).__name__}: argument {i} is not a torch tensor")
        if a.device.type != "cuda":
            raise ValueError(f"{type(op).__name__}: argument {i} is not on the GPU")
        if not a.is_contiguous():
            raise ValueError(f"{type(op).__name__}: argument {i} is not contiguous")
        if a.numel() * a.element_size() < s.nbytes:
            raise ValueError(
                f"{type(op).__name__}: argument {i} holds {a.numel() * a.element_size()} bytes, "
                f"spec {s.shape} {s.dtype} needs {s.nbytes}"
            )
        out.append(a)
    return out
