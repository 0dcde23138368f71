"""Operator base classes, context, sequence executor and test utilities."""

from .base import (AIEOperatorBase, AIERuntimeArgSpec, CompositeOperator, MLIROperator,
                   register_reference_provider)
from .context import AIEContext

__all__ = ["AIEOperatorBase", "AIERuntimeArgSpec", "CompositeOperator", "MLIROperator",
           "AIEContext", "register_reference_provider"]
