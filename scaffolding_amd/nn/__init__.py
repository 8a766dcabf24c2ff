"""nn surface of the path: Module, Parameter, Linear, SiLU, GELU and the
functional ops (reference nn/__init__.py)."""
from . import functional
from .layers import GELU, Linear, Module, Parameter, SiLU

__all__ = ["functional", "Module", "Parameter", "Linear", "SiLU", "GELU"]
