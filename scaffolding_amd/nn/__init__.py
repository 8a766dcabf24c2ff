"""nn surface of the path: Module, Parameter, Sequential, Linear, LayerNorm,
RMSNorm, Dropout, SiLU, GELU and the functional ops (reference
nn/__init__.py)."""
from . import functional
from .layers import GELU, Dropout, LayerNorm, Linear, Module, Parameter, RMSNorm, Sequential, SiLU

__all__ = ["functional", "Module", "Parameter", "Sequential", "Linear", "LayerNorm", "RMSNorm", "Dropout",
           "SiLU", "GELU"]
