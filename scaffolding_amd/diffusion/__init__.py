"""Diffusion-transformer glue around the matmul path (reference
diffusion/__init__.py): the adaptive layer norm and the DiT block, GPU
resident from input to output."""
from .models import AdaLayerNorm, DiTBlock

__all__ = ["AdaLayerNorm", "DiTBlock"]
