"""Backend flags (reference backends/__init__.py)."""
from . import cuda  # noqa: F401
