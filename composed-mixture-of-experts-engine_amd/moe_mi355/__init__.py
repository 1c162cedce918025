"""moe_mi355 -- MI355X (gfx950) native MoE hot path.

Hand-written HIP kernels (``csrc/``) behind a plain C ABI
(``include/moe_mi355.h``), loaded with ctypes (``_lib``), wrapped as torch
autograd Functions (``router``).  The reference-compatible modules live in
the ``pkg`` package next to this one.
"""

from . import _lib, ops  # noqa: F401
from .router import RouterCore, route  # noqa: F401

__version__ = "0.1.0"


def native_available() -> bool:
    """True when libmoe_mi355.so is built and a ROCm GPU is visible."""
    import os

    import torch

    return os.path.exists(_lib.LIB_PATH) and torch.cuda.is_available()
