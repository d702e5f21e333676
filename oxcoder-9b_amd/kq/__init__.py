"""kq -- MI355X (gfx950) quantized matrix products of the Kindi Q4 path.

Modules:
  formats  -- block formats, Kindi 8-row repack (numpy)
  quantize -- seeded synthetic Q4_K/Q6_K weights (libkqhost.so)
  ops      -- tensor-level calls into libkq.so (HIP kernels, include/kq.h)
  gpu4     -- Weights / Engine: the operator surface of scripts/kindi_q4/kindi/gpu4.py
"""
from .formats import BLOCK, PAGE, Q4_K, Q6_K, Q8K_BYTES, QK  # noqa: F401

__version__ = "1.0"
