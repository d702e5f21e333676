"""Synthetic quantized weights: seeded fp32 matrices quantized to Q4_K/Q6_K and repacked.

The reference has no quantizer (Kindi reads pre-quantized GGUF, q4pack.py:110-180); this module
uses the repository's own one in libkqhost.so (include/kq_host.h documents the algorithm).

Seeds: W ~ N(0, 0.02) from ``np.random.default_rng(seed).standard_normal(dtype=float32) * 0.02``;
activations ~ N(0, 1) from ``default_rng(1_000_000 + seed)``.
"""
import numpy as np

from . import _lib
from .formats import BLOCK, Q4_K, Q6_K, QK, check_shape


def _ptr(a):
    return a.ctypes.data


def quantize(w, ty):
    """fp32 [R][C] -> blocks in GGUF row order, uint8 [R*(C/256)*bs]."""
    w = np.ascontiguousarray(w, np.float32)
    R, C = w.shape
    if C % QK:
        raise ValueError("C must be a multiple of 256")
    out = np.empty(R * (C // QK) * BLOCK[ty], np.uint8)
    fn = _lib.kqhost().kq_host_quantize_q4k if ty == Q4_K else _lib.kqhost().kq_host_quantize_q6k
    if fn(_ptr(w), R, C, _ptr(out)) != 0:
        raise ValueError("quantize: bad arguments")
    return out


def tile(raw, R, C, ty):
    """[R][G][bs] -> Kindi [R/8][G][8][bs] (same as formats.tile, parallel native copy)."""
    check_shape(R, C, ty)
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty_like(raw)
    if _lib.kqhost().kq_host_tile(_ptr(raw), R, C, ty, _ptr(out)) != 0:
        raise ValueError("tile: bad arguments")
    return out


def untile(packed, R, C, ty):
    check_shape(R, C, ty)
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.empty_like(packed)
    if _lib.kqhost().kq_host_untile(_ptr(packed), R, C, ty, _ptr(out)) != 0:
        raise ValueError("untile: bad arguments")
    return out


def synthetic_fp32(R, C, seed, sigma=0.02):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((R, C), dtype=np.float32) * np.float32(sigma)


def synthetic_matrix(R, C, ty, seed, sigma=0.02):
    """Seeded N(0, sigma) matrix, quantized and repacked: uint8 Kindi-layout bytes."""
    check_shape(R, C, ty)
    return tile(quantize(synthetic_fp32(R, C, seed, sigma), ty), R, C, ty)


def synthetic_activations(N, C, seed):
    rng = np.random.default_rng(1_000_000 + seed)
    return rng.standard_normal((N, C), dtype=np.float32)


__all__ = ["quantize", "tile", "untile", "synthetic_fp32", "synthetic_matrix",
           "synthetic_activations", "Q4_K", "Q6_K"]
