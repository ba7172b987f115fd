"""Seeded synthetic GGUF weights and activations (host), over libcima_synth.so.

The reference has no quantiser (it only decodes, ``src/quant.rs:571-896``);
these produce valid packed blocks from seeded N(0, sigma^2) weights for the
benchmark configurations.  See ``include/cima_synth.h``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import gguf

LIBSYNTH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libcima_synth.so")
_lib = None


def _L():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBSYNTH):
            raise RuntimeError(f"{LIBSYNTH} is not built (run python -m cima_amd.build)")
        L = ctypes.CDLL(LIBSYNTH)
        P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.cima_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_float, P, S, I]
        L.cima_synth_normal.restype = None
        L.cima_synth_quantize.argtypes = [I, P, S, S, P, I]
        L.cima_synth_weights.argtypes = [I, ctypes.c_uint64, ctypes.c_float, S, S, P, I]
        _lib = L
    return _lib


def _threads(threads: int | None) -> int:
    if threads:
        return threads
    return max(1, min(16, len(os.sched_getaffinity(0))))


def normal(seed: int, stddev: float, count: int, threads: int | None = None) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    _L().cima_synth_normal(seed, stddev, out.ctypes.data_as(ctypes.c_void_p), count, _threads(threads))
    return out


def quantize(t: int, w: np.ndarray, threads: int | None = None) -> np.ndarray:
    """Quantise a [rows, k] fp32 matrix into packed GGUF bytes [rows, row_bytes]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    out = np.empty((rows, gguf.row_bytes(t, k)), dtype=np.uint8)
    rc = _L().cima_synth_quantize(int(t), w.ctypes.data_as(ctypes.c_void_p), rows, k,
                                  out.ctypes.data_as(ctypes.c_void_p), _threads(threads))
    if rc:
        raise ValueError(f"quantize: unsupported type {t} or k={k}")
    return out


def weights(t: int, seed: int, stddev: float, rows: int, k: int, threads: int | None = None) -> np.ndarray:
    """Seeded N(0, stddev^2) [rows, k] weights, quantised: [rows, row_bytes] u8."""
    out = np.empty((rows, gguf.row_bytes(t, k)), dtype=np.uint8)
    rc = _L().cima_synth_weights(int(t), seed, stddev, rows, k, out.ctypes.data_as(ctypes.c_void_p),
                                 _threads(threads))
    if rc:
        raise ValueError(f"weights: unsupported type {t} or k={k}")
    return out
