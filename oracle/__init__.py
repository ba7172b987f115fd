"""CPU oracle for the GGUF dequant-GEMV path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
path (``cima_amd``) never imports it.

The arithmetic lives in ``gguf_oracle.c`` (a C restatement of the reference's
``src/traits.rs:832-896`` f16 primitives, ``src/quant.rs:571-896`` GGUF
decoders and ``src/quant.rs:258-437`` bitsandbytes NF4/FP4 decoding); this module is a thin numpy/ctypes front end over ``liboracle.so``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 2, 3, 6, 7, 8, 12, 13, 14, 23
BLOCK_ELEMS = {Q8_0: 32, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ4_XS: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ4_XS: 136}

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile."""
    if force or not os.path.exists(LIB_PATH):
        cmd = ["make", "-s", "-C", HERE]
        if force:
            cmd.insert(1, "-B")
        subprocess.run(cmd, check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_block_elems.argtypes = [I]
        L.oracle_block_bytes.argtypes = [I]
        L.oracle_storage_bytes.argtypes = [I, S]
        L.oracle_storage_bytes.restype = S
        L.oracle_dequant.argtypes = [I, P, S, S, P]
        L.oracle_gemv_f32.argtypes = [P, P, P, P, P, I, I, I, I]
        L.oracle_gemv_f64.argtypes = [P, P, P, P, I, I]
        L.oracle_gguf_gemv_packed.argtypes = [I, P, P, P, I, I, I]
        L.oracle_gemm_f32.argtypes = [P, P, P, I, I, I, I]
        L.oracle_gguf_gather.argtypes = [I, P, S, P, P, I, I]
        L.oracle_scale_min_k4.argtypes = [I, P, P, P]
        L.oracle_f16_to_f32_array.argtypes = [P, P, S]
        L.oracle_f32_to_f16_array.argtypes = [P, P, S]
        L.oracle_nf4_fold_absmax.argtypes = [P, S, P, P, S, S, ctypes.c_float, P]
        L.oracle_nf4_dequant.argtypes = [P, P, P, P, S, S]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def f32_to_f16(v: float) -> int:
    return lib().oracle_f32_to_f16(v)


def f16_to_f32_array(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16_array(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_p(v), _p(out), v.size)
    return out


def storage_bytes(t: int, numel: int) -> int:
    return lib().oracle_storage_bytes(t, numel)


def dequant(t: int, src: np.ndarray, numel: int) -> np.ndarray:
    """f16 bits (uint16) of the first ``numel`` elements; raises on the
    reference's size-mismatch error."""
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.zeros(numel, dtype=np.uint16)
    rc = lib().oracle_dequant(t, _p(src), src.nbytes, numel, _p(out))
    if rc:
        raise ValueError(f"oracle dequant(type {t}) failed: rc={rc}")
    return out


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def gemv(w16: np.ndarray, x: np.ndarray, n: int, k: int, mode: int = 0,
         bias: np.ndarray | None = None, y_old: np.ndarray | None = None,
         threads: int = 1) -> np.ndarray:
    """Reference CPU GEMV over decoded f16 weights, fp32 accumulate."""
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y_old = None if y_old is None else np.ascontiguousarray(y_old, dtype=np.float32)
    y = np.zeros(n, dtype=np.float32)
    lib().oracle_gemv_f32(_p(w16), _p(x), _p(bias), _p(y_old), _p(y), n, k, mode, threads)
    return y


def gemv_f64(w16: np.ndarray, x: np.ndarray, n: int, k: int):
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(n, dtype=np.float64)
    l2 = np.zeros(n, dtype=np.float64)
    lib().oracle_gemv_f64(_p(w16), _p(x), _p(y), _p(l2), n, k)
    return y, l2


def gguf_gemv_packed(t: int, w: np.ndarray, x: np.ndarray, n: int, k: int,
                     threads: int = 1) -> np.ndarray:
    """The CPU baseline: decode each packed row to f16, fp32 dot."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(n, dtype=np.float32)
    rc = lib().oracle_gguf_gemv_packed(t, _p(w), _p(x), _p(y), n, k, threads)
    if rc:
        raise ValueError("oracle gguf_gemv_packed failed")
    return y


def gemm(x: np.ndarray, w16: np.ndarray, m: int, n: int, k: int, threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w16 = np.ascontiguousarray(w16, dtype=np.uint16)
    y = np.zeros((m, n), dtype=np.float32)
    lib().oracle_gemm_f32(_p(x), _p(w16), _p(y), m, n, k, threads)
    return y


def gather(t: int, table: np.ndarray, ids: np.ndarray, hidden: int) -> np.ndarray:
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.zeros((len(ids), hidden), dtype=np.uint16)
    rc = lib().oracle_gguf_gather(t, _p(table), table.nbytes, _p(ids), _p(out), len(ids), hidden)
    if rc:
        raise ValueError("oracle gather failed")
    return out


def scale_min_k4(j: int, scales: np.ndarray):
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    sc, m = ctypes.c_float(), ctypes.c_float()
    lib().oracle_scale_min_k4(j, _p(s), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


# ------------------------------------------------------------ bitsandbytes 4-bit

def nf4_fold_absmax(codes: np.ndarray, nested_quant_map: np.ndarray, nested_absmax: np.ndarray,
                    nested_blocksize: int, nested_offset: float) -> np.ndarray:
    """folded_absmax (src/quant.rs:258-330), double-quantised branch."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    nmap = np.ascontiguousarray(nested_quant_map, dtype=np.float32)
    nabs = np.ascontiguousarray(nested_absmax, dtype=np.float32)
    if nmap.size != 256:
        raise ValueError("nested_quant_map must have 256 entries")
    out = np.zeros(codes.size, dtype=np.float32)
    rc = lib().oracle_nf4_fold_absmax(_p(codes), codes.size, _p(nmap), _p(nabs), nabs.size, nested_blocksize,
                                      float(nested_offset), _p(out))
    if rc:
        raise ValueError("nested_absmax too short")
    return out


def nf4_dequant(packed: np.ndarray, absmax: np.ndarray, qmap: np.ndarray, n: int, blocksize: int) -> np.ndarray:
    """dequant_host (src/quant.rs:401-437): f16 bits of qmap[nib(i)] * absmax[i // blocksize]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32)
    qmap = np.ascontiguousarray(qmap, dtype=np.float32)
    if packed.size * 2 < n or absmax.size * blocksize < n or qmap.size != 16:
        raise ValueError("nf4 operands too short")
    out = np.zeros(n, dtype=np.uint16)
    if lib().oracle_nf4_dequant(_p(packed), _p(absmax), _p(qmap), _p(out), n, blocksize):
        raise ValueError("nf4_dequant: n must be even and a multiple of blocksize")
    return out


def nf4_gemv(packed: np.ndarray, absmax: np.ndarray, qmap: np.ndarray, x: np.ndarray, n: int, k: int,
             blocksize: int, threads: int = 1) -> np.ndarray:
    """The reference CPU path for a packed weight: dequant_host, then the fp32 GEMV over the f16 weights."""
    return gemv(nf4_dequant(packed, absmax, qmap, n * k, blocksize), x, n, k, threads=threads)
