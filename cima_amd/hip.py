"""Python host mirror of the reference's CudaCtx GGUF surface, over the C ABI.

``HipCtx`` exposes the same methods, argument order and meaning as the
reference's Rust ``CudaCtx`` (``src/cuda.rs``): ``gguf_gemv``
(``:2161-2220``), ``gguf_dequant`` (``:2285-2320``), ``gguf_gather``
(``:2226-2283``), plus the fused ``gguf_gemv_swiglu``.  Arguments are device
pointers (``int``) or torch CUDA tensors (their ``data_ptr()`` is used; torch
is only the allocator here).  Failures raise :class:`EngineError`, the
counterpart of the reference's ``EngineError{scope: "cuda"}``
(``src/traits.rs:29-84``); ``fatal`` is set for sticky device faults
(``cu_fatal``, ``src/cuda.rs:122-127``).

There is no fallback: if ``libcima_hip.so`` or the gfx950 code object is
missing, construction raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

from . import gguf

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
LIBHIP = os.path.join(LIB_DIR, "libcima_hip.so")
CODE_OBJECTS = [os.path.join(LIB_DIR, f"cima_{n}.hsaco") for n in ("gemv", "gemm", "dequant")]

# declared in include/cima_hip.h, in order
EXPORTS = (
    "cima_hip_init", "cima_hip_destroy", "cima_hip_bind", "cima_hip_set_stream", "cima_hip_get_stream",
    "cima_hip_sync", "cima_hip_last_error", "cima_hip_is_fatal", "cima_hip_num_cu", "cima_hip_set_gemv_tuning",
    "cima_hip_set_gemv_grid", "cima_hip_set_gemm_tile",
    "cima_hip_gguf_gemv",
    "cima_hip_gguf_gemv_swiglu", "cima_hip_gguf_gemm", "cima_hip_gguf_dequant", "cima_hip_gguf_gather",
)

E_INVALID, E_FORMAT, E_NO_KERNEL, E_NOT_INIT = -1, -2, -3, -4


class EngineError(RuntimeError):
    def __init__(self, scope: str, code: int, message: str, fatal: bool = False):
        super().__init__(f"[{scope}] {message}")
        self.scope = scope
        self.code = code
        self.fatal = fatal


_lib = None


def load_library(path: str = LIBHIP) -> ctypes.CDLL:
    """Load libcima_hip.so and declare the C ABI signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise EngineError("hip", E_NOT_INIT, f"{path} is not built (run python -m cima_amd.build)")
    L = ctypes.CDLL(path)
    P, I, LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    L.cima_hip_init.argtypes = [I, ctypes.c_char_p, ctypes.POINTER(P)]
    L.cima_hip_destroy.argtypes = [P]
    L.cima_hip_bind.argtypes = [P]
    L.cima_hip_set_stream.argtypes = [P, P]
    L.cima_hip_get_stream.argtypes = [P]
    L.cima_hip_get_stream.restype = P
    L.cima_hip_sync.argtypes = [P]
    L.cima_hip_last_error.argtypes = []
    L.cima_hip_last_error.restype = ctypes.c_char_p
    L.cima_hip_is_fatal.argtypes = [I]
    L.cima_hip_num_cu.argtypes = [P]
    L.cima_hip_set_gemv_tuning.argtypes = [P, I, I]
    L.cima_hip_set_gemv_grid.argtypes = [P, I]
    L.cima_hip_set_gemm_tile.argtypes = [P, I]
    L.cima_hip_gguf_gemv.argtypes = [P, I, P, P, P, P, I, I, I, I]
    L.cima_hip_gguf_gemv_swiglu.argtypes = [P, I, P, P, P, P, P, P, I, I, I]
    L.cima_hip_gguf_gemm.argtypes = [P, I, P, P, P, I, I, I, I, I, I]
    L.cima_hip_gguf_dequant.argtypes = [P, I, P, P, LL]
    L.cima_hip_gguf_gather.argtypes = [P, I, P, P, P, I, I]
    _lib = L
    return L


def _ptr(a) -> Optional[int]:
    if a is None or (isinstance(a, int) and a == 0):
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):
        if not a.is_cuda:
            raise EngineError("hip", E_INVALID, "tensor argument is not on a HIP device")
        if not a.is_contiguous():
            raise EngineError("hip", E_INVALID, "tensor argument is not contiguous")
        return a.data_ptr()
    raise TypeError(f"expected a device pointer or a torch tensor, got {type(a)!r}")


def _act_of(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return gguf.DT_F32
    if t.dtype == torch.float16:
        return gguf.DT_F16
    raise EngineError("hip", E_INVALID, f"activation dtype {t.dtype} is not float32 or float16")


class HipCtx:
    """One device context: a loaded gfx950 module and a launch stream."""

    def __init__(self, device: int = 0, code_dir: Optional[str] = None):
        self.lib = load_library()
        if code_dir is None:
            missing = [p for p in CODE_OBJECTS if not os.path.exists(p)]
            if missing:
                raise EngineError("hip", E_NOT_INIT, f"{missing[0]} is not built (run python -m cima_amd.build)")
        h = ctypes.c_void_p()
        co = (code_dir or LIB_DIR).encode()
        self._check(self.lib.cima_hip_init(device, co, ctypes.byref(h)))
        self.handle = h
        self.device = device

    # -- plumbing ---------------------------------------------------------
    def _check(self, rc: int) -> None:
        if rc != 0:
            msg = self.lib.cima_hip_last_error().decode(errors="replace")
            raise EngineError("hip", rc, msg, fatal=bool(self.lib.cima_hip_is_fatal(rc)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.cima_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind(self) -> None:
        self._check(self.lib.cima_hip_bind(self.handle))

    def set_stream(self, stream) -> None:
        """Launch on ``stream`` (a torch stream, a raw hipStream_t, or None
        for the context's own non-blocking stream)."""
        raw = getattr(stream, "cuda_stream", stream)
        self._check(self.lib.cima_hip_set_stream(self.handle, raw or None))

    def use_torch_stream(self) -> None:
        import torch

        self.set_stream(torch.cuda.current_stream(self.device).cuda_stream)

    def sync(self) -> None:
        self._check(self.lib.cima_hip_sync(self.handle))

    @property
    def num_cu(self) -> int:
        return self.lib.cima_hip_num_cu(self.handle)

    def set_gemv_tuning(self, rows: int = 0, lanes_per_row: int = 0) -> None:
        """Override the GEMV launch plan (0, 0 = built-in heuristic)."""
        self._check(self.lib.cima_hip_set_gemv_tuning(self.handle, rows, lanes_per_row))

    def set_gemv_grid(self, wgs_per_cu: int = 0) -> None:
        """Cap the persistent GEMV grid at this many workgroups per CU (0 = fill)."""
        self._check(self.lib.cima_hip_set_gemv_grid(self.handle, wgs_per_cu))

    # -- the GGUF hot path --------------------------------------------------
    def gguf_gemv(self, fmt: int, x, w, bias, y, n: int, k: int, mode: int = 0,
                  act_dtype: Optional[int] = None) -> None:
        """``y[n] = W[n,k]·x[k]`` (+bias); mode 1 accumulates into y; mode 2
        treats W as the ``[2n,k]`` gate|up pair with a SwiGLU epilogue."""
        if act_dtype is None:
            act_dtype = _act_of(x) if hasattr(x, "dtype") else gguf.DT_F32
        self._check(self.lib.cima_hip_gguf_gemv(self.handle, int(fmt), _ptr(x), _ptr(w), _ptr(bias), _ptr(y),
                                                n, k, mode, act_dtype))

    def gguf_gemv_swiglu(self, fmt: int, x, w_gate, w_up, bias_gate, bias_up, y, n: int, k: int,
                         act_dtype: Optional[int] = None) -> None:
        """``y = silu(Wg·x + bg) * (Wu·x + bu)`` in one pass."""
        if act_dtype is None:
            act_dtype = _act_of(x) if hasattr(x, "dtype") else gguf.DT_F32
        self._check(self.lib.cima_hip_gguf_gemv_swiglu(self.handle, int(fmt), _ptr(x), _ptr(w_gate), _ptr(w_up),
                                                       _ptr(bias_gate), _ptr(bias_up), _ptr(y), n, k, act_dtype))

    def gguf_gemm(self, fmt: int, x, w, y, m: int, n: int, k: int, ldy: Optional[int] = None,
                  x_dtype: Optional[int] = None, y_dtype: Optional[int] = None) -> None:
        """``Y[m,n] = X[m,k]·dequant(W)[n,k]^T`` (prefill, MFMA); ldy defaults to n."""
        def dt(t, default):
            if t is not None:
                return t
            import torch

            return {torch.float32: gguf.DT_F32, torch.float16: gguf.DT_F16,
                    torch.bfloat16: gguf.DT_BF16}.get(getattr(x if default == "x" else y, "dtype", None), gguf.DT_F32)
        xd = dt(x_dtype, "x") if hasattr(x, "dtype") or x_dtype is not None else gguf.DT_F32
        yd = dt(y_dtype, "y") if hasattr(y, "dtype") or y_dtype is not None else gguf.DT_F32
        self._check(self.lib.cima_hip_gguf_gemm(self.handle, int(fmt), _ptr(x), _ptr(w), _ptr(y), m, n, k,
                                                n if ldy is None else ldy, xd, yd))

    def gguf_dequant(self, fmt: int, src, out, nblocks: int) -> None:
        """Decode ``nblocks`` blocks to f16 (bit-exact with the host decoders)."""
        self._check(self.lib.cima_hip_gguf_dequant(self.handle, int(fmt), _ptr(src), _ptr(out), nblocks))

    def gguf_gather(self, fmt: int, table, ids, out, n: int, hidden: int) -> None:
        """``out[i,:] = dequant(table[ids[i]])`` as f16."""
        self._check(self.lib.cima_hip_gguf_gather(self.handle, int(fmt), _ptr(table), _ptr(ids), _ptr(out),
                                                  n, hidden))
