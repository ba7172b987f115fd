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
# the gfx950 code objects cima_hip_init loads (names as cima_amd/build.py
# writes them)
CODE_OBJECTS = [os.path.join(LIB_DIR, f"cima_{n}.hsaco")
                for n in ("gemv_a", "gemv_b", "gemv_c", "gemm", "dequant", "decode", "bnb4")]

# declared in include/cima_hip.h, in order
EXPORTS = (
    "cima_hip_init", "cima_hip_destroy", "cima_hip_bind", "cima_hip_set_stream", "cima_hip_use_own_stream",
    "cima_hip_get_stream",
    "cima_hip_sync", "cima_hip_last_error", "cima_hip_is_fatal", "cima_hip_num_cu", "cima_hip_set_gemv_tuning",
    "cima_hip_set_gemv_dma", "cima_hip_set_gemv_wsplit", "cima_hip_set_gemv_grid", "cima_hip_gemm_status", "cima_hip_set_gemm_tile",
    "cima_hip_gguf_gemv", "cima_hip_rmsnorm_gguf_gemv",
    "cima_hip_gguf_gemv_swiglu", "cima_hip_gguf_gemm", "cima_hip_gguf_gemm_slab", "cima_hip_gguf_dequant", "cima_hip_gguf_gather",
    "cima_hip_rmsnorm", "cima_hip_rope", "cima_hip_kv_append", "cima_hip_attn_decode_split", "cima_hip_attn_reduce",
    "cima_hip_attn_decode_noalloc", "cima_hip_attn_decode", "cima_hip_attn_gguf_gemv", "cima_hip_gguf_gemv_argmax", "cima_hip_argmax",
    "cima_hip_argmax_to_ids", "cima_hip_pos_bump", "cima_hip_decode_step",
    "cima_hip_capture_begin", "cima_hip_capture_end", "cima_hip_graph_launch", "cima_hip_graph_destroy",
    "cima_hip_nf4_dequant", "cima_hip_nf4_gemv", "cima_hip_set_nf4_tuning", "cima_hip_nf4_gemm_slab",
    "cima_hip_stream_read", "cima_hip_stream_read_cfg",
)


class DecoderLayer(ctypes.Structure):
    """``cima_decoder_layer`` (include/cima_hip.h)."""
    _fields_ = ([(n, ctypes.c_void_p) for n in (
        "attn_norm", "wqkv", "bqkv", "wo", "ffn_norm", "w_gate_up", "w_down", "k_cache", "v_cache", "wk", "wv",
        "w_up")]
        + [(n, ctypes.c_int) for n in ("type_q", "type_k", "type_v", "type_o", "type_gate", "type_up", "type_down",
                                       "window")])


class Decoder(ctypes.Structure):
    """``cima_decoder`` (include/cima_hip.h)."""
    _fields_ = ([(n, ctypes.c_int) for n in (
        "ggml_type", "embed_type", "head_type", "n_layers", "hidden", "q_heads", "kv_heads", "head_dim", "ffn",
        "vocab", "max_seq", "attn_chunk")]
        + [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]
        + [(n, ctypes.c_void_p) for n in ("embed", "head", "final_norm")]
        + [("layers", ctypes.POINTER(DecoderLayer))]
        + [(n, ctypes.c_void_p) for n in (
            "x", "qkv", "act", "logits", "part", "slot", "ids", "pos")])

E_INVALID, E_FORMAT, E_NO_KERNEL, E_NOT_INIT, E_LIBRARY = -1, -2, -3, -4, -5


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
    L.cima_hip_use_own_stream.argtypes = [P]
    L.cima_hip_get_stream.argtypes = [P]
    L.cima_hip_get_stream.restype = P
    L.cima_hip_sync.argtypes = [P]
    L.cima_hip_last_error.argtypes = []
    L.cima_hip_last_error.restype = ctypes.c_char_p
    L.cima_hip_is_fatal.argtypes = [I]
    L.cima_hip_num_cu.argtypes = [P]
    L.cima_hip_set_gemv_tuning.argtypes = [P, I, I]
    L.cima_hip_set_gemv_dma.argtypes = [P, I]
    L.cima_hip_set_gemv_wsplit.argtypes = [P, I]
    L.cima_hip_gemm_status.argtypes = [P, ctypes.POINTER(ctypes.c_uint), I]
    L.cima_hip_set_gemv_grid.argtypes = [P, I]
    L.cima_hip_set_gemm_tile.argtypes = [P, I]
    L.cima_hip_gguf_gemv.argtypes = [P, I, P, P, P, P, I, I, I, I]
    F = ctypes.c_float
    L.cima_hip_rmsnorm_gguf_gemv.argtypes = [P, I, P, P, F, P, P, P, I, I, I, I]
    L.cima_hip_rmsnorm.argtypes = [P, P, P, P, I, I, F]
    L.cima_hip_rope.argtypes = [P, P, I, I, I, I, F, I, P]
    L.cima_hip_kv_append.argtypes = [P, P, P, P, P, I, I, I, I, I, P]
    L.cima_hip_attn_decode_split.argtypes = [P, P, P, P, P, I, I, I, I, I, I, I, F, I, P]
    L.cima_hip_attn_reduce.argtypes = [P, P, P, I, I, I, I, I, I, I, P]
    L.cima_hip_attn_decode_noalloc.argtypes = [P, P, P, P, P, I, I, I, I, I, I, I, F, I, P]
    L.cima_hip_attn_decode.argtypes = [P, P, P, P, P, I, I, I, I, I, I, F, F, I, P]
    L.cima_hip_attn_gguf_gemv.argtypes = [P, I, P, I, I, I, I, I, I, P, P, P, P, I, I]
    L.cima_hip_gguf_gemv_argmax.argtypes = [P, I, P, P, F, P, P, I, I, P]
    L.cima_hip_argmax.argtypes = [P, P, P, I, F]
    L.cima_hip_argmax_to_ids.argtypes = [P, P, P, P]
    L.cima_hip_pos_bump.argtypes = [P, P]
    L.cima_hip_decode_step.argtypes = [P, ctypes.POINTER(Decoder)]
    L.cima_hip_capture_begin.argtypes = [P]
    L.cima_hip_stream_read.argtypes = [P, P, LL, P]
    L.cima_hip_stream_read_cfg.argtypes = [P, P, LL, P, I, I, I, I]
    L.cima_hip_nf4_dequant.argtypes = [P, P, P, P, P, LL, I]
    L.cima_hip_nf4_gemv.argtypes = [P, P, P, P, P, P, I, I, I, I]
    L.cima_hip_set_nf4_tuning.argtypes = [P, I, I]
    L.cima_hip_nf4_gemm_slab.argtypes = [P, P, P, P, P, P, I, I, I, I, I, I, P, ctypes.c_ulonglong]
    L.cima_hip_capture_end.argtypes = [P, ctypes.POINTER(P)]
    L.cima_hip_graph_launch.argtypes = [P, P]
    L.cima_hip_graph_destroy.argtypes = [P]
    L.cima_hip_gguf_gemv_swiglu.argtypes = [P, I, P, P, P, P, P, P, I, I, I]
    L.cima_hip_gguf_gemm.argtypes = [P, I, P, P, P, I, I, I, I, I, I]
    L.cima_hip_gguf_gemm_slab.argtypes = [P, I, P, P, P, I, I, I, I, I, I, P, ctypes.c_ulonglong]
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
        """Launch on ``stream``: a torch stream or a raw hipStream_t (0 is
        the null stream); None returns to the context's own stream."""
        if stream is None:
            self._check(self.lib.cima_hip_use_own_stream(self.handle))
            return
        raw = getattr(stream, "cuda_stream", stream)
        self._check(self.lib.cima_hip_set_stream(self.handle, raw))

    def use_torch_stream(self) -> None:
        """Launch on torch's current stream of this device (ordered with
        torch's own kernels there)."""
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

    def set_gemv_dma(self, mode: int = 0) -> None:
        """GEMV main loop: 0 = heuristic, 1 = direct-to-LDS streaming where built, 2 = register loops."""
        self._check(self.lib.cima_hip_set_gemv_dma(self.handle, int(mode)))

    def set_gemv_wsplit(self, mode: int = 0) -> None:
        """GEMV rows split over the workgroup's waves: 0 = heuristic, 1 = wherever it applies, 2 = never."""
        self._check(self.lib.cima_hip_set_gemv_wsplit(self.handle, int(mode)))

    def gemm_status(self, clear: bool = True) -> int:
        """X range flags of the prefill GEMMs since the last clear (waits for the
        stream): bit 0 = values beyond f16's range / non-finite, bit 1 = bf16
        values below 2^-17 (cima_hip_gemm_status)."""
        v = ctypes.c_uint(0)
        self._check(self.lib.cima_hip_gemm_status(self.handle, ctypes.byref(v), 1 if clear else 0))
        return int(v.value)

    def set_gemm_tile(self, tokens: int = 0) -> None:
        """Prefill GEMM token-tile width (16, 32, 64, 128 or 256; 0 = built-in choice)."""
        self._check(self.lib.cima_hip_set_gemm_tile(self.handle, int(tokens)))

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

    @staticmethod
    def _gemm_dtypes(x, y, x_dtype, y_dtype):
        def dt(t, default):
            if t is not None:
                return t
            import torch

            return {torch.float32: gguf.DT_F32, torch.float16: gguf.DT_F16,
                    torch.bfloat16: gguf.DT_BF16}.get(getattr(x if default == "x" else y, "dtype", None), gguf.DT_F32)
        xd = dt(x_dtype, "x") if hasattr(x, "dtype") or x_dtype is not None else gguf.DT_F32
        yd = dt(y_dtype, "y") if hasattr(y, "dtype") or y_dtype is not None else gguf.DT_F32
        return xd, yd

    def gguf_gemm(self, fmt: int, x, w, y, m: int, n: int, k: int, ldy: Optional[int] = None,
                  x_dtype: Optional[int] = None, y_dtype: Optional[int] = None) -> None:
        """``Y[m,n] = X[m,k]·dequant(W)[n,k]^T`` (prefill, MFMA); ldy defaults to n."""
        xd, yd = self._gemm_dtypes(x, y, x_dtype, y_dtype)
        self._check(self.lib.cima_hip_gguf_gemm(self.handle, int(fmt), _ptr(x), _ptr(w), _ptr(y), m, n, k,
                                                n if ldy is None else ldy, xd, yd))

    def gguf_gemm_slab(self, fmt: int, x, w, y, m: int, n: int, k: int, slab=None, slab_bytes: Optional[int] = None,
                       ldy: Optional[int] = None, x_dtype: Optional[int] = None,
                       y_dtype: Optional[int] = None) -> None:
        """The same product through the reference's lin_gemm signature (the
        engine's scratch slab is accepted and left untouched: the fused
        kernels never expand W)."""
        xd, yd = self._gemm_dtypes(x, y, x_dtype, y_dtype)
        if slab_bytes is None:
            slab_bytes = 0 if slab is None else slab.numel() * slab.element_size()
        self._check(self.lib.cima_hip_gguf_gemm_slab(self.handle, int(fmt), _ptr(x), _ptr(w), _ptr(y), m, n, k,
                                                     n if ldy is None else ldy, xd, yd, _ptr(slab),
                                                     int(slab_bytes)))

    @staticmethod
    def nf4_slab_bytes(m: int, n: int, k: int, x_f16: bool = False) -> int:
        """Slab size with which ``nf4_gemm_slab``'s slab route decodes W in
        one slice (W as f16); the fused route needs none.  ``m`` and
        ``x_f16`` are kept for callers written for a slab that also held X."""
        return (2 * n * k + 255) // 256 * 256

    def gguf_dequant(self, fmt: int, src, out, nblocks: int) -> None:
        """Decode ``nblocks`` blocks to f16 (bit-exact with the host decoders)."""
        self._check(self.lib.cima_hip_gguf_dequant(self.handle, int(fmt), _ptr(src), _ptr(out), nblocks))

    def gguf_gather(self, fmt: int, table, ids, out, n: int, hidden: int) -> None:
        """``out[i,:] = dequant(table[ids[i]])`` as f16."""
        self._check(self.lib.cima_hip_gguf_gather(self.handle, int(fmt), _ptr(table), _ptr(ids), _ptr(out),
                                                  n, hidden))

    # -- bitsandbytes 4-bit (src/quant.rs:18-437) ----------------------------
    def nf4_dequant(self, packed, absmax, qmap, out, n: int, blocksize: int) -> None:
        """CudaCtx::nf4_dequant (src/cuda.rs:2321): ``out[i] = f16(qmap[nib(i)] * absmax[i // blocksize])``."""
        self._check(self.lib.cima_hip_nf4_dequant(self.handle, _ptr(packed), _ptr(absmax), _ptr(qmap), _ptr(out),
                                                  n, blocksize))

    def nf4_gemv(self, x, packed, absmax, qmap, y, n: int, k: int, blocksize: int,
                 act_dtype: Optional[int] = None) -> None:
        """CudaCtx::nf4_gemv (src/cuda.rs:2347): ``y[n] = W[n, k] . x`` over the packed weight."""
        if act_dtype is None:
            act_dtype = _act_of(x) if hasattr(x, "dtype") else gguf.DT_F16
        self._check(self.lib.cima_hip_nf4_gemv(self.handle, _ptr(x), _ptr(packed), _ptr(absmax), _ptr(qmap), _ptr(y),
                                               n, k, blocksize, act_dtype))

    def nf4_gemm_slab(self, x, packed, absmax, qmap, y, m: int, n: int, k: int, blocksize: int, slab,
                      slab_bytes: Optional[int] = None, x_dtype: Optional[int] = None,
                      y_dtype: Optional[int] = None) -> None:
        """WTensor::gemm for an NF4 weight (src/quant.rs:131-162): ``Y[m, n] = X . W^T``
        on this library's f16-MFMA tiles, W decoded inside them (or, for shapes
        they do not take, into the f16 ``slab`` first)."""
        xd, yd = self._gemm_dtypes(x, y, x_dtype, y_dtype)
        if slab_bytes is None:
            slab_bytes = slab.numel() * slab.element_size()
        self._check(self.lib.cima_hip_nf4_gemm_slab(self.handle, _ptr(x), _ptr(packed), _ptr(absmax), _ptr(qmap),
                                                    _ptr(y), m, n, k, blocksize, xd, yd, _ptr(slab),
                                                    int(slab_bytes)))

    def set_nf4_tuning(self, rows: int = 0, kernel: int = 0) -> None:
        """Fast NF4 GEMV: rows per wave (1, 2, 4) and kernel (1 = LDS pair table,
        2 = codebook in registers); 0 = heuristic."""
        self._check(self.lib.cima_hip_set_nf4_tuning(self.handle, int(rows), int(kernel)))

    def rmsnorm_gguf_gemv(self, fmt: int, x, norm_w, eps: float, w, bias, y, n: int, k: int, mode: int = 0,
                          act_dtype: Optional[int] = None) -> None:
        """``gguf_gemv`` of ``rmsnorm(x) * norm_w`` (the norm is never written out)."""
        if act_dtype is None:
            act_dtype = _act_of(x) if hasattr(x, "dtype") else gguf.DT_F32
        self._check(self.lib.cima_hip_rmsnorm_gguf_gemv(self.handle, int(fmt), _ptr(x), _ptr(norm_w), eps, _ptr(w),
                                                        _ptr(bias), _ptr(y), n, k, mode, act_dtype))

    # -- decode-step support (f16) ------------------------------------------
    def rmsnorm(self, x, w, y, rows: int, n: int, eps: float) -> None:
        """CudaCtx::rmsnorm (src/cuda.rs:1180)."""
        self._check(self.lib.cima_hip_rmsnorm(self.handle, _ptr(x), _ptr(w), _ptr(y), rows, n, eps))

    def rope(self, x, rows: int, heads: int, dim: int, pos0: int, theta: float, nfreqs: int, pos_dev=None) -> None:
        """CudaCtx::rope (src/cuda.rs:1302), in place."""
        self._check(self.lib.cima_hip_rope(self.handle, _ptr(x), rows, heads, dim, pos0, theta, nfreqs,
                                           _ptr(pos_dev)))

    def kv_append(self, k, v, kc, vc, rows: int, kv_heads: int, dim: int, pos: int, max_seq: int,
                  pos_dev=None) -> None:
        """CudaCtx::kv_append (src/cuda.rs:1344)."""
        self._check(self.lib.cima_hip_kv_append(self.handle, _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), rows, kv_heads,
                                                dim, pos, max_seq, _ptr(pos_dev)))

    def attn_decode_split(self, q, kc, vc, part, q_heads: int, kv_heads: int, dim: int, seq: int, max_seq: int,
                          csz: int, n_chunks: int, scale: float, window: int = 0, pos_dev=None) -> None:
        """CudaCtx::attn_decode_split (src/cuda.rs:1418)."""
        self._check(self.lib.cima_hip_attn_decode_split(self.handle, _ptr(q), _ptr(kc), _ptr(vc), _ptr(part),
                                                        q_heads, kv_heads, dim, seq, max_seq, csz, n_chunks, scale,
                                                        window, _ptr(pos_dev)))

    def attn_reduce(self, part, out, q_heads: int, dim: int, csz: int, n_chunks: int, seq: int, max_seq: int,
                    window: int = 0, pos_dev=None) -> None:
        """CudaCtx::attn_reduce (src/cuda.rs:1476)."""
        self._check(self.lib.cima_hip_attn_reduce(self.handle, _ptr(part), _ptr(out), q_heads, dim, csz, n_chunks,
                                                  seq, max_seq, window, _ptr(pos_dev)))

    def attn_decode_noalloc(self, q, kc, vc, out, q_heads: int, kv_heads: int, dim: int, seq: int, max_seq: int,
                            csz: int, n_chunks: int, scale: float, window: int = 0, pos_dev=None) -> None:
        """attn_decode_split + attn_reduce with the partials in the library's
        fixed device scratch (allocates nothing; calls on one device must
        not overlap)."""
        self._check(self.lib.cima_hip_attn_decode_noalloc(self.handle, _ptr(q), _ptr(kc), _ptr(vc), _ptr(out),
                                                          q_heads, kv_heads, dim, seq, max_seq, csz, n_chunks, scale,
                                                          window, _ptr(pos_dev)))

    def attn_decode(self, qkv, kc, vc, part, q_heads: int, kv_heads: int, dim: int, max_seq: int, csz: int,
                    n_chunks: int, theta: float, scale: float, pos_dev, window: int = 0) -> None:
        """RoPE + KV append + split attention partials in one launch
        (window > 0: the last `window` positions only)."""
        self._check(self.lib.cima_hip_attn_decode(self.handle, _ptr(qkv), _ptr(kc), _ptr(vc), _ptr(part), q_heads,
                                                  kv_heads, dim, max_seq, csz, n_chunks, theta, scale, window,
                                                  _ptr(pos_dev)))

    def attn_gguf_gemv(self, fmt: int, part, q_heads: int, dim: int, csz: int, n_chunks: int, max_seq: int,
                       pos_dev, w, bias, y, n: int, mode: int = 0, window: int = 0) -> None:
        """o projection of the attention merged from split partials (f16;
        window > 0: merged over the last `window` positions)."""
        self._check(self.lib.cima_hip_attn_gguf_gemv(self.handle, int(fmt), _ptr(part), q_heads, dim, csz, n_chunks,
                                                     max_seq, window, _ptr(pos_dev), _ptr(w), _ptr(bias), _ptr(y), n,
                                                     mode))

    def gguf_gemv_argmax(self, fmt: int, x, norm_w, eps: float, w, y, n: int, k: int, slot) -> None:
        """Head GEMV (optional RMSNorm prologue) with the greedy argmax into slot."""
        self._check(self.lib.cima_hip_gguf_gemv_argmax(self.handle, int(fmt), _ptr(x), _ptr(norm_w), eps, _ptr(w),
                                                       _ptr(y), n, k, _ptr(slot)))

    def argmax(self, x, slot, n: int, cap: float = 0.0) -> None:
        """CudaCtx::argmax_softcap_enqueue (src/cuda.rs:2036); slot must be 0."""
        self._check(self.lib.cima_hip_argmax(self.handle, _ptr(x), _ptr(slot), n, cap))

    def argmax_to_ids(self, slot, ids, pos_dev=None) -> None:
        """CudaCtx::argmax_to_ids (+ pos_bump when pos_dev is given); clears slot."""
        self._check(self.lib.cima_hip_argmax_to_ids(self.handle, _ptr(slot), _ptr(ids), _ptr(pos_dev)))

    def pos_bump(self, pos_dev) -> None:
        self._check(self.lib.cima_hip_pos_bump(self.handle, _ptr(pos_dev)))

    def decode_step(self, desc: "Decoder") -> None:
        """One greedy decode step of a whole decoder (cima_hip_decode_step)."""
        self._check(self.lib.cima_hip_decode_step(self.handle, ctypes.byref(desc)))

    def stream_read_cfg(self, src, nbytes: int, sink, dest: int, depth: int, width: int = 16,
                        wgs_per_cu: int = 2) -> None:
        """Read ceiling in a chosen form: dest 0 = registers (depth loads of width
        bytes per thread), 1 = LDS ring of depth 1 KB copies per wave."""
        self._check(self.lib.cima_hip_stream_read_cfg(self.handle, _ptr(src), nbytes, _ptr(sink), dest, depth, width,
                                                      wgs_per_cu))

    def stream_read(self, src, nbytes: int, sink) -> None:
        """Read nbytes once (bandwidth reference)."""
        self._check(self.lib.cima_hip_stream_read(self.handle, _ptr(src), nbytes, _ptr(sink)))

    # -- graphs ---------------------------------------------------------------
    def capture_begin(self) -> None:
        """Start recording the context stream (CudaCtx::capture_begin)."""
        self._check(self.lib.cima_hip_capture_begin(self.handle))

    def capture_end(self) -> "Graph":
        """Stop recording and instantiate (CudaCtx::capture_end)."""
        g = ctypes.c_void_p()
        self._check(self.lib.cima_hip_capture_end(self.handle, ctypes.byref(g)))
        return Graph(self, g)


class Graph:
    """An instantiated graph of the context's stream; launch() replays it."""

    def __init__(self, ctx: HipCtx, handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self) -> None:
        self.ctx._check(self.ctx.lib.cima_hip_graph_launch(self.ctx.handle, self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx.lib.cima_hip_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
