"""cima_amd -- MI355X (gfx950) GGUF dequant-GEMV hot path of the cima engine.

Native parts (built by ``cima_amd.build`` into ``cima_amd/lib``):
  * ``cima_gemv_{a,b,c}.hsaco``, ``cima_gemm.hsaco``, ``cima_dequant.hsaco``,
    ``cima_decode.hsaco`` -- hand-written HIP kernels for gfx950
  * ``libcima_hip.so``  -- the C ABI of ``include/cima_hip.h``
  * ``libcima_synth.so`` -- seeded synthetic weights (``include/cima_synth.h``)

``cima_amd.hip.HipCtx`` is the Python mirror of the reference's ``CudaCtx``
GGUF methods.
"""
from . import gguf  # noqa: F401
from .gguf import DType, block_elems, storage_bytes  # noqa: F401

__all__ = ["gguf", "DType", "block_elems", "storage_bytes"]
