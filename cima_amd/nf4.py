"""bitsandbytes 4-bit (NF4 / FP4) weights: host side of the packed path.

Mirrors the reference's ``quant::bnb`` module (src/quant.rs:18-437):

* a quantised ``nn.Linear`` weight ``W`` is stored (safetensors, as
  ``transformers`` saves it) as a family of tensors -- ``W`` (U8 packed
  nibbles, element 2j in the HIGH nibble of byte j), ``W.absmax`` (F32, or
  U8 codes when double-quantised), ``W.quant_map`` (16 f32), optionally
  ``W.nested_absmax`` / ``W.nested_quant_map`` and the JSON quant state
  ``W.quant_state.bitsandbytes__{nf4,fp4}``;
* on load the double quantisation is folded on the host into one f32 absmax
  per ``blocksize`` elements (``fold_absmax``), and the weight stays resident
  as packed nibbles + absmax + codebook (``Nf4Weight``);
* decode (m == 1) runs the fused GEMV, prefill dequantises to an f16 slab
  and multiplies (``Nf4Weight.gemm``, the reference's WTensor::gemm,
  src/quant.rs:82-163).

The kernels are in ``csrc/bnb4.hip``; this module never computes weights on
the CPU except for the load-time fold and the synthetic quantiser.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Mapping, Optional

import numpy as np

from .hip import E_INVALID, EngineError

# The NF4 codebook (normal-float 4-bit: quantiles of N(0, 1) scaled to
# [-1, 1], with an exact zero), as bitsandbytes stores it in W.quant_map.
NF4_CODE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)

QUANT_TYPES = ("nf4", "fp4")


def _err(msg: str) -> EngineError:
    return EngineError("quant", E_INVALID, msg)


@dataclass
class BnbState:
    """Parsed ``W.quant_state.bitsandbytes__*`` (src/quant.rs:40-47)."""
    blocksize: int
    rows: int
    cols: int
    nested_blocksize: int
    nested_offset: float


def state_name(tensors: Mapping[str, np.ndarray], name: str) -> Optional[str]:
    """Name of the quant-state sibling if ``name`` is a bnb-packed weight (src/quant.rs:166-178)."""
    for qt in QUANT_TYPES:
        n = f"{name}.quant_state.bitsandbytes__{qt}"
        if n in tensors:
            return n
    return None


def is_aux(name: str) -> bool:
    """True for the auxiliary tensors of a packed family (src/quant.rs:180-188)."""
    return (name.endswith(".absmax") or name.endswith(".quant_map") or name.endswith(".nested_absmax")
            or name.endswith(".nested_quant_map") or ".quant_state.bitsandbytes__" in name)


def parse_state(tensors: Mapping[str, np.ndarray], name: str) -> BnbState:
    """parse_state (src/quant.rs:197-255): the JSON quant state with its defaults."""
    sname = state_name(tensors, name)
    if sname is None:
        raise _err(f"tensor '{name}' has no bitsandbytes quant_state sibling")
    raw = np.ascontiguousarray(tensors[sname]).view(np.uint8).tobytes()
    try:
        txt = raw.decode("utf-8")
    except UnicodeDecodeError:
        raise _err(f"quant_state of '{name}' is not UTF-8 JSON") from None
    try:
        j = json.loads(txt)
    except json.JSONDecodeError as e:
        raise _err(f"quant_state of '{name}' is not valid JSON: {e}") from None
    shape = [int(v) for v in j.get("shape", []) if isinstance(v, (int, float)) and v >= 0]
    if len(shape) != 2:
        raise _err(f"quant_state of '{name}' has shape {shape} -- only 2-D linear weights are executable")
    blocksize = int(j.get("blocksize", 64))
    if blocksize <= 0 or (shape[0] * shape[1]) % blocksize:
        raise _err(f"'{name}': numel {shape[0] * shape[1]} not divisible by blocksize {blocksize}")
    return BnbState(blocksize=blocksize, rows=shape[0], cols=shape[1],
                    nested_blocksize=int(j.get("nested_blocksize", 256)),
                    nested_offset=float(np.float32(j.get("nested_offset", 0.0))))


def fold_absmax(tensors: Mapping[str, np.ndarray], name: str, st: BnbState, nblocks: int) -> np.ndarray:
    """folded_absmax (src/quant.rs:258-330): one f32 scale per block.

    Double-quantised (U8 absmax): ``nested_quant_map[code[i]] *
    nested_absmax[i // nested_blocksize] + nested_offset``, each operation
    rounded in f32 (no fused multiply-add).
    """
    am = tensors.get(f"{name}.absmax")
    if am is None:
        raise _err(f"'{name}': missing .absmax sibling")
    am = np.asarray(am)
    if am.dtype == np.float32:
        v = am.reshape(-1)
        if v.size != nblocks:
            raise _err(f"'{name}': absmax has {v.size} entries, expected {nblocks}")
        return np.ascontiguousarray(v)
    if am.dtype != np.uint8:
        raise _err(f"'{name}': absmax stored as {am.dtype} -- expected U8 (double-quant) or F32")
    nmap = tensors.get(f"{name}.nested_quant_map")
    if nmap is None:
        raise _err(f"'{name}': double-quantized but .nested_quant_map is missing")
    nabs = tensors.get(f"{name}.nested_absmax")
    if nabs is None:
        raise _err(f"'{name}': double-quantized but .nested_absmax is missing")
    nmap = np.asarray(nmap, dtype=np.float32).reshape(-1)
    nabs = np.asarray(nabs, dtype=np.float32).reshape(-1)
    codes = am.reshape(-1)
    if codes.size != nblocks:
        raise _err(f"'{name}': absmax has {codes.size} entries, expected {nblocks}")
    if nmap.size < 256:
        raise _err(f"'{name}': nested_quant_map has {nmap.size} entries, expected 256")
    j = np.arange(nblocks, dtype=np.int64) // st.nested_blocksize
    if nblocks and j[-1] >= nabs.size:
        raise _err(f"'{name}': nested_absmax too short ({nabs.size} for block {int(np.argmax(j >= nabs.size))})")
    prod = nmap[codes] * nabs[j]  # f32 x f32 -> f32
    return np.ascontiguousarray(prod + np.float32(st.nested_offset), dtype=np.float32)


@dataclass
class HostNf4:
    """A packed weight on the host: what upload_nf4 sends to the device."""
    packed: np.ndarray  # [rows*cols/2] u8
    absmax: np.ndarray  # [rows*cols/blocksize] f32 (folded)
    qmap: np.ndarray    # [16] f32
    rows: int
    cols: int
    blocksize: int

    def device_bytes(self) -> int:
        return nf4_device_bytes(self.rows * self.cols, self.blocksize)


def nf4_device_bytes(numel: int, blocksize: int) -> int:
    """Bytes a packed weight occupies once resident (src/quant.rs:392-396)."""
    return numel // 2 + (numel // blocksize) * 4 + 64


def load_bnb4(tensors: Mapping[str, np.ndarray], name: str) -> HostNf4:
    """upload_nf4's host half (src/quant.rs:333-390): checks and the absmax fold."""
    st = parse_state(tensors, name)
    numel = st.rows * st.cols
    w = tensors.get(name)
    if w is None:
        raise _err(f"'{name}': no such tensor")
    w = np.asarray(w)
    if w.dtype != np.uint8 or w.nbytes != numel // 2:
        raise _err(f"'{name}': packed payload is {w.nbytes} bytes of {w.dtype}, expected {numel // 2} u8 bytes "
                   f"for [{st.rows} x {st.cols}] nibbles")
    nblocks = numel // st.blocksize
    absmax = fold_absmax(tensors, name, st, nblocks)
    qm = tensors.get(f"{name}.quant_map")
    if qm is None:
        raise _err(f"'{name}': missing .quant_map sibling")
    qm = np.asarray(qm, dtype=np.float32).reshape(-1)
    if qm.size != 16:
        raise _err(f"'{name}': quant_map has {qm.size} entries, expected 16")
    return HostNf4(packed=np.ascontiguousarray(w.reshape(-1)), absmax=absmax, qmap=np.ascontiguousarray(qm),
                   rows=st.rows, cols=st.cols, blocksize=st.blocksize)


def read_safetensors(path: str) -> dict:
    """Every tensor of a safetensors file as numpy arrays (no code is executed from the file)."""
    from safetensors.numpy import load_file

    return load_file(path)


# ------------------------------------------------------------ synthetic weights

def quantize(w: np.ndarray, blocksize: int = 64, code: np.ndarray = NF4_CODE, quant_type: str = "nf4",
             double_quant: bool = False, nested_blocksize: int = 256, name: str = "weight") -> dict:
    """Quantise a 2-D f32 weight the way bitsandbytes' quantize_4bit does
    (absmax per block, nearest codebook entry of w / absmax), returning the
    tensor family as it appears in a checkpoint.  With ``double_quant`` the
    absmax is itself quantised: offset = mean(absmax), then one 256-entry
    code per block against a per-``nested_blocksize`` scale."""
    w = np.asarray(w, dtype=np.float32)
    rows, cols = w.shape
    flat = w.reshape(-1)
    if flat.size % blocksize or flat.size % 2:
        raise ValueError("numel must be even and a multiple of blocksize")
    blocks = flat.reshape(-1, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    safe = np.where(absmax > 0, absmax, np.float32(1.0))
    norm = blocks / safe[:, None]
    idx = np.abs(norm[..., None] - code[None, None, :]).argmin(axis=-1).astype(np.uint8).reshape(-1)
    packed = ((idx[0::2] << 4) | idx[1::2]).astype(np.uint8)
    state = {"quant_type": quant_type, "blocksize": blocksize, "shape": [rows, cols], "dtype": "float16"}
    out = {name: packed.reshape(-1, 1), f"{name}.quant_map": np.asarray(code, dtype=np.float32)}
    if double_quant:
        offset = np.float32(absmax.mean())
        centred = absmax - offset
        nmap = np.linspace(-1.0, 1.0, 256, dtype=np.float32)
        nb = (absmax.size + nested_blocksize - 1) // nested_blocksize
        pad = np.zeros(nb * nested_blocksize, dtype=np.float32)
        pad[:absmax.size] = centred
        nabs = np.abs(pad.reshape(nb, nested_blocksize)).max(axis=1).astype(np.float32)
        nabs = np.where(nabs > 0, nabs, np.float32(1.0)).astype(np.float32)
        scaled = pad.reshape(nb, nested_blocksize) / nabs[:, None]
        codes = np.abs(scaled[..., None] - nmap).argmin(axis=-1).astype(np.uint8).reshape(-1)[:absmax.size]
        out[f"{name}.absmax"] = codes
        out[f"{name}.nested_absmax"] = nabs
        out[f"{name}.nested_quant_map"] = nmap
        state.update(nested_blocksize=nested_blocksize, nested_offset=float(offset))
    else:
        out[f"{name}.absmax"] = absmax
    out[f"{name}.quant_state.bitsandbytes__{quant_type}"] = np.frombuffer(json.dumps(state).encode(), dtype=np.uint8)
    return out


# ------------------------------------------------------------ device residency

class Nf4Weight:
    """A packed weight resident on the device (BnbNf4, src/quant.rs:49-58)."""

    def __init__(self, host: HostNf4, device: str = "cuda"):
        import torch

        self.rows, self.cols, self.blocksize = host.rows, host.cols, host.blocksize
        self.packed = torch.from_numpy(np.require(host.packed, requirements=["C", "W"])).to(device)
        self.absmax = torch.from_numpy(np.require(host.absmax, requirements=["C", "W"])).to(device)
        self.qmap = torch.from_numpy(np.require(host.qmap, requirements=["C", "W"])).to(device)

    def _check_shape(self, n: int, k: int) -> None:
        if self.rows != n or self.cols != k:
            raise _err(f"nf4 weight is [{self.rows}, {self.cols}] but the GEMM expects [{n}, {k}] -- "
                       "graph/checkpoint mismatch")

    def gemv(self, ctx, x, y) -> None:
        """y[n] = W . x (x, y f16 or f32 on the device)."""
        ctx.nf4_gemv(x, self.packed, self.absmax, self.qmap, y, self.rows, self.cols, self.blocksize)

    def dequant(self, ctx, out) -> None:
        """out[rows*cols] = f16 weights, bit-exact with the host decoder."""
        ctx.nf4_dequant(self.packed, self.absmax, self.qmap, out, self.rows * self.cols, self.blocksize)

    def gemm(self, ctx, x, y, scratch=None) -> None:
        """WTensor::gemm for a packed weight (src/quant.rs:131-162): y[m, n] = x[m, k] . W^T.
        m == 1 runs the fused GEMV; m > 1 runs cima_hip_nf4_gemm_slab: the
        f16-MFMA prefill tiles decode W themselves for every checkpoint
        shape, other shapes decode it into the ``scratch`` slab a row slice
        at a time; any slab that holds one slice works (the reference's is
        32 MiB), ``HipCtx.nf4_slab_bytes(m, n, k)`` bytes hold W whole."""
        m = x.shape[0] if x.dim() == 2 else 1
        n, k = y.shape[-1], x.shape[-1]
        self._check_shape(n, k)
        if m == 1:
            self.gemv(ctx, x.reshape(-1), y.reshape(-1))
            return
        if scratch is None:
            raise _err("nf4 prefill GEMM requires a dequant scratch buffer")
        ctx.nf4_gemm_slab(x, self.packed, self.absmax, self.qmap, y, m, n, k, self.blocksize, scratch)
