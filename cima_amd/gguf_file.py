"""GGUF container files: reader, writer, and the decoder model they hold.

The reader mirrors the reference's GGUF parser (``src/formats.rs``): the
header (magic ``GGUF``, version 2 or 3, tensor and metadata counts,
``:513-545``), typed metadata values (``:176-216``, types 0-12, arrays
nested at most twice), tensor records with dims stored innermost-first and
returned outermost-first (``:546-570``), the data section aligned to
``general.alignment`` (default 32, ``:572-576``), every tensor's extent
checked against the file (``:582-597``) and the ggml type ids it accepts
(``:90-117``).  ``decoder_config`` restates ``model_config`` (``:940-1007``):
the ``ARCH.*`` metadata keys, defaults included.  Tensor names are ggml's
(``blk.N.attn_q.weight`` ...; ``translate_name``, ``:610-660``, maps them
for the reference's builders; ``load_model`` maps them onto the decode
step's layout directly).

The file is memory-mapped; ``tensor_data`` returns views into the map.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from typing import Any, Iterable

import numpy as np

from . import gguf

MAGIC = b"GGUF"

# metadata value types (GGUF spec; src/formats.rs:183-214)
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<u1", T_I8: "<i1", T_U16: "<u2", T_I16: "<i2", T_U32: "<u4", T_I32: "<i4", T_F32: "<f4",
           T_BOOL: "<u1", T_U64: "<u8", T_I64: "<i8", T_F64: "<f8"}

# non-block ggml tensor types the container may hold (src/formats.rs:90-117)
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
_PLAIN = {GGML_F32: 4, GGML_F16: 2, GGML_BF16: 2}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file (the reference's ``gguf`` errors)."""


def tensor_type_name(t: int) -> str:
    if t in _PLAIN:
        return {GGML_F32: "F32", GGML_F16: "F16", GGML_BF16: "BF16"}[t]
    return gguf.DType(t).name


def check_tensor_type(t: int) -> int:
    """The ggml type ids the reference registers (src/formats.rs:90-117)."""
    if t in _PLAIN or gguf.is_gguf_block(t):
        return t
    raise GGUFError(f"ggml tensor type {t} is not registered in this build (supported: F32, F16, BF16, Q8_0, "
                    "Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K, IQ4_XS)")


def tensor_bytes(t: int, numel: int) -> int:
    """Bytes a tensor occupies on disk (src/formats.rs:119-132)."""
    if t in _PLAIN:
        return numel * _PLAIN[t]
    return gguf.storage_bytes(t, numel)


@dataclass
class TensorInfo:
    name: str
    ggml_type: int
    shape: tuple        # outermost-first (row-major)
    offset: int         # absolute byte offset in the file
    nbytes: int

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1


class _Cursor:
    def __init__(self, b, pos: int = 0):
        self.b, self.pos = b, pos

    def take(self, n: int):
        if self.pos + n > len(self.b):
            raise GGUFError(f"truncated file: need {n} bytes at offset {self.pos}, "
                            f"have {len(self.b) - min(self.pos, len(self.b))}")
        s = self.b[self.pos:self.pos + n]
        self.pos += n
        return s

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def string(self) -> str:
        n = self.u64()
        if n > 1 << 24:
            raise GGUFError(f"implausible string length {n} -- corrupt header")
        return bytes(self.take(n)).decode("utf-8", errors="replace")

    def value(self, ty: int, depth: int = 0) -> Any:
        if depth > 2:
            raise GGUFError("metadata arrays nested deeper than the spec allows")
        if ty in _SCALAR:
            dt = np.dtype(_SCALAR[ty])
            v = np.frombuffer(self.take(dt.itemsize), dt)[0]
            return bool(v) if ty == T_BOOL else v.item()
        if ty == T_STR:
            return self.string()
        if ty == T_ARR:
            et, n = self.u32(), self.u64()
            if n > 1 << 26:
                raise GGUFError(f"implausible array length {n} -- corrupt header")
            if et in _SCALAR:  # numeric arrays in one read
                dt = np.dtype(_SCALAR[et])
                a = np.frombuffer(self.take(dt.itemsize * n), dt).copy()
                return a.astype(bool) if et == T_BOOL else a
            return [self.value(et, depth + 1) for _ in range(n)]
        raise GGUFError(f"unknown metadata value type {ty}")


class GGUFFile:
    """A parsed, memory-mapped GGUF file (``GgufWeights::open``,
    src/formats.rs:247-345, one part)."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            try:
                self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            except ValueError as e:  # an empty file
                raise GGUFError(f"'{path}' is not a GGUF file (empty)") from e
        b = memoryview(self._map)
        if len(b) < 24 or bytes(b[0:4]) != MAGIC:
            raise GGUFError(f"'{path}' is not a GGUF file (bad magic)")
        c = _Cursor(b, 4)
        self.version = c.u32()
        if not 2 <= self.version <= 3:
            raise GGUFError(f"GGUF version {self.version} unsupported (this build reads v2/v3)")
        n_tensors, n_kv = c.u64(), c.u64()
        if n_tensors > 1 << 20 or n_kv > 1 << 20:
            raise GGUFError(f"implausible header counts (tensors={n_tensors}, kv={n_kv})")
        self.meta: dict[str, Any] = {}
        for _ in range(n_kv):
            key = c.string()
            self.meta[key] = c.value(c.u32())
        raw = []
        for _ in range(n_tensors):
            name = c.string()
            n_dims = c.u32()
            if n_dims > 4:
                raise GGUFError(f"tensor '{name}' has {n_dims} dims (max 4)")
            dims = [c.u64() for _ in range(n_dims)]
            t = check_tensor_type(c.u32())
            raw.append((name, t, tuple(reversed(dims)), c.u64()))
        self.alignment = int(self.meta.get("general.alignment", 32))
        if self.alignment <= 0:
            raise GGUFError(f"general.alignment {self.alignment} is not positive")
        self.data_start = -(-c.pos // self.alignment) * self.alignment
        self.tensors: dict[str, TensorInfo] = {}
        for name, t, shape, off in raw:
            numel = int(np.prod(shape, dtype=np.int64)) if shape else 1
            be = gguf.block_elems(t) if gguf.is_gguf_block(t) else 1
            if numel % be:
                raise GGUFError(f"tensor '{name}': {numel} elements are not a whole number of {be}-element blocks")
            nbytes = tensor_bytes(t, numel)
            start = self.data_start + off
            if start + nbytes > len(b):
                raise GGUFError(f"tensor '{name}' data ends at {start + nbytes} but '{path}' is {len(b)} bytes "
                                "-- truncated")
            self.tensors[name] = TensorInfo(name, t, shape, start, nbytes)
        self.architecture = str(self.meta.get("general.architecture", ""))

    def close(self) -> None:
        """Unmap the file, unless arrays returned by tensor_data (or a model
        loaded from it) still use it: then the map lives until they go."""
        try:
            self._map.close()
        except BufferError:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tensor_data(self, name: str) -> np.ndarray:
        """The tensor as stored: block formats as uint8 rows [rows, row
        bytes] (rows = all but the innermost dim), F32 / F16 typed arrays of
        the tensor's shape, BF16 as uint16.  A view into the file."""
        ti = self.tensors[name]
        a = np.frombuffer(self._map, np.uint8, ti.nbytes, ti.offset)
        if gguf.is_gguf_block(ti.ggml_type):
            k = ti.shape[-1] if ti.shape else 1
            return a.reshape(-1, gguf.storage_bytes(ti.ggml_type, k))
        dt = {GGML_F32: np.float32, GGML_F16: np.float16, GGML_BF16: np.uint16}[ti.ggml_type]
        return a.view(dt).reshape(ti.shape)

    def meta_int(self, key: str):
        v = self.meta.get(key)
        return None if v is None or isinstance(v, (list, np.ndarray, str)) else int(v)

    def meta_float(self, key: str):
        v = self.meta.get(key)
        return None if v is None or isinstance(v, (list, np.ndarray, str)) else float(v)


# ------------------------------------------------------------------ writer

def _pack_value(ty: int, v: Any) -> bytes:
    if ty in _SCALAR:
        return np.array([v], _SCALAR[ty]).tobytes()
    if ty == T_STR:
        s = v.encode("utf-8")
        return struct.pack("<Q", len(s)) + s
    if ty == T_ARR:
        et, items = v
        if et in _SCALAR:
            a = np.asarray(items, _SCALAR[et])
            return struct.pack("<IQ", et, a.size) + a.tobytes()
        return struct.pack("<IQ", et, len(items)) + b"".join(_pack_value(et, x) for x in items)
    raise GGUFError(f"unknown metadata value type {ty}")


def write(path: str, meta: Iterable[tuple], tensors: Iterable[tuple], version: int = 3,
          alignment: int = 32) -> None:
    """Write a GGUF file.  meta: (key, value type, value) with arrays as
    (element type, items); tensors: (name, ggml type, shape outermost-first,
    bytes).  general.alignment is written when it is not 32."""
    meta = list(meta)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", T_U32, alignment))
    tensors = list(tensors)
    out = bytearray(MAGIC + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for key, ty, v in meta:
        k = key.encode("utf-8")
        out += struct.pack("<Q", len(k)) + k + struct.pack("<I", ty) + _pack_value(ty, v)
    offs, pos = [], 0
    for name, t, shape, data in tensors:
        if len(data) != tensor_bytes(t, int(np.prod(shape, dtype=np.int64))):
            raise GGUFError(f"tensor '{name}': {len(data)} bytes for shape {tuple(shape)} of type {t}")
        offs.append(pos)
        pos = -(-(pos + len(data)) // alignment) * alignment
    for (name, t, shape, data), off in zip(tensors, offs):
        n = name.encode("utf-8")
        out += struct.pack("<Q", len(n)) + n + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", d) for d in reversed(shape))
        out += struct.pack("<IQ", t, off)
    out += bytes(-len(out) % alignment)
    data_start = len(out)
    for (name, t, shape, data), off in zip(tensors, offs):
        out += bytes(data_start + off - len(out))  # each tensor at its aligned offset
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)


# ------------------------------------------------- the decoder in the file

def decoder_config(g: GGUFFile, max_seq: int | None = None, attn_chunk: int = 128,
                   use_sliding_window: bool = False):
    """DecoderConfig from the metadata (``model_config``,
    src/formats.rs:940-1007), for the qwen2 / llama tensor family.

    The reference's model_config ignores ``{arch}.attention.sliding_window``
    for these architectures and always decodes with full causal attention,
    so by default this loader does too (window 0): a file that carries the
    key -- one converted from an HF config with use_sliding_window=false,
    say -- decodes as the reference decodes it.  ``use_sliding_window=True``
    opts in to the file's single window (a per-layer pattern is refused
    then rather than decoded with the wrong span)."""
    from .decoder import DecoderConfig

    a = g.architecture

    def need(attr):
        v = g.meta_int(f"{a}.{attr}")
        if v is None:
            raise GGUFError(f"metadata is missing {a}.{attr} -- cannot synthesize the model config")
        return v

    n_heads, hidden = need("attention.head_count"), need("embedding_length")
    vocab = g.meta_int(f"{a}.vocab_size")
    if vocab is None and "tokenizer.ggml.tokens" in g.meta:
        vocab = len(g.meta["tokenizer.ggml.tokens"])
    if vocab is None:
        raise GGUFError("cannot determine vocab size from metadata")
    ctx = g.meta_int(f"{a}.context_length") or 8192
    ms = min(ctx, 8192) if max_seq is None else min(ctx, max_seq)
    q = g.tensors.get("blk.0.attn_q.weight")
    if q is None:
        raise GGUFError("blk.0.attn_q.weight is missing -- not a qwen2 / llama-family decoder")
    eps = g.meta_float(f"{a}.attention.layer_norm_rms_epsilon")
    theta = g.meta_float(f"{a}.rope.freq_base")
    # sliding-window attention, opt-in: one window for every layer is
    # supported; a per-layer pattern (alternating local / global layers) is
    # not, and is refused rather than decoded with the wrong attention span
    window = (g.meta_int(f"{a}.attention.sliding_window") or 0) if use_sliding_window else 0
    if window and any(k.startswith(f"{a}.attention.sliding_window_") for k in g.meta):
        raise GGUFError(f"{a}: per-layer sliding-window patterns are not supported by this decoder")
    return DecoderConfig(
        n_layers=need("block_count"), hidden=hidden, q_heads=n_heads,
        kv_heads=g.meta_int(f"{a}.attention.head_count_kv") or n_heads,
        head_dim=g.meta_int(f"{a}.attention.key_length") or hidden // n_heads,
        ffn=need("feed_forward_length"), vocab=vocab,
        rope_theta=1e4 if theta is None else theta, rms_eps=1e-6 if eps is None else eps,
        qkv_bias="blk.0.attn_q.bias" in g.tensors, tied="output.weight" not in g.tensors,
        ggml_type=q.ggml_type, max_seq=ms, attn_chunk=attn_chunk, window=window)


def _f16_vector(g: GGUFFile, name: str, n: int) -> np.ndarray:
    ti = g.tensors.get(name)
    if ti is None:
        raise GGUFError(f"tensor '{name}' is missing")
    if ti.numel != n or ti.ggml_type not in (GGML_F32, GGML_F16):
        raise GGUFError(f"tensor '{name}': {ti.shape} {tensor_type_name(ti.ggml_type)}, want {n} F32/F16 values")
    return g.tensor_data(name).reshape(-1).astype(np.float16)


def _matrix(g: GGUFFile, name: str, rows: int, k: int):
    ti = g.tensors.get(name)
    if ti is None:
        raise GGUFError(f"tensor '{name}' is missing")
    if not gguf.is_gguf_block(ti.ggml_type):
        raise GGUFError(f"tensor '{name}' is {tensor_type_name(ti.ggml_type)}: the decode step runs GGUF block "
                        "formats")
    if tuple(ti.shape) != (rows, k):
        raise GGUFError(f"tensor '{name}' has shape {tuple(ti.shape)}, want {(rows, k)}")
    return g.tensor_data(name), int(ti.ggml_type)


def load_model(g: GGUFFile, max_seq: int | None = None, attn_chunk: int = 128,
               use_sliding_window: bool = False):
    """The qwen2 / llama-family decoder of a GGUF file as a HostModel, in
    the decode step's layout: q, k, v as one matrix when they share a
    format (else separate), gate and up as one; norms and biases as f16.
    Full causal attention unless ``use_sliding_window`` (decoder_config)."""
    from .decoder import HostModel

    c = decoder_config(g, max_seq, attn_chunk, use_sliding_window)
    qd, kvd = c.q_heads * c.head_dim, c.kv_heads * c.head_dim
    embed, et = _matrix(g, "token_embd.weight", c.vocab, c.hidden)
    m = HostModel(c, embed, _f16_vector(g, "output_norm.weight", c.hidden), embed_type=et)
    if not c.tied:
        m.head, m.head_type = _matrix(g, "output.weight", c.vocab, c.hidden)
    for i in range(c.n_layers):
        p = f"blk.{i}."
        wq, tq = _matrix(g, p + "attn_q.weight", qd, c.hidden)
        wk, tk = _matrix(g, p + "attn_k.weight", kvd, c.hidden)
        wv, tv = _matrix(g, p + "attn_v.weight", kvd, c.hidden)
        wo, to = _matrix(g, p + "attn_output.weight", c.hidden, qd)
        wg, tg = _matrix(g, p + "ffn_gate.weight", c.ffn, c.hidden)
        wu, tu = _matrix(g, p + "ffn_up.weight", c.ffn, c.hidden)
        wd, td = _matrix(g, p + "ffn_down.weight", c.hidden, c.ffn)
        if tg != tu:
            raise GGUFError(f"layer {i}: ffn_gate ({tensor_type_name(tg)}) and ffn_up ({tensor_type_name(tu)}) "
                            "formats differ")
        L = {"attn_norm": _f16_vector(g, p + "attn_norm.weight", c.hidden),
             "ffn_norm": _f16_vector(g, p + "ffn_norm.weight", c.hidden),
             "wo": np.ascontiguousarray(wo), "w_down": np.ascontiguousarray(wd),
             "w_gate_up": np.concatenate([wg, wu]),
             "types": dict(q=tq, k=tk, v=tv, o=to, gate=tg, up=tu, down=td),
             "bqkv": (np.concatenate([_f16_vector(g, p + f"attn_{x}.bias", n) for x, n in
                                      (("q", qd), ("k", kvd), ("v", kvd))]) if c.qkv_bias else None)}
        if tq == tk == tv:
            L["wqkv"] = np.concatenate([wq, wk, wv])
        else:
            L["wqkv"], L["wk"], L["wv"] = (np.ascontiguousarray(a) for a in (wq, wk, wv))
        m.layers.append(L)
    return m


def save_model(path: str, m, arch: str = "qwen2", alignment: int = 32) -> None:
    """Write a HostModel as a GGUF file with ggml tensor names and the
    ``ARCH.*`` metadata decoder_config reads (norms and biases as F32)."""
    c = m.cfg
    qd, kvd = c.q_heads * c.head_dim, c.kv_heads * c.head_dim
    meta = [("general.architecture", T_STR, arch), (f"{arch}.block_count", T_U32, c.n_layers),
            (f"{arch}.embedding_length", T_U32, c.hidden), (f"{arch}.feed_forward_length", T_U32, c.ffn),
            (f"{arch}.attention.head_count", T_U32, c.q_heads),
            (f"{arch}.attention.head_count_kv", T_U32, c.kv_heads),
            (f"{arch}.attention.key_length", T_U32, c.head_dim), (f"{arch}.context_length", T_U32, c.max_seq),
            (f"{arch}.rope.freq_base", T_F32, c.rope_theta),
            (f"{arch}.attention.layer_norm_rms_epsilon", T_F32, c.rms_eps),
            (f"{arch}.vocab_size", T_U32, c.vocab)]
    if c.window:
        meta.append((f"{arch}.attention.sliding_window", T_U32, c.window))
    f32 = lambda a: np.asarray(a, np.float32).tobytes()  # noqa: E731
    ts = [("token_embd.weight", m.embed_type, (c.vocab, c.hidden), m.embed.tobytes()),
          ("output_norm.weight", GGML_F32, (c.hidden,), f32(m.final_norm))]
    if m.head is not None:
        ts.append(("output.weight", m.head_type, (c.vocab, c.hidden), m.head.tobytes()))
    for i, L in enumerate(m.layers):
        p = f"blk.{i}."
        ty = {k: L["types"].get(k, int(c.ggml_type)) for k in ("q", "k", "v", "o", "gate", "up", "down")}
        if L.get("wk") is None:
            rq = gguf.row_bytes(ty["q"], c.hidden)
            wq, wk, wv = L["wqkv"][:qd], L["wqkv"][qd:qd + kvd], L["wqkv"][qd + kvd:]
            assert wq.shape[1] == rq
        else:
            wq, wk, wv = L["wqkv"], L["wk"], L["wv"]
        ts += [(p + "attn_norm.weight", GGML_F32, (c.hidden,), f32(L["attn_norm"])),
               (p + "attn_q.weight", ty["q"], (qd, c.hidden), wq.tobytes()),
               (p + "attn_k.weight", ty["k"], (kvd, c.hidden), wk.tobytes()),
               (p + "attn_v.weight", ty["v"], (kvd, c.hidden), wv.tobytes())]
        if L.get("bqkv") is not None:
            b = L["bqkv"]
            ts += [(p + "attn_q.bias", GGML_F32, (qd,), f32(b[:qd])),
                   (p + "attn_k.bias", GGML_F32, (kvd,), f32(b[qd:qd + kvd])),
                   (p + "attn_v.bias", GGML_F32, (kvd,), f32(b[qd + kvd:]))]
        ts += [(p + "attn_output.weight", ty["o"], (c.hidden, qd), L["wo"].tobytes()),
               (p + "ffn_norm.weight", GGML_F32, (c.hidden,), f32(L["ffn_norm"])),
               (p + "ffn_gate.weight", ty["gate"], (c.ffn, c.hidden), L["w_gate_up"][:c.ffn].tobytes()),
               (p + "ffn_up.weight", ty["up"], (c.ffn, c.hidden), L["w_gate_up"][c.ffn:].tobytes()),
               (p + "ffn_down.weight", ty["down"], (c.hidden, c.ffn), L["w_down"].tobytes())]
    write(path, meta, ts, alignment=alignment)
