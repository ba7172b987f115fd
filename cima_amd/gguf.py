"""GGUF block-format tables (host side).

Mirrors the reference's format metadata: ggml type ids
(``src/formats.rs:90-117``), ``storage_bytes`` (``src/formats.rs:119-132``),
``block_elems`` (``src/traits.rs:264-272``) and ``is_gguf_block``
(``src/traits.rs:244-257``), restricted to the formats this library executes.
"""
from __future__ import annotations

import enum


class DType(enum.IntEnum):
    """GGUF block formats by ggml tensor type id."""

    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ4_XS = 23

    @property
    def block_elems(self) -> int:
        return block_elems(self)

    @property
    def block_bytes(self) -> int:
        return _BLOCK_BYTES[self]


_BLOCK_ELEMS = {DType.Q8_0: 32, DType.Q4_0: 32, DType.Q4_1: 32, DType.Q5_0: 32, DType.Q5_1: 32,
                DType.Q4_K: 256, DType.Q5_K: 256, DType.Q6_K: 256, DType.IQ4_XS: 256}
_BLOCK_BYTES = {DType.Q8_0: 34, DType.Q4_0: 18, DType.Q4_1: 20, DType.Q5_0: 22, DType.Q5_1: 24,
                DType.Q4_K: 144, DType.Q5_K: 176, DType.Q6_K: 210, DType.IQ4_XS: 136}

# activation / output element types of the C ABI
DT_F32, DT_F16, DT_BF16 = 0, 1, 2


def is_gguf_block(t: int) -> bool:
    return t in _BLOCK_ELEMS


def block_elems(t: int) -> int:
    """Elements per block (the row-length grain); 1 for non-block types."""
    return _BLOCK_ELEMS.get(t, 1)


def storage_bytes(t: int, numel: int) -> int:
    """Bytes a tensor of ``numel`` elements of block format ``t`` occupies."""
    if t not in _BLOCK_ELEMS:
        raise ValueError(f"ggml type {t} is not a supported GGUF block format")
    return (numel // _BLOCK_ELEMS[t]) * _BLOCK_BYTES[t]


def row_bytes(t: int, k: int) -> int:
    return storage_bytes(t, k)
