"""Independent numpy decoder for the GGUF formats + golden-fixture generator.

This is a second, separate coding of the block decoders, written from the
closed form rather than from the reference's loop structure: every product
in Q8_0 / Q4_0 / Q4_K / Q6_K is exact in binary32, so each decoded value is
the exact real number (d*sc)*q - dmin*m (computed in float64, where it is
exact), rounded once to float32 and once to float16 -- the reference's
f32 arithmetic followed by f32_to_f16 (src/quant.rs:599-896,
src/traits.rs:857-896).  Element/nibble/bit placement is derived from the
block layout comments of src/quant.rs:547-564 and the decoders' index maps,
expressed as whole-array reshapes.

Fixtures (``gguf_golden.npz``) hold random blocks drawn from the reference
selftest's xorshift64 stream (seed 0x9E3779B97F4A7C15, src/selftest.rs:
911-917), the f16 bits this decoder assigns them, and small GEMV cases
(x, y in float64 over the decoded weights).  Regenerate with
``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import os

import numpy as np

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 2, 3, 6, 7, 8, 12, 13, 14, 23
BLOCK = {Q8_0: (32, 34), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210), IQ4_XS: (256, 136)}
# ggml's kvalues_iq4nl
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float64)
HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "gguf_golden.npz")


def xorshift_bytes(nbytes: int, seed: int = 0x9E3779B97F4A7C15) -> np.ndarray:
    """The selftest's xorshift64 stream, little-endian u64 words as bytes."""
    M = (1 << 64) - 1
    words = []
    s = seed
    for _ in range((nbytes + 7) // 8):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        words.append(s)
    return np.array(words, dtype="<u8").view(np.uint8)[:nbytes].copy()


def _f16(b: np.ndarray, off: int) -> np.ndarray:
    """f16 field at byte offset `off` of each block row -> float64."""
    return b[:, off:off + 2].copy().view("<f2").astype(np.float64)[:, 0]


def _round(v64: np.ndarray) -> np.ndarray:
    """exact value -> binary32 -> binary16 bits"""
    with np.errstate(all="ignore"):
        return v64.astype(np.float32).astype(np.float16).view(np.uint16)


def decode(t: int, src: np.ndarray) -> np.ndarray:
    """Packed blocks -> f16 bits, one row of elements per block, flattened."""
    return _round(decode_exact(t, src))


def decode_exact(t: int, src: np.ndarray) -> np.ndarray:
    """Packed blocks -> the exact real value of every element (float64, no
    rounding at all), flattened."""
    be, bb = BLOCK[t]
    b = np.asarray(src, dtype=np.uint8).reshape(-1, bb)
    nb = b.shape[0]
    with np.errstate(all="ignore"):
        if t == Q8_0:
            d = _f16(b, 0)
            q = b[:, 2:34].view(np.int8).astype(np.float64)
            v = d[:, None] * q
        elif t == Q4_0:
            d = _f16(b, 0)
            qs = b[:, 2:18]
            q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float64) - 8.0
            v = d[:, None] * q
        elif t in (Q4_1, Q5_0, Q5_1):
            # 32 elements: nibble bytes (low = element j, high = j + 16), a
            # 5th bit per element from a 32-bit mask (bit e = element e)
            d = _f16(b, 0)
            qoff = {Q4_1: 4, Q5_0: 6, Q5_1: 8}[t]
            qs = b[:, qoff:qoff + 16].astype(np.int64)
            q = np.concatenate([qs & 15, qs >> 4], axis=1)
            if t != Q4_1:
                hoff = 2 if t == Q5_0 else 4
                qh = b[:, hoff:hoff + 4].copy().view("<u4")[:, 0].astype(np.int64)
                q = q | (((qh[:, None] >> np.arange(32)[None, :]) & 1) << 4)
            if t == Q5_0:
                v = d[:, None] * (q - 16).astype(np.float64)      # no min term (keeps -0)
            else:
                v = d[:, None] * q.astype(np.float64) + _f16(b, 2)[:, None]
        elif t == IQ4_XS:
            d = _f16(b, 0)
            sh = b[:, 2:4].copy().view("<u2")[:, 0].astype(np.int64)
            sl = b[:, 4:8].astype(np.int64)
            ib = np.arange(8)
            ls = ((sl[:, ib // 2] >> (4 * (ib % 2))) & 15) | (((sh[:, None] >> (2 * ib)) & 3) << 4)
            qs = b[:, 8:136].reshape(nb, 8, 16).astype(np.int64)
            q = np.concatenate([qs & 15, qs >> 4], axis=2)            # sub-block, 32 elements
            v = (d[:, None, None] * (ls - 32)[:, :, None]) * IQ4NL[q]
            v = v.reshape(nb, 256)
        elif t in (Q4_K, Q5_K):
            d, dmin = _f16(b, 0), _f16(b, 2)
            s = b[:, 4:16].astype(np.int64)
            # 6-bit (scale, min) of sub-blocks 0..7
            sc = np.empty((nb, 8)); mn = np.empty((nb, 8))
            sc[:, :4] = s[:, 0:4] & 63
            mn[:, :4] = s[:, 4:8] & 63
            sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
            mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
            qs = b[:, 16:144].reshape(nb, 4, 32) if t == Q4_K else b[:, 48:176].reshape(nb, 4, 32)
            # chunk c: low nibbles -> sub-block 2c, high nibbles -> 2c+1
            q = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.int64)
            if t == Q5_K:
                # sub-block j's 5th bits: bit j of qh[l] (l = 0..31)
                qh = b[:, 16:48].astype(np.int64)
                q = q | (((qh[:, None, :] >> np.arange(8)[None, :, None]) & 1) << 4)
            q = q.astype(np.float64)
            v = (d[:, None, None] * sc[:, :, None]) * q - (dmin[:, None] * mn)[:, :, None]
            v = v.reshape(nb, 256)
        elif t == Q6_K:
            ql = b[:, 0:128].reshape(nb, 2, 2, 32).astype(np.int64)   # half, (l / l+32), l
            qh = b[:, 128:192].reshape(nb, 2, 32).astype(np.int64)    # half, l
            sc = b[:, 192:208].view(np.int8).astype(np.float64).reshape(nb, 2, 8)
            d = _f16(b, 208)
            q = np.empty((nb, 2, 4, 32), dtype=np.int64)              # half, group g, l
            for g in range(4):
                nib = (ql[:, :, g & 1, :] >> (4 * (g >> 1))) & 15
                q[:, :, g, :] = (nib | (((qh >> (2 * g)) & 3) << 4)) - 32
            # scale of (half, g, l) is sc[half, l // 16 + 2g]
            scl = np.empty((nb, 2, 4, 32))
            for g in range(4):
                scl[:, :, g, :16] = sc[:, :, 2 * g][:, :, None]
                scl[:, :, g, 16:] = sc[:, :, 2 * g + 1][:, :, None]
            v = (d[:, None, None, None] * scl) * q.astype(np.float64)
            v = v.reshape(nb, 256)
        else:
            raise ValueError(t)
    return v.reshape(-1)


def sane_scales(t: int, blocks: np.ndarray) -> np.ndarray:
    """Pin the f16 scale fields to exponent 14 (magnitude ~0.5..1), as the
    reference's GEMV selftest does (src/selftest.rs:1042-1063)."""
    be, bb = BLOCK[t]
    b = blocks.reshape(-1, bb).copy()
    offs = {Q6_K: [208], Q4_K: [0, 2], Q5_K: [0, 2], Q4_1: [0, 2], Q5_1: [0, 2]}.get(t, [0])
    for o in offs:
        h = b[:, o:o + 2].copy().view("<u2")[:, 0]
        h = (h & 0x83FF) | (14 << 10)
        b[:, o:o + 2] = h.astype("<u2").view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def gemv64(w16: np.ndarray, x: np.ndarray, n: int, k: int) -> np.ndarray:
    w = w16.view(np.float16).astype(np.float64).reshape(n, k)
    return w @ x.astype(np.float64)


def make() -> dict:
    out = {}
    for t, name in ((Q8_0, "q8_0"), (Q4_0, "q4_0"), (Q4_1, "q4_1"), (Q5_0, "q5_0"), (Q5_1, "q5_1"), (Q4_K, "q4_k"),
                    (Q5_K, "q5_k"), (Q6_K, "q6_k"), (IQ4_XS, "iq4_xs")):
        be, bb = BLOCK[t]
        nblocks = 24 if be == 256 else 64
        src = xorshift_bytes(nblocks * bb, seed=0x9E3779B97F4A7C15 + t)
        out[f"{name}_blocks"] = src
        out[f"{name}_f16"] = decode(t, src)
        # a tiny GEMV with sane scales: n rows of k
        n, k = 6, 2 * be if be == 256 else 4 * be
        w = sane_scales(t, xorshift_bytes(n * (k // be) * bb, seed=0xC1A5EED + t))
        rng = np.random.default_rng(1234 + t)
        x = rng.uniform(-1, 1, k).astype(np.float32)
        w16 = decode(t, w)
        out[f"{name}_gemv_w"] = w
        out[f"{name}_gemv_x"] = x
        out[f"{name}_gemv_y64"] = gemv64(w16, x, n, k)
        out[f"{name}_gemv_shape"] = np.array([n, k])
    return out


if __name__ == "__main__":
    np.savez_compressed(GOLDEN, **make())
    print("wrote", GOLDEN, os.path.getsize(GOLDEN), "bytes")
