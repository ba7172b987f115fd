"""CPU tests: pin the oracle.

The reference's own known-answer tests (src/quant.rs:1010-1218) are restated
here against the C oracle, then the oracle is checked against independent
codings: numpy's IEEE float16 casts, the closed-form numpy decoder in
tests/golden/make_golden.py and its committed fixtures, and float64 dots.
"""
import numpy as np
import pytest

import oracle
import make_golden as mg

Q4_0, Q8_0, Q4_K, Q6_K = oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q6_K
Q4_1, Q5_0, Q5_1, Q5_K, IQ4_XS = oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q5_K, oracle.IQ4_XS
FORMATS = [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K, IQ4_XS]
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q4_K: "q4_k", Q5_K: "q5_k",
         Q6_K: "q6_k", IQ4_XS: "iq4_xs"}


def f16le(v: float) -> bytes:
    return int(oracle.f32_to_f16(v)).to_bytes(2, "little")


def is_nan16(v):
    v = np.asarray(v, dtype=np.uint16)
    return ((v & 0x7C00) == 0x7C00) & ((v & 0x3FF) != 0)


def same_bits(a, b):
    """bit equality, NaNs equal as a class (src/selftest.rs:970-975)"""
    a = np.asarray(a, dtype=np.uint16)
    b = np.asarray(b, dtype=np.uint16)
    return (a == b) | (is_nan16(a) & is_nan16(b))


# --------------------------------------------- reference known-answer tests

def test_q8_0_block_reference():
    """src/quant.rs:1011-1024"""
    blk = bytearray(34)
    blk[0:2] = f16le(0.5)
    for i in range(32):
        blk[2 + i] = (i * 3 - 40) & 0xFF
    out = oracle.f16_bits_to_f32(oracle.dequant(Q8_0, np.frombuffer(bytes(blk), np.uint8), 32))
    for i in range(32):
        assert abs(out[i] - 0.5 * (i * 3 - 40)) < 1e-3, i
        assert out[i] == 0.5 * (i * 3 - 40)  # exact: small multiples of 0.5


def test_q4_k_sub_block_scales_and_mins():
    """src/quant.rs:1027-1072: scale[j] = j+1, min[j] = j, packed across the
    j<4 / j>=4 boundary of the 6-bit layout."""
    blk = bytearray(144)
    blk[0:2] = f16le(1.0)
    blk[2:4] = f16le(1.0)
    sc = [j + 1 for j in range(8)]
    mn = list(range(8))
    s = [0] * 12
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = mn[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 0x0F) | ((mn[j] & 0x0F) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (mn[j] >> 4) << 6
    blk[4:16] = bytes(s)
    for i in range(128):
        blk[16 + i] = (i % 16) | ((15 - i % 16) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q4_K, np.frombuffer(bytes(blk), np.uint8), 256))
    for c in range(4):
        for i in range(32):
            q = blk[16 + c * 32 + i]
            want_lo = (2 * c + 1) * (q & 0x0F) - (2 * c)
            want_hi = (2 * c + 2) * (q >> 4) - (2 * c + 1)
            assert abs(out[c * 64 + i] - want_lo) < 0.51, (c, i)
            assert abs(out[c * 64 + 32 + i] - want_hi) < 0.51, (c, i)
            assert out[c * 64 + i] == want_lo and out[c * 64 + 32 + i] == want_hi  # exact integers


def test_q6_k_reconstructs_signed_six_bit():
    """src/quant.rs:1075-1100"""
    blk = bytearray(210)
    for j in range(16):
        blk[192 + j] = 2
    blk[208:210] = f16le(1.0)
    for l in range(32):
        v = max(-32, min(31, l * 2 - 31))
        q = v + 32
        blk[l] = (blk[l] & 0xF0) | (q & 0x0F)
        blk[128 + l] = (blk[128 + l] & ~0x03 & 0xFF) | ((q >> 4) & 0x03)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q6_K, np.frombuffer(bytes(blk), np.uint8), 256))
    for l in range(32):
        v = max(-32, min(31, l * 2 - 31))
        assert abs(out[l] - 2.0 * v) < 1e-2, l


def test_q4_0_nibble_order_and_offset():
    """src/quant.rs:1220-1240"""
    blk = bytearray(18)
    blk[0:2] = f16le(0.25)
    for j in range(16):
        blk[2 + j] = j | ((15 - j) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q4_0, np.frombuffer(bytes(blk), np.uint8), 32))
    for j in range(16):
        assert abs(out[j] - 0.25 * (j - 8)) < 1e-3
        assert abs(out[j + 16] - 0.25 * ((15 - j) - 8)) < 1e-3


def test_q4_1_scale_plus_min():
    """src/quant.rs:1245-1259"""
    blk = bytearray(20)
    blk[0:2] = f16le(0.5)
    blk[2:4] = f16le(-1.5)
    for j in range(16):
        blk[4 + j] = j | ((15 - j) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q4_1, np.frombuffer(bytes(blk), np.uint8), 32))
    for j in range(16):
        assert abs(out[j] - (0.5 * j - 1.5)) < 1e-3
        assert abs(out[j + 16] - (0.5 * (15 - j) - 1.5)) < 1e-3


def test_q5_0_fifth_bit_mapping():
    """src/quant.rs:1261-1279: bit r of qh is element r's 5th bit (exact
    values, so equality)"""
    blk = bytearray(22)
    blk[0:2] = f16le(1.0)
    qh = 0xA5F00F5A
    blk[2:6] = qh.to_bytes(4, "little")
    for j in range(16):
        blk[6 + j] = (j % 16) | ((j % 16) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q5_0, np.frombuffer(bytes(blk), np.uint8), 32))
    for r in range(32):
        assert out[r] == (r % 16) + ((qh >> r) & 1) * 16 - 16, r


def test_q5_1_fifth_bit_plus_min():
    """src/quant.rs:1281-1305 (exact values here, so equality)"""
    blk = bytearray(24)
    blk[0:2] = f16le(0.5)
    blk[2:4] = f16le(2.0)
    qh = 0x1234ABCD
    blk[4:8] = qh.to_bytes(4, "little")
    for j in range(16):
        blk[8 + j] = j | ((15 - j) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(Q5_1, np.frombuffer(bytes(blk), np.uint8), 32))
    for r in range(32):
        nib = r if r < 16 else 15 - (r - 16)
        assert out[r] == 0.5 * (nib + ((qh >> r) & 1) * 16) + 2.0, r


def test_q5_k_fifth_bit_and_rotating_masks():
    """src/quant.rs:1101-1138: d = 1, dmin = 0, scales 1; qh bit 2 lifts
    chunk 1's low half by 16 and leaves chunk 0 alone"""
    blk = bytearray(176)
    blk[0:2] = f16le(1.0)
    blk[2:4] = f16le(0.0)
    for j in range(4):
        blk[4 + j] = 1
        blk[4 + j + 4] = 0
    for j in range(4, 8):
        blk[4 + j + 4] = 1
    for i in range(128):
        blk[48 + i] = (i % 16) | ((i % 16) << 4)
    for i in range(32):
        blk[16 + i] = 0b0000_0100
    out = oracle.f16_bits_to_f32(oracle.dequant(Q5_K, np.frombuffer(bytes(blk), np.uint8), 256))
    for l in range(32):
        nib = l % 16
        assert out[l] == nib, l
        assert out[64 + l] == nib + 16, l


def test_iq4_xs_codebook_and_split_scales():
    """src/quant.rs:1140-1169: sub-block 0 scale 33 (ls - 32 = 1) from
    scales_l's low nibble 1 and scales_h bits 10b; sub-block 1 scale 0 -> -32"""
    blk = bytearray(136)
    blk[0:2] = f16le(1.0)
    blk[2] = 0b0000_0010
    blk[4] = 0x01
    for i in range(16):
        blk[8 + i] = (i % 16) | ((i % 16) << 4)
    out = oracle.f16_bits_to_f32(oracle.dequant(IQ4_XS, np.frombuffer(bytes(blk), np.uint8), 256))
    for j in range(16):
        assert out[j] == mg.IQ4NL[j], j
    assert out[32] == -32.0 * mg.IQ4NL[0]


def test_f16_converters_are_ieee_exact():
    """src/quant.rs:1171-1204: exhaustive round trip, NaN class, RTNE ties."""
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.f16_to_f32_array(h)
    back = oracle.f32_to_f16_array(f)
    nan = is_nan16(h)
    assert np.all(back[~nan] == h[~nan])
    assert np.all(np.isnan(f[nan]))
    assert np.all((back[nan] & 0x7C00) == 0x7C00) and np.all((back[nan] & 0x3FF) != 0)
    for hv in [0, 1, 2, 0x3FF, 0x400, 0x7BFE, 0x1234]:
        a = float(oracle.f16_to_f32(hv))
        b = float(oracle.f16_to_f32(hv + 1))
        mid = np.float32((a + b) / 2.0)
        r = oracle.f32_to_f16(float(mid))
        assert r in (hv, hv + 1)
        assert r & 1 == 0, hex(hv)


def test_storage_sizes_match_ggml():
    """src/quant.rs:1207-1218"""
    assert oracle.storage_bytes(Q8_0, 1024) == 1024 // 32 * 34
    assert oracle.storage_bytes(Q4_0, 1024) == 1024 // 32 * 18
    assert oracle.storage_bytes(Q4_1, 1024) == 1024 // 32 * 20
    assert oracle.storage_bytes(Q5_0, 1024) == 1024 // 32 * 22
    assert oracle.storage_bytes(Q5_1, 1024) == 1024 // 32 * 24
    assert oracle.storage_bytes(Q4_K, 1024) == 1024 // 256 * 144
    assert oracle.storage_bytes(Q5_K, 1024) == 1024 // 256 * 176
    assert oracle.storage_bytes(IQ4_XS, 1024) == 1024 // 256 * 136
    assert oracle.storage_bytes(Q6_K, 1024) == 1024 // 256 * 210


# ------------------------------------------------ independent library oracle

def test_f16_to_f32_matches_numpy_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_to_f32_array(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(ours[nan]))


def test_f32_to_f16_matches_numpy_rtne():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 1_000_000, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    # concentrate samples on the f16 range, subnormals and ties
    near = (rng.standard_normal(500_000) * 10.0 ** rng.uniform(-9, 5, 500_000)).astype(np.float32)
    ties = (np.arange(1, 65535, dtype=np.uint16).view(np.float16).astype(np.float64))
    with np.errstate(all="ignore"):
        ties = ((ties[:-1] + ties[1:]) / 2).astype(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8,
                         2.9802322e-08, -2.9802322e-08, 1e-10], dtype=np.float32)
    allv = np.concatenate([v, near, ties[np.isfinite(ties)], specials])
    ours = oracle.f32_to_f16_array(allv)
    with np.errstate(all="ignore"):
        ref = allv.astype(np.float16).view(np.uint16)
    assert np.all(same_bits(ours, ref))
    # NaN canonicalises to sign|0x7e00
    nan = np.isnan(allv)
    sign = (allv[nan].view(np.uint32) >> 16) & 0x8000
    assert np.all(ours[nan] == (sign | 0x7E00))


# --------------------------------------------------- decoders vs closed form

@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_dequant_matches_closed_form_random_blocks(t):
    be, bb = mg.BLOCK[t]
    src = np.random.default_rng(t).integers(0, 256, bb * 3000, dtype=np.uint8)
    ours = oracle.dequant(t, src, 3000 * be)
    ref = mg.decode(t, src)
    assert np.all(same_bits(ours, ref))


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_dequant_golden_fixture(t):
    g = np.load(mg.GOLDEN)
    be, bb = mg.BLOCK[t]
    src = g[f"{NAMES[t]}_blocks"]
    ours = oracle.dequant(t, src, len(src) // bb * be)
    assert np.all(same_bits(ours, g[f"{NAMES[t]}_f16"]))


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_dequant_exactly_one_rounding(t):
    """Each value equals the exact real value rounded to f32 then to f16:
    scales pinned sane, every block checked against float64 by element."""
    be, bb = mg.BLOCK[t]
    src = mg.sane_scales(t, np.random.default_rng(100 + t).integers(0, 256, bb * 500, dtype=np.uint8))
    ours = oracle.dequant(t, src, 500 * be)
    assert not np.any(is_nan16(ours))
    assert np.all(same_bits(ours, mg.decode(t, src)))


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_dequant_size_mismatch_errors(t):
    be, bb = mg.BLOCK[t]
    src = np.zeros(bb * 4, dtype=np.uint8)
    with pytest.raises(ValueError):
        oracle.dequant(t, src, 4 * be + 1)  # not a block multiple
    with pytest.raises(ValueError):
        oracle.dequant(t, src[:-1], 4 * be)  # too few bytes
    assert oracle.dequant(t, src, 0).size == 0  # empty is fine


def test_unsupported_format_rejected():
    with pytest.raises(ValueError):
        oracle.dequant(10, np.zeros(84, np.uint8), 256)  # Q2_K: not a format the reference executes


# ----------------------------------------------------------- gemv / gemm

@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_gemv_golden_fixture(t):
    g = np.load(mg.GOLDEN)
    n, k = (int(v) for v in g[f"{NAMES[t]}_gemv_shape"])
    w = g[f"{NAMES[t]}_gemv_w"]
    x = g[f"{NAMES[t]}_gemv_x"]
    w16 = oracle.dequant(t, w, n * k)
    y = oracle.gemv(w16, x, n, k)
    y64 = g[f"{NAMES[t]}_gemv_y64"]
    terms = np.abs(oracle.f16_bits_to_f32(w16).reshape(n, k).astype(np.float64) * x).sum(1)
    assert np.all(np.abs(y - y64) <= 1e-6 * terms + 1e-30)
    assert np.allclose(oracle.gguf_gemv_packed(t, w, x, n, k), y, rtol=0, atol=0)


def test_gemv_epilogues_closed_form():
    rng = np.random.default_rng(3)
    n, k = 37, 96
    w16 = rng.standard_normal((2 * n, k)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(k).astype(np.float32)
    bias = rng.standard_normal(2 * n).astype(np.float32)
    y_old = rng.standard_normal(n).astype(np.float32)
    W = w16.view(np.float16).astype(np.float64)
    dot = W @ x.astype(np.float64)
    y0 = oracle.gemv(w16, x, n, k, mode=0, bias=bias)
    assert np.allclose(y0, dot[:n] + bias[:n], rtol=1e-5, atol=1e-5)
    y1 = oracle.gemv(w16, x, n, k, mode=1, bias=bias, y_old=y_old)
    assert np.allclose(y1, y_old + dot[:n] + bias[:n], rtol=1e-5, atol=1e-5)
    y2 = oracle.gemv(w16, x, n, k, mode=2, bias=bias)
    g = dot[:n] + bias[:n]
    u = dot[n:] + bias[n:]
    assert np.allclose(y2, g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-5)


def test_gemm_matches_float64():
    rng = np.random.default_rng(4)
    m, n, k = 5, 33, 256
    w16 = (rng.standard_normal((n, k)) * 0.02).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = oracle.gemm(x, w16, m, n, k)
    ref = x.astype(np.float64) @ w16.view(np.float16).astype(np.float64).T
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_gather_is_rowwise_dequant(t):
    be, bb = mg.BLOCK[t]
    hidden, vocab = 2 * 256, 40
    rb = hidden // be * bb
    table = np.random.default_rng(t).integers(0, 256, vocab * rb, dtype=np.uint8)
    ids = np.array([3, 0, 39, 3, 17], dtype=np.uint32)
    got = oracle.gather(t, table, ids, hidden)
    for i, r in enumerate(ids):
        assert np.all(same_bits(got[i], mg.decode(t, table[r * rb:(r + 1) * rb])))
    with pytest.raises(ValueError):
        oracle.gather(t, table, np.array([vocab], np.uint32), hidden)  # out of range
