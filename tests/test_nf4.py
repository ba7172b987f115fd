"""bitsandbytes 4-bit (NF4 / FP4): the oracle and the host-side loader.

The reference holds no NF4 known-answer test or fixture, so the oracle's
dequant_host restatement (src/quant.rs:401-437) is pinned by
  * an independent numpy statement of the closed form (one f32 product,
    rounded once to f16 by numpy's own conversion),
  * the nibble order the reference states (element 2j = HIGH nibble,
    src/kernels.cu:320-329, src/quant.rs:28) on a hand-made byte,
  * exact special cases: power-of-two codes and scales, round-half-to-even
    ties, overflow to infinity, f16 subnormals and the sign of zero,
and the absmax fold (src/quant.rs:258-330) by the same closed form
computed with float64 products that are exact for the chosen operands.
"""
import json

import numpy as np
import pytest

import oracle
from cima_amd import nf4
from cima_amd.hip import EngineError


def closed_form(packed, absmax, qmap, n, bs):
    i = np.arange(n)
    b = packed[i // 2].astype(np.int64)
    nib = np.where(i % 2 == 0, b >> 4, b & 15)
    prod = qmap.astype(np.float32)[nib] * absmax.astype(np.float32)[i // bs]  # f32 x f32 -> f32
    return prod.astype(np.float16).view(np.uint16)


def rand_case(seed, n, bs, signed_zero=True):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    absmax = (rng.standard_normal(n // bs) * 3).astype(np.float32)
    qmap = rng.standard_normal(16).astype(np.float32)
    if signed_zero:
        qmap[3] = -0.0
        qmap[7] = 0.0
    return packed, absmax, qmap


@pytest.mark.parametrize("bs", [2, 32, 64, 128, 4096, 48])
def test_oracle_dequant_matches_closed_form(bs):
    n = 4096 * 3
    packed, absmax, qmap = rand_case(bs, n, bs)
    got = oracle.nf4_dequant(packed, absmax, qmap, n, bs)
    np.testing.assert_array_equal(got, closed_form(packed, absmax, qmap, n, bs))


def test_oracle_nibble_order():
    q = np.arange(16, dtype=np.float32)
    got = oracle.f16_bits_to_f32(oracle.nf4_dequant(np.array([0xAB, 0x3C], np.uint8), np.ones(1, np.float32),
                                                    q, 4, 4))
    np.testing.assert_array_equal(got, [10.0, 11.0, 3.0, 12.0])


def test_oracle_exact_special_cases():
    # one element per block: element 2j high nibble -> code 1, element 2j+1 low -> code 2
    qmap = np.zeros(16, np.float32)
    qmap[1] = 1.0 + 2.0 ** -11   # exactly between f16 1.0 and its successor: ties to even (1.0)
    qmap[2] = 1.0 + 3 * 2.0 ** -11  # between 1+2^-10 and 1+2^-9: ties to even (1+2^-9)
    qmap[3] = -0.0
    qmap[4] = 2.0 ** -20           # f16 subnormal
    qmap[5] = 1.0
    packed = np.array([0x12, 0x34, 0x55, 0x35], np.uint8)
    absmax = np.array([1.0, 1.0, -1.0, 1.0, 70000.0, 2.0 ** -10, 3.0, -0.0], np.float32)
    got = oracle.nf4_dequant(packed, absmax, qmap, 8, 1)
    # signs of zero: -0 * -1 = +0, -0 * 3 = -0, 1 * -0 = -0
    want = np.array([0x3C00, 0x3C02, 0x0000, 0x0010, 0x7C00, 0x1400, 0x8000, 0x8000], np.uint16)
    np.testing.assert_array_equal(got, want)


def test_oracle_rejects_ragged():
    with pytest.raises(ValueError):
        oracle.nf4_dequant(np.zeros(8, np.uint8), np.ones(4, np.float32), np.zeros(16, np.float32), 12, 5)


def test_oracle_fold_exact():
    rng = np.random.default_rng(7)
    nblocks, nbs = 1000, 256
    codes = rng.integers(0, 256, nblocks, dtype=np.uint8)
    nmap = (rng.integers(-512, 512, 256) / 512.0).astype(np.float32)   # 10-bit values
    nabs = (rng.integers(1, 1024, (nblocks + nbs - 1) // nbs) / 64.0).astype(np.float32)
    off = np.float32(0.375)
    want = (nmap[codes].astype(np.float64) * nabs[np.arange(nblocks) // nbs] + off).astype(np.float32)  # exact
    np.testing.assert_array_equal(oracle.nf4_fold_absmax(codes, nmap, nabs, nbs, off), want)
    with pytest.raises(ValueError):
        oracle.nf4_fold_absmax(codes, nmap, nabs[:-1], nbs, off)


def test_oracle_fold_rounds_each_step():
    # product and sum rounded separately in f32 (no fused multiply-add)
    nmap = np.zeros(256, np.float32)
    nmap[1] = np.float32(1.0 + 2.0 ** -12)
    nabs = np.array([1.0 + 2.0 ** -12], np.float32)
    off = np.float32(-1.0)
    got = oracle.nf4_fold_absmax(np.array([1], np.uint8), nmap, nabs, 256, off)
    p = np.float32(nmap[1]) * np.float32(nabs[0])  # 1 + 2^-11 (the 2^-24 term rounds away)
    assert p == np.float32(1.0 + 2.0 ** -11)
    assert got[0] == np.float32(2.0 ** -11)


def test_oracle_gemv_against_float64():
    n, k, bs = 64, 512, 64
    packed, absmax, qmap = rand_case(3, n * k, bs, signed_zero=False)
    x = np.random.default_rng(4).standard_normal(k).astype(np.float32)
    y = oracle.nf4_gemv(packed, absmax, qmap, x, n, k, bs)
    w = oracle.f16_bits_to_f32(closed_form(packed, absmax, qmap, n * k, bs)).astype(np.float64).reshape(n, k)
    ref = w @ x.astype(np.float64)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6


# ------------------------------------------------------------ host loader

def test_host_fold_matches_oracle():
    w = np.random.default_rng(1).standard_normal((96, 256)).astype(np.float32)
    fam = nf4.quantize(w, blocksize=64, double_quant=True, nested_blocksize=128, name="m.w")
    st = nf4.parse_state(fam, "m.w")
    got = nf4.fold_absmax(fam, "m.w", st, 96 * 256 // 64)
    want = oracle.nf4_fold_absmax(fam["m.w.absmax"], fam["m.w.nested_quant_map"], fam["m.w.nested_absmax"],
                                  st.nested_blocksize, st.nested_offset)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("double_quant", [False, True])
def test_quantize_load_round_trip(double_quant):
    rows, cols, bs = 64, 512, 64
    w = np.random.default_rng(2).standard_normal((rows, cols)).astype(np.float32)
    fam = nf4.quantize(w, blocksize=bs, double_quant=double_quant, name="w")
    h = nf4.load_bnb4(fam, "w")
    assert (h.rows, h.cols, h.blocksize) == (rows, cols, bs)
    assert h.device_bytes() == rows * cols // 2 + rows * cols // bs * 4 + 64
    deq = oracle.f16_bits_to_f32(oracle.nf4_dequant(h.packed, h.absmax, h.qmap, rows * cols, bs))
    # adjacent NF4 codes are at most 0.304 apart (-1 .. -0.696): error <= 0.153 of the block absmax
    amax = np.abs(w.reshape(-1, bs)).max(axis=1)
    err = np.abs(deq - w.reshape(-1)).reshape(-1, bs).max(axis=1)
    assert np.all(err <= 0.153 * amax + (0.05 * amax if double_quant else 1e-3 * amax))


def test_safetensors_round_trip(tmp_path):
    from safetensors.numpy import save_file

    w = np.random.default_rng(5).standard_normal((32, 128)).astype(np.float32)
    fam = nf4.quantize(w, blocksize=64, double_quant=True, name="layer.0.q_proj.weight")
    fam["other.bias"] = np.ones(4, np.float32)
    path = str(tmp_path / "m.safetensors")
    save_file(fam, path)
    t = nf4.read_safetensors(path)
    assert nf4.state_name(t, "layer.0.q_proj.weight").endswith("bitsandbytes__nf4")
    assert nf4.state_name(t, "other.bias") is None
    assert sorted(n for n in t if nf4.is_aux(n)) == sorted(n for n in fam if n != "layer.0.q_proj.weight"
                                                         and n != "other.bias")
    a, b = nf4.load_bnb4(t, "layer.0.q_proj.weight"), nf4.load_bnb4(fam, "layer.0.q_proj.weight")
    np.testing.assert_array_equal(a.packed, b.packed)
    np.testing.assert_array_equal(a.absmax, b.absmax)


def _family(**state):
    st = {"quant_type": "nf4", "blocksize": 64, "shape": [4, 64]}
    st.update(state)
    return {"w": np.zeros((128, 1), np.uint8), "w.absmax": np.ones(4, np.float32),
            "w.quant_map": nf4.NF4_CODE.copy(),
            "w.quant_state.bitsandbytes__nf4": np.frombuffer(json.dumps(st).encode(), np.uint8)}


@pytest.mark.parametrize("mutate, msg", [
    (lambda f: f.pop("w.quant_state.bitsandbytes__nf4"), "no bitsandbytes quant_state"),
    (lambda f: f.update({"w.quant_state.bitsandbytes__nf4": np.frombuffer(b"{oops", np.uint8)}), "not valid JSON"),
    (lambda f: f.update({"w.quant_state.bitsandbytes__nf4": np.frombuffer(b"\xff\xfe", np.uint8)}), "UTF-8"),
    (lambda f: f.update(_family(shape=[256])), "only 2-D"),
    (lambda f: f.update(_family(blocksize=48)), "not divisible by blocksize"),
    (lambda f: f.update({"w": np.zeros(100, np.uint8)}), "packed payload"),
    (lambda f: f.update({"w": np.zeros(64, np.uint16)}), "packed payload"),
    (lambda f: f.pop("w.absmax"), "missing .absmax"),
    (lambda f: f.update({"w.absmax": np.ones(5, np.float32)}), "absmax has 5 entries"),
    (lambda f: f.update({"w.absmax": np.ones(4, np.float16)}), "expected U8"),
    (lambda f: f.update({"w.absmax": np.ones(4, np.uint8)}), "nested_quant_map is missing"),
    (lambda f: f.update({"w.absmax": np.ones(4, np.uint8), "w.nested_quant_map": np.ones(256, np.float32)}),
     "nested_absmax is missing"),
    (lambda f: f.update({"w.absmax": np.ones(4, np.uint8), "w.nested_quant_map": np.ones(256, np.float32),
                         "w.nested_absmax": np.ones(0, np.float32)}), "nested_absmax too short"),
    (lambda f: f.pop("w.quant_map"), "missing .quant_map"),
    (lambda f: f.update({"w.quant_map": np.ones(15, np.float32)}), "15 entries"),
])
def test_load_rejects(mutate, msg):
    f = _family()
    mutate(f)
    with pytest.raises(EngineError, match=msg):
        nf4.load_bnb4(f, "w")


def test_state_defaults():
    f = _family()
    f["w.quant_state.bitsandbytes__nf4"] = np.frombuffer(json.dumps({"shape": [2, 64]}).encode(), np.uint8)
    st = nf4.parse_state(f, "w")
    assert (st.blocksize, st.nested_blocksize, st.nested_offset) == (64, 256, 0.0)
