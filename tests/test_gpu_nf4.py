"""GPU parity of the bitsandbytes 4-bit path, through the C ABI.

Bars: dequantisation bit-exact in f16 bits against the oracle's
dequant_host restatement (src/quant.rs:401-437); the GEMV within 1e-3
normwise relative error of the reference CPU path (f16 dequant + fp32 dot),
and within 5e-4 (f32 y) / 8e-4 (f16 y, whose rounding adds up to 2^-11 per
element) of the exact float64 product of the same weights: the fast kernel
rounds each code to f16 (relative error <= 2^-11 per weight) where the
reference path rounds each decoded weight.
"""
import numpy as np
import pytest

import oracle
from cima_amd import nf4
from cima_amd.hip import EngineError, E_INVALID

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def dev(a: np.ndarray):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host_u16(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def case(seed, n, bs, code=None, double_quant=False):
    """A random packed weight family folded by the host loader."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
    qmap = nf4.NF4_CODE.copy() if code is None else code
    if double_quant:
        fam = {"w": packed, "w.quant_map": qmap,
               "w.absmax": rng.integers(0, 256, n // bs, dtype=np.uint8),
               "w.nested_absmax": (rng.random((n // bs + 255) // 256) + 0.5).astype(np.float32),
               "w.nested_quant_map": np.linspace(-1, 1, 256, dtype=np.float32),
               "w.quant_state.bitsandbytes__nf4": np.frombuffer(
                   f'{{"blocksize": {bs}, "shape": [1, {n}], "nested_offset": 1.25}}'.encode(), np.uint8)}
        h = nf4.load_bnb4(fam, "w")
        return h.packed, h.absmax, h.qmap
    absmax = (rng.random(n // bs) * 2 + 0.01).astype(np.float32)
    return packed, absmax, qmap


RANDOM_CODE = np.random.default_rng(99).standard_normal(16).astype(np.float32)
RANDOM_CODE[5] = -0.0


@pytest.mark.parametrize("n, bs", [(1 << 22, 64), (1 << 20, 32), (1 << 20, 4096), (96 * 1024, 128),
                                   (3 * 1024, 48), (1000, 20), (2, 2), (1 << 20, 2)])
@pytest.mark.parametrize("code", ["nf4", "random"])
def test_dequant_bitexact(hip, n, bs, code):
    packed, absmax, qmap = case(n + bs, n, bs, None if code == "nf4" else RANDOM_CODE)
    if code == "random":
        absmax[::7] *= -1  # negative scales: signs of zero and of every product
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    hip.nf4_dequant(dev(packed), dev(absmax), dev(qmap), out, n, bs)
    np.testing.assert_array_equal(host_u16(out), oracle.nf4_dequant(packed, absmax, qmap, n, bs))


def test_dequant_double_quantised_family(hip):
    n, bs = 1 << 20, 64
    packed, absmax, qmap = case(11, n, bs, double_quant=True)
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    hip.nf4_dequant(dev(packed), dev(absmax), dev(qmap), out, n, bs)
    np.testing.assert_array_equal(host_u16(out), oracle.nf4_dequant(packed, absmax, qmap, n, bs))


def test_dequant_overflow_and_subnormals(hip):
    n, bs = 4096, 32
    packed = np.arange(n // 2, dtype=np.int64).astype(np.uint8)
    qmap = np.array([2.0 ** -k for k in range(16)], np.float32)
    absmax = np.array([70000.0 if i % 3 == 0 else 2.0 ** -12 for i in range(n // bs)], np.float32)
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    hip.nf4_dequant(dev(packed), dev(absmax), dev(qmap), out, n, bs)
    np.testing.assert_array_equal(host_u16(out), oracle.nf4_dequant(packed, absmax, qmap, n, bs))


# ------------------------------------------------------------------- GEMV

SHAPES = [(4096, 4096, 64), (14336, 4096, 64), (4096, 14336, 64), (1000, 4096, 64), (7, 2048, 64),
          (4096, 4096, 32), (512, 4096, 256), (256, 4096, 4096), (300, 96, 32), (64, 8192, 128)]


@pytest.mark.parametrize("n, k, bs", SHAPES, ids=[f"{n}x{k}_bs{b}" for n, k, b in SHAPES])
@pytest.mark.parametrize("act", ["f16", "f32"])
def test_gemv_parity(hip, n, k, bs, act):
    packed, absmax, qmap = case(n * 7 + k + bs, n * k, bs)
    x = np.random.default_rng(n + k).standard_normal(k).astype(np.float32)
    xh = x.astype(np.float16)
    y = torch.empty(n, dtype=torch.float16 if act == "f16" else torch.float32, device="cuda")
    xd = dev(xh) if act == "f16" else dev(x)
    hip.nf4_gemv(xd, dev(packed), dev(absmax), dev(qmap), y, n, k, bs)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    x_eff = xh.astype(np.float32)  # the kernel's activations are f16 in both modes
    want = oracle.nf4_gemv(packed, absmax, qmap, x_eff, n, k, bs, threads=8)
    assert rel(got, want) < 1e-3, rel(got, want)
    w64 = oracle.f16_bits_to_f32(oracle.nf4_dequant(packed, absmax, qmap, n * k, bs)).astype(np.float64)
    exact = w64.reshape(n, k) @ x_eff.astype(np.float64)
    assert rel(got, exact) < (8e-4 if act == "f16" else 5e-4), rel(got, exact)


@pytest.mark.parametrize("kernel", [1, 2], ids=["pair_table", "reg_codebook"])
@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("n, k", [(999, 4096), (333, 14336), (64, 96)])
def test_gemv_every_kernel_and_row_grouping(hip, kernel, rows, n, k):
    bs = 32
    packed, absmax, qmap = case(5 + n, n * k, bs, RANDOM_CODE)
    absmax[::5] *= -1
    x = np.random.default_rng(6).standard_normal(k).astype(np.float16)
    y = torch.empty(n, dtype=torch.float16, device="cuda")
    try:
        hip.set_nf4_tuning(rows, kernel)
        hip.nf4_gemv(dev(x), dev(packed), dev(absmax), dev(qmap), y, n, k, bs)
        torch.cuda.synchronize()
    finally:
        hip.set_nf4_tuning(0, 0)
    want = oracle.nf4_gemv(packed, absmax, qmap, x.astype(np.float32), n, k, bs, threads=8)
    assert rel(y.float().cpu().numpy(), want) < 1e-3


def test_gemv_general_shapes(hip):
    # k not a multiple of 32 and a blocksize that is not a power of two: the general kernel, which decodes
    # each weight exactly like the dequantiser
    for n, k, bs in ((33, 100, 50), (17, 62, 2), (5, 1000, 40)):
        packed, absmax, qmap = case(n + k, n * k, bs, RANDOM_CODE)
        x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        hip.nf4_gemv(dev(x), dev(packed), dev(absmax), dev(qmap), y, n, k, bs)
        torch.cuda.synchronize()
        want = oracle.nf4_gemv(packed, absmax, qmap, x.astype(np.float16).astype(np.float32), n, k, bs)
        assert rel(y.cpu().numpy(), want) < 1e-5


def test_gemv_double_quantised_from_safetensors(hip, tmp_path):
    from safetensors.numpy import save_file

    n, k, bs = 2048, 4096, 64
    w = np.random.default_rng(3).standard_normal((n, k)).astype(np.float32) * 0.02
    fam = nf4.quantize(w, blocksize=bs, double_quant=True, name="model.layers.0.mlp.up_proj.weight")
    path = str(tmp_path / "w.safetensors")
    save_file(fam, path)
    h = nf4.load_bnb4(nf4.read_safetensors(path), "model.layers.0.mlp.up_proj.weight")
    wt = nf4.Nf4Weight(h)
    x = torch.randn(k, device="cuda", dtype=torch.float16)
    y = torch.empty(n, device="cuda", dtype=torch.float16)
    wt.gemm(hip, x.reshape(1, k), y.reshape(1, n))
    torch.cuda.synchronize()
    want = oracle.nf4_gemv(h.packed, h.absmax, h.qmap, x.float().cpu().numpy(), n, k, bs, threads=8)
    assert rel(y.float().cpu().numpy(), want) < 1e-3
    # prefill: the MFMA prefill tiles (the scratch slab is checked, not used)
    m = 5
    xs = torch.randn(m, k, device="cuda", dtype=torch.float16)
    ys = torch.empty(m, n, device="cuda", dtype=torch.float16)
    scratch = torch.empty(hip.nf4_slab_bytes(m, n, k, x_f16=True), device="cuda", dtype=torch.uint8)
    wt.gemm(hip, xs, ys, scratch)
    torch.cuda.synchronize()
    w16 = oracle.f16_bits_to_f32(oracle.nf4_dequant(h.packed, h.absmax, h.qmap, n * k, bs)).reshape(n, k)
    want = xs.float().cpu().numpy() @ w16.T
    assert rel(ys.float().cpu().numpy(), want) < 1e-3
    with pytest.raises(EngineError, match="scratch"):
        wt.gemm(hip, xs, ys)
    with pytest.raises(EngineError, match="GEMM expects"):
        wt.gemm(hip, xs[:, :64], ys)


def test_argument_errors(hip):
    x = torch.zeros(64, dtype=torch.float16, device="cuda")
    p = torch.zeros(64 * 32, dtype=torch.uint8, device="cuda")
    a = torch.ones(64, dtype=torch.float32, device="cuda")
    q = torch.zeros(16, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, dtype=torch.float16, device="cuda")
    for args in ((x, p, a, q, y, 64, 0, 64), (x, p, a, q, y, 64, 64, 0), (x, p, a, q, y, -1, 64, 64)):
        with pytest.raises(EngineError) as e:
            hip.nf4_gemv(*args)
        assert e.value.code == E_INVALID
    with pytest.raises(EngineError):
        hip.nf4_gemv(x, p, a, q, y, 64, 64, 64, act_dtype=2)
    with pytest.raises(EngineError):
        hip.nf4_dequant(p, a, q, y, 64, 0)
    with pytest.raises(EngineError):
        hip.set_nf4_tuning(3, 0)
    with pytest.raises(EngineError):
        hip.set_nf4_tuning(0, 3)
    hip.nf4_gemv(x, p, a, q, y, 0, 64, 64)  # n == 0: nothing to do
    hip.nf4_dequant(p, a, q, y, 0, 64)


@pytest.mark.parametrize("kernel", [1, 2], ids=["pair_table", "reg_codebook"])
@pytest.mark.parametrize("rows", [1, 4])
def test_gemv_many_rows_per_wave(hip, rows, kernel):
    # a small grid cap would leave each wave more than the 64 rows it can hold: the host widens the grid
    n, k, bs = 70001, 256, 64
    packed, absmax, qmap = case(8, n * k, bs)
    x = np.random.default_rng(9).standard_normal(k).astype(np.float16)
    y = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    try:
        hip.set_nf4_tuning(rows, kernel)
        hip.set_gemv_grid(1)
        hip.nf4_gemv(dev(x), dev(packed), dev(absmax), dev(qmap), y, n, k, bs)
        torch.cuda.synchronize()
    finally:
        hip.set_nf4_tuning(0, 0)
        hip.set_gemv_grid(0)
    got = y.float().cpu().numpy()
    assert not np.isnan(got).any()
    want = oracle.nf4_gemv(packed, absmax, qmap, x.astype(np.float32), n, k, bs, threads=8)
    assert rel(got, want) < 1e-3


TDT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


@pytest.mark.parametrize("m, n, k, bs", [(2, 256, 512, 64), (17, 320, 1024, 128), (300, 512, 2048, 64),
                                         (40, 200, 4096, 4096), (5, 96, 640, 96), (33, 192, 384, 48),
                                         (9, 130, 200, 20)])
def test_gemm_slab_parity(hip, m, n, k, bs):
    """cima_hip_nf4_gemm_slab (WTensor::gemm's Nf4 arm, src/quant.rs:131-162)
    against the CPU path: the oracle's bit-exact f16 W times the f16-rounded X
    in float64; 1e-5 with fp32 Y (only the summation order differs), the
    north star's 1e-3 with f16 Y.  The first five shapes take the fused
    route (the tiles decode W; blocksize 96 is not a power of two), the
    sixth the slab route's f16-weight tiles (blocksize 48 splits 32-element
    runs), the last the slab route's plain kernel (k % 64 != 0)."""
    packed, absmax, qmap = case(700 + m, n * k, bs, code=RANDOM_CODE)
    w16 = oracle.f16_bits_to_f32(oracle.nf4_dequant(packed, absmax, qmap, n * k, bs)).reshape(n, k)
    xf = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    p, a, q = dev(packed), dev(absmax), dev(qmap)
    for xd, yd in ((2, 0), (1, 1), (0, 0)):
        x = torch.from_numpy(xf).to(TDT[xd]).cuda()
        y = torch.full((m, n), 3.0, dtype=TDT[yd], device="cuda")
        slab = torch.empty(hip.nf4_slab_bytes(m, n, k, x_f16=xd == 1), dtype=torch.uint8, device="cuda")
        hip.nf4_gemm_slab(x, p, a, q, y, m, n, k, bs, slab)
        torch.cuda.synchronize()
        xh = x.float().cpu().numpy().astype(np.float16).astype(np.float64)
        r = rel(y.float().cpu().numpy(), xh @ w16.astype(np.float64).T)
        assert r <= (1e-5 if yd == 0 else 1e-3), (xd, yd, r)


def test_gemm_slab_argument_errors(hip):
    m, n, k, bs = 4, 64, 256, 64
    packed, absmax, qmap = case(5, n * k, bs)
    p, a, q = dev(packed), dev(absmax), dev(qmap)
    x = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    y = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    slab = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    hip.nf4_gemm_slab(x, p, a, q, y, 0, n, k, bs, slab)  # m = 0: no-op
    for bad in (dict(slab_bytes=256), dict(k=100)):  # 256 B: not one 256-element f16 row
        kk = bad.get("k", k)
        with pytest.raises(EngineError) as e:
            hip.nf4_gemm_slab(x, p, a, q, y, m, n, kk, bs, slab, slab_bytes=bad.get("slab_bytes"))
        assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.nf4_gemm_slab(x, p, a, q, y, m, n, k, bs, slab[64:])
    assert e.value.code == E_INVALID


def test_gemm_slab_row_slices(hip):
    """The slab route with a slab far smaller than the f16 weight: W is
    decoded and multiplied a row slice at a time, each slice writing its
    columns of Y; the result equals the one-slice run bit for bit (same
    kernels, same per-row summation) and the CPU path to 1e-5.  Blocksizes
    that do not divide k make the slices start on absmax block boundaries;
    one slab holds exactly one slice."""
    for n, k, bs, m, slab_bytes in ((600, 192, 48, 5, 100 << 10), (300, 200, 20, 7, 40 << 10),
                                    (96, 320, 80, 3, 2 * 320 * 4)):
        packed, absmax, qmap = case(900 + n, n * k, bs, code=RANDOM_CODE)
        p, a, q = dev(packed), dev(absmax), dev(qmap)
        x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        small = torch.empty(slab_bytes, dtype=torch.uint8, device="cuda")
        big = torch.empty(hip.nf4_slab_bytes(m, n, k), dtype=torch.uint8, device="cuda")
        ys = torch.empty((m, n), device="cuda")
        yb = torch.empty((m, n), device="cuda")
        hip.nf4_gemm_slab(x, p, a, q, ys, m, n, k, bs, small)
        hip.nf4_gemm_slab(x, p, a, q, yb, m, n, k, bs, big)
        torch.cuda.synchronize()
        assert np.array_equal(ys.cpu().numpy(), yb.cpu().numpy()), (n, k)
        w16 = oracle.f16_bits_to_f32(oracle.nf4_dequant(packed, absmax, qmap, n * k, bs)).reshape(n, k)
        xh = x.float().cpu().numpy().astype(np.float16).astype(np.float64)
        assert rel(ys.cpu().numpy(), xh @ w16.astype(np.float64).T) <= 1e-5, (n, k)


@pytest.mark.parametrize("m", [16, 128, 512])
def test_gemm_fused_full_shape(hip, m):
    """The fused NF4 prefill at the Llama-3-8B gate/up shape (14336 x 4096,
    blocksize 64), every output row, against the oracle's bit-exact f16 W
    times the f16-rounded bf16 X in float64 (1e-5, fp32 Y); the caller's
    slab is left as it was."""
    n, k, bs = 14336, 4096, 64
    packed, absmax, qmap = case(77, n * k, bs)
    w16 = oracle.f16_bits_to_f32(oracle.nf4_dequant(packed, absmax, qmap, n * k, bs)).reshape(n, k)
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    y = torch.full((m, n), float("nan"), device="cuda")
    slab = torch.full((1 << 20,), 0x5A, dtype=torch.uint8, device="cuda")
    hip.nf4_gemm_slab(x, dev(packed), dev(absmax), dev(qmap), y, m, n, k, bs, slab)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert not np.isnan(got).any()
    xh = x.float().cpu().numpy().astype(np.float16).astype(np.float64)
    want = xh @ w16.astype(np.float64).T
    assert rel(got, want) <= 1e-5
    assert bool((slab == 0x5A).all())
