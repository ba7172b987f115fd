"""GPU parity of the prefill dequant-GEMM (MFMA) against the reference CPU
path: decode W to f16 (bit-exact decoders), then an fp32 GEMM
(src/models/transformer.rs:618-655 does the same on the GPU with an f16
slab).  The kernel multiplies the same f16 weights with fp32 accumulation,
so the bar is far inside the north star's 1e-3: normwise 1e-5 when x is
exactly representable in f16 (f16 / bf16 inputs), 1e-3 when fp32 x is
rounded to f16."""
import numpy as np
import pytest

import oracle
import make_golden as mg
from cima_amd import gguf, synth
from cima_amd.hip import EngineError, E_INVALID

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 2, 3, 6, 7, 8, 12, 13, 14, 23
FORMATS = [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K, IQ4_XS]
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q4_K: "q4_k", Q5_K: "q5_k",
         Q6_K: "q6_k", IQ4_XS: "iq4_xs"}
TDT = {gguf.DT_F32: torch.float32, gguf.DT_F16: torch.float16, gguf.DT_BF16: torch.bfloat16}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def run(hip, t, w, xf, m, n, k, xd, yd, ldy=None):
    ldy = n if ldy is None else ldy
    x = torch.from_numpy(xf).to(TDT[xd]).cuda()
    xh = x.float().cpu().numpy()  # the exact x the kernel receives
    y = torch.full((m, ldy), 3.0, dtype=TDT[yd], device="cuda")
    hip.gguf_gemm(t, x, torch.from_numpy(w).cuda(), y, m, n, k, ldy, xd, yd)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), xh


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
@pytest.mark.parametrize("m", [1, 7, 16, 33, 64, 129])
def test_gemm_small_shapes(hip, t, m):
    n, k = 200, 512
    w = synth.weights(t, 50 + t, 0.02, n, k)
    xf = synth.normal(51 + m, 1.0, m * k).reshape(m, k)
    w16 = oracle.dequant(t, w, n * k)
    for xd, yd in ((gguf.DT_BF16, gguf.DT_F32), (gguf.DT_F16, gguf.DT_F16), (gguf.DT_F32, gguf.DT_F32)):
        y, xh = run(hip, t, w, xf, m, n, k, xd, yd, ldy=n + 8)
        want = oracle.gemm(xh, w16, m, n, k)
        tol = 1e-5 if (xd != gguf.DT_F32 and yd == gguf.DT_F32) else 1e-3
        r = rel(y[:, :n], want)
        assert r <= tol, (xd, yd, r)
        assert np.all(y[:, n:] == 3.0), "wrote past n into the ldy padding"


@pytest.mark.parametrize("m", [16, 128, 512])
def test_gemm_config4_full_shape(hip, m):
    """Benchmark config 4: Q4_K W 14336x4096 x X (m tokens, bf16), Y fp32,
    every output row against the CPU path (the oracle's bit-exact f16 decode
    of all of W, then the product in float64), so a wrong tile anywhere in
    the row range fails; also per 128-row block, so one bad tile cannot hide
    in the norm of the whole."""
    n, k = 14336, 4096
    w = synth.weights(Q4_K, 60, 0.02, n, k)
    xf = synth.normal(61, 1.0, m * k).reshape(m, k)
    y, xh = run(hip, Q4_K, w, xf, m, n, k, gguf.DT_BF16, gguf.DT_F32)
    assert gguf.row_bytes(Q4_K, k) == w.shape[1]
    w16 = oracle.f16_bits_to_f32(oracle.dequant(Q4_K, w.reshape(-1), n * k)).reshape(n, k)
    want = xh.astype(np.float64) @ w16.astype(np.float64).T
    r = rel(y, want)
    print(f"config 4 m={m}: rel err vs CPU path {r:.2e} over all {n} rows")
    assert r <= 1e-5
    for r0 in range(0, n, 128):
        rb = rel(y[:, r0:r0 + 128], want[:, r0:r0 + 128])
        assert rb <= 1e-5, (r0, rb)


def test_gemm_tile_variants_agree(hip):
    """Every token-tile width gives the same product (exact f16 inputs),
    with one partial tile (40 tokens) and ragged ones (300 tokens)."""
    n, k = 300, 1024
    w = synth.weights(Q4_K, 70, 0.02, n, k)
    w16 = oracle.dequant(Q4_K, w, n * k)
    lib = hip.lib
    for m in (40, 300):
        xf = synth.normal(71 + m, 1.0, m * k).reshape(m, k)
        x = torch.from_numpy(xf).to(torch.float16).cuda()
        want = oracle.gemm(x.float().cpu().numpy(), w16, m, n, k)
        for bn in (16, 32, 64, 128, 256):
            rc = lib.cima_hip_set_gemm_tile(hip.handle, bn)
            assert rc == 0
            y = torch.empty((m, n), device="cuda")
            hip.gguf_gemm(Q4_K, x, torch.from_numpy(w).cuda(), y, m, n, k)
            torch.cuda.synchronize()
            assert rel(y.cpu().numpy(), want) <= 1e-5, (m, bn)
    lib.cima_hip_set_gemm_tile(hip.handle, 0)


def test_gemm_argument_errors(hip):
    x = torch.zeros((4, 256), device="cuda")
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    y = torch.zeros((4, 4), device="cuda")
    hip.gguf_gemm(Q4_K, x, w, y, 0, 4, 256)  # m = 0: no-op
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm(Q4_K, x, w, y, 4, 4, 100)
    assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm(Q4_K, x, w, y, 4, 4, 256, ldy=3)
    assert e.value.code == E_INVALID
    xs = torch.zeros(4 * 256 + 2, device="cuda")[2:].view(4, 256)  # 8-byte aligned only
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm(Q4_K, xs, w, y, 4, 4, 256)
    assert e.value.code == E_INVALID


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
@pytest.mark.parametrize("bn", [16, 32, 64, 128, 256])
def test_gemm_dequantises_bit_exactly(hip, t, bn):
    """With X the identity, Y = dequant(W)^T: every f16 weight the kernel
    multiplies, read back exactly (an f16 times 1.0, summed with exact
    zeros in fp32), must equal the host decoder's f16 bits -- random block
    bytes (scales of every exponent, NaN-free) through each token tile."""
    k = 256
    n = 96
    nbytes = n * k // oracle.BLOCK_ELEMS[t] * oracle.BLOCK_BYTES[t]
    raw = mg.xorshift_bytes(nbytes, seed=0x9E3779B97F4A7C15 + bn)
    # half the rows with raw random scale fields, half with the scales
    # pinned near 1 (the selftest's choice) so that no row overflows
    w = np.concatenate([raw[:nbytes // 2], mg.sane_scales(t, raw[nbytes // 2:])]).reshape(n, -1)
    want = oracle.f16_bits_to_f32(oracle.dequant(t, w.reshape(-1), n * k)).reshape(n, k)
    ok = np.isfinite(want).all(axis=1)
    x = np.eye(k, dtype=np.float32)
    hip.set_gemm_tile(bn)
    try:
        y, _ = run(hip, t, w, x, k, n, k, gguf.DT_F16, gguf.DT_F32)
    finally:
        hip.set_gemm_tile(0)
    got = y.T  # [n, k]
    assert np.array_equal(got[ok], want[ok]), (int(ok.sum()), np.argwhere(got[ok] != want[ok])[:4])


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
@pytest.mark.parametrize("n,m", [(8192, 13), (8191, 13), (1000, 13), (4000, 32), (1000, 32), (3000, 17)])
def test_gemm_16_token_tiles_wide_and_narrow(hip, t, n, m):
    """Up to 32 tokens the grid picks the split-k tile: 32 rows per
    workgroup where that grid (rows / 32 x tokens / 16) fills more than
    half the CUs (8192 rows at 13 tokens, 4000 or 3000 rows at 17-32),
    16 rows (the _b16n_ kernels) otherwise; both against the CPU path,
    ragged row and token counts included."""
    k = 256
    w = synth.weights(t, 140 + t, 0.02, n, k)
    xf = synth.normal(141, 1.0, m * k).reshape(m, k)
    w16 = oracle.dequant(t, w, n * k)
    for xd, yd in ((gguf.DT_BF16, gguf.DT_F32), (gguf.DT_F32, gguf.DT_F16)):
        y, xh = run(hip, t, w, xf, m, n, k, xd, yd, ldy=n + 4)
        want = oracle.gemm(xh, w16, m, n, k)
        tol = 1e-5 if xd != gguf.DT_F32 and yd == gguf.DT_F32 else 1e-3
        assert rel(y[:, :n], want) <= tol, (xd, yd)
        assert np.all(y[:, n:] == 3.0)


@pytest.mark.parametrize("n,k,m", [(1024, 4096, 512), (4096, 4096, 256)], ids=["1024x4096_m512", "4096x4096_m256"])
def test_gemm_narrow_weight_many_tokens(hip, n, k, m):
    """Weights too narrow for the 128-token grid to fill the CUs run the
    register-A tiles (32 or 64 tokens) past 128 tokens; the default route at
    those shapes against the reference CPU path, bf16 X, fp32 Y."""
    w = synth.weights(Q4_K, 90, 0.02, n, k)
    xf = synth.normal(91, 1.0, m * k).reshape(m, k)
    y, xh = run(hip, Q4_K, w, xf, m, n, k, gguf.DT_BF16, gguf.DT_F32)
    want = oracle.gemm(xh, oracle.dequant(Q4_K, w, n * k), m, n, k)
    assert rel(y, want) <= 1e-5


@pytest.mark.parametrize("m", [16, 64, 256], ids=["sk16", "reg_a", "lds_pipe"])
def test_gemm_x_range_flags(hip, m):
    """bf16 X beyond f16's range, or too small for it, no longer turns into
    inf / zero silently: the tiles flag it (cima_hip_gemm_status) on every
    tile kind, for the GGUF and the bitsandbytes weights; in-range bf16 and
    any f16 X leave the word clear; f32 X flags only overflow."""
    n, k = 256, 1024
    w = torch.from_numpy(synth.weights(Q4_K, 70, 0.02, n, k)).cuda()
    y = torch.empty((m, n), device="cuda")
    hip.gemm_status(clear=True)

    def flags(x, xd):
        hip.gguf_gemm(Q4_K, x, w, y, m, n, k, n, xd, gguf.DT_F32)
        return hip.gemm_status(clear=True)

    base = torch.randn(m, k)
    base[base.abs() < 1e-3] = 1e-3  # normal draws can land below 2^-17 themselves
    assert flags(base.to(torch.bfloat16).cuda(), gguf.DT_BF16) == 0
    assert flags(base.to(torch.float16).cuda(), gguf.DT_F16) == 0
    assert flags(base.cuda(), gguf.DT_F32) == 0
    big = base.clone()
    big[m // 2, 777] = 70000.0
    assert flags(big.to(torch.bfloat16).cuda(), gguf.DT_BF16) == 1
    assert torch.isinf(y[m // 2]).any(), "the overflowing value reached the product as inf"
    assert flags(big.cuda(), gguf.DT_F32) == 1
    tiny = base.clone()
    tiny[m - 1, 5] = 3e-7  # below 2^-17, nonzero
    assert flags(tiny.to(torch.bfloat16).cuda(), gguf.DT_BF16) == 2
    assert flags(tiny.cuda(), gguf.DT_F32) == 0
    edge = base.clone()
    edge[0, 0], edge[0, 1] = 65280.0, 2.0 ** -17  # the exact extremes
    assert flags(edge.to(torch.bfloat16).cuda(), gguf.DT_BF16) == 0
    # the bitsandbytes tiles report through the same word
    from cima_amd import nf4
    packed = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8).cuda()
    absmax = torch.rand(n * k // 64).cuda() + 0.1
    qmap = torch.from_numpy(nf4.NF4_CODE.copy()).cuda()
    slab = torch.empty(2 * n * k, dtype=torch.uint8, device="cuda")
    hip.nf4_gemm_slab(big.to(torch.bfloat16).cuda(), packed, absmax, qmap, y, m, n, k, 64, slab)
    assert hip.gemm_status(clear=True) == 1
