"""GPU parity: the HIP kernels, called through the C ABI, against the oracle.

Bars (the north star's): dequantisation and gather bit-exact in f16 bits
(NaN equal as a class, as src/selftest.rs:970-975 does); GEMV within 1e-3
normwise relative error of the reference CPU path (f16 dequant + fp32 dot),
plus the selftest's per-row noise bound (src/selftest.rs:1104-1121) without
its q8_1 term (the kernels stage x as 16-bit fixed point, not 8-bit), plus a
tight bound against the exact float64 product of the undecoded-to-f16
weights: rel err <= 5e-5, the size of the 16-bit activation rounding.
"""
import numpy as np
import pytest

import oracle
import make_golden as mg
from cima_amd import gguf, synth
from cima_amd.hip import EngineError, E_INVALID, E_FORMAT

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 2, 3, 6, 7, 8, 12, 13, 14, 23
FORMATS = [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K, IQ4_XS]
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q4_K: "q4_k", Q5_K: "q5_k",
         Q6_K: "q6_k", IQ4_XS: "iq4_xs"}
fid = [NAMES[t] for t in FORMATS]


def dev(a: np.ndarray):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host_u16(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def is_nan16(v):
    return ((v & 0x7C00) == 0x7C00) & ((v & 0x3FF) != 0)


def assert_bits(got, want, what):
    bad = (got != want) & ~(is_nan16(got) & is_nan16(want))
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"{what}: {int(bad.sum())} f16 mismatches, first at {i}: "
                             f"want {want[i]:#06x} got {got[i]:#06x}")


def rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def rand_blocks(t, nblocks, seed, sane=False):
    be, bb = mg.BLOCK[t]
    src = np.random.default_rng(seed).integers(0, 256, nblocks * bb, dtype=np.uint8)
    return mg.sane_scales(t, src) if sane else src


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_dequant_bitexact_random_blocks(hip, t):
    be, bb = mg.BLOCK[t]
    nblocks = (4 << 20) // bb
    src = rand_blocks(t, nblocks, seed=0x9E37 + t)
    out = torch.empty(nblocks * be, dtype=torch.float16, device="cuda")
    hip.gguf_dequant(t, dev(src), out, nblocks)
    assert_bits(host_u16(out), oracle.dequant(t, src, nblocks * be), f"{NAMES[t]} dequant")


@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_dequant_golden_fixture(hip, t):
    g = np.load(mg.GOLDEN)
    be, bb = mg.BLOCK[t]
    src = g[f"{NAMES[t]}_blocks"]
    nb = len(src) // bb
    out = torch.empty(nb * be, dtype=torch.float16, device="cuda")
    hip.gguf_dequant(t, dev(src), out, nb)
    assert_bits(host_u16(out), g[f"{NAMES[t]}_f16"], f"{NAMES[t]} golden")


@pytest.mark.parametrize("t", FORMATS, ids=fid)
@pytest.mark.parametrize("nb", [1, 3, 257, 1001])
def test_dequant_ragged_block_counts(hip, t, nb):
    be, bb = mg.BLOCK[t]
    src = rand_blocks(t, nb, seed=nb * 31 + t)
    out = torch.full((nb * be + 64,), 7.0, dtype=torch.float16, device="cuda")
    hip.gguf_dequant(t, dev(src), out, nb)
    got = host_u16(out)
    assert_bits(got[: nb * be], oracle.dequant(t, src, nb * be), f"{NAMES[t]} nb={nb}")
    assert np.all(got[nb * be:] == np.float16(7.0).view(np.uint16))  # nothing written past the end


def test_dequant_zero_blocks_is_noop(hip):
    hip.gguf_dequant(Q4_K, 0, 0, 0)


# ------------------------------------------------------------------- gather

@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_gather_bitexact(hip, t):
    """src/selftest.rs:1142-1196: vocab 512, hidden 2048, 96 ids"""
    be, bb = mg.BLOCK[t]
    vocab, hidden, n_ids = 512, 2048, 96
    rb = hidden // be * bb
    table = np.random.default_rng(t).integers(0, 256, vocab * rb, dtype=np.uint8)
    ids = np.random.default_rng(t + 1).integers(0, vocab, n_ids).astype(np.uint32)
    out = torch.empty(n_ids * hidden, dtype=torch.float16, device="cuda")
    hip.gguf_gather(t, dev(table), dev(ids), out, n_ids, hidden)
    want = oracle.gather(t, table, ids, hidden).reshape(-1)
    assert_bits(host_u16(out), want, f"{NAMES[t]} gather")


# --------------------------------------------------------------------- gemv

SELFTEST_SHAPES = [(8192, 4096), (4096, 1536), (512, 1536), (1536, 512), (1536, 4096), (6144, 1536),
                   (1536, 6144)]


def check_rows(y, w16, x, n, k, what):
    """per-row bound of src/selftest.rs:1104-1121 without the q8_1 term"""
    y64, l2 = oracle.gemv_f64(w16, x, n, k)
    unit = l2 * 4.9e-4
    err = np.abs(y.astype(np.float64) - y64)
    worst = float(np.max(err / np.maximum(unit, 1e-12)))
    assert np.all(err <= 4 * unit + 1e-6), f"{what}: worst {worst:.2f} noise units"
    return worst


@pytest.mark.parametrize("t", FORMATS, ids=fid)
@pytest.mark.parametrize("n,k", SELFTEST_SHAPES, ids=[f"{n}x{k}" for n, k in SELFTEST_SHAPES])
def test_gemv_selftest_shapes(hip, t, n, k):
    w = rand_blocks(t, n * k // mg.BLOCK[t][0], seed=n + k + t, sane=True)
    rng = np.random.default_rng(k)
    x = (rng.uniform(-1, 1, k) * (1.0 + (np.arange(k) % 7) * 0.1) * 0.03).astype(np.float32)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, dev(x), dev(w), None, y, n, k, 0)
    yg = host(y)
    w16 = oracle.dequant(t, w, n * k)
    check_rows(yg, w16, x, n, k, f"{NAMES[t]} {n}x{k}")
    assert rel(yg, oracle.gemv(w16, x, n, k)) <= 1e-3


BENCH_SHAPES = [
    (Q8_0, 4864, 896),      # config 1
    (Q4_K, 14336, 4096),    # config 2: gate / up
    (Q4_K, 4096, 14336),    # down
    (Q4_K, 4096, 4096),     # q / o
    (Q4_K, 1024, 4096),     # k / v
    (Q6_K, 128256, 4096),   # config 3: output head
    (Q8_0, 151936, 896),    # config 5: tied Qwen2.5-0.5B head
    (Q8_0, 4096, 4096),
    (Q4_0, 4096, 4096),
    (Q5_K, 14336, 4096),    # the other formats of Q4_K_M / IQ4_XS files
    (IQ4_XS, 4096, 14336),
    (Q5_0, 4864, 896),
    (Q5_1, 896, 4864),
    (Q4_1, 1152, 896),
]


@pytest.mark.parametrize("t,n,k", BENCH_SHAPES, ids=[f"{NAMES[t]}-{n}x{k}" for t, n, k in BENCH_SHAPES])
def test_gemv_baseline_shapes_vs_cpu_path(hip, t, n, k):
    """Seeded N(0,0.02) weights, x ~ N(0,1): rel err <= 1e-3 vs the reference
    CPU path (decode to f16, fp32 dot) at the benchmark's full sizes."""
    w = synth.weights(t, seed=1000 + t, stddev=0.02, rows=n, k=k)
    x = synth.normal(2000 + t, 1.0, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, dev(x), dev(w), None, y, n, k, 0)
    ycpu = oracle.gguf_gemv_packed(t, w, x, n, k, threads=16)
    r = rel(host(y), ycpu)
    print(f"{NAMES[t]} {n}x{k}: rel err vs CPU path {r:.3e}")
    assert r <= 1e-3


@pytest.mark.parametrize("t", FORMATS, ids=fid)
@pytest.mark.parametrize("n,k", [(4096, 4096), (1000, 14336), (333, 1536)], ids=["4096x4096", "1000x14336", "333x1536"])
def test_gemv_tight_vs_exact_weights(hip, t, n, k):
    """Against W (exact decoded values, float64) . x: the only error left is
    the 16-bit fixed-point staging of x and fp32 scaling, ~1e-5."""
    w = synth.weights(t, seed=40 + t, stddev=0.02, rows=n, k=k)
    x = synth.normal(41 + t, 1.0, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, dev(x), dev(w), None, y, n, k, 0)
    W = mg.decode_exact(t, w).reshape(n, k)
    r = rel(host(y), W @ x.astype(np.float64))
    print(f"{NAMES[t]} {n}x{k}: rel err vs exact {r:.2e}")
    assert r <= 5e-5


@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_gemv_modes_bias_residual_pair(hip, t):
    be = mg.BLOCK[t][0]
    n, k = 1000, 4 * 256
    w = synth.weights(t, seed=5 + t, stddev=0.02, rows=2 * n, k=k)
    x = synth.normal(6, 1.0, k)
    bias = synth.normal(7, 0.1, 2 * n)
    y_old = synth.normal(8, 1.0, n)
    w16 = oracle.dequant(t, w, 2 * n * k)
    wd, xd, bd = dev(w), dev(x), dev(bias)
    # mode 0 + bias
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, xd, wd, bd, y, n, k, 0)
    assert rel(host(y), oracle.gemv(w16, x, n, k, 0, bias=bias)) <= 1e-3
    # mode 1: residual accumulate (+bias)
    y = dev(y_old)
    hip.gguf_gemv(t, xd, wd, bd, y, n, k, 1)
    assert rel(host(y), oracle.gemv(w16, x, n, k, 1, bias=bias, y_old=y_old)) <= 1e-3
    # mode 2: [2n, k] gate|up pair, SwiGLU, 2n biases
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, xd, wd, bd, y, n, k, 2)
    assert rel(host(y), oracle.gemv(w16, x, n, k, 2, bias=bias)) <= 1e-3
    # separate gate / up buffers: the fused SwiGLU entry point
    rb = gguf.row_bytes(t, k)
    wg, wu = dev(w[:n]), dev(w[n:])
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv_swiglu(t, xd, wg, wu, dev(bias[:n]), dev(bias[n:]), y, n, k)
    assert rel(host(y), oracle.gemv(w16, x, n, k, 2, bias=bias)) <= 1e-3
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv_swiglu(t, xd, wg, wu, None, None, y, n, k)
    assert rel(host(y), oracle.gemv(w16, x, n, k, 2)) <= 1e-3
    assert w.shape[1] == rb


@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_gemv_f16_activations(hip, t):
    """The engine's drop-in: x, bias, y in f16 (src/cuda.rs:2161)."""
    n, k = 777, 2048
    w = synth.weights(t, seed=9 + t, stddev=0.02, rows=2 * n, k=k)
    x16 = synth.normal(10, 1.0, k).astype(np.float16)
    b16 = synth.normal(11, 0.1, 2 * n).astype(np.float16)
    yo16 = synth.normal(12, 1.0, n).astype(np.float16)
    w16 = oracle.dequant(t, w, 2 * n * k)
    x, b, yo = x16.astype(np.float32), b16.astype(np.float32), yo16.astype(np.float32)
    wd, xd, bd = dev(w), dev(x16), dev(b16)
    for mode in (0, 1, 2):
        y = dev(yo16.copy())
        hip.gguf_gemv(t, xd, wd, bd, y, n, k, mode)
        want = oracle.gemv(w16, x, n, k, mode, bias=b, y_old=yo)
        assert rel(host(y).astype(np.float32), want) <= 1e-3, mode


@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_gemv_every_launch_plan(hip, t):
    """Each (rows, lanes) variant the tuner can pick computes the same GEMV;
    ragged n exercises the tail row groups."""
    n, k = 333, 1536
    w = synth.weights(t, seed=13 + t, stddev=0.02, rows=n, k=k)
    x = synth.normal(14, 1.0, k)
    want = oracle.gguf_gemv_packed(t, w, x, n, k, threads=16)
    wd, xd = dev(w), dev(x)
    ref = None
    try:
        for rows in (1, 2):
            for lpr in (16, 32, 64, 128, 256):
                hip.set_gemv_tuning(rows, lpr)
                y = torch.empty(n, dtype=torch.float32, device="cuda")
                hip.gguf_gemv(t, xd, wd, None, y, n, k, 0)
                yg = host(y)
                assert rel(yg, want) <= 1e-3, (rows, lpr)
                if ref is None:
                    ref = yg
                # same lanes-per-row => same summation order only within a plan;
                # across plans results agree to fp32 rounding
                assert rel(yg, ref) <= 1e-5, (rows, lpr)
    finally:
        hip.set_gemv_tuning(0, 0)


@pytest.mark.parametrize("t", FORMATS, ids=fid)
@pytest.mark.parametrize("n", [1, 2, 7, 65])
def test_gemv_tiny_shapes(hip, t, n):
    k = mg.BLOCK[t][0]  # one block per row
    w = rand_blocks(t, n, seed=n + 100 * t, sane=True)
    x = np.random.default_rng(n).uniform(-0.03, 0.03, k).astype(np.float32)
    y = torch.full((n + 8,), 5.0, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(t, dev(x), dev(w), None, y, n, k, 0)
    yg = host(y)
    check_rows(yg[:n], oracle.dequant(t, w, n * k), x, n, k, f"{NAMES[t]} n={n}")
    assert np.all(yg[n:] == 5.0)


def test_gemv_deterministic(hip):
    n, k = 14336, 4096
    w = dev(synth.weights(Q4_K, seed=21, stddev=0.02, rows=n, k=k))
    x = dev(synth.normal(22, 1.0, k))
    ys = []
    for _ in range(3):
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        hip.gguf_gemv(Q4_K, x, w, None, y, n, k, 0)
        ys.append(host(y))
    assert np.array_equal(ys[0], ys[1]) and np.array_equal(ys[0], ys[2])


@pytest.mark.parametrize("t, n, k", [(Q8_0, 14336, 4096), (Q8_0, 4864, 896), (Q4_K, 4096, 4096),
                                     (Q6_K, 512, 14336), (Q4_0, 300, 2048)],
                         ids=["q8_0-big", "q8_0-896", "q4_k", "q6_k-long", "q4_0"])
@pytest.mark.parametrize("act", [gguf.DT_F16, gguf.DT_F32], ids=["f16", "f32"])
def test_gemv_x_at_element_offset(hip, t, n, k, act):
    """x, bias and y may sit at any element offset, as the reference's
    pointers may (src/cuda.rs:2161): the result equals the aligned call's
    bit for bit, with the residual epilogue, on every main loop the
    heuristic picks for these shapes (the direct-to-LDS one for the large
    Q8_0 matrix)."""
    td = torch.float16 if act == gguf.DT_F16 else torch.float32
    w = dev(synth.weights(t, seed=31, stddev=0.02, rows=n, k=k))
    xv = torch.from_numpy(synth.normal(32, 1.0, k)).to(td).cuda()
    bv = torch.from_numpy(synth.normal(33, 0.1, n)).to(td).cuda()
    y0v = torch.from_numpy(synth.normal(34, 1.0, n)).to(td).cuda()
    ya = y0v.clone()
    hip.gguf_gemv(t, xv, w, bv, ya, n, k, 1, act)
    for off in (1, 3):
        xb = torch.zeros(k + 8, dtype=td, device="cuda")
        bb = torch.zeros(n + 8, dtype=td, device="cuda")
        yb = torch.zeros(n + 8, dtype=td, device="cuda")
        xb[off:off + k] = xv
        bb[off:off + n] = bv
        yb[off:off + n] = y0v
        hip.gguf_gemv(t, xb[off:off + k], w, bb[off:off + n], yb[off:off + n], n, k, 1, act)
        torch.cuda.synchronize()
        assert torch.equal(yb[off:off + n], ya), off
        assert not yb[:off].any() and not yb[off + n:].any()


def test_gemv_argument_errors(hip):
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    y = torch.zeros(4, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(Q4_K, x, w, None, y, 0, 256, 0)  # n = 0: no-op
    for bad in [dict(k=100), dict(k=0), dict(mode=3)]:
        a = dict(k=256, mode=0)
        a.update(bad)
        with pytest.raises(EngineError) as e:
            hip.gguf_gemv(Q4_K, x, w, None, y, 4, a["k"], a["mode"])
        assert e.value.code == E_INVALID and not e.value.fatal
    with pytest.raises(EngineError) as e:
        hip.gguf_gemv(10, x, w, None, y, 4, 256, 0)  # Q2_K: not a format the reference executes
    assert e.value.code == E_FORMAT
    with pytest.raises(EngineError) as e:
        hip.gguf_gemv(Q4_K, x.data_ptr() + 2, w, None, y, 1, 128 * 2, 0)  # f32 x not 4-B aligned
    assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.gguf_gemv(Q4_K, x, w.data_ptr() + 2, None, y, 1, 256, 0)  # Q4_K weights need 16 B
    assert e.value.code == E_INVALID


def test_gemv_graph_replay(hip):
    """Captured into a HIP graph (as the engine's decode step is), every replay
    matches the eager result; eager work runs between the replays."""
    n, k = 4096, 4096
    w = dev(synth.weights(Q4_K, seed=31, stddev=0.02, rows=n, k=k))
    x = dev(synth.normal(32, 1.0, k))
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hip.gguf_gemv(Q4_K, x, w, None, y, n, k, 0)
    eager = host(y).copy()
    g = torch.cuda.CUDAGraph()
    yg = torch.zeros(n, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            hip.set_stream(s.cuda_stream)
            hip.gguf_gemv(Q4_K, x, w, None, yg, n, k, 0)
    hip.use_torch_stream()
    torch.cuda.synchronize()
    for i in range(4):
        yg.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(yg), eager), i
        hip.gguf_gemv(Q4_K, x, w, None, y, n, k, 0)  # eager work between replays
        torch.cuda.synchronize()


def test_launches_order_with_torch_default_stream(hip):
    """On torch's default stream the library's kernels are ordered with
    torch's own: a dependent GEMV pair behind a torch fill of the
    intermediate never sees the fill (the null stream handle is the null
    stream, not the context's unsynchronised own stream)."""
    t = 12
    w1 = torch.from_numpy(synth.weights(t, 1, 0.02, 2048, 1024)).cuda()
    w2 = torch.from_numpy(synth.weights(t, 2, 0.02, 512, 2048)).cuda()
    x = torch.from_numpy(synth.normal(2, 1.0, 1024)).cuda()
    y1 = torch.empty(2048, device="cuda")
    hip.use_torch_stream()
    hip.gguf_gemv(t, x, w1, None, y1, 2048, 1024, 0)
    ref = torch.empty(512, device="cuda")
    hip.gguf_gemv(t, y1, w2, None, ref, 512, 2048, 0)
    torch.cuda.synchronize()
    outs = [torch.empty(512, device="cuda") for _ in range(16)]
    for o in outs:
        y1.fill_(float("nan"))
        hip.gguf_gemv(t, x, w1, None, y1, 2048, 1024, 0)
        hip.gguf_gemv(t, y1, w2, None, o, 512, 2048, 0)
    torch.cuda.synchronize()
    assert all(torch.equal(o, ref) for o in outs)
    # the context's own stream, explicitly synchronised, still works
    hip.set_stream(None)
    o = torch.empty(512, device="cuda")
    torch.cuda.synchronize()
    hip.gguf_gemv(t, y1, w2, None, o, 512, 2048, 0)
    hip.sync()
    assert torch.equal(o, ref)
    hip.use_torch_stream()


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_wave_split_rows_match(hip, t):
    """Long rows split over the workgroup's four waves (the _ksplit kernels,
    forced on) against the lane-split loops (forced off): the same product
    up to the order of the k sum -- 1e-6 with fp32 y, one f16 rounding with
    f16 y -- with and without the residual and bias epilogue, ragged row
    counts and rows of 132-512 units (one and two units per lane and wave),
    and against exact float64 within the kernels' 5e-5."""
    be = mg.BLOCK[t][0]
    ue = 64 if be == 256 else 32
    try:
        for n, units in ((37, 132), (300, 200), (1000, 448), (5, 512)):
            k = units * ue
            wh = synth.weights(t, 90 + n, 0.02, n, k)
            w = torch.from_numpy(wh).cuda()
            for dt in (torch.float32, torch.float16):
                x = torch.from_numpy(synth.normal(91, 1.0, k)).to(dt).cuda()
                b = torch.from_numpy(synth.normal(92, 0.1, n)).to(dt).cuda()
                outs = []
                for mode in (1, 2):
                    hip.set_gemv_wsplit(mode)
                    y = torch.from_numpy(synth.normal(93, 1.0, n)).to(dt).cuda()
                    hip.gguf_gemv(t, x, w, b, y, n, k, 1)
                    y0 = torch.empty(n, dtype=dt, device="cuda")
                    hip.gguf_gemv(t, x, w, None, y0, n, k, 0)
                    outs.append((host(y).astype(np.float64), host(y0).astype(np.float64)))
                tol = 1e-6 if dt == torch.float32 else 1e-3
                assert rel(outs[0][0], outs[1][0]) <= tol and rel(outs[0][1], outs[1][1]) <= tol, (n, k, dt)
                if dt == torch.float32:
                    w64 = oracle.f16_bits_to_f32(oracle.dequant(t, wh.reshape(-1), n * k)).reshape(n, k)
                    # the decoded weights are f16-rounded for some formats: compare against the
                    # exact product only through the CPU path's 1e-3 bar here
                    want = w64.astype(np.float64) @ x.cpu().numpy().astype(np.float64)
                    assert rel(outs[0][1], want) <= 1e-3, (n, k)
    finally:
        hip.set_gemv_wsplit(0)


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_item_ring_matches_double_buffer(t):
    """The item-ring main loops (forced on with CIMA_GEMV_RING=1, forced off
    with 2) compute every row exactly as the row-group double buffer does:
    identical outputs, f32 and f16, with and without the epilogue, for rows
    of one and of two units per lane and for long rows of several steps
    (ragged included), and for the fused gate+up pair."""
    import os
    from cima_amd.hip import HipCtx

    ctxs = {}
    for mode in ("1", "2"):
        os.environ["CIMA_GEMV_RING"] = mode
        try:
            ctxs[mode] = HipCtx(0)
        finally:
            del os.environ["CIMA_GEMV_RING"]
        ctxs[mode].use_torch_stream()
    be = mg.BLOCK[t][0]
    ue = 64 if be == 256 else 32  # elements per unit
    # one unit per lane at 32 lanes; two per lane at 64 (ragged: 100 units);
    # long rows of 4-7 steps of 64 units (the stepped ring; ragged: 200, 300)
    for n, k in ((1, 32 * ue), (37, 32 * ue), (1000, 32 * ue), (37, 128 * ue), (300, 100 * ue), (37, 200 * ue),
                 (300, 448 * ue), (1, 300 * ue)):
        w = torch.from_numpy(synth.weights(t, 80 + n, 0.02, n, k)).cuda()
        for dt in (torch.float32, torch.float16):
            x = torch.from_numpy(synth.normal(81, 1.0, k)).to(dt).cuda()
            b = torch.from_numpy(synth.normal(82, 0.1, n)).to(dt).cuda()
            outs = []
            for mode, c in ctxs.items():
                y = torch.from_numpy(synth.normal(83, 1.0, n)).to(dt).cuda()
                c.gguf_gemv(t, x, w, b, y, n, k, 1)
                y0 = torch.empty(n, dtype=dt, device="cuda")
                c.gguf_gemv(t, x, w, None, y0, n, k, 0)
                outs.append((y, y0))
            torch.cuda.synchronize()
            assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), (n, k, dt)
    # the gate+up SwiGLU pair (each item one gate row and one up row), with
    # and without biases
    for n, k in ((37, 32 * ue), (1000, 32 * ue), (300, 100 * ue)):
        wg = torch.from_numpy(synth.weights(t, 84 + n, 0.02, n, k)).cuda()
        wu = torch.from_numpy(synth.weights(t, 85 + n, 0.02, n, k)).cuda()
        for dt in (torch.float32, torch.float16):
            x = torch.from_numpy(synth.normal(86, 1.0, k)).to(dt).cuda()
            bg = torch.from_numpy(synth.normal(87, 0.1, n)).to(dt).cuda()
            bu = torch.from_numpy(synth.normal(88, 0.1, n)).to(dt).cuda()
            outs = []
            for mode, c in ctxs.items():
                y = torch.empty(n, dtype=dt, device="cuda")
                c.gguf_gemv_swiglu(t, x, wg, wu, bg, bu, y, n, k)
                y0 = torch.empty(n, dtype=dt, device="cuda")
                c.gguf_gemv_swiglu(t, x, wg, wu, None, None, y0, n, k)
                outs.append((y, y0))
            torch.cuda.synchronize()
            assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), ("pair", n, k, dt)
    for c in ctxs.values():
        c.close()


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
def test_streaming_matches_register_loops(t):
    """The direct-to-LDS streaming kernels (the _dma<D> family, forced on
    with CIMA_GEMV_DMA=1 for one item in flight and 3 for two) against the
    register loops (forced off with CIMA_GEMV_DMA=2): the same product up
    to the order of the k sum (1e-6 with fp32 y, one f16 rounding with f16
    y) for plain, residual + bias and gate+up pair GEMVs, ragged row
    counts, rows of one and of several segments, and the argmax head's
    index exactly."""
    import os
    from cima_amd.hip import HipCtx

    ctxs = {}
    for dma in ("2", "1", "3"):
        os.environ["CIMA_GEMV_DMA"] = dma
        try:
            ctxs[dma] = HipCtx(0)
        finally:
            del os.environ["CIMA_GEMV_DMA"]
        ctxs[dma].use_torch_stream()
    ref_key = "2"
    be = mg.BLOCK[t][0]
    ue = 64 if be == 256 else 32
    for n, k in ((37, 32 * ue), (1000, 128 * ue), (300, 300 * ue)):
        w = torch.from_numpy(synth.weights(t, 70 + n, 0.02, n, k)).cuda()
        wu = torch.from_numpy(synth.weights(t, 71 + n, 0.02, n, k)).cuda()
        for dt in (torch.float32, torch.float16):
            x = torch.from_numpy(synth.normal(72, 1.0, k)).to(dt).cuda()
            b = torch.from_numpy(synth.normal(73, 0.1, n)).to(dt).cuda()
            outs = {}
            for key, c in ctxs.items():
                y0 = torch.empty(n, dtype=dt, device="cuda")
                c.gguf_gemv(t, x, w, None, y0, n, k, 0)
                y1 = torch.from_numpy(synth.normal(74, 1.0, n)).to(dt).cuda()
                c.gguf_gemv(t, x, w, b, y1, n, k, 1)
                y2 = torch.empty(n, dtype=dt, device="cuda")
                c.gguf_gemv_swiglu(t, x, w, wu, b, b, y2, n, k)
                outs[key] = [host(v).astype(np.float64) for v in (y0, y1, y2)]
            tol = 1e-6 if dt == torch.float32 else 1e-3
            for key, o in outs.items():
                for i in range(3):
                    assert rel(o[i], outs[ref_key][i]) <= tol, (key, i, n, k, dt)
        # the head: f16 x and logits, the argmax key's index
        xh = torch.from_numpy(synth.normal(75, 1.0, k)).half().cuda()
        idx = {}
        for key, c in ctxs.items():
            y = torch.empty(n, dtype=torch.float16, device="cuda")
            slot = torch.zeros(1, dtype=torch.int64, device="cuda")
            c.gguf_gemv_argmax(t, xh, None, 0.0, w, y, n, k, slot)
            idx[key] = (int(host(slot)[0]) & 0xFFFFFFFF, host(y).astype(np.float64))
        for key, (i, y) in idx.items():
            assert rel(y, idx[ref_key][1]) <= 1e-3, (key, "argmax logits", n, k)
            assert y[i] == y.max(), (key, "argmax index", n, k)
    for c in ctxs.values():
        c.close()


def swiglu64(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


@pytest.mark.parametrize("t", [Q4_K, Q8_0], ids=["q4_k", "q8_0"])
@pytest.mark.parametrize("act", ["f32", "f16"])
@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
def test_swiglu_full_config2_shape(hip, t, act, with_bias):
    """The benchmark's roofline kernel on its own launch plan: fused gate+up
    SwiGLU at 2 x 14336 x 4096 (64 lanes per row), against the reference CPU
    path (each row decoded to f16, fp32 dot) on the stacked [2n, k] weight,
    then g / (1 + e^-g) * u in float64 (k_gemv_f16 mode 2, src/kernels.cu:
    516-537).  Both the separate-weight entry point and mode 2 of the plain
    GEMV on the stacked weight; rel <= 1e-3."""
    n, k = 14336, 4096
    w = synth.weights(t, seed=77 + t, stddev=0.02, rows=2 * n, k=k)
    x = synth.normal(78, 1.0, k)
    bias = synth.normal(79, 0.1, 2 * n) if with_bias else None
    if act == "f16":
        x = x.astype(np.float16).astype(np.float32)
        if bias is not None:
            bias = bias.astype(np.float16).astype(np.float32)
    dots = oracle.gguf_gemv_packed(t, w, x, 2 * n, k, threads=16).astype(np.float64)
    if bias is not None:
        dots = dots + bias
    want = swiglu64(dots[:n], dots[n:])
    cast = (lambda a: dev(a.astype(np.float16))) if act == "f16" else dev
    xd = cast(x)
    ydt = torch.float16 if act == "f16" else torch.float32
    wg, wu = dev(w[:n]), dev(w[n:])
    bg = cast(bias[:n]) if bias is not None else None
    bu = cast(bias[n:]) if bias is not None else None
    y = torch.empty(n, dtype=ydt, device="cuda")
    hip.gguf_gemv_swiglu(t, xd, wg, wu, bg, bu, y, n, k)
    r = rel(host(y).astype(np.float64), want)
    print(f"{NAMES[t]} swiglu 2x{n}x{k} {act} bias={with_bias}: rel {r:.2e}")
    assert r <= 1e-3
    y2 = torch.empty(n, dtype=ydt, device="cuda")
    hip.gguf_gemv(t, xd, dev(w), cast(bias) if bias is not None else None, y2, n, k, 2)
    assert rel(host(y2).astype(np.float64), want) <= 1e-3
    # the two entry points run the same kernel on the same operands
    assert np.array_equal(host(y2), host(y))


@pytest.mark.parametrize("t", FORMATS, ids=fid)
def test_swiglu_every_launch_plan(hip, t):
    """Mode 2 (gate|up pair) under each (rows, lanes) plan the tuner can
    pick, ragged n, against the CPU path + the SwiGLU closed form."""
    n, k = 333, 1536
    w = synth.weights(t, seed=23 + t, stddev=0.02, rows=2 * n, k=k)
    x = synth.normal(24, 1.0, k)
    dots = oracle.gguf_gemv_packed(t, w, x, 2 * n, k, threads=16)
    want = swiglu64(dots[:n], dots[n:])
    wd, xd = dev(w), dev(x)
    try:
        for rows in (1, 2):
            for lpr in (16, 32, 64):
                hip.set_gemv_tuning(rows, lpr)
                y = torch.empty(n, dtype=torch.float32, device="cuda")
                hip.gguf_gemv(t, xd, wd, None, y, n, k, 2)
                assert rel(host(y), want) <= 1e-3, (rows, lpr)
    finally:
        hip.set_gemv_tuning(0, 0)
