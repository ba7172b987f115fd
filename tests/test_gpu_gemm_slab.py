"""GPU parity of the dequant-slab prefill route (cima_hip_gguf_gemm_slab):
the reference's lin_gemm (src/models/transformer.rs:618-655) decodes W into
an f16 slab with gguf_dequant and multiplies it with cublasGemmEx
(src/cuda.rs:2468-2541); here the slab is decoded by the bit-exact dequant
kernel and multiplied by hipBLASLt.  Checked against the CPU path (f16
dequant + fp64 GEMM of the f16-rounded X) at the north star's 1e-3 bar,
and against the fused MFMA kernel on the same inputs."""
import numpy as np
import pytest

import oracle
from cima_amd import gguf, synth
from cima_amd.hip import EngineError, E_INVALID, HipCtx

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


@pytest.fixture
def route_all(hip):
    """Send every token count to the library route for the test's duration."""
    hip.set_gemm_route(1)
    yield hip
    hip.set_gemm_route(0)


def slab_for(m, n, k, xd):
    nbytes = HipCtx.gemm_slab_bytes(m, n, k, x_f16=xd == gguf.DT_F16)
    return torch.empty(nbytes, dtype=torch.uint8, device="cuda")


def run_slab(hip, t, w, xf, m, n, k, xd, yd, ldy=None, slab=None):
    ldy = n if ldy is None else ldy
    x = torch.from_numpy(xf).to(TDT[xd]).cuda()
    y = torch.full((m, ldy), 3.0, dtype=TDT[yd], device="cuda")
    slab = slab_for(m, n, k, xd) if slab is None else slab
    route = hip.gguf_gemm_slab(t, x, torch.from_numpy(w).cuda(), y, m, n, k, slab, ldy=ldy, x_dtype=xd, y_dtype=yd)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), x.float().cpu().numpy(), route


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
@pytest.mark.parametrize("m", [1, 7, 33, 130])
def test_slab_route_all_formats(route_all, t, m):
    hip = route_all
    n, k = 200, 512
    w = synth.weights(t, 80 + t, 0.02, n, k)
    xf = synth.normal(81 + m, 1.0, m * k).reshape(m, k)
    w16 = oracle.dequant(t, w, n * k)
    for xd, yd in ((gguf.DT_BF16, gguf.DT_F32), (gguf.DT_F16, gguf.DT_F16), (gguf.DT_F32, gguf.DT_F32)):
        y, xh, route = run_slab(hip, t, w, xf, m, n, k, xd, yd)
        assert route == 1, "hipBLASLt route not taken"
        want = oracle.gemm(xh.astype(np.float16).astype(np.float32), w16, m, n, k)
        r = rel(y, want)
        assert r <= (1e-5 if yd == gguf.DT_F32 else 1e-3), (xd, yd, r)


@pytest.mark.parametrize("m", [512, 600])
def test_slab_route_config4_shape(hip, m):
    """Benchmark config 4 shape (Q4_K W 14336x4096, X bf16, Y fp32) at and
    past the route threshold: library route, checked on 256 sampled rows
    against the CPU path and in full against the fused kernel."""
    n, k = 14336, 4096
    w = synth.weights(Q4_K, 60, 0.02, n, k)
    xf = synth.normal(61, 1.0, m * k).reshape(m, k)
    y, xh, route = run_slab(hip, Q4_K, w, xf, m, n, k, gguf.DT_BF16, gguf.DT_F32)
    assert route == 1
    rows = np.random.default_rng(m).choice(n, 256, replace=False)
    w16 = oracle.dequant(Q4_K, np.stack([w[r] for r in rows]).reshape(-1), 256 * k)
    r = rel(y[:, rows], oracle.gemm(xh, w16, m, 256, k))
    print(f"slab route m={m}: rel err vs CPU path {r:.2e}")
    assert r <= 1e-5
    yf = torch.empty((m, n), device="cuda")
    hip.gguf_gemm(Q4_K, torch.from_numpy(xf).to(torch.bfloat16).cuda(), torch.from_numpy(w).cuda(), yf, m, n, k)
    torch.cuda.synchronize()
    assert rel(y, yf.cpu().numpy()) <= 1e-5


def test_slab_fused_fallbacks(route_all):
    """ldy != n, a slab too small for W and X, and the threshold all run the
    fused kernel, with the same result and the ldy padding untouched."""
    hip = route_all
    n, k, m = 96, 256, 20
    w = synth.weights(Q4_K, 90, 0.02, n, k)
    xf = synth.normal(91, 1.0, m * k).reshape(m, k)
    want = oracle.gemm(xf.astype(np.float16).astype(np.float32), oracle.dequant(Q4_K, w, n * k), m, n, k)
    y, _, route = run_slab(hip, Q4_K, w, xf, m, n, k, gguf.DT_F16, gguf.DT_F32, ldy=n + 8)
    assert route == 0 and rel(y[:, :n], want) <= 1e-5 and np.all(y[:, n:] == 3.0)
    small = torch.empty(2 * n * k - 256, dtype=torch.uint8, device="cuda")
    y, _, route = run_slab(hip, Q4_K, w, xf, m, n, k, gguf.DT_F16, gguf.DT_F32, slab=small)
    assert route == 0 and rel(y, want) <= 1e-5
    hip.set_gemm_route(m + 1)
    y, _, route = run_slab(hip, Q4_K, w, xf, m, n, k, gguf.DT_F16, gguf.DT_F32)
    assert route == 0 and rel(y, want) <= 1e-5
    hip.set_gemm_route(m)
    y, _, route = run_slab(hip, Q4_K, w, xf, m, n, k, gguf.DT_F16, gguf.DT_F32)
    assert route == 1 and rel(y, want) <= 1e-5


@pytest.mark.parametrize("n, k, m, want_route", [
    (1024, 4096, 32, 0),    # split-k 16-token tiles: always fused
    (1024, 4096, 33, 1),    # 8 workgroups of 64-token tiles: narrow grid
    (14336, 1024, 128, 0),  # 112 workgroups of rows 1024 long
    (14336, 1024, 129, 0),  # 224 workgroups of 128-token tiles, rows 1024 long
    (4096, 4096, 129, 1),   # 64 workgroups of 128-token tiles, rows 4096 long
    (256, 256, 256, 1),     # narrow grid
    (14336, 256, 256, 0),
    (14336, 256, 257, 1),   # past 256 tokens: always the slab
])
def test_slab_builtin_route(hip, n, k, m, want_route):
    """The built-in route (slab_route_pays in cima_hip.cpp), and both
    routes' results against the CPU path on 64 sampled rows."""
    w = synth.weights(Q5_K, 95, 0.02, n, k)
    xf = synth.normal(96 + m, 1.0, m * k).reshape(m, k)
    y, xh, route = run_slab(hip, Q5_K, w, xf, m, n, k, gguf.DT_BF16, gguf.DT_F32)
    assert route == want_route
    rows = np.random.default_rng(n + m).choice(n, 64, replace=False)
    w16 = oracle.dequant(Q5_K, np.stack([w[r] for r in rows]).reshape(-1), 64 * k)
    assert rel(y[:, rows], oracle.gemm(xh, w16, m, 64, k)) <= 1e-5


def test_slab_repeat_and_shape_change(route_all):
    """Cached plans: two shapes alternately through one slab, each result
    unchanged on the repeat (the slab keeps the previous call's contents)."""
    hip = route_all
    k = 512
    cases = []
    for n, m, seed in ((160, 24, 1), (64, 9, 2)):
        w = synth.weights(Q6_K, 100 + seed, 0.02, n, k)
        xf = synth.normal(110 + seed, 1.0, m * k).reshape(m, k)
        cases.append((n, m, w, xf))
    slab = slab_for(24, 160, k, gguf.DT_F32)
    first = [run_slab(hip, Q6_K, w, xf, m, n, k, gguf.DT_F32, gguf.DT_F32, slab=slab) for n, m, w, xf in cases]
    again = [run_slab(hip, Q6_K, w, xf, m, n, k, gguf.DT_F32, gguf.DT_F32, slab=slab) for n, m, w, xf in cases]
    for (n, m, w, xf), a, b in zip(cases, first, again):
        assert a[2] == 1 and b[2] == 1
        np.testing.assert_array_equal(a[0], b[0])
        want = oracle.gemm(xf.astype(np.float16).astype(np.float32), oracle.dequant(Q6_K, w, n * k), m, n, k)
        assert rel(a[0], want) <= 1e-5


def test_slab_argument_errors(hip):
    x = torch.zeros((4, 256), device="cuda")
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    y = torch.zeros((4, 4), device="cuda")
    slab = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    assert hip.gguf_gemm_slab(Q4_K, x, w, y, 0, 4, 256, slab) == 0  # m = 0: no-op
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm_slab(Q4_K, x, w, y, 4, 4, 100, slab)
    assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm_slab(Q4_K, x, w, y, 4, 4, 256, slab[16:])  # slab not 256-byte aligned
    assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.set_gemm_route(-1)
    assert e.value.code == E_INVALID


def test_slab_route_graph_replay(hip):
    """After a first (plan-making) call, the library route captured into a
    HIP graph replays to the eager result every time, with eager work
    between the replays (a library that recorded a memset node would show
    here)."""
    n, k, m = 2048, 1024, 300
    w = torch.from_numpy(synth.weights(Q4_K, 120, 0.02, n, k)).cuda()
    x = torch.from_numpy(synth.normal(121, 1.0, m * k).reshape(m, k)).to(torch.bfloat16).cuda()
    slab = slab_for(m, n, k, gguf.DT_BF16)
    y = torch.empty((m, n), device="cuda")
    assert hip.gguf_gemm_slab(Q4_K, x, w, y, m, n, k, slab) == 1
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    yg = torch.zeros((m, n), device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            hip.set_stream(s.cuda_stream)
            hip.gguf_gemm_slab(Q4_K, x, w, yg, m, n, k, slab)
    hip.use_torch_stream()
    torch.cuda.synchronize()
    for i in range(4):
        yg.zero_()
        slab.fill_(0xFF)  # the replay must rebuild the slab itself
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(yg.cpu().numpy(), eager), i
        hip.gguf_gemm_slab(Q4_K, x, w, y, m, n, k, slab)  # eager work between replays
        torch.cuda.synchronize()


def test_slab_route_autotuned(monkeypatch):
    """CIMA_GEMM_AUTOTUNE=1 (read by the context at init): hipBLASLt's
    candidates are timed on the first call of a shape; every later result
    still matches the CPU path."""
    monkeypatch.setenv("CIMA_GEMM_AUTOTUNE", "1")
    ctx = HipCtx(0)
    ctx.use_torch_stream()
    n, k, m = 512, 1024, 300
    w = synth.weights(Q4_K, 130, 0.02, n, k)
    xf = synth.normal(131, 1.0, m * k).reshape(m, k)
    w16 = oracle.dequant(Q4_K, w, n * k)
    for _ in range(2):
        y, xh, route = run_slab(ctx, Q4_K, w, xf, m, n, k, gguf.DT_BF16, gguf.DT_F32)
        assert route == 1
        assert rel(y, oracle.gemm(xh, w16, m, n, k)) <= 1e-5
