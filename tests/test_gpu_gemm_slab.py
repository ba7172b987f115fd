"""GPU parity of the prefill entry point with the engine's scratch slab
(cima_hip_gguf_gemm_slab): the reference's lin_gemm (src/models/
transformer.rs:618-655) decodes W into an f16 slab with gguf_dequant and
multiplies it with cublasGemmEx (src/cuda.rs:2468-2541); here the same
call runs the fused MFMA kernels, which dequantise W bit-exactly tile by
tile, so W is never expanded and no library GEMM runs; the slab only holds
the partial tiles of narrow weights split along k at up to 32 tokens.  Checked
against the CPU path (f16 dequant + fp64 GEMM of the f16-rounded X): 1e-5
with fp32 Y, where only the summation order differs, and the north star's
1e-3 with f16 Y."""
import numpy as np
import pytest

import oracle
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


def want_of(t, w, xh, m, n, k):
    """The CPU path on X as the kernels see it: rounded to f16."""
    xh16 = np.asarray(xh, np.float32).astype(np.float16).astype(np.float32)
    return oracle.gemm(xh16, oracle.dequant(t, w, n * k), m, n, k, threads=16)


@pytest.mark.parametrize("t", FORMATS, ids=[NAMES[t] for t in FORMATS])
@pytest.mark.parametrize("m", [1, 33, 300])
def test_slab_entry_all_formats(hip, t, m):
    """Every format, ragged token counts, all X / Y types: the slab entry
    point gives cima_hip_gguf_gemm's bits, within the bars of the CPU path,
    and leaves the slab as it found it."""
    n, k = 200, 512
    w = synth.weights(t, 80 + t, 0.02, n, k)
    wd = torch.from_numpy(w).cuda()
    xf = synth.normal(81 + m, 1.0, m * k).reshape(m, k)
    slab = torch.full((1 << 16,), 0x5A, dtype=torch.uint8, device="cuda")
    for xd, yd in ((gguf.DT_BF16, gguf.DT_F32), (gguf.DT_F16, gguf.DT_F16), (gguf.DT_F32, gguf.DT_F32)):
        x = torch.from_numpy(xf).to(TDT[xd]).cuda()
        ys = torch.full((m, n), 3.0, dtype=TDT[yd], device="cuda")
        yg = torch.full((m, n), 3.0, dtype=TDT[yd], device="cuda")
        hip.gguf_gemm_slab(t, x, wd, ys, m, n, k, slab, x_dtype=xd, y_dtype=yd)
        hip.gguf_gemm(t, x, wd, yg, m, n, k, x_dtype=xd, y_dtype=yd)
        torch.cuda.synchronize()
        assert torch.equal(ys, yg)
        r = rel(ys.float().cpu().numpy(), want_of(t, w, x.float().cpu().numpy(), m, n, k))
        assert r <= (1e-5 if yd == gguf.DT_F32 else 1e-3), (NAMES[t], m, xd, yd, r)
    assert bool((slab == 0x5A).all())


@pytest.mark.parametrize("m", [16, 128, 512])
def test_slab_entry_config4_shape(hip, m):
    """Benchmark config 4 (Q4_K 14336 x 4096, bf16 X, fp32 Y) through the
    slab entry point with a reference-sized 32 MiB slab (DQ_SCRATCH,
    src/models/transformer.rs:744-747), checked on 256 sampled rows."""
    n, k = 14336, 4096
    w = synth.weights(Q4_K, 90, 0.02, n, k)
    xf = synth.normal(91 + m, 1.0, m * k).reshape(m, k)
    x = torch.from_numpy(xf).to(torch.bfloat16).cuda()
    y = torch.empty((m, n), device="cuda")
    slab = torch.empty(32 << 20, dtype=torch.uint8, device="cuda")
    hip.gguf_gemm_slab(Q4_K, x, torch.from_numpy(w).cuda(), y, m, n, k, slab)
    torch.cuda.synchronize()
    rows = np.random.default_rng(m).choice(n, 256, replace=False)
    w16 = oracle.dequant(Q4_K, np.stack([w[r] for r in rows]).reshape(-1), 256 * k)
    xh = x.float().cpu().numpy()
    r = rel(y.cpu().numpy()[:, rows], oracle.gemm(xh, w16, m, 256, k, threads=16))
    print(f"config 4 m={m}: rel err vs CPU path {r:.2e}")
    assert r <= 1e-5


def test_slab_argument_errors(hip):
    x = torch.zeros((4, 256), device="cuda")
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    y = torch.zeros((4, 4), device="cuda")
    slab = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    hip.gguf_gemm_slab(Q4_K, x, w, y, 0, 4, 256, slab)  # m = 0: no-op
    hip.gguf_gemm_slab(Q4_K, x, w, y, 4, 4, 256)  # no slab: fine
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm_slab(Q4_K, x, w, y, 4, 4, 100, slab)
    assert e.value.code == E_INVALID
    with pytest.raises(EngineError) as e:
        hip.gguf_gemm_slab(Q4_K, x, w, y, 4, 4, 256, slab[16:])  # slab not 256-byte aligned
    assert e.value.code == E_INVALID


def test_slab_entry_graph_replay(hip):
    """The slab entry point captured into a HIP graph replays to the eager
    result every time, with eager work between the replays."""
    n, k, m = 2048, 1024, 300
    w = torch.from_numpy(synth.weights(Q4_K, 120, 0.02, n, k)).cuda()
    x = torch.from_numpy(synth.normal(121, 1.0, m * k).reshape(m, k)).to(torch.bfloat16).cuda()
    slab = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.empty((m, n), device="cuda")
    hip.gguf_gemm_slab(Q4_K, x, w, y, m, n, k, slab)
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
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(yg.cpu().numpy(), eager), i
        hip.gguf_gemm_slab(Q4_K, x, w, y, m, n, k, slab)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("t, n, k, m", [(Q4_K, 4096, 14336, 16), (Q4_K, 4096, 14336, 32), (Q8_0, 4096, 14336, 32),
                                        (Q4_K, 1024, 4096, 16), (Q4_K, 1024, 4096, 32), (Q4_K, 6144, 4096, 16),
                                        (Q6_K, 1024, 4096, 20)],
                         ids=["q4k-down-m16", "q4k-down-m32", "q8-down-m32", "q4k-kv-m16", "q4k-kv-m32",
                              "q4k-qkv-m16", "q6k-kv-m20"])
def test_slab_entry_k_split(hip, t, n, k, m):
    """Narrow weights at up to 32 tokens split along k over more workgroups,
    with the partial tiles in the caller's slab and a fixed-order sum (the
    long-row down projection at 32 tokens among them): every output row
    against the CPU path (1e-5), against the unsplit product (1e-6: only
    the order of the k sum differs), bit-identical run to run and in a
    replayed graph; a slab too small for the partials runs unsplit, giving
    cima_hip_gguf_gemm's bits."""
    w = synth.weights(t, 130, 0.02, n, k)
    wd = torch.from_numpy(w).cuda()
    x = torch.from_numpy(synth.normal(131 + m, 1.0, m * k).reshape(m, k)).to(torch.bfloat16).cuda()
    slab = torch.empty(32 << 20, dtype=torch.uint8, device="cuda")
    y1 = torch.empty((m, n), device="cuda")
    y2 = torch.empty((m, n), device="cuda")
    yu = torch.empty((m, n), device="cuda")
    hip.gguf_gemm_slab(t, x, wd, y1, m, n, k, slab)
    hip.gguf_gemm_slab(t, x, wd, y2, m, n, k, slab)
    hip.gguf_gemm(t, x, wd, yu, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    got, unsplit = y1.cpu().numpy(), yu.cpu().numpy()
    assert rel(got, unsplit) <= 1e-6
    w16 = oracle.f16_bits_to_f32(oracle.dequant(t, w, n * k)).reshape(n, k)
    xh = x.float().cpu().numpy().astype(np.float64)
    assert rel(got, xh @ w16.astype(np.float64).T) <= 1e-5
    tiny = torch.empty(1024, dtype=torch.uint8, device="cuda")
    ys = torch.empty((m, n), device="cuda")
    hip.gguf_gemm_slab(t, x, wd, ys, m, n, k, tiny)
    torch.cuda.synchronize()
    assert torch.equal(ys, yu)
    # captured and replayed, eager work between replays
    g = torch.cuda.CUDAGraph()
    yg = torch.zeros((m, n), device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            hip.set_stream(s.cuda_stream)
            hip.gguf_gemm_slab(t, x, wd, yg, m, n, k, slab)
    hip.use_torch_stream()
    torch.cuda.synchronize()
    for i in range(3):
        yg.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), i
        hip.gguf_gemm_slab(t, x, wd, y2, m, n, k, slab)
        torch.cuda.synchronize()
