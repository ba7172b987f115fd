"""The allocation-free entry point cima_hip_attn_decode_noalloc against the
entry points it combines (cima_hip_attn_decode_split into a caller's
workspace, then cima_hip_attn_reduce), through the C ABI: two calls in a
row on different shapes, the second smaller (the device scratch keeps the
first call's partials, which the second must not read), bit-identical
outputs; and the size limit."""
import numpy as np
import pytest

from cima_amd.hip import E_INVALID, EngineError

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _case(dim, qh, kvh, max_seq, seed):
    r = np.random.default_rng(seed)
    f = lambda *s: torch.from_numpy(r.standard_normal(s).astype(np.float16)).cuda()  # noqa: E731
    return f(qh, dim), f(kvh, max_seq, dim), f(kvh, max_seq, dim)


@pytest.mark.parametrize("window", [0, 300])
def test_noalloc_attention_matches_workspace_entry_points(hip, window):
    for dim, qh, kvh, seq, csz, max_seq in ((128, 32, 8, 3000, 256, 4096), (64, 14, 2, 777, 64, 1024)):
        q, kc, vc = _case(dim, qh, kvh, max_seq, seq)
        nch = max_seq // csz
        scale = 1.0 / np.sqrt(dim)
        part = torch.zeros(qh * nch * (dim + 2), device="cuda")
        want = torch.empty((qh, dim), dtype=torch.float16, device="cuda")
        hip.attn_decode_split(q, kc, vc, part, qh, kvh, dim, seq, max_seq, csz, nch, scale, window)
        hip.attn_reduce(part, want, qh, dim, csz, nch, seq, max_seq, window)
        got = torch.full((qh, dim), float("nan"), dtype=torch.float16, device="cuda")
        hip.attn_decode_noalloc(q, kc, vc, got, qh, kvh, dim, seq, max_seq, csz, nch, scale, window)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (dim, qh, seq)
        # the device position form as well
        posd = torch.tensor([seq - 1], dtype=torch.int32, device="cuda")
        got2 = torch.full((qh, dim), float("nan"), dtype=torch.float16, device="cuda")
        hip.attn_decode_noalloc(q, kc, vc, got2, qh, kvh, dim, 0, max_seq, csz, nch, scale, window, posd)
        torch.cuda.synchronize()
        assert torch.equal(got2, want)


def test_noalloc_attention_rejects_oversize(hip):
    q, kc, vc = _case(128, 64, 8, 64, 1)
    out = torch.empty((64, 128), dtype=torch.float16, device="cuda")
    # 64 heads x 128 chunks x 130 floats = 4.3 MB > 4 MiB
    with pytest.raises(EngineError) as e:
        hip.attn_decode_noalloc(q, kc, vc, out, 64, 8, 128, 1, 32768, 256, 128, 0.1)
    assert e.value.code == E_INVALID
