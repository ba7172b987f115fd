"""CPU pins of the decode-step oracle (oracle/decode.py): each function is
checked against what the mathematics fixes -- closed forms, invariants and
special cases -- so that a dropped term, a wrong sign or a transposed index
fails here before the oracle is trusted as the GPU checker."""
import math

import numpy as np
import pytest

import oracle
from oracle import decode as od


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- rmsnorm

def test_rmsnorm_constant_row_closed_form():
    for c in (0.5, -3.0, 100.0):
        x = np.full((1, 96), c, np.float16)
        got = od.rmsnorm(x, None, 1e-6)
        want = np.float16(c / math.sqrt(c * c + 1e-6))
        assert np.all(got == want)


def test_rmsnorm_weight_and_eps():
    x = np.array([[3.0, 4.0]], np.float16)  # mean square 12.5
    w = np.array([2.0, -1.0], np.float16)
    got = od.rmsnorm(x, w, 0.5).astype(np.float64)[0]
    inv = 1.0 / math.sqrt(12.5 + 0.5)
    assert got[0] == np.float16(3 * inv * 2) and got[1] == np.float16(4 * inv * -1)


def test_rmsnorm_saturates_like_g_sat16():
    x = np.array([[65504.0, -65504.0, 1.0, 0.0]], np.float16)
    got = od.rmsnorm(x, None, 0.0).astype(np.float64)[0]
    s = np.array([65000.0, -65000.0, 1.0, 0.0])
    want = (s / math.sqrt((s * s).mean())).astype(np.float16)
    assert np.all(got == want)


def test_rmsnorm_rows_independent():
    x = rng(1).normal(size=(3, 64)).astype(np.float16)
    both = od.rmsnorm(x, None, 1e-6)
    for r in range(3):
        assert np.all(both[r] == od.rmsnorm(x[r:r + 1], None, 1e-6)[0])


# ------------------------------------------------------------------- RoPE

def test_rope_position_zero_is_identity():
    x = rng(2).normal(size=(1, 3, 64)).astype(np.float16)
    assert np.all(od.rope(x, 0, 1e6) == x)


def test_rope_single_pair_is_the_2d_rotation():
    # dim 2: one pair with frequency theta^0 = 1, so the angle is the position
    a, b = 0.75, -0.5
    x = np.array([[[a, b]]], np.float16)
    for p in (1, 7, 1000):
        got = od.rope(x, p, 10000.0).astype(np.float64)[0, 0]
        want = [a * math.cos(p) - b * math.sin(p), a * math.sin(p) + b * math.cos(p)]
        assert np.allclose(got, want, atol=1e-3)


def test_rope_pairs_halves_not_neighbours():
    # NeoX layout: element i pairs with i + dim/2.  A vector with only
    # x[1] set rotates into x[1 + dim/2], never into x[0] or x[2].
    x = np.zeros((1, 1, 8), np.float16)
    x[0, 0, 1] = 1.0
    got = od.rope(x, 3, 100.0).astype(np.float64)[0, 0]
    assert np.count_nonzero(got) == 2 and got[5] != 0
    ang = od.rope_angles(3, 8, 100.0)
    assert math.isclose(got[1], math.cos(ang[1]), abs_tol=1e-3)
    assert math.isclose(got[5], math.sin(ang[1]), abs_tol=1e-3)
    # frequency of pair i is theta^(-2i/dim): pair 1 of dim 8 -> 100^(-1/4)
    assert math.isclose(ang[1], 3 * 100.0 ** -0.25, rel_tol=1e-6)


def test_rope_preserves_pair_norms_and_adds_angles():
    x = rng(3).normal(size=(1, 2, 64)).astype(np.float16)
    r1 = od.rope(x, 500, 1e6)
    xf, rf = x.astype(np.float64), r1.astype(np.float64)
    n0 = xf[..., :32] ** 2 + xf[..., 32:] ** 2
    n1 = rf[..., :32] ** 2 + rf[..., 32:] ** 2
    assert np.allclose(n0, n1, rtol=4e-3, atol=1e-3)
    # rotating by p1 then p2 equals rotating by p1 + p2 (up to f16 rounding)
    r12 = od.rope(od.rope(x, 200, 1e6), 300, 1e6).astype(np.float64)
    assert np.allclose(r12, rf, atol=4e-3)


def test_rope_nfreqs_leaves_tail_pairs():
    x = rng(4).normal(size=(1, 1, 16)).astype(np.float16)
    got = od.rope(x, 9, 1e4, nfreqs=3)
    keep = [i for i in range(8) if i >= 3]
    assert np.all(got[0, 0, keep] == x[0, 0, keep])
    assert np.all(got[0, 0, [k + 8 for k in keep]] == x[0, 0, [k + 8 for k in keep]])
    assert not np.all(got[0, 0, :3] == x[0, 0, :3])


def test_rope_rows_take_consecutive_positions():
    x = rng(5).normal(size=(1, 1, 32)).astype(np.float16)
    two = od.rope(np.concatenate([x, x]), 10, 1e4)
    assert np.all(two[1] == od.rope(x, 11, 1e4)[0])


# -------------------------------------------------------------- attention

def test_attention_single_position_returns_v():
    kc = rng(6).normal(size=(1, 8, 64)).astype(np.float16)
    vc = rng(7).normal(size=(1, 8, 64)).astype(np.float16)
    q = rng(8).normal(size=(2, 64)).astype(np.float16)
    out = od.attention(q, kc, vc, 1, 0.125)
    assert np.allclose(out, vc[0, 0].astype(np.float64)[None, :].repeat(2, 0), rtol=0, atol=1e-12)


def test_attention_equal_scores_average_v():
    kc = np.zeros((2, 16, 64), np.float16)
    vc = rng(9).normal(size=(2, 16, 64)).astype(np.float16)
    q = rng(10).normal(size=(4, 64)).astype(np.float16)
    out = od.attention(q, kc, vc, 10, 0.125)
    for h in range(4):  # GQA: heads 0,1 -> kv 0; 2,3 -> kv 1
        assert np.allclose(out[h], vc[h // 2, :10].astype(np.float64).mean(0), atol=1e-12)


def test_attention_softmax_weights_brute_force():
    kc = rng(11).normal(size=(1, 5, 4)).astype(np.float16)
    vc = rng(12).normal(size=(1, 5, 4)).astype(np.float16)
    q = rng(13).normal(size=(1, 4)).astype(np.float16)
    s = [sum(float(q[0, d]) * float(kc[0, j, d]) for d in range(4)) * 0.5 for j in range(5)]
    w = [math.exp(v) for v in s]
    want = [sum(w[j] * float(vc[0, j, d]) for j in range(5)) / sum(w) for d in range(4)]
    assert np.allclose(od.attention(q, kc, vc, 5, 0.5)[0], want, atol=1e-12)


@pytest.mark.parametrize("seq,csz,window", [(1, 128, 0), (300, 128, 0), (256, 128, 0), (700, 64, 0), (700, 64, 100)])
def test_split_merge_equals_direct(seq, csz, window):
    kc = rng(14).normal(size=(2, 1024, 64)).astype(np.float16)
    vc = rng(15).normal(size=(2, 1024, 64)).astype(np.float16)
    q = (3 * rng(16).normal(size=(14, 64))).astype(np.float16)
    nch = 1024 // csz
    parts = od.attn_partials(q, kc, vc, seq, 0.125, csz, nch, window)
    assert all(parts[0][c] is None for c in range(-(-seq // csz), nch))
    assert np.allclose(od.attn_merge(parts), od.attention(q, kc, vc, seq, 0.125, window), rtol=1e-12, atol=1e-12)


def test_kv_append_positions_and_overflow():
    kc = np.zeros((2, 4, 3), np.float16)
    vc = np.zeros_like(kc)
    k = np.arange(12, dtype=np.float16).reshape(2, 2, 3)
    od.kv_append(kc, vc, k, -k, 3)  # row 0 -> pos 3, row 1 -> pos 4 dropped
    assert np.all(kc[:, 3] == k[0]) and np.all(vc[:, 3] == -k[0])
    assert np.all(kc[:, :3] == 0)


# ----------------------------------------------------------------- argmax

def test_argmax_matches_numpy_and_ties_go_high():
    x = rng(17).normal(size=5000).astype(np.float16)
    idx, _ = od.argmax_packed(x)
    assert idx == int(np.argmax(x.astype(np.float32))) or x[idx] == x.max()
    x[[10, 4000]] = np.float16(9.0)
    assert od.argmax_packed(x)[0] == 4000


def test_argmax_sign_order():
    x = np.array([-3.0, -0.0, 0.0, -1.0], np.float16)
    assert od.argmax_packed(x)[0] == 2  # +0 above -0
    x = np.array([-3.0, -1.0, -2.0], np.float16)
    assert od.argmax_packed(x)[0] == 1
    packed = od.argmax_packed(np.array([1.0], np.float16))[1]
    assert packed >> 32 == (0x3F800000 | 0x80000000)


def test_argmax_softcap_keeps_order():
    x = (5 * rng(18).normal(size=300)).astype(np.float16)
    assert od.argmax_packed(x, 30.0)[0] == od.argmax_packed(x)[0]


# ------------------------------------------------------------ decode step

def _tiny_model(zero_layers: bool):
    from cima_amd import synth

    cfg = dict(hidden=64, q_heads=2, kv_heads=1, head_dim=32, ffn=96, vocab=50, rope_theta=1e4, rms_eps=1e-6,
               type=8, embed_type=8)
    hid, qd, kvd, ffn = 64, 64, 32, 96

    def w(seed, rows, k):
        if zero_layers:
            return np.zeros((rows, k // 32 * 34), np.uint8)
        return synth.weights(8, seed, 0.05, rows, k)
    layers = []
    for i in range(2):
        layers.append(dict(attn_norm=np.ones(hid, np.float16), wqkv=w(10 * i + 1, qd + 2 * kvd, hid),
                           bqkv=None, wo=w(10 * i + 2, hid, qd), ffn_norm=np.ones(hid, np.float16),
                           w_gate_up=w(10 * i + 3, 2 * ffn, hid), w_down=w(10 * i + 4, hid, ffn),
                           k_cache=np.zeros((1, 16, 32), np.float16), v_cache=np.zeros((1, 16, 32), np.float16)))
    embed = synth.weights(8, 99, 0.5, 50, hid)
    return dict(cfg=cfg, embed=embed, final_norm=np.ones(hid, np.float16), layers=layers)


def test_decode_step_zero_layers_is_norm_then_tied_head():
    m = _tiny_model(True)
    logits, tok = od.decode_step(m, 7, 0)
    e = oracle.dequant(8, m["embed"], 50 * 64).view(np.float16).reshape(50, 64).astype(np.float64)
    h = od.rmsnorm(e[7].astype(np.float16), None, 1e-6)[0].astype(np.float64)
    want = e @ h
    assert np.allclose(logits.astype(np.float64), want, rtol=2e-3, atol=2e-3)
    assert tok == int(np.argmax(want))


def test_decode_step_writes_cache_at_pos_and_is_deterministic():
    m1, m2 = _tiny_model(False), _tiny_model(False)
    l1, t1 = od.decode_step(m1, 3, 5)
    l2, t2 = od.decode_step(m2, 3, 5)
    assert np.all(l1 == l2) and t1 == t2
    for L in m1["layers"]:
        assert np.any(L["k_cache"][:, 5] != 0) and np.all(L["k_cache"][:, 6:] == 0)
        assert np.all(L["k_cache"][:, :5] == 0)
