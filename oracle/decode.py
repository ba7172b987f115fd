"""CPU oracle for the decode-step support ops -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may use this module, and only as the checker.

numpy restatements of the reference's decode-step kernels, f16 in and out
like the engine's activations, with the arithmetic carried in float64 so the
oracle sits closer to the exact result than either the reference's fp32 or
the device kernels:

* ``rmsnorm``      k_rmsnorm            src/kernels.cu:30-50
* ``rope``         k_rope               src/kernels.cu:397-414
* ``kv_append``    k_kv_append          src/kernels.cu:440-454
* ``attn_partials`` / ``attn_merge``
                   k_attn_decode_split / k_attn_reduce  src/kernels.cu:547-639
* ``attention``    the softmax they compute, evaluated directly
* ``argmax_packed`` k_argmax_softcap    src/kernels.cu:244-262
* ``decode_step``  enqueue_decode_device + forward_chunk_at (rows == 1)
                   src/models/transformer.rs:1440-1461, :1012-1300

Pins (tests/test_decode_oracle.py): closed forms of rmsnorm on constant
rows, RoPE as a rotation (norm-preserving, identity at position 0, angle
additivity, the explicit 2x2 rotation), attention reducing to v for one
position and to the mean of v for equal scores, the split/merge identity
against the direct softmax, argmax's tie and sign order against numpy, and
the decode step's pieces against one another.
"""
from __future__ import annotations

import numpy as np

from . import gguf_gemv_packed, gather


def f16(a) -> np.ndarray:
    """Round to f16 (RTNE, numpy's IEEE conversion)."""
    return np.asarray(a, dtype=np.float64).astype(np.float16)


def sat16(v: np.ndarray) -> np.ndarray:
    """g_sat16 (src/kernels.cu:30-35): clamp to +-65000; NaN -> -65000 as
    CUDA's fminf/fmaxf return the non-NaN operand."""
    v = np.asarray(v, dtype=np.float64)
    out = np.clip(v, -65000.0, 65000.0)
    return np.where(np.isnan(v), -65000.0, out)


def rmsnorm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    """Rows of x (f16) -> f16(sat(x) / sqrt(mean(sat(x)^2) + eps) * w)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.float16))
    s = sat16(x.astype(np.float64))
    inv = 1.0 / np.sqrt((s * s).mean(axis=1, keepdims=True) + eps)
    g = 1.0 if w is None else np.asarray(w, dtype=np.float16).astype(np.float64)
    return f16(s * inv * g)


def rope_angles(pos: int, dim: int, theta: float, nfreqs: int | None = None) -> np.ndarray:
    """Angle of each pair i < dim/2: p * theta^(-2i/dim), in fp32 like the
    reference's powf and product, so arguments match to the last bit of the
    fp32 angle; pairs >= nfreqs get no rotation (angle 0)."""
    i = np.arange(dim // 2, dtype=np.float32)
    expo = (np.float32(-2.0) * i) / np.float32(dim)
    freq = np.power(np.float64(np.float32(theta)), expo.astype(np.float64)).astype(np.float32)
    ang = (np.float32(pos) * freq).astype(np.float64)
    if nfreqs is not None:
        ang[int(nfreqs):] = 0.0
    return ang


def rope(x: np.ndarray, pos0: int, theta: float, nfreqs: int | None = None) -> np.ndarray:
    """x [rows, heads, dim] f16 -> rotated f16: row r at position pos0 + r;
    pair i = (x[i], x[i + dim/2]) -> (a cos - b sin, a sin + b cos)."""
    x = np.asarray(x, dtype=np.float16)
    rows, heads, dim = x.shape
    h = dim // 2
    out = x.astype(np.float64).copy()
    for r in range(rows):
        ang = rope_angles(pos0 + r, dim, theta, nfreqs)
        c, s = np.cos(ang), np.sin(ang)
        a = out[r, :, :h].copy()
        b = out[r, :, h:].copy()
        out[r, :, :h] = a * c - b * s
        out[r, :, h:] = a * s + b * c
    return f16(out)


def kv_append(kc: np.ndarray, vc: np.ndarray, k: np.ndarray, v: np.ndarray, pos: int) -> None:
    """caches [kv_heads, max_seq, dim]; k, v [rows, kv_heads, dim]: row r goes
    to position pos + r (dropped past max_seq), in place."""
    rows = k.shape[0]
    for r in range(rows):
        if 0 <= pos + r < kc.shape[1]:
            kc[:, pos + r, :] = k[r]
            vc[:, pos + r, :] = v[r]


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, seq: int, scale: float,
              window: int = 0) -> np.ndarray:
    """Direct softmax attention of q [q_heads, dim] over the first seq cache
    positions (GQA: head h reads kv head h // (q_heads / kv_heads)); window
    > 0 keeps the last `window` positions.  Returns float64 [q_heads, dim]."""
    qh, dim = q.shape
    kvh = kc.shape[0]
    grp = qh // kvh
    lo = seq - window if (window > 0 and seq > window) else 0
    out = np.zeros((qh, dim))
    for h in range(qh):
        K = kc[h // grp, lo:seq].astype(np.float64)
        V = vc[h // grp, lo:seq].astype(np.float64)
        s = K @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = (p @ V) / p.sum()
    return out


def attn_partials(q, kc, vc, seq: int, scale: float, csz: int, n_chunks: int, window: int = 0):
    """Per-(head, chunk) {m, l, acc[dim]} of k_attn_decode_split; chunks past
    seq (or before the window) are None."""
    qh, dim = q.shape
    grp = qh // kc.shape[0]
    lo = seq - window if (window > 0 and seq > window) else 0
    parts = [[None] * n_chunks for _ in range(qh)]
    for h in range(qh):
        for c in range(n_chunks):
            s0, s1 = max(c * csz, lo), min(c * csz + csz, seq)
            if s0 >= s1:
                continue
            K = kc[h // grp, s0:s1].astype(np.float64)
            V = vc[h // grp, s0:s1].astype(np.float64)
            s = K @ q[h].astype(np.float64) * scale
            m = s.max()
            e = np.exp(s - m)
            parts[h][c] = (m, e.sum(), e @ V)
    return parts


def attn_merge(parts) -> np.ndarray:
    """k_attn_reduce: M = max m_c; out = sum e^(m_c-M) acc_c / sum e^(m_c-M) l_c."""
    out = []
    for ph in parts:
        live = [p for p in ph if p is not None]
        M = max(p[0] for p in live)
        L = sum(np.exp(p[0] - M) * p[1] for p in live)
        A = sum(np.exp(p[0] - M) * p[2] for p in live)
        out.append(A / L)
    return np.array(out)


def argmax_packed(x: np.ndarray, cap: float = 0.0) -> tuple[int, int]:
    """(index, packed u64) of k_argmax_softcap: the maximum of
    (orderable f32 bits << 32 | index), ties to the higher index."""
    v = np.asarray(x, dtype=np.float16).astype(np.float32)
    if cap > 0:
        v = (np.float32(cap) * np.tanh(v / np.float32(cap))).astype(np.float32)
    b = v.view(np.uint32).astype(np.uint64)
    neg = (b & 0x80000000) != 0
    key = np.where(neg, (~b) & 0xFFFFFFFF, b | 0x80000000)
    packed = (key << np.uint64(32)) | np.arange(len(v), dtype=np.uint64)
    best = int(packed.max())
    return best & 0xFFFFFFFF, best


def _gemv(t, w, x, n, k, threads):
    return gguf_gemv_packed(t, w, np.asarray(x, np.float32), n, k, threads=threads).astype(np.float64)


def decode_step(m: dict, token: int, pos: int, threads: int = 8, trace: list | None = None):
    """One greedy decode step of a Qwen2-shaped model held in numpy.

    ``m``: cfg (dict with hidden, q_heads, kv_heads, head_dim, ffn, vocab,
    rope_theta, rms_eps, type, embed_type, head_type), embed (packed [vocab,
    row]), final_norm (f16), layers (list of dicts: attn_norm, wqkv, bqkv,
    wo, ffn_norm, w_gate_up, w_down packed/f16, optional types (format per
    projection, default cfg type) and wk / wv (separate k and v; wqkv is then
    q alone), k_cache, v_cache f16 arrays [kv_heads, max_seq, dim], modified
    in place).  The f16 roundings sit
    where the reference writes f16 activations: the gathered x, the normed
    h, q/k/v after the bias add (rounded twice: GEMV output, then bias),
    q/k after RoPE, the attention output, x after each residual add, the
    SwiGLU gate/up/product and the logits.  A layer's optional ``window`` >
    0 keeps its last `window` positions (the split kernel's window,
    src/kernels.cu:557-559).  With ``trace`` a list, each layer appends
    {"attn": x after the attention residual, "ffn": x after the FFN
    residual} (f16).

    Returns (logits f16 [vocab], next token).
    """
    c = m["cfg"]
    hid, qh, kvh, hd, ffn = c["hidden"], c["q_heads"], c["kv_heads"], c["head_dim"], c["ffn"]
    t, eps = c["type"], c["rms_eps"]
    qd, kvd = qh * hd, kvh * hd
    x = gather(c["embed_type"], m["embed"], np.array([token], np.uint32), hid).view(np.float16)[0]
    scale = 1.0 / np.sqrt(hd)
    for L in m["layers"]:
        ty = {p: (L.get("types") or {}).get(p) or t for p in ("q", "k", "v", "o", "gate", "up", "down")}
        h = rmsnorm(x, L["attn_norm"], eps)[0]
        if L.get("wk") is None:
            qkv = f16(_gemv(ty["q"], L["wqkv"], h, qd + 2 * kvd, hid, threads))
        else:  # separate q, k, v matrices (formats of their own)
            qkv = f16(np.concatenate([_gemv(ty["q"], L["wqkv"], h, qd, hid, threads),
                                      _gemv(ty["k"], L["wk"], h, kvd, hid, threads),
                                      _gemv(ty["v"], L["wv"], h, kvd, hid, threads)]))
        if L.get("bqkv") is not None:
            qkv = f16(qkv.astype(np.float64) + L["bqkv"].astype(np.float64))
        q = rope(qkv[:qd].reshape(1, qh, hd), pos, c["rope_theta"])[0]
        k = rope(qkv[qd:qd + kvd].reshape(1, kvh, hd), pos, c["rope_theta"])
        v = qkv[qd + kvd:].reshape(1, kvh, hd)
        kv_append(L["k_cache"], L["v_cache"], k, v, pos)
        att = f16(attention(q, L["k_cache"], L["v_cache"], pos + 1, scale, L.get("window", 0))).reshape(-1)
        x = f16(x.astype(np.float64) + _gemv(ty["o"], L["wo"], att, hid, qd, threads))
        x_attn = x
        h = rmsnorm(x, L["ffn_norm"], eps)[0]
        gu = _gemv(ty["gate"], L["w_gate_up"], h, 2 * ffn, hid, threads)
        g, u = f16(gu[:ffn]).astype(np.float64), f16(gu[ffn:]).astype(np.float64)
        act = f16(g / (1.0 + np.exp(-g)) * u)
        x = f16(x.astype(np.float64) + _gemv(ty["down"], L["w_down"], act, hid, ffn, threads))
        if trace is not None:
            trace.append({"attn": x_attn, "ffn": x})
    h = rmsnorm(x, m["final_norm"], eps)[0]
    head = m.get("head")
    ht = c.get("head_type", c["embed_type"]) if head is not None else c["embed_type"]
    logits = f16(_gemv(ht, m["embed"] if head is None else head, h, c["vocab"], hid, threads))
    return logits, argmax_packed(logits)[0]
