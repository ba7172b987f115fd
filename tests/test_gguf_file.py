"""CPU tests of GGUF container ingestion (cima_amd/gguf_file.py), restating
the reference parser's rules (src/formats.rs:134-600) and model_config
(:940-1007).  The spec is pinned by a file assembled byte by byte here,
independently of the writer."""
import os
import struct

import numpy as np
import pytest

import oracle
import oracle.decode as od
from cima_amd import gguf, synth
from cima_amd import gguf_file as gf
from cima_amd.decoder import DecoderConfig, synthetic_kv, synthetic_model

Q8_0, Q4_K, Q5_0, Q6_K = 8, 12, 6, 14


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def hand_built(version=3) -> bytes:
    """A GGUF file per the spec: 2 metadata pairs, a 2x32 Q8_0 tensor and a
    3-element F32 tensor, 32-byte aligned data."""
    kv = gstr("general.architecture") + struct.pack("<I", 8) + gstr("qwen2")
    kv += gstr("qwen2.block_count") + struct.pack("<I", 4) + struct.pack("<I", 7)
    w = synth.weights(Q8_0, 1, 0.02, 2, 32).tobytes()          # 68 bytes
    v = np.array([1.5, -2.0, 3.25], np.float32).tobytes()     # 12 bytes
    ti = gstr("w") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", Q8_0, 0)
    ti += gstr("v") + struct.pack("<I", 1) + struct.pack("<Q", 3) + struct.pack("<IQ", 0, 96)
    head = b"GGUF" + struct.pack("<IQQ", version, 2, 2) + kv + ti
    head += bytes(-len(head) % 32)
    return head + w + bytes(96 - len(w)) + v


def test_reads_a_hand_built_file(tmp_path):
    p = tmp_path / "a.gguf"
    p.write_bytes(hand_built())
    with gf.GGUFFile(str(p)) as g:
        assert g.version == 3 and g.architecture == "qwen2" and g.meta["qwen2.block_count"] == 7
        assert g.tensors["w"].shape == (2, 32) and g.tensors["w"].ggml_type == Q8_0   # dims reversed
        assert g.tensors["v"].shape == (3,)
        assert np.array_equal(g.tensor_data("w"), synth.weights(Q8_0, 1, 0.02, 2, 32))
        assert np.array_equal(g.tensor_data("v"), [1.5, -2.0, 3.25])
        assert g.data_start % 32 == 0 and g.tensors["v"].offset == g.data_start + 96


def test_writer_produces_the_spec_bytes(tmp_path):
    p = tmp_path / "b.gguf"
    gf.write(str(p), [("general.architecture", gf.T_STR, "qwen2"), ("qwen2.block_count", gf.T_U32, 7)],
             [("w", Q8_0, (2, 32), synth.weights(Q8_0, 1, 0.02, 2, 32).tobytes()),
              ("v", gf.GGML_F32, (3,), np.array([1.5, -2.0, 3.25], np.float32).tobytes())])
    assert p.read_bytes() == hand_built()


def test_every_metadata_value_type_round_trips(tmp_path):
    meta = [("u8", gf.T_U8, 200), ("i8", gf.T_I8, -100), ("u16", gf.T_U16, 60000), ("i16", gf.T_I16, -30000),
            ("u32", gf.T_U32, 4000000000), ("i32", gf.T_I32, -2000000000), ("f32", gf.T_F32, 0.5),
            ("bool", gf.T_BOOL, True), ("str", gf.T_STR, "héllo"), ("u64", gf.T_U64, 1 << 40),
            ("i64", gf.T_I64, -(1 << 40)), ("f64", gf.T_F64, 1e-300),
            ("arr_i32", gf.T_ARR, (gf.T_I32, [1, -2, 3])), ("arr_str", gf.T_ARR, (gf.T_STR, ["a", "", "ccc"])),
            ("arr_arr", gf.T_ARR, (gf.T_ARR, [(gf.T_U8, [1, 2]), (gf.T_U8, [])]))]
    p = str(tmp_path / "m.gguf")
    gf.write(p, meta, [], version=2, alignment=64)
    with gf.GGUFFile(p) as g:
        assert g.version == 2 and g.alignment == 64
        m = g.meta
        for k in ("u8", "i8", "u16", "i16", "u32", "i32", "f32", "bool", "str", "u64", "i64", "f64"):
            assert m[k] == dict((a, c) for a, _, c in meta)[k], k
        assert list(m["arr_i32"]) == [1, -2, 3] and m["arr_str"] == ["a", "", "ccc"]
        assert [list(a) for a in m["arr_arr"]] == [[1, 2], []]


@pytest.mark.parametrize("t", list(gguf.DType) + [gf.GGML_F32, gf.GGML_F16, gf.GGML_BF16])
def test_tensors_of_every_type_round_trip(tmp_path, t):
    rows, k = 3, 256
    data = np.random.default_rng(t).integers(0, 256, gf.tensor_bytes(t, rows * k), dtype=np.uint8)
    p = str(tmp_path / "t.gguf")
    gf.write(p, [], [("a", t, (rows, k), data.tobytes()), ("b", t, (1, 1, 2, k), data[:gf.tensor_bytes(t, 2 * k)]
                                                              .tobytes())])
    with gf.GGUFFile(p) as g:
        assert g.tensors["a"].shape == (rows, k) and g.tensors["b"].shape == (1, 1, 2, k)
        assert np.array_equal(g.tensor_data("a").view(np.uint8).reshape(-1), data)


def _corrupt(tmp_path, b: bytes):
    p = tmp_path / "c.gguf"
    p.write_bytes(b)
    with pytest.raises(gf.GGUFError) as e:
        gf.GGUFFile(str(p))
    return str(e.value)


def test_rejects_what_the_reference_rejects(tmp_path):
    good = hand_built()
    assert "bad magic" in _corrupt(tmp_path, b"GGUX" + good[4:])
    assert "bad magic" in _corrupt(tmp_path, good[:20])
    for v in (1, 4):
        assert "unsupported" in _corrupt(tmp_path, good[:4] + struct.pack("<I", v) + good[8:])
    assert "truncated" in _corrupt(tmp_path, good[:-1])                    # tensor data cut short
    assert "truncated" in _corrupt(tmp_path, good[:40])                    # header cut short
    assert "implausible" in _corrupt(tmp_path, good[:8] + struct.pack("<QQ", 1 << 21, 2) + good[24:])
    ty_at = good.index(struct.pack("<IQ", Q8_0, 0))                        # Q8_0 -> Q2_K (10)
    assert "not registered" in _corrupt(tmp_path, good[:ty_at] + struct.pack("<I", 10) + good[ty_at + 4:])
    kv_ty = good.index(gstr("qwen2")) - 4                                  # metadata type 8 -> 13
    assert "unknown metadata value type" in _corrupt(tmp_path, good[:kv_ty] + struct.pack("<I", 13)
                                                     + good[kv_ty + 4:])
    nd = good.index(gstr("w")) + len(gstr("w"))                            # n_dims 2 -> 5
    assert "dims" in _corrupt(tmp_path, good[:nd] + struct.pack("<I", 5) + good[nd + 4:])


def test_decoder_config_from_metadata_and_defaults(tmp_path):
    cfg = DecoderConfig(n_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                        max_seq=512)
    m = synthetic_model(cfg, seed=1)
    p = str(tmp_path / "q.gguf")
    gf.save_model(p, m)
    with gf.GGUFFile(p) as g:
        c = gf.decoder_config(g)
        for f in ("n_layers", "hidden", "q_heads", "kv_heads", "head_dim", "ffn", "vocab", "max_seq", "qkv_bias",
                  "tied", "ggml_type"):
            assert getattr(c, f) == getattr(cfg, f), f
        assert c.rope_theta == np.float32(cfg.rope_theta) and c.rms_eps == np.float32(cfg.rms_eps)
    # defaults: kv heads = heads, head_dim = hidden / heads, theta 1e4, eps 1e-6,
    # vocab from the tokenizer's token list, context 8192 capped
    w = synth.weights(Q8_0, 2, 0.02, 256, 256).tobytes()
    meta = [("general.architecture", gf.T_STR, "llama"), ("llama.block_count", gf.T_U32, 0),
            ("llama.embedding_length", gf.T_U32, 256), ("llama.feed_forward_length", gf.T_U32, 512),
            ("llama.attention.head_count", gf.T_U32, 4),
            ("tokenizer.ggml.tokens", gf.T_ARR, (gf.T_STR, [f"t{i}" for i in range(300)]))]
    gf.write(p, meta, [("blk.0.attn_q.weight", Q8_0, (256, 256), w)])
    with gf.GGUFFile(p) as g:
        c = gf.decoder_config(g, max_seq=1024)
        assert (c.kv_heads, c.head_dim, c.rope_theta, c.rms_eps, c.vocab, c.max_seq) == (4, 64, 1e4, 1e-6, 300, 1024)
        assert c.tied and not c.qkv_bias
    gf.write(p, meta[:1] + meta[2:], [("blk.0.attn_q.weight", Q8_0, (256, 256), w)])
    with gf.GGUFFile(p) as g, pytest.raises(gf.GGUFError, match="block_count"):
        gf.decoder_config(g)


def test_model_round_trip_with_mixed_formats(tmp_path):
    cfg = DecoderConfig(n_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=600,
                        max_seq=256, tied=False)
    m = synthetic_model(cfg, seed=2, tensor_types={"v": Q6_K, "down": Q6_K, "o": Q5_0, "head": Q4_K})
    p = str(tmp_path / "mixed.gguf")
    gf.save_model(p, m, alignment=64)
    with gf.GGUFFile(p) as g:
        m2 = gf.load_model(g)
        assert m2.head_type == Q4_K and m2.embed_type == Q8_0 and np.array_equal(m2.head, m.head)
        for a, b in zip(m.layers, m2.layers):
            assert a["types"] == b["types"]
            for key in ("wqkv", "wk", "wv", "wo", "w_gate_up", "w_down", "bqkv", "attn_norm", "ffn_norm"):
                assert np.array_equal(a[key], b[key]), key


def test_load_rejects_unsupported_layouts(tmp_path):
    cfg = DecoderConfig(n_layers=1, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=300,
                        max_seq=256)
    m = synthetic_model(cfg, seed=4)
    p = str(tmp_path / "x.gguf")
    gf.save_model(p, m)
    with gf.GGUFFile(p) as g:
        names = {k: (ti.ggml_type, ti.shape, bytes(g.tensor_data(k).view(np.uint8).reshape(-1)))
                 for k, ti in g.tensors.items()}
        meta = [(k, gf.T_STR if isinstance(v, str) else (gf.T_F32 if isinstance(v, float) else gf.T_U32), v)
                for k, v in g.meta.items()]
    # gate and up in different formats
    t, shp, _ = names["blk.0.ffn_up.weight"]
    ts = [(k, *v) for k, v in names.items() if k != "blk.0.ffn_up.weight"]
    ts.append(("blk.0.ffn_up.weight", Q4_K, shp, synth.weights(Q4_K, 9, 0.02, *shp).tobytes()))
    gf.write(p, meta, ts)
    with gf.GGUFFile(p) as g, pytest.raises(gf.GGUFError, match="formats differ"):
        gf.load_model(g)
    # a weight matrix stored as F16 is not a block format
    ts = [(k, *v) for k, v in names.items() if k != "blk.0.attn_output.weight"]
    ts.append(("blk.0.attn_output.weight", gf.GGML_F16, (256, 256), np.zeros(256 * 256, np.float16).tobytes()))
    gf.write(p, meta, ts)
    with gf.GGUFFile(p) as g, pytest.raises(gf.GGUFError, match="block formats"):
        gf.load_model(g)


def _oracle_dict(m, kvs):
    c = m.cfg
    return dict(cfg=dict(hidden=c.hidden, q_heads=c.q_heads, kv_heads=c.kv_heads, head_dim=c.head_dim, ffn=c.ffn,
                         vocab=c.vocab, rope_theta=c.rope_theta, rms_eps=c.rms_eps, type=int(c.ggml_type),
                         embed_type=int(m.embed_type), head_type=int(m.head_type)),
                embed=m.embed, head=m.head, final_norm=m.final_norm,
                layers=[dict(L, k_cache=kv[0].copy(), v_cache=kv[1].copy()) for L, kv in zip(m.layers, kvs)])


def test_oracle_split_qkv_equals_fused():
    """The oracle's separate-q/k/v path (formats of their own) computes what
    the fused matrix does when the formats agree."""
    cfg = DecoderConfig(n_layers=1, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=300,
                        max_seq=128)
    m = synthetic_model(cfg, seed=6)
    kvs = [synthetic_kv(cfg, 0, 50)]
    qd, kvd = 256, 128
    fused = _oracle_dict(m, kvs)
    split = _oracle_dict(m, kvs)
    L = split["layers"][0]
    w = L["wqkv"]
    L["wqkv"], L["wk"], L["wv"] = w[:qd], w[qd:qd + kvd], w[qd + kvd:]
    a = od.decode_step(fused, 7, 50, threads=2)
    b = od.decode_step(split, 7, 50, threads=2)
    assert np.array_equal(a[0], b[0]) and a[1] == b[1]
    assert oracle.BLOCK_ELEMS[Q8_0] == 32


def test_sliding_window_metadata(tmp_path):
    """The reference's model_config (src/formats.rs:940-1007) ignores the
    sliding-window key for qwen2 / llama files, so by default the loader
    decodes with full attention (window 0) even when the file carries one;
    with the opt-in, a single window reaches the decoder config and a
    per-layer window pattern is refused."""
    from cima_amd.decoder import DecoderConfig, synthetic_model

    cfg = DecoderConfig(n_layers=1, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=100,
                        max_seq=256, window=96)
    m = synthetic_model(cfg, seed=2)
    path = str(tmp_path / "win.gguf")
    gf.save_model(path, m)
    g = gf.GGUFFile(path)
    assert gf.decoder_config(g).window == 0
    assert gf.load_model(g).cfg.window == 0
    assert gf.decoder_config(g, use_sliding_window=True).window == 96
    g.meta["qwen2.attention.sliding_window_pattern"] = 2
    assert gf.decoder_config(g).window == 0
    with pytest.raises(gf.GGUFError):
        gf.decoder_config(g, use_sliding_window=True)
    g.close()
