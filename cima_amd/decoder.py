"""Batch-1 greedy decoder over the C ABI: a Qwen2/Llama-family model whose
layer weights stay in GGUF blocks, stepped by ``cima_hip_decode_step`` and
replayed as one HIP graph per token.

This mirrors the reference's ``Transformer`` decode path
(``src/models/transformer.rs``): the workspace of ``enqueue_decode_device``
(``:1440-1461``), the device position counter and token feedback that let
``arm_decode_graph`` (``:1467-1497``) capture one step and replay it per
token.  torch is only the allocator and the graph recorder here; every
kernel is the library's.

Weights are synthetic (seeded N(0, sigma^2), quantised by ``cima_amd.synth``)
-- there are no checkpoints in this build.  The q, k and v projections are
stored as one [q + 2 kv, hidden] matrix and gate/up as one [2 ffn, hidden]
matrix, the reference's fused ``LayerW`` layouts
(``src/models/transformer.rs:1062-1085``).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import gguf, synth
from .hip import Decoder, DecoderLayer, HipCtx


@dataclass
class DecoderConfig:
    """Architecture of the decoder.  Defaults: Qwen2.5-0.5B."""
    n_layers: int = 24
    hidden: int = 896
    q_heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 4864
    vocab: int = 151936
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    qkv_bias: bool = True
    tied: bool = True
    ggml_type: int = gguf.DType.Q8_0
    max_seq: int = 4096
    attn_chunk: int = 128
    window: int = 0      # sliding-window attention (> 0: the last `window` positions), every layer


# the projections of a layer, as named in a layer's "types" dict
PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class HostModel:
    """A model on the host (packed GGUF bytes and f16 arrays).

    Each layer dict holds attn_norm, wqkv, bqkv, wo, ffn_norm, w_gate_up,
    w_down and a "types" dict (ggml type per projection).  q, k and v are
    one fused [q + 2 kv, hidden] matrix in wqkv when they share a format;
    otherwise wqkv is q alone and "wk" / "wv" hold k and v.  gate and up
    (one format) are one fused [2 ffn, hidden] matrix."""
    cfg: DecoderConfig
    embed: np.ndarray
    final_norm: np.ndarray
    layers: list = field(default_factory=list)
    head: np.ndarray | None = None
    embed_type: int | None = None
    head_type: int | None = None

    def __post_init__(self):
        if self.embed_type is None:
            self.embed_type = int(self.cfg.ggml_type)
        if self.head_type is None:
            self.head_type = self.embed_type


def _f16(seed: int, sigma: float, n: int, mean: float = 0.0) -> np.ndarray:
    return (synth.normal(seed, sigma, n) + np.float32(mean)).astype(np.float16)


def synthetic_model(cfg: DecoderConfig, seed: int = 5, sigma: float = 0.02,
                    tensor_types: dict | None = None) -> HostModel:
    """Seeded random-init weights of the configured shape, every matrix
    quantised to cfg.ggml_type (the tied embedding/head too) unless
    ``tensor_types`` names another format for a projection ("q" ... "down",
    as in PROJECTIONS; gate and up must agree) or for "embed" / "head"."""
    t = int(cfg.ggml_type)
    tt = {k: int(v) for k, v in (tensor_types or {}).items()}
    types = {p: tt.get(p, t) for p in PROJECTIONS}
    if types["gate"] != types["up"]:
        raise ValueError("gate and up projections must share a format")
    qd, kvd = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    s = seed * 1000
    et = tt.get("embed", t)
    embed = synth.weights(et, s + 1, sigma, cfg.vocab, cfg.hidden)
    m = HostModel(cfg, embed, _f16(s + 2, 0.1, cfg.hidden, 1.0), embed_type=et)
    if not cfg.tied:
        m.head_type = tt.get("head", t)
        m.head = synth.weights(m.head_type, s + 3, sigma, cfg.vocab, cfg.hidden)
    for i in range(cfg.n_layers):
        b = s + 100 * (i + 1)
        L = {
            "attn_norm": _f16(b + 1, 0.1, cfg.hidden, 1.0),
            "bqkv": _f16(b + 3, 0.1, qd + 2 * kvd) if cfg.qkv_bias else None,
            "wo": synth.weights(types["o"], b + 4, sigma, cfg.hidden, qd),
            "ffn_norm": _f16(b + 5, 0.1, cfg.hidden, 1.0),
            "w_gate_up": synth.weights(types["gate"], b + 6, sigma, 2 * cfg.ffn, cfg.hidden),
            "w_down": synth.weights(types["down"], b + 7, sigma, cfg.hidden, cfg.ffn),
            "types": dict(types),
        }
        if cfg.window:
            L["window"] = int(cfg.window)
        if types["q"] == types["k"] == types["v"]:
            L["wqkv"] = synth.weights(types["q"], b + 2, sigma, qd + 2 * kvd, cfg.hidden)
        else:
            L["wqkv"] = synth.weights(types["q"], b + 2, sigma, qd, cfg.hidden)
            L["wk"] = synth.weights(types["k"], b + 8, sigma, kvd, cfg.hidden)
            L["wv"] = synth.weights(types["v"], b + 9, sigma, kvd, cfg.hidden)
        m.layers.append(L)
    return m


def synthetic_kv(cfg: DecoderConfig, layer: int, ctx_len: int, seed: int = 9):
    """Seeded N(0, 1) f16 keys and values for positions [0, ctx_len) of one
    layer's caches [kv_heads, max_seq, head_dim] (zeros beyond)."""
    shape = (cfg.kv_heads, cfg.max_seq, cfg.head_dim)
    kc = np.zeros(shape, np.float16)
    vc = np.zeros(shape, np.float16)
    n = cfg.kv_heads * ctx_len * cfg.head_dim
    kc[:, :ctx_len] = _f16(seed * 7919 + 2 * layer, 1.0, n).reshape(cfg.kv_heads, ctx_len, cfg.head_dim)
    vc[:, :ctx_len] = _f16(seed * 7919 + 2 * layer + 1, 1.0, n).reshape(cfg.kv_heads, ctx_len, cfg.head_dim)
    return kc, vc


class DeviceDecoder:
    """The model, its KV caches and the decode workspace in device memory."""

    def __init__(self, hip: HipCtx, model: HostModel, device: str = "cuda"):
        import torch

        self.hip = hip
        self.cfg = c = model.cfg
        self.torch = torch
        dev = torch.device(device)
        # contiguous and writable (weights read from a GGUF map are views
        # of a read-only mapping, which torch will not wrap)
        up = lambda a: torch.from_numpy(np.require(a, requirements=["C", "W"])).to(dev)  # noqa: E731
        self._keep = []
        qd, kvd = c.q_heads * c.head_dim, c.kv_heads * c.head_dim
        self.embed = up(model.embed)
        self.head = None if model.head is None else up(model.head)
        self.embed_type, self.head_type = int(model.embed_type), int(model.head_type)
        self.final_norm = up(model.final_norm)
        self.layers = []
        for L in model.layers:
            d = {k: (None if v is None else up(v)) for k, v in L.items() if k not in ("types", "window")}
            d["types"] = dict(L.get("types") or {})
            d["window"] = int(L.get("window", c.window))
            d["k_cache"] = torch.zeros((c.kv_heads, c.max_seq, c.head_dim), dtype=torch.float16, device=dev)
            d["v_cache"] = torch.zeros_like(d["k_cache"])
            self.layers.append(d)
        n_chunks = -(-c.max_seq // c.attn_chunk)
        f16 = torch.float16
        self.x = torch.zeros(c.hidden, dtype=f16, device=dev)
        self.qkv = torch.zeros(qd + 2 * kvd, dtype=f16, device=dev)
        self.act = torch.zeros(c.ffn, dtype=f16, device=dev)
        self.logits = torch.zeros(c.vocab, dtype=f16, device=dev)
        self.part = torch.zeros(c.q_heads * n_chunks * (c.head_dim + 2), dtype=torch.float32, device=dev)
        self.slot = torch.zeros(1, dtype=torch.int64, device=dev)
        self.ids = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graph = None
        self.desc = self._describe()

    def _describe(self) -> Decoder:
        c = self.cfg
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        arr = (DecoderLayer * c.n_layers)()
        for i, L in enumerate(self.layers):
            ty = L["types"]
            arr[i] = DecoderLayer(p(L["attn_norm"]), p(L["wqkv"]), p(L.get("bqkv")), p(L["wo"]), p(L["ffn_norm"]),
                                  p(L["w_gate_up"]), p(L["w_down"]), p(L["k_cache"]), p(L["v_cache"]),
                                  p(L.get("wk")), p(L.get("wv")), None,
                                  *[int(ty.get(n, 0)) for n in PROJECTIONS], int(L["window"]))
        self._keep.append(arr)
        t = int(c.ggml_type)
        return Decoder(
            ggml_type=t, embed_type=self.embed_type, head_type=self.head_type, n_layers=c.n_layers,
            hidden=c.hidden, q_heads=c.q_heads,
            kv_heads=c.kv_heads, head_dim=c.head_dim, ffn=c.ffn, vocab=c.vocab, max_seq=c.max_seq,
            attn_chunk=c.attn_chunk, rope_theta=c.rope_theta, rms_eps=c.rms_eps, embed=p(self.embed),
            head=p(self.head), final_norm=p(self.final_norm),
            layers=ctypes.cast(arr, ctypes.POINTER(DecoderLayer)),
            x=p(self.x), qkv=p(self.qkv), act=p(self.act), logits=p(self.logits),
            part=p(self.part), slot=p(self.slot), ids=p(self.ids), pos=p(self.pos))

    def load_kv(self, layer: int, kc: np.ndarray, vc: np.ndarray) -> None:
        L = self.layers[layer]
        L["k_cache"].copy_(self.torch.from_numpy(kc))
        L["v_cache"].copy_(self.torch.from_numpy(vc))

    def set_state(self, token: int, pos: int) -> None:
        """Input token and its position (synchronous)."""
        if not 0 <= pos < self.cfg.max_seq:
            raise ValueError(f"position {pos} outside the cache (max_seq {self.cfg.max_seq})")
        self.ids.fill_(int(token))
        self.pos.fill_(int(pos))
        self.torch.cuda.synchronize()

    def step(self) -> None:
        """Enqueue one decode step on torch's current stream."""
        self.hip.use_torch_stream()
        self.hip.decode_step(self.desc)

    def capture(self, native: bool = True) -> None:
        """Record one step as a graph (arm_decode_graph, src/models/
        transformer.rs:1467-1497); replay() runs it.  native: the library's
        own capture of a dedicated stream (cima_hip_capture_begin/end);
        otherwise torch's CUDAGraph around the same calls."""
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        self.stream = s
        self.hip.set_stream(s)
        if native:
            self.hip.capture_begin()
            try:
                self.hip.decode_step(self.desc)
            finally:
                g = self.hip.capture_end()
            self.graph = g
        else:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    self.hip.decode_step(self.desc)
            self.graph = g
        torch.cuda.current_stream().wait_stream(s)

    def replay(self) -> None:
        """One step: a graph launch on the decoder's stream (self.stream)."""
        self.hip.set_stream(self.stream)
        if hasattr(self.graph, "launch"):
            self.graph.launch()
        else:
            with self.torch.cuda.stream(self.stream):
                self.graph.replay()

    def token(self) -> int:
        return int(self.ids.item())

    def position(self) -> int:
        return int(self.pos.item())
