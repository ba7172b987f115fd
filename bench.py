#!/usr/bin/env python3
"""Benchmark of the GGUF dequant-GEMV hot path on one MI355X.

Workload (benchmark config 2): the batch-1 decode GEMVs of one Llama-3-8B
decoder layer with Q4_K weights -- q|k|v as one 6144 x 4096 matrix (4096 +
1024 + 1024 rows), o (4096 x 4096, residual epilogue), the fused gate+up
SwiGLU (2 x 14336 x 4096) and down (4096 x 14336, residual epilogue),
chained on one stream as an engine decode step issues them (down consumes
the SwiGLU output).  A
"step" is one layer; the timed region cycles through 32 distinct layer
copies (3.9 GB, like a real 32-layer model) so every step streams its
weights cold from HBM.  The launches are captured once in a HIP graph.
Weights are seeded synthetic N(0, 0.02) quantised to Q4_K; x ~ N(0, 1).

value = algorithmic bytes per step (packed weights + fp32 x and y) x steps /
time, in GB/s.  Per-shape us/call (cold, graph-batched) for configs 1-3 are
reported under "shapes" (with the plain streaming-read time of the same
weight bytes, the best any kernel reads them here, and Q8_0 and
bitsandbytes NF4 at the same Llama-3-8B shapes); "roofline" is for the fused gate+up kernel, the
largest share of a step, timed with HIP events on its launch stream;
"cpu_baseline" runs the CPU restatement of the reference's host path
(decode to f16, fp32 dot) on a bounded sample of the same step, single
threaded like the reference's loops and again on all host cores.

Every figure is the median of --repeats timed runs (graph replays): the
headline over exactly --steps layer steps per replay, each per-shape leg
cold (copies cycled) and hot (one buffer), the decode step over
--decode-tokens tokens split across the repeats.  The device's sustained
read bandwidth is re-measured (1 GiB transfers) and reported beside the
8 TB/s datasheet figure.

Usage: python bench.py [--gpus 1] [--steps 320] [--warmup 64] [--repeats 21]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X published HBM3E bandwidth
Q4_K, Q6_K, Q8_0 = 12, 14, 8
N_LAYERS = 32
HID, FFN, KV = 4096, 14336, 1024


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--repeats", type=int, default=21, help="timed replays; the median is reported")
    ap.add_argument("--cpu-steps", type=int, default=4, help="layer steps in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-shapes", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode-step leg")
    ap.add_argument("--decode-tokens", type=int, default=200)
    ap.add_argument("--calib", action="store_true",
                    help="also run a 256 MiB device copy (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--leg", choices=["q8_0_14336x4096", "q8_0_pair", "q8_0_head_151936x896", "q4_k_14336x4096",
                                        "q4_k_4096x14336", "q4_k_gemm_m16", "q4_k_gemm_m128", "q4_k_gemm_m512"], default=None,
                    help="run only this GEMV or prefill GEMM --steps times on cycled cold copies (and --calib), "
                         "for counter passes of rocprofv3; prints nothing")
    return ap.parse_args()


def wbytes(t, n, k):
    from cima_amd import gguf

    return gguf.storage_bytes(t, n * k)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the decode GEMV path has no multi-GPU mode here -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import cima_amd.build as cbuild

    cbuild.ensure()
    import torch
    from cima_amd import nf4, synth
    from cima_amd.hip import HipCtx

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    ctx = HipCtx(0)
    ctx.use_torch_stream()

    # ---- one layer of seeded weights, replicated into 32 distinct copies.
    # q, k and v are stored as one [q | k | v] matrix (the reference's fused
    # wqkv layout, src/models/transformer.rs:1062-1085): one GEMV instead of
    # three over the same bytes
    shapes = {"q": (HID, HID), "k": (KV, HID), "v": (KV, HID), "o": (HID, HID),
              "gate": (FFN, HID), "up": (FFN, HID), "down": (HID, FFN)}
    host = {name: synth.weights(Q4_K, 100 + i, 0.02, n, k) for i, (name, (n, k)) in enumerate(shapes.items())}
    fused = {"qkv": np.concatenate([host["q"], host["k"], host["v"]]), "o": host["o"], "gate": host["gate"],
             "up": host["up"], "down": host["down"]}
    layers = [{name: torch.from_numpy(w).to(dev) for name, w in fused.items()} for _ in range(N_LAYERS)]
    x = torch.from_numpy(synth.normal(7, 1.0, HID)).to(dev)
    attn = torch.from_numpy(synth.normal(8, 1.0, HID)).to(dev)
    NQKV = HID + 2 * KV
    qkv = torch.empty(NQKV, device=dev)
    h = torch.zeros(HID, device=dev)
    act = torch.empty(FFN, device=dev)
    step_bytes = sum(wbytes(Q4_K, n, k) for n, k in shapes.values())
    # fp32 activations: x -> qkv; attn + residual -> h; h -> act; act + residual -> h
    step_bytes += 4 * (HID + NQKV + (2 * HID + HID) + (HID + FFN) + (FFN + 2 * HID))

    def layer(L):
        ctx.gguf_gemv(Q4_K, x, L["qkv"], None, qkv, NQKV, HID, 0)
        ctx.gguf_gemv(Q4_K, attn, L["o"], None, h, HID, HID, 1)
        ctx.gguf_gemv_swiglu(Q4_K, h, L["gate"], L["up"], None, None, act, FFN, HID)
        ctx.gguf_gemv(Q4_K, act, L["down"], None, h, HID, FFN, 1)

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                ctx.set_stream(s.cuda_stream)
                fn()
        ctx.use_torch_stream()
        torch.cuda.synchronize()
        return g

    def replay_ms(g):
        """One replay of g bracketed by synchronisations, timed with HIP
        events on torch's stream (the replay's launch stream)."""
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    if args.calib:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).normal_()
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.leg:
        # one GEMV shape alone, for per-dispatch counters (FETCH_SIZE /
        # WRITE_SIZE): Q8_0 or Q4_K at Llama-3-8B gate/up, Q4_K down, the
        # Q8_0 gate+up pair, or the Qwen2.5-0.5B Q8_0 tied head with its
        # argmax (f16 x)
        if args.leg.startswith("q4_k_gemm_m"):
            # config 4's prefill dequant-GEMM at one token count (X bf16, Y fp32)
            m = int(args.leg[len("q4_k_gemm_m"):])
            gbufs = [torch.from_numpy(synth.weights(Q4_K, 300, 0.02, FFN, HID)).to(dev)]
            gbufs += [gbufs[0].clone() for _ in range(11)]
            gslab = torch.empty(32 << 20, dtype=torch.uint8, device=dev)
            gx = torch.from_numpy(synth.normal(301, 1.0, m * HID)).to(dev).to(torch.bfloat16).reshape(m, HID)
            gy = torch.empty((m, FFN), device=dev)
            for i in range(args.steps):
                ctx.gguf_gemm_slab(Q4_K, gx, gbufs[i % len(gbufs)], gy, m, FFN, HID, gslab)
            torch.cuda.synchronize()
            return
        n, k = {"q8_0_head_151936x896": (151936, 896), "q4_k_4096x14336": (HID, FFN)}.get(args.leg, (FFN, HID))
        pair = args.leg == "q8_0_pair"
        t = Q4_K if args.leg.startswith("q4_k") else Q8_0
        copies = [torch.from_numpy(synth.weights(t, 400 + i, 0.02, n, k)).to(dev) for i in range(2 if pair else 1)]
        copies = [c.clone() for c in copies for _ in range(6)]
        if args.leg == "q8_0_head_151936x896":
            xs = torch.from_numpy(synth.normal(9, 1.0, k)).to(dev).half()
            ys = torch.empty(n, device=dev, dtype=torch.float16)
            slot = torch.zeros(1, dtype=torch.int64, device=dev)
        else:
            xs = torch.from_numpy(synth.normal(9, 1.0, k)).to(dev)
            ys = torch.empty(n, device=dev)
        for i in range(args.steps):
            if pair:
                ctx.gguf_gemv_swiglu(Q8_0, xs, copies[(2 * i) % len(copies)], copies[(2 * i + 1) % len(copies)],
                                     None, None, ys, n, k)
            elif args.leg == "q8_0_head_151936x896":
                ctx.gguf_gemv_argmax(Q8_0, xs, None, 0.0, copies[i % len(copies)], ys, n, k, slot)
            else:
                ctx.gguf_gemv(t, xs, copies[i % len(copies)], None, ys, n, k, 0)
        torch.cuda.synchronize()
        return

    # eager pass first (loads kernels, checks arguments)
    for L in layers[:2]:
        layer(L)
    torch.cuda.synchronize()
    # exactly --steps layer steps per replay (step i runs layer copy i % 32),
    # and a --warmup-step graph run once before timing
    g_steps = capture(lambda: [layer(layers[i % N_LAYERS]) for i in range(args.steps)])
    if args.warmup > 0:
        g_warm = capture(lambda: [layer(layers[i % N_LAYERS]) for i in range(args.warmup)])
        g_warm.replay()
        torch.cuda.synchronize()
        del g_warm
    t0 = time.perf_counter()
    rep_ms = [replay_ms(g_steps) for _ in range(args.repeats)]
    wall = time.perf_counter() - t0
    steps = args.steps
    ms = float(np.median(rep_ms))
    ms_per_step = ms / steps
    value = step_bytes * steps / (ms / 1e3) / 1e9
    del g_steps

    # ---- per-shape us/call: a graph of back-to-back calls, replayed
    # --repeats times, median per call.  Cold: the calls cycle over copies
    # of the weight (more bytes than the 256 MB last-level cache); hot: every
    # call reads one buffer.
    def time_calls(launch, bufs, calls=64, reps=None):
        g = capture(lambda: [launch(bufs[i % len(bufs)]) for i in range(calls)])
        g.replay()
        torch.cuda.synchronize()
        us = [replay_ms(g) * 1e3 / calls for _ in range(reps or args.repeats)]
        return float(np.median(us))

    per_shape = {}
    read_us = {}
    read_cfg = {}
    SWEEP_SHAPES = ("q4_k 14336x4096 (gate/up)", "q8_0 14336x4096 (gate/up)", "q4_k 4096x4096 (q/o)")
    hot_us = {}
    gemm_flops = {}
    # the roofline kernel: fused gate+up SwiGLU, cold over the 32 layers
    pair_bytes = 2 * wbytes(Q4_K, FFN, HID) + 4 * HID + 4 * FFN
    pair_us = time_calls(lambda L: ctx.gguf_gemv_swiglu(Q4_K, h, L["gate"], L["up"], None, None, act, FFN, HID),
                         layers)
    per_shape["q4_k gate+up swiglu 2x14336x4096"] = (pair_us, pair_bytes)
    hot_us["q4_k gate+up swiglu 2x14336x4096"] = time_calls(
        lambda L: ctx.gguf_gemv_swiglu(Q4_K, h, L["gate"], L["up"], None, None, act, FFN, HID), layers[:1])
    # the plain streaming-read rate of the same byte count, measured the same
    # way (cold copies, graph replay): what any kernel can reach here
    rbytes = 2 * wbytes(Q4_K, FFN, HID)
    rbufs = [torch.empty(rbytes + 16, dtype=torch.uint8, device=dev) for _ in range(12)]
    for b in rbufs:
        b.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    # read-ceiling sweep: loads in flight per lane, load width, registers or
    # LDS (global_load_lds_dwordx4) and workgroups per CU; a GEMV is held
    # against the best of them (cima_hip_stream_read_cfg)
    READ_CFGS = [(0, 2, 16, 2), (0, 4, 16, 1), (0, 4, 16, 2), (0, 4, 16, 4), (0, 8, 16, 1), (0, 8, 16, 2),
                 (0, 16, 16, 1), (0, 8, 8, 2), (0, 16, 8, 2), (1, 4, 16, 2), (1, 8, 16, 1), (1, 16, 16, 1)]

    def cfg_name(c):
        return (f"reg {c[1]}x{c[2]}B" if c[0] == 0 else f"lds ring {c[1]} KB/wave") + f", {c[3]} wg/CU"

    def read_best(bufs, nb, calls=64, keep=None):
        best = None
        for c in READ_CFGS:
            us = time_calls(lambda b: ctx.stream_read_cfg(b, nb, sink, *c), bufs, calls=calls)
            if keep is not None:
                keep[cfg_name(c)] = round(us, 3)
            if best is None or us < best[0]:
                best = (us, cfg_name(c))
        return best

    read_sweep = {}
    pair_read_us, pair_read_cfg = read_best(rbufs, rbytes, keep=read_sweep.setdefault("q4_k 2x14336x4096 (66 MB)", {}))
    del rbufs
    # the device's sustained read bandwidth, re-measured: the same read kernel
    # over 1 GiB transfers (two buffers, so nothing is served from cache)
    pbytes = 1 << 30
    pbufs = [torch.empty(pbytes, dtype=torch.uint8, device=dev) for _ in range(2)]
    for b in pbufs:
        b.fill_(1)
    peak_us = time_calls(lambda b: ctx.stream_read(b, pbytes, sink), pbufs, calls=8)
    peak_measured = pbytes / peak_us / 1e3
    del pbufs
    torch.cuda.empty_cache()
    if not args.no_shapes:
        def shape_leg(name, t, n, k, copies_mb=600):
            w = synth.weights(t, 200 + n % 97, 0.02, n, k)
            ncopy = max(2, int(np.ceil(copies_mb * 1e6 / w.nbytes)))
            bufs = [torch.from_numpy(w).to(dev) for _ in range(ncopy)]
            xs = torch.from_numpy(synth.normal(9, 1.0, k)).to(dev)
            ys = torch.empty(n, device=dev)
            calls = 64  # the copies are cycled, so each call still reads cold weights
            us = time_calls(lambda b: ctx.gguf_gemv(t, xs, b, None, ys, n, k, 0), bufs, calls=calls)
            per_shape[name] = (us, wbytes(t, n, k) + 4 * (n + k))
            hot_us[name] = time_calls(lambda b: ctx.gguf_gemv(t, xs, b, None, ys, n, k, 0), bufs[:1], calls=calls)
            # the best streaming-read time of the same weight bytes, same method
            rb = w.nbytes // 16 * 16
            read_us[name], read_cfg[name] = read_best(bufs, rb, calls=calls, keep=read_sweep.setdefault(
                f"{w.nbytes / 1e6:.1f} MB", {}) if name in SWEEP_SHAPES else None)
            return us
        for nm, (n, k) in [("q4_k 6144x4096 (q|k|v)", (HID + 2 * KV, HID)),
                           ("q4_k 14336x4096 (gate/up)", (FFN, HID)), ("q4_k 4096x14336 (down)", (HID, FFN)),
                           ("q4_k 4096x4096 (q/o)", (HID, HID)), ("q4_k 1024x4096 (k/v)", (KV, HID))]:
            shape_leg(nm, Q4_K, n, k)
        # Q8_0 at the same Llama-3-8B layer shapes
        for nm, (n, k) in [("q8_0 14336x4096 (gate/up)", (FFN, HID)), ("q8_0 4096x14336 (down)", (HID, FFN)),
                           ("q8_0 4096x4096 (q/o)", (HID, HID))]:
            shape_leg(nm, Q8_0, n, k)
        shape_leg("q8_0 4864x896 (config 1)", Q8_0, 4864, 896)

        # bitsandbytes NF4 (blocksize 64, folded f32 absmax, f16 x / y) at the same shapes
        def nf4_leg(name, n, k, bs=64, copies_mb=600):
            g = torch.Generator(device=dev)
            g.manual_seed(n + k)
            nb = n * k // 2 + n * k // bs * 4  # packed nibbles + absmax, one buffer
            ncopy = max(2, int(np.ceil(copies_mb * 1e6 / nb)))
            bufs = []
            for _ in range(ncopy):
                b = torch.randint(0, 256, (nb,), dtype=torch.uint8, device=dev, generator=g)
                b[n * k // 2:].view(torch.float32).uniform_(0.01, 0.05, generator=g)
                bufs.append(b)
            qm = torch.from_numpy(nf4.NF4_CODE).to(dev)
            xs = torch.from_numpy(synth.normal(9, 1.0, k)).to(dev).half()
            ys = torch.empty(n, device=dev, dtype=torch.float16)
            calls = 64
            us = time_calls(lambda b: ctx.nf4_gemv(xs, b, b[n * k // 2:].view(torch.float32), qm, ys, n, k, bs),
                            bufs, calls=calls)
            per_shape[name] = (us, nb + 2 * (n + k))
            hot_us[name] = time_calls(lambda b: ctx.nf4_gemv(xs, b, b[n * k // 2:].view(torch.float32), qm, ys, n, k,
                                                             bs), bufs[:1], calls=calls)
            read_us[name], read_cfg[name] = read_best(bufs, nb // 16 * 16, calls=calls)
        for nm, (n, k) in [("nf4 14336x4096 (gate/up)", (FFN, HID)), ("nf4 4096x14336 (down)", (HID, FFN)),
                           ("nf4 4096x4096 (q/o)", (HID, HID))]:
            nf4_leg(nm, n, k)
        nf4_leg("nf4 128256x4096 (head)", 128256, HID, copies_mb=900)
        shape_leg("q6_k 128256x4096 (config 3 head)", Q6_K, 128256, HID, copies_mb=900)
        # config 4: prefill dequant-GEMM on MFMA, Q4_K 14336x4096, X bf16 (m tokens), Y fp32
        gw = synth.weights(Q4_K, 300, 0.02, FFN, HID)
        gbufs = [torch.from_numpy(gw).to(dev) for _ in range(12)]
        # the prefill entry point of the engine (cima_hip_gguf_gemm_slab, with
        # the reference's 32 MiB scratch): the fused MFMA kernels
        gslab = torch.empty(32 << 20, dtype=torch.uint8, device=dev)
        for m in (16, 128, 512):
            gx = torch.from_numpy(synth.normal(301, 1.0, m * HID)).to(dev).to(torch.bfloat16).reshape(m, HID)
            gy = torch.empty((m, FFN), device=dev)
            us = time_calls(lambda b: ctx.gguf_gemm_slab(Q4_K, gx, b, gy, m, FFN, HID, gslab), gbufs, calls=24)
            b = wbytes(Q4_K, FFN, HID) + 2 * m * HID + 4 * m * FFN
            per_shape[f"q4_k gemm 14336x4096 m={m} (config 4)"] = (us, b)
            hot_us[f"q4_k gemm 14336x4096 m={m} (config 4)"] = time_calls(
                lambda b: ctx.gguf_gemm_slab(Q4_K, gx, b, gy, m, FFN, HID, gslab), gbufs[:1], calls=24)
            gemm_flops[f"q4_k gemm 14336x4096 m={m} (config 4)"] = 2.0 * FFN * HID * m
        del gbufs
        # the same prefill over bitsandbytes NF4 weights (blocksize 64): the
        # MFMA tiles decode the packed weight themselves
        nn, kk, bs = FFN, HID, 64
        nb = nn * kk // 2 + nn * kk // bs * 4
        g = torch.Generator(device=dev)
        g.manual_seed(5)
        nbufs = []
        for _ in range(12):
            b = torch.randint(0, 256, (nb,), dtype=torch.uint8, device=dev, generator=g)
            b[nn * kk // 2:].view(torch.float32).uniform_(0.01, 0.05, generator=g)
            nbufs.append(b)
        qm = torch.from_numpy(nf4.NF4_CODE).to(dev)
        for m in (16, 128, 512):
            gx = torch.from_numpy(synth.normal(302, 1.0, m * HID)).to(dev).to(torch.bfloat16).reshape(m, HID)
            gy = torch.empty((m, FFN), device=dev)
            leg = f"nf4 gemm 14336x4096 m={m} (bitsandbytes prefill)"
            fn = lambda b: ctx.nf4_gemm_slab(gx, b, b[nn * kk // 2:].view(torch.float32), qm, gy, m, nn, kk, bs, gslab)  # noqa: E731
            per_shape[leg] = (time_calls(fn, nbufs, calls=24), nb + 2 * m * HID + 4 * m * FFN)
            hot_us[leg] = time_calls(fn, nbufs[:1], calls=24)
            gemm_flops[leg] = 2.0 * FFN * HID * m
        del nbufs
        # the Q8_0 gate+up pair (the direct-to-LDS streaming kernels)
        q8g = synth.weights(Q8_0, 310, 0.02, FFN, HID)
        q8u = synth.weights(Q8_0, 311, 0.02, FFN, HID)
        qb = [(torch.from_numpy(q8g).to(dev), torch.from_numpy(q8u).to(dev)) for _ in range(6)]
        xq = torch.from_numpy(synth.normal(9, 1.0, HID)).to(dev)
        yq = torch.empty(FFN, device=dev)
        fn = lambda b: ctx.gguf_gemv_swiglu(Q8_0, xq, b[0], b[1], None, None, yq, FFN, HID)  # noqa: E731
        per_shape["q8_0 gate+up swiglu 2x14336x4096"] = (time_calls(fn, qb, calls=24),
                                                         2 * wbytes(Q8_0, FFN, HID) + 4 * (HID + FFN))
        hot_us["q8_0 gate+up swiglu 2x14336x4096"] = time_calls(fn, qb[:1], calls=24)
        del qb

    shapes_out = {}
    for name, (us, b) in per_shape.items():
        shapes_out[name] = {"us_per_call": round(us, 3), "gb_s": round(b / us / 1e3, 1),
                            "hbm_frac": round(b / us / 1e3 / PEAK_HBM_GBS, 4),
                            "frac_of_measured_peak": round(b / us / 1e3 / peak_measured, 4), "bytes": b}
        if name in hot_us:
            shapes_out[name]["hot_us_per_call"] = round(hot_us[name], 3)
        if name in read_us:
            shapes_out[name]["read_ceiling_us"] = round(read_us[name], 3)
            shapes_out[name]["read_ceiling_cfg"] = read_cfg[name]
            shapes_out[name]["frac_of_read_ceiling"] = round(read_us[name] / us, 4)
        if name in gemm_flops:
            tf = gemm_flops[name] / us / 1e6
            shapes_out[name].update({"tflop_s": round(tf, 1), "mfma_frac_f16_dense": round(tf / 2500.0, 4)})
            shapes_out[name]["route"] = "fused MFMA"

    achieved = pair_bytes / pair_us / 1e3
    traffic = None
    tf = os.path.join(ROOT, "profiles", "gemv_q4k_swiglu_traffic.txt")
    if os.path.exists(tf):
        for line in open(tf):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":")[1]))
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                "kernel": "cima_gemv_q4_k_r1_i1_f32_ring_pair", "alg_bytes_per_launch": pair_bytes,
                "avg_launch_us": round(pair_us, 3),
                "hot_us": round(hot_us["q4_k gate+up swiglu 2x14336x4096"], 3),
                "read_ceiling_gb_s": round(rbytes / pair_read_us / 1e3, 1), "read_ceiling_cfg": pair_read_cfg,
                "frac_of_read_ceiling": round(achieved / (rbytes / pair_read_us / 1e3), 4),
                "peak_measured_gb_s": round(peak_measured, 1),
                "frac_of_measured_peak": round(achieved / peak_measured, 4),
                "peak_measured_how": "cima_stream_read over 1 GiB, two buffers cycled, graph replay, median"}

    # ---- config 5: whole greedy decode step of a Qwen2.5-0.5B-shaped Q8_0
    # model, KV prefilled to 2048, one graph replay per token
    decode = None
    if not args.no_decode:
        from cima_amd.decoder import DecoderConfig, DeviceDecoder, synthetic_kv, synthetic_model

        dcfg = DecoderConfig()
        dm = synthetic_model(dcfg, seed=5)
        dd = DeviceDecoder(ctx, dm)
        ctx_len = 2048
        for i in range(dcfg.n_layers):
            dd.load_kv(i, *synthetic_kv(dcfg, i, ctx_len))
        wbytes_tok = dm.embed.nbytes + sum(sum(v.nbytes for v in L.values() if isinstance(v, np.ndarray))
                                           for L in dm.layers)
        del dm
        def time_tokens(run, stream, n):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(n):
                run()
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / n

        # per-launch (no graph) for reference, then the captured step
        dd.set_state(1, ctx_len)
        for _ in range(10):
            dd.step()
        eager_ms = time_tokens(dd.step, torch.cuda.current_stream(), 50)
        dd.set_state(1, ctx_len)
        dd.capture()
        for _ in range(20):
            dd.replay()
        torch.cuda.synchronize()
        p0 = dd.position()
        # --repeats timed runs of decode_tokens / repeats tokens each; median
        per_rep = max(1, args.decode_tokens // args.repeats)
        tok_ms = [time_tokens(dd.replay, dd.stream, per_rep) for _ in range(args.repeats)]
        dms = float(np.median(tok_ms))
        assert dd.position() == p0 + per_rep * args.repeats
        kv_bytes = dcfg.n_layers * 2 * dcfg.kv_heads * dcfg.head_dim * 2 * (p0 + args.decode_tokens // 2)
        decode = {"workload": "qwen2.5-0.5b-shaped Q8_0 greedy decode step (24 layers, tied 151936 head), "
                              "KV prefilled to 2048, one hipGraph replay per token (5 launches/layer + 3)",
                  "tok_s": round(1e3 / dms, 1), "ms_per_token": round(dms, 4), "tokens": per_rep * args.repeats,
                  "ms_per_token_min_max": [round(min(tok_ms), 4), round(max(tok_ms), 4)],
                  "repeats": args.repeats, "tokens_per_repeat": per_rep,
                  "tok_s_without_graph": round(1e3 / eager_ms, 1),
                  "context": [p0, p0 + per_rep * args.repeats],
                  "bytes_per_token": wbytes_tok + kv_bytes,
                  "gb_s": round((wbytes_tok + kv_bytes) / dms / 1e6, 1)}
        del dd
        torch.cuda.empty_cache()

    # ---- CPU baseline: the reference's host path on a bounded sample
    cpu = None
    if not args.no_cpu:
        import oracle

        xh = x.cpu().numpy()
        actn = synth.normal(10, 1.0, FFN)
        order = [("q", xh), ("k", xh), ("v", xh), ("o", xh), ("gate", xh), ("up", xh), ("down", actn)]
        t0 = time.perf_counter()
        for _ in range(args.cpu_steps):
            for name, xin in order:
                n, k = shapes[name]
                oracle.gguf_gemv_packed(Q4_K, host[name], xin, n, k, threads=1)
        cpu_s = time.perf_counter() - t0
        # the same sample on every host core this process may use (at most
        # 16, the box's CPU share per GPU), rows split over OpenMP threads
        ncores = min(16, len(os.sched_getaffinity(0)))
        t0 = time.perf_counter()
        for _ in range(args.cpu_steps):
            for name, xin in order:
                n, k = shapes[name]
                oracle.gguf_gemv_packed(Q4_K, host[name], xin, n, k, threads=ncores)
        mt_s = time.perf_counter() - t0
        # dequant only (the reference's dequant_host, src/quant.rs:578-597):
        # one 14336 x 4096 Q4_K matrix decoded to f16, single thread
        dq_us = []
        for _ in range(5):
            t0 = time.perf_counter()
            oracle.dequant(Q4_K, host["gate"], FFN * HID)
            dq_us.append((time.perf_counter() - t0) * 1e6)
        cpu_model = "unknown"
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        cpu = {"value": round(step_bytes * args.cpu_steps / cpu_s / 1e9, 4), "unit": "GB/s", "cores": 1,
               "kind": "port",
               "sample": f"{args.cpu_steps} layer steps (same 7 Q4_K GEMVs, same weights), single thread, "
                         f"{cpu_s:.1f} s; oracle/gguf_oracle.c decode-to-f16 + fp32 dot",
               "ms_per_step": round(cpu_s * 1e3 / args.cpu_steps, 1),
               "cpu_model": cpu_model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
               "dequant_only": {"us_per_call": round(float(np.median(dq_us)), 1), "cores": 1,
                                "sample": "oracle dequant of one Q4_K 14336x4096 matrix to f16, median of 5"},
               "all_cores": {"value": round(step_bytes * args.cpu_steps / mt_s / 1e9, 4), "unit": "GB/s",
                             "cores": ncores, "ms_per_step": round(mt_s * 1e3 / args.cpu_steps, 1),
                             "sample": f"the same {args.cpu_steps} layer steps, rows over {ncores} threads, "
                                       f"{mt_s:.1f} s"}}

    out = {
        "metric": "dequant-GEMV µs/call + % HBM roofline (Q4_K/Q8_0, 8B shapes); decode tok/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x int16 fixed-point activations, int32 dot, fp32 scale",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q4_K, x ~ N(0,1))",
        "config": {"workload": "llama-3-8b decoder layer decode GEMVs, batch 1, Q4_K: q|k|v (one 6144x4096 "
                               "matrix), o(+residual), gate+up SwiGLU fused, down(+residual); 32 distinct layers "
                               "cycled (cold HBM), hipGraph replay",
                   "bytes_per_step": step_bytes, "layers_cycled": N_LAYERS,
                   "hbm_frac_of_8TBs": round(value / PEAK_HBM_GBS, 4),
                   "wall_s": round(wall, 3), "repeats": args.repeats,
                   "ms_per_step_min_max": [round(min(rep_ms) / steps, 5), round(max(rep_ms) / steps, 5)],
                   "timing": "median of --repeats graph replays of exactly --steps layer steps"},
        "shapes": shapes_out,
        "read_ceiling_sweep_us": read_sweep,
        "decode_step": decode,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
