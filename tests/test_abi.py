"""CPU tests of the product's host side: the C ABI exports, format tables,
the synthetic quantisers (decoded by the oracle), and loud failure without
a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from cima_amd import gguf, synth
from cima_amd import hip as hipmod
from cima_amd import build as cbuild

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FORMATS = list(gguf.DType)


def header_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(cima_\w+)\s*\(", text)


@pytest.mark.parametrize("header,lib", [("cima_hip.h", cbuild.LIBHIP), ("cima_synth.h", cbuild.LIBSYNTH)])
def test_library_exports_every_declared_symbol(header, lib):
    names = header_functions(os.path.join(ROOT, "include", header))
    assert names, header
    L = ctypes.CDLL(lib)
    for n in names:
        assert hasattr(L, n), f"{os.path.basename(lib)} does not export {n}"


def test_python_binding_covers_header():
    names = header_functions(os.path.join(ROOT, "include", "cima_hip.h"))
    assert set(names) == set(hipmod.EXPORTS)


def test_code_object_holds_every_kernel():
    blobs = {}
    for name, path in cbuild.HSACOS.items():
        blob = open(path, "rb").read()
        assert blob[:4] == b"\x7fELF" or blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
        assert b"gfx950" in blob
        blobs[name] = blob
    gemv = b"".join(blobs[o] for o in cbuild.GEMV_OBJECTS)
    for f in [t.name.lower() for t in FORMATS]:
        blob = gemv
        for r, it in ((1, 1), (1, 2), (1, 4), (1, 8), (2, 1), (2, 2), (2, 4)):
            for a in ("f32", "f16"):
                for sfx in ("", "_epi", "_pair", "_pair_epi") + (("_att_epi", "_amax") if a == "f16" else ()):
                    assert f"cima_gemv_{f}_r{r}_i{it}_{a}{sfx}".encode() in blob
        for it in (1, 2):
            for rk in ("_f32_ring", "_f32_ring_epi", "_f16_ring", "_f16_ring_epi", "_f16_ring_amax"):
                assert f"cima_gemv_{f}_r1_i{it}{rk}".encode() in blob
        for rk in ("_f32_ringl", "_f32_ringl_epi", "_f16_ringl", "_f16_ringl_epi"):
            assert f"cima_gemv_{f}_r1_i1{rk}".encode() in blob
        assert f"cima_dequant_{f}".encode() in blobs["dequant"]
        assert f"cima_gather_{f}".encode() in blobs["dequant"]
        for bn in (16, 32, 64, 128):
            for xt in ("f32", "f16", "bf16"):
                for yt in ("f32", "f16"):
                    assert f"cima_gemm_{f}_b{bn}_{xt}_{yt}".encode() in blobs["gemm"]
                    if bn == 16:
                        assert f"cima_gemm_{f}_b16n_{xt}_{yt}".encode() in blobs["gemm"]


def test_stream_read_kernel_present():
    assert b"cima_stream_read" in open(cbuild.HSACOS["dequant"], "rb").read()


def test_decode_object_holds_every_kernel():
    blob = open(cbuild.HSACOS["decode"], "rb").read()
    names = ["cima_rmsnorm_f16", "cima_rope_f16", "cima_kv_append_f16", "cima_argmax_f16", "cima_argmax_to_ids",
             "cima_pos_bump"]
    names += [f"cima_attn_{k}_d{d}" for k in ("split", "reduce", "decode") for d in (64, 128)]
    for n in names:
        assert n.encode() in blob, n


def test_bnb4_object_holds_every_kernel():
    blob = open(cbuild.HSACOS["bnb4"], "rb").read()
    names = ["cima_nf4_dequant_v", "cima_nf4_dequant_e"]
    names += [f"cima_nf4_gemv_{v}_r{r}_{a}_{a}" for v in ("t", "c") for r in (1, 2, 4) for a in ("f16", "f32")]
    names += [f"cima_nf4_gemv_e_{a}_{a}" for a in ("f16", "f32")]
    for n in names:
        assert n.encode() in blob, n


def test_decoder_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors of cima_decoder / cima_decoder_layer have the C
    layout (compiled with the header by the host compiler)."""
    src = tmp_path / "layout.c"
    fields = [f[0] for f in hipmod.Decoder._fields_]
    lfields = [f[0] for f in hipmod.DecoderLayer._fields_]
    body = "".join(f'printf("%zu ", offsetof(cima_decoder, {f}));' for f in fields)
    body += "".join(f'printf("%zu ", offsetof(cima_decoder_layer, {f}));' for f in lfields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "cima_hip.h"\nint main(void){'
                   + body + 'printf("%zu %zu", sizeof(cima_decoder), sizeof(cima_decoder_layer));return 0;}')
    exe = tmp_path / "layout"
    import subprocess
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(hipmod.Decoder, f).offset for f in fields] + [getattr(hipmod.DecoderLayer, f).offset
                                                                    for f in lfields]
    want += [ctypes.sizeof(hipmod.Decoder), ctypes.sizeof(hipmod.DecoderLayer)]
    assert got == want


def test_error_classification():
    L = hipmod.load_library()
    for c in (700, 702, 710, 713, 719):
        assert L.cima_hip_is_fatal(c) == 1
    for c in (0, 1, 2, 701, 98, -1):
        assert L.cima_hip_is_fatal(c) == 0


def test_null_context_is_rejected():
    L = hipmod.load_library()
    rc = L.cima_hip_gguf_gemv(None, 12, None, None, None, None, 1, 256, 0, 0)
    assert rc == hipmod.E_NOT_INIT
    assert b"not initialised" in L.cima_hip_last_error()
    assert L.cima_hip_gguf_dequant(None, 12, None, None, 1) == hipmod.E_NOT_INIT
    assert L.cima_hip_sync(None) == hipmod.E_NOT_INIT


def test_hipctx_fails_loudly_without_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is present")
    with pytest.raises(hipmod.EngineError):
        hipmod.HipCtx(0)


@pytest.mark.parametrize("t", FORMATS, ids=lambda t: t.name)
def test_format_tables_match_oracle(t):
    assert gguf.block_elems(t) == oracle.BLOCK_ELEMS[t]
    assert t.block_bytes == oracle.BLOCK_BYTES[t]
    for numel in (0, 256, 4096, 14336 * 4096):
        assert gguf.storage_bytes(t, numel) == oracle.storage_bytes(t, numel)
    with pytest.raises(ValueError):
        gguf.storage_bytes(10, 256)


def test_synth_normal_is_deterministic_and_normal():
    a = synth.normal(42, 0.02, 1 << 20, threads=4)
    b = synth.normal(42, 0.02, 1 << 20, threads=1)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    c = synth.normal(43, 0.02, 1 << 10)
    assert not np.array_equal(a[:1024], c)


# relative normwise quantisation error bounds of the synthetic quantisers
QERR = {gguf.DType.Q8_0: 0.01, gguf.DType.Q4_0: 0.2, gguf.DType.Q4_1: 0.12, gguf.DType.Q5_0: 0.08,
        gguf.DType.Q5_1: 0.07, gguf.DType.Q4_K: 0.12, gguf.DType.Q5_K: 0.07, gguf.DType.Q6_K: 0.04,
        gguf.DType.IQ4_XS: 0.12}


@pytest.mark.parametrize("t", FORMATS, ids=lambda t: t.name)
def test_synth_quantisers_roundtrip_through_oracle(t):
    rows, k = 64, 1024
    w = synth.normal(7, 0.02, rows * k).reshape(rows, k)
    packed = synth.quantize(t, w)
    assert packed.shape == (rows, gguf.row_bytes(t, k))
    deq = oracle.f16_bits_to_f32(oracle.dequant(t, packed.reshape(-1), rows * k)).reshape(rows, k)
    err = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert err < QERR[t], err
    # weights() is normal() + quantize() without the fp32 matrix
    assert np.array_equal(synth.weights(t, 7, 0.02, rows, k), packed)


def test_synth_rejects_bad_shapes():
    with pytest.raises(ValueError):
        synth.quantize(12, np.zeros((2, 100), np.float32))
    with pytest.raises(ValueError):
        synth.weights(10, 1, 0.02, 2, 256)


def _kernel_notes(hsaco):
    """(vgpr_count, private_segment_fixed_size) per kernel of a built code
    object, read from its AMDGPU metadata with the ROCm LLVM tools."""
    import shutil
    import subprocess
    import tempfile

    llvm = "/opt/rocm/llvm/bin"
    if not (shutil.which(f"{llvm}/clang-offload-bundler") and shutil.which(f"{llvm}/llvm-readelf")):
        pytest.skip("ROCm LLVM tools not found")
    with tempfile.TemporaryDirectory() as d:
        co = os.path.join(d, "k.co")
        subprocess.run([f"{llvm}/clang-offload-bundler", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={hsaco}", f"--output={co}", "--unbundle"], check=True)
        notes = subprocess.run([f"{llvm}/llvm-readelf", "--notes", co], capture_output=True, text=True,
                               check=True).stdout
    out = {}
    for blk in notes.split("- .agpr_count")[1:]:
        name = re.search(r"\.name:\s+(\S+)", blk).group(1)
        out[name] = (int(re.search(r"\.vgpr_count:\s+(\d+)", blk).group(1)),
                     int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", blk).group(1)))
    return out


def test_hot_gemv_kernels_do_not_spill():
    """The GEMV variants the decode shapes and the benchmark run keep every
    value in registers: a scratch spill is a vector memory access queued
    behind the weight loads in flight, which stalls the x staging."""
    notes = {}
    for o in cbuild.GEMV_OBJECTS:
        notes.update(_kernel_notes(cbuild.HSACOS[o]))
    fmts = [t.name.lower() for t in FORMATS]
    hot = [f"cima_gemv_{f}_r1_i{it}_{a}{sfx}" for f in fmts for it in (1, 2, 4)
           for a in ("f32", "f16") for sfx in ("", "_epi", "_pair")]
    hot += [f"cima_gemv_{f}_r1_i{it}_{a}_ring{e}" for f in fmts for it in (1, 2)
            for a in ("f32", "f16") for e in ("", "_epi")]
    hot += [f"cima_gemv_{f}_r1_i1_{a}_ringl{e}" for f in fmts for a in ("f32", "f16") for e in ("", "_epi")]
    hot += [f"cima_gemv_{f}_r1_i1_f16_{v}" for f in ("q8_0", "q4_k") for v in ("att_epi", "amax", "ring_amax")]
    spills = {k: notes[k] for k in hot if notes[k][1] > 0}
    assert not spills, spills
    notes = _kernel_notes(cbuild.HSACOS["bnb4"])
    spills = {k: v for k, v in notes.items() if (k.startswith("cima_nf4_gemv_t") or k.startswith("cima_nf4_gemv_c")) and v[1] > 0}
    assert not spills, spills


def test_python_binding_checks_every_code_object():
    """HipCtx refuses to start without any of the code objects the build
    writes (the list the C library loads)."""
    assert sorted(hipmod.CODE_OBJECTS) == sorted(cbuild.HSACOS.values())


def test_gemm_kernels_do_not_spill():
    """Every prefill GEMM variant keeps its load ring in registers (a ring
    left in scratch memory -- register pressure, or an aggregate copy the
    compiler does not promote -- turns each stage into scratch traffic)."""
    notes = _kernel_notes(cbuild.HSACOS["gemm"])
    # nine GGUF formats, bitsandbytes 4-bit and f16 weights: six tile kinds
    # x six (x, y) dtype pairs each, plus the six plain f16-weight kernels
    # and the two k-split sums
    assert len(notes) == 11 * 6 * 6 + 6 + 2
    spills = {k: v for k, v in notes.items() if v[1] > 0}
    assert not spills, spills


def test_error_codes_match_header():
    """The Python error-code constants are the header's CIMA_E_* values."""
    from cima_amd import hip as h

    text = open(os.path.join(os.path.dirname(__file__), "..", "include", "cima_hip.h")).read()
    codes = {name: int(v) for name, v in re.findall(r"#define CIMA_(E_[A-Z_]+)\s+(-?\d+)", text)}
    assert codes == {n: getattr(h, n) for n in codes}
    assert set(codes) == {"E_INVALID", "E_FORMAT", "E_NO_KERNEL", "E_NOT_INIT", "E_LIBRARY"}


def test_x_range_flag_arithmetic():
    """The prefill tiles' X range test (XRange in gguf_gemm.hip) is word
    arithmetic on two bf16 halves at once; restated here in numpy and
    checked over all 65536 x 2 half pairs' magnitudes against the
    definition: overflow = |x| >= 65536 or not finite (f16 cannot hold it),
    tiny = 0 < |x| < 2^-17 (f16 may drop its bits)."""
    import numpy as np

    h = np.arange(65536, dtype=np.uint32)
    for lo_fixed in (0x0000, 0x3f80, 0x4780, 0x0001):
        w = (h << 16) | lo_fixed
        a = w & 0x7FFF7FFF
        acc = ((a + 0x38803880) & 0x80008000) | ((~(a + 0x49004900) & (a + 0x7FFF7FFF) & 0x80008000) >> 1)
        acc &= 0xFFFFFFFF
        over = (acc & 0x80008000) != 0
        tiny = (acc & 0x40004000) != 0

        def ok(bits):
            v = (bits.astype(np.uint32) << 16).view(np.float32)
            return (~np.isfinite(v)) | (np.abs(v) >= 65536.0), (v != 0) & (np.abs(v) < 2.0 ** -17)

        o_hi, t_hi = ok(h.astype(np.uint16))
        o_lo, t_lo = ok(np.full(65536, lo_fixed, np.uint16))
        assert np.array_equal(over, o_hi | o_lo)
        assert np.array_equal(tiny, t_hi | t_lo)
    # f32: bit 31 <- |x| >= 65520, the first value f16 rounds to inf
    xs = np.array([65504.0, 65519.99, 65520.0, 1e9, np.inf, -70000.0, 1.0], np.float32)
    f = ((xs.view(np.uint32) & 0x7FFFFFFF) + 0x38801000) & 0x80000000
    assert list(f != 0) == [False, False, True, True, True, True, False]
    assert np.isinf(np.float32(65520.0).astype(np.float16)) and not np.isinf(np.float32(65519.99).astype(np.float16))
