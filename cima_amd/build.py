"""Build recipe for the native parts of cima_amd (runs on a CPU-only host).

Produces, in ``cima_amd/lib/``:
  cima_gemv_a/b/c.hsaco  gfx950 code objects (hipcc --genco): decode GEMVs,
  cima_gemm.hsaco       prefill dequant-GEMMs (MFMA),
  cima_dequant.hsaco    dequant-to-f16 and packed gather,
  cima_decode.hsaco     decode-step support (norm, RoPE, attention, argmax)
  cima_bnb4.hsaco       bitsandbytes NF4/FP4 dequant and decode GEMV
  libcima_hip.so      host C ABI (include/cima_hip.h), links libamdhip64
  libcima_synth.so    seeded synthetic weights + quantisers (include/cima_synth.h)

``python -m cima_amd.build`` rebuilds everything.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# code object -> (HIP source, defines); the GEMVs are split over three code
# objects by format set so that they compile in parallel
SOURCES = {"gemv_a": ("gguf_gemv.hip", ["-DCIMA_GEMV_SET=0"]), "gemv_b": ("gguf_gemv.hip", ["-DCIMA_GEMV_SET=1"]),
           "gemv_c": ("gguf_gemv.hip", ["-DCIMA_GEMV_SET=2"]), "gemm": ("gguf_gemm.hip", []),
           "dequant": ("gguf_dequant.hip", []), "decode": ("decode_ops.hip", []),
           "bnb4": ("bnb4.hip", [])}
HSACOS = {name: os.path.join(LIB, f"cima_{name}.hsaco") for name in SOURCES}
GEMV_OBJECTS = ("gemv_a", "gemv_b", "gemv_c")
LIBHIP = os.path.join(LIB, "libcima_hip.so")
LIBSYNTH = os.path.join(LIB, "libcima_synth.so")

# Device code: gfx950 only.  Packed-FP32 VALU ops are disabled (they have
# produced silently wrong results on this hardware pool).  No implicit FP
# contraction: the dequantisers must round exactly like the host decoders
# (a fused f32->f16 multiply would drop the sign of -0 and the intermediate
# f32 rounding of Q4_K); the GEMV code asks for its FMAs explicitly.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _cmds():
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    return {
        **{path: [hipcc, *HIPCC_FLAGS, *SOURCES[name][1], f"-I{CSRC}", "--genco", "-o", path,
                  os.path.join(CSRC, SOURCES[name][0])]
           for name, path in HSACOS.items()},
        LIBHIP: ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__",
                 f"-I{INCLUDE}", f"-I{ROCM}/include", os.path.join(CSRC, "cima_hip.cpp"),
                 f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl", "-o", LIBHIP],
        LIBSYNTH: ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-Wall", f"-I{INCLUDE}",
                   os.path.join(CSRC, "gguf_synth.cpp"), "-o", LIBSYNTH],
    }


STAMP = os.path.join(LIB, "build.stamp")


def source_hash() -> str:
    """Hash of everything the native artefacts are built from: the sources
    and headers under csrc/ and include/, and the compile commands."""
    h = hashlib.sha256()
    for d in (CSRC, INCLUDE):
        for name in sorted(os.listdir(d)):
            path = os.path.join(d, name)
            if os.path.isfile(path):
                h.update(name.encode())
                with open(path, "rb") as f:
                    h.update(f.read())
    # the commands with the checkout's own path taken out, so a copy of the
    # tree at another path (a GPU host's scratch directory) hashes the same
    for cmd in _cmds().values():
        h.update(" ".join(cmd).replace(ROOT, "<root>").encode())
    return h.hexdigest()


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> None:
    """Compile every native artefact (always recompiles)."""
    os.makedirs(LIB, exist_ok=True)
    cmds = _cmds()
    if os.path.exists(STAMP):
        os.remove(STAMP)
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        outs = list(ex.map(_run, cmds.values()))
    with open(STAMP, "w") as f:
        f.write(source_hash() + "\n")
    if verbose:
        for o in outs:
            if o.strip():
                print(o, file=sys.stderr)


def built() -> bool:
    """True when every artefact exists (whether or not it is current)."""
    return all(os.path.exists(p) for p in (*HSACOS.values(), LIBHIP, LIBSYNTH))


def current() -> bool:
    """True when the artefacts were built from the sources as they are now
    (the stamp written by build() matches source_hash())."""
    if not (built() and os.path.exists(STAMP)):
        return False
    with open(STAMP) as f:
        return f.read().strip() == source_hash()


def ensure() -> None:
    """Load what is built: compile only when an artefact is missing, and warn
    (without rebuilding) when the sources changed since the last build."""
    if not built():
        build()
    elif not current():
        print("cima_amd: the native artefacts predate the sources under csrc/ or include/; "
              "run python -m cima_amd.build to rebuild them", file=sys.stderr)


if __name__ == "__main__":
    build(verbose=True)
    print("built:", *HSACOS.values(), LIBHIP, LIBSYNTH)
