"""The build stamp: a copy of the tree at another path (as on a GPU host)
must count as built from the same sources, so tests, smoke() and bench.py
load the shipped artefacts instead of recompiling them."""
import importlib
import shutil

import cima_amd.build as b


def test_source_hash_is_independent_of_the_checkout_path(tmp_path):
    h0 = b.source_hash()
    root = tmp_path / "elsewhere" / "repo"
    shutil.copytree(b.CSRC, root / "cima_amd" / "csrc")
    shutil.copytree(b.INCLUDE, root / "include")
    mod = importlib.reload(b)
    try:
        mod.ROOT = str(root)
        mod.PKG = str(root / "cima_amd")
        mod.CSRC = str(root / "cima_amd" / "csrc")
        mod.INCLUDE = str(root / "include")
        mod.LIB = str(root / "cima_amd" / "lib")
        mod.HSACOS = {n: str(root / "cima_amd" / "lib" / f"cima_{n}.hsaco") for n in mod.SOURCES}
        mod.LIBHIP = str(root / "cima_amd" / "lib" / "libcima_hip.so")
        mod.LIBSYNTH = str(root / "cima_amd" / "lib" / "libcima_synth.so")
        assert mod.source_hash() == h0
        # a changed source is noticed
        (root / "cima_amd" / "csrc" / "gguf_gemv.hip").write_text("// changed\n")
        assert mod.source_hash() != h0
    finally:
        importlib.reload(b)


def test_ensure_does_not_rebuild_what_exists(monkeypatch):
    calls = []
    monkeypatch.setattr(b, "built", lambda: True)
    monkeypatch.setattr(b, "current", lambda: False)
    monkeypatch.setattr(b, "build", lambda *a, **k: calls.append(1))
    b.ensure()
    assert calls == []
