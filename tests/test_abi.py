"""CPU checks of the C-ABI boundary (no GPU compute): libhipinfer.so is built for gfx950, loads,
and exports every symbol include/hipinfer.h declares -- and nothing else of the hi_ namespace
(reference CI checks its exports the same way, .github/workflows/ci.yml:78: nm -D ... " T hi_").
The host mirror imports without a GPU, and the product path has no CPU fallback."""
import ctypes
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "hipinfer_amd", "libhipinfer.so")


def declared():
    src = open(os.path.join(ROOT, "include", "hipinfer.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hi_\w+)\s*\(", src)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return sorted({l.split()[-1] for l in out.splitlines() if " T hi_" in l})


def test_library_exports_exactly_the_header():
    assert os.path.exists(LIB), "build first: python -m hipinfer_amd.build"
    assert declared() == exported()


def test_library_loads_and_resolves_every_symbol():
    lib = ctypes.CDLL(LIB)
    for name in declared():
        assert getattr(lib, name) is not None


def test_library_holds_gfx950_code_objects():
    blob = open(LIB, "rb").read()
    assert b"gfx950" in blob


def test_host_mirror_imports_and_binds(monkeypatch):
    from hipinfer_amd import hipinfer
    for name in ["hi_gemv", "hi_gemv_w8", "hi_gemv_qkv_rope", "hi_gemv_qkv_rope_w8", "hi_rmsnorm"]:
        assert getattr(hipinfer.lib, name).argtypes is not None


def test_product_path_never_loads_the_oracle():
    """Nothing under hipinfer_amd/ imports, links or names the oracle library."""
    for dirpath, _, files in os.walk(os.path.join(ROOT, "hipinfer_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), f"{f} mentions the oracle"
    out = subprocess.run(["ldd", LIB], capture_output=True, text=True).stdout
    assert "oracle" not in out
