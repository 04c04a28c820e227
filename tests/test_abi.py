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


def header_prototypes():
    """{name: (return kind, [argument kinds])} from include/hipinfer.h, in the Python module's kinds:
    pointers are ptr, except char pointers (strings) str; long long i64; size_t size."""
    src = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "hipinfer.h")).read(), flags=re.S)

    def kind(decl):
        decl = decl.replace("const ", "").strip()
        if "char*" in decl.replace(" ", ""):
            return "str"
        if "*" in decl:
            return "ptr"
        t = decl.split()[0]
        return {"long": "i64", "size_t": "size", "int": "int", "float": "float", "void": "void"}[t]

    out = {}
    for m in re.finditer(r"(?m)^([A-Za-z_][\w* ]*?)\s*\b(hi_\w+)\s*\(([^)]*)\)\s*;", src):
        args = [a for a in m.group(3).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(2)] = (kind(m.group(1)), [kind(a) for a in args])
    return out


def test_host_mirror_binds_the_header_prototypes():
    """The Python module's prototype table (its ctypes argtypes / restype) is the header's, symbol
    for symbol and argument for argument."""
    from hipinfer_amd import hipinfer
    hdr = header_prototypes()
    assert set(hipinfer.SIGNATURES) == set(hdr)
    for name, sig in hdr.items():
        assert hipinfer.SIGNATURES[name] == sig, name
        assert getattr(hipinfer.lib, name).argtypes is not None


def test_interleave_gate_up_layout():
    """Rows 32j .. 32j+15 are gate rows 16j .., rows 32j+16 .. 32j+31 the same up rows (the reference
    exporter's layout, export.py:97-101), on the CPU (no GPU needed)."""
    import torch
    from hipinfer_amd import hipinfer
    I, H = 48, 3
    g = torch.arange(I * H, dtype=torch.float32).reshape(I, H)
    u = -g - 1
    f = hipinfer.interleave_gate_up(g, u)
    for r in range(2 * I):
        grp, i = divmod(r, 32)
        src = g if i < 16 else u
        assert torch.equal(f[r], src[grp * 16 + i % 16])


def test_product_path_never_loads_the_oracle():
    """Nothing under hipinfer_amd/ imports, links or names the oracle library."""
    for dirpath, _, files in os.walk(os.path.join(ROOT, "hipinfer_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), f"{f} mentions the oracle"
    out = subprocess.run(["ldd", LIB], capture_output=True, text=True).stdout
    assert "oracle" not in out
