"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
exactly the entry points include/kansai_hip.h declares, and the Python
binding covers all of them.  No compute call is made (no GPU here)."""

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kansai_hip.h")
LIB = os.path.join(ROOT, "kansaiml_amd", "lib", "libkansai_hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kh_[a-z0-9_]+)\s*\(", text))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T kh_" in line}


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_exports_every_declared_symbol():
    d = declared()
    assert len(d) >= 25
    missing = d - exported()
    assert not missing, f"declared but not exported: {sorted(missing)}"
    extra = exported() - d
    assert not extra, f"exported but not declared: {sorted(extra)}"


def test_binding_covers_header():
    from kansaiml_amd import _native
    assert set(_native.exported_symbols()) == declared()


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_loads_and_resolves_symbols():
    from kansaiml_amd import _native
    lib = _native.load_library()
    for name in _native.exported_symbols():
        assert getattr(lib, name) is not None


def test_product_package_never_imports_oracle():
    """The product path has no CPU fallback: nothing under kansaiml_amd/
    imports, loads or names the oracle."""
    pkg = os.path.join(ROOT, "kansaiml_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in src.lower(), f"{f} mentions the oracle"
