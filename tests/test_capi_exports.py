"""The C-ABI library loads without a GPU and exports every function that
include/kvx.h declares; the ctypes prototypes cover exactly that set."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(inc, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(kvx_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_header_symbols_exported(kvx):
    lib = kvx._capi.load()
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", kvx.library_path()],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names <= exported


def test_prototypes_match_header(kvx):
    assert set(kvx._capi.PROTOTYPES) == declared_functions()


def test_version_and_last_error(kvx):
    lib = kvx._capi.load()
    assert b"gfx950" in lib.kvx_version()
    assert lib.kvx_future_await(None) == 3
    assert "null" in kvx._capi.last_error()
