"""The C-ABI from plain C: include/kvx.h compiles as C11 (-pedantic) and a C
client (tests/c_abi_client.c) linked against libkvx.so runs the reference's
known answers for block accessors, pools, copy specs, wire bytes and the
allocator. CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_c11_client_links_and_runs(kvx, tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lib_dir = os.path.dirname(kvx.library_path())
    exe = tmp_path / "c_abi_client"
    extra = []
    if os.environ.get("KVX_LIBRARY"):
        # A sanitizer build: its runtime comes from LD_PRELOAD (inherited by
        # the client below), not from the link.
        extra = ["-Wl,--allow-shlib-undefined"]
    subprocess.run([cc, "-std=c11", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c_abi_client.c"), "-o", str(exe),
                    "-L", lib_dir, "-lkvx", f"-Wl,-rpath,{lib_dir}", *extra],
                   check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "c client ok" in r.stdout
