"""The C-ABI library loads without a GPU and exports every function that
include/kvx.h declares; the ctypes prototypes cover exactly that set."""
import os
import re
import shutil
import subprocess

import pytest

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


def test_device_address_checks_refuse_before_issue(tmp_path):
    """Entry points that take raw device addresses refuse host, unknown,
    managed, wrong-device and overrunning ones with INVALID_ARGUMENT before
    anything is issued (tests/device_address_check.cc drives the C-ABI with
    a made-up address map in place of the HIP runtime's lookup). GPUs are
    hidden from the program: none of its calls may reach a device."""
    cxx = shutil.which("g++") or shutil.which("c++")
    libdir = os.path.join(ROOT, "tpu-sync_amd")
    if cxx is None or not os.path.exists(os.path.join(libdir, "libkvx.so")):
        pytest.skip("no C++ compiler or libkvx.so not built")
    exe = tmp_path / "device_address_check"
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    env.update(HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run([cxx, "-O1", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", "-I", os.path.join(ROOT, "include"),
                        "-I", os.path.join(ROOT, "tpu-sync_amd", "csrc", "host"),
                        os.path.join(ROOT, "tests", "device_address_check.cc"), "-o", str(exe),
                        "-L", libdir, "-lkvx", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout
