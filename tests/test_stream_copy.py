"""The bounce lanes' host copy (csrc/host/stream_copy.cc) against memcpy, with
each of its two bodies (32-byte and 16-byte streaming stores), built from the
source with the host compiler. CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tpu-sync_amd", "csrc", "host")


@pytest.mark.parametrize("avx2", ["true", "false"])
def test_stream_copy_matches_memcpy(tmp_path, avx2):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no C++ compiler")
    if avx2 == "true":
        with open("/proc/cpuinfo") as f:
            if " avx2" not in f.read():
                pytest.skip("this CPU has no AVX2")
    exe = tmp_path / "stream_copy_check"
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    subprocess.run([cxx, "-O2", "-std=c++17", "-Wall", "-Werror", "-I", HOST,
                    f"-DKVX_STREAM_COPY_AVX2={avx2}",
                    os.path.join(ROOT, "tests", "stream_copy_check.cc"),
                    os.path.join(HOST, "stream_copy.cc"), "-o", str(exe)],
                   check=True, capture_output=True, text=True, env=env)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "stream copy ok" in r.stdout
