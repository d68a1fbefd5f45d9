"""The pageable lanes' host copy pool (csrc/host/host_copy_pool.cc) built from
the source with the host compiler and checked byte for byte; the second build
runs under ThreadSanitizer, which fails the run on any data race in the
pool's batch handoffs. CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "tpu-sync_amd", "csrc", "host")


@pytest.mark.parametrize("sanitize", [False, True], ids=["plain", "tsan"])
def test_host_copy_pool(tmp_path, sanitize):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no C++ compiler")
    exe = tmp_path / "host_copy_pool_check"
    flags = ["-O1", "-g", "-fsanitize=thread", "-DKVX_CHECK_LIGHT"] if sanitize else ["-O2"]
    # Neither the compiler nor the check inherits a sanitizer runtime preloaded
    # into this process (the library's sanitizer targets do that).
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    r = subprocess.run([cxx, *flags, "-std=c++17", "-Wall", "-Werror", "-pthread", "-I", HOST,
                        os.path.join(ROOT, "tests", "host_copy_pool_check.cc"),
                        os.path.join(HOST, "host_copy_pool.cc"),
                        os.path.join(HOST, "stream_copy.cc"), "-o", str(exe)],
                       capture_output=True, text=True, env=env)
    if sanitize and r.returncode != 0 and "tsan" in (r.stderr + r.stdout).lower():
        pytest.skip("no ThreadSanitizer runtime for the host compiler")
    assert r.returncode == 0, r.stderr
    env["TSAN_OPTIONS"] = "halt_on_error=1:exitcode=66"
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "host copy pool ok" in run.stdout
