"""The host-pointer path's parallel host memcpy (tomoul_amd/csrc/host_copier.hpp)
under ThreadSanitizer: tests/c/test_host_copier.cpp copies buffers of many
sizes, offsets and from several requesting threads, and checks every byte.
CPU only; skipped without g++."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
@pytest.mark.parametrize("sanitizer", ["thread", "address,undefined"])
def test_host_copier(tmp_path, sanitizer):
    exe = tmp_path / "host_copier"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-pthread", f"-fsanitize={sanitizer}", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "tomoul_amd", "csrc"), os.path.join(ROOT, "tests", "c", "test_host_copier.cpp"),
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = {**os.environ, "TSAN_OPTIONS": "halt_on_error=1", "ASAN_OPTIONS": "detect_leaks=0"}
    p = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "host copier ok" in p.stdout
    assert "WARNING: ThreadSanitizer" not in p.stderr, p.stderr
