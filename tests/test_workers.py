"""The staging worker pool (sym_amd/csrc/workers.cpp) under ThreadSanitizer:
tests/native/workers_stress.cpp built with g++ and run on the CPU."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "sym_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workers_visit_every_element_once_under_tsan(tmp_path):
    exe = str(tmp_path / "workers_stress")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=thread", "-pthread", "-I" + CSRC,
           os.path.join(HERE, "native", "workers_stress.cpp"), os.path.join(CSRC, "workers.cpp"),
           "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok" in r.stdout
