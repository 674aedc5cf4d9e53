"""The halo conv's load / barrier schedule (k_conv3_sched.h) replayed on the
host by tests/conv3_schedule_check.cpp for every tile width and 1..48
channel chunks: reads only of completed loads, buffer refills only after a
barrier that follows the last read, wait counts within vmcnt's range; the
checker also proves it detects a schedule with too little waiting."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_halo_conv_schedule(tmp_path):
    exe = tmp_path / "conv3_schedule_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    "-I", os.path.join(REPO, "draw-instant_amd", "csrc"),
                    os.path.join(REPO, "tests", "conv3_schedule_check.cpp"), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
