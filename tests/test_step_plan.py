"""CPU enumeration check of the persistent decode-step kernel's index math.

tests/cpu/step_plan_check.cpp includes axiomlm_amd/csrc/step_plan.h -- the functions
the kernel itself calls for every offset it forms -- and walks whole launches at the
C1 / smoke shapes, a wide GQA-2 group-128 model, the 7B layer shape (group 128 and 64,
4096 slots, 256 and 80 CUs) and a GQA 8:1 model with a 49152-token vocabulary.  Every
offset is asserted inside its buffer and used to read a host buffer of exactly that
size, built with AddressSanitizer; chunk, row, unit and key-split coverage is checked.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpu", "step_plan_check.cpp")
INC = os.path.join(ROOT, "axiomlm_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_step_plan_offsets_in_bounds_under_asan(tmp_path):
    exe = str(tmp_path / "step_plan_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", f"-I{INC}",
                    SRC, "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.count("ok ") == 7, res.stdout
