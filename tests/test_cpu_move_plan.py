"""The slot-move planner on the CPU: the host C++ that cuts a canonical
layout's moves into chain segments (kvmem-llama.cpp_amd/csrc/move_plan.cpp),
compiled here with g++ beside a fuzz driver (tests/move_plan_fuzz.cpp) that
replays the segments as the device kernel runs them and compares with
"read every source, then write every destination" (the gather/scatter of
layout_gpu_slots_by_orig_pos, llama-memory-kvmem.cpp:1003-1093)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "kvmem-llama.cpp_amd" / "csrc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_move_plan_fuzz(tmp_path):
    exe = tmp_path / "move_plan_fuzz"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{CSRC}", str(ROOT / "tests" / "move_plan_fuzz.cpp"),
                    str(CSRC / "move_plan.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe), "20000"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    cases, refused, bad = (int(x) for x in r.stdout.split()[1::2])
    assert bad == 0 and cases == 20000 and 0 < refused < cases
