"""The host store, runtime and slot pool (csrc/kvmem_store.{hpp,cpp}) under
AddressSanitizer and UndefinedBehaviorSanitizer.

tests/store_fuzz.cpp is built with g++ next to csrc/kvmem_store.cpp and run
over three seeds: 40 random configurations each (block size, budget, sink,
recent, tie rule, forced reload, pool size), 400 random operations per
configuration (history appends, resident appends, truncations, reselects over
random scores with mandatory blocks, commits, attention views and the
continuation checks), the store's invariants checked after every operation.
The reference's own host tests drive the same classes with recorded sequences
(kvmem/tests/kvmem_store_test.cpp, kvmem_runtime_test.cpp).
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "kvmem-llama.cpp_amd" / "csrc"


@pytest.fixture(scope="module")
def store_fuzz(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path_factory.mktemp("store_fuzz") / "store_fuzz"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", f"-I{CSRC}", str(ROOT / "tests" / "store_fuzz.cpp"),
           str(CSRC / "kvmem_store.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_store_sequences_under_sanitizers(store_fuzz, seed):
    r = subprocess.run([str(store_fuzz), str(seed), "40", "400"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.startswith("ok"), (seed, r.stdout, r.stderr[-3000:])
