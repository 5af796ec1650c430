"""The C++ blocks of INTEGRATION.md, run on the GPU as an adapter would call
them: tests/integration_driver/driver.cpp links the blocks as the document
shows them with libkvmem_hip.so and checks every result against the oracle's
C library (bit-exact pool rows, scores within 1e-3 / 1e-5, the engine's
selections equal to the oracle's top-k).  The driver is built by
__graft_entry__.build() (tests/integration_driver/build.py) and runs here as a
child process."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "integration_driver" / "_bin" / "integration_driver"


@pytest.mark.gpu
def test_integration_blocks_on_gpu():
    assert BIN.exists(), f"{BIN} is not built: run __graft_entry__.build()"
    print("running the integration driver", flush=True)
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.rstrip().endswith("[driver] ok"), r.stdout
    assert r.stdout.count("[driver] kvmem_") == 6, r.stdout
