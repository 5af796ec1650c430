"""The C-ABI library loads on a machine without a GPU and exports every
function include/*.h declares (no compute call is made here)."""
from __future__ import annotations

import re
import subprocess

from conftest import PKG_DIR, ROOT, load_pkg

LIB = PKG_DIR / "libkvmem_hip.so"


def declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"KVMEM_HIP_API\s+[^;{]*?\b(kvmem_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_path():
    names = declared_functions()
    for required in ("kvmem_hip_create", "kvmem_hip_score", "kvmem_hip_topk", "kvmem_hip_stagein_blocks",
                     "kvmem_hip_stagein_blocks_host", "kvmem_hip_stagein_quant", "kvmem_engine_preview",
                     "kvmem_engine_apply", "kvmem_engine_apply_retrieval", "kvmem_store_pick_topk",
                     "kvmem_store_apply"):
        assert required in names


def test_library_exports_every_declared_symbol():
    kv = load_pkg()
    lib = kv.load_library()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_no_unexpected_exports():
    """Every exported kvmem_* symbol is declared in a header."""
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T kvmem_" in line}
    assert exported <= declared_functions(), sorted(exported - declared_functions())


def test_host_only_calls_without_gpu():
    kv = load_pkg()
    lib = kv.load_library()
    assert lib.kvmem_hip_row_size(kv.TYPE_Q8_0, 1024) == 1088
    assert lib.kvmem_hip_row_size(kv.TYPE_Q5_0, 1024) == 704
    assert lib.kvmem_hip_row_size(kv.TYPE_Q4_0, 1024) == 576
    assert lib.kvmem_hip_row_size(kv.TYPE_Q8_0, 1000) == 0
    assert lib.kvmem_hip_quant_ok(kv.TYPE_Q5_0) == 1 and lib.kvmem_hip_quant_ok(3) == 0
    assert lib.kvmem_hip_last_error(None) == b"null context"
    assert lib.kvmem_hip_sync(None) == kv.ERR_INVALID
