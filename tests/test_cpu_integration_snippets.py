"""The C ABI as a C or C++ caller sees it (no GPU needed).

- Every struct of include/kvmem_hip.h and include/kvmem_host.h: sizeof and
  the offset of every member, printed by a C program compiled from the
  headers, equal the ctypes mirrors the Python view and the tests use.
  A member the mirror names that the header lacks fails the compile.
- Every C++ block of INTEGRATION.md (the calls an adapter would make)
  compiles against the headers, and links against libkvmem_hip.so.
- The integration driver (tests/integration_driver), which runs those
  blocks on the GPU against the oracle, builds from them.
"""
from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from conftest import PKG_DIR, ROOT, load_pkg

kv = load_pkg()
from kvmem_amd import host  # noqa: E402

INCLUDE = ROOT / "include"
STRUCTS = {
    "kvmem_hip_reserve_args": kv.ReserveArgs, "kvmem_hip_scratch": kv.Scratch,
    "kvmem_hip_quant_op": kv.QuantOp, "kvmem_hip_history": kv.History,
    "kvmem_hip_transform": kv.Transform, "kvmem_hip_pool": kv.Pool,
    "kvmem_hip_host_history": kv.HostHistory, "kvmem_hip_packed_host": kv.PackedHost,
    "kvmem_hip_score_args": kv.ScoreArgs, "kvmem_hip_meank_args": kv.MeanKArgs,
    "kvmem_hip_perf": kv.Perf, "kvmem_plan_stats": host.PlanStats,
    "kvmem_engine_params": host.EngineParams, "kvmem_row_range": host.RowRange,
    "kvmem_attention_view": host.AttentionViewC, "kvmem_hip_transfer_stats": kv.TransferStats,
}


def header_structs() -> set[str]:
    names = set()
    for h in INCLUDE.glob("*.h"):
        names |= set(re.findall(r"typedef struct (kvmem_\w+)\s*\{", h.read_text()))
    return names


def test_every_header_struct_has_a_mirror():
    assert header_structs() == set(STRUCTS), header_structs() ^ set(STRUCTS)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_struct_layouts_match_the_ctypes_mirrors(tmp_path):
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "kvmem_host.h"', "int main(void) {"]
    for name, cls in STRUCTS.items():
        lines.append(f'    printf("{name} size %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'    printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines += ["    return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{INCLUDE}", str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, field, value = line.split()
        got[(name, field)] = int(value)
    for name, cls in STRUCTS.items():
        assert got[(name, "size")] == __import__("ctypes").sizeof(cls), name
        for field, _ in cls._fields_:
            assert got[(name, field)] == getattr(cls, field).offset, (name, field)


def test_perf_stage_bits_match_the_header():
    text = (INCLUDE / "kvmem_hip.h").read_text()
    bits = dict(re.findall(r"#define KVMEM_PERF_STAGE_(\w+) (\d+)u", text))
    assert len(bits) >= 8
    for name, value in bits.items():
        assert getattr(kv, f"PERF_STAGE_{name}") == int(value), name


def snippets() -> list[str]:
    text = (ROOT / "INTEGRATION.md").read_text()
    return re.findall(r"```cpp\n(.*?)```", text, flags=re.S)


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_integration_snippets_compile_and_link(tmp_path):
    blocks = snippets()
    assert len(blocks) >= 5
    objs = []
    for i, code in enumerate(blocks):
        src = tmp_path / f"snippet{i}.cpp"
        src.write_text(code)
        obj = tmp_path / f"snippet{i}.o"
        r = subprocess.run(["g++", "-std=c++17", "-fPIC", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                            f"-I{INCLUDE}", "-I/opt/rocm/include", "-c", str(src), "-o", str(obj)],
                           capture_output=True, text=True)
        assert r.returncode == 0, f"INTEGRATION.md block {i}:\n{r.stderr}"
        objs.append(str(obj))
    # every symbol the snippets call resolves in the library
    lib = PKG_DIR / "libkvmem_hip.so"
    r = subprocess.run(["g++", "-shared", "-o", str(tmp_path / "snippets.so"), *objs, str(lib),
                        "-Wl,--no-undefined", "-L/opt/rocm/lib", "-lamdhip64"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_integration_driver_builds(tmp_path):
    import importlib.util
    spec = importlib.util.spec_from_file_location("integration_driver_build",
                                                  ROOT / "tests" / "integration_driver" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert len(mod.blocks()) == len(snippets())
    exe = mod.build(tmp_path / "gen", tmp_path / "bin" / "integration_driver")
    assert exe.exists()
