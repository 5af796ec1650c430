"""Build the integration driver: every ```cpp block of INTEGRATION.md, as the
document shows it, compiled and linked with driver.cpp against the built
libkvmem_hip.so and the oracle's liboracle.so.

The blocks are written to _gen/block_<n>.cpp (one translation unit each, so a
block that does not compile on its own fails here) and the program to
_bin/integration_driver, whose run path finds both libraries relative to
itself.  Host code only: g++ with the HIP runtime headers, no GPU code.
"""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
PKG = ROOT / "kvmem-llama.cpp_amd"
ORACLE = ROOT / "oracle"
GEN = HERE / "_gen"
BIN = HERE / "_bin" / "integration_driver"
ROCM = Path("/opt/rocm")

CXX = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
       f"-I{ROOT / 'include'}", f"-I{ORACLE}", f"-I{ROCM / 'include'}"]


def blocks(doc: Path = ROOT / "INTEGRATION.md") -> list[str]:
    """The ```cpp fenced blocks of the document, in order."""
    return re.findall(r"^```cpp\n(.*?)^```", doc.read_text(), re.S | re.M)


def build(gen: Path = GEN, out: Path = BIN) -> Path:
    for lib in (PKG / "libkvmem_hip.so", ORACLE / "liboracle.so"):
        if not lib.exists():
            raise RuntimeError(f"{lib} is not built")
    gen.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    srcs = []
    for i, text in enumerate(blocks()):
        src = gen / f"block_{i}.cpp"
        src.write_text(text)
        srcs.append(src)
    if len(srcs) < 6:
        raise RuntimeError(f"INTEGRATION.md holds {len(srcs)} cpp blocks, the driver calls six")
    objs = []
    for src in [*srcs, HERE / "driver.cpp"]:
        obj = gen / (src.stem + ".o")
        r = subprocess.run([*CXX, "-c", str(src), "-o", str(obj)], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compiling {src.name} failed:\n{r.stderr}")
        objs.append(obj)
    rpath = ":".join(["$ORIGIN/../../../kvmem-llama.cpp_amd", "$ORIGIN/../../../oracle", str(ROCM / "lib")])
    tmp = out.with_suffix(".tmp")
    cmd = ["g++", "-o", str(tmp), *map(str, objs),
           f"-L{PKG}", "-lkvmem_hip", f"-L{ORACLE}", "-loracle", f"-L{ROCM / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,{rpath}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"linking the integration driver failed:\n{r.stderr}")
    tmp.replace(out)
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
