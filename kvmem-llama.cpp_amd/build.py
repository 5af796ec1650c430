"""Build libkvmem_hip.so (gfx950) in-tree, and the CPU oracle beside it.

    python kvmem-llama.cpp_amd/build.py            # library + oracle (+ _ref)
    python kvmem-llama.cpp_amd/build.py --lib-only

The library is compiled with hipcc for gfx950 only.  Every HIP translation
unit disables packed-FP32 instruction selection, and the stage-in unit
disables FP contraction (ggml's reference quantizers round products and sums
separately).  Host C++ units (csrc/*.cpp) are compiled by hipcc in C++ mode so that one
shared object carries both the device ABI (include/kvmem_hip.h) and the host
mirror of the reference's store / runtime / reselect interface
(include/kvmem_host.h).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ = PKG / "_build"
LIB = PKG / "libkvmem_hip.so"
ORACLE = ROOT / "oracle"
REFERENCE = Path("/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-fPIC", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}",
          "-fvisibility=hidden", "-Wall", "-Wno-unused-result"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-x", "hip",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-fno-gpu-flush-denormals-to-zero"]
# per-file extras
EXTRA = {
    "stagein.hip": ["-ffp-contract=off"],
    "score.hip": ["-ffinite-math-only"],
    "meank.hip": ["-ffp-contract=off"],
}


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = OBJ / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *HIP_FLAGS, *COMMON, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", *COMMON,
               "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build_lib(jobs: int = 8, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, warn in results:
        if verbose and warn.strip():
            print(warn, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results], "-Wl,-Bsymbolic", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


CALIB_SRC = PKG / "calib" / "hbm_rates.hip"
CALIB_BIN = PKG / "calib" / "hbm_rates"


def build_calib() -> Path:
    """The plain streaming kernels that give this device's reachable HBM
    read, write and copy rates (bench.py --workload copy_calibration)."""
    tmp = CALIB_BIN.with_suffix(".tmp")
    cmd = [HIPCC, *HIP_FLAGS, "-O3", "-std=c++17", "-Wall", str(CALIB_SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"calibration build failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CALIB_BIN)
    return CALIB_BIN


def build_oracle(with_ref: bool = True) -> None:
    make = shutil.which("make") or "make"
    r = subprocess.run([make, "-s", "-C", str(ORACLE), "all"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{r.stdout}\n{r.stderr}")
    if with_ref and (REFERENCE / "kvmem" / "src" / "host" / "kvmem_store.cpp").exists():
        r = subprocess.run([make, "-s", "-C", str(ORACLE), "ref", f"REFROOT={REFERENCE}"],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"reference kvmem build failed\n{r.stdout}\n{r.stderr}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    build_lib(a.jobs, a.verbose)
    if not a.lib_only:
        build_calib()
        build_oracle()
    print(f"built {LIB}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
