"""bench.py's command line on a machine without a GPU: it measures one GPU
only and says so for any other count, and its headline line carries every
key of the one-line JSON contract (checked on the source, since producing
the line needs the GPU)."""
from __future__ import annotations

import ast
import os
import subprocess
import sys

from conftest import ROOT

BENCH = ROOT / "bench.py"


def run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, str(BENCH), *args], capture_output=True, text=True, env=e,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    for args, env in ((["--gpus", "2"], None), (["--gpus", "8"], None), ([], {"WORLD_SIZE": "2"})):
        r = run(args, env)
        assert r.returncode == 2, (args, env, r.returncode)
        assert "one GPU" in r.stderr
        assert r.stdout == ""


def test_help_lists_the_workloads():
    r = run(["--help"])
    assert r.returncode == 0
    for w in ("reselect_256k", "mixed_precision", "recall_1m", "cache_transform", "meank_256k"):
        assert w in r.stdout


def headline_keys() -> set[str]:
    """String keys of the dict literal that run_reselect_256k names `result`."""
    tree = ast.parse(BENCH.read_text())
    fn = next(n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == "run_reselect_256k")
    for node in ast.walk(fn):
        if (isinstance(node, ast.Assign) and any(isinstance(t, ast.Name) and t.id == "result"
                                                  for t in node.targets)
                and isinstance(node.value, ast.Dict)):
            return {k.value for k in node.value.keys if isinstance(k, ast.Constant)}
    raise AssertionError("no result dict in run_reselect_256k")


def test_headline_line_carries_the_contract_keys():
    keys = headline_keys()
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in keys, k
    src = BENCH.read_text()
    # added to the line after the dict is built
    assert 'result["cpu_baseline"]' in src
    # the roofline object's fields
    for k in ('"bound"', '"achieved"', '"peak"', '"unit"', '"frac"', '"traffic"'):
        assert k in src, k


def test_calibration_program_is_built_and_checks_its_size():
    """build() makes kvmem-llama.cpp_amd/calib/hbm_rates, which
    `bench.py --workload copy_calibration` runs; a size that is not a
    positive multiple of 16 MiB is refused before any device call."""
    exe = ROOT / "kvmem-llama.cpp_amd" / "calib" / "hbm_rates"
    assert exe.exists(), "build first"
    for arg in ("17", "0", "-16", "131072"):
        r = subprocess.run([str(exe), arg], capture_output=True, text=True, timeout=60)
        assert r.returncode == 2, (arg, r.returncode, r.stderr)
        assert "multiple of 16 MiB" in r.stderr
