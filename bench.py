"""Reselect benchmark: one KVMem agent step at 256K context on one MI355X.

Workload (the full reselect step at 256K, 16 attention layers):
  history  K, V [16 layers][2048 blocks][128 tokens][4 KV heads][256] f16,
           device resident (K = N(0,1) + per-(layer, block) offset N(0, 0.3^2)
           per channel, V = N(0,1)), seeded, synthetic
  query    Q [16][64 tokens][24 heads][256] bf16, GQA group 6
  pool     256 + 128 slots of 128 cells per layer, K and V q8_0
  step     score every block (per-token max of q.k/16, mean over layers) ->
           top-256 with block 0 kept as sink, ascending -> diff against the
           resident selection -> stage-in of the changed blocks (77 of 256,
           ~30 %) quantized to q8_0 into the slots the outgoing blocks free.
Each timed step starts from the same previous selection: between timed
steps an untimed restore re-applies it (the same stage-in path).

Prints ONE JSON line.  `value` is ms per agent step (lower is better) with
history and query resident in HBM.  `roofline` is the MFMA block scorer
(the dominant kernel); `stagein_roofline` the q8_0 stage-in kernel against
HBM; `pinned_host` the same stage-in fed over PCIe from pinned host memory;
`cpu_baseline` the oracle's restatement of the step on the host cores.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG_DIR = ROOT / "kvmem-llama.cpp_amd"

L, B, T, HKV, HQ, D, TQ = 16, 2048, 128, 4, 24, 256, 64
E = HKV * D
BUDGET = 256            # blocks (32K tokens)
RESERVE = 128           # generation reserve blocks (16K tokens)
N_SLOTS = BUDGET + RESERVE
N_CHANGED = round(0.3 * BUDGET)   # 77

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
PCIE_PEAK_GBS = 64.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "kvmem_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["kvmem_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def make_engine(kv, torch, k, v):
    """The reselect engine over the device-resident history (C++ host store
    + slot plan, gfx950 kernels)."""
    from kvmem_amd import host
    eng = host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                      budget_blocks=BUDGET, reserve_blocks=RESERVE, sink_blocks=1, recent_blocks=0,
                      type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q8_0, tie_lower_index=1,
                      layer_reduce=kv.LAYER_MEAN)
    eng.set_device_history(k.data_ptr(), v.data_ptr(), B, B * T)
    return eng


def make_previous(sel: list[int], seed: int = 7) -> list[int]:
    """The previous step's selection: N_CHANGED seeded blocks of `sel`
    (never the sink) swapped for seeded blocks outside it."""
    rng = np.random.default_rng(seed)
    cur = np.array(sel)
    drop = rng.choice(cur[cur != 0], N_CHANGED, replace=False)
    outside = np.setdiff1d(np.arange(B), cur)
    add = rng.choice(outside, N_CHANGED, replace=False)
    return sorted(set(sel) - set(drop.tolist()) | set(add.tolist()))


# ------------------------------------------------------------ cpu baseline
def cpu_baseline(torch, k, v, q, sel_ids: list[int], budget_s: float = 12.0) -> dict:
    """The oracle's restatement of the step on the host cores: fp32 per-token
    max scorer (OpenMP) on a sample of blocks, sort-based top-k, and the
    reference q8_0 quantizer over a sample of the staged blocks (thread
    pool), each scaled to the full step."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import kvmem_oracle as oracle

    threads = min(16, len(os.sched_getaffinity(0)))
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    qf = q.float().cpu().numpy()

    def host_blocks(t, ids):
        idx = torch.tensor(ids, dtype=torch.long, device=t.device)
        return t[:, idx].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

    # scoring: probe 8 blocks, then a sample sized to ~budget_s * 0.8
    probe = host_blocks(k, list(range(8)))
    t0 = time.perf_counter()
    oracle.score_pertoken_max_f32(qf, probe, 0, 8, threads)
    per_block = (time.perf_counter() - t0) / 8
    n_sample = int(min(B, max(16, (0.8 * budget_s) / max(per_block, 1e-6))))
    sample_ids = list(range(0, B, max(1, B // n_sample)))[:n_sample]
    ks = host_blocks(k, sample_ids)
    t0 = time.perf_counter()
    ls = oracle.score_pertoken_max_f32(qf, ks, 0, len(sample_ids), threads)
    score_s = (time.perf_counter() - t0) * B / len(sample_ids)
    del ks
    # top-k over a full score vector (the sampled ones tiled)
    sc = np.resize(ls.mean(axis=0).astype(np.float64), B)
    t0 = time.perf_counter()
    oracle.pick_topk(sc, BUDGET, sink=1)
    topk_s = time.perf_counter() - t0
    # stage-in quantize: 8 staged blocks x 16 layers x K/V, thread pool
    n_q = min(8, len(sel_ids))
    kb = host_blocks(k, sel_ids[:n_q])
    vb = host_blocks(v, sel_ids[:n_q])
    jobs = [(src[l, i].reshape(T, E)) for src in (kb, vb) for l in range(L) for i in range(n_q)]
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda r: oracle.quantize_rows_f16(oracle.TYPE_Q8_0, r), jobs))
    quant_s = (time.perf_counter() - t0) * N_CHANGED / n_q
    total_ms = (score_s + topk_s + quant_s) * 1e3
    return {
        "value": round(total_ms, 1), "unit": "ms/step", "cores": threads, "kind": "port",
        "sample": (f"fp32 per-token max scorer on {len(sample_ids)} of {B} blocks x {L} layers "
                   f"(OpenMP, {threads} threads) scaled x{B / len(sample_ids):.1f}; top-256 over "
                   f"{B} scores; q8_0 quantize of {n_q} of {N_CHANGED} staged blocks x {L} layers "
                   f"x K/V ({threads} threads) scaled x{N_CHANGED / n_q:.2f}"),
        "parts_ms": {"score": round(score_s * 1e3, 1), "topk": round(topk_s * 1e3, 3),
                     "quantize": round(quant_s * 1e3, 1)},
    }


# --------------------------------------------------------- pinned host mode
def pinned_host_mode(kv, ctx, torch, k, v, eng, incoming: list[int], reps: int = 3) -> dict:
    """Stage-in of the changed blocks from pinned host memory (block-major
    [block][layer][K rows, V rows]) through the copy stream and device ring
    into free slots of the engine's pool."""
    n = len(incoming)
    span_el = L * 2 * T * E
    host = torch.empty((n, span_el), dtype=torch.float16, pin_memory=True)
    idx = torch.tensor(incoming, dtype=torch.long, device="cuda")
    kk = k[:, idx].permute(1, 0, 2, 3, 4).reshape(n, L, T * E)
    vv = v[:, idx].permute(1, 0, 2, 3, 4).reshape(n, L, T * E)
    host.copy_(torch.cat([kk, vv], dim=2).reshape(n, span_el).cpu())
    del kk, vv
    hh = kv.HostHistory(host.data_ptr(), L, n, T, E, E, 0)
    used = set(s for s in eng.block_slots() if s >= 0)
    slots = [s for s in range(eng.n_slots()) if s not in used][:n]
    assert len(slots) == n
    layers = [eng.pool_layer(l) for l in range(L)]
    pool = ctx.make_pool(L, eng.n_slots(), T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                         [p[0] for p in layers], [p[1] for p in layers])
    ctx.stagein_blocks_host(hh, pool, list(range(n)), slots)   # warm the ring
    ctx.sync()
    best = None
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ctx.stagein_blocks_host(hh, pool, list(range(n)), slots)
        ctx.sync()
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    h2d = n * span_el * 2
    return {"ms": round(best * 1e3, 3), "h2d_bytes": h2d, "h2d_GBs": round(h2d / best / 1e9, 2),
            "link_peak_GBs": PCIE_PEAK_GBS, "frac": round(h2d / best / 1e9 / PCIE_PEAK_GBS, 3)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pinned", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the reselect path runs on a single MI355X "
              "(multi-GPU sharding is described in DESIGN.md, not run)", file=sys.stderr)
        return 2

    import torch
    kv = load_pkg()
    from kvmem_amd import host, workloads

    log("generating history K/V [16][2048][128][4][256] f16 and query [16][64][24][256] bf16")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=2, with_v=True)
    torch.cuda.synchronize()
    eng = make_engine(kv, torch, k, v)
    ctx = kv.Context.borrow(eng.ctx_handle())

    sel = eng.preview(q.data_ptr(), TQ).blocks
    prev = make_previous(sel)

    def restore():
        """Apply the previous step's selection (untimed between steps)."""
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))

    restore()
    changed = len(set(sel) - set(prev))
    log(f"selection {len(sel)} blocks, {changed} changed vs previous step")

    def step() -> dict:
        return eng.apply_retrieval(q.data_ptr(), TQ)

    for _ in range(a.warmup):
        step()
        restore()
    ctx.perf_enable(True)
    times, staged, score_ms, set_ms, sel_ms = [], [], 0.0, 0.0, 0.0
    for _ in range(a.steps):
        ctx.perf_reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st = step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        pf = ctx.perf()
        score_ms += pf["score_ms"]
        set_ms += pf["set_ms"]
        sel_ms += pf["topk_ms"]
        staged.append(st["n_staged"])
        restore()
    ctx.perf_enable(False)
    K = a.steps
    ms_step = 1e3 * sum(times) / K
    score_ms /= K
    set_ms /= K
    sel_ms /= K
    n_staged = staged[0]
    assert all(x == n_staged for x in staged), staged
    log(f"step {ms_step:.3f} ms: score kernel {score_ms:.3f} ms, combine+top-k {sel_ms:.3f} ms, "
        f"stage-in kernel {set_ms:.3f} ms ({n_staged} blocks)")

    flops = 2.0 * TQ * HQ * D * (B * T) * L
    k_bytes = L * B * T * E * 2
    score_tflops = flops / (score_ms * 1e-3) / 1e12
    stage_bytes = n_staged * L * 2 * (T * E * 2 + T * kv.row_size(kv.TYPE_Q8_0, E))
    stage_gbs = stage_bytes / (set_ms * 1e-3) / 1e9

    result = {
        "metric": "reselect latency ms/agent-step @256K ctx; stage-in GB/s vs HBM peak",
        "value": round(ms_step, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16/bf16->f32 scoring, f16->q8_0 stage-in",
        "data": "synthetic (seeded N(0,1) keys with per-block offsets, bf16 query)",
        "config": {"workload": "full reselect step @256K: 16 layers x 2048 blocks x 128 tokens, "
                               "4 KV heads x 256, 64-token query x 24 heads (GQA 6), top-256 + sink, "
                               f"{n_staged} changed blocks -> q8_0 K/V pool of 256+128 slots",
                   "history": "device-resident", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "score_kernel<256>",
                     "achieved": round(score_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(score_tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": None, "algorithmic_bytes": k_bytes, "flops": flops,
                     "hbm_GBs_algorithmic": round(k_bytes / (score_ms * 1e-3) / 1e9, 1)},
        "stagein_roofline": {"bound": "hbm", "kernel": "quant_scatter_kv_kernel<q8_0,q8_0>",
                             "achieved": round(stage_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(stage_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                             "algorithmic_bytes": stage_bytes, "kernel_ms": round(set_ms, 4)},
        "parts_ms": {"score_kernel": round(score_ms, 4), "combine_topk": round(sel_ms, 4),
                     "stagein_kernel": round(set_ms, 4)},
    }
    if not a.no_pinned:
        incoming = sorted(set(sel) - set(prev))
        result["pinned_host"] = pinned_host_mode(kv, ctx, torch, k, v, eng, incoming)
    if not a.no_cpu_baseline:
        log("cpu baseline (oracle restatement on host cores)")
        result["cpu_baseline"] = cpu_baseline(torch, k, v, q, sorted(set(sel) - set(prev)))
    eng.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
