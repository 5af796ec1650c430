"""Reselect benchmark: one KVMem agent step at 256K context on one MI355X.

Workload (the full reselect step at 256K, 16 attention layers):
  history  K, V [16 layers][2048 blocks][128 tokens][4 KV heads][256] f16,
           device resident (K = N(0,1) + per-(layer, block) offset N(0, 0.3^2)
           per channel, V = N(0,1)), seeded, synthetic
  query    Q [16][64 tokens][24 heads][256] bf16, GQA group 6
  pool     256 + 128 slots of 128 cells per layer, K and V q8_0
  step     score every block (per-token max of q.k/16, mean over layers) ->
           top-256 with block 0 kept as sink, ascending -> diff against the
           resident selection and slot plan on the device -> slot moves
           (slot i = i-th selected block) -> stage-in of the changed blocks
           (77 of 256, ~30 %) quantized to q8_0.
Each timed step starts from the same previous selection: between timed
steps an untimed restore re-applies it (the same stage-in path).

Prints ONE JSON line.  `value` is ms per agent step (lower is better) with
history and query resident in HBM, the pool laid out as the reference lays
it out (slot i = i-th selected block), with the HIP timing events of the
two rooflines on (scorer and stage-in); `ms_per_step_no_timing_events` is
the same steps timed again without any event, and
`ms_per_step_all_timing_events` with every stage timed (the source of the
top-k and slot-move parts); `host_planned` is the same step with the diff and slot plan
on the host, `lifo_layout` the same step without the slot moves.  `mixed_precision` (Student-t history, K q8_0 +
V q4_0, then K and V q5_0) and `recall_1m` (8192 blocks, 512-token query,
32 planted blocks, budget 512) are the other workloads' steps, and
`meank_256k` (the reference's own mean-K scorer) and `cache_transform` (RoPE +
attn_rot before q8_0) the same 256K step in its other modes, in the same
line unless --no-configs.  `transfers_per_step` is one step's data movement
per direction (kvmem_hip_transfer_get).  `roofline` is the MFMA block scorer
(the dominant kernel); `stagein_roofline` the q8_0 stage-in kernel against
HBM; `pinned_host` the same stage-in fed over PCIe from pinned host memory,
and the same blocks as packed q8_0 rows copied out to (`packed_stageout`)
and restored from (`packed_stagein`) a pinned packed store, and `step` the
whole reselect step with the F16 history staged from pinned host memory
(the keys also in HBM for the scorer), again with a packed host store
(`with_packed_store`: incoming blocks restored from their q8_0 rows); `cpu_baseline`
the oracle's restatement of the whole step measured on the host cores.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import importlib.util
import json
import os
import subprocess
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
# HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE on this
# workload, scaled by the copy-kernel calibration (profiles/traffic_reselect_256k.md)
SCORE_TRAFFIC_BYTES = 8.597e9 + 2.10e6
STAGEIN_TRAFFIC_BYTES = 6.458e8 + 3.431e8
MFMA_F16_PEAK_TFLOPS = 2500.0
PCIE_PEAK_GBS = 64.0
HOST_CPU_SHARE = 16           # host cores a one-GPU job may use, whatever the node shows


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "kvmem_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["kvmem_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def make_engine(kv, torch, k, v, n_blocks: int = B, budget: int = BUDGET, reserve: int = RESERVE,
                type_k: int | None = None, type_v: int | None = None, **extra):
    """The reselect engine over the device-resident history (C++ host store
    + slot plan, gfx950 kernels)."""
    from kvmem_amd import host
    eng = host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                      budget_blocks=budget, reserve_blocks=reserve, sink_blocks=1, recent_blocks=0,
                      type_k=kv.TYPE_Q8_0 if type_k is None else type_k,
                      type_v=kv.TYPE_Q8_0 if type_v is None else type_v, tie_lower_index=1,
                      layer_reduce=kv.LAYER_MEAN, **extra)
    eng.set_device_history(k.data_ptr(), v.data_ptr(), n_blocks, n_blocks * T)
    return eng


def timed_steps(eng, ctx, torch, q, n_q_tokens: int, prev: list, steps: int, warmup: int) -> dict:
    """`warmup` untimed then `steps` timed agent steps, each from the
    previous selection `prev` (restored, untimed, between steps).  Returns
    mean wall ms per step and the per-stage device ms of the engine stream."""
    import kvmem_amd as kv
    from kvmem_amd import host

    def restore():
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))

    def step() -> dict:
        return eng.apply_retrieval(q.data_ptr(), n_q_tokens)

    restore()
    for _ in range(warmup):
        step()
        restore()
    times, bare, full, staged, moved = [], [], [], [], []
    score_ms = set_ms = sel_ms = layout_ms = after_ms = cos_ms = 0.0
    planned = []
    d2d_bytes = 0
    for _ in range(steps):
        # the timed step: only the scorer and the stage-in carry timing
        # events (each event holds the stream idle a few microseconds),
        # the two the rooflines need
        ctx.perf_stages(kv.PERF_STAGE_SCORE | kv.PERF_STAGE_SET)
        ctx.perf_enable(True)
        ctx.perf_reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st = step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        pf = ctx.perf()
        xfer = ctx.transfers()  # this step's data movement, per direction
        ctx.perf_enable(False)
        score_ms += pf["score_ms"]
        set_ms += pf["set_ms"]
        after_ms += pf["after_score_ms"]
        staged.append(st["n_staged"])
        moved.append(st["n_moved"])
        planned.append(st.get("device_planned", 0))
        restore()
        # the same step without any timing event, interleaved so that every
        # kind sees the same clocks: the step's latency as a caller sees it
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        bare.append(time.perf_counter() - t0)
        restore()
        # and with every stage timed, for the top-k and slot-move parts
        ctx.perf_stages(kv.PERF_STAGE_ALL)
        ctx.perf_enable(True)
        ctx.perf_reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        full.append(time.perf_counter() - t0)
        pf = ctx.perf()
        ctx.perf_enable(False)
        sel_ms += pf["topk_ms"]
        layout_ms += pf["layout_ms"]
        cos_ms += pf["meank_cos_ms"]
        d2d_bytes += pf["d2d_bytes"]
        restore()
    assert all(x == staged[0] for x in staged), staged
    return {"ms_step": 1e3 * sum(times) / steps, "ms_step_no_events": 1e3 * sum(bare) / steps,
            "ms_step_all_events": 1e3 * sum(full) / steps,
            "score_ms": score_ms / steps,
            "set_ms": set_ms / steps, "sel_ms": sel_ms / steps, "n_staged": staged[0],
            "layout_ms": layout_ms / steps, "n_moved": max(moved), "d2d_bytes": d2d_bytes // steps,
            "cos_ms": cos_ms / steps,
            "device_planned": min(planned), "after_score_ms": after_ms / steps, "transfers": xfer}


def stage_bytes(kv, n_blocks: int, type_k: int, type_v: int) -> int:
    """Algorithmic HBM bytes of a stage-in: F16 K and V read once, packed
    rows written once."""
    return n_blocks * L * T * (2 * E * 2 + kv.row_size(type_k, E) + kv.row_size(type_v, E))


# ------------------------------------------------------------ cpu baseline
def cpu_baseline(torch, k, v, q, sel_ids: list[int]) -> dict:
    """The oracle's restatement of the whole step on the host cores, over
    the same inputs, measured in full: the fp32 per-token max scorer
    (OpenMP) on every block of every layer, the sort-based top-k over the
    2048 scores, and the reference q8_0 quantizer on every staged block's K
    and V rows of every layer (thread pool).  Beside it, measured in full
    too: the reference's own mean-K scorer (one thread, as the adapter runs
    it) over every block's key sums, the q8_0 quantizer on one thread, and
    the host memcpy of the staged blocks' packed rows."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import kvmem_oracle as oracle

    visible = len(os.sched_getaffinity(0))
    threads = min(HOST_CPU_SHARE, visible)  # a one-GPU job's share of the host's cores
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    qf = q.float().cpu().numpy()

    def host_blocks(t, ids):
        idx = torch.tensor(ids, dtype=torch.long, device=t.device)
        return t[:, idx].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

    # scoring: every block of every layer (the keys copied to the host first, untimed)
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16)
    t0 = time.perf_counter()
    ls = oracle.score_pertoken_max_f32(qf, kh, 0, B, threads)
    score_s = time.perf_counter() - t0
    del kh
    sc = ls.astype(np.float64).mean(axis=0)
    t0 = time.perf_counter()
    oracle.pick_topk(sc, BUDGET, sink=1)
    topk_s = time.perf_counter() - t0
    # stage-in quantize: every staged block x 16 layers x K/V, thread pool
    n_q = len(sel_ids)
    kb = host_blocks(k, sel_ids)
    vb = host_blocks(v, sel_ids)
    jobs = [(src[l, i].reshape(T, E)) for src in (kb, vb) for l in range(L) for i in range(n_q)]
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda r: oracle.quantize_rows_f16(oracle.TYPE_Q8_0, r), jobs))
    quant_s = time.perf_counter() - t0
    total_ms = (score_s + topk_s + quant_s) * 1e3
    # the reference's own scorer (mean-K cosine, one thread as in the
    # adapter) over the real key sums of every block (made on the device,
    # untimed: they are kept per block, not made per step)
    k_sum = k.float().sum(dim=2).reshape(L, B, E).cpu().numpy()
    q_sum = qf.sum(axis=1).reshape(L, HQ * D).astype(np.float32)
    t0 = time.perf_counter()
    oracle.score_meank(q_sum, [TQ] * L, k_sum, np.full((L, B), T, np.uint32), HQ, HKV, D)
    meank_s = time.perf_counter() - t0
    del k_sum
    # q8_0 quantize on one thread (the same jobs, serial)
    t0 = time.perf_counter()
    for r in jobs:
        oracle.quantize_rows_f16(oracle.TYPE_Q8_0, r)
    quant1_s = time.perf_counter() - t0
    # the reference's live stage-in on the host: a memcpy of the changed
    # blocks' packed q8_0 rows into the staging slab (write_block_to_gpu)
    packed = np.ones(n_q * L * 2 * T * 1088, dtype=np.uint8)
    slab = np.zeros_like(packed)
    slab.fill(2)  # the slab's pages are resident, as the reference's pinned slab
    memcpy_s = None
    for _ in range(3):
        t0 = time.perf_counter()
        np.copyto(slab, packed)
        dt = time.perf_counter() - t0
        memcpy_s = dt if memcpy_s is None else min(memcpy_s, dt)
    return {
        "value": round(total_ms, 1), "unit": "ms/step", "cores": threads, "kind": "port",
        "host_cpus_visible": visible, "cpu_share_per_gpu": HOST_CPU_SHARE,
        "sample": (f"the whole step measured, no scaling: fp32 per-token max scorer on all {B} blocks "
                   f"x {L} layers (OpenMP, {threads} threads); top-{BUDGET} over {B} scores; q8_0 "
                   f"quantize of all {n_q} staged blocks x {L} layers x K/V ({threads} threads)"),
        "parts_ms": {"score": round(score_s * 1e3, 1), "topk": round(topk_s * 1e3, 3),
                     "quantize": round(quant_s * 1e3, 1)},
        "other_legs": {
            "meank_score_ms": round(meank_s * 1e3, 2),
            "meank_sample": f"mean-K cosine scorer (1 thread) on all {B} blocks x {L} layers",
            "quantize_1thread_ms": round(quant1_s * 1e3, 1),
            "packed_memcpy_ms": round(memcpy_s * 1e3, 2),
            "packed_memcpy_GBs": round(packed.nbytes / memcpy_s / 1e9, 2),
        },
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
    out = {"ms": round(best * 1e3, 3), "h2d_bytes": h2d, "h2d_GBs": round(h2d / best / 1e9, 2),
           "link_peak_GBs": PCIE_PEAK_GBS, "frac": round(h2d / best / 1e9 / PCIE_PEAK_GBS, 3)}
    # the same blocks as packed q8_0 rows: stage-out (gather + D2H) into a
    # pinned packed store, then the packed stage-in back into the slots
    row = kv.row_size(kv.TYPE_Q8_0, E)
    span = L * T * 2 * row
    store = torch.empty(n * span, dtype=torch.uint8, pin_memory=True)
    ph = kv.PackedHost(store.data_ptr(), L, n, T)
    ids, nts = list(range(n)), [T] * n
    for name, fn in (("packed_stageout", lambda: ctx.stageout_blocks(pool, ph, ids, slots, nts)),
                     ("packed_stagein", lambda: ctx.stagein_packed_host(ph, pool, ids, slots, nts))):
        fn()
        ctx.sync()
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            ctx.sync()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        nbytes = n * span
        out[name] = {"ms": round(best * 1e3, 3), "bytes": nbytes, "GBs": round(nbytes / best / 1e9, 2),
                     "frac": round(nbytes / best / 1e9 / PCIE_PEAK_GBS, 3)}
    return out


def pinned_host_step(a, torch, kv, k, v, q, prev: list) -> dict:
    """The whole step with the history's K and V F16 in pinned host memory
    (block-major [block][layer][K rows, V rows], every block), the keys also
    in HBM for the per-token scorer: the stage-in kernel reads the changed
    blocks over PCIe and quantizes them in the same pass."""
    log("pinned-host step: the K/V history mirrored block-major in 16 GiB of pinned host memory")
    span_el = L * 2 * T * E
    host = torch.empty((B, span_el), dtype=torch.float16, pin_memory=True)
    hv = host.view(B, L, 2, T * E)
    for l in range(L):
        hv[:, l, 0].copy_(k[l].reshape(B, T * E))
        hv[:, l, 1].copy_(v[l].reshape(B, T * E))
    eng = make_engine(kv, torch, k, v)
    eng.set_host_history(host.data_ptr(), B)
    ctx = kv.Context.borrow(eng.ctx_handle())
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    h2d = m["n_staged"] * span_el * 2
    out = {"ms_per_step": round(m["ms_step"], 4),
           "ms_per_step_no_timing_events": round(m["ms_step_no_events"], 4),
           "score_kernel_ms": round(m["score_ms"], 4), "layout_ms": round(m["layout_ms"], 4),
           "stagein_kernel_ms": round(m["set_ms"], 4), "n_staged": m["n_staged"], "n_moved": m["n_moved"],
           "h2d_bytes": h2d, "h2d_GBs": round(h2d / (m["set_ms"] * 1e-3) / 1e9, 2),
           "link_peak_GBs": PCIE_PEAK_GBS}
    # with a pinned packed store (every block's q8_0 rows, block-major): the
    # warmup steps copy evicted blocks out once, then each step restores its
    # incoming blocks from their packed rows, half the link bytes of F16
    log("pinned-host step with a packed host store (q8_0 rows of every block, pinned)")
    row = kv.row_size(kv.TYPE_Q8_0, E)
    packed_span = L * 2 * T * row
    packed = torch.empty((B, packed_span), dtype=torch.uint8, pin_memory=True)
    eng.set_packed_host(packed.data_ptr(), B)
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, max(a.warmup, 2))
    eng.close()
    del hv, host, packed
    h2d = m["n_staged"] * packed_span
    out["with_packed_store"] = {
        "ms_per_step": round(m["ms_step"], 4), "ms_per_step_no_timing_events": round(m["ms_step_no_events"], 4),
        "score_kernel_ms": round(m["score_ms"], 4), "layout_ms": round(m["layout_ms"], 4),
        "stagein_ms": round(m["set_ms"], 4), "n_staged": m["n_staged"], "h2d_bytes": h2d,
        "h2d_GBs": round(h2d / (m["set_ms"] * 1e-3) / 1e9, 2) if m["set_ms"] > 0 else None}
    return out


def run_reselect_256k(a, torch, kv, workloads) -> dict:
    log("generating history K/V [16][2048][128][4][256] f16 and query [16][64][24][256] bf16")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=2, with_v=True)
    torch.cuda.synchronize()
    eng = make_engine(kv, torch, k, v)   # canonical layout: slot i = i-th selected block
    ctx = kv.Context.borrow(eng.ctx_handle())
    sel = eng.preview(q.data_ptr(), TQ).blocks
    prev = workloads.previous_selection(sel, B, N_CHANGED)
    log(f"selection {len(sel)} blocks, {len(set(sel) - set(prev))} changed vs previous step")
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    n_staged = m["n_staged"]
    log(f"step {m['ms_step']:.3f} ms: score kernel {m['score_ms']:.3f} ms, top-k "
        f"{m['sel_ms']:.3f} ms, slot moves {m['layout_ms']:.3f} ms ({m['n_moved']} blocks), "
        f"stage-in kernel {m['set_ms']:.3f} ms ({n_staged} blocks)")

    flops = 2.0 * TQ * HQ * D * (B * T) * L
    k_bytes = L * B * T * E * 2
    score_tflops = flops / (m["score_ms"] * 1e-3) / 1e12
    sbytes = stage_bytes(kv, n_staged, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    stage_gbs = sbytes / (m["set_ms"] * 1e-3) / 1e9
    row = kv.row_size(kv.TYPE_Q8_0, E)
    moved_bytes = m["n_moved"] * L * 2 * T * row  # one copy of the moved blocks' K and V rows
    result = {
        "metric": "reselect latency ms/agent-step @256K ctx; stage-in GB/s vs HBM peak",
        "value": round(m["ms_step"], 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(m["ms_step"], 4),
        "ms_per_step_no_timing_events": round(m["ms_step_no_events"], 4),
        "ms_per_step_all_timing_events": round(m["ms_step_all_events"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16/bf16->f32 scoring, f16->q8_0 stage-in",
        "data": "synthetic (seeded N(0,1) keys with per-block offsets, bf16 query)",
        "config": {"workload": "full reselect step @256K: 16 layers x 2048 blocks x 128 tokens, "
                               "4 KV heads x 256, 64-token query x 24 heads (GQA 6), top-256 + sink, "
                               f"{n_staged} changed blocks -> q8_0 K/V pool of 256+128 slots, "
                               "canonical layout (slot i = i-th selected block)",
                   "history": "device-resident", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "score_kernel<256>",
                     "achieved": round(score_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(score_tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": SCORE_TRAFFIC_BYTES, "algorithmic_bytes": k_bytes, "flops": flops,
                     "hbm_GBs_algorithmic": round(k_bytes / (m["score_ms"] * 1e-3) / 1e9, 1)},
        "stagein_roofline": {"bound": "hbm", "kernel": "quant_scatter_kv_kernel<q8_0,q8_0>",
                             "achieved": round(stage_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(stage_gbs / HBM_PEAK_GBS, 4), "traffic": STAGEIN_TRAFFIC_BYTES,
                             "algorithmic_bytes": sbytes, "kernel_ms": round(m["set_ms"], 4)},
        "layout": {"n_moved": m["n_moved"], "layout_ms": round(m["layout_ms"], 4),
                   "algorithmic_bytes": 2 * moved_bytes, "device_bytes": 2 * m["d2d_bytes"],
                   "GBs_algorithmic": (round(2 * moved_bytes / (m["layout_ms"] * 1e-3) / 1e9, 1)
                                       if m["layout_ms"] > 0 else None)},
        "parts_ms": {"score_kernel": round(m["score_ms"], 4), "topk_kernel": round(m["sel_ms"], 4),
                     "layout_kernels": round(m["layout_ms"], 4), "stagein_kernel": round(m["set_ms"], 4)},
        "after_score_ms": round(m["after_score_ms"], 4),
        "transfers_per_step": m["transfers"],
    }
    if not a.no_pinned:
        incoming = sorted(set(sel) - set(prev))
        result["pinned_host"] = pinned_host_mode(kv, ctx, torch, k, v, eng, incoming)
    if not a.no_cpu_baseline:
        log("cpu baseline (oracle restatement on host cores)")
        result["cpu_baseline"] = cpu_baseline(torch, k, v, q, sorted(set(sel) - set(prev)))
    eng.close()
    result["device_planned"] = m["device_planned"]
    result["host_planned"] = host_planned_mode(a, torch, kv, k, v, q, prev)
    result["lifo_layout"] = lifo_layout_mode(a, torch, kv, k, v, q, prev)
    if not a.no_configs:
        result["meank_256k"] = run_meank_256k(a, torch, kv, workloads, (k, v, q))
        result["cache_transform"] = run_cache_transform(a, torch, kv, workloads, (k, v, q))
    if not a.no_pinned:
        result["pinned_host"]["step"] = pinned_host_step(a, torch, kv, k, v, q, prev)
    del k, v, q
    torch.cuda.empty_cache()
    if not a.no_configs:
        result["mixed_precision"] = run_mixed_precision(a, torch, kv, workloads)["runs"]
        torch.cuda.empty_cache()
        result["recall_1m"] = run_recall_1m(a, torch, kv, workloads)
        torch.cuda.empty_cache()
    return result


def host_planned_mode(a, torch, kv, k, v, q, prev: list) -> dict:
    """The same step planned on the host (device_plan = 0): the host waits
    for the selection, plans the diff and the slot moves and launches them.
    `after_score_ms` is the device span from the scorer's end to the
    stage-in's end, the part the plan changes (the scorer's own duration
    follows the power-capped clock)."""
    log("host-planned: the same step with the diff and slot plan on the host")
    eng = make_engine(kv, torch, k, v, device_plan=0)
    ctx = kv.Context.borrow(eng.ctx_handle())
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    eng.close()
    assert m["device_planned"] == 0
    return {"ms_per_step": round(m["ms_step"], 4),
            "ms_per_step_no_timing_events": round(m["ms_step_no_events"], 4),
            "after_score_ms": round(m["after_score_ms"], 4),
            "score_kernel_ms": round(m["score_ms"], 4), "layout_ms": round(m["layout_ms"], 4),
            "stagein_kernel_ms": round(m["set_ms"], 4), "n_moved": m["n_moved"], "n_staged": m["n_staged"]}


def lifo_layout_mode(a, torch, kv, k, v, q, prev: list) -> dict:
    """The same step with the LIFO slot plan alone (canonical_layout = 0):
    incoming blocks take the slots the outgoing ones free and resident
    blocks never move.  Reported beside the default step."""
    log("LIFO layout: the same step without the canonical slot moves")
    eng = make_engine(kv, torch, k, v, canonical_layout=0)
    ctx = kv.Context.borrow(eng.ctx_handle())
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    eng.close()
    return {"ms_per_step": round(m["ms_step"], 4), "n_moved": m["n_moved"], "n_staged": m["n_staged"],
            "score_kernel_ms": round(m["score_ms"], 4), "stagein_kernel_ms": round(m["set_ms"], 4)}


def run_mixed_precision(a, torch, kv, workloads) -> dict:
    """Student-t (nu = 4) history; run A K q8_0 + V q4_0 (reserve 128
    blocks), run B K and V q5_0 (reserve 96 blocks)."""
    log("generating Student-t history K/V [16][2048][128][4][256] f16")
    k, v, q = workloads.student_t_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=4)
    torch.cuda.synchronize()
    runs = {}
    for name, tk, tv, reserve in (("A_q8_0_q4_0", kv.TYPE_Q8_0, kv.TYPE_Q4_0, 128),
                                  ("B_q5_0_q5_0", kv.TYPE_Q5_0, kv.TYPE_Q5_0, 96)):
        eng = make_engine(kv, torch, k, v, reserve=reserve, type_k=tk, type_v=tv)
        ctx = kv.Context.borrow(eng.ctx_handle())
        sel = eng.preview(q.data_ptr(), TQ).blocks
        prev = workloads.previous_selection(sel, B, N_CHANGED)
        m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
        sb = stage_bytes(kv, m["n_staged"], tk, tv)
        runs[name] = {"ms_per_step": round(m["ms_step"], 4), "score_kernel_ms": round(m["score_ms"], 4),
                      "stagein_kernel_ms": round(m["set_ms"], 4), "n_staged": m["n_staged"],
                      "stagein_algorithmic_bytes": sb,
                      "stagein_GBs": round(sb / (m["set_ms"] * 1e-3) / 1e9, 1),
                      "stagein_frac_hbm": round(sb / (m["set_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                      "layout_ms": round(m["layout_ms"], 4), "n_moved": m["n_moved"],
                      "pool_slots": BUDGET + reserve}
        log(f"{name}: {runs[name]}")
        eng.close()
    del k, v, q
    return {"metric": "mixed-precision reselect @256K (Student-t nu=4 history)", "unit": "ms/step",
            "higher_is_better": False, "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
            "data": "synthetic (seeded Student-t nu=4 K/V, bf16 query)", "runs": runs}


def run_cache_transform(a, torch, kv, workloads, tensors=None) -> dict:
    """The 256K step with the cache row transform on: the 77 changed blocks
    are RoPE'd at their original positions (256 rotary dims, base 1e6) and
    Walsh-Hadamard rotated (K width 256, V width 64) before q8_0.  Beside it,
    `transform_parts`: the stage-in alone (no scorer before it), 77 distinct
    random blocks per call, with each part of the transform on its own.
    `tensors` = (k, v, q) of the 256K workload when the caller has them."""
    if tensors is None:
        log("generating history K/V [16][2048][128][4][256] f16 and query")
        k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=2, with_v=True)
        torch.cuda.synchronize()
    else:
        k, v, q = tensors
    log("cache transform step: RoPE 256 + attn_rot before q8_0")
    eng = make_engine(kv, torch, k, v, n_rot=256, rope_freq_base=1e6, attn_rot=1)
    ctx = kv.Context.borrow(eng.ctx_handle())
    sel = eng.preview(q.data_ptr(), TQ).blocks
    prev = workloads.previous_selection(sel, B, N_CHANGED)
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    eng.close()
    sb = stage_bytes(kv, m["n_staged"], kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    gbs = sb / (m["set_ms"] * 1e-3) / 1e9
    parts = transform_parts(kv, torch, k, v, sb)
    return {"metric": "reselect @256K with RoPE + attn_rot stage-in", "unit": "ms/step",
            "value": round(m["ms_step"], 4), "higher_is_better": False, "n_gpus": 1,
            "steps": a.steps, "warmup": a.warmup, "data": "synthetic (seeded N(0,1) keys, bf16 query)",
            "stagein_roofline": {"bound": "hbm", "kernel": "x64_kv_kernel<q8_0,q8_0>",
                                 "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": sb,
                                 "kernel_ms": round(m["set_ms"], 4), "n_staged": m["n_staged"]},
            "parts_ms": {"score_kernel": round(m["score_ms"], 4), "stagein_kernel": round(m["set_ms"], 4)},
            "transform_parts": parts}


def transform_parts(kv, torch, k, v, sb: int, calls: int = 12) -> dict:
    """Stage-in device ms (events on the library stream) of 77 random blocks
    x 16 layers into a q8_0 pool, per transform: none, RoPE only (K), K
    Hadamard 256 only, V Hadamard 64 only, and all of them."""
    import numpy as np
    # RoPE frequencies base^(-2i/n_rot) (the timing does not depend on their last bits)
    theta = (1e6 ** (-2.0 * np.arange(128) / 256)).astype(np.float32)
    ctx = kv.Context(0)
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    n_slots = N_CHANGED
    pk = [torch.empty(n_slots * T * rb, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.empty(n_slots * T * rb, dtype=torch.uint8, device="cuda") for _ in range(L)]
    hist = ctx.make_history(k.data_ptr(), v.data_ptr(), L, B, T, E, E)
    rng = np.random.default_rng(5)
    sets = [sorted(rng.choice(B, N_CHANGED, replace=False).tolist()) for _ in range(calls + 2)]
    slots = list(range(n_slots))
    variants = {"none": None, "rope_k": (D, 256, theta, 0, 0), "hadamard_k256": (D, 0, None, 256, 0),
                "hadamard_v64": (D, 0, None, 0, 64), "all": (D, 256, theta, 256, 64)}
    out = {}
    ctx.perf_enable(True)
    for name, xf in variants.items():
        x = ctx.make_transform(*xf) if xf else None
        pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p.data_ptr() for p in pk],
                             [p.data_ptr() for p in pv], x)
        for ids in sets[:2]:
            ctx.stagein_blocks(hist, pool, ids, slots)
        ctx.sync()
        ctx.perf_reset()
        for ids in sets[2:]:
            ctx.stagein_blocks(hist, pool, ids, slots)
        ctx.sync()
        ms = ctx.perf()["set_ms"] / calls
        out[name] = {"kernel_ms": round(ms, 4), "GBps": round(sb / (ms * 1e-3) / 1e9, 1),
                     "frac": round(sb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    ctx.perf_enable(False)
    ctx.close()
    del pk, pv
    return out


def sample_power_clocks() -> dict | None:
    """One `amd-smi metric -c -p` reading: socket power (W) and the GFX
    clocks (MHz) of the XCDs; None where the tool is missing or fails."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-c", "-p"], capture_output=True, text=True,
                             timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    power = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", out)
    clocks = [int(m) for m in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*([0-9]+)\s*MHz", out)]
    if not power and not clocks:
        return None
    return {"socket_power_W": float(power.group(1)) if power else None, "gfx_clk_MHz": clocks}


def run_scorer_sustained(a, torch, kv, workloads) -> dict:
    """The 256K scorer (16 layers x 2048 blocks, 64-token query) back to
    back for `--seconds`, with socket power and GFX clocks sampled in the
    middle: the power-capped regime the kernel runs in when it is the whole
    load, and the dense fp16 MFMA ceiling at the sampled clock."""
    import threading
    log("generating history K [16][2048][128][4][256] f16 and query")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=2)
    torch.cuda.synchronize()
    scores = torch.empty(B, dtype=torch.float32, device="cuda")
    ctx = kv.Context(0)
    hist = ctx.make_history(k.data_ptr(), None, L, B, T, E, 0)
    for _ in range(3):
        ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, TQ, HQ, HKV, D, scores.data_ptr())
    ctx.sync()
    sample: dict = {}
    timer = threading.Timer(a.seconds / 2, lambda: sample.update(s=sample_power_clocks()))
    timer.start()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < a.seconds:
        for _ in range(20):
            ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, TQ, HQ, HKV, D, scores.data_ptr())
        ctx.sync()
        n += 20
    dt = time.perf_counter() - t0
    timer.join()
    ctx.close()
    ms = 1e3 * dt / n
    flops = 2.0 * TQ * HQ * D * B * T * L
    pc = sample.get("s")
    out = {"metric": "scorer back to back @256K", "unit": "ms/call", "value": round(ms, 4),
           "higher_is_better": False, "n_gpus": 1, "calls": n,
           "data": "synthetic (seeded N(0,1) keys with per-block offsets, bf16 query)",
           "achieved_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1), "power_clocks": pc}
    if pc and pc["gfx_clk_MHz"]:
        mhz = sum(pc["gfx_clk_MHz"]) / len(pc["gfx_clk_MHz"])
        # 1024 SIMDs x 1024 dense fp16 FLOP per clock (2.5 PFLOP/s at 2.4 GHz)
        peak = 1024 * 1024 * mhz * 1e6 / 1e12
        out["mfma_peak_at_clock_TFLOPs"] = round(peak, 1)
        out["frac_at_clock"] = round(flops / (ms * 1e-3) / 1e12 / peak, 4)
    return out


def run_meank_256k(a, torch, kv, workloads, tensors=None) -> dict:
    """The 256K step with the reference's mean-K cosine scorer: per-block
    key sums are produced once (untimed warmup) and kept; a step sums the
    query rows, scores every block from the sums (128 MiB of fp32) and
    stages the changed blocks.  `tensors` = (k, v, q) of the 256K workload
    when the caller has them."""
    if tensors is None:
        log("generating history K/V [16][2048][128][4][256] f16 and query")
        k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=TQ, seed=2, with_v=True)
        torch.cuda.synchronize()
    else:
        k, v, q = tensors
    log("mean-K step: the reference's scorer over kept key sums")
    eng = make_engine(kv, torch, k, v, scorer=1)
    ctx = kv.Context.borrow(eng.ctx_handle())
    sel = eng.preview(q.data_ptr(), TQ).blocks
    prev = workloads.previous_selection(sel, B, N_CHANGED)
    m = timed_steps(eng, ctx, torch, q, TQ, prev, a.steps, a.warmup)
    eng.close()
    sums_bytes = L * B * E * 4
    return {"metric": "reselect @256K with the mean-K cosine scorer", "unit": "ms/step",
            "value": round(m["ms_step"], 4), "higher_is_better": False, "n_gpus": 1,
            "steps": a.steps, "warmup": a.warmup, "data": "synthetic (seeded N(0,1) keys, bf16 query)",
            "score_roofline": {"bound": "hbm", "kernel": "meank_cos_kernel<256>",
                               "achieved": round(sums_bytes / (m["cos_ms"] * 1e-3) / 1e9, 1),
                               "peak": HBM_PEAK_GBS, "unit": "GB/s", "algorithmic_bytes": sums_bytes,
                               "frac": round(sums_bytes / (m["cos_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                               "kernel_ms": round(m["cos_ms"], 4),
                               "scoring_span_ms": round(m["score_ms"], 4)},
            "ms_per_step_no_timing_events": round(m["ms_step_no_events"], 4),
            "parts_ms": {"score": round(m["score_ms"], 4), "stagein_kernel": round(m["set_ms"], 4),
                         "topk": round(m["sel_ms"], 4), "layout_kernels": round(m["layout_ms"], 4)},
            "n_staged": m["n_staged"], "n_moved": m["n_moved"]}


def run_recall_1m(a, torch, kv, workloads) -> dict:
    """1M-token workspace: 8192 blocks x 16 layers, 512-token query, 32
    planted blocks (Zipf relevance), budget 512.  A cold step (empty pool,
    every selected block staged), the recall of the planted blocks, then
    reselect steps that each start from a previous selection with 30 % of
    the 512 blocks different (154 staged)."""
    nb, tq, budget = 8192, 512, 512
    n_changed = round(0.3 * budget)
    log("generating history K/V [16][8192][128][4][256] f16 (64 GiB) and query [16][512][24][256]")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=tq, seed=6, with_v=True)
    planted = workloads.plant_blocks(torch, k, q, n_planted=32, seed=5)
    torch.cuda.synchronize()
    eng = make_engine(kv, torch, k, v, n_blocks=nb, budget=budget, reserve=128)
    ctx = kv.Context.borrow(eng.ctx_handle())
    ctx.perf_enable(True)
    ctx.perf_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    st = eng.apply_retrieval(q.data_ptr(), tq)
    torch.cuda.synchronize()
    cold_ms = 1e3 * (time.perf_counter() - t0)
    pf_cold = ctx.perf()
    ctx.perf_enable(False)
    sel = eng.preview(q.data_ptr(), tq).blocks
    recall = sum(int(b) in set(sel) for b in planted) / len(planted)
    prev = workloads.previous_selection(sel, nb, n_changed)
    m = timed_steps(eng, ctx, torch, q, tq, prev, max(2, a.steps // 2), 1)
    eng.close()
    del k, v, q
    flops = 2.0 * tq * HQ * D * (nb * T) * L
    sb = stage_bytes(kv, m["n_staged"], kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    log(f"1M: reselect step {m['ms_step']:.3f} ms, cold step {cold_ms:.3f} ms, recall {recall:.3f}")
    return {"metric": "1M-workspace reselect step + planted-block recall", "unit": "ms/step",
            "higher_is_better": False, "n_gpus": 1,
            "config": {"workload": "16 layers x 8192 blocks x 128 tokens, 512-token query, budget 512 "
                                   "(+128 reserve), 32 planted blocks, q8_0 K/V, canonical layout",
                       "changed_per_step": n_changed},
            "ms_per_step": round(m["ms_step"], 3), "n_staged": m["n_staged"], "n_moved": m["n_moved"],
            "score_kernel_ms": round(m["score_ms"], 3),
            "score_TFLOPs": round(flops / (m["score_ms"] * 1e-3) / 1e12, 1),
            "score_frac_mfma": round(flops / (m["score_ms"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "topk_kernel_ms": round(m["sel_ms"], 4), "layout_ms": round(m["layout_ms"], 4),
            "stagein_kernel_ms": round(m["set_ms"], 4),
            "stagein_frac_hbm": round(sb / (m["set_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "cold_step_ms": round(cold_ms, 3), "cold_staged": st["n_staged"],
            "cold_stagein_kernel_ms": round(pf_cold["set_ms"], 4),
            "recall_planted": recall, "n_planted": len(planted)}


def run_copy_calibration(a, torch, kv, workloads) -> dict:
    """A plain device copy of known size (1 GiB in 4096 ops of 256 KiB,
    batched_copy_kernel): the reference point for HBM byte counters."""
    n_ops, op = 4096, 256 << 10
    src = torch.randint(0, 255, (n_ops * op,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    ctx = kv.Context(0)
    srcs = [src.data_ptr() + i * op for i in range(n_ops)]
    dsts = [dst.data_ptr() + i * op for i in range(n_ops)]
    ctx.d2d_batched(srcs, dsts, [op] * n_ops)
    ctx.sync()
    ctx.perf_enable(True)
    ctx.perf_reset()
    for _ in range(a.steps):
        ctx.d2d_batched(srcs, dsts, [op] * n_ops)
    ctx.sync()
    ms = ctx.perf()["layout_ms"] / a.steps
    ok = bool(torch.equal(src, dst))
    ctx.close()
    # the runtime's own device copy of the same bytes, for comparison
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    e0.record()
    for _ in range(a.steps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    rt_ms = e0.elapsed_time(e1) / a.steps
    # the host link: one 512 MiB pinned buffer each way, the runtime's copies
    link = {}
    hbuf = torch.empty(512 << 20, dtype=torch.uint8, pin_memory=True)
    dbuf = src[: 512 << 20]
    for name, fn in (("h2d", lambda: dbuf.copy_(hbuf, non_blocking=True)),
                     ("d2h", lambda: hbuf.copy_(dbuf, non_blocking=True))):
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(3):
            fn()
        e1.record()
        e1.synchronize()
        t = e0.elapsed_time(e1) / 3
        link[name + "_GBs"] = round((512 << 20) / (t * 1e-3) / 1e9, 1)
    # plain streaming kernels (kvmem-llama.cpp_amd/calib/hbm_rates.hip, a
    # child process): the read, write and copy rates this device reaches
    calib = Path(__file__).resolve().parent / "kvmem-llama.cpp_amd" / "calib" / "hbm_rates"
    if not calib.exists():
        raise SystemExit(f"{calib} is missing: build first (__graft_entry__.build())")
    log("plain streaming kernels: 1 GiB read, write and copy")
    r = subprocess.run([str(calib)], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        raise SystemExit(f"hbm_rates failed ({r.returncode}): {r.stderr.strip()}")
    plain = json.loads(r.stdout.strip().splitlines()[-1])
    return {"metric": "device copy calibration", "bytes_read": n_ops * op, "bytes_written": n_ops * op,
            "kernel_ms": round(ms, 4), "GBs_read_plus_write": round(2 * n_ops * op / (ms * 1e-3) / 1e9, 1),
            "runtime_copy_ms": round(rt_ms, 4),
            "runtime_copy_GBs": round(2 * n_ops * op / (rt_ms * 1e-3) / 1e9, 1), "copy_ok": ok,
            "pinned_link": link, "plain_kernels": plain}


def run_mfma_calibration(a, torch, kv, workloads) -> dict:
    """The runtime's own dense GEMM (torch.matmul, i.e. hipBLASLt) on
    8192 x 8192 x 8192 f16 and bf16 operands, each back to back for half of
    `--seconds`, with socket power and GFX clocks sampled in the middle of
    each loop: the dense MFMA rate a tuned library reaches on this chip under
    the same power cap as the scorer, the reference point for the scorer's
    TFLOP/s."""
    import threading
    n = 8192
    flops = 2.0 * n * n * n
    out = {"metric": "dense GEMM calibration (torch.matmul 8192^3)", "unit": "TFLOP/s",
           "higher_is_better": True, "n_gpus": 1}
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        g = torch.Generator(device="cuda").manual_seed(5)
        x = torch.randn(n, n, device="cuda", dtype=dt, generator=g)
        w = torch.randn(n, n, device="cuda", dtype=dt, generator=g)
        y = torch.empty(n, n, device="cuda", dtype=dt)
        for _ in range(3):
            torch.matmul(x, w, out=y)
        torch.cuda.synchronize()
        sample: dict = {}
        secs = a.seconds / 2
        timer = threading.Timer(secs / 2, lambda: sample.update(s=sample_power_clocks()))
        timer.start()
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < secs:
            for _ in range(10):
                torch.matmul(x, w, out=y)
            torch.cuda.synchronize()
            calls += 10
        el = time.perf_counter() - t0
        timer.join()
        tf = flops * calls / el / 1e12
        entry = {"ms_per_call": round(1e3 * el / calls, 4), "TFLOPs": round(tf, 1), "calls": calls,
                 "frac_of_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "power_clocks": sample.get("s")}
        pc = sample.get("s")
        if pc and pc["gfx_clk_MHz"]:
            mhz = sum(pc["gfx_clk_MHz"]) / len(pc["gfx_clk_MHz"])
            entry["frac_at_clock"] = round(tf / (1024 * 1024 * mhz * 1e6 / 1e12), 4)
        out[name] = entry
        del x, w, y
    out["value"] = out["f16"]["TFLOPs"]
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="reselect_256k",
                    choices=["reselect_256k", "mixed_precision", "recall_1m", "copy_calibration",
                             "cache_transform", "meank_256k", "scorer_sustained", "mfma_calibration"])
    ap.add_argument("--seconds", type=float, default=8.0,
                    help="scorer_sustained, mfma_calibration: loop length")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pinned", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="reselect_256k: leave out the mixed-precision and 1M-workspace sub-objects")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the reselect path runs on a single MI355X; "
              "sharding it across GPUs is a design, not a run", file=sys.stderr)
        return 2

    import torch
    kv = load_pkg()
    from kvmem_amd import workloads
    run = {"reselect_256k": run_reselect_256k, "mixed_precision": run_mixed_precision,
           "recall_1m": run_recall_1m, "copy_calibration": run_copy_calibration,
           "cache_transform": run_cache_transform, "meank_256k": run_meank_256k,
           "scorer_sustained": run_scorer_sustained, "mfma_calibration": run_mfma_calibration}[a.workload]
    result = run(a, torch, kv, workloads)
    print(json.dumps(result), flush=True)
    # every engine and context is released here, with the runtime fully up,
    # not by finalizers during interpreter shutdown
    torch.cuda.synchronize()
    kv.close_all()
    log("closed every engine and context")
    return 0


if __name__ == "__main__":
    sys.exit(main())
