"""Transfer accounting and the profiling buckets on the GPU
(kvmem_hip_transfer_get, kvmem_hip_perf_*).

- Bytes and calls per direction, exact, for each data path of the device
  layer: the pinned-host stage-in (one host-to-device kernel read), the
  stage-out to a pinned packed store (one device-to-host launch), the packed
  stage-in, kvmem_hip_h2d_async, kvmem_hip_d2d_batched and a slot move
  (device to device), against the byte counts worked out from the pool and
  history geometry; and the timed calls of the set, stage-out, copy and
  layout buckets.  The reference counts the same directions at its copy
  call sites (src/adapter/llama-kvmem-transfer.h:9-31).
- A failed call leaves no stage open: after a stage-in failed on the host
  (kvmem_hip_debug_fail_after) and a 300 ms pause, the next stage-in's time
  is its own, not measured from the failed call's start.
- The engine's plan bucket and n_skip: a host-planned apply adds host plan
  time, a device-planned apply_retrieval the plan kernel's; n_skip counts
  the window blocks whose baked position equals their window position.
"""
from __future__ import annotations

import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()

from engine_helpers import T, history, make_engine  # noqa: E402

L, B, E = 2, 6, 1024


def announce(msg: str) -> None:
    print(f"[perf] {msg}", flush=True)


def delta(after: dict, before: dict) -> dict:
    return {k: after[k] - before[k] for k in after}


def test_transfer_counts_per_direction():
    announce("transfer bytes and calls: pinned stage-in, stage-out, packed stage-in, h2d, d2d, move")
    rk = kv.row_size(kv.TYPE_Q8_0, E)
    span = L * T * 2 * E * 2                     # one block, every layer, K then V, F16
    pspan = L * T * 2 * rk                        # the same block packed
    rng = np.random.default_rng(3)
    host_hist = torch.from_numpy(rng.standard_normal(B * span // 2).astype(np.float16)).pin_memory()
    packed = torch.zeros(B * pspan, dtype=torch.uint8).pin_memory()
    n_slots = 8
    pk = [torch.zeros(n_slots * T * rk, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.zeros(n_slots * T * rk, dtype=torch.uint8, device="cuda") for _ in range(L)]
    with kv.Context(0) as ctx:
        pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p.data_ptr() for p in pk],
                             [p.data_ptr() for p in pv])
        ctx.perf_enable(True)
        ctx.perf_reset()
        t0 = ctx.transfers()
        assert all(v == 0 for v in t0.values()), t0
        hh = kv.HostHistory(host_hist.data_ptr(), L, B, T, E, E, 0)
        ctx.stagein_blocks_host(hh, pool, [1, 4, 5], [0, 2, 3])
        t1 = ctx.transfers()
        assert delta(t1, t0) == dict(t0, h2d_bytes=3 * span, h2d_calls=1)
        ph = kv.PackedHost(packed.data_ptr(), L, B, T)
        ctx.stageout_blocks(pool, ph, [1, 4], [0, 2], [T, 50])
        t2 = ctx.transfers()
        assert delta(t2, t1) == dict(t0, d2h_bytes=L * (T + 50) * 2 * rk, d2h_calls=1)
        ctx.stagein_packed_host(ph, pool, [1], [5], [T])
        t3 = ctx.transfers()
        assert delta(t3, t2) == dict(t0, h2d_bytes=pspan, h2d_calls=1)
        dst = torch.zeros(4096, dtype=torch.uint8, device="cuda")
        ctx.h2d_async(dst.data_ptr(), packed.data_ptr(), 4096)
        t4 = ctx.transfers()
        assert delta(t4, t3) == dict(t0, h2d_bytes=4096, h2d_calls=1)
        ctx.d2d_batched([pk[0].data_ptr(), pk[1].data_ptr()], [dst.data_ptr(), dst.data_ptr() + 1024],
                        [1000, 24])
        t5 = ctx.transfers()
        assert delta(t5, t4) == dict(t0, d2d_bytes=1024, d2d_calls=1)
        ctx.move_slots(pool, [0], [7])
        t6 = ctx.transfers()
        assert delta(t6, t5) == dict(t0, d2d_bytes=pspan, d2d_calls=1)
        ctx.sync()
        perf = ctx.perf()
        assert perf["n_set"] == 2 and perf["n_stage_out"] == 1 and perf["n_copy"] == 1
        assert perf["n_layout"] == 2
        assert perf["h2d_bytes"] == t6["h2d_bytes"] and perf["d2h_bytes"] == t6["d2h_bytes"]
        assert perf["d2d_bytes"] == t6["d2d_bytes"]
        assert perf["stage_out_ms"] > 0 and perf["set_ms"] > 0
        # the stage-out wrote the oracle's bytes where the pool held them
        got = packed.numpy().reshape(B, L, 2, T, rk)
        for layer in range(L):
            assert np.array_equal(got[4, layer, 0, :50], pk[layer].cpu().numpy().reshape(n_slots, T, rk)[2, :50])
        ctx.perf_reset()
        assert all(v == 0 for v in ctx.transfers().values())
        ctx.perf_enable(False)


def test_failed_stagein_leaves_no_open_stage():
    announce("stage-ins failed on the host, then good ones 300 ms later: set_ms is their own")
    rk = kv.row_size(kv.TYPE_Q8_0, E)
    span = L * T * 2 * E * 2
    host_hist = torch.zeros(B * span // 2, dtype=torch.float16).pin_memory()
    src = torch.zeros(T * E, dtype=torch.float16, device="cuda")
    n_slots = 8
    pk = [torch.zeros(n_slots * T * rk, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.zeros(n_slots * T * rk, dtype=torch.uint8, device="cuda") for _ in range(L)]
    ops = [(src.data_ptr(), pk[0].data_ptr(), T, E, kv.TYPE_Q8_0)]
    with kv.Context(0) as ctx:
        pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p.data_ptr() for p in pk],
                             [p.data_ptr() for p in pv])
        hh = kv.HostHistory(host_hist.data_ptr(), L, B, T, E, E, 0)
        ctx.stagein_quant(ops)                            # first calls: tables and code loaded
        ctx.stagein_blocks_host(hh, pool, [0], [0])
        ctx.sync()
        ctx.perf_enable(True)
        for name, call in (("stagein_quant", lambda: ctx.stagein_quant(ops)),
                           ("stagein_blocks_host", lambda: ctx.stagein_blocks_host(hh, pool, [1, 2], [1, 2]))):
            ctx.perf_reset()
            ctx.debug_fail_after(kv.FAIL_LAUNCH, 1)
            with pytest.raises(kv.KvMemError):
                call()
            ctx.debug_fail_after(0, 0)
            assert ctx.transfers()["h2d_calls"] == 0, name    # nothing was issued
            ctx.sync()
            time.sleep(0.3)
            call()
            ctx.sync()
            perf = ctx.perf()
            assert perf["n_set"] == 1, (name, perf)
            assert perf["set_ms"] < 100.0, (name, perf)       # its own time, not the 300 ms pause
        ctx.perf_enable(False)


def test_engine_plan_bucket_and_skip_count():
    announce("engine: host plan time, device plan kernel time, n_skip")
    cap, nb = 40, 40
    k, v, q = history(cap, seed=61)
    with make_engine(8, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        ctx = kv.Context.borrow(eng.ctx_handle())
        ctx.perf_enable(True)
        ctx.perf_reset()
        sel = eng.preview(q.data_ptr(), q.shape[1])
        st = eng.apply(sel)
        perf = ctx.perf()
        assert perf["n_plan"] == 1 and perf["plan_ms"] > 0, perf
        # first apply: every block is baked at its own start; block id i at index i keeps it
        assert st["n_skip"] == sum(1 for i, b in enumerate(sel.blocks) if b == i)
        assert st["n_skip"] >= 1                          # the sink block 0
        q2 = (q.float() * -1.0).to(torch.bfloat16)
        ctx.perf_reset()
        st2 = eng.apply_retrieval(q2.data_ptr(), q2.shape[1])
        assert st2["device_planned"] == 1
        perf = ctx.perf()
        assert perf["n_plan"] == 1 and perf["plan_ms"] > 0, perf
        tr = ctx.transfers()
        assert tr["d2d_bytes"] == perf["d2d_bytes"]
        if st2["n_moved"]:
            moved = st2["n_moved"] * L * T * 2 * kv.row_size(kv.TYPE_Q8_0, E)
            assert tr["d2d_calls"] >= 1 and tr["d2d_bytes"] >= moved, (tr, st2)
        ctx.perf_enable(False)


def test_meank_cosine_kernel_timed_alone():
    """score_ms covers the mean-K scorer's three kernels; meank_cos_ms the
    cosine kernel alone, one timed launch per call, inside the score span;
    the stage mask switches it off."""
    announce("mean-K scorer: cosine kernel bucket")
    nl, nb, hq, hkv, d = 4, 512, 8, 4, 256
    ks = torch.randn((nl, nb, hkv * d), device="cuda")
    mt = torch.full((nl, nb), 128, dtype=torch.int32, device="cuda")
    q_sum = torch.randn((nl, hq * d), device="cuda")
    scores = torch.empty(nb, dtype=torch.float32, device="cuda")
    with kv.Context(0) as ctx:
        def score():
            ctx.score_meank(q_sum.data_ptr(), [4] * nl, ks.data_ptr(), mt.data_ptr(), nl, nb, hq, hkv, d,
                            scores.data_ptr())
        torch.cuda.synchronize()
        score()
        ctx.sync()
        ctx.perf_enable(True)
        ctx.perf_reset()
        for _ in range(3):
            score()
        ctx.sync()
        pf = ctx.perf()
        assert pf["n_score"] == 3 and pf["n_meank_cos"] == 3
        assert 0.0 < pf["meank_cos_ms"] < pf["score_ms"]
        ctx.perf_stages(kv.PERF_STAGE_ALL & ~kv.PERF_STAGE_MEANK_COS)
        ctx.perf_reset()
        score()
        ctx.sync()
        pf = ctx.perf()
        assert pf["n_score"] == 1 and pf["n_meank_cos"] == 0 and pf["meank_cos_ms"] == 0.0
        ctx.perf_stages(kv.PERF_STAGE_ALL)
        ctx.perf_enable(False)
