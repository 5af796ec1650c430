"""Up-front sizing (kvmem_hip_reserve) and the plain host-to-device copy
(kvmem_hip_h2d_async) on the GPU.

A context reserved for a set of shapes must run every entry point at those
shapes without a single further device or pinned allocation, and give the
same bytes as a context that grew its scratch on demand.  The copy must
move pinned and pageable host bytes unchanged, accept n == 0 and reject
null pointers, like kvmem_stagein_h2d_bytes (llama-kvmem-stagein.cu:607-613).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import workloads  # noqa: E402

T = 128
L, B, HQ, HKV, D, TQ = 2, 16, 24, 4, 256, 8
E = HKV * D
N_SLOTS = 8


def announce(msg: str) -> None:
    print(f"[reserve] {msg}", flush=True)
    sys.stdout.flush()


def run_path(ctx, inputs):
    """Every entry point once at the reserved shapes; returns host copies of
    all outputs."""
    kd, vd, q, hb = inputs["k"], inputs["v"], inputs["q"], inputs["host"]
    hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), L, B, T, E, E)
    torch.cuda.synchronize()
    scores = torch.empty(B, dtype=torch.float32, device="cuda")
    ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, TQ, HQ, HKV, D, scores.data_ptr())
    sel = ctx.topk(scores.data_ptr(), B, 5, forced=[0])
    tk, tv = kv.TYPE_Q8_0, kv.TYPE_Q4_0
    rk, rv = kv.row_size(tk, E), kv.row_size(tv, E)
    pk = [torch.zeros(N_SLOTS * T * rk, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.zeros(N_SLOTS * T * rv, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pool = ctx.make_pool(L, N_SLOTS, T, E, E, tk, tv, [p.data_ptr() for p in pk], [p.data_ptr() for p in pv])
    torch.cuda.synchronize()  # the pools were cleared on torch's stream
    ctx.stagein_blocks(hist, pool, [3, 9], [0, 1])
    hh = kv.HostHistory(hb.data_ptr(), L, B, T, E, E, 0)
    ctx.stagein_blocks_host(hh, pool, [1, 4, 15], [2, 3, 4])
    span = L * T * (rk + rv)
    store = torch.full((B * span,), 0xA5, dtype=torch.uint8, pin_memory=True)
    ph = kv.PackedHost(store.data_ptr(), L, B, T)
    ctx.stageout_blocks(pool, ph, [3, 9, 1], [0, 1, 2], [T, T, T])
    ctx.stagein_packed_host(ph, pool, [3, 9], [5, 6], [T, T])
    ctx.move_slots(pool, [4, 2], [7, 2])
    ks = torch.empty((L, B, E), dtype=torch.float32, device="cuda")
    mt = torch.empty((L, B), dtype=torch.int32, device="cuda")
    ctx.meank_sums(hist, list(range(B)), ks.data_ptr(), mt.data_ptr())
    q_sum = torch.empty((L, HQ * D), dtype=torch.float32, device="cuda")
    ctx.q_accumulate(q.data_ptr(), kv.TYPE_BF16, L, TQ, HQ * D, q_sum.data_ptr())
    mscores = torch.empty(B, dtype=torch.float32, device="cuda")
    ctx.score_meank(q_sum.data_ptr(), [TQ] * L, ks.data_ptr(), mt.data_ptr(), L, B, HQ, HKV, D,
                    mscores.data_ptr())
    ctx.sync()
    return {"scores": scores.cpu().numpy(), "sel": np.array(sel), "store": store.numpy().copy(),
            "pk": [p.cpu().numpy() for p in pk], "pv": [p.cpu().numpy() for p in pv],
            "ks": ks.cpu().numpy(), "mscores": mscores.cpu().numpy()}


def make_inputs():
    kh = workloads.heavy_tailed(31, (L, B, T, E))
    vh = workloads.heavy_tailed(32, (L, B, T, E))
    rng = np.random.default_rng(33)
    qf = rng.standard_normal((L, TQ, HQ, D)).astype(np.float32)
    q = torch.from_numpy(qf).to(torch.bfloat16).cuda()
    # host history: [block][layer][K rows][V rows] f16
    hk = np.transpose(kh, (1, 0, 2, 3)).reshape(B, L, T * E)
    hv = np.transpose(vh, (1, 0, 2, 3)).reshape(B, L, T * E)
    host = torch.empty((B, L * 2 * T * E), dtype=torch.int16, pin_memory=True)
    host.copy_(torch.from_numpy(np.concatenate([hk, hv], axis=2).reshape(B, -1).view(np.int16)))
    return {"k": torch.from_numpy(kh.view(np.int16)).cuda(), "v": torch.from_numpy(vh.view(np.int16)).cuda(),
            "q": q, "host": host}


def test_reserved_context_allocates_nothing_and_matches():
    announce(f"L={L} B={B} Hq={HQ} Hkv={HKV} D={D} Tq={TQ}: reserve, then every entry point")
    inputs = make_inputs()
    rk, rv = kv.row_size(kv.TYPE_Q8_0, E), kv.row_size(kv.TYPE_Q4_0, E)
    with kv.Context(0) as grown, kv.Context(0) as held:
        held.reserve(n_layers=L, n_blocks=B, n_head=HQ, n_head_kv=HKV, head_dim=D, n_q_tokens=TQ,
                     max_items=B, h2d_block_bytes=L * T * 2 * E * 2, d2h_block_bytes=L * T * (rk + rv),
                     move_bytes=2 * L * T * (rk + rv))
        before = held.scratch_info()
        assert before["allocations"] > 0 and before["device_bytes"] > 0
        got = run_path(held, inputs)
        after = held.scratch_info()
        assert after == before, (before, after)
        want = run_path(grown, inputs)
        assert grown.scratch_info()["allocations"] > 0
        for key in ("scores", "sel", "store", "ks", "mscores"):
            assert np.array_equal(got[key], want[key]), key
        for a, b in zip(got["pk"] + got["pv"], want["pk"] + want["pv"]):
            assert np.array_equal(a, b)
        # a second pass at the same shapes still allocates nothing
        run_path(held, inputs)
        assert held.scratch_info() == before


def test_reserve_rejects_bad_shapes():
    announce("reserve argument checks")
    with kv.Context(0) as c:
        with pytest.raises(kv.KvMemError):
            c.reserve(n_head=25, n_head_kv=4)
        with pytest.raises(kv.KvMemError):
            c.reserve(head_dim=192)
        c.reserve()  # nothing asked, nothing reserved
        assert c.scratch_info()["allocations"] == 0


def test_h2d_async_pinned_and_pageable():
    announce("h2d_async: 3 MiB + 5 bytes pinned, 1 MiB pageable, n == 0, null pointers")
    rng = np.random.default_rng(34)
    n = (3 << 20) + 5
    src = torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)).pin_memory()
    dst = torch.zeros(n + 64, dtype=torch.uint8, device="cuda")
    page = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    dst2 = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()  # the destinations were cleared on torch's stream
    with kv.Context(0) as c:
        c.perf_enable(True)
        c.h2d_async(dst.data_ptr() + 64, src.data_ptr(), n)
        c.h2d_async(dst2.data_ptr(), page.ctypes.data, page.nbytes)
        c.h2d_async(0, 0, 0)
        with pytest.raises(kv.KvMemError):
            c.h2d_async(dst.data_ptr(), 0, 16)
        c.sync()
        perf = c.perf()
        assert perf["h2d_bytes"] == n + page.nbytes
        assert perf["n_copy"] == 2
    out = dst.cpu().numpy()
    assert (out[:64] == 0).all()
    assert np.array_equal(out[64:], src.numpy())
    assert np.array_equal(dst2.cpu().numpy(), page)
