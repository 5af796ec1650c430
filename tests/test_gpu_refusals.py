"""Every device entry point of include/kvmem_hip.h refuses bad arguments on
the host, before anything is issued.

One context meets a table of calls that break each entry point's stated
limits: null pointers and empty ops, misaligned buffers, block ids, slots,
token rows, forced ids and window rows out of range, token counts above
the block, geometry that does not match (head grouping, row width,
capacity below the block count, a pool of other layers), unsupported
types, head sizes and layer counts.  Each call must return the documented
status (KVMEM_HIP_ERR_INVALID or _UNSUPPORTED) with kvmem_hip_last_error
naming the entry point or the argument; afterwards the context's stream
holds no error, every output and pool buffer still holds its sentinel
bytes, and valid calls on the same context work (a stage-in bit-exact
against the oracle, a score).  Each refused case was checked against the
entry point's source to be refused before its first launch or copy.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import workloads  # noqa: E402

L, B, T, HKV, HQ, D = 2, 4, 128, 4, 24, 256
E = HKV * D
EQ = HQ * D
SLOTS = 4
INV, UNS = kv.ERR_INVALID, kv.ERR_UNSUPPORTED


def announce(msg: str) -> None:
    print(f"[refusals] {msg}", flush=True)


def test_entry_points_refuse_bad_arguments(oracle):
    announce("refusal table over every device entry point")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=8, seed=3, with_v=True)
    rk = kv.row_size(kv.TYPE_Q8_0, E)
    pool_k = [torch.full((SLOTS * T * rk,), 0x5A, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pool_v = [torch.full((SLOTS * T * rk,), 0x5A, dtype=torch.uint8, device="cuda") for _ in range(L)]
    scores = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda")
    k_sum = torch.full((L, B, E), -9.0, dtype=torch.float32, device="cuda")
    mean_t = torch.full((L, B), 77, dtype=torch.int32, device="cuda")
    acc = torch.full((E,), -9.0, dtype=torch.float32, device="cuda")
    qf = torch.randn((L, 8, EQ), dtype=torch.float32, device="cuda")
    q_sum = torch.full((L, EQ), -9.0, dtype=torch.float32, device="cuda")
    window = torch.full((16, EQ), -9.0, dtype=torch.float32, device="cuda")
    copy_dst = torch.full((64,), 0x11, dtype=torch.uint8, device="cuda")
    pinned_hist = torch.zeros((B, L * 2 * T * E), dtype=torch.float16, pin_memory=True)
    packed = torch.full((B * L * T * 2 * rk,), 0x33, dtype=torch.uint8, pin_memory=True)
    pageable = np.zeros(B * L * 2 * T * E, dtype=np.float16)
    host_src = torch.zeros(64, dtype=torch.uint8, pin_memory=True)
    torch.cuda.synchronize()
    sentinels = [(t, t.clone()) for t in (*pool_k, *pool_v, k_sum, mean_t, acc, q_sum, window, copy_dst)]
    packed0 = packed.clone()

    with kv.Context(0) as ctx:
        hist = ctx.make_history(k.data_ptr(), v.data_ptr(), L, B, T, E, E)
        pool = ctx.make_pool(L, SLOTS, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                             [t.data_ptr() for t in pool_k], [t.data_ptr() for t in pool_v])
        hh = kv.HostHistory(pinned_hist.data_ptr(), L, B, T, E, E, 0)
        ph = kv.PackedHost(packed.data_ptr(), L, B, T)

        def with_hist(**kw):
            a = dict(k_ptr=k.data_ptr(), v_ptr=v.data_ptr(), n_layers=L, n_blocks=B, block_tokens=T,
                     n_embd_k=E, n_embd_v=E)
            a.update(kw)
            return ctx.make_history(**a)

        def with_pool(n_layers=L, type_k=kv.TYPE_Q8_0):
            return ctx.make_pool(n_layers, SLOTS, T, E, E, type_k, kv.TYPE_Q8_0,
                                 [pool_k[i % L].data_ptr() for i in range(n_layers)],
                                 [pool_v[i % L].data_ptr() for i in range(n_layers)])

        def score(hist_=hist, q_ptr=q.data_ptr(), q_type=kv.TYPE_BF16, n_q=8, n_head_kv=HKV, head_dim=D,
                  reduce=kv.LAYER_MEAN, fn="score"):
            getattr(ctx, fn)(hist_, q_ptr, q_type, n_q, HQ, n_head_kv, head_dim, scores.data_ptr(),
                             layer_reduce=reduce)

        # (call, status, a word the message holds)
        cases = [
            (lambda: ctx.h2d_async(0, host_src.data_ptr(), 16), INV, "null"),
            (lambda: ctx.d2d_batched([k.data_ptr()], [copy_dst.data_ptr()], [0]), INV, "empty op"),
            (lambda: ctx.d2d_batched([0], [copy_dst.data_ptr()], [16]), INV, "null"),
            (lambda: ctx.reserve(n_layers=L, n_blocks=B, n_head=HQ, n_head_kv=5, head_dim=D), INV, "multiple"),
            (lambda: ctx.reserve(n_layers=L, n_blocks=B, n_head=HQ, n_head_kv=HKV, head_dim=64), UNS, "head_dim"),
            (lambda: ctx.stagein_quant([(k.data_ptr(), pool_k[0].data_ptr(), 4, 48, kv.TYPE_Q8_0)]), INV, "n_embd"),
            (lambda: ctx.stagein_quant([(k.data_ptr(), pool_k[0].data_ptr(), 4, E, 3)]), UNS, "type"),
            (lambda: ctx.stagein_quant([(k.data_ptr() + 2, pool_k[0].data_ptr(), 4, E, kv.TYPE_Q8_0)]), INV,
             "aligned"),
            (lambda: ctx.stagein_blocks(hist, pool, [B], [0]), INV, "out of range"),
            (lambda: ctx.stagein_blocks(hist, pool, [0], [SLOTS]), INV, "out of range"),
            (lambda: ctx.stagein_blocks(with_hist(capacity_blocks=B - 1), pool, [0], [0]), INV, "capacity"),
            (lambda: ctx.stagein_blocks(with_hist(k_ptr=k.data_ptr() + 2), pool, [0], [0]), INV, "alignment"),
            (lambda: ctx.stagein_blocks(hist, with_pool(n_layers=L + 1), [0], [0]), INV, "geometry"),
            (lambda: ctx.stagein_blocks(hist, with_pool(type_k=3), [0], [0]), UNS, "type"),
            (lambda: ctx.stagein_blocks_host(hh, pool, [B], [0]), INV, "out of range"),
            (lambda: ctx.stagein_blocks_host(hh, pool, [0], [SLOTS]), INV, "out of range"),
            (lambda: ctx.move_slots(pool, [0], [SLOTS]), INV, "out of range"),
            (lambda: ctx.move_slots(pool, [0], [1], [T + 1]), INV, "n_tokens"),
            (lambda: ctx.stageout_blocks(pool, ph, [B], [0], [T]), INV, "out of range"),
            (lambda: ctx.stageout_blocks(pool, ph, [0], [0], [T + 1]), INV, "out of range"),
            (lambda: ctx.stagein_packed_host(ph, pool, [0], [SLOTS], [T]), INV, "out of range"),
            (lambda: score(head_dim=64), UNS, "head_dim"),
            (lambda: score(n_head_kv=2), INV, "n_embd_k"),
            (lambda: score(hist_=with_hist(last_block_tokens=T + 1)), UNS, "block_tokens"),
            (lambda: score(q_ptr=q.data_ptr() + 2), INV, "aligned"),
            (lambda: score(q_type=kv.TYPE_F32), UNS, "bf16"),
            (lambda: score(reduce=7), INV, "layer_reduce"),
            (lambda: score(n_q=0), INV, "multiple"),
            (lambda: score(head_dim=64, fn="score_noalloc"), UNS, "head_dim"),
            (lambda: ctx.topk(scores.data_ptr(), B, 2, forced=[B]), INV, "forced"),
            (lambda: ctx.topk(scores.data_ptr(), (1 << 20) + 1, 1), UNS, "1048576"),
            (lambda: ctx.meank_sums(hist, [B], k_sum.data_ptr(), mean_t.data_ptr()), INV, "out of range"),
            (lambda: ctx.meank_sums(with_hist(last_block_tokens=T + 1), [0], k_sum.data_ptr(), mean_t.data_ptr()),
             INV, "last_block_tokens"),
            (lambda: ctx.meank_sums(with_hist(n_embd_k=E - 4), [0], k_sum.data_ptr(), mean_t.data_ptr()), INV,
             "multiple of 8"),
            (lambda: ctx.meank_sums(hist, [0], k_sum.data_ptr() + 4, mean_t.data_ptr()), INV, "aligned"),
            (lambda: ctx.meank_sums_host(kv.HostHistory(pageable.ctypes.data, L, B, T, E, E, 0), [0],
                                         k_sum.data_ptr(), mean_t.data_ptr()), UNS, "pinned"),
            (lambda: ctx.meank_add(k.data_ptr(), kv.TYPE_Q8_0, E, D, 2, D * 2, E * 2, 0, 4, acc.data_ptr()), UNS,
             "k_type"),
            (lambda: ctx.meank_add(k.data_ptr(), kv.TYPE_F16, 1000, D, 2, D * 2, E * 2, 0, 4, acc.data_ptr()),
             INV, "geometry"),
            (lambda: ctx.meank_add(k.data_ptr(), kv.TYPE_F16, E, D, 2, 3, E * 2, 0, 4, acc.data_ptr()), INV,
             "strides"),
            (lambda: ctx.q_accumulate(qf.data_ptr(), kv.TYPE_F32, L, 8, EQ, q_sum.data_ptr(), tokens=[8]), INV,
             "out of range"),
            (lambda: ctx.q_accumulate(qf.data_ptr(), kv.TYPE_Q8_0, L, 8, EQ, q_sum.data_ptr()), UNS, "q_type"),
            (lambda: ctx.q_window_write(q.data_ptr(), kv.TYPE_BF16, HQ, D, 2, D * 2, EQ * 2, [0], [16],
                                        window.data_ptr(), 16), INV, "capacity"),
            (lambda: ctx.q_window_write(q.data_ptr(), kv.TYPE_BF16, HQ, D, 2, D * 2, EQ * 2, [0, 1], [3, 3],
                                        window.data_ptr(), 16), INV, "twice"),
            (lambda: ctx.q_window_gather(window.data_ptr(), 1, 16, EQ, [16], kv.TYPE_F32, q_sum.data_ptr()), INV,
             "capacity"),
            (lambda: ctx.score_meank(q_sum.data_ptr(), [8] * L, k_sum.data_ptr(), mean_t.data_ptr(), L, B, HQ, 5, D,
                                     scores.data_ptr()), INV, "geometry"),
            (lambda: ctx.score_meank(q_sum.data_ptr(), [8] * L, k_sum.data_ptr(), mean_t.data_ptr(), L, B, HQ, HKV,
                                     64, scores.data_ptr()), INV, "geometry"),
            (lambda: ctx.score_meank(q_sum.data_ptr(), [8] * L, k_sum.data_ptr(), mean_t.data_ptr(), L, B, HQ, HKV,
                                     D, scores.data_ptr(), capacity_blocks=B - 1), INV, "geometry"),
            (lambda: ctx.score_meank(q_sum.data_ptr(), [8] * 257, k_sum.data_ptr(), mean_t.data_ptr(), 257, B, HQ,
                                     HKV, D, scores.data_ptr()), UNS, "256 layers"),
        ]
        for i, (call, code, word) in enumerate(cases):
            with pytest.raises(kv.KvMemError) as ex:
                call()
            assert ex.value.code == code, f"case {i}: {ex.value}"
            assert word in ctx.last_error(), f"case {i}: {ctx.last_error()!r} lacks {word!r}"
        announce(f"{len(cases)} calls refused")

        ctx.sync()
        torch.cuda.synchronize()
        for t, before in sentinels:
            assert torch.equal(t, before), "a refused call wrote device memory"
        assert torch.isnan(scores).all(), "a refused call wrote scores"
        assert torch.equal(packed, packed0), "a refused call wrote the packed store"

        # the context still works
        ctx.stagein_blocks(hist, pool, [1], [2])
        score()
        ctx.sync()
        kb = workloads.to_bits(torch, k)
        got = pool_k[0].cpu().numpy().reshape(SLOTS * T, rk)[2 * T:3 * T]
        assert np.array_equal(got, oracle.quantize_rows_f16(kv.TYPE_Q8_0, kb[0, 1].reshape(T, E)))
        assert torch.isfinite(scores).all()
