"""The reselect engine (include/kvmem_host.h) on the GPU against the oracle.

One agent step = preview (device scorer + device top-k with the store's
sink / mandatory / recent charge) then apply (store diff, slot plan, one
stage-in launch).  Checked: scores within 1e-3 relative of the fp64
oracle, the selection equal to the oracle's top-k over the engine's own
scores, every selected block's pool rows bit-exact against the oracle's
quantizer, the stale-selection rule, canonical slot layout, a growing
partial tail block, stage-in from pinned host history, and a pinned-host
stage-in long enough to cycle the device upload ring many times.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

from engine_helpers import (E, HKV, HQ, D, L, RTOL, T, block_major_pinned, check_pool,  # noqa: E402,F401
                            decode_rows, history, make_engine, oracle_scores)


def announce(msg: str) -> None:
    print(f"[engine] {msg}", flush=True)


def test_engine_two_steps_vs_oracle(oracle):
    announce("two agent steps, 40 blocks, budget 8 + 4 reserve, K q8_0 / V q4_0")
    cap, nb = 48, 40
    k, v, q1 = history(cap, seed=31)
    q2 = (q1.float() * -1.0).to(torch.bfloat16)     # a different query direction
    with make_engine(8, 4, kv.TYPE_Q8_0, kv.TYPE_Q4_0, canonical_layout=0) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        assert eng.block_count() == nb
        sel1 = eng.preview(q1.data_ptr(), q1.shape[1])
        got_scores = np.array(eng.scores(), dtype=np.float64)
        want_scores = oracle_scores(oracle, q1, k, nb)
        rel = np.abs(got_scores - want_scores) / np.maximum(np.abs(want_scores), 1e-6)
        assert rel.max() <= RTOL, f"scores: max rel err {rel.max():.3e}"
        assert sel1.blocks == oracle.pick_topk(got_scores.astype(np.float32).astype(np.float64), 8, sink=1)
        st1 = eng.apply(sel1)
        assert st1["n_staged"] == 8 and st1["n_stage_in"] == 8
        check_pool(eng, oracle, k, v, sel1.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)

        sel2 = eng.preview(q2.data_ptr(), q2.shape[1])
        s2 = np.array(eng.scores(), dtype=np.float64)
        assert sel2.blocks == oracle.pick_topk(s2.astype(np.float32).astype(np.float64), 8, sink=1)
        st2 = eng.apply(sel2)
        new = set(sel2.blocks) - set(sel1.blocks)
        assert st2["n_staged"] == len(new)
        assert st2["selection_overlap_blocks"] == len(set(sel1.blocks) & set(sel2.blocks))
        check_pool(eng, oracle, k, v, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)
        # the stage-in slots came from the LIFO free list of the store mirror
        st = host.Store(T, 8, 1, 0, True, eng.n_slots())
        st.register_append(nb * T)
        st.apply(sel1.blocks)
        st.apply(sel2.blocks)
        assert st.blocks()["gpu_slot"] == eng.block_slots()


def test_engine_stale_selection():
    announce("stale selection after the history grows")
    cap = 12
    k, v, q = history(cap, seed=5)
    with make_engine(4, 2) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 10 * T)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        eng.append_tokens(T)
        with pytest.raises(kv.StaleSelection):
            eng.apply(sel)
        fresh = eng.preview(q.data_ptr(), q.shape[1])
        eng.apply(fresh)


@pytest.mark.parametrize("budget,reserve", [(10, 4), (24, 8)])
def test_engine_canonical_layout(oracle, budget, reserve):
    """Selected block i in slot i after each reselection; with 24 of 30
    blocks selected the resident blocks' moves form chains longer than one
    segment of the chain walk."""
    announce(f"canonical layout: selected block i in slot i (budget {budget})")
    cap, nb = 32, 30
    k, v, q1 = history(cap, seed=9)
    q2 = (q1.float() * -1.0).to(torch.bfloat16)
    with make_engine(budget, reserve, canonical_layout=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        for q in (q1, q2, q1):
            sel = eng.preview(q.data_ptr(), q.shape[1])
            eng.apply(sel)
            slots = eng.block_slots()
            assert [slots[b] for b in sel.blocks] == list(range(len(sel.blocks)))
            check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0)


def test_engine_partial_tail_grows(oracle):
    announce("partial tail block kept by recent=1, then grown and re-staged")
    cap = 16
    k, v, q = history(cap, seed=13)
    n_tok = 9 * T + 37
    with make_engine(4, 2, recent_blocks=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, n_tok)
        assert eng.block_count() == 10
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert 9 in sel.blocks and 0 in sel.blocks
        eng.apply(sel)
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 37 if b == 9 else T)
        eng.append_tokens(50)      # the tail now has 87 tokens
        sel = eng.preview(q.data_ptr(), q.shape[1])
        st = eng.apply(sel)
        assert st["n_staged"] >= 1
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 87 if b == 9 else T)


def test_engine_pinned_host_history(oracle):
    announce("stage-in from pinned host history")
    cap, nb = 24, 24
    k, v, q = history(cap, seed=17)
    hb = block_major_pinned(k, v, nb)
    with make_engine(12, 4, kv.TYPE_Q5_0, kv.TYPE_Q8_0) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        eng.set_host_history(hb.data_ptr(), nb)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        eng.apply(sel)
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q5_0, kv.TYPE_Q8_0)


@pytest.mark.parametrize("memory", ["pinned", "pageable"])
def test_stagein_host_many_ring_batches(ctx, oracle, memory):
    """A host-history stage-in of 47 blocks, K q8_0 / V q4_0.  From pinned
    memory the kernel reads the blocks itself in one launch; from pageable
    memory they go through five device-ring batches (regression: the
    per-call tables must stay valid through every batch)."""
    announce(f"{memory} host stage-in, 4 layers, 47 blocks, K q8_0 / V q4_0")
    Lh, Ek, Ev, nb, n_slots = 4, 2048, 1024, 60, 64
    rng = np.random.default_rng(21)
    kh = workloads.heavy_tailed(22, (nb, Lh, T, Ek))
    vh = workloads.heavy_tailed(23, (nb, Lh, T, Ev))
    span = Lh * T * (Ek + Ev)
    rows = np.concatenate([kh.reshape(nb, Lh, -1), vh.reshape(nb, Lh, -1)], axis=2).reshape(nb, span)
    if memory == "pinned":
        hb = torch.empty((nb, span), dtype=torch.int16, pin_memory=True)
        hb.copy_(torch.from_numpy(rows.view(np.int16)))
    else:
        hb = torch.from_numpy(np.ascontiguousarray(rows.view(np.int16)))
    ids = sorted(rng.choice(nb, 47, replace=False).tolist())
    slots = rng.permutation(n_slots)[:47].tolist()
    rbk, rbv = kv.row_size(kv.TYPE_Q8_0, Ek), kv.row_size(kv.TYPE_Q4_0, Ev)
    pk = [torch.zeros(n_slots * T * rbk, dtype=torch.uint8, device="cuda") for _ in range(Lh)]
    pv = [torch.zeros(n_slots * T * rbv, dtype=torch.uint8, device="cuda") for _ in range(Lh)]
    pool = ctx.make_pool(Lh, n_slots, T, Ek, Ev, kv.TYPE_Q8_0, kv.TYPE_Q4_0,
                         [p.data_ptr() for p in pk], [p.data_ptr() for p in pv])
    hh = kv.HostHistory(hb.data_ptr(), Lh, nb, T, Ek, Ev, 0)
    torch.cuda.synchronize()
    ctx.stagein_blocks_host(hh, pool, ids, slots)
    ctx.sync()
    for layer in range(Lh):
        gk = pk[layer].cpu().numpy().reshape(n_slots * T, rbk)
        gv = pv[layer].cpu().numpy().reshape(n_slots * T, rbv)
        for b, s in zip(ids, slots):
            assert np.array_equal(gk[s * T:(s + 1) * T], oracle.quantize_rows_f16(kv.TYPE_Q8_0, kh[b, layer]))
            assert np.array_equal(gv[s * T:(s + 1) * T], oracle.quantize_rows_f16(kv.TYPE_Q4_0, vh[b, layer]))


def test_engine_request_and_turn_spans(oracle):
    """Mandatory blocks from the request span / turn spans and force_pos
    (retrieval_mandatory) are charged in preview: the selection equals the
    oracle's top-k with those ids as the mandatory list."""
    announce("request span, turn spans and force_pos -> mandatory blocks")
    cap, nb, budget = 40, 40, 8
    k, v, q = history(cap, seed=37)
    with make_engine(budget, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        cases = [
            (lambda: eng.set_request_span(20 * T + 5, 23 * T, 3 * T + 1), [20, 21, 22, 3]),
            (lambda: eng.set_request_span(37 * T, 0, -1), [37, 38, 39]),
            (lambda: eng.set_turn_spans(query=[(0, 10)], mandatory=[(35 * T, 36 * T + 1), (2, 3)]),
             [0, 35, 36]),
            (lambda: eng.set_request_span(-1, 0, -1), []),
        ]
        for set_span, want_mand in cases:
            set_span()
            mand = eng.retrieval_mandatory()
            assert mand == want_mand
            sel = eng.preview(q.data_ptr(), q.shape[1])
            s = np.array(eng.scores(), dtype=np.float64).astype(np.float32).astype(np.float64)
            assert sel.blocks == oracle.pick_topk(s, budget, sink=1, mandatory=mand)
            assert set(want_mand) <= set(sel.blocks)
            eng.apply(sel)
            check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
        with pytest.raises(kv.KvMemError):
            eng.set_turn_spans(query=[(5, 4)])


def test_engine_own_pool_starts_cleared():
    """The engine's own pool is zero before any stage-in, as llama.cpp
    clears its KV cache buffers: cells that no stage-in or decode has
    written (free slots, rows past a partial tail) hold no NaN bits for the
    attention that reads them under a mask.  The same after set_pool(NULL)
    replaces a borrowed pool with a new own one."""
    announce("own pool cleared at creation and after set_pool(NULL)")
    with make_engine(6, 2, kv.TYPE_Q8_0, kv.TYPE_Q4_0) as eng:
        ctx = kv.Context(0)
        try:
            def all_zero() -> bool:
                for layer in range(L):
                    for ptr, ty in zip(eng.pool_layer(layer), (kv.TYPE_Q8_0, kv.TYPE_Q4_0)):
                        n = eng.n_slots() * T * kv.row_size(ty, E)
                        buf = torch.full((n,), 0xA5, dtype=torch.uint8, device="cuda")
                        torch.cuda.synchronize()
                        ctx.d2d_batched([ptr], [buf.data_ptr()], [n])
                        ctx.sync()
                        if bool(buf.any()):
                            return False
                return True

            assert all_zero()
            n = eng.n_slots() * T * kv.row_size(kv.TYPE_Q8_0, E)
            borrowed = [torch.full((n,), 0x7F, dtype=torch.uint8, device="cuda") for _ in range(2 * L)]
            torch.cuda.synchronize()
            eng.set_pool([t.data_ptr() for t in borrowed[:L]], [t.data_ptr() for t in borrowed[L:]])
            eng.set_pool(None)
            assert all_zero()
        finally:
            ctx.close()


@pytest.mark.parametrize("scorer", [0, 1], ids=["per_token_max", "mean_k"])
def test_engine_scores_when_every_block_fits(oracle, scorer):
    """A budget that takes every block still scores them: the preview's
    scores are this preview's (the reference scores before it selects,
    llama-memory-kvmem.cpp:3047-3067), within 1e-3 of the fp64 oracle for
    the per-token scorer, and not those of an earlier, larger history."""
    announce(f"every block fits the budget: scores still computed (scorer {scorer})")
    cap = 12
    k, v, q = history(cap, seed=23)
    with make_engine(8, 2, scorer=scorer) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 12 * T)
        sel = eng.preview(q.data_ptr(), q.shape[1])          # 12 blocks, budget 8: scored
        assert len(sel.blocks) == 8
        eng.truncate_to(5 * T + 40)                          # 6 blocks: all fit
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert sel.blocks == list(range(6))
        got = np.array(eng.scores(), dtype=np.float64)
        assert np.all(got != 0.0)
        if scorer == 0:
            want = oracle_scores(oracle, q, k, 6, last_T=40)
            rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-6)
            assert rel.max() <= RTOL, f"max rel err {rel.max():.3e}"
        eng.apply(sel)
        st = eng.apply_retrieval(q.data_ptr(), q.shape[1])   # all fit: the host path
        assert st["n_staged"] == 0
        again = np.array(eng.scores(), dtype=np.float64)
        assert np.array_equal(again, got)


def test_engine_second_grown_tail_evicts_the_first(oracle):
    """The engine marks one block whose pool rows are stale.  A resident
    partial tail grows (block 2: 40 rows in the pool, 128 in the history);
    rows decoded after it go into a new block (3) that takes a slot; block 3
    then grows too.  Block 2 leaves the pool rather than lose its mark, and
    the next apply stages both again: every row bit-exact, none stale."""
    announce("a second grown tail: the first leaves the pool and is staged again")
    cap = 8
    k, v, q = history(cap, seed=29)
    with make_engine(6, 2) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 2 * T + 40)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert sel.blocks == [0, 1, 2]
        eng.apply(sel)
        eng.append_tokens(T - 40)                       # block 2 full in the history, stale in the pool
        decode_rows(eng, k, v, 3 * T, 3 * T + 50)       # block 3 takes a slot, its 50 rows written
        assert eng.block_slots()[3] >= 0
        before = eng.attention_epoch()
        eng.append_tokens(30)                           # block 3 grows: block 2 leaves the pool
        slots = eng.block_slots()
        assert slots[2] == -1 and slots[3] >= 0, slots
        assert eng.attention_epoch() > before
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert sel.blocks == [0, 1, 2, 3]
        st = eng.apply(sel)
        assert st["n_staged"] == 2                      # blocks 2 and 3, both whole again
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 80 if b == 3 else T)
