"""Continuation checks of the two-phase API on the host store (no GPU).

The adapter's attention_view / selection_fits / commit_unchanged /
commit_resident / can_append (src/adapter/llama-memory-kvmem.cpp:2982-3024,
3069-3102) run in this library's host C++ over the store and a pool state.
The engine calls the same functions with its device pool; here the store
alone stands in for it (a block holding a slot is complete).  Pinned by:
  - the reference's own expectations of these calls in its GPU test
    (tests/mtp-kv-test.cpp:334-361): an identical attention view is
    accepted, a selection with its mandatory tail trimmed does not fit, an
    oversized generation reserve cannot append, and after a restore the old
    view and selection are stale;
  - closed forms for every condition of each check and every reason string
    of can_append, worked out by hand on small stores;
  - the attention epoch: appended rows never move it; cuts and applies that
    change the working set do;
  - where oracle/_ref is built, the reference's own KvMemStore::
    prefill_needs_offload (can_append's pressure test) and KvMemRuntime::
    commit_resident_selection (what commit_unchanged / commit_resident end
    in), live over random and edge inputs.
"""
from __future__ import annotations

import pytest

from conftest import load_pkg

kv = load_pkg()
from kvmem_amd import host  # noqa: E402


def make_store(bt=32, budget=64, n_slots=40, **kw):
    return host.Store(block_tokens=bt, budget_blocks=budget, sink_blocks=1, recent_blocks=0,
                      n_slots=n_slots, **kw)


def preview(st, mandatory=()):
    return host.Selection(st.epoch(), st.total_tokens(), st.pick_topk_blocks(mandatory))


def test_reference_logits_fixture_flow():
    """mtp-kv-test.cpp:300-361 on the store: prefill to the query start,
    take the view, decode the 24 query rows, preview with the query span
    mandatory, then the checks the reference test requires."""
    bt, end = 32, 600
    query = end - 24
    st = make_store(bt=bt, budget=64, n_slots=40)
    st.append_resident(query)                   # decode(0, query): rows land in the pool
    before = st.attention_view()
    assert before.valid and before.rows == query
    assert before.blocks == list(range((query + bt - 1) // bt))
    st.append_resident(end - query)             # decode(query, end)
    mandatory = st.blocks_overlapping([(query, end)])
    sel = preview(st, mandatory)
    assert sel.blocks == list(range((end + bt - 1) // bt))   # everything fits the budget
    assert st.commit_unchanged(before, sel), "identical attention view rejected"
    assert st.blocks()["in_ws"] == [1] * st.block_count()
    trimmed = host.Selection(sel.epoch, sel.rows, sel.blocks[:-1])
    assert not st.selection_fits(trimmed, end, 0, mandatory), "trimmed mandatory tail accepted"
    assert st.selection_fits(sel, end, 0, mandatory)
    ok, why = st.can_append(end, 40 * bt, True)
    assert not ok and why == "insufficient_slots", "oversized generation reserve accepted"
    # restore the checkpoint at the query start and remove the suffix
    st.truncate_to(query)
    assert not st.commit_unchanged(before, sel), "stale attention view accepted after restore"
    assert st.epoch() != sel.epoch, "stale selection accepted after restore"
    # replay the query rows; a fresh preview is current again, the old view is not
    st.append_resident(end - query)
    again = preview(st, mandatory)
    assert again.blocks == sel.blocks and again.epoch == st.epoch()
    assert not st.commit_unchanged(before, again)
    assert st.commit_unchanged(st.attention_view(), again)


def test_attention_epoch_moves_with_the_pool_not_with_rows():
    st = make_store(bt=4, budget=3, n_slots=4)
    e0 = st.epoch()
    st.register_append(10)
    assert st.epoch() == e0
    st.append_resident(3)
    assert st.epoch() == e0
    st.apply([0, 1, 2])                         # stage-in and stage-out: moves
    e1 = st.epoch()
    assert e1 > e0
    st.apply([0, 1, 2])                         # the same working set: no change
    assert st.epoch() == e1
    st.truncate_to(st.total_tokens())           # cuts nothing
    assert st.epoch() == e1
    st.truncate_to(9)
    assert st.epoch() > e1


def test_append_resident_slots_and_refusal():
    st = make_store(bt=4, budget=8, n_slots=3)
    st.register_append(6)                       # blocks 0 (full), 1 (2 rows), no slots
    st.append_resident(5)                       # tail 1 takes a slot, new block 2 (3 rows) too
    b = st.blocks()
    assert b["gpu_slot"] == [-1, 0, 1] and b["tier"] == [1, 0, 0]
    assert st.total_tokens() == 11
    with pytest.raises(kv.KvMemError):          # block 3 and 4 need two slots; one is free
        st.append_resident(6)
    assert st.total_tokens() == 11 and st.blocks()["gpu_slot"] == [-1, 0, 1]
    st.append_resident(5)                       # fills block 2, opens block 3 in the last slot
    assert st.blocks()["gpu_slot"] == [-1, 0, 1, 2]


def test_attention_view_validity():
    st = make_store(bt=4, budget=4, n_slots=6)
    st.register_append(24)                      # 6 blocks, none resident
    v = st.attention_view()
    assert v.valid and v.blocks == [] and v.rows == 24
    st.apply([0, 2, 4])                         # LIFO slots 0, 1, 2 in stage-in order
    assert st.blocks()["gpu_slot"][:5] == [0, -1, 1, -1, 2]
    assert st.attention_view(canonical=False) == host.AttentionView(st.epoch(), 24, True, [0, 2, 4])
    assert st.attention_view(canonical=True).valid          # i-th resident block in slot i
    st.apply([0, 1, 2, 4])                      # block 1 takes slot 3
    assert st.blocks()["gpu_slot"][:5] == [0, 3, 1, -1, 2]
    assert not st.attention_view(canonical=True).valid
    assert st.attention_view(canonical=False).valid


def test_selection_fits_closed_forms():
    bt = 4
    st = make_store(bt=bt, budget=5, n_slots=6)
    st.register_append(40)                      # 10 blocks
    sel = host.Selection(st.epoch(), 40, [0, 7, 8, 9])
    # first = 40/4 = 10; rows [40, 48) add blocks 10, 11: 4 + 2 = 6 <= 6
    assert st.selection_fits(sel, 40, 8)
    assert not st.selection_fits(sel, 40, 9)    # block 12 too: 7 > 6
    assert st.selection_fits(sel, 44, 4)
    assert not st.selection_fits(sel, 39, 0)    # end < rows
    assert not st.selection_fits(host.Selection(sel.epoch + 1, 40, sel.blocks), 40, 0)
    assert not st.selection_fits(host.Selection(sel.epoch, 36, sel.blocks), 40, 0)
    assert st.selection_fits(sel, 40, 0, mandatory=[7, 9])
    assert not st.selection_fits(sel, 40, 0, mandatory=[6])
    # final - first beyond the pool on its own
    assert not st.selection_fits(host.Selection(sel.epoch, 40, []), 40, 7 * bt)
    # a selection that already holds the continuation blocks counts them once
    st.register_append(8)                       # rows 48, blocks 10, 11
    sel2 = host.Selection(st.epoch(), 48, [0, 8, 9, 10, 11])
    assert st.selection_fits(sel2, 48, 4)       # block 12 is the one extra: 6 <= 6
    assert not st.selection_fits(sel2, 48, 5)   # 13 too


def test_commit_unchanged_closed_forms():
    st = make_store(bt=4, budget=3, n_slots=4)
    st.register_append(16)                      # 4 blocks
    st.apply([0, 1, 2])
    view = st.attention_view()
    sel = host.Selection(st.epoch(), 16, [0, 1, 2])
    bad_valid = host.AttentionView(view.epoch, view.rows, False, view.blocks)
    assert not st.commit_unchanged(bad_valid, sel)
    assert not st.commit_unchanged(host.AttentionView(view.epoch - 1, 16, True, view.blocks), sel)
    assert not st.commit_unchanged(host.AttentionView(view.epoch, 17, True, view.blocks), sel)
    assert not st.commit_unchanged(view, host.Selection(sel.epoch, 15, sel.blocks))
    assert not st.commit_unchanged(view, host.Selection(sel.epoch, 16, [0, 1, 3]))   # not the pool
    assert not st.commit_unchanged(host.AttentionView(view.epoch, 16, True, [0, 1, 2, 3]), sel)
    assert st.commit_unchanged(view, sel)
    assert st.blocks()["in_ws"] == [1, 1, 1, 0]
    # non-canonical pools are never "unchanged"
    st.apply([0, 2, 3])                         # block 3 takes slot 1 (freed by block 1)
    v2 = st.attention_view(canonical=False)
    assert v2.valid and not st.attention_view().valid
    assert not st.commit_unchanged(v2, host.Selection(st.epoch(), 16, [0, 2, 3]))


def test_commit_resident():
    st = make_store(bt=4, budget=3, n_slots=4)
    st.register_append(16)
    st.apply([0, 2, 3])
    st.apply([0, 1, 2])                         # block 1 lands in slot 2: not canonical
    assert not st.commit_resident_selection([0, 2])
    st.append_resident(2)                       # block 4 takes the last slot
    assert st.blocks()["in_ws"] == [1, 1, 1, 0, 0]
    assert st.commit_resident_selection([0, 1, 2, 4])
    assert st.blocks()["in_ws"] == [1, 1, 1, 0, 1]


def test_can_append_reasons():
    bt = 4
    st = make_store(bt=bt, budget=4, n_slots=6)
    assert st.can_append(0, 0, False) == (True, "same_query")
    assert st.can_append(0, 0, True) == (True, "all_resident")
    st.append_resident(12)                      # 3 resident blocks in slots 0..2
    assert st.can_append(11, 0, False) == (False, "invalid_boundary")
    assert st.can_append(12, 0, True) == (True, "all_resident")
    assert st.can_append(16, 0, True) == (True, "all_resident")       # end_blocks 4 = budget
    assert st.can_append(17, 0, True) == (False, "selection_budget")
    # resident 12 + incoming 11 = 23 > max(0.95 * 24 = 22, 4): prefill pressure
    big = make_store(bt=bt, budget=8, n_slots=6)
    big.append_resident(12)
    assert big.can_append(22, 0, True) == (True, "all_resident")
    assert big.can_append(23, 0, True) == (False, "prefill_pressure")
    assert big.can_append(23, 0, False) == (True, "same_query")
    # slots: 3 free; rows [12, 12 + g) need ceil(g / 4) new blocks
    assert st.can_append(12, 12, False) == (True, "same_query")
    assert st.can_append(12, 13, False) == (False, "insufficient_slots")
    # final_blocks beyond every slot and block together
    assert st.can_append(12, 4 * (6 + 3) - 12 + 1, False) == (False, "insufficient_slots")
    # history_not_resident: a block without a slot
    st.register_append(4)                       # block 3, not in the pool
    assert st.can_append(16, 0, True) == (False, "history_not_resident")
    assert st.can_append(16, 0, False) == (True, "same_query")
    # partial_tail_missing: the partial tail holds no slot
    st.register_append(2)                       # block 4 with 2 rows
    assert st.can_append(18, 0, False) == (False, "partial_tail_missing")
    # coverage_or_layout: the canonical view is broken
    lay = make_store(bt=bt, budget=4, n_slots=6)
    lay.register_append(16)
    lay.apply([0, 2])
    lay.apply([0, 1, 2])                        # block 1 in slot 2, block 2 in slot 1
    assert lay.can_append(16, 0, True) == (False, "coverage_or_layout")
    assert lay.can_append(16, 0, False) == (True, "same_query")


def test_query_replay_fits_closed_forms():
    """query_replay_fits (llama-memory-kvmem.cpp:3502-3524): the blocks from
    the query's first block to the prompt's end plus the sink must fit the
    budget; a query starting inside the sink needs every block."""
    bt = 4
    st = make_store(bt=bt, budget=5, n_slots=8)     # sink 1
    assert st.query_replay_fits(40, 40) and st.query_replay_fits(41, 40)   # empty
    assert st.query_replay_fits(32, 40)             # blocks 8, 9 + sink = 3
    assert st.query_replay_fits(24, 40)             # 6..9 + sink = 5
    assert not st.query_replay_fits(20, 40)         # 5..9 + sink = 6
    assert st.query_replay_fits(39, 40)             # block 9 + sink
    assert not st.query_replay_fits(0, 40)          # inside the sink: all 10 blocks
    assert st.query_replay_fits(0, 20)              # all 5 blocks
    assert st.query_replay_fits(3, 17)              # inside the sink: 17 rows = 5 blocks
    assert not st.query_replay_fits(3, 21)          # 21 rows = 6 blocks
    assert make_store(bt=bt, budget=0, n_slots=8).query_replay_fits(0, 400)   # no budget


def test_free_slots_follow_the_lifo_list():
    st = make_store(bt=4, budget=3, n_slots=5)
    assert st.free_slots() == 5
    st.register_append(20)
    st.apply([0, 1, 2])
    assert st.free_slots() == 2
    st.append_resident(4)                           # block 5 takes a slot
    assert st.free_slots() == 1
    st.truncate_to(12)                              # blocks 3.. gone, block 5's slot freed
    assert st.free_slots() == 2


REF = __import__("conftest").ROOT / "oracle" / "_ref" / "libkvmem_ref.so"


def _ref_lib():
    import ctypes as C
    ref = C.CDLL(str(REF))
    pu32 = C.POINTER(C.c_uint32)
    ref.kref_prefill_needs_offload.argtypes = [C.c_uint32] * 4
    ref.kref_runtime_new.restype = C.c_void_p
    ref.kref_runtime_new.argtypes = [C.c_uint32] * 6
    ref.kref_runtime_free.argtypes = [C.c_void_p]
    ref.kref_runtime_apply.argtypes = [C.c_void_p, pu32, C.c_uint32, pu32, pu32, pu32, pu32, pu32]
    ref.kref_runtime_commit_resident.argtypes = [C.c_void_p, pu32, C.c_uint32]
    ref.kref_runtime_blocks.restype = C.c_uint32
    ref.kref_runtime_blocks.argtypes = [C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_uint8),
                                        C.POINTER(C.c_uint8), C.POINTER(C.c_int64)]
    return ref


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (needs the reference tree)")
def test_prefill_needs_offload_matches_the_reference_library():
    """can_append's prefill-pressure test against the reference's own
    KvMemStore::prefill_needs_offload, on the watermark's edges and at
    random."""
    import numpy as np
    ref = _ref_lib()
    rng = np.random.default_rng(12)
    n = 0
    for bt in (16, 32, 128):
        st = make_store(bt=bt)
        cases = [(0, 0, 0), (5, 0, 100), (0, 5, 0), (0, bt, bt), (0, bt + 1, bt), (10, 1, 10)]
        for pool in (bt, 7 * bt, 384 * bt, 49152, 40000):
            w = max(int(pool * 0.95), bt)
            for r in (0, 1, w // 2):
                for inc in (w - r - 1, w - r, w - r + 1, pool - r, pool - r + 1):
                    if inc >= 0:
                        cases.append((r, inc, pool))
        cases += [tuple(int(x) for x in rng.integers(0, 60000, 3)) for _ in range(500)]
        for r, inc, pool in cases:
            assert st.prefill_needs_offload(r, inc, pool) == bool(ref.kref_prefill_needs_offload(bt, r, inc, pool)), \
                (bt, r, inc, pool)
            n += 1
    assert n > 1500


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (needs the reference tree)")
def test_commit_resident_selection_matches_the_reference_library():
    """commit_resident_selection after random applies: the same accept or
    refuse, and the same working-set flags, as the reference's own runtime
    for the resident set itself, a trimmed one, one with an extra block and
    an unsorted one."""
    import ctypes as C
    import numpy as np
    ref = _ref_lib()
    rng = np.random.default_rng(21)
    bt, nb, budget, n_slots = 16, 40, 12, 16
    for trial in range(30):
        st = make_store(bt=bt, budget=budget, n_slots=n_slots)
        st.register_append(nb * bt)
        h = ref.kref_runtime_new(bt, budget, 1, 0, n_slots, nb * bt)
        try:
            for step in range(4):
                sel = sorted(rng.choice(nb, int(rng.integers(1, budget + 1)), replace=False).tolist())
                st.apply(sel)
                arr = (C.c_uint32 * nb)(*sel)
                si, so, ctr = (C.c_uint32 * nb)(), (C.c_uint32 * nb)(), (C.c_uint32 * 5)()
                ni, no = C.c_uint32(), C.c_uint32()
                ref.kref_runtime_apply(h, arr, len(sel), si, C.byref(ni), so, C.byref(no), ctr)
                resident = [b for b, s in enumerate(st.blocks()["gpu_slot"]) if s >= 0]
                extra = sorted(set(resident) | {int(rng.integers(0, nb))})
                for cand in (resident, resident[:-1], extra, resident[::-1]):
                    a = (C.c_uint32 * max(1, len(cand)))(*cand)
                    want = bool(ref.kref_runtime_commit_resident(h, a, len(cand)))
                    assert st.commit_resident_selection(cand) == want, (trial, step, cand)
                gs, tr = (C.c_int32 * nb)(), (C.c_uint8 * nb)()
                ws, bk = (C.c_uint8 * nb)(), (C.c_int64 * nb)()
                ref.kref_runtime_blocks(h, gs, tr, ws, bk)
                b = st.blocks()
                assert b["in_ws"] == list(ws) and b["gpu_slot"] == list(gs), (trial, step)
        finally:
            ref.kref_runtime_free(h)
