"""The host store of libkvmem_hip.so (no GPU) against the reference.

  - the reference library's own multi-step sequences (golden fixture made
    from kvmem/src/host/kvmem_store.cpp + kvmem_runtime.cpp): selection,
    stage_in / stage_out, plan counters, per-block slot / tier /
    working-set flag / baked position after every step;
  - the reference's unit-test cases for this path, restated
    (kvmem/tests/kvmem_store_test.cpp, kvmem_runtime_test.cpp);
  - where oracle/_ref is built, a live randomized cross-check.
"""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT, load_pkg

kv = load_pkg()
from kvmem_amd import host  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"
REF = ROOT / "oracle" / "_ref" / "libkvmem_ref.so"


def test_golden_reference_sequences():
    sc_all = json.loads((GOLDEN / "select_sequences.json").read_text())["scenarios"]
    steps = 0
    for sc in sc_all:
        st = host.Store(sc["block_tokens"], sc["budget_blocks"], sc["sink"], sc["recent"],
                        tie_lower_index=False, n_slots=sc["n_slots"])
        st.register_append(sc["n_tokens"])
        for s in sc["steps"]:
            st.set_retrieval_scores(s["scores"])
            sel = st.pick_topk_blocks(s["mandatory"])
            assert sel == s["selection"]
            stage_in, stage_out, stats = st.apply(sel)
            assert stage_in == s["stage_in"] and stage_out == s["stage_out"]
            for k, v in s["counters"].items():
                assert stats[k] == v, k
            b = st.blocks()
            assert b["gpu_slot"] == s["gpu_slot"]
            assert b["tier"] == s["tier"]
            assert b["in_ws"] == s["in_ws"]
            assert b["baked_pos"] == s["baked_pos"]
            steps += 1
    assert steps >= 100


# ------------------------------------------- reference unit tests, restated
def test_register_append_partial_blocks():
    """kvmem_store_test.cpp:25-51."""
    st = host.Store(128, 4, 1, 0)
    st.register_append(100)
    assert st.block_count() == 1
    st.register_append(50)
    assert st.block_count() == 2 and st.total_tokens() == 150
    st.register_append(384)
    assert st.block_count() == 5 and st.total_tokens() == 534


def test_selection_diff_and_remap():
    """kvmem_store_test.cpp:53-110: select {4,0,2}, then {0,2,3}."""
    st = host.Store(128, 8, 1, 0, n_slots=8)
    st.register_append(128 * 5)
    sin, sout, stats = st.apply([4, 0, 2])
    assert sin == [0, 2, 4]
    assert stats["total_window_tokens"] == 384
    b = st.blocks()
    assert [b["baked_pos"][i] for i in (0, 2, 4)] == [0, 128, 256]
    sin, sout, stats = st.apply([0, 2, 3])
    assert sin == [3] and sout == [4]
    assert stats["retained_position_stable"] == 2 and stats["gpu_reused_blocks"] == 2
    assert st.blocks()["baked_pos"][3] == 256


def test_topk_budget_sink_recent():
    """kvmem_store_test.cpp:284-314."""
    st = host.Store(128, 4, sink_blocks=1, recent_blocks=1, tie_lower_index=False)
    st.register_append(128 * 10)
    s = [0.0] * 10
    s[5], s[6], s[3] = 100.0, 90.0, 10.0
    st.set_retrieval_scores(s)
    assert st.pick_topk_blocks() == [0, 5, 6, 9]


def test_topk_zero_recent_keeps_no_suffix():
    """kvmem_store_test.cpp:316-339."""
    st = host.Store(128, 4, sink_blocks=1, recent_blocks=0, tie_lower_index=False)
    st.register_append(128 * 10)
    s = [0.0] * 10
    s[3], s[5], s[6], s[9] = 80.0, 100.0, 90.0, -100.0
    st.set_retrieval_scores(s)
    assert st.pick_topk_blocks() == [0, 3, 5, 6]


def test_topk_mandatory_blocks_stay_inside_budget():
    """kvmem_store_test.cpp:433-456."""
    st = host.Store(32, 4, sink_blocks=1, recent_blocks=0, tie_lower_index=False)
    st.register_append(32 * 10)
    s = [0.0] * 10
    s[2], s[3], s[4], s[8], s[9] = 100.0, 90.0, 80.0, -10.0, -20.0
    st.set_retrieval_scores(s)
    assert st.pick_topk_blocks([8, 9]) == [0, 2, 8, 9]


def test_mandatory_overlap_and_best_effort_recent():
    """kvmem_store_test.cpp:458-475."""
    st = host.Store(32, 4, sink_blocks=2, recent_blocks=3, tie_lower_index=False)
    st.register_append(32 * 10)
    assert st.pick_topk_blocks([0, 0, 5]) == [0, 1, 5, 9]


def test_mandatory_hard_union_overflow_trims_newest():
    """kvmem_store_test.cpp:477-493."""
    st = host.Store(32, 4, sink_blocks=1, recent_blocks=2, tie_lower_index=False)
    st.register_append(32 * 10)
    assert st.pick_topk_blocks([1, 2, 3, 4]) == [0, 2, 3, 4]


def test_topk_all_fit_and_empty():
    """kvmem_store_test.cpp:763-781."""
    st = host.Store(128, 100)
    st.register_append(128 * 3)
    assert st.pick_topk_blocks() == [0, 1, 2]
    empty = host.Store(128, 4)
    assert empty.pick_topk_blocks() == []
    sin, sout, stats = empty.apply([0, 1])
    assert sin == [] and stats["total_window_tokens"] == 0


def test_high_overlap_skips_stage_in():
    """kvmem_runtime_test.cpp:78-97: the same selection twice stages nothing
    the second time and reuses every block."""
    st = host.Store(32, 4, sink_blocks=1, recent_blocks=1, n_slots=8)
    st.register_append(32 * 10)
    sel = st.pick_topk_blocks()
    st.apply(sel)
    sin, sout, stats = st.apply(st.pick_topk_blocks())
    assert sin == [] and sout == []
    assert stats["gpu_reused_blocks"] == 4


def test_preview_and_resident_commit():
    """kvmem_runtime_test.cpp:218-246 (commit refused for a wrong set,
    accepted for the resident one, window tokens of a partial tail)."""
    st = host.Store(32, 4, sink_blocks=1, recent_blocks=1, n_slots=8)
    st.register_append(32 * 3 + 7)
    sel = st.pick_topk_blocks()
    assert sel == [0, 1, 2, 3]
    assert not st.commit_resident_selection([0, 1, 2])
    sin, _, stats = st.apply(sel)
    assert stats["total_window_tokens"] == 103
    assert st.commit_resident_selection(sel)
    assert not st.commit_resident_selection([0, 1])


def test_stage_out_frees_before_stage_in_slots():
    """kvmem_runtime_test.cpp:50-76: frees precede allocs, so the outgoing
    block's slot is the one the incoming block receives (LIFO)."""
    st = host.Store(128, 2, sink_blocks=1, recent_blocks=0, n_slots=2)
    st.register_append(128 * 4)
    st.apply([0, 2])
    slot_of_2 = st.blocks()["gpu_slot"][2]
    st.apply([0, 3])
    b = st.blocks()
    assert b["gpu_slot"][3] == slot_of_2 and b["gpu_slot"][2] == -1 and b["tier"][2] == 1


def test_truncate_frees_slots():
    st = host.Store(128, 4, n_slots=4)
    st.register_append(128 * 6)
    st.apply([0, 1, 4, 5])
    st.truncate_to(128 * 4 + 10)
    assert st.block_count() == 5 and st.total_tokens() == 522
    st.apply([0, 1, 2, 3])
    assert sorted(st.blocks()["gpu_slot"][:4]) == [0, 1, 2, 3]


def test_lower_index_tie_rule():
    """The reselect contract: equal scores rank the lower block id first."""
    st = host.Store(128, 3, sink_blocks=1, recent_blocks=0, tie_lower_index=True)
    st.register_append(128 * 6)
    st.set_retrieval_scores([0.0, 1.0, 1.0, 1.0, 1.0, 0.5])
    assert st.pick_topk_blocks() == [0, 1, 2]
    ref_rule = host.Store(128, 3, sink_blocks=1, recent_blocks=0, tie_lower_index=False)
    ref_rule.register_append(128 * 6)
    ref_rule.set_retrieval_scores([0.0, 1.0, 1.0, 1.0, 1.0, 0.5])
    assert ref_rule.pick_topk_blocks() == [0, 3, 4]


# --------------------------------------------- live reference cross-check
@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (needs the reference tree)")
def test_live_reference_random_sequences():
    ref = C.CDLL(str(REF))
    ref.kref_runtime_new.restype = C.c_void_p
    ref.kref_runtime_new.argtypes = [C.c_uint32] * 6
    ref.kref_runtime_free.argtypes = [C.c_void_p]
    ref.kref_runtime_set_scores.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.c_uint32]
    pu32 = C.POINTER(C.c_uint32)
    ref.kref_runtime_preview.argtypes = [C.c_void_p, pu32, C.c_uint32, pu32, pu32]
    ref.kref_runtime_apply.argtypes = [C.c_void_p, pu32, C.c_uint32, pu32, pu32, pu32, pu32, pu32]
    ref.kref_runtime_blocks.restype = C.c_uint32
    ref.kref_runtime_blocks.argtypes = [C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_uint8),
                                        C.POINTER(C.c_uint8), C.POINTER(C.c_int64)]
    rng = np.random.default_rng(77)
    for trial in range(120):
        bt = int(rng.choice([16, 128]))
        n_tok = int(rng.integers(1, 70)) * bt + int(rng.integers(0, bt))
        budget, sink, recent = int(rng.integers(1, 30)), int(rng.integers(0, 3)), int(rng.integers(0, 3))
        n_slots = budget + int(rng.integers(0, 4))
        h = ref.kref_runtime_new(bt, budget, sink, recent, n_slots, n_tok)
        st = host.Store(bt, budget, sink, recent, tie_lower_index=False, n_slots=n_slots)
        st.register_append(n_tok)
        n = st.block_count()
        for _ in range(4):
            s = rng.integers(-2, 3, n).astype(np.float64) if trial % 2 else rng.standard_normal(n)
            st.set_retrieval_scores(s.tolist())
            ref.kref_runtime_set_scores(h, s.ctypes.data_as(C.POINTER(C.c_double)), n)
            mand = rng.choice(n, int(rng.integers(0, 3))).tolist() if n else []
            ma = (C.c_uint32 * max(1, len(mand)))(*mand)
            out, cnt = (C.c_uint32 * max(1, n))(), C.c_uint32()
            ref.kref_runtime_preview(h, ma, len(mand), out, C.byref(cnt))
            want = list(out[: cnt.value])
            assert st.pick_topk_blocks(mand) == want
            sa = (C.c_uint32 * max(1, n))(*want)
            si, so = (C.c_uint32 * max(1, n))(), (C.c_uint32 * max(1, n))()
            ni, no, ctr = C.c_uint32(), C.c_uint32(), (C.c_uint32 * 5)()
            ref.kref_runtime_apply(h, sa, len(want), si, C.byref(ni), so, C.byref(no), ctr)
            gi, go, stats = st.apply(want)
            assert gi == list(si[: ni.value]) and go == list(so[: no.value])
            gs = (C.c_int32 * max(1, n))()
            tr, ws, bk = (C.c_uint8 * max(1, n))(), (C.c_uint8 * max(1, n))(), (C.c_int64 * max(1, n))()
            ref.kref_runtime_blocks(h, gs, tr, ws, bk)
            b = st.blocks()
            assert b["gpu_slot"] == list(gs[:n]) and b["baked_pos"] == list(bk[:n])
        ref.kref_runtime_free(h)


def test_apply_without_free_slots_changes_nothing():
    """A selection the slot pool cannot hold (admit_incoming gets slot -1
    from an empty free list) is refused as a whole: the block table is as
    before the call."""
    st = host.Store(block_tokens=16, budget_blocks=6, sink_blocks=1, recent_blocks=0,
                    tie_lower_index=True, n_slots=4)
    st.register_append(10 * 16)
    st.apply([0, 1, 2])
    before = st.blocks()
    with pytest.raises(kv.KvMemError) as ex:
        st.apply([0, 3, 4, 5, 6, 7])
    assert ex.value.code == kv.ERR_NOMEM
    assert st.blocks() == before
    stage_in, _, _ = st.apply([0, 1, 5])
    assert stage_in == [5]


def test_blocks_overlapping_closed_forms():
    """retrieval_mandatory's row-range mapping (llama-memory-kvmem.cpp:
    3026-3045) on 10 blocks of 16 tokens with a 5-token tail (149 rows):
    half-open ranges, straddles, the tail, several ranges (each block once,
    block order), force_pos appended last (even when already listed), and
    the reference's overlap test, under which an empty range [20, 20) still
    names the block holding row 20."""
    st = host.Store(block_tokens=16, budget_blocks=4, n_slots=8)
    st.register_append(9 * 16 + 5)
    assert st.blocks_overlapping([(0, 1)]) == [0]
    assert st.blocks_overlapping([(15, 17)]) == [0, 1]
    assert st.blocks_overlapping([(16, 32)]) == [1]
    assert st.blocks_overlapping([(144, 1000)]) == [9]
    assert st.blocks_overlapping([(149, 1000)]) == []
    assert st.blocks_overlapping([(100, 120), (0, 20), (110, 130)]) == [0, 1, 6, 7, 8]
    assert st.blocks_overlapping([(20, 20)]) == [1]
    assert st.blocks_overlapping([(32, 48)], force_pos=40) == [2, 2]
    assert st.blocks_overlapping([], force_pos=148) == [9]
    assert st.blocks_overlapping([], force_pos=149) == []
    assert st.blocks_overlapping([], force_pos=-1) == []
    for bad in ([(-1, 5)], [(8, 7)]):
        with pytest.raises(kv.KvMemError):
            st.blocks_overlapping(bad)


def test_mandatory_blocks_feed_pick_topk_like_the_reference():
    """The mapped ids go to pick_topk_blocks as its mandatory list: with a
    budget of 5, sink 1 and the query rows [100, 130) (blocks 6, 7, 8), the
    selection is the sink, the three query blocks and the best other block
    (2); a force_pos block is listed last, hence charged first, so it
    survives a tight budget."""
    st = host.Store(block_tokens=16, budget_blocks=5, sink_blocks=1, n_slots=8)
    st.register_append(9 * 16 + 5)
    st.set_retrieval_scores([0.0, 0.1, 0.9, 0.2, 0.3, 0.4, 0.0, 0.0, 0.0, 0.5])
    assert st.pick_topk_blocks(st.blocks_overlapping([(100, 130)])) == [0, 2, 6, 7, 8]
    tight = host.Store(block_tokens=16, budget_blocks=3, sink_blocks=1, n_slots=8)
    tight.register_append(9 * 16 + 5)
    tight.set_retrieval_scores([0.0] * 10)
    # charged newest-listed first: force block 3, then blocks 8, 7 ... until full
    assert tight.pick_topk_blocks(tight.blocks_overlapping([(100, 130)], force_pos=50)) == [0, 3, 8]
