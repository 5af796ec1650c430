"""Recovery of the reselect engine from failed device work, and history
changes through set_device_history, on the GPU against the oracle.

The reference falls back to host writes when a device call fails
(src/adapter/llama-memory-kvmem.cpp:2752-2758, 993-998, 1094-1099).  Here
a failed apply leaves the store as it was before the apply, minus the
blocks whose pool slots the failed work may have written, so the next
apply stages them again.  Failures are injected on the host
(kvmem_hip_debug_fail_after: the n-th allocation / copy / launch is
refused before it is issued), so no kernel ever faults.  Every injection
point of an apply is tried in turn; after each failure every block the
engine still calls resident must hold its exact bytes, and the next apply
must produce the oracle's pool bytes.
"""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from engine_helpers import E, L, T, block_major_pinned, check_pool, history, make_engine  # noqa: E402

ALL_KINDS = kv.FAIL_ALLOC | kv.FAIL_COPY | kv.FAIL_LAUNCH


def announce(msg: str) -> None:
    print(f"[recovery] {msg}", flush=True)


def resident(eng) -> list[int]:
    return [b for b, s in enumerate(eng.block_slots()) if s >= 0]


@pytest.mark.parametrize("mode", ["device", "canonical", "pinned_packed"])
def test_failed_apply_is_recovered_bit_exact(oracle, mode):
    announce(f"injected failures at every operation of an apply ({mode})")
    cap, nb, budget = 40, 40, 8
    k, v, q1 = history(cap, seed=41)
    q2 = (q1.float() * -1.0).to(torch.bfloat16)
    hb = store = None
    span = L * T * (kv.row_size(kv.TYPE_Q8_0, E) + kv.row_size(kv.TYPE_Q4_0, E))
    if mode == "pinned_packed":
        hb = block_major_pinned(k, v, nb)
        store = torch.zeros(nb * span, dtype=torch.uint8, pin_memory=True)

    def fresh_engine():
        """The same starting state for every injection point: sel1 applied."""
        eng = make_engine(budget, 4, kv.TYPE_Q8_0, kv.TYPE_Q4_0, canonical_layout=int(mode == "canonical"))
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        if mode == "pinned_packed":
            store.zero_()
            eng.set_host_history(hb.data_ptr(), nb)
            eng.set_packed_host(store.data_ptr(), nb)
        return eng

    n_failed = 0
    for nth in range(1, 64):
        with fresh_engine() as eng:
            ctx = kv.Context.borrow(eng.ctx_handle())
            sel1 = eng.preview(q1.data_ptr(), q1.shape[1])
            sel2 = eng.preview(q2.data_ptr(), q2.shape[1])
            assert set(sel1.blocks) != set(sel2.blocks)
            eng.apply(sel1)
            check_pool(eng, oracle, k, v, sel1.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)
            ctx.debug_fail_after(ALL_KINDS, nth)
            try:
                eng.apply(sel2)
                failed = False
            except kv.KvMemError as ex:
                assert "injected failure" in str(ex), str(ex)
                failed = True
            left = ctx.debug_fail_left()
            ctx.debug_fail_after(0, 0)
            if not failed:
                assert left > 0, "an apply succeeded although its injected failure fired"
                check_pool(eng, oracle, k, v, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)
                break
            n_failed += 1
            print(f"[recovery] {mode}: failure at operation {nth}: "
                  f"{ctx.last_error()!r}; {len(resident(eng))} blocks still resident", flush=True)
            # what the engine still calls resident holds its exact bytes
            check_pool(eng, oracle, k, v, resident(eng), kv.TYPE_Q8_0, kv.TYPE_Q4_0)
            assert set(resident(eng)) <= set(sel1.blocks)
            # the next apply recovers: every selected block bit-exact
            eng.apply(sel2)
            check_pool(eng, oracle, k, v, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)
            if mode == "canonical":
                slots = eng.block_slots()
                assert [slots[b] for b in sel2.blocks] == list(range(len(sel2.blocks)))
            eng.apply(sel1)
            check_pool(eng, oracle, k, v, sel1.blocks, kv.TYPE_Q8_0, kv.TYPE_Q4_0)
    else:
        raise AssertionError("apply never ran to completion")
    # a device-history apply is one launch (its tables travel in the kernel
    # arguments); slot moves add the chain launch (and saves), the pinned
    # packed store the stage-out of evicted blocks
    assert n_failed >= {"device": 1, "canonical": 2, "pinned_packed": 2}[mode], n_failed
    del hb, store


def test_set_device_history_grows_resident_tail(oracle):
    """The same history pointers with more tokens: a resident partial tail
    block is staged again (as append_tokens)."""
    announce("set_device_history grows a resident partial tail")
    cap = 16
    k, v, q = history(cap, seed=43)
    with make_engine(4, 2, recent_blocks=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 9 * T + 37)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert 9 in sel.blocks
        eng.apply(sel)
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 37 if b == 9 else T)
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 9 * T + 100)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        st = eng.apply(sel)
        assert st["n_staged"] >= 1
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 100 if b == 9 else T)


def test_set_device_history_new_buffers_restage(oracle):
    """Other history buffers (new content): nothing staged from the old
    ones stays resident, so the same selection is staged again in full."""
    announce("set_device_history to new buffers")
    cap, nb = 24, 24
    k1, v1, q = history(cap, seed=45)
    k2, v2, _ = history(cap, seed=46)
    with make_engine(6, 2) as eng:
        eng.set_device_history(k1.data_ptr(), v1.data_ptr(), cap, nb * T)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        eng.apply(sel)
        check_pool(eng, oracle, k1, v1, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
        eng.set_device_history(k2.data_ptr(), v2.data_ptr(), cap, nb * T)
        assert resident(eng) == []
        sel2 = eng.preview(q.data_ptr(), q.shape[1])
        st = eng.apply(sel2)
        assert st["n_staged"] == len(sel2.blocks)
        check_pool(eng, oracle, k2, v2, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
