"""Continuation calls of the engine on the GPU (include/kvmem_host.h):
attention_view, selection_fits, commit_unchanged, commit_resident,
can_append and append_resident over the engine's own pool.

- The reference GPU test's expectations (tests/mtp-kv-test.cpp:300-361):
  prefill to the query start with the rows written into the pool as they
  are decoded, take the view, decode the query rows, preview with the query
  span mandatory; the identical view is accepted, a trimmed mandatory tail
  does not fit, an oversized generation reserve cannot append, and after a
  restore (truncate to the query start) the old view and selection are
  stale.  Every pool row stays the oracle's quantization of the history.
- An identical preview after an apply commits with no device work: the
  pool is byte for byte the same and no stage-in or slot move is timed.
- A changed selection or a changed pool is refused; commit_resident and
  canonical / LIFO views.
- Rows appended resident in canonical mode continue the slot order and are
  not staged again by the next apply, host-planned or device-planned.
"""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host  # noqa: E402

from engine_helpers import E, L, T, check_pool, decode_rows, history, make_engine  # noqa: E402


def announce(msg: str) -> None:
    print(f"[continuation] {msg}", flush=True)


def pool_bytes(eng) -> list:
    out = []
    for layer in range(L):
        for ptr, ty in zip(eng.pool_layer(layer), (eng.params.type_k, eng.params.type_v)):
            n = eng.n_slots() * T * kv.row_size(ty, E)
            buf = torch.empty(n, dtype=torch.uint8, device="cuda")
            c = kv.Context(0)
            c.d2d_batched([ptr], [buf.data_ptr()], [n])
            c.sync()
            c.close()
            out.append(buf.cpu())
    return out


def test_reference_logits_fixture_flow(oracle):
    announce("mtp-kv-test flow: prefill 576 rows, 24 query rows, all blocks fit the budget")
    cap, end = 8, 600
    query = end - 24
    k, v, q = history(cap, seed=41)
    with make_engine(16, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 0)
        decode_rows(eng, k, v, 0, query)
        before = eng.attention_view()
        assert before.valid and before.rows == query and before.blocks == [0, 1, 2, 3, 4]
        decode_rows(eng, k, v, query, end)
        eng.set_request_span(query, end)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        assert sel.blocks == [0, 1, 2, 3, 4] and sel.rows == end
        snap = pool_bytes(eng)
        assert eng.commit_unchanged(before, sel), "identical attention view rejected"
        assert all(torch.equal(a, b) for a, b in zip(snap, pool_bytes(eng)))
        last = end - 4 * T
        check_pool(eng, oracle, k, v, sel.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: last if b == 4 else T)
        trimmed = host.Selection(sel.epoch, sel.rows, sel.blocks[:-1])
        assert not eng.selection_fits(trimmed, end, 0), "trimmed mandatory tail accepted"
        assert eng.selection_fits(sel, end, 0)
        ok, why = eng.can_append(end, eng.n_slots() * T, True)
        assert not ok and why == "insufficient_slots", "oversized generation reserve accepted"
        assert eng.can_append(end, T, False) == (True, "same_query")
        eng.truncate_to(query)                  # restore the checkpoint at the query start
        assert not eng.commit_unchanged(before, sel), "stale attention view accepted after restore"
        with pytest.raises(kv.StaleSelection):
            eng.apply(sel)
        decode_rows(eng, k, v, query, end)      # replay the query rows
        again = eng.preview(q.data_ptr(), q.shape[1])
        assert again.blocks == sel.blocks
        assert eng.commit_unchanged(eng.attention_view(), again)
        check_pool(eng, oracle, k, v, again.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: last if b == 4 else T)


def test_commit_unchanged_after_identical_preview(oracle):
    announce("apply, then an identical preview: commit_unchanged moves no byte")
    cap, nb = 40, 40
    k, v, q = history(cap, seed=43)
    q2 = (q.float() * -1.0).to(torch.bfloat16)
    with make_engine(8, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        sel1 = eng.preview(q.data_ptr(), q.shape[1])
        eng.apply(sel1)
        view = eng.attention_view()
        assert view.valid and view.blocks == sel1.blocks
        assert eng.commit_resident(True)
        snap = pool_bytes(eng)
        ctx = kv.Context.borrow(eng.ctx_handle())
        ctx.perf_enable(True)
        ctx.perf_reset()
        same = eng.preview(q.data_ptr(), q.shape[1])
        assert same.blocks == sel1.blocks
        assert eng.commit_unchanged(view, same)
        ctx.sync()
        perf = ctx.perf()
        ctx.perf_enable(False)
        assert perf["n_set"] == 0 and perf["n_layout"] == 0, perf
        assert all(torch.equal(a, b) for a, b in zip(snap, pool_bytes(eng)))
        st = eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), same.blocks))
        assert st["n_staged"] == 0 and st["n_moved"] == 0 and st["n_stage_in"] == 0
        # a different selection is refused and leaves the working set alone
        other = eng.preview(q2.data_ptr(), q2.shape[1])
        assert other.blocks != sel1.blocks
        assert not eng.commit_unchanged(view, other)
        assert not eng.selection_fits(host.Selection(other.epoch + 1, other.rows, other.blocks),
                                      other.rows, 0)
        eng.apply(other)
        # the pool changed: the old view is stale even for the new resident set
        assert eng.attention_epoch() != view.epoch
        assert not eng.commit_unchanged(view, host.Selection(eng.epoch(), eng.total_tokens(),
                                                             other.blocks))
        check_pool(eng, oracle, k, v, other.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0)


def test_views_in_lifo_layout(oracle):
    announce("LIFO slots: the canonical view breaks, the plain one holds")
    cap, nb = 24, 24
    k, v, q = history(cap, seed=47)
    q2 = (q.float() * -1.0).to(torch.bfloat16)
    with make_engine(6, 2, canonical_layout=0) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        eng.apply(eng.preview(q.data_ptr(), q.shape[1]))
        eng.apply(eng.preview(q2.data_ptr(), q2.shape[1]))
        slots = eng.block_slots()
        resident = [b for b in range(nb) if slots[b] >= 0]
        canonical = all(slots[b] == i for i, b in enumerate(resident))
        plain = eng.attention_view(canonical=False)
        assert plain.valid and plain.blocks == resident
        assert eng.attention_view(canonical=True).valid == canonical
        assert eng.commit_resident(False)
        assert eng.commit_resident(True) == canonical
        ok, why = eng.can_append(nb * T, 0, True)
        assert not ok and why in ("coverage_or_layout", "history_not_resident")


def test_append_resident_in_canonical_layout(oracle):
    announce("rows appended resident continue the window and are not staged again")
    cap, nb = 20, 16
    k, v, q = history(cap, seed=53)
    with make_engine(8, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        eng.apply(sel)
        view = eng.attention_view()
        decode_rows(eng, k, v, nb * T, nb * T + 70)     # block 16, 70 rows
        assert eng.block_slots()[nb] == len(sel.blocks)
        after = eng.attention_view()
        assert after.valid and after.blocks == sel.blocks + [nb]
        assert after.epoch == view.epoch                # appended rows leave the attention epoch
        # the selection now needs the new block: with it mandatory, it is kept
        eng.set_request_span(nb * T, 0)
        sel2 = eng.preview(q.data_ptr(), q.shape[1])
        assert nb in sel2.blocks
        st = eng.apply(sel2)
        assert st["n_staged"] == len(set(sel2.blocks) - set(sel.blocks) - {nb})
        check_pool(eng, oracle, k, v, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 70 if b == nb else T)
        # a partial tail without a slot gets one, but is staged again by the next apply
        eng.set_request_span(-1)
        far = [b for b in range(nb) if b not in sel2.blocks][:1]
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), sorted(set(sel2.blocks[:4]) | set(far))))
        assert eng.block_slots()[nb] == -1
        eng.append_resident(10)                         # the tail (80 rows) takes a slot
        assert eng.block_slots()[nb] >= 0
        assert not eng.attention_view(canonical=False).valid
        st = eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), [0, nb]))
        assert st["n_staged"] >= 1
        check_pool(eng, oracle, k, v, [0, nb], kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 80 if b == nb else T)
        assert eng.attention_view().valid


def test_append_resident_then_device_planned_step(oracle):
    """Blocks appended resident enter the device plan's resident list like
    staged ones: a device-planned apply_retrieval after them stages only the
    blocks it newly selects, moves the rest into window order, and every
    selected block's rows are the oracle's."""
    announce("append_resident, then apply_retrieval through the device plan")
    cap, nb = 24, 18
    k, v, q = history(cap, seed=59)
    q2 = (q.float() * -1.0).to(torch.bfloat16)
    with make_engine(8, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        st = eng.apply_retrieval(q.data_ptr(), q.shape[1])
        assert st["device_planned"] == 1
        first = [b for b, s in enumerate(eng.block_slots()) if s >= 0]
        decode_rows(eng, k, v, nb * T, (nb + 2) * T)        # blocks 18, 19 written in the pool
        slots = eng.block_slots()
        assert slots[nb] == len(first) and slots[nb + 1] == len(first) + 1
        eng.set_request_span(nb * T, 0)                      # the new rows are the query
        st = eng.apply_retrieval(q2.data_ptr(), q2.shape[1])
        assert st["device_planned"] == 1
        sel = [b for b, s in enumerate(eng.block_slots()) if s >= 0]
        assert nb in sel and nb + 1 in sel
        assert st["n_staged"] == len(set(sel) - set(first) - {nb, nb + 1})
        assert [eng.block_slots()[b] for b in sel] == list(range(len(sel)))
        check_pool(eng, oracle, k, v, sel, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
        assert eng.attention_view().valid


def test_truncated_grown_tail_leaves_no_stale_mark(oracle):
    """A resident partial tail that grew (so the next apply would quantize it
    again) and is then cut away by a truncation leaves no mark behind: rows
    decoded afterwards into a new block under the same id make a complete
    block, the attention view is valid, and the next apply does not stage
    it again."""
    announce("grown tail truncated away, then a new block decoded under its id")
    cap, nb = 20, 10
    k, v, q = history(cap, seed=67)
    with make_engine(6, 4) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T + 50)
        sel = eng.preview(q.data_ptr(), q.shape[1], mandatory=[nb])
        assert nb in sel.blocks
        eng.apply(sel)
        eng.append_tokens(30)                     # the resident tail grows: stale in the pool
        assert not eng.attention_view().valid
        eng.truncate_to(nb * T)                   # ... and is cut away with its slot
        assert eng.block_slots()[nb:] == []
        decode_rows(eng, k, v, nb * T, nb * T + 40)   # a new block 10, written in the pool
        view = eng.attention_view()
        assert view.valid and view.blocks[-1] == nb, view
        check_pool(eng, oracle, k, v, view.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 40 if b == nb else T)
        sel2 = eng.preview(q.data_ptr(), q.shape[1], mandatory=[nb])
        st = eng.apply(sel2)
        assert st["n_staged"] == len(set(sel2.blocks) - set(view.blocks)), st
        check_pool(eng, oracle, k, v, sel2.blocks, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                   ntok_of=lambda b: 40 if b == nb else T)
