"""ctypes view of the reselect engine and host store (include/kvmem_host.h).

Store  -- the host block table / top-k / diff / slot plan alone (no GPU);
          method names follow KvMemStore / KvMemRuntime
          (kvmem/include/kvmem/kvmem_store.hpp, kvmem_runtime.hpp).
Engine -- one agent step on the GPU: preview (score + top-k) then apply
          (diff, slots, stage-in), as llama_memory_kvmem::preview_retrieval /
          apply_selection (src/adapter/llama-memory-kvmem.cpp:3047-3263).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Sequence

import sys

from . import (ERR_STALE, OK, KvMemError, StaleSelection, TYPE_BF16, TYPE_Q8_0, LAYER_MEAN,
               load_library, track)


class PlanStats(C.Structure):
    _fields_ = [("n_stage_in", C.c_uint32), ("n_stage_out", C.c_uint32), ("n_staged", C.c_uint32),
                ("n_moved", C.c_uint32), ("selection_overlap_blocks", C.c_uint32),
                ("gpu_reused_blocks", C.c_uint32), ("retained_position_stable", C.c_uint32),
                ("retained_position_moved", C.c_uint32), ("total_window_tokens", C.c_uint32),
                ("n_saved", C.c_uint32), ("n_restored", C.c_uint32), ("device_planned", C.c_uint32),
                ("n_skip", C.c_uint32)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class RowRange(C.Structure):
    """kvmem_row_range: rows [begin, end) (llama_kvmem_row_range)."""
    _fields_ = [("begin", C.c_int32), ("end", C.c_int32)]


class AttentionViewC(C.Structure):
    """kvmem_attention_view (llama_kvmem_attention_view)."""
    _fields_ = [("epoch", C.c_uint64), ("rows", C.c_uint32), ("valid", C.c_int32),
                ("n_blocks", C.c_uint32), ("capacity", C.c_uint32), ("blocks", C.POINTER(C.c_uint32))]


@dataclass
class AttentionView:
    """llama_kvmem_attention_view (src/adapter/llama-kvmem-hooks.h:143-148)."""
    epoch: int
    rows: int
    valid: bool
    blocks: list

    def to_c(self):
        arr = (C.c_uint32 * max(1, len(self.blocks)))(*self.blocks)
        v = AttentionViewC(self.epoch, self.rows, int(self.valid), len(self.blocks), len(self.blocks),
                           C.cast(arr, C.POINTER(C.c_uint32)))
        return v, arr


def _get_view(fn, h, canonical: bool, cap: int) -> AttentionView:
    arr = (C.c_uint32 * max(1, cap))()
    v = AttentionViewC(0, 0, 0, 0, max(1, cap), C.cast(arr, C.POINTER(C.c_uint32)))
    rc = fn(h, int(canonical), C.byref(v))
    if rc != OK:
        raise KvMemError(rc, "attention view failed")
    return AttentionView(v.epoch, v.rows, bool(v.valid), list(arr[: v.n_blocks]))


def _ranges(rs):
    rs = list(rs)
    return (RowRange * max(1, len(rs)))(*[RowRange(int(b), int(e)) for b, e in rs]), len(rs)


class EngineParams(C.Structure):
    _fields_ = [("device", C.c_int32), ("n_layers", C.c_uint32), ("block_tokens", C.c_uint32),
                ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32),
                ("n_embd_v", C.c_uint32), ("budget_blocks", C.c_uint32),
                ("reserve_blocks", C.c_uint32), ("sink_blocks", C.c_uint32),
                ("recent_blocks", C.c_uint32), ("type_k", C.c_int32), ("type_v", C.c_int32),
                ("tie_lower_index", C.c_int32), ("layer_reduce", C.c_int32),
                ("canonical_layout", C.c_int32), ("scorer", C.c_int32), ("n_rot", C.c_uint32),
                ("rope_freq_base", C.c_float), ("rope_freq_scale", C.c_float), ("attn_rot", C.c_int32),
                ("query_max_tokens", C.c_uint32), ("query_last", C.c_uint32), ("device_plan", C.c_int32)]


_bound = set()


def bind(lib: C.CDLL) -> C.CDLL:
    if id(lib) in _bound:
        return lib
    vp, u32, i32, u64 = C.c_void_p, C.c_uint32, C.c_int, C.c_uint64
    pu32, pi32, pu8, pi64 = (C.POINTER(C.c_uint32), C.POINTER(C.c_int32), C.POINTER(C.c_uint8),
                             C.POINTER(C.c_int64))
    pd = C.POINTER(C.c_double)

    def sig(name, res, *args):
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = list(args)

    sig("kvmem_store_create", i32, u32, u32, u32, u32, i32, u32, C.POINTER(vp))
    sig("kvmem_store_destroy", None, vp)
    sig("kvmem_store_register_append", i32, vp, u32)
    sig("kvmem_store_truncate_to", i32, vp, u32)
    sig("kvmem_store_block_count", u32, vp)
    sig("kvmem_store_total_tokens", u32, vp)
    sig("kvmem_store_set_scores", i32, vp, pd, u32)
    sig("kvmem_store_pick_topk", i32, vp, pu32, u32, pu32, pu32)
    sig("kvmem_store_apply", i32, vp, pu32, u32, pu32, pu32, pu32, pu32, C.POINTER(PlanStats))
    sig("kvmem_store_blocks", i32, vp, pi32, pu8, pu8, pi64)
    sig("kvmem_store_commit_resident", i32, vp, pu32, u32)
    sig("kvmem_store_blocks_overlapping", i32, vp, C.POINTER(RowRange), u32, C.c_int32, pu32, u32, pu32)
    pview, pstr = C.POINTER(AttentionViewC), C.POINTER(C.c_char_p)
    sig("kvmem_store_epoch", u64, vp)
    sig("kvmem_store_append_resident", i32, vp, u32)
    sig("kvmem_store_attention_view", i32, vp, i32, pview)
    sig("kvmem_store_selection_fits", i32, vp, pu32, u32, u64, u32, pu32, u32, u32, u32)
    sig("kvmem_store_commit_unchanged", i32, vp, pview, u64, u32, pu32, u32)
    sig("kvmem_store_can_append", i32, vp, u32, u32, i32, pstr)
    sig("kvmem_engine_append_resident", i32, vp, u32)
    sig("kvmem_engine_attention_epoch", u64, vp)
    sig("kvmem_engine_attention_view", i32, vp, i32, pview)
    sig("kvmem_engine_selection_fits", i32, vp, u64, u32, pu32, u32, u32, u32)
    sig("kvmem_engine_commit_unchanged", i32, vp, pview, u64, u32, pu32, u32)
    sig("kvmem_engine_commit_resident", i32, vp, i32)
    sig("kvmem_engine_can_append", i32, vp, u32, u32, i32, pstr)
    sig("kvmem_store_query_replay_fits", i32, vp, u32, u32)
    sig("kvmem_store_free_slots", u32, vp)
    sig("kvmem_store_prefill_needs_offload", i32, vp, u32, u32, u32)
    sig("kvmem_engine_query_replay_fits", i32, vp, u32, u32)
    sig("kvmem_engine_free_slots", u32, vp)
    pf32 = C.POINTER(C.c_float)
    sig("kvmem_engine_get_query", i32, vp, pf32, pu32)
    sig("kvmem_engine_set_query", i32, vp, pf32, pu32)
    sig("kvmem_engine_freeze_query", i32, vp, i32)
    sig("kvmem_engine_set_request_span", i32, vp, C.c_int32, C.c_int32, C.c_int32)
    sig("kvmem_engine_set_turn_spans", i32, vp, C.POINTER(RowRange), u32, C.POINTER(RowRange), u32)
    sig("kvmem_engine_retrieval_mandatory", i32, vp, pu32, u32, pu32)
    sig("kvmem_engine_capture_q", i32, vp, u32, vp, i32, C.c_size_t, C.c_size_t, C.c_size_t, u32, pi32)
    sig("kvmem_engine_reset_query", i32, vp)
    sig("kvmem_engine_query_rows", i32, vp, pu32)
    sig("kvmem_engine_default_params", EngineParams)
    sig("kvmem_engine_create", i32, C.POINTER(EngineParams), C.POINTER(vp))
    sig("kvmem_engine_destroy", None, vp)
    sig("kvmem_engine_last_error", C.c_char_p, vp)
    sig("kvmem_engine_ctx", vp, vp)
    sig("kvmem_engine_set_device_history", i32, vp, vp, vp, u32, u32)
    sig("kvmem_engine_set_host_history", i32, vp, vp, u32)
    sig("kvmem_engine_set_packed_host", i32, vp, vp, u32)
    sig("kvmem_engine_packed_valid", i32, vp, u32)
    sig("kvmem_engine_append_tokens", i32, vp, u32)
    sig("kvmem_engine_truncate_to", i32, vp, u32)
    sig("kvmem_engine_block_count", u32, vp)
    sig("kvmem_engine_total_tokens", u32, vp)
    sig("kvmem_engine_epoch", u64, vp)
    sig("kvmem_engine_n_slots", u32, vp)
    sig("kvmem_engine_pool_layer", i32, vp, u32, C.POINTER(vp), C.POINTER(vp))
    sig("kvmem_engine_set_pool", i32, vp, C.POINTER(vp), C.POINTER(vp))
    sig("kvmem_engine_block_slots", i32, vp, pi32)
    sig("kvmem_engine_preview", i32, vp, vp, i32, u32, pu32, u32, pu32, pu32, C.POINTER(u64), pu32)
    sig("kvmem_engine_preview_meank", i32, vp, vp, pu32, pu32, u32, pu32, pu32, C.POINTER(u64), pu32)
    sig("kvmem_engine_apply", i32, vp, u64, u32, pu32, u32, C.POINTER(PlanStats))
    sig("kvmem_engine_apply_retrieval", i32, vp, vp, i32, u32, pu32, u32, C.POINTER(PlanStats))
    sig("kvmem_engine_scores", i32, vp, C.POINTER(C.c_float), u32)
    _bound.add(id(lib))
    return lib


def _u32(xs: Sequence[int]):
    xs = list(xs)
    return (C.c_uint32 * max(1, len(xs)))(*xs), len(xs)


@dataclass
class Selection:
    """llama_kvmem_selection (src/adapter/llama-kvmem-hooks.h:140-144)."""
    epoch: int
    rows: int
    blocks: list


class Store:
    """Host store + slot plan (no device).  Every block starts outside the
    pool; apply() runs prepare_selection + finish_reselect."""

    def __init__(self, block_tokens: int = 128, budget_blocks: int = 256, sink_blocks: int = 1,
                 recent_blocks: int = 0, tie_lower_index: bool = True, n_slots: int = 384):
        self.lib = bind(load_library())
        h = C.c_void_p()
        rc = self.lib.kvmem_store_create(block_tokens, budget_blocks, sink_blocks, recent_blocks,
                                         int(tie_lower_index), n_slots, C.byref(h))
        if rc != OK:
            raise KvMemError(rc, "kvmem_store_create failed")
        self.h = h
        track(self)

    _close_rank = 0

    def close(self):
        if getattr(self, "h", None):
            self.lib.kvmem_store_destroy(self.h)
            self.h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals (sys among them) may already be
        # gone when an object is collected during interpreter shutdown
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def register_append(self, n_tokens: int) -> None:
        self.lib.kvmem_store_register_append(self.h, n_tokens)

    def truncate_to(self, token_pos: int) -> None:
        self.lib.kvmem_store_truncate_to(self.h, token_pos)

    def block_count(self) -> int:
        return self.lib.kvmem_store_block_count(self.h)

    def total_tokens(self) -> int:
        return self.lib.kvmem_store_total_tokens(self.h)

    def set_retrieval_scores(self, scores: Sequence[float]) -> None:
        arr = (C.c_double * max(1, len(scores)))(*[float(x) for x in scores])
        self.lib.kvmem_store_set_scores(self.h, arr, len(scores))

    def pick_topk_blocks(self, mandatory: Sequence[int] = ()) -> list:
        m, nm = _u32(mandatory)
        out = (C.c_uint32 * max(1, self.block_count()))()
        n = C.c_uint32(0)
        self.lib.kvmem_store_pick_topk(self.h, m, nm, out, C.byref(n))
        return list(out[: n.value])

    def apply(self, sel: Sequence[int]) -> tuple[list, list, dict]:
        s, ns = _u32(sel)
        cap = max(1, self.block_count())
        si, so = (C.c_uint32 * cap)(), (C.c_uint32 * cap)()
        ni, no = C.c_uint32(0), C.c_uint32(0)
        st = PlanStats()
        rc = self.lib.kvmem_store_apply(self.h, s, ns, si, C.byref(ni), so, C.byref(no), C.byref(st))
        if rc != OK:
            raise KvMemError(rc, "kvmem_store_apply failed")
        return list(si[: ni.value]), list(so[: no.value]), st.as_dict()

    def blocks(self) -> dict:
        n = self.block_count()
        slot = (C.c_int32 * max(1, n))()
        tier = (C.c_uint8 * max(1, n))()
        ws = (C.c_uint8 * max(1, n))()
        baked = (C.c_int64 * max(1, n))()
        self.lib.kvmem_store_blocks(self.h, slot, tier, ws, baked)
        return {"gpu_slot": list(slot[:n]), "tier": list(tier[:n]), "in_ws": list(ws[:n]),
                "baked_pos": list(baked[:n])}

    def commit_resident_selection(self, sel: Sequence[int]) -> bool:
        s, n = _u32(sel)
        return bool(self.lib.kvmem_store_commit_resident(self.h, s, n))

    # ---- continuation checks (the store alone: a block holding a slot is complete)
    def epoch(self) -> int:
        """Attention epoch: moves with applies that change the working set and cuts."""
        return self.lib.kvmem_store_epoch(self.h)

    def append_resident(self, n_tokens: int) -> None:
        """Rows written into the pool as they are decoded (new blocks take slots)."""
        rc = self.lib.kvmem_store_append_resident(self.h, n_tokens)
        if rc != OK:
            raise KvMemError(rc, "kvmem_store_append_resident failed")

    def attention_view(self, canonical: bool = True) -> AttentionView:
        return _get_view(self.lib.kvmem_store_attention_view, self.h, canonical, self.block_count())

    def selection_fits(self, sel: Selection, end: int, generation_rows: int,
                       mandatory: Sequence[int] = ()) -> bool:
        m, nm = _u32(mandatory)
        s, ns = _u32(sel.blocks)
        return bool(self.lib.kvmem_store_selection_fits(self.h, m, nm, sel.epoch, sel.rows, s, ns, end,
                                                        generation_rows))

    def commit_unchanged(self, before: AttentionView, sel: Selection) -> bool:
        v, keep = before.to_c()
        s, ns = _u32(sel.blocks)
        return bool(self.lib.kvmem_store_commit_unchanged(self.h, C.byref(v), sel.epoch, sel.rows, s, ns))

    def can_append(self, end: int, generation_rows: int, all_history: bool) -> tuple[bool, str]:
        why = C.c_char_p()
        ok = self.lib.kvmem_store_can_append(self.h, end, generation_rows, int(all_history), C.byref(why))
        return bool(ok), why.value.decode()

    def query_replay_fits(self, query_begin: int, prompt_end: int) -> bool:
        return bool(self.lib.kvmem_store_query_replay_fits(self.h, query_begin, prompt_end))

    def free_slots(self) -> int:
        return self.lib.kvmem_store_free_slots(self.h)

    def prefill_needs_offload(self, resident_tokens: int, incoming_tokens: int, pool_tokens: int) -> bool:
        return bool(self.lib.kvmem_store_prefill_needs_offload(self.h, resident_tokens, incoming_tokens,
                                                               pool_tokens))

    def blocks_overlapping(self, ranges, force_pos: int = -1) -> list:
        """retrieval_mandatory's mapping of row ranges (+ force_pos) to ids."""
        r, nr = _ranges(ranges)
        cap = max(1, self.block_count() + 1)
        out = (C.c_uint32 * cap)()
        n = C.c_uint32(0)
        rc = self.lib.kvmem_store_blocks_overlapping(self.h, r, nr, force_pos, out, cap, C.byref(n))
        if rc != OK:
            raise KvMemError(rc, "kvmem_store_blocks_overlapping failed")
        return list(out[: n.value])


class Engine:
    """The reselect engine on one GPU (owns its context, pool and store)."""

    def __init__(self, **params):
        self.lib = bind(load_library())
        p = self.lib.kvmem_engine_default_params()
        for k, v in params.items():
            if not hasattr(p, k):
                raise TypeError(f"unknown engine parameter {k}")
            setattr(p, k, float(v) if k.startswith("rope_freq") else int(v))
        self.params = p
        h = C.c_void_p()
        rc = self.lib.kvmem_engine_create(C.byref(p), C.byref(h))
        if rc != OK:
            raise KvMemError(rc, "kvmem_engine_create failed")
        self.h = h
        track(self)

    _close_rank = 0

    def close(self):
        if getattr(self, "h", None):
            self.lib.kvmem_engine_destroy(self.h)
            self.h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # bound at definition: module globals (sys among them) may already be
        # gone when an object is collected during interpreter shutdown
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check(self, rc: int, what: str) -> None:
        if rc == OK:
            return
        msg = self.lib.kvmem_engine_last_error(self.h).decode()
        raise (StaleSelection if rc == ERR_STALE else KvMemError)(rc, f"{what}: {msg}")

    def ctx_handle(self) -> int:
        return self.lib.kvmem_engine_ctx(self.h)

    def set_device_history(self, k_ptr: int, v_ptr: int, capacity_blocks: int, n_tokens: int):
        self.check(self.lib.kvmem_engine_set_device_history(self.h, k_ptr, v_ptr, capacity_blocks,
                                                            n_tokens), "set_device_history")

    def set_host_history(self, base_ptr: int | None, capacity_blocks: int = 0):
        self.check(self.lib.kvmem_engine_set_host_history(self.h, base_ptr or None, capacity_blocks),
                   "set_host_history")

    def set_packed_host(self, base_ptr: int | None, capacity_blocks: int = 0):
        """Pinned packed host store (block spans in the pool's formats)."""
        self.check(self.lib.kvmem_engine_set_packed_host(self.h, base_ptr or None, capacity_blocks),
                   "set_packed_host")

    def packed_valid(self, block_id: int) -> bool:
        return bool(self.lib.kvmem_engine_packed_valid(self.h, block_id))

    def append_tokens(self, n: int):
        self.check(self.lib.kvmem_engine_append_tokens(self.h, n), "append_tokens")

    def truncate_to(self, pos: int):
        self.check(self.lib.kvmem_engine_truncate_to(self.h, pos), "truncate_to")

    def block_count(self) -> int:
        return self.lib.kvmem_engine_block_count(self.h)

    def total_tokens(self) -> int:
        return self.lib.kvmem_engine_total_tokens(self.h)

    def epoch(self) -> int:
        return self.lib.kvmem_engine_epoch(self.h)

    def n_slots(self) -> int:
        return self.lib.kvmem_engine_n_slots(self.h)

    def pool_layer(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        self.check(self.lib.kvmem_engine_pool_layer(self.h, layer, C.byref(k), C.byref(v)), "pool_layer")
        return k.value, v.value

    def set_pool(self, k_ptrs: Sequence[int] | None, v_ptrs: Sequence[int] | None = None):
        """Borrow caller-owned per-layer pool tensors (None: engine-owned)."""
        if k_ptrs is None:
            self.check(self.lib.kvmem_engine_set_pool(self.h, None, None), "set_pool")
            return
        ka = (C.c_void_p * len(k_ptrs))(*k_ptrs)
        va = (C.c_void_p * len(v_ptrs))(*v_ptrs)
        self._pool_keep = (ka, va)
        self.check(self.lib.kvmem_engine_set_pool(self.h, ka, va), "set_pool")

    def set_request_span(self, query_begin: int, query_end: int = 0, force_pos: int = -1) -> None:
        self.check(self.lib.kvmem_engine_set_request_span(self.h, query_begin, query_end, force_pos),
                   "set_request_span")

    def set_turn_spans(self, query=(), mandatory=()) -> None:
        q, nq = _ranges(query)
        m, nm = _ranges(mandatory)
        self.check(self.lib.kvmem_engine_set_turn_spans(self.h, q, nq, m, nm), "set_turn_spans")

    def retrieval_mandatory(self) -> list:
        cap = max(1, self.block_count() + 1)
        out = (C.c_uint32 * cap)()
        n = C.c_uint32(0)
        self.check(self.lib.kvmem_engine_retrieval_mandatory(self.h, out, cap, C.byref(n)),
                   "retrieval_mandatory")
        return list(out[: n.value])

    def capture_q(self, layer: int, q_ptr: int, q_type: int, nb0: int, nb1: int, nb2: int,
                  positions: Sequence[int]) -> None:
        """Query rows of one layer's strided Qcur view, at these positions."""
        pos = (C.c_int32 * max(1, len(positions)))(*[int(p) for p in positions])
        self.check(self.lib.kvmem_engine_capture_q(self.h, layer, q_ptr, q_type, nb0, nb1, nb2,
                                                   len(positions), pos), "capture_q")

    def reset_query(self) -> None:
        self.check(self.lib.kvmem_engine_reset_query(self.h), "reset_query")

    def query_rows(self) -> int:
        n = C.c_uint32(0)
        self.check(self.lib.kvmem_engine_query_rows(self.h, C.byref(n)), "query_rows")
        return n.value

    def preview_window(self, mandatory: Sequence[int] = ()) -> Selection:
        """Preview over the captured query window (q = NULL)."""
        m, nm = _u32(mandatory)
        out = (C.c_uint32 * max(1, self.block_count()))()
        n, rows = C.c_uint32(0), C.c_uint32(0)
        ep = C.c_uint64(0)
        self.check(self.lib.kvmem_engine_preview(self.h, None, TYPE_BF16, 0, m, nm, out, C.byref(n),
                                                 C.byref(ep), C.byref(rows)), "preview (query window)")
        return Selection(ep.value, rows.value, list(out[: n.value]))

    def block_slots(self) -> list:
        n = self.block_count()
        out = (C.c_int32 * max(1, n))()
        self.check(self.lib.kvmem_engine_block_slots(self.h, out), "block_slots")
        return list(out[:n])

    def preview(self, q_ptr: int, n_q_tokens: int, q_type: int = TYPE_BF16,
                mandatory: Sequence[int] = ()) -> Selection:
        m, nm = _u32(mandatory)
        out = (C.c_uint32 * max(1, self.block_count()))()
        n, rows = C.c_uint32(0), C.c_uint32(0)
        ep = C.c_uint64(0)
        self.check(self.lib.kvmem_engine_preview(self.h, q_ptr, q_type, n_q_tokens, m, nm, out,
                                                 C.byref(n), C.byref(ep), C.byref(rows)), "preview")
        return Selection(ep.value, rows.value, list(out[: n.value]))

    def preview_meank(self, q_sum_ptr: int, q_count: Sequence[int],
                      mandatory: Sequence[int] = ()) -> Selection:
        """Preview with the reference's mean-K cosine scorer (q_sum: device
        [n_layers][n_head*head_dim] f32 sums of query rows, q_count per layer)."""
        qc, _ = _u32(q_count)
        m, nm = _u32(mandatory)
        out = (C.c_uint32 * max(1, self.block_count()))()
        n, rows = C.c_uint32(0), C.c_uint32(0)
        ep = C.c_uint64(0)
        self.check(self.lib.kvmem_engine_preview_meank(self.h, q_sum_ptr, qc, m, nm, out, C.byref(n),
                                                       C.byref(ep), C.byref(rows)), "preview_meank")
        return Selection(ep.value, rows.value, list(out[: n.value]))

    def apply(self, sel: Selection) -> dict:
        s, n = _u32(sel.blocks)
        st = PlanStats()
        self.check(self.lib.kvmem_engine_apply(self.h, sel.epoch, sel.rows, s, n, C.byref(st)), "apply")
        return st.as_dict()

    def apply_retrieval(self, q_ptr: int, n_q_tokens: int, q_type: int = TYPE_BF16,
                        mandatory: Sequence[int] = ()) -> dict:
        m, nm = _u32(mandatory)
        st = PlanStats()
        self.check(self.lib.kvmem_engine_apply_retrieval(self.h, q_ptr, q_type, n_q_tokens, m, nm,
                                                         C.byref(st)), "apply_retrieval")
        return st.as_dict()

    # ---- continuation (two-phase API)
    def append_resident(self, n: int) -> None:
        """Rows the caller's decode writes into the pool itself (see block_slots)."""
        self.check(self.lib.kvmem_engine_append_resident(self.h, n), "append_resident")

    def attention_epoch(self) -> int:
        return self.lib.kvmem_engine_attention_epoch(self.h)

    def attention_view(self, canonical: bool = True) -> AttentionView:
        return _get_view(self.lib.kvmem_engine_attention_view, self.h, canonical, self.block_count())

    def selection_fits(self, sel: Selection, end: int, generation_rows: int) -> bool:
        s, ns = _u32(sel.blocks)
        return bool(self.lib.kvmem_engine_selection_fits(self.h, sel.epoch, sel.rows, s, ns, end,
                                                         generation_rows))

    def commit_unchanged(self, before: AttentionView, sel: Selection) -> bool:
        v, keep = before.to_c()
        s, ns = _u32(sel.blocks)
        return bool(self.lib.kvmem_engine_commit_unchanged(self.h, C.byref(v), sel.epoch, sel.rows, s, ns))

    def commit_resident(self, canonical: bool = True) -> bool:
        return bool(self.lib.kvmem_engine_commit_resident(self.h, int(canonical)))

    def can_append(self, end: int, generation_rows: int, all_history: bool) -> tuple[bool, str]:
        why = C.c_char_p()
        ok = self.lib.kvmem_engine_can_append(self.h, end, generation_rows, int(all_history), C.byref(why))
        return bool(ok), why.value.decode()

    def query_replay_fits(self, query_begin: int, prompt_end: int) -> bool:
        return bool(self.lib.kvmem_engine_query_replay_fits(self.h, query_begin, prompt_end))

    def free_slots(self) -> int:
        return self.lib.kvmem_engine_free_slots(self.h)

    def get_query(self):
        """(sums [n_layers][n_head*head_dim] f32, counts [n_layers]) a window preview uses."""
        import numpy as np
        L = self.params.n_layers
        sums = np.zeros((L, self.params.n_head * self.params.head_dim), np.float32)
        cnt = (C.c_uint32 * L)()
        self.check(self.lib.kvmem_engine_get_query(self.h, sums.ctypes.data_as(C.POINTER(C.c_float)), cnt),
                   "get_query")
        return sums, list(cnt)

    def set_query(self, sums, counts) -> None:
        import numpy as np
        a = np.ascontiguousarray(sums, dtype=np.float32)
        cnt = (C.c_uint32 * len(counts))(*counts)
        self.check(self.lib.kvmem_engine_set_query(self.h, a.ctypes.data_as(C.POINTER(C.c_float)), cnt),
                   "set_query")

    def freeze_query(self, frozen: bool) -> None:
        self.check(self.lib.kvmem_engine_freeze_query(self.h, int(frozen)), "freeze_query")

    def scores(self) -> list:
        n = self.block_count()
        out = (C.c_float * max(1, n))()
        self.check(self.lib.kvmem_engine_scores(self.h, out, n), "scores")
        return list(out[:n])


__all__ = ["Store", "Engine", "Selection", "AttentionView", "PlanStats", "EngineParams", "bind",
           "TYPE_Q8_0", "LAYER_MEAN"]
