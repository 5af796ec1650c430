"""kvmem-llama.cpp_amd -- MI355X-native KVMem reselect path.

Python view of libkvmem_hip.so (built in-tree by build.py): the device ABI of
include/kvmem_hip.h (stage-in quantize-scatter, MFMA block scorer, top-k)
and the host mirror of the reference's store / runtime / reselect interface
of include/kvmem_host.h (KvMemStore, KvMemRuntime, ReselectEngine).

The directory name is not a Python identifier; load it with
`load_package()` from tests/conftest.py or __graft_entry__.py, which imports
this file under the module name ``kvmem_amd``.

Nothing here falls back to a CPU path: if the shared library is missing or
a call fails, an exception is raised.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import sys
import weakref
from pathlib import Path
from typing import Iterable, Sequence

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libkvmem_hip.so"

# ggml type codes (include/kvmem_hip.h)
TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q5_0 = 6
TYPE_Q8_0 = 8
TYPE_BF16 = 30
TYPE_NAMES = {TYPE_F16: "f16", TYPE_Q4_0: "q4_0", TYPE_Q5_0: "q5_0", TYPE_Q8_0: "q8_0"}
GROUP_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_0: 18, TYPE_Q5_0: 22, TYPE_F16: 64}

LAYER_MEAN, LAYER_MAX, LAYER_SUM = 0, 1, 2

OK, ERR_INVALID, ERR_RUNTIME, ERR_NOMEM, ERR_STALE, ERR_UNSUPPORTED, ERR_BUSY = range(7)

# stage bits of Context.perf_stages (KVMEM_PERF_STAGE_*)
PERF_STAGE_SCORE, PERF_STAGE_TOPK, PERF_STAGE_SET, PERF_STAGE_COPY, PERF_STAGE_LAYOUT = 1, 2, 4, 8, 16
PERF_STAGE_STAGE_OUT, PERF_STAGE_PLAN, PERF_STAGE_MEANK_COS = 32, 64, 128
PERF_STAGE_ALL = 0xffffffff

# operation kinds of Context.debug_fail_after (kvmem_hip_fail_kind)
FAIL_ALLOC, FAIL_COPY, FAIL_LAUNCH = 1, 2, 4


def row_size(type_: int, n: int) -> int:
    """ggml_row_size for the types on this path (n % 32 == 0)."""
    return GROUP_BYTES[type_] * (n // 32)


class KvMemError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class StaleSelection(KvMemError):
    """The selection's epoch / row count no longer matches the memory
    (the reference throws std::runtime_error("stale KVMem selection"),
    llama-memory-kvmem.cpp:3144-3147)."""


# ----------------------------------------------------------------- ABI types
class QuantOp(C.Structure):
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p), ("n_rows", C.c_uint32),
                ("n_embd", C.c_uint32), ("type", C.c_int32), ("src_stride", C.c_uint32)]


class History(C.Structure):
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("n_layers", C.c_uint32),
                ("n_blocks", C.c_uint32), ("block_tokens", C.c_uint32),
                ("n_embd_k", C.c_uint32), ("n_embd_v", C.c_uint32),
                ("last_block_tokens", C.c_uint32), ("capacity_blocks", C.c_uint32)]


class HostHistory(C.Structure):
    _fields_ = [("base", C.c_void_p), ("n_layers", C.c_uint32), ("n_blocks", C.c_uint32),
                ("block_tokens", C.c_uint32), ("n_embd_k", C.c_uint32),
                ("n_embd_v", C.c_uint32), ("last_block_tokens", C.c_uint32)]


class Transform(C.Structure):
    _fields_ = [("head_dim", C.c_uint32), ("n_rot", C.c_uint32), ("theta", C.POINTER(C.c_float)),
                ("hadamard_k", C.c_uint32), ("hadamard_v", C.c_uint32),
                ("pos0", C.POINTER(C.c_int32))]


class Pool(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_slots", C.c_uint32), ("block_tokens", C.c_uint32),
                ("n_embd_k", C.c_uint32), ("n_embd_v", C.c_uint32), ("type_k", C.c_int32),
                ("type_v", C.c_int32), ("k_layers", C.POINTER(C.c_void_p)),
                ("v_layers", C.POINTER(C.c_void_p)), ("xf", C.POINTER(Transform))]


class PackedHost(C.Structure):
    _fields_ = [("base", C.c_void_p), ("n_layers", C.c_uint32), ("n_blocks", C.c_uint32),
                ("block_tokens", C.c_uint32)]


class ScoreArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("q_type", C.c_int32), ("n_q_tokens", C.c_uint32),
                ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32),
                ("layer_reduce", C.c_int32), ("layer_scores", C.c_void_p), ("scores", C.c_void_p)]


class MeanKArgs(C.Structure):
    _fields_ = [("q_sum", C.c_void_p), ("q_count", C.POINTER(C.c_uint32)), ("k_sum", C.c_void_p),
                ("mean_tokens", C.c_void_p), ("n_layers", C.c_uint32), ("n_blocks", C.c_uint32),
                ("capacity_blocks", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("head_dim", C.c_uint32), ("scores", C.c_void_p)]


class ReserveArgs(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_blocks", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32), ("n_q_tokens", C.c_uint32),
                ("max_items", C.c_uint32), ("pad0", C.c_uint32), ("h2d_block_bytes", C.c_uint64),
                ("d2h_block_bytes", C.c_uint64), ("move_bytes", C.c_uint64)]


class Scratch(C.Structure):
    _fields_ = [("device_bytes", C.c_uint64), ("pinned_bytes", C.c_uint64), ("allocations", C.c_uint64)]


class TransferStats(C.Structure):
    """kvmem_hip_transfer_stats: bytes / calls per direction (H2D, D2H, D2D)."""
    _fields_ = [("bytes", C.c_uint64 * 3), ("calls", C.c_uint64 * 3)]

    def as_dict(self) -> dict:
        names = ("h2d", "d2h", "d2d")
        return {f"{n}_{what}": int(getattr(self, what)[i]) for i, n in enumerate(names)
                for what in ("bytes", "calls")}


class Perf(C.Structure):
    _fields_ = [("score_ms", C.c_double), ("topk_ms", C.c_double), ("set_ms", C.c_double),
                ("copy_ms", C.c_double), ("layout_ms", C.c_double), ("n_score", C.c_uint64),
                ("n_topk", C.c_uint64), ("n_set", C.c_uint64), ("n_copy", C.c_uint64),
                ("n_layout", C.c_uint64), ("h2d_bytes", C.c_uint64), ("d2d_bytes", C.c_uint64),
                ("after_score_ms", C.c_double), ("n_after_score", C.c_uint64),
                ("stage_out_ms", C.c_double), ("plan_ms", C.c_double), ("n_stage_out", C.c_uint64),
                ("n_plan", C.c_uint64), ("d2h_bytes", C.c_uint64), ("meank_cos_ms", C.c_double),
                ("n_meank_cos", C.c_uint64)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_lib: C.CDLL | None = None

# Every open handle (contexts, engines, stores).  They are closed at
# interpreter exit by close_all(), an atexit hook, while the HIP runtime is
# fully up; a finalizer running later, during interpreter shutdown, does
# nothing (the process is ending and the runtime may already be tearing
# down), so no HIP call is made from module teardown.
_live: "weakref.WeakSet" = weakref.WeakSet()


def track(obj) -> None:
    """Register a handle owner (an object with close() and a _close_rank:
    lower ranks close first) for close_all()."""
    _live.add(obj)


def close_all() -> None:
    """Close every open engine, store and context: engines and stores
    first (they destroy their own contexts), then stand-alone contexts."""
    for obj in sorted(list(_live), key=lambda o: getattr(o, "_close_rank", 1)):
        try:
            obj.close()
        except Exception:
            pass


atexit.register(close_all)


def _sig(lib: C.CDLL, name: str, res, *args) -> None:
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def load_library(path: os.PathLike | str | None = None) -> C.CDLL:
    """Load libkvmem_hip.so (raises if it was not built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} not built: run `python kvmem-llama.cpp_amd/build.py`")
    lib = C.CDLL(str(p), mode=C.RTLD_LOCAL)
    vp, u32, i32, sz = C.c_void_p, C.c_uint32, C.c_int, C.c_size_t
    pu32 = C.POINTER(C.c_uint32)
    _sig(lib, "kvmem_hip_create", i32, i32, C.POINTER(vp))
    _sig(lib, "kvmem_hip_destroy", None, vp)
    _sig(lib, "kvmem_hip_last_error", C.c_char_p, vp)
    _sig(lib, "kvmem_hip_set_stream", i32, vp, vp)
    _sig(lib, "kvmem_hip_get_stream", vp, vp)
    _sig(lib, "kvmem_hip_sync", i32, vp)
    _sig(lib, "kvmem_hip_quant_ok", i32, i32)
    _sig(lib, "kvmem_hip_row_size", sz, i32, C.c_int64)
    _sig(lib, "kvmem_hip_stagein_quant", i32, vp, C.POINTER(QuantOp), i32)
    _sig(lib, "kvmem_hip_stagein_blocks", i32, vp, C.POINTER(History), C.POINTER(Pool), pu32, pu32, u32)
    _sig(lib, "kvmem_hip_stagein_blocks_host", i32, vp, C.POINTER(HostHistory), C.POINTER(Pool),
         pu32, pu32, u32)
    _sig(lib, "kvmem_hip_move_slots", i32, vp, C.POINTER(Pool), pu32, pu32, pu32, u32)
    _sig(lib, "kvmem_hip_d2d_batched", i32, vp, C.POINTER(vp), C.POINTER(vp), C.POINTER(sz), i32)
    _sig(lib, "kvmem_hip_score", i32, vp, C.POINTER(History), C.POINTER(ScoreArgs))
    _sig(lib, "kvmem_hip_score_noalloc", i32, vp, C.POINTER(History), C.POINTER(ScoreArgs))
    _sig(lib, "kvmem_hip_topk", i32, vp, vp, u32, pu32, u32, u32, i32, pu32, pu32)
    _sig(lib, "kvmem_hip_meank_sums", i32, vp, C.POINTER(History), pu32, u32, vp, vp)
    _sig(lib, "kvmem_hip_meank_sums_host", i32, vp, C.POINTER(HostHistory), pu32, u32, u32, vp, vp)
    _sig(lib, "kvmem_hip_score_meank", i32, vp, C.POINTER(MeanKArgs))
    _sig(lib, "kvmem_hip_q_accumulate", i32, vp, vp, i32, u32, u32, u32, pu32, u32, i32, vp)
    _sig(lib, "kvmem_hip_meank_add", i32, vp, vp, i32, u32, u32, sz, sz, sz, u32, u32, i32, vp, vp)
    _sig(lib, "kvmem_hip_check_scale_arith", i32, vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64))
    _sig(lib, "kvmem_hip_stageout_blocks", i32, vp, C.POINTER(Pool), C.POINTER(PackedHost), pu32, pu32,
         pu32, u32)
    _sig(lib, "kvmem_hip_stagein_packed_host", i32, vp, C.POINTER(PackedHost), C.POINTER(Pool), pu32, pu32,
         pu32, u32)
    _sig(lib, "kvmem_hip_reserve", i32, vp, C.POINTER(ReserveArgs))
    _sig(lib, "kvmem_hip_scratch_info", i32, vp, C.POINTER(Scratch))
    _sig(lib, "kvmem_hip_h2d_async", i32, vp, vp, vp, sz)
    _sig(lib, "kvmem_hip_debug_fail_after", i32, vp, u32, C.c_uint64)
    _sig(lib, "kvmem_hip_debug_fail_left", C.c_uint64, vp)
    _sig(lib, "kvmem_hip_perf_enable", i32, vp, i32)
    _sig(lib, "kvmem_hip_perf_stages", i32, vp, C.c_uint32)
    _sig(lib, "kvmem_hip_perf_get", i32, vp, C.POINTER(Perf))
    _sig(lib, "kvmem_hip_perf_reset", None, vp)
    _sig(lib, "kvmem_hip_q_window_write", i32, vp, vp, i32, C.c_uint32, C.c_uint32, C.c_size_t, C.c_size_t,
         C.c_size_t, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32, vp, C.c_uint32)
    _sig(lib, "kvmem_hip_q_window_gather", i32, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32,
         C.POINTER(C.c_uint32), C.c_uint32, i32, vp)
    _sig(lib, "kvmem_hip_transfer_get", i32, vp, C.POINTER(TransferStats))
    if path is None:
        _lib = lib
    return lib


def _u32_array(xs: Iterable[int]):
    xs = list(xs)
    return (C.c_uint32 * max(1, len(xs)))(*xs), len(xs)


def _ptr_array(ptrs: Sequence[int]):
    return (C.c_void_p * max(1, len(ptrs)))(*ptrs)


class Context:
    """A kvmem_hip_ctx on one GPU (explicit handle, own stream by default)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        rc = self.lib.kvmem_hip_create(device, C.byref(h))
        if rc != OK:
            raise KvMemError(rc, f"kvmem_hip_create(device={device}) failed")
        self.h = h
        self._keep: list = []
        track(self)

    _close_rank = 1

    @classmethod
    def borrow(cls, handle: int) -> "Context":
        """Wrap a context owned elsewhere (e.g. a reselect engine's); close()
        leaves it alive."""
        c = cls.__new__(cls)
        c.lib = load_library()
        c.h = C.c_void_p(handle)
        c._keep = []
        c._borrowed = True
        return c

    def close(self) -> None:
        if getattr(self, "h", None):
            if not getattr(self, "_borrowed", False):
                self.lib.kvmem_hip_destroy(self.h)
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

    # -- errors
    def check(self, rc: int, what: str) -> None:
        if rc == OK:
            return
        msg = self.lib.kvmem_hip_last_error(self.h).decode()
        cls = StaleSelection if rc == ERR_STALE else KvMemError
        raise cls(rc, f"{what}: {msg}")

    def last_error(self) -> str:
        return self.lib.kvmem_hip_last_error(self.h).decode()

    # -- streams
    def set_stream(self, stream_handle: int | None) -> None:
        self.check(self.lib.kvmem_hip_set_stream(self.h, stream_handle or None), "set_stream")

    def stream(self) -> int:
        return self.lib.kvmem_hip_get_stream(self.h) or 0

    def sync(self) -> None:
        self.check(self.lib.kvmem_hip_sync(self.h), "sync")

    # -- stage-in
    def stagein_quant(self, ops: Sequence[tuple]) -> None:
        """ops: (src_ptr, dst_ptr, n_rows, n_embd, type[, src_stride])."""
        arr = (QuantOp * max(1, len(ops)))()
        for i, op in enumerate(ops):
            src, dst, n_rows, n_embd, type_ = op[:5]
            stride = op[5] if len(op) > 5 else 0
            arr[i] = QuantOp(src, dst, n_rows, n_embd, type_, stride)
        self.check(self.lib.kvmem_hip_stagein_quant(self.h, arr, len(ops)), "stagein_quant")

    @staticmethod
    def make_history(k_ptr, v_ptr, n_layers, n_blocks, block_tokens, n_embd_k, n_embd_v,
                     last_block_tokens=0, capacity_blocks=0) -> History:
        return History(k_ptr or None, v_ptr or None, n_layers, n_blocks, block_tokens,
                       n_embd_k, n_embd_v, last_block_tokens, capacity_blocks)

    def make_pool(self, n_layers, n_slots, block_tokens, n_embd_k, n_embd_v, type_k, type_v,
                  k_ptrs: Sequence[int], v_ptrs: Sequence[int] | None,
                  xf: "Transform | None" = None) -> Pool:
        ka = _ptr_array(k_ptrs)
        va = _ptr_array(v_ptrs) if v_ptrs is not None else None
        self._keep.extend([ka, va, xf])
        return Pool(n_layers, n_slots, block_tokens, n_embd_k, n_embd_v, type_k, type_v,
                    C.cast(ka, C.POINTER(C.c_void_p)),
                    C.cast(va, C.POINTER(C.c_void_p)) if va is not None else None,
                    C.pointer(xf) if xf is not None else None)

    def make_transform(self, head_dim: int, n_rot: int = 0, theta=None, hadamard_k: int = 0,
                       hadamard_v: int = 0, pos0=None) -> Transform:
        """The cache's row transform (RoPE frequencies theta[n_rot/2], optional
        per-block positions of token 0 for the next stage-in call)."""
        vals = [float(t) for t in theta][: n_rot // 2] if theta is not None else []
        th = (C.c_float * max(1, n_rot // 2))(*vals)
        ps = (C.c_int32 * len(pos0))(*[int(p) for p in pos0]) if pos0 is not None else None
        self._keep.extend([th, ps])
        return Transform(head_dim, n_rot, C.cast(th, C.POINTER(C.c_float)) if theta is not None else None,
                         hadamard_k, hadamard_v, C.cast(ps, C.POINTER(C.c_int32)) if ps is not None else None)

    def stagein_blocks(self, hist: History, pool: Pool, block_ids, slots) -> None:
        ids, n = _u32_array(block_ids)
        sl, m = _u32_array(slots)
        assert n == m
        self.check(self.lib.kvmem_hip_stagein_blocks(self.h, C.byref(hist), C.byref(pool), ids, sl, n),
                   "stagein_blocks")

    def stageout_blocks(self, pool: Pool, dst: PackedHost, block_ids, slots, n_tokens) -> None:
        """Pool slots -> packed host blocks (asynchronous until sync())."""
        ids, n = _u32_array(block_ids)
        sl, m = _u32_array(slots)
        nt, k = _u32_array(n_tokens)
        assert n == m == k
        self.check(self.lib.kvmem_hip_stageout_blocks(self.h, C.byref(pool), C.byref(dst), ids, sl, nt, n),
                   "stageout_blocks")

    def stagein_packed_host(self, src: PackedHost, pool: Pool, block_ids, slots, n_tokens) -> None:
        """Packed host blocks -> pool slots, no quantization."""
        ids, n = _u32_array(block_ids)
        sl, m = _u32_array(slots)
        nt, k = _u32_array(n_tokens)
        assert n == m == k
        self.check(self.lib.kvmem_hip_stagein_packed_host(self.h, C.byref(src), C.byref(pool), ids, sl, nt, n),
                   "stagein_packed_host")

    def stagein_blocks_host(self, hist: HostHistory, pool: Pool, block_ids, slots) -> None:
        ids, n = _u32_array(block_ids)
        sl, m = _u32_array(slots)
        assert n == m
        self.check(self.lib.kvmem_hip_stagein_blocks_host(self.h, C.byref(hist), C.byref(pool), ids,
                                                          sl, n), "stagein_blocks_host")

    def move_slots(self, pool: Pool, src_slots, dst_slots, n_tokens=None) -> None:
        """Move the first n_tokens[i] rows (default: whole slots) of slot
        src_slots[i] to dst_slots[i]."""
        s, n = _u32_array(src_slots)
        d, m = _u32_array(dst_slots)
        assert n == m
        nt = None
        if n_tokens is not None:
            nt, k = _u32_array(n_tokens)
            assert k == n
        self.check(self.lib.kvmem_hip_move_slots(self.h, C.byref(pool), s, d, nt, n), "move_slots")

    def reserve(self, **sizes) -> None:
        """Grow scratch for calls of at most these sizes (ReserveArgs fields)."""
        self.check(self.lib.kvmem_hip_reserve(self.h, C.byref(ReserveArgs(**sizes))), "reserve")

    def scratch_info(self) -> dict:
        out = Scratch()
        self.check(self.lib.kvmem_hip_scratch_info(self.h, C.byref(out)), "scratch_info")
        return {name: getattr(out, name) for name, _ in out._fields_}

    def h2d_async(self, dst_ptr: int, src_ptr: int, n: int) -> None:
        """Enqueue an n-byte host-to-device copy on the context stream."""
        self.check(self.lib.kvmem_hip_h2d_async(self.h, dst_ptr or None, src_ptr or None, n), "h2d_async")

    def d2d_batched(self, srcs, dsts, nbytes) -> None:
        n = len(srcs)
        s = (C.c_void_p * max(1, n))(*srcs)
        d = (C.c_void_p * max(1, n))(*dsts)
        b = (C.c_size_t * max(1, n))(*nbytes)
        self.check(self.lib.kvmem_hip_d2d_batched(self.h, s, d, b, n), "d2d_batched")

    # -- scoring / selection
    def score(self, hist: History, q_ptr: int, q_type: int, n_q_tokens: int, n_head: int,
              n_head_kv: int, head_dim: int, scores_ptr: int, layer_scores_ptr: int = 0,
              layer_reduce: int = LAYER_MEAN) -> None:
        a = ScoreArgs(q_ptr, q_type, n_q_tokens, n_head, n_head_kv, head_dim, layer_reduce,
                      layer_scores_ptr or None, scores_ptr)
        self.check(self.lib.kvmem_hip_score(self.h, C.byref(hist), C.byref(a)), "score")

    def score_noalloc(self, hist: History, q_ptr: int, q_type: int, n_q_tokens: int, n_head: int,
                      n_head_kv: int, head_dim: int, scores_ptr: int, layer_scores_ptr: int = 0,
                      layer_reduce: int = LAYER_MEAN) -> None:
        """score() with the library's static per-GPU scratch (allocates nothing)."""
        a = ScoreArgs(q_ptr, q_type, n_q_tokens, n_head, n_head_kv, head_dim, layer_reduce,
                      layer_scores_ptr or None, scores_ptr)
        self.check(self.lib.kvmem_hip_score_noalloc(self.h, C.byref(hist), C.byref(a)), "score_noalloc")

    def topk(self, scores_ptr: int, n: int, need: int, forced=(), tie_lower_index: bool = True) -> list[int]:
        f, nf = _u32_array(forced)
        out = (C.c_uint32 * max(1, n))()
        cnt = C.c_uint32(0)
        self.check(self.lib.kvmem_hip_topk(self.h, scores_ptr, n, f, nf, need, int(tie_lower_index),
                                           out, C.byref(cnt)), "topk")
        return list(out[: cnt.value])

    # -- mean-K cosine scorer (reference semantics)
    def meank_sums(self, hist: History, block_ids, k_sum_ptr: int, mean_tokens_ptr: int) -> None:
        ids, n = _u32_array(block_ids)
        self.check(self.lib.kvmem_hip_meank_sums(self.h, C.byref(hist), ids, n, k_sum_ptr,
                                                 mean_tokens_ptr), "meank_sums")

    def meank_sums_host(self, hist: HostHistory, block_ids, k_sum_ptr: int, mean_tokens_ptr: int,
                        capacity_blocks: int = 0) -> None:
        """Key sums of pinned host blocks (block-major history)."""
        ids, n = _u32_array(block_ids)
        self.check(self.lib.kvmem_hip_meank_sums_host(self.h, C.byref(hist), ids, n, capacity_blocks,
                                                      k_sum_ptr, mean_tokens_ptr), "meank_sums_host")

    def meank_add(self, k_ptr: int, k_type: int, n_embd: int, head_dim: int, nb0: int, nb1: int,
                  nb2: int, tok0: int, n_keep: int, acc_ptr: int, count_ptr: int = 0,
                  reset: bool = False) -> None:
        """acc (+)= the kept tokens' K rows (strided view), token order."""
        self.check(self.lib.kvmem_hip_meank_add(self.h, k_ptr, k_type, n_embd, head_dim, nb0, nb1, nb2,
                                                tok0, n_keep, int(reset), acc_ptr, count_ptr or None),
                   "meank_add")

    def check_scale_arith(self) -> tuple[int, int]:
        """(div127 mismatches, reciprocal mismatches) over their full ranges."""
        a, b = C.c_uint64(0), C.c_uint64(0)
        self.check(self.lib.kvmem_hip_check_scale_arith(self.h, C.byref(a), C.byref(b)), "check_scale_arith")
        return a.value, b.value

    def q_accumulate(self, q_ptr: int, q_type: int, n_layers: int, n_tokens: int, n_embd_q: int,
                     q_sum_ptr: int, tokens=None, reset: bool = True) -> None:
        """q_sum[l] (+)= the listed query rows of layer l, in list order."""
        if tokens is None:
            ids, n = None, 0
        else:
            ids, n = _u32_array(tokens)
        self.check(self.lib.kvmem_hip_q_accumulate(self.h, q_ptr, q_type, n_layers, n_tokens, n_embd_q,
                                                   ids, n, int(reset), q_sum_ptr), "q_accumulate")

    def score_meank(self, q_sum_ptr: int, q_count, k_sum_ptr: int, mean_tokens_ptr: int,
                    n_layers: int, n_blocks: int, n_head: int, n_head_kv: int, head_dim: int,
                    scores_ptr: int, capacity_blocks: int = 0) -> None:
        qc, _ = _u32_array(q_count)
        a = MeanKArgs(q_sum_ptr, C.cast(qc, C.POINTER(C.c_uint32)), k_sum_ptr, mean_tokens_ptr,
                      n_layers, n_blocks, capacity_blocks, n_head, n_head_kv, head_dim, scores_ptr)
        self.check(self.lib.kvmem_hip_score_meank(self.h, C.byref(a)), "score_meank")

    # -- failure injection (host side: nothing faults on the device)
    def debug_fail_after(self, kinds: int, nth_op: int) -> None:
        """The nth_op-th later operation of `kinds` (FAIL_* mask) fails before
        it is issued; 0 switches injection off."""
        self.check(self.lib.kvmem_hip_debug_fail_after(self.h, kinds, nth_op), "debug_fail_after")

    def debug_fail_left(self) -> int:
        """Operations left before the injected failure (0: fired or off)."""
        return self.lib.kvmem_hip_debug_fail_left(self.h)

    # -- profiling
    def perf_enable(self, on: bool = True) -> None:
        self.check(self.lib.kvmem_hip_perf_enable(self.h, int(on)), "perf_enable")

    def perf_stages(self, mask: int) -> None:
        """Time only the stages in `mask` (PERF_STAGE_* bits) while enabled."""
        self.check(self.lib.kvmem_hip_perf_stages(self.h, mask), "perf_stages")

    def perf(self) -> dict:
        p = Perf()
        self.check(self.lib.kvmem_hip_perf_get(self.h, C.byref(p)), "perf_get")
        return p.as_dict()

    def perf_reset(self) -> None:
        self.lib.kvmem_hip_perf_reset(self.h)

    def q_window_write(self, q_ptr: int, q_type: int, n_head: int, head_dim: int, nb0: int, nb1: int,
                       nb2: int, tokens, rows, window_ptr: int, capacity: int) -> None:
        """Tokens of a strided query view into rows of a [capacity][n_head*head_dim] f32 window."""
        t, n = _u32_array(tokens)
        r, m = _u32_array(rows)
        assert n == m
        self.check(self.lib.kvmem_hip_q_window_write(self.h, q_ptr, q_type, n_head, head_dim, nb0, nb1, nb2,
                                                     t, r, n, window_ptr, capacity), "q_window_write")

    def q_window_gather(self, window_ptr: int, n_layers: int, capacity: int, n_embd_q: int, rows,
                        out_type: int, out_ptr: int) -> None:
        """out[l][i] = window[l][rows[i]] for every layer, converted to out_type."""
        r, n = _u32_array(rows)
        self.check(self.lib.kvmem_hip_q_window_gather(self.h, window_ptr, n_layers, capacity, n_embd_q, r, n,
                                                      out_type, out_ptr), "q_window_gather")

    def transfers(self) -> dict:
        """Bytes and calls per direction since the last perf_reset."""
        t = TransferStats()
        self.check(self.lib.kvmem_hip_transfer_get(self.h, C.byref(t)), "transfer_get")
        return t.as_dict()
