"""ctypes view of oracle/liboracle.so -- the CPU restatement of the reselect
path that the tests compare the product against.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

TYPE_F16, TYPE_Q4_0, TYPE_Q5_0, TYPE_Q8_0 = 1, 2, 6, 8
GROUP_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_0: 18, TYPE_Q5_0: 22, TYPE_F16: 64}

_lib = None


def build() -> None:
    r = subprocess.run(["make", "-s", "-C", str(HERE), "all"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    L = C.CDLL(str(LIB))
    u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
    u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
    u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
    u32 = C.c_uint32
    L.ko_f32_to_f16.restype = C.c_uint16
    L.ko_f32_to_f16.argtypes = [C.c_float]
    L.ko_f16_to_f32.restype = C.c_float
    L.ko_f16_to_f32.argtypes = [C.c_uint16]
    L.ko_quantize_rows_f16.restype = C.c_int
    L.ko_quantize_rows_f16.argtypes = [C.c_int, u16p, u8p, C.c_int64, C.c_int64]
    for nm in ("ko_quantize_row_q8_0", "ko_quantize_row_q4_0", "ko_quantize_row_q5_0"):
        getattr(L, nm).restype = None
        getattr(L, nm).argtypes = [f32p, u8p, C.c_int64]
    L.ko_dequantize_row.restype = None
    L.ko_dequantize_row.argtypes = [C.c_int, u8p, f32p, C.c_int64]
    L.ko_stagein_blocks.restype = C.c_int
    L.ko_stagein_blocks.argtypes = [C.c_int, u16p, u32p, u32, u32, u32, u8p, u32]
    L.ko_score_pertoken_max.restype = None
    L.ko_score_pertoken_max.argtypes = [f32p, u16p, u32, u32, u32, u32, u32, u32, u32, u32,
                                        C.c_void_p, u32, f64p]
    L.ko_score_pertoken_max_f32.restype = None
    L.ko_score_pertoken_max_f32.argtypes = [f32p, u16p, u32, u32, u32, u32, u32, u32, u32,
                                            u32, u32, u32, f32p, C.c_int]
    L.ko_combine_layers.restype = None
    L.ko_combine_layers.argtypes = [f64p, u32, u32, C.c_int, f64p]
    L.ko_pick_topk.restype = None
    L.ko_pick_topk.argtypes = [f64p, u32, u32, u32, u32, C.c_void_p, u32, C.c_int, u32p,
                               C.POINTER(C.c_uint32)]
    L.ko_meank_sum_f16.restype = None
    L.ko_meank_sum_f16.argtypes = [u16p, u32, u32, C.c_uint64, f32p]
    L.ko_mean_k.restype = None
    L.ko_mean_k.argtypes = [f32p, u32, u32, f32p]
    L.ko_score_meank.restype = None
    L.ko_score_meank.argtypes = [f32p, u32p, f32p, u32p, u32, u32, u32, u32, u32, f64p]
    L.ko_rope_sincos_n.restype = None
    L.ko_rope_sincos_n.argtypes = [f32p, C.c_uint64, f32p, f32p]
    L.ko_rope_rows.restype = None
    L.ko_rope_rows.argtypes = [f32p, u32, u32, u32, u32, f32p, C.c_int32]
    L.ko_hadamard_rows.restype = None
    L.ko_hadamard_rows.argtypes = [f32p, C.c_uint64, u32]
    L.ko_quantize_rows_f32.restype = C.c_int
    L.ko_quantize_rows_f32.argtypes = [C.c_int, f32p, u8p, C.c_int64, C.c_int64]
    L.ko_q_accumulate.restype = None
    L.ko_q_accumulate.argtypes = [f32p, u32, u32, u32, C.c_void_p, u32, C.c_int, f32p]
    L.ko_div127_mismatches.restype = C.c_uint64
    L.ko_div127_mismatches.argtypes = [C.c_uint32, C.c_uint32]
    L.ko_round_trick_mismatches.restype = C.c_uint64
    L.ko_round_trick_mismatches.argtypes = [C.c_float, C.c_float]
    L.ko_max_threads.restype = C.c_int
    L.ko_max_threads.argtypes = []
    _lib = L
    return L


def row_bytes(type_: int, n: int) -> int:
    return GROUP_BYTES[type_] * (n // 32)


def f32_to_f16(x) -> np.ndarray:
    f = lib().ko_f32_to_f16
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in x], dtype=np.uint16)


def f16_to_f32(h) -> np.ndarray:
    f = lib().ko_f16_to_f32
    h = np.asarray(h, dtype=np.uint16).ravel()
    return np.array([f(int(v)) for v in h], dtype=np.float32)


def quantize_row(type_: int, x: np.ndarray) -> np.ndarray:
    """ggml quantize_row_*_ref on an f32 row (len % 32 == 0)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(row_bytes(type_, x.size), dtype=np.uint8)
    fn = {TYPE_Q8_0: lib().ko_quantize_row_q8_0, TYPE_Q4_0: lib().ko_quantize_row_q4_0,
          TYPE_Q5_0: lib().ko_quantize_row_q5_0}[type_]
    fn(x, out, x.size)
    return out


def quantize_rows_f16(type_: int, rows: np.ndarray) -> np.ndarray:
    """F16 rows [n_rows, n_embd] (uint16 bits) -> packed rows [n_rows, row_bytes]."""
    rows = np.ascontiguousarray(rows, dtype=np.uint16)
    n_rows, n_embd = rows.shape
    out = np.zeros((n_rows, row_bytes(type_, n_embd)), dtype=np.uint8)
    if lib().ko_quantize_rows_f16(type_, rows, out, n_rows, n_embd) != 0:
        raise ValueError("ko_quantize_rows_f16 failed")
    return out


def dequantize_row(type_: int, y: np.ndarray, n: int) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.uint8).ravel()
    out = np.zeros(n, dtype=np.float32)
    lib().ko_dequantize_row(type_, y, out, n)
    return out


def stagein_blocks(type_: int, src: np.ndarray, slots, n_slots: int) -> np.ndarray:
    """src [n_blocks, T, E] uint16 -> pool bytes [n_slots*T, row_bytes] with
    block i written at rows slots[i]*T .. +T."""
    src = np.ascontiguousarray(src, dtype=np.uint16)
    nb, T, E = src.shape
    pool = np.zeros((n_slots * T, row_bytes(type_, E)), dtype=np.uint8)
    sl = np.ascontiguousarray(slots, dtype=np.uint32)
    if lib().ko_stagein_blocks(type_, src, sl, nb, T, E, pool, n_slots) != 0:
        raise ValueError("ko_stagein_blocks failed")
    return pool


def score_pertoken_max(q: np.ndarray, k: np.ndarray, last_block_tokens: int = 0,
                       block_ids=None) -> np.ndarray:
    """q [L,Tq,Hq,D] f32, k [L,B,T,Hkv,D] uint16 (f16 bits) -> [L,B] f64
    (only the columns of block_ids are filled when given)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    L, Tq, Hq, D = q.shape
    L2, B, T, Hkv, D2 = k.shape
    assert L == L2 and D == D2 and Hq % Hkv == 0
    out = np.full((L, B), np.nan, dtype=np.float64)
    if block_ids is None:
        ids_ptr, n_ids = None, 0
    else:
        ids = np.ascontiguousarray(block_ids, dtype=np.uint32)
        ids_ptr, n_ids = ids.ctypes.data, ids.size
    lib().ko_score_pertoken_max(q, k, L, Tq, Hq, Hkv, D, B, T, last_block_tokens, ids_ptr, n_ids, out)
    return out


def score_pertoken_max_f32(q, k, b_begin: int, b_end: int, n_threads: int = 0,
                           last_block_tokens: int = 0) -> np.ndarray:
    """fp32 per-token max scorer: q [L,Tq,Hq,D] f32, k [L,B,T,Hkv,D] f16 bits
    -> [L,B] f32 with columns [b_begin, b_end) filled (the rest NaN)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    L, Tq, Hq, D = q.shape
    L2, B, T, Hkv, D2 = k.shape
    if L != L2 or D != D2 or Hq % Hkv or not 0 <= b_begin <= b_end <= B or last_block_tokens > T:
        raise ValueError("score_pertoken_max_f32: shapes or block range do not match")
    out = np.full((L, B), np.nan, dtype=np.float32)
    lib().ko_score_pertoken_max_f32(q, k, L, Tq, Hq, Hkv, D, B, T, last_block_tokens, b_begin, b_end,
                                    out, n_threads)
    return out


def combine_layers(layer_scores: np.ndarray, mode: int = 0) -> np.ndarray:
    ls = np.ascontiguousarray(layer_scores, dtype=np.float64)
    L, B = ls.shape
    out = np.zeros(B, dtype=np.float64)
    lib().ko_combine_layers(ls, L, B, mode, out)
    return out


def pick_topk(scores, budget: int, sink: int = 1, recent: int = 0, mandatory=(),
              tie_lower_index: bool = True) -> list[int]:
    s = np.ascontiguousarray(scores, dtype=np.float64)
    n = s.size
    mand = np.ascontiguousarray(list(mandatory), dtype=np.uint32)
    out = np.zeros(max(1, n), dtype=np.uint32)
    cnt = C.c_uint32(0)
    lib().ko_pick_topk(s, n, budget, sink, recent, mand.ctypes.data if mand.size else None,
                       mand.size, int(tie_lower_index), out, C.byref(cnt))
    return out[: cnt.value].tolist()


def meank_sum_f16(rows: np.ndarray) -> np.ndarray:
    """[n_tokens, n_embd] f16 bits -> fp32 token-order sum (capture_mean_f16)."""
    rows = np.ascontiguousarray(rows, dtype=np.uint16)
    n, e = rows.shape
    out = np.zeros(e, dtype=np.float32)
    lib().ko_meank_sum_f16(rows, n, e, e, out)
    return out


def mean_k(k_sum: np.ndarray, mean_tokens: int) -> np.ndarray:
    k_sum = np.ascontiguousarray(k_sum, dtype=np.float32)
    out = np.zeros_like(k_sum)
    lib().ko_mean_k(k_sum, mean_tokens, k_sum.size, out)
    return out


def score_meank(q_sum: np.ndarray, q_count, k_sum: np.ndarray, mean_tokens: np.ndarray,
                Hq: int, Hkv: int, D: int) -> np.ndarray:
    """q_sum [L, Hq*D] f32, q_count [L], k_sum [L, B, Hkv*D] f32,
    mean_tokens [L, B] -> scores [B] f64 (score_retrieval)."""
    q_sum = np.ascontiguousarray(q_sum, dtype=np.float32)
    k_sum = np.ascontiguousarray(k_sum, dtype=np.float32)
    mt = np.ascontiguousarray(mean_tokens, dtype=np.uint32)
    qc = np.ascontiguousarray(q_count, dtype=np.uint32)
    L, B = mt.shape
    out = np.zeros(B, dtype=np.float64)
    lib().ko_score_meank(q_sum, qc, k_sum, mt, L, B, Hq, Hkv, D, out)
    return out


def rope_sincos(a) -> tuple[np.ndarray, np.ndarray]:
    """sin, cos (f32) of f32 angles, the library's own evaluation."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    s = np.zeros_like(a)
    c = np.zeros_like(a)
    lib().ko_rope_sincos_n(a, a.size, s, c)
    return s, c


def rope_theta(n_rot: int, freq_base: float = 10000.0, freq_scale: float = 1.0) -> np.ndarray:
    """Pair frequencies as rope.cpp:20-23 forms them: powf(freq_base,
    -2.0f*i/n_rot) * freq_scale, every step in fp32 (the C library's powf,
    which std::pow(float, float) calls)."""
    import ctypes.util
    libm = C.CDLL(ctypes.util.find_library("m"))
    libm.powf.restype = C.c_float
    libm.powf.argtypes = [C.c_float, C.c_float]
    out = np.zeros(n_rot // 2, dtype=np.float32)
    for i in range(n_rot // 2):
        ex = np.float32(np.float32(-2.0) * np.float32(i)) / np.float32(n_rot)
        out[i] = np.float32(libm.powf(float(np.float32(freq_base)), float(ex))) * np.float32(freq_scale)
    return out


def transform_rows(rows: np.ndarray, head_dim: int, n_rot: int = 0, theta=None, pos0: int = 0,
                   hadamard: int = 0) -> np.ndarray:
    """[n_rows, n_embd] f32 -> RoPE'd (n_rot > 0) then Hadamard-rotated
    (hadamard > 0) copy, the raw-K stage-in transform."""
    x = np.array(rows, dtype=np.float32, copy=True, order="C")
    n, e = x.shape
    if n_rot:
        th = np.ascontiguousarray(theta, dtype=np.float32)
        lib().ko_rope_rows(x, n, e, head_dim, n_rot, th, int(pos0))
    if hadamard:
        lib().ko_hadamard_rows(x, x.size, hadamard)
    return x


def quantize_rows_f32(type_: int, rows: np.ndarray) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n, e = rows.shape
    out = np.zeros((n, row_bytes(type_, e)), dtype=np.uint8)
    if lib().ko_quantize_rows_f32(type_, rows, out, n, e) != 0:
        raise ValueError("ko_quantize_rows_f32 failed")
    return out


def q_accumulate(q: np.ndarray, tokens=None, q_sum: np.ndarray | None = None) -> np.ndarray:
    """q [L, T, E] (f32 values; widen bf16/f16 first) -> q_sum [L, E] f32:
    the listed tokens added in order onto q_sum (zeros when None)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    L, T, E = q.shape
    reset = q_sum is None
    out = np.zeros((L, E), np.float32) if reset else np.array(q_sum, dtype=np.float32, copy=True)
    if tokens is None:
        tk, n = None, T
    else:
        tk = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = tk.size
    lib().ko_q_accumulate(q, L, T, E, tk.ctypes.data if tk is not None and n else None, n,
                          int(reset), out)
    return out


def max_threads() -> int:
    return lib().ko_max_threads()
