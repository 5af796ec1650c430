"""Writes the golden fixtures of the CPU tests (run in a container that has
the reference tree; the fixtures are committed, this script is how they
were made).

quant_vectors.npz
    F16 rows (crafted special groups + N(0,1) with x20 outlier channels +
    Student-t nu=4) and their ggml q8_0 / q4_0 / q5_0 bytes, computed by
    an independent numpy restatement of ggml's quantize_row_*_ref
    (float32 arithmetic, one rounding per operation, roundf = half away
    from zero, f16 scale by round-to-nearest-even).  Independent of
    oracle/kvmem_oracle_quant.c, which the tests check against it.

meank_vectors.npz
    F16 key rows of 2.6 blocks and the mean-K of each block as the
    reference's own RawKvStore computes it (kvmem/src/host/raw_kv_store.cpp,
    compiled into oracle/_ref).

select_sequences.json
    Multi-step reselect scenarios produced by the reference's own host
    library (kvmem/src/host/kvmem_store.cpp + kvmem_runtime.cpp, compiled
    from its sources into oracle/_ref by `make -C oracle ref`): per step
    the scores, mandatory ids, KvMemStore::pick_topk_blocks' selection,
    the KvMemPlan of set_selection (stage_in, stage_out, counters) and the
    per-block slot / tier / working-set / baked position after
    finish_reselect with the adapter's LIFO slot allocator.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF_LIB = HERE.parents[1] / "oracle" / "_ref" / "libkvmem_ref.so"

F32 = np.float32


# ------------------------------------------------------------- quantizers
def _f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _scale_bits(d: np.float32) -> int:
    return int(np.array([d], dtype=np.float32).astype(np.float16).view(np.uint16)[0])


def _roundf(v: np.ndarray) -> np.ndarray:
    """C roundf on float32 values: half away from zero (exact in float64)."""
    v64 = v.astype(np.float64)
    return np.sign(v64) * np.floor(np.abs(v64) + 0.5)


def np_q8_0(x: np.ndarray) -> bytes:
    out = bytearray()
    for g in x.reshape(-1, 32).astype(np.float32):
        amax = F32(np.max(np.abs(g)))
        d = F32(amax / F32(127.0))
        idv = F32(F32(1.0) / d) if d != 0 else F32(0.0)
        q = _roundf((g * idv).astype(np.float32)).astype(np.int64)
        out += _scale_bits(d).to_bytes(2, "little")
        out += bytes((q & 0xFF).astype(np.uint8).tolist())
    return bytes(out)


def _signed_absmax(g: np.ndarray) -> np.float32:
    a = np.abs(g)
    if a.max() == 0:
        return F32(0.0)
    return F32(g[int(np.argmax(a))])   # first index of the largest magnitude


def _codes(g: np.ndarray, idv: np.float32, bias: float, top: int) -> np.ndarray:
    s = (g * idv).astype(np.float32)
    t = (s + F32(bias)).astype(np.float32)
    return np.minimum(top, np.trunc(t.astype(np.float64)).astype(np.int64))


def np_q4_0(x: np.ndarray) -> bytes:
    out = bytearray()
    for g in x.reshape(-1, 32).astype(np.float32):
        d = F32(_signed_absmax(g) / F32(-8.0))
        idv = F32(F32(1.0) / d) if d != 0 else F32(0.0)
        c = _codes(g, idv, 8.5, 15)
        out += _scale_bits(d).to_bytes(2, "little")
        out += bytes(((c[:16] & 0xF) | ((c[16:] & 0xF) << 4)).astype(np.uint8).tolist())
    return bytes(out)


def np_q5_0(x: np.ndarray) -> bytes:
    out = bytearray()
    for g in x.reshape(-1, 32).astype(np.float32):
        d = F32(_signed_absmax(g) / F32(-16.0))
        idv = F32(F32(1.0) / d) if d != 0 else F32(0.0)
        c = _codes(g, idv, 16.5, 31)
        qh = 0
        for j in range(32):
            qh |= ((int(c[j]) >> 4) & 1) << j
        out += _scale_bits(d).to_bytes(2, "little")
        out += qh.to_bytes(4, "little")
        out += bytes(((c[:16] & 0xF) | ((c[16:] & 0xF) << 4)).astype(np.uint8).tolist())
    return bytes(out)


def special_groups() -> list[np.ndarray]:
    """Groups (f16 bits) that pin edge behaviour."""
    rng = np.random.default_rng(101)
    g = []
    z = np.zeros(32, np.float32)
    g.append(_f16_bits(z))                                          # all zero
    x = z.copy(); x[0] = -0.0; g.append(_f16_bits(x))               # -0 only
    x = z.copy(); x[7] = 3.0; g.append(_f16_bits(x))                # single positive
    x = z.copy(); x[7] = -3.0; g.append(_f16_bits(x))               # single negative
    x = z.copy(); x[:8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5]; g.append(_f16_bits(x))
    x = z.copy(); x[2] = -3.0; x[5] = 3.0; g.append(_f16_bits(x))   # tie, negative first
    x = z.copy(); x[2] = 3.0; x[5] = -3.0; g.append(_f16_bits(x))   # tie, positive first
    x = z.copy(); x[31] = -8.0; x[:4] = [7.5, 0.5, -0.5, 1.0]; g.append(_f16_bits(x))
    x = z.copy(); x[31] = -16.0; x[:6] = [15.5, 0.5, -0.5, 1.5, 7.5, -15.5]; g.append(_f16_bits(x))
    x = z.copy(); x[3] = 65504.0; x[4] = -65504.0; x[5] = 1.0; g.append(_f16_bits(x))
    b = np.zeros(32, np.uint16); b[9] = 0x0001; g.append(b)         # smallest subnormal
    b = np.zeros(32, np.uint16); b[0] = 0x8001; b[1] = 0x0001; g.append(b)
    g.append(rng.integers(0, 0x0400, 32).astype(np.uint16))         # all subnormal
    g.append(_f16_bits(rng.standard_normal(32) * 1e-5))             # subnormal scale
    g.append(_f16_bits(np.full(32, 0.75)))                          # constant
    x = np.full(32, -1.0, np.float32); x[::2] = 1.0; g.append(_f16_bits(x))
    g.append(_f16_bits(np.arange(-16, 16, dtype=np.float32)))       # every q4 code
    g.append(_f16_bits(np.arange(32, dtype=np.float32) - 15.5))     # half-way grid
    return g


def quant_inputs() -> np.ndarray:
    """96 rows x 256 elements (8 groups each) of f16 bits."""
    rng = np.random.default_rng(7)
    rows = np.zeros((96, 256), np.uint16)
    x = rng.standard_normal((32, 256)).astype(np.float32)
    x[:, [3, 77, 130, 255]] *= 20.0                                 # outlier channels
    rows[:32] = _f16_bits(x)
    rows[32:64] = _f16_bits(np.clip(rng.standard_t(4.0, (32, 256)), -6e4, 6e4))
    rows[64:] = _f16_bits(rng.standard_normal((32, 256)) * 3.0)
    for i, gb in enumerate(special_groups()):
        r, c = divmod(i, 8)
        rows[64 + r, c * 32:(c + 1) * 32] = gb
    return rows


def write_quant() -> None:
    rows = quant_inputs()
    xs = rows.view(np.float16).astype(np.float32)
    out = {"rows": rows}
    for name, fn, gb in (("q8_0", np_q8_0, 34), ("q4_0", np_q4_0, 18), ("q5_0", np_q5_0, 22)):
        out[name] = np.frombuffer(b"".join(fn(r) for r in xs), np.uint8).reshape(len(rows), 8 * gb)
    np.savez_compressed(HERE / "quant_vectors.npz", **out)


# ------------------------------------------------ selection / diff / slots
def _ref_lib() -> C.CDLL:
    lib = C.CDLL(str(REF_LIB))
    u32, vp = C.c_uint32, C.c_void_p
    pu32 = C.POINTER(C.c_uint32)
    lib.kref_runtime_new.restype = vp
    lib.kref_runtime_new.argtypes = [u32] * 6
    lib.kref_runtime_free.argtypes = [vp]
    lib.kref_runtime_set_scores.argtypes = [vp, C.POINTER(C.c_double), u32]
    lib.kref_runtime_preview.argtypes = [vp, pu32, u32, pu32, pu32]
    lib.kref_runtime_apply.argtypes = [vp, pu32, u32, pu32, pu32, pu32, pu32, pu32]
    lib.kref_runtime_blocks.argtypes = [vp, C.POINTER(C.c_int32), C.POINTER(C.c_uint8),
                                        C.POINTER(C.c_uint8), C.POINTER(C.c_int64)]
    lib.kref_runtime_blocks.restype = u32
    return lib


def write_select(n_scenarios: int = 40, steps: int = 3) -> None:
    lib = _ref_lib()
    rng = np.random.default_rng(2024)
    scenarios = []
    for sc in range(n_scenarios):
        bt = int(rng.choice([32, 128]))
        n_tok = int(rng.integers(1, 48)) * bt + int(rng.integers(0, bt))
        budget = int(rng.integers(1, 24))
        sink = int(rng.integers(0, 3))
        recent = int(rng.integers(0, 3))
        n_slots = budget + int(rng.integers(0, 4))
        h = lib.kref_runtime_new(bt, budget, sink, recent, n_slots, n_tok)
        n = (n_tok + bt - 1) // bt
        rec = {"block_tokens": bt, "n_tokens": n_tok, "budget_blocks": budget, "sink": sink,
               "recent": recent, "n_slots": n_slots, "steps": []}
        for _ in range(steps):
            if sc % 3 == 0:
                scores = rng.integers(-2, 3, n).astype(np.float64)   # many exact ties
            else:
                scores = np.round(rng.standard_normal(n), 6)
            mand = sorted(rng.choice(n, int(rng.integers(0, 3)), replace=True).tolist()) if n else []
            lib.kref_runtime_set_scores(h, scores.ctypes.data_as(C.POINTER(C.c_double)), n)
            ma = (C.c_uint32 * max(1, len(mand)))(*mand)
            out = (C.c_uint32 * max(1, n))()
            cnt = C.c_uint32()
            lib.kref_runtime_preview(h, ma, len(mand), out, C.byref(cnt))
            sel = list(out[: cnt.value])
            sa = (C.c_uint32 * max(1, n))(*sel)
            si, so = (C.c_uint32 * max(1, n))(), (C.c_uint32 * max(1, n))()
            ni, no = C.c_uint32(), C.c_uint32()
            ctr = (C.c_uint32 * 5)()
            lib.kref_runtime_apply(h, sa, len(sel), si, C.byref(ni), so, C.byref(no), ctr)
            gs, tr = (C.c_int32 * max(1, n))(), (C.c_uint8 * max(1, n))()
            ws, bk = (C.c_uint8 * max(1, n))(), (C.c_int64 * max(1, n))()
            lib.kref_runtime_blocks(h, gs, tr, ws, bk)
            rec["steps"].append({
                "scores": scores.tolist(), "mandatory": mand, "selection": sel,
                "stage_in": list(si[: ni.value]), "stage_out": list(so[: no.value]),
                "counters": {"selection_overlap_blocks": ctr[0], "gpu_reused_blocks": ctr[1],
                             "retained_position_stable": ctr[2], "retained_position_moved": ctr[3],
                             "total_window_tokens": ctr[4]},
                "gpu_slot": list(gs[:n]), "tier": list(tr[:n]), "in_ws": list(ws[:n]),
                "baked_pos": list(bk[:n]),
            })
        lib.kref_runtime_free(h)
        scenarios.append(rec)
    (HERE / "select_sequences.json").write_text(json.dumps({
        "source": "reference kvmem host library (KvMemStore/KvMemRuntime) via oracle/ref_shim.cpp; "
                  "blocks start outside the GPU pool; LIFO slot allocator; TopK policy; "
                  "ties rank the higher block id first",
        "scenarios": scenarios}, separators=(",", ":")))


def write_meank() -> None:
    """F16 key rows and the reference RawKvStore's mean-K of each block
    (write_layer_tokens_f16 then mean_k, the capture_mean_f16 path)."""
    lib = C.CDLL(str(REF_LIB))
    lib.kref_mean_k_f16.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                    C.c_void_p]
    rng = np.random.default_rng(33)
    E, bt, n = 256, 32, 75                       # two full blocks and a partial one
    x = rng.standard_normal((n, E)).astype(np.float32)
    x[:, 5] *= 3e3                                # large channel: rounding in the sums
    x[::3, 9] = -x[::3, 9] * 1e4
    rows = x.astype(np.float16).view(np.uint16)
    means = np.zeros((3, E), np.float32)
    for b in range(3):
        lib.kref_mean_k_f16(E, bt, rows.ctypes.data, n, b, means[b].ctypes.data)
    np.savez_compressed(HERE / "meank_vectors.npz", rows=rows, block_tokens=np.array(bt),
                        means=means)


if __name__ == "__main__":
    write_quant()
    if REF_LIB.exists():
        write_select()
        write_meank()
    else:
        print(f"{REF_LIB} not built: `make -C oracle ref` (needs the reference tree)")
