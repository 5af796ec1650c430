"""The engine's per-token query window on the GPU.

Query rows of strided Qcur views (F32 / F16 / BF16, padded head stride)
are captured per layer over several ubatches, kept by the request span
(the reference's query_contains), capped to the newest query_max_tokens
rows, or the newest query_last when no span is set.  A preview over the
window must equal a preview over the same rows passed explicitly (bit for
bit: the same scorer input), and the oracle chain: per-token max scores
within 1e-3 relative of the fp64 oracle on the bf16-rounded rows; mean-K
scores within 1e-5 of the oracle over the f32 row sums in token order.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

L, T, HKV, HQ, D = 2, 128, 4, 24, 256
E = HKV * D
EQ = HQ * D
PAD = 8
DTYPES = {"f32": (torch.float32, kv.TYPE_F32), "f16": (torch.float16, kv.TYPE_F16),
          "bf16": (torch.bfloat16, kv.TYPE_BF16)}


def announce(msg: str) -> None:
    print(f"[qwindow] {msg}", flush=True)


def engine(**kw):
    p = dict(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D, budget_blocks=8,
             reserve_blocks=4)
    p.update(kw)
    return host.Engine(**p)


class Capture:
    """Seeded Qcur ubatches: per layer a padded [n][HQ][D + PAD] tensor of
    `dtype`; `rows(layer, positions)` gives the captured rows as f32."""

    def __init__(self, dtype: str, seed: int):
        self.tdt, self.code = DTYPES[dtype]
        self.g = torch.Generator(device="cpu").manual_seed(seed)
        self.by_pos = {}

    def ubatch(self, eng, pos0: int, n: int):
        positions = list(range(pos0, pos0 + n))
        for layer in range(L):
            x = (torch.randn((n, HQ, D + PAD), generator=self.g) * 2).to(self.tdt)
            for i, p in enumerate(positions):
                self.by_pos[(layer, p)] = x[i, :, :D].float().reshape(EQ).numpy()
            xd = x.cuda()
            esz = xd.element_size()
            torch.cuda.synchronize()
            eng.capture_q(layer, xd.data_ptr(), self.code, esz, (D + PAD) * esz, HQ * (D + PAD) * esz,
                          positions)
            kv.Context.borrow(eng.ctx_handle()).sync()   # the view is freed after this

    def rows(self, positions) -> np.ndarray:
        """[L][len][HQ][D] f32 rows at these positions."""
        return np.stack([[self.by_pos[(layer, p)] for p in positions] for layer in range(L)]).reshape(
            L, len(positions), HQ, D)


def explicit_q(rows_f32: np.ndarray):
    """The same rows as the bf16 device query kvmem_engine_preview takes."""
    return torch.from_numpy(np.ascontiguousarray(rows_f32)).to(torch.bfloat16).cuda()


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_window_span_per_token_scorer(oracle, dtype):
    announce(f"request span [100, 160) over 3 ubatches of {dtype} Qcur")
    cap, nb = 40, 40
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=71, with_v=True)
    with engine() as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        eng.set_request_span(100, 160, -1)
        cp = Capture(dtype, 72)
        for p0, n in ((64, 64), (128, 64), (192, 8)):
            cp.ubatch(eng, p0, n)
        assert eng.query_rows() == 60
        sel = eng.preview_window()
        got = np.array(eng.scores(), dtype=np.float64)
        rows = cp.rows(range(100, 160))
        qe = explicit_q(rows)
        torch.cuda.synchronize()
        sel2 = eng.preview(qe.data_ptr(), 60)
        got2 = np.array(eng.scores(), dtype=np.float64)
        assert sel.blocks == sel2.blocks and np.array_equal(got, got2)
        qb = qe.float().cpu().numpy()                      # the bf16-rounded rows
        want = oracle.combine_layers(oracle.score_pertoken_max(qb, workloads.to_bits(torch, k)), 0)
        assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-6)) <= 1e-3
        mand = eng.retrieval_mandatory()
        assert mand == [0, 1]
        assert sel.blocks == oracle.pick_topk(got.astype(np.float32).astype(np.float64), 8, sink=1,
                                              mandatory=mand)


def test_window_meank_scorer_sums_in_token_order(oracle):
    announce("mean-K scorer over the window: f32 sums in token order")
    cap, nb = 40, 40
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=73, with_v=True)
    with engine(scorer=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        eng.set_turn_spans(query=[(10, 30), (50, 70)], mandatory=[])
        cp = Capture("f32", 74)
        cp.ubatch(eng, 0, 40)
        cp.ubatch(eng, 40, 40)
        assert eng.query_rows() == 40
        sel = eng.preview_window()
        got = np.array(eng.scores(), dtype=np.float64)
        pos = list(range(10, 30)) + list(range(50, 70))
        q_sum = oracle.q_accumulate(cp.rows(pos).reshape(L, 40, EQ))
        kb = workloads.to_bits(torch, k)
        sums = np.stack([[oracle.meank_sum_f16(kb[l, b].reshape(T, E)) for b in range(nb)]
                         for l in range(L)])
        want = oracle.score_meank(q_sum, [40] * L, sums, np.full((L, nb), T, np.uint32), HQ, HKV, D)
        assert np.max(np.abs(got - want)) <= 1e-5
        assert sel.blocks == oracle.pick_topk(got.astype(np.float32).astype(np.float64), 8, sink=1)


def test_window_cap_and_query_last_fallback(oracle):
    announce("cap 32 keeps the newest rows; no span: the newest query_last = 24")
    cap, nb = 40, 40
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=75, with_v=True)
    with engine(query_max_tokens=32, query_last=24) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        cp = Capture("bf16", 76)
        for p0 in (0, 20, 40):                              # no span: every row captured
            cp.ubatch(eng, p0, 20)
        assert eng.query_rows() == 24
        sel = eng.preview_window()
        got = np.array(eng.scores(), dtype=np.float64)
        qe = explicit_q(cp.rows(range(36, 60)))
        torch.cuda.synchronize()
        assert eng.preview(qe.data_ptr(), 24).blocks == sel.blocks
        assert np.array_equal(np.array(eng.scores(), dtype=np.float64), got)
        eng.reset_query()
        eng.set_request_span(5, 0, -1)                      # open-ended span: rows 5.. (then capped)
        for p0 in (0, 20):
            cp.ubatch(eng, p0, 20)
        assert eng.query_rows() == 32                       # 35 rows kept, the newest 32 read
        sel = eng.preview_window()
        got = np.array(eng.scores(), dtype=np.float64)
        qe = explicit_q(cp.rows(range(8, 40)))
        torch.cuda.synchronize()
        assert eng.preview(qe.data_ptr(), 32).blocks == sel.blocks
        assert np.array_equal(np.array(eng.scores(), dtype=np.float64), got)
        # one layer ahead of the other, then an empty window: refused
        x = torch.zeros((1, HQ, D), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        eng.capture_q(0, x.data_ptr(), kv.TYPE_F32, 4, D * 4, HQ * D * 4, [39])
        with pytest.raises(kv.KvMemError):
            eng.preview_window()
        eng.reset_query()
        with pytest.raises(kv.KvMemError):
            eng.query_rows()


def test_window_write_checks_rows_against_capacity():
    """kvmem_hip_q_window_write refuses a row at or past the window's
    capacity, and a row written twice, before anything is issued; rows in
    range receive their tokens widened exactly."""
    announce("q_window_write: rows checked against the capacity")
    cap, nt = 6, 4
    q = torch.randn((nt, HQ, D), dtype=torch.float32, device="cuda").to(torch.bfloat16)
    win = torch.full((cap, EQ), -7.0, dtype=torch.float32, device="cuda")
    nb0, nb1, nb2 = 2, D * 2, HQ * D * 2
    with kv.Context(0) as ctx:
        for rows in ([0, 6], [5, 5]):
            with pytest.raises(kv.KvMemError):
                ctx.q_window_write(q.data_ptr(), kv.TYPE_BF16, HQ, D, nb0, nb1, nb2, [0, 1], rows,
                                   win.data_ptr(), cap)
        ctx.sync()
        assert bool((win == -7.0).all())
        ctx.q_window_write(q.data_ptr(), kv.TYPE_BF16, HQ, D, nb0, nb1, nb2, [3, 1], [5, 0], win.data_ptr(), cap)
        ctx.sync()
    assert torch.equal(win[5], q[3].float().reshape(-1)) and torch.equal(win[0], q[1].float().reshape(-1))
    assert bool((win[1:5] == -7.0).all())


def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_window_gather_converts_round_to_nearest_even():
    """kvmem_hip_q_window_gather: out[l][i] = window[l][rows[i]] for every
    layer, rows in any order and repeated, copied as f32 or rounded to f16
    or bf16 to nearest even -- halfway cases, f16 subnormals and f16
    overflow included (numpy's conversions are the reference); a row at or
    past the capacity, or an output type other than F32 / F16 / BF16, is
    refused with nothing written."""
    announce("q_window_gather: row order, repeats, f32 / f16 / bf16 rounding")
    cap, n_layers = 9, 2
    rng = np.random.default_rng(17)
    win = (rng.standard_normal((n_layers, cap, EQ)) * 3.0).astype(np.float32)
    special = np.array([1 + 2**-11, 1 + 3 * 2**-11, -(1 + 2**-11), 1.5 * 2**-24, 2**-25, 3 * 2**-26,
                        65504.0, 65519.0, 65520.0, -70000.0, 1 + 2**-8, 1 + 3 * 2**-8, -(1 + 3 * 2**-8),
                        3.0e38, 1e-40, 0.0, -0.0], dtype=np.float32)
    win[:, :, :special.size] = special
    win[1, 2, -special.size:] = special[::-1]
    rows = [4, 0, 8, 4, 2]
    wd = torch.from_numpy(win).to("cuda")
    want32 = win[:, rows]
    with np.errstate(over="ignore"):
        want16 = want32.astype(np.float16).view(np.uint16)
    wantbf = bf16_rne_bits(want32)
    with kv.Context(0) as ctx:
        for name, (tdt, ty) in DTYPES.items():
            out = torch.full((n_layers, len(rows), EQ), 7, dtype=tdt, device="cuda")
            torch.cuda.synchronize()
            ctx.q_window_gather(wd.data_ptr(), n_layers, cap, EQ, rows, ty, out.data_ptr())
            ctx.sync()
            if name == "f32":
                got = out.cpu().numpy().view(np.uint32)
                assert np.array_equal(got, want32.view(np.uint32)), name
            else:
                got = out.cpu().view(torch.int16).numpy().view(np.uint16)
                want = want16 if name == "f16" else wantbf
                bad = np.flatnonzero(got.ravel() != want.ravel())
                assert bad.size == 0, f"{name}: {bad.size} differ, first at {bad[:4]}: " \
                                      f"{want32.ravel()[bad[:4]]} -> {got.ravel()[bad[:4]]} not {want.ravel()[bad[:4]]}"
        out = torch.full((n_layers, 2, EQ), -3.0, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for rows_bad, ty, code in (([0, cap], kv.TYPE_F32, kv.ERR_INVALID),
                                   ([0, 1], kv.TYPE_Q8_0, kv.ERR_UNSUPPORTED)):
            with pytest.raises(kv.KvMemError) as ex:
                ctx.q_window_gather(wd.data_ptr(), n_layers, cap, EQ, rows_bad, ty, out.data_ptr())
            assert ex.value.code == code, str(ex.value)
        ctx.sync()
        assert bool((out == -3.0).all())


@pytest.mark.parametrize("n_rows", [768, 769, 800])
def test_window_gather_long_row_list(n_rows):
    """Row lists at the kernel arguments' capacity (768 entries, the table
    full) and past it (uploaded), in random order with repeats: f32 copies
    bit-exact and bf16 rounded to nearest even, in every layer."""
    announce(f"q_window_gather: {n_rows} rows")
    cap, n_layers, e = 1024, 2, 256
    rng = np.random.default_rng(41)
    win = (rng.standard_normal((n_layers, cap, e)) * 5).astype(np.float32)
    rows = rng.integers(0, cap, n_rows).tolist()
    wd = torch.from_numpy(win).to("cuda")
    with kv.Context(0) as ctx:
        for tdt, ty in ((torch.float32, kv.TYPE_F32), (torch.bfloat16, kv.TYPE_BF16)):
            out = torch.zeros((n_layers, len(rows), e), dtype=tdt, device="cuda")
            torch.cuda.synchronize()
            ctx.q_window_gather(wd.data_ptr(), n_layers, cap, e, rows, ty, out.data_ptr())
            ctx.sync()
            if ty == kv.TYPE_F32:
                assert np.array_equal(out.cpu().numpy().view(np.uint32), win[:, rows].view(np.uint32))
            else:
                got = out.cpu().view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(got, bf16_rne_bits(np.ascontiguousarray(win[:, rows])))


def test_misaligned_device_history_is_refused():
    """Every reader of the device history (scorer, key sums, stage-in)
    loads 16-byte words: set_device_history refuses a misaligned K or V
    and keeps the history it had."""
    announce("set_device_history: 16-byte alignment")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=4, Tq=4, seed=9, with_v=True)
    with engine() as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), 4, 4 * T)
        with pytest.raises(kv.KvMemError):
            eng.set_device_history(k.data_ptr() + 8, v.data_ptr(), 4, 4 * T)
        assert eng.block_count() == 4
        st = eng.apply_retrieval(q.data_ptr(), 4)
        assert st["n_staged"] == 4


def test_query_state_get_set_freeze(oracle):
    """The query state {sum, count} (llama_kvmem_get_query / set_query /
    freeze_query, llama-memory-kvmem.cpp:3104-3137): get returns the window
    rows summed in token order, bit-exact against the oracle's ordered sum;
    set on a second engine makes its window preview score from the given
    sums (the same scores and selection as the first engine's window) and
    freezes the query, so later captures keep no rows; reset_query drops the
    set state; bad states and the per-token scorer are refused."""
    announce("query state: get, set on another engine, freeze, reset")
    cap, nb = 40, 40
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=83, with_v=True)
    cp = Capture("bf16", 84)
    with engine(scorer=1) as a, engine(scorer=1) as b:
        for eng in (a, b):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        a.set_turn_spans(query=[(20, 60)], mandatory=[])
        cp.ubatch(a, 0, 40)
        cp.ubatch(a, 40, 40)
        sums, counts = a.get_query()
        assert counts == [40] * L
        want = oracle.q_accumulate(cp.rows(range(20, 60)).reshape(L, 40, EQ))
        assert np.array_equal(sums.view(np.uint32), want.view(np.uint32))
        sel_a = a.preview_window()
        scores_a = np.array(a.scores(), dtype=np.float64)
        with pytest.raises(kv.KvMemError):
            b.get_query()                                   # nothing captured yet
        bad = sums.copy()
        bad[0, 3] = np.inf
        for s_, c_ in ((bad, counts), (sums, [40] * (L - 1) + [39]), (sums, [0] * L)):
            with pytest.raises(kv.KvMemError):
                b.set_query(s_, c_)
        b.set_query(sums, counts)
        got_sums, got_counts = b.get_query()
        assert np.array_equal(got_sums.view(np.uint32), sums.view(np.uint32)) and got_counts == counts
        sel_b = b.preview_window()
        assert sel_b.blocks == sel_a.blocks
        assert np.array_equal(np.array(b.scores(), dtype=np.float64), scores_a)
        # frozen: a capture keeps no rows, the set state stays
        b.set_turn_spans(query=[(0, 80)], mandatory=[])
        cp.ubatch(b, 0, 40)
        assert np.array_equal(b.get_query()[0].view(np.uint32), sums.view(np.uint32))
        b.reset_query()                                     # the set state goes; still frozen
        with pytest.raises(kv.KvMemError):
            b.get_query()
        cp.ubatch(b, 0, 40)
        with pytest.raises(kv.KvMemError):
            b.query_rows()
        b.freeze_query(False)
        cp.ubatch(b, 0, 40)
        assert b.query_rows() == 40
    with engine() as t:
        t.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        with pytest.raises(kv.KvMemError):
            t.set_query(sums, counts)                       # the per-token scorer reads rows


def test_set_query_then_unfrozen_rows_add_on(oracle):
    """After set_query, rows captured once the query is unfrozen add onto the
    set state, as the reference's harvest adds each row onto q_sum_ and
    q_count_ after set_query (llama-memory-kvmem.cpp:2164-2172, 3121-3137):
    the sums are the set ones plus the new rows in token order, the counts
    the set ones plus the rows; rows captured while frozen, or before the
    state was set, do not count; a window preview scores from that state."""
    announce("set state, capture frozen (kept nothing), unfreeze, capture: rows add onto the state")
    cap, nb = 40, 40
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=85, with_v=True)
    cp = Capture("bf16", 86)
    rng = np.random.default_rng(87)
    with engine(scorer=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, nb * T)
        eng.set_turn_spans(query=[(0, 200)], mandatory=[])
        cp.ubatch(eng, 0, 12)                           # before the state: replaced by it
        state = (rng.standard_normal((L, EQ)) * 7).astype(np.float32)
        eng.set_query(state, [7] * L)
        cp.ubatch(eng, 12, 5)                           # frozen: kept nothing
        got, counts = eng.get_query()
        assert counts == [7] * L and np.array_equal(got.view(np.uint32), state.view(np.uint32))
        eng.freeze_query(False)
        cp.ubatch(eng, 17, 6)                           # added onto the state
        got, counts = eng.get_query()
        want = oracle.q_accumulate(cp.rows(range(17, 23)).reshape(L, 6, EQ), q_sum=state)
        assert counts == [13] * L
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        sel = eng.preview_window()
        scores = np.array(eng.scores(), dtype=np.float64)
        kb = workloads.to_bits(torch, k)
        sums = np.stack([[oracle.meank_sum_f16(kb[l, b].reshape(T, E)) for b in range(nb)]
                         for l in range(L)])
        want_s = oracle.score_meank(want, [13] * L, sums, np.full((L, nb), T, np.uint32), HQ, HKV, D)
        assert np.max(np.abs(scores - want_s)) <= 1e-5
        assert sel.blocks == oracle.pick_topk(scores.astype(np.float32).astype(np.float64), 8, sink=1)
        eng.reset_query()                               # the state and the rows go
        with pytest.raises(kv.KvMemError):
            eng.get_query()
