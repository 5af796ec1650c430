"""Seeded random operation sequences on the reselect engine, checked
against the oracle after every operation.

The reference drives its reselect path from the server loop: retrieval
steps, rows decoded into the pool, rows appended to the host history,
restores that truncate to a checkpoint, and host fallbacks after a failed
device call (src/adapter/llama-memory-kvmem.cpp:2752-2758, 3047-3263;
tests/mtp-kv-test.cpp:144-214, 300-361).  Here those operations come in a
seeded random order:

- a retrieval step through the device plan (apply_retrieval), whose
  resident set must be the preview of the same query and mandatory blocks;
- preview + apply, and apply of a caller's own selection (any order,
  repeated ids, ids past the history; more blocks than slots is refused
  with nothing changed, as the reference's set_selection sorts, de-duplicates
  and drops out-of-range ids, kvmem_store.cpp:758-770);
- a preview made stale by rows appended or cut before its apply;
- rows appended to the history only (append_tokens);
- rows decoded resident (append_resident, then the caller writes the pool
  cells of the blocks they touch, whole blocks from the history);
- a truncation;
- a swap to other history buffers of the same shape (set_device_history):
  every block leaves the pool, and the key sums and saved rows go with it;
- an apply whose n-th device operation is refused on the host
  (kvmem_hip_debug_fail_after: nothing faults);
- commit_unchanged after a preview with the last apply's query and
  mandatory blocks, which must succeed exactly when the selection equals
  the pool's canonical attention view;
- a request span (query rows and force_pos) or turn spans (query and
  mandatory row ranges; a reversed range is refused) set, or the spans
  cleared: the blocks retrieval_mandatory derives are checked after every
  operation, as
  the history grows and shrinks under it, every preview keeps them with the
  sink and the caller's mandatory blocks whenever they fit the budget, and
  selection_fits holds exactly when a preview kept every derived block
  (llama-memory-kvmem.cpp:3026-3045, 3069-3084);
- query rows captured into the engine's window (bf16 Qcur views at random
  positions, kept when the span holds them, the newest 48), or the window
  emptied; then a preview over the window, whose selection and scores must
  equal a preview over the same rows passed explicitly, bit for bit (the
  newest 48 rows with a span set, the newest 16 without), and its apply
  (llama-memory-kvmem.cpp:2157-2172, 2206-2219; tools/llama-kvmem-server.cpp:1032-1038);
- the query state: get_query bit-exact against the oracle's token-order sum
  of the rows the model holds, set_query of a state read back or of a random
  finite one (refused as unsupported by the per-token scorer), freeze and
  unfreeze; a frozen query keeps no captured rows, and rows captured once it
  is unfrozen add onto a set state, as the reference's harvest adds onto
  q_sum_ after set_query (llama-memory-kvmem.cpp:2164-2172, 3104-3137); a
  window preview with a set state scores as the oracle does over it.

A model in the test tracks how many rows of each resident block the pool
holds.  After every operation: the engine's resident set is the model's;
slots are distinct and in range; every resident block's pool rows are the
oracle's quantization of its history rows; after a successful apply the
resident set is the selection, in window order when the layout is canonical.
With a pinned host history and a pinned packed store, every block the engine
marks as saved holds the oracle's rows in the store.  With the row transform
(NeoX RoPE 256 on K at the original positions, then attn_rot), the pool rows
are the oracle's transform and quantization; decoded rows are left out there,
since a transformed pool's decoded cells are the model's to write.  With the
reference's mean-K scorer, every preview's scores are the oracle's over the
history as it stands.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

from engine_helpers import D, E, HQ, L, T, block_major_pinned, decode_rows, history, make_engine  # noqa: E402
from test_gpu_transform import expected_rows  # noqa: E402

ALL_KINDS = kv.FAIL_ALLOC | kv.FAIL_COPY | kv.FAIL_LAUNCH

CASES = [
    # (canonical layout, type_k, type_v, seed, pinned host history + packed store,
    #  row transform: NeoX RoPE 256 on K at the original positions, then attn_rot)
    (1, kv.TYPE_Q8_0, kv.TYPE_Q8_0, 101, False, False),
    (0, kv.TYPE_Q8_0, kv.TYPE_Q4_0, 102, False, False),
    (1, kv.TYPE_Q5_0, kv.TYPE_Q8_0, 103, False, False),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q4_0, 104, True, False),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q4_0, 105, False, True),
    (1, kv.TYPE_Q5_0, kv.TYPE_Q8_0, 108, True, True),
]
# the reference's mean-K cosine scorer over key sums the engine keeps current
MEANK_CASE = (1, kv.TYPE_Q8_0, kv.TYPE_Q8_0, 106, False, False)
XF = dict(n_rot=256, rope_freq_base=1e6, attn_rot=1)
OPS = ["retrieve", "preview_apply", "stale", "append", "decode", "truncate", "fail", "unchanged", "span",
       "capture", "wretrieve", "qstate", "apply_ids", "swap"]
WEIGHTS = np.array([4, 3, 1, 2, 2, 1, 1, 2, 1, 2, 2, 1, 1, 0.5], dtype=float)
QWIN_CAP, QWIN_LAST = 48, 16   # query_max_tokens, query_last
# KVMEM_SEQ_OPS / KVMEM_SEQ_SEED_OFFSET lengthen a run or draw other seeds
N_OPS = int(os.environ.get("KVMEM_SEQ_OPS", "150"))
SEED_OFFSET = int(os.environ.get("KVMEM_SEQ_SEED_OFFSET", "0"))


def announce(msg: str) -> None:
    print(f"[sequences] {msg}", flush=True)


class Model:
    """What the pool must hold: rows of each resident block, and the token count."""

    def __init__(self, eng, oracle, k, v, types, store=None, xf=False):
        self.eng, self.oracle, self.types, self.store = eng, oracle, types, store
        self.theta = oracle.rope_theta(XF["n_rot"], XF["rope_freq_base"]) if xf else None
        self.bits = (workloads.to_bits(torch, k), workloads.to_bits(torch, v))
        self.hist = 0   # which history the engine reads (its rows key the cache)
        self.total = eng.total_tokens()
        self.valid: dict[int, int] = {}
        # the one resident block whose pool rows the engine knows to be stale
        # (a partial tail that grew, or a decoded tail that had no slot)
        self.stale: int | None = None
        self.cache: dict[tuple, np.ndarray] = {}
        self.n_packed_checked = 0
        self.n_scores_checked = 0

    def ntok(self, b: int) -> int:
        return min(T, self.total - b * T)

    def resident(self) -> dict[int, int]:
        return {b: s for b, s in enumerate(self.eng.block_slots()) if s >= 0}

    def applied(self, sel: list[int]) -> None:
        self.valid = {b: self.ntok(b) for b in sel}
        self.stale = None

    def tail_grows(self) -> None:
        """Before append_tokens: a partial tail in the pool becomes the stale
        block; an earlier stale block leaves the pool (the engine marks one)."""
        nb = (self.total + T - 1) // T
        tail = nb - 1
        if nb and self.ntok(tail) < T and tail in self.valid:
            if self.stale is not None and self.stale != tail:
                self.valid.pop(self.stale, None)
            self.stale = tail

    def cut(self, total: int) -> None:
        """truncate_to(total): blocks past it gone, the cut one shortened."""
        self.total = total
        self.valid = {b: min(r, self.ntok(b)) for b, r in self.valid.items() if b * T < total}
        if self.stale is not None and self.stale * T >= total:
            self.stale = None

    def use_history(self, hist: int, k, v) -> None:
        self.hist = hist
        self.bits = (workloads.to_bits(torch, k), workloads.to_bits(torch, v))

    def want(self, layer: int, which: int, b: int, n: int) -> np.ndarray:
        key = (self.hist, layer, which, b, n)
        if key not in self.cache:
            rows = self.bits[which][layer, b].reshape(T, E)[:n]
            if self.theta is None:
                self.cache[key] = self.oracle.quantize_rows_f16(self.types[which], rows)
            else:
                # K: RoPE 256 at positions b*T.. then the width-256 rotation; V: width 64
                n_rot, width = (XF["n_rot"], 256) if which == 0 else (0, 64)
                self.cache[key] = expected_rows(self.oracle, self.types[which], rows, D, n_rot,
                                                self.theta if n_rot else None, b * T, width)
        return self.cache[key]

    def check_meank_scores(self, q, what: str, cache_q: bool = True, state=None) -> None:
        """The last preview's scores against the oracle's mean-K chain over the
        history as it is now: token-order query sums, token-order key sums of
        every block's rows (the tail's partial ones included), score_retrieval."""
        got = np.array(self.eng.scores(), dtype=np.float64)
        nb = self.eng.block_count()
        assert got.size == nb, (what, got.size, nb)
        if state is not None:   # (sums [L][HQ*D], counts [L]): a query state
            q_sum, q_count = state
        else:
            key = ("q", q.data_ptr())
            if not cache_q or key not in self.cache:
                q_sum = self.oracle.q_accumulate(q.float().cpu().numpy().reshape(L, q.shape[1], -1))
                if cache_q:   # only for the run's fixed query tensors: a freed pointer is reused
                    self.cache[key] = q_sum
            q_sum = self.cache[key] if cache_q else q_sum
            q_count = [q.shape[1]] * L
        sums = np.zeros((L, nb, E), np.float32)
        mt = np.zeros((L, nb), np.uint32)
        for b in range(nb):
            n = self.ntok(b)
            for layer in range(L):
                k2 = ("sum", self.hist, layer, b, n)
                if k2 not in self.cache:
                    self.cache[k2] = self.oracle.meank_sum_f16(self.bits[0][layer, b].reshape(T, E)[:n])
                sums[layer, b] = self.cache[k2]
                mt[layer, b] = n
        want = self.oracle.score_meank(q_sum, q_count, sums, mt, HQ, E // D, D)
        assert np.max(np.abs(got - want)) <= 1e-5, (what, float(np.max(np.abs(got - want))))
        self.n_scores_checked += 1

    def check(self, what: str, canonical_sel: list[int] | None = None) -> None:
        eng = self.eng
        assert eng.total_tokens() == self.total, what
        res = self.resident()
        assert set(res) == set(self.valid), (what, sorted(res), sorted(self.valid))
        slots = list(res.values())
        assert len(set(slots)) == len(slots) and all(0 <= s < eng.n_slots() for s in slots), (what, res)
        if canonical_sel is not None:
            assert [res[b] for b in canonical_sel] == list(range(len(canonical_sel))), (what, res)
        c = kv.Context(0)
        pools = []
        for layer in range(L):
            for which in (0, 1):
                rb = kv.row_size(self.types[which], E)
                n = eng.n_slots() * T * rb
                buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                c.d2d_batched([eng.pool_layer(layer)[which]], [buf.data_ptr()], [n])
                pools.append((buf, rb))
        c.sync()
        c.close()
        for i, (buf, rb) in enumerate(pools):
            layer, which = divmod(i, 2)
            pool = buf.cpu().numpy().reshape(eng.n_slots() * T, rb)
            for b, s in res.items():
                n = self.valid[b]
                got = pool[s * T: s * T + n]
                assert np.array_equal(got, self.want(layer, which, b, n)), (what, layer, "KV"[which], b, s, n)
        if self.store is not None:
            # packed rows the engine restores from: full blocks saved at eviction, each
            # [layer][T rows of K][T rows of V]
            rk, rv = (kv.row_size(t, E) for t in self.types)
            span = L * T * (rk + rv)
            host = self.store.numpy()
            for b in range(eng.block_count()):
                if not eng.packed_valid(b):
                    continue
                assert self.ntok(b) == T, (what, b)
                for layer in range(L):
                    at = b * span + layer * T * (rk + rv)
                    kr = host[at: at + T * rk].reshape(T, rk)
                    vr = host[at + T * rk: at + T * (rk + rv)].reshape(T, rv)
                    assert np.array_equal(kr, self.want(layer, 0, b, T)), (what, "packed K", b, layer)
                    assert np.array_equal(vr, self.want(layer, 1, b, T)), (what, "packed V", b, layer)
                self.n_packed_checked += 1


@pytest.mark.parametrize("case", CASES, ids=["canonical_q8", "lifo_q8_q4", "canonical_q5_q8",
                                             "pinned_packed_q8_q4", "rope_hadamard_q8_q4",
                                             "rope_hadamard_pinned_packed_q5_q8"])
def test_random_operation_sequences(oracle, case):
    run_sequence(oracle, case, meank=False)


def test_random_operation_sequences_meank_scorer(oracle):
    """The same operations with the reference's mean-K scorer: after every
    preview the scores are within 1e-5 of the oracle's over the history as it
    stands, so the key sums the engine keeps across appended, decoded and
    truncated rows are current."""
    run_sequence(oracle, MEANK_CASE, meank=True)


def test_random_operation_sequences_host_only_history(oracle):
    """The reference's deployment shape: every block only in pinned host
    memory (no history in HBM), a pinned packed store, the mean-K scorer over
    key sums the device reads from the pinned blocks."""
    run_sequence(oracle, (1, kv.TYPE_Q8_0, kv.TYPE_Q4_0, 107, True, False), meank=True, host_only=True)


def run_sequence(oracle, case, meank: bool, host_only: bool = False) -> None:
    canonical, tk, tv, seed, pinned, xf = case
    seed += SEED_OFFSET
    cap, budget, reserve = 40, 8, 6
    announce(f"{N_OPS} random operations, canonical={canonical}, types {kv.TYPE_NAMES[tk]}/"
             f"{kv.TYPE_NAMES[tv]}, seed {seed}, pinned host history and packed store: {pinned}, "
             f"row transform: {xf}, mean-K scorer: {meank}, host-only history: {host_only}")
    k, v, q = history(cap, seed=seed)
    k2, v2, _ = history(cap, seed=seed + 500)   # another history of the same shape
    hists = [(k, v), (k2, v2)]
    hb = store = None
    if pinned:
        hb = block_major_pinned(k, v, cap)
        span = L * T * (kv.row_size(tk, E) + kv.row_size(tv, E))
        store = torch.zeros(cap * span, dtype=torch.uint8, pin_memory=True)
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(q.shape[2], generator=g).tolist()
    queries = [q, (q.float() * -1.0).to(torch.bfloat16), q[:, :, perm].contiguous()]
    rng = np.random.default_rng(seed)
    counts = dict.fromkeys(OPS, 0)
    hits = {"unchanged_ok": 0, "failed_apply": 0, "decode_refused": 0, "stale_refused": 0, "spans": 0,
            "captures": 0, "window_previews": 0, "states_read": 0, "states_set": 0, "state_previews": 0,
            "caller_selections": 0, "swaps": 0}
    with make_engine(budget, reserve, tk, tv, canonical_layout=canonical, scorer=int(meank),
                     query_max_tokens=QWIN_CAP, query_last=QWIN_LAST, **(XF if xf else {})) as eng:
        if host_only:
            eng.set_host_history(hb.data_ptr(), cap)
            eng.append_tokens(20 * T + 37)
        else:
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, 20 * T + 37)
            if pinned:
                eng.set_host_history(hb.data_ptr(), cap)
        if pinned:
            eng.set_packed_host(store.data_ptr(), cap)
        ctx = kv.Context.borrow(eng.ctx_handle())
        m = Model(eng, oracle, k, v, (tk, tv), store, xf)
        m.check("start")
        last_q, last_mand = 0, []
        # the spans: none, a request span (query rows [qb, qe), qe <= 0 to the end) or turn
        # spans (query and mandatory row ranges); force_pos stays from the last request span
        spans = {"kind": None, "qb": -1, "qe": 0, "query": [], "mand": [], "force": -1}

        def derived() -> list[int]:
            """retrieval_mandatory as the history stands: the blocks overlapping
            the mandatory rows in block order, then the block holding force_pos."""
            if spans["kind"] == "turns":
                ranges = spans["mand"]
            elif spans["kind"] == "req":
                ranges = [(spans["qb"], spans["qe"] if spans["qe"] > 0 else m.total)]
            else:
                ranges = []
            out = [b for b in range(eng.block_count())
                   if any(b * T + m.ntok(b) > lo and b * T < hi for lo, hi in ranges)]
            if 0 <= spans["force"] < m.total:
                out.append(spans["force"] // T)
            return out

        window = []   # captured query rows, oldest first: [L][HQ][D] bf16 each
        # the query state: rows captured since the last reset, a state set by set_query
        # (sums, counts, rows captured before it) and the frozen flag
        qs = {"captured": 0, "imported": None, "base": 0, "frozen": False}

        def limit() -> int:
            return QWIN_CAP if spans["kind"] is not None else QWIN_LAST

        def expected_state():
            """What get_query returns: the newest window rows summed in token order, or a
            set state with the rows captured since added onto it; None with neither."""
            if qs["imported"] is None:
                n = min(len(window), limit())
                if n == 0:
                    return None
                rows = torch.stack(window[-n:], dim=1).float().numpy().reshape(L, n, -1)
                return oracle.q_accumulate(rows), [n] * L
            sums, counts = qs["imported"]
            n = min(qs["captured"] - qs["base"], limit(), len(window))
            if n == 0:
                return sums.copy(), list(counts)
            rows = torch.stack(window[-n:], dim=1).float().numpy().reshape(L, n, -1)
            return oracle.q_accumulate(rows, q_sum=sums), [c + n for c in counts]

        def contains(pos: int) -> bool:
            """query_contains; with no span every row is a query row."""
            if spans["kind"] == "turns":
                return any(lo <= pos < hi for lo, hi in spans["query"])
            if spans["kind"] == "req":
                return spans["qb"] <= pos and (spans["qe"] <= 0 or pos < spans["qe"])
            return True

        def ranges(k: int) -> list[tuple[int, int]]:
            out = []
            for _ in range(k):
                lo = int(rng.integers(0, m.total + 1))
                out.append((lo, lo + int(rng.integers(0, 3 * T))))
            return out

        def kept(sel_blocks: list[int], mand: list[int], what: str) -> None:
            need = {0} | set(mand) | set(derived())
            if len(need) <= budget:
                assert need <= set(sel_blocks), (what, sorted(need), sel_blocks)

        def mandatory() -> list[int]:
            nb = eng.block_count()
            n = int(rng.integers(0, 3))
            return sorted({int(x) for x in rng.integers(0, nb, n)})

        def grow(n: int) -> int:
            return int(min(n, cap * T - m.total))

        for step in range(N_OPS):
            op = OPS[int(rng.choice(len(OPS), p=WEIGHTS / WEIGHTS.sum()))]
            if xf and op == "decode":
                op = "append"   # a transformed pool's decoded cells are the model's to write
            qi = int(rng.integers(0, len(queries)))
            qq = queries[qi]
            what = f"step {step} {op}"
            counts[op] += 1
            if op == "retrieve":
                mand = mandatory()
                want = eng.preview(qq.data_ptr(), qq.shape[1], mandatory=mand).blocks
                if meank:
                    m.check_meank_scores(qq, what)
                st = eng.apply_retrieval(qq.data_ptr(), qq.shape[1], mandatory=mand)
                got = sorted(m.resident())
                assert got == want, (what, got, want, st)
                kept(got, mand, what)
                m.applied(want)
                last_q, last_mand = qi, mand
                m.check(what, want if canonical else None)
            elif op == "preview_apply":
                mand = mandatory()
                sel = eng.preview(qq.data_ptr(), qq.shape[1], mandatory=mand)
                if meank:
                    m.check_meank_scores(qq, what)
                kept(sel.blocks, mand, what)
                assert eng.selection_fits(sel, m.total, 0) == (set(derived()) <= set(sel.blocks)), what
                before = dict(m.valid)
                need = sum(1 for b in sel.blocks if before.get(b, -1) < m.ntok(b))
                st = eng.apply(sel)
                # a decoded tail that had no slot is staged once more by the engine
                assert need <= st["n_staged"] <= need + 1, (what, need, st)
                m.applied(sel.blocks)
                last_q, last_mand = qi, mand
                m.check(what, sel.blocks if canonical else None)
            elif op == "stale":
                sel = eng.preview(qq.data_ptr(), qq.shape[1])
                n = grow(int(rng.integers(1, 100)))
                if n > 0:
                    m.tail_grows()
                    eng.append_tokens(n)
                    m.total += n
                else:
                    cut = m.total - int(rng.integers(1, 60))
                    eng.truncate_to(cut)
                    m.cut(cut)
                with pytest.raises(kv.StaleSelection):
                    eng.apply(sel)
                hits["stale_refused"] += 1
                m.check(what)
            elif op == "append":
                n = grow(int(rng.integers(1, 300)))
                if n:
                    m.tail_grows()
                    eng.append_tokens(n)
                    m.total += n
                m.check(what)
            elif op == "decode":
                n = grow(int(rng.integers(1, 200)))
                if n == 0:
                    continue
                t0 = m.total
                tail = (t0 + T - 1) // T - 1
                gets_slot = t0 % T != 0 and tail not in m.valid   # a partial tail taking a slot
                try:
                    decode_rows(eng, *hists[m.hist], t0, t0 + n)
                except kv.KvMemError as ex:
                    # no free slot, or another grown tail waits: nothing changed, and the
                    # caller appends the rows to the history instead
                    assert ex.code in (kv.ERR_NOMEM, kv.ERR_UNSUPPORTED), (what, str(ex))
                    assert eng.total_tokens() == t0, what
                    m.check(what + " refused")
                    m.tail_grows()
                    eng.append_tokens(n)
                    m.total += n
                    hits["decode_refused"] += 1
                else:
                    m.total += n
                    for b in range(t0 // T, (t0 + n + T - 1) // T):
                        m.valid[b] = m.ntok(b)
                    if gets_slot:
                        m.stale = tail   # its cells were written whole here, yet it is staged again
                m.check(what)
            elif op == "truncate":
                if m.total <= 2 * T:
                    continue
                cut = int(rng.integers(max(T, m.total - 3 * T), m.total))
                eng.truncate_to(cut)
                m.cut(cut)
                m.check(what)
            elif op == "fail":
                sel = eng.preview(qq.data_ptr(), qq.shape[1])
                before = dict(m.valid)
                device = bool(rng.integers(0, 2))      # through the device plan, or the host plan
                ctx.debug_fail_after(ALL_KINDS, int(rng.integers(1, 4)))
                try:
                    if device:
                        eng.apply_retrieval(qq.data_ptr(), qq.shape[1])
                    else:
                        eng.apply(sel)
                    failed = False
                except kv.KvMemError as ex:
                    assert "injected failure" in str(ex), (what, str(ex))
                    failed = True
                ctx.debug_fail_after(0, 0)
                if failed:
                    hits["failed_apply"] += 1
                    res = m.resident()
                    assert set(res) <= set(before), (what, sorted(res), sorted(before))
                    m.valid = {b: before[b] for b in res}
                    if m.stale not in res:   # the mark goes with its block's slot
                        m.stale = None
                    m.check(what + " (failed)")
                else:
                    assert sorted(m.resident()) == sel.blocks, what
                    m.applied(sel.blocks)
                    last_q, last_mand = qi, []
                    m.check(what, sel.blocks if canonical else None)
            elif op == "unchanged":
                # the check runs against the pool's canonical view, as the reference's
                # commit_unchanged does (llama-memory-kvmem.cpp:3086-3096)
                view = eng.attention_view(canonical=bool(canonical))
                canon = eng.attention_view(canonical=True)
                qq = queries[last_q]          # the last apply's query and mandatory blocks
                sel = eng.preview(qq.data_ptr(), qq.shape[1], mandatory=last_mand)
                ok = eng.commit_unchanged(view, sel)
                assert ok == (view.valid and canon.valid and sel.blocks == canon.blocks), (what, view, sel.blocks)
                hits["unchanged_ok"] += int(ok)
                m.check(what)
            elif op == "span":
                r = int(rng.integers(0, 4))
                if r == 0 or m.total == 0:
                    eng.set_request_span(-1)
                    spans.update(kind=None, force=-1)
                elif r == 1:   # turn spans: query and mandatory row ranges
                    q_r, m_r = ranges(int(rng.integers(1, 3))), ranges(int(rng.integers(0, 3)))
                    if rng.integers(0, 6) == 0:   # a reversed range is refused, nothing changes
                        with pytest.raises(kv.KvMemError):
                            eng.set_turn_spans(query=q_r + [(5, 2)], mandatory=m_r)
                    else:
                        eng.set_turn_spans(query=q_r, mandatory=m_r)
                        spans.update(kind="turns", query=q_r, mand=m_r)
                else:
                    qb = int(rng.integers(0, m.total))
                    qe = 0 if rng.integers(0, 2) == 0 else int(rng.integers(qb + 1, m.total + 1))
                    fp = -1 if rng.integers(0, 2) == 0 else int(rng.integers(0, m.total))
                    eng.set_request_span(qb, qe, fp)
                    spans.update(kind="req", qb=qb, qe=qe, force=fp)
                hits["spans"] += int(spans["kind"] is not None)
                m.check(what)
            elif op == "capture":
                if rng.integers(0, 8) == 0:
                    eng.reset_query()   # a frozen query stays frozen
                    window = []
                    qs.update(captured=0, imported=None, base=0)
                else:
                    n = int(rng.integers(1, 40))
                    pos0 = int(rng.integers(0, m.total + 1))
                    positions = list(range(pos0, pos0 + n))
                    x = (torch.randn((L, n, HQ, D), generator=g) * 2).to(torch.bfloat16)
                    for layer in range(L):
                        xd = x[layer].contiguous().cuda()
                        torch.cuda.synchronize()
                        eng.capture_q(layer, xd.data_ptr(), kv.TYPE_BF16, 2, D * 2, HQ * D * 2, positions)
                        ctx.sync()   # the view is freed after this
                    if not qs["frozen"]:   # a frozen query keeps no rows
                        kept_rows = [x[:, i] for i, p in enumerate(positions) if contains(p)]
                        window = (window + kept_rows)[-QWIN_CAP:]
                        qs["captured"] += len(kept_rows)
                hits["captures"] += 1
                m.check(what)
            elif op == "wretrieve" and qs["imported"] is not None and meank:
                # a set state (with rows captured since): the oracle's scores over it
                sel = eng.preview_window()
                m.check_meank_scores(None, what, state=expected_state())
                kept(sel.blocks, [], what)
                eng.apply(sel)
                m.applied(sel.blocks)
                hits["state_previews"] += 1
                m.check(what, sel.blocks if canonical else None)
            elif op == "wretrieve":
                n = min(len(window), limit())
                if n == 0:   # an empty window is refused
                    with pytest.raises(kv.KvMemError):
                        eng.query_rows()
                    continue
                assert eng.query_rows() == n, (what, eng.query_rows(), n)
                sel = eng.preview_window()
                got = np.array(eng.scores(), dtype=np.float64)
                qe = torch.stack(window[-n:], dim=1).contiguous().cuda()   # [L][n][HQ][D]
                torch.cuda.synchronize()
                sel2 = eng.preview(qe.data_ptr(), n)
                assert sel.blocks == sel2.blocks, (what, sel.blocks, sel2.blocks)
                assert np.array_equal(got, np.array(eng.scores(), dtype=np.float64)), what
                if meank:
                    m.check_meank_scores(qe, what, cache_q=False)
                kept(sel.blocks, [], what)
                eng.apply(sel2)
                m.applied(sel2.blocks)
                hits["window_previews"] += 1
                m.check(what, sel2.blocks if canonical else None)
            elif op == "swap":
                if pinned or host_only:   # their stage-in reads the pinned copy of the first history
                    continue
                # other buffers: a new history, so residency, key sums and saved rows go
                cur = 1 - m.hist
                kk, vv = hists[cur]
                eng.set_device_history(kk.data_ptr(), vv.data_ptr(), cap, m.total)
                m.use_history(cur, kk, vv)
                m.valid = {}
                m.stale = None
                hits["swaps"] += 1
                m.check(what)
            elif op == "apply_ids":
                # a caller's own selection: any order, repeats, ids past the history, at times
                # more blocks than slots (refused, nothing changes), at times none
                nb = eng.block_count()
                ids = [int(x) for x in rng.integers(0, nb + 3, int(rng.integers(0, eng.n_slots() + 4)))]
                uniq = sorted({i for i in ids if i < nb})
                before = dict(m.valid)
                if len(uniq) > eng.n_slots():
                    with pytest.raises(kv.KvMemError) as ex:
                        eng.apply(host.Selection(eng.epoch(), m.total, ids))
                    assert ex.value.code == kv.ERR_INVALID, what
                    assert m.valid == before
                    m.check(what + " (refused)")
                else:
                    eng.apply(host.Selection(eng.epoch(), m.total, ids))
                    assert sorted(m.resident()) == uniq, (what, sorted(m.resident()), uniq)
                    m.applied(uniq)
                    m.check(what, uniq if canonical else None)
                hits["caller_selections"] += 1
            elif op == "qstate":
                r = int(rng.integers(0, 3))
                want = expected_state()
                if r == 0:   # get_query
                    if want is None:
                        with pytest.raises(kv.KvMemError):
                            eng.get_query()
                    else:
                        got_sums, got_counts = eng.get_query()
                        assert got_counts == want[1], (what, got_counts, want[1])
                        assert np.array_equal(got_sums.view(np.uint32), want[0].view(np.uint32)), what
                        hits["states_read"] += 1
                elif r == 1:   # set_query: a state read back, or a random finite one
                    if want is not None and rng.integers(0, 2) == 0:
                        new_state = (want[0], want[1])
                    else:
                        c = int(rng.integers(1, 50))
                        new_state = ((rng.standard_normal((L, HQ * D)) * c).astype(np.float32), [c] * L)
                    if not meank:
                        with pytest.raises(kv.KvMemError) as ex:
                            eng.set_query(*new_state)
                        assert ex.value.code == kv.ERR_UNSUPPORTED
                    else:
                        eng.set_query(*new_state)
                        qs.update(imported=(np.array(new_state[0], np.float32), list(new_state[1])),
                                  base=qs["captured"], frozen=True)
                        hits["states_set"] += 1
                else:   # freeze or unfreeze
                    frozen = bool(rng.integers(0, 2))
                    eng.freeze_query(frozen)
                    qs["frozen"] = frozen
                m.check(what)
            assert eng.retrieval_mandatory() == derived(), (what, spans, eng.retrieval_mandatory())
    announce(f"operations {counts}; {hits}; packed blocks checked {m.n_packed_checked}; "
             f"mean-K score sets checked {m.n_scores_checked}")
    assert hits["stale_refused"] >= 1 and hits["failed_apply"] >= 1, hits
    if canonical:
        assert hits["unchanged_ok"] >= 1, hits
    if pinned:
        assert m.n_packed_checked >= 1
    if meank:
        assert m.n_scores_checked >= 10
    del hb, store
