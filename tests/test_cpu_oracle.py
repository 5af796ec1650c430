"""The CPU oracle pinned against things other than itself (no GPU).

Quantizers (ggml quantize_row_q8_0/q4_0/q5_0_ref restated in
oracle/kvmem_oracle_quant.c):
  - golden bytes from an independent numpy restatement (tests/golden);
  - closed forms: all-zero groups, single non-zero element, half-way
    rounding, sign ties (first index wins), every q4 code once;
  - dequantisation error bounds (|x - deq| <= d/2, plus the clamp step);
  - planted mistakes in the numpy restatement (round-half-even for
    roundf, the last instead of the first element of largest magnitude)
    are rejected by the golden bytes.
Half precision: f16 -> f32 over all 65536 codes and f32 -> f16 on edge and
random values against numpy's IEEE conversion.
Per-token max scorer (fp64): numpy brute force on tiny shapes, permutation
and scaling invariants.  Its fp32 twin (the full-size tests' checker): the
fp64 scorer and the brute force within 1e-5, over block sub-ranges, thread
counts, head_dim 128 / 256, GQA groups and partial last blocks; GQA-map,
block-offset, layer-stride and partial-tail slips planted through its inputs
fail the same comparison.
Top-k: the reference library's selections (tests/golden/select_sequences
.json, ties to the higher id) and a sort-based brute force (both tie rules).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"

Q8, Q4, Q5, F16 = 8, 2, 6, 1


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN / "quant_vectors.npz")


@pytest.mark.parametrize("name,type_", [("q8_0", Q8), ("q4_0", Q4), ("q5_0", Q5)])
def test_quantizers_match_numpy_restatement(oracle, gold, name, type_):
    got = oracle.quantize_rows_f16(type_, gold["rows"])
    want = gold[name]
    assert np.array_equal(got, want), np.flatnonzero(got.ravel() != want.ravel())[:8]


def _golden_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_golden_rejects_planted_mistakes(gold, monkeypatch):
    """The golden vectors discriminate plausible mistakes: round-half-even
    instead of roundf in q8_0, and the LAST element of largest magnitude
    as the q4_0 / q5_0 scale source."""
    mg = _golden_module()
    xs = gold["rows"].view(np.float16).astype(np.float32)
    monkeypatch.setattr(mg, "_roundf", lambda v: np.rint(v.astype(np.float64)))
    q8 = np.frombuffer(b"".join(mg.np_q8_0(r) for r in xs), np.uint8).reshape(gold["q8_0"].shape)
    assert not np.array_equal(q8, gold["q8_0"])

    def last_absmax(g):
        a = np.abs(g)
        if a.max() == 0:
            return np.float32(0.0)
        return np.float32(g[len(g) - 1 - int(np.argmax(a[::-1]))])

    monkeypatch.setattr(mg, "_signed_absmax", last_absmax)
    for name, fn in (("q4_0", mg.np_q4_0), ("q5_0", mg.np_q5_0)):
        q = np.frombuffer(b"".join(fn(r) for r in xs), np.uint8).reshape(gold[name].shape)
        assert not np.array_equal(q, gold[name]), name


def groups_f16(*groups) -> np.ndarray:
    return np.asarray(groups, dtype=np.float32).astype(np.float16).view(np.uint16).reshape(1, -1)


def test_all_zero_group_closed_form(oracle):
    z = groups_f16(np.zeros(32))
    q8 = oracle.quantize_rows_f16(Q8, z)[0]
    assert q8[:2].tolist() == [0, 0] and not q8[2:].any()
    q4 = oracle.quantize_rows_f16(Q4, z)[0]
    assert q4[:2].tolist() == [0x00, 0x80]            # d = 0/-8 = -0.0
    assert (q4[2:] == 0x88).all()
    q5 = oracle.quantize_rows_f16(Q5, z)[0]
    assert q5[:2].tolist() == [0x00, 0x80]
    assert q5[2:6].tolist() == [0xFF] * 4 and not q5[6:].any()


def test_single_nonzero_q8_is_127(oracle):
    for v in (3.0, -3.0, 1e-3, 60000.0):
        g = np.zeros(32)
        g[11] = v
        q = oracle.quantize_rows_f16(Q8, groups_f16(g))[0]
        assert np.int8(q[2 + 11]) == (127 if v > 0 else -127)
        assert not np.delete(q[2:], 11).any()


def test_q8_half_way_rounds_away_from_zero(oracle):
    g = np.zeros(32)
    g[0] = 127.0                                      # d = 1, id = 1
    g[1:7] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5]
    q = oracle.quantize_rows_f16(Q8, groups_f16(g))[0].view(np.int8)
    assert q[2 + 1: 2 + 7].tolist() == [3, -3, 1, -1, 2, -2]


def test_q4_sign_tie_first_index_wins(oracle):
    a = np.zeros(32); a[2] = -3.0; a[5] = 3.0
    b = np.zeros(32); b[2] = 3.0; b[5] = -3.0
    qa = oracle.quantize_rows_f16(Q4, groups_f16(a))[0]
    qb = oracle.quantize_rows_f16(Q4, groups_f16(b))[0]
    da = np.frombuffer(qa[:2].tobytes(), np.float16)[0]
    db = np.frombuffer(qb[:2].tobytes(), np.float16)[0]
    assert da == np.float16(3.0 / 8) and db == np.float16(-3.0 / 8)


def test_q4_every_code(oracle):
    """x = -8..7 scaled by d = 1 (vmax = -8 first): codes 0..15 in order."""
    g = np.concatenate([np.arange(-8, 8), np.arange(-8, 8)]).astype(np.float32)
    q = oracle.quantize_rows_f16(Q4, groups_f16(g))[0]
    lo = q[2:] & 0xF
    hi = q[2:] >> 4
    assert lo.tolist() == list(range(16)) and hi.tolist() == list(range(16))


@pytest.mark.parametrize("type_,levels", [(Q8, 127), (Q4, 8), (Q5, 16)])
def test_dequant_error_bound(oracle, type_, levels):
    rng = np.random.default_rng(3)
    x = rng.standard_t(4, (64, 256)).astype(np.float16)
    rows = x.view(np.uint16)
    q = oracle.quantize_rows_f16(type_, rows)
    for r in range(rows.shape[0]):
        deq = oracle.dequantize_row(type_, q[r], 256)
        xs = x[r].astype(np.float32)
        for gi in range(8):
            g = xs[gi * 32:(gi + 1) * 32]
            gb = {Q8: 34, Q4: 18, Q5: 22}[type_]
            d = abs(float(np.frombuffer(q[r, gi * gb: gi * gb + 2].tobytes(), np.float16)[0]))
            err = np.abs(g - deq[gi * 32:(gi + 1) * 32])
            # half a step, plus the f16 rounding of d over `levels` steps and
            # the top clamp of the 4/5-bit codes (one step)
            bound = 0.5 * d + levels * d * 2.0 ** -11 + (d if type_ != Q8 else 0.0) + 1e-7
            assert err.max() <= bound * 1.0001, (r, gi, err.max(), d)


def test_f16_to_f32_exhaustive(oracle):
    import ctypes as C
    lib = oracle.lib()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    f = lib.ko_f16_to_f32
    got = np.array([f(int(v)) for v in h], dtype=np.float32)
    w = want
    same = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
    assert same.all()
    del C


def test_f32_to_f16_rne(oracle):
    rng = np.random.default_rng(5)
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e-8, 2.0 ** -25,
                     2.0 ** -25 * 1.0000001, 2.0 ** -24, 3 * 2.0 ** -26, 6.1e-5, 6.097555e-5,
                     np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    xs = np.concatenate([edge, (rng.standard_normal(4000) * 10.0 ** rng.integers(-8, 5, 4000)).astype(np.float32)])
    got = oracle.f32_to_f16(xs)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ scorer
def brute_scores(q, kbits, last_T=0):
    k = kbits.view(np.float16).astype(np.float64)
    L, Tq, Hq, D = q.shape
    _, B, T, Hkv, _ = k.shape
    g = Hq // Hkv
    out = np.zeros((L, B))
    for l in range(L):
        for b in range(B):
            nt = last_T if (b == B - 1 and last_T) else T
            best = -np.inf
            for h in range(Hkv):
                qq = q[l, :, h * g:(h + 1) * g].reshape(-1, D).astype(np.float64)
                s = qq @ k[l, b, :nt, h].T
                best = max(best, s.max())
            out[l, b] = best / np.sqrt(D)
    return out


def test_scorer_vs_numpy_brute_force(oracle):
    rng = np.random.default_rng(8)
    L, Tq, Hq, Hkv, D, B, T = 2, 5, 6, 2, 64, 4, 16
    q = rng.standard_normal((L, Tq, Hq, D)).astype(np.float32)
    k = rng.standard_normal((L, B, T, Hkv, D)).astype(np.float16).view(np.uint16)
    for last in (0, 7):
        got = oracle.score_pertoken_max(q, k, last)
        assert np.allclose(got, brute_scores(q, k, last), rtol=1e-12, atol=1e-12)


def test_scorer_gqa_map_is_contiguous_groups(oracle):
    """Query head hq reads KV head hq // g: moving the only large query to
    head g (first head of group 1) must change which KV head scores it."""
    L, Tq, Hq, Hkv, D, B, T = 1, 1, 4, 2, 32, 1, 4
    k = np.zeros((L, B, T, Hkv, D), np.float32)
    k[0, 0, :, 0, 0] = 1.0                     # KV head 0 answers direction e0
    k[0, 0, :, 1, 1] = 1.0                     # KV head 1 answers direction e1
    kb = k.astype(np.float16).view(np.uint16)
    q = np.zeros((L, Tq, Hq, D), np.float32)
    q[0, 0, 1, 0] = 4.0                        # head 1 -> KV head 0 (g = 2)
    assert oracle.score_pertoken_max(q, kb)[0, 0] == pytest.approx(4.0 / np.sqrt(D))
    q[:] = 0
    q[0, 0, 2, 0] = 4.0                        # head 2 -> KV head 1: sees nothing on e0
    assert oracle.score_pertoken_max(q, kb)[0, 0] == 0.0


def test_scorer_invariants(oracle):
    rng = np.random.default_rng(9)
    L, Tq, Hq, Hkv, D, B, T = 1, 3, 4, 2, 32, 3, 8
    q = rng.standard_normal((L, Tq, Hq, D)).astype(np.float32)
    k = rng.standard_normal((L, B, T, Hkv, D)).astype(np.float16).view(np.uint16)
    base = oracle.score_pertoken_max(q, k)
    perm = rng.permutation(T)
    assert np.array_equal(oracle.score_pertoken_max(q, k[:, :, perm].copy()), base)
    assert np.allclose(oracle.score_pertoken_max(q * 2, k), 2 * base, rtol=1e-12)
    swapped = q[:, :, [1, 0, 3, 2]].copy()        # heads swapped inside each group
    assert np.allclose(oracle.score_pertoken_max(swapped, k), base, rtol=1e-12)


# ------------------------------------------------ fp32 scorer (full-size checker)
def _f32_inputs(seed, L, Tq, Hq, Hkv, D, B, T):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((L, Tq, Hq, D)).astype(np.float32)
    k = (rng.standard_normal((L, B, T, Hkv, D)) + rng.normal(0, 0.3, (L, B, 1, 1, D)))
    return q, k.astype(np.float16).view(np.uint16)


def _f32_close(got, want, rtol=1e-5):
    """fp32 accumulation over D <= 256 products: 1e-5 of the score's scale."""
    scale = np.maximum(np.abs(want), 1e-3)
    return bool(np.all(np.abs(got.astype(np.float64) - want) <= rtol * scale))


@pytest.mark.parametrize("D,Hq,Hkv,last", [(256, 24, 4, 0), (256, 24, 4, 37), (128, 8, 2, 0),
                                          (128, 6, 6, 91)])
def test_scorer_f32_vs_fp64_and_brute_force(oracle, D, Hq, Hkv, last):
    """The fp32 scorer the full-size tests check the device against equals
    the fp64 scorer and a numpy brute force to fp32 accumulation error, on
    128-token blocks with a partial last block."""
    L, Tq, B, T = 2, 4, 5, 128
    q, k = _f32_inputs(21 + D + last, L, Tq, Hq, Hkv, D, B, T)
    got = oracle.score_pertoken_max_f32(q, k, 0, B, last_block_tokens=last)
    assert not np.isnan(got).any()
    assert _f32_close(got, oracle.score_pertoken_max(q, k, last))
    assert _f32_close(got, brute_scores(q, k, last))


def test_scorer_f32_block_range_and_threads(oracle):
    """Columns outside [b_begin, b_end) stay untouched; inside they equal the
    full-range call bit for bit, for 1, 3 and all threads (one block is one
    thread's work, so the sums never depend on the split)."""
    L, Tq, Hq, Hkv, D, B, T = 3, 3, 24, 4, 256, 7, 128
    q, k = _f32_inputs(5, L, Tq, Hq, Hkv, D, B, T)
    full = oracle.score_pertoken_max_f32(q, k, 0, B, n_threads=1, last_block_tokens=50)
    for threads in (1, 3, 0):
        assert np.array_equal(oracle.score_pertoken_max_f32(q, k, 0, B, threads, 50), full)
        part = oracle.score_pertoken_max_f32(q, k, 2, 6, threads, 50)
        assert np.isnan(part[:, :2]).all() and np.isnan(part[:, 6:]).all()
        assert np.array_equal(part[:, 2:6], full[:, 2:6])
        tail = oracle.score_pertoken_max_f32(q, k, 6, 7, threads, 50)
        assert np.array_equal(tail[:, 6], full[:, 6])
    assert np.isnan(oracle.score_pertoken_max_f32(q, k, 3, 3)).all()
    with pytest.raises(ValueError):
        oracle.score_pertoken_max_f32(q, k, 4, 8)


def test_scorer_f32_checks_reject_planted_slips(oracle):
    """The comparison the fp32 scorer passes above fails for the slips a
    rewrite of it could make.  Each slip is planted by feeding the correct
    scorer the inputs that make it compute the wrong thing:
      - GQA map hq -> hq % Hkv instead of hq // g;
      - keys read one block further on (a block-offset slip);
      - the layer stride off by one block (layer l reads layer l's keys
        starting one block early);
      - the partial last block scored over all T rows."""
    L, Tq, Hq, Hkv, D, B, T, last = 2, 4, 24, 4, 256, 5, 128, 40
    g = Hq // Hkv
    q, k = _f32_inputs(77, L, Tq, Hq, Hkv, D, B, T)
    kf = k.view(np.float16).copy()
    kf[:, B - 1, last:] = 8.0          # rows past the tail: large, never to be scored
    k = kf.view(np.uint16)
    want = oracle.score_pertoken_max(q, k, last)
    assert _f32_close(oracle.score_pertoken_max_f32(q, k, 0, B, last_block_tokens=last), want)

    perm = [gi * Hkv + h for h in range(Hkv) for gi in range(g)]
    slips = {
        "gqa": (q[:, :, perm].copy(), k, last),
        "block_offset": (q, np.roll(k, -1, axis=1).copy(), last),
        "layer_stride": (q, np.roll(k.reshape(L * B, T, Hkv, D), 1, axis=0).reshape(k.shape).copy(), last),
        "partial_tail": (q, k, 0),
    }
    for name, (qq, kk, lt) in slips.items():
        got = oracle.score_pertoken_max_f32(qq, kk, 0, B, last_block_tokens=lt)
        assert not _f32_close(got, want), name


def test_combine_layers_modes(oracle):
    ls = np.array([[1.0, -2.0], [3.0, 4.0], [-5.0, 0.5]])
    assert np.allclose(oracle.combine_layers(ls, 0), ls.mean(axis=0))
    assert np.allclose(oracle.combine_layers(ls, 1), ls.max(axis=0))
    assert np.allclose(oracle.combine_layers(ls, 2), ls.sum(axis=0))


# ------------------------------------------------------------------- top-k
@pytest.fixture(scope="module")
def sequences():
    return json.loads((GOLDEN / "select_sequences.json").read_text())["scenarios"]


def test_pick_topk_matches_reference_library(oracle, sequences):
    n_checked = 0
    for sc in sequences:
        for st in sc["steps"]:
            got = oracle.pick_topk(st["scores"], sc["budget_blocks"], sink=sc["sink"],
                                   recent=sc["recent"], mandatory=st["mandatory"],
                                   tie_lower_index=False)
            assert got == st["selection"], sc
            n_checked += 1
    assert n_checked >= 100


@pytest.mark.parametrize("tie_lower", [True, False])
def test_pick_topk_vs_sort_brute_force(oracle, tie_lower):
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(1, 80))
        budget = int(rng.integers(1, 40))
        s = rng.integers(-3, 4, n).astype(np.float64)
        got = oracle.pick_topk(s, budget, sink=1, tie_lower_index=tie_lower)
        if n <= budget:
            assert got == list(range(n))
            continue
        rest = list(range(1, n))
        key = (lambda i: (-s[i], i)) if tie_lower else (lambda i: (-s[i], -i))
        want = sorted([0] + sorted(rest, key=key)[: budget - 1])
        assert got == want


def test_q8_rounding_shortcut_exhaustive(oracle):
    """The kernel rounds q8_0 codes as trunc(s + copysign(0.49999997, s));
    over every float in [0, 128.5) (|x*id| <= 127 * (1 + 2^-22)) that equals
    roundf, and both are odd functions, so the codes are ggml's."""
    assert oracle.lib().ko_round_trick_mismatches(0.0, 128.5) == 0
    # the check itself sees a wrong constant: 0.5 rounds 0.49999997 up
    assert oracle.lib().ko_round_trick_mismatches(0.0, 1.0) == 0
    s = np.float32(0.49999997)
    assert np.trunc(np.float32(s + np.float32(0.5))) != np.round(s)


def test_q8_scale_division_shortcut_exhaustive(oracle):
    """q8_0's d = amax / 127 is computed as a * RN(1/127) plus one exact FMA
    correction; over every non-negative float (zero, subnormals, normals)
    that equals the IEEE quotient.  The reciprocal shortcut depends on the
    device's rcp and is checked on the GPU (test_gpu_stagein)."""
    assert oracle.lib().ko_div127_mismatches(0x00000000, 0x7F800000) == 0


# ------------------------------------------------ q5_0 byte layout, literal
from q5_literals import ggml_q5_0_decode_codes, q5_literal_failures  # noqa: E402


def test_q5_0_literal_bytes(oracle):
    assert q5_literal_failures(lambda r: oracle.quantize_rows_f16(Q5, r)) == []


def test_q5_0_literal_checks_reject_planted_layouts(oracle):
    """Plausible q5_0 layout mistakes, planted in the oracle's output, fail
    the literal checks: qh stored big-endian, element j's bit 4 stored at
    qh bit j + 16 (halves swapped), and the nibbles of qs swapped."""
    def planted(mutate):
        return lambda r: np.stack([mutate(bytearray(b.tobytes())) for b in
                                   oracle.quantize_rows_f16(Q5, r)])

    def qh_big_endian(b):
        b[2:6] = b[2:6][::-1]
        return np.frombuffer(bytes(b), np.uint8)

    def qh_halves_swapped(b):
        qh = int.from_bytes(b[2:6], "little")
        b[2:6] = (((qh & 0xFFFF) << 16) | (qh >> 16)).to_bytes(4, "little")
        return np.frombuffer(bytes(b), np.uint8)

    def qs_nibbles_swapped(b):
        for j in range(16):
            b[6 + j] = ((b[6 + j] & 15) << 4) | (b[6 + j] >> 4)
        return np.frombuffer(bytes(b), np.uint8)

    for mutate in (qh_big_endian, qh_halves_swapped, qs_nibbles_swapped):
        assert q5_literal_failures(planted(mutate)), mutate.__name__


def test_q5_0_dequantizer_statement_round_trips_random_codes(oracle):
    """Random groups of exact codes (d = 1 set by a -16 at a random first
    position) round-trip through the published dequantizer bit for bit."""
    rng = np.random.default_rng(21)
    for _ in range(200):
        pos = int(rng.integers(0, 32))
        codes = rng.integers(-15, 16, 32)        # -15..15, so -16 at pos is the first max
        codes[pos] = -16
        g = codes.astype(np.float32)
        blk = bytes(oracle.quantize_rows_f16(Q5, groups_f16(g))[0].tobytes())
        assert blk[:2] == bytes([0x00, 0x3C])
        assert ggml_q5_0_decode_codes(blk) == codes.tolist()
