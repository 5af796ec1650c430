"""The oracle's mean-K producer and mean-K cosine scorer (the reference's
retrieval scorer), pinned without the GPU.

  - mean-K: bit-exact against the reference RawKvStore's own output
    (tests/golden/meank_vectors.npz, and live through oracle/_ref when it
    is built), including a partial last block and large-magnitude channels;
  - scorer: an independent float64 numpy restatement (1e-6), closed forms
    (parallel -> 1, antiparallel -> -1, orthogonal -> 0), invariance to the
    query-sum scale and to head order inside a GQA group, layer skipping
    and blocks without keys.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT

GOLDEN = Path(__file__).resolve().parent / "golden"
REF = ROOT / "oracle" / "_ref" / "libkvmem_ref.so"


def block_means(oracle, rows: np.ndarray, bt: int) -> np.ndarray:
    n = rows.shape[0]
    out = []
    for b in range((n + bt - 1) // bt):
        seg = rows[b * bt:min(n, (b + 1) * bt)]
        out.append(oracle.mean_k(oracle.meank_sum_f16(seg), seg.shape[0]))
    return np.stack(out)


def test_mean_k_matches_reference_golden(oracle):
    g = np.load(GOLDEN / "meank_vectors.npz")
    got = block_means(oracle, g["rows"], int(g["block_tokens"]))
    assert np.array_equal(got.view(np.uint32), g["means"].view(np.uint32))


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (needs the reference tree)")
def test_mean_k_matches_reference_live(oracle):
    ref = C.CDLL(str(REF))
    ref.kref_mean_k_f16.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                                    C.c_void_p]
    rng = np.random.default_rng(4)
    for _ in range(30):
        E = int(rng.choice([64, 512, 1024]))
        bt = int(rng.choice([16, 128]))
        n = int(rng.integers(1, 3 * bt))
        rows = (rng.standard_normal((n, E)) * rng.choice([1.0, 300.0, 2e3])).astype(np.float16)
        rows = rows.view(np.uint16)
        mine = block_means(oracle, rows, bt)
        for b in range(mine.shape[0]):
            want = np.zeros(E, np.float32)
            ref.kref_mean_k_f16(E, bt, rows.ctypes.data, n, b, want.ctypes.data)
            assert np.array_equal(mine[b].view(np.uint32), want.view(np.uint32))


def numpy_score(q_sum, q_count, k_sum, mean_tokens, Hq, Hkv, D):
    L, B = mean_tokens.shape
    g = Hq // Hkv
    out = np.zeros(B)
    for b in range(B):
        if not mean_tokens[:, b].any():
            continue
        acc, nlay = 0.0, 0
        for l in range(L):
            if q_count[l] == 0:
                continue
            mt = mean_tokens[l, b]
            mk = k_sum[l, b].astype(np.float64) / mt if mt else np.zeros(Hkv * D)
            layer = 0.0
            for h in range(Hkv):
                qh = q_sum[l].reshape(Hq, D)[h * g:(h + 1) * g].astype(np.float64).sum(0) / (q_count[l] * g)
                kh = mk[h * D:(h + 1) * D]
                layer += qh @ kh / (np.linalg.norm(qh) * np.linalg.norm(kh) + 1e-6)
            acc += layer / Hkv
            nlay += 1
        out[b] = acc / nlay
    return out


def test_score_meank_vs_numpy(oracle):
    rng = np.random.default_rng(6)
    L, B, Hq, Hkv, D = 3, 9, 8, 2, 64
    q_sum = rng.standard_normal((L, Hq * D)).astype(np.float32) * 5
    q_count = np.array([4, 0, 7], np.uint32)                     # layer 1 not scored
    k_sum = rng.standard_normal((L, B, Hkv * D)).astype(np.float32) * 40
    mt = rng.integers(1, 129, (L, B)).astype(np.uint32)
    mt[:, 4] = 0                                                  # block without keys
    mt[2, 6] = 0                                                  # one layer without keys
    got = oracle.score_meank(q_sum, q_count, k_sum, mt, Hq, Hkv, D)
    want = numpy_score(q_sum, q_count, k_sum, mt, Hq, Hkv, D)
    assert got[4] == 0.0
    assert np.allclose(got, want, rtol=0, atol=1e-6)


def test_score_meank_closed_forms(oracle):
    L, B, Hq, Hkv, D = 1, 3, 4, 1, 32
    rng = np.random.default_rng(1)
    u = rng.standard_normal(D).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    w -= (w @ u) / (u @ u) * u                                    # w orthogonal to u
    q_sum = np.tile(u, Hq).reshape(L, Hq * D) * 3.0              # every head of the group = u
    k_sum = np.stack([u * 10, -u * 10, w * 10]).reshape(L, B, D).astype(np.float32)
    mt = np.full((L, B), 10, np.uint32)
    s = oracle.score_meank(q_sum.astype(np.float32), [5], k_sum, mt, Hq, Hkv, D)
    assert s[0] == pytest.approx(1.0, abs=1e-5)
    assert s[1] == pytest.approx(-1.0, abs=1e-5)
    assert s[2] == pytest.approx(0.0, abs=1e-5)


def test_score_meank_invariances(oracle):
    rng = np.random.default_rng(2)
    L, B, Hq, Hkv, D = 2, 6, 6, 2, 64
    q_sum = rng.standard_normal((L, Hq * D)).astype(np.float32)
    k_sum = rng.standard_normal((L, B, Hkv * D)).astype(np.float32)
    mt = np.full((L, B), 128, np.uint32)
    base = oracle.score_meank(q_sum, [3, 3], k_sum, mt, Hq, Hkv, D)
    # a larger query sum over proportionally more rows: same direction
    assert np.allclose(oracle.score_meank(q_sum * 4, [12, 12], k_sum, mt, Hq, Hkv, D), base, atol=1e-6)
    perm = q_sum.reshape(L, Hq, D)[:, [2, 0, 1, 5, 3, 4]].reshape(L, Hq * D).copy()
    assert np.allclose(oracle.score_meank(perm, [3, 3], k_sum, mt, Hq, Hkv, D), base, atol=1e-6)


def test_q_accumulate_exact_integers(oracle):
    rng = np.random.default_rng(8)
    q = rng.integers(-1000, 1000, (3, 40, 96)).astype(np.float32)
    got = oracle.q_accumulate(q)
    assert np.array_equal(got, q.astype(np.int64).sum(axis=1).astype(np.float32))
    sub = [5, 0, 39, 7]
    assert np.array_equal(oracle.q_accumulate(q, sub),
                          q[:, sub].astype(np.int64).sum(axis=1).astype(np.float32))


def test_q_accumulate_token_order(oracle):
    # fp32: (1e8 + 5) rounds to 1e8 + 8, so the token-order sum is 8, while
    # pairing 1e8 with -1e8 first gives 5: only the reference's sequential
    # order reproduces 8, and the list order is honoured
    q = np.array([1e8, 5.0, -1e8], np.float32).reshape(1, 3, 1)
    assert oracle.q_accumulate(q)[0, 0] == 8.0
    assert oracle.q_accumulate(q, [0, 2, 1])[0, 0] == 5.0


def test_q_accumulate_continues_and_bounds(oracle):
    rng = np.random.default_rng(9)
    q = (rng.standard_normal((2, 64, 256)) * 3).astype(np.float32)
    first = oracle.q_accumulate(q, list(range(20)))
    both = oracle.q_accumulate(q, list(range(20, 64)), q_sum=first)
    assert np.array_equal(both, oracle.q_accumulate(q))
    exact = q.astype(np.float64).sum(axis=1)
    bound = 64 * np.finfo(np.float32).eps * np.abs(q).astype(np.float64).sum(axis=1)
    assert np.all(np.abs(both - exact) <= bound)
