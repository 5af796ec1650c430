"""Several reselect engines on one GPU, driven from as many host threads at
once.

Each engine has its own device context, stream, pool, history and store;
the library keeps no other state per process than the allocation-free
scorer's scratch guard.  Four engines of different pool formats and slot
layouts each run six agent steps over their own history (the history grows
by a partial block before every step after the first; even steps preview
and apply, odd ones run apply_retrieval), all four threads at the same
time.  The same four sequences then run one after another on one thread.
Checked:
  - concurrent and sequential runs agree bit for bit: every step's scores,
    selection and slot map, and each engine's final pool bytes;
  - the sequential run against the oracle: the last step's scores within
    1e-3 of the fp64 scorer, its selection the oracle's top-k over the
    engine's scores, and every selected block's pool rows bit-exact.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()

from engine_helpers import RTOL, T, check_pool, history, make_engine, oracle_scores  # noqa: E402

CAP, N0, STEPS, GROW = 48, 30, 6, 50


@dataclass(frozen=True)
class Cfg:
    type_k: int
    type_v: int
    budget: int
    reserve: int
    canonical: int
    seed: int


CFGS = (Cfg(kv.TYPE_Q8_0, kv.TYPE_Q8_0, 12, 4, 1, 101),
        Cfg(kv.TYPE_Q4_0, kv.TYPE_Q8_0, 10, 6, 0, 102),
        Cfg(kv.TYPE_Q5_0, kv.TYPE_Q5_0, 16, 4, 1, 103),
        Cfg(kv.TYPE_Q8_0, kv.TYPE_F16, 8, 4, 1, 104))


def announce(msg: str) -> None:
    print(f"[threads] {msg}", flush=True)


def inputs(cfg: Cfg):
    k, v, q0 = history(CAP, seed=cfg.seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(cfg.seed + 1000)
    queries = [torch.randn(q0.shape, generator=g, device="cuda").to(q0.dtype) for _ in range(STEPS)]
    torch.cuda.synchronize()
    return k, v, queries


def pool_bytes(eng) -> list:
    out = []
    ctx = kv.Context(0)
    try:
        for layer in range(2):
            for ptr, ty in zip(eng.pool_layer(layer), (eng.params.type_k, eng.params.type_v)):
                n = eng.n_slots() * T * kv.row_size(ty, 1024)
                buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                torch.cuda.synchronize()
                ctx.d2d_batched([ptr], [buf.data_ptr()], [n])
                ctx.sync()
                out.append(buf.cpu().numpy())
    finally:
        ctx.close()
    return out


def run(cfg: Cfg, data, check=None):
    """The six steps of one engine: per step (blocks, selection, scores,
    slots); then the final pool bytes.  `check(eng, last)` runs on the live
    engine after the last step."""
    k, v, queries = data
    steps = []
    with make_engine(cfg.budget, cfg.reserve, cfg.type_k, cfg.type_v, canonical_layout=cfg.canonical) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), CAP, N0 * T)
        for s, q in enumerate(queries):
            if s:
                eng.append_tokens(GROW)
            if s % 2 == 0:
                sel = eng.preview(q.data_ptr(), q.shape[1])
                eng.apply(sel)
                chosen = list(sel.blocks)
            else:
                eng.apply_retrieval(q.data_ptr(), q.shape[1])
                chosen = [b for b, slot in enumerate(eng.block_slots()) if slot >= 0]
            steps.append((eng.block_count(), chosen, np.array(eng.scores(), dtype=np.float32),
                          list(eng.block_slots())))
        pool = pool_bytes(eng)
        if check:
            check(eng, steps[-1])
    return steps, pool


def test_engines_in_threads_match_sequential_and_oracle(oracle):
    announce(f"{len(CFGS)} engines x {STEPS} steps, concurrently from {len(CFGS)} threads")
    data = [inputs(c) for c in CFGS]
    results: list = [None] * len(CFGS)
    errors: list = []
    start = threading.Barrier(len(CFGS))

    def worker(i: int) -> None:
        try:
            start.wait()
            results[i] = run(CFGS[i], data[i])
        except BaseException as ex:  # reported on the main thread
            errors.append((i, ex))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(CFGS))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    announce("concurrent run done; sequential run with the oracle checks")

    total = N0 * T + (STEPS - 1) * GROW
    n_blocks = (total + T - 1) // T
    last_T = total - (n_blocks - 1) * T

    for i, cfg in enumerate(CFGS):
        k, v, queries = data[i]

        def check(eng, last, cfg=cfg, k=k, v=v, q=queries[-1]):
            nb, chosen, scores, _ = last
            assert nb == n_blocks
            want = oracle_scores(oracle, q, k, nb, last_T)
            rel = np.abs(scores.astype(np.float64) - want) / np.maximum(np.abs(want), 1e-6)
            assert rel.max() <= RTOL, f"engine {i}: max rel err {rel.max():.3e}"
            assert chosen == oracle.pick_topk(scores.astype(np.float64), cfg.budget, sink=1)
            check_pool(eng, oracle, k, v, chosen, cfg.type_k, cfg.type_v,
                       ntok_of=lambda b: last_T if b == nb - 1 else T)

        steps, pool = run(cfg, data[i], check)
        c_steps, c_pool = results[i]
        for s, (a, b) in enumerate(zip(steps, c_steps)):
            assert a[0] == b[0] and a[1] == b[1] and a[3] == b[3], f"engine {i} step {s}: selection or slots"
            assert np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32)), f"engine {i} step {s}: scores"
        for j, (a, b) in enumerate(zip(pool, c_pool)):
            assert np.array_equal(a, b), f"engine {i} pool tensor {j}"
