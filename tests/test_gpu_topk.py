"""Device top-k vs the oracle's KvMemStore top-k restatement (same f32
scores in, identical ids out), ties in both tie modes, forced ids."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()


def announce(msg: str) -> None:
    print(f"[topk] {msg}", flush=True)


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("n,budget", [(1, 1), (7, 3), (100, 37), (2048, 256), (2049, 256),
                                      (8192, 512), (16384, 4096), (300, 299)])
def test_topk_sink_matches_oracle(ctx, oracle, n, budget):
    announce(f"n={n} budget={budget}")
    rng = np.random.default_rng(n + budget)
    s = rng.standard_normal(n).astype(np.float32)
    d = dev(s)
    torch.cuda.synchronize()
    need = max(0, budget - 1) if n > budget else n
    forced = [0] if n > budget else []
    got = ctx.topk(d.data_ptr(), n, need, forced=forced)
    want = oracle.pick_topk(s.astype(np.float64), budget, sink=1)
    assert got == want


@pytest.mark.parametrize("tie_lower", [True, False])
def test_topk_ties(ctx, oracle, tie_lower):
    announce(f"ties tie_lower={tie_lower}")
    rng = np.random.default_rng(9)
    n = 3000
    s = rng.integers(-3, 4, n).astype(np.float32) * 0.5  # 7 distinct values
    s[rng.choice(n, 20, replace=False)] = -0.0
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, 700, forced=[0, 1], tie_lower_index=tie_lower)
    want = oracle.pick_topk(s.astype(np.float64), 702, sink=2, tie_lower_index=tie_lower)
    assert got == want


def test_topk_forced_mandatory_recent(ctx, oracle):
    """Forced = sink + mandatory + recent as the store charges them."""
    announce("forced sink/mandatory/recent")
    rng = np.random.default_rng(5)
    n, budget, sink, recent = 1000, 64, 2, 3
    mand = [700, 701, 702, 999]
    s = rng.standard_normal(n).astype(np.float32)
    want = oracle.pick_topk(s.astype(np.float64), budget, sink=sink, recent=recent, mandatory=mand)
    forced = sorted(set(list(range(sink)) + mand + [n - 1 - i for i in range(recent)]))
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, budget - len(forced), forced=forced)
    assert got == want


def test_topk_need_exceeds_candidates(ctx):
    announce("need > candidates")
    s = np.arange(10, dtype=np.float32)
    d = dev(s)
    torch.cuda.synchronize()
    assert ctx.topk(d.data_ptr(), 10, 50, forced=[3]) == list(range(10))
    assert ctx.topk(d.data_ptr(), 10, 0, forced=[3, 7]) == [3, 7]
    with pytest.raises(kv.KvMemError):
        ctx.topk(d.data_ptr(), 10, 1, forced=[10])


@pytest.mark.parametrize("n_mand", [63, 64, 300])
def test_topk_many_forced(ctx, oracle, n_mand):
    """Up to 64 distinct forced ids travel in the kernel arguments, more go
    through an upload: both sides of that limit, with repeated ids (which
    count once)."""
    announce(f"sink + {n_mand} mandatory ids, repeats included")
    rng = np.random.default_rng(40 + n_mand)
    n, fill = 5000, 200
    s = rng.standard_normal(n).astype(np.float32)
    mand = sorted(rng.choice(np.arange(1, n), n_mand, replace=False).tolist())
    budget = 1 + n_mand + fill
    want = oracle.pick_topk(s.astype(np.float64), budget, sink=1, mandatory=mand)
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, fill, forced=[0] + mand + mand[:5])
    assert got == want
    assert len(got) == budget


@pytest.mark.parametrize("n,budget,tie_lower", [(16385, 512, True), (20000, 512, False),
                                                (65536, 4096, True), (300000, 2048, False)])
def test_topk_beyond_lds_keys(ctx, oracle, n, budget, tie_lower):
    """More blocks than the keys LDS holds: the keys are recomputed from the
    scores in every radix pass.  Ties (a coarse score grid), a sink and 100
    mandatory ids (the upload path), both tie rules."""
    announce(f"n={n} budget={budget} tie_lower={tie_lower}")
    rng = np.random.default_rng(n)
    s = (rng.integers(-400, 400, n) * 0.25).astype(np.float32)
    mand = sorted(rng.choice(np.arange(1, n), 100, replace=False).tolist())
    want = oracle.pick_topk(s.astype(np.float64), budget, sink=1, mandatory=mand,
                            tie_lower_index=tie_lower)
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, budget - 101, forced=[0] + mand, tie_lower_index=tie_lower)
    assert got == want


@pytest.mark.parametrize("n,budget,tie_lower", [(2048, 257, True), (16384, 1024, False),
                                                (50000, 2048, True), (300000, 512, False)])
def test_topk_distinct_scores_early_exit(ctx, oracle, n, budget, tie_lower):
    """Continuous scores (no ties but the forced ids): the radix select
    stops once the threshold key stands alone in its digit, in the LDS
    kernel (n <= 16384) and in the streaming one."""
    announce(f"distinct scores n={n} budget={budget} tie_lower={tie_lower}")
    rng = np.random.default_rng(n + 7)
    s = rng.standard_normal(n).astype(np.float32)
    want = oracle.pick_topk(s.astype(np.float64), budget, sink=1, tie_lower_index=tie_lower)
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, budget - 1, forced=[0], tie_lower_index=tie_lower)
    assert got == want


def test_engine_selects_over_20000_blocks(oracle):
    """The engine's preview over 20000 blocks of 32 tokens (a 640K-token
    history at --kvmem-block-tokens 32): the device top-k equals the
    oracle's over the same scores."""
    from kvmem_amd import host, workloads
    announce("engine preview over 20000 blocks of 32 tokens")
    L, nb, bt, tq = 1, 20000, 32, 8
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=tq, seed=12, T=bt, with_v=True)
    torch.cuda.synchronize()
    with host.Engine(n_layers=L, block_tokens=bt, n_head=24, n_head_kv=4, head_dim=256,
                     budget_blocks=512, reserve_blocks=64) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * bt)
        sel = eng.preview(q.data_ptr(), tq)
        s = np.array(eng.scores(), dtype=np.float64)
        assert sel.blocks == oracle.pick_topk(s.astype(np.float32).astype(np.float64), 512, sink=1)
        st = eng.apply(sel)
        assert st["n_staged"] == 512
    del k, v, q
    torch.cuda.empty_cache()


@pytest.mark.parametrize("n", [5000, 40000], ids=["lds", "streamed"])
@pytest.mark.parametrize("tie_lower", [True, False])
def test_topk_many_forced_ids_uploaded(ctx, oracle, n, tie_lower):
    """More forced ids than travel in the kernel arguments (64): 150 of them,
    20 repeated, uploaded instead; scores rounded to integers so that many
    tie.  Both kernels (keys in LDS, and recomputed per pass above 16384
    blocks), both tie rules: the oracle's selection."""
    announce(f"{n} blocks, 150 forced ids (uploaded), lower-id ties {tie_lower}")
    rng = np.random.default_rng(n + int(tie_lower))
    s = np.round(rng.standard_normal(n) * 8).astype(np.float32)
    forced = sorted(rng.choice(n, 150, replace=False).tolist())
    need = 77
    want = oracle.pick_topk(s.astype(np.float64), len(forced) + need, sink=0, mandatory=forced,
                            tie_lower_index=tie_lower)
    d = dev(s)
    torch.cuda.synchronize()
    got = ctx.topk(d.data_ptr(), n, need, forced=forced + forced[:20], tie_lower_index=tie_lower)
    assert got == want
