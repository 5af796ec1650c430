"""apply_retrieval's device plan: the selection diff and the slot moves
sized on the device behind the top-k, and the stage-in of the items the
plan kernel wrote (kvmem_engine_params.device_plan).  Two engines over the
same history, one planning on the device and one on the host, must leave
the same pool bytes, the same slots and the same plan counts after every
step, and both must equal the oracle's quantization of every selected
block; a failure anywhere in the device pipeline leaves no block called
resident with wrong bytes."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from engine_helpers import D, E, HQ, L, T, check_pool, history, host, kv, make_engine, workloads  # noqa: E402


def announce(msg: str) -> None:
    print(f"[test_gpu_device_plan] {msg}", flush=True)

ALL_KINDS = kv.FAIL_ALLOC | kv.FAIL_COPY | kv.FAIL_LAUNCH


def queries(seed: int, n: int, tq: int = 8):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return [torch.randn((L, tq, HQ, 256), generator=g, device="cuda").to(torch.bfloat16) for _ in range(n)]


def window(eng, type_k, type_v, ntok_of):
    """Bytes of every selected block's rows, slot by slot, both tensors."""
    out = {}
    slots = eng.block_slots()
    c = kv.Context(0)
    for layer in range(L):
        for which, ty in ((0, type_k), (1, type_v)):
            rb = kv.row_size(ty, E)
            n = eng.n_slots() * T * rb
            buf = torch.empty(n, dtype=torch.uint8, device="cuda")
            c.d2d_batched([eng.pool_layer(layer)[which]], [buf.data_ptr()], [n])
            c.sync()
            pool = buf.cpu().numpy().reshape(eng.n_slots() * T, rb)
            for b, s in enumerate(slots):
                if s >= 0:
                    out[(layer, which, b)] = pool[s * T: s * T + ntok_of(b)].copy()
    c.close()
    return out


def same_step(dev, ref, q, mandatory, types, ntok_of, oracle, k, v):
    sd = dev.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=mandatory)
    sr = ref.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=mandatory)
    assert sd["device_planned"] == 1 and sr["device_planned"] == 0
    sd.pop("device_planned")
    sr.pop("device_planned")
    assert sd == sr
    slots = dev.block_slots()
    assert slots == ref.block_slots()
    sel = [b for b, s in enumerate(slots) if s >= 0]
    assert sorted(slots[b] for b in sel) == list(range(len(sel)))  # canonical: slot i = i-th block
    wd, wr = window(dev, *types, ntok_of), window(ref, *types, ntok_of)
    assert wd.keys() == wr.keys()
    for key in wd:
        assert np.array_equal(wd[key], wr[key]), key
    check_pool(dev, oracle, k, v, sel, *types, ntok_of=ntok_of)
    return sd


TYPES = [(kv.TYPE_Q8_0, kv.TYPE_Q8_0), (kv.TYPE_Q8_0, kv.TYPE_Q4_0), (kv.TYPE_Q5_0, kv.TYPE_Q5_0),
         (kv.TYPE_F16, kv.TYPE_Q8_0)]


@pytest.mark.parametrize("types", TYPES, ids=["q8q8", "q8q4", "q5q5", "f16q8"])
def test_device_plan_equals_host_plan(oracle, types):
    announce(f"device plan vs host plan: 6 steps, 48-block history with a growing partial tail, types {types}")
    cap = 48
    k, v, _ = history(cap, seed=61)
    tail = {"n": 77}
    n_tok = 47 * T + tail["n"]
    ntok_of = lambda b: tail["n"] if b == 47 else T  # noqa: E731
    with make_engine(24, 8, *types, recent_blocks=1) as dev, \
            make_engine(24, 8, *types, recent_blocks=1, device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, n_tok)
        moved = 0
        for step, q in enumerate(queries(62, 6)):
            if step == 3:  # the resident tail grows: it is staged again
                for eng in (dev, ref):
                    eng.append_tokens(30)
                tail["n"] = 107
            st = same_step(dev, ref, q, (), types, ntok_of, oracle, k, v)
            moved += st["n_moved"]
        assert moved > 0


@pytest.mark.parametrize("types", [(kv.TYPE_Q8_0, kv.TYPE_Q4_0), (kv.TYPE_Q5_0, kv.TYPE_F16)],
                         ids=["q8q4", "q5f16"])
def test_device_plan_many_staged_blocks(oracle, types):
    """64 blocks staged at once, K and V in different formats: the stage-in
    reads the plan kernel's items, as many as the store stages."""
    announce(f"device plan: 64 staged blocks, several chunks per workgroup, types {types}")
    cap = 160
    k, v, _ = history(cap, seed=69)
    with make_engine(64, 16, *types) as dev, make_engine(64, 16, *types, device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        staged = 0
        for q in queries(70, 3):
            st = same_step(dev, ref, q, (), types, lambda b: T, oracle, k, v)
            staged = max(staged, st["n_staged"])
        assert staged == 64


def test_device_plan_long_chains_and_saves(oracle):
    announce("device plan: forced selections whose slot moves form chains longer than a segment")
    cap = 64
    k, v, q = history(cap, seed=63)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q4_0)
    steps = [
        [0] + list(range(10, 33)),                             # 24 blocks
        [0, 1, 2] + list(range(10, 31)),                       # 10..30 shift right by 2: chains of 10
        [0] + list(range(3, 12)) + list(range(20, 34)),        # shifts both ways
        [0] + list(range(40, 63)),                             # everything new
        [0] + list(range(39, 62)),                             # every block one slot right
        [0] + list(range(41, 64)),                             # and two slots left
    ]
    with make_engine(24, 8, *types) as dev, make_engine(24, 8, *types, device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        longest = 0
        for sel in steps:
            st = same_step(dev, ref, q, sel, types, lambda b: T, oracle, k, v)
            assert sorted(b for b, s in enumerate(dev.block_slots()) if s >= 0) == sel
            longest = max(longest, st["n_moved"])
        assert longest >= 20


def test_device_plan_budget_edges(oracle):
    announce("device plan: every block fits (host path), then a selection of one block past the sink")
    cap = 20
    k, v, q = history(cap, seed=65)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    with make_engine(24, 4, *types) as dev:
        dev.set_device_history(k.data_ptr(), v.data_ptr(), cap, 12 * T)
        st = dev.apply_retrieval(q.data_ptr(), q.shape[1])  # 12 blocks <= budget 24
        assert st["device_planned"] == 0 and st["n_staged"] == 12
        check_pool(dev, oracle, k, v, list(range(12)), *types)
    with make_engine(2, 2, *types) as dev, make_engine(2, 2, *types, device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        for q2 in queries(66, 3):
            same_step(dev, ref, q2, (), types, lambda b: T, oracle, k, v)


def test_device_plan_failure_leaves_exact_pool(oracle):
    announce("device plan: every allocation / copy / launch of an apply_retrieval failed in turn")
    cap = 40
    k, v, q = history(cap, seed=67)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q4_0)
    first = [0] + list(range(5, 28))
    second = [0, 1] + list(range(8, 30))
    n_failed = 0
    for nth in range(1, 64):
        with make_engine(24, 8, *types) as eng:
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
            eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=first)
            ctx = kv.Context.borrow(eng.ctx_handle())
            ctx.debug_fail_after(ALL_KINDS, nth)
            try:
                st = eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=second)
            except kv.KvMemError:
                n_failed += 1
                ctx.debug_fail_after(0, 0)
                slots = eng.block_slots()
                resident = [b for b, s in enumerate(slots) if s >= 0]
                check_pool(eng, oracle, k, v, resident, *types)
                st = eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=second)
                assert st["device_planned"] == 1
                check_pool(eng, oracle, k, v, second, *types)
                continue
            ctx.debug_fail_after(0, 0)
            assert st["device_planned"] == 1
            check_pool(eng, oracle, k, v, second, *types)
            break
    else:
        raise AssertionError("apply_retrieval never ran to completion")
    assert n_failed >= 4, n_failed  # scorer, top-k, plan, saves, chain walk, stage-in


def test_perf_stage_mask_and_after_score_span():
    """kvmem_hip_perf_stages: with SCORE | SET only the scorer and the
    stage-in are timed, and after_score_ms spans the scorer's end to the
    stage-in's end; with every stage the top-k and the slot moves are timed
    too."""
    announce("perf stage mask: scorer + stage-in only, then every stage")
    cap = 40
    k, v, q = history(cap, seed=71)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    first = [0] + list(range(10, 33))
    second = [0, 1, 2] + list(range(10, 31))   # 2 staged, the rest move right by 2
    with make_engine(24, 8, *types) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        ctx = kv.Context.borrow(eng.ctx_handle())
        eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=first)
        ctx.perf_stages(kv.PERF_STAGE_SCORE | kv.PERF_STAGE_SET)
        ctx.perf_enable(True)
        ctx.perf_reset()
        st = eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=second)
        pf = ctx.perf()
        assert st["n_staged"] == 2 and st["n_moved"] > 0 and st["device_planned"] == 1
        assert pf["n_score"] == 1 and pf["n_set"] == 1
        assert pf["n_topk"] == 0 and pf["n_layout"] == 0
        assert pf["n_after_score"] == 1
        assert pf["after_score_ms"] >= pf["set_ms"] > 0.0
        ctx.perf_stages(kv.PERF_STAGE_ALL)
        ctx.perf_reset()
        st = eng.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=first)
        pf = ctx.perf()
        ctx.perf_enable(False)
        assert st["n_moved"] > 0
        assert pf["n_score"] == 1 and pf["n_topk"] == 1 and pf["n_layout"] == 1
        assert pf["n_set"] == (1 if st["n_staged"] else 0)
        assert pf["after_score_ms"] >= pf["topk_ms"] + pf["layout_ms"] + pf["set_ms"]


XF_CASES = [
    # (n_rot, type_k, type_v): RoPE 256 + attn_rot on the 64-elements-per-lane kernel,
    # RoPE 64 + attn_rot on the 8-per-lane kernel, attn_rot alone
    (256, kv.TYPE_Q8_0, kv.TYPE_Q4_0),
    (64, kv.TYPE_Q5_0, kv.TYPE_Q5_0),
    (0, kv.TYPE_Q8_0, kv.TYPE_Q8_0),
]


@pytest.mark.parametrize("case", XF_CASES, ids=["rope256_q8q4", "rope64_q5q5", "hadamard_q8q8"])
def test_device_plan_with_row_transform(oracle, case):
    """A transformed pool (RoPE at the original positions, then attn_rot)
    through the device plan: the plan kernel carries the RoPE frequencies
    to the stage-in; pools equal the host-planned engine's byte for byte,
    and with RoPE 256 every selected block equals the oracle's transform
    and quantization."""
    from test_gpu_transform import expected_rows
    n_rot, tk, tv = case
    announce(f"device plan with the row transform: n_rot {n_rot} + attn_rot, types {(tk, tv)}, 4 steps")
    cap = 48
    k, v, _ = history(cap, seed=73)
    xf = dict(n_rot=n_rot, rope_freq_base=1e6, attn_rot=1)
    with make_engine(24, 8, tk, tv, **xf) as dev, make_engine(24, 8, tk, tv, device_plan=0, **xf) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        moved = 0
        for q in queries(74, 4):
            sd = dev.apply_retrieval(q.data_ptr(), q.shape[1])
            sr = ref.apply_retrieval(q.data_ptr(), q.shape[1])
            assert sd.pop("device_planned") == 1 and sr.pop("device_planned") == 0
            assert sd == sr
            assert dev.block_slots() == ref.block_slots()
            wd, wr = window(dev, tk, tv, lambda b: T), window(ref, tk, tv, lambda b: T)
            assert wd.keys() == wr.keys()
            for key in wd:
                assert np.array_equal(wd[key], wr[key]), key
            moved += sd["n_moved"]
        assert moved > 0
        if n_rot == 256:
            theta = oracle.rope_theta(256, 1e6)
            kb = workloads.to_bits(torch, k)
            vb = workloads.to_bits(torch, v)
            for (layer, which, b), got in wd.items():
                src, ty, nr, width = (kb, tk, 256, 256) if which == 0 else (vb, tv, 0, 64)
                want = expected_rows(oracle, ty, src[layer, b].reshape(T, E), D, nr,
                                     theta if nr else None, b * T, width)
                assert np.array_equal(got, want), (layer, which, b)


def test_device_plan_random_selections():
    """40 seeded random selections of 24 blocks (sink kept) over 64 blocks,
    some steps with a grown tail, every tenth step a repeat (nothing to
    stage or move): the device plan's diff, chain ranks, cut slots and stage
    items leave the same pool bytes and slots as the host plan after every
    step."""
    announce("device plan: 40 random selections vs the host plan, q8_0 K / q5_0 V")
    cap = 64
    k, v, q = history(cap, seed=75)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q5_0)
    rng = np.random.default_rng(76)
    tail = {"n": 60}
    ntok_of = lambda b: tail["n"] if b == cap - 1 else T  # noqa: E731
    with make_engine(24, 8, *types) as dev, make_engine(24, 8, *types, device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, (cap - 1) * T + tail["n"])
        moved = staged = 0
        for step in range(40):
            if step in (13, 27):  # the partial tail grows: staged again if resident
                for eng in (dev, ref):
                    eng.append_tokens(20)
                tail["n"] += 20
            # runs of neighbours as well as scattered ids, so chains of every length occur
            start = int(rng.integers(1, cap - 30))
            pool_ids = np.concatenate([np.arange(start, start + 30), rng.choice(np.arange(1, cap), 20)])
            if step % 10 != 9:  # every tenth step repeats the last: nothing staged or moved
                sel = sorted({0, *rng.choice(np.unique(pool_ids), 23, replace=False).tolist()})
            sd = dev.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=sel)
            sr = ref.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=sel)
            assert sd.pop("device_planned") == 1 and sr.pop("device_planned") == 0, step
            assert sd == sr, step
            slots = dev.block_slots()
            assert slots == ref.block_slots(), step
            assert sorted(b for b, s in enumerate(slots) if s >= 0) == sel, step
            wd, wr = window(dev, *types, ntok_of), window(ref, *types, ntok_of)
            for key in wd:
                assert np.array_equal(wd[key], wr[key]), (step, key)
            if step % 10 == 9:
                assert sd["n_staged"] == 0 and sd["n_moved"] == 0, step
            moved += sd["n_moved"]
            staged += sd["n_staged"]
        assert moved > 100 and staged > 100, (moved, staged)


GEOMETRIES = [
    # (block_tokens, n_head, n_head_kv, head_dim, type_k, type_v)
    (32, 8, 2, 128, kv.TYPE_Q8_0, kv.TYPE_Q4_0),
    (64, 16, 2, 128, kv.TYPE_Q5_0, kv.TYPE_Q8_0),
]


@pytest.mark.parametrize("geom", GEOMETRIES, ids=["T32_d128", "T64_d128"])
def test_device_plan_other_block_sizes(oracle, geom):
    """32- and 64-token blocks over 128-wide heads (256-element rows): 16
    random selections through the device and the host plan leave the same
    pool bytes and slots, and the last window equals the oracle's
    quantization of every selected block."""
    from kvmem_amd import host
    bt, hq, hkv, hd, tk, tv = geom
    nl, cap, budget = 2, 48, 16
    e = hkv * hd
    announce(f"device plan: {bt}-token blocks, {hkv} KV heads x {hd}, types {(tk, tv)}, 16 steps")
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=nl, B=cap, Tq=8, seed=77, T=bt, Hkv=hkv, Hq=hq,
                                        D=hd, with_v=True)
    torch.cuda.synchronize()
    rng = np.random.default_rng(78)

    def engine(**kw):
        return host.Engine(n_layers=nl, block_tokens=bt, n_head=hq, n_head_kv=hkv, head_dim=hd,
                           budget_blocks=budget, reserve_blocks=4, type_k=tk, type_v=tv, **kw)

    def pool_rows(eng, layer, which, ty):
        rb = kv.row_size(ty, e)
        n = eng.n_slots() * bt * rb
        buf = torch.empty(n, dtype=torch.uint8, device="cuda")
        c = kv.Context(0)
        c.d2d_batched([eng.pool_layer(layer)[which]], [buf.data_ptr()], [n])
        c.sync()
        c.close()
        return buf.cpu().numpy().reshape(eng.n_slots() * bt, rb)

    with engine() as dev, engine(device_plan=0) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * bt)
        moved = 0
        for step in range(16):
            sel = sorted({0, *rng.choice(np.arange(1, cap), budget - 1, replace=False).tolist()})
            sd = dev.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=sel)
            sr = ref.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=sel)
            assert sd.pop("device_planned") == 1 and sr.pop("device_planned") == 0, step
            assert sd == sr, step
            slots = dev.block_slots()
            assert slots == ref.block_slots(), step
            for layer in range(nl):
                for which, ty in ((0, tk), (1, tv)):
                    pd, pr = pool_rows(dev, layer, which, ty), pool_rows(ref, layer, which, ty)
                    for b in sel:
                        s = slots[b]
                        assert np.array_equal(pd[s * bt:(s + 1) * bt], pr[s * bt:(s + 1) * bt]), (step, b)
            moved += sd["n_moved"]
        assert moved > 0
        kb, vb = workloads.to_bits(torch, k), workloads.to_bits(torch, v)
        for layer in range(nl):
            for which, src, ty in ((0, kb, tk), (1, vb, tv)):
                pd = pool_rows(dev, layer, which, ty)
                for b in sel:
                    s = slots[b]
                    want = oracle.quantize_rows_f16(ty, src[layer, b].reshape(bt, e))
                    assert np.array_equal(pd[s * bt:(s + 1) * bt], want), (layer, which, b)


@pytest.mark.parametrize("scorer", [0, 1], ids=["per_token_max", "mean_k"])
def test_device_plan_query_window_both_scorers(scorer):
    """apply_retrieval through the device plan from the captured query
    window (q = NULL: the newest 64 captured rows) with either scorer: 5
    steps, each after a fresh ubatch of Qcur, leave the same slots, counts
    and pool bytes as the host-planned engine fed the same rows."""
    from test_gpu_qwindow import Capture
    announce(f"device plan from the query window, scorer {scorer}, 5 steps")
    cap = 40
    k, v, _ = history(cap, seed=79)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q4_0)
    with make_engine(16, 4, *types, scorer=scorer) as dev, \
            make_engine(16, 4, *types, scorer=scorer, device_plan=0) as ref:
        caps = (Capture("bf16", 80), Capture("bf16", 80))   # the same rows for both
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, cap * T)
        moved = 0
        for step in range(5):
            for eng, cp in zip((dev, ref), caps):
                cp.ubatch(eng, 64 * step, 64)
            sd = dev.apply_retrieval(0, 0)
            sr = ref.apply_retrieval(0, 0)
            assert sd.pop("device_planned") == 1 and sr.pop("device_planned") == 0, step
            assert sd == sr, step
            assert dev.block_slots() == ref.block_slots(), step
            wd, wr = window(dev, *types, lambda b: T), window(ref, *types, lambda b: T)
            assert wd.keys() == wr.keys()
            for key in wd:
                assert np.array_equal(wd[key], wr[key]), (step, key)
            moved += sd["n_moved"] + sd["n_staged"]
        assert moved > 0


def test_device_plan_transform_growing_tail(oracle):
    """RoPE 256 + attn_rot through the device plan while the last block is
    partial and grows between steps: the re-staged tail is RoPE'd at its
    original positions on its valid rows only; pools equal the host-planned
    engine's, and the tail equals the oracle's transform of its rows."""
    from test_gpu_transform import expected_rows
    announce("device plan, RoPE 256 + attn_rot, partial tail growing 50 -> 90 -> 128 tokens")
    cap = 32
    k, v, _ = history(cap, seed=81)
    types = (kv.TYPE_Q8_0, kv.TYPE_Q4_0)
    xf = dict(n_rot=256, rope_freq_base=1e6, attn_rot=1)
    tail = {"n": 50}
    ntok_of = lambda b: tail["n"] if b == cap - 1 else T  # noqa: E731
    mand = [0, cap - 1] + list(range(8, 20))   # the tail is always selected
    with make_engine(16, 4, *types, **xf) as dev, make_engine(16, 4, *types, device_plan=0, **xf) as ref:
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, (cap - 1) * T + tail["n"])
        for step, q in enumerate(queries(82, 3)):
            if step:
                for eng in (dev, ref):
                    eng.append_tokens(40 if step == 1 else 38)
                tail["n"] = 90 if step == 1 else 128
            sd = dev.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=mand)
            sr = ref.apply_retrieval(q.data_ptr(), q.shape[1], mandatory=mand)
            assert sd.pop("device_planned") == 1 and sr.pop("device_planned") == 0, step
            assert sd == sr, step
            if step:
                assert sd["n_staged"] >= 1  # the grown tail
            wd, wr = window(dev, *types, ntok_of), window(ref, *types, ntok_of)
            for key in wd:
                assert np.array_equal(wd[key], wr[key]), (step, key)
            theta = oracle.rope_theta(256, 1e6)
            kb = workloads.to_bits(torch, k)
            vb = workloads.to_bits(torch, v)
            b = cap - 1
            nt = tail["n"]
            for layer in range(L):
                want_k = expected_rows(oracle, types[0], kb[layer, b].reshape(T, E)[:nt], D, 256, theta,
                                       b * T, 256)
                want_v = expected_rows(oracle, types[1], vb[layer, b].reshape(T, E)[:nt], D, 0, None, b * T, 64)
                assert np.array_equal(wd[(layer, 0, b)], want_k), (step, layer, "K")
                assert np.array_equal(wd[(layer, 1, b)], want_v), (step, layer, "V")


@pytest.mark.parametrize("budget,reserve,on_device", [(1100, 20, 0), (1000, 3200, 0), (1024, 3072, 1)],
                         ids=["selection_1100", "slots_4200", "at_both_limits"])
def test_device_plan_at_and_past_its_limits(oracle, budget, reserve, on_device):
    """Past the device plan's limits (1024 selected blocks, 4096 pool
    slots) apply_retrieval plans on the host even when the device plan is
    asked for; at exactly both limits it plans on the device.  Over three
    queries either leaves the same stats, slots and pool bytes as an engine
    without the device plan, selects the oracle's top-k over its scores,
    and sampled blocks hold the oracle's q8_0 rows."""
    announce(f"device plan limits: budget {budget}, reserve {reserve}")
    lg, tg, hkv, hq, d = 2, 16, 1, 2, 256
    eg = hkv * d
    nb = 1300
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=lg, B=nb, Tq=1, seed=budget, T=tg, Hkv=hkv, Hq=hq,
                                        D=d, with_v=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(reserve)
    qs = [torch.randn((lg, 4, hq, d), generator=g, device="cuda").to(torch.bfloat16) for _ in range(3)]
    kb, vb = workloads.to_bits(torch, k), workloads.to_bits(torch, v)
    rb = kv.row_size(kv.TYPE_Q8_0, eg)
    rng = np.random.default_rng(budget + reserve)

    def engine(plan):
        return host.Engine(n_layers=lg, block_tokens=tg, n_head=hq, n_head_kv=hkv, head_dim=d,
                           budget_blocks=budget, reserve_blocks=reserve, device_plan=plan)

    def pool_bytes(eng):
        c = kv.Context.borrow(eng.ctx_handle())
        out = []
        for layer in range(lg):
            for ptr in eng.pool_layer(layer):
                n = eng.n_slots() * tg * rb
                buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                c.d2d_batched([ptr], [buf.data_ptr()], [n])
                c.sync()
                out.append(buf.cpu().numpy().reshape(eng.n_slots(), tg, rb))
        return out

    with engine(1) as dev, engine(0) as ref:
        assert dev.n_slots() == budget + reserve
        for eng in (dev, ref):
            eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * tg)
        for q in qs:
            torch.cuda.synchronize()
            sd = dev.apply_retrieval(q.data_ptr(), q.shape[1])
            sr = ref.apply_retrieval(q.data_ptr(), q.shape[1])
            assert sd.pop("device_planned") == on_device and sr.pop("device_planned") == 0
            assert sd == sr
            slots = dev.block_slots()
            assert slots == ref.block_slots()
            sel = [b for b, s in enumerate(slots) if s >= 0]
            assert sorted(slots[b] for b in sel) == list(range(len(sel)))  # canonical layout
            scores = np.array(dev.scores(), dtype=np.float64)
            assert sel == oracle.pick_topk(scores.astype(np.float32).astype(np.float64), budget, sink=1)
            pd, pr = pool_bytes(dev), pool_bytes(ref)
            for a, b in zip(pd, pr):
                assert np.array_equal(a[[slots[x] for x in sel]], b[[slots[x] for x in sel]])
            for b in rng.choice(sel, 24, replace=False).tolist():
                for layer in range(lg):
                    for which, src in ((0, kb), (1, vb)):
                        want = oracle.quantize_rows_f16(kv.TYPE_Q8_0, src[layer, b].reshape(tg, eg))
                        assert np.array_equal(pd[2 * layer + which][slots[b]], want), (layer, which, b)
    del k, v
    torch.cuda.empty_cache()
