"""Mean-K producer and mean-K cosine scorer on the GPU vs the oracle.

Sums are compared bit-exact (the producer adds the F16 keys in token order,
as the reference); scores within 1e-5 absolute of the oracle (cosines in
[-1, 1]; the GPU reduces channels in a lane-then-tree order).  Covers a
partial last block, a capacity larger than the history, layers without
query rows and blocks without keys, and the full 16-layer x 2048-block
history shape on sampled blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

T, HKV, HQ, D = 128, 4, 24, 256
E = HKV * D


def announce(msg: str) -> None:
    print(f"[meank] {msg}", flush=True)


def device_sums(ctx, k, n_blocks, cap, last_T=0, ids=None):
    L = k.shape[0]
    ks = torch.full((L, cap, E), float("nan"), dtype=torch.float32, device="cuda")
    mt = torch.zeros((L, cap), dtype=torch.int32, device="cuda")
    hist = ctx.make_history(k.data_ptr(), None, L, n_blocks, T, E, 0, last_T, cap)
    torch.cuda.synchronize()
    ctx.meank_sums(hist, list(range(n_blocks)) if ids is None else ids, ks.data_ptr(), mt.data_ptr())
    ctx.sync()
    return ks, mt


def test_meank_sums_bit_exact(ctx, oracle):
    announce("sums: 3 layers, 11 of 14 capacity blocks, partial last block of 53 tokens")
    L, nb, cap, last = 3, 11, 14, 53
    k, _, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=1, seed=21)
    k[0, 7] *= 900.0                       # large values: rounding inside the sums
    ks, mt = device_sums(ctx, k, nb, cap, last)
    kb = workloads.to_bits(torch, k)
    got, mtn = ks.cpu().numpy(), mt.cpu().numpy()
    for l in range(L):
        for b in range(nb):
            nt = last if b == nb - 1 else T
            assert mtn[l, b] == nt
            want = oracle.meank_sum_f16(kb[l, b].reshape(T, E)[:nt])
            assert np.array_equal(got[l, b].view(np.uint32), want.view(np.uint32)), (l, b)
    assert np.isnan(got[:, nb:]).all()     # blocks past the history are untouched


def test_meank_scores_vs_oracle(ctx, oracle):
    announce("scores: 4 layers x 40 blocks, layer 2 without query rows, block 9 without keys")
    L, nb = 4, 40
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=16, seed=22)
    ks, mt = device_sums(ctx, k, nb, nb)
    mt[:, 9] = 0
    q_sum = q.float().sum(dim=1).contiguous()          # [L][Hq*D] sums of 16 query rows
    q_count = [16, 16, 0, 16]
    scores = torch.empty(nb, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.score_meank(q_sum.data_ptr(), q_count, ks.data_ptr(), mt.data_ptr(), L, nb, HQ, HKV, D,
                    scores.data_ptr())
    ctx.sync()
    got = scores.cpu().numpy().astype(np.float64)
    want = oracle.score_meank(q_sum.cpu().numpy().reshape(L, HQ * D), q_count, ks.cpu().numpy(),
                              mt.cpu().numpy().astype(np.uint32), HQ, HKV, D)
    assert got[9] == 0.0
    assert np.max(np.abs(got - want)) <= 1e-5, np.max(np.abs(got - want))


@pytest.mark.parametrize("Tb,Hq,Hkv,Dh,last_T", [
    (32, 8, 8, 128, 5),      # no grouping, 1024-element rows
    (64, 6, 2, 256, 0),      # groups of 3, 512-element rows
    (16, 32, 16, 128, 16),   # groups of 2, 2048-element rows (the key sums' widest)
    (128, 16, 2, 128, 100),  # groups of 8, 256-element rows
])
def test_meank_other_groupings(ctx, oracle, Tb, Hq, Hkv, Dh, last_T):
    """Key sums bit-exact and mean-K scores within 1e-5 of the oracle's chain
    over head groupings of 1, 2, 3 and 8, row widths from 256 to 2048 and
    block lengths from 16 to 128 tokens, a partial last block included."""
    announce(f"mean-K: T={Tb} Hq={Hq} Hkv={Hkv} D={Dh} last_T={last_T}")
    L, nb, Tq = 3, 9, 5
    e = Hkv * Dh
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=Tq, seed=Tb + Hq + Dh, T=Tb, Hkv=Hkv, Hq=Hq,
                                        D=Dh)
    ks = torch.full((L, nb, e), float("nan"), dtype=torch.float32, device="cuda")
    mt = torch.zeros((L, nb), dtype=torch.int32, device="cuda")
    hist = ctx.make_history(k.data_ptr(), None, L, nb, Tb, e, 0, last_T, nb)
    torch.cuda.synchronize()
    ctx.meank_sums(hist, list(range(nb)), ks.data_ptr(), mt.data_ptr())
    ctx.sync()
    kb = workloads.to_bits(torch, k)
    got_s, got_mt = ks.cpu().numpy(), mt.cpu().numpy()
    for layer in range(L):
        for b in range(nb):
            nt = last_T if (b == nb - 1 and last_T) else Tb
            assert got_mt[layer, b] == nt
            want = oracle.meank_sum_f16(kb[layer, b].reshape(Tb, e)[:nt])
            assert np.array_equal(got_s[layer, b].view(np.uint32), want.view(np.uint32)), (layer, b)
    q_sum = torch.from_numpy(oracle.q_accumulate(q.float().cpu().numpy().reshape(L, Tq, -1))).to("cuda")
    scores = torch.empty(nb, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.score_meank(q_sum.data_ptr(), [Tq] * L, ks.data_ptr(), mt.data_ptr(), L, nb, Hq, Hkv, Dh, scores.data_ptr())
    ctx.sync()
    want = oracle.score_meank(q_sum.cpu().numpy(), [Tq] * L, got_s, got_mt.astype(np.uint32), Hq, Hkv, Dh)
    assert np.max(np.abs(scores.cpu().numpy().astype(np.float64) - want)) <= 1e-5


def test_meank_full_history_sampled(ctx, oracle):
    announce("full history 16 layers x 2048 blocks, sampled blocks")
    L, nb = 16, 2048
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=64, seed=2)
    ks, mt = device_sums(ctx, k, nb, nb)
    q_sum = q.float().sum(dim=1).contiguous()
    scores = torch.empty(nb, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.score_meank(q_sum.data_ptr(), [64] * L, ks.data_ptr(), mt.data_ptr(), L, nb, HQ, HKV, D,
                    scores.data_ptr())
    ctx.sync()
    ids = np.array([0, 1, 777, 1500, 2047])
    idx = torch.from_numpy(ids).cuda()
    kb = workloads.to_bits(torch, k[:, idx])
    sums = np.stack([[oracle.meank_sum_f16(kb[l, i].reshape(T, E)) for i in range(len(ids))]
                     for l in range(L)])
    assert np.array_equal(ks[:, idx].cpu().numpy().view(np.uint32), sums.view(np.uint32))
    want = oracle.score_meank(q_sum.cpu().numpy().reshape(L, HQ * D), [64] * L, sums,
                              np.full((L, len(ids)), T, np.uint32), HQ, HKV, D)
    got = scores.cpu().numpy()[ids].astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5
    del k, ks
    torch.cuda.empty_cache()


def test_engine_meank_preview_apply(oracle):
    """The engine with the reference scorer: scores within 1e-5 of the
    oracle over sums it produced itself, selection = the oracle's top-k over
    the engine's scores, sums refreshed after the history grows."""
    announce("engine mean-K preview: 2 layers x 30 blocks, grown tail")
    L, cap = 2, 32
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=8, seed=23, with_v=True)
    q_sum = q.float().sum(dim=1).contiguous()
    n_tok = 29 * T + 40
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=6, reserve_blocks=2, recent_blocks=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), cap, n_tok)
        for step in range(2):
            sel = eng.preview_meank(q_sum.data_ptr(), [8] * L)
            nb = eng.block_count()
            kb = workloads.to_bits(torch, k)
            last = eng.total_tokens() - (nb - 1) * T
            sums = np.stack([[oracle.meank_sum_f16(kb[l, b].reshape(T, E)[:(T if b < nb - 1 else last)])
                              for b in range(nb)] for l in range(L)])
            mt = np.full((L, nb), T, np.uint32)
            mt[:, nb - 1] = last
            want = oracle.score_meank(q_sum.cpu().numpy().reshape(L, HQ * D), [8] * L, sums, mt, HQ, HKV, D)
            got = np.array(eng.scores(), dtype=np.float64)
            assert np.max(np.abs(got - want)) <= 1e-5, step
            assert sel.blocks == oracle.pick_topk(got.astype(np.float32).astype(np.float64), 6, sink=1,
                                                  recent=1)
            eng.apply(sel)
            eng.append_tokens(50)           # the partial tail grows: its sums are redone


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_q_accumulate_bit_exact(ctx, oracle, dtype):
    announce(f"query sums {dtype}: 3 layers x 40 tokens x 6144, token list, continue")
    L, Tq, E = 3, 40, HQ * D
    g = torch.Generator(device="cpu").manual_seed(31)
    qf = torch.randn((L, Tq, E), generator=g) * 4
    qf[0, :3, 0] = torch.tensor([1e4, 3.0, -1e4])  # order-sensitive in fp32 for narrow types too
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    code = {"f32": kv.TYPE_F32, "f16": kv.TYPE_F16, "bf16": kv.TYPE_BF16}[dtype]
    q = qf.to(tdt).cuda()
    wide = q.float().cpu().numpy()
    qs = torch.full((L, E), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.q_accumulate(q.data_ptr(), code, L, Tq, E, qs.data_ptr())
    ctx.sync()
    want = oracle.q_accumulate(wide)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), want.view(np.uint32))
    sub = [7, 0, 33, 2]
    ctx.q_accumulate(q.data_ptr(), code, L, Tq, E, qs.data_ptr(), tokens=sub, reset=False)
    ctx.sync()
    want = oracle.q_accumulate(wide, sub, q_sum=want)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n_list", [768, 769, 1000])
def test_q_accumulate_long_token_list(ctx, oracle, n_list):
    """Token lists at the kernel arguments' capacity (768 entries, the
    table full) and past it (uploaded), repeats included: the sums
    bit-exact in list order, then continued by a second list."""
    announce(f"query sums over a {n_list}-entry token list")
    L, Tq, E = 2, 1200, 256
    rng = np.random.default_rng(37)
    wide = (rng.standard_normal((L, Tq, E)) * 3).astype(np.float32)
    q = torch.from_numpy(wide).to("cuda")
    qs = torch.full((L, E), float("nan"), dtype=torch.float32, device="cuda")
    tokens = rng.integers(0, Tq, n_list).tolist()
    torch.cuda.synchronize()
    ctx.q_accumulate(q.data_ptr(), kv.TYPE_F32, L, Tq, E, qs.data_ptr(), tokens=tokens)
    ctx.sync()
    want = oracle.q_accumulate(wide, tokens)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), want.view(np.uint32))
    more = rng.integers(0, Tq, 900).tolist()
    ctx.q_accumulate(q.data_ptr(), kv.TYPE_F32, L, Tq, E, qs.data_ptr(), tokens=more, reset=False)
    ctx.sync()
    want = oracle.q_accumulate(wide, more, q_sum=want)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_engine_scorer_meank_from_query_rows(oracle):
    """scorer = mean-K: preview takes the per-token query itself; the query
    sums, key sums and scores agree with the oracle chain."""
    announce("engine scorer=mean-K from query rows: 3 layers x 40 blocks")
    L, nb, Tq = 3, 40, 16
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=Tq, seed=24, with_v=True)
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=8, reserve_blocks=2, scorer=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * T)
        sel = eng.preview(q.data_ptr(), Tq)
        q_sum = oracle.q_accumulate(q.float().cpu().numpy().reshape(L, Tq, HQ * D))
        kb = workloads.to_bits(torch, k)
        sums = np.stack([[oracle.meank_sum_f16(kb[l, b].reshape(T, E)) for b in range(nb)]
                         for l in range(L)])
        want = oracle.score_meank(q_sum, [Tq] * L, sums, np.full((L, nb), T, np.uint32), HQ, HKV, D)
        got = np.array(eng.scores(), dtype=np.float64)
        assert np.max(np.abs(got - want)) <= 1e-5
        assert sel.blocks == oracle.pick_topk(got.astype(np.float32).astype(np.float64), 8, sink=1)
        stats = eng.apply(sel)
        assert stats["n_stage_in"] == len(sel.blocks)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_meank_add_decode_running_sum(ctx, oracle, dtype):
    """The decode producer over a strided K view (padded heads): two calls
    (reset, then continue) equal the oracle's token-order sums, and the
    count follows the kept tokens."""
    announce(f"decode running key sum {dtype}: 40 tokens x 4 heads x 256, padded strides")
    n_tok, dpad = 40, D + 8
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    code = {"f32": kv.TYPE_F32, "f16": kv.TYPE_F16, "bf16": kv.TYPE_BF16}[dtype]
    g = torch.Generator(device="cpu").manual_seed(41)
    full = (torch.randn((n_tok, HKV, dpad), generator=g) * 3).to(tdt).cuda()
    full[0, 0, 0] = 1e4 if dtype != "f32" else 1e8   # order-sensitive large first value
    esz = full.element_size()
    acc = torch.full((E,), float("nan"), dtype=torch.float32, device="cuda")
    cnt = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ctx.meank_add(full.data_ptr(), code, E, D, esz, dpad * esz, HKV * dpad * esz, 0, 25,
                  acc.data_ptr(), cnt.data_ptr(), reset=True)
    ctx.meank_add(full.data_ptr(), code, E, D, esz, dpad * esz, HKV * dpad * esz, 25, 15,
                  acc.data_ptr(), cnt.data_ptr(), reset=False)
    ctx.sync()
    rows = full[:, :, :D].float().cpu().numpy().reshape(1, n_tok, E)
    want = oracle.q_accumulate(rows)[0]            # every token in order from zero
    assert np.array_equal(acc.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert int(cnt.item()) == n_tok


def pinned_block_major(k, v):
    """Host history [block][layer][K rows, V rows] halves in one pinned
    allocation, from CPU tensors k, v [L][B][T][Hkv][D]."""
    L_, nb = k.shape[0], k.shape[1]
    kk = k.permute(1, 0, 2, 3, 4).reshape(nb, L_, -1)
    vv = v.permute(1, 0, 2, 3, 4).reshape(nb, L_, -1)
    hb = torch.empty((nb, L_ * (kk.shape[2] + vv.shape[2])), dtype=torch.float16, pin_memory=True)
    hb.copy_(torch.cat([kk, vv], dim=2).reshape(nb, -1))
    return hb


def test_meank_sums_from_pinned_host_bit_exact(ctx, oracle):
    """Key sums read by the device from a pinned block-major host history
    (partial last block, capacity above the block count) equal the
    oracle's token-order sums bit for bit."""
    announce("key sums from pinned host blocks: 3 layers x 21 blocks, 50-token tail")
    L, nb, cap, last = 3, 21, 24, 50
    k, v, _ = workloads.scoring_tensors(torch, "cpu", L=L, B=nb, Tq=1, seed=61, with_v=True)
    hb = pinned_block_major(k, v)
    hh = kv.HostHistory(hb.data_ptr(), L, nb, T, E, E, last)
    ks = torch.full((L, cap, E), float("nan"), dtype=torch.float32, device="cuda")
    mt = torch.zeros((L, cap), dtype=torch.int32, device="cuda")
    ids = [20, 0, 7, 13]
    torch.cuda.synchronize()
    ctx.meank_sums_host(hh, ids, ks.data_ptr(), mt.data_ptr(), capacity_blocks=cap)
    ctx.sync()
    kb = workloads.to_bits(torch, k)
    got, got_t = ks.cpu().numpy(), mt.cpu().numpy()
    for l in range(L):
        for b in ids:
            nt = last if b == nb - 1 else T
            want = oracle.meank_sum_f16(kb[l, b].reshape(T, E)[:nt])
            assert np.array_equal(got[l, b].view(np.uint32), want.view(np.uint32)), (l, b)
            assert got_t[l, b] == nt


def test_engine_host_only_history_meank(oracle):
    """The reference's deployment shape: every block in pinned host memory
    and no key mirror in HBM.  The mean-K scorer runs on key sums the device
    reads from the pinned blocks; stage-in reads the same blocks.  Scores
    within 1e-5 of the oracle chain, the selection equal to the oracle's
    top-k over those scores, pool rows bit-exact -- then the partial tail
    grows and is summed and staged again."""
    announce("host-only history: mean-K scorer, 2 layers x 40 blocks")
    L, nb, cap, Tq, budget = 2, 40, 48, 16, 8
    k, v, q = workloads.scoring_tensors(torch, "cpu", L=L, B=cap, Tq=Tq, seed=62, with_v=True)
    hb = pinned_block_major(k, v)
    qd = q.cuda()
    kb = workloads.to_bits(torch, k)
    vb = workloads.to_bits(torch, v)
    q_sum = oracle.q_accumulate(q.float().numpy().reshape(L, Tq, HQ * D))
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=budget, reserve_blocks=4, scorer=1, recent_blocks=1) as eng:
        eng.set_host_history(hb.data_ptr(), cap)
        for n_tok in (nb * T - 70, nb * T - 20):
            if eng.total_tokens() == 0:
                eng.append_tokens(n_tok)
            else:
                eng.append_tokens(n_tok - eng.total_tokens())   # the tail grows by 50 rows
            last = n_tok - (nb - 1) * T
            announce(f"{n_tok} tokens, tail block of {last}")
            sel = eng.preview(qd.data_ptr(), Tq)
            got = np.array(eng.scores(), dtype=np.float64)
            sums = np.stack([[oracle.meank_sum_f16(kb[l, b].reshape(T, E)[:(T if b < nb - 1 else last)])
                              for b in range(nb)] for l in range(L)])
            mt = np.full((L, nb), T, np.uint32)
            mt[:, nb - 1] = last
            want = oracle.score_meank(q_sum, [Tq] * L, sums, mt, HQ, HKV, D)
            assert np.max(np.abs(got - want)) <= 1e-5
            assert sel.blocks == oracle.pick_topk(got.astype(np.float32).astype(np.float64), budget,
                                                  sink=1, recent=1)
            eng.apply(sel)
            slots = eng.block_slots()
            for l in range(L):
                for which, src in ((0, kb), (1, vb)):
                    ptr = eng.pool_layer(l)[which]
                    n = eng.n_slots() * T * 1088
                    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                    c = kv.Context(0)
                    c.d2d_batched([ptr], [buf.data_ptr()], [n])
                    c.sync()
                    c.close()
                    pool = buf.cpu().numpy().reshape(-1, 1088)
                    for b in sel.blocks:
                        nt = T if b < nb - 1 else last
                        s = slots[b]
                        want_rows = oracle.quantize_rows_f16(kv.TYPE_Q8_0, src[l, b].reshape(T, E)[:nt])
                        assert np.array_equal(pool[s * T:s * T + nt], want_rows), (l, which, b)
        # the per-token scorer needs keys in HBM
        with pytest.raises(kv.KvMemError):
            with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                             budget_blocks=budget, reserve_blocks=4) as e2:
                e2.set_host_history(hb.data_ptr(), cap)
                e2.append_tokens(nb * T)
                e2.preview(qd.data_ptr(), Tq)
