"""The reselect workloads at their full sizes on the GPU, against the oracle.

- Scoring @256K (16 layers x 2048 blocks, 64-token bf16 query x 24 heads):
  every layer score of every block within 1e-3 relative of the oracle's fp32
  scorer, and the device top-256 (block 0 kept, ties to the lower id) equal
  to the top-256 over the ORACLE's scores, except blocks whose oracle score
  lies within 1e-3 relative of the k-th one.
- The full reselect step @256K through the engine (canonical layout, 77 of
  256 blocks changed): every staged block and a sample of the moved ones
  bit-exact in their slots, slot i holding the i-th selected block.
- The same step with the history in pinned host memory, block-major as the
  reference keeps it in host RAM (16 GiB, every block): the 77 changed
  blocks read over the link and quantized, every one bit-exact; then with a
  pinned packed host store, the evicted blocks' q8_0 rows saved bit-exact
  and the 77 blocks restored from them bit-exact.
- Mixed precision @256K (Student-t nu = 4): K q8_0 + V q4_0, then K and V
  q5_0 with a 96-block reserve; every staged block bit-exact.
- 1M workspace (16 layers x 8192 blocks, 512-token query, 32 planted
  blocks, budget 512): every planted block recalled, sampled blocks' scores
  against the oracle, the selection equal to the oracle's top-k over the
  same scores, and the cold stage-in of all 512 blocks sampled bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

L, T, HKV, HQ, D = 16, 128, 4, 24, 256
E = HKV * D
RTOL = 1e-3


def announce(msg: str) -> None:
    print(f"[fullsize] {msg}", flush=True)


def rel_err(got, want) -> np.ndarray:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.abs(got - want) / np.maximum(np.abs(want), 1e-6)


def check_selection_band(sel, oracle_scores, forced, need, rtol=RTOL) -> int:
    """`sel` holds every forced id and `need` others: all candidates scored
    (by the oracle) above the k-th best by more than rtol relative, and none
    scored below it by more.  Returns how many candidates fell in the band."""
    s = np.asarray(oracle_scores, np.float64)
    forced = set(int(b) for b in forced)
    cand = np.array([b for b in range(s.size) if b not in forced])
    order = cand[np.lexsort((cand, -s[cand]))]       # score desc, then lower id
    kth = s[order[need - 1]]
    band = rtol * abs(kth)
    chosen = set(int(b) for b in sel)
    assert forced <= chosen
    assert len(chosen) == len(sel) == len(forced) + need
    must_in = {int(b) for b in cand if s[b] > kth + band}
    must_out = {int(b) for b in cand if s[b] < kth - band}
    assert must_in <= chosen, sorted(must_in - chosen)[:8]
    assert not (must_out & chosen), sorted(must_out & chosen)[:8]
    return int(np.sum(np.abs(s[cand] - kth) <= band))


def pool_rows(eng, layer: int, which: int, type_) -> np.ndarray:
    ptr = eng.pool_layer(layer)[which]
    rb = kv.row_size(type_, E)
    n = eng.n_slots() * T * rb
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    c = kv.Context(0)
    c.d2d_batched([ptr], [buf.data_ptr()], [n])
    c.sync()
    c.close()
    return buf.cpu().numpy().reshape(eng.n_slots() * T, rb)


def check_blocks_in_pool(eng, oracle, k, v, blocks, type_k, type_v) -> None:
    """The pool rows of every listed block (all layers, K and V) equal the
    oracle's quantization of its history rows."""
    idx = torch.tensor(sorted(blocks), dtype=torch.long, device="cuda")
    kb = workloads.to_bits(torch, k[:, idx])
    vb = workloads.to_bits(torch, v[:, idx])
    slots = eng.block_slots()
    for layer in range(k.shape[0]):
        for which, src, ty in ((0, kb, type_k), (1, vb, type_v)):
            pool = pool_rows(eng, layer, which, ty)
            for j, b in enumerate(sorted(blocks)):
                s = slots[b]
                assert s >= 0, f"block {b} not in the pool"
                want = oracle.quantize_rows_f16(ty, src[layer, j].reshape(T, E))
                assert np.array_equal(pool[s * T:(s + 1) * T], want), (layer, "KV"[which], b, s)


def engine(**kw):
    p = dict(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D, budget_blocks=256,
             reserve_blocks=128, sink_blocks=1, recent_blocks=0, tie_lower_index=1)
    p.update(kw)
    return host.Engine(**p)


def test_scoring_256k_every_block_and_selection_band(oracle):
    announce("scoring 16 x 2048 blocks: every block vs the fp32 oracle, top-256 band rule")
    B, Tq = 2048, 64
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=2)
    scores = torch.empty(B, dtype=torch.float32, device="cuda")
    layer = torch.empty((L, B), dtype=torch.float32, device="cuda")
    with kv.Context(0) as ctx:
        hist = ctx.make_history(k.data_ptr(), None, L, B, T, E, 0)
        torch.cuda.synchronize()
        ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, scores.data_ptr(), layer.data_ptr())
        sel = ctx.topk(scores.data_ptr(), B, 255, forced=[0], tie_lower_index=True)
        ctx.sync()
    got_l = layer.cpu().numpy()
    got_s = scores.cpu().numpy()
    qf = q.float().cpu().numpy()
    kb = workloads.to_bits(torch, k)
    del k
    announce("oracle: fp32 per-token max scorer over all 2048 blocks x 16 layers (OpenMP)")
    want_l = oracle.score_pertoken_max_f32(qf, kb, 0, B)
    del kb
    assert np.isfinite(want_l).all()
    err_l = rel_err(got_l, want_l)
    assert err_l.max() <= RTOL, f"layer scores: max rel err {err_l.max():.3e}"
    want_s = oracle.combine_layers(want_l.astype(np.float64), 0)
    err_s = rel_err(got_s, want_s)
    assert err_s.max() <= RTOL, f"scores: max rel err {err_s.max():.3e}"
    n_band = check_selection_band(sel, want_s, forced=[0], need=255)
    announce(f"max rel err {err_l.max():.2e} (layers) {err_s.max():.2e} (mean); "
             f"{n_band} candidates inside the 1e-3 band of the 256th score")
    torch.cuda.empty_cache()


def test_reselect_256k_engine_step_bit_exact(oracle):
    announce("engine step @256K: 77 changed blocks, canonical layout, q8_0 K/V")
    B, Tq = 2048, 64
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=2, with_v=True)
    torch.cuda.synchronize()
    with engine() as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), B, B * T)
        sel = eng.preview(q.data_ptr(), Tq)
        prev = workloads.previous_selection(sel.blocks, B, 77)
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))
        old_slots = eng.block_slots()
        st = eng.apply_retrieval(q.data_ptr(), Tq)
        assert st["n_staged"] == 77 and st["n_stage_in"] == 77 and st["n_stage_out"] == 77
        slots = eng.block_slots()
        assert [slots[b] for b in sel.blocks] == list(range(256))
        staged = sorted(set(sel.blocks) - set(prev))
        moved = [b for b in sel.blocks if b in set(prev) and old_slots[b] != slots[b]]
        assert st["n_moved"] == len(moved)
        rng = np.random.default_rng(3)
        sample = sorted(rng.choice(moved, 16, replace=False).tolist()) if len(moved) > 16 else moved
        check_blocks_in_pool(eng, oracle, k, v, staged + sample, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    del k, v, q
    torch.cuda.empty_cache()


def test_reselect_256k_pinned_host_step_bit_exact(oracle):
    announce("pinned-host step @256K: 77 changed blocks read over the link from 16 GiB of block-major "
             "pinned history, then saved to and restored from a pinned packed store")
    B, Tq = 2048, 64
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=2, with_v=True)
    span_el = L * 2 * T * E
    hist = torch.empty((B, span_el), dtype=torch.float16, pin_memory=True)
    hv = hist.view(B, L, 2, T * E)
    for layer in range(L):
        hv[:, layer, 0].copy_(k[layer].reshape(B, T * E))
        hv[:, layer, 1].copy_(v[layer].reshape(B, T * E))
    torch.cuda.synchronize()
    row = kv.row_size(kv.TYPE_Q8_0, E)
    with engine() as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), B, B * T)   # the scorer's keys
        eng.set_host_history(hist.data_ptr(), B)                        # the stage-in's source
        sel = eng.preview(q.data_ptr(), Tq)
        prev = workloads.previous_selection(sel.blocks, B, 77)
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))
        st = eng.apply_retrieval(q.data_ptr(), Tq)
        assert st["n_staged"] == 77 and st["n_restored"] == 0
        staged = sorted(set(sel.blocks) - set(prev))
        check_blocks_in_pool(eng, oracle, k, v, staged, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
        announce("packed host store: the 77 blocks evicted (saved), then restored from their rows")
        packed = torch.zeros((B, L * 2 * T * row), dtype=torch.uint8, pin_memory=True)
        eng.set_packed_host(packed.data_ptr(), B)
        back = eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))
        assert back["n_saved"] == 77 and back["n_staged"] == 77
        assert all(eng.packed_valid(b) for b in staged)
        idx = torch.tensor(staged, dtype=torch.long, device="cuda")
        kb = workloads.to_bits(torch, k[:, idx])
        vb = workloads.to_bits(torch, v[:, idx])
        pk = packed.numpy()[staged].reshape(len(staged), L, 2, T, row)
        for layer in range(L):
            for j in range(len(staged)):
                for which, src in ((0, kb), (1, vb)):
                    want = oracle.quantize_rows_f16(kv.TYPE_Q8_0, src[layer, j].reshape(T, E))
                    assert np.array_equal(pk[j, layer, which], want), (layer, "KV"[which], staged[j])
        fwd = eng.apply_retrieval(q.data_ptr(), Tq)
        assert fwd["n_staged"] == 77 and fwd["n_restored"] == 77
        check_blocks_in_pool(eng, oracle, k, v, staged, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    del k, v, q, hist, hv, packed
    torch.cuda.empty_cache()


@pytest.mark.parametrize("tk,tv,reserve", [(kv.TYPE_Q8_0, kv.TYPE_Q4_0, 128),
                                           (kv.TYPE_Q5_0, kv.TYPE_Q5_0, 96)])
def test_mixed_precision_256k_bit_exact(oracle, tk, tv, reserve):
    announce(f"mixed precision @256K, Student-t history, K type {tk} / V type {tv}, reserve {reserve}")
    B, Tq = 2048, 64
    k, v, q = workloads.student_t_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=4)
    torch.cuda.synchronize()
    with engine(type_k=tk, type_v=tv, reserve_blocks=reserve) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), B, B * T)
        sel = eng.preview(q.data_ptr(), Tq)
        prev = workloads.previous_selection(sel.blocks, B, 77)
        eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), prev))
        st = eng.apply_retrieval(q.data_ptr(), Tq)
        assert st["n_staged"] == 77
        staged = sorted(set(sel.blocks) - set(prev))
        check_blocks_in_pool(eng, oracle, k, v, staged, tk, tv)
    del k, v, q
    torch.cuda.empty_cache()


def test_recall_1m_full(oracle):
    announce("1M workspace: 16 x 8192 blocks, 512-token query, 32 planted, budget 512")
    B, Tq, budget = 8192, 512, 512
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=6, with_v=True)
    planted = workloads.plant_blocks(torch, k, q, n_planted=32, seed=5)
    torch.cuda.synchronize()
    with engine(budget_blocks=budget, reserve_blocks=128) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), B, B * T)
        sel = eng.preview(q.data_ptr(), Tq)
        s = np.array(eng.scores(), dtype=np.float64)
        missing = [int(b) for b in planted if int(b) not in set(sel.blocks)]
        assert not missing, f"planted blocks not recalled: {missing}"
        assert sel.blocks == oracle.pick_topk(s.astype(np.float32).astype(np.float64), budget, sink=1)
        rng = np.random.default_rng(9)
        others = rng.choice(np.setdiff1d(np.arange(B), planted), 32, replace=False)
        ids = np.sort(np.concatenate([planted, others])).astype(np.int64)
        ksub = workloads.to_bits(torch, k[:, torch.from_numpy(ids).cuda()])
        want_l = oracle.score_pertoken_max_f32(q.float().cpu().numpy(), ksub, 0, ids.size)
        want = oracle.combine_layers(want_l.astype(np.float64), 0)
        err = rel_err(s[ids], want)
        assert err.max() <= RTOL, f"sampled scores: max rel err {err.max():.3e}"
        st = eng.apply(sel)
        assert st["n_staged"] == budget
        slots = eng.block_slots()
        assert [slots[b] for b in sel.blocks] == list(range(budget))
        sample = sorted(set(rng.choice(sel.blocks, 24, replace=False).tolist()) | set(planted[:8].tolist()))
        check_blocks_in_pool(eng, oracle, k, v, sample, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    del k, v, q
    torch.cuda.empty_cache()
