"""MFMA per-token max scorer vs the fp64 oracle (1e-3 relative, fp32
accumulation on the GPU), plus the full 16-layer x 2048-block scoring
workload checked on sampled blocks and through its top-k."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import workloads  # noqa: E402

RTOL = 1e-3


def announce(msg: str) -> None:
    print(f"[score] {msg}", flush=True)


def run_score(ctx, k, q, q_type, Hq, Hkv, D, last_T=0, reduce=kv.LAYER_MEAN):
    L, B, T = k.shape[0], k.shape[1], k.shape[2]
    scores = torch.empty(B, dtype=torch.float32, device="cuda")
    layer = torch.empty((L, B), dtype=torch.float32, device="cuda")
    hist = ctx.make_history(k.data_ptr(), None, L, B, T, Hkv * D, 0, last_T)
    torch.cuda.synchronize()
    ctx.score(hist, q.data_ptr(), q_type, q.shape[1], Hq, Hkv, D, scores.data_ptr(), layer.data_ptr(),
              reduce)
    ctx.sync()
    return scores.cpu().numpy().astype(np.float64), layer.cpu().numpy().astype(np.float64)


def q_f32(q) -> np.ndarray:
    return q.float().cpu().numpy()


def assert_close(got, want, what):
    err = np.abs(got - want) / np.maximum(np.abs(want), 1e-6)
    i = int(np.argmax(err))
    assert err.max() <= RTOL, f"{what}: max rel err {err.max():.3e} at {i}: got {got.flat[i]} want {want.flat[i]}"


@pytest.mark.parametrize("D,Tq,q_dtype,last_T", [
    (256, 16, "bf16", 77),
    (256, 80, "bf16", 0),      # 480 query rows: two 384-row slices
    (128, 64, "f16", 5),
    (256, 7, "f16", 128),
])
def test_score_small_vs_fp64_oracle(ctx, oracle, D, Tq, q_dtype, last_T):
    announce(f"small scorer D={D} Tq={Tq} q={q_dtype} last_T={last_T}")
    L, B, T, Hkv, Hq = 2, 19, 128, 4, 24
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=3 + D + Tq, D=D)
    qt = kv.TYPE_BF16
    if q_dtype == "f16":
        q = q.to(torch.float16)
        qt = kv.TYPE_F16
    s, ls = run_score(ctx, k, q, qt, Hq, Hkv, D, last_T)
    want_ls = oracle.score_pertoken_max(q_f32(q), workloads.to_bits(torch, k), last_T)
    assert_close(ls, want_ls, "layer scores")
    assert_close(s, oracle.combine_layers(want_ls, 0), "mean scores")


@pytest.mark.parametrize("T,Hq,Hkv,D,Tq,last_T", [
    (32, 8, 8, 128, 12, 9),      # no grouping: one query head per KV head
    (64, 6, 2, 256, 10, 1),      # groups of 3
    (16, 32, 4, 128, 50, 16),    # groups of 8, 400 rows: two slices, full last block
    (96, 8, 2, 128, 100, 95),    # groups of 4, 400 rows over 128-wide heads: two slices
    (128, 16, 16, 256, 1, 127),  # one query token
    (1, 24, 4, 256, 8, 0),       # one-token blocks
])
def test_score_other_groupings_and_block_sizes(ctx, oracle, T, Hq, Hkv, D, Tq, last_T):
    """Head groupings (1, 3, 4, 8 query heads per KV head), block lengths from
    1 to 128 tokens and queries of several row slices at both head sizes:
    every layer score and block score within 1e-3 of the fp64 oracle."""
    announce(f"scorer: T={T} Hq={Hq} Hkv={Hkv} D={D} Tq={Tq} last_T={last_T}")
    L, B = 3, 13
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=5 * T + Hq + Tq, T=T, Hkv=Hkv, Hq=Hq,
                                        D=D)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, Hq, Hkv, D, last_T)
    want_ls = oracle.score_pertoken_max(q_f32(q), workloads.to_bits(torch, k), last_T)
    assert_close(ls, want_ls, "layer scores")
    assert_close(s, oracle.combine_layers(want_ls, 0), "mean scores")


@pytest.mark.parametrize("mode", [kv.LAYER_MEAN, kv.LAYER_MAX, kv.LAYER_SUM])
def test_score_layer_reduce_modes(ctx, oracle, mode):
    announce(f"layer reduce mode {mode}")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=3, B=9, Tq=8, seed=17)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, 24, 4, 256, reduce=mode)
    want = oracle.combine_layers(oracle.score_pertoken_max(q_f32(q), workloads.to_bits(torch, k)), mode)
    assert_close(s, want, f"mode {mode}")


@pytest.mark.parametrize("mode", [kv.LAYER_MEAN, kv.LAYER_MAX, kv.LAYER_SUM])
def test_score_fold_many_layers_exact(ctx, oracle, mode):
    """20 layers, 37 blocks (the last workgroup of the fold partly empty), an
    80-token query (two 384-row slices: 32 partial maxima per layer).  The
    block score is exactly the f32 reduction, in layer order, of the layer
    scores the same call returns; the layer scores of two blocks match the
    oracle."""
    announce(f"fold: 20 layers x 37 blocks, Tq=80, mode {mode}")
    L, B, Tq = 20, 37, 80
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=29)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, 24, 4, 256, reduce=mode)
    ls32 = ls.astype(np.float32)
    if mode == kv.LAYER_MAX:
        acc = ls32.max(axis=0)
    else:
        acc = np.zeros(B, dtype=np.float32)
        for lay in range(L):
            acc = (acc + ls32[lay]).astype(np.float32)
        if mode == kv.LAYER_MEAN:
            acc = (acc / np.float32(L)).astype(np.float32)
    assert np.array_equal(s.astype(np.float32), acc)
    want = oracle.score_pertoken_max(q_f32(q), workloads.to_bits(torch, k[:, :2].contiguous()))
    assert_close(ls[:, :2], want, "layer scores")


def test_score_bf16_query_past_f16_range(ctx, oracle):
    """bf16 query values beyond f16's range (|q| >= 65536) in a few rows: the
    waves holding them convert their rows scaled by a power of two and scale
    their maxima back, so scores stay finite and match the oracle; waves
    without them are untouched."""
    announce("bf16 query rows past f16 range")
    L, B, Tq = 2, 7, 16
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=41)
    qf = q.float()
    g = torch.Generator(device="cuda").manual_seed(42)
    qf[0, 3, 5] = 3.0e5 * torch.sign(torch.randn(256, device="cuda", generator=g))  # a whole row
    qf[1, 10, 17, 7] = -2.0e6                                                           # one element
    q = qf.to(torch.bfloat16)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, 24, 4, 256)
    assert np.isfinite(s).all() and np.isfinite(ls).all()
    want_ls = oracle.score_pertoken_max(q_f32(q), workloads.to_bits(torch, k))
    assert_close(ls, want_ls, "layer scores")
    assert ls.max() > 1e4  # the large rows decide some blocks' scores


def test_score_invariants(ctx):
    """Permuting tokens inside a block and query heads inside a GQA group
    leaves scores unchanged; scaling Q by 2 scales them by 2."""
    announce("scorer invariants")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=2, B=6, Tq=8, seed=23)
    base, _ = run_score(ctx, k, q, kv.TYPE_BF16, 24, 4, 256)
    perm = torch.randperm(128, generator=torch.Generator().manual_seed(1)).cuda()
    s1, _ = run_score(ctx, k[:, :, perm].contiguous(), q, kv.TYPE_BF16, 24, 4, 256)
    assert np.array_equal(s1, base) or np.allclose(s1, base, rtol=1e-6, atol=0)
    hp = torch.tensor([5, 4, 3, 2, 1, 0] + list(range(6, 24)), device="cuda")
    s2, _ = run_score(ctx, k, q[:, :, hp].contiguous(), kv.TYPE_BF16, 24, 4, 256)
    assert np.allclose(s2, base, rtol=1e-6, atol=0)
    s3, _ = run_score(ctx, k, (q.float() * 2).to(torch.bfloat16), kv.TYPE_BF16, 24, 4, 256)
    assert np.allclose(s3, 2 * base, rtol=1e-6, atol=0)


def test_score_full_256k_sampled_and_topk(ctx, oracle):
    """16 layers x 2048 blocks x 64-token query: every block scored on the
    GPU; 6 sampled blocks checked against the fp64 oracle; the device top-256
    (sink 0, ties to the lower id) equal to the oracle's top-k over the same
    scores."""
    announce("full scoring workload 16 x 2048 blocks")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=16, B=2048, Tq=64, seed=2)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, 24, 4, 256)
    assert np.isfinite(s).all()
    rng = np.random.default_rng(0)
    ids = np.sort(rng.choice(2048, 6, replace=False)).astype(np.uint32)
    ksub = workloads.to_bits(torch, k[:, torch.from_numpy(ids.astype(np.int64)).cuda()])
    want = oracle.score_pertoken_max(q_f32(q), ksub)
    assert_close(ls[:, ids], want, "sampled layer scores")
    assert_close(s[ids], want.mean(axis=0), "sampled mean scores")
    scores_dev = torch.from_numpy(s.astype(np.float32)).cuda()
    torch.cuda.synchronize()
    sel = ctx.topk(scores_dev.data_ptr(), 2048, 255, forced=[0], tie_lower_index=True)
    want_sel = oracle.pick_topk(s.astype(np.float32).astype(np.float64), 256, sink=1)
    assert sel == want_sel
    del k
    torch.cuda.empty_cache()


@pytest.mark.parametrize("Tq", [80, 200, 512], ids=["2_slices", "4_slices", "8_slices"])
def test_score_multi_slice_short_chunks(ctx, oracle, Tq):
    """Queries of several 384-row slices over 4100 blocks, the last one
    partial: the launch splits the blocks into short chunks (32, 64 and 16
    blocks for 2, 4 and 8 slices, the last chunk ragged).  Blocks on both
    sides of chunk boundaries, the last chunk's and the partial last block
    are checked against the oracle's fp32 scorer."""
    L, B, Hkv, Hq, D, last_T = 2, 4100, 4, 24, 256, 50
    announce(f"scorer over {B} blocks, {Tq}-token query ({-(-Tq * Hq // Hkv // 384)} slices)")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=90 + Tq)
    s, ls = run_score(ctx, k, q, kv.TYPE_BF16, Hq, Hkv, D, last_T)
    assert np.isfinite(s).all()
    rng = np.random.default_rng(Tq)
    edges = [0, 1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 4031, 4032, 4095, 4096, 4097, 4098]
    ids = np.unique(np.concatenate([edges, rng.choice(B - 1, 12, replace=False), [B - 1]]))
    ksub = workloads.to_bits(torch, k[:, torch.from_numpy(ids.astype(np.int64)).cuda()])
    want = oracle.score_pertoken_max_f32(q_f32(q), ksub, 0, ids.size, last_block_tokens=last_T)
    assert_close(ls[:, ids], want, "layer scores")
    del k
    torch.cuda.empty_cache()
