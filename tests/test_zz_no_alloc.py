"""kvmem_hip_score_noalloc: the per-token max scorer with the library's
static per-GPU scratch instead of allocated buffers.

Two calls in a row through the C ABI -- the 256K workload (16 layers x 2048
blocks, 64-token bf16 query x 24 heads) and then a smaller one (2 layers x
300 blocks with a partial last block, 8-token f16 query, per-layer scores
left to the scratch) -- each equal bit for bit to kvmem_hip_score on the
same inputs, with no allocation by the context in between.  A call that
needs more scratch than the array holds is refused before any work.  Two
contexts on one GPU share the array in turn; a call from the second while
the first one's call is still queued is refused with KVMEM_HIP_ERR_BUSY
and writes nothing.  A call captured into a HIP graph replays with the
scorer's results for whatever query its buffer holds at each replay.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import workloads  # noqa: E402

T, HKV, HQ, D = 128, 4, 24, 256
E = HKV * D


def announce(msg: str) -> None:
    print(f"[no_alloc] {msg}", flush=True)


def both_scores(ctx, L, B, Tq, q_type, last_T, seed):
    """(scores, layer scores) of kvmem_hip_score and of
    kvmem_hip_score_noalloc on the same seeded inputs."""
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=seed)
    if q_type == kv.TYPE_F16:
        q = q.to(torch.float16)
    torch.cuda.synchronize()
    hist = ctx.make_history(k.data_ptr(), None, L, B, T, E, 0, last_T)
    want = torch.empty(B, dtype=torch.float32, device="cuda")
    want_l = torch.empty((L, B), dtype=torch.float32, device="cuda")
    ctx.score(hist, q.data_ptr(), q_type, Tq, HQ, HKV, D, want.data_ptr(), want_l.data_ptr())
    ctx.sync()
    got = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda")
    got_l = torch.full((L, B), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    before = ctx.scratch_info()["allocations"]
    ctx.score_noalloc(hist, q.data_ptr(), q_type, Tq, HQ, HKV, D, got.data_ptr(), got_l.data_ptr())
    ctx.sync()
    # the layer scores left to the static scratch: same final scores
    got2 = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.score_noalloc(hist, q.data_ptr(), q_type, Tq, HQ, HKV, D, got2.data_ptr())
    ctx.sync()
    assert ctx.scratch_info()["allocations"] == before
    return [t.cpu().numpy() for t in (want, want_l, got, got_l, got2)]


def test_score_noalloc_equals_score_two_calls():
    with kv.Context(0) as ctx:
        for L, B, Tq, q_type, last_T, seed in ((16, 2048, 64, kv.TYPE_BF16, 0, 2),
                                               (2, 300, 8, kv.TYPE_F16, 37, 5)):
            announce(f"L={L} B={B} Tq={Tq} q_type={q_type} last_T={last_T}")
            want, want_l, got, got_l, got2 = both_scores(ctx, L, B, Tq, q_type, last_T, seed)
            assert np.isfinite(want).all()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            assert np.array_equal(got_l.view(np.uint32), want_l.view(np.uint32))
            assert np.array_equal(got2.view(np.uint32), want.view(np.uint32))


def test_score_noalloc_refuses_past_its_scratch():
    """16 layers x 8192 blocks with a 512-token query needs 64 MiB of
    partial maxima: refused on the host, nothing launched."""
    announce("oversized call refused")
    with kv.Context(0) as ctx:
        buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")
        out = torch.zeros(8192, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        hist = ctx.make_history(buf.data_ptr(), None, 16, 8192, T, E, 0)
        with pytest.raises(kv.KvMemError) as ex:
            ctx.score_noalloc(hist, buf.data_ptr(), kv.TYPE_BF16, 512, HQ, HKV, D, out.data_ptr())
        assert ex.value.code == kv.ERR_INVALID and "maximum" in str(ex.value)
        ctx.sync()


def test_score_noalloc_two_contexts_share_then_refuse_overlap():
    announce("two contexts on one GPU: in turn, then overlapping")
    L, B, Tq = 2, 300, 8
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=7)
    busy = torch.cuda.Stream()
    torch.cuda.synchronize()

    def out():
        t = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        return t

    def occupy():
        # about 10 ms of matrix products queued on `busy` ahead of the next call
        with torch.cuda.stream(busy):
            x = torch.ones((4096, 4096), dtype=torch.float16, device="cuda")
            for _ in range(64):
                x = (x @ x) * 1e-3

    with kv.Context(0) as a, kv.Context(0) as b:
        ha = a.make_history(k.data_ptr(), None, L, B, T, E, 0)
        hb = b.make_history(k.data_ptr(), None, L, B, T, E, 0)
        want = out()
        a.score(ha, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, want.data_ptr())
        a.sync()
        want = want.cpu().numpy()
        # in turn: each call waited for before the other context's
        for ctx, h in ((a, ha), (b, hb), (a, ha)):
            got = out()
            ctx.score_noalloc(h, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, got.data_ptr())
            ctx.sync()
            assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
        # overlapping: a's call is queued behind the products, b's is refused
        a.set_stream(busy.cuda_stream)
        occupy()
        got_a, got_b = out(), out()
        a.score_noalloc(ha, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, got_a.data_ptr())
        with pytest.raises(kv.KvMemError) as ex:
            b.score_noalloc(hb, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, got_b.data_ptr())
        assert ex.value.code == kv.ERR_BUSY, str(ex.value)
        busy.synchronize()
        assert np.isnan(got_b.cpu().numpy()).all()          # the refused call wrote nothing
        assert np.array_equal(got_a.cpu().numpy().view(np.uint32), want.view(np.uint32))
        # one context never overlaps itself: set_stream waits for the old stream
        occupy()
        a.score_noalloc(ha, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, got_a.data_ptr())
        a.set_stream(None)
        again = out()
        a.score_noalloc(ha, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, again.data_ptr())
        a.sync()
        assert np.array_equal(again.cpu().numpy().view(np.uint32), want.view(np.uint32))
        # once the work is done, b takes the array
        b.score_noalloc(hb, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, got_b.data_ptr())
        b.sync()
        assert np.array_equal(got_b.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_score_noalloc_under_graph_capture():
    """One call captured into a HIP graph on the context's stream
    (torch.cuda.graph in global capture mode, where an allocation or a
    synchronisation fails the capture), then replayed four times, a new
    query copied into the captured query buffer and the output cleared
    before each replay, eager work and synchronisations in between: every
    replay equals kvmem_hip_score on that query, bit for bit, and the
    context allocates nothing while capturing or replaying."""
    L, B, Tq, last_T = 4, 512, 16, 50
    announce(f"graph capture: L={L} B={B} Tq={Tq} last_T={last_T}")
    k, _, q = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=Tq, seed=11)
    g = torch.Generator(device="cuda")
    g.manual_seed(12)
    queries = [torch.randn(q.shape, generator=g, device="cuda").to(q.dtype) for _ in range(4)]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with kv.Context(0) as ctx:
        ctx.set_stream(stream.cuda_stream)
        hist = ctx.make_history(k.data_ptr(), None, L, B, T, E, 0, last_T)
        out = torch.full((B,), float("nan"), dtype=torch.float32, device="cuda")
        want = torch.empty(B, dtype=torch.float32, device="cuda")
        ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, want.data_ptr())
        ctx.score_noalloc(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, out.data_ptr())
        ctx.sync()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))
        before = ctx.scratch_info()["allocations"]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ctx.score_noalloc(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, out.data_ptr())
        torch.cuda.synchronize()
        for i, qi in enumerate(queries):
            q.copy_(qi)
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            assert ctx.scratch_info()["allocations"] == before
            ctx.score(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, want.data_ptr())
            ctx.sync()
            w = want.cpu().numpy()
            assert np.isfinite(w).all()
            assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), f"replay {i}"
        # eager calls from the capturing context go on as before
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        ctx.score_noalloc(hist, q.data_ptr(), kv.TYPE_BF16, Tq, HQ, HKV, D, out.data_ptr())
        ctx.sync()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))
        del graph
        ctx.set_stream(None)
