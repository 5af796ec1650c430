"""Packed host rows on the GPU: stage-out (pool slots -> pinned host) and the
packed stage-in (pinned host -> pool slots), bit-exact.

The packed host store holds each block as [layer][K rows][V rows] in the
pool's formats.  Stage-out after a quantizing stage-in must give the
oracle's quantized rows at the block's span (only the block's own rows of
a partial block; everything else untouched); a packed stage-in of those
spans into other slots must reproduce the pool bytes; batches spanning
several 32 MiB ring slots keep every block intact.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import workloads  # noqa: E402

T = 128
SENT = 0xA5


def announce(msg: str) -> None:
    print(f"[packed] {msg}", flush=True)
    sys.stdout.flush()


def pinned(nbytes: int, fill: int = SENT):
    t = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    t.fill_(fill)
    return t


def pool_of(ctx, L, n_slots, Ek, Ev, tk, tv, fill=0):
    rk, rv = kv.row_size(tk, Ek), kv.row_size(tv, Ev)
    pk = [torch.full((n_slots * T * rk,), fill, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.full((n_slots * T * rv,), fill, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pool = ctx.make_pool(L, n_slots, T, Ek, Ev, tk, tv, [p.data_ptr() for p in pk], [p.data_ptr() for p in pv])
    return pool, pk, pv, rk, rv


def test_stageout_after_quantize_and_restore(ctx, oracle):
    announce("3 layers x 9 blocks, K q8_0 / V q4_0, partial last block: quantize, stage out, restore")
    L, B, Ek, Ev, last = 3, 9, 1024, 512, 77
    tk, tv = kv.TYPE_Q8_0, kv.TYPE_Q4_0
    Kh = workloads.heavy_tailed(5, (L, B, T, Ek))
    Vh = workloads.heavy_tailed(6, (L, B, T, Ev))
    kd = torch.from_numpy(Kh.view(np.int16)).cuda()
    vd = torch.from_numpy(Vh.view(np.int16)).cuda()
    ids, slots, n_slots = [8, 0, 5, 3], [11, 2, 7, 0], 12
    pool, pk, pv, rk, rv = pool_of(ctx, L, n_slots, Ek, Ev, tk, tv)
    hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), L, B, T, Ek, Ev, last)
    torch.cuda.synchronize()
    ctx.stagein_blocks(hist, pool, ids, slots)
    span = L * T * (rk + rv)
    store = pinned(B * span)
    ph = kv.PackedHost(store.data_ptr(), L, B, T)
    ntok = [last if b == B - 1 else T for b in ids]
    ctx.stageout_blocks(pool, ph, ids, slots, ntok)
    ctx.sync()
    got = store.numpy().reshape(B, L, T * (rk + rv))
    for b in range(B):
        if b not in ids:
            assert (got[b] == SENT).all(), f"block {b} was not staged out but changed"
            continue
        nt = last if b == B - 1 else T
        for l in range(L):
            krun = got[b, l, :T * rk].reshape(T, rk)
            vrun = got[b, l, T * rk:].reshape(T, rv)
            assert np.array_equal(krun[:nt], oracle.quantize_rows_f16(tk, Kh[l, b, :nt])), (b, l)
            assert np.array_equal(vrun[:nt], oracle.quantize_rows_f16(tv, Vh[l, b, :nt])), (b, l)
            assert (krun[nt:] == SENT).all() and (vrun[nt:] == SENT).all()
    # restore the packed rows into other slots of a fresh pool: same bytes as the quantized pool
    pool2, pk2, pv2, _, _ = pool_of(ctx, L, n_slots, Ek, Ev, tk, tv, fill=0x3C)
    slots2 = [1, 9, 4, 6]
    ctx.stagein_packed_host(ph, pool2, ids, slots2, ntok)
    ctx.sync()
    for l in range(L):
        a_k = pk[l].cpu().numpy().reshape(n_slots * T, rk)
        b_k = pk2[l].cpu().numpy().reshape(n_slots * T, rk)
        a_v = pv[l].cpu().numpy().reshape(n_slots * T, rv)
        b_v = pv2[l].cpu().numpy().reshape(n_slots * T, rv)
        for s1, s2, nt in zip(slots, slots2, ntok):
            assert np.array_equal(a_k[s1 * T:s1 * T + nt], b_k[s2 * T:s2 * T + nt])
            assert np.array_equal(a_v[s1 * T:s1 * T + nt], b_v[s2 * T:s2 * T + nt])
            assert (b_k[s2 * T + nt:(s2 + 1) * T] == 0x3C).all()


@pytest.mark.parametrize("memory", ["pinned", "pageable"])
def test_packed_many_ring_batches(ctx, memory):
    """Both directions, 47 blocks of 5.5 MiB.  A pinned store is read and
    written by one copy launch each way; a pageable one goes through batches
    that fill several device-ring slots, with alternating slots reused."""
    announce(f"{memory} store: 4 layers, F16 K 2048 / q8_0 V 1024, 47 blocks each way")
    L, Ek, Ev, n_slots, nb = 4, 2048, 1024, 64, 60
    tk, tv = kv.TYPE_F16, kv.TYPE_Q8_0
    g = torch.Generator(device="cuda").manual_seed(7)
    pool, pk, pv, rk, rv = pool_of(ctx, L, n_slots, Ek, Ev, tk, tv)
    for p in pk + pv:
        p.copy_(torch.randint(0, 256, p.shape, dtype=torch.uint8, device="cuda", generator=g))
    rng = np.random.default_rng(3)
    ids = sorted(rng.choice(nb, 47, replace=False).tolist())
    slots = rng.permutation(n_slots)[:47].tolist()
    span = L * T * (rk + rv)
    if memory == "pinned":
        store = pinned(nb * span)
    else:
        store = torch.from_numpy(np.full(nb * span, SENT, dtype=np.uint8))
    ph = kv.PackedHost(store.data_ptr(), L, nb, T)
    torch.cuda.synchronize()
    ctx.stageout_blocks(pool, ph, ids, slots, [T] * 47)
    ctx.stageout_blocks(pool, ph, ids[:5], slots[:5], [T] * 5)   # a second call reuses the ring
    ctx.sync()
    got = store.numpy().reshape(nb, L, T * (rk + rv))
    for b, s in zip(ids, slots):
        for l in range(L):
            assert np.array_equal(got[b, l, :T * rk], pk[l][s * T * rk:(s + 1) * T * rk].cpu().numpy())
            assert np.array_equal(got[b, l, T * rk:], pv[l][s * T * rv:(s + 1) * T * rv].cpu().numpy())
    pool2, pk2, pv2, _, _ = pool_of(ctx, L, n_slots, Ek, Ev, tk, tv)
    slots2 = rng.permutation(n_slots)[:47].tolist()
    ctx.stagein_packed_host(ph, pool2, ids, slots2, [T] * 47)
    ctx.sync()
    for s1, s2 in zip(slots, slots2):
        for l in range(L):
            assert torch.equal(pk[l][s1 * T * rk:(s1 + 1) * T * rk], pk2[l][s2 * T * rk:(s2 + 1) * T * rk])
            assert torch.equal(pv[l][s1 * T * rv:(s1 + 1) * T * rv], pv2[l][s2 * T * rv:(s2 + 1) * T * rv])


def test_packed_rejects_bad_arguments(ctx):
    announce("packed argument checks")
    L, Ek, Ev, n_slots = 2, 1024, 1024, 4
    pool, pk, pv, rk, rv = pool_of(ctx, L, n_slots, Ek, Ev, kv.TYPE_Q8_0, kv.TYPE_Q8_0)
    store = pinned(3 * L * T * (rk + rv))
    good = kv.PackedHost(store.data_ptr(), L, 3, T)
    cases = [(good, [3], [0], [T]),                                   # block beyond the store
             (good, [0], [n_slots], [T]),                             # slot beyond the pool
             (good, [0], [0], [T + 1]),                               # more rows than a block
             (kv.PackedHost(store.data_ptr(), L + 1, 3, T), [0], [0], [T]),   # layer mismatch
             (kv.PackedHost(store.data_ptr(), L, 3, 64), [0], [0], [64])]     # block size mismatch
    for ph, ids, slots, nt in cases:
        with pytest.raises(kv.KvMemError):
            ctx.stageout_blocks(pool, ph, ids, slots, nt)
        with pytest.raises(kv.KvMemError):
            ctx.stagein_packed_host(ph, pool, ids, slots, nt)
    ctx.sync()
    assert (store.numpy() == SENT).all()


def read_pool(eng, layer, which, rb):
    n = eng.n_slots() * T * rb
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    c = kv.Context(0)
    c.d2d_batched([eng.pool_layer(layer)[which]], [buf.data_ptr()], [n])
    c.sync()
    c.close()
    return buf.cpu().numpy().reshape(eng.n_slots() * T, rb)


def test_engine_packed_store_save_and_restore(oracle):
    """Pinned-host history with a packed store: blocks evicted by a step are
    saved (bytes = the oracle's quantized rows), and selecting them again
    restores them from the packed rows (no quantization) with the same pool
    bytes."""
    from kvmem_amd import host
    announce("engine: pinned host history + packed store, evict then restore")
    L, HQ, HKV, D, nb = 2, 24, 4, 256, 24
    E = HKV * D
    tk, tv = kv.TYPE_Q8_0, kv.TYPE_Q4_0
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=8, seed=91, with_v=True)
    _, _, q2 = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=8, seed=92, with_v=True)
    kk = k.permute(1, 0, 2, 3, 4).reshape(nb, L, T * E)
    vv = v.permute(1, 0, 2, 3, 4).reshape(nb, L, T * E)
    hb = torch.empty((nb, L * 2 * T * E), dtype=torch.float16, pin_memory=True)
    hb.copy_(torch.cat([kk, vv], dim=2).reshape(nb, -1).cpu())
    rk, rv = kv.row_size(tk, E), kv.row_size(tv, E)
    span = L * T * (rk + rv)
    store = pinned(nb * span)
    kb = workloads.to_bits(torch, k)
    vb = workloads.to_bits(torch, v)
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=6, reserve_blocks=2, type_k=tk, type_v=tv) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * T)   # the scorer's keys
        eng.set_host_history(hb.data_ptr(), nb)                           # stage-in source
        eng.set_packed_host(store.data_ptr(), nb)
        sel1 = eng.preview(q.data_ptr(), 8)
        st1 = eng.apply(sel1)
        assert st1["n_saved"] == 0 and st1["n_restored"] == 0
        sel2 = eng.preview(q2.data_ptr(), 8)
        st2 = eng.apply(sel2)
        evicted = sorted(set(sel1.blocks) - set(sel2.blocks))
        assert evicted and st2["n_saved"] == len(evicted)
        got = store.numpy().reshape(nb, L, T * (rk + rv))
        for b in range(nb):
            assert eng.packed_valid(b) == (b in evicted)
            if b not in evicted:
                continue
            for l in range(L):
                assert np.array_equal(got[b, l, :T * rk].reshape(T, rk),
                                      oracle.quantize_rows_f16(tk, kb[l, b].reshape(T, E))), (b, l)
                assert np.array_equal(got[b, l, T * rk:].reshape(T, rv),
                                      oracle.quantize_rows_f16(tv, vb[l, b].reshape(T, E))), (b, l)
        # select the first step's blocks again: the evicted ones come back packed
        st3 = eng.apply(host.Selection(eng.epoch(), eng.total_tokens(), sel1.blocks))
        assert st3["n_restored"] == len(evicted)
        slots = eng.block_slots()
        for l in range(L):
            pk = read_pool(eng, l, 0, rk)
            pv = read_pool(eng, l, 1, rv)
            for b in sel1.blocks:
                s = slots[b]
                assert np.array_equal(pk[s * T:(s + 1) * T], oracle.quantize_rows_f16(tk, kb[l, b].reshape(T, E)))
                assert np.array_equal(pv[s * T:(s + 1) * T], oracle.quantize_rows_f16(tv, vb[l, b].reshape(T, E)))
        # a truncate drops the packed rows of the blocks it cuts
        eng.truncate_to(10 * T + 5)
        assert not any(eng.packed_valid(b) for b in range(10, nb))
