"""Shared set-up of the reselect-engine GPU tests: seeded device history,
engines of the test shape, and the pool check against the oracle's
quantizer."""
from __future__ import annotations

import numpy as np
import torch

from conftest import load_pkg

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

RTOL = 1e-3
L, T, HKV, HQ, D = 2, 128, 4, 24, 256
E = HKV * D


def history(cap: int, seed: int, Tq: int = 8):
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=cap, Tq=Tq, seed=seed, with_v=True)
    torch.cuda.synchronize()
    return k, v, q


def make_engine(budget: int, reserve: int, type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q8_0, **kw):
    return host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                       budget_blocks=budget, reserve_blocks=reserve, type_k=type_k, type_v=type_v,
                       **kw)


def check_pool(eng, oracle, k, v, sel, type_k, type_v, ntok_of=None):
    kb = workloads.to_bits(torch, k)
    vb = workloads.to_bits(torch, v)
    slots = eng.block_slots()
    for layer in range(L):
        for which, src, ty in ((0, kb, type_k), (1, vb, type_v)):
            rb = kv.row_size(ty, E)
            ptr = eng.pool_layer(layer)[which]
            n = eng.n_slots() * T * rb
            buf = torch.empty(n, dtype=torch.uint8, device="cuda")
            c = kv.Context(0)
            c.d2d_batched([ptr], [buf.data_ptr()], [n])
            c.sync()
            c.close()
            pool = buf.cpu().numpy().reshape(eng.n_slots() * T, rb)
            for b in sel:
                s = slots[b]
                assert s >= 0, f"block {b} has no slot"
                nt = T if ntok_of is None else ntok_of(b)
                rows = src[layer, b].reshape(T, E)[:nt]
                want = oracle.quantize_rows_f16(ty, rows)
                got = pool[s * T: s * T + nt]
                assert np.array_equal(got, want), f"layer {layer} {'KV'[which]} block {b} slot {s}"


def oracle_scores(oracle, q, k, n_blocks, last_T=0):
    ls = oracle.score_pertoken_max(q.float().cpu().numpy(), workloads.to_bits(torch, k[:, :n_blocks]),
                                   last_T)
    return oracle.combine_layers(ls, 0)


def block_major_pinned(k, v, n_blocks):
    """[block][layer][K rows, V rows] halves in pinned host memory."""
    kk = k[:, :n_blocks].permute(1, 0, 2, 3, 4).reshape(n_blocks, L, T * E)
    vv = v[:, :n_blocks].permute(1, 0, 2, 3, 4).reshape(n_blocks, L, T * E)
    host_buf = torch.empty((n_blocks, L * 2 * T * E), dtype=torch.float16, pin_memory=True)
    host_buf.copy_(torch.cat([kk, vv], dim=2).reshape(n_blocks, -1).cpu())
    return host_buf


def decode_rows(eng, k, v, begin: int, end: int) -> None:
    """The caller's decode of rows [begin, end): append them resident, then
    write the pool cells of every block they touch (whole blocks, from the
    history that already holds the rows), as llama.cpp writes a batch's
    K/V cells."""
    eng.append_resident(end - begin)
    slots = eng.block_slots()
    ids = list(range(begin // T, (end + T - 1) // T))
    n_blocks = eng.block_count()
    last = eng.total_tokens() - (n_blocks - 1) * T
    c = kv.Context(0)
    hist = c.make_history(k.data_ptr(), v.data_ptr(), L, n_blocks, T, E, E, 0 if last == T else last,
                          k.shape[1])
    pk = [eng.pool_layer(layer)[0] for layer in range(L)]
    pv = [eng.pool_layer(layer)[1] for layer in range(L)]
    pool = c.make_pool(L, eng.n_slots(), T, E, E, eng.params.type_k, eng.params.type_v, pk, pv)
    c.stagein_blocks(hist, pool, ids, [slots[b] for b in ids])
    c.sync()
    c.close()
