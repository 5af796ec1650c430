"""The mixed-precision and planted-recall workloads at test size.

Mixed precision (Student-t nu = 4 history, all 16 layers, 4 KV heads x 256,
a 96-block slice of the history): run A stages K as q8_0 and V as q4_0, run
B stages K and V as q5_0 with a 96-block generation reserve; every staged
block's pool rows are compared bit-exact with the oracle's quantizers.

Planted recall (4 layers x 1024 blocks, 512-token query, 32 blocks planted
with Zipf-weighted query directions, budget 128): every planted block is
selected, and the selection equals the oracle's top-k over the engine's
own scores.
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
    print(f"[configs] {msg}", flush=True)


def pool_bytes(eng, layer: int, which: int, type_) -> np.ndarray:
    ptr = eng.pool_layer(layer)[which]
    rb = kv.row_size(type_, E)
    n = eng.n_slots() * T * rb
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    c = kv.Context(0)
    c.d2d_batched([ptr], [buf.data_ptr()], [n])
    c.sync()
    c.close()
    return buf.cpu().numpy().reshape(eng.n_slots() * T, rb)


@pytest.mark.parametrize("tk,tv,budget,reserve", [(kv.TYPE_Q8_0, kv.TYPE_Q4_0, 24, 16),
                                                  (kv.TYPE_Q5_0, kv.TYPE_Q5_0, 24, 12)])
def test_mixed_precision_16_layers_bit_exact(oracle, tk, tv, budget, reserve):
    announce(f"Student-t history, 16 layers x 96 blocks, K type {tk} / V type {tv}")
    L, nb = 16, 96
    k, v, q = workloads.student_t_tensors(torch, "cuda", L=L, B=nb, Tq=16, seed=40 + tk)
    torch.cuda.synchronize()
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=budget, reserve_blocks=reserve, type_k=tk, type_v=tv) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * T)
        sel = eng.preview(q.data_ptr(), q.shape[1])
        st = eng.apply(sel)
        assert st["n_staged"] == budget
        kb, vb = workloads.to_bits(torch, k), workloads.to_bits(torch, v)
        slots = eng.block_slots()
        for layer in range(L):
            for which, src, ty in ((0, kb, tk), (1, vb, tv)):
                pool = pool_bytes(eng, layer, which, ty)
                for b in sel.blocks:
                    s = slots[b]
                    want = oracle.quantize_rows_f16(ty, src[layer, b].reshape(T, E))
                    assert np.array_equal(pool[s * T:(s + 1) * T], want), (layer, which, b)


def test_planted_blocks_recalled(oracle):
    announce("planted recall: 4 layers x 1024 blocks, 512-token query, 32 planted, budget 128")
    L, nb, tq, budget = 4, 1024, 512, 128
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=tq, seed=8, with_v=True)
    planted = workloads.plant_blocks(torch, k, q, n_planted=32, seed=5)
    torch.cuda.synchronize()
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=budget, reserve_blocks=16) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * T)
        sel = eng.preview(q.data_ptr(), tq)
        scores = np.array(eng.scores(), dtype=np.float64)
        assert sel.blocks == oracle.pick_topk(scores.astype(np.float32).astype(np.float64), budget, sink=1)
        missing = [int(b) for b in planted if int(b) not in set(sel.blocks)]
        assert not missing, f"planted blocks not recalled: {missing}"
        # scores of a few planted and unplanted blocks against the fp64 oracle
        ids = np.array(sorted(list(planted[:3]) + [1, 500, 1023]), dtype=np.uint32)
        ksub = workloads.to_bits(torch, k[:, torch.from_numpy(ids.astype(np.int64)).cuda()])
        want = oracle.combine_layers(oracle.score_pertoken_max(q.float().cpu().numpy(), ksub), 0)
        got = scores[ids]
        assert np.all(np.abs(got - want) <= 1e-3 * np.maximum(np.abs(want), 1e-6))
