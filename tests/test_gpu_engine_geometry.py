"""The reselect engine over other geometries, in random operation sequences.

Mostly 3 layers, 32-token blocks, 8 query heads over 2 KV heads of 128 (GQA
4, 256-element rows), a 4-token bf16 query; also one-token blocks, and
7-token blocks over one KV head of 128 and 5-token blocks over three, whose
slots are not a whole
number of 16 bytes (the stage-in's 2-byte stores, the slot moves' gather
path); pools of q8_0, q5_0, q4_0 and F16
in both slot layouts, the per-token max scorer and the reference's mean-K
scorer, the row transform (NeoX RoPE 128 at the original positions, then
attn_rot: Hadamard 128 on K, 64 on V), and a pinned host history as the only
history.  Each case runs a seeded sequence of previews and applies,
retrievals (device-planned where the engine plans on the device), appended
rows (growing a partial tail), rows decoded into the pool by the caller
(append_resident, then the cells written), truncations to any row, and
request spans with a force_pos.  Checked against the oracle after every
operation:
  - each preview's scores: within 1e-3 relative of the fp64 per-token
    scorer, or within 1e-5 of the oracle's mean-K chain (token-order query
    and key sums, score_retrieval), over the history as it stands;
  - its selection: the oracle's top-k over the engine's scores with the sink
    blocks (the first one, two or none), the blocks retrieval_mandatory
    derives (the span's rows and force_pos's block, as the history stands)
    and the newest `recent` blocks charged first, equal scores going to the
    lower id or, as the reference's rule, to the higher;
  - the resident blocks are exactly the last selection's plus the decoded
    ones, cut to the history, in distinct slots, slot i = the i-th selected
    block in the canonical layout;
  - every resident block's pool rows, up to the rows it held when it was
    staged or decoded, are the oracle's (transformed) quantization of its
    history rows;
  - a decode the free list cannot take, or one behind a grown tail still
    to be staged, is refused with nothing changed.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()
from kvmem_amd import host, workloads  # noqa: E402

GEOM = (3, 32, 8, 2, 128)     # layers, block tokens, query heads, KV heads, head_dim
CAP, TQ = 40, 4
RTOL = 1e-3
# KVMEM_GEOM_OPS / KVMEM_GEOM_SEED_OFFSET lengthen a run or draw other seeds
N_OPS = int(os.environ.get("KVMEM_GEOM_OPS", "120"))
SEED_OFFSET = int(os.environ.get("KVMEM_GEOM_SEED_OFFSET", "0"))
XF = dict(n_rot=128, rope_freq_base=1e6, attn_rot=1)   # attn_rot widths: K 128, V 64
OPS = ["preview_apply", "retrieve", "append", "truncate", "decode", "span"]
WEIGHTS = [0.25, 0.25, 0.12, 0.1, 0.15, 0.13]

CASES = [
    # (canonical layout, type_k, type_v, budget, reserve, seed, scorer, row transform, host history only,
    #  geometry, other engine parameters)
    (1, kv.TYPE_Q8_0, kv.TYPE_Q8_0, 6, 3, 201, 0, False, False, GEOM, {}),
    (0, kv.TYPE_Q4_0, kv.TYPE_Q5_0, 7, 2, 202, 0, False, False, GEOM, {}),
    (1, kv.TYPE_Q5_0, kv.TYPE_Q4_0, 5, 4, 203, 0, False, False, GEOM, {}),
    (1, kv.TYPE_Q8_0, kv.TYPE_F16, 6, 3, 204, 0, False, False, GEOM, {}),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q4_0, 6, 3, 205, 1, False, False, GEOM, {}),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q8_0, 6, 3, 206, 0, True, False, GEOM, {}),
    (1, kv.TYPE_Q5_0, kv.TYPE_Q8_0, 6, 3, 207, 1, False, True, GEOM, {}),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q5_0, 6, 3, 208, 0, False, False, (2, 7, 4, 1, 128), {}),
    (0, kv.TYPE_Q4_0, kv.TYPE_Q8_0, 7, 2, 209, 0, False, False, (2, 7, 4, 1, 128), {}),
    (1, kv.TYPE_Q5_0, kv.TYPE_Q4_0, 6, 3, 210, 1, False, False, (3, 5, 12, 3, 128), {}),
    (1, kv.TYPE_Q8_0, kv.TYPE_Q8_0, 6, 3, 211, 0, False, False, (2, 1, 8, 2, 128), {}),
    (1, kv.TYPE_Q4_0, kv.TYPE_Q4_0, 8, 3, 212, 0, False, False, GEOM,
     {"sink_blocks": 2, "recent_blocks": 2, "tie_lower_index": 0}),
    (0, kv.TYPE_Q8_0, kv.TYPE_Q5_0, 7, 2, 213, 1, False, False, GEOM,
     {"sink_blocks": 0, "recent_blocks": 1, "tie_lower_index": 0}),
]
IDS = ["canonical_q8", "lifo_q4_q5", "canonical_q5_q4", "canonical_q8_f16", "meank_q8_q4", "transform_q8",
       "host_only_meank_q5_q8", "T7_canonical_q8_q5", "T7_lifo_q4_q8", "T5_meank_q5_q4", "T1_canonical_q8",
       "sink2_recent2_higher_ties_q4", "lifo_meank_nosink_recent1_q8_q5"]


def announce(msg: str) -> None:
    print(f"[geometry] {msg}", flush=True)


def read_pool(eng, types, L: int, T: int, E: int) -> list:
    """[layer][K or V] -> the pool tensor's rows on the host."""
    out = []
    ctx = kv.Context(0)
    try:
        for layer in range(L):
            pair = []
            for ptr, ty in zip(eng.pool_layer(layer), types):
                rb = kv.row_size(ty, E)
                n = eng.n_slots() * T * rb
                buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                torch.cuda.synchronize()
                ctx.d2d_batched([ptr], [buf.data_ptr()], [n])
                ctx.sync()
                pair.append(buf.cpu().numpy().reshape(eng.n_slots() * T, rb))
            out.append(pair)
    finally:
        ctx.close()
    return out


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_engine_sequences_other_geometry(oracle, case):
    canon, tk, tv, budget, reserve, seed, scorer, xf, host_only, (L, T, HQ, HKV, D), extra = case
    sink = extra.get("sink_blocks", 1)
    recent = extra.get("recent_blocks", 0)
    lower_ties = bool(extra.get("tie_lower_index", 1))
    E = HKV * D
    announce(f"{N_OPS} operations, canonical={canon}, types {kv.TYPE_NAMES[tk]}/{kv.TYPE_NAMES[tv]}, "
             f"budget {budget} + {reserve}, scorer {scorer}, transform {xf}, host history only {host_only}, "
             f"geometry (L, T, Hq, Hkv, D) = {(L, T, HQ, HKV, D)}, {extra}")
    rng = np.random.default_rng(seed + SEED_OFFSET)
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=CAP, Tq=TQ, seed=seed, T=T, Hkv=HKV, Hq=HQ, D=D,
                                        with_v=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    torch.cuda.synchronize()
    bits = (workloads.to_bits(torch, k), workloads.to_bits(torch, v))
    types = (tk, tv)
    theta = oracle.rope_theta(XF["n_rot"], XF["rope_freq_base"]) if xf else None
    quant: dict = {}
    sums: dict = {}
    pinned = None
    if host_only:
        # block-major [block][layer][K rows, V rows]
        kk = k.permute(1, 0, 2, 3, 4).reshape(CAP, L, T * E)
        vv = v.permute(1, 0, 2, 3, 4).reshape(CAP, L, T * E)
        pinned = torch.empty((CAP, L * 2 * T * E), dtype=torch.float16, pin_memory=True)
        pinned.copy_(torch.cat([kk, vv], dim=2).reshape(CAP, -1).cpu())

    def want(layer: int, which: int, b: int, n: int) -> np.ndarray:
        key = (layer, which, b)
        if key not in quant:
            rows = bits[which][layer, b].reshape(T, E)
            if xf:
                x = oracle.transform_rows(oracle.f16_to_f32(rows).reshape(T, E), D,
                                          XF["n_rot"] if which == 0 else 0, theta,
                                          b * T, 128 if which == 0 else 64)
                quant[key] = oracle.quantize_rows_f32(types[which], x)
            else:
                quant[key] = oracle.quantize_rows_f16(types[which], rows)
        return quant[key][:n]

    def ksum(layer: int, b: int, n: int) -> np.ndarray:
        key = (layer, b, n)
        if key not in sums:
            sums[key] = oracle.meank_sum_f16(bits[0][layer, b].reshape(T, E)[:n])
        return sums[key]

    total = int(rng.integers(8 * T, 20 * T))
    valid: dict[int, int] = {}   # resident block -> rows the pool holds for it
    stale: list = [None]         # the resident block whose pool rows the engine knows are stale
    span = {"qb": -1, "qe": 0, "force": -1}
    counts = {op: 0 for op in OPS}
    hits = {"decode_refused": 0, "span_set": 0, "mandatory_checked": 0, "evicted": 0}
    last_sel: list[int] = []

    def ntok(b: int) -> int:
        return min(T, total - b * T)

    def derived() -> list[int]:
        """retrieval_mandatory as the history stands: the blocks overlapping
        the span's rows in block order, then the block holding force_pos."""
        nb = (total + T - 1) // T
        out = []
        if span["qb"] >= 0:
            out = [b for b in range(nb) if b * T < span["qe"] and b * T + ntok(b) > span["qb"]]
        if 0 <= span["force"] < total:
            out.append(span["force"] // T)
        return out

    def check_scores(q, scores, nb) -> None:
        last_t = total - (nb - 1) * T
        if scorer == 0:
            ref = oracle.combine_layers(oracle.score_pertoken_max(q.float().cpu().numpy(), bits[0][:, :nb],
                                                                  last_t if last_t < T else 0), 0)
            rel = np.abs(scores.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-6)
            assert rel.max() <= RTOL, f"max rel err {rel.max():.3e}"
        else:
            q_sum = oracle.q_accumulate(q.float().cpu().numpy().reshape(L, TQ, -1))
            ks = np.zeros((L, nb, E), np.float32)
            mt = np.zeros((L, nb), np.uint32)
            for b in range(nb):
                for layer in range(L):
                    ks[layer, b] = ksum(layer, b, ntok(b))
                    mt[layer, b] = ntok(b)
            ref = oracle.score_meank(q_sum, [TQ] * L, ks, mt, HQ, HKV, D)
            assert np.max(np.abs(scores.astype(np.float64) - ref)) <= 1e-5

    def decode(eng, begin: int, end: int) -> None:
        """The caller's decode: rows appended resident, then the cells of every
        block they touch written (whole blocks, from the history)."""
        eng.append_resident(end - begin)
        slots = eng.block_slots()
        ids = list(range(begin // T, (end + T - 1) // T))
        nb = eng.block_count()
        last = eng.total_tokens() - (nb - 1) * T
        c = kv.Context(0)
        try:
            pk = [eng.pool_layer(layer)[0] for layer in range(L)]
            pv = [eng.pool_layer(layer)[1] for layer in range(L)]
            pool = c.make_pool(L, eng.n_slots(), T, E, E, tk, tv, pk, pv)
            if host_only:
                hh = kv.HostHistory(pinned.data_ptr(), L, nb, T, E, E, 0 if last == T else last)
                c.stagein_blocks_host(hh, pool, ids, [slots[b] for b in ids])
            else:
                hist = c.make_history(k.data_ptr(), v.data_ptr(), L, nb, T, E, E, 0 if last == T else last, CAP)
                c.stagein_blocks(hist, pool, ids, [slots[b] for b in ids])
            c.sync()
        finally:
            c.close()

    params = dict(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D, budget_blocks=budget,
                  reserve_blocks=reserve, type_k=tk, type_v=tv, canonical_layout=canon, scorer=scorer, **extra)
    if xf:
        params.update(XF)
    with host.Engine(**params) as eng:
        if host_only:
            eng.set_host_history(pinned.data_ptr(), CAP)
            eng.append_tokens(total)
        else:
            eng.set_device_history(k.data_ptr(), v.data_ptr(), CAP, total)
        for step in range(N_OPS):
            op = OPS[int(rng.choice(len(OPS), p=WEIGHTS))]
            if op == "decode" and xf:
                op = "append"   # a transformed pool's decoded cells are the caller's to transform
            what = f"step {step} ({op})"
            nb = (total + T - 1) // T
            if op in ("preview_apply", "retrieve"):
                q = torch.randn((L, TQ, HQ, D), generator=gen, device="cuda").to(torch.bfloat16)
                torch.cuda.synchronize()
                if op == "preview_apply":
                    sel = eng.preview(q.data_ptr(), TQ)
                    chosen = sel.blocks
                    scores = np.array(eng.scores(), dtype=np.float32)
                    eng.apply(sel)
                else:
                    eng.apply_retrieval(q.data_ptr(), TQ)
                    chosen = [b for b, s in enumerate(eng.block_slots()) if s >= 0]
                    scores = np.array(eng.scores(), dtype=np.float32)
                assert scores.size == nb, what
                check_scores(q, scores, nb)
                mand = derived()
                hits["mandatory_checked"] += bool(mand)
                assert chosen == oracle.pick_topk(scores.astype(np.float64), budget, sink=sink, recent=recent,
                                                  mandatory=mand, tie_lower_index=lower_ties), what
                valid = {b: ntok(b) for b in chosen}
                stale[0] = None
                last_sel = chosen
                if canon:
                    slots = eng.block_slots()
                    assert [slots[b] for b in chosen] == list(range(len(chosen))), f"{what}: layout"
            elif op == "append":
                n = min(int(rng.integers(1, 3 * T)), CAP * T - total)
                if n == 0:
                    continue
                tail = (total + T - 1) // T - 1
                if ntok(tail) < T and tail in valid:
                    # the grown tail is the stale block now; an earlier one leaves the pool
                    if stale[0] is not None and stale[0] != tail:
                        valid.pop(stale[0], None)
                        hits["evicted"] += 1
                    stale[0] = tail
                eng.append_tokens(n)
                total += n
            elif op == "truncate":
                total = int(rng.integers(1, total + 1))
                eng.truncate_to(total)
                nb = (total + T - 1) // T
                valid = {b: min(c, ntok(b)) for b, c in valid.items() if b < nb}
                if stale[0] is not None and stale[0] >= nb:
                    stale[0] = None
            elif op == "decode":
                n = min(int(rng.integers(1, 2 * T)), CAP * T - total)
                if n == 0:
                    continue
                before = (list(eng.block_slots()), eng.total_tokens())
                tail = (total + T - 1) // T - 1
                gets_slot = total % T != 0 and tail not in valid   # a partial tail taking a slot
                try:
                    decode(eng, total, total + n)
                except kv.KvMemError as ex:
                    assert ex.code in (kv.ERR_NOMEM, kv.ERR_UNSUPPORTED), (what, str(ex))
                    assert (list(eng.block_slots()), eng.total_tokens()) == before, f"{what}: refused, yet changed"
                    hits["decode_refused"] += 1
                else:
                    begin = total
                    total += n
                    for b in range(begin // T, (total + T - 1) // T):
                        valid[b] = ntok(b)
                    if gets_slot:
                        stale[0] = tail
            else:
                if rng.random() < 0.3:
                    span = {"qb": -1, "qe": 0, "force": -1}
                    eng.set_request_span(-1)
                else:
                    qb = int(rng.integers(0, total))
                    force = int(rng.integers(0, total)) if rng.random() < 0.6 else -1
                    span = {"qb": qb, "qe": qb + int(rng.integers(1, T + 1)), "force": force}
                    eng.set_request_span(span["qb"], span["qe"], span["force"])
                    hits["span_set"] += 1
            counts[op] += 1
            assert eng.total_tokens() == total and eng.block_count() == (total + T - 1) // T, what
            assert eng.retrieval_mandatory() == derived(), (what, eng.retrieval_mandatory(), derived())
            slots = eng.block_slots()
            resident = {b: s for b, s in enumerate(slots) if s >= 0}
            assert set(resident) == set(valid), f"{what}: resident {sorted(resident)} vs {sorted(valid)}"
            assert len(set(resident.values())) == len(resident), f"{what}: shared slots"
            pool = read_pool(eng, types, L, T, E)
            for b, s in resident.items():
                n = valid[b]
                for layer in range(L):
                    for which in (0, 1):
                        got = pool[layer][which][s * T: s * T + n]
                        assert np.array_equal(got, want(layer, which, b, n)), \
                            f"{what}: layer {layer} {'KV'[which]} block {b} slot {s}"
    announce(f"operations {counts}; {hits}; last selection {last_sel}")
