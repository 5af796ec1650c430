"""Stage-in quantize-scatter on the GPU vs the oracle: bit-exact pool bytes.

Covers the single-layer q8_0 stage-in workload (64 blocks x 128 tokens x
4 heads x 256, outlier channels, seeded slot permutation), heavy-tailed
q4_0 / q5_0 / q8_0 / F16, partial last blocks, strided op sources, crafted
special groups (zeros, -0, half-way codes, first-index sign ties, f16
extremes, subnormal scales) and that untouched pool rows keep their bytes.
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

SENTINEL = 0xA5
TYPES = [kv.TYPE_Q8_0, kv.TYPE_Q5_0, kv.TYPE_Q4_0, kv.TYPE_F16]


def dev_bits(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def new_pool(n_slots: int, T: int, row_bytes: int):
    return torch.full((n_slots * T * row_bytes,), SENTINEL, dtype=torch.uint8, device="cuda")


def expected_pool(oracle, type_, blocks: np.ndarray, slots, n_slots, T, ntoks=None):
    """Sentinel pool with block i's rows quantized at slot slots[i]."""
    E = blocks.shape[-1]
    rb = oracle.row_bytes(type_, E)
    out = np.full((n_slots * T, rb), SENTINEL, dtype=np.uint8)
    for i, s in enumerate(slots):
        nt = T if ntoks is None else ntoks[i]
        out[s * T: s * T + nt] = oracle.quantize_rows_f16(type_, blocks[i, :nt])
    return out


def first_diff(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.flatnonzero(a.ravel() != b.ravel())
    if idx.size == 0:
        return "identical"
    i = int(idx[0])
    return f"{idx.size} bytes differ; first at byte {i}: got {a.ravel()[i]:#x} want {b.ravel()[i]:#x}"


def announce(msg: str) -> None:
    print(f"[stagein] {msg}", flush=True)
    sys.stdout.flush()


def test_stagein_1layer_q8_0_bit_exact(ctx, oracle):
    announce("1-layer q8_0 stage-in, 64 blocks -> permuted slots of 256")
    K, V, slots = workloads.stagein_1layer(seed=1)
    nb, T, E = K.shape
    kd, vd = dev_bits(K), dev_bits(V)
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    pk, pv = new_pool(256, T, rb), new_pool(256, T, rb)
    hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), 1, nb, T, E, E)
    pool = ctx.make_pool(1, 256, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [pk.data_ptr()], [pv.data_ptr()])
    torch.cuda.synchronize()
    ctx.stagein_blocks(hist, pool, list(range(nb)), slots.tolist())
    ctx.sync()
    for name, src, p in (("K", K, pk), ("V", V, pv)):
        got = p.cpu().numpy().reshape(256 * T, rb)
        want = expected_pool(oracle, kv.TYPE_Q8_0, src, slots, 256, T)
        assert np.array_equal(got, want), f"{name}: {first_diff(got, want)}"


@pytest.mark.parametrize("type_", TYPES)
def test_stagein_heavy_tailed_multilayer_partial(ctx, oracle, type_):
    announce(f"heavy-tailed 3-layer stage-in type={type_}, partial last block")
    L, B, T, Ek, Ev = 3, 9, 128, 1024, 512
    last = 77
    Kh = workloads.heavy_tailed(11 + type_, (L, B, T, Ek))
    Vh = workloads.heavy_tailed(31 + type_, (L, B, T, Ev))
    ids = [8, 0, 5, 3]           # includes the partial last block
    n_slots = 12
    slots = [11, 2, 7, 0]
    kd, vd = dev_bits(Kh), dev_bits(Vh)
    rbk, rbv = kv.row_size(type_, Ek), kv.row_size(type_, Ev)
    pks = [new_pool(n_slots, T, rbk) for _ in range(L)]
    pvs = [new_pool(n_slots, T, rbv) for _ in range(L)]
    hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), L, B, T, Ek, Ev, last)
    pool = ctx.make_pool(L, n_slots, T, Ek, Ev, type_, type_, [p.data_ptr() for p in pks],
                         [p.data_ptr() for p in pvs])
    torch.cuda.synchronize()
    ctx.stagein_blocks(hist, pool, ids, slots)
    ctx.sync()
    ntoks = [last if b == B - 1 else T for b in ids]
    for l in range(L):
        for name, src, p, rb in (("K", Kh, pks[l], rbk), ("V", Vh, pvs[l], rbv)):
            got = p.cpu().numpy().reshape(n_slots * T, rb)
            want = expected_pool(oracle, type_, src[l][ids], slots, n_slots, T, ntoks)
            assert np.array_equal(got, want), f"layer {l} {name}: {first_diff(got, want)}"


@pytest.mark.parametrize("T,E,type_,had", [
    (7, 96, kv.TYPE_Q8_0, 0),     # 21 groups per slot
    (100, 160, kv.TYPE_Q5_0, 0),  # 500 groups per slot
    (1, 32, kv.TYPE_Q4_0, 0),     # one group per slot
    (13, 96, kv.TYPE_F16, 0),     # F16 slots stay 16-byte aligned
    (5, 192, kv.TYPE_Q8_0, 64),   # the 64-elements-per-lane transform kernel, 30 groups per slot
    (3, 64, kv.TYPE_Q4_0, 64),    # 6 groups per slot, one partial lane unit
])
def test_stagein_slots_not_16_byte_aligned(ctx, oracle, T, E, type_, had):
    """Block lengths and row widths whose slots are not a whole number of 16
    bytes (block_tokens x groups per row not a multiple of 8), so slots start
    2-byte aligned: every staged block's rows bit-exact at its slot, the
    partial last block included, and every other pool byte untouched, with
    and without a Hadamard rotation (64-wide, the 64-elements-per-lane
    kernel)."""
    announce(f"unaligned slots: T={T} E={E} type={type_} hadamard={had}")
    L, B, n_slots = 2, 6, 9
    last = max(1, T - 3) if T > 1 else 0
    rng = np.random.default_rng(T * 31 + E)
    K = workloads.f16_bits((rng.standard_normal((L, B, T, E)) * 2).astype(np.float32))
    V = workloads.f16_bits(rng.standard_normal((L, B, T, E)).astype(np.float32))
    ids, slots = [5, 0, 3, 1], [8, 1, 4, 6]   # block 5: the partial last one
    kd, vd = dev_bits(K), dev_bits(V)
    rb = kv.row_size(type_, E)
    pks = [new_pool(n_slots, T, rb) for _ in range(L)]
    pvs = [new_pool(n_slots, T, rb) for _ in range(L)]
    xf = ctx.make_transform(64, 0, None, had, had) if had else None
    hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), L, B, T, E, E, last)
    pool = ctx.make_pool(L, n_slots, T, E, E, type_, type_, [p.data_ptr() for p in pks],
                         [p.data_ptr() for p in pvs], xf)
    torch.cuda.synchronize()
    ctx.stagein_blocks(hist, pool, ids, slots)
    ctx.sync()
    ntoks = [last if (b == B - 1 and last) else T for b in ids]
    for layer in range(L):
        for name, src, p in (("K", K, pks[layer]), ("V", V, pvs[layer])):
            got = p.cpu().numpy().reshape(n_slots * T, rb)
            want = np.full((n_slots * T, rb), SENTINEL, dtype=np.uint8)
            for b, s, nt in zip(ids, slots, ntoks):
                rows = src[layer, b, :nt]
                if had:
                    x = oracle.transform_rows(oracle.f16_to_f32(rows).reshape(nt, E), 64, 0, None, 0, had)
                    want[s * T: s * T + nt] = oracle.quantize_rows_f32(type_, x)
                else:
                    want[s * T: s * T + nt] = oracle.quantize_rows_f16(type_, rows)
            assert np.array_equal(got, want), f"layer {layer} {name}: {first_diff(got, want)}"


def special_rows(E: int = 1024) -> np.ndarray:
    """128 rows of crafted groups (f16 bits), remaining groups random."""
    rng = np.random.default_rng(7)
    rows = workloads.f16_bits(rng.standard_normal((128, E), dtype=np.float32))
    groups = []
    groups.append(np.zeros(32, np.float32))                                 # all zero
    g = np.zeros(32, np.float32); g[0] = -0.0; groups.append(g)             # -0 first
    g = np.zeros(32, np.float32)
    g[:8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5]; groups.append(g)  # q8 half-way
    g = np.zeros(32, np.float32); g[2] = -3.0; g[5] = 3.0; groups.append(g)  # sign tie, neg first
    g = np.zeros(32, np.float32); g[2] = 3.0; g[5] = -3.0; groups.append(g)  # sign tie, pos first
    g = np.zeros(32, np.float32); g[31] = -8.0; g[0] = 7.5; g[1] = 0.5; g[2] = -0.5; groups.append(g)
    g = np.zeros(32, np.float32); g[31] = -16.0; g[:6] = [15.5, 0.5, -0.5, 1.5, 7.5, -15.5]; groups.append(g)
    g = np.zeros(32, np.float32); g[3] = 65504.0; g[4] = -65504.0; g[5] = 1.0; groups.append(g)
    gb = np.zeros(32, np.uint16); gb[9] = 0x0001                             # 2^-24 only
    gb_rows = [gb]
    gb = np.zeros(32, np.uint16); gb[0] = 0x8001; gb[1] = 0x0001; gb_rows.append(gb)  # +-min subnormal
    gb = (rng.integers(0, 0x0400, 32)).astype(np.uint16); gb_rows.append(gb)          # subnormal group
    g = (rng.standard_normal(32) * 1e-6).astype(np.float32); groups.append(g)        # tiny scale
    g = np.full(32, 0.75, np.float32); groups.append(g)                               # constant
    g = np.full(32, -1.0, np.float32); g[::2] = 1.0; groups.append(g)                 # +-1 alternating
    groups.append(np.arange(-16, 16, dtype=np.float32))                               # every q5 code
    g = np.full(32, -5.0, np.float32); g[0], g[3], g[20] = -16.0, 2.0, 7.0; groups.append(g)  # q5 qh bits 3, 20
    g = np.zeros(32, np.float32); g[16], g[17], g[1] = 16.0, -15.0, -3.0; groups.append(g)    # q5 d < 0
    all_groups = [workloads.f16_bits(x) for x in groups] + gb_rows
    for i, gbits in enumerate(all_groups):
        r, c = divmod(i, E // 32)
        rows[r, c * 32:(c + 1) * 32] = gbits
        # the same group again at the last column of a later row
        rows[64 + i, E - 32:] = gbits
    return rows


@pytest.mark.parametrize("type_", TYPES)
def test_stagein_special_groups(ctx, oracle, type_):
    announce(f"special groups type={type_}")
    rows = special_rows()
    T, E = rows.shape
    src = dev_bits(rows)
    rb = kv.row_size(type_, E)
    out = torch.full((T * rb,), SENTINEL, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ctx.stagein_quant([(src.data_ptr(), out.data_ptr(), T, E, type_)])
    ctx.sync()
    got = out.cpu().numpy().reshape(T, rb)
    want = oracle.quantize_rows_f16(type_, rows)
    assert np.array_equal(got, want), first_diff(got, want)


def test_stagein_q5_0_literal_bytes(ctx):
    """The kernel's q5_0 blocks equal literal bytes worked out from ggml's
    published block_q5_0 layout and dequantizer (no oracle involved)."""
    from q5_literals import q5_literal_failures
    announce("q5_0 literal blocks (qh bit order, qs nibble pairing)")

    def quantize(rows):
        src = dev_bits(rows)
        out = torch.full((rows.shape[0] * 22 * (rows.shape[1] // 32),), SENTINEL, dtype=torch.uint8,
                         device="cuda")
        torch.cuda.synchronize()
        ctx.stagein_quant([(src.data_ptr(), out.data_ptr(), rows.shape[0], rows.shape[1],
                            kv.TYPE_Q5_0)])
        ctx.sync()
        return out.cpu().numpy().reshape(rows.shape[0], -1)

    assert q5_literal_failures(quantize) == []


def test_stagein_ops_strided_mixed_types(ctx, oracle):
    announce("op list: strided sources, mixed types in one call")
    rng = np.random.default_rng(3)
    E = 512
    buf = workloads.f16_bits(rng.standard_normal((40, 2 * E), dtype=np.float32) * 3)
    src = dev_bits(buf)
    stride = 2 * E * 2
    outs, ops, want = [], [], []
    for i, (type_, r0, nr) in enumerate([(kv.TYPE_Q8_0, 0, 17), (kv.TYPE_Q4_0, 5, 33),
                                         (kv.TYPE_Q5_0, 3, 1), (kv.TYPE_F16, 9, 31),
                                         (kv.TYPE_Q8_0, 20, 20)]):
        rb = kv.row_size(type_, E)
        o = torch.full((nr * rb,), SENTINEL, dtype=torch.uint8, device="cuda")
        outs.append(o)
        col = (i % 2) * E          # left or right half of each row
        ops.append((src.data_ptr() + r0 * stride + col * 2, o.data_ptr(), nr, E, type_, stride))
        want.append(oracle.quantize_rows_f16(type_, buf[r0:r0 + nr, col:col + E]))
    torch.cuda.synchronize()
    ctx.stagein_quant(ops)
    ctx.sync()
    for o, w in zip(outs, want):
        got = o.cpu().numpy().reshape(w.shape)
        assert np.array_equal(got, w), first_diff(got, w)


def test_stagein_full_256k_sampled(ctx, oracle):
    """The benchmark's stage-in at full size: 77 random blocks of the 16-layer
    x 2048-block history (16 GiB of F16 K and V on the device) into random
    slots of a 384-slot q8_0 pool, one launch.  Eight sampled blocks are
    checked bit for bit against the oracle quantizer in every layer, K and
    V; every other staged block's rows must have been written (the pool
    starts as a sentinel no q8_0 row of these values can equal)."""
    announce("full-size stage-in: 77 of 2048 blocks x 16 layers, K/V q8_0 -> 384 slots")
    L, B, T, E, n_slots = 16, 2048, 128, 1024, 384
    k, v, _ = workloads.scoring_tensors(torch, "cuda", L=L, B=B, Tq=1, seed=12, with_v=True)
    rng = np.random.default_rng(13)
    ids = sorted(rng.choice(B, 77, replace=False).tolist())
    slots = rng.permutation(n_slots)[:77].tolist()
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    pk = [torch.full((n_slots * T * rb,), 0xFF, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pv = [torch.full((n_slots * T * rb,), 0xFF, dtype=torch.uint8, device="cuda") for _ in range(L)]
    hist = ctx.make_history(k.data_ptr(), v.data_ptr(), L, B, T, E, E)
    pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p.data_ptr() for p in pk],
                         [p.data_ptr() for p in pv])
    torch.cuda.synchronize()
    ctx.stagein_blocks(hist, pool, ids, slots)
    ctx.sync()
    sample = set(rng.choice(77, 8, replace=False).tolist())
    for l in range(L):
        for src, p in ((k, pk[l]), (v, pv[l])):
            got = p.cpu().numpy().reshape(n_slots, T, rb)
            for i, (b, s_) in enumerate(zip(ids, slots)):
                if i in sample:
                    rows = src[l, b].reshape(T, E).cpu().view(torch.int16).numpy().view(np.uint16)
                    assert np.array_equal(got[s_], oracle.quantize_rows_f16(kv.TYPE_Q8_0, rows)), (l, b)
                else:
                    assert not (got[s_] == 0xFF).all(axis=1).any(), (l, b)
    del k, v


def test_stagein_rejects_bad_arguments(ctx):
    announce("argument validation")
    a = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(kv.KvMemError):
        ctx.stagein_quant([(a.data_ptr() + 2, a.data_ptr(), 1, 64, kv.TYPE_Q8_0)])  # misaligned
    with pytest.raises(kv.KvMemError):
        ctx.stagein_quant([(a.data_ptr(), a.data_ptr(), 1, 48, kv.TYPE_Q8_0)])      # n_embd % 32
    with pytest.raises(kv.KvMemError):
        ctx.stagein_quant([(a.data_ptr(), a.data_ptr(), 1, 64, 3)])                 # q4_1
    hist = ctx.make_history(a.data_ptr(), None, 1, 1, 1, 64, 0)
    pool = ctx.make_pool(1, 2, 1, 64, 0, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [a.data_ptr()], None)
    with pytest.raises(kv.KvMemError):
        ctx.stagein_blocks(hist, pool, [0], [2])                                    # slot range
    with pytest.raises(kv.KvMemError):
        ctx.stagein_blocks(hist, pool, [1], [0])                                    # block range


def test_move_slots_overlapping(ctx):
    announce("move_slots with overlapping source/destination slots")
    L, n_slots, T, E = 2, 8, 16, 256
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    pk = [torch.randint(0, 256, (n_slots * T * rb,), dtype=torch.uint8, device="cuda", generator=g)
          for _ in range(L)]
    pv = [torch.randint(0, 256, (n_slots * T * rb,), dtype=torch.uint8, device="cuda", generator=g)
          for _ in range(L)]
    before_k = [p.cpu().numpy().reshape(n_slots, -1).copy() for p in pk]
    before_v = [p.cpu().numpy().reshape(n_slots, -1).copy() for p in pv]
    pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0,
                         [p.data_ptr() for p in pk], [p.data_ptr() for p in pv])
    src, dst = [1, 2, 3, 6], [0, 1, 2, 3]     # a left shift chain + a jump
    torch.cuda.synchronize()
    ctx.move_slots(pool, src, dst)
    ctx.sync()
    for l in range(L):
        for before, p in ((before_k[l], pk[l]), (before_v[l], pv[l])):
            want = before.copy()
            for s, d in zip(src, dst):
                want[d] = before[s]
            got = p.cpu().numpy().reshape(n_slots, -1)
            assert np.array_equal(got, want)


def test_move_slots_null_layer_refused_unaligned_layers_moved(ctx):
    announce("move_slots: a null V layer is refused; layers at 2-byte offsets move by gather/scatter")
    L, n_slots, T, E = 2, 8, 16, 256
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    span = n_slots * T * rb
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    raw = [torch.randint(0, 256, (span + 16,), dtype=torch.uint8, device="cuda", generator=g)
           for _ in range(2 * L)]
    ptrs = [r.data_ptr() + 2 for r in raw]  # every layer tensor 2 bytes past 16-byte alignment
    null_v = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, ptrs[:L], [ptrs[L], 0])
    torch.cuda.synchronize()
    with pytest.raises(kv.KvMemError):
        ctx.move_slots(null_v, [1], [0])
    before = [r.cpu().numpy()[2:2 + span].reshape(n_slots, -1).copy() for r in raw]
    pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, ptrs[:L], ptrs[L:])
    src, dst = [1, 2, 3, 5, 0], [0, 1, 2, 3, 5]     # a chain and a cycle through slot 0
    ctx.move_slots(pool, src, dst)
    ctx.sync()
    for i, r in enumerate(raw):
        out = r.cpu().numpy()
        want = before[i].copy()
        for s, d in zip(src, dst):
            want[d] = before[i][s]
        assert np.array_equal(out[2:2 + span].reshape(n_slots, -1), want)


def move_case(case: str, n_slots: int, rng):
    """(src, dst) slot lists: long chains, cycles, or a set with a shared
    source (which takes the gather/scatter path)."""
    perm = rng.permutation(n_slots).tolist()
    if case == "chains":      # one chain of 39 moves (five segments) and two short ones
        chain = [(perm[i], perm[i + 1]) for i in range(39)]
        chain += [(perm[41], perm[42]), (perm[42], perm[43]), (perm[45], perm[46])]
        return [a for a, _ in chain], [b for _, b in chain]
    if case == "cycles":      # cycles of 20, 3 and 2, and two self-moves
        moves = [(perm[i], perm[(i + 1) % 20]) for i in range(20)]
        moves += [(perm[20 + i], perm[20 + (i + 1) % 3]) for i in range(3)]
        moves += [(perm[23], perm[24]), (perm[24], perm[23]), (perm[30], perm[30]), (perm[31], perm[31])]
        order = rng.permutation(len(moves))
        return [moves[i][0] for i in order], [moves[i][1] for i in order]
    src = perm[:12] + [perm[0]]            # slot perm[0] copied to two places
    dst = perm[12:24] + [perm[40]]
    return src, dst


@pytest.mark.parametrize("E", [256, 32])
@pytest.mark.parametrize("case", ["chains", "cycles", "shared_source"])
def test_move_slots_chains_and_cycles(ctx, case, E):
    """Slot moves equal gathering every source first and scattering in
    order, for chains longer than one segment, cycles, self-moves and
    partial token counts (K q8_0 and V q4_0 rows of different widths; at
    n_embd 32 the rows are 34 and 18 bytes, which takes the gather/scatter
    path even for chains)."""
    announce(f"move_slots {case}, n_embd {E}")
    L, n_slots, T = 3, 64, 16
    rng = np.random.default_rng({"chains": 1, "cycles": 2, "shared_source": 3}[case])
    tk, tv = kv.TYPE_Q8_0, kv.TYPE_Q4_0
    rk, rv = kv.row_size(tk, E), kv.row_size(tv, E)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    pk = [torch.randint(0, 256, (n_slots * T * rk,), dtype=torch.uint8, device="cuda", generator=g)
          for _ in range(L)]
    pv = [torch.randint(0, 256, (n_slots * T * rv,), dtype=torch.uint8, device="cuda", generator=g)
          for _ in range(L)]
    pool = ctx.make_pool(L, n_slots, T, E, E, tk, tv, [p.data_ptr() for p in pk], [p.data_ptr() for p in pv])
    src, dst = move_case(case, n_slots, rng)
    ntok = [int(x) for x in rng.integers(0, T + 1, len(src))]
    ntok[:3] = [T, T, 0]
    before = [(p.cpu().numpy().reshape(n_slots, T, -1).copy()) for p in pk + pv]
    torch.cuda.synchronize()
    ctx.move_slots(pool, src, dst, ntok)
    ctx.sync()
    for b, p in zip(before, pk + pv):
        want = b.copy()
        gathered = [b[s_, :nt].copy() for s_, nt in zip(src, ntok)]
        for d, nt, rows in zip(dst, ntok, gathered):
            want[d, :nt] = rows
        assert np.array_equal(p.cpu().numpy().reshape(n_slots, T, -1), want)


def test_move_slots_pool_beyond_16_bit_slots(ctx):
    """A pool of 70 000 slots: the chain kernel's segment records switch
    from 16-bit to 32-bit entries.  A shift chain across slot 65 535 (two
    segments), a chain between far slots and a 3-cycle through slots above
    65 535, with partial token counts: the result equals gathering every
    source first and scattering in order."""
    announce("move_slots over 70 000 slots (32-bit chain records)")
    L, n_slots, T, E = 2, 70000, 2, 256
    rng = np.random.default_rng(71)
    rb = kv.row_size(kv.TYPE_Q8_0, E)
    g = torch.Generator(device="cuda")
    g.manual_seed(71)
    layers = [torch.randint(0, 256, (n_slots * T * rb,), dtype=torch.uint8, device="cuda", generator=g)
              for _ in range(2 * L)]
    pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p.data_ptr() for p in layers[:L]],
                         [p.data_ptr() for p in layers[L:]])
    shift = list(range(65530, 65546))                      # slot i+1 -> slot i
    src, dst = shift[1:], shift[:-1]
    far = rng.choice(np.arange(100, 65000), 10, replace=False).tolist() + [69990, 66001, 65999]
    far = rng.permutation(far).tolist()                    # a chain far[0] <- far[1] <- ...
    src += far[1:]
    dst += far[:-1]
    src += [69999, 7, 66500]                               # a 3-cycle
    dst += [7, 66500, 69999]
    assert len(set(src)) == len(src) and len(set(dst)) == len(dst)
    ntok = [int(x) for x in rng.integers(0, T + 1, len(src))]
    ntok[:2] = [T, 0]
    before = [p.cpu().numpy().reshape(n_slots, T, rb).copy() for p in layers]
    torch.cuda.synchronize()
    ctx.move_slots(pool, src, dst, ntok)
    ctx.sync()
    for b, p in zip(before, layers):
        want = b.copy()
        gathered = [b[s_, :nt].copy() for s_, nt in zip(src, ntok)]
        for d, nt, rows in zip(dst, ntok, gathered):
            want[d, :nt] = rows
        assert np.array_equal(p.cpu().numpy().reshape(n_slots, T, rb), want)
    del layers
    torch.cuda.empty_cache()


def test_scale_shortcuts_exhaustive(ctx):
    """The quantizers' division-free scale arithmetic equals the IEEE
    quotients over every float of its range, on this device."""
    announce("scale arithmetic: a/127 over all non-negative floats, 1/d over all normal |d| <= 2^126")
    div, rec = ctx.check_scale_arith()
    assert (div, rec) == (0, 0)
