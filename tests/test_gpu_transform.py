"""Stage-in with the cache row transform on the GPU vs the oracle:
bit-exact pool bytes.

The oracle widens each staged block's F16 rows, RoPEs K at the block's
positions (the library's own sin/cos), rotates K and V with the attn_rot
Walsh-Hadamard transform and quantizes the fp32 rows; the kernel does the
same arithmetic in registers.  Covers K q8_0/q4_0/q5_0/F16 with V q8_0/
q5_0/q4_0, head_dim 256 (full rotary, widths 256 / 64) and 128 (partial
rotary 64, width 128 whose scale 1/sqrtf(128) is inexact), default and
explicit positions up to 2^20, a partial last block, RoPE only, Hadamard
only, the pinned-host path, and the argument checks.
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
SENTINEL = 0x5A


def announce(msg: str) -> None:
    print(f"[transform] {msg}", flush=True)
    sys.stdout.flush()


def dev_bits(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.view(np.float16).astype(np.float32)


def expected_rows(oracle, type_, bits, head_dim, n_rot, theta, pos0, width):
    x = oracle.transform_rows(f16_to_f32(bits), head_dim, n_rot, theta, pos0, width)
    return oracle.quantize_rows_f32(type_, x)


def first_diff(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.flatnonzero(a.ravel() != b.ravel())
    if idx.size == 0:
        return "identical"
    i = int(idx[0])
    return f"{idx.size} bytes differ; first at byte {i}: got {a.ravel()[i]:#x} want {b.ravel()[i]:#x}"


def run_case(ctx, oracle, *, L, B, Hkv, D, type_k, type_v, n_rot, had_k, had_v, ids, slots,
             n_slots, last=0, pos0=None, seed=0, host=False):
    E = Hkv * D
    rng = np.random.default_rng(seed)
    Kh = workloads.heavy_tailed(seed + 1, (L, B, T, E))
    Vh = (rng.standard_normal((L, B, T, E)) * 2).astype(np.float16).view(np.uint16)
    theta = oracle.rope_theta(n_rot, 1e6) if n_rot else None
    xf = ctx.make_transform(D, n_rot, theta, had_k, had_v, pos0)
    rbk, rbv = kv.row_size(type_k, E), kv.row_size(type_v, E)
    pks = [torch.full((n_slots * T * rbk,), SENTINEL, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pvs = [torch.full((n_slots * T * rbv,), SENTINEL, dtype=torch.uint8, device="cuda") for _ in range(L)]
    pool = ctx.make_pool(L, n_slots, T, E, E, type_k, type_v, [p.data_ptr() for p in pks],
                         [p.data_ptr() for p in pvs], xf)
    if host:
        span = L * T * 2 * E
        blk = np.concatenate([Kh.transpose(1, 0, 2, 3).reshape(B, L, T * E),
                              Vh.transpose(1, 0, 2, 3).reshape(B, L, T * E)], axis=2)
        hb = torch.empty((B, span), dtype=torch.int16, pin_memory=True)
        hb.copy_(torch.from_numpy(np.ascontiguousarray(blk.reshape(B, span)).view(np.int16)))
        hh = kv.HostHistory(hb.data_ptr(), L, B, T, E, E, last)
        torch.cuda.synchronize()
        ctx.stagein_blocks_host(hh, pool, ids, slots)
    else:
        kd, vd = dev_bits(Kh), dev_bits(Vh)
        hist = ctx.make_history(kd.data_ptr(), vd.data_ptr(), L, B, T, E, E, last)
        torch.cuda.synchronize()
        ctx.stagein_blocks(hist, pool, ids, slots)
    ctx.sync()
    for l in range(L):
        gk = pks[l].cpu().numpy().reshape(n_slots * T, rbk)
        gv = pvs[l].cpu().numpy().reshape(n_slots * T, rbv)
        for i, (b, s) in enumerate(zip(ids, slots)):
            nt = last if (b == B - 1 and last) else T
            p0 = pos0[i] if pos0 is not None else b * T
            wk = expected_rows(oracle, type_k, Kh[l, b, :nt], D, n_rot, theta, p0, had_k)
            wv = expected_rows(oracle, type_v, Vh[l, b, :nt], D, 0, None, 0, had_v)
            assert np.array_equal(gk[s * T:s * T + nt], wk), f"layer {l} block {b} K: {first_diff(gk[s*T:s*T+nt], wk)}"
            assert np.array_equal(gv[s * T:s * T + nt], wv), f"layer {l} block {b} V: {first_diff(gv[s*T:s*T+nt], wv)}"
            if nt < T:
                assert (gk[s * T + nt:(s + 1) * T] == SENTINEL).all()


@pytest.mark.parametrize("type_k,type_v", [(kv.TYPE_Q8_0, kv.TYPE_Q8_0), (kv.TYPE_Q4_0, kv.TYPE_Q5_0),
                                           (kv.TYPE_Q5_0, kv.TYPE_Q4_0), (kv.TYPE_F16, kv.TYPE_Q8_0)])
def test_transform_rope_hadamard_256(ctx, oracle, type_k, type_v):
    announce(f"RoPE 256 + Hadamard 256/64, 2 layers x 6 blocks, K={type_k} V={type_v}, partial last")
    run_case(ctx, oracle, L=2, B=6, Hkv=4, D=256, type_k=type_k, type_v=type_v, n_rot=256,
             had_k=256, had_v=64, ids=[5, 0, 3], slots=[1, 7, 4], n_slots=8, last=77, seed=3 + type_k)


def test_transform_partial_rotary_128_positions(ctx, oracle):
    announce("head_dim 128, RoPE 64, Hadamard 128/64, explicit positions up to 2^20")
    run_case(ctx, oracle, L=2, B=5, Hkv=8, D=128, type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q4_0,
             n_rot=64, had_k=128, had_v=64, ids=[4, 1, 2], slots=[0, 3, 2], n_slots=4,
             pos0=[1 << 20, 5, 262_016], seed=41)


# Shapes of both stage-in kernels: the 64-elements-per-lane one (rotary
# pairs across lanes l ^ 1 and l ^ 2 or inside a lane, Hadamard stages
# across lanes ^ 1, ^ 2, ^ 4, inexact scales 1/sqrtf(128) and 1/sqrtf(512),
# rotary dims short of head_dim, an untransformed V) and the
# 8-elements-per-lane one it leaves to (n_rot 48 and 512; F16 with
# cross-lane butterflies is covered above).
SHAPES = [
    # D, Hkv, n_rot, had_k, had_v, type_k, type_v
    (128, 8, 128, 128, 128, kv.TYPE_Q8_0, kv.TYPE_Q5_0),
    (256, 4, 128, 256, 256, kv.TYPE_Q4_0, kv.TYPE_Q8_0),
    (512, 2, 256, 512, 512, kv.TYPE_Q8_0, kv.TYPE_Q4_0),
    (128, 8, 32, 64, 0, kv.TYPE_Q5_0, kv.TYPE_Q8_0),
    (64, 16, 64, 64, 64, kv.TYPE_Q8_0, kv.TYPE_F16),
    (256, 4, 256, 256, 64, kv.TYPE_Q8_0, kv.TYPE_F16),
    (256, 4, 48, 256, 64, kv.TYPE_Q8_0, kv.TYPE_Q8_0),
    (512, 2, 512, 512, 128, kv.TYPE_Q5_0, kv.TYPE_Q8_0),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"D{s[0]}-rot{s[2]}-h{s[3]}-{s[4]}-k{s[5]}-v{s[6]}")
def test_transform_shapes(ctx, oracle, shape):
    D, hkv, n_rot, hk, hv, tk, tv = shape
    announce(f"head_dim {D} x {hkv}, n_rot {n_rot}, Hadamard {hk}/{hv}, K={tk} V={tv}, partial last")
    run_case(ctx, oracle, L=3, B=5, Hkv=hkv, D=D, type_k=tk, type_v=tv, n_rot=n_rot, had_k=hk, had_v=hv,
             ids=[4, 1, 3], slots=[2, 0, 1], n_slots=3, last=45, pos0=[70_000, 3, 1 << 19], seed=D + n_rot + hk)


def test_transform_rope_only_f16(ctx, oracle):
    announce("RoPE only into an F16 pool (RNE of the rotated values)")
    run_case(ctx, oracle, L=1, B=4, Hkv=4, D=256, type_k=kv.TYPE_F16, type_v=kv.TYPE_F16,
             n_rot=256, had_k=0, had_v=0, ids=[3, 1], slots=[0, 1], n_slots=2, seed=51)


def test_transform_hadamard_only_q8(ctx, oracle):
    announce("Hadamard only (no RoPE), q8_0 K/V")
    run_case(ctx, oracle, L=1, B=3, Hkv=4, D=256, type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q8_0,
             n_rot=0, had_k=256, had_v=64, ids=[0, 2], slots=[1, 0], n_slots=2, seed=61)


def test_transform_pinned_host(ctx, oracle):
    announce("pinned-host stage-in with RoPE + Hadamard, q8_0 K / q5_0 V")
    run_case(ctx, oracle, L=2, B=6, Hkv=4, D=256, type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q5_0,
             n_rot=256, had_k=256, had_v=64, ids=[2, 5, 0], slots=[0, 2, 1], n_slots=3, last=100,
             seed=71, host=True)


def test_transform_rejects_bad_arguments(ctx):
    announce("transform argument checks")
    E, L, n_slots = 1024, 1, 2
    k = torch.zeros((L, 2, T, E), dtype=torch.float16, device="cuda")
    pk = torch.zeros(n_slots * T * kv.row_size(kv.TYPE_Q8_0, E), dtype=torch.uint8, device="cuda")
    hist = ctx.make_history(k.data_ptr(), None, L, 2, T, E, E)
    th = np.ones(128, np.float32)
    bad = [ctx.make_transform(96, 0, None, 64, 0),      # head_dim not a power of two
           ctx.make_transform(256, 40, th, 0, 0),       # n_rot not a multiple of 16
           ctx.make_transform(256, 256, None, 0, 0),    # RoPE without theta
           ctx.make_transform(128, 0, None, 256, 0),    # width above head_dim
           ctx.make_transform(256, 0, None, 32, 0)]     # width below 64
    for xf in bad:
        pool = ctx.make_pool(L, n_slots, T, E, E, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [pk.data_ptr()], None, xf)
        with pytest.raises(kv.KvMemError):
            ctx.stagein_blocks(hist, pool, [0], [0])
    # RoPE table too large for a workgroup: 256-element rows touch 64 rows per chunk
    k2 = torch.zeros((1, 2, T, 256), dtype=torch.float16, device="cuda")
    p2 = torch.zeros(n_slots * T * kv.row_size(kv.TYPE_Q8_0, 256), dtype=torch.uint8, device="cuda")
    h2 = ctx.make_history(k2.data_ptr(), None, 1, 2, T, 256, 256)
    pool = ctx.make_pool(1, n_slots, T, 256, 256, kv.TYPE_Q8_0, kv.TYPE_Q8_0, [p2.data_ptr()], None,
                         ctx.make_transform(256, 256, th, 0, 0))
    with pytest.raises(kv.KvMemError):
        ctx.stagein_blocks(h2, pool, [0], [0])
    assert (pk.cpu().numpy() == 0).all() and (p2.cpu().numpy() == 0).all()


def test_engine_rope_attn_rot(oracle):
    """The engine with n_rot / attn_rot: every selected block lands in its
    slot RoPE'd at its original positions and rotated (K width 256 on q8_0,
    V width 64 on q4_0), bit-exact."""
    from kvmem_amd import host
    announce("engine: RoPE 256 (base 1e6) + attn_rot, q8_0 K / q4_0 V, 2 layers x 20 blocks")
    L, HQ, HKV, D, nb = 2, 24, 4, 256, 20
    E = HKV * D
    k, v, q = workloads.scoring_tensors(torch, "cuda", L=L, B=nb, Tq=8, seed=81, with_v=True)
    theta = oracle.rope_theta(256, 1e6)
    with host.Engine(n_layers=L, block_tokens=T, n_head=HQ, n_head_kv=HKV, head_dim=D,
                     budget_blocks=6, reserve_blocks=2, type_k=kv.TYPE_Q8_0, type_v=kv.TYPE_Q4_0,
                     n_rot=256, rope_freq_base=1e6, attn_rot=1) as eng:
        eng.set_device_history(k.data_ptr(), v.data_ptr(), nb, nb * T)
        sel = eng.preview(q.data_ptr(), 8)
        eng.apply(sel)
        slots = eng.block_slots()
        kb = workloads.to_bits(torch, k)
        vb = workloads.to_bits(torch, v)
        c = kv.Context(0)
        for layer in range(L):
            for which, src, ty, n_rot, width in ((0, kb, kv.TYPE_Q8_0, 256, 256),
                                                 (1, vb, kv.TYPE_Q4_0, 0, 64)):
                rb = kv.row_size(ty, E)
                n = eng.n_slots() * T * rb
                buf = torch.empty(n, dtype=torch.uint8, device="cuda")
                c.d2d_batched([eng.pool_layer(layer)[which]], [buf.data_ptr()], [n])
                c.sync()
                pool = buf.cpu().numpy().reshape(eng.n_slots() * T, rb)
                for b in sel.blocks:
                    s = slots[b]
                    want = expected_rows(oracle, ty, src[layer, b].reshape(T, E), D, n_rot,
                                         theta if n_rot else None, b * T, width)
                    got = pool[s * T:(s + 1) * T]
                    assert np.array_equal(got, want), f"layer {layer} {'KV'[which]} block {b}: {first_diff(got, want)}"
        c.close()
