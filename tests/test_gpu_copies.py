"""kvmem_hip_d2d_batched (the reference's kvmem_d2d_batched + copy_bytes,
src/adapter/llama-kvmem-stagein.cu:235-260, 965-998) on the GPU.

10 000 ops in one call (past the reference's 8192-op limit) with random
sizes from 1 byte to 70 KB and random source / destination alignments, so
both the 16-byte and the byte path run, every byte compared with the
expected buffer, bytes outside the ops untouched.  As the reference's entry
point, a call holding a null pointer or an empty op is refused before any
copy (stagein.cu:977-979), and n = 0 is a no-op.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()


def test_d2d_batched_many_unaligned_ops(ctx):
    print("[copies] 10000 ops, random sizes and alignments", flush=True)
    rng = np.random.default_rng(17)
    n = 10000
    sizes = np.where(rng.random(n) < 0.3, rng.integers(1, 64, n), rng.integers(64, 70000, n)).astype(np.int64)
    sizes[::7] = (sizes[::7] + 15) // 16 * 16           # some 16-byte multiples
    src_off = np.cumsum(np.concatenate([[0], sizes[:-1] + rng.integers(0, 40, n - 1)]))
    src_off[::5] = (src_off[::5] + 15) // 16 * 16        # some aligned sources (reads may overlap)
    # destinations laid out in another order, disjoint, some 16-byte aligned
    dst_off = np.zeros(n, np.int64)
    pos = 3
    for j, i in enumerate(rng.permutation(n)):
        if j % 5 == 0:
            pos = (pos + 15) // 16 * 16
        dst_off[i] = pos
        pos += int(sizes[i]) + int(rng.integers(0, 40))
    sizes_d = sizes
    total_src = int((src_off + sizes).max()) + 64
    total_dst = int((dst_off + sizes_d).max()) + 64
    src_h = rng.integers(0, 256, total_src, dtype=np.uint8)
    src = torch.from_numpy(src_h).cuda()
    dst = torch.full((total_dst,), 0xA5, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ctx.d2d_batched([src.data_ptr() + int(o) for o in src_off], [dst.data_ptr() + int(o) for o in dst_off],
                    [int(s) for s in sizes_d])
    ctx.sync()
    got = dst.cpu().numpy()
    want = np.full(total_dst, 0xA5, np.uint8)
    for so, do, sz in zip(src_off, dst_off, sizes_d):
        want[do:do + sz] = src_h[so:so + sz]
    assert np.array_equal(got, want), int(np.flatnonzero(got != want)[0])


@pytest.mark.parametrize("big", [(5 << 20), (1 << 20) + 7, (64 << 20) + 48])
def test_d2d_batched_large_and_tiny_ops_together(ctx, big):
    """Ops are cut into pieces sized from the largest op (about 16 KiB,
    at most 64 per op): one op of several MiB, aligned or not, beside
    16-byte, 3-byte and 70 KB ops in the same launch; every byte equal to
    the source, bytes outside the ops untouched."""
    print(f"[copies] one {big}-byte op with small ones", flush=True)
    rng = np.random.default_rng(big & 0xffff)
    sizes = [big, 16, 3, 70000, 1, 4096, big // 3]
    src_off, dst_off, pos_s, pos_d = [], [], 0, 5
    for i, sz in enumerate(sizes):
        src_off.append(pos_s if i % 2 == 0 else pos_s + 7)
        pos_s = src_off[-1] + sz + 32
        dst_off.append((pos_d + 15) // 16 * 16 if i % 3 == 0 else pos_d)
        pos_d = dst_off[-1] + sz + 32
    src_h = rng.integers(0, 256, pos_s + 64, dtype=np.uint8)
    src = torch.from_numpy(src_h).cuda()
    dst = torch.full((pos_d + 64,), 0x3C, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ctx.d2d_batched([src.data_ptr() + o for o in src_off], [dst.data_ptr() + o for o in dst_off], sizes)
    ctx.sync()
    want = np.full(pos_d + 64, 0x3C, np.uint8)
    for so, do, sz in zip(src_off, dst_off, sizes):
        want[do:do + sz] = src_h[so:so + sz]
    got = dst.cpu().numpy()
    assert np.array_equal(got, want), int(np.flatnonzero(got != want)[0])


def test_d2d_batched_refuses_null_and_empty_ops(ctx):
    print("[copies] null / empty ops refused, n = 0 a no-op", flush=True)
    src = torch.arange(256, dtype=torch.uint8, device="cuda")
    dst = torch.zeros(256, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for srcs, dsts, sizes in (([src.data_ptr(), 0], [dst.data_ptr(), dst.data_ptr() + 64], [16, 16]),
                              ([src.data_ptr(), src.data_ptr()], [dst.data_ptr(), 0], [16, 16]),
                              ([src.data_ptr(), src.data_ptr()], [dst.data_ptr(), dst.data_ptr() + 64],
                               [16, 0])):
        with pytest.raises(kv.KvMemError):
            ctx.d2d_batched(srcs, dsts, sizes)
    ctx.d2d_batched([], [], [])
    ctx.sync()
    assert not dst.cpu().numpy().any()
