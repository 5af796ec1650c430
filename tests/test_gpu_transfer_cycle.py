"""The reference's GPU transfer cycle (tests/mtp-kv-test.cpp:144-214), restated
through the C ABI and compared byte for byte, untouched rows included.

Every pool tensor (K and V of each layer) is filled with the reference's LCG
byte pattern (mtp-kv-test.cpp:38-45, seed 123 + number of tensors).  Blocks
0, 1, 2 sit in slots 3, 5, 7; they are saved (stage-out into a packed host
store), the pool is overwritten with 0x5a, the blocks are restored into
slots 2, 4, 6 (packed stage-in) and then laid out into slots 0, 1, 2 (device
slot moves).  After the restore only the blocks' own rows in slots 2, 4, 6
differ from 0x5a; after the layout slots 0, 1, 2 also hold them.  The last
block is partial (77 of 128 tokens), as a trailing block can be.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from conftest import load_pkg  # noqa: E402

kv = load_pkg()

T = 128
L = 2
N_SLOTS = 8
IDS = [0, 1, 2]
NTOK = [T, T, 77]


def announce(msg: str) -> None:
    print(f"[transfer] {msg}", flush=True)
    sys.stdout.flush()


def lcg_pattern(size: int, seed: int) -> np.ndarray:
    """bytes[i] = top byte of the i+1-th state of s' = s*1664525 + 1013904223
    (mod 2^32), vectorised by composing the affine step in chunks."""
    a, c, m = 1664525, 1013904223, (1 << 32) - 1
    chunk = 4096
    A = np.empty(chunk, dtype=np.uint64)
    C = np.empty(chunk, dtype=np.uint64)
    ak, ck = 1, 0
    for k in range(chunk):                     # state after k+1 steps = A[k]*s + C[k]
        ak, ck = (a * ak) & m, (a * ck + c) & m
        A[k], C[k] = ak, ck
    out = np.empty(size, dtype=np.uint8)
    s = np.uint64(seed & m)
    for off in range(0, size, chunk):
        n = min(chunk, size - off)
        st = (A[:n] * s + C[:n]) & np.uint64(m)
        out[off:off + n] = (st >> np.uint64(24)).astype(np.uint8)
        s = st[n - 1]
    return out


def test_lcg_pattern_matches_sequential():
    seed, n = 129, 10000
    want = np.empty(n, dtype=np.uint8)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        want[i] = s >> 24
    assert np.array_equal(lcg_pattern(n, seed), want)


@pytest.mark.parametrize("tk,tv", [(kv.TYPE_Q8_0, kv.TYPE_Q4_0), (kv.TYPE_F16, kv.TYPE_F16),
                                   (kv.TYPE_Q5_0, kv.TYPE_Q8_0)])
def test_save_clear_restore_layout_cycle(ctx, tk, tv):
    announce(f"types {tk}/{tv}: save blocks {IDS} from slots 3,5,7, clear, restore to 2,4,6, "
             f"layout to 0,1,2 (tokens {NTOK})")
    E = 1024
    rk, rv = kv.row_size(tk, E), kv.row_size(tv, E)
    rows = [rk, rv] * L
    n_tensors = 2 * L
    original = [lcg_pattern(N_SLOTS * T * r, 123 + n_tensors) for r in rows]
    tensors = [torch.from_numpy(o.copy()).cuda() for o in original]
    pool = ctx.make_pool(L, N_SLOTS, T, E, E, tk, tv, [tensors[2 * l].data_ptr() for l in range(L)],
                         [tensors[2 * l + 1].data_ptr() for l in range(L)])
    span = L * T * (rk + rv)
    store = torch.zeros(len(IDS) * span, dtype=torch.uint8, pin_memory=True)
    ph = kv.PackedHost(store.data_ptr(), L, len(IDS), T)
    torch.cuda.synchronize()

    # save: block id lives in slot 3 + 2*id
    ctx.stageout_blocks(pool, ph, IDS, [3 + 2 * i for i in IDS], NTOK)
    ctx.sync()
    # clear every pool tensor
    for t in tensors:
        t.fill_(0x5A)
    torch.cuda.synchronize()
    expected = [np.full_like(o, 0x5A) for o in original]
    for i, r in enumerate(rows):
        for b, nt in zip(IDS, NTOK):
            src = (3 + 2 * b) * T * r
            dst = (2 + 2 * b) * T * r
            expected[i][dst:dst + nt * r] = original[i][src:src + nt * r]

    # restore into slot 2 + 2*id
    ctx.stagein_packed_host(ph, pool, IDS, [2 + 2 * i for i in IDS], NTOK)
    ctx.sync()
    for i, t in enumerate(tensors):
        assert np.array_equal(t.cpu().numpy(), expected[i]), f"restore: tensor {i} differs"

    # layout: slot 2 + 2*id -> slot id
    before = [e.copy() for e in expected]
    for i, r in enumerate(rows):
        for b, nt in zip(IDS, NTOK):
            src = (2 + 2 * b) * T * r
            expected[i][b * T * r:b * T * r + nt * r] = before[i][src:src + nt * r]
    ctx.move_slots(pool, [2 + 2 * i for i in IDS], IDS, NTOK)
    ctx.sync()
    for i, t in enumerate(tensors):
        assert np.array_equal(t.cpu().numpy(), expected[i]), f"layout: tensor {i} differs"
