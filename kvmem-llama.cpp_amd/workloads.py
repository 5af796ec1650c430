"""Seeded synthetic workloads of the reselect path (shapes of the reselect
benchmark configurations).  No parity logic lives here.

Shapes (L layers, B history blocks, T = 128 tokens per block, Hkv = 4 KV
heads, Hq = 24 query heads, D = 256):
  stagein_1layer : K, V [64][128][4][256] f16, N(0,1) with 4 fixed outlier
                   channels per head scaled x20, slots = seeded permutation
                   of 0..255 (pool of 256 slots), q8_0.
  scoring_256k   : K [16][2048][128][4][256] f16 = N(0,1) + per-(layer,
                   block) offset N(0, 0.3^2) per channel; Q [16][64][24][256]
                   bf16 N(0,1); GQA group 6; top-256 with block 0 as sink.
  reselect_256k  : the scoring workload plus V, a pool of 256 + 128 slots,
                   and a second query whose selection differs by ~30 %.
  mixed_precision: the same shapes with Student-t (nu = 4) values.
  recall_1m      : 8192 blocks x 16 layers, 512-token query, 32 planted
                   blocks with Zipf relevance, budget 512.
"""
from __future__ import annotations

import numpy as np

T_BLOCK = 128
HKV = 4
HQ = 24
HEAD_DIM = 256
N_EMBD = HKV * HEAD_DIM


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x.astype(np.float16)).view(np.uint16)


def outlier_channels(rng: np.random.Generator, n_head: int = HKV, head_dim: int = HEAD_DIM,
                     per_head: int = 4) -> np.ndarray:
    """Channel indices (within n_head*head_dim) scaled x20: 4 per head."""
    ch = [h * head_dim + rng.choice(head_dim, per_head, replace=False) for h in range(n_head)]
    return np.sort(np.concatenate(ch))


def stagein_1layer(seed: int = 1, n_blocks: int = 64, n_slots: int = 256, T: int = T_BLOCK,
                   n_embd: int = N_EMBD):
    """K, V f16 bits [n_blocks][T][n_embd] and the slot of each block."""
    rng = np.random.default_rng(seed)
    ch = outlier_channels(rng, n_embd // HEAD_DIM)
    out = []
    for _ in range(2):
        x = rng.standard_normal((n_blocks, T, n_embd), dtype=np.float32)
        x[..., ch] *= 20.0
        out.append(f16_bits(x))
    slots = rng.permutation(n_slots)[:n_blocks].astype(np.uint32)
    return out[0], out[1], slots


def heavy_tailed(seed: int, shape, nu: float = 4.0) -> np.ndarray:
    """Student-t values as f16 bits (clipped to the f16 range)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_t(nu, size=shape).astype(np.float32)
    return f16_bits(np.clip(x, -60000.0, 60000.0))


# ----------------------------------------------------------------- device
def scoring_tensors(torch, device: str, L: int = 16, B: int = 2048, Tq: int = 64, seed: int = 2,
                    T: int = T_BLOCK, Hkv: int = HKV, Hq: int = HQ, D: int = HEAD_DIM,
                    with_v: bool = False, offset_std: float = 0.3):
    """K (and V) history [L][B][T][Hkv][D] f16 and Q [L][Tq][Hq][D] bf16 on
    `device`, generated there from a seeded generator, one layer at a time."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    k = torch.empty((L, B, T, Hkv, D), dtype=torch.float16, device=device)
    v = torch.empty_like(k) if with_v else None
    for l in range(L):
        off = torch.randn((B, 1, Hkv, D), generator=g, device=device, dtype=torch.float32) * offset_std
        k[l] = (torch.randn((B, T, Hkv, D), generator=g, device=device, dtype=torch.float32) + off).half()
        if v is not None:
            v[l] = torch.randn((B, T, Hkv, D), generator=g, device=device, dtype=torch.float32).half()
    q = torch.randn((L, Tq, Hq, D), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    return k, v, q


def student_t_tensors(torch, device: str, L: int = 16, B: int = 2048, Tq: int = 64, seed: int = 4,
                      T: int = T_BLOCK, Hkv: int = HKV, Hq: int = HQ, D: int = HEAD_DIM,
                      nu: int = 4):
    """K, V history [L][B][T][Hkv][D] f16 with Student-t (nu = 4) values,
    t = z / sqrt(chi2_nu / nu) with chi2_nu a sum of nu squared normals,
    generated on `device` one layer at a time; Q [L][Tq][Hq][D] bf16 N(0,1)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    k = torch.empty((L, B, T, Hkv, D), dtype=torch.float16, device=device)
    v = torch.empty_like(k)
    for dst in (k, v):
        for l in range(L):
            chi2 = torch.zeros((B, T, Hkv, D), device=device, dtype=torch.float32)
            for _ in range(nu):
                chi2.addcmul_(z := torch.randn((B, T, Hkv, D), generator=g, device=device), z)
            z = torch.randn((B, T, Hkv, D), generator=g, device=device)
            dst[l] = (z / torch.sqrt(chi2 / nu)).clamp_(-60000.0, 60000.0).half()
            del chi2, z
    q = torch.randn((L, Tq, Hq, D), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    return k, v, q


def plant_blocks(torch, k, q, n_planted: int = 32, seed: int = 5, alpha: float = 48.0):
    """Add alpha * rank-scaled unit query directions to the keys of
    n_planted seeded blocks (Zipf relevance: the r-th planted block gets
    weight 1/r^0.5 of alpha).  Returns the planted block ids.

    Scale: a unit direction raises a block's per-token max by about
    w * 4.3 / sqrt(head_dim) (the largest projection of 3072 N(0,1) query
    rows on their mean direction), while the max over ~4e5 random dot
    products already spreads unplanted blocks by ~0.3; alpha = 48 lifts
    the weakest rank (r = 32) by ~2.3, clear of that spread."""
    L, B, T, Hkv, D = k.shape
    rng = np.random.default_rng(seed)
    ids = np.sort(rng.choice(np.arange(1, B), n_planted, replace=False))
    ranks = rng.permutation(n_planted) + 1
    g = q.shape[2] // Hkv
    for l in range(L):
        # one unit direction per KV head: the mean of the group's query heads
        qd = q[l].float().mean(dim=0).view(Hkv, g, D).mean(dim=1)
        qd = qd / qd.norm(dim=-1, keepdim=True)
        for b, r in zip(ids, ranks):
            w = alpha / float(r) ** 0.5
            k[l, int(b)] += (w * qd).half().unsqueeze(0)
    return ids.astype(np.uint32)


def previous_selection(sel, n_blocks: int, n_changed: int, seed: int = 7) -> list[int]:
    """The previous agent step's selection for a reselect workload:
    `n_changed` seeded blocks of `sel` (never block 0, the sink) swapped for
    seeded blocks outside it, so the next step stages exactly those."""
    rng = np.random.default_rng(seed)
    cur = np.array(sel)
    drop = rng.choice(cur[cur != 0], n_changed, replace=False)
    outside = np.setdiff1d(np.arange(n_blocks), cur)
    add = rng.choice(outside, n_changed, replace=False)
    return sorted(set(int(x) for x in sel) - set(drop.tolist()) | set(add.tolist()))


def to_bits(torch, t) -> np.ndarray:
    """Device f16/bf16 tensor -> numpy uint16 bits on the host."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
