"""The oracle's cache row transform (raw-K stage-in: NeoX RoPE at the
block's positions, then the attn_rot Walsh-Hadamard rotation), pinned
without the GPU.

  - sin/cos: equal to float64 libm sin/cos rounded to fp32 on 5*10^5 seeded
    angles (small, up to 10^6 rad, near multiples of pi/2, signed zeros, up
    to 2^39 rad);
  - RoPE: the reference's own rope_neox_apply (kvmem/src/host/rope.cpp, built
    into oracle/_ref) within fp32 rounding, its unit test (position 0 is the
    identity, position 1 is not), a float64 rotation, pair norms preserved,
    elements past n_rot untouched, frequencies as rope.cpp forms them;
  - Hadamard: float64 products with the Sylvester matrix / sqrt(n), H H = I,
    exact images of unit vectors (+-1/sqrt(n) with the (-1)^popcount(i&j)
    sign pattern), runs of `width` inside longer rows.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
from scipy.linalg import hadamard

from conftest import ROOT

REF = ROOT / "oracle" / "_ref" / "libkvmem_ref.so"


def test_sincos_correctly_rounded(oracle):
    rng = np.random.default_rng(11)
    a = np.concatenate([
        rng.uniform(-8, 8, 200_000),
        rng.uniform(-1e6, 1e6, 200_000),
        np.float32(np.pi / 2) * rng.integers(-100_000, 100_000, 100_000) +
        rng.uniform(-1e-3, 1e-3, 100_000),
        np.float32(np.pi / 2) * np.arange(-64, 64),
        [0.0, -0.0, 1e-30, -1e-30, 2.0 ** -126, 2.0 ** 31, -1.5e9, 2.0 ** 39],
    ]).astype(np.float32)
    s, c = oracle.rope_sincos(a)
    ws = np.sin(a.astype(np.float64)).astype(np.float32)
    wc = np.cos(a.astype(np.float64)).astype(np.float32)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(c.view(np.uint32), wc.view(np.uint32))


def test_rope_theta_as_reference(oracle):
    th = oracle.rope_theta(128, 10000.0, 0.5)
    assert th[0] == np.float32(0.5)
    want = (10000.0 ** (-2.0 * np.arange(64) / 128)) * 0.5
    assert np.allclose(th, want, rtol=3e-7, atol=0)


def rope64(x, head_dim, n_rot, theta, pos0):
    """float64 NeoX rotation with the fp32 angle of the reference."""
    x = x.astype(np.float64).copy()
    n, e = x.shape
    half = n_rot // 2
    for t in range(n):
        a = (np.float32(pos0 + t) * theta).astype(np.float32).astype(np.float64)
        c, s = np.cos(a), np.sin(a)
        for h in range(e // head_dim):
            base = h * head_dim
            x0 = x[t, base:base + half].copy()
            x1 = x[t, base + half:base + n_rot].copy()
            x[t, base:base + half] = x0 * c - x1 * s
            x[t, base + half:base + n_rot] = x0 * s + x1 * c
    return x


@pytest.mark.parametrize("head_dim,n_rot,pos0", [(256, 256, 0), (256, 128, 4096), (128, 64, 777_777)])
def test_rope_float64_and_invariants(oracle, head_dim, n_rot, pos0):
    rng = np.random.default_rng(head_dim + n_rot)
    x = rng.standard_normal((24, 4 * head_dim)).astype(np.float32) * 3
    th = oracle.rope_theta(n_rot, 1e6)
    got = oracle.transform_rows(x, head_dim, n_rot, th, pos0)
    want = rope64(x, head_dim, n_rot, th, pos0)
    assert np.max(np.abs(got - want)) <= 4e-7 * np.max(np.abs(x))
    half = n_rot // 2
    for h in range(4):
        b = h * head_dim
        assert np.array_equal(got[:, b + n_rot:b + head_dim], x[:, b + n_rot:b + head_dim])
        n_in = x[:, b:b + half] ** 2 + x[:, b + half:b + n_rot] ** 2
        n_out = got[:, b:b + half] ** 2 + got[:, b + half:b + n_rot] ** 2
        assert np.allclose(n_in, n_out, rtol=2e-6, atol=1e-6)


def test_rope_reference_unit_case(oracle):
    # raw_kv_store_test.cpp:143-157: n_rot 4, one head, base 10000; x = e0 + e2
    th = oracle.rope_theta(4, 10000.0)
    x64 = np.zeros((1, 64), np.float32)
    x64[0, 0] = x64[0, 2] = 1.0
    at0 = oracle.transform_rows(x64[:, :64], 64, 4, th, 0)
    assert np.array_equal(at0, x64)
    at1 = oracle.transform_rows(x64, 64, 4, th, 1)
    assert not np.array_equal(at1, x64)


@pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (needs the reference tree)")
@pytest.mark.parametrize("n_rot,head_dim,pos0", [(128, 128, 0), (256, 256, 131_000), (64, 128, 9)])
def test_rope_matches_reference(oracle, n_rot, head_dim, pos0):
    ref = C.CDLL(str(REF))
    fp = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    ref.kref_rope_neox.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, C.c_float, fp,
                                   C.c_uint32, C.c_int32, fp]
    rng = np.random.default_rng(n_rot + pos0)
    hkv, n = 4, 16
    x = rng.standard_normal((n, hkv * head_dim)).astype(np.float32)
    want = np.zeros_like(x)
    assert ref.kref_rope_neox(n_rot, head_dim, hkv, 1e6, 1.0, x, n, pos0, want) == 0
    got = oracle.transform_rows(x, head_dim, n_rot, oracle.rope_theta(n_rot, 1e6), pos0)
    # same fp32 angles; sin/cos of the C library within one rounding
    assert np.max(np.abs(got - want)) <= 4e-7 * np.max(np.abs(x))


@pytest.mark.parametrize("width", [64, 128, 256, 512])
def test_hadamard_matches_sylvester(oracle, width):
    rng = np.random.default_rng(width)
    x = rng.standard_normal((6, 1024)).astype(np.float32)
    got = oracle.transform_rows(x, 512, 0, None, 0, width).astype(np.float64)
    H = hadamard(width) / np.sqrt(width)
    want = (x.astype(np.float64).reshape(-1, width) @ H.T).reshape(x.shape)
    assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(x)) * np.log2(width)
    back = oracle.transform_rows(got.astype(np.float32), 512, 0, None, 0, width)
    assert np.allclose(back, x, atol=1e-5)


@pytest.mark.parametrize("width", [64, 128, 256])
def test_hadamard_unit_vectors_exact(oracle, width):
    scale = np.float32(1.0) / np.sqrt(np.float32(width))
    eye = np.eye(width, dtype=np.float32)
    got = oracle.transform_rows(eye, width, 0, None, 0, width)
    i = np.arange(width)
    signs = np.array([[(-1) ** bin(a & b).count("1") for b in i] for a in i], np.float32)
    assert np.array_equal(got, signs.T * scale)


def test_transform_then_quantize_roundtrip(oracle):
    """Dequantized q8_0 of the rotated rows, rotated back, stays within the
    quantization error of the input (the cache round trip)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 1024)).astype(np.float32)
    r = oracle.transform_rows(x, 256, 0, None, 0, 256)
    q = oracle.quantize_rows_f32(oracle.TYPE_Q8_0, r)
    deq = np.stack([oracle.dequantize_row(oracle.TYPE_Q8_0, q[i], 1024) for i in range(8)])
    back = oracle.transform_rows(deq, 256, 0, None, 0, 256)
    assert np.max(np.abs(back - x)) <= 0.02 * np.max(np.abs(r))
