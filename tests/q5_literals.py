"""Literal q5_0 blocks from ggml's published layout (shared by the CPU
oracle tests and the GPU stage-in tests).

ggml publishes block_q5_0 as {ggml_half d; uint8_t qh[4]; uint8_t qs[16]}
and reads it back in dequantize_row_q5_0 as
    qh   = the 4 bytes as a little-endian uint32 (memcpy on x86 / gfx9)
    xh_0 = ((qh >> (j +  0)) << 4) & 0x10     element j,      j < 16
    xh_1 = ((qh >> (j + 12))     ) & 0x10     element j + 16
    x0   = ((qs[j] & 0x0F) | xh_0) - 16
    x1   = ((qs[j] >>   4) | xh_1) - 16
The decoder below states exactly that (a different formula from the
quantizer's packing loop), and the expected bytes of the groups are
literals worked out by hand from the codes.
"""
from __future__ import annotations

import numpy as np


def groups_f16(*groups) -> np.ndarray:
    return np.asarray(groups, dtype=np.float32).astype(np.float16).view(np.uint16).reshape(1, -1)


def ggml_q5_0_decode_codes(block: bytes) -> list[int]:
    """Signed codes (-16..15) of one 22-byte block_q5_0, per the published
    dequantizer's bit extraction."""
    qh = int.from_bytes(block[2:6], "little")
    qs = block[6:22]
    out = [0] * 32
    for j in range(16):
        xh_0 = ((qh >> (j + 0)) << 4) & 0x10
        xh_1 = (qh >> (j + 12)) & 0x10
        out[j] = ((qs[j] & 0x0F) | xh_0) - 16
        out[j + 16] = ((qs[j] >> 4) | xh_1) - 16
    return out


def _q5_every_code():
    # x = -16..15: vmax = -16 (element 0, first of largest magnitude), d = 1,
    # code of x is x + 16, so element j has code j.
    g = np.arange(-16, 16, dtype=np.float32)
    d_bits = bytes([0x00, 0x3C])                  # f16 1.0
    qh = bytes([0x00, 0x00, 0xFF, 0xFF])          # codes 16..31 sit at elements 16..31
    qs = bytes([j | (j << 4) for j in range(16)])  # lo nibble j, hi nibble (j + 16) & 15 = j
    return g, d_bits + qh + qs


def _q5_asymmetric():
    # d = 1 from x[0] = -16; every other element -5 (code 11 = 0x0B) except
    # x[3] = 2 (code 18 = 0x12) and x[20] = 7 (code 23 = 0x17): bit 4 is set
    # for elements 3 and 20 only, i.e. qh = (1 << 3) | (1 << 20).
    g = np.full(32, -5.0, np.float32)
    g[0], g[3], g[20] = -16.0, 2.0, 7.0
    d_bits = bytes([0x00, 0x3C])
    qh = bytes([0x08, 0x00, 0x10, 0x00])
    qs = [0xBB] * 16
    qs[0] = 0x0 | (0xB << 4)                     # element 0 code 0, element 16 code 11
    qs[3] = 0x2 | (0xB << 4)                     # element 3 code 18 -> low nibble 2
    qs[4] = 0xB | (0x7 << 4)                     # element 20 code 23 -> high nibble 7
    return g, d_bits + qh + bytes(qs)


def _q5_high_half_only():
    # d = -1 from x[16] = 16 (vmax = +16, the first of largest magnitude):
    # codes are trunc(-x + 16.5) capped at 31.  x[16] -> 0, x[17] = -15 -> 31,
    # x[1] = -3 -> 19, the rest 0 -> 16.
    g = np.zeros(32, np.float32)
    g[16], g[17], g[1] = 16.0, -15.0, -3.0
    d_bits = bytes([0x00, 0xBC])                  # f16 -1.0
    codes = [16] * 32
    codes[16], codes[17], codes[1] = 0, 31, 19
    qh_v = sum(((c >> 4) & 1) << j for j, c in enumerate(codes))
    assert qh_v == 0xFFFEFFFF                     # every bit but element 16's
    qh = bytes([0xFF, 0xFF, 0xFE, 0xFF])
    qs = bytes([(codes[j] & 15) | ((codes[j + 16] & 15) << 4) for j in range(16)])
    assert qs[0] == 0x00 and qs[1] == 0xF3 and qs[2] == 0x00
    return g, d_bits + qh + qs


Q5_LITERAL_GROUPS = [_q5_every_code, _q5_asymmetric, _q5_high_half_only]


def q5_literal_failures(quantize) -> list[str]:
    """Every literal check of the q5_0 layout against `quantize(rows_f16)`;
    returns the failures (empty when the layout is ggml's)."""
    bad = []
    for make in Q5_LITERAL_GROUPS:
        g, want = make()
        got = bytes(quantize(groups_f16(g))[0].tobytes())
        if got != want:
            bad.append(f"{make.__name__}: {got.hex()} != {want.hex()}")
        d = float(np.frombuffer(want[:2], np.float16)[0])
        codes = ggml_q5_0_decode_codes(got)
        # these groups are exact multiples of d in the code range: the
        # published dequantizer gives them back exactly
        if not np.array_equal(np.array(codes, np.float32) * np.float32(d), g):
            bad.append(f"{make.__name__}: decodes to {codes}")
    return bad
