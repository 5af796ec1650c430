/*
 * kvmem_oracle_quant.c -- half-precision conversion and the ggml q8_0 / q4_0 /
 * q5_0 reference quantizers, restated as the tests' reference for the KVMem
 * stage-in.
 *
 * TEST INFRASTRUCTURE ONLY (see kvmem_oracle.h).  Compiled with
 * -ffp-contract=off: ggml's reference quantizers are specified by their C
 * source, in which `x*id` and `+ 8.5f` are two separately rounded float
 * operations.
 */
#include "kvmem_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* f32 <-> f16 (raw_kv_store.cpp:22-83 semantics: IEEE binary16, RNE)       */
/* ------------------------------------------------------------------------ */

uint16_t ko_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {                     /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x0200u : 0u));
    }
    if (a >= 0x477ff000u) {                     /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a < 0x38800000u) {                      /* below 2^-14: subnormal */
        if (a <= 0x33000000u) {                 /* <= 2^-25 (tie -> even 0) */
            return sign;
        }
        const uint32_t e = a >> 23;             /* biased exponent, 103..112 */
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;        /* value * 2^24 = m >> shift */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) {
            ++q;                                /* may carry into 0x400 */
        }
        return (uint16_t)(sign | q);
    }
    uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        ++h;                                    /* carry rolls the exponent */
    }
    return (uint16_t)(sign | h);
}

float ko_f16_to_f32(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    float v;
    if (e == 0x1fu) {
        uint32_t bits = 0x7f800000u | (m << 13);
        memcpy(&v, &bits, sizeof(v));
    } else if (e == 0) {
        v = ldexpf((float) m, -24);
    } else {
        v = ldexpf((float) (m | 0x400u), (int) e - 25);
    }
    return (h & 0x8000u) ? -v : v;
}

float ko_bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t) h << 16;
    float v;
    memcpy(&v, &bits, sizeof(v));
    return v;
}

/* ------------------------------------------------------------------------ */
/* Block formats                                                            */
/*   q8_0: f16 d, int8 qs[32]                 = 34 B  (stagein.cu:19-22)    */
/*   q4_0: f16 d, u8 qs[16]                   = 18 B  (stagein.cu:24-27)    */
/*   q5_0: f16 d, u8 qh[4], u8 qs[16]         = 22 B  (ggml block_q5_0)     */
/* ------------------------------------------------------------------------ */

size_t ko_group_bytes(int type) {
    switch (type) {
        case KO_TYPE_Q8_0: return 34;
        case KO_TYPE_Q4_0: return 18;
        case KO_TYPE_Q5_0: return 22;
        case KO_TYPE_F16:  return 64;
        case KO_TYPE_F32:  return 128;
        default:           return 0;
    }
}

size_t ko_row_bytes(int type, int64_t n) {
    return ko_group_bytes(type) * (size_t) (n / 32);
}

static void put_f16(uint8_t *p, float d) {
    const uint16_t h = ko_f32_to_f16(d);
    p[0] = (uint8_t) (h & 0xffu);
    p[1] = (uint8_t) (h >> 8);
}

static float get_f16(const uint8_t *p) {
    return ko_f16_to_f32((uint16_t) (p[0] | (p[1] << 8)));
}

/* quantize_row_q8_0_ref: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id). */
void ko_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k) {
    for (int64_t g = 0; g < k / 32; ++g) {
        const float *xs = x + g * 32;
        uint8_t *out = y + g * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float a = fabsf(xs[j]);
            if (a > amax) {
                amax = a;
            }
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(out, d);
        for (int j = 0; j < 32; ++j) {
            const float v = xs[j] * id;
            out[2 + j] = (uint8_t) (int8_t) roundf(v);
        }
    }
}

/* Signed value of largest magnitude; the first such element wins. */
static float signed_absmax(const float *xs) {
    float amax = 0.0f;
    float vmax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        if (fabsf(xs[j]) > amax) {
            amax = fabsf(xs[j]);
            vmax = xs[j];
        }
    }
    return vmax;
}

/* Truncating code of ggml's `MIN(top, (int8_t)(v + bias))`. */
static uint8_t trunc_code(float v, float bias, int top) {
    const float s = v + bias;                   /* one rounded float add */
    const int q = (int) s;                      /* truncation toward zero */
    return (uint8_t) (q < top ? q : top);
}

/* quantize_row_q4_0_ref: d = vmax/-8, q = min(15, trunc(x*id + 8.5)),
 * low nibble = element j, high nibble = element j+16. */
void ko_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k) {
    for (int64_t g = 0; g < k / 32; ++g) {
        const float *xs = x + g * 32;
        uint8_t *out = y + g * 18;
        const float d = signed_absmax(xs) / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(out, d);
        for (int j = 0; j < 16; ++j) {
            const uint8_t lo = trunc_code(xs[j] * id, 8.5f, 15);
            const uint8_t hi = trunc_code(xs[j + 16] * id, 8.5f, 15);
            out[2 + j] = (uint8_t) (lo | (hi << 4));
        }
    }
}

/* quantize_row_q5_0_ref: d = vmax/-16, q = min(31, trunc(x*id + 16.5)),
 * low 4 bits as in q4_0, bit 4 of element j goes to qh bit j (qh is a
 * little-endian uint32 after d). */
void ko_quantize_row_q5_0(const float *x, uint8_t *y, int64_t k) {
    for (int64_t g = 0; g < k / 32; ++g) {
        const float *xs = x + g * 32;
        uint8_t *out = y + g * 22;
        const float d = signed_absmax(xs) / -16.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(out, d);
        uint32_t qh = 0;
        for (int j = 0; j < 16; ++j) {
            const uint8_t lo = trunc_code(xs[j] * id, 16.5f, 31);
            const uint8_t hi = trunc_code(xs[j + 16] * id, 16.5f, 31);
            out[6 + j] = (uint8_t) ((lo & 0x0fu) | ((hi & 0x0fu) << 4));
            qh |= (uint32_t) ((lo >> 4) & 1u) << j;
            qh |= (uint32_t) ((hi >> 4) & 1u) << (j + 16);
        }
        out[2] = (uint8_t) (qh & 0xffu);
        out[3] = (uint8_t) ((qh >> 8) & 0xffu);
        out[4] = (uint8_t) ((qh >> 16) & 0xffu);
        out[5] = (uint8_t) (qh >> 24);
    }
}

void ko_dequantize_row(int type, const uint8_t *y, float *x, int64_t k) {
    for (int64_t g = 0; g < k / 32; ++g) {
        float *xs = x + g * 32;
        if (type == KO_TYPE_Q8_0) {
            const uint8_t *b = y + g * 34;
            const float d = get_f16(b);
            for (int j = 0; j < 32; ++j) {
                xs[j] = (float) (int8_t) b[2 + j] * d;
            }
        } else if (type == KO_TYPE_Q4_0) {
            const uint8_t *b = y + g * 18;
            const float d = get_f16(b);
            for (int j = 0; j < 16; ++j) {
                xs[j] = (float) ((int) (b[2 + j] & 0x0f) - 8) * d;
                xs[j + 16] = (float) ((int) (b[2 + j] >> 4) - 8) * d;
            }
        } else if (type == KO_TYPE_Q5_0) {
            const uint8_t *b = y + g * 22;
            const float d = get_f16(b);
            const uint32_t qh = (uint32_t) b[2] | ((uint32_t) b[3] << 8) |
                                ((uint32_t) b[4] << 16) | ((uint32_t) b[5] << 24);
            for (int j = 0; j < 16; ++j) {
                const int lo = (b[6 + j] & 0x0f) | (int) (((qh >> j) & 1u) << 4);
                const int hi = (b[6 + j] >> 4) | (int) (((qh >> (j + 16)) & 1u) << 4);
                xs[j] = (float) (lo - 16) * d;
                xs[j + 16] = (float) (hi - 16) * d;
            }
        }
    }
}

int ko_quantize_rows_f16(int type, const uint16_t *src, uint8_t *dst,
                         int64_t n_rows, int64_t n_embd) {
    if (n_embd % 32 != 0) {
        return -1;
    }
    const size_t rb = ko_row_bytes(type, n_embd);
    if (rb == 0) {
        return -1;
    }
    float row[8192];
    if (n_embd > 8192) {
        return -1;
    }
    for (int64_t r = 0; r < n_rows; ++r) {
        const uint16_t *s = src + r * n_embd;
        uint8_t *o = dst + (size_t) r * rb;
        if (type == KO_TYPE_F16) {
            memcpy(o, s, (size_t) n_embd * 2);
            continue;
        }
        for (int64_t i = 0; i < n_embd; ++i) {
            row[i] = ko_f16_to_f32(s[i]);
        }
        switch (type) {
            case KO_TYPE_Q8_0: ko_quantize_row_q8_0(row, o, n_embd); break;
            case KO_TYPE_Q4_0: ko_quantize_row_q4_0(row, o, n_embd); break;
            case KO_TYPE_Q5_0: ko_quantize_row_q5_0(row, o, n_embd); break;
            default: return -1;
        }
    }
    return 0;
}

int ko_stagein_blocks(int type, const uint16_t *src, const uint32_t *slots,
                      uint32_t n_blocks, uint32_t block_tokens, uint32_t n_embd,
                      uint8_t *pool, uint32_t n_slots) {
    const size_t rb = ko_row_bytes(type, n_embd);
    for (uint32_t i = 0; i < n_blocks; ++i) {
        if (slots[i] >= n_slots) {
            return -1;
        }
        const uint16_t *s = src + (size_t) i * block_tokens * n_embd;
        uint8_t *d = pool + (size_t) slots[i] * block_tokens * rb;
        if (ko_quantize_rows_f16(type, s, d, block_tokens, n_embd) != 0) {
            return -1;
        }
    }
    return 0;
}

/* Number of floats in [lo, hi) (both non-negative) whose roundf differs
 * from the truncation of s + 0.49999997f (the float below 0.5): checks the
 * three-instruction rounding the stage-in kernel uses for q8_0 codes over
 * every float of the range. */
uint64_t ko_round_trick_mismatches(float lo, float hi) {
    uint32_t b0, b1;
    memcpy(&b0, &lo, 4);
    memcpy(&b1, &hi, 4);
    const float c = 0x1.fffffep-2f;
    uint64_t bad = 0;
    for (uint32_t b = b0; b < b1; ++b) {
        float s;
        memcpy(&s, &b, 4);
        const float t = s + c;
        if (truncf(t) != roundf(s)) {
            ++bad;
        }
    }
    return bad;
}

/* Non-negative floats a in bit range [lo_bits, hi_bits) where the stage-in's
 * q8_0 scale shortcut, q0 = a * RN(1/127), q = fma(fma(-q0, 127, a),
 * RN(1/127), q0), differs from the IEEE quotient a / 127.0f. */
uint64_t ko_div127_mismatches(uint32_t lo_bits, uint32_t hi_bits) {
    const float r127 = 1.0f / 127.0f;
    uint64_t bad = 0;
    for (uint32_t b = lo_bits; b < hi_bits; ++b) {
        float a;
        memcpy(&a, &b, 4);
        const float q0 = a * r127;
        const float q = fmaf(fmaf(-q0, 127.0f, a), r127, q0);
        const float want = a / 127.0f;
        if (memcmp(&q, &want, 4) != 0) {
            ++bad;
        }
    }
    return bad;
}
