/*
 * kvmem_oracle_xf.c -- the cache row transform of the raw-K stage-in
 * (NeoX RoPE at the block's positions, then the attn_rot Walsh-Hadamard
 * rotation), restated as the tests' reference.
 *
 * TEST INFRASTRUCTURE ONLY (see kvmem_oracle.h).  Compiled with
 * -ffp-contract=off: every product and sum is one IEEE operation, and the
 * fused multiply-adds of the sin/cos evaluation are explicit fma() calls.
 */
#include "kvmem_oracle.h"

#include <math.h>

/* sin and cos of an fp32 angle (the library's own evaluation, stated here
 * step by step): k = rint(a * 2/pi) in double, r = a - k*pi/2 by two fused
 * multiply-adds with pi/2 split into two doubles (Cody-Waite), Taylor series
 * of sin to r^17 and of cos to r^16 by Horner's rule in double, quadrant
 * k mod 4, one rounding to fp32 at the end.  Finite |a| < 2^40. */
void ko_rope_sincos(float a, float *sn, float *cs) {
    const double x = (double) a;
    const double k = rint(x * 0x1.45f306dc9c883p-1);
    double r = x;  /* |a| < pi/4: no reduction (keeps the sign of zero) */
    if (k != 0.0) {
        r = fma(-k, 0x1.921fb54442d18p+0, x);
        r = fma(-k, 0x1.1a62633145c07p-54, r);
    }
    const double r2 = r * r;
    /* sin: -1/3!, 1/5!, ..., 1/17!; cos: -1/2!, 1/4!, ..., 1/16! */
    static const double S[8] = {-0x1.5555555555555p-3, 0x1.1111111111111p-7,
                                -0x1.a01a01a01a01ap-13, 0x1.71de3a556c734p-19,
                                -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33,
                                -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49};
    static const double Cc[8] = {-0.5, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
                                 0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22,
                                 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
                                 0x1.ae7f3e733b81fp-45};
    double ps = S[7];
    for (int i = 6; i >= 0; --i) {
        ps = fma(ps, r2, S[i]);
    }
    double pc = Cc[7];
    for (int i = 6; i >= 0; --i) {
        pc = fma(pc, r2, Cc[i]);
    }
    const double sr = r == 0.0 ? r : fma(r * r2, ps, r);  /* sin(+-0) = +-0 */
    const double cr = fma(r2, pc, 1.0);
    const int quadrant = (int) (k - 4.0 * floor(k * 0.25));  /* k mod 4, exact */
    const double sv = (quadrant & 1) ? cr : sr;
    const double cv = (quadrant & 1) ? sr : cr;
    *sn = (float) ((quadrant & 2) ? -sv : sv);
    *cs = (float) (((quadrant + 1) & 2) ? -cv : cv);
}

void ko_rope_sincos_n(const float *a, uint64_t n, float *sn, float *cs) {
    for (uint64_t i = 0; i < n; ++i) {
        ko_rope_sincos(a[i], sn + i, cs + i);
    }
}

/* NeoX RoPE in place (rope_neox_kernel, llama-kvmem-stagein.cu:159-178;
 * kvmem/src/host/rope.cpp:8-45): rows [n_rows][n_embd] token-major, heads of
 * head_dim; token t sits at position pos0 + t; for i < n_rot/2 the pair
 * (x0, x1) = (x[i], x[i + n_rot/2]) becomes (x0*c - x1*s, x0*s + x1*c) with
 * a = (float)(pos0 + t) * theta[i]; elements from n_rot on are unchanged. */
void ko_rope_rows(float *rows, uint32_t n_rows, uint32_t n_embd, uint32_t head_dim,
                  uint32_t n_rot, const float *theta, int32_t pos0) {
    const uint32_t half = n_rot / 2;
    for (uint32_t t = 0; t < n_rows; ++t) {
        const float pos = (float) (pos0 + (int32_t) t);
        for (uint32_t h = 0; h < n_embd / head_dim; ++h) {
            float *x = rows + (size_t) t * n_embd + (size_t) h * head_dim;
            for (uint32_t i = 0; i < half; ++i) {
                float s, c;
                ko_rope_sincos(pos * theta[i], &s, &c);
                const float x0 = x[i];
                const float x1 = x[i + half];
                x[i] = x0 * c - x1 * s;
                x[i + half] = x0 * s + x1 * c;
            }
        }
    }
}

/* attn_rot Walsh-Hadamard rotation in place of every run of `width`
 * elements (fwht_kernel, llama-kvmem-stagein.cu:104-130, launched with
 * scale = 1.0f / sqrtf(width), :557): scale first, then butterflies
 * (a + b, a - b) of span 1, 2, ..., width/2. */
void ko_hadamard_rows(float *x, uint64_t n_elems, uint32_t width) {
    const float scale = 1.0f / sqrtf((float) width);
    for (uint64_t base = 0; base + width <= n_elems; base += width) {
        float *v = x + base;
        for (uint32_t i = 0; i < width; ++i) {
            v[i] = v[i] * scale;
        }
        for (uint32_t h = 1; h < width; h *= 2) {
            for (uint32_t i = 0; i < width; i += 2 * h) {
                for (uint32_t j = 0; j < h; ++j) {
                    const float a = v[i + j];
                    const float b = v[i + j + h];
                    v[i + j] = a + b;
                    v[i + j + h] = a - b;
                }
            }
        }
    }
}

/* fp32 rows -> packed rows of `type` (ggml_quantize_chunk row by row, or
 * ggml_fp32_to_fp16_row RNE for F16; llama-kvmem-quant.h:96-119). */
int ko_quantize_rows_f32(int type, const float *src, uint8_t *dst, int64_t n_rows, int64_t n_embd) {
    const size_t rb = ko_row_bytes(type, n_embd);
    if (rb == 0) {
        return -1;
    }
    for (int64_t r = 0; r < n_rows; ++r) {
        const float *x = src + r * n_embd;
        uint8_t *y = dst + (size_t) r * rb;
        switch (type) {
            case KO_TYPE_Q8_0: ko_quantize_row_q8_0(x, y, n_embd); break;
            case KO_TYPE_Q4_0: ko_quantize_row_q4_0(x, y, n_embd); break;
            case KO_TYPE_Q5_0: ko_quantize_row_q5_0(x, y, n_embd); break;
            case KO_TYPE_F16:
                for (int64_t e = 0; e < n_embd; ++e) {
                    const uint16_t h = ko_f32_to_f16(x[e]);
                    y[2 * e] = (uint8_t) (h & 0xff);
                    y[2 * e + 1] = (uint8_t) (h >> 8);
                }
                break;
            default: return -1;
        }
    }
    return 0;
}
