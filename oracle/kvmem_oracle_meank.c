/*
 * kvmem_oracle_meank.c -- the reference's retrieval scorer (mean-K cosine)
 * and its mean-K producer, restated as the tests' reference.
 *
 * TEST INFRASTRUCTURE ONLY (see kvmem_oracle.h).  Compiled with
 * -ffp-contract=off: every product and sum below is one IEEE operation in
 * the order of the reference source.
 */
#include "kvmem_oracle.h"

#include <math.h>
#include <string.h>

/* RawKvStore::capture_mean_f16 (kvmem/src/host/raw_kv_store.cpp:184-202):
 * k_sum[e] = 0.0f + f16(row 0)[e] + f16(row 1)[e] + ... in token order. */
void ko_meank_sum_f16(const uint16_t *rows, uint32_t n_tokens, uint32_t n_embd,
                      uint64_t row_stride, float *k_sum) {
    for (uint32_t e = 0; e < n_embd; ++e) {
        k_sum[e] = 0.0f;
    }
    for (uint32_t t = 0; t < n_tokens; ++t) {
        const uint16_t *r = rows + (size_t) t * row_stride;
        for (uint32_t e = 0; e < n_embd; ++e) {
            k_sum[e] += ko_f16_to_f32(r[e]);
        }
    }
}

/* RawKvStore::mean_k normalisation (raw_kv_store.cpp:984-995): one fp32
 * reciprocal of the token count, then one multiplication per element. */
void ko_mean_k(const float *k_sum, uint32_t mean_tokens, uint32_t n_embd, float *out) {
    if (mean_tokens == 0) {
        for (uint32_t e = 0; e < n_embd; ++e) {
            out[e] = 0.0f;
        }
        return;
    }
    const float inv = 1.0f / (float) mean_tokens;
    for (uint32_t e = 0; e < n_embd; ++e) {
        out[e] = k_sum[e] * inv;
    }
}

/* llama_memory_kvmem::score_retrieval (src/adapter/llama-memory-kvmem.cpp:
 * 2869-2916).  For block b, every layer l with q_count[l] > 0:
 *   mk      = mean_k(b, l)
 *   per KV head h: qh = sum_{gi<g} q_sum[l][(h*g+gi)*D ..] (float, in gi
 *                  order); qv = qh * (1 / (q_count*g)); cos = dot(qv, mk_h) /
 *                  (sqrt(|qv|^2) * sqrt(|mk_h|^2) + 1e-6f), float sums in d order
 *   layer   = sum_h cos (double);  acc += layer / Hkv (double)
 * score = acc / (layers counted) (double); a block with no mean in any layer
 * (RawKvStore::has_block false) scores 0. */
void ko_score_meank(const float *q_sum, const uint32_t *q_count, const float *k_sum,
                    const uint32_t *mean_tokens, uint32_t L, uint32_t B, uint32_t Hq,
                    uint32_t Hkv, uint32_t D, double *scores) {
    const uint32_t g = Hkv == 0 ? 1 : Hq / Hkv;
    const uint32_t E = Hkv * D;
    float mk[8192];
    float qh[1024];
    for (uint32_t b = 0; b < B; ++b) {
        scores[b] = 0.0;
        int has = 0;
        for (uint32_t l = 0; l < L; ++l) {
            has |= mean_tokens[(size_t) l * B + b] != 0;
        }
        if (!has || E > 8192 || D > 1024) {
            continue;
        }
        double acc = 0.0;
        uint32_t nlay = 0;
        for (uint32_t l = 0; l < L; ++l) {
            if (q_count[l] == 0) {
                continue;
            }
            ko_mean_k(k_sum + ((size_t) l * B + b) * E, mean_tokens[(size_t) l * B + b], E, mk);
            double layer = 0.0;
            const float invq = 1.0f / (float) (q_count[l] * (g > 1 ? g : 1));
            for (uint32_t h = 0; h < Hkv; ++h) {
                for (uint32_t d = 0; d < D; ++d) {
                    qh[d] = 0.0f;
                }
                for (uint32_t gi = 0; gi < g; ++gi) {
                    const uint32_t qi = h * g + gi;
                    if (qi >= Hq) {
                        break;
                    }
                    const float *q = q_sum + (size_t) l * Hq * D + (size_t) qi * D;
                    for (uint32_t d = 0; d < D; ++d) {
                        qh[d] += q[d];
                    }
                }
                const float *kh = mk + (size_t) h * D;
                float dot = 0.0f, nq = 0.0f, nk = 0.0f;
                for (uint32_t d = 0; d < D; ++d) {
                    const float qv = qh[d] * invq;
                    dot += qv * kh[d];
                    nq += qv * qv;
                    nk += kh[d] * kh[d];
                }
                layer += dot / (sqrtf(nq) * sqrtf(nk) + 1e-6f);
            }
            acc += layer / (double) (Hkv > 1 ? Hkv : 1);
            nlay++;
        }
        scores[b] = nlay ? acc / nlay : 0.0;
    }
}

/* The reference's query harvest into q_sum_ (src/adapter/llama-memory-
 * kvmem.cpp:2164-2172 and :2206-2219): per layer, every listed token's row
 * (already widened to f32) is added element by element onto q_sum in list
 * order.  reset != 0 starts from zeros (q_sum_ assigned 0.0f). */
void ko_q_accumulate(const float *q, uint32_t L, uint32_t T, uint32_t E, const uint32_t *tokens,
                     uint32_t n_list, int reset, float *q_sum) {
    for (uint32_t l = 0; l < L; ++l) {
        float *dst = q_sum + (size_t) l * E;
        if (reset) {
            for (uint32_t e = 0; e < E; ++e) {
                dst[e] = 0.0f;
            }
        }
        for (uint32_t i = 0; i < n_list; ++i) {
            const uint32_t t = tokens ? tokens[i] : i;
            const float *src = q + ((size_t) l * T + t) * E;
            for (uint32_t e = 0; e < E; ++e) {
                dst[e] += src[e];
            }
        }
    }
}
