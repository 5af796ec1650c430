/*
 * kvmem_oracle_select.c -- per-token max block scorer (fp64 truth), layer
 * combination and the KvMemStore top-k selection, restated as the tests'
 * reference.
 *
 * TEST INFRASTRUCTURE ONLY (see kvmem_oracle.h).
 */
#include "kvmem_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int ko_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* s[l][b] = max over query rows (t, hq) of group h and keys j < n_tok(b) of
 * q.k / sqrt(D), accumulated in double.  GQA: query head hq reads KV head
 * hq / g (llama-memory-kvmem.cpp:2890-2892, qh_i = h*g + gi). */
void ko_score_pertoken_max(const float *q, const uint16_t *k,
                           uint32_t L, uint32_t Tq, uint32_t Hq, uint32_t Hkv,
                           uint32_t D, uint32_t B, uint32_t T,
                           uint32_t last_block_tokens,
                           const uint32_t *block_ids, uint32_t n_ids,
                           double *layer_scores) {
    const uint32_t g = Hq / Hkv;
    const double inv = 1.0 / sqrt((double) D);
    const uint32_t n = block_ids ? n_ids : B;
#pragma omp parallel
    {
        double *kd = (double *) malloc(sizeof(double) * (size_t) T * D);
        double *qd = (double *) malloc(sizeof(double) * (size_t) D);
#pragma omp for schedule(dynamic, 1)
        for (uint32_t ii = 0; ii < n; ++ii) {
            const uint32_t b = block_ids ? block_ids[ii] : ii;
            const uint32_t ntok =
                (b + 1 == B && last_block_tokens != 0) ? last_block_tokens : T;
            for (uint32_t l = 0; l < L; ++l) {
                double best = -INFINITY;
                for (uint32_t h = 0; h < Hkv; ++h) {
                    for (uint32_t j = 0; j < ntok; ++j) {
                        const uint16_t *kr =
                            k + ((((size_t) l * B + b) * T + j) * Hkv + h) * D;
                        for (uint32_t d = 0; d < D; ++d) {
                            kd[(size_t) j * D + d] = (double) ko_f16_to_f32(kr[d]);
                        }
                    }
                    for (uint32_t t = 0; t < Tq; ++t) {
                        for (uint32_t gi = 0; gi < g; ++gi) {
                            const float *qr =
                                q + (((size_t) l * Tq + t) * Hq + h * g + gi) * D;
                            for (uint32_t d = 0; d < D; ++d) {
                                qd[d] = (double) qr[d];
                            }
                            for (uint32_t j = 0; j < ntok; ++j) {
                                const double *kj = kd + (size_t) j * D;
                                double dot = 0.0;
                                for (uint32_t d = 0; d < D; ++d) {
                                    dot += qd[d] * kj[d];
                                }
                                if (dot > best) {
                                    best = dot;
                                }
                            }
                        }
                    }
                }
                layer_scores[(size_t) l * B + b] = best * inv;
            }
        }
        free(kd);
        free(qd);
    }
}

/* Layer combination.  Mean follows the reference's layer averaging
 * (llama-memory-kvmem.cpp:2910-2913: acc += layer, score = acc / nlay). */
void ko_combine_layers(const double *layer_scores, uint32_t L, uint32_t B,
                       int mode, double *scores) {
    for (uint32_t b = 0; b < B; ++b) {
        double acc = mode == 1 ? -INFINITY : 0.0;
        for (uint32_t l = 0; l < L; ++l) {
            const double v = layer_scores[(size_t) l * B + b];
            if (mode == 1) {
                acc = v > acc ? v : acc;
            } else {
                acc += v;
            }
        }
        scores[b] = (mode == 0 && L > 0) ? acc / (double) L : acc;
    }
}

/* ------------------------------------------------------------------------ */
/* Top-k (kvmem_store.cpp:482-623, KvMemSelectPolicy::TopK)                 */
/* ------------------------------------------------------------------------ */

static const double *g_scores;
static int g_tie_lower;

/* Strict total order "a ranks before b": higher score first; equal scores
 * by id (lower first for the reselect contract, higher first for the
 * reference's recency rule, kvmem_store.cpp:602-609). */
static int rank_cmp(const void *pa, const void *pb) {
    const uint32_t a = *(const uint32_t *) pa;
    const uint32_t b = *(const uint32_t *) pb;
    const double sa = g_scores[a];
    const double sb = g_scores[b];
    if (sa != sb) {
        return sa > sb ? -1 : 1;
    }
    if (g_tie_lower) {
        return a < b ? -1 : 1;
    }
    return a > b ? -1 : 1;
}

void ko_pick_topk(const double *scores, uint32_t n, uint32_t budget,
                  uint32_t sink, uint32_t recent,
                  const uint32_t *mandatory, uint32_t n_mandatory,
                  int tie_lower_index, uint32_t *out, uint32_t *n_out) {
    *n_out = 0;
    if (n == 0) {
        return;
    }
    if (budget == 0 || n <= budget) {                 /* everything fits */
        for (uint32_t i = 0; i < n; ++i) {
            out[i] = i;
        }
        *n_out = n;
        return;
    }
    uint8_t *kept = (uint8_t *) calloc(n, 1);
    uint32_t count = 0;
#define KO_KEEP(id)                                      \
    do {                                                 \
        const uint32_t id_ = (id);                       \
        if (id_ < n && !kept[id_]) {                     \
            kept[id_] = 1;                               \
            ++count;                                     \
        }                                                \
    } while (0)
    const uint32_t s = sink < n ? sink : n;
    for (uint32_t i = 0; i < s && count < budget; ++i) {
        KO_KEEP(i);
    }
    /* mandatory ids: the last listed (newest) first, until the budget */
    for (uint32_t i = n_mandatory; i > 0 && count < budget; --i) {
        KO_KEEP(mandatory[i - 1]);
    }
    const uint32_t r = recent < n ? recent : n;
    for (uint32_t i = 0; i < r && count < budget; ++i) {
        KO_KEEP(n - 1 - i);
    }
    if (count < budget) {
        uint32_t *cand = (uint32_t *) malloc(sizeof(uint32_t) * n);
        uint32_t nc = 0;
        for (uint32_t i = 0; i < n; ++i) {
            if (!kept[i]) {
                cand[nc++] = i;
            }
        }
        const uint32_t need = budget - count;
        g_scores = scores;
        g_tie_lower = tie_lower_index;
        qsort(cand, nc, sizeof(uint32_t), rank_cmp);
        for (uint32_t i = 0; i < need && i < nc; ++i) {
            KO_KEEP(cand[i]);
        }
        free(cand);
    }
#undef KO_KEEP
    for (uint32_t i = 0; i < n; ++i) {
        if (kept[i]) {
            out[(*n_out)++] = i;
        }
    }
    free(kept);
}
