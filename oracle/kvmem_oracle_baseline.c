/*
 * kvmem_oracle_baseline.c -- fp32 CPU implementation of the per-token max
 * scorer, written to vectorise (K transposed per head so the inner loop runs
 * over keys).  Two uses: the CPU baseline timed beside the GPU scorer, and
 * the checker of the full-size scoring tests (16 layers x 2048 blocks is out
 * of reach of the fp64 scorer in test time).  It is pinned on the CPU
 * against the fp64 ko_score_pertoken_max and an independent numpy brute
 * force, over block sub-ranges, thread counts, head_dim 128 / 256, GQA
 * groups and a partial last block (tests/test_cpu_oracle.py).
 *
 * TEST INFRASTRUCTURE ONLY (see kvmem_oracle.h).
 */
#include "kvmem_oracle.h"

#include <math.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void ko_score_pertoken_max_f32(const float *q, const uint16_t *k,
                               uint32_t L, uint32_t Tq, uint32_t Hq, uint32_t Hkv,
                               uint32_t D, uint32_t B, uint32_t T,
                               uint32_t last_block_tokens,
                               uint32_t b_begin, uint32_t b_end,
                               float *layer_scores, int n_threads) {
    const uint32_t g = Hq / Hkv;
    const float inv = 1.0f / sqrtf((float) D);
#ifdef _OPENMP
    if (n_threads <= 0) {
        n_threads = omp_get_max_threads();
    }
#endif
#pragma omp parallel num_threads(n_threads)
    {
        float *kt = (float *) malloc(sizeof(float) * (size_t) T * D);
        float *acc = (float *) malloc(sizeof(float) * (size_t) T);
#pragma omp for schedule(dynamic, 1)
        for (uint32_t b = b_begin; b < b_end; ++b) {
            /* keys of the block: T, or last_block_tokens for a partial tail */
            const uint32_t nt = (b + 1 == B && last_block_tokens) ? last_block_tokens : T;
            for (uint32_t l = 0; l < L; ++l) {
                float best = -INFINITY;
                for (uint32_t h = 0; h < Hkv; ++h) {
                    for (uint32_t j = 0; j < nt; ++j) {
                        const uint16_t *kr =
                            k + ((((size_t) l * B + b) * T + j) * Hkv + h) * D;
                        for (uint32_t d = 0; d < D; ++d) {
                            kt[(size_t) d * nt + j] = ko_f16_to_f32(kr[d]);
                        }
                    }
                    for (uint32_t r = 0; r < Tq * g; ++r) {
                        const uint32_t t = r / g;
                        const uint32_t gi = r % g;
                        const float *qr =
                            q + (((size_t) l * Tq + t) * Hq + h * g + gi) * D;
                        for (uint32_t j = 0; j < nt; ++j) {
                            acc[j] = 0.0f;
                        }
                        for (uint32_t d = 0; d < D; ++d) {
                            const float qv = qr[d];
                            const float *kd = kt + (size_t) d * nt;
                            for (uint32_t j = 0; j < nt; ++j) {
                                acc[j] += qv * kd[j];
                            }
                        }
                        for (uint32_t j = 0; j < nt; ++j) {
                            best = acc[j] > best ? acc[j] : best;
                        }
                    }
                }
                layer_scores[(size_t) l * B + b] = best * inv;
            }
        }
        free(kt);
        free(acc);
    }
}
