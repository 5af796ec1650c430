/*
 * kvmem_oracle.h -- CPU restatement of the KVMem reselect path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code: only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only to check or time the product against.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the CrKcel/kvmem-llama.cpp tree).  The ggml quantizers
 * live in the un-vendored llama.cpp submodule (CrKcel/llama.cpp, branch
 * kvmem/prism on PrismML prism 9a9394a, see .gitmodules:1-3 and
 * patches/README.md:3); they are restated from ggml's published
 * quantize_row_{q8_0,q4_0,q5_0}_ref algorithm and anchored on the
 * reference's own CUDA restatement (src/adapter/llama-kvmem-stagein.cu:180-233).
 *
 * Pinning (what checks each function against something other than itself):
 *   ko_f32_to_f16 / ko_f16_to_f32 : numpy float16 (IEEE RNE), exhaustive f16.
 *   ko_quantize_row_*             : golden vectors from an independent numpy
 *                                   restatement (tests/golden), closed-form
 *                                   special groups, dequantisation bounds.
 *   ko_score_pertoken_max         : brute force fp64 numpy on tiny shapes,
 *                                   permutation / scaling invariants.
 *   ko_score_pertoken_max_f32     : the fp64 scorer above and an independent
 *                                   numpy brute force (1e-5 relative), over
 *                                   block sub-ranges, thread counts, head
 *                                   widths, GQA groups, partial tails.
 *   ko_pick_topk                  : the reference kvmem library compiled from
 *                                   its own sources (oracle/_ref), the
 *                                   reference's own unit-test cases, sort-based
 *                                   brute force.
 *   ko_meank_sum_f16 / ko_mean_k  : the reference RawKvStore (oracle/_ref),
 *                                   bit-exact; the reference's own
 *                                   cancellation pattern (raw_kv_store_test).
 *   ko_score_meank                : an independent float64 numpy restatement,
 *                                   closed forms (parallel / orthogonal /
 *                                   scaled directions, GQA head sums).
 *   ko_rope_sincos                : float64 libm sin/cos rounded to fp32 over
 *                                   10^6 angles up to 2^20 rad, quadrant
 *                                   identities, exact multiples of pi/2.
 *   ko_rope_rows                  : the reference's own RoPE (rope.cpp via
 *                                   oracle/_ref) within fp32 rounding, its unit
 *                                   test (position 0 = identity), float64
 *                                   rotation, pair norms preserved.
 *   ko_hadamard_rows              : float64 Sylvester matrix products, H H = I,
 *                                   exact images of unit vectors.
 *   ko_q_accumulate               : exact integer sums, an order-sensitive
 *                                   cancellation sequence only the token-order
 *                                   fp32 sum reproduces, float64 error bound.
 */
#ifndef KVMEM_ORACLE_H
#define KVMEM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type codes for the formats on this path (ggml.h enum values). */
enum { KO_TYPE_F32 = 0, KO_TYPE_F16 = 1, KO_TYPE_Q4_0 = 2, KO_TYPE_Q5_0 = 6, KO_TYPE_Q8_0 = 8 };

/* Half precision <-> single precision, IEEE round-to-nearest-even.
 * raw_kv_store.cpp:22-56 (f32_to_f16) and :58-83 (f16_to_f32). */
uint16_t ko_f32_to_f16(float f);
float    ko_f16_to_f32(uint16_t h);
float    ko_bf16_to_f32(uint16_t h);

/* Bytes of one 32-element group, and of a row of n elements. */
size_t ko_group_bytes(int type);
size_t ko_row_bytes(int type, int64_t n);

/* ggml quantize_row_*_ref restated; k must be a multiple of 32.
 * q8_0: llama-kvmem-stagein.cu:180-198; q4_0: :200-233; q5_0: ggml only. */
void ko_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k);
void ko_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k);
void ko_quantize_row_q5_0(const float *x, uint8_t *y, int64_t k);

/* Floats in [lo, hi) (non-negative) where roundf(s) differs from
 * truncf(s + 0.49999997f): the stage-in's q8_0 rounding, checked over every
 * float of the range |x*id| can take. */
uint64_t ko_round_trick_mismatches(float lo, float hi);
/* Floats with bits in [lo_bits, hi_bits) where the stage-in's division-free
 * a / 127 (product with RN(1/127), one FMA residual, one FMA correction)
 * differs from the IEEE quotient. */
uint64_t ko_div127_mismatches(uint32_t lo_bits, uint32_t hi_bits);

/* Dequantisation (inverse maps, used for error-bound invariants).
 * q8_0 / q4_0: llama-kvmem-stagein.cu:132-157. */
void ko_dequantize_row(int type, const uint8_t *y, float *x, int64_t k);

/* F16 rows -> packed rows of `type` (F16 rows are converted exactly to f32
 * first, as ggml_quantize_chunk does; llama-kvmem-quant.h:96-119).
 * type KO_TYPE_F16 copies the rows unchanged. */
int ko_quantize_rows_f16(int type, const uint16_t *src, uint8_t *dst,
                         int64_t n_rows, int64_t n_embd);

/* Stage-in of whole blocks into a slot pool:
 * src  : [n_blocks][block_tokens][n_embd] f16 (one layer, one of K/V)
 * slots: slot of each block; pool row (cell) = slot*block_tokens + t
 *        (llama-kvmem-batch.cpp:48, llama-memory-kvmem.cpp:2742)
 * pool : n_slots*block_tokens rows of ko_row_bytes(type, n_embd).
 * Returns 0, or -1 on a bad argument (slot out of range). */
int ko_stagein_blocks(int type, const uint16_t *src, const uint32_t *slots,
                      uint32_t n_blocks, uint32_t block_tokens, uint32_t n_embd,
                      uint8_t *pool, uint32_t n_slots);

/* Per-token max scorer (the retrieval scorer of the reselect step):
 *   s[l][b] = max_{t, hq, j<n_tok(b)} (q[l][t][hq] . k[l][b][j][hq/g]) / sqrt(D)
 * q: [L][Tq][Hq][D] f32 (exact image of the bf16 query), k: [L][B][T][Hkv][D]
 * f16 bits.  Accumulates in double.  layer_scores: [L][B].  The reference
 * scorer it replaces is mean-K cosine (llama-memory-kvmem.cpp:2869-2916);
 * GQA head map hq -> hq/g follows :2890-2892.  block_ids (optional) restricts
 * the computation to the listed blocks (others untouched). */
void ko_score_pertoken_max(const float *q, const uint16_t *k,
                           uint32_t L, uint32_t Tq, uint32_t Hq, uint32_t Hkv,
                           uint32_t D, uint32_t B, uint32_t T,
                           uint32_t last_block_tokens,
                           const uint32_t *block_ids, uint32_t n_ids,
                           double *layer_scores);

/* Same computation with fp32 accumulation, written for speed: the CPU
 * baseline of the scoring step and the checker of the full-size scoring
 * tests.  Fills columns [b_begin, b_end) of layer_scores; block B-1 has
 * last_block_tokens keys when nonzero.  n_threads <= 0 = all. */
void ko_score_pertoken_max_f32(const float *q, const uint16_t *k,
                               uint32_t L, uint32_t Tq, uint32_t Hq, uint32_t Hkv,
                               uint32_t D, uint32_t B, uint32_t T,
                               uint32_t last_block_tokens,
                               uint32_t b_begin, uint32_t b_end,
                               float *layer_scores, int n_threads);

/* Layer combination of per-layer scores into one score per block:
 * mode 0 = mean (layer averaging as llama-memory-kvmem.cpp:2910-2913),
 * 1 = max, 2 = sum. */
void ko_combine_layers(const double *layer_scores, uint32_t L, uint32_t B,
                       int mode, double *scores);

/* Top-k selection of KvMemStore::pick_topk_ungrouped (TopK policy),
 * kvmem_store.cpp:482-623: keep [0,sink), then mandatory ids newest-first,
 * then the last `recent` ids, then the best remaining scores; returns the
 * kept ids ascending in out (capacity n), count in *n_out.
 * tie_lower_index = 1: equal scores prefer the LOWER id (reselect contract);
 *                   0: equal scores prefer the higher id (kvmem_store.cpp:602-609). */
void ko_pick_topk(const double *scores, uint32_t n, uint32_t budget,
                  uint32_t sink, uint32_t recent,
                  const uint32_t *mandatory, uint32_t n_mandatory,
                  int tie_lower_index, uint32_t *out, uint32_t *n_out);

/* Mean-K producer of the reference (RawKvStore::capture_mean_f16,
 * raw_kv_store.cpp:184-202): fp32 sum of n_tokens F16 rows in token order. */
void ko_meank_sum_f16(const uint16_t *rows, uint32_t n_tokens, uint32_t n_embd,
                      uint64_t row_stride, float *k_sum);
/* RawKvStore::mean_k normalisation (raw_kv_store.cpp:984-995). */
void ko_mean_k(const float *k_sum, uint32_t mean_tokens, uint32_t n_embd, float *out);
/* The reference's retrieval scorer, mean-K cosine
 * (llama-memory-kvmem.cpp:2869-2916): q_sum [L][Hq*D], q_count [L],
 * k_sum [L][B][Hkv*D], mean_tokens [L][B] -> scores [B] (double). */
void ko_score_meank(const float *q_sum, const uint32_t *q_count, const float *k_sum,
                    const uint32_t *mean_tokens, uint32_t L, uint32_t B, uint32_t Hq,
                    uint32_t Hkv, uint32_t D, double *scores);

/* Cache row transform of the raw-K stage-in (llama-kvmem-stagein.cu:
 * 704-740): ko_rope_sincos is the library's own sin/cos of an fp32 angle
 * (fp64 Cody-Waite reduction, Taylor polynomials, one rounding);
 * ko_rope_rows the NeoX RoPE of rope_neox_kernel (:159-178, rope.cpp:8-45)
 * at positions pos0 + t; ko_hadamard_rows fwht_kernel (:104-130) over runs
 * of `width` with scale 1/sqrtf(width); ko_quantize_rows_f32 quantizes fp32
 * rows (F16: RNE). */
void ko_rope_sincos(float a, float *sn, float *cs);
void ko_rope_sincos_n(const float *a, uint64_t n, float *sn, float *cs);
void ko_rope_rows(float *rows, uint32_t n_rows, uint32_t n_embd, uint32_t head_dim,
                  uint32_t n_rot, const float *theta, int32_t pos0);
void ko_hadamard_rows(float *x, uint64_t n_elems, uint32_t width);
int ko_quantize_rows_f32(int type, const float *src, uint8_t *dst, int64_t n_rows, int64_t n_embd);

/* The reference's query harvest (llama-memory-kvmem.cpp:2164-2172):
 * q [L][T][E] f32; q_sum[l] (+)= q[l][tokens[i]] for i < n_list in order
 * (tokens NULL = 0..n_list-1); reset != 0 starts from zeros. */
void ko_q_accumulate(const float *q, uint32_t L, uint32_t T, uint32_t E, const uint32_t *tokens,
                     uint32_t n_list, int reset, float *q_sum);

/* Number of OpenMP threads the oracle uses (for the baseline's core count). */
int ko_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
