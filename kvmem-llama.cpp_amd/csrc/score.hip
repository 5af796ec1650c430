// Per-token max block scorer on the CDNA4 matrix cores.
//
// For layer l, KV head h and block b the scorer needs
//     max_{query rows r of group h, keys j of block b} q_r . k_j
// where the query rows of group h are the (token, head) pairs with head in
// [h*g, (h+1)*g) (GQA, llama-memory-kvmem.cpp:2890-2892).  That is a small
// GEMM (rows x 128 keys x head_dim) whose output is reduced by max at once.
//
// Mapping.  A workgroup of 8 waves owns one (layer, KV head, 384-row slice)
// and a contiguous range of blocks.  Each wave keeps 48 query rows resident
// in VGPRs as f16 A-fragments of v_mfma_f32_16x16x32_f16 (loaded once;
// bf16 queries are converted to f16 on the way, exact for normal-range
// values).  Every block's K tile (128 keys x head_dim halves) is copied
// from HBM to LDS once per workgroup (row stride padded by 16 bytes so the
// 16 keys of a B-fragment read hit distinct banks) and consumed by all 8
// waves; the next block's tile is prefetched into registers while the
// current one is multiplied.  Out-of-range query rows and keys (partial
// last block, row count not a multiple of 384) are replaced by duplicates
// of valid ones, which leaves the max unchanged and needs no masking.
//
// Dispatch order is XCD-aware: consecutive workgroup ids go to different
// XCDs, so the id is decoded such that each XCD works through its own set
// of (layer, head) pairs, keeping their query rows resident in that XCD's
// L2, and row slices of the same block range run next to each other.
#include "kvmem_internal.hpp"

#include <algorithm>
#include <cmath>

namespace kvmem_hip {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kScoreWaves = 8;
constexpr int kScoreThreads = kScoreWaves * 64;
constexpr int kRowTiles = 3;                            // 16-row tiles per wave
constexpr int kRowsPerWave = kRowTiles * 16;            // 48
constexpr int kRowsPerGroup = kScoreWaves * kRowsPerWave;  // 384
constexpr int kMaxTokens = 128;                         // keys per LDS tile

struct ScoreParams {
    const uint16_t *q;       // [L][Tq][Hq][D] bf16 or f16 bits
    const uint8_t *k;        // [L][B][T][Hkv][D] f16
    float *partial;          // [RG][L][Hkv][B]
    uint32_t L, Tq, Hq, Hkv, B, T, last_T, g, R, RG;
    uint32_t cap;            // blocks per layer in memory (>= B)
    uint32_t n_chunks;       // block chunks per (l, h, row slice)
    uint32_t blocks_per_chunk;
    uint32_t q_bf16;
    uint32_t xcd_major;      // 1 if (L*Hkv) % 8 == 0
    float scale;             // 1/sqrt(D)
};

__device__ inline _Float16 q_elem_to_half(uint16_t bits, bool bf16) {
    if (bf16) {
        const float f = __uint_as_float(static_cast<uint32_t>(bits) << 16);
        return static_cast<_Float16>(f);
    }
    return __builtin_bit_cast(_Float16, bits);
}

template <int D>
__global__ __launch_bounds__(kScoreThreads, 1) void score_kernel(ScoreParams p) {
    constexpr int KS = D / 32;                       // k-steps of 32
    constexpr int ROW_BYTES = D * 2;
    constexpr int LDS_STRIDE = ROW_BYTES + 16;       // padded key row
    constexpr int PIECES = kMaxTokens * D / 8;       // 16-byte pieces per tile
    constexpr int PER_THREAD = PIECES / kScoreThreads;
    static_assert(PIECES % kScoreThreads == 0, "tile must split evenly");
    constexpr int PIECES_PER_ROW = D / 8;

    __shared__ __attribute__((aligned(16))) uint8_t tile[kMaxTokens * LDS_STRIDE];
    __shared__ float red[kScoreWaves];

    // ---- decode (layer, head, row slice, chunk) from the workgroup id
    const uint32_t pairs = p.L * p.Hkv;
    uint32_t lh, chunk, rg;
    {
        const uint32_t i = blockIdx.x;
        if (p.xcd_major) {
            const uint32_t xcd = i & 7u;
            const uint32_t local = i >> 3;
            rg = local % p.RG;
            const uint32_t rest = local / p.RG;
            chunk = rest % p.n_chunks;
            lh = (rest / p.n_chunks) * 8u + xcd;
        } else {
            rg = i % p.RG;
            const uint32_t rest = i / p.RG;
            chunk = rest % p.n_chunks;
            lh = rest / p.n_chunks;
        }
    }
    if (lh >= pairs) {
        return;
    }
    const uint32_t l = lh / p.Hkv;
    const uint32_t h = lh - l * p.Hkv;
    const uint32_t b_begin = chunk * p.blocks_per_chunk;
    const uint32_t b_end = min(p.B, b_begin + p.blocks_per_chunk);
    if (b_begin >= b_end) {
        return;
    }

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t lrow = lane & 15u;   // row (A) / key (B) within a 16-tile
    const uint32_t kgrp = lane >> 4;    // which 8 of the 32 k-values

    // ---- query rows -> A fragments (resident for the whole workgroup)
    half8_t a[kRowTiles][KS];
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
        uint32_t r = rg * kRowsPerGroup + wave * kRowsPerWave + rt * 16 + lrow;
        r = min(r, p.R - 1u);                       // duplicate the last valid row
        const uint32_t t = r / p.g;
        const uint32_t hq = h * p.g + (r - t * p.g);
        const uint16_t *qrow = p.q + ((static_cast<uint64_t>(l) * p.Tq + t) * p.Hq + hq) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(qrow + ks * 32 + kgrp * 8);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
            half8_t v;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = q_elem_to_half(static_cast<uint16_t>(w[i] & 0xffffu), p.q_bf16 != 0);
                v[2 * i + 1] = q_elem_to_half(static_cast<uint16_t>(w[i] >> 16), p.q_bf16 != 0);
            }
            a[rt][ks] = v;
        }
    }

    // ---- K tile prefetch: piece -> (key, part); keys beyond the block's
    // tokens read the block's last valid key.
    const uint64_t key_stride = static_cast<uint64_t>(p.Hkv) * ROW_BYTES;  // bytes between keys
    auto block_base = [&](uint32_t b) -> const uint8_t * {
        return p.k + ((static_cast<uint64_t>(l) * p.cap + b) * p.T) * key_stride +
               static_cast<uint64_t>(h) * ROW_BYTES;
    };
    auto n_tokens = [&](uint32_t b) -> uint32_t {
        return (b + 1 == p.B && p.last_T != 0) ? p.last_T : p.T;
    };
    uint4 pre[PER_THREAD];
    auto prefetch = [&](uint32_t b) {
        const uint8_t *base = block_base(b);
        const uint32_t nt = n_tokens(b);
#pragma unroll
        for (int s = 0; s < PER_THREAD; ++s) {
            const uint32_t piece = tid + s * kScoreThreads;
            const uint32_t key = min(piece / PIECES_PER_ROW, nt - 1u);
            const uint32_t part = piece % PIECES_PER_ROW;
            pre[s] = load_stream16(base + key * key_stride + part * 16u);
        }
    };

    prefetch(b_begin);
    for (uint32_t b = b_begin; b < b_end; ++b) {
        __syncthreads();  // previous block's tile fully consumed, red[] written
        if (tid == 0 && b > b_begin) {
            float m = red[0];
#pragma unroll
            for (int w = 1; w < kScoreWaves; ++w) {
                m = fmaxf(m, red[w]);
            }
            p.partial[((static_cast<uint64_t>(rg) * p.L + l) * p.Hkv + h) * p.B + (b - 1)] = m * p.scale;
        }
#pragma unroll
        for (int s = 0; s < PER_THREAD; ++s) {
            const uint32_t piece = tid + s * kScoreThreads;
            const uint32_t key = piece / PIECES_PER_ROW;
            const uint32_t part = piece % PIECES_PER_ROW;
            *reinterpret_cast<uint4 *>(tile + key * LDS_STRIDE + part * 16u) = pre[s];
        }
        __syncthreads();
        if (b + 1 < b_end) {
            prefetch(b + 1);
        }

        float m = -INFINITY;
#pragma unroll 1
        for (int kt = 0; kt < kMaxTokens / 16; ++kt) {
            const uint8_t *krow = tile + (kt * 16 + lrow) * LDS_STRIDE + kgrp * 16;
            half8_t bf[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                bf[ks] = *reinterpret_cast<const half8_t *>(krow + ks * 64);
            }
            float4_t acc[kRowTiles];
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                acc[rt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int rt = 0; rt < kRowTiles; ++rt) {
                    acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rt][ks], bf[ks], acc[rt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                m = fmaxf(m, fmaxf(fmaxf(acc[rt][0], acc[rt][1]), fmaxf(acc[rt][2], acc[rt][3])));
            }
        }
        // wave max -> red[wave]
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            m = fmaxf(m, __shfl_xor(m, off, 64));
        }
        if (lane == 0) {
            red[wave] = m;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float m = red[0];
#pragma unroll
        for (int w = 1; w < kScoreWaves; ++w) {
            m = fmaxf(m, red[w]);
        }
        p.partial[((static_cast<uint64_t>(rg) * p.L + l) * p.Hkv + h) * p.B + (b_end - 1)] = m * p.scale;
    }
}

// scores[b] = reduce_l max_{rg, h} partial[rg][l][h][b]
__global__ __launch_bounds__(256) void score_finalize_kernel(const float *partial, uint32_t RG,
                                                             uint32_t L, uint32_t Hkv, uint32_t B,
                                                             int mode, float *layer_scores,
                                                             float *scores) {
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) {
        return;
    }
    float acc = mode == KVMEM_LAYER_MAX ? -INFINITY : 0.0f;
    for (uint32_t l = 0; l < L; ++l) {
        float best = -INFINITY;
        for (uint32_t rg = 0; rg < RG; ++rg) {
            for (uint32_t h = 0; h < Hkv; ++h) {
                best = fmaxf(best, partial[((static_cast<uint64_t>(rg) * L + l) * Hkv + h) * B + b]);
            }
        }
        if (layer_scores) {
            layer_scores[static_cast<uint64_t>(l) * B + b] = best;
        }
        acc = mode == KVMEM_LAYER_MAX ? fmaxf(acc, best) : acc + best;
    }
    if (mode == KVMEM_LAYER_MEAN && L > 0) {
        acc = acc / static_cast<float>(L);
    }
    scores[b] = acc;
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" int kvmem_hip_score(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                               const kvmem_hip_score_args *args) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!hist || !args || !hist->k || !args->q || !args->scores) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: null argument");
    }
    const uint32_t D = args->head_dim;
    if (D != 128 && D != 256) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "score: head_dim must be 128 or 256");
    }
    if (args->n_head_kv == 0 || args->n_head % args->n_head_kv != 0 || args->n_q_tokens == 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: n_head must be a positive multiple of n_head_kv");
    }
    if (hist->n_embd_k != args->n_head_kv * D) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: history n_embd_k != n_head_kv*head_dim");
    }
    if (hist->block_tokens == 0 || hist->block_tokens > static_cast<uint32_t>(kMaxTokens) ||
        hist->last_block_tokens > hist->block_tokens) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "score: block_tokens must be in [1, 128]");
    }
    if (args->q_type != KVMEM_TYPE_BF16 && args->q_type != KVMEM_TYPE_F16) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "score: query must be bf16 or f16");
    }
    if (args->layer_reduce < KVMEM_LAYER_MEAN || args->layer_reduce > KVMEM_LAYER_SUM) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: bad layer_reduce");
    }
    if ((reinterpret_cast<uintptr_t>(hist->k) & 15u) || (reinterpret_cast<uintptr_t>(args->q) & 15u)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: q and k must be 16-byte aligned");
    }
    const uint32_t L = hist->n_layers;
    const uint32_t B = hist->n_blocks;
    if (L == 0 || B == 0) {
        return KVMEM_HIP_OK;
    }
    ScoreParams p{};
    p.q = static_cast<const uint16_t *>(args->q);
    p.k = static_cast<const uint8_t *>(hist->k);
    p.L = L;
    p.Tq = args->n_q_tokens;
    p.Hq = args->n_head;
    p.Hkv = args->n_head_kv;
    p.B = B;
    p.cap = hist->capacity_blocks ? hist->capacity_blocks : B;
    if (p.cap < B) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: capacity_blocks below n_blocks");
    }
    p.T = hist->block_tokens;
    p.last_T = hist->last_block_tokens;
    p.g = args->n_head / args->n_head_kv;
    p.R = p.Tq * p.g;
    p.RG = (p.R + kRowsPerGroup - 1) / kRowsPerGroup;
    p.q_bf16 = args->q_type == KVMEM_TYPE_BF16;
    p.scale = 1.0f / std::sqrt(static_cast<float>(D));
    const uint32_t pairs = L * p.Hkv;
    // about four workgroups per CU over the whole launch
    const uint32_t target = 1024;
    const uint32_t per_chunk_target = std::max<uint32_t>(1, target / std::max<uint32_t>(1, pairs * p.RG));
    p.n_chunks = std::min(B, per_chunk_target);
    p.blocks_per_chunk = (B + p.n_chunks - 1) / p.n_chunks;
    p.n_chunks = (B + p.blocks_per_chunk - 1) / p.blocks_per_chunk;
    p.xcd_major = (pairs % 8u) == 0;

    (void) hipSetDevice(ctx->device);
    const size_t partial_bytes = sizeof(float) * static_cast<size_t>(p.RG) * L * p.Hkv * B;
    if (!ensure_dev(ctx, ctx->score_partial, partial_bytes, "score partial")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    p.partial = static_cast<float *>(ctx->score_partial.ptr);
    const uint64_t n_wg = static_cast<uint64_t>(pairs) * p.RG * p.n_chunks;
    const uint64_t grid = p.xcd_major ? n_wg : n_wg;
    if (grid > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: problem too large for one launch");
    }
    perf_begin(ctx, kPerfScore);
    if (D == 256) {
        score_kernel<256><<<static_cast<uint32_t>(grid), kScoreThreads, 0, ctx->stream>>>(p);
    } else {
        score_kernel<128><<<static_cast<uint32_t>(grid), kScoreThreads, 0, ctx->stream>>>(p);
    }
    perf_end(ctx, kPerfScore);
    if (!hip_ok(ctx, hipGetLastError(), "score kernel launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    // the layer combination is timed with the selection stage
    perf_begin(ctx, kPerfTopk);
    score_finalize_kernel<<<(B + 255) / 256, 256, 0, ctx->stream>>>(
        p.partial, p.RG, L, p.Hkv, B, args->layer_reduce, args->layer_scores, args->scores);
    perf_end(ctx, kPerfTopk);
    if (!hip_ok(ctx, hipGetLastError(), "score finalize launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    return KVMEM_HIP_OK;
}
