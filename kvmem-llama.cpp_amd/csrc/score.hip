// Per-token max block scorer on the CDNA4 matrix cores.
//
// For layer l, KV head h and block b the scorer needs
//     max_{query rows r of group h, keys j of block b} q_r . k_j
// where the query rows of group h are the (token, head) pairs with head in
// [h*g, (h+1)*g) (GQA, llama-memory-kvmem.cpp:2890-2892).  That is a small
// GEMM (rows x 128 keys x head_dim) whose output is reduced by max at once,
// so no score ever goes to memory.
//
// Mapping.  A workgroup of 4 waves (one per SIMD) owns one (layer, KV head,
// 384-row slice) and a contiguous range of blocks; two workgroups share a
// CU, so each SIMD runs two waves that cover each other's barrier and
// load waits.  Each wave keeps 96 query rows resident in VGPRs as f16
// A-fragments of v_mfma_f32_16x16x32_f16 (loaded once; bf16 queries are
// converted to f16 on the way, exact for normal-range values, a wave's rows
// scaled by a power of two first when they would overflow f16), so every
// 16-byte B-fragment read from LDS feeds six MFMAs (two reads kept in
// flight ahead of their MFMAs).  Half a block's K tile
// (64 keys x head_dim halves of one KV head, 32 KiB) moves HBM -> LDS with
// global_load_lds_dwordx4 (no register staging) into one of two LDS
// buffers while the other buffer's keys are multiplied: one barrier per
// half block.  The per-block max over the wave's lanes uses DPP and the
// row-swap permutes, not LDS.  Inside a tile the
// 16-byte chunk c of key j sits at chunk position c ^ (j mod chunks-per-
// key), so the 16 keys of a B-fragment read hit 16 different bank groups;
// the swizzle is applied on the global side (each lane of a direct LDS load
// fetches the chunk that belongs to its fixed LDS slot).  Out-of-range
// query rows and keys (partial last block, row count not a multiple of
// 384) are replaced by duplicates of valid ones, which leaves the max
// unchanged and needs no masking.  Each wave writes its own per-block max
// to a partial array; a small kernel folds waves, row slices, KV heads and
// layers.
//
// The file is built with finite-math semantics (max needs no NaN
// canonicalisation); every identity is -FLT_MAX and inputs are finite F16.
//
// Dispatch order is XCD-aware: consecutive workgroup ids go to different
// XCDs, so the id is decoded such that each XCD works through its own set
// of (layer, head) pairs, keeping their query rows resident in that XCD's
// L2.
#include "kvmem_internal.hpp"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <mutex>
#include <string>

namespace kvmem_hip {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kScoreWaves = 4;
constexpr int kScoreThreads = kScoreWaves * 64;
constexpr int kRowTiles = 6;                               // 16-row tiles per wave
constexpr int kRowsPerWave = kRowTiles * 16;               // 96
constexpr int kRowsPerGroup = kScoreWaves * kRowsPerWave;  // 384
constexpr int kMaxTokens = 128;                            // keys per block (at most)
constexpr int kTileKeys = 64;                              // keys per LDS tile (half a block)
// Cache policy of the tile DMA: nt (streamed once; keeps L2 for the query
// rows, and costs less energy in the power-capped regime this kernel runs in).
constexpr int kDmaNonTemporal = 2;

struct ScoreParams {
    const uint16_t *q;       // [L][Tq][Hq][D] bf16 or f16 bits
    const uint8_t *k;        // [L][cap][T][Hkv][D] f16
    float *partial;          // [RG * kScoreWaves][L][Hkv][B]
    uint32_t L, Tq, Hq, Hkv, B, T, last_T, g, R, RG;
    uint32_t cap;            // blocks per layer in memory (>= B)
    uint32_t n_chunks;       // block chunks per (l, h, row slice)
    uint32_t blocks_per_chunk;
    uint32_t q_bf16;
    uint32_t xcd_major;      // 1 if (L*Hkv) % 8 == 0
    float scale;             // 1/sqrt(D)
};

// Max over the 64 lanes of a wave without LDS: DPP within each 16-lane row
// (quad permutes, then row rotations by 4 and 8; max is idempotent, so the
// overlapping windows are harmless), then the gfx950 row swaps, which hand
// every lane the value of the other 16-lane row and of the other 32-lane
// half.  Every lane ends with the wave maximum.
__device__ inline float wave_max(float m) {
    int x = __float_as_int(m);
    m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false)));
    x = __float_as_int(m);
    m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false)));
    x = __float_as_int(m);
    m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x124, 0xF, 0xF, false)));
    x = __float_as_int(m);
    m = __builtin_fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x128, 0xF, 0xF, false)));
    const uint32_t u = __float_as_uint(m);
    const auto s16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    m = __builtin_fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
    const uint32_t v = __float_as_uint(m);
    const auto s32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __builtin_fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

// A bf16 value (its bits in the top half of `f32_bits`, the rest zero) ->
// f16, times qscale (a power of two, exact) before the rounding.
__device__ inline _Float16 bf16_to_half(uint32_t f32_bits, float qscale) {
    return static_cast<_Float16>(__uint_as_float(f32_bits) * qscale);
}

// A wave's query rows as raw 16-bit A fragments (bf16 or f16 bits, not yet
// converted).  Returns the largest |q| bit pattern the lane loaded.
template <int D, int KS>
__device__ __forceinline__ uint32_t load_query_bits(const ScoreParams &p, half8_t (&a)[kRowTiles][KS],
                                                    uint32_t l, uint32_t h, uint32_t rg, uint32_t wave,
                                                    uint32_t lrow, uint32_t kgrp) {
    uint32_t mx = 0;
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
        uint32_t r = rg * kRowsPerGroup + wave * kRowsPerWave + rt * 16 + lrow;
        r = min(r, p.R - 1u);                       // duplicate the last valid row
        const uint32_t t = r / p.g;
        const uint32_t hq = h * p.g + (r - t * p.g);
        const uint16_t *qrow = p.q + ((static_cast<uint64_t>(l) * p.Tq + t) * p.Hq + hq) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4_t w = *reinterpret_cast<const u32x4_t *>(qrow + ks * 32 + kgrp * 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mx = max(mx, max(w[i] & 0x7fffu, (w[i] >> 16) & 0x7fffu));
            }
            a[rt][ks] = __builtin_bit_cast(half8_t, w);
        }
    }
    return mx;
}

template <int D>
__global__ __launch_bounds__(kScoreThreads, 2) void score_kernel(ScoreParams p) {
    constexpr int KS = D / 32;                       // k-steps of 32
    constexpr int ROW_BYTES = D * 2;                 // one key of one head
    constexpr int CH = D / 8;                        // 16-byte chunks per key
    constexpr int TILE = kTileKeys * ROW_BYTES;      // 32 KiB (D = 256)
    constexpr int LOADS = TILE / 1024;               // wave-wide 1 KiB loads per tile
    constexpr int LOADS_PER_WAVE = LOADS / kScoreWaves;
    static_assert(LOADS % kScoreWaves == 0, "tile must split over the waves");

    __shared__ __attribute__((aligned(1024))) uint8_t tiles[2][TILE];

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
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63u;
    const uint32_t lrow = lane & 15u;   // row (A) / key (B) within a 16-tile
    const uint32_t kgrp = lane >> 4;    // which 8 of the 32 k-values

    // ---- K tiles: direct HBM -> LDS, swizzled chunk order
    const uint64_t key_stride = static_cast<uint64_t>(p.Hkv) * ROW_BYTES;
    // A full tile (64 keys inside the block) has no duplicated keys: the
    // source offset of load `inst` (key j = KPI*inst + lane/CH, chunk
    // (lane mod CH) ^ (j mod CH)) splits into a uniform part in SGPRs,
    // KPI*inst*key_stride, and a per-lane part XOR a per-load constant:
    //   lane_src ^ ((KPI*inst mod CH) * 16),
    //   lane_src = (lane/CH)*key_stride + ((lane mod CH) ^ (lane/CH))*16
    // (the XORed bits lie below ROW_BYTES, and key_stride is a multiple of
    // it), one VALU per load.  The last tile of a partial block takes the
    // general path, which clamps keys to the last valid one.
    constexpr uint32_t KPI = 1024u / ROW_BYTES;  // keys per wave-wide 1 KiB load
    const uint32_t lane_src = (lane / CH) * static_cast<uint32_t>(key_stride) +
                              (((lane % CH) ^ (lane / CH)) * 16u);
    // tile `it` = keys [64*(it&1), 64*(it&1) + 64) of block b_begin + it/2
    auto issue_tile = [&](uint32_t it, int buf) {
        const uint32_t b = b_begin + (it >> 1);
        const uint32_t k0 = (it & 1u) * kTileKeys;
        const uint8_t *base = p.k + ((static_cast<uint64_t>(l) * p.cap + b) * p.T) * key_stride +
                              static_cast<uint64_t>(h) * ROW_BYTES;
        const uint32_t nt = (b + 1 == p.B && p.last_T != 0) ? p.last_T : p.T;
        // the lane terms pass through an empty asm so the per-load offsets
        // are recomputed here (a VALU or a few per load) instead of being
        // kept live across the loop next to the 192 registers of query rows
        if (k0 + kTileKeys <= nt) {
            uint32_t ls = lane_src;
            asm volatile("" : "+v"(ls));
            const uint8_t *tbase = base + static_cast<uint64_t>(k0) * key_stride;
#pragma unroll
            for (int i = 0; i < LOADS_PER_WAVE; ++i) {
                const uint32_t inst = wave * LOADS_PER_WAVE + i;
                const uint32_t voff = ls ^ (((KPI * inst) & (CH - 1u)) * 16u);
                const uint8_t *src = tbase + static_cast<uint64_t>(KPI * inst) * key_stride + voff;
                __builtin_amdgcn_global_load_lds(
                    src, (lds_void_t *) (&tiles[buf][inst * 1024u]), 16, 0, kDmaNonTemporal);
            }
            return;
        }
        uint32_t ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int i = 0; i < LOADS_PER_WAVE; ++i) {
            const uint32_t inst = wave * LOADS_PER_WAVE + i;
            const uint32_t slot = inst * 64u + ln;              // 16-byte LDS slot
            const uint32_t j = slot / CH;                       // key within the tile
            const uint32_t c = (slot % CH) ^ (j % CH);          // global chunk held there
            const uint32_t jj = min(k0 + j, nt - 1u);           // duplicate the last key
            const uint8_t *src = base + jj * key_stride + c * 16u;
            __builtin_amdgcn_global_load_lds(
                src, (lds_void_t *) (&tiles[buf][inst * 1024u]), 16, 0, kDmaNonTemporal);
        }
    };

    issue_tile(0u, 0);

    // ---- query rows -> A fragments (resident for the whole workgroup).  The
    // raw bits are loaded first; bf16 rows are then converted to f16 in
    // place.  A bf16 value past f16's range (|q| >= 65536, bf16 exponent
    // >= 143) would turn infinite, so the wave's rows are converted times
    // 2^-qexp, which brings its largest |q| below 65536, and its maxima are
    // scaled back on the way out.  Both scalings are exact (qexp is 0 for
    // rows in range), so scores do not change.
    half8_t a[kRowTiles][KS];
    const uint32_t qmax = load_query_bits<D, KS>(p, a, l, h, rg, wave, lrow, kgrp);
    int qexp = 0;
    if (p.q_bf16 != 0) {
        const uint32_t e = static_cast<uint32_t>(wave_max(static_cast<float>(qmax))) >> 7;
        qexp = (e > 142u && e < 255u) ? static_cast<int>(e) - 142 : 0;
        const float qscale = __builtin_ldexpf(1.0f, -qexp);
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4_t w = __builtin_bit_cast(u32x4_t, a[rt][ks]);
                half8_t v;
#pragma unroll
                for (int i = 0; i < 4; ++i) {  // two bf16 per word, the low one first
                    v[2 * i] = bf16_to_half(w[i] << 16, qscale);
                    v[2 * i + 1] = bf16_to_half(w[i] & 0xffff0000u, qscale);
                }
                a[rt][ks] = v;
            }
        }
    }
    const float out_scale = __builtin_ldexpf(p.scale, qexp);

    // LDS byte address of B fragment (kt, ks) in buffer buf, i.e. of the
    // swizzled chunk (ks*4 + kgrp) ^ (key mod CH) of key kt*16 + lrow:
    //   (tiles + buf*TILE + kt*16*ROW_BYTES + lrow*ROW_BYTES + (kgrp ^ lrow)*16)
    //     ^ (ks*64 ^ ((kt*16) mod CH)*16)
    // -- everything at or above the row size is added, the swizzle bits
    // below it XORed in, so one VALU per read and one register per lane.
    const uint32_t lds0 = (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) uint8_t *)(&tiles[0][0]));
    const uint32_t lane_b = lrow * ROW_BYTES + ((kgrp ^ lrow) * 16u);

    float *out = p.partial +
                 ((static_cast<uint64_t>(rg * kScoreWaves + wave) * p.L + l) * p.Hkv + h) * p.B;
    const uint32_t n_tiles = 2u * (b_end - b_begin);
    float m = -FLT_MAX;
    for (uint32_t it = 0; it < n_tiles; ++it) {
        const int buf = static_cast<int>(it & 1u);
        // this thread's loads of tile it have landed; after the barrier every
        // thread's have, and every wave is done reading the other buffer
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (it + 1 < n_tiles) {
            issue_tile(it + 1, buf ^ 1);
        }
        // B fragments of the tile: f = kt * KS + ks covers keys kt*16 .. +16
        // and k-slice ks.  The reads are inline asm with explicit
        // lgkmcnt waits that carry the fragment register as an operand:
        // two reads stay in flight ahead of the six MFMAs that consume a
        // fragment, in three registers.  (Compiler-issued reads ended up
        // with a single register, each read waiting out the MFMAs before
        // it and its own latency after.)  Every read is waited for inside
        // the tile, before the next barrier.
        uint32_t tb = lds0 + static_cast<uint32_t>(buf) * TILE + lane_b;
        asm volatile("" : "+v"(tb));  // recompute the read addresses per tile
        auto read_b = [&](int f) {
            const uint32_t kt = static_cast<uint32_t>(f / KS);
            const uint32_t ks = static_cast<uint32_t>(f % KS);
            const uint32_t addr = (tb + kt * (16u * ROW_BYTES)) ^ (ks * 64u ^ ((kt * 16u) & (CH - 1u)) * 16u);
            half8_t r;
            asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
            return r;
        };
        constexpr int NF = (kTileKeys / 16) * KS;
        constexpr int PF = 2;  // reads in flight ahead of the consumed one
        half8_t bq[PF + 1];
#pragma unroll
        for (int f = 0; f < PF; ++f) {
            bq[f] = read_b(f);
        }
        float4_t acc[kRowTiles];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int ks = f % KS;
            half8_t &bf = bq[f % (PF + 1)];
            if (f + PF < NF) {
                bq[(f + PF) % (PF + 1)] = read_b(f + PF);
            }
            // LDS reads return in order: wait until only the newer ones
            // (at most PF) are outstanding
            const int newer = (NF - 1 - f) < PF ? (NF - 1 - f) : PF;
            if (newer == 2) {
                asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(bf) :: "memory");
            } else if (newer == 1) {
                asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(bf) :: "memory");
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bf) :: "memory");
            }
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    a[rt][ks], bf, ks == 0 ? float4_t{0.0f, 0.0f, 0.0f, 0.0f} : acc[rt], 0, 0, 0);
            }
            if (ks == KS - 1) {
#pragma unroll
                for (int rt = 0; rt < kRowTiles; ++rt) {
                    m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(acc[rt][0], acc[rt][1]),
                                                           __builtin_fmaxf(acc[rt][2], acc[rt][3])));
                }
            }
        }
        if (it & 1u) {  // both halves of the block are in m
            m = wave_max(m);
            if (lane == 0) {
                out[b_begin + (it >> 1)] = m * out_scale;
            }
            m = -FLT_MAX;
        }
    }
}

// The fold after the scorer, one launch:
//   layer_scores[l][b] = max_{slice, h} partial[slice][l][h][b]
//   scores[b]          = reduce over layers, in layer order, of layer_scores[l][b]
//                        (sum then / L for the mean, or max).
// A workgroup takes 16 blocks; 16 threads per block take the layers l,
// l + 16, ... and issue a layer's partial maxima as one batch of loads.
// After the barrier one thread per block reduces its layers in layer order,
// again loading 16 layers per batch.  The arithmetic is the plain loops'
// (a max chain in (slice, head) order, an ordered float sum), so batching
// changes no bit.
constexpr uint32_t kFoldBlocks = 16;
constexpr uint32_t kFoldLanes = 256 / kFoldBlocks;
constexpr uint32_t kFoldBatch = 16;

__global__ __launch_bounds__(256) void score_fold_kernel(const float *partial, uint32_t S,
                                                         uint32_t L, uint32_t Hkv, uint32_t B,
                                                         float *layer_scores, int mode,
                                                         float *scores) {
    const uint32_t bl = threadIdx.x % kFoldBlocks;
    const uint32_t lane = threadIdx.x / kFoldBlocks;
    const uint32_t b = blockIdx.x * kFoldBlocks + bl;
    const uint32_t per_layer = S * Hkv;
    if (b < B) {
        for (uint32_t l = lane; l < L; l += kFoldLanes) {
            float best = -FLT_MAX;
            for (uint32_t i0 = 0; i0 < per_layer; i0 += kFoldBatch) {
                float v[kFoldBatch];
#pragma unroll
                for (uint32_t j = 0; j < kFoldBatch; ++j) {
                    const uint32_t i = i0 + j;
                    v[j] = -FLT_MAX;
                    if (i < per_layer) {
                        const uint32_t sl = i / Hkv;
                        const uint32_t h = i - sl * Hkv;
                        v[j] = partial[((static_cast<uint64_t>(sl) * L + l) * Hkv + h) * B + b];
                    }
                }
#pragma unroll
                for (uint32_t j = 0; j < kFoldBatch; ++j) {
                    best = fmaxf(best, v[j]);
                }
            }
            layer_scores[static_cast<uint64_t>(l) * B + b] = best;
        }
    }
    __syncthreads();
    if (lane != 0 || b >= B) {
        return;
    }
    const bool max_mode = mode == KVMEM_LAYER_MAX;
    float acc = max_mode ? -FLT_MAX : 0.0f;
    for (uint32_t l0 = 0; l0 < L; l0 += kFoldBatch) {
        float v[kFoldBatch];
#pragma unroll
        for (uint32_t j = 0; j < kFoldBatch; ++j) {
            v[j] = l0 + j < L ? layer_scores[static_cast<uint64_t>(l0 + j) * B + b] : 0.0f;
        }
#pragma unroll
        for (uint32_t j = 0; j < kFoldBatch; ++j) {
            if (l0 + j < L) {
                acc = max_mode ? fmaxf(acc, v[j]) : acc + v[j];
            }
        }
    }
    if (mode == KVMEM_LAYER_MEAN && L > 0) {
        acc = acc / static_cast<float>(L);
    }
    scores[b] = acc;
}

size_t score_partial_bytes(uint32_t L, uint32_t Hkv, uint32_t B, uint32_t n_q_tokens, uint32_t g) {
    const size_t rows = static_cast<size_t>(n_q_tokens) * g;
    const size_t slices = (rows + kRowsPerGroup - 1) / kRowsPerGroup * kScoreWaves;
    return sizeof(float) * slices * L * Hkv * B;
}

bool load_score_kernels() {
    return load_kernel_object(&score_kernel<256>);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

namespace {

// Validates a scorer call and fills its launch shape (everything but the
// partial-maxima buffer).  Sets *empty when there is nothing to score.
int score_setup(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist, const kvmem_hip_score_args *args,
                ScoreParams &p, uint64_t &grid, bool *empty) {
    *empty = false;
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
        *empty = true;
        return KVMEM_HIP_OK;
    }
    p = ScoreParams{};
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
    // two workgroups per CU hold their LDS double buffers; eight per CU
    // over the launch keep every XCD busy to the end
    const uint32_t target = 2048;
    const uint32_t per_chunk_target = std::max<uint32_t>(1, target / std::max<uint32_t>(1, pairs * p.RG));
    p.n_chunks = std::min(B, per_chunk_target);
    p.blocks_per_chunk = (B + p.n_chunks - 1) / p.n_chunks;
    if (p.RG > 1) {
        // Several row slices read the same key tiles.  Their workgroups are
        // consecutive on one XCD, and short chunks keep them close enough
        // together for each tile to come from that XCD's L2.  At 16 x 8192
        // blocks with a 512-token query (8 slices), 16 blocks per chunk cut
        // HBM reads from 5.6 to 1.9 times the key bytes and the call by
        // 5.7 %.  Shorter chunks lose more in workgroup start-up (query
        // rows loaded and converted) than they gain.  4 slices do best with
        // 64 blocks, 2 with 32.
        const uint32_t most = p.RG >= 8 ? 16u : (p.RG >= 4 ? 64u : 32u);
        p.blocks_per_chunk = std::min(p.blocks_per_chunk, most);
    }
    p.n_chunks = (B + p.blocks_per_chunk - 1) / p.blocks_per_chunk;
    p.xcd_major = (pairs % 8u) == 0;
    grid = static_cast<uint64_t>(pairs) * p.RG * p.n_chunks;
    if (grid > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score: problem too large for one launch");
    }
    return KVMEM_HIP_OK;
}

// The scorer and the fold on the context stream: p.partial receives the
// per-slice maxima, `layers` the per-layer scores.  `timed` brackets the
// scorer with the profiling events of kPerfScore.
int score_launch(kvmem_hip_ctx *ctx, const kvmem_hip_score_args *args, const ScoreParams &p,
                 uint64_t grid, float *layers, bool timed) {
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "score kernel launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (timed) {
        (void) perf_attach(ctx, kPerfScore);  // the scorer's events ride on its launch
    }
    if (args->head_dim == 256) {
        ctx_launch(ctx, score_kernel<256>, dim3(static_cast<uint32_t>(grid)), dim3(kScoreThreads), 0, p);
    } else {
        ctx_launch(ctx, score_kernel<128>, dim3(static_cast<uint32_t>(grid)), dim3(kScoreThreads), 0, p);
    }
    const bool launched = hip_ok(ctx, hipGetLastError(), "score kernel launch");
    if (timed) {
        perf_detach(ctx, kPerfScore, launched);
    }
    if (!launched) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    // the fold is not bracketed: a timing event costs the stream a few
    // microseconds, as much as the fold itself
    score_fold_kernel<<<(p.B + kFoldBlocks - 1) / kFoldBlocks, 256, 0, ctx->stream>>>(
        p.partial, p.RG * kScoreWaves, p.L, p.Hkv, p.B, layers, args->layer_reduce, args->scores);
    if (!hip_ok(ctx, hipGetLastError(), "score fold launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    return KVMEM_HIP_OK;
}

// Scratch of kvmem_hip_score_noalloc, one copy per GPU for the life of the
// process: the per-slice maxima, then (when the caller passes no
// layer_scores) the per-layer scores.  The 256K workload (16 layers x 2048
// blocks, 4 KV heads, a 64-token query of 24 heads) needs 2 MiB + 128 KiB.
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Device address of `scratch` on each GPU, looked up once per device, and
// its owner: the context and stream of the last call, whose completion
// event tells when the array is free again.  A call from another context
// while that event is pending would race on the array and is refused
// instead (a context's own calls are ordered: set_stream waits for the old
// stream).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_addr[kMaxDevices] = {};
struct ScratchOwner {
    const kvmem_hip_ctx *ctx = nullptr;
    hipStream_t stream = nullptr;
};
ScratchOwner g_scratch_owner[kMaxDevices];

}  // namespace

namespace kvmem_hip {

bool score_scratch_setup(kvmem_hip_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) {
        fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "score scratch: device ordinal beyond 63");
        return false;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[ctx->device]) {
        // the caller made ctx->device current
        void *addr = nullptr;
        if (!hip_ok(ctx, hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "score scratch address")) {
            return false;
        }
        g_scratch_addr[ctx->device] = addr;
    }
    ctx->noalloc_scratch = g_scratch_addr[ctx->device];
    // the owner record's completion event (no timing: cheap to record)
    return hip_ok(ctx, hipEventCreateWithFlags(&ctx->noalloc_done, hipEventDisableTiming), "score scratch event");
}

void score_scratch_release(kvmem_hip_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) {
        return;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_owner[ctx->device].ctx == ctx) {
        g_scratch_owner[ctx->device] = ScratchOwner{};
    }
}

}  // namespace kvmem_hip

extern "C" int kvmem_hip_score(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                               const kvmem_hip_score_args *args) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    ScoreParams p;
    uint64_t grid = 0;
    bool empty = false;
    int st = score_setup(ctx, hist, args, p, grid, &empty);
    if (st != KVMEM_HIP_OK || empty) {
        return st;
    }
    (void) hipSetDevice(ctx->device);
    const size_t partial_bytes = score_partial_bytes(p.L, p.Hkv, p.B, p.Tq, p.g);
    if (!ensure_dev(ctx, ctx->score_partial, partial_bytes, "score partial")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    p.partial = static_cast<float *>(ctx->score_partial.ptr);
    float *layers = args->layer_scores;
    if (!layers) {
        if (!ensure_dev(ctx, ctx->score_layers, sizeof(float) * static_cast<size_t>(p.L) * p.B,
                        "score layer buffer")) {
            return KVMEM_HIP_ERR_NOMEM;
        }
        layers = static_cast<float *>(ctx->score_layers.ptr);
    }
    return score_launch(ctx, args, p, grid, layers, true);
}

extern "C" int kvmem_hip_score_noalloc(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                                       const kvmem_hip_score_args *args) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    ScoreParams p;
    uint64_t grid = 0;
    bool empty = false;
    int st = score_setup(ctx, hist, args, p, grid, &empty);
    if (st != KVMEM_HIP_OK || empty) {
        return st;
    }
    if (!ctx->noalloc_scratch) {
        return fail(ctx, KVMEM_HIP_ERR_RUNTIME, "score_noalloc: no scratch address for this device");
    }
    const size_t partial_bytes = score_partial_bytes(p.L, p.Hkv, p.B, p.Tq, p.g);
    const size_t layer_off = (partial_bytes + 255) / 256 * 256;
    const size_t need = args->layer_scores ? partial_bytes
                                           : layer_off + sizeof(float) * static_cast<size_t>(p.L) * p.B;
    if (need > kNoAllocScratchBytes) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID,
                    "score_noalloc: " + std::to_string(need) + " bytes of scratch needed, the maximum is " +
                        std::to_string(kNoAllocScratchBytes) + " (use kvmem_hip_score)");
    }
    (void) hipSetDevice(ctx->device);
    // Under graph capture the launches become graph nodes and the call's
    // completion cannot be tracked: its replays run when the caller launches
    // them.  An event recorded in a capture cannot be queried afterwards,
    // so none is recorded and the capturing context stays the owner.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (!hip_ok(ctx, hipStreamIsCapturing(ctx->stream, &capture), "score_noalloc capture status")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const bool capturing = capture != hipStreamCaptureStatusNone;
    // Take the device's array: free when no call is recorded, when the last
    // one came from this context on this stream (queued behind it), or when
    // the last call's completion event has fired.
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchOwner &own = g_scratch_owner[ctx->device];
    if (own.ctx && !(own.ctx == ctx && own.stream == ctx->stream)) {
        const hipError_t q = hipEventQuery(own.ctx->noalloc_done);
        if (q == hipErrorNotReady) {
            return fail(ctx, KVMEM_HIP_ERR_BUSY,
                        "score_noalloc: another context or stream is still using this GPU's scratch");
        }
        if (q != hipSuccess) {
            return fail(ctx, KVMEM_HIP_ERR_RUNTIME,
                        std::string("score_noalloc: owner event: ") + hipGetErrorString(q));
        }
    }
    uint8_t *base = static_cast<uint8_t *>(ctx->noalloc_scratch);
    p.partial = reinterpret_cast<float *>(base);
    float *layers = args->layer_scores ? args->layer_scores : reinterpret_cast<float *>(base + layer_off);
    st = score_launch(ctx, args, p, grid, layers, false);
    if (st != KVMEM_HIP_OK) {
        // a launch that failed after the scorer kernel was queued leaves that
        // kernel on the array with no owner record: let it drain first (a
        // capture holds nothing that runs)
        if (!capturing) {
            (void) hipStreamSynchronize(ctx->stream);
        }
        return st;
    }
    if (capturing) {
        own.ctx = ctx;
        own.stream = ctx->stream;
        return KVMEM_HIP_OK;
    }
    if (!hip_ok(ctx, hipEventRecord(ctx->noalloc_done, ctx->stream), "score_noalloc completion event")) {
        own = ScratchOwner{};  // nothing tells when the launched work ends: no owner to wait for
        (void) hipStreamSynchronize(ctx->stream);
        return KVMEM_HIP_ERR_RUNTIME;
    }
    own.ctx = ctx;
    own.stream = ctx->stream;
    return KVMEM_HIP_OK;
}
