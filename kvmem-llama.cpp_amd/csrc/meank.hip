// Mean-K cosine block scorer (the reference's retrieval scorer) and its
// producers: per-block key sums from the F16 history, the decode-time
// running key sum, and the per-layer query sums.
//
// Producer: k_sum[l][b][e] = fp32 sum of the block's F16 keys in token
// order, mean_tokens[l][b] = tokens summed (RawKvStore::capture_mean_f16,
// kvmem/src/host/raw_kv_store.cpp:184-202).  A thread owns 8 consecutive
// channels and adds token after token, so every channel's sum is the same
// sequence of IEEE additions as the reference's: bit-identical.
//
// Scorer (llama_memory_kvmem::score_retrieval, src/adapter/
// llama-memory-kvmem.cpp:2869-2916):
//   qv[l][h]   = (sum_{gi<g} q_sum[l][h*g+gi]) * (1 / (q_count[l]*g))
//   mk         = k_sum[l][b] * (1 / mean_tokens[l][b])
//   cos[l][b][h] = (qv . mk_h) / (sqrt(|qv|^2) * sqrt(|mk_h|^2) + 1e-6)
//   score[b]   = mean over layers with q_count > 0 of (sum_h cos) / Hkv,
// layer and block sums in double as the reference; blocks with no keys in
// any layer score 0.  Sixteen lanes per (block, layer) compute each head's
// dot products with a lane-then-tree reduction (the reference sums in
// channel order: results agree to ~1e-7 of the norms).  HBM-bound: the
// 16 x 2048-block scorer reads 128 MiB of fp32 sums.
#include "kvmem_internal.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

namespace kvmem_hip {

// grid: (items * L) workgroups of E/8 threads; item i = block_ids[i].  The
// keys of (block b, layer l) are T rows of E halves at k + b*block_stride +
// l*layer_stride: a device history [L][cap][T][E] or the K rows of a
// block-major pinned host history.
__global__ __launch_bounds__(256) void meank_sum_kernel(const uint8_t *k, uint64_t block_stride,
                                                        uint64_t layer_stride, const uint32_t *items,
                                                        uint32_t L, uint32_t cap, uint32_t T,
                                                        uint32_t E, uint32_t last_block,
                                                        uint32_t last_tokens, float *k_sum,
                                                        uint32_t *mean_tokens) {
    const uint32_t job = blockIdx.x;
    const uint32_t item = job / L;
    const uint32_t l = job - item * L;
    const uint32_t b = items[item];
    const uint32_t e0 = threadIdx.x * 8u;
    if (e0 >= E) {
        return;
    }
    const uint32_t nt = (b == last_block && last_tokens != 0) ? last_tokens : T;
    const uint8_t *base = k + b * block_stride + l * layer_stride + e0 * 2u;
    float s[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t t = 0; t < nt; ++t) {
        const uint4 raw = *reinterpret_cast<const uint4 *>(base + static_cast<uint64_t>(t) * E * 2u);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s[2 * i] += static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] & 0xffffu)));
            s[2 * i + 1] += static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] >> 16)));
        }
    }
    float *out = k_sum + (static_cast<uint64_t>(l) * cap + b) * E + e0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        out[i] = s[i];
    }
    if (threadIdx.x == 0) {
        mean_tokens[static_cast<uint64_t>(l) * cap + b] = nt;
    }
}

// Query-sum producer: one thread per (layer, channel) adds the listed
// tokens' values in list order onto (or from zero into) q_sum, as the
// reference's harvest loop does per layer (llama-memory-kvmem.cpp:2164-2172).
template <typename QT>
__global__ __launch_bounds__(256) void q_accumulate_kernel(const QT *q, const uint8_t *tok_dev,
                                                           ArgTables tok_args, int listed,
                                                           uint32_t n_list, uint32_t n_tokens,
                                                           uint32_t E, uint32_t L, int reset,
                                                           float *q_sum) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t l = blockIdx.y;
    if (e >= E || l >= L) {
        return;
    }
    float *dst = q_sum + static_cast<uint64_t>(l) * E + e;
    float acc = reset ? 0.0f : *dst;
    const QT *src = q + static_cast<uint64_t>(l) * n_tokens * E + e;
    // the rows of a batch are loaded before any is added (one memory latency
    // per batch); they are added in list order as the sequential loop does
    constexpr uint32_t kBatch = 16;
    uint32_t i = 0;
    for (; i + kBatch <= n_list; i += kBatch) {
        float v[kBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t t = listed ? tab_read<uint32_t>(tok_dev, tok_args, 4u * (i + j)) : i + j;
            v[j] = static_cast<float>(src[static_cast<uint64_t>(t) * E]);
        }
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            acc += v[j];
        }
    }
    for (; i < n_list; ++i) {
        const uint32_t t = listed ? tab_read<uint32_t>(tok_dev, tok_args, 4u * i) : i;
        acc += static_cast<float>(src[static_cast<uint64_t>(t) * E]);
    }
    *dst = acc;
}

// Decode running sum: one thread per channel adds the kept tokens' values
// in token order (strided K view of type KT).
template <typename KT>
__global__ __launch_bounds__(256) void meank_add_kernel(const uint8_t *k, uint32_t n_embd,
                                                        uint32_t head_dim, uint64_t nb0, uint64_t nb1,
                                                        uint64_t nb2, uint32_t tok0, uint32_t n_keep,
                                                        int reset, float *acc, uint32_t *count) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e == 0 && count) {
        *count = (reset ? 0u : *count) + n_keep;
    }
    if (e >= n_embd) {
        return;
    }
    const uint32_t head = e / head_dim;
    const uint32_t dim = e - head * head_dim;
    const uint8_t *base = k + static_cast<uint64_t>(head) * nb1 + static_cast<uint64_t>(dim) * nb0;
    float s = reset ? 0.0f : acc[e];
    for (uint32_t t = 0; t < n_keep; ++t) {
        s += static_cast<float>(*reinterpret_cast<const KT *>(base + static_cast<uint64_t>(tok0 + t) * nb2));
    }
    acc[e] = s;
}

// Per-layer 1 / (query rows x group size), 0 for a layer without query
// rows, carried in the query kernel's arguments (no upload before it).
constexpr uint32_t kMeankMaxL = 256;
struct LayerScales {
    float v[kMeankMaxL];
};

// One workgroup per (layer, KV head), one thread per channel: the group's
// query sum (heads added in group order) scaled by invq, and its squared
// norm reduced over the channels.  The (layer, 0) workgroups also copy the
// layer's scale to invq_out in device memory for the kernels after it.
__global__ __launch_bounds__(256) void meank_query_kernel(const float *q_sum, LayerScales invq,
                                                          float *invq_out, uint32_t L, uint32_t Hq,
                                                          uint32_t Hkv, uint32_t D, float *qv, float *nq) {
    __shared__ float part[4];
    const uint32_t i = blockIdx.x;  // l * Hkv + h
    const uint32_t d = threadIdx.x;
    const uint32_t l = i / Hkv;
    const uint32_t h = i - l * Hkv;
    const uint32_t g = Hq / Hkv;
    const float scale = invq.v[l];  // uniform index: read from the argument bytes
    if (h == 0 && d == 0) {
        invq_out[l] = scale;
    }
    float v = 0.0f;
    if (d < D) {
        float acc = 0.0f;
        for (uint32_t gi = 0; gi < g; ++gi) {
            acc += q_sum[(static_cast<uint64_t>(l) * Hq + h * g + gi) * D + d];
        }
        v = acc * scale;
        qv[static_cast<uint64_t>(i) * D + d] = v;
    }
    float n = v * v;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        n += __shfl_xor(n, off, 64);
    }
    if ((threadIdx.x & 63u) == 0u) {
        part[threadIdx.x >> 6] = n;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (uint32_t w = 0; w < (blockDim.x + 63u) / 64u; ++w) {
            t += part[w];
        }
        nq[i] = t;
    }
}

// Sum of v over the 16 lanes of a DPP row (quad permutes, bank-masked row
// shifts for distance 4, row rotation by 8); every lane must be active.
__device__ inline float row16_sum(float v) {
    int x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));  // ^1
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));  // ^2
    x = __float_as_int(v);
    const int t = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0x5, false);        // +4 (banks 0, 2)
    v += __int_as_float(__builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false));  // -4 (banks 1, 3)
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));  // ^8
    return v;
}

// 16 lanes per (layer, block) item, 16 items per 256-thread workgroup.  A
// lane holds D/16 channels of each head as float4s.  The key sums of every
// head (up to kMaxHeads) are loaded before the first head is reduced, so an
// item waits for memory once; the query vectors (shared by the layer's
// blocks, cache hits) are loaded per head.
template <int D>
__global__ __launch_bounds__(256) void meank_cos_kernel(const float *k_sum, const uint32_t *mean_tokens,
                                                        const float *qv, const float *nq,
                                                        const float *invq, uint32_t L, uint32_t B,
                                                        uint32_t cap, uint32_t Hkv, double *layer_cos) {
    constexpr int P4 = D / 64;  // float4s per lane per head
    constexpr int kMaxHeads = 4;  // heads whose key sums are in flight together
    const uint32_t item = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const uint32_t sub = threadIdx.x & 15u;
    const bool live = item < L * B;
    const uint32_t l = live ? item / B : 0u;
    const uint32_t b = live ? item - l * B : 0u;
    const float iq = invq[l];
    const uint32_t mt_raw = mean_tokens[static_cast<uint64_t>(l) * cap + b];
    const bool scored = live && iq != 0.0f;  // layers without query rows are skipped
    const uint32_t mt = scored ? mt_raw : 0u;
    const float inv = mt ? 1.0f / static_cast<float>(mt) : 0.0f;
    const float4 *ks = reinterpret_cast<const float4 *>(k_sum + (static_cast<uint64_t>(l) * cap + b) * Hkv * D);
    const float4 *qs = reinterpret_cast<const float4 *>(qv + static_cast<uint64_t>(l) * Hkv * D);
    const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    double layer = 0.0;
    for (uint32_t h0 = 0; h0 < Hkv; h0 += kMaxHeads) {
        const uint32_t nh = min(Hkv - h0, static_cast<uint32_t>(kMaxHeads));
        float4 kc[kMaxHeads][P4];
#pragma unroll
        for (int hh = 0; hh < kMaxHeads; ++hh) {
#pragma unroll
            for (int j = 0; j < P4; ++j) {
                // loaded whatever mt is (every row up to capacity is in bounds),
                // chosen after: the load need not wait for mean_tokens
                const float4 kv = static_cast<uint32_t>(hh) < nh ? ks[(h0 + hh) * (D / 4) + j * 16 + sub] : zero;
                kc[hh][j] = mt ? kv : zero;
            }
        }
#pragma unroll
        for (int hh = 0; hh < kMaxHeads; ++hh) {
            if (static_cast<uint32_t>(hh) >= nh) {
                break;
            }
            const uint32_t h = h0 + hh;
            float dot = 0.0f, nk = 0.0f;
#pragma unroll
            for (int j = 0; j < P4; ++j) {
                const float4 qv4 = qs[h * (D / 4) + j * 16 + sub];
                const float4 qc = scored ? qv4 : zero;
                const float m[4] = {kc[hh][j].x * inv, kc[hh][j].y * inv, kc[hh][j].z * inv, kc[hh][j].w * inv};
                const float q[4] = {qc.x, qc.y, qc.z, qc.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dot += q[e] * m[e];
                    nk += m[e] * m[e];
                }
            }
            dot = row16_sum(dot);
            nk = row16_sum(nk);
            const float nqh = nq[l * Hkv + h];
            const float c = dot / (sqrtf(scored ? nqh : 0.0f) * sqrtf(nk) + 1e-6f);
            layer += static_cast<double>(c);
        }
    }
    if (scored && sub == 0u) {
        layer_cos[static_cast<uint64_t>(l) * B + b] = layer;
    }
}

// A block's score: the mean over scored layers of its layer cosine sum / Hkv
// (in double, in layer order); 0 when no layer holds keys of the block.
// Threads take (layer slice, block) pairs so every load is issued at once:
// the workgroup covers 256 / kCombineLayers blocks, each thread its block's
// layers l = slice, slice + kCombineLayers, ..., and one thread per block
// adds the terms from LDS in layer order.
constexpr uint32_t kCombineLayers = 16;
constexpr uint32_t kCombineMaxL = 256;  // layers held in LDS per block

__global__ __launch_bounds__(256) void meank_combine_kernel(const double *layer_cos,
                                                            const uint32_t *mean_tokens,
                                                            const float *invq, uint32_t L, uint32_t B,
                                                            uint32_t cap, uint32_t Hkv, float *scores) {
    constexpr uint32_t kBlocks = 256 / kCombineLayers;
    __shared__ double term[kBlocks][kCombineMaxL];
    __shared__ uint32_t any_keys[kBlocks];
    const uint32_t lb = threadIdx.x / kCombineLayers;  // block within the workgroup
    const uint32_t slice = threadIdx.x - lb * kCombineLayers;
    const uint32_t b = blockIdx.x * kBlocks + lb;
    if (slice == 0) {
        any_keys[lb] = 0u;
    }
    __syncthreads();
    if (b < B) {
        uint32_t has = 0;
        for (uint32_t l = slice; l < L; l += kCombineLayers) {
            has |= mean_tokens[static_cast<uint64_t>(l) * cap + b] != 0 ? 1u : 0u;
            term[lb][l] = invq[l] != 0.0f ? layer_cos[static_cast<uint64_t>(l) * B + b] : 0.0;
        }
        if (has) {
            atomicOr(&any_keys[lb], 1u);
        }
    }
    __syncthreads();
    if (b >= B || slice != 0) {
        return;
    }
    double acc = 0.0;
    uint32_t nlay = 0;
    for (uint32_t l = 0; l < L; ++l) {
        if (invq[l] != 0.0f) {
            acc += term[lb][l] / static_cast<double>(Hkv ? Hkv : 1);
            ++nlay;
        }
    }
    scores[b] = static_cast<float>((any_keys[lb] && nlay) ? acc / nlay : 0.0);
}

// Per-(layer, block) cosine sums in double, rounded up to 256 bytes so the
// query vectors after them start aligned.
static size_t meank_cos_bytes(uint32_t L, uint32_t B) {
    return (sizeof(double) * static_cast<size_t>(L) * B + 255) & ~static_cast<size_t>(255);
}

size_t meank_scratch_bytes(uint32_t L, uint32_t Hkv, uint32_t B, uint32_t D) {
    const size_t qv_bytes = sizeof(float) * static_cast<size_t>(L) * Hkv * (D + 1);
    return meank_cos_bytes(L, B) + qv_bytes + sizeof(float) * static_cast<size_t>(L) + 256;
}

bool load_meank_kernels() {
    return load_kernel_object(&meank_cos_kernel<256>);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" {

int kvmem_hip_meank_sums(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                         const uint32_t *block_ids, uint32_t n, float *k_sum,
                         uint32_t *mean_tokens) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!hist || !hist->k || !block_ids || !k_sum || !mean_tokens) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums: null argument");
    }
    const uint32_t E = hist->n_embd_k;
    const uint32_t cap = hist->capacity_blocks ? hist->capacity_blocks : hist->n_blocks;
    if (E == 0 || E % 8 != 0 || E / 8 > 256 || hist->block_tokens == 0 || cap < hist->n_blocks ||
        (reinterpret_cast<uintptr_t>(hist->k) & 15u) || (reinterpret_cast<uintptr_t>(k_sum) & 15u)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID,
                    "meank_sums: n_embd_k must be a multiple of 8 and at most 2048, 16-byte aligned");
    }
    if (hist->last_block_tokens > hist->block_tokens) {
        // the kernel sums the last block's rows up to this count
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums: last_block_tokens above block_tokens");
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (block_ids[i] >= hist->n_blocks) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums: block id out of range");
        }
    }
    const uint64_t jobs = static_cast<uint64_t>(n) * hist->n_layers;
    if (jobs > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums: too many blocks in one call");
    }
    (void) hipSetDevice(ctx->device);
    const void *items = upload(ctx, block_ids, sizeof(uint32_t) * n, "meank_sums ids");
    if (!items) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "meank_sums launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const uint64_t block_stride = static_cast<uint64_t>(hist->block_tokens) * E * 2u;
    meank_sum_kernel<<<static_cast<uint32_t>(jobs), E / 8, 0, ctx->stream>>>(
        static_cast<const uint8_t *>(hist->k), block_stride, block_stride * cap,
        static_cast<const uint32_t *>(items), hist->n_layers, cap, hist->block_tokens, E,
        hist->n_blocks - 1, hist->last_block_tokens, k_sum, mean_tokens);
    return hip_ok(ctx, hipGetLastError(), "meank_sums launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

int kvmem_hip_meank_sums_host(kvmem_hip_ctx *ctx, const kvmem_hip_host_history *hist,
                              const uint32_t *block_ids, uint32_t n, uint32_t capacity_blocks,
                              float *k_sum, uint32_t *mean_tokens) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!hist || !hist->base || !block_ids || !k_sum || !mean_tokens) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums_host: null argument");
    }
    const uint32_t E = hist->n_embd_k;
    const uint32_t T = hist->block_tokens;
    const uint32_t cap = capacity_blocks ? capacity_blocks : hist->n_blocks;
    if (E == 0 || E % 8 != 0 || E / 8 > 256 || T == 0 || cap < hist->n_blocks ||
        hist->last_block_tokens > T || (reinterpret_cast<uintptr_t>(hist->base) & 15u) ||
        (reinterpret_cast<uintptr_t>(k_sum) & 15u) || (hist->n_embd_v % 8 != 0)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID,
                    "meank_sums_host: n_embd_k must be a multiple of 8 and at most 2048, 16-byte aligned");
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (block_ids[i] >= hist->n_blocks) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums_host: block id out of range");
        }
    }
    const uint64_t jobs = static_cast<uint64_t>(n) * hist->n_layers;
    if (jobs > 0x7fffffffu) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_sums_host: too many blocks in one call");
    }
    const uint64_t layer_bytes = static_cast<uint64_t>(T) * (hist->n_embd_k + hist->n_embd_v) * 2u;
    const uint64_t span = layer_bytes * hist->n_layers;
    (void) hipSetDevice(ctx->device);
    // the kernel reads the pinned rows over the link itself
    const uint8_t *view = host_device_view(hist->base, span * hist->n_blocks);
    if (!view) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED,
                    "meank_sums_host: the history must lie inside one pinned host allocation");
    }
    const void *items = upload(ctx, block_ids, sizeof(uint32_t) * n, "meank_sums_host ids");
    if (!items) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "meank_sums_host launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    meank_sum_kernel<<<static_cast<uint32_t>(jobs), E / 8, 0, ctx->stream>>>(
        view, span, layer_bytes, static_cast<const uint32_t *>(items), hist->n_layers, cap, T, E,
        hist->n_blocks - 1, hist->last_block_tokens, k_sum, mean_tokens);
    if (!hip_ok(ctx, hipGetLastError(), "meank_sums_host launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    // the kernel reads the listed blocks' K rows over the link
    uint64_t rows = 0;
    for (uint32_t i = 0; i < n; ++i) {
        rows += (block_ids[i] + 1 == hist->n_blocks && hist->last_block_tokens) ? hist->last_block_tokens : T;
    }
    note_xfer(ctx, kXferH2D, rows * hist->n_layers * E * 2u);
    return KVMEM_HIP_OK;
}

int kvmem_hip_meank_add(kvmem_hip_ctx *ctx, const void *k, int32_t k_type, uint32_t n_embd,
                        uint32_t head_dim, size_t nb0, size_t nb1, size_t nb2, uint32_t tok0,
                        uint32_t n_keep, int reset, float *acc, uint32_t *count) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!k || !acc || n_embd == 0 || head_dim == 0 || n_embd % head_dim != 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_add: null pointer or bad geometry");
    }
    const size_t esz = k_type == KVMEM_TYPE_F32 ? 4 : 2;
    if (k_type != KVMEM_TYPE_F32 && k_type != KVMEM_TYPE_F16 && k_type != KVMEM_TYPE_BF16) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "meank_add: k_type must be F32, F16 or BF16");
    }
    if (nb0 % esz || nb1 % esz || nb2 % esz || (reinterpret_cast<uintptr_t>(k) % esz)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "meank_add: strides must be multiples of the element size");
    }
    if (n_keep == 0 && !reset) {
        return KVMEM_HIP_OK;
    }
    (void) hipSetDevice(ctx->device);
    const uint32_t grid = (n_embd + 255) / 256;
    const uint8_t *kb = static_cast<const uint8_t *>(k);
    if (k_type == KVMEM_TYPE_F32) {
        meank_add_kernel<float><<<grid, 256, 0, ctx->stream>>>(kb, n_embd, head_dim, nb0, nb1, nb2, tok0,
                                                              n_keep, reset, acc, count);
    } else if (k_type == KVMEM_TYPE_F16) {
        meank_add_kernel<_Float16><<<grid, 256, 0, ctx->stream>>>(kb, n_embd, head_dim, nb0, nb1, nb2, tok0,
                                                                 n_keep, reset, acc, count);
    } else {
        meank_add_kernel<__bf16><<<grid, 256, 0, ctx->stream>>>(kb, n_embd, head_dim, nb0, nb1, nb2, tok0,
                                                               n_keep, reset, acc, count);
    }
    return hip_ok(ctx, hipGetLastError(), "meank_add launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

int kvmem_hip_q_accumulate(kvmem_hip_ctx *ctx, const void *q, int32_t q_type, uint32_t n_layers,
                           uint32_t n_tokens, uint32_t n_embd_q, const uint32_t *tokens,
                           uint32_t n_list, int reset, float *q_sum) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!q || !q_sum) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_accumulate: null argument");
    }
    if (q_type != KVMEM_TYPE_F32 && q_type != KVMEM_TYPE_F16 && q_type != KVMEM_TYPE_BF16) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "q_accumulate: q_type must be F32, F16 or BF16");
    }
    if (!tokens) {
        n_list = n_tokens;
    }
    for (uint32_t i = 0; tokens && i < n_list; ++i) {
        if (tokens[i] >= n_tokens) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_accumulate: token index out of range");
        }
    }
    if (n_layers == 0 || n_embd_q == 0 || (n_list == 0 && !reset)) {
        return KVMEM_HIP_OK;
    }
    if (n_layers > 65535) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "q_accumulate: too many layers");
    }
    (void) hipSetDevice(ctx->device);
    // the token list travels in the kernel arguments when it fits (768
    // rows), else it is uploaded
    LaunchTables lt;
    const int listed = tokens && n_list ? 1 : 0;
    if (listed && !stage_tables(ctx, tokens, sizeof(uint32_t) * n_list, lt, "q_accumulate tokens")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const dim3 grid((n_embd_q + 255) / 256, n_layers);
    if (q_type == KVMEM_TYPE_F32) {
        q_accumulate_kernel<float><<<grid, 256, 0, ctx->stream>>>(
            static_cast<const float *>(q), lt.dev, lt.args, listed, n_list, n_tokens, n_embd_q, n_layers, reset,
            q_sum);
    } else if (q_type == KVMEM_TYPE_F16) {
        q_accumulate_kernel<_Float16><<<grid, 256, 0, ctx->stream>>>(
            static_cast<const _Float16 *>(q), lt.dev, lt.args, listed, n_list, n_tokens, n_embd_q, n_layers,
            reset, q_sum);
    } else {
        q_accumulate_kernel<__bf16><<<grid, 256, 0, ctx->stream>>>(
            static_cast<const __bf16 *>(q), lt.dev, lt.args, listed, n_list, n_tokens, n_embd_q, n_layers,
            reset, q_sum);
    }
    return hip_ok(ctx, hipGetLastError(), "q_accumulate launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

int kvmem_hip_score_meank(kvmem_hip_ctx *ctx, const kvmem_hip_meank_args *a) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!a || !a->q_sum || !a->q_count || !a->k_sum || !a->mean_tokens || !a->scores) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score_meank: null argument");
    }
    const uint32_t L = a->n_layers, B = a->n_blocks, D = a->head_dim;
    const uint32_t cap = a->capacity_blocks ? a->capacity_blocks : B;
    if (a->n_head_kv == 0 || a->n_head % a->n_head_kv != 0 || (D != 128 && D != 256) || cap < B) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score_meank: bad head geometry");
    }
    if (reinterpret_cast<uintptr_t>(a->k_sum) & 15u) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "score_meank: k_sum must be 16-byte aligned");
    }
    static_assert(kMeankMaxL == kCombineMaxL, "layer bound");
    if (L > kMeankMaxL) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "score_meank: more than 256 layers");
    }
    if (L == 0 || B == 0) {
        return KVMEM_HIP_OK;
    }
    const uint32_t g = a->n_head / a->n_head_kv;
    // per-layer 1 / (q_count * g) as the reference computes it in fp32; 0
    // marks a layer without query rows
    LayerScales invq{};
    for (uint32_t l = 0; l < L; ++l) {
        invq.v[l] = a->q_count[l] ? 1.0f / static_cast<float>(a->q_count[l] * g) : 0.0f;
    }
    (void) hipSetDevice(ctx->device);
    // the fp32 query vectors start 256-byte aligned (read as float4)
    const size_t cos_bytes = meank_cos_bytes(L, B);
    if (!ensure_dev(ctx, ctx->meank_scratch, meank_scratch_bytes(L, a->n_head_kv, B, D),
                    "score_meank scratch")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    uint8_t *scratch = static_cast<uint8_t *>(ctx->meank_scratch.ptr);
    double *layer_cos = reinterpret_cast<double *>(scratch);
    float *qv = reinterpret_cast<float *>(scratch + cos_bytes);
    float *nq = qv + static_cast<size_t>(L) * a->n_head_kv * D;
    float *invq_dev = nq + static_cast<size_t>(L) * a->n_head_kv;
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "score_meank launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    perf_begin(ctx, kPerfScore);
    const uint32_t lh = L * a->n_head_kv;
    meank_query_kernel<<<lh, D, 0, ctx->stream>>>(a->q_sum, invq, invq_dev, L, a->n_head, a->n_head_kv, D,
                                                  qv, nq);
    const uint64_t items = static_cast<uint64_t>(L) * B;  // 16 lanes each
    const uint32_t grid = static_cast<uint32_t>((items * 16 + 255) / 256);
    {
        // the cosine kernel, which streams the key sums, also timed alone
        PerfLaunchScope timed(ctx, kPerfMeankCos);
        ctx_launch(ctx, D == 256 ? meank_cos_kernel<256> : meank_cos_kernel<128>, dim3(grid), dim3(256), 0,
                   a->k_sum, a->mean_tokens, qv, nq, invq_dev, L, B, cap, a->n_head_kv, layer_cos);
        if (hip_ok(ctx, hipGetLastError(), "score_meank launch")) {
            timed.ok();
        } else {
            perf_drop(ctx, kPerfScore);
            return KVMEM_HIP_ERR_RUNTIME;
        }
    }
    constexpr uint32_t kCombineBlocks = 256 / kCombineLayers;
    meank_combine_kernel<<<(B + kCombineBlocks - 1) / kCombineBlocks, 256, 0, ctx->stream>>>(layer_cos, a->mean_tokens, invq_dev,
                                                                   L, B, cap, a->n_head_kv, a->scores);
    perf_end(ctx, kPerfScore);
    return hip_ok(ctx, hipGetLastError(), "score_meank launch") ? KVMEM_HIP_OK : KVMEM_HIP_ERR_RUNTIME;
}

}  // extern "C"
