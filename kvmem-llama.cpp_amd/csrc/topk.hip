// Top-k block selection in one workgroup.
//
// Keys are 64-bit: the high word is the score mapped to an unsigned order
// (negative floats bit-inverted, positive floats with the sign bit set,
// -0 folded to +0), the low word encodes the id so that equal scores rank
// by id (lower id first: ~id; higher id first: id).  Forced ids and padding
// get key 0, below every finite score.  A bitonic sort of the keys in LDS
// (descending) puts the `need` best candidates first; their ids plus the
// forced ids are then flagged and compacted in ascending id order with a
// workgroup prefix sum, which is the window order of
// KvMemStore::pick_topk_ungrouped (kvmem_store.cpp:618-622).
#include "kvmem_internal.hpp"

#include <algorithm>
#include <vector>

namespace kvmem_hip {

constexpr int kTopkThreads = 1024;
constexpr int kTopkMaxN = 16384;
constexpr int kTopkMaxPerThread = kTopkMaxN / kTopkThreads;  // 16

__device__ inline uint64_t rank_key(float s, uint32_t id, bool tie_lower) {
    if (s == 0.0f) {
        s = 0.0f;  // -0 == +0 as a score
    }
    const uint32_t u = __float_as_uint(s);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t lo = tie_lower ? (0xffffffffu - id) : id;
    return (static_cast<uint64_t>(ord) << 32) | lo;
}

__device__ inline uint32_t key_id(uint64_t key, bool tie_lower) {
    const uint32_t lo = static_cast<uint32_t>(key);
    return tie_lower ? (0xffffffffu - lo) : lo;
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float *scores, uint32_t n,
                                                            uint32_t npow2, const uint32_t *forced,
                                                            uint32_t n_forced, uint32_t need,
                                                            int tie_lower, uint32_t *sel,
                                                            uint32_t *n_sel) {
    __shared__ uint64_t keys[kTopkMaxN];
    __shared__ uint32_t scan[kTopkThreads];
    const uint32_t tid = threadIdx.x;
    const bool tl = tie_lower != 0;

    for (uint32_t i = tid; i < npow2; i += kTopkThreads) {
        keys[i] = i < n ? rank_key(scores[i], i, tl) : 0ull;
    }
    __syncthreads();
    for (uint32_t f = tid; f < n_forced; f += kTopkThreads) {
        keys[forced[f]] = 0ull;  // position == id before the sort
    }
    __syncthreads();

    // bitonic sort, descending
    for (uint32_t k = 2; k <= npow2; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < npow2; i += kTopkThreads) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = keys[i];
                    const uint64_t b = keys[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) {
                        keys[i] = b;
                        keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }

    // the winners' ids leave LDS before it is reused for flags
    uint32_t mine[kTopkMaxPerThread];
    uint32_t n_mine = 0;
    for (uint32_t i = tid; i < need; i += kTopkThreads) {
        const uint64_t key = keys[i];
        if (key != 0ull) {
            mine[n_mine++] = key_id(key, tl);
        }
    }
    __syncthreads();
    uint8_t *flags = reinterpret_cast<uint8_t *>(keys);
    for (uint32_t i = tid; i < n; i += kTopkThreads) {
        flags[i] = 0;
    }
    __syncthreads();
    for (uint32_t j = 0; j < n_mine; ++j) {
        flags[mine[j]] = 1;
    }
    for (uint32_t f = tid; f < n_forced; f += kTopkThreads) {
        flags[forced[f]] = 1;
    }
    __syncthreads();

    // ordered compaction: thread t owns ids [t*seg, (t+1)*seg)
    const uint32_t seg = (n + kTopkThreads - 1) / kTopkThreads;
    const uint32_t lo = min(n, tid * seg);
    const uint32_t hi = min(n, lo + seg);
    uint32_t cnt = 0;
    for (uint32_t i = lo; i < hi; ++i) {
        cnt += flags[i];
    }
    scan[tid] = cnt;
    __syncthreads();
    for (uint32_t off = 1; off < kTopkThreads; off <<= 1) {
        const uint32_t v = tid >= off ? scan[tid - off] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t pos = scan[tid] - cnt;  // exclusive prefix
    for (uint32_t i = lo; i < hi; ++i) {
        if (flags[i]) {
            sel[pos++] = i;
        }
    }
    if (tid == kTopkThreads - 1) {
        *n_sel = scan[tid];
    }
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" int kvmem_hip_topk(kvmem_hip_ctx *ctx, const float *scores, uint32_t n,
                              const uint32_t *forced, uint32_t n_forced, uint32_t need,
                              int tie_lower_index, uint32_t *sel_out, uint32_t *n_sel) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!sel_out || !n_sel || (n > 0 && !scores) || (n_forced > 0 && !forced)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "topk: null argument");
    }
    *n_sel = 0;
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (n > static_cast<uint32_t>(kTopkMaxN)) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "topk: more than 16384 blocks");
    }
    std::vector<uint8_t> seen(n, 0);
    std::vector<uint32_t> uniq;
    uniq.reserve(n_forced);
    for (uint32_t i = 0; i < n_forced; ++i) {
        if (forced[i] >= n) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "topk: forced id out of range");
        }
        if (!seen[forced[i]]) {
            seen[forced[i]] = 1;
            uniq.push_back(forced[i]);
        }
    }
    const uint32_t candidates = n - static_cast<uint32_t>(uniq.size());
    need = std::min(need, candidates);
    uint32_t npow2 = 1;
    while (npow2 < n) {
        npow2 <<= 1;
    }
    (void) hipSetDevice(ctx->device);
    const size_t out_cap = static_cast<size_t>(n) + 1;
    if (!ensure_dev(ctx, ctx->topk_sel, out_cap * sizeof(uint32_t), "topk output") ||
        !ensure_pin(ctx, ctx->topk_sel_host, out_cap * sizeof(uint32_t), "topk pinned output")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    const uint32_t *forced_dev = nullptr;
    if (!uniq.empty()) {
        forced_dev = static_cast<const uint32_t *>(
            upload(ctx, uniq.data(), uniq.size() * sizeof(uint32_t), "topk forced ids"));
        if (!forced_dev) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
    }
    uint32_t *sel_dev = static_cast<uint32_t *>(ctx->topk_sel.ptr);
    perf_begin(ctx, kPerfTopk);
    topk_kernel<<<1, kTopkThreads, 0, ctx->stream>>>(scores, n, npow2, forced_dev,
                                                     static_cast<uint32_t>(uniq.size()), need,
                                                     tie_lower_index, sel_dev, sel_dev + n);
    perf_end(ctx, kPerfTopk);
    if (!hip_ok(ctx, hipGetLastError(), "topk launch") ||
        !hip_ok(ctx, hipMemcpyAsync(ctx->topk_sel_host.ptr, sel_dev, out_cap * sizeof(uint32_t),
                                    hipMemcpyDeviceToHost, ctx->stream), "topk D2H") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "topk sync")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const uint32_t *h = static_cast<const uint32_t *>(ctx->topk_sel_host.ptr);
    const uint32_t cnt = h[n];
    if (cnt > static_cast<uint32_t>(uniq.size()) + need) {
        return fail(ctx, KVMEM_HIP_ERR_RUNTIME, "topk: selection larger than requested");
    }
    std::copy(h, h + cnt, sel_out);
    *n_sel = cnt;
    return KVMEM_HIP_OK;
}
