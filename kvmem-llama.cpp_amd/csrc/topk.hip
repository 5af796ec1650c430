// Top-k block selection in one workgroup.  Up to 16384 blocks the keys sit
// in LDS (topk_kernel); beyond, up to 2^20, they are recomputed from the
// scores in every pass (topk_stream_kernel).
//
// Keys are 64-bit: the high word is the score mapped to an unsigned order
// (negative floats bit-inverted, positive floats with the sign bit set,
// -0 folded to +0), the low word encodes the id so that equal scores rank
// by id (lower id first: ~id; higher id first: id).  Every candidate key is
// therefore distinct, and the selection is "the `need` largest keys".
// Forced ids get key 0, below every finite score, and a bit in a mask.
//
// The need-th largest key is found by radix select, eight passes of 8 bits
// from the top: each pass histograms the digit of the keys that match the
// digits fixed so far, and one wave picks the digit where the running count
// from the top reaches the remaining rank.  Winners are the keys at or above
// that threshold; they and the forced ids are compacted in ascending id
// order with a workgroup prefix sum, which is the window order of
// KvMemStore::pick_topk_ungrouped (kvmem_store.cpp:618-622).
//
// The selection goes straight to coherent pinned host memory: the ids are
// compacted in LDS, one wave writes them out with coalesced stores, and a
// completion word is set after its system-scope fence.  The host spins on that word
// instead of sleeping in a stream synchronize: the wait spans the scorer
// (milliseconds), long enough for a blocking wait to fall back to an
// interrupt, whose wake-up cost tens of microseconds per step.  A few forced
// ids (the sink) travel in the kernel arguments, so no upload precedes the
// launch.
#include "kvmem_internal.hpp"
#include "device_reselect.h"

#include <algorithm>
#include <chrono>
#include <vector>

namespace kvmem_hip {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkMaxN = 16384;
constexpr int kTopkForcedInline = 64;  // forced ids passed by value

struct TopkForced {
    uint32_t id[kTopkForcedInline];
};

__device__ inline uint64_t rank_key(float s, uint32_t id, bool tie_lower) {
    if (s == 0.0f) {
        s = 0.0f;  // -0 == +0 as a score
    }
    const uint32_t u = __float_as_uint(s);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t lo = tie_lower ? (0xffffffffu - id) : id;
    return (static_cast<uint64_t>(ord) << 32) | lo;
}

// Inclusive prefix sum over the workgroup (every thread passes one value).
__device__ inline uint32_t block_inclusive_scan(uint32_t v, uint32_t *wave_tot) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(v, off, 64);
        if (lane >= static_cast<uint32_t>(off)) {
            v += t;
        }
    }
    if (lane == 63u) {
        wave_tot[wave] = v;
    }
    __syncthreads();
    if (wave == 0) {
        uint32_t w = lane < static_cast<uint32_t>(kTopkWaves) ? wave_tot[lane] : 0u;
#pragma unroll
        for (int off = 1; off < kTopkWaves; off <<= 1) {
            const uint32_t t = __shfl_up(w, off, 64);
            if (lane >= static_cast<uint32_t>(off)) {
                w += t;
            }
        }
        if (lane < static_cast<uint32_t>(kTopkWaves)) {
            wave_tot[lane] = w;  // inclusive totals of waves 0..lane
        }
    }
    __syncthreads();
    return v + (wave > 0 ? wave_tot[wave - 1] : 0u);
}

// `forced` is a device list, or null with the ids in `forced_inline`.
// `out` (host-mapped) receives the ids at [0, count) and the count at [n];
// `done` is set to `epoch` once both are visible to the host.  `dev_out`,
// when set, receives the count at [0] and the ids at [1, 1 + count) in
// device memory, for kernels that follow on the stream.
__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const float *scores, uint32_t n,
                                                            const uint32_t *forced,
                                                            TopkForced forced_inline,
                                                            uint32_t n_forced, uint32_t need,
                                                            int tie_lower, uint32_t *out,
                                                            uint32_t *done, uint32_t epoch,
                                                            uint32_t *dev_out) {
    __shared__ uint64_t keys[kTopkMaxN];
    __shared__ uint32_t forced_bits[kTopkMaxN / 32];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wave_tot[kTopkWaves];
    __shared__ uint64_t s_prefix;
    __shared__ uint32_t s_rank;
    __shared__ uint32_t s_alone;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const bool tl = tie_lower != 0;

    for (uint32_t i = tid; i < n; i += kTopkThreads) {
        keys[i] = rank_key(scores[i], i, tl);
    }
    for (uint32_t w = tid; w < (n + 31u) / 32u; w += kTopkThreads) {
        forced_bits[w] = 0u;
    }
    __syncthreads();
    for (uint32_t f = tid; f < n_forced; f += kTopkThreads) {
        const uint32_t id = forced ? forced[f] : forced_inline.id[f];
        keys[id] = 0ull;  // out of the race
        atomicOr(&forced_bits[id >> 5], 1u << (id & 31u));
    }
    __syncthreads();

    // ---- radix select: threshold = the need-th largest candidate key.
    // Keys are unique, so once the digit holding that rank has a single key
    // it is the threshold, and the digits decided so far (`mask`) order
    // every other key against it: the later passes are skipped.
    uint64_t prefix = 0ull;
    uint64_t mask = 0ull;
    uint32_t rank = need;  // rank still to find among keys matching `prefix`
    if (need > 0u) {
        for (int shift = 56; shift >= 0; shift -= 8) {
            if (tid < 256u) {
                hist[tid] = 0u;
            }
            if (tid == 0u) {
                s_alone = 0u;
            }
            __syncthreads();
            for (uint32_t i = tid; i < n; i += kTopkThreads) {
                const uint64_t k = keys[i];
                if (k != 0ull && (k & mask) == prefix) {
                    atomicAdd(&hist[static_cast<uint32_t>(k >> shift) & 255u], 1u);
                }
            }
            __syncthreads();
            if (tid < 64u) {
                // lane owns digits 4*lane .. 4*lane+3; above(d) = count of
                // matching keys whose digit exceeds d
                uint32_t c[4];
                uint32_t own = 0u;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    c[j] = hist[4u * lane + j];
                    own += c[j];
                }
                uint32_t suffix = own;  // sum over lanes >= this one
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t t = __shfl_down(suffix, off, 64);
                    if (lane + off < 64u) {
                        suffix += t;
                    }
                }
                uint32_t above = suffix - own;  // digits of higher lanes
#pragma unroll
                for (int j = 3; j >= 0; --j) {
                    if (above < rank && rank <= above + c[j]) {
                        s_prefix = prefix | (static_cast<uint64_t>(4u * lane + j) << shift);
                        s_rank = rank - above;
                        s_alone = c[j] == 1u ? 1u : 0u;
                    }
                    above += c[j];
                }
            }
            __syncthreads();
            prefix = s_prefix;
            rank = s_rank;
            mask |= 0xffull << shift;
            const bool alone = s_alone != 0u;
            __syncthreads();  // s_prefix / s_alone / hist are rewritten by the next pass
            if (alone) {
                break;
            }
        }
    }
    // the key of rank `need`, on the bits decided (all 64 unless it stood
    // alone earlier): a candidate wins when its key on those bits is >= it
    const uint64_t threshold = prefix;

    // ---- ordered compaction: thread t owns ids [t*seg, (t+1)*seg)
    const uint32_t seg = (n + kTopkThreads - 1) / kTopkThreads;
    const uint32_t lo = min(n, tid * seg);
    const uint32_t hi = min(n, lo + seg);
    auto chosen = [&](uint32_t i) -> bool {
        const uint64_t k = keys[i];
        if (k == 0ull) {
            return (forced_bits[i >> 5] >> (i & 31u)) & 1u;
        }
        return need > 0u && (k & mask) >= threshold;
    };
    uint32_t cnt = 0;
    uint32_t picked = 0;  // bit j: id lo + j chosen (seg <= 16)
    for (uint32_t i = lo; i < hi; ++i) {
        if (chosen(i)) {
            picked |= 1u << (i - lo);
            ++cnt;
        }
    }
    const uint32_t incl = block_inclusive_scan(cnt, wave_tot);
    const uint32_t total = wave_tot[kTopkWaves - 1];
    // the keys are no longer read: their LDS holds the compacted ids
    uint32_t *ids = reinterpret_cast<uint32_t *>(keys);
    uint32_t pos = incl - cnt;
    for (uint32_t i = lo; i < hi; ++i) {
        if ((picked >> (i - lo)) & 1u) {
            ids[pos++] = i;
        }
    }
    __syncthreads();
    // one wave writes the host copy, so one fence covers it
    if (tid >= 64u) {
        return;
    }
    for (uint32_t i = tid; i < total; i += 64u) {
        out[i] = ids[i];
        if (dev_out) {
            dev_out[1u + i] = ids[i];
        }
    }
    if (tid == 0) {
        out[n] = total;
        if (dev_out) {
            dev_out[0] = total;
        }
    }
    __threadfence_system();
    if (tid == 0) {
        __hip_atomic_store(done, epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// More blocks than the keys LDS holds (n > kTopkMaxN, up to kTopkStreamMaxN):
// the same radix select and ordered compaction, but no key is kept -- each
// pass recomputes the keys it needs from the scores (L2-resident: 4 bytes a
// block) and only the forced-id bitmask lives in LDS.  The ids go straight
// from each thread's segment to the host buffer.
constexpr uint32_t kTopkStreamMaxN = 1u << 20;

__global__ __launch_bounds__(kTopkThreads) void topk_stream_kernel(
    const float *scores, uint32_t n, const uint32_t *forced, TopkForced forced_inline,
    uint32_t n_forced, uint32_t need, int tie_lower, uint32_t *out, uint32_t *done, uint32_t epoch,
    uint32_t *dev_out) {
    __shared__ uint32_t forced_bits[kTopkStreamMaxN / 32];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t wave_tot[kTopkWaves];
    __shared__ uint64_t s_prefix;
    __shared__ uint32_t s_rank;
    __shared__ uint32_t s_alone;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const bool tl = tie_lower != 0;
    for (uint32_t w = tid; w < (n + 31u) / 32u; w += kTopkThreads) {
        forced_bits[w] = 0u;
    }
    __syncthreads();
    for (uint32_t f = tid; f < n_forced; f += kTopkThreads) {
        const uint32_t id = forced ? forced[f] : forced_inline.id[f];
        atomicOr(&forced_bits[id >> 5], 1u << (id & 31u));
    }
    __syncthreads();
    auto is_forced = [&](uint32_t i) -> bool { return (forced_bits[i >> 5] >> (i & 31u)) & 1u; };
    auto key_of = [&](uint32_t i) -> uint64_t { return is_forced(i) ? 0ull : rank_key(scores[i], i, tl); };

    // the same radix select as topk_kernel's, its passes skipped once the
    // threshold key stands alone in its digit
    uint64_t prefix = 0ull;
    uint64_t mask = 0ull;
    uint32_t rank = need;
    if (need > 0u) {
        for (int shift = 56; shift >= 0; shift -= 8) {
            if (tid < 256u) {
                hist[tid] = 0u;
            }
            if (tid == 0u) {
                s_alone = 0u;
            }
            __syncthreads();
            for (uint32_t i = tid; i < n; i += kTopkThreads) {
                const uint64_t k = key_of(i);
                if (k != 0ull && (k & mask) == prefix) {
                    atomicAdd(&hist[static_cast<uint32_t>(k >> shift) & 255u], 1u);
                }
            }
            __syncthreads();
            if (tid < 64u) {
                uint32_t c[4];
                uint32_t own = 0u;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    c[j] = hist[4u * lane + j];
                    own += c[j];
                }
                uint32_t suffix = own;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t t = __shfl_down(suffix, off, 64);
                    if (lane + off < 64u) {
                        suffix += t;
                    }
                }
                uint32_t above = suffix - own;
#pragma unroll
                for (int j = 3; j >= 0; --j) {
                    if (above < rank && rank <= above + c[j]) {
                        s_prefix = prefix | (static_cast<uint64_t>(4u * lane + j) << shift);
                        s_rank = rank - above;
                        s_alone = c[j] == 1u ? 1u : 0u;
                    }
                    above += c[j];
                }
            }
            __syncthreads();
            prefix = s_prefix;
            rank = s_rank;
            mask |= 0xffull << shift;
            const bool alone = s_alone != 0u;
            __syncthreads();
            if (alone) {
                break;
            }
        }
    }
    const uint64_t threshold = prefix;  // on the bits in `mask`
    auto chosen = [&](uint32_t i) -> bool {
        if (is_forced(i)) {
            return true;
        }
        return need > 0u && (rank_key(scores[i], i, tl) & mask) >= threshold;
    };
    const uint32_t seg = (n + kTopkThreads - 1) / kTopkThreads;
    const uint32_t lo = min(n, tid * seg);
    const uint32_t hi = min(n, lo + seg);
    uint32_t cnt = 0;
    for (uint32_t i = lo; i < hi; ++i) {
        cnt += chosen(i) ? 1u : 0u;
    }
    const uint32_t incl = block_inclusive_scan(cnt, wave_tot);
    const uint32_t total = wave_tot[kTopkWaves - 1];
    uint32_t pos = incl - cnt;
    for (uint32_t i = lo; i < hi; ++i) {
        if (chosen(i)) {
            if (dev_out) {
                dev_out[1u + pos] = i;
            }
            out[pos++] = i;
        }
    }
    if (tid == 0) {
        out[n] = total;
        if (dev_out) {
            dev_out[0] = total;
        }
    }
    __threadfence_system();  // every thread's ids are visible to the host ...
    __syncthreads();
    if (tid == 0) {          // ... before the completion word
        __hip_atomic_store(done, epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

bool load_topk_kernels() {
    return load_kernel_object(&topk_kernel) && load_kernel_object(&topk_stream_kernel);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

namespace {

inline void cpu_relax() {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
}

}  // namespace

namespace kvmem_hip {

// Launch half of kvmem_hip_topk: validates, uploads nothing but an overlong
// forced list, and enqueues the kernel.  With `to_device` the selection is
// also written to ctx->topk_dev ([0] = count, then the ids) for kernels
// that follow on the stream.  topk_wait() collects the selection.
int topk_launch(kvmem_hip_ctx *ctx, const float *scores, uint32_t n, const uint32_t *forced,
                uint32_t n_forced, uint32_t need, int tie_lower_index, bool to_device) {
    ctx->topk_pending = false;
    if (!scores || (n_forced > 0 && !forced)) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "topk: null argument");
    }
    if (n > kTopkStreamMaxN) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "topk: more than 1048576 blocks");
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
    (void) hipSetDevice(ctx->device);
    if (!ensure_pin(ctx, ctx->topk_sel_host, topk_out_bytes(n), "topk host output",
                    hipHostMallocCoherent | hipHostMallocMapped)) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    if (to_device && !ensure_dev(ctx, ctx->topk_dev, sizeof(uint32_t) * (static_cast<size_t>(n) + 1),
                                 "topk device output")) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    uint32_t *h = static_cast<uint32_t *>(ctx->topk_sel_host.ptr);
    void *out_dev = nullptr;
    if (!hip_ok(ctx, hipHostGetDevicePointer(&out_dev, h, 0), "topk host output mapping")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    const size_t flag = topk_flag_index(n);
    TopkForced inl{};
    const uint32_t *forced_dev = nullptr;
    if (uniq.size() > static_cast<size_t>(kTopkForcedInline)) {
        forced_dev = static_cast<const uint32_t *>(
            upload(ctx, uniq.data(), uniq.size() * sizeof(uint32_t), "topk forced ids"));
        if (!forced_dev) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
    } else {
        std::copy(uniq.begin(), uniq.end(), inl.id);
    }
    ctx->topk_epoch = ctx->topk_epoch + 1 == 0 ? 1 : ctx->topk_epoch + 1;
    const uint32_t epoch = ctx->topk_epoch;
    uint32_t *out = static_cast<uint32_t *>(out_dev);
    uint32_t *dev_out = to_device ? static_cast<uint32_t *>(ctx->topk_dev.ptr) : nullptr;
    // pinned memory comes uninitialised: clear the word before the kernel
    // can set it (the previous call's write has landed; it was waited for)
    __atomic_store_n(h + flag, 0u, __ATOMIC_RELEASE);
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, "topk launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    perf_begin(ctx, kPerfTopk);
    if (n <= static_cast<uint32_t>(kTopkMaxN)) {
        topk_kernel<<<1, kTopkThreads, 0, ctx->stream>>>(scores, n, forced_dev, inl,
                                                         static_cast<uint32_t>(uniq.size()), need,
                                                         tie_lower_index, out, out + flag, epoch, dev_out);
    } else {
        topk_stream_kernel<<<1, kTopkThreads, 0, ctx->stream>>>(
            scores, n, forced_dev, inl, static_cast<uint32_t>(uniq.size()), need, tie_lower_index, out,
            out + flag, epoch, dev_out);
    }
    perf_end(ctx, kPerfTopk);
    if (!hip_ok(ctx, hipGetLastError(), "topk launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    ctx->topk_pending = true;
    ctx->topk_n = n;
    ctx->topk_limit = static_cast<uint32_t>(uniq.size()) + need;
    return KVMEM_HIP_OK;
}

// Wait half: spin on the completion word of the last topk_launch.  Once the
// wait has lasted hold_off_us, every few thousand rounds ask the stream
// whether it has drained (then the word must be set) or failed.  A caller
// with work queued behind the top-k holds the query back: the runtime
// answers it by attaching a completion signal, with a system-scope cache
// release, to the last command queued -- in a device-planned apply the
// chain walk, whose release would then stall the stage-in queued behind it
// by several microseconds.  There a failed stream is seen after
// kTopkQueryAfterUs; kvmem_hip_topk, with nothing behind the top-k, asks
// from the first round.
constexpr int64_t kTopkQueryAfterUs = 20000;

int topk_wait(kvmem_hip_ctx *ctx, uint32_t *sel_out, uint32_t *n_sel, int64_t hold_off_us) {
    if (!ctx->topk_pending) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "topk: no launch to wait for");
    }
    ctx->topk_pending = false;
    const uint32_t n = ctx->topk_n;
    const uint32_t epoch = ctx->topk_epoch;
    const uint32_t *h = static_cast<const uint32_t *>(ctx->topk_sel_host.ptr);
    const uint32_t *done = h + topk_flag_index(n);
    const auto t0 = std::chrono::steady_clock::now();
    bool query = hold_off_us <= 0;
    for (uint32_t spin = 1; __atomic_load_n(done, __ATOMIC_ACQUIRE) != epoch; ++spin) {
        cpu_relax();
        if ((spin & 4095u) == 0 && !query) {
            query = std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(hold_off_us);
        }
        if (query && (spin & 4095u) == 0) {
            const hipError_t q = hipStreamQuery(ctx->stream);
            if (q == hipErrorNotReady) {
                continue;
            }
            if (!hip_ok(ctx, q, "topk wait")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
            if (__atomic_load_n(done, __ATOMIC_ACQUIRE) != epoch) {
                return fail(ctx, KVMEM_HIP_ERR_RUNTIME, "topk: kernel ended without its completion word");
            }
        }
    }
    const uint32_t cnt = h[n];
    if (cnt > ctx->topk_limit) {
        return fail(ctx, KVMEM_HIP_ERR_RUNTIME, "topk: selection larger than requested");
    }
    std::copy(h, h + cnt, sel_out);
    *n_sel = cnt;
    return KVMEM_HIP_OK;
}

}  // namespace kvmem_hip

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
    const int rc = topk_launch(ctx, scores, n, forced, n_forced, need, tie_lower_index, false);
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    return topk_wait(ctx, sel_out, n_sel, 0);
}

extern "C" int kvmem_hip_topk_launch_dev(kvmem_hip_ctx *ctx, const float *scores, uint32_t n,
                                         const uint32_t *forced, uint32_t n_forced, uint32_t need,
                                         int tie_lower_index) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "topk: no blocks");
    }
    return topk_launch(ctx, scores, n, forced, n_forced, need, tie_lower_index, true);
}

extern "C" int kvmem_hip_topk_wait(kvmem_hip_ctx *ctx, uint32_t *sel_out, uint32_t *n_sel) {
    if (!ctx || !sel_out || !n_sel) {
        return KVMEM_HIP_ERR_INVALID;
    }
    *n_sel = 0;
    return topk_wait(ctx, sel_out, n_sel, kTopkQueryAfterUs);
}
