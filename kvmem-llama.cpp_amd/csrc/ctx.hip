// Context lifetime, error reporting, streams, upload ring, profiling and the
// batched device copy of libkvmem_hip.so.
#include "kvmem_internal.hpp"
#include "device_reselect.h"

#include <algorithm>

#include <cstring>
#include <new>
#include <vector>

namespace kvmem_hip {

int fail(kvmem_hip_ctx *ctx, int code, const std::string &msg) {
    if (ctx) {
        ctx->last_error = msg;
    }
    return code;
}

bool hip_ok(kvmem_hip_ctx *ctx, hipError_t e, const char *what) {
    if (e == hipSuccess) {
        return true;
    }
    if (ctx) {
        ctx->last_error = std::string(what) + ": " + hipGetErrorString(e);
    }
    return false;
}

bool injected_fail(kvmem_hip_ctx *ctx, uint32_t kind, const char *what) {
    if (!ctx || !(ctx->fail_kinds & kind)) {
        return false;
    }
    if (ctx->fail_countdown > 1) {
        --ctx->fail_countdown;
        return false;
    }
    ctx->fail_kinds = 0;
    ctx->fail_countdown = 0;
    ctx->last_error = std::string(what) + ": injected failure";
    return true;
}

bool ensure_dev(kvmem_hip_ctx *ctx, DevBuf &b, size_t bytes, const char *what) {
    if (b.ptr && b.bytes >= bytes) {
        return true;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_ALLOC, what)) {
        return false;
    }
    if (b.ptr) {
        // the old buffer may still be read by enqueued work
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), what)) {
            return false;
        }
        (void) hipFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (!hip_ok(ctx, hipMalloc(&b.ptr, want), what)) {
        b.ptr = nullptr;
        return false;
    }
    b.bytes = want;
    ctx->n_allocs += 1;
    return true;
}

bool ensure_pin(kvmem_hip_ctx *ctx, PinBuf &b, size_t bytes, const char *what, unsigned flags) {
    if (b.ptr && b.bytes >= bytes) {
        return true;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_ALLOC, what)) {
        return false;
    }
    if (b.ptr) {
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), what)) {
            return false;
        }
        (void) hipHostFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (!hip_ok(ctx, hipHostMalloc(&b.ptr, want, flags), what)) {
        b.ptr = nullptr;
        return false;
    }
    b.bytes = want;
    ctx->n_allocs += 1;
    return true;
}

void *upload(kvmem_hip_ctx *ctx, const void *src, size_t bytes, const char *what) {
    UploadSlot &s = ctx->upload[ctx->upload_next];
    ctx->upload_next = (ctx->upload_next + 1) % kUploadRing;
    if (s.pending) {
        // the pinned staging area is still the source of an enqueued copy
        if (!hip_ok(ctx, hipEventSynchronize(s.done), what)) {
            return nullptr;
        }
        s.pending = false;
    }
    if (!ensure_pin(ctx, s.host, bytes, what) || !ensure_dev(ctx, s.dev, bytes, what)) {
        return nullptr;
    }
    if (!s.done && !hip_ok(ctx, hipEventCreateWithFlags(&s.done, hipEventDisableTiming), what)) {
        return nullptr;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_COPY, what)) {
        return nullptr;
    }
    std::memcpy(s.host.ptr, src, bytes);
    if (!hip_ok(ctx, hipMemcpyAsync(s.dev.ptr, s.host.ptr, bytes, hipMemcpyHostToDevice,
                                    ctx->stream), what) ||
        !hip_ok(ctx, hipEventRecord(s.done, ctx->stream), what)) {
        return nullptr;
    }
    s.pending = true;
    return s.dev.ptr;
}

static hipEvent_t perf_event(kvmem_hip_ctx *ctx) {
    if (!ctx->perf_free.empty()) {
        hipEvent_t e = ctx->perf_free.back();
        ctx->perf_free.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        return nullptr;
    }
    return e;
}

void perf_begin(kvmem_hip_ctx *ctx, PerfStage s) {
    if (!ctx->perf_on || !(ctx->perf_mask & (1u << s)) || ctx->perf_open[s]) {
        return;  // off, not timed, or already inside this stage
    }
    hipEvent_t e = perf_event(ctx);
    if (e && hipEventRecord(e, ctx->stream) == hipSuccess) {
        ctx->perf_open[s] = e;
    } else if (e) {
        ctx->perf_free.push_back(e);
    }
}

void perf_drop(kvmem_hip_ctx *ctx, PerfStage s) {
    if (ctx->perf_open[s]) {
        ctx->perf_free.push_back(ctx->perf_open[s]);
        ctx->perf_open[s] = nullptr;
    }
}

void note_xfer(kvmem_hip_ctx *ctx, XferKind k, uint64_t bytes, uint64_t calls) {
    ctx->xfer_bytes[k] += bytes;
    ctx->xfer_calls[k] += calls;
}

// The open scorer-to-stage-in span, if it reached a stage-in, joins the
// done list; either way a new one may start.
static void span_close(kvmem_hip_ctx *ctx) {
    if (ctx->span_score_end && ctx->span_set_end) {
        ctx->span_done.emplace_back(ctx->span_score_end, ctx->span_set_end);
    }
    ctx->span_score_end = nullptr;
    ctx->span_set_end = nullptr;
}

// A stage's timed pair, its end also closing or extending the open
// scorer-to-stage-in span.
static void perf_file(kvmem_hip_ctx *ctx, PerfStage s, hipEvent_t start, hipEvent_t end) {
    ctx->perf_done[s].emplace_back(start, end);
    if (s == kPerfScore) {
        span_close(ctx);
        ctx->span_score_end = end;
    } else if (s == kPerfSet && ctx->span_score_end) {
        ctx->span_set_end = end;
    }
}

void perf_end(kvmem_hip_ctx *ctx, PerfStage s) {
    hipEvent_t start = ctx->perf_open[s];
    if (!start) {
        return;
    }
    ctx->perf_open[s] = nullptr;
    hipEvent_t end = perf_event(ctx);
    if (end && hipEventRecord(end, ctx->stream) == hipSuccess) {
        perf_file(ctx, s, start, end);
        return;
    }
    ctx->perf_free.push_back(start);
    if (end) {
        ctx->perf_free.push_back(end);
    }
}

bool perf_attach(kvmem_hip_ctx *ctx, PerfStage s) {
    if (!ctx->perf_on || !(ctx->perf_mask & (1u << s)) || ctx->perf_open[s] || ctx->attach_start) {
        return false;  // off, not timed, inside this stage, or a pair already waits
    }
    hipEvent_t start = perf_event(ctx);
    hipEvent_t end = start ? perf_event(ctx) : nullptr;
    if (!end) {
        if (start) {
            ctx->perf_free.push_back(start);
        }
        return false;
    }
    ctx->attach_start = start;
    ctx->attach_stop = end;
    ctx->attach_armed = true;
    return true;
}

void perf_detach(kvmem_hip_ctx *ctx, PerfStage s, bool ok) {
    hipEvent_t start = ctx->attach_start;
    hipEvent_t end = ctx->attach_stop;
    const bool launched = !ctx->attach_armed;
    ctx->attach_start = nullptr;
    ctx->attach_stop = nullptr;
    ctx->attach_armed = false;
    if (!start) {
        return;
    }
    if (ok && launched) {
        perf_file(ctx, s, start, end);
        return;
    }
    ctx->perf_free.push_back(start);
    ctx->perf_free.push_back(end);
}

void perf_collect(kvmem_hip_ctx *ctx) {
    // the spans first: their events belong to the stage pairs freed below
    span_close(ctx);
    for (auto &pr : ctx->span_done) {
        float ms = 0.0f;
        if (hipEventSynchronize(pr.second) == hipSuccess &&
            hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
            ctx->after_score_ms += ms;
            ctx->n_after_score += 1;
        }
    }
    ctx->span_done.clear();
    for (int s = 0; s < kPerfStages; ++s) {
        for (auto &pr : ctx->perf_done[s]) {
            float ms = 0.0f;
            if (hipEventSynchronize(pr.second) == hipSuccess &&
                hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
                ctx->perf_ms[s] += ms;
                ctx->perf_n[s] += 1;
            }
            ctx->perf_free.push_back(pr.first);
            ctx->perf_free.push_back(pr.second);
        }
        ctx->perf_done[s].clear();
    }
}

// ------------------------------------------------------------------------
// Batched byte copies: `pieces` workgroups per op, each a contiguous share
// of it, 16-byte vectors when both addresses and the size are 16-byte
// aligned.  A launch with few ops splits them so the chip fills.
// ------------------------------------------------------------------------
// Piece `piece` of `pieces` of one copy op, by the calling workgroup.
__device__ inline void copy_piece(const CopyOpDev &op, int piece, int pieces) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(op.src) | reinterpret_cast<uintptr_t>(op.dst);
    if ((a & 15u) == 0 && (op.nbytes & 15u) == 0) {
        // four 16-byte loads in flight per thread, nontemporal both ways (a
        // copy streams at ~6.0 TB/s so, against ~4.5-5.4 with one load)
        const u32x4_t *s = reinterpret_cast<const u32x4_t *>(op.src);
        u32x4_t *d = reinterpret_cast<u32x4_t *>(op.dst);
        const uint64_t n16 = op.nbytes >> 4;
        const uint64_t j1 = n16 * (piece + 1) / pieces;
        uint64_t j = n16 * piece / pieces + threadIdx.x;
        for (; j + 3u * blockDim.x < j1; j += 4u * blockDim.x) {
            u32x4_t v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v[u] = __builtin_nontemporal_load(s + j + u * blockDim.x);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                __builtin_nontemporal_store(v[u], d + j + u * blockDim.x);
            }
        }
        for (; j < j1; j += blockDim.x) {
            __builtin_nontemporal_store(__builtin_nontemporal_load(s + j), d + j);
        }
        return;
    }
    const uint64_t b1 = op.nbytes * (piece + 1) / pieces;
    for (uint64_t j = op.nbytes * piece / pieces + threadIdx.x; j < b1; j += blockDim.x) {
        op.dst[j] = op.src[j];
    }
}

__global__ __launch_bounds__(256) void batched_copy_kernel(const CopyOpDev *ops_dev, ArgTables t, int n,
                                                           int pieces) {
    const int i = blockIdx.x / pieces;
    const int piece = blockIdx.x - i * pieces;
    if (i >= n) {
        return;
    }
    const CopyOpDev op = reinterpret_cast<const CopyOpDev *>(
        table_base(reinterpret_cast<const uint8_t *>(ops_dev), t))[i];
    copy_piece(op, piece, pieces);
}

// The same copies with their count in device memory (written by an earlier
// kernel on the stream): min(*count, max_ops) ops of a device table, the
// grid's workgroups taking (op, piece) pairs in turn.
__global__ __launch_bounds__(256) void batched_copy_dev_kernel(const CopyOpDev *ops, const uint32_t *count,
                                                               uint32_t max_ops, uint32_t pieces) {
    const uint32_t n = min(*count, max_ops) * pieces;
    for (uint32_t v = blockIdx.x; v < n; v += gridDim.x) {
        const uint32_t i = v / pieces;
        copy_piece(ops[i], static_cast<int>(v - i * pieces), static_cast<int>(pieces));
    }
}

bool launch_dev_copies(kvmem_hip_ctx *ctx, const CopyOpDev *ops, const uint32_t *count, uint32_t max_ops,
                       const char *what) {
    if (max_ops == 0) {
        return true;
    }
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, what)) {
        return false;
    }
    constexpr uint32_t kPieces = 8;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>(1024, uint64_t{max_ops} * kPieces));
    batched_copy_dev_kernel<<<grid, 256, 0, ctx->stream>>>(ops, count, max_ops, kPieces);
    return hip_ok(ctx, hipGetLastError(), what);
}

bool stage_tables(kvmem_hip_ctx *ctx, const void *src, size_t bytes, LaunchTables &out, const char *what) {
    if (bytes <= kArgTableBytes) {
        out.dev = nullptr;
        std::memcpy(out.args.bytes, src, bytes);
        return true;
    }
    out.dev = static_cast<const uint8_t *>(upload(ctx, src, bytes, what));
    return out.dev != nullptr;
}

bool stage_copy_ops(kvmem_hip_ctx *ctx, const std::vector<CopyOpDev> &ops, LaunchTables &out, const char *what) {
    if (ops.size() > 0x7fffffffu / 8u) {
        fail(ctx, KVMEM_HIP_ERR_INVALID, std::string(what) + ": too many copies");
        return false;
    }
    return stage_tables(ctx, ops.data(), ops.size() * sizeof(CopyOpDev), out, what);
}

uint64_t max_op_bytes(const std::vector<CopyOpDev> &ops) {
    uint64_t m = 0;
    for (const CopyOpDev &op : ops) {
        m = std::max<uint64_t>(m, op.nbytes);
    }
    return m;
}

bool launch_staged_copies(kvmem_hip_ctx *ctx, const LaunchTables &tables, size_t n, uint64_t max_bytes,
                          const char *what) {
    if (n == 0) {
        return true;
    }
    // Pieces of about 16 KiB, one pass of a workgroup's four loads per
    // thread: a copy streams at ~6.3 TB/s so, against ~5.5 with one
    // workgroup looping over each 256 KiB op (the addresses in flight then
    // spread over every op).  Few small ops are still split so that ~2048
    // workgroups fill the chip; at most 64 pieces per op.
    constexpr uint64_t kPieceBytes = 16384;
    const uint64_t by_size = (max_bytes + kPieceBytes - 1) / kPieceBytes;
    const uint64_t to_fill = std::min<uint64_t>(8, std::max<uint64_t>(1, 2048 / n));
    const uint64_t cap = std::max<uint64_t>(1, 0x7fffffffu / n);  // grid below 2^31
    const int pieces = static_cast<int>(std::min<uint64_t>({64, cap, std::max(by_size, to_fill)}));
    if (injected_fail(ctx, KVMEM_HIP_FAIL_LAUNCH, what)) {
        return false;
    }
    ctx_launch(ctx, batched_copy_kernel, dim3(static_cast<uint32_t>(n * pieces)), dim3(256), 0,
               reinterpret_cast<const CopyOpDev *>(tables.dev), tables.args, static_cast<int>(n), pieces);
    return hip_ok(ctx, hipGetLastError(), what);
}

bool launch_copy_ops(kvmem_hip_ctx *ctx, const std::vector<CopyOpDev> &ops, const char *what) {
    if (ops.empty()) {
        return true;
    }
    LaunchTables tables;
    return stage_copy_ops(ctx, ops, tables, what) &&
           launch_staged_copies(ctx, tables, ops.size(), max_op_bytes(ops), what);
}

bool ensure_h2d_ring(kvmem_hip_ctx *ctx, size_t min_slot_bytes) {
    const size_t want = std::max<size_t>(size_t{32} << 20, min_slot_bytes);
    if (ctx->h2d_ring.ptr && ctx->h2d_slot_bytes >= want) {
        return true;
    }
    // earlier users of the ring must be done before it is replaced
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->copy_stream), "h2d ring sync") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "h2d ring sync")) {
        return false;
    }
    if (ctx->h2d_ring.ptr) {
        (void) hipFree(ctx->h2d_ring.ptr);
        ctx->h2d_ring.ptr = nullptr;
        ctx->h2d_ring.bytes = 0;
    }
    if (!ensure_dev(ctx, ctx->h2d_ring, want * kH2dRing, "h2d ring")) {
        ctx->h2d_slot_bytes = 0;
        return false;
    }
    ctx->h2d_slot_bytes = want;
    ctx->h2d_slots = kH2dRing;
    for (int r = 0; r < kH2dRing; ++r) {
        if (!ctx->h2d_copied[r]) {
            if (!hip_ok(ctx, hipEventCreateWithFlags(&ctx->h2d_copied[r], hipEventDisableTiming), "h2d event") ||
                !hip_ok(ctx, hipEventCreateWithFlags(&ctx->h2d_consumed[r], hipEventDisableTiming), "h2d event")) {
                return false;
            }
        }
        // a fresh "consumed" marker on the compute stream
        if (!hip_ok(ctx, hipEventRecord(ctx->h2d_consumed[r], ctx->stream), "h2d event")) {
            return false;
        }
    }
    return true;
}

uint8_t *host_device_view(const void *p, uint64_t bytes) {
    if (!p || bytes == 0) {
        return nullptr;
    }
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, p) != hipSuccess || a.type != hipMemoryTypeHost ||
        !a.devicePointer) {
        (void) hipGetLastError();
        return nullptr;
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, static_cast<hipDeviceptr_t>(a.devicePointer)) != hipSuccess) {
        (void) hipGetLastError();
        return nullptr;
    }
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    const uintptr_t v = reinterpret_cast<uintptr_t>(a.devicePointer);
    if (v < b || v - b > size || bytes > size - (v - b)) {
        return nullptr;
    }
    return static_cast<uint8_t *>(a.devicePointer);
}

bool load_ctx_kernels() {
    return load_kernel_object(&batched_copy_kernel);
}

}  // namespace kvmem_hip

using namespace kvmem_hip;

extern "C" {

int kvmem_hip_create(int device, kvmem_hip_ctx **out) {
    if (!out) {
        return KVMEM_HIP_ERR_INVALID;
    }
    *out = nullptr;
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || device < 0 || device >= n_dev) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    kvmem_hip_ctx *ctx = new (std::nothrow) kvmem_hip_ctx();
    if (!ctx) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    ctx->device = device;
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking) != hipSuccess ||
        !load_ctx_kernels() || !load_meank_kernels() || !load_score_kernels() ||
        !load_stagein_kernels() || !load_topk_kernels() || !load_qwindow_kernels() ||
        !score_scratch_setup(ctx)) {
        kvmem_hip_destroy(ctx);
        return KVMEM_HIP_ERR_RUNTIME;
    }
    ctx->stream = ctx->own_stream;
    *out = ctx;
    return KVMEM_HIP_OK;
}

void kvmem_hip_destroy(kvmem_hip_ctx *ctx) {
    if (!ctx) {
        return;
    }
    (void) hipSetDevice(ctx->device);
    if (ctx->stream) {
        (void) hipStreamSynchronize(ctx->stream);
    }
    if (ctx->copy_stream) {
        (void) hipStreamSynchronize(ctx->copy_stream);
    }
    for (auto &s : ctx->upload) {
        if (s.host.ptr) (void) hipHostFree(s.host.ptr);
        if (s.dev.ptr) (void) hipFree(s.dev.ptr);
        if (s.done) (void) hipEventDestroy(s.done);
    }
    for (DevBuf *b : {&ctx->score_partial, &ctx->score_layers, &ctx->meank_scratch,
                      &ctx->move_scratch, &ctx->h2d_ring, &ctx->d2h_ring, &ctx->topk_dev, &ctx->plan}) {
        if (b->ptr) (void) hipFree(b->ptr);
    }
    if (ctx->topk_sel_host.ptr) (void) hipHostFree(ctx->topk_sel_host.ptr);
    if (ctx->plan_counts.ptr) (void) hipHostFree(ctx->plan_counts.ptr);
    for (int i = 0; i < 8; ++i) {
        if (ctx->h2d_copied[i]) (void) hipEventDestroy(ctx->h2d_copied[i]);
        if (ctx->h2d_consumed[i]) (void) hipEventDestroy(ctx->h2d_consumed[i]);
    }
    for (int i = 0; i < 2; ++i) {
        if (ctx->d2h_gathered[i]) (void) hipEventDestroy(ctx->d2h_gathered[i]);
        if (ctx->d2h_done[i]) (void) hipEventDestroy(ctx->d2h_done[i]);
    }
    for (int s = 0; s < kPerfStages; ++s) {
        if (ctx->perf_open[s]) (void) hipEventDestroy(ctx->perf_open[s]);
        for (auto &pr : ctx->perf_done[s]) {
            (void) hipEventDestroy(pr.first);
            (void) hipEventDestroy(pr.second);
        }
    }
    for (hipEvent_t e : ctx->perf_free) {
        (void) hipEventDestroy(e);
    }
    if (ctx->attach_start) (void) hipEventDestroy(ctx->attach_start);
    if (ctx->attach_stop) (void) hipEventDestroy(ctx->attach_stop);
    score_scratch_release(ctx);
    if (ctx->noalloc_done) (void) hipEventDestroy(ctx->noalloc_done);
    if (ctx->own_stream) (void) hipStreamDestroy(ctx->own_stream);
    if (ctx->copy_stream) (void) hipStreamDestroy(ctx->copy_stream);
    delete ctx;
}

const char *kvmem_hip_last_error(const kvmem_hip_ctx *ctx) {
    return ctx ? ctx->last_error.c_str() : "null context";
}

int kvmem_hip_set_stream(kvmem_hip_ctx *ctx, void *stream) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
    if (next != ctx->stream) {
        // work on the old stream must not overtake later work on the new one
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "set_stream sync")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        ctx->stream = next;
    }
    return KVMEM_HIP_OK;
}

void *kvmem_hip_get_stream(const kvmem_hip_ctx *ctx) {
    return ctx ? static_cast<void *>(ctx->stream) : nullptr;
}

int kvmem_hip_sync(kvmem_hip_ctx *ctx) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->copy_stream), "sync copy stream") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "sync")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    return KVMEM_HIP_OK;
}

int kvmem_hip_reserve(kvmem_hip_ctx *ctx, const kvmem_hip_reserve_args *a) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!a) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reserve: null arguments");
    }
    const uint32_t L = a->n_layers;
    const uint32_t B = a->n_blocks;
    if (a->n_head_kv && a->n_head % a->n_head_kv != 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "reserve: n_head must be a multiple of n_head_kv");
    }
    if (a->head_dim != 0 && a->head_dim != 128 && a->head_dim != 256) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, "reserve: head_dim must be 128 or 256");
    }
    (void) hipSetDevice(ctx->device);
    const int nomem = KVMEM_HIP_ERR_NOMEM;  // the failing call is in last_error
    if (L && B && a->n_head_kv && a->n_q_tokens &&
        !ensure_dev(ctx, ctx->score_partial,
                    score_partial_bytes(L, a->n_head_kv, B, a->n_q_tokens, a->n_head / a->n_head_kv),
                    "reserve score partial")) {
        return nomem;
    }
    if (L && B && !ensure_dev(ctx, ctx->score_layers, sizeof(float) * static_cast<size_t>(L) * B,
                              "reserve score layers")) {
        return nomem;
    }
    if (L && B && a->n_head_kv && a->head_dim &&
        !ensure_dev(ctx, ctx->meank_scratch, meank_scratch_bytes(L, a->n_head_kv, B, a->head_dim),
                    "reserve score_meank scratch")) {
        return nomem;
    }
    if (B && !ensure_pin(ctx, ctx->topk_sel_host, topk_out_bytes(B), "reserve topk host output",
                         hipHostMallocCoherent | hipHostMallocMapped)) {
        return nomem;
    }
    if (a->max_items || L) {
        const size_t up = upload_bytes_for(std::max(a->max_items, B), L);
        for (auto &slot : ctx->upload) {
            if (!ensure_pin(ctx, slot.host, up, "reserve upload") ||
                !ensure_dev(ctx, slot.dev, up, "reserve upload")) {
                return nomem;
            }
            if (!slot.done && !hip_ok(ctx, hipEventCreateWithFlags(&slot.done, hipEventDisableTiming),
                                      "reserve upload event")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
        }
    }
    if (a->h2d_block_bytes && !ensure_h2d_ring(ctx, a->h2d_block_bytes)) {
        return nomem;
    }
    if (a->d2h_block_bytes && !ensure_d2h_ring(ctx, a->d2h_block_bytes)) {
        return nomem;
    }
    if (a->move_bytes && !ensure_dev(ctx, ctx->move_scratch, a->move_bytes, "reserve move_slots scratch")) {
        return nomem;
    }
    return KVMEM_HIP_OK;
}

int kvmem_hip_scratch_info(const kvmem_hip_ctx *ctx, kvmem_hip_scratch *out) {
    if (!ctx || !out) {
        return KVMEM_HIP_ERR_INVALID;
    }
    uint64_t dev = 0;
    uint64_t pin = 0;
    for (const auto &s : ctx->upload) {
        dev += s.dev.bytes;
        pin += s.host.bytes;
    }
    for (const DevBuf *b : {&ctx->score_partial, &ctx->score_layers, &ctx->meank_scratch,
                            &ctx->move_scratch, &ctx->h2d_ring, &ctx->d2h_ring}) {
        dev += b->bytes;
    }
    pin += ctx->topk_sel_host.bytes;
    out->device_bytes = dev;
    out->pinned_bytes = pin;
    out->allocations = ctx->n_allocs;
    return KVMEM_HIP_OK;
}

int kvmem_hip_h2d_async(kvmem_hip_ctx *ctx, void *dst, const void *src, size_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!dst || !src) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "h2d_async: null pointer");
    }
    (void) hipSetDevice(ctx->device);
    if (injected_fail(ctx, KVMEM_HIP_FAIL_COPY, "h2d_async")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    PerfScope timed(ctx, kPerfCopy);
    if (!hip_ok(ctx, hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ctx->stream), "h2d_async")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    timed.ok();
    note_xfer(ctx, kXferH2D, n);
    return KVMEM_HIP_OK;
}

int kvmem_hip_quant_ok(int type) {
    return type == KVMEM_TYPE_Q8_0 || type == KVMEM_TYPE_Q5_0 || type == KVMEM_TYPE_Q4_0 ||
           type == KVMEM_TYPE_F16;
}

size_t kvmem_hip_row_size(int type, int64_t n) {
    if (n <= 0 || n % 32 != 0) {
        return 0;
    }
    return static_cast<size_t>(group_bytes(type)) * static_cast<size_t>(n / 32);
}

int kvmem_hip_d2d_batched(kvmem_hip_ctx *ctx, const void *const *src, void *const *dst,
                          const size_t *nbytes, int n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n <= 0) {
        return KVMEM_HIP_OK;
    }
    if (!src || !dst || !nbytes) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "d2d_batched: null array");
    }
    std::vector<CopyOpDev> ops(static_cast<size_t>(n));
    uint64_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (!src[i] || !dst[i] || nbytes[i] == 0) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, "d2d_batched: null pointer or empty op");
        }
        ops[i] = {static_cast<const uint8_t *>(src[i]), static_cast<uint8_t *>(dst[i]), nbytes[i]};
        total += nbytes[i];
    }
    (void) hipSetDevice(ctx->device);
    LaunchTables tables;
    if (!stage_copy_ops(ctx, ops, tables, "d2d_batched ops")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    PerfLaunchScope timed(ctx, kPerfLayout);  // events on the copy kernel's launch
    if (!launch_staged_copies(ctx, tables, ops.size(), max_op_bytes(ops), "d2d_batched launch")) {
        return KVMEM_HIP_ERR_RUNTIME;
    }
    timed.ok();
    note_xfer(ctx, kXferD2D, total);
    return KVMEM_HIP_OK;
}

int kvmem_hip_debug_fail_after(kvmem_hip_ctx *ctx, uint32_t kinds, uint64_t nth_op) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint32_t all = KVMEM_HIP_FAIL_ALLOC | KVMEM_HIP_FAIL_COPY | KVMEM_HIP_FAIL_LAUNCH;
    if (kinds & ~all) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, "debug_fail_after: unknown operation kind");
    }
    ctx->fail_kinds = nth_op ? kinds : 0u;
    ctx->fail_countdown = kinds ? nth_op : 0u;
    return KVMEM_HIP_OK;
}

uint64_t kvmem_hip_debug_fail_left(const kvmem_hip_ctx *ctx) {
    return ctx && ctx->fail_kinds ? ctx->fail_countdown : 0u;
}

int kvmem_hip_perf_enable(kvmem_hip_ctx *ctx, int on) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    ctx->perf_on = on != 0;
    return KVMEM_HIP_OK;
}

int kvmem_hip_perf_stages(kvmem_hip_ctx *ctx, uint32_t mask) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    ctx->perf_mask = mask;
    return KVMEM_HIP_OK;
}

int kvmem_hip_perf_get(kvmem_hip_ctx *ctx, kvmem_hip_perf *out) {
    if (!ctx || !out) {
        return KVMEM_HIP_ERR_INVALID;
    }
    perf_collect(ctx);
    out->score_ms = ctx->perf_ms[kPerfScore];
    out->topk_ms = ctx->perf_ms[kPerfTopk];
    out->set_ms = ctx->perf_ms[kPerfSet];
    out->copy_ms = ctx->perf_ms[kPerfCopy];
    out->layout_ms = ctx->perf_ms[kPerfLayout];
    out->n_score = ctx->perf_n[kPerfScore];
    out->n_topk = ctx->perf_n[kPerfTopk];
    out->n_set = ctx->perf_n[kPerfSet];
    out->n_copy = ctx->perf_n[kPerfCopy];
    out->n_layout = ctx->perf_n[kPerfLayout];
    out->h2d_bytes = ctx->xfer_bytes[kXferH2D];
    out->d2d_bytes = ctx->xfer_bytes[kXferD2D];
    out->after_score_ms = ctx->after_score_ms;
    out->n_after_score = ctx->n_after_score;
    out->stage_out_ms = ctx->perf_ms[kPerfStageOut];
    out->plan_ms = ctx->perf_ms[kPerfPlan];
    out->n_stage_out = ctx->perf_n[kPerfStageOut];
    out->n_plan = ctx->perf_n[kPerfPlan];
    out->d2h_bytes = ctx->xfer_bytes[kXferD2H];
    out->meank_cos_ms = ctx->perf_ms[kPerfMeankCos];
    out->n_meank_cos = ctx->perf_n[kPerfMeankCos];
    return KVMEM_HIP_OK;
}

void kvmem_hip_perf_add_plan_ms(kvmem_hip_ctx *ctx, double ms) {
    if (ctx && ctx->perf_on && (ctx->perf_mask & (1u << kPerfPlan))) {
        ctx->perf_ms[kPerfPlan] += ms;
        ctx->perf_n[kPerfPlan] += 1;
    }
}

int kvmem_hip_transfer_get(const kvmem_hip_ctx *ctx, kvmem_hip_transfer_stats *out) {
    if (!ctx || !out) {
        return KVMEM_HIP_ERR_INVALID;
    }
    for (int k = 0; k < 3; ++k) {
        out->bytes[k] = ctx->xfer_bytes[k];
        out->calls[k] = ctx->xfer_calls[k];
    }
    return KVMEM_HIP_OK;
}

void kvmem_hip_perf_reset(kvmem_hip_ctx *ctx) {
    if (!ctx) {
        return;
    }
    perf_collect(ctx);
    for (int s = 0; s < kPerfStages; ++s) {
        // a stage a failed or unfinished call left open starts no later span
        perf_drop(ctx, static_cast<PerfStage>(s));
        ctx->perf_ms[s] = 0.0;
        ctx->perf_n[s] = 0;
    }
    for (int k = 0; k < 3; ++k) {
        ctx->xfer_bytes[k] = 0;
        ctx->xfer_calls[k] = 0;
    }
    ctx->after_score_ms = 0.0;
    ctx->n_after_score = 0;
}

}  // extern "C"
