// Internal definitions shared by the gfx950 translation units of
// libkvmem_hip.so: the context object, status helpers, scratch buffers.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "kvmem_hip.h"

namespace kvmem_hip {

// Grow-only device buffer owned by a context.
struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Grow-only pinned host buffer owned by a context.
struct PinBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};

// Ring slot for small host->device uploads (op tables, id lists): a pinned
// staging area, a device copy and the event that marks the copy consumed.
struct UploadSlot {
    PinBuf host;
    DevBuf dev;
    hipEvent_t done = nullptr;
    bool pending = false;
};

constexpr int kUploadRing = 4;
constexpr int kPerfStages = 8;  // score, topk, set, copy, layout, stage-out, plan, mean-K cosine
enum PerfStage {
    kPerfScore = 0,
    kPerfTopk = 1,
    kPerfSet = 2,
    kPerfCopy = 3,
    kPerfLayout = 4,
    kPerfStageOut = 5,
    kPerfPlan = 6,
    kPerfMeankCos = 7
};
// Directions of the transfer counters (llama_kvmem_transfer_stats order).
enum XferKind { kXferH2D = 0, kXferD2H = 1, kXferD2D = 2 };

}  // namespace kvmem_hip

struct kvmem_hip_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;       // active compute stream
    hipStream_t copy_stream = nullptr;  // side stream for H2D of host blocks
    std::string last_error;

    kvmem_hip::UploadSlot upload[kvmem_hip::kUploadRing];
    int upload_next = 0;

    kvmem_hip::DevBuf score_partial;    // [slices][L][Hkv][B] f32
    kvmem_hip::DevBuf score_layers;     // [L][B] f32 when the caller passes none
    kvmem_hip::DevBuf meank_scratch;    // mean-K scorer: layer cosines, query vectors
    kvmem_hip::DevBuf move_scratch;     // gathered slots for kvmem_hip_move_slots
    // Selection written by the top-k kernel straight into coherent pinned
    // host memory: [n] ids, [n] count, and a completion word the kernel
    // sets to topk_epoch after the rest is visible (topk_flag_index).
    kvmem_hip::PinBuf topk_sel_host;
    uint32_t topk_epoch = 0;
    // a launched top-k not yet waited for: its block count and largest
    // selection; with a device copy of the selection in topk_dev ([0] =
    // count, then the ids) for the device reselect plan
    bool topk_pending = false;
    uint32_t topk_n = 0;
    uint32_t topk_limit = 0;
    kvmem_hip::DevBuf topk_dev;
    // device reselect plan: its tables (stage items, chain segments, slot
    // saves) and counts, and the counts in host-mapped memory
    kvmem_hip::DevBuf plan;
    kvmem_hip::PinBuf plan_counts;
    size_t plan_stage_off = 0;     // the stage table's offset in `plan`
    uint32_t plan_max_sel = 0;     // stage entries the last plan wrote
    uint32_t plan_theta_off = 0;   // RoPE frequencies in the stage table
    uint64_t plan_row_bytes = 0;   // one moved row over every layer, K and V
    uint64_t plan_save_bytes = 0;  // one saved slot over every layer, K and V

    // pinned-host stage-in: device ring of block buffers + events
    kvmem_hip::DevBuf h2d_ring;
    size_t h2d_slot_bytes = 0;
    int h2d_slots = 0;
    hipEvent_t h2d_copied[8] = {};
    hipEvent_t h2d_consumed[8] = {};

    // stage-out: device ring the pool rows are gathered into before D2H
    kvmem_hip::DevBuf d2h_ring;
    size_t d2h_slot_bytes = 0;
    int d2h_next = 0;
    hipEvent_t d2h_gathered[2] = {};
    hipEvent_t d2h_done[2] = {};

    // profiling: start/end event pairs per stage, harvested when read
    bool perf_on = false;
    uint32_t perf_mask = 0xffffffffu;  // stages timed while perf_on (bit = PerfStage)
    std::vector<hipEvent_t> perf_free;                       // reusable events
    hipEvent_t perf_open[kvmem_hip::kPerfStages] = {};       // started, not ended
    // a stage's event pair handed to the next kernel launch (perf_attach):
    // the runtime stamps them with that kernel's own start and end
    hipEvent_t attach_start = nullptr, attach_stop = nullptr;
    bool attach_armed = false;  // not yet taken by a launch
    std::vector<std::pair<hipEvent_t, hipEvent_t>> perf_done[kvmem_hip::kPerfStages];
    double perf_ms[kvmem_hip::kPerfStages] = {};
    uint64_t perf_n[kvmem_hip::kPerfStages] = {};
    // from a scoring stage's end event to the end event of the last
    // stage-in after it (events owned by their stages' pairs)
    hipEvent_t span_score_end = nullptr, span_set_end = nullptr;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> span_done;
    double after_score_ms = 0.0;
    uint64_t n_after_score = 0;
    // bytes and calls per direction (kXferH2D, kXferD2H, kXferD2D) of the
    // data this context moved: one call = one copy launch or runtime copy
    uint64_t xfer_bytes[3] = {};
    uint64_t xfer_calls[3] = {};
    uint64_t n_allocs = 0;  // device + pinned allocations since creation

    // Host-side failure injection (kvmem_hip_debug_fail_after): the
    // fail_countdown-th operation of a kind in fail_kinds fails before it
    // is issued.
    uint32_t fail_kinds = 0;
    uint64_t fail_countdown = 0;

    // Device address of the scorer's static scratch array on this device
    // (kvmem_hip_score_noalloc), looked up when the context is created.
    void *noalloc_scratch = nullptr;
    // Completion of this context's last kvmem_hip_score_noalloc, recorded on
    // the stream it ran on; the device's scratch owner record points here.
    hipEvent_t noalloc_done = nullptr;
};

namespace kvmem_hip {

// Record `msg` as the context's last error and return `code`.
int fail(kvmem_hip_ctx *ctx, int code, const std::string &msg);
// Check a HIP call; on failure record "<what>: <hip error string>".
bool hip_ok(kvmem_hip_ctx *ctx, hipError_t e, const char *what);

// True when this operation (an allocation, a host<->device copy or a
// kernel launch; kvmem_hip_fail_kind) is the one kvmem_hip_debug_fail_after
// chose to fail: the error is recorded and the caller returns before
// issuing anything.
bool injected_fail(kvmem_hip_ctx *ctx, uint32_t kind, const char *what);

bool ensure_dev(kvmem_hip_ctx *ctx, DevBuf &b, size_t bytes, const char *what);
bool ensure_pin(kvmem_hip_ctx *ctx, PinBuf &b, size_t bytes, const char *what,
                unsigned flags = hipHostMallocDefault);

// One device byte copy of the batched copy kernel.
struct CopyOpDev {
    const uint8_t *src;
    uint8_t *dst;
    uint64_t nbytes;
};

// Launch tables small enough travel in the kernel's arguments instead of an
// upload (a pinned copy, an H2D transfer and a blit on the stream before the
// kernel): the kernel reads them in place from its argument segment.  A
// kernel that takes ArgTables binds its table pointers to `dev` when the
// tables were uploaded (too large for the arguments), else to the bytes.
constexpr size_t kArgTableBytes = 3072;
struct ArgTables {
    alignas(16) uint8_t bytes[kArgTableBytes];
};
__device__ inline const uint8_t *table_base(const uint8_t *dev, const ArgTables &t) {
    return dev ? dev : t.bytes;
}
// Table pointers stay generic: a pointer into a kernel's ArgTables must never
// go through an integer (its parameter would be copied to private memory and
// the integer would hold a private-aperture address).  tab_read() reads a
// value at a byte offset of a launch's tables without forming one: from an
// uploaded table through the constant address space (a scalar load when the
// offset is uniform), else from the argument bytes by direct indexing (a
// scalar load from the argument segment).
template <typename T>
__device__ inline T tab_read(const uint8_t *dev, const ArgTables &t, uint32_t off) {
    if (dev) {
        return *reinterpret_cast<const __attribute__((address_space(4))) T *>(
            reinterpret_cast<uintptr_t>(dev) + off);
    }
    T v;
    __builtin_memcpy(&v, &t.bytes[off], sizeof(T));
    return v;
}

// A value at byte offset `off` of a table in device memory (an allocation,
// never a kernel parameter), read through the constant address space: a
// scalar load when the offset is uniform.  The table is not written by the
// reading kernel.
template <typename T>
__device__ inline T cload(const uint8_t *dev, uint32_t off) {
    return *reinterpret_cast<const __attribute__((address_space(4))) T *>(reinterpret_cast<uintptr_t>(dev) + off);
}

// A device-memory address (an allocation, never a kernel parameter) in the
// global address space: global_load / global_store instead of flat ones.
template <typename T>
using global_ptr = __attribute__((address_space(1))) T *;
template <typename T>
__device__ inline global_ptr<T> as_global(T *p) {
    return reinterpret_cast<global_ptr<T>>(reinterpret_cast<uintptr_t>(p));
}

// Tables for one launch: copied into `args` when they fit (dev = null),
// else uploaded (dev = the device copy).  False on an upload failure.
struct LaunchTables {
    const uint8_t *dev = nullptr;
    ArgTables args;
};
bool stage_tables(kvmem_hip_ctx *ctx, const void *src, size_t bytes, LaunchTables &out, const char *what);

// Upload `ops` and copy them in one launch on the context stream (each op
// split into pieces of about 16 KiB, one per workgroup, and few small ops
// into more so that a launch fills the chip; 16-byte vectors where
// aligned).  The two halves apart: the upload, then launches of the
// uploaded table (e.g. inside a timing bracket), which take the largest
// op's size to size the pieces.
bool launch_copy_ops(kvmem_hip_ctx *ctx, const std::vector<CopyOpDev> &ops, const char *what);
bool stage_copy_ops(kvmem_hip_ctx *ctx, const std::vector<CopyOpDev> &ops, LaunchTables &out, const char *what);
bool launch_staged_copies(kvmem_hip_ctx *ctx, const LaunchTables &tables, size_t n, uint64_t max_bytes,
                          const char *what);
uint64_t max_op_bytes(const std::vector<CopyOpDev> &ops);
// Copies whose count an earlier kernel on the stream writes: min(*count,
// max_ops) ops of the device table `ops` (a grid sized for max_ops).
bool launch_dev_copies(kvmem_hip_ctx *ctx, const CopyOpDev *ops, const uint32_t *count, uint32_t max_ops,
                       const char *what);

// The pinned-host stage-in ring: kH2dRing device slots of at least
// `min_slot_bytes` (32 MiB or more, grown only), with their events.
constexpr int kH2dRing = 4;
bool ensure_h2d_ring(kvmem_hip_ctx *ctx, size_t min_slot_bytes);

// The stage-out ring: two device slots of at least `min_slot_bytes`
// (128 MiB or more, grown only), with their events.
bool ensure_d2h_ring(kvmem_hip_ctx *ctx, size_t min_slot_bytes);

// Scratch sizes of the entry points, shared with kvmem_hip_reserve.
// Per-token scorer partial maxima for `n_q_tokens` query tokens of `g` query
// heads per KV head.
size_t score_partial_bytes(uint32_t L, uint32_t Hkv, uint32_t B, uint32_t n_q_tokens, uint32_t g);
// Mean-K scorer: query vectors and per-(layer, block) cosines.
size_t meank_scratch_bytes(uint32_t L, uint32_t Hkv, uint32_t B, uint32_t D);
// Selection output of kvmem_hip_topk over `n` blocks (device and pinned).
// Top-k host output: n ids, the count, then the completion word on its own
// 64-byte line.
inline size_t topk_flag_index(uint32_t n) { return (static_cast<size_t>(n) + 1 + 15) / 16 * 16; }
inline size_t topk_out_bytes(uint32_t n) { return (topk_flag_index(n) + 16) * sizeof(uint32_t); }
// Largest table one call with `items` ids / ops / blocks over `L` layers
// uploads: 32-byte quantize ops, 24-byte copies of K and V per layer for a
// block (packed stage-in/out, slot moves), 16-byte block items after 2L
// pool pointers and up to 128 RoPE frequencies, or 76-byte slot-move chain
// segments after 2L pool pointers.
inline size_t upload_bytes_for(uint32_t items, uint32_t L) {
    const size_t per_item = std::max<size_t>(80, 48 * static_cast<size_t>(L));
    return per_item * items + 16 * static_cast<size_t>(L) + 1024;
}

// The device's address for host memory [p, p + bytes) when the whole range
// lies inside one pinned host allocation (kernels may then read or write it
// directly over the link); nullptr otherwise (pageable memory, a range past
// the allocation).  Clears the runtime error a failed query leaves behind.
uint8_t *host_device_view(const void *p, uint64_t bytes);

// Copy `bytes` of host data to device memory through the upload ring,
// ordered on the context stream.  Returns the device address or nullptr.
void *upload(kvmem_hip_ctx *ctx, const void *src, size_t bytes, const char *what);

// Top-k in two halves (kvmem_hip_topk is both): topk_launch enqueues the
// selection kernel (with `to_device`, also writing the selection to
// ctx->topk_dev); topk_wait spins until the selection is on the host,
// asking the stream for a failure once hold_off_us have passed.
int topk_launch(kvmem_hip_ctx *ctx, const float *scores, uint32_t n, const uint32_t *forced,
                uint32_t n_forced, uint32_t need, int tie_lower_index, bool to_device);
int topk_wait(kvmem_hip_ctx *ctx, uint32_t *sel_out, uint32_t *n_sel, int64_t hold_off_us);

// Profiling brackets around a stage's launches on the context stream.
void perf_begin(kvmem_hip_ctx *ctx, PerfStage s);
void perf_end(kvmem_hip_ctx *ctx, PerfStage s);
// Forget a started stage without timing it (the call failed).
void perf_drop(kvmem_hip_ctx *ctx, PerfStage s);
// A timed stage of exactly one kernel launch: perf_attach hands a start and
// an end event to the next ctx_launch, which passes them to the runtime with
// the kernel, so they carry the kernel's own start and end times -- no
// marker packets around it, which hold the stream idle a few microseconds
// each.  perf_detach files the pair as the stage's when the launch took it
// (`ok`), else returns it.  Returns false when the stage is not timed.
bool perf_attach(kvmem_hip_ctx *ctx, PerfStage s);
void perf_detach(kvmem_hip_ctx *ctx, PerfStage s, bool ok);

// A kernel launch on the context stream, carrying the events perf_attach
// left for it, if any.
template <typename... Params, typename... Args>
inline void ctx_launch(kvmem_hip_ctx *ctx, void (*kernel)(Params...), dim3 grid, dim3 block, uint32_t shmem,
                       const Args &...args) {
    if (ctx->attach_armed) {
        ctx->attach_armed = false;  // one launch per attachment; perf_detach files the pair
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, ctx->stream, ctx->attach_start, ctx->attach_stop, 0u,
                              static_cast<Params>(args)...);
    } else {
        kernel<<<grid, block, shmem, ctx->stream>>>(args...);
    }
}

// A timed stage over a scope: started on construction, ended by ok() once
// the work is enqueued, dropped on destruction otherwise, so that no
// return path leaves the stage open.
class PerfScope {
public:
    PerfScope(kvmem_hip_ctx *ctx, PerfStage s) : ctx_(ctx), s_(s) { perf_begin(ctx_, s_); }
    ~PerfScope() {
        if (!done_) {
            perf_drop(ctx_, s_);
        }
    }
    void ok() {
        if (!done_) {
            perf_end(ctx_, s_);
            done_ = true;
        }
    }
    PerfScope(const PerfScope &) = delete;
    PerfScope &operator=(const PerfScope &) = delete;

private:
    kvmem_hip_ctx *ctx_;
    PerfStage s_;
    bool done_ = false;
};

// A timed stage of one kernel launch over a scope, with the events carried
// by the launch (perf_attach): filed by ok() once the kernel is enqueued,
// returned on destruction otherwise.
class PerfLaunchScope {
public:
    PerfLaunchScope(kvmem_hip_ctx *ctx, PerfStage s) : ctx_(ctx), s_(s), on_(perf_attach(ctx, s)) {}
    ~PerfLaunchScope() {
        if (on_) {
            perf_detach(ctx_, s_, false);
        }
    }
    void ok() {
        if (on_) {
            perf_detach(ctx_, s_, true);
            on_ = false;
        }
    }
    PerfLaunchScope(const PerfLaunchScope &) = delete;
    PerfLaunchScope &operator=(const PerfLaunchScope &) = delete;

private:
    kvmem_hip_ctx *ctx_;
    PerfStage s_;
    bool on_;
};

// Count `bytes` moved in direction k by `calls` copy operations.
void note_xfer(kvmem_hip_ctx *ctx, XferKind k, uint64_t bytes, uint64_t calls = 1);
// Harvest finished event pairs into the accumulators (blocking).
void perf_collect(kvmem_hip_ctx *ctx);

// Each .hip file's kernels make one code object, which HIP loads onto the
// device at the first launch of any of them (about 5 ms for the stage-in
// object).  Context creation asks each object for one kernel's attributes,
// which loads it there, so no reselect step pays the load.
bool load_ctx_kernels();
bool load_meank_kernels();
bool load_score_kernels();
bool load_stagein_kernels();
bool load_topk_kernels();
bool load_qwindow_kernels();
// Looks up, once per device (the context's, made current by the caller),
// the device address of the static scratch array of
// kvmem_hip_score_noalloc and keeps it in ctx->noalloc_scratch.
bool score_scratch_setup(kvmem_hip_ctx *ctx);
// Forgets ctx as the owner of its device's scratch (the context goes away).
void score_scratch_release(kvmem_hip_ctx *ctx);

template <typename K>
inline bool load_kernel_object(K *kernel) {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void *>(kernel)) == hipSuccess;
}

// 16-byte load that is not expected to be reused (streamed history data).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ inline uint4 load_stream16(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t *>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Block format helpers (ggml layouts).
inline uint32_t group_bytes(int type) {
    switch (type) {
        case KVMEM_TYPE_Q8_0: return 34;
        case KVMEM_TYPE_Q4_0: return 18;
        case KVMEM_TYPE_Q5_0: return 22;
        case KVMEM_TYPE_F16: return 64;
        default: return 0;
    }
}

}  // namespace kvmem_hip
