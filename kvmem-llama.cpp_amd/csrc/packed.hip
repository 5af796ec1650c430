// Packed host rows: stage-out (pool slots -> pinned host, the rows as the
// cache holds them) and the packed stage-in (pinned host -> pool slots, no
// quantization), the two directions of the reference's packed-row traffic
// (stage-out gather + D2H, llama-kvmem-stagein.cu:842-963; the live
// write_block_to_gpu upload, llama-memory-kvmem.cpp:2726-2791).
//
// A store in pinned memory is read or written by the copy kernel itself:
// one launch moves every row over the link at its full rate (runtime copies
// of a few MB each leave ~10 us gaps between them).  A pageable store goes
// through copy pipelines over two streams.  Stage-out gathers a batch of
// blocks (every layer, K and V) into a 128 MiB device ring slot in the host
// layout with one copy launch on the context stream, then copies the spans
// device-to-host on the side stream (runs of consecutive blocks as one
// copy); two ring slots alternate so the next gather overlaps the previous
// copies.  The packed stage-in
// copies block spans host-to-device into the stage-in ring on the side
// stream and scatters each batch into the slots with one copy launch.  HBM
// work is a few hundred MB per step; the bound is the PCIe link.
#include "kvmem_internal.hpp"

#include <algorithm>
#include <vector>

using namespace kvmem_hip;

namespace {

struct PackedGeom {
    uint64_t row_k = 0;
    uint64_t row_v = 0;
    uint64_t run_k = 0;        // block_tokens * row_k
    uint64_t run_v = 0;        // block_tokens * row_v
    uint64_t layer_bytes = 0;  // run_k + run_v
    uint64_t span = 0;         // bytes of one block, every layer
};

int check_packed(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool, const kvmem_hip_packed_host *host,
                 const uint32_t *block_ids, const uint32_t *slots, const uint32_t *n_tokens,
                 uint32_t n, PackedGeom &g, const char *who) {
    if (!pool || !pool->k_layers || !host || !host->base || !block_ids || !slots || !n_tokens) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, std::string(who) + ": null argument");
    }
    const bool want_v = pool->v_layers != nullptr;
    if (host->n_layers != pool->n_layers || host->block_tokens != pool->block_tokens ||
        pool->block_tokens == 0 || pool->n_layers == 0) {
        return fail(ctx, KVMEM_HIP_ERR_INVALID, std::string(who) + ": packed store geometry does not match the pool");
    }
    g.row_k = kvmem_hip_row_size(pool->type_k, pool->n_embd_k);
    g.row_v = want_v ? kvmem_hip_row_size(pool->type_v, pool->n_embd_v) : 0;
    if (g.row_k == 0 || (want_v && g.row_v == 0)) {
        return fail(ctx, KVMEM_HIP_ERR_UNSUPPORTED, std::string(who) + ": unsupported cache type or row width");
    }
    for (uint32_t l = 0; l < pool->n_layers; ++l) {
        if (!pool->k_layers[l] || (want_v && !pool->v_layers[l])) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID, std::string(who) + ": null layer pointer");
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (block_ids[i] >= host->n_blocks || slots[i] >= pool->n_slots ||
            n_tokens[i] > pool->block_tokens) {
            return fail(ctx, KVMEM_HIP_ERR_INVALID,
                        std::string(who) + ": block id, slot or token count out of range");
        }
    }
    g.run_k = g.row_k * pool->block_tokens;
    g.run_v = g.row_v * pool->block_tokens;
    g.layer_bytes = g.run_k + g.run_v;
    g.span = g.layer_bytes * pool->n_layers;
    return KVMEM_HIP_OK;
}

}  // namespace

namespace kvmem_hip {

bool ensure_d2h_ring(kvmem_hip_ctx *ctx, size_t min_slot_bytes) {
    // device-to-host copies reach the link rate only in large pieces
    const size_t want = std::max<size_t>(size_t{128} << 20, min_slot_bytes);
    if (ctx->d2h_ring.ptr && ctx->d2h_slot_bytes >= want) {
        return true;
    }
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->copy_stream), "d2h ring sync") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "d2h ring sync")) {
        return false;
    }
    if (ctx->d2h_ring.ptr) {
        (void) hipFree(ctx->d2h_ring.ptr);
        ctx->d2h_ring.ptr = nullptr;
        ctx->d2h_ring.bytes = 0;
    }
    if (!ensure_dev(ctx, ctx->d2h_ring, want * 2, "d2h ring")) {
        ctx->d2h_slot_bytes = 0;
        return false;
    }
    ctx->d2h_slot_bytes = want;
    for (int r = 0; r < 2; ++r) {
        if (!ctx->d2h_done[r]) {
            if (!hip_ok(ctx, hipEventCreateWithFlags(&ctx->d2h_gathered[r], hipEventDisableTiming), "d2h event") ||
                !hip_ok(ctx, hipEventCreateWithFlags(&ctx->d2h_done[r], hipEventDisableTiming), "d2h event")) {
                return false;
            }
        }
        // a fresh "copied out" marker: the slot is free
        if (!hip_ok(ctx, hipEventRecord(ctx->d2h_done[r], ctx->copy_stream), "d2h event")) {
            return false;
        }
    }
    return true;
}

}  // namespace kvmem_hip

extern "C" {

int kvmem_hip_stageout_blocks(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool,
                              const kvmem_hip_packed_host *dst, const uint32_t *block_ids,
                              const uint32_t *slots, const uint32_t *n_tokens, uint32_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    PackedGeom g;
    int st = check_packed(ctx, pool, dst, block_ids, slots, n_tokens, n, g, "stageout_blocks");
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    (void) hipSetDevice(ctx->device);
    // Pinned store: one copy launch writes the rows over the link.
    if (uint8_t *view = host_device_view(dst->base, static_cast<uint64_t>(dst->n_blocks) * g.span)) {
        std::vector<CopyOpDev> ops;
        ops.reserve(static_cast<size_t>(n) * pool->n_layers * 2);
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t nt = n_tokens[i];
            for (uint32_t l = 0; l < pool->n_layers && nt > 0; ++l) {
                uint8_t *d = view + static_cast<uint64_t>(block_ids[i]) * g.span + l * g.layer_bytes;
                ops.push_back({static_cast<const uint8_t *>(pool->k_layers[l]) + slots[i] * g.run_k, d,
                               nt * g.row_k});
                if (g.row_v) {
                    ops.push_back({static_cast<const uint8_t *>(pool->v_layers[l]) + slots[i] * g.run_v,
                                   d + g.run_k, nt * g.row_v});
                }
            }
        }
        uint64_t bytes = 0;
        for (const CopyOpDev &op : ops) bytes += op.nbytes;
        PerfScope timed(ctx, kPerfStageOut);
        if (!launch_copy_ops(ctx, ops, "stage-out to the pinned store")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        timed.ok();
        note_xfer(ctx, kXferD2H, bytes);
        return KVMEM_HIP_OK;
    }
    // Pageable store: gather into the device ring, then runtime copies.
    if (!ensure_d2h_ring(ctx, g.span)) {
        return KVMEM_HIP_ERR_NOMEM;  // the failing call is in kvmem_hip_last_error
    }
    const uint64_t slot_bytes = ctx->d2h_slot_bytes;
    const uint32_t per_slot = static_cast<uint32_t>(slot_bytes / g.span);
    const uint32_t T = pool->block_tokens;
    uint8_t *host = static_cast<uint8_t *>(dst->base);
    uint8_t *ring = static_cast<uint8_t *>(ctx->d2h_ring.ptr);
    PerfScope timed(ctx, kPerfStageOut);
    int r = ctx->d2h_next;
    for (uint32_t first = 0; first < n; first += per_slot) {
        const uint32_t cnt = std::min(per_slot, n - first);
        uint8_t *slot_base = ring + static_cast<uint64_t>(r) * slot_bytes;
        // the copy-out of this ring slot's previous batch must be done
        if (!hip_ok(ctx, hipStreamWaitEvent(ctx->stream, ctx->d2h_done[r], 0), "d2h wait free")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        std::vector<CopyOpDev> ops;
        ops.reserve(static_cast<size_t>(cnt) * pool->n_layers * 2);
        for (uint32_t j = 0; j < cnt; ++j) {
            const uint32_t i = first + j;
            const uint32_t nt = n_tokens[i];
            if (nt == 0) {
                continue;
            }
            for (uint32_t l = 0; l < pool->n_layers; ++l) {
                uint8_t *d = slot_base + j * g.span + l * g.layer_bytes;
                ops.push_back({static_cast<const uint8_t *>(pool->k_layers[l]) + slots[i] * g.run_k, d,
                               nt * g.row_k});
                if (g.row_v) {
                    ops.push_back({static_cast<const uint8_t *>(pool->v_layers[l]) + slots[i] * g.run_v,
                                   d + g.run_k, nt * g.row_v});
                }
            }
        }
        if (!launch_copy_ops(ctx, ops, "stage-out gather")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        uint64_t gathered = 0;
        for (const CopyOpDev &op : ops) gathered += op.nbytes;
        note_xfer(ctx, kXferD2D, gathered);
        if (!hip_ok(ctx, hipEventRecord(ctx->d2h_gathered[r], ctx->stream), "d2h record") ||
            !hip_ok(ctx, hipStreamWaitEvent(ctx->copy_stream, ctx->d2h_gathered[r], 0), "d2h wait gathered")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        for (uint32_t j = 0; j < cnt; ++j) {
            const uint32_t i = first + j;
            const uint32_t nt = n_tokens[i];
            uint8_t *hb = host + static_cast<uint64_t>(block_ids[i]) * g.span;
            const uint8_t *db = slot_base + j * g.span;
            if (nt == T) {
                // full blocks are contiguous spans on both sides; a run of
                // consecutive full blocks goes out as one copy
                uint32_t run = 1;
                while (j + run < cnt && n_tokens[i + run] == T && block_ids[i + run] == block_ids[i] + run) {
                    ++run;
                }
                if (injected_fail(ctx, KVMEM_HIP_FAIL_COPY, "d2h block copy")) {
                    return KVMEM_HIP_ERR_RUNTIME;
                }
                if (!hip_ok(ctx, hipMemcpyAsync(hb, db, run * g.span, hipMemcpyDeviceToHost, ctx->copy_stream),
                            "d2h block copy")) {
                    return KVMEM_HIP_ERR_RUNTIME;
                }
                note_xfer(ctx, kXferD2H, run * g.span);
                j += run - 1;
                continue;
            }
            // a partial block: only its rows, so the rest of the host run is untouched
            for (uint32_t l = 0; l < pool->n_layers && nt > 0; ++l) {
                const uint64_t o = l * g.layer_bytes;
                if (!hip_ok(ctx, hipMemcpyAsync(hb + o, db + o, nt * g.row_k, hipMemcpyDeviceToHost,
                                                ctx->copy_stream), "d2h rows copy")) {
                    return KVMEM_HIP_ERR_RUNTIME;
                }
                note_xfer(ctx, kXferD2H, nt * g.row_k);
                if (g.row_v &&
                    !hip_ok(ctx, hipMemcpyAsync(hb + o + g.run_k, db + o + g.run_k, nt * g.row_v,
                                                hipMemcpyDeviceToHost, ctx->copy_stream), "d2h rows copy")) {
                    return KVMEM_HIP_ERR_RUNTIME;
                }
                if (g.row_v) {
                    note_xfer(ctx, kXferD2H, nt * g.row_v);
                }
            }
        }
        if (!hip_ok(ctx, hipEventRecord(ctx->d2h_done[r], ctx->copy_stream), "d2h record done")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        r ^= 1;
    }
    ctx->d2h_next = r;
    timed.ok();
    return KVMEM_HIP_OK;
}

int kvmem_hip_stagein_packed_host(kvmem_hip_ctx *ctx, const kvmem_hip_packed_host *src,
                                  const kvmem_hip_pool *pool, const uint32_t *block_ids,
                                  const uint32_t *slots, const uint32_t *n_tokens, uint32_t n) {
    if (!ctx) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    PackedGeom g;
    int st = check_packed(ctx, pool, src, block_ids, slots, n_tokens, n, g, "stagein_packed_host");
    if (st != KVMEM_HIP_OK) {
        return st;
    }
    (void) hipSetDevice(ctx->device);
    // Pinned store: one copy launch reads the rows over the link.
    if (const uint8_t *view = host_device_view(src->base, static_cast<uint64_t>(src->n_blocks) * g.span)) {
        std::vector<CopyOpDev> ops;
        ops.reserve(static_cast<size_t>(n) * pool->n_layers * 2);
        uint64_t bytes = 0;
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t nt = n_tokens[i];
            for (uint32_t l = 0; l < pool->n_layers && nt > 0; ++l) {
                const uint8_t *s = view + static_cast<uint64_t>(block_ids[i]) * g.span + l * g.layer_bytes;
                ops.push_back({s, static_cast<uint8_t *>(pool->k_layers[l]) + slots[i] * g.run_k, nt * g.row_k});
                bytes += nt * g.row_k;
                if (g.row_v) {
                    ops.push_back({s + g.run_k, static_cast<uint8_t *>(pool->v_layers[l]) + slots[i] * g.run_v,
                                   nt * g.row_v});
                    bytes += nt * g.row_v;
                }
            }
        }
        PerfScope timed(ctx, kPerfSet);
        if (!launch_copy_ops(ctx, ops, "packed stage-in from the pinned store")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        timed.ok();
        note_xfer(ctx, kXferH2D, bytes);
        return KVMEM_HIP_OK;
    }
    // Pageable store: runtime copies into the stage-in ring, then a scatter.
    if (!ensure_h2d_ring(ctx, g.span)) {
        return KVMEM_HIP_ERR_NOMEM;  // the failing call is in kvmem_hip_last_error
    }
    const uint64_t slot_bytes = ctx->h2d_slot_bytes;
    const uint32_t per_slot = static_cast<uint32_t>(slot_bytes / g.span);
    const uint8_t *host = static_cast<const uint8_t *>(src->base);
    uint8_t *ring = static_cast<uint8_t *>(ctx->h2d_ring.ptr);
    PerfScope timed(ctx, kPerfSet);
    int r = 0;
    for (uint32_t first = 0; first < n; first += per_slot) {
        const uint32_t cnt = std::min(per_slot, n - first);
        uint8_t *slot_base = ring + static_cast<uint64_t>(r) * slot_bytes;
        // the scatter that last read this ring slot must be done
        if (!hip_ok(ctx, hipStreamWaitEvent(ctx->copy_stream, ctx->h2d_consumed[r], 0), "h2d wait consumed")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        for (uint32_t j = 0; j < cnt; ++j) {
            // a run of consecutive blocks comes in as one copy
            const uint32_t b = block_ids[first + j];
            uint32_t run = 1;
            while (j + run < cnt && block_ids[first + j + run] == b + run) {
                ++run;
            }
            if (injected_fail(ctx, KVMEM_HIP_FAIL_COPY, "h2d packed block copy")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
            if (!hip_ok(ctx, hipMemcpyAsync(slot_base + j * g.span, host + static_cast<uint64_t>(b) * g.span,
                                            run * g.span, hipMemcpyHostToDevice, ctx->copy_stream),
                        "h2d packed block copy")) {
                return KVMEM_HIP_ERR_RUNTIME;
            }
            note_xfer(ctx, kXferH2D, run * g.span);
            j += run - 1;
        }
        if (!hip_ok(ctx, hipEventRecord(ctx->h2d_copied[r], ctx->copy_stream), "h2d record") ||
            !hip_ok(ctx, hipStreamWaitEvent(ctx->stream, ctx->h2d_copied[r], 0), "h2d wait copied")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        std::vector<CopyOpDev> ops;
        ops.reserve(static_cast<size_t>(cnt) * pool->n_layers * 2);
        for (uint32_t j = 0; j < cnt; ++j) {
            const uint32_t i = first + j;
            const uint32_t nt = n_tokens[i];
            if (nt == 0) {
                continue;
            }
            for (uint32_t l = 0; l < pool->n_layers; ++l) {
                const uint8_t *s = slot_base + j * g.span + l * g.layer_bytes;
                ops.push_back({s, static_cast<uint8_t *>(pool->k_layers[l]) + slots[i] * g.run_k, nt * g.row_k});
                if (g.row_v) {
                    ops.push_back({s + g.run_k, static_cast<uint8_t *>(pool->v_layers[l]) + slots[i] * g.run_v,
                                   nt * g.row_v});
                }
            }
        }
        if (!launch_copy_ops(ctx, ops, "packed stage-in scatter")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        uint64_t scattered = 0;
        for (const CopyOpDev &op : ops) scattered += op.nbytes;
        note_xfer(ctx, kXferD2D, scattered);
        if (!hip_ok(ctx, hipEventRecord(ctx->h2d_consumed[r], ctx->stream), "h2d record consumed")) {
            return KVMEM_HIP_ERR_RUNTIME;
        }
        r = (r + 1) % kH2dRing;
    }
    timed.ok();
    return KVMEM_HIP_OK;
}

}  // extern "C"
