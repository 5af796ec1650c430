/* Internal to libkvmem_hip.so (not exported): the device halves that the
 * reselect engine's one-call path (kvmem_engine_apply_retrieval) strings
 * together, so that top-k, the selection diff and the slot moves run back
 * to back on the stream with no host round trip between them, and the
 * stage-in the host queues meanwhile follows the moves.  Plain C types,
 * for the engine's host C++. */
#pragma once

#include <stdint.h>

#include "kvmem_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest selection and pool the device plan takes (one selected block per
 * thread of its workgroup; slot tables in its LDS). */
#define KVMEM_PLAN_MAX_SEL 1024u
#define KVMEM_PLAN_MAX_SLOTS 4096u

/* Counts of a device plan, read with kvmem_hip_reselect_device_counts. */
enum {
    KVMEM_PLAN_STAGE = 0,    /* blocks staged */
    KVMEM_PLAN_MOVES = 1,    /* slot moves */
    KVMEM_PLAN_SEGS = 2,     /* chain segments */
    KVMEM_PLAN_SAVES = 3,    /* slots saved before the chain walk */
    KVMEM_PLAN_SAVE_OPS = 4, /* their copies */
    KVMEM_PLAN_SEL = 5,      /* selected blocks */
    KVMEM_PLAN_ERROR = 6,    /* nonzero: the plan was refused, nothing moved or staged */
    KVMEM_PLAN_ROWS = 7,     /* rows the moves carry */
    KVMEM_PLAN_N_COUNTS = 8
};

/* kvmem_hip_topk's launch half, also leaving the selection in device memory
 * for kvmem_hip_reselect_device; kvmem_hip_topk_wait is its wait half. */
int kvmem_hip_topk_launch_dev(kvmem_hip_ctx *ctx, const float *scores, uint32_t n,
                              const uint32_t *forced, uint32_t n_forced, uint32_t need,
                              int tie_lower_index);
int kvmem_hip_topk_wait(kvmem_hip_ctx *ctx, uint32_t *sel_out, uint32_t *n_sel);

/* Behind the launched top-k: the plan kernel, the slot saves and the chain
 * walk of a canonical-layout apply (window slot i = the i-th selected
 * block), sized on the device.  res_block / res_slot list the blocks whose
 * pool rows are valid, ascending in id and in slot; dirty is a resident
 * block to stage again (UINT32_MAX for none); max_sel bounds the selection
 * size.  Device history, no pool transform, 16-byte rows. */
int kvmem_hip_reselect_device(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                              const kvmem_hip_pool *pool, const uint32_t *res_block,
                              const uint32_t *res_slot, uint32_t n_res, uint32_t dirty,
                              uint32_t max_sel);

/* The stage-in of the plan's n_staged blocks (the count the host's store
 * finds for the same selection), queued behind the chain walk; their items
 * are the plan kernel's. */
int kvmem_hip_reselect_device_stagein(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                                      const kvmem_hip_pool *pool, uint32_t n_staged);

/* The counts of the last device plan (out[0 .. n), KVMEM_PLAN_*), valid
 * once the stream has drained. */
int kvmem_hip_reselect_device_counts(kvmem_hip_ctx *ctx, uint32_t *out, uint32_t n);

/* Host time of the engine's own diff and slot plan, added to the plan
 * bucket of kvmem_hip_perf when that stage is timed. */
void kvmem_hip_perf_add_plan_ms(kvmem_hip_ctx *ctx, double ms);

#ifdef __cplusplus
}
#endif
