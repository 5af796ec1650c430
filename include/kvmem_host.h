/*
 * kvmem_host.h -- C ABI of the reselect engine: the per-agent-step
 * score -> top-k -> diff -> stage-in path of the reference adapter,
 * driving the gfx950 kernels of kvmem_hip.h.
 *
 * It replaces, for this path, llama_memory_kvmem's preview_retrieval /
 * apply_selection / apply_retrieval (src/adapter/llama-memory-kvmem.cpp:
 * 3047-3067, 3139-3263; C API llama_kvmem_preview_retrieval /
 * llama_kvmem_apply_selection / llama_kvmem_apply_retrieval,
 * src/adapter/llama-kvmem-hooks.h:100,149-160) together with the host
 * library calls they make (KvMemStore::set_retrieval_scores,
 * pick_topk_blocks, set_selection; KvMemRuntime::prepare_selection,
 * spill_outgoing, admit_incoming; kvmem/src/host/kvmem_store.cpp,
 * kvmem_runtime.cpp).  The two-phase shape is kept: preview returns a
 * selection stamped with an epoch and the history row count, apply rejects
 * a stale one (KVMEM_HIP_ERR_STALE; the reference throws
 * std::runtime_error("stale KVMem selection"), llama-memory-kvmem.cpp:
 * 3144-3147).
 *
 * Also exported: the host store alone (kvmem_store_*), with no device, for
 * callers and tests that exercise selection and diff semantics.
 *
 * Lifetimes: history pointers (device K/V, pinned host blocks) and query
 * pointers are borrowed; the caller keeps them valid until the call that
 * uses them returns (preview and apply synchronise the engine's stream
 * before returning).  Pool memory is owned by the engine unless borrowed
 * with kvmem_engine_set_pool.  An engine is
 * not re-entrant: one engine per host thread.
 */
#ifndef KVMEM_HOST_H
#define KVMEM_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "kvmem_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------ selection & plan */

/* Counters of one applied selection (KvMemPlan, kvmem_store.hpp:108-124,
 * plus the device work it caused). */
typedef struct kvmem_plan_stats {
    uint32_t n_stage_in;               /* blocks entering the working set */
    uint32_t n_stage_out;              /* resident blocks leaving it */
    uint32_t n_staged;                 /* blocks written into the pool (quantized
                                          or restored from packed rows) */
    uint32_t n_moved;                  /* resident blocks moved (canonical layout) */
    uint32_t selection_overlap_blocks;
    uint32_t gpu_reused_blocks;
    uint32_t retained_position_stable;
    uint32_t retained_position_moved;
    uint32_t total_window_tokens;
    uint32_t n_saved;                  /* evicted blocks copied to the packed host store */
    uint32_t n_restored;               /* staged blocks restored from packed rows */
    uint32_t device_planned;           /* 1: the diff and slot plan ran on the device
                                          (kvmem_engine_params.device_plan) */
    uint32_t n_skip;                   /* window blocks whose baked position equals
                                          their window position (KvMemRemap.skip,
                                          the reference's n_skip,
                                          llama-memory-kvmem.cpp:3152-3158) */
} kvmem_plan_stats;

/* A half-open range [begin, end) of history rows (token positions);
 * llama_kvmem_row_range (src/adapter/llama-kvmem-hooks.h:123-126). */
typedef struct kvmem_row_range {
    int32_t begin;
    int32_t end;
} kvmem_row_range;

/* An attention view (llama_kvmem_attention_view, src/adapter/
 * llama-kvmem-hooks.h:143-148): the blocks attention reads -- every block
 * holding a pool slot, ascending -- with the attention epoch and the history
 * rows it was taken at.  valid = 1 when every one of them has all its rows
 * in the pool (and, for a canonical view, the i-th of them sits in slot i).
 * The attention epoch moves whenever pool contents or residency change (an
 * apply that stages, moves or evicts, a truncate, a new pool or history, a
 * failed apply); rows appended do not move it (the adapter's
 * attention_epoch_, llama-memory-kvmem.cpp:630-1495, 2735).  The caller
 * owns `blocks` (capacity entries); calls that fill a view set n_blocks
 * always and the ids when they fit. */
typedef struct kvmem_attention_view {
    uint64_t epoch;
    uint32_t rows;
    int32_t valid;
    uint32_t n_blocks;
    uint32_t capacity;
    uint32_t *blocks;
} kvmem_attention_view;

/* ----------------------------------------------------------- host store */

typedef struct kvmem_store kvmem_store;

/* Store with block_tokens per block and a budget of budget_blocks, keeping
 * sink_blocks first and recent_blocks last blocks (KvMemStoreConfig,
 * kvmem_store.hpp:223-232).  tie_lower_index = 1 ranks equal scores by
 * lower block id; 0 by higher id as the reference (kvmem_store.cpp:602-609).
 * The store has a slot pool of n_slots (LIFO, llama-memory-kvmem.cpp:
 * 621-627, 693-707) and every registered block starts outside the pool. */
KVMEM_HIP_API int kvmem_store_create(uint32_t block_tokens, uint32_t budget_blocks,
                                     uint32_t sink_blocks, uint32_t recent_blocks,
                                     int tie_lower_index, uint32_t n_slots,
                                     kvmem_store **out);
KVMEM_HIP_API void kvmem_store_destroy(kvmem_store *s);
/* KvMemStore::register_append (kvmem_store.cpp:179-205). */
KVMEM_HIP_API int kvmem_store_register_append(kvmem_store *s, uint32_t n_tokens);
/* KvMemRuntime::truncate_to (kvmem_runtime.cpp:75-92): frees pool slots. */
KVMEM_HIP_API int kvmem_store_truncate_to(kvmem_store *s, uint32_t token_pos);
KVMEM_HIP_API uint32_t kvmem_store_block_count(const kvmem_store *s);
KVMEM_HIP_API uint32_t kvmem_store_total_tokens(const kvmem_store *s);
/* KvMemStore::set_retrieval_scores (kvmem_store.cpp:242-248). */
KVMEM_HIP_API int kvmem_store_set_scores(kvmem_store *s, const double *scores, uint32_t n);
/* KvMemStore::pick_topk_blocks(mandatory) (kvmem_store.cpp:482-623):
 * ascending ids into out (capacity block count). */
KVMEM_HIP_API int kvmem_store_pick_topk(kvmem_store *s, const uint32_t *mandatory,
                                        uint32_t n_mandatory, uint32_t *out, uint32_t *n_out);
/* prepare_selection + finish_reselect (kvmem_runtime.cpp:108-113,
 * 223-236): the diff, then slots freed for stage-out and allocated for
 * stage-in.  stage_in / stage_out (capacity block count each) receive the
 * plan's lists. */
KVMEM_HIP_API int kvmem_store_apply(kvmem_store *s, const uint32_t *sel, uint32_t n_sel,
                                    uint32_t *stage_in, uint32_t *n_in, uint32_t *stage_out,
                                    uint32_t *n_out, kvmem_plan_stats *stats);
/* Per block: pool slot (-1 = none), tier (0 GPU, 1 CPU), in-working-set
 * flag, baked window position.  Arrays of block count entries. */
KVMEM_HIP_API int kvmem_store_blocks(const kvmem_store *s, int32_t *gpu_slot, uint8_t *tier,
                                     uint8_t *in_ws, int64_t *baked_pos);
/* KvMemStore::commit_resident_selection (kvmem_store.cpp:884-895):
 * 1 if committed, 0 if refused. */
KVMEM_HIP_API int kvmem_store_commit_resident(kvmem_store *s, const uint32_t *sel, uint32_t n);
/* The block ids the adapter's retrieval_mandatory derives from row ranges
 * (llama-memory-kvmem.cpp:3026-3045): in block order every block
 * overlapping one of the n_ranges ranges, then the block holding force_pos
 * (KvMemStore::block_id_containing, kvmem_store.cpp:158-176; -1 = none).
 * out holds `capacity` ids; *n_out receives the count (ERR_INVALID when it
 * exceeds capacity, or for a range with begin < 0 or end < begin). */
KVMEM_HIP_API int kvmem_store_blocks_overlapping(const kvmem_store *s, const kvmem_row_range *ranges,
                                                 uint32_t n_ranges, int32_t force_pos,
                                                 uint32_t *out, uint32_t capacity, uint32_t *n_out);

/* Continuation checks of the two-phase API over the store alone, where a
 * block holding a slot counts as complete (no device).  The store's
 * attention epoch moves with every apply that changes the working set and
 * every truncate that cuts rows; kvmem_store_register_append and
 * kvmem_store_append_resident leave it.  These restate the adapter's
 * attention_view / selection_fits / commit_unchanged / can_append
 * (llama-memory-kvmem.cpp:2982-3024, 3069-3096), which the engine calls
 * below exports with the pool's own state. */
KVMEM_HIP_API uint64_t kvmem_store_epoch(const kvmem_store *s);
/* Rows that enter the pool as they are written (llama.cpp's decode writing
 * K/V cells): register_append, and every block the rows touch that has no
 * slot takes one from the LIFO free list (prepare_working_set with the
 * working set pinned, llama-memory-kvmem.cpp:1256-1337).  ERR_NOMEM (no
 * change) when the free list is short. */
KVMEM_HIP_API int kvmem_store_append_resident(kvmem_store *s, uint32_t n_tokens);
KVMEM_HIP_API int kvmem_store_attention_view(const kvmem_store *s, int canonical,
                                             kvmem_attention_view *view);
/* 1 when the selection (epoch, rows, ids) is current, keeps every listed
 * mandatory id, and the rows up to end plus generation_rows fit the slot
 * pool beside it; else 0 (llama_kvmem_selection_fits, llama-kvmem-hooks.h:
 * 158; llama-memory-kvmem.cpp:3069-3084). */
KVMEM_HIP_API int kvmem_store_selection_fits(const kvmem_store *s, const uint32_t *mandatory,
                                             uint32_t n_mandatory, uint64_t epoch, uint32_t rows,
                                             const uint32_t *sel, uint32_t n_sel, uint32_t end,
                                             uint32_t generation_rows);
/* 1 and the selection committed as the working set when the view taken
 * before is still current, the canonical view now equals the selection and
 * keeps every block of the view before; else 0, nothing changed
 * (llama_kvmem_commit_unchanged, llama-kvmem-hooks.h:159;
 * llama-memory-kvmem.cpp:3086-3096). */
KVMEM_HIP_API int kvmem_store_commit_unchanged(kvmem_store *s, const kvmem_attention_view *before,
                                               uint64_t epoch, uint32_t rows, const uint32_t *sel,
                                               uint32_t n_sel);
/* 1 when rows up to end plus generation_rows can be decoded onto the pool
 * as it is; *reason (static string) gets the adapter's reason: "same_query"
 * / "all_resident" or "invalid_boundary", "coverage_or_layout",
 * "partial_tail_missing", "history_not_resident", "selection_budget",
 * "prefill_pressure", "insufficient_slots" (llama_kvmem_can_append,
 * llama-kvmem-hooks.h:156; llama-memory-kvmem.cpp:3002-3024). */
KVMEM_HIP_API int kvmem_store_can_append(const kvmem_store *s, uint32_t end, uint32_t generation_rows,
                                         int all_history, const char **reason);
/* 1 when replaying the query rows [query_begin, prompt_end) fits the
 * selection budget beside the sink blocks (the blocks from query_begin's on
 * plus the sink; 1 with no budget or an empty range) -- the adapter's
 * query_replay_fits (llama_kvmem_query_replay_fits, llama-kvmem-hooks.h:103;
 * llama-memory-kvmem.cpp:3502-3524). */
KVMEM_HIP_API int kvmem_store_query_replay_fits(const kvmem_store *s, uint32_t query_begin,
                                                uint32_t prompt_end);
/* KvMemStore::prefill_needs_offload (kvmem_store.cpp:340-351): 1 when
 * incoming_tokens more rows over resident_tokens overflow pool_tokens or
 * its high watermark (0.95 of it, at least one block), the test can_append
 * makes for a whole resident history. */
KVMEM_HIP_API int kvmem_store_prefill_needs_offload(const kvmem_store *s, uint32_t resident_tokens,
                                                    uint32_t incoming_tokens, uint32_t pool_tokens);
/* Slots the LIFO free list still holds (llama_kvmem_free_slots,
 * llama-kvmem-hooks.h:85). */
KVMEM_HIP_API uint32_t kvmem_store_free_slots(const kvmem_store *s);

/* ------------------------------------------------------ reselect engine */

typedef struct kvmem_engine kvmem_engine;

typedef struct kvmem_engine_params {
    int32_t device;            /* HIP ordinal */
    uint32_t n_layers;         /* attention layers */
    uint32_t block_tokens;     /* --kvmem-block-tokens (<= 128) */
    uint32_t n_head;           /* query heads */
    uint32_t n_head_kv;        /* KV heads */
    uint32_t head_dim;         /* 128 or 256 */
    uint32_t n_embd_v;         /* V row elements (0 = n_head_kv*head_dim) */
    uint32_t budget_blocks;    /* --kvmem-budget / block_tokens */
    uint32_t reserve_blocks;   /* --kvmem-gen-reserve / block_tokens */
    uint32_t sink_blocks;      /* default 1 (llama-memory-kvmem.cpp:295-297) */
    uint32_t recent_blocks;    /* default 0 */
    int32_t type_k;            /* KVMEM_TYPE_Q8_0 / Q5_0 / Q4_0 / F16 (-ctk) */
    int32_t type_v;            /* (-ctv) */
    int32_t tie_lower_index;   /* 1: equal scores -> lower id first */
    int32_t layer_reduce;      /* kvmem_hip_layer_reduce */
    int32_t canonical_layout;  /* 1 (default): selected block i (ascending)
                                  lives in slot i after every apply, as
                                  apply_selection lays the window out with
                                  layout_gpu_slots_by_orig_pos
                                  (llama-memory-kvmem.cpp:3209, 931-1254);
                                  0: blocks keep the slot the LIFO free list
                                  gave them (resident blocks never move) */
    int32_t scorer;            /* kvmem_engine_scorer used by preview */
    /* Cache row transform of the stage-in (kvmem_hip_transform), for a
     * history of pre-RoPE keys and a cache that holds RoPE'd, rotated rows: */
    uint32_t n_rot;            /* K rotary dims, RoPE at each block's original
                                  positions (0 = keys stored as given) */
    float rope_freq_base;      /* theta_i = powf(base, -2i/n_rot) * scale, */
    float rope_freq_scale;     /*   as kvmem/src/host/rope.cpp:20-23 */
    int32_t attn_rot;          /* 1: the reference's attn_rot rule
                                  (kvmem_attn_rot_on, llama-kvmem-quant.h:
                                  22-38): a quantized K (V) cache gets the
                                  Walsh-Hadamard rotation of width
                                  kvmem_hadamard_nrot_k(head_dim) (64) */
    uint32_t query_max_tokens; /* query window: rows kept per layer, the newest
                                  (--kvmem-query-max-tokens, default 512,
                                  tools/llama-kvmem-server.cpp:226, 1089-1096) */
    uint32_t query_last;       /* with no request / turn span: rows the
                                  preview takes, the newest captured
                                  (--kvmem-query-last, default 64,
                                  tools/llama-kvmem-server.cpp:225, 1032-1038) */
    int32_t device_plan;       /* 1 (default): apply_retrieval diffs the
                                  selection and plans the slot moves on the
                                  device, behind the top-k, so scoring,
                                  top-k, the plan, the slot saves and the
                                  chain walk run back to back with no host
                                  round trip; the host meanwhile takes the
                                  selection, commits the same plan to its
                                  store and queues the stage-in behind the
                                  walk (canonical layout, device-resident
                                  history, no packed store, budget <= 1024
                                  blocks, pool <= 4096 slots, 16-byte rows;
                                  a row transform is carried).  0, or
                                  outside those bounds: the host plans, as
                                  apply */
} kvmem_engine_params;

/* Block scorer of kvmem_engine_preview / apply_retrieval. */
enum kvmem_engine_scorer {
    KVMEM_SCORER_TOKEN_MAX = 0, /* per-token max of q.k / sqrt(head_dim) on MFMA */
    KVMEM_SCORER_MEAN_K = 1     /* the reference's mean-K cosine (score_retrieval,
                                   llama-memory-kvmem.cpp:2869-2916) over the
                                   sum of the query rows */
};

/* Defaults: 16 layers, 128-token blocks, 24/4 heads x 256, budget 256 +
 * reserve 128 blocks, sink 1, recent 0, q8_0 K and V, lower-id ties, mean
 * layer reduce, canonical layout (slot i = i-th selected block), per-token
 * max scorer, no row transform (RoPE base 10000, scale 1 when n_rot is
 * set). */
KVMEM_HIP_API kvmem_engine_params kvmem_engine_default_params(void);

/* Create the engine: its kvmem_hip_ctx, the slot pool of
 * (budget + reserve) slots per layer for K and V (kv_size = budget +
 * gen_reserve blocks, llama-memory-kvmem.cpp:363-426), cleared to zero as
 * llama.cpp clears its KV cache buffers, and the store. */
KVMEM_HIP_API int kvmem_engine_create(const kvmem_engine_params *p, kvmem_engine **out);
KVMEM_HIP_API void kvmem_engine_destroy(kvmem_engine *e);
KVMEM_HIP_API const char *kvmem_engine_last_error(const kvmem_engine *e);
/* The device context (stream, perf counters) the engine runs on. */
KVMEM_HIP_API kvmem_hip_ctx *kvmem_engine_ctx(kvmem_engine *e);

/* Device-resident F16 history: K and V [n_layers][capacity_blocks]
 * [block_tokens][n_embd] (K doubles as the scorer's key mirror).  The
 * store's block table is brought to n_tokens tokens (register_append /
 * truncate_to); capacity_blocks bounds later appends.  Bumps the epoch. */
KVMEM_HIP_API int kvmem_engine_set_device_history(kvmem_engine *e, const void *k, const void *v,
                                                  uint32_t capacity_blocks, uint32_t n_tokens);
/* Pinned host history, block-major (see kvmem_hip_host_history): when
 * set, stage-in reads changed blocks from it over PCIe instead of from the
 * device history.  It may also be the only history, as the reference keeps
 * every block in host RAM (RawKvStore): then append_tokens registers its
 * blocks, and preview runs the mean-K scorer (scorer = KVMEM_SCORER_MEAN_K;
 * the per-token scorer needs keys in HBM) on key sums the device reads from
 * the pinned blocks once per block (kvmem_hip_meank_sums_host).  NULL
 * clears it. */
KVMEM_HIP_API int kvmem_engine_set_host_history(kvmem_engine *e, const void *pinned_base,
                                                uint32_t capacity_blocks);
/* Packed host store (see kvmem_hip_packed_host), pinned, capacity_blocks
 * block spans in the pool's row formats, as the reference keeps packed GPU
 * rows per block (RawKvStore k_gpu / v_gpu).  When set:
 *   - apply copies every evicted full block whose packed rows the store
 *     does not hold yet to it (apply_plan_to_kv's stage-out of missing
 *     packed rows, llama-memory-kvmem.cpp:784-830);
 *   - with pinned host history, a selected block the store holds is
 *     restored from its packed rows (half the PCIe bytes of F16 at q8_0)
 *     instead of being quantized again (write_block_to_gpu,
 *     :2726-2791).  With device history the quantizing stage-in from HBM
 *     stays faster and is kept.
 * A block's packed rows are dropped when its history changes (truncate,
 * new history).  NULL clears the store. */
KVMEM_HIP_API int kvmem_engine_set_packed_host(kvmem_engine *e, void *pinned_base,
                                               uint32_t capacity_blocks);
/* 1 if the packed host store holds block_id's rows. */
KVMEM_HIP_API int kvmem_engine_packed_valid(const kvmem_engine *e, uint32_t block_id);
/* The history grew (caller wrote the new tokens): register_append.
 * Bumps the epoch. */
KVMEM_HIP_API int kvmem_engine_append_tokens(kvmem_engine *e, uint32_t n_new_tokens);
/* Rewind to token_pos tokens (truncate_to); frees their pool slots. */
KVMEM_HIP_API int kvmem_engine_truncate_to(kvmem_engine *e, uint32_t token_pos);

KVMEM_HIP_API uint32_t kvmem_engine_block_count(const kvmem_engine *e);
KVMEM_HIP_API uint32_t kvmem_engine_total_tokens(const kvmem_engine *e);
KVMEM_HIP_API uint64_t kvmem_engine_epoch(const kvmem_engine *e);
/* Borrow caller-owned pool tensors instead of the engine's own (the
 * llama.cpp K/V cache tensors, whose data pointers the reference adapter
 * takes with kvmem_cuda_tensor_ptr, llama-memory-kvmem.cpp:196-205):
 * k_layers / v_layers are host arrays of n_layers device pointers, each to
 * at least n_slots * block_tokens rows of the pool type, 16-byte aligned.
 * The engine's own pool is released.  The caller keeps the tensors alive
 * while the engine uses them; the working set is cleared (every block is
 * staged again by the next apply).  NULL k_layers returns to an engine-owned
 * pool, cleared to zero. */
KVMEM_HIP_API int kvmem_engine_set_pool(kvmem_engine *e, void *const *k_layers,
                                        void *const *v_layers);
/* Pool slots and per-layer device pool tensors. */
KVMEM_HIP_API uint32_t kvmem_engine_n_slots(const kvmem_engine *e);
KVMEM_HIP_API int kvmem_engine_pool_layer(const kvmem_engine *e, uint32_t layer, void **k,
                                          void **v);
/* Slot of every block (-1 = not in the pool), block count entries. */
KVMEM_HIP_API int kvmem_engine_block_slots(const kvmem_engine *e, int32_t *slots);

/* Request span (llama_kvmem_set_request_span, llama-kvmem-hooks.h:112):
 * the query rows [query_begin, query_end) (query_end <= 0: to the end of
 * the history; query_begin < 0: no span) and force_pos, a row whose block
 * every selection keeps (-1 = none).  Drops explicit turn spans. */
KVMEM_HIP_API int kvmem_engine_set_request_span(kvmem_engine *e, int32_t query_begin,
                                                int32_t query_end, int32_t force_pos);
/* Explicit turn spans (llama_kvmem_set_turn_spans, llama-kvmem-hooks.h:
 * 133-137, 154): query ranges and mandatory ranges replace the request
 * span; ERR_INVALID for a range with begin < 0 or end < begin (the
 * reference throws std::invalid_argument, llama-memory-kvmem.cpp:2936-2944). */
KVMEM_HIP_API int kvmem_engine_set_turn_spans(kvmem_engine *e, const kvmem_row_range *query,
                                              uint32_t n_query, const kvmem_row_range *mandatory,
                                              uint32_t n_mandatory);
/* The blocks every preview keeps (retrieval_mandatory,
 * llama-memory-kvmem.cpp:3026-3045): with turn spans, the blocks
 * overlapping their mandatory ranges; else those overlapping the request
 * span's query rows; then the block holding force_pos.  Block order; out
 * holds `capacity` ids. */
KVMEM_HIP_API int kvmem_engine_retrieval_mandatory(const kvmem_engine *e, uint32_t *out,
                                                   uint32_t capacity, uint32_t *n_out);

/* Query capture (the reference's Q harvest, harvest_capture('q') /
 * harvest_from_host('q'), llama-memory-kvmem.cpp:2157-2172, 2206-2219):
 * the rows of the strided device view q (pre-RoPE, post-q_norm Qcur of
 * `layer`: element (d, h, t) at d*nb0 + h*nb1 + t*nb2 bytes, F32 / F16 /
 * BF16; n_head x head_dim per token) whose position positions[t] (host) is
 * a query row (query_contains, llama-memory-kvmem.cpp:2950-2955; every row
 * when no span is set) are widened to f32 into the engine's query window,
 * a ring of the newest query_max_tokens rows per layer in HBM.  Enqueued on
 * the engine stream: q stays valid until the next preview / apply returns
 * or kvmem_hip_sync(kvmem_engine_ctx(e)) does.  Layers are captured
 * independently but must end up with the same number of rows. */
KVMEM_HIP_API int kvmem_engine_capture_q(kvmem_engine *e, uint32_t layer, const void *q,
                                         int32_t q_type, size_t nb0, size_t nb1, size_t nb2,
                                         uint32_t n_tokens, const int32_t *positions);
/* Empty the query window and drop a state set by kvmem_engine_set_query
 * (llama_kvmem_reset_query, llama-kvmem-hooks.h:71; reset_query_acc,
 * llama-memory-kvmem.cpp:2059-2064); a frozen query stays frozen. */
KVMEM_HIP_API int kvmem_engine_reset_query(kvmem_engine *e);
/* Query rows a window preview would read: the newest query_max_tokens
 * captured rows, or the newest query_last with no span set. */
KVMEM_HIP_API int kvmem_engine_query_rows(kvmem_engine *e, uint32_t *n_rows);

/* Phase 1 (preview_retrieval): score every block over q (device
 * [n_layers][n_q_tokens][n_head][head_dim], bf16 or f16) with the engine's
 * scorer -- the per-token max, or mean-K cosine over the sum of the
 * n_q_tokens rows (q_count_ = n_q_tokens in every layer) -- then top-k
 * with sink / mandatory / recent charged first: mandatory is the caller's
 * host ids (newest last) followed by kvmem_engine_retrieval_mandatory's.
 * q = NULL scores the captured query window instead (kvmem_engine_capture_q,
 * n_q_tokens and q_type ignored): its rows in token order, as bf16 for the
 * per-token scorer and summed in f32 for mean-K (q_count_ = the rows).
 * Writes the ascending selection (capacity block count), its epoch and rows
 * (history tokens). */
KVMEM_HIP_API int kvmem_engine_preview(kvmem_engine *e, const void *q, int32_t q_type,
                                       uint32_t n_q_tokens, const uint32_t *mandatory,
                                       uint32_t n_mandatory, uint32_t *sel, uint32_t *n_sel,
                                       uint64_t *epoch, uint32_t *rows);
/* Phase 2 (apply_selection): reject a stale selection, diff it against the
 * working set, free and allocate slots, quantize every incoming block into
 * its slot (one launch for K and V, from device or pinned host history),
 * and in canonical mode move resident blocks to their window slots.
 * Synchronises the engine stream. */
KVMEM_HIP_API int kvmem_engine_apply(kvmem_engine *e, uint64_t epoch, uint32_t rows,
                                     const uint32_t *sel, uint32_t n_sel,
                                     kvmem_plan_stats *stats);
/* Phase 1 with the reference's own scorer, mean-K cosine
 * (score_retrieval, llama-memory-kvmem.cpp:2869-2916): q_sum is device
 * [n_layers][n_head*head_dim] f32 (the per-layer sum of query rows the
 * reference keeps in q_sum_), q_count host [n_layers] (q_count_).  The
 * per-block key sums are produced on the device from the history and kept
 * current across appends.  Same outputs as kvmem_engine_preview. */
KVMEM_HIP_API int kvmem_engine_preview_meank(kvmem_engine *e, const float *q_sum,
                                             const uint32_t *q_count, const uint32_t *mandatory,
                                             uint32_t n_mandatory, uint32_t *sel, uint32_t *n_sel,
                                             uint64_t *epoch, uint32_t *rows);
/* preview + apply (apply_retrieval, llama-memory-kvmem.cpp:3139-3142). */
KVMEM_HIP_API int kvmem_engine_apply_retrieval(kvmem_engine *e, const void *q, int32_t q_type,
                                               uint32_t n_q_tokens, const uint32_t *mandatory,
                                               uint32_t n_mandatory, kvmem_plan_stats *stats);
/* ------------------------------------------- continuation (two-phase API)
 * The calls a caller makes between preview and apply to skip or check an
 * apply (llama-kvmem-hooks.h:155-161; the multimodal server's cached-query
 * and unchanged-selection paths, tools/kvmem-multimodal-server.h:309-389).
 * Selections are checked against the engine's epoch and rows as apply
 * checks them; views against the attention epoch. */

/* Rows the caller's decode writes into the pool itself, as llama.cpp writes
 * a batch's K/V cells (the adapter's prepare_working_set with the working
 * set pinned, llama-memory-kvmem.cpp:1256-1337): the history grows by
 * n_new_tokens (the caller writes them there too), and every block they
 * touch that holds no slot takes the next one of the free list --
 * kvmem_engine_block_slots tells where; row t of block b goes to cell
 * slot*block_tokens + (t - b*block_tokens) of every layer's K and V pool
 * tensor, in the pool's row format.  In canonical layout the new blocks
 * continue the window's slot order.  A partial tail that held no slot gets
 * one but its older rows are not in the pool: the next apply stages it
 * again.  Moves the selection epoch, not the attention epoch.  ERR_NOMEM
 * (nothing changed) when the free list is short. */
KVMEM_HIP_API int kvmem_engine_append_resident(kvmem_engine *e, uint32_t n_new_tokens);
KVMEM_HIP_API uint64_t kvmem_engine_attention_epoch(const kvmem_engine *e);
/* llama_kvmem_get_attention_view (llama-kvmem-hooks.h:155;
 * llama-memory-kvmem.cpp:2982-3000): a block holding a slot is complete
 * unless it is a partial tail whose newer rows wait to be staged.  The
 * pool has no cells outside blocks, so the reference's check of extra live
 * cells has nothing to count here. */
KVMEM_HIP_API int kvmem_engine_attention_view(const kvmem_engine *e, int canonical,
                                              kvmem_attention_view *view);
/* llama_kvmem_selection_fits (llama-kvmem-hooks.h:158; llama-memory-kvmem.cpp:
 * 3069-3084): 1 when the selection is current (epoch, rows), end >= rows,
 * it keeps every block kvmem_engine_retrieval_mandatory names (a selector
 * that trimmed a mandatory range to its budget made a plan unfit for
 * continuation), and its blocks plus those rows [rows, end +
 * generation_rows) still need fit the slot pool; else 0. */
KVMEM_HIP_API int kvmem_engine_selection_fits(const kvmem_engine *e, uint64_t epoch, uint32_t rows,
                                              const uint32_t *sel, uint32_t n_sel, uint32_t end,
                                              uint32_t generation_rows);
/* llama_kvmem_commit_unchanged (llama-kvmem-hooks.h:159; llama-memory-kvmem.cpp:
 * 3086-3096): when the view taken before is valid and still current (same
 * attention epoch, no more rows than now), the selection is current, the
 * canonical view now is valid and equals it and keeps every block of the
 * view before, the selection becomes the working set with no device work
 * (commit_resident_selection) and 1 is returned; else 0 and nothing
 * changes.  A caller that gets 1 skips kvmem_engine_apply. */
KVMEM_HIP_API int kvmem_engine_commit_unchanged(kvmem_engine *e, const kvmem_attention_view *before,
                                                uint64_t epoch, uint32_t rows, const uint32_t *sel,
                                                uint32_t n_sel);
/* llama_kvmem_commit_resident (llama-kvmem-hooks.h:161; llama-memory-kvmem.cpp:
 * 3098-3102): commit the blocks now in the pool as the working set when the
 * view (canonical or not) is valid; 1 on success, 0 otherwise. */
KVMEM_HIP_API int kvmem_engine_commit_resident(kvmem_engine *e, int canonical);
/* llama_kvmem_can_append (llama-kvmem-hooks.h:156; llama-memory-kvmem.cpp:
 * 3002-3024): as kvmem_store_can_append, over the engine's pool. */
KVMEM_HIP_API int kvmem_engine_can_append(const kvmem_engine *e, uint32_t end, uint32_t generation_rows,
                                          int all_history, const char **reason);
/* As kvmem_store_query_replay_fits / kvmem_store_free_slots, over the
 * engine's store and pool (llama-kvmem-hooks.h:85, 103). */
KVMEM_HIP_API int kvmem_engine_query_replay_fits(const kvmem_engine *e, uint32_t query_begin,
                                                 uint32_t prompt_end);
KVMEM_HIP_API uint32_t kvmem_engine_free_slots(const kvmem_engine *e);

/* Query state (llama_kvmem_query_state {sum, count}, llama-kvmem-hooks.h:
 * 139-142, 162-164): per layer the sum of the query rows (n_head*head_dim
 * f32) and their count, the input of the reference's mean-K scorer.
 * get: host q_sum [n_layers][n_head*head_dim], q_count [n_layers] receive
 * the state a preview with q = NULL would use -- the rows of the query
 * window summed in token order, or the state set_query set (ERR_INVALID
 * with neither; llama-memory-kvmem.cpp:3104-3119).
 * set: the caller's state replaces the rows captured so far for previews
 * with q = NULL, and freezes the query (capture_q keeps no rows) until
 * freeze_query(0); rows captured after that add onto the state (sums in
 * token order, counts), as the reference's harvest adds onto q_sum_ and
 * q_count_ (llama-memory-kvmem.cpp:2164-2172, 3121-3137).  reset_query
 * drops the state.  Sums must be finite and the counts equal and nonzero
 * (ERR_INVALID, nothing changed).  The
 * per-token scorer reads the rows themselves, not their sum:
 * ERR_UNSUPPORTED on an engine with scorer = KVMEM_SCORER_TOKEN_MAX.
 * freeze: while frozen, capture_q keeps no rows (query_contains is false,
 * llama-memory-kvmem.cpp:2950-2951). */
KVMEM_HIP_API int kvmem_engine_get_query(kvmem_engine *e, float *q_sum, uint32_t *q_count);
KVMEM_HIP_API int kvmem_engine_set_query(kvmem_engine *e, const float *q_sum, const uint32_t *q_count);
KVMEM_HIP_API int kvmem_engine_freeze_query(kvmem_engine *e, int frozen);

/* Scores of the last preview (host copy, block count entries).  Every
 * preview scores every block, also when the budget takes them all, as the
 * reference's preview_retrieval scores before it selects
 * (llama-memory-kvmem.cpp:3047-3067). */
KVMEM_HIP_API int kvmem_engine_scores(kvmem_engine *e, float *out, uint32_t n);

#ifdef __cplusplus
}
#endif
#endif
