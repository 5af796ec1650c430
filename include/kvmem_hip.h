/*
 * kvmem_hip.h -- C ABI of the MI355X (gfx950) KVMem reselect library.
 *
 * This is the device layer that replaces the reference's CUDA stage-in helper
 * (src/adapter/llama-kvmem-stagein.h:12-62, free functions over a global
 * singleton on cudaStreamPerThread) and the host scoring loop of the adapter
 * (src/adapter/llama-memory-kvmem.cpp:2869-2916).  Differences by design:
 *   - explicit context handle instead of the global `g_st` (stagein.cu:60-90);
 *   - explicit HIP stream (default: a stream owned by the context);
 *   - integer status codes (0 = ok) plus kvmem_hip_last_error() instead of
 *     `bool` + stderr (stagein.cu:92-98); no exception crosses this ABI.
 *
 * Pointer lifetimes: every `const void *` / `void *` that names device memory
 * is borrowed for the duration of the call and of the asynchronous work it
 * enqueues on the context stream; the caller keeps it alive until
 * kvmem_hip_sync() (or its own stream synchronisation) returns.  Host arrays
 * passed in (op lists, ids, slots, pointer tables) are copied before the call
 * returns and may be reused immediately.  Calls on one context are not
 * re-entrant: use one context per host thread.
 *
 * Numeric formats use ggml's type codes and block layouts:
 *   Q8_0 (8)  {f16 d; int8 qs[32]}             34 bytes / 32 elements
 *   Q5_0 (6)  {f16 d; u8 qh[4]; u8 qs[16]}     22 bytes / 32 elements
 *   Q4_0 (2)  {f16 d; u8 qs[16]}               18 bytes / 32 elements
 *   F16  (1)  raw half rows (copy)
 * Quantized bytes are bit-identical to ggml's quantize_row_*_ref applied to
 * the F16 rows converted to f32.
 */
#ifndef KVMEM_HIP_H
#define KVMEM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define KVMEM_HIP_API __attribute__((visibility("default")))
#else
#define KVMEM_HIP_API
#endif

/* ---------------------------------------------------------------- status */
enum kvmem_hip_status {
    KVMEM_HIP_OK = 0,
    KVMEM_HIP_ERR_INVALID = 1,    /* bad argument (shape, alignment, range) */
    KVMEM_HIP_ERR_RUNTIME = 2,    /* a HIP runtime call failed */
    KVMEM_HIP_ERR_NOMEM = 3,      /* device or pinned allocation failed */
    KVMEM_HIP_ERR_STALE = 4,      /* selection epoch/rows mismatch */
    KVMEM_HIP_ERR_UNSUPPORTED = 5, /* type / head_dim not built */
    KVMEM_HIP_ERR_BUSY = 6         /* a shared resource is in use by overlapping work */
};

/* ggml_type codes (ggml.h) for the formats on this path. */
enum kvmem_hip_type {
    KVMEM_TYPE_F32 = 0,
    KVMEM_TYPE_F16 = 1,
    KVMEM_TYPE_Q4_0 = 2,
    KVMEM_TYPE_Q5_0 = 6,
    KVMEM_TYPE_Q8_0 = 8,
    KVMEM_TYPE_BF16 = 30
};

/* Layer combination of per-layer block scores. */
enum kvmem_hip_layer_reduce {
    KVMEM_LAYER_MEAN = 0, /* layer averaging, llama-memory-kvmem.cpp:2910-2913 */
    KVMEM_LAYER_MAX = 1,
    KVMEM_LAYER_SUM = 2
};

typedef struct kvmem_hip_ctx kvmem_hip_ctx;

/* ------------------------------------------------------------- lifetime */

/* Create a context on `device` (HIP ordinal).  Replaces the lazy singleton
 * set-up of kvmem_stagein_gpu_ready (llama-kvmem-stagein.h:12,
 * stagein.cu:319-393).  Scratch grows on demand inside later calls. */
KVMEM_HIP_API int kvmem_hip_create(int device, kvmem_hip_ctx **out);

/* Release every device/pinned buffer the context owns.  Replaces
 * kvmem_stagein_gpu_free (llama-kvmem-stagein.h:13, stagein.cu:395-438). */
KVMEM_HIP_API void kvmem_hip_destroy(kvmem_hip_ctx *ctx);

/* Message of the last failing call on this context ("" if none).  Replaces
 * the stderr line of cuda_ok (stagein.cu:92-98). */
KVMEM_HIP_API const char *kvmem_hip_last_error(const kvmem_hip_ctx *ctx);

/* Use `stream` (a hipStream_t; NULL = the context's own stream) for all
 * later work.  The reference hard-wires cudaStreamPerThread
 * (stagein.cu:100-102). */
KVMEM_HIP_API int kvmem_hip_set_stream(kvmem_hip_ctx *ctx, void *stream);
KVMEM_HIP_API void *kvmem_hip_get_stream(const kvmem_hip_ctx *ctx);

/* Block the host until all work enqueued by this context has finished.
 * Replaces kvmem_stagein_sync (llama-kvmem-stagein.h:27, stagein.cu:615-617). */
KVMEM_HIP_API int kvmem_hip_sync(kvmem_hip_ctx *ctx);

/* Shapes a caller will use, so that later calls of at most these sizes run
 * without allocating device or pinned memory.  Zero fields reserve nothing
 * for their part. */
typedef struct kvmem_hip_reserve_args {
    uint32_t n_layers;         /* scored history layers */
    uint32_t n_blocks;         /* history blocks scored / selected over */
    uint32_t n_head;           /* query heads */
    uint32_t n_head_kv;        /* KV heads */
    uint32_t head_dim;         /* 128 or 256 */
    uint32_t n_q_tokens;       /* query tokens per layer (per-token scorer) */
    uint32_t max_items;        /* largest id / op list passed in one call */
    uint32_t pad0;
    uint64_t h2d_block_bytes;  /* one block over every layer in a host source:
                                  F16 K+V rows (stagein_blocks_host) or packed
                                  rows (stagein_packed_host); 0 = none */
    uint64_t d2h_block_bytes;  /* one block's packed rows over every layer
                                  (stageout_blocks); 0 = none */
    uint64_t move_bytes;       /* bytes one kvmem_hip_move_slots call gathers */
} kvmem_hip_reserve_args;

/* Grow every scratch buffer, ring and upload slot to fit `args`.  Replaces
 * the up-front sizing of kvmem_stagein_gpu_ready(n_f32, n_packed)
 * (llama-kvmem-stagein.h:12, stagein.cu:319-393); buffers only grow, and
 * growing waits for work still reading the old ones. */
KVMEM_HIP_API int kvmem_hip_reserve(kvmem_hip_ctx *ctx, const kvmem_hip_reserve_args *args);

/* Memory the context holds and the number of device/pinned allocations it
 * has made since creation (a call that allocated nothing leaves the count
 * unchanged).  No counterpart in the reference; the singleton's sizes
 * n_f32 / n_q (stagein.cu:60-90) are the nearest. */
typedef struct kvmem_hip_scratch {
    uint64_t device_bytes;
    uint64_t pinned_bytes;
    uint64_t allocations;
} kvmem_hip_scratch;
KVMEM_HIP_API int kvmem_hip_scratch_info(const kvmem_hip_ctx *ctx, kvmem_hip_scratch *out);

/* Enqueue a copy of `n` host bytes to device memory `dst` on the context
 * stream.  Replaces kvmem_stagein_h2d_bytes (llama-kvmem-stagein.h:26,
 * stagein.cu:607-613): n == 0 is a no-op that succeeds, and no fence is
 * taken, so the host buffer stays unchanged until kvmem_hip_sync returns
 * (pinned buffers are read asynchronously; the runtime stages pageable ones
 * before it returns).  Counted in the profiling copy stage and h2d_bytes. */
KVMEM_HIP_API int kvmem_hip_h2d_async(kvmem_hip_ctx *ctx, void *dst, const void *src, size_t n);

/* 1 if `type` can be produced by the stage-in kernels.  Replaces
 * kvmem_stagein_quant_ok (llama-kvmem-stagein.h:16; the reference accepts
 * only Q8_0 and Q4_0, stagein.cu:444-446). */
KVMEM_HIP_API int kvmem_hip_quant_ok(int type);

/* Bytes of a row of n elements of `type` (ggml_row_size), 0 if unsupported
 * or n % 32 != 0.  Used as at llama-memory-kvmem.cpp:2738-2739. */
KVMEM_HIP_API size_t kvmem_hip_row_size(int type, int64_t n);

/* ------------------------------------------------------------- stage-in */

/* One quantize-scatter operation: n_rows rows of n_embd F16 values at `src`
 * (row stride src_stride bytes, 0 = n_embd*2) become n_rows contiguous rows
 * of kvmem_hip_row_size(type, n_embd) bytes at `dst`.  src and dst must be
 * 16-byte aligned, src_stride a multiple of 16, n_embd a multiple of 32. */
typedef struct kvmem_hip_quant_op {
    const void *src;
    void *dst;
    uint32_t n_rows;
    uint32_t n_embd;
    int32_t type;
    uint32_t src_stride;
} kvmem_hip_quant_op;

/* Enqueue a batch of quantize-scatter operations (one kernel launch per
 * output type present).  Replaces the enqueue_k/enqueue_v + flush slab
 * sequence and kvmem_stagein_quantize (llama-kvmem-stagein.h:25,31-40;
 * stagein.cu:579-605, 632-753, 776-840), fused: F16 rows are read once from
 * HBM and written once in the pool's format. */
KVMEM_HIP_API int kvmem_hip_stagein_quant(kvmem_hip_ctx *ctx,
                                          const kvmem_hip_quant_op *ops,
                                          int n_ops);

/* Device-resident F16 block history: for each of K and V, the layer-major
 * array [n_layers][capacity_blocks][block_tokens][n_embd] of halves (one
 * 128-token block of one layer is contiguous, as RawKvStore keeps it per
 * (block, layer), raw_kv_store.hpp:98-117), of which blocks
 * [0, n_blocks) hold history.  v may be NULL (K only). */
typedef struct kvmem_hip_history {
    const void *k;
    const void *v;
    uint32_t n_layers;
    uint32_t n_blocks;
    uint32_t block_tokens;
    uint32_t n_embd_k;
    uint32_t n_embd_v;
    uint32_t last_block_tokens; /* tokens in block n_blocks-1 (0 = full) */
    uint32_t capacity_blocks;   /* blocks per layer in memory (0 = n_blocks) */
} kvmem_hip_history;

/* How the cache expects its rows: the transform the stage-in applies to the
 * F16 history rows before it quantizes them, in the order of the reference's
 * raw-K stage-in (kvmem_stagein_flush for K items, llama-kvmem-stagein.cu:
 * 704-740: widen -> NeoX RoPE -> Walsh-Hadamard -> quantize):
 *   RoPE (K only; rope_neox_kernel stagein.cu:159-178, kvmem/src/host/
 *   rope.cpp:8-45): in every head, for i < n_rot/2, with a = (float)p *
 *   theta[i] at the token's position p,
 *       x'[i]          = x[i]*cos(a) - x[i+n_rot/2]*sin(a)
 *       x'[i+n_rot/2]  = x[i]*sin(a) + x[i+n_rot/2]*cos(a)
 *   (separate IEEE products and sums; cos/sin of the fp32 angle are the
 *   library's own, within one rounding of the exact values); elements at
 *   n_rot and beyond are unchanged.
 *   attn_rot (llama-kvmem-quant.h:22-94; fwht_kernel stagein.cu:104-130):
 *   every run of `width` elements of a head becomes H x, H the orthonormal
 *   Walsh-Hadamard matrix: the run is first scaled by 1/sqrtf(width), then
 *   butterflies (a+b, a-b) of span 1, 2, 4, ... width/2.  The reference
 *   uses width = the largest power of two dividing head_dim (>= 64) for K
 *   (kvmem_hadamard_nrot_k) and 64 for V, on quantized caches.
 * Limits: head_dim 64, 128, 256 or 512 dividing n_embd; n_rot a multiple of
 * 16 up to head_dim; widths 64..512 dividing head_dim; a workgroup chunk of
 * 512 groups may span at most 4096 (row, rotary pair) entries, i.e.
 * (16384 / n_embd + 1) * n_rot / 2 <= 4096. */
typedef struct kvmem_hip_transform {
    uint32_t head_dim;
    uint32_t n_rot;           /* K rotary dims (0 = no RoPE) */
    const float *theta;       /* host [n_rot/2] pair frequencies (rope.cpp:
                                 freq_base^(-2i/n_rot) * freq_scale) */
    uint32_t hadamard_k;      /* K rotation width (0 = none) */
    uint32_t hadamard_v;      /* V rotation width (0 = none) */
    const int32_t *pos0;      /* host, one per staged block of a call: the
                                 position of its token 0 (NULL = block_id *
                                 block_tokens, the block's original start) */
} kvmem_hip_transform;

/* Slot pool: per layer one K and one V tensor of n_slots*block_tokens rows
 * of kvmem_hip_row_size(type, n_embd) bytes (the cache tensors of
 * llama-memory-kvmem.cpp:2736-2742; cell = slot*block_tokens + t,
 * llama-kvmem-batch.cpp:48).  k_layers/v_layers are host arrays of device
 * pointers, 16-byte aligned.  v_layers may be NULL.  xf (may be NULL: rows
 * stored as given) is applied by the block stage-in calls. */
typedef struct kvmem_hip_pool {
    uint32_t n_layers;
    uint32_t n_slots;
    uint32_t block_tokens;
    uint32_t n_embd_k;
    uint32_t n_embd_v;
    int32_t type_k;
    int32_t type_v;
    void *const *k_layers;
    void *const *v_layers;
    const kvmem_hip_transform *xf;
} kvmem_hip_pool;

/* Quantize blocks block_ids[i] of a device-resident history into pool slot
 * slots[i], every layer, K and V.  The single-launch-per-kind replacement
 * of write_block_to_gpu's per-(block, layer) slab items
 * (llama-memory-kvmem.cpp:2726-2791). */
KVMEM_HIP_API int kvmem_hip_stagein_blocks(kvmem_hip_ctx *ctx,
                                           const kvmem_hip_history *hist,
                                           const kvmem_hip_pool *pool,
                                           const uint32_t *block_ids,
                                           const uint32_t *slots,
                                           uint32_t n);

/* Host-resident history, block-major: block b occupies one contiguous span
 * of n_layers*(block_tokens*(n_embd_k+n_embd_v)) halves laid out
 * [layer][K rows then V rows].  When all n_blocks spans lie inside one
 * pinned allocation (hipHostMalloc, torch pin_memory), the quantize kernel
 * reads them over the link itself: one launch, no device staging.  Other
 * host memory is copied with hipMemcpyAsync on a side stream into a device
 * ring and quantized on the context stream as each copy lands.  Replaces
 * the 32 MiB slab H2D of kvmem_stagein_flush (stagein.cu:632-753), which
 * event-synchronises every H2D. */
typedef struct kvmem_hip_host_history {
    const void *base;           /* pinned host memory */
    uint32_t n_layers;
    uint32_t n_blocks;
    uint32_t block_tokens;
    uint32_t n_embd_k;
    uint32_t n_embd_v;
    uint32_t last_block_tokens;
} kvmem_hip_host_history;

KVMEM_HIP_API int kvmem_hip_stagein_blocks_host(kvmem_hip_ctx *ctx,
                                                const kvmem_hip_host_history *hist,
                                                const kvmem_hip_pool *pool,
                                                const uint32_t *block_ids,
                                                const uint32_t *slots,
                                                uint32_t n);

/* Packed host rows: the pool's own row formats kept in pinned host memory
 * per block, as the reference's RawKvStore keeps packed GPU rows per (block,
 * layer) (k_gpu / v_gpu, kvmem/include/kvmem/raw_kv_store.hpp:98-117).
 * Block-major: block b occupies one span of
 *     n_layers * block_tokens * (row_k + row_v) bytes
 * laid out [layer][block_tokens rows of K][block_tokens rows of V], rows of
 * kvmem_hip_row_size(pool type, n_embd) bytes; a block of n_tokens rows
 * uses the first n_tokens rows of each run. */
typedef struct kvmem_hip_packed_host {
    void *base;                 /* pinned host memory */
    uint32_t n_layers;
    uint32_t n_blocks;          /* blocks the memory holds */
    uint32_t block_tokens;
} kvmem_hip_packed_host;

/* Stage-out: copy the packed rows of pool slot slots[i] (every layer, K and
 * V, n_tokens[i] rows) to block block_ids[i] of the packed host store.
 * A store inside one pinned allocation is written by one copy launch on the
 * context stream.  Otherwise the rows are gathered into a device ring in
 * the host layout by one copy launch per 128 MiB batch, then copied
 * device-to-host on the side stream, so a later call's gathers overlap
 * earlier copies.
 * Asynchronous: the host rows are complete after kvmem_hip_sync.  Replaces
 * kvmem_stageout_enqueue / submit / wait (llama-kvmem-stagein.h:40-47,
 * stagein.cu:842-963: gather kernel into a 32 MiB slab, D2H into two
 * pinned slabs) and the per-block harvest of packed rows
 * (llama-memory-kvmem.cpp:2317-2394). */
KVMEM_HIP_API int kvmem_hip_stageout_blocks(kvmem_hip_ctx *ctx, const kvmem_hip_pool *pool,
                                            const kvmem_hip_packed_host *dst,
                                            const uint32_t *block_ids, const uint32_t *slots,
                                            const uint32_t *n_tokens, uint32_t n);

/* Stage-in of packed rows, the reference's live path (write_block_to_gpu:
 * copy_k_gpu / copy_v_gpu into the slab, enqueue_v, flush,
 * llama-memory-kvmem.cpp:2726-2791): the rows go into slot slots[i] of
 * every layer (n_tokens[i] rows), no quantization.  A store inside one
 * pinned allocation is read by one copy launch; otherwise block spans go
 * host-to-device into the device ring on the side stream and one copy
 * launch per batch scatters them.  The pool transform (xf) does not apply: packed rows are
 * already in the cache's form. */
KVMEM_HIP_API int kvmem_hip_stagein_packed_host(kvmem_hip_ctx *ctx,
                                                const kvmem_hip_packed_host *src,
                                                const kvmem_hip_pool *pool,
                                                const uint32_t *block_ids, const uint32_t *slots,
                                                const uint32_t *n_tokens, uint32_t n);

/* Move slots inside the pool: the first n_tokens[i] rows of slot
 * src_slots[i] -> slot dst_slots[i] for every layer, K and V (quantized
 * bytes copied unchanged; the destination's rows past n_tokens[i] keep
 * their bytes).  n_tokens == NULL moves whole slots.  The result is as if
 * every source were read before any destination is written, whatever the
 * overlap.  When sources are distinct and destinations are distinct (a
 * canonical layout's moves) and the layer tensors and rows are 16-byte
 * aligned, chains and cycles of moves are walked in segments and the bytes
 * move once; other sets are gathered to device scratch and scattered,
 * destinations in list order.  Every layer tensor of the pool must be
 * non-null (KVMEM_HIP_ERR_INVALID otherwise, nothing issued).  Replaces the
 * gather/scatter D2D of layout_gpu_slots_by_orig_pos, which moves each
 * block's n_tokens rows (llama-memory-kvmem.cpp:1003-1093). */
KVMEM_HIP_API int kvmem_hip_move_slots(kvmem_hip_ctx *ctx,
                                       const kvmem_hip_pool *pool,
                                       const uint32_t *src_slots,
                                       const uint32_t *dst_slots,
                                       const uint32_t *n_tokens,
                                       uint32_t n);

/* Batched device-to-device byte copies in one launch.  Replaces
 * kvmem_d2d_batched (llama-kvmem-stagein.h:52-53, stagein.cu:965-998);
 * no 8192-op limit. */
KVMEM_HIP_API int kvmem_hip_d2d_batched(kvmem_hip_ctx *ctx,
                                        const void *const *src,
                                        void *const *dst,
                                        const size_t *nbytes,
                                        int n);

/* -------------------------------------------------------------- scoring */

/* Per-token max block scorer on the matrix cores:
 *   s[l][b] = max_{t<n_q_tokens, hq<n_head, j<n_tok(b)}
 *             (q[l][t][hq] . k[l][b][j][hq / (n_head/n_head_kv)]) / sqrt(head_dim)
 * with fp32 accumulation, and scores[b] = reduce_l s[l][b].
 *   q       : device [n_layers][n_q_tokens][n_head][head_dim], bf16 or f16
 *   hist->k : device history (see kvmem_hip_history), n_embd_k must equal
 *             n_head_kv*head_dim
 *   layer_scores (device [n_layers][n_blocks] f32, may be NULL), scores
 *   (device [n_blocks] f32).
 * The reference's scorer is mean-K cosine on the host
 * (llama-memory-kvmem.cpp:2869-2916, per-block std::vector per head); its
 * GQA head map (qh_i = h*g + gi, :2890-2892) is kept. */
typedef struct kvmem_hip_score_args {
    const void *q;
    int32_t q_type;             /* KVMEM_TYPE_BF16 or KVMEM_TYPE_F16 */
    uint32_t n_q_tokens;
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t head_dim;          /* 128 or 256 */
    int32_t layer_reduce;       /* kvmem_hip_layer_reduce */
    float *layer_scores;
    float *scores;
} kvmem_hip_score_args;

KVMEM_HIP_API int kvmem_hip_score(kvmem_hip_ctx *ctx,
                                  const kvmem_hip_history *hist,
                                  const kvmem_hip_score_args *args);

/* kvmem_hip_score that allocates nothing: no counterpart in the reference.
 * For callers that cannot allocate (tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and the same scores, bit for bit.
 * The scorer's partial maxima (and the per-layer scores when
 * args->layer_scores is NULL) live in a static device array of 8 MiB that
 * every GPU the library runs on holds until the process ends; a call
 * needing more returns KVMEM_HIP_ERR_INVALID before any work (the 256K
 * workload -- 16 layers x 2048 blocks, 4 KV heads, 64 query tokens x 24
 * heads -- needs 2.1 MiB).  Every call on one GPU shares that GPU's array
 * and overwrites it (nothing in it has to start at zero).  One context's
 * calls follow each other (kvmem_hip_set_stream waits for the old stream);
 * a call from another context while the last call on the array has not
 * finished returns KVMEM_HIP_ERR_BUSY with nothing issued (the caller
 * synchronises, or uses kvmem_hip_score).  The array's last
 * user is tracked on the host: two processes on one GPU each have their
 * own array.  A call on a stream under HIP graph capture issues only two
 * kernel launches (no allocation, copy, memset or synchronisation), so it
 * can be captured; the capturing context becomes the array's owner, but
 * the replays run outside the library's view: the caller orders them with
 * its own calls and keeps other contexts' calls on this GPU from
 * overlapping them (such calls are not refused).  Not timed by
 * kvmem_hip_perf_*. */
KVMEM_HIP_API int kvmem_hip_score_noalloc(kvmem_hip_ctx *ctx,
                                          const kvmem_hip_history *hist,
                                          const kvmem_hip_score_args *args);

/* Top-k block selection on device.  From scores[0..n) (device, finite),
 * keep every id in forced[] (host array, the sink / mandatory / recent
 * blocks already charged by the host), then the `need` best remaining ids
 * by score (equal scores: lower id first if tie_lower_index, else higher id
 * first as kvmem_store.cpp:602-609), and write the union in ascending id
 * order to sel_out (host array, capacity n_forced + need); *n_sel receives
 * its length.  Replaces the nth_element fill of pick_topk_ungrouped
 * (kvmem_store.cpp:594-622).  Returns once the selection is on the host:
 * the kernel writes it to the context's coherent pinned buffer and sets a
 * completion word there, on which the calling thread spins (work queued
 * earlier on the context stream, e.g. the scorer, completes first).
 * n <= 1048576 (more than 16384 blocks take a kernel that recomputes
 * the keys from the scores in every radix pass). */
KVMEM_HIP_API int kvmem_hip_topk(kvmem_hip_ctx *ctx,
                                 const float *scores, uint32_t n,
                                 const uint32_t *forced, uint32_t n_forced,
                                 uint32_t need, int tie_lower_index,
                                 uint32_t *sel_out, uint32_t *n_sel);

/* ---------------------------------------------- mean-K cosine (reference) */

/* Mean-K producer: for every listed block and every layer of a device
 * history, k_sum[l][b][e] = fp32 sum of the block's F16 keys in token order
 * and mean_tokens[l][b] = the tokens summed (RawKvStore::capture_mean_f16,
 * kvmem/src/host/raw_kv_store.cpp:184-202; bit-identical sums).  k_sum is
 * device [n_layers][capacity][n_embd_k] f32 (16-byte aligned), mean_tokens
 * device [n_layers][capacity] u32; n_embd_k a multiple of 8, <= 2048. */
KVMEM_HIP_API int kvmem_hip_meank_sums(kvmem_hip_ctx *ctx, const kvmem_hip_history *hist,
                                       const uint32_t *block_ids, uint32_t n,
                                       float *k_sum, uint32_t *mean_tokens);

/* The same producer over a pinned host history (kvmem_hip_host_history,
 * block-major), for a deployment that keeps the history on the host only,
 * as the reference's RawKvStore does (its key sums are made on the host,
 * raw_kv_store.cpp:674-694, 976-1043): the kernel reads the listed blocks'
 * K rows over the link itself.  The whole history must lie inside one
 * pinned allocation (KVMEM_HIP_ERR_UNSUPPORTED otherwise).  k_sum /
 * mean_tokens are [n_layers][capacity_blocks] (0 = hist->n_blocks) as
 * kvmem_hip_meank_sums writes them; the sums are bit-identical. */
KVMEM_HIP_API int kvmem_hip_meank_sums_host(kvmem_hip_ctx *ctx, const kvmem_hip_host_history *hist,
                                            const uint32_t *block_ids, uint32_t n,
                                            uint32_t capacity_blocks, float *k_sum,
                                            uint32_t *mean_tokens);

/* Query-sum producer (the reference's Q harvest into q_sum_,
 * src/adapter/llama-memory-kvmem.cpp:2164-2172 and :2206-2219): for every
 * layer and channel, q_sum[l][e] += q[l][t][e] over the listed tokens in
 * list order, fp32 additions as the reference (bit-identical).
 *   q       device [n_layers][n_tokens][n_embd_q], F32, F16 or BF16
 *   tokens  host list of token indices (the query span; NULL = every token
 *           in order), n_list entries
 *   reset   nonzero: start from 0 (q_sum_ cleared), else add onto q_sum
 *   q_sum   device [n_layers][n_embd_q] f32
 * The caller counts the rows (q_count_) itself. */
KVMEM_HIP_API int kvmem_hip_q_accumulate(kvmem_hip_ctx *ctx, const void *q, int32_t q_type,
                                         uint32_t n_layers, uint32_t n_tokens, uint32_t n_embd_q,
                                         const uint32_t *tokens, uint32_t n_list, int reset,
                                         float *q_sum);

/* Decode-time mean-K producer (the reference's running sum on the GPU,
 * kvmem_meank_zero / kvmem_meank_add, llama-kvmem-stagein.cu:1020-1063):
 * for e < n_embd, acc[e] (+)= K[t][e / head_dim][e % head_dim] over the
 * tokens t = tok0 .. tok0 + n_keep - 1 in token order (fp32 additions,
 * bit-identical to the reference's loop).  K is device memory of k_type
 * F32, F16 or BF16 addressed with byte strides nb0 (element), nb1 (head),
 * nb2 (token), as the ggml K view the reference reads.  acc is device
 * [n_embd] f32, e.g. a row of the key sums kvmem_hip_meank_sums writes;
 * count (device, may be NULL) is that row's token count, increased by
 * n_keep.  reset != 0 starts both from zero (kvmem_meank_zero). */
KVMEM_HIP_API int kvmem_hip_meank_add(kvmem_hip_ctx *ctx, const void *k, int32_t k_type,
                                      uint32_t n_embd, uint32_t head_dim, size_t nb0, size_t nb1,
                                      size_t nb2, uint32_t tok0, uint32_t n_keep, int reset,
                                      float *acc, uint32_t *count);

/* Per-token query window (the rows the per-token scorer reads; the
 * reference keeps only their sum, q_sum_, from the pre-RoPE post-q_norm
 * query rows of its query span, llama-memory-kvmem.cpp:2157-2172,
 * 2206-2219).  Write: for i < n, row rows[i] of `window` (device
 * [capacity][n_head*head_dim] f32, one layer) receives token tokens[i] of
 * the strided device view q (element (d, h, t) at d*nb0 + h*nb1 + t*nb2
 * bytes, as ggml lays Qcur out and the reference reads it,
 * bytes_to_f32_token_major :2066-2090), widened exactly to f32 from F32,
 * F16 or BF16.  Rows must be distinct within a call and below capacity
 * (KVMEM_HIP_ERR_INVALID, nothing issued, otherwise). */
KVMEM_HIP_API int kvmem_hip_q_window_write(kvmem_hip_ctx *ctx, const void *q, int32_t q_type,
                                           uint32_t n_head, uint32_t head_dim, size_t nb0, size_t nb1,
                                           size_t nb2, const uint32_t *tokens, const uint32_t *rows,
                                           uint32_t n, float *window, uint32_t capacity);
/* Gather: out[l][i][:] = window[l][rows[i]][:] for every layer (window
 * device [n_layers][capacity][n_embd_q] f32), converted to out_type (BF16
 * and F16 round to nearest even; F32 copies) -- the [n_layers][n][n_head]
 * [head_dim] query kvmem_hip_score reads. */
KVMEM_HIP_API int kvmem_hip_q_window_gather(kvmem_hip_ctx *ctx, const float *window, uint32_t n_layers,
                                            uint32_t capacity, uint32_t n_embd_q, const uint32_t *rows,
                                            uint32_t n, int32_t out_type, void *out);

/* The reference's retrieval scorer (llama_memory_kvmem::score_retrieval,
 * src/adapter/llama-memory-kvmem.cpp:2869-2916): per block the mean over
 * layers with query rows of the mean over KV heads of
 *   cos(sum_{gi<g} q_sum[h*g+gi] / (q_count*g), k_sum_h / mean_tokens)
 * (denominator sqrt|q|^2 * sqrt|k|^2 + 1e-6), layer and block sums in
 * double; blocks without keys in any layer score 0.
 *   q_sum       device [n_layers][n_head*head_dim] f32 (sums of query rows)
 *   q_count     host   [n_layers] rows summed (0 = layer not scored)
 *   k_sum, mean_tokens as produced by kvmem_hip_meank_sums
 *   scores      device [n_blocks] f32
 * At most 256 layers (KVMEM_HIP_ERR_UNSUPPORTED beyond). */
typedef struct kvmem_hip_meank_args {
    const float *q_sum;
    const uint32_t *q_count;
    const float *k_sum;
    const uint32_t *mean_tokens;
    uint32_t n_layers;
    uint32_t n_blocks;
    uint32_t capacity_blocks;   /* 0 = n_blocks */
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t head_dim;          /* 128 or 256 */
    float *scores;
} kvmem_hip_meank_args;

KVMEM_HIP_API int kvmem_hip_score_meank(kvmem_hip_ctx *ctx, const kvmem_hip_meank_args *args);

/* -------------------------------------------------------- self-check */

/* Check, on this device and over every float of their ranges, the two
 * shortcuts the quantizers use for ggml's scale divisions: a / 127 for
 * every non-negative float a (q8_0's d) and 1 / d for every normal |d| <=
 * 2^126 (the id of all three formats); each count is the number of inputs
 * where the shortcut differs from the IEEE quotient (0 expected).  Takes a
 * few hundred milliseconds; no counterpart in the reference. */
KVMEM_HIP_API int kvmem_hip_check_scale_arith(kvmem_hip_ctx *ctx, uint64_t *div127_mismatches,
                                              uint64_t *recip_mismatches);

/* ---------------------------------------------------- failure injection */

/* Kinds of operation kvmem_hip_debug_fail_after can fail. */
enum kvmem_hip_fail_kind {
    KVMEM_HIP_FAIL_ALLOC = 1,  /* a device or pinned allocation */
    KVMEM_HIP_FAIL_COPY = 2,   /* a host<->device copy (table uploads included) */
    KVMEM_HIP_FAIL_LAUNCH = 4  /* a kernel launch */
};

/* Make the nth_op-th later operation of a kind in `kinds` (a mask of
 * kvmem_hip_fail_kind) on this context fail before it is issued: the entry
 * point that reaches it returns an error and kvmem_hip_last_error names
 * it ("...: injected failure"); nothing is enqueued for that operation and
 * injection then switches off.  nth_op = 0 or kinds = 0 switches it off.
 * Host-side only, it never makes a kernel fault.  The reference's callers
 * recover from a failed device call by falling back to host writes
 * (llama-memory-kvmem.cpp:2752-2758, 993-998, 1094-1099); this is how such
 * recovery is tested here.  No counterpart in the reference. */
KVMEM_HIP_API int kvmem_hip_debug_fail_after(kvmem_hip_ctx *ctx, uint32_t kinds, uint64_t nth_op);
/* Operations still to pass before the injected failure (0 = not armed:
 * it fired, or was never set). */
KVMEM_HIP_API uint64_t kvmem_hip_debug_fail_left(const kvmem_hip_ctx *ctx);

/* ------------------------------------------------------------ profiling */

/* Per-stage GPU time (hipEvent pairs on the context stream), the device
 * analogue of the KVMEM_RETR_SUM buckets (llama-memory-kvmem.cpp:2918-2936):
 * score = scoring kernels, topk = selection kernel, set = stage-in kernels
 * (quantizing or packed), copy = kvmem_hip_h2d_async, layout = slot moves
 * and their slot saves, stage_out = packed rows gathered and copied to the
 * host (kvmem_hip_stageout_blocks), plan = the slot plan (the device plan
 * kernel of the engine's apply_retrieval, or the host time of the engine's
 * own diff and slot plan when it plans on the host).  Milliseconds summed
 * over calls since the last reset; counts are numbers of timed calls; a
 * call that fails is not timed.
 * after_score_ms: from the end of a call's scoring to the end of the last
 * stage-in before the next scoring (top-k, the slot plan, moves, stage-in
 * and the idle stream between them); n_after_score such spans.
 * h2d_bytes / d2h_bytes / d2d_bytes: the bytes of kvmem_hip_transfer_get.
 * meank_cos_ms: the mean-K scorer's cosine kernel alone (events attached to
 * its launch), the one kernel of that scorer that streams the key sums;
 * score_ms covers all of its kernels (query, cosine, combine) and the gaps
 * between them.  The per-token scorer is one kernel, timed in score_ms the
 * same way. */
typedef struct kvmem_hip_perf {
    double score_ms;
    double topk_ms;
    double set_ms;
    double copy_ms;
    double layout_ms;
    uint64_t n_score;
    uint64_t n_topk;
    uint64_t n_set;
    uint64_t n_copy;
    uint64_t n_layout;
    uint64_t h2d_bytes;
    uint64_t d2d_bytes;
    double after_score_ms;
    uint64_t n_after_score;
    double stage_out_ms;
    double plan_ms;
    uint64_t n_stage_out;
    uint64_t n_plan;
    uint64_t d2h_bytes;
    double meank_cos_ms;
    uint64_t n_meank_cos;
} kvmem_hip_perf;

/* Data this context moved, per direction: [0] host to device, [1] device
 * to host, [2] device to device -- llama_kvmem_transfer_stats
 * (src/adapter/llama-kvmem-hooks.h:127-132), whose copy call sites
 * kvmem_copy_async / kvmem_tensor_set / _get count the same way
 * (src/adapter/llama-kvmem-transfer.h:9-31).  A call is one copy launch or
 * one runtime copy: a stage-in kernel reading pinned host blocks over the
 * link is one host-to-device call of the F16 (or packed) bytes it reads; a
 * slot-move chain walk and its slot saves are one device-to-device call
 * each; a stage-out through the device ring is its gather launches (device
 * to device) and its runtime copies (device to host).  Quantizing kernels
 * reading a device-resident history are compute, not transfers, and launch
 * tables are not counted.  Always counted (perf_enable not needed); cleared
 * by kvmem_hip_perf_reset. */
typedef struct kvmem_hip_transfer_stats {
    uint64_t bytes[3];
    uint64_t calls[3];
} kvmem_hip_transfer_stats;

KVMEM_HIP_API int kvmem_hip_transfer_get(const kvmem_hip_ctx *ctx, kvmem_hip_transfer_stats *out);

KVMEM_HIP_API int kvmem_hip_perf_enable(kvmem_hip_ctx *ctx, int on);
/* Which stages perf_enable times (default all): a mask of
 * KVMEM_PERF_STAGE_* bits.  Each timed stage records two events on the
 * stream, and each event holds the stream idle for a few microseconds, so
 * timing fewer stages perturbs a call less.  after_score_ms needs SCORE and
 * SET. */
#define KVMEM_PERF_STAGE_SCORE 1u
#define KVMEM_PERF_STAGE_TOPK 2u
#define KVMEM_PERF_STAGE_SET 4u
#define KVMEM_PERF_STAGE_COPY 8u
#define KVMEM_PERF_STAGE_LAYOUT 16u
#define KVMEM_PERF_STAGE_STAGE_OUT 32u
#define KVMEM_PERF_STAGE_PLAN 64u
#define KVMEM_PERF_STAGE_MEANK_COS 128u
KVMEM_HIP_API int kvmem_hip_perf_stages(kvmem_hip_ctx *ctx, uint32_t mask);
KVMEM_HIP_API int kvmem_hip_perf_get(kvmem_hip_ctx *ctx, kvmem_hip_perf *out);
/* Zero every bucket, count and transfer counter; a stage a failed call
 * left open is dropped. */
KVMEM_HIP_API void kvmem_hip_perf_reset(kvmem_hip_ctx *ctx);

#ifdef __cplusplus
}
#endif
#endif
