// Reselect engine and host-store C ABI (include/kvmem_host.h).
//
// The engine owns a kvmem_hip_ctx, the K/V slot pool and the host store;
// one agent step is preview (device scorer + device top-k with the store's
// sink / mandatory / recent charge) then apply (store diff and slot plan,
// one stage-in launch for every incoming block, optional canonical slot
// layout).  It stands where llama_memory_kvmem::preview_retrieval /
// apply_selection stand in the reference (src/adapter/llama-memory-kvmem.cpp:
// 3047-3067, 3139-3263); the per-block write_block_to_gpu loop
// (:2726-2791) becomes a single batched device call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include "kvmem_host.h"
#include "device_reselect.h"
#include "kvmem_store.hpp"

using kvmem_amd::Block;
using kvmem_amd::KvMemRuntime;
using kvmem_amd::Plan;
using kvmem_amd::SlotPool;
using kvmem_amd::StoreConfig;
using kvmem_amd::Tier;

namespace {

// Slot pool that records the blocks admitted in one apply.
class RecordingSlots final : public kvmem_amd::KvMemBackend {
public:
    explicit RecordingSlots(uint32_t n) : pool_(n) {}
    int32_t alloc_gpu_slot() override { return pool_.alloc_gpu_slot(); }
    void free_gpu_slot(int32_t s) override { pool_.free_gpu_slot(s); }
    uint32_t free_slot_count() const override { return pool_.n_free(); }
    uint32_t n_slots() const { return pool_.n_slots(); }
    void block_staged_in(uint32_t id, int32_t slot) override {
        staged_ids.push_back(id);
        staged_slots.push_back(static_cast<uint32_t>(slot));
    }
    // Free list holding every slot except [0, n_used), lowest on top.
    void reset_after(uint32_t n_used) {
        pool_.reset();
        for (uint32_t i = 0; i < n_used; ++i) {
            (void) pool_.alloc_gpu_slot();
        }
    }
    uint32_t n_free() const { return pool_.n_free(); }
    std::vector<uint32_t> staged_ids;
    std::vector<uint32_t> staged_slots;

private:
    SlotPool pool_;
};

void fill_stats(const Plan &p, uint32_t n_staged, uint32_t n_moved, uint32_t n_saved,
                uint32_t n_restored, kvmem_plan_stats *st) {
    if (!st) {
        return;
    }
    st->n_saved = n_saved;
    st->n_restored = n_restored;
    st->n_stage_in = static_cast<uint32_t>(p.stage_in.size());
    st->n_stage_out = static_cast<uint32_t>(p.stage_out.size());
    st->n_staged = n_staged;
    st->n_moved = n_moved;
    st->selection_overlap_blocks = p.selection_overlap_blocks;
    st->gpu_reused_blocks = p.gpu_reused_blocks;
    st->retained_position_stable = p.retained_position_stable;
    st->retained_position_moved = p.retained_position_moved;
    st->total_window_tokens = p.total_window_tokens;
    st->device_planned = 0;
    st->n_skip = 0;
    for (const kvmem_amd::Remap &r : p.remaps) {
        st->n_skip += r.skip ? 1u : 0u;
    }
}

// admit_incoming gives a block no slot when the free list is empty
// (alloc_gpu_slot returns -1, kvmem_runtime.cpp:294-328): such a plan
// cannot be applied.
bool every_stage_in_has_slot(const KvMemRuntime &rt, const Plan &p) {
    for (uint32_t id : p.stage_in) {
        const Block &b = rt.store().blocks()[id];
        if (b.tier != Tier::GPU || b.gpu_slot < 0) {
            return false;
        }
    }
    return true;
}

// Row ranges from the ABI; false for a range with begin < 0 or end < begin
// (the reference's std::invalid_argument, llama-memory-kvmem.cpp:2938-2944).
bool copy_ranges(const kvmem_row_range *r, uint32_t n, std::vector<std::pair<int32_t, int32_t>> &out) {
    out.clear();
    for (uint32_t i = 0; i < n; ++i) {
        if (r[i].begin < 0 || r[i].end < r[i].begin) {
            return false;
        }
        out.emplace_back(r[i].begin, r[i].end);
    }
    return true;
}

// An attention view into the ABI struct: header fields always, the block
// ids when they fit the caller's capacity (ERR_INVALID otherwise).
int export_view(const kvmem_amd::AttentionView &v, kvmem_attention_view *out) {
    out->epoch = v.epoch;
    out->rows = v.rows;
    out->valid = v.valid ? 1 : 0;
    out->n_blocks = static_cast<uint32_t>(v.blocks.size());
    if (v.blocks.size() > out->capacity || (!v.blocks.empty() && !out->blocks)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::copy(v.blocks.begin(), v.blocks.end(), out->blocks);
    return KVMEM_HIP_OK;
}

// The ABI struct back into a view (its first n_blocks ids); false when the
// ids cannot be read.
bool import_view(const kvmem_attention_view *in, kvmem_amd::AttentionView &v) {
    if (!in || (in->n_blocks && !in->blocks) || in->n_blocks > in->capacity) {
        return false;
    }
    v.epoch = in->epoch;
    v.rows = in->rows;
    v.valid = in->valid != 0;
    v.blocks.assign(in->blocks, in->blocks + in->n_blocks);
    return true;
}

StoreConfig store_config(uint32_t block_tokens, uint32_t budget_blocks, uint32_t sink,
                         uint32_t recent, bool tie_lower) {
    StoreConfig c;
    c.block_tokens = block_tokens;
    c.select_budget = budget_blocks * block_tokens;
    c.sink_blocks = sink;
    c.recent_blocks = recent;
    c.tie_lower_index = tie_lower;
    return c;
}

}  // namespace

// ================================================================ store

struct kvmem_store {
    RecordingSlots slots;
    KvMemRuntime rt;
    // attention epoch: bumped by applies that change the working set and by
    // cuts, never by appended rows (the adapter's attention_epoch_)
    uint64_t epoch = 1;
    kvmem_store(const StoreConfig &c, uint32_t n_slots) : slots(n_slots), rt(c, &slots) {}
    // The store alone has no device: a block holding a slot is complete.
    kvmem_amd::PoolState pool_state() const {
        kvmem_amd::PoolState p;
        p.epoch = epoch;
        p.n_slots = slots.n_slots();
        p.n_free = slots.n_free();
        p.complete = [](const Block &b) { return b.tier == Tier::GPU; };
        return p;
    }
};

extern "C" {

int kvmem_store_create(uint32_t block_tokens, uint32_t budget_blocks, uint32_t sink_blocks,
                       uint32_t recent_blocks, int tie_lower_index, uint32_t n_slots,
                       kvmem_store **out) {
    if (!out || block_tokens == 0) {
        return KVMEM_HIP_ERR_INVALID;
    }
    *out = new (std::nothrow) kvmem_store(
        store_config(block_tokens, budget_blocks, sink_blocks, recent_blocks, tie_lower_index != 0),
        n_slots);
    return *out ? KVMEM_HIP_OK : KVMEM_HIP_ERR_NOMEM;
}

void kvmem_store_destroy(kvmem_store *s) {
    delete s;
}

int kvmem_store_register_append(kvmem_store *s, uint32_t n_tokens) {
    if (!s) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint32_t first_new = s->rt.store().block_count();
    s->rt.register_append(n_tokens);
    // new blocks live in the host history until a selection stages them in
    for (uint32_t id = first_new; id < s->rt.store().block_count(); ++id) {
        s->rt.store().set_block_tier(id, Tier::CPU);
    }
    return KVMEM_HIP_OK;
}

int kvmem_store_truncate_to(kvmem_store *s, uint32_t token_pos) {
    if (!s) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (token_pos < s->rt.store().total_tokens()) {
        ++s->epoch;
    }
    s->rt.truncate_to(token_pos);
    return KVMEM_HIP_OK;
}

int kvmem_store_append_resident(kvmem_store *s, uint32_t n_tokens) {
    if (!s) {
        return KVMEM_HIP_ERR_INVALID;
    }
    return s->rt.append_resident(n_tokens, nullptr) ? KVMEM_HIP_OK : KVMEM_HIP_ERR_NOMEM;
}

uint64_t kvmem_store_epoch(const kvmem_store *s) {
    return s ? s->epoch : 0;
}

int kvmem_store_attention_view(const kvmem_store *s, int canonical, kvmem_attention_view *view) {
    if (!s || !view) {
        return KVMEM_HIP_ERR_INVALID;
    }
    return export_view(kvmem_amd::attention_view(s->rt.store(), s->pool_state(), canonical != 0), view);
}

int kvmem_store_selection_fits(const kvmem_store *s, const uint32_t *mandatory, uint32_t n_mandatory,
                               uint64_t epoch, uint32_t rows, const uint32_t *sel, uint32_t n_sel,
                               uint32_t end, uint32_t generation_rows) {
    if (!s || (n_mandatory && !mandatory) || (n_sel && !sel)) {
        return 0;
    }
    return kvmem_amd::selection_fits(s->rt.store(), s->pool_state(),
                                     std::vector<uint32_t>(mandatory, mandatory + n_mandatory), epoch,
                                     rows, std::vector<uint32_t>(sel, sel + n_sel), end, generation_rows)
               ? 1
               : 0;
}

int kvmem_store_commit_unchanged(kvmem_store *s, const kvmem_attention_view *before, uint64_t epoch,
                                 uint32_t rows, const uint32_t *sel, uint32_t n_sel) {
    kvmem_amd::AttentionView v;
    if (!s || (n_sel && !sel) || !import_view(before, v)) {
        return 0;
    }
    return kvmem_amd::commit_unchanged(s->rt, s->pool_state(), v, epoch, rows,
                                       std::vector<uint32_t>(sel, sel + n_sel))
               ? 1
               : 0;
}

int kvmem_store_query_replay_fits(const kvmem_store *s, uint32_t query_begin, uint32_t prompt_end) {
    return !s || kvmem_amd::query_replay_fits(s->rt.store(), query_begin, prompt_end) ? 1 : 0;
}

int kvmem_store_prefill_needs_offload(const kvmem_store *s, uint32_t resident_tokens, uint32_t incoming_tokens,
                                      uint32_t pool_tokens) {
    return s && s->rt.store().prefill_needs_offload(resident_tokens, incoming_tokens, pool_tokens) ? 1 : 0;
}

uint32_t kvmem_store_free_slots(const kvmem_store *s) {
    return s ? s->slots.n_free() : 0u;
}

int kvmem_store_can_append(const kvmem_store *s, uint32_t end, uint32_t generation_rows, int all_history,
                           const char **reason) {
    if (!s) {
        if (reason) *reason = "invalid_boundary";
        return 0;
    }
    return kvmem_amd::can_append(s->rt.store(), s->pool_state(), end, generation_rows, all_history != 0,
                                 reason)
               ? 1
               : 0;
}

uint32_t kvmem_store_block_count(const kvmem_store *s) {
    return s ? s->rt.store().block_count() : 0;
}

uint32_t kvmem_store_total_tokens(const kvmem_store *s) {
    return s ? s->rt.store().total_tokens() : 0;
}

int kvmem_store_set_scores(kvmem_store *s, const double *scores, uint32_t n) {
    if (!s || (n && !scores)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    s->rt.store().set_retrieval_scores(std::vector<double>(scores, scores + n));
    return KVMEM_HIP_OK;
}

int kvmem_store_pick_topk(kvmem_store *s, const uint32_t *mandatory, uint32_t n_mandatory,
                          uint32_t *out, uint32_t *n_out) {
    if (!s || !out || !n_out || (n_mandatory && !mandatory)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const std::vector<uint32_t> sel =
        s->rt.preview_reselect(std::vector<uint32_t>(mandatory, mandatory + n_mandatory));
    std::copy(sel.begin(), sel.end(), out);
    *n_out = static_cast<uint32_t>(sel.size());
    return KVMEM_HIP_OK;
}

int kvmem_store_apply(kvmem_store *s, const uint32_t *sel, uint32_t n_sel, uint32_t *stage_in,
                      uint32_t *n_in, uint32_t *stage_out, uint32_t *n_out,
                      kvmem_plan_stats *stats) {
    if (!s || (n_sel && !sel)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    s->slots.staged_ids.clear();
    s->slots.staged_slots.clear();
    const KvMemRuntime rt_before = s->rt;
    const RecordingSlots slots_before = s->slots;
    const Plan p = s->rt.prepare_selection(std::vector<uint32_t>(sel, sel + n_sel));
    s->rt.finish_reselect();
    if (!every_stage_in_has_slot(s->rt, p)) {
        // the pool ran out of slots: nothing was applied
        s->rt = rt_before;
        s->slots = slots_before;
        return KVMEM_HIP_ERR_NOMEM;
    }
    if (!p.stage_in.empty() || !p.stage_out.empty()) {
        ++s->epoch;  // the working set changed (apply_plan_to_kv, llama-memory-kvmem.cpp:785)
    }
    if (stage_in) {
        std::copy(p.stage_in.begin(), p.stage_in.end(), stage_in);
    }
    if (stage_out) {
        std::copy(p.stage_out.begin(), p.stage_out.end(), stage_out);
    }
    if (n_in) {
        *n_in = static_cast<uint32_t>(p.stage_in.size());
    }
    if (n_out) {
        *n_out = static_cast<uint32_t>(p.stage_out.size());
    }
    fill_stats(p, static_cast<uint32_t>(s->slots.staged_ids.size()), 0, 0, 0, stats);
    return KVMEM_HIP_OK;
}

int kvmem_store_blocks(const kvmem_store *s, int32_t *gpu_slot, uint8_t *tier, uint8_t *in_ws,
                       int64_t *baked_pos) {
    if (!s) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const auto &bl = s->rt.store().blocks();
    for (size_t i = 0; i < bl.size(); ++i) {
        if (gpu_slot) gpu_slot[i] = bl[i].gpu_slot;
        if (tier) tier[i] = static_cast<uint8_t>(bl[i].tier);
        if (in_ws) in_ws[i] = bl[i].in_working_set ? 1 : 0;
        if (baked_pos) baked_pos[i] = bl[i].baked_pos;
    }
    return KVMEM_HIP_OK;
}

int kvmem_store_commit_resident(kvmem_store *s, const uint32_t *sel, uint32_t n) {
    if (!s || (n && !sel)) {
        return 0;
    }
    return s->rt.commit_resident_selection(std::vector<uint32_t>(sel, sel + n)) ? 1 : 0;
}

int kvmem_store_blocks_overlapping(const kvmem_store *s, const kvmem_row_range *ranges,
                                   uint32_t n_ranges, int32_t force_pos, uint32_t *out,
                                   uint32_t capacity, uint32_t *n_out) {
    std::vector<std::pair<int32_t, int32_t>> rr;
    if (!s || !n_out || (n_ranges && !ranges) || (capacity && !out) ||
        !copy_ranges(ranges, n_ranges, rr)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const std::vector<uint32_t> ids = s->rt.store().blocks_overlapping(rr, force_pos);
    *n_out = static_cast<uint32_t>(ids.size());
    if (ids.size() > capacity) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::copy(ids.begin(), ids.end(), out);
    return KVMEM_HIP_OK;
}

}  // extern "C"

// =============================================================== engine

struct kvmem_engine {
    kvmem_engine_params p{};
    uint32_t n_embd_k = 0;
    uint32_t n_embd_v = 0;
    uint32_t n_slots = 0;
    kvmem_hip_ctx *ctx = nullptr;
    RecordingSlots slots;
    KvMemRuntime rt;
    std::vector<void *> pool_k, pool_v;
    bool own_pool = true;
    const void *hist_k = nullptr;
    const void *hist_v = nullptr;
    uint32_t hist_capacity = 0;
    const void *host_base = nullptr;
    uint32_t host_capacity = 0;
    float *d_scores = nullptr;
    uint32_t d_scores_n = 0;
    int64_t dirty_tail = -1;   // resident partial block that grew since staged
    float *d_ksum = nullptr;   // mean-K sums [L][capacity][n_embd_k]
    uint32_t *d_mt = nullptr;  // mean-K token counts [L][capacity]
    uint32_t meank_cap = 0;    // capacity the sums are allocated for
    uint32_t meank_valid = 0;  // leading blocks whose sums are current
    float *d_qsum = nullptr;   // query sums [L][n_head*head_dim] (mean-K scorer)
    float *d_qwin = nullptr;   // query window [L][qwin_cap][n_head*head_dim] f32
    void *d_qgather = nullptr; // its rows in token order for the scorer, bf16
    uint32_t qwin_cap = 0;
    std::vector<uint64_t> qwin_count;  // rows captured per layer since the reset
    bool query_frozen = false;         // capture_q keeps no rows (freeze_query, set_query)
    bool query_imported = false;       // a state set by set_query is in use
    float *d_qimp = nullptr;           // its sums [L][n_head*head_dim]
    std::vector<uint32_t> imp_count;   // its row counts per layer
    uint64_t imp_base = 0;             // window rows captured before it was set
    void *packed_base = nullptr;        // pinned packed host store (may be null)
    uint32_t packed_capacity = 0;       // blocks it holds
    std::vector<uint8_t> packed_valid;  // block's packed rows are in the store
    kvmem_hip_transform xf{};  // cache row transform (unused when has_xf is false)
    std::vector<float> theta;  // RoPE pair frequencies
    bool has_xf = false;
    uint64_t epoch = 1;        // selection epoch: history rows or contents changed
    uint64_t attn_epoch = 1;   // attention epoch: pool contents or residency changed
    std::string err;
    // request span / turn spans (llama-memory-kvmem.h:164-170, .cpp:2938-2948)
    int32_t query_begin = -1;
    int32_t query_end = 0;
    int32_t force_pos = -1;
    bool explicit_spans = false;
    std::vector<std::pair<int32_t, int32_t>> span_query, span_mandatory;

    // retrieval_mandatory (llama-memory-kvmem.cpp:3026-3045)
    std::vector<uint32_t> retrieval_mandatory() const {
        std::vector<std::pair<int32_t, int32_t>> ranges;
        if (explicit_spans) {
            ranges = span_mandatory;
        } else if (query_begin >= 0) {
            ranges.emplace_back(query_begin, query_end > 0
                                                 ? query_end
                                                 : static_cast<int32_t>(rt.store().total_tokens()));
        }
        return rt.store().blocks_overlapping(ranges, force_pos);
    }
    bool spans_set() const { return explicit_spans || query_begin >= 0; }
    // query_contains (llama-memory-kvmem.cpp:2950-2955): a row of the query
    bool query_contains(int32_t row) const {
        if (!explicit_spans) {
            return query_begin >= 0 && row >= query_begin && (query_end <= 0 || row < query_end);
        }
        for (const auto &r : span_query) {
            if (row >= r.first && row < r.second) {
                return true;
            }
        }
        return false;
    }

    kvmem_engine(const kvmem_engine_params &pp, uint32_t n)
        : p(pp),
          n_slots(n),
          slots(n),
          rt(store_config(pp.block_tokens, pp.budget_blocks, pp.sink_blocks, pp.recent_blocks,
                          pp.tie_lower_index != 0),
             &slots) {}

    int fail(int code, const std::string &msg) {
        err = msg;
        return code;
    }
    int fail_ctx(int code, const char *what) {
        err = std::string(what) + ": " + kvmem_hip_last_error(ctx);
        return code;
    }

    // The pool as the continuation checks see it: a block holding a slot is
    // complete unless it is a partial tail whose newer rows are not staged.
    kvmem_amd::PoolState pool_state() const {
        kvmem_amd::PoolState ps;
        ps.epoch = attn_epoch;
        ps.n_slots = n_slots;
        ps.n_free = slots.n_free();
        const int64_t dirty = dirty_tail;
        ps.complete = [dirty](const Block &b) {
            return b.tier == Tier::GPU && static_cast<int64_t>(b.block_id) != dirty;
        };
        return ps;
    }

    kvmem_hip_pool pool_desc() const {
        kvmem_hip_pool d{};
        d.n_layers = p.n_layers;
        d.n_slots = n_slots;
        d.block_tokens = p.block_tokens;
        d.n_embd_k = n_embd_k;
        d.n_embd_v = n_embd_v;
        d.type_k = p.type_k;
        d.type_v = p.type_v;
        d.k_layers = pool_k.data();
        d.v_layers = pool_v.data();
        d.xf = has_xf ? &xf : nullptr;
        return d;
    }

    uint32_t last_block_tokens() const {
        const auto &bl = rt.store().blocks();
        if (bl.empty() || bl.back().n_tokens == p.block_tokens) {
            return 0;
        }
        return bl.back().n_tokens;
    }

    // Blocks the key-sum arrays are laid out for: the device history's
    // capacity, or the pinned host history's when there is no device one.
    uint32_t sums_capacity() const { return hist_k ? hist_capacity : host_capacity; }

    kvmem_hip_host_history host_history() const {
        kvmem_hip_host_history h{};
        h.base = host_base;
        h.n_layers = p.n_layers;
        h.n_blocks = rt.store().block_count();
        h.block_tokens = p.block_tokens;
        h.n_embd_k = n_embd_k;
        h.n_embd_v = n_embd_v;
        h.last_block_tokens = last_block_tokens();
        return h;
    }

    kvmem_hip_history device_history() const {
        kvmem_hip_history h{};
        h.k = hist_k;
        h.v = hist_v;
        h.n_layers = p.n_layers;
        h.n_blocks = rt.store().block_count();
        h.block_tokens = p.block_tokens;
        h.n_embd_k = n_embd_k;
        h.n_embd_v = n_embd_v;
        h.last_block_tokens = last_block_tokens();
        h.capacity_blocks = hist_capacity;
        return h;
    }
};

namespace {

kvmem_hip_packed_host packed_desc(const kvmem_engine *e) {
    kvmem_hip_packed_host ph{};
    ph.base = e->packed_base;
    ph.n_layers = e->p.n_layers;
    ph.n_blocks = e->packed_capacity;
    ph.block_tokens = e->p.block_tokens;
    return ph;
}

// Write blocks `ids` into pool slots `slots`: from the packed host store
// when the history is on the host and the store holds the block, else by
// quantizing the F16 history (device or pinned host).
int engine_stage(kvmem_engine *e, const std::vector<uint32_t> &ids,
                 const std::vector<uint32_t> &slots, uint32_t *n_restored) {
    *n_restored = 0;
    if (ids.empty()) {
        return KVMEM_HIP_OK;
    }
    const kvmem_hip_pool pool = e->pool_desc();
    std::vector<uint32_t> q_ids, q_slots;
    std::vector<uint32_t> p_ids, p_slots, p_nt;
    for (size_t i = 0; i < ids.size(); ++i) {
        const uint32_t id = ids[i];
        if (e->host_base && e->packed_base && id < e->packed_capacity && e->packed_valid[id]) {
            p_ids.push_back(id);
            p_slots.push_back(slots[i]);
            p_nt.push_back(e->p.block_tokens);  // only full blocks are kept
        } else {
            q_ids.push_back(id);
            q_slots.push_back(slots[i]);
        }
    }
    int rc = KVMEM_HIP_OK;
    if (!p_ids.empty()) {
        const kvmem_hip_packed_host ph = packed_desc(e);
        rc = kvmem_hip_stagein_packed_host(e->ctx, &ph, &pool, p_ids.data(), p_slots.data(), p_nt.data(),
                                           static_cast<uint32_t>(p_ids.size()));
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "packed stage-in");
        }
        *n_restored = static_cast<uint32_t>(p_ids.size());
    }
    if (q_ids.empty()) {
        return KVMEM_HIP_OK;
    }
    if (e->host_base) {
        const kvmem_hip_host_history h = e->host_history();
        rc = kvmem_hip_stagein_blocks_host(e->ctx, &h, &pool, q_ids.data(), q_slots.data(),
                                           static_cast<uint32_t>(q_ids.size()));
    } else {
        const kvmem_hip_history h = e->device_history();
        rc = kvmem_hip_stagein_blocks(e->ctx, &h, &pool, q_ids.data(), q_slots.data(),
                                      static_cast<uint32_t>(q_ids.size()));
    }
    return rc == KVMEM_HIP_OK ? rc : e->fail_ctx(rc, "stage-in");
}

}  // namespace

static bool alloc_own_pool(kvmem_engine *e);

namespace {

// No block is in the pool any more: every block goes back to the host tier,
// the working set is empty and every slot is free (the next apply stages
// its whole selection).
// Take one block out of the pool, its slot back to the free list: a
// selection that holds it stages it again.
void evict_block(kvmem_engine *e, uint32_t id) {
    if (id >= e->rt.store().block_count()) {
        return;
    }
    const Block &b = e->rt.store().blocks()[id];
    if (b.tier == Tier::GPU && b.gpu_slot >= 0) {
        e->slots.free_gpu_slot(b.gpu_slot);
    }
    e->rt.store().set_block_tier(id, Tier::CPU);
    e->rt.store().drop_from_working_set(id);
    if (e->dirty_tail == static_cast<int64_t>(id)) {
        e->dirty_tail = -1;
    }
    ++e->attn_epoch;
}

void drop_residency(kvmem_engine *e) {
    for (const Block &b : e->rt.store().blocks()) {
        if (b.tier == Tier::GPU) {
            e->rt.store().set_block_tier(b.block_id, Tier::CPU);
        }
    }
    e->rt.store().clear_working_set();
    e->slots.reset_after(0);
    e->dirty_tail = -1;
    ++e->attn_epoch;
}

// The stage-in row transform from the engine parameters: RoPE frequencies
// as rope.cpp:20-23 forms them, and the reference's attn_rot widths
// (llama-kvmem-quant.h:22-38): on a quantized cache, K gets the largest
// power of two dividing head_dim (at least 64), V gets 64.
bool setup_transform(kvmem_engine *e) {
    const kvmem_engine_params &p = e->p;
    const auto quantized = [](int t) { return t != KVMEM_TYPE_F16 && t != KVMEM_TYPE_F32; };
    const bool rot_ok = p.attn_rot && p.head_dim >= 64 && p.head_dim % 64 == 0;
    uint32_t had_k = 0;
    if (rot_ok && quantized(p.type_k)) {
        uint32_t n = 64;
        do {
            n *= 2;
        } while (p.head_dim % n == 0);
        had_k = n / 2;
    }
    const uint32_t had_v = rot_ok && quantized(p.type_v) ? 64u : 0u;
    if (p.n_rot == 0 && had_k == 0 && had_v == 0) {
        e->has_xf = false;
        return true;
    }
    if (p.n_rot % 16 != 0 || p.n_rot > p.head_dim) {
        return false;
    }
    e->theta.resize(p.n_rot / 2);
    for (uint32_t i = 0; i < p.n_rot / 2; ++i) {
        const float ex = -2.0f * static_cast<float>(i) / static_cast<float>(p.n_rot);
        e->theta[i] = powf(p.rope_freq_base, ex) * p.rope_freq_scale;
    }
    e->xf = kvmem_hip_transform{};
    e->xf.head_dim = p.head_dim;
    e->xf.n_rot = p.n_rot;
    e->xf.theta = e->theta.empty() ? nullptr : e->theta.data();
    e->xf.hadamard_k = had_k;
    e->xf.hadamard_v = had_v;
    e->xf.pos0 = nullptr;  // original positions: block_id * block_tokens
    e->has_xf = true;
    return true;
}

}  // namespace

extern "C" {

kvmem_engine_params kvmem_engine_default_params(void) {
    kvmem_engine_params p{};
    p.device = 0;
    p.n_layers = 16;
    p.block_tokens = 128;
    p.n_head = 24;
    p.n_head_kv = 4;
    p.head_dim = 256;
    p.n_embd_v = 0;
    p.budget_blocks = 256;
    p.reserve_blocks = 128;
    p.sink_blocks = 1;
    p.recent_blocks = 0;
    p.type_k = KVMEM_TYPE_Q8_0;
    p.type_v = KVMEM_TYPE_Q8_0;
    p.tie_lower_index = 1;
    p.layer_reduce = KVMEM_LAYER_MEAN;
    p.canonical_layout = 1;
    p.scorer = KVMEM_SCORER_TOKEN_MAX;
    p.n_rot = 0;
    p.rope_freq_base = 10000.0f;
    p.rope_freq_scale = 1.0f;
    p.attn_rot = 0;
    p.query_max_tokens = 512;
    p.query_last = 64;
    p.device_plan = 1;
    return p;
}

int kvmem_engine_create(const kvmem_engine_params *pp, kvmem_engine **out) {
    if (!pp || !out) {
        return KVMEM_HIP_ERR_INVALID;
    }
    *out = nullptr;
    const kvmem_engine_params &p = *pp;
    if (p.n_layers == 0 || p.block_tokens == 0 || p.block_tokens > 128 || p.n_head_kv == 0 ||
        p.n_head % p.n_head_kv != 0 || (p.head_dim != 128 && p.head_dim != 256) ||
        p.budget_blocks == 0 || !kvmem_hip_quant_ok(p.type_k) || !kvmem_hip_quant_ok(p.type_v) ||
        (p.scorer != KVMEM_SCORER_TOKEN_MAX && p.scorer != KVMEM_SCORER_MEAN_K)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint32_t n_slots = p.budget_blocks + p.reserve_blocks;
    kvmem_engine *e = new (std::nothrow) kvmem_engine(p, n_slots);
    if (!e) {
        return KVMEM_HIP_ERR_NOMEM;
    }
    e->n_embd_k = p.n_head_kv * p.head_dim;
    e->n_embd_v = p.n_embd_v ? p.n_embd_v : e->n_embd_k;
    if (e->p.query_max_tokens == 0) e->p.query_max_tokens = 512;  // zero-initialised params
    if (e->p.query_last == 0) e->p.query_last = 64;
    e->qwin_cap = e->p.query_max_tokens;
    e->qwin_count.assign(p.n_layers, 0);
    if (e->n_embd_v % 32 != 0) {
        delete e;
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!setup_transform(e)) {
        delete e;
        return KVMEM_HIP_ERR_INVALID;
    }
    int rc = kvmem_hip_create(p.device, &e->ctx);
    if (rc != KVMEM_HIP_OK) {
        delete e;
        return rc;
    }
    if (!alloc_own_pool(e)) {
        kvmem_engine_destroy(e);
        return KVMEM_HIP_ERR_NOMEM;
    }
    *out = e;
    return KVMEM_HIP_OK;
}

void kvmem_engine_destroy(kvmem_engine *e) {
    if (!e) {
        return;
    }
    if (e->ctx) {
        kvmem_hip_sync(e->ctx);
    }
    if (e->own_pool) {
        for (void *ptr : e->pool_k) {
            if (ptr) (void) hipFree(ptr);
        }
        for (void *ptr : e->pool_v) {
            if (ptr) (void) hipFree(ptr);
        }
    }
    if (e->d_scores) {
        (void) hipFree(e->d_scores);
    }
    if (e->d_ksum) {
        (void) hipFree(e->d_ksum);
    }
    if (e->d_qsum) {
        (void) hipFree(e->d_qsum);
    }
    if (e->d_qimp) {
        (void) hipFree(e->d_qimp);
    }
    if (e->d_mt) {
        (void) hipFree(e->d_mt);
    }
    if (e->d_qwin) {
        (void) hipFree(e->d_qwin);
    }
    if (e->d_qgather) {
        (void) hipFree(e->d_qgather);
    }
    kvmem_hip_destroy(e->ctx);
    delete e;
}

const char *kvmem_engine_last_error(const kvmem_engine *e) {
    return e ? e->err.c_str() : "null engine";
}

kvmem_hip_ctx *kvmem_engine_ctx(kvmem_engine *e) {
    return e ? e->ctx : nullptr;
}

int kvmem_engine_set_device_history(kvmem_engine *e, const void *k, const void *v,
                                    uint32_t capacity_blocks, uint32_t n_tokens) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!k || !v) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_device_history: null K or V");
    }
    if ((reinterpret_cast<uintptr_t>(k) & 15u) || (reinterpret_cast<uintptr_t>(v) & 15u)) {
        // the scorer, the key sums and every stage-in read it in 16-byte words
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_device_history: K and V must be 16-byte aligned");
    }
    const uint64_t cap_tokens = static_cast<uint64_t>(capacity_blocks) * e->p.block_tokens;
    if (n_tokens > cap_tokens) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_device_history: n_tokens exceeds the capacity");
    }
    if (k != e->hist_k || v != e->hist_v || capacity_blocks != e->hist_capacity) {
        // A new history: the pool rows, key sums and packed rows of every
        // block were made from the old one.
        if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {  // work reading the old one is done
            return e->fail_ctx(KVMEM_HIP_ERR_RUNTIME, "set_device_history");
        }
        e->hist_k = k;
        e->hist_v = v;
        e->hist_capacity = capacity_blocks;
        drop_residency(e);
        e->meank_valid = 0;
        std::fill(e->packed_valid.begin(), e->packed_valid.end(), 0);
    }
    // The same history grown or cut: as append_tokens / truncate_to (a
    // resident partial tail that grows is staged again, its key sums redone).
    const uint32_t have = e->rt.store().total_tokens();
    if (n_tokens < have) {
        return kvmem_engine_truncate_to(e, n_tokens);
    }
    if (n_tokens > have) {
        return kvmem_engine_append_tokens(e, n_tokens - have);
    }
    ++e->epoch;
    return KVMEM_HIP_OK;
}

int kvmem_engine_set_host_history(kvmem_engine *e, const void *pinned_base,
                                  uint32_t capacity_blocks) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (pinned_base && capacity_blocks < e->rt.store().block_count()) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_host_history: capacity below the block count");
    }
    e->host_base = pinned_base;
    e->host_capacity = pinned_base ? capacity_blocks : 0;
    std::fill(e->packed_valid.begin(), e->packed_valid.end(), 0);  // a new history
    if (!e->hist_k) {
        e->meank_valid = 0;  // the key sums come from this history
    }
    return KVMEM_HIP_OK;
}

int kvmem_engine_set_packed_host(kvmem_engine *e, void *pinned_base, uint32_t capacity_blocks) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {  // copies into the old store are done
        return e->fail_ctx(KVMEM_HIP_ERR_RUNTIME, "set_packed_host");
    }
    e->packed_base = pinned_base;
    e->packed_capacity = pinned_base ? capacity_blocks : 0;
    e->packed_valid.assign(e->packed_capacity, 0);
    return KVMEM_HIP_OK;
}

int kvmem_engine_packed_valid(const kvmem_engine *e, uint32_t block_id) {
    return e && block_id < e->packed_capacity && e->packed_valid[block_id] ? 1 : 0;
}

int kvmem_engine_append_tokens(kvmem_engine *e, uint32_t n_new_tokens) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint64_t want = static_cast<uint64_t>(e->rt.store().total_tokens()) + n_new_tokens;
    if ((!e->hist_k && !e->host_base) ||
        (e->hist_k && want > static_cast<uint64_t>(e->hist_capacity) * e->p.block_tokens) ||
        (e->host_base && want > static_cast<uint64_t>(e->host_capacity) * e->p.block_tokens)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "append_tokens: history capacity exceeded");
    }
    const uint32_t first_new = e->rt.store().block_count();
    if (first_new > 0 && n_new_tokens > 0 &&
        e->rt.store().blocks().back().n_tokens < e->p.block_tokens) {
        e->meank_valid = std::min(e->meank_valid, first_new - 1);  // the tail grows
    }
    if (first_new > 0 && n_new_tokens > 0) {
        // a partial tail that is in the pool must be staged again
        const Block &tail = e->rt.store().blocks().back();
        if (tail.n_tokens < e->p.block_tokens && tail.tier == Tier::GPU && tail.gpu_slot >= 0) {
            const int64_t tail_id = tail.block_id;
            if (e->dirty_tail >= 0 && e->dirty_tail != tail_id) {
                // The engine tracks one block whose pool rows are stale.  An
                // earlier one (a tail that grew, then rows decoded after it)
                // leaves the pool rather than lose its mark: the next
                // selection that holds it stages it again.
                evict_block(e, static_cast<uint32_t>(e->dirty_tail));
            }
            e->dirty_tail = tail_id;
        }
    }
    e->rt.register_append(n_new_tokens);
    for (uint32_t id = first_new; id < e->rt.store().block_count(); ++id) {
        e->rt.store().set_block_tier(id, Tier::CPU);
    }
    ++e->epoch;
    return KVMEM_HIP_OK;
}

int kvmem_engine_truncate_to(kvmem_engine *e, uint32_t token_pos) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (token_pos < e->rt.store().total_tokens()) {
        ++e->attn_epoch;  // rows attention read are gone
    }
    e->rt.truncate_to(token_pos);
    // blocks from the one holding token_pos on are cut short or gone
    for (uint32_t id = token_pos / e->p.block_tokens; id < e->packed_capacity; ++id) {
        e->packed_valid[id] = 0;
    }
    const uint32_t nb = e->rt.store().block_count();
    if (e->dirty_tail >= static_cast<int64_t>(nb)) {
        // the grown tail is gone: a block appended later under its id is a
        // new one, complete once its rows are written
        e->dirty_tail = -1;
    }
    // a block cut short has stale sums
    e->meank_valid = std::min(e->meank_valid, nb > 0 ? nb - 1 : 0u);
    ++e->epoch;
    return KVMEM_HIP_OK;
}

uint32_t kvmem_engine_block_count(const kvmem_engine *e) {
    return e ? e->rt.store().block_count() : 0;
}

uint32_t kvmem_engine_total_tokens(const kvmem_engine *e) {
    return e ? e->rt.store().total_tokens() : 0;
}

uint64_t kvmem_engine_epoch(const kvmem_engine *e) {
    return e ? e->epoch : 0;
}

uint32_t kvmem_engine_n_slots(const kvmem_engine *e) {
    return e ? e->n_slots : 0;
}

static bool alloc_own_pool(kvmem_engine *e) {
    const size_t kbytes = static_cast<size_t>(e->n_slots) * e->p.block_tokens *
                          kvmem_hip_row_size(e->p.type_k, e->n_embd_k);
    const size_t vbytes = static_cast<size_t>(e->n_slots) * e->p.block_tokens *
                          kvmem_hip_row_size(e->p.type_v, e->n_embd_v);
    e->pool_k.assign(e->p.n_layers, nullptr);
    e->pool_v.assign(e->p.n_layers, nullptr);
    e->own_pool = true;
    // Cleared, as llama.cpp clears its KV cache buffers: attention reads
    // every cell of the pool under a mask, and a cell no stage-in or decode
    // has written (a free slot, the rows past a partial tail) must not hold
    // NaN bits.
    hipStream_t s = static_cast<hipStream_t>(kvmem_hip_get_stream(e->ctx));
    for (uint32_t l = 0; l < e->p.n_layers; ++l) {
        if (hipMalloc(&e->pool_k[l], kbytes) != hipSuccess ||
            hipMalloc(&e->pool_v[l], vbytes) != hipSuccess ||
            hipMemsetAsync(e->pool_k[l], 0, kbytes, s) != hipSuccess ||
            hipMemsetAsync(e->pool_v[l], 0, vbytes, s) != hipSuccess) {
            return false;
        }
    }
    return kvmem_hip_sync(e->ctx) == KVMEM_HIP_OK;
}

int kvmem_engine_set_pool(kvmem_engine *e, void *const *k_layers, void *const *v_layers) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (k_layers && !v_layers) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_pool: V tensors missing");
    }
    if (k_layers) {
        for (uint32_t l = 0; l < e->p.n_layers; ++l) {
            if (!k_layers[l] || !v_layers[l] || (reinterpret_cast<uintptr_t>(k_layers[l]) & 15u) ||
                (reinterpret_cast<uintptr_t>(v_layers[l]) & 15u)) {
                return e->fail(KVMEM_HIP_ERR_INVALID, "set_pool: null or misaligned layer tensor");
            }
        }
    }
    if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {
        return e->fail_ctx(KVMEM_HIP_ERR_RUNTIME, "set_pool");
    }
    // the old tensors go: no block is resident in the pool from here on,
    // also when the new pool cannot be allocated
    drop_residency(e);
    if (e->own_pool) {
        for (void *ptr : e->pool_k) {
            if (ptr) (void) hipFree(ptr);
        }
        for (void *ptr : e->pool_v) {
            if (ptr) (void) hipFree(ptr);
        }
    }
    if (k_layers) {
        e->pool_k.assign(k_layers, k_layers + e->p.n_layers);
        e->pool_v.assign(v_layers, v_layers + e->p.n_layers);
        e->own_pool = false;
    } else if (!alloc_own_pool(e)) {
        // the layers allocated before the failure are freed with the
        // engine; the null ones make every apply fail until a pool is set
        return e->fail(KVMEM_HIP_ERR_NOMEM, "set_pool: pool allocation");
    }
    return KVMEM_HIP_OK;
}

int kvmem_engine_pool_layer(const kvmem_engine *e, uint32_t layer, void **k, void **v) {
    if (!e || layer >= e->p.n_layers) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (k) *k = e->pool_k[layer];
    if (v) *v = e->pool_v[layer];
    return KVMEM_HIP_OK;
}

int kvmem_engine_block_slots(const kvmem_engine *e, int32_t *slots) {
    if (!e || !slots) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const auto &bl = e->rt.store().blocks();
    for (size_t i = 0; i < bl.size(); ++i) {
        slots[i] = bl[i].tier == Tier::GPU ? bl[i].gpu_slot : -1;
    }
    return KVMEM_HIP_OK;
}

}  // extern "C"

namespace {

bool ensure_scores(kvmem_engine *e, uint32_t n) {
    if (e->d_scores_n >= n) {
        return true;
    }
    if (e->d_scores) {
        if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {
            return false;
        }
        (void) hipFree(e->d_scores);
        e->d_scores = nullptr;
    }
    if (hipMalloc(&e->d_scores, sizeof(float) * n) != hipSuccess) {
        e->d_scores_n = 0;
        return false;
    }
    e->d_scores_n = n;
    return true;
}

// The store's charge (sink, mandatory, recent) then the device top-k over
// d_scores for the remaining budget; ascending selection into sel.
int select_topk(kvmem_engine *e, const kvmem_amd::TopkCharge &charge, uint32_t *sel, uint32_t *n_sel) {
    const uint32_t n = e->rt.store().block_count();
    std::vector<uint32_t> out;
    if (charge.all_fit) {
        out.resize(n);
        for (uint32_t i = 0; i < n; ++i) out[i] = i;
    } else {
        std::vector<uint32_t> got(n);
        uint32_t cnt = 0;
        const int rc = kvmem_hip_topk(e->ctx, e->d_scores, n, charge.forced.data(),
                                      static_cast<uint32_t>(charge.forced.size()), charge.need,
                                      e->p.tie_lower_index, got.data(), &cnt);
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "preview top-k");
        }
        got.resize(cnt);
        out.swap(got);
    }
    std::copy(out.begin(), out.end(), sel);
    *n_sel = static_cast<uint32_t>(out.size());
    return KVMEM_HIP_OK;
}

// Mean-K cosine scores of every block into d_scores.  The per-block key
// sums are produced on the device for the blocks written since the last
// call (a partial tail block is summed again once it grows).
int meank_scores(kvmem_engine *e, const float *q_sum, const uint32_t *q_count) {
    const uint32_t n = e->rt.store().block_count();
    const uint32_t cap = e->sums_capacity();
    if (e->meank_cap != cap) {
        if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {
            return e->fail_ctx(KVMEM_HIP_ERR_RUNTIME, "mean-K scorer");
        }
        if (e->d_ksum) (void) hipFree(e->d_ksum);
        if (e->d_mt) (void) hipFree(e->d_mt);
        e->d_ksum = nullptr;
        e->d_mt = nullptr;
        const size_t lc = static_cast<size_t>(e->p.n_layers) * cap;
        if (hipMalloc(&e->d_ksum, sizeof(float) * lc * e->n_embd_k) != hipSuccess ||
            hipMalloc(&e->d_mt, sizeof(uint32_t) * lc) != hipSuccess) {
            e->meank_cap = 0;
            return e->fail(KVMEM_HIP_ERR_NOMEM, "mean-K scorer: key sums");
        }
        e->meank_cap = cap;
        e->meank_valid = 0;
    }
    if (e->meank_valid < n) {
        std::vector<uint32_t> ids;
        for (uint32_t b = e->meank_valid; b < n; ++b) ids.push_back(b);
        int rc;
        if (e->hist_k) {
            const kvmem_hip_history h = e->device_history();
            rc = kvmem_hip_meank_sums(e->ctx, &h, ids.data(), static_cast<uint32_t>(ids.size()), e->d_ksum,
                                      e->d_mt);
        } else {
            // host-only history: the sums are read from the pinned blocks
            const kvmem_hip_host_history h = e->host_history();
            rc = kvmem_hip_meank_sums_host(e->ctx, &h, ids.data(), static_cast<uint32_t>(ids.size()), cap,
                                           e->d_ksum, e->d_mt);
        }
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "mean-K key sums");
        }
        const bool tail_partial = e->rt.store().blocks().back().n_tokens < e->p.block_tokens;
        e->meank_valid = tail_partial ? n - 1 : n;
    }
    kvmem_hip_meank_args a{};
    a.q_sum = q_sum;
    a.q_count = q_count;
    a.k_sum = e->d_ksum;
    a.mean_tokens = e->d_mt;
    a.n_layers = e->p.n_layers;
    a.n_blocks = n;
    a.capacity_blocks = cap;
    a.n_head = e->p.n_head;
    a.n_head_kv = e->p.n_head_kv;
    a.head_dim = e->p.head_dim;
    a.scores = e->d_scores;
    const int rc = kvmem_hip_score_meank(e->ctx, &a);
    return rc == KVMEM_HIP_OK ? rc : e->fail_ctx(rc, "mean-K score");
}

// The store state before an apply, and the pool slots that apply's device
// work has been asked to write so far.
struct ApplyUndo {
    KvMemRuntime rt;
    RecordingSlots slots;
    int64_t dirty_tail;
    std::vector<uint8_t> packed_valid;
    std::vector<uint32_t> written_slots;
};

// A failed apply leaves the store as before it, except that a block whose
// slot the failed work may have written (a move destination or a stage-in
// slot) is no longer trusted: it leaves the pool and the working set, so the
// next apply that selects it stages it in again.  Packed rows copied out by
// the failed apply are not marked kept.  The device error stays in the
// engine's last error; the return value is `code`.
int rollback(kvmem_engine *e, ApplyUndo &u, int code) {
    ++e->attn_epoch;  // the failed work may have changed pool rows
    e->rt = std::move(u.rt);
    e->slots = std::move(u.slots);
    e->dirty_tail = u.dirty_tail;
    e->packed_valid = std::move(u.packed_valid);
    if (!u.written_slots.empty()) {
        std::vector<uint8_t> hit(e->n_slots, 0);
        for (uint32_t s : u.written_slots) {
            if (s < e->n_slots) hit[s] = 1;
        }
        for (const Block &b : e->rt.store().blocks()) {
            if (b.tier == Tier::GPU && b.gpu_slot >= 0 && hit[static_cast<uint32_t>(b.gpu_slot)]) {
                const uint32_t id = b.block_id;
                e->slots.free_gpu_slot(b.gpu_slot);
                e->rt.store().set_block_tier(id, Tier::CPU);
                e->rt.store().drop_from_working_set(id);
                if (e->dirty_tail == static_cast<int64_t>(id)) {
                    e->dirty_tail = -1;
                }
            }
        }
    }
    return code;
}

// The query window rows a preview reads, oldest first: the newest
// query_max_tokens captured rows (query_last when no span is set; the
// server's clamp and fallback, tools/llama-kvmem-server.cpp:1032-1038,
// 1089-1096).  Every layer must hold the same number of rows.
int window_rows(kvmem_engine *e, std::vector<uint32_t> &rows, uint64_t since = 0, bool allow_none = false) {
    rows.clear();
    const uint64_t c = e->qwin_count.empty() ? 0 : e->qwin_count[0];
    for (uint64_t x : e->qwin_count) {
        if (x != c) {
            return e->fail(KVMEM_HIP_ERR_INVALID, "query window: layers hold different numbers of rows");
        }
    }
    // only rows captured after `since` rows (those since a set_query)
    const uint64_t limit = e->spans_set() ? e->qwin_cap : std::min<uint32_t>(e->qwin_cap, e->p.query_last);
    const uint64_t n = std::min<uint64_t>(c > since ? c - since : 0, limit);
    if (n == 0) {
        return allow_none ? KVMEM_HIP_OK : e->fail(KVMEM_HIP_ERR_INVALID, "query window: no query rows captured");
    }
    for (uint64_t i = c - n; i < c; ++i) {
        rows.push_back(static_cast<uint32_t>(i % e->qwin_cap));
    }
    return KVMEM_HIP_OK;
}

// The query state a preview with q = NULL reads, into d_qsum and `counts`:
// the window's rows summed in token order; after set_query, the set sums
// with the rows captured since (the query unfrozen) added onto them in
// token order, and the set counts plus those rows -- as the reference's
// harvest adds each row onto q_sum_ and q_count_ after set_query
// (llama-memory-kvmem.cpp:2164-2172, 3121-3137).
int query_state(kvmem_engine *e, std::vector<uint32_t> &counts) {
    const uint32_t L = e->p.n_layers;
    const uint32_t n_embd_q = e->p.n_head * e->p.head_dim;
    const size_t bytes = sizeof(float) * static_cast<size_t>(L) * n_embd_q;
    if (!e->d_qsum && hipMalloc(&e->d_qsum, bytes) != hipSuccess) {
        e->d_qsum = nullptr;
        return e->fail(KVMEM_HIP_ERR_NOMEM, "query sums");
    }
    std::vector<uint32_t> rows;
    int rc = window_rows(e, rows, e->query_imported ? e->imp_base : 0, e->query_imported);
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    if (e->query_imported) {
        hipStream_t st = static_cast<hipStream_t>(kvmem_hip_get_stream(e->ctx));
        if (hipMemcpyAsync(e->d_qsum, e->d_qimp, bytes, hipMemcpyDeviceToDevice, st) != hipSuccess) {
            return e->fail(KVMEM_HIP_ERR_RUNTIME, "query state: copy of the set sums");
        }
    }
    if (!rows.empty()) {
        rc = kvmem_hip_q_accumulate(e->ctx, e->d_qwin, KVMEM_TYPE_F32, L, e->qwin_cap, n_embd_q, rows.data(),
                                    static_cast<uint32_t>(rows.size()), e->query_imported ? 0 : 1, e->d_qsum);
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "query state: sums");
        }
    }
    counts.assign(L, static_cast<uint32_t>(rows.size()));
    if (e->query_imported) {
        for (uint32_t l = 0; l < L; ++l) {
            counts[l] += e->imp_count[l];
        }
    }
    return KVMEM_HIP_OK;
}

// The scoring half of a preview: the mandatory ids (the caller's, then the
// spans'), the store's charge, and the scores of every block launched into
// d_scores (not waited for) -- also when every block fits the budget and the
// selection needs none, as the reference scores on every preview
// (preview_retrieval, llama-memory-kvmem.cpp:3047-3067), so that the scores
// a caller reads back are always this preview's.  *empty: the store has no
// block.
int preview_scores(kvmem_engine *e, const void *q, int32_t q_type, uint32_t n_q_tokens,
                   const uint32_t *mandatory, uint32_t n_mandatory, kvmem_amd::TopkCharge &charge,
                   bool *empty) {
    *empty = false;
    if (!e->hist_k && (e->p.scorer != KVMEM_SCORER_MEAN_K || !e->host_base)) {
        // the per-token scorer reads every key in HBM; the mean-K scorer
        // also runs from a pinned host history's key sums
        return e->fail(KVMEM_HIP_ERR_INVALID, "preview: no device history (the scorer reads keys in HBM)");
    }
    const uint32_t n = e->rt.store().block_count();
    // no query pointer: the sums set by set_query, or the captured query
    // window, its newest rows in token order
    std::vector<uint32_t> win_rows;
    const bool imported = !q && e->query_imported;
    if (imported && e->p.scorer != KVMEM_SCORER_MEAN_K) {
        return e->fail(KVMEM_HIP_ERR_UNSUPPORTED, "preview: a set query holds row sums; the per-token scorer needs rows");
    }
    if (!q && !imported) {
        const int rc = window_rows(e, win_rows);
        if (rc != KVMEM_HIP_OK) {
            return rc;
        }
        n_q_tokens = static_cast<uint32_t>(win_rows.size());
    }
    if (n == 0) {
        *empty = true;
        return KVMEM_HIP_OK;
    }
    if (!ensure_scores(e, n)) {
        return e->fail(KVMEM_HIP_ERR_NOMEM, "preview: score buffer");
    }
    std::vector<uint32_t> mand(mandatory, mandatory + n_mandatory);
    const std::vector<uint32_t> spans = e->retrieval_mandatory();
    mand.insert(mand.end(), spans.begin(), spans.end());
    charge = e->rt.store().charge_topk(mand);
    const uint32_t n_embd_q = e->p.n_head * e->p.head_dim;
    if (imported) {
        // the set query's sums and counts, with the rows captured since
        std::vector<uint32_t> counts;
        const int rc = query_state(e, counts);
        return rc == KVMEM_HIP_OK ? meank_scores(e, e->d_qsum, counts.data()) : rc;
    }
    if (e->p.scorer == KVMEM_SCORER_MEAN_K) {
        // the reference's scorer over the sum of the query rows
        if (!e->d_qsum &&
            hipMalloc(&e->d_qsum, sizeof(float) * e->p.n_layers * n_embd_q) != hipSuccess) {
            e->d_qsum = nullptr;
            return e->fail(KVMEM_HIP_ERR_NOMEM, "preview: query sums");
        }
        int rc = q ? kvmem_hip_q_accumulate(e->ctx, q, q_type, e->p.n_layers, n_q_tokens, n_embd_q, nullptr,
                                            0, 1, e->d_qsum)
                   // the window's rows summed in token order, as the harvest adds them
                   : kvmem_hip_q_accumulate(e->ctx, e->d_qwin, KVMEM_TYPE_F32, e->p.n_layers, e->qwin_cap,
                                            n_embd_q, win_rows.data(), n_q_tokens, 1, e->d_qsum);
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "preview query sums");
        }
        const std::vector<uint32_t> q_count(e->p.n_layers, n_q_tokens);
        return meank_scores(e, e->d_qsum, q_count.data());
    }
    if (!q) {
        // the window's rows in token order, as the bf16 query the scorer reads
        const size_t bytes = 2u * static_cast<size_t>(e->p.n_layers) * e->qwin_cap * n_embd_q;
        if (!e->d_qgather && hipMalloc(&e->d_qgather, bytes) != hipSuccess) {
            e->d_qgather = nullptr;
            return e->fail(KVMEM_HIP_ERR_NOMEM, "preview: query window gather buffer");
        }
        const int rc = kvmem_hip_q_window_gather(e->ctx, e->d_qwin, e->p.n_layers, e->qwin_cap, n_embd_q,
                                                 win_rows.data(), n_q_tokens, KVMEM_TYPE_BF16,
                                                 e->d_qgather);
        if (rc != KVMEM_HIP_OK) {
            return e->fail_ctx(rc, "preview query window");
        }
        q = e->d_qgather;
        q_type = KVMEM_TYPE_BF16;
    }
    const kvmem_hip_history h = e->device_history();
    kvmem_hip_score_args a{};
    a.q = q;
    a.q_type = q_type;
    a.n_q_tokens = n_q_tokens;
    a.n_head = e->p.n_head;
    a.n_head_kv = e->p.n_head_kv;
    a.head_dim = e->p.head_dim;
    a.layer_reduce = e->p.layer_reduce;
    a.layer_scores = nullptr;
    a.scores = e->d_scores;
    const int rc = kvmem_hip_score(e->ctx, &h, &a);
    return rc == KVMEM_HIP_OK ? rc : e->fail_ctx(rc, "preview score");
}

// The store's side of a canonical-layout apply of `ids` (ascending, unique,
// in range): the plan committed (prepare_selection + finish_reselect), the
// grown partial tail staged again, window slot i given to the i-th id.
// Counts the blocks staged and the resident blocks that change slot.
void commit_canonical(kvmem_engine *e, const std::vector<uint32_t> &ids, Plan &plan, uint32_t *n_staged,
                      uint32_t *n_moved) {
    const uint32_t n = e->rt.store().block_count();
    std::vector<int32_t> old_slot(n, -1);
    for (const Block &b : e->rt.store().blocks()) {
        old_slot[b.block_id] = b.tier == Tier::GPU ? b.gpu_slot : -1;
    }
    e->slots.staged_ids.clear();
    e->slots.staged_slots.clear();
    plan = e->rt.prepare_selection(ids);
    e->rt.finish_reselect();
    std::vector<uint8_t> staged(n, 0);
    for (uint32_t id : e->slots.staged_ids) staged[id] = 1;
    if (e->dirty_tail >= 0) {
        const uint32_t id = static_cast<uint32_t>(e->dirty_tail);
        if (id < n && e->rt.store().blocks()[id].tier == Tier::GPU && e->rt.store().blocks()[id].gpu_slot >= 0) {
            staged[id] = 1;
        }
        e->dirty_tail = -1;
    }
    *n_staged = 0;
    *n_moved = 0;
    for (uint32_t i = 0; i < ids.size(); ++i) {
        const uint32_t id = ids[i];
        if (staged[id]) {
            ++*n_staged;
        } else if (old_slot[id] >= 0 && static_cast<uint32_t>(old_slot[id]) != i) {
            ++*n_moved;
        }
        e->rt.store().set_block_gpu_slot(id, static_cast<int32_t>(i));
    }
    e->slots.reset_after(static_cast<uint32_t>(ids.size()));
}

// Whether apply_retrieval can take the device plan: the parameters, the
// history and the pool it covers -- every condition under which
// kvmem_hip_reselect_device refuses a plan, so that a refusal never comes
// after the top-k is launched (the selection size and the resident blocks'
// order are checked per call).
bool device_plan_ok(const kvmem_engine *e) {
    if (!e->p.device_plan || !e->p.canonical_layout || !e->hist_k || !e->hist_v || e->host_base ||
        e->packed_base || e->n_slots > KVMEM_PLAN_MAX_SLOTS || e->p.block_tokens > 65535u ||
        kvmem_hip_row_size(e->p.type_k, e->n_embd_k) % 16 != 0 ||
        kvmem_hip_row_size(e->p.type_v, e->n_embd_v) % 16 != 0 || e->n_embd_k % 32 != 0 ||
        e->n_embd_v % 32 != 0 || (reinterpret_cast<uintptr_t>(e->hist_k) & 15u) ||
        (reinterpret_cast<uintptr_t>(e->hist_v) & 15u) || e->hist_capacity < e->rt.store().block_count() ||
        (e->has_xf && e->xf.pos0)) {
        return false;
    }
    for (uint32_t l = 0; l < e->p.n_layers; ++l) {
        if (!e->pool_k[l] || !e->pool_v[l]) {
            return false;
        }
    }
    return true;
}

// A device plan that failed part way may have moved or written any slot of
// the window: nothing in the pool is trusted any more.
int device_plan_failed(kvmem_engine *e, int code, const char *what) {
    e->fail_ctx(code, what);
    (void) kvmem_hip_sync(e->ctx);
    drop_residency(e);
    return code;
}

// apply_retrieval as one device pipeline: scorer, top-k, then (queued
// behind it, sized on the device) the diff and slot plan, the slot saves
// and the chain walk.  The host meanwhile waits for the selection, commits
// the same plan to the store and queues the stage-in of the blocks it
// stages while the walk runs, then checks the device's counts against its
// own.  KVMEM_HIP_ERR_UNSUPPORTED (nothing issued):
// take the host path.
int apply_retrieval_device(kvmem_engine *e, const void *q, int32_t q_type, uint32_t n_q_tokens,
                           const uint32_t *mandatory, uint32_t n_mandatory, kvmem_plan_stats *stats) {
    const uint32_t n = e->rt.store().block_count();
    if (n == 0 || (!e->hist_k && !e->host_base)) {
        return KVMEM_HIP_ERR_UNSUPPORTED;
    }
    kvmem_amd::TopkCharge charge;
    bool empty = false;
    int rc = preview_scores(e, q, q_type, n_q_tokens, mandatory, n_mandatory, charge, &empty);
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    // while the scorer runs: the blocks whose pool rows are valid,
    // ascending in id; a canonical pool holds them at ascending slots
    std::vector<uint32_t> res_block, res_slot;
    bool canonical = true;
    for (const Block &b : e->rt.store().blocks()) {
        if (b.tier == Tier::GPU && b.gpu_slot >= 0) {
            if (!res_slot.empty() && static_cast<uint32_t>(b.gpu_slot) <= res_slot.back()) {
                canonical = false;
                break;
            }
            res_block.push_back(b.block_id);
            res_slot.push_back(static_cast<uint32_t>(b.gpu_slot));
        }
    }
    const uint32_t max_sel = static_cast<uint32_t>(charge.forced.size()) + charge.need;
    if (!canonical || empty || charge.all_fit || max_sel == 0 || max_sel > KVMEM_PLAN_MAX_SEL ||
        max_sel > e->n_slots) {
        // outside the device plan: the host selects over the scores on the
        // stream and plans
        std::vector<uint32_t> sel(std::max<uint32_t>(1, n));
        uint32_t n_sel = 0;
        if (!empty) {
            rc = select_topk(e, charge, sel.data(), &n_sel);
            if (rc != KVMEM_HIP_OK) {
                return rc;
            }
        }
        return kvmem_engine_apply(e, e->epoch, e->rt.store().total_tokens(), sel.data(), n_sel, stats);
    }
    rc = kvmem_hip_topk_launch_dev(e->ctx, e->d_scores, n, charge.forced.data(),
                                   static_cast<uint32_t>(charge.forced.size()), charge.need,
                                   e->p.tie_lower_index);
    if (rc != KVMEM_HIP_OK) {
        return e->fail_ctx(rc, "apply_retrieval: top-k");
    }
    const uint32_t dirty = e->dirty_tail >= 0 ? static_cast<uint32_t>(e->dirty_tail) : UINT32_MAX;
    const kvmem_hip_history h = e->device_history();
    const kvmem_hip_pool pool = e->pool_desc();
    rc = kvmem_hip_reselect_device(e->ctx, &h, &pool, res_block.data(), res_slot.data(),
                                   static_cast<uint32_t>(res_block.size()), dirty, max_sel);
    std::vector<uint32_t> sel(max_sel);
    uint32_t n_sel = 0;
    const int wrc = kvmem_hip_topk_wait(e->ctx, sel.data(), &n_sel);
    if (rc != KVMEM_HIP_OK) {
        return device_plan_failed(e, rc, "apply_retrieval: device plan");
    }
    if (wrc != KVMEM_HIP_OK) {
        return device_plan_failed(e, wrc, "apply_retrieval: top-k");
    }
    sel.resize(n_sel);
    Plan plan;
    uint32_t n_staged = 0, n_moved = 0;
    commit_canonical(e, sel, plan, &n_staged, &n_moved);
    // queued while the chain walk runs: the stage-in of the blocks the
    // device plan listed, as many as the store stages
    rc = kvmem_hip_reselect_device_stagein(e->ctx, &h, &pool, n_staged);
    if (rc != KVMEM_HIP_OK) {
        return device_plan_failed(e, rc, "apply_retrieval: stage-in");
    }
    if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {
        return device_plan_failed(e, KVMEM_HIP_ERR_RUNTIME, "apply_retrieval sync");
    }
    uint32_t c[KVMEM_PLAN_N_COUNTS] = {};
    (void) kvmem_hip_reselect_device_counts(e->ctx, c, KVMEM_PLAN_N_COUNTS);
    if (c[KVMEM_PLAN_ERROR] != 0 || c[KVMEM_PLAN_SEL] != n_sel || c[KVMEM_PLAN_STAGE] != n_staged ||
        c[KVMEM_PLAN_MOVES] != n_moved) {
        e->fail(KVMEM_HIP_ERR_RUNTIME, "apply_retrieval: the device plan differs from the store's");
        drop_residency(e);
        return KVMEM_HIP_ERR_RUNTIME;
    }
    if (!plan.stage_in.empty() || !plan.stage_out.empty() || n_staged || n_moved) {
        ++e->attn_epoch;
    }
    fill_stats(plan, n_staged, n_moved, 0, 0, stats);
    if (stats) {
        stats->device_planned = 1;
    }
    return KVMEM_HIP_OK;
}

}  // namespace

extern "C" {

int kvmem_engine_set_request_span(kvmem_engine *e, int32_t query_begin, int32_t query_end,
                                  int32_t force_pos) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    e->explicit_spans = false;
    e->query_begin = query_begin;
    e->query_end = query_end;
    e->force_pos = force_pos;
    return KVMEM_HIP_OK;
}

int kvmem_engine_set_turn_spans(kvmem_engine *e, const kvmem_row_range *query, uint32_t n_query,
                                const kvmem_row_range *mandatory, uint32_t n_mandatory) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::vector<std::pair<int32_t, int32_t>> q, m;
    if ((n_query && !query) || (n_mandatory && !mandatory) || !copy_ranges(query, n_query, q) ||
        !copy_ranges(mandatory, n_mandatory, m)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_turn_spans: invalid KVMem row range");
    }
    e->span_query.swap(q);
    e->span_mandatory.swap(m);
    e->explicit_spans = true;
    return KVMEM_HIP_OK;
}

int kvmem_engine_retrieval_mandatory(const kvmem_engine *e, uint32_t *out, uint32_t capacity,
                                     uint32_t *n_out) {
    if (!e || !n_out || (capacity && !out)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const std::vector<uint32_t> ids = e->retrieval_mandatory();
    *n_out = static_cast<uint32_t>(ids.size());
    if (ids.size() > capacity) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::copy(ids.begin(), ids.end(), out);
    return KVMEM_HIP_OK;
}

int kvmem_engine_preview(kvmem_engine *e, const void *q, int32_t q_type, uint32_t n_q_tokens,
                         const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *sel,
                         uint32_t *n_sel, uint64_t *epoch, uint32_t *rows) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!sel || !n_sel || (n_mandatory && !mandatory)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "preview: null argument");
    }
    *n_sel = 0;
    if (epoch) *epoch = e->epoch;
    if (rows) *rows = e->rt.store().total_tokens();
    kvmem_amd::TopkCharge charge;
    bool empty = false;
    const int rc = preview_scores(e, q, q_type, n_q_tokens, mandatory, n_mandatory, charge, &empty);
    if (rc != KVMEM_HIP_OK || empty) {
        return rc;
    }
    return select_topk(e, charge, sel, n_sel);
}

int kvmem_engine_capture_q(kvmem_engine *e, uint32_t layer, const void *q, int32_t q_type, size_t nb0,
                           size_t nb1, size_t nb2, uint32_t n_tokens, const int32_t *positions) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (layer >= e->p.n_layers || (n_tokens && (!q || !positions))) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "capture_q: bad layer or null argument");
    }
    // the rows of the query (all of them when no span is set: the preview
    // then takes the newest query_last); none while the query is frozen
    // (query_contains is false then, llama-memory-kvmem.cpp:2950-2951)
    std::vector<uint32_t> kept;
    for (uint32_t i = 0; i < n_tokens && !e->query_frozen; ++i) {
        if (!e->spans_set() || e->query_contains(positions[i])) {
            kept.push_back(i);
        }
    }
    if (kept.empty()) {
        return KVMEM_HIP_OK;
    }
    const uint32_t n_embd_q = e->p.n_head * e->p.head_dim;
    if (!e->d_qwin) {
        const size_t bytes = sizeof(float) * static_cast<size_t>(e->p.n_layers) * e->qwin_cap * n_embd_q;
        if (hipMalloc(&e->d_qwin, bytes) != hipSuccess) {
            e->d_qwin = nullptr;
            return e->fail(KVMEM_HIP_ERR_NOMEM, "capture_q: query window");
        }
    }
    // ring of qwin_cap rows: only the newest qwin_cap of this call are written
    uint64_t &count = e->qwin_count[layer];
    const size_t skip = kept.size() > e->qwin_cap ? kept.size() - e->qwin_cap : 0;
    std::vector<uint32_t> tokens, rows;
    for (size_t j = skip; j < kept.size(); ++j) {
        tokens.push_back(kept[j]);
        rows.push_back(static_cast<uint32_t>((count + j) % e->qwin_cap));
    }
    const int rc = kvmem_hip_q_window_write(e->ctx, q, q_type, e->p.n_head, e->p.head_dim, nb0, nb1, nb2,
                                            tokens.data(), rows.data(), static_cast<uint32_t>(tokens.size()),
                                            e->d_qwin + static_cast<size_t>(layer) * e->qwin_cap * n_embd_q,
                                            e->qwin_cap);
    if (rc != KVMEM_HIP_OK) {
        return e->fail_ctx(rc, "capture_q");
    }
    count += kept.size();
    return KVMEM_HIP_OK;
}

int kvmem_engine_reset_query(kvmem_engine *e) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::fill(e->qwin_count.begin(), e->qwin_count.end(), 0);
    e->query_imported = false;  // reset_query_acc zeroes q_sum_ / q_count_
    return KVMEM_HIP_OK;
}

int kvmem_engine_query_rows(kvmem_engine *e, uint32_t *n_rows) {
    if (!e || !n_rows) {
        return KVMEM_HIP_ERR_INVALID;
    }
    std::vector<uint32_t> r;
    const int rc = window_rows(e, r);
    *n_rows = static_cast<uint32_t>(r.size());
    return rc;
}

int kvmem_engine_preview_meank(kvmem_engine *e, const float *q_sum, const uint32_t *q_count,
                               const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *sel,
                               uint32_t *n_sel, uint64_t *epoch, uint32_t *rows) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!q_sum || !q_count || !sel || !n_sel || (n_mandatory && !mandatory)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "preview_meank: null argument");
    }
    if (!e->hist_k && !e->host_base) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "preview_meank: no history");
    }
    const uint32_t n = e->rt.store().block_count();
    *n_sel = 0;
    if (epoch) *epoch = e->epoch;
    if (rows) *rows = e->rt.store().total_tokens();
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    if (!ensure_scores(e, n)) {
        return e->fail(KVMEM_HIP_ERR_NOMEM, "preview_meank: score buffer");
    }
    std::vector<uint32_t> mand(mandatory, mandatory + n_mandatory);
    const std::vector<uint32_t> spans = e->retrieval_mandatory();
    mand.insert(mand.end(), spans.begin(), spans.end());
    const kvmem_amd::TopkCharge charge = e->rt.store().charge_topk(mand);
    const int rc = meank_scores(e, q_sum, q_count);  // also when every block fits, as preview_scores
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    return select_topk(e, charge, sel, n_sel);
}

int kvmem_engine_apply(kvmem_engine *e, uint64_t epoch, uint32_t rows, const uint32_t *sel,
                       uint32_t n_sel, kvmem_plan_stats *stats) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n_sel && !sel) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "apply: null selection");
    }
    if (epoch != e->epoch || rows != e->rt.store().total_tokens()) {
        return e->fail(KVMEM_HIP_ERR_STALE, "stale KVMem selection");
    }
    if (!e->hist_k && !e->host_base) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "apply: no history");
    }
    for (uint32_t l = 0; l < e->p.n_layers; ++l) {
        if (!e->pool_k[l] || !e->pool_v[l]) {
            return e->fail(KVMEM_HIP_ERR_INVALID, "apply: no pool (a failed set_pool)");
        }
    }
    std::vector<uint32_t> ids(sel, sel + n_sel);
    const uint32_t n = e->rt.store().block_count();
    std::sort(ids.begin(), ids.end());
    ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
    ids.erase(std::remove_if(ids.begin(), ids.end(), [n](uint32_t id) { return id >= n; }), ids.end());
    if (ids.size() > e->n_slots) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "apply: selection larger than the slot pool");
    }
    // slots the selection keeps before the plan changes them
    const int64_t dirty_at_start = e->dirty_tail;  // its pool rows are stale
    std::vector<int32_t> old_slot(n, -1);
    for (const Block &b : e->rt.store().blocks()) {
        old_slot[b.block_id] = b.tier == Tier::GPU ? b.gpu_slot : -1;
    }
    // The plan is committed to the store before the device work it asks
    // for; on any failure the store goes back to this state, minus the
    // blocks whose pool slots the failed work may have written.
    ApplyUndo undo{e->rt, e->slots, e->dirty_tail, e->packed_valid, {}};
    const auto t_plan = std::chrono::steady_clock::now();
    e->slots.staged_ids.clear();
    e->slots.staged_slots.clear();
    const Plan plan = e->rt.prepare_selection(ids);
    e->rt.finish_reselect();
    if (!every_stage_in_has_slot(e->rt, plan)) {
        e->fail(KVMEM_HIP_ERR_NOMEM, "apply: slot pool exhausted");
        return rollback(e, undo, KVMEM_HIP_ERR_NOMEM);
    }
    std::vector<uint32_t> stage_ids = e->slots.staged_ids;
    std::vector<uint32_t> stage_slots = e->slots.staged_slots;
    if (e->dirty_tail >= 0) {
        // the grown tail keeps its slot and is quantized again
        const uint32_t id = static_cast<uint32_t>(e->dirty_tail);
        if (id < n) {
            const Block &b = e->rt.store().blocks()[id];
            if (b.tier == Tier::GPU && b.gpu_slot >= 0 &&
                std::find(stage_ids.begin(), stage_ids.end(), id) == stage_ids.end()) {
                auto at = std::lower_bound(stage_ids.begin(), stage_ids.end(), id);
                const size_t k = static_cast<size_t>(at - stage_ids.begin());
                stage_ids.insert(at, id);
                stage_slots.insert(stage_slots.begin() + static_cast<std::ptrdiff_t>(k),
                                   static_cast<uint32_t>(b.gpu_slot));
            }
        }
        e->dirty_tail = -1;
    }
    for (uint32_t s : stage_slots) {
        if (s >= e->n_slots) {
            e->fail(KVMEM_HIP_ERR_RUNTIME, "apply: slot out of range");
            return rollback(e, undo, KVMEM_HIP_ERR_RUNTIME);
        }
    }
    int rc = KVMEM_HIP_OK;
    // the diff and slot plan so far, plus the canonical layout's slot
    // assignment below, are the host's plan
    double plan_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_plan).count();
    // Evicted full blocks whose packed rows the host store lacks are copied
    // out first: the copies are ordered before the moves and stage-ins that
    // reuse their slots on the same stream.
    uint32_t n_saved = 0;
    if (e->packed_base) {
        std::vector<uint32_t> sid, sslot, snt;
        for (uint32_t id : plan.stage_out) {
            if (id < n && old_slot[id] >= 0 && id < e->packed_capacity && !e->packed_valid[id] &&
                static_cast<int64_t>(id) != dirty_at_start &&
                e->rt.store().blocks()[id].n_tokens == e->p.block_tokens) {
                sid.push_back(id);
                sslot.push_back(static_cast<uint32_t>(old_slot[id]));
                snt.push_back(e->p.block_tokens);
            }
        }
        if (!sid.empty()) {
            const kvmem_hip_pool pool = e->pool_desc();
            const kvmem_hip_packed_host ph = packed_desc(e);
            rc = kvmem_hip_stageout_blocks(e->ctx, &pool, &ph, sid.data(), sslot.data(), snt.data(),
                                           static_cast<uint32_t>(sid.size()));
            if (rc != KVMEM_HIP_OK) {
                e->fail_ctx(rc, "apply: stage-out");
                return rollback(e, undo, rc);  // reads the pool only
            }
            for (uint32_t id : sid) e->packed_valid[id] = 1;
            n_saved = static_cast<uint32_t>(sid.size());
        }
    }
    uint32_t n_moved = 0;
    if (e->p.canonical_layout) {
        // window slot i holds the i-th selected block
        const auto t_layout = std::chrono::steady_clock::now();
        std::vector<uint32_t> src, dst, ntok;
        std::vector<uint8_t> staged(n, 0);
        for (uint32_t id : stage_ids) staged[id] = 1;
        stage_slots.clear();
        for (uint32_t i = 0; i < ids.size(); ++i) {
            const uint32_t id = ids[i];
            if (staged[id]) {
                stage_slots.push_back(i);
            } else if (old_slot[id] >= 0 && static_cast<uint32_t>(old_slot[id]) != i) {
                src.push_back(static_cast<uint32_t>(old_slot[id]));
                dst.push_back(i);
                ntok.push_back(e->rt.store().blocks()[id].n_tokens);
            }
            e->rt.store().set_block_gpu_slot(id, static_cast<int32_t>(i));
        }
        // staged ids come in ascending order, so stage_slots pairs with stage_ids
        e->slots.reset_after(static_cast<uint32_t>(ids.size()));
        plan_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_layout).count();
        if (!src.empty()) {
            undo.written_slots.insert(undo.written_slots.end(), dst.begin(), dst.end());
            const kvmem_hip_pool pool = e->pool_desc();
            rc = kvmem_hip_move_slots(e->ctx, &pool, src.data(), dst.data(), ntok.data(),
                                      static_cast<uint32_t>(src.size()));
            if (rc != KVMEM_HIP_OK) {
                e->fail_ctx(rc, "apply: canonical layout");
                return rollback(e, undo, rc);
            }
            n_moved = static_cast<uint32_t>(src.size());
        }
    }
    uint32_t n_restored = 0;
    undo.written_slots.insert(undo.written_slots.end(), stage_slots.begin(), stage_slots.end());
    rc = engine_stage(e, stage_ids, stage_slots, &n_restored);
    if (rc != KVMEM_HIP_OK) {
        return rollback(e, undo, rc);
    }
    if (kvmem_hip_sync(e->ctx) != KVMEM_HIP_OK) {
        e->fail_ctx(KVMEM_HIP_ERR_RUNTIME, "apply sync");
        return rollback(e, undo, KVMEM_HIP_ERR_RUNTIME);
    }
    if (!plan.stage_in.empty() || !plan.stage_out.empty() || !stage_ids.empty() || n_moved) {
        ++e->attn_epoch;  // apply_plan_to_kv / layout / write_block_to_gpu (llama-memory-kvmem.cpp:785, 964, 2735)
    }
    kvmem_hip_perf_add_plan_ms(e->ctx, plan_ms);
    fill_stats(plan, static_cast<uint32_t>(stage_ids.size()), n_moved, n_saved, n_restored, stats);
    return KVMEM_HIP_OK;
}

int kvmem_engine_apply_retrieval(kvmem_engine *e, const void *q, int32_t q_type,
                                 uint32_t n_q_tokens, const uint32_t *mandatory,
                                 uint32_t n_mandatory, kvmem_plan_stats *stats) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if ((n_mandatory && !mandatory)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "apply_retrieval: null mandatory list");
    }
    if (device_plan_ok(e)) {
        const int drc = apply_retrieval_device(e, q, q_type, n_q_tokens, mandatory, n_mandatory, stats);
        if (drc != KVMEM_HIP_ERR_UNSUPPORTED) {
            return drc;
        }
    }
    std::vector<uint32_t> sel(std::max<uint32_t>(1, e->rt.store().block_count()));
    uint32_t n_sel = 0, rows = 0;
    uint64_t epoch = 0;
    int rc = kvmem_engine_preview(e, q, q_type, n_q_tokens, mandatory, n_mandatory, sel.data(),
                                  &n_sel, &epoch, &rows);
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    return kvmem_engine_apply(e, epoch, rows, sel.data(), n_sel, stats);
}

int kvmem_engine_append_resident(kvmem_engine *e, uint32_t n_new_tokens) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    const uint64_t want = static_cast<uint64_t>(e->rt.store().total_tokens()) + n_new_tokens;
    if ((!e->hist_k && !e->host_base) ||
        (e->hist_k && want > static_cast<uint64_t>(e->hist_capacity) * e->p.block_tokens) ||
        (e->host_base && want > static_cast<uint64_t>(e->host_capacity) * e->p.block_tokens)) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "append_resident: history capacity exceeded");
    }
    if (n_new_tokens == 0) {
        return KVMEM_HIP_OK;
    }
    const auto &bl = e->rt.store().blocks();
    const uint32_t first_new = e->rt.store().block_count();
    const bool tail_partial = first_new > 0 && bl.back().n_tokens < e->p.block_tokens;
    // A partial tail without a slot gets one, but its older rows are not in
    // the pool: it is staged again by the next apply.  One such block at a
    // time (the engine tracks a single stale tail).
    const bool tail_gets_slot = tail_partial && !(bl.back().tier == Tier::GPU && bl.back().gpu_slot >= 0);
    if (tail_gets_slot && e->dirty_tail >= 0 && e->dirty_tail != static_cast<int64_t>(first_new - 1)) {
        return e->fail(KVMEM_HIP_ERR_UNSUPPORTED, "append_resident: another block still waits to be staged again");
    }
    const uint32_t tail_id = first_new - 1;
    std::vector<uint32_t> placed;
    if (!e->rt.append_resident(n_new_tokens, &placed)) {
        return e->fail(KVMEM_HIP_ERR_NOMEM, "append_resident: no free pool slot for the new rows");
    }
    if (tail_partial) {
        e->meank_valid = std::min(e->meank_valid, tail_id);  // the tail grows: its sums are redone
    }
    if (tail_gets_slot) {
        e->dirty_tail = tail_id;
    }
    ++e->epoch;  // the history grew: earlier selections are stale (their rows differ)
    return KVMEM_HIP_OK;
}

uint32_t kvmem_engine_free_slots(const kvmem_engine *e) {
    return e ? e->slots.n_free() : 0u;
}

int kvmem_engine_query_replay_fits(const kvmem_engine *e, uint32_t query_begin, uint32_t prompt_end) {
    return !e || kvmem_amd::query_replay_fits(e->rt.store(), query_begin, prompt_end) ? 1 : 0;
}

int kvmem_engine_get_query(kvmem_engine *e, float *q_sum, uint32_t *q_count) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!q_sum || !q_count) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "get_query: null argument");
    }
    std::vector<uint32_t> counts;
    const int rc = query_state(e, counts);
    if (rc != KVMEM_HIP_OK) {
        return rc;
    }
    const size_t bytes = sizeof(float) * static_cast<size_t>(e->p.n_layers) * e->p.n_head * e->p.head_dim;
    hipStream_t st = static_cast<hipStream_t>(kvmem_hip_get_stream(e->ctx));
    if (hipMemcpyAsync(q_sum, e->d_qsum, bytes, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        return e->fail(KVMEM_HIP_ERR_RUNTIME, "get_query: copy");
    }
    std::copy(counts.begin(), counts.end(), q_count);
    return KVMEM_HIP_OK;
}

int kvmem_engine_set_query(kvmem_engine *e, const float *q_sum, const uint32_t *q_count) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (!q_sum || !q_count) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "set_query: null argument");
    }
    if (e->p.scorer != KVMEM_SCORER_MEAN_K) {
        return e->fail(KVMEM_HIP_ERR_UNSUPPORTED,
                       "set_query: the state holds row sums, which only the mean-K scorer reads");
    }
    const uint32_t L = e->p.n_layers;
    const size_t n = static_cast<size_t>(L) * e->p.n_head * e->p.head_dim;
    // llama-memory-kvmem.cpp:3124-3137: finite sums, one nonzero row count
    for (size_t i = 0; i < n; ++i) {
        if (!std::isfinite(q_sum[i])) {
            return e->fail(KVMEM_HIP_ERR_INVALID, "set_query: a sum is not finite");
        }
    }
    for (uint32_t l = 0; l < L; ++l) {
        if (q_count[l] == 0 || q_count[l] != q_count[0]) {
            return e->fail(KVMEM_HIP_ERR_INVALID, "set_query: row counts must be equal and nonzero");
        }
    }
    if (!e->d_qimp && hipMalloc(&e->d_qimp, sizeof(float) * n) != hipSuccess) {
        e->d_qimp = nullptr;
        return e->fail(KVMEM_HIP_ERR_NOMEM, "set_query: query sums");
    }
    hipStream_t st = static_cast<hipStream_t>(kvmem_hip_get_stream(e->ctx));
    if (hipMemcpyAsync(e->d_qimp, q_sum, sizeof(float) * n, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        return e->fail(KVMEM_HIP_ERR_RUNTIME, "set_query: copy");
    }
    // the state replaces the rows captured so far; rows captured once the
    // query is unfrozen add onto it
    e->imp_count.assign(q_count, q_count + L);
    e->imp_base = e->qwin_count.empty() ? 0 : e->qwin_count[0];
    e->query_imported = true;
    e->query_frozen = true;
    return KVMEM_HIP_OK;
}

int kvmem_engine_freeze_query(kvmem_engine *e, int frozen) {
    if (!e) {
        return KVMEM_HIP_ERR_INVALID;
    }
    e->query_frozen = frozen != 0;
    return KVMEM_HIP_OK;
}

uint64_t kvmem_engine_attention_epoch(const kvmem_engine *e) {
    return e ? e->attn_epoch : 0;
}

int kvmem_engine_attention_view(const kvmem_engine *e, int canonical, kvmem_attention_view *view) {
    if (!e || !view) {
        return KVMEM_HIP_ERR_INVALID;
    }
    return export_view(kvmem_amd::attention_view(e->rt.store(), e->pool_state(), canonical != 0), view);
}

int kvmem_engine_selection_fits(const kvmem_engine *e, uint64_t epoch, uint32_t rows, const uint32_t *sel,
                                uint32_t n_sel, uint32_t end, uint32_t generation_rows) {
    if (!e || (n_sel && !sel) || epoch != e->epoch) {
        return 0;
    }
    kvmem_amd::PoolState ps = e->pool_state();
    ps.epoch = epoch;  // the selection's own staleness is checked above
    return kvmem_amd::selection_fits(e->rt.store(), ps, e->retrieval_mandatory(), epoch, rows,
                                     std::vector<uint32_t>(sel, sel + n_sel), end, generation_rows)
               ? 1
               : 0;
}

int kvmem_engine_commit_unchanged(kvmem_engine *e, const kvmem_attention_view *before, uint64_t epoch,
                                  uint32_t rows, const uint32_t *sel, uint32_t n_sel) {
    kvmem_amd::AttentionView v;
    if (!e || (n_sel && !sel) || !import_view(before, v) || epoch != e->epoch) {
        return 0;
    }
    // the view against the attention epoch, the selection against its own
    kvmem_amd::PoolState ps = e->pool_state();
    return kvmem_amd::commit_unchanged(e->rt, ps, v, ps.epoch, rows, std::vector<uint32_t>(sel, sel + n_sel))
               ? 1
               : 0;
}

int kvmem_engine_commit_resident(kvmem_engine *e, int canonical) {
    if (!e) {
        return 0;
    }
    return kvmem_amd::commit_resident(e->rt, e->pool_state(), canonical != 0) ? 1 : 0;
}

int kvmem_engine_can_append(const kvmem_engine *e, uint32_t end, uint32_t generation_rows, int all_history,
                            const char **reason) {
    if (!e) {
        if (reason) *reason = "invalid_boundary";
        return 0;
    }
    return kvmem_amd::can_append(e->rt.store(), e->pool_state(), end, generation_rows, all_history != 0, reason)
               ? 1
               : 0;
}

int kvmem_engine_scores(kvmem_engine *e, float *out, uint32_t n) {
    if (!e || (n && !out)) {
        return KVMEM_HIP_ERR_INVALID;
    }
    if (n > e->d_scores_n) {
        return e->fail(KVMEM_HIP_ERR_INVALID, "scores: more than the last preview produced");
    }
    if (n == 0) {
        return KVMEM_HIP_OK;
    }
    hipStream_t s = static_cast<hipStream_t>(kvmem_hip_get_stream(e->ctx));
    if (hipMemcpyAsync(out, e->d_scores, sizeof(float) * n, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        return e->fail(KVMEM_HIP_ERR_RUNTIME, "scores: copy");
    }
    return KVMEM_HIP_OK;
}

}  // extern "C"
