// C entry points over the reference's own host kvmem library (KvMemStore /
// KvMemRuntime / RawKvStore compiled from kvmem/src/host/*.cpp where the
// reference tree lies), so that the tests can drive it through ctypes as a
// second reference.
//
// TEST INFRASTRUCTURE ONLY: built into oracle/_ref/ by `make ref`; used by
// tests/golden/make_golden.py to write fixtures and by CPU tests when the
// library is present.  Nothing in the product links it.
//
// The slot allocator of the recording backend mirrors the adapter's free
// list (llama-memory-kvmem.cpp:621-627 reset_slots, :693-707 alloc/free):
// slots are handed out from the back of a vector initialised n-1..0, freed
// slots are pushed back (LIFO).
#include "kvmem/kvmem_runtime.hpp"
#include "kvmem/kvmem_store.hpp"
#include "kvmem/raw_kv_store.hpp"
#include "kvmem/rope.hpp"

#include <cstdint>
#include <cstring>
#include <vector>

namespace {

class SlotBackend final : public kvmem::KvMemBackend {
public:
    explicit SlotBackend(uint32_t n_slots) {
        for (int32_t i = static_cast<int32_t>(n_slots) - 1; i >= 0; --i) {
            free_.push_back(i);
        }
    }
    int32_t alloc_gpu_slot() override {
        if (free_.empty()) {
            return -1;
        }
        const int32_t s = free_.back();
        free_.pop_back();
        return s;
    }
    void free_gpu_slot(int32_t slot) override {
        if (slot >= 0) {
            free_.push_back(slot);
        }
    }

private:
    std::vector<int32_t> free_;
};

struct RefRuntime {
    SlotBackend backend;
    kvmem::KvMemRuntime rt;
    RefRuntime(const kvmem::KvMemRuntimeConfig &cfg, uint32_t n_slots)
        : backend(n_slots), rt(cfg, &backend) {}
};

kvmem::KvMemStoreConfig make_cfg(uint32_t block_tokens, uint32_t budget_blocks, uint32_t sink,
                                 uint32_t recent) {
    kvmem::KvMemStoreConfig c;
    c.block_tokens = block_tokens;
    c.select_budget = budget_blocks * block_tokens;
    c.sink_blocks = sink;
    c.recent_blocks = recent;
    return c;
}

}  // namespace

#define KREF_API extern "C" __attribute__((visibility("default")))

// KvMemStore::pick_topk_blocks over explicit scores (one full block per
// score, n blocks).  Writes the ascending ids to out (capacity n).
KREF_API int kref_pick_topk(const double *scores, uint32_t n, uint32_t block_tokens,
                            uint32_t budget_blocks, uint32_t sink, uint32_t recent,
                            const uint32_t *mandatory, uint32_t n_mandatory, uint32_t *out,
                            uint32_t *n_out) {
    try {
        kvmem::KvMemStore st(make_cfg(block_tokens, budget_blocks, sink, recent));
        st.register_append(n * block_tokens);
        st.set_retrieval_scores(std::vector<double>(scores, scores + n));
        std::vector<uint32_t> mand(mandatory, mandatory + n_mandatory);
        const std::vector<uint32_t> sel = st.pick_topk_blocks(mand);
        std::memcpy(out, sel.data(), sel.size() * sizeof(uint32_t));
        *n_out = static_cast<uint32_t>(sel.size());
        return 0;
    } catch (...) {
        return -1;
    }
}

// A runtime with `n_tokens` appended tokens whose blocks all start outside
// the GPU (history on the host), and a slot pool of n_slots.
KREF_API void *kref_runtime_new(uint32_t block_tokens, uint32_t budget_blocks, uint32_t sink,
                                uint32_t recent, uint32_t n_slots, uint32_t n_tokens) {
    try {
        kvmem::KvMemRuntimeConfig cfg;
        cfg.store = make_cfg(block_tokens, budget_blocks, sink, recent);
        auto *r = new RefRuntime(cfg, n_slots);
        r->rt.register_append(n_tokens);
        for (uint32_t id = 0; id < r->rt.store().block_count(); ++id) {
            r->rt.store().set_block_tier(id, kvmem::KvTier::CPU);
        }
        return r;
    } catch (...) {
        return nullptr;
    }
}

KREF_API void kref_runtime_free(void *h) {
    delete static_cast<RefRuntime *>(h);
}

KREF_API void kref_runtime_set_scores(void *h, const double *scores, uint32_t n) {
    static_cast<RefRuntime *>(h)->rt.store().set_retrieval_scores(
        std::vector<double>(scores, scores + n));
}

KREF_API int kref_runtime_preview(void *h, const uint32_t *mandatory, uint32_t n_mandatory,
                                  uint32_t *out, uint32_t *n_out) {
    auto *r = static_cast<RefRuntime *>(h);
    const std::vector<uint32_t> sel =
        r->rt.preview_reselect(std::vector<uint32_t>(mandatory, mandatory + n_mandatory));
    std::memcpy(out, sel.data(), sel.size() * sizeof(uint32_t));
    *n_out = static_cast<uint32_t>(sel.size());
    return 0;
}

// prepare_selection + finish_reselect.  Outputs: stage_in / stage_out ids
// (capacity = block count each), counters[4] = selection_overlap_blocks,
// gpu_reused_blocks, retained_position_stable, retained_position_moved,
// total_window_tokens into counters[4].
KREF_API int kref_runtime_apply(void *h, const uint32_t *sel, uint32_t n_sel, uint32_t *stage_in,
                                uint32_t *n_in, uint32_t *stage_out, uint32_t *n_out,
                                uint32_t *counters) {
    try {
        auto *r = static_cast<RefRuntime *>(h);
        const kvmem::KvMemPlan p =
            r->rt.prepare_selection(std::vector<uint32_t>(sel, sel + n_sel));
        r->rt.finish_reselect();
        std::memcpy(stage_in, p.stage_in.data(), p.stage_in.size() * sizeof(uint32_t));
        std::memcpy(stage_out, p.stage_out.data(), p.stage_out.size() * sizeof(uint32_t));
        *n_in = static_cast<uint32_t>(p.stage_in.size());
        *n_out = static_cast<uint32_t>(p.stage_out.size());
        counters[0] = p.selection_overlap_blocks;
        counters[1] = p.gpu_reused_blocks;
        counters[2] = p.retained_position_stable;
        counters[3] = p.retained_position_moved;
        counters[4] = p.total_window_tokens;
        return 0;
    } catch (...) {
        return -1;
    }
}

// KvMemRuntime::commit_resident_selection: 1 if committed, 0 if refused.
KREF_API int kref_runtime_commit_resident(void *h, const uint32_t *sel, uint32_t n) {
    auto *r = static_cast<RefRuntime *>(h);
    return r->rt.commit_resident_selection(std::vector<uint32_t>(sel, sel + n)) ? 1 : 0;
}

// KvMemStore::prefill_needs_offload of a store with block_tokens per block
// and the default high watermark.
KREF_API int kref_prefill_needs_offload(uint32_t block_tokens, uint32_t resident_tokens,
                                        uint32_t incoming_tokens, uint32_t pool_tokens) {
    kvmem::KvMemStore st(make_cfg(block_tokens, 1, 0, 0));
    return st.prefill_needs_offload(resident_tokens, incoming_tokens, pool_tokens) ? 1 : 0;
}

// Per block: gpu slot (-1 if none), tier, in_working_set, baked_pos.
KREF_API uint32_t kref_runtime_blocks(void *h, int32_t *gpu_slot, uint8_t *tier, uint8_t *in_ws,
                                      int64_t *baked_pos) {
    auto *r = static_cast<RefRuntime *>(h);
    const auto &bl = r->rt.store().blocks();
    for (size_t i = 0; i < bl.size(); ++i) {
        gpu_slot[i] = bl[i].gpu_slot;
        tier[i] = static_cast<uint8_t>(bl[i].tier);
        in_ws[i] = bl[i].in_working_set ? 1 : 0;
        baked_pos[i] = bl[i].baked_pos;
    }
    return static_cast<uint32_t>(bl.size());
}

// RawKvStore mean-K of block `block` after writing n_tokens F16 K rows
// (token-major [n_tokens][n_embd]) from position 0 with
// write_layer_tokens_f16 (capture_mean_f16 path), one layer.
KREF_API int kref_mean_k_f16(uint32_t n_embd, uint32_t block_tokens, const uint16_t *k_rows,
                             uint32_t n_tokens, uint32_t block, float *out) {
    try {
        kvmem::RawKvStoreConfig cfg;
        cfg.n_layer = 1;
        cfg.n_embd_k = n_embd;
        cfg.n_embd_v = n_embd;
        cfg.block_tokens = block_tokens;
        kvmem::RawKvStore raw(cfg);
        raw.write_layer_tokens_f16(0, n_tokens, 0, k_rows, nullptr);
        raw.mean_k(block, 0, out);
        return 0;
    } catch (...) {
        return -1;
    }
}

// RawKvStore mean-K after write_layer_mean_k of f32 rows in batches of
// `batch` tokens (the add_mean_f32 path), one layer.
KREF_API int kref_mean_k_f32(uint32_t n_embd, uint32_t block_tokens, const float *rows,
                             uint32_t n_tokens, uint32_t batch, uint32_t block, float *out) {
    try {
        kvmem::RawKvStoreConfig cfg;
        cfg.n_layer = 1;
        cfg.n_embd_k = n_embd;
        cfg.n_embd_v = n_embd;
        cfg.block_tokens = block_tokens;
        cfg.k_row_bytes = 1088;
        kvmem::RawKvStore raw(cfg);
        for (uint32_t pos = 0; pos < n_tokens; pos += batch) {
            const uint32_t n = n_tokens - pos < batch ? n_tokens - pos : batch;
            raw.write_layer_mean_k(pos, n, 0, rows + static_cast<size_t>(pos) * n_embd);
        }
        raw.mean_k(block, 0, out);
        return 0;
    } catch (...) {
        return -1;
    }
}

// kvmem::rope_neox_apply (kvmem/src/host/rope.cpp): k_prerope token-major
// [n_tokens][n_head_kv][n_embd_head] f32 rotated at positions pos0, pos0+1, ...
KREF_API int kref_rope_neox(uint32_t n_rot, uint32_t n_embd_head, uint32_t n_head_kv, float freq_base,
                            float freq_scale, const float *src, uint32_t n_tokens, int32_t pos0,
                            float *out) {
    try {
        kvmem::RopeConfig cfg;
        cfg.n_rot = n_rot;
        cfg.n_embd_head = n_embd_head;
        cfg.n_head_kv = n_head_kv;
        cfg.freq_base = freq_base;
        cfg.freq_scale = freq_scale;
        kvmem::rope_neox_apply(cfg, src, n_tokens, pos0, out);
        return 0;
    } catch (...) {
        return -1;
    }
}
