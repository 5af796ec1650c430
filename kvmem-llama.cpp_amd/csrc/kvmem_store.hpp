// Host mirror of the reference's KVMem block table, selection and diff
// (kvmem/include/kvmem/kvmem_store.hpp, kvmem_runtime.hpp,
// kvmem_backend.hpp), restricted to what the reselect step uses.  Pure host
// logic: no HIP call is made here.
//
// Kept from the reference interface: the names register_append,
// truncate_to, set_retrieval_scores, pick_topk_blocks(mandatory),
// set_selection -> KvMemPlan, commit_resident_selection, clear_working_set,
// preview_reselect, prepare_selection, spill_outgoing, admit_incoming,
// finish_reselect, and the backend hooks alloc_gpu_slot / free_gpu_slot.
// Their argument meaning and results follow the reference (file:line on
// each declaration).  Left out: CPU/NVMe tiers, the quota and media
// policies, semantic groups and the immutable-source-K refresh counters
// (the latter's remap_count / remap_abs_delta bookkeeping is kept).
#pragma once

#include <cstdint>
#include <functional>
#include <stdexcept>
#include <utility>
#include <vector>

namespace kvmem_amd {

enum class Tier : uint8_t { GPU = 0, CPU = 1, SSD = 2 };

// kvmem_store.hpp:36-73 (fields on this path).
struct Block {
    uint32_t block_id = 0;
    uint32_t orig_pos_start = 0;
    uint32_t n_tokens = 0;
    Tier tier = Tier::GPU;
    int32_t gpu_slot = -1;
    int64_t baked_pos = -1;
    uint32_t remap_count = 0;
    uint64_t remap_abs_delta = 0;
    bool in_working_set = false;
    double retrieval_score = 0.0;
    uint32_t orig_pos_end() const { return orig_pos_start + n_tokens; }
};

// kvmem_store.hpp:80-94.
struct Remap {
    uint32_t block_id = 0;
    uint32_t n_tokens = 0;
    int32_t from_base = 0;
    int32_t to_base = 0;
    bool working_k_resident = false;
    bool skip = false;
};

// kvmem_store.hpp:108-124.
struct Plan {
    std::vector<uint32_t> stage_in;
    std::vector<uint32_t> stage_out;
    std::vector<Remap> remaps;
    uint32_t total_window_tokens = 0;
    uint32_t selection_overlap_blocks = 0;
    uint32_t gpu_reused_blocks = 0;
    uint32_t retained_position_stable = 0;
    uint32_t retained_position_moved = 0;
};

struct StoreConfig {
    uint32_t block_tokens = 128;      // --kvmem-block-tokens
    uint32_t select_budget = 131072;  // tokens; budget_blocks = select_budget / block_tokens
    uint32_t sink_blocks = 1;
    uint32_t recent_blocks = 0;
    // Equal scores: true ranks the lower block id first (the reselect
    // contract); false ranks the higher id first, the reference's recency
    // rule (kvmem_store.cpp:602-609).
    bool tie_lower_index = true;
    // false forces every selected block to be staged in again
    // (optimize_stage_in, kvmem_store.hpp:229-231).
    bool optimize_stage_in = true;
    // Share of the pool's tokens above which a prefill must offload
    // (gpu_high_watermark, kvmem_store.hpp:311).
    double gpu_high_watermark = 0.95;
};

// Blocks charged before the score fill of pick_topk: sink, mandatory
// (newest listed first) and recent, each while the budget has room.
struct TopkCharge {
    bool all_fit = false;             // n <= budget: every block is selected
    std::vector<uint32_t> forced;     // charged ids, in charge order
    uint32_t need = 0;                // best-scored blocks still to add
};

// Ranks the uncharged blocks: writes the `need` best ids (any order) given
// the charged-id mask.  The default ranks the store's retrieval scores on
// the host; the reselect engine plugs in the device top-k.
using Ranker = std::function<std::vector<uint32_t>(const std::vector<uint8_t> &charged,
                                                   uint32_t need)>;

class KvMemStore {
public:
    explicit KvMemStore(StoreConfig cfg) : cfg_(cfg) {
        if (cfg_.block_tokens == 0) {
            throw std::invalid_argument("block_tokens must be positive");
        }
    }

    const StoreConfig &config() const { return cfg_; }
    uint32_t block_count() const { return static_cast<uint32_t>(blocks_.size()); }
    uint32_t total_tokens() const { return total_tokens_; }
    const std::vector<Block> &blocks() const { return blocks_; }
    uint32_t budget_blocks() const { return cfg_.select_budget / cfg_.block_tokens; }

    // kvmem_store.cpp:179-205: fill the trailing partial block, then open
    // new blocks of up to block_tokens, each baked at its true position.
    void register_append(uint32_t n_new_tokens);
    // kvmem_store.cpp:207-227: drop blocks starting at or past token_pos,
    // shrink a straddling last block.  Returns the dropped ids.
    std::vector<uint32_t> truncate_to(uint32_t token_pos);

    // kvmem_store.cpp:242-248: replace every block's score; blocks past
    // scores.size() get 0.
    void set_retrieval_scores(const std::vector<double> &scores);

    // kvmem_store.cpp:482-623 (TopK policy): sink, mandatory newest-first,
    // recent, then the best scores; ids returned ascending.
    std::vector<uint32_t> pick_topk_blocks(const std::vector<uint32_t> &mandatory = {},
                                           const Ranker &ranker = nullptr) const;
    // The charge phase of pick_topk_blocks alone.
    TopkCharge charge_topk(const std::vector<uint32_t> &mandatory) const;

    // kvmem_store.cpp:158-176: the block holding token position pos, -1 if
    // none.
    int32_t block_id_containing(uint32_t pos) const;
    // The adapter's retrieval_mandatory (llama-memory-kvmem.cpp:3026-3045):
    // in block order, every block overlapping one of the half-open row
    // ranges [begin, end), then the block holding force_pos (>= 0).
    std::vector<uint32_t> blocks_overlapping(const std::vector<std::pair<int32_t, int32_t>> &ranges,
                                             int32_t force_pos) const;

    // kvmem_store.cpp:340-351 with gpu_high_watermark_tokens (:320-327):
    // whether incoming_tokens more rows over resident_tokens overflow the
    // pool's pool_tokens or its high watermark.
    bool prefill_needs_offload(uint32_t resident_tokens, uint32_t incoming_tokens,
                               uint32_t pool_tokens) const;

    // kvmem_store.cpp:250-277 with optimize_stage_out: leaving the GPU
    // clears the slot.
    void set_block_tier(uint32_t id, Tier tier);
    void set_block_gpu_slot(uint32_t id, int32_t slot);

    // kvmem_store.cpp:758-882: diff a selection against the working set.
    Plan set_selection(std::vector<uint32_t> selected_ids);
    // kvmem_store.cpp:884-895.
    bool commit_resident_selection(const std::vector<uint32_t> &selected_ids);
    // kvmem_store.cpp:897-901.
    void clear_working_set();
    // One block leaves the window (its pool rows can no longer be trusted);
    // the next selection that keeps it stages it in again.
    void drop_from_working_set(uint32_t id);

private:
    StoreConfig cfg_;
    std::vector<Block> blocks_;
    uint32_t total_tokens_ = 0;
};

// kvmem_backend.hpp:11-27 (slot hooks; block bytes move in batches through
// the reselect engine instead of one copy call per block).
class KvMemBackend {
public:
    virtual ~KvMemBackend() = default;
    virtual int32_t alloc_gpu_slot() { return -1; }
    virtual void free_gpu_slot(int32_t /*slot*/) {}
    // Slots alloc_gpu_slot can still hand out (the adapter's
    // free_slots_.size()).
    virtual uint32_t free_slot_count() const { return 0; }
    // A block entered `slot` (called once per staged block, ascending ids).
    virtual void block_staged_in(uint32_t /*block_id*/, int32_t /*slot*/) {}
};

// LIFO slot free list of the adapter (llama-memory-kvmem.cpp:621-627
// reset_slots, :693-707 alloc_slot / free_slot): slot 0 is handed out
// first, a freed slot is the next one handed out.
class SlotPool final : public KvMemBackend {
public:
    explicit SlotPool(uint32_t n_slots);
    int32_t alloc_gpu_slot() override;
    void free_gpu_slot(int32_t slot) override;
    uint32_t free_slot_count() const override { return n_free(); }
    uint32_t n_slots() const { return n_slots_; }
    uint32_t n_free() const { return static_cast<uint32_t>(free_.size()); }
    void reset();

private:
    uint32_t n_slots_;
    std::vector<int32_t> free_;
};

// kvmem_runtime.hpp:28-100 / kvmem_runtime.cpp:104-113, 212-236, 294-328:
// the stage-out-before-stage-in ordering and the slot plan, with no
// lower tiers (a block leaving the GPU keeps its host history copy).
class KvMemRuntime {
public:
    KvMemRuntime(StoreConfig cfg, KvMemBackend *backend);

    KvMemStore &store() { return store_; }
    const KvMemStore &store() const { return store_; }
    const Plan &last_plan() const { return last_plan_; }
    bool pending() const { return pending_; }

    void register_append(uint32_t n_tokens) { store_.register_append(n_tokens); }
    std::vector<uint32_t> truncate_to(uint32_t token_pos);

    std::vector<uint32_t> preview_reselect(const std::vector<uint32_t> &mandatory = {},
                                           const Ranker &ranker = nullptr) const;
    Plan prepare_selection(const std::vector<uint32_t> &selected);
    bool commit_resident_selection(const std::vector<uint32_t> &selected);
    // Rows the caller writes into the pool itself, as llama.cpp's decode
    // writes the K/V cells of a batch: register_append, then every block
    // the new rows touch that has no slot gets one from the free list
    // (prepare_working_set with the working set pinned,
    // llama-memory-kvmem.cpp:1256-1337).  Refused (false, nothing changed)
    // while a plan is pending or when the free list is short; `placed`
    // receives the blocks given a slot.
    bool append_resident(uint32_t n_tokens, std::vector<uint32_t> *placed);
    void spill_outgoing();
    void admit_incoming();
    void finish_reselect();

private:
    KvMemStore store_;
    KvMemBackend *backend_;
    Plan last_plan_;
    bool pending_ = false;
    std::vector<int32_t> pending_frees_;
};

// ------------------------------------------------- continuation checks

// llama_kvmem_attention_view (src/adapter/llama-kvmem-hooks.h:143-148): the
// blocks attention reads (every block holding a pool slot, in block order),
// the attention epoch and history rows it was taken at, and whether every
// one of them has all its rows in the pool (and, canonical, block i of the
// view in slot i).
struct AttentionView {
    uint64_t epoch = 0;
    uint32_t rows = 0;
    bool valid = false;
    std::vector<uint32_t> blocks;
};

// What the checks need of the pool beside the store: the attention epoch
// (bumped whenever pool contents or residency change, never by appended
// rows: the adapter's attention_epoch_), the slot count and free slots, and
// whether a block's rows are all in the pool (gpu_kv_complete,
// llama-memory-kvmem.cpp:2964-2980; called for blocks holding a slot).
struct PoolState {
    uint64_t epoch = 0;
    uint32_t n_slots = 0;
    uint32_t n_free = 0;
    std::function<bool(const Block &)> complete;
};

// attention_view (llama-memory-kvmem.cpp:2982-3000).
AttentionView attention_view(const KvMemStore &s, const PoolState &p, bool canonical);
// selection_fits (llama-memory-kvmem.cpp:3069-3084): the selection is
// current, keeps every mandatory block, and with the rows up to end plus
// generation_rows fits the slot pool.
bool selection_fits(const KvMemStore &s, const PoolState &p, const std::vector<uint32_t> &mandatory,
                    uint64_t sel_epoch, uint32_t sel_rows, const std::vector<uint32_t> &sel,
                    uint32_t end, uint32_t generation_rows);
// commit_unchanged (llama-memory-kvmem.cpp:3086-3096): the attention view
// taken before (same epoch, no more rows) is kept by the current one, which
// equals the selection; then commit_resident_selection.
bool commit_unchanged(KvMemRuntime &rt, const PoolState &p, const AttentionView &before,
                      uint64_t sel_epoch, uint32_t sel_rows, const std::vector<uint32_t> &sel);
// commit_resident (llama-memory-kvmem.cpp:3098-3102).
bool commit_resident(KvMemRuntime &rt, const PoolState &p, bool canonical);
// query_replay_fits (llama-memory-kvmem.cpp:3502-3524): whether replaying
// the query rows [query_begin, prompt_end) fits the selection budget beside
// the sink blocks (true with no budget or an empty query).
bool query_replay_fits(const KvMemStore &s, uint32_t query_begin, uint32_t prompt_end);
// can_append (llama-memory-kvmem.cpp:3002-3024): whether rows up to end
// plus generation_rows can be decoded onto the current pool without a
// reselect; *reason receives the adapter's reason string.
bool can_append(const KvMemStore &s, const PoolState &p, uint32_t end, uint32_t generation_rows,
                bool all_history, const char **reason);

}  // namespace kvmem_amd
