// Host block table, top-k selection, selection diff and slot plan of the
// reselect step.  Behaviour follows the reference host library file:line
// cited on each function; the code is written for this library.
#include "kvmem_store.hpp"

#include <algorithm>
#include <cstdlib>

namespace kvmem_amd {

namespace {

uint64_t abs_diff(int64_t a, int64_t b) {
    return static_cast<uint64_t>(a > b ? a - b : b - a);
}

}  // namespace

// ------------------------------------------------------------ block table

void KvMemStore::register_append(uint32_t n_new_tokens) {
    const uint32_t bt = cfg_.block_tokens;
    uint32_t left = n_new_tokens;
    if (left && !blocks_.empty() && blocks_.back().n_tokens < bt) {
        Block &tail = blocks_.back();
        const uint32_t add = std::min(bt - tail.n_tokens, left);
        tail.n_tokens += add;
        total_tokens_ += add;
        left -= add;
    }
    while (left) {
        Block b;
        b.block_id = block_count();
        b.orig_pos_start = total_tokens_;
        b.n_tokens = std::min(bt, left);
        b.baked_pos = b.orig_pos_start;
        total_tokens_ += b.n_tokens;
        left -= b.n_tokens;
        blocks_.push_back(b);
    }
}

std::vector<uint32_t> KvMemStore::truncate_to(uint32_t token_pos) {
    std::vector<uint32_t> dropped;
    if (token_pos >= total_tokens_) {
        return dropped;
    }
    while (!blocks_.empty() && blocks_.back().orig_pos_start >= token_pos) {
        dropped.push_back(blocks_.back().block_id);
        total_tokens_ -= blocks_.back().n_tokens;
        blocks_.pop_back();
    }
    if (!blocks_.empty() && blocks_.back().orig_pos_end() > token_pos) {
        Block &tail = blocks_.back();
        const uint32_t keep = token_pos - tail.orig_pos_start;
        total_tokens_ -= tail.n_tokens - keep;
        tail.n_tokens = keep;
    }
    return dropped;
}

void KvMemStore::set_retrieval_scores(const std::vector<double> &scores) {
    for (Block &b : blocks_) {
        b.retrieval_score = b.block_id < scores.size() ? scores[b.block_id] : 0.0;
    }
}

void KvMemStore::set_block_tier(uint32_t id, Tier tier) {
    if (id >= block_count()) {
        return;
    }
    blocks_[id].tier = tier;
    if (tier != Tier::GPU) {
        blocks_[id].gpu_slot = -1;
    }
}

void KvMemStore::set_block_gpu_slot(uint32_t id, int32_t slot) {
    if (id < block_count()) {
        blocks_[id].gpu_slot = slot;
    }
}

int32_t KvMemStore::block_id_containing(uint32_t pos) const {
    if (blocks_.empty() || pos >= total_tokens_) {
        return -1;
    }
    const uint32_t guess = std::min(pos / cfg_.block_tokens, block_count() - 1);
    const Block &g = blocks_[guess];
    if (pos >= g.orig_pos_start && pos < g.orig_pos_end()) {
        return static_cast<int32_t>(guess);
    }
    for (const Block &b : blocks_) {
        if (pos >= b.orig_pos_start && pos < b.orig_pos_end()) {
            return static_cast<int32_t>(b.block_id);
        }
    }
    return -1;
}

std::vector<uint32_t> KvMemStore::blocks_overlapping(
    const std::vector<std::pair<int32_t, int32_t>> &ranges, int32_t force_pos) const {
    std::vector<uint32_t> out;
    for (const Block &b : blocks_) {
        for (const auto &r : ranges) {
            if (static_cast<int64_t>(b.orig_pos_end()) > r.first &&
                static_cast<int64_t>(b.orig_pos_start) < r.second) {
                out.push_back(b.block_id);
                break;
            }
        }
    }
    if (force_pos >= 0) {
        const int32_t id = block_id_containing(static_cast<uint32_t>(force_pos));
        if (id >= 0) {
            out.push_back(static_cast<uint32_t>(id));
        }
    }
    return out;
}

// ---------------------------------------------------------------- top-k

TopkCharge KvMemStore::charge_topk(const std::vector<uint32_t> &mandatory) const {
    TopkCharge c;
    const uint32_t n = block_count();
    const uint32_t budget = budget_blocks();
    if (n == 0) {
        return c;
    }
    if (budget == 0 || n <= budget) {
        c.all_fit = true;
        return c;
    }
    std::vector<uint8_t> charged(n, 0);
    auto charge = [&](uint32_t id) {
        if (id < n && !charged[id] && c.forced.size() < budget) {
            charged[id] = 1;
            c.forced.push_back(id);
        }
    };
    for (uint32_t i = 0; i < std::min(cfg_.sink_blocks, n); ++i) {
        charge(i);
    }
    for (auto it = mandatory.rbegin(); it != mandatory.rend(); ++it) {
        charge(*it);
    }
    for (uint32_t i = 0; i < std::min(cfg_.recent_blocks, n); ++i) {
        charge(n - 1 - i);
    }
    c.need = budget - static_cast<uint32_t>(c.forced.size());
    return c;
}

std::vector<uint32_t> KvMemStore::pick_topk_blocks(const std::vector<uint32_t> &mandatory,
                                                   const Ranker &ranker) const {
    const uint32_t n = block_count();
    std::vector<uint32_t> out;
    const TopkCharge c = charge_topk(mandatory);
    if (n == 0) {
        return out;
    }
    if (c.all_fit) {
        out.resize(n);
        for (uint32_t i = 0; i < n; ++i) {
            out[i] = i;
        }
        return out;
    }
    std::vector<uint8_t> keep(n, 0);
    for (uint32_t id : c.forced) {
        keep[id] = 1;
    }
    const uint32_t candidates = n - static_cast<uint32_t>(c.forced.size());
    const uint32_t need = std::min(c.need, candidates);
    if (need > 0) {
        std::vector<uint32_t> best;
        if (ranker) {
            best = ranker(keep, need);
        } else {
            // strict total order: higher score first, then the tie rule
            const bool lower_first = cfg_.tie_lower_index;
            auto before = [&](uint32_t a, uint32_t b) {
                const double sa = blocks_[a].retrieval_score;
                const double sb = blocks_[b].retrieval_score;
                if (sa != sb) {
                    return sa > sb;
                }
                return lower_first ? a < b : a > b;
            };
            best.reserve(candidates);
            for (uint32_t i = 0; i < n; ++i) {
                if (!keep[i]) {
                    best.push_back(i);
                }
            }
            std::partial_sort(best.begin(), best.begin() + need, best.end(), before);
            best.resize(need);
        }
        for (uint32_t id : best) {
            if (id < n) {
                keep[id] = 1;
            }
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (keep[i]) {
            out.push_back(i);
        }
    }
    return out;
}

// ------------------------------------------------------------------ diff

Plan KvMemStore::set_selection(std::vector<uint32_t> ids) {
    const uint32_t n = block_count();
    std::sort(ids.begin(), ids.end());
    ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
    ids.erase(std::remove_if(ids.begin(), ids.end(), [n](uint32_t id) { return id >= n; }),
              ids.end());

    Plan plan;
    std::vector<uint8_t> selected(n, 0);
    for (uint32_t id : ids) {
        selected[id] = 1;
    }
    std::vector<uint8_t> was_ws(n, 0);
    for (const Block &b : blocks_) {
        was_ws[b.block_id] = b.in_working_set;
        plan.selection_overlap_blocks += (b.in_working_set && selected[b.block_id]) ? 1u : 0u;
    }
    const bool reload_all = !cfg_.optimize_stage_in;

    // outgoing: GPU-tier blocks the new selection drops (all of them on a
    // forced full reload), in id order
    for (Block &b : blocks_) {
        if (b.tier == Tier::GPU && (reload_all || !selected[b.block_id])) {
            plan.stage_out.push_back(b.block_id);
            b.in_working_set = false;
        }
    }

    // window order = ascending id, packed from position 0
    int64_t pos = 0;
    for (uint32_t id : ids) {
        Block &b = blocks_[id];
        const bool on_gpu = b.tier == Tier::GPU;
        if (was_ws[id] && on_gpu) {
            if (b.baked_pos == pos) {
                ++plan.retained_position_stable;
            } else {
                ++plan.retained_position_moved;
            }
            if (!reload_all) {
                ++plan.gpu_reused_blocks;
            }
        }
        if (!b.in_working_set) {
            plan.stage_in.push_back(id);
        }
        Remap r;
        r.block_id = id;
        r.n_tokens = b.n_tokens;
        r.from_base = static_cast<int32_t>(b.baked_pos);
        r.to_base = static_cast<int32_t>(pos);
        r.working_k_resident = on_gpu && !reload_all;
        r.skip = b.baked_pos == pos;
        plan.remaps.push_back(r);
        if (!r.skip) {
            ++b.remap_count;
            b.remap_abs_delta += abs_diff(b.baked_pos, pos);
        }
        b.in_working_set = true;
        b.baked_pos = pos;
        pos += b.n_tokens;
    }
    plan.total_window_tokens = static_cast<uint32_t>(pos);
    return plan;
}

bool KvMemStore::commit_resident_selection(const std::vector<uint32_t> &ids) {
    std::vector<uint32_t> resident;
    for (const Block &b : blocks_) {
        if (b.gpu_slot < 0 || b.n_tokens == 0) {
            continue;
        }
        if (b.tier != Tier::GPU) {
            return false;
        }
        resident.push_back(b.block_id);
    }
    if (resident != ids) {
        return false;
    }
    for (Block &b : blocks_) {
        b.in_working_set = b.gpu_slot >= 0 && b.n_tokens > 0;
    }
    return true;
}

bool KvMemStore::prefill_needs_offload(uint32_t resident_tokens, uint32_t incoming_tokens,
                                       uint32_t pool_tokens) const {
    if (incoming_tokens == 0 || pool_tokens == 0) {
        return false;
    }
    const uint64_t next = static_cast<uint64_t>(resident_tokens) + incoming_tokens;
    if (next > pool_tokens) {
        return true;
    }
    double r = cfg_.gpu_high_watermark;
    if (r <= 0.0 || r > 1.0) {
        r = 1.0;
    }
    const uint32_t high = std::max(static_cast<uint32_t>(pool_tokens * r), cfg_.block_tokens);
    return next > high;
}

void KvMemStore::clear_working_set() {
    for (Block &b : blocks_) {
        b.in_working_set = false;
    }
}

void KvMemStore::drop_from_working_set(uint32_t id) {
    if (id < block_count()) {
        blocks_[id].in_working_set = false;
    }
}

// ------------------------------------------------------------ slot pool

SlotPool::SlotPool(uint32_t n_slots) : n_slots_(n_slots) {
    reset();
}

void SlotPool::reset() {
    free_.clear();
    free_.reserve(n_slots_);
    for (uint32_t i = n_slots_; i > 0; --i) {
        free_.push_back(static_cast<int32_t>(i - 1));
    }
}

int32_t SlotPool::alloc_gpu_slot() {
    if (free_.empty()) {
        return -1;
    }
    const int32_t s = free_.back();
    free_.pop_back();
    return s;
}

void SlotPool::free_gpu_slot(int32_t slot) {
    if (slot >= 0) {
        free_.push_back(slot);
    }
}

// --------------------------------------------------------------- runtime

KvMemRuntime::KvMemRuntime(StoreConfig cfg, KvMemBackend *backend)
    : store_(cfg), backend_(backend) {
    if (!backend_) {
        throw std::invalid_argument("KvMemRuntime needs a backend");
    }
}

std::vector<uint32_t> KvMemRuntime::truncate_to(uint32_t token_pos) {
    std::vector<int32_t> slots;
    for (const Block &b : store_.blocks()) {
        if (b.orig_pos_start >= token_pos && b.gpu_slot >= 0) {
            slots.push_back(b.gpu_slot);
        }
    }
    std::vector<uint32_t> dropped = store_.truncate_to(token_pos);
    for (int32_t s : slots) {
        backend_->free_gpu_slot(s);
    }
    return dropped;
}

std::vector<uint32_t> KvMemRuntime::preview_reselect(const std::vector<uint32_t> &mandatory,
                                                     const Ranker &ranker) const {
    return store_.pick_topk_blocks(mandatory, ranker);
}

Plan KvMemRuntime::prepare_selection(const std::vector<uint32_t> &selected) {
    last_plan_ = store_.set_selection(selected);
    pending_ = true;
    return last_plan_;
}

bool KvMemRuntime::commit_resident_selection(const std::vector<uint32_t> &selected) {
    if (pending_ || !store_.commit_resident_selection(selected)) {
        return false;
    }
    last_plan_ = Plan{};
    for (uint32_t id : selected) {
        last_plan_.total_window_tokens += store_.blocks()[id].n_tokens;
    }
    return true;
}

bool KvMemRuntime::append_resident(uint32_t n_tokens, std::vector<uint32_t> *placed) {
    if (placed) {
        placed->clear();
    }
    if (pending_) {
        return false;
    }
    if (n_tokens == 0) {
        return true;
    }
    // blocks the new rows [t0, t0 + n_tokens) touch: the partial tail, then
    // the new ones
    const uint32_t bt = store_.config().block_tokens;
    const uint32_t t0 = store_.total_tokens();
    const auto &bl = store_.blocks();
    uint32_t need = 0;
    const bool tail_partial = !bl.empty() && bl.back().n_tokens < bt;
    if (tail_partial && bl.back().gpu_slot < 0) {
        ++need;
    }
    const uint32_t into_tail = tail_partial ? std::min(bt - bl.back().n_tokens, n_tokens) : 0u;
    need += (n_tokens - into_tail + bt - 1) / bt;
    if (need > backend_->free_slot_count()) {
        return false;
    }
    store_.register_append(n_tokens);
    for (const Block &b : store_.blocks()) {
        if (b.orig_pos_end() <= t0 || b.gpu_slot >= 0) {
            continue;
        }
        const int32_t slot = backend_->alloc_gpu_slot();
        store_.set_block_tier(b.block_id, Tier::GPU);
        store_.set_block_gpu_slot(b.block_id, slot);
        if (placed) {
            placed->push_back(b.block_id);
        }
    }
    return true;
}

void KvMemRuntime::spill_outgoing() {
    if (!pending_) {
        return;
    }
    pending_frees_.clear();
    for (uint32_t id : last_plan_.stage_out) {
        const int32_t slot = store_.blocks()[id].gpu_slot;
        store_.set_block_tier(id, Tier::CPU);   // the host history keeps the block
        if (slot >= 0) {
            pending_frees_.push_back(slot);
        }
    }
}

void KvMemRuntime::admit_incoming() {
    if (!pending_) {
        return;
    }
    for (int32_t s : pending_frees_) {
        backend_->free_gpu_slot(s);
    }
    pending_frees_.clear();
    for (uint32_t id : last_plan_.stage_in) {
        const Block &b = store_.blocks()[id];
        if (b.tier == Tier::GPU && b.gpu_slot >= 0) {
            continue;  // still resident (only a working-set transition)
        }
        const int32_t slot = backend_->alloc_gpu_slot();
        store_.set_block_tier(id, Tier::GPU);
        store_.set_block_gpu_slot(id, slot);
        if (slot >= 0) {
            backend_->block_staged_in(id, slot);
        }
    }
    pending_ = false;
}

void KvMemRuntime::finish_reselect() {
    spill_outgoing();
    admit_incoming();
}

// ------------------------------------------------- continuation checks

namespace {

bool holds(const std::vector<uint32_t> &sorted, uint32_t id) {
    return std::binary_search(sorted.begin(), sorted.end(), id);
}

// gpu_kv_complete (llama-memory-kvmem.cpp:2964-2980) for block id.
bool block_complete(const KvMemStore &s, const PoolState &p, uint64_t id) {
    if (id >= s.block_count()) {
        return false;
    }
    const Block &b = s.blocks()[id];
    return b.gpu_slot >= 0 && b.tier == Tier::GPU && b.n_tokens > 0 && p.complete && p.complete(b);
}

}  // namespace

AttentionView attention_view(const KvMemStore &s, const PoolState &p, bool canonical) {
    AttentionView v;
    v.epoch = p.epoch;
    v.rows = s.total_tokens();
    v.valid = s.config().optimize_stage_in;
    for (const Block &b : s.blocks()) {
        if (b.gpu_slot < 0 || b.n_tokens == 0) {
            continue;
        }
        if ((canonical && b.gpu_slot != static_cast<int32_t>(v.blocks.size())) ||
            !block_complete(s, p, b.block_id)) {
            v.valid = false;
        }
        v.blocks.push_back(b.block_id);
    }
    return v;
}

bool selection_fits(const KvMemStore &s, const PoolState &p, const std::vector<uint32_t> &mandatory,
                    uint64_t sel_epoch, uint32_t sel_rows, const std::vector<uint32_t> &sel,
                    uint32_t end, uint32_t generation_rows) {
    if (sel_epoch != p.epoch || sel_rows != s.total_tokens() || end < sel_rows) {
        return false;
    }
    std::vector<uint32_t> ids(sel);
    std::sort(ids.begin(), ids.end());
    // a selector that trimmed a mandatory range to its budget made a plan
    // unfit for continuation
    for (uint32_t id : mandatory) {
        if (!holds(ids, id)) {
            return false;
        }
    }
    const uint64_t bt = s.config().block_tokens;
    const uint64_t final_block = (static_cast<uint64_t>(end) + generation_rows + bt - 1) / bt;
    const uint64_t first = sel_rows / bt;
    if (final_block < first || final_block - first > p.n_slots) {
        return false;
    }
    uint64_t count = ids.size();
    for (uint64_t id = first; id < final_block; ++id) {
        if (!holds(ids, static_cast<uint32_t>(id))) {
            ++count;
        }
    }
    return count <= p.n_slots;
}

bool commit_unchanged(KvMemRuntime &rt, const PoolState &p, const AttentionView &before,
                      uint64_t sel_epoch, uint32_t sel_rows, const std::vector<uint32_t> &sel) {
    const KvMemStore &s = rt.store();
    if (!before.valid || before.epoch != p.epoch || before.rows > s.total_tokens() ||
        sel_epoch != p.epoch || sel_rows != s.total_tokens()) {
        return false;
    }
    const AttentionView after = attention_view(s, p, true);
    if (!after.valid || after.blocks != sel) {
        return false;
    }
    for (uint32_t id : before.blocks) {
        if (!holds(after.blocks, id)) {
            return false;
        }
    }
    return rt.commit_resident_selection(sel);
}

bool commit_resident(KvMemRuntime &rt, const PoolState &p, bool canonical) {
    const AttentionView v = attention_view(rt.store(), p, canonical);
    return v.valid && rt.commit_resident_selection(v.blocks);
}

bool query_replay_fits(const KvMemStore &s, uint32_t query_begin, uint32_t prompt_end) {
    if (query_begin >= prompt_end) {
        return true;
    }
    const uint64_t bt = std::max(1u, s.config().block_tokens);
    const uint64_t budget = s.budget_blocks();
    if (budget == 0) {
        return true;
    }
    const uint64_t total_blocks = (static_cast<uint64_t>(prompt_end) + bt - 1) / bt;
    const uint64_t boundary = query_begin / bt;
    if (boundary >= total_blocks) {
        return true;
    }
    const uint64_t sink = std::min<uint64_t>(s.config().sink_blocks, total_blocks);
    // the query blocks from the boundary on, plus the sink ahead of them
    const uint64_t required = boundary < sink ? total_blocks : sink + (total_blocks - boundary);
    return required <= budget;
}

bool can_append(const KvMemStore &s, const PoolState &p, uint32_t end, uint32_t generation_rows,
                bool all_history, const char **reason) {
    const char *why = nullptr;
    const uint64_t bt = s.config().block_tokens;
    const AttentionView v = attention_view(s, p, all_history);
    uint32_t resident_tokens = 0;
    for (const Block &b : s.blocks()) {
        if (b.gpu_slot >= 0) {
            resident_tokens += b.n_tokens;
        }
    }
    const uint64_t end_blocks = (static_cast<uint64_t>(end) + bt - 1) / bt;
    const uint64_t final_blocks = (static_cast<uint64_t>(end) + generation_rows + bt - 1) / bt;
    if (end < s.total_tokens()) {
        why = "invalid_boundary";
    } else if (!v.valid) {
        why = "coverage_or_layout";
    } else if (v.rows % bt && !block_complete(s, p, v.rows / bt)) {
        why = "partial_tail_missing";
    } else if (all_history && v.blocks.size() != s.block_count()) {
        why = "history_not_resident";
    } else if (all_history && s.budget_blocks() && end_blocks > s.budget_blocks()) {
        why = "selection_budget";
    } else if (all_history &&
               s.prefill_needs_offload(resident_tokens, end - v.rows,
                                       static_cast<uint32_t>(static_cast<uint64_t>(p.n_slots) * bt))) {
        why = "prefill_pressure";
    } else if (final_blocks > static_cast<uint64_t>(p.n_slots) + s.block_count()) {
        why = "insufficient_slots";
    } else {
        uint64_t needed = 0;
        for (uint64_t id = v.rows / bt; id < final_blocks; ++id) {
            if (id >= s.block_count() || s.blocks()[id].gpu_slot < 0) {
                ++needed;
            }
        }
        if (needed > p.n_free) {
            why = "insufficient_slots";
        }
    }
    if (reason) {
        *reason = why ? why : (all_history ? "all_resident" : "same_query");
    }
    return why == nullptr;
}

}  // namespace kvmem_amd
