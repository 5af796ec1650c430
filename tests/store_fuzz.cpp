// Randomized sequences over the host store, runtime and slot pool
// (csrc/kvmem_store.{hpp,cpp}), built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_cpu_store_sanitized.py.
//
// Each trial draws a store configuration (block size, budget, sink, recent,
// tie rule, forced reload) and a pool of more slots than the budget, then
// runs random operations: rows appended to the history, rows appended
// resident (KvMemRuntime::append_resident), truncations, reselects over
// random scores with random mandatory blocks (preview, prepare, stage-out
// then stage-in), commits of the resident set, and the continuation checks
// (attention_view, selection_fits, commit_unchanged, commit_resident,
// can_append, query_replay_fits) with random arguments.  After every
// operation:
//   - blocks tile the history: block i starts at i * block_tokens, only the
//     last one is partial, and their tokens add up to the total;
//   - slots held by blocks are distinct and in range, and with the free
//     list they account for every slot of the pool;
//   - no plan is left pending;
//   - after a reselect, the resident set is the selection: ascending, within
//     the budget, holding the sink and mandatory blocks whenever they fit it;
//   - an attention view lists exactly the blocks holding slots.
// Prints "ok" and exits 0, or names the trial, step and broken rule and
// exits 1.
#include "kvmem_store.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

using namespace kvmem_amd;

namespace {

int g_trial = 0;
int g_step = 0;

void expect(bool ok, const char *rule) {
    if (!ok) {
        std::fprintf(stderr, "trial %d step %d: %s\n", g_trial, g_step, rule);
        std::exit(1);
    }
}

std::vector<uint32_t> resident(const KvMemStore &s) {
    std::vector<uint32_t> out;
    for (const Block &b : s.blocks()) {
        if (b.gpu_slot >= 0) {
            out.push_back(b.block_id);
        }
    }
    return out;
}

void check_invariants(const KvMemRuntime &rt, const SlotPool &pool) {
    const KvMemStore &s = rt.store();
    const uint32_t bt = s.config().block_tokens;
    uint64_t sum = 0;
    const auto &bl = s.blocks();
    std::vector<uint8_t> used(pool.n_slots(), 0);
    uint32_t n_res = 0;
    for (size_t i = 0; i < bl.size(); ++i) {
        const Block &b = bl[i];
        expect(b.block_id == i, "block ids are their index");
        expect(b.orig_pos_start == i * bt, "block i starts at i * block_tokens");
        expect(b.n_tokens > 0 && b.n_tokens <= bt, "a block holds 1..block_tokens rows");
        expect(i + 1 == bl.size() || b.n_tokens == bt, "only the last block is partial");
        sum += b.n_tokens;
        if (b.gpu_slot >= 0) {
            expect(static_cast<uint32_t>(b.gpu_slot) < pool.n_slots(), "slot in range");
            expect(!used[b.gpu_slot], "slots are distinct");
            used[b.gpu_slot] = 1;
            ++n_res;
        }
    }
    expect(sum == s.total_tokens(), "block tokens add up to the total");
    expect(n_res + pool.n_free() == pool.n_slots(), "held and free slots account for the pool");
    expect(!rt.pending(), "no plan left pending");
}

PoolState pool_state(const SlotPool &pool, uint64_t epoch) {
    PoolState p;
    p.epoch = epoch;
    p.n_slots = pool.n_slots();
    p.n_free = pool.n_free();
    p.complete = [](const Block &b) { return b.tier == Tier::GPU && b.gpu_slot >= 0; };
    return p;
}

}  // namespace

int main(int argc, char **argv) {
    const uint64_t seed = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
    const int trials = argc > 2 ? std::atoi(argv[2]) : 40;
    const int steps = argc > 3 ? std::atoi(argv[3]) : 400;
    std::mt19937_64 rng(seed);
    auto pick = [&rng](uint64_t n) { return n ? rng() % n : 0; };
    uint64_t n_reselect = 0, n_commit_unchanged = 0, n_append_resident = 0;
    for (g_trial = 0; g_trial < trials; ++g_trial) {
        StoreConfig cfg;
        cfg.block_tokens = 8u << pick(3);
        const uint32_t budget_blocks = 2 + static_cast<uint32_t>(pick(10));
        cfg.select_budget = cfg.block_tokens * budget_blocks;
        cfg.sink_blocks = static_cast<uint32_t>(pick(3));
        cfg.recent_blocks = static_cast<uint32_t>(pick(3));
        cfg.tie_lower_index = pick(2) == 0;
        cfg.optimize_stage_in = pick(8) != 0;
        const uint32_t n_slots = budget_blocks + 1 + static_cast<uint32_t>(pick(6));
        SlotPool pool(n_slots);
        KvMemRuntime rt(cfg, &pool);
        uint64_t epoch = 0;  // the attention epoch: moves with every pool change
        const uint32_t bt = cfg.block_tokens;
        for (g_step = 0; g_step < steps; ++g_step) {
            KvMemStore &s = rt.store();
            const uint32_t total = s.total_tokens();
            switch (pick(9)) {
            case 0:
            case 1: {  // rows appended to the history only
                if (total < 4000) {
                    rt.register_append(static_cast<uint32_t>(pick(3 * bt)));
                }
                break;
            }
            case 2: {  // rows appended resident
                const std::vector<uint32_t> before = resident(s);
                std::vector<uint32_t> placed;
                const uint32_t n = static_cast<uint32_t>(pick(2 * bt));
                const bool ok = rt.append_resident(n, &placed);
                if (ok) {
                    n_append_resident += n > 0;
                    for (uint32_t id : placed) {
                        expect(s.blocks()[id].gpu_slot >= 0, "a placed block holds a slot");
                        expect(!std::binary_search(before.begin(), before.end(), id),
                               "only blocks without a slot are placed");
                    }
                    expect(s.total_tokens() == total + n, "append_resident adds its rows");
                } else {
                    expect(s.total_tokens() == total && resident(s) == before,
                           "a refused append_resident changes nothing");
                }
                break;
            }
            case 3: {  // truncation
                const uint32_t pos = static_cast<uint32_t>(pick(uint64_t{total} + 1));
                rt.truncate_to(pos);
                expect(s.total_tokens() == std::min(pos, total), "truncation sets the total");
                if (pos < total) {
                    ++epoch;
                }
                break;
            }
            case 4:
            case 5: {  // reselect over random scores
                const uint32_t nb = s.block_count();
                std::vector<double> scores(nb);
                for (double &x : scores) {
                    x = static_cast<double>(pick(1000)) / 7.0;  // ties happen
                }
                s.set_retrieval_scores(scores);
                std::vector<uint32_t> mand;
                for (uint64_t i = 0, m = pick(3); i < m && nb; ++i) {
                    mand.push_back(static_cast<uint32_t>(pick(nb)));
                }
                const std::vector<uint32_t> sel = rt.preview_reselect(mand);
                expect(std::is_sorted(sel.begin(), sel.end()) &&
                           std::adjacent_find(sel.begin(), sel.end()) == sel.end(),
                       "the selection is ascending and unique");
                expect(sel.size() <= (nb <= budget_blocks ? nb : budget_blocks), "the selection fits the budget");
                for (uint32_t i = 0; i < std::min(cfg.sink_blocks, nb) && nb > budget_blocks; ++i) {
                    if (i < budget_blocks) {
                        expect(std::binary_search(sel.begin(), sel.end(), i), "sink blocks are kept");
                    }
                }
                if (nb <= budget_blocks) {
                    expect(sel.size() == nb, "everything fits: every block is selected");
                } else {
                    std::vector<uint32_t> keep(mand);
                    for (uint32_t i = 0; i < std::min(cfg.sink_blocks, nb); ++i) {
                        keep.push_back(i);
                    }
                    std::sort(keep.begin(), keep.end());
                    keep.erase(std::unique(keep.begin(), keep.end()), keep.end());
                    if (keep.size() <= budget_blocks) {
                        for (uint32_t id : keep) {
                            expect(std::binary_search(sel.begin(), sel.end(), id),
                                   "sink and mandatory blocks that fit the budget are kept");
                        }
                    }
                }
                rt.prepare_selection(sel);
                rt.finish_reselect();
                expect(resident(s) == sel, "after a reselect the resident set is the selection");
                ++epoch;
                ++n_reselect;
                break;
            }
            case 6: {  // commit of the resident set
                const std::vector<uint32_t> res = resident(s);
                expect(rt.commit_resident_selection(res), "the resident set commits");
                std::vector<uint32_t> other = res;
                if (!other.empty()) {
                    other.pop_back();
                    expect(!rt.commit_resident_selection(other), "another set does not commit");
                }
                break;
            }
            case 7: {  // attention view, commit_unchanged, commit_resident
                const PoolState p = pool_state(pool, epoch);
                const bool canonical = pick(2) == 0;
                const AttentionView v = attention_view(s, p, canonical);
                expect(v.blocks == resident(s), "the view lists the blocks holding slots");
                expect(v.epoch == epoch && v.rows == total, "the view carries epoch and rows");
                std::vector<uint32_t> sel = v.blocks;
                if (pick(3) == 0 && !sel.empty()) {
                    sel.erase(sel.begin() + static_cast<long>(pick(sel.size())));
                }
                const AttentionView canon = attention_view(s, p, true);
                const bool want = v.valid && canon.valid && sel == canon.blocks;
                const bool ok = commit_unchanged(rt, p, v, epoch, total, sel);
                expect(ok == want, "commit_unchanged accepts exactly an unchanged view");
                n_commit_unchanged += ok;
                expect(!commit_unchanged(rt, p, v, epoch + 1, total, sel), "a stale selection is refused");
                expect(commit_resident(rt, p, canonical) == attention_view(s, p, canonical).valid,
                       "commit_resident follows the view");
                break;
            }
            case 8: {  // checks with random arguments
                const PoolState p = pool_state(pool, epoch);
                const uint32_t end = static_cast<uint32_t>(pick(uint64_t{total} + 2 * bt));
                const uint32_t gen = static_cast<uint32_t>(pick(4 * bt));
                const char *reason = nullptr;
                (void) can_append(s, p, end, gen, pick(2) == 0, &reason);
                expect(reason != nullptr, "can_append names a reason");
                const std::vector<uint32_t> res = resident(s);
                (void) selection_fits(s, p, {}, epoch, total, res, end, gen);
                expect(!selection_fits(s, p, {}, epoch + 1, total, res, end, gen),
                       "a stale selection does not fit");
                const uint32_t qb = static_cast<uint32_t>(pick(uint64_t{total} + 1));
                (void) query_replay_fits(s, qb, qb + static_cast<uint32_t>(pick(3 * bt)));
                (void) s.prefill_needs_offload(static_cast<uint32_t>(pick(4000)),
                                               static_cast<uint32_t>(pick(4000)), n_slots * bt);
                break;
            }
            default:
                break;
            }
            check_invariants(rt, pool);
        }
    }
    std::printf("ok: %d trials x %d steps, %llu reselects, %llu unchanged commits, %llu resident appends\n",
                trials, steps, static_cast<unsigned long long>(n_reselect),
                static_cast<unsigned long long>(n_commit_unchanged),
                static_cast<unsigned long long>(n_append_resident));
    return 0;
}
