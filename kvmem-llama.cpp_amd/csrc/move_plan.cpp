// Slot-move planning (see move_plan.hpp).
#include "move_plan.hpp"

#include <algorithm>

namespace kvmem_hip {

bool build_chains(const uint32_t *src, const uint32_t *dst, const uint32_t *n_tokens, uint32_t n,
                  uint32_t T, uint32_t n_slots, std::vector<ChainSeg> &segs, std::vector<uint32_t> &saved) {
    std::vector<int32_t> from(n_slots, -1), into(n_slots, -1);
    std::vector<uint32_t> keep;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t nt = n_tokens ? n_tokens[i] : T;
        if (nt == 0) {
            continue;
        }
        if (from[src[i]] >= 0 || into[dst[i]] >= 0) {
            return false;
        }
        from[src[i]] = static_cast<int32_t>(i);
        into[dst[i]] = static_cast<int32_t>(i);
        if (src[i] != dst[i]) {
            keep.push_back(i);
        }
    }
    for (uint32_t i = 0; i < n; ++i) {  // self-moves leave the chain maps
        const uint32_t nt = n_tokens ? n_tokens[i] : T;
        if (nt != 0 && src[i] == dst[i]) {
            from[src[i]] = -1;
            into[dst[i]] = -1;
        }
    }
    std::vector<uint8_t> done(n, 0);
    std::vector<uint32_t> chain;
    auto emit = [&](bool cycle) {
        const uint32_t k = static_cast<uint32_t>(chain.size());
        for (uint32_t g0 = 0; g0 < k; g0 += kChainSeg) {
            ChainSeg sg{};
            sg.len = std::min<uint32_t>(kChainSeg, k - g0);
            for (uint32_t j = 0; j < sg.len; ++j) {
                const uint32_t m = chain[g0 + j];
                sg.slot[j] = src[m];
                sg.slot[j + 1] = dst[m];
                sg.nt[j] = n_tokens ? n_tokens[m] : T;
            }
            sg.saved = -1;
            if (g0 > 0 || cycle) {
                sg.saved = static_cast<int32_t>(saved.size());
                saved.push_back(sg.slot[0]);
            }
            segs.push_back(sg);
        }
    };
    for (uint32_t i : keep) {  // chains start at a source no move writes
        if (into[src[i]] >= 0) {
            continue;
        }
        chain.clear();
        for (int32_t m = static_cast<int32_t>(i); m >= 0; m = from[dst[m]]) {
            chain.push_back(static_cast<uint32_t>(m));
            done[m] = 1;
        }
        emit(false);
    }
    for (uint32_t i : keep) {  // what is left are cycles
        if (done[i]) {
            continue;
        }
        chain.clear();
        for (int32_t m = static_cast<int32_t>(i); !done[m]; m = from[dst[m]]) {
            chain.push_back(static_cast<uint32_t>(m));
            done[m] = 1;
        }
        emit(true);
    }
    return true;
}

}  // namespace kvmem_hip
