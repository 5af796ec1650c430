// Fuzz of the slot-move planner (kvmem-llama.cpp_amd/csrc/move_plan.cpp).
//
// For random move sets (permutations with chains, cycles and self-moves,
// partial token counts, and sets with shared sources or destinations) the
// planned segments, replayed the way the device kernel runs them (each
// segment: every load, then every store; segments interleaved at random;
// one row at a time), must leave the slots as "read every source, then
// write every destination in list order" does.  Also checked: the planner
// refuses exactly the sets with a shared source or destination among the
// moves that carry rows, segments hold 1..kChainSeg moves, and a segment's
// slots are distinct except a cycle's closing slot, which is read from
// scratch.  Prints "cases C refused R bad B"; exit status 1 when B > 0.
#include "move_plan.hpp"

#include <algorithm>
#include <cstdio>
#include <random>
#include <set>

using kvmem_hip::ChainSeg;
using kvmem_hip::kChainSeg;

int main(int argc, char **argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
    std::mt19937 g(7);
    int bad = 0, refused = 0, cases = 0;
    for (int it = 0; it < iters; ++it) {
        const uint32_t n_slots = 1 + g() % 48, T = 1 + g() % 6;
        std::vector<uint32_t> ps(n_slots), pd(n_slots);
        for (uint32_t i = 0; i < n_slots; ++i) ps[i] = pd[i] = i;
        std::shuffle(ps.begin(), ps.end(), g);
        const int kind = g() % 6;
        std::vector<uint32_t> src, dst;
        if (kind == 0) {  // a cycle over a random subset, in random order
            const uint32_t k = 1 + g() % n_slots;
            for (uint32_t i = 0; i < k; ++i) { src.push_back(ps[i]); dst.push_back(ps[(i + 1) % k]); }
        } else if (kind == 1) {  // one long chain
            for (uint32_t i = 0; i + 1 < n_slots; ++i) { src.push_back(ps[i]); dst.push_back(ps[i + 1]); }
        } else if (kind == 5) {  // arbitrary (often shared) sources and destinations
            const uint32_t n = g() % (n_slots + 3);
            for (uint32_t i = 0; i < n; ++i) { src.push_back(g() % n_slots); dst.push_back(g() % n_slots); }
        } else {  // a random partial permutation: chains, cycles, self-moves
            std::shuffle(pd.begin(), pd.end(), g);
            const uint32_t n = g() % (n_slots + 1);
            for (uint32_t i = 0; i < n; ++i) { src.push_back(ps[i]); dst.push_back(pd[i]); }
        }
        const uint32_t n = static_cast<uint32_t>(src.size());
        std::vector<uint32_t> perm(n);
        for (uint32_t i = 0; i < n; ++i) perm[i] = i;
        std::shuffle(perm.begin(), perm.end(), g);
        std::vector<uint32_t> s2(n), d2(n), nt(n);
        for (uint32_t i = 0; i < n; ++i) { s2[i] = src[perm[i]]; d2[i] = dst[perm[i]]; nt[i] = g() % 3 ? T : g() % (T + 1); }
        ++cases;
        // expected refusal: a shared source or destination among moves with rows
        std::set<uint32_t> ss, dd;
        bool shared = false;
        for (uint32_t i = 0; i < n; ++i) {
            if (nt[i] == 0) continue;
            shared |= !ss.insert(s2[i]).second || !dd.insert(d2[i]).second;
        }
        std::vector<ChainSeg> segs;
        std::vector<uint32_t> saved;
        const bool ok = kvmem_hip::build_chains(s2.data(), d2.data(), nt.data(), n, T, n_slots, segs, saved);
        if (ok == shared) { ++bad; if (bad < 5) printf("it %d: refusal %d, shared %d\n", it, !ok, shared); continue; }
        if (!ok) { ++refused; continue; }
        for (const ChainSeg &sg : segs) {
            std::set<uint32_t> seen;
            bool distinct = true;
            for (uint32_t j = 0; j <= sg.len; ++j) {
                const bool closing = j == sg.len && sg.saved >= 0 && sg.slot[j] == sg.slot[0];
                if (!closing) distinct &= seen.insert(sg.slot[j]).second;
            }
            if (sg.len < 1 || sg.len > static_cast<uint32_t>(kChainSeg) || !distinct ||
                (sg.saved >= 0 && static_cast<size_t>(sg.saved) >= saved.size()) ||
                (sg.saved >= 0 && saved[sg.saved] != sg.slot[0])) {
                ++bad; if (bad < 5) printf("it %d: bad segment\n", it);
            }
        }
        // reference: read every source, then write every destination in order
        std::vector<int> mem(n_slots * T);
        for (size_t i = 0; i < mem.size(); ++i) mem[i] = static_cast<int>(i) * 7 + 1;
        std::vector<int> ref = mem, out = mem;
        {
            std::vector<std::vector<int>> rows(n);
            for (uint32_t i = 0; i < n; ++i)
                for (uint32_t r = 0; r < nt[i]; ++r) rows[i].push_back(mem[s2[i] * T + r]);
            for (uint32_t i = 0; i < n; ++i)
                for (uint32_t r = 0; r < nt[i]; ++r) ref[d2[i] * T + r] = rows[i][r];
        }
        std::vector<int> scratch(saved.size() * T);
        for (size_t e = 0; e < saved.size(); ++e)
            for (uint32_t r = 0; r < T; ++r) scratch[e * T + r] = mem[saved[e] * T + r];
        for (uint32_t r = 0; r < T; ++r) {
            std::vector<int> phase(segs.size(), 0);
            std::vector<std::vector<int>> vals(segs.size(), std::vector<int>(kChainSeg));
            size_t live = segs.size();
            while (live) {
                const size_t si = g() % segs.size();
                if (phase[si] == 2) continue;
                const ChainSeg &sg = segs[si];
                if (phase[si] == 0) {  // the device loads every source row, rows past nt included
                    for (uint32_t j = 0; j < sg.len; ++j)
                        vals[si][j] = (j == 0 && sg.saved >= 0) ? scratch[sg.saved * T + r] : out[sg.slot[j] * T + r];
                    phase[si] = 1;
                } else {
                    for (uint32_t j = 0; j < sg.len; ++j)
                        if (r < sg.nt[j]) out[sg.slot[j + 1] * T + r] = vals[si][j];
                    phase[si] = 2;
                    --live;
                }
            }
        }
        if (out != ref) { ++bad; if (bad < 5) printf("it %d: slots differ (n %u, slots %u, T %u)\n", it, n, n_slots, T); }
    }
    printf("cases %d refused %d bad %d\n", cases, refused, bad);
    return bad ? 1 : 0;
}
