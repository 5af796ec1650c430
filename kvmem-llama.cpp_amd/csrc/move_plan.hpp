// Slot-move planning: a set of pool slot moves with distinct sources and
// distinct destinations is a set of chains (s0 -> s1 -> ... -> sk) and
// cycles.  They are cut into segments of at most kChainSeg moves that the
// device walks with no synchronisation (move_chain_kernel in stagein.hip):
// one thread reads every source of its segment, then writes every
// destination.  The first source of every segment but a chain's first, and
// a cycle's first source, is overwritten by another segment, so it is saved
// to scratch before the walk and read from there.
//
// Host-only C++ (no HIP), so the planner is tested on its own on the CPU.
#pragma once

#include <cstdint>
#include <vector>

namespace kvmem_hip {

constexpr int kChainSeg = 8;

struct ChainSeg {
    uint32_t slot[kChainSeg + 1];  // move j: slot[j] -> slot[j + 1]
    uint32_t nt[kChainSeg];        // rows move j carries
    uint32_t len;                  // moves in the segment
    int32_t saved;                 // >= 0: slot[0]'s rows are this scratch entry
};

static_assert(sizeof(ChainSeg) == 76, "upload_bytes_for counts 76-byte chain segments");

// Segments of the moves src[i] -> dst[i] that carry rows (n_tokens[i] rows,
// every one of block_tokens when n_tokens is null; slots < n_slots), and in
// `saved` the slots to save first (entry e of scratch holds saved[e]).
// Returns false when two moves that carry rows share a source or a
// destination (self-moves included); the caller then gathers and scatters.
// Self-moves are dropped: their slot is neither read nor written by any
// other move.  Unused slot/nt entries of a segment are zero.
bool build_chains(const uint32_t *src, const uint32_t *dst, const uint32_t *n_tokens, uint32_t n,
                  uint32_t block_tokens, uint32_t n_slots, std::vector<ChainSeg> &segs,
                  std::vector<uint32_t> &saved);

}  // namespace kvmem_hip
