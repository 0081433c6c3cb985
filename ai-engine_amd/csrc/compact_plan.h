// compact_plan.h -- host planning of in-place block compaction (no HIP:
// also built on its own, with the sanitizers, by the CPU tests).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace pkv {

// Bytes of the largest plan for a pool of n blocks.
size_t plan_capacity_bytes(size_t n);

// Decomposes the moves src[i] -> dst[i] (block ids in [0, num_blocks), no
// source or destination twice) into chains and cycles that one thread per
// byte range can execute in order, in place.  ops holds (src, dst) pairs;
// chain c is ops pairs starts[c] .. starts[c + 1] - 1.  src == -1 reads the
// chain's held copy, dst == -1 stores into it (a cycle parks one block first
// and restores it last).  Moves onto themselves are dropped.  Every block
// occurs in at most one chain.  Returns false with the reason in why on an
// id out of range or a repeated source or destination.
bool plan_compaction(int num_blocks, const int32_t* src, const int32_t* dst, int n,
                     std::vector<int32_t>& ops, std::vector<int32_t>& starts, std::string& why);

}  // namespace pkv
