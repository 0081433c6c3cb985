// compact_plan.cpp -- host planning of in-place block compaction (the
// block renumbering of pkv_compact; no reference counterpart).  Plain C++,
// no HIP.
#include "compact_plan.h"

#include <cstdio>

namespace pkv {

// Bytes of the largest plan for a pool of n blocks: at most n moves (2 ints
// each), at most n / 2 cycles (a cycle has >= 2 moves) adding 2 ops (4 ints)
// each, and one start per chain or cycle plus the end marker.
size_t plan_capacity_bytes(size_t n) { return (5 * n + 2) * sizeof(int32_t); }

// Moves m = (s -> d).  A move whose destination is still some other move's
// source must wait until that block has been read: the chain is built from
// a move whose dst is free, then repeatedly the move that fills the block
// just vacated.  Moves left over form cycles; each cycle first parks one
// block (dst = -1) and finally restores it (src = -1).
bool plan_compaction(int num_blocks, const int32_t* src, const int32_t* dst, int n,
                     std::vector<int32_t>& ops, std::vector<int32_t>& starts, std::string& why) {
  const int N = num_blocks;
  char buf[160];
  std::vector<int32_t> move_from(N > 0 ? N : 0, -1);  // move_from[d] = s
  std::vector<int32_t> move_to(N > 0 ? N : 0, -1);    // move_to[s] = d
  for (int i = 0; i < n; ++i) {
    int s = src[i], d = dst[i];
    if (s < 0 || s >= N || d < 0 || d >= N) {
      std::snprintf(buf, sizeof buf, "pair %d (%d -> %d) out of range [0, %d)", i, s, d, N);
      why = buf;
      return false;
    }
    if (move_to[s] != -1) {
      std::snprintf(buf, sizeof buf, "source block %d appears twice", s);
      why = buf;
      return false;
    }
    if (move_from[d] != -1) {
      std::snprintf(buf, sizeof buf, "destination block %d appears twice", d);
      why = buf;
      return false;
    }
    move_to[s] = d;
    move_from[d] = s;
  }
  std::vector<char> done(N, 0);  // indexed by source block
  starts.clear();
  ops.clear();
  for (int i = 0; i < n; ++i) {
    int s = src[i], d = dst[i];
    if (s == d) {
      done[s] = 1;
      continue;
    }
    if (move_to[d] != -1) continue;  // d is still someone's source: not a chain head
    starts.push_back((int32_t)(ops.size() / 2));
    // execute s -> d, then the move that fills s, and so on
    int cs = s, cd = d;
    while (true) {
      ops.push_back(cs);
      ops.push_back(cd);
      done[cs] = 1;
      int prev = move_from[cs];
      if (prev == -1 || prev == cs || done[prev]) break;
      cd = cs;
      cs = prev;
    }
  }
  for (int i = 0; i < n; ++i) {
    int s = src[i];
    if (done[s]) continue;
    // s lies on a cycle s -> d -> ... -> s.  Park the block that moves into
    // s's destination chain end: walk backwards from s.
    starts.push_back((int32_t)(ops.size() / 2));
    int first_dst = move_to[s];
    ops.push_back(first_dst);  // park first_dst's content (it moves on)
    ops.push_back(-1);
    int cs = s, cd = first_dst;
    while (true) {
      ops.push_back(cs);
      ops.push_back(cd);
      done[cs] = 1;
      int prev = move_from[cs];
      if (prev == first_dst) break;  // first_dst's content is parked
      cd = cs;
      cs = prev;
    }
    ops.push_back(-1);  // parked content -> its destination
    ops.push_back(cs);
    done[first_dst] = 1;
  }
  starts.push_back((int32_t)(ops.size() / 2));
  return true;
}

}  // namespace pkv
