// host_check.cpp -- the library's host C++ (block allocator and tables,
// scheduler step machine, compaction planner) driven through its own entry
// points on seeded random workloads, built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_sanitize.py.  Besides running
// every path under the sanitizers, it checks:
//   * allocator: free count, table contents, locate and the no-partial-
//     allocation rule against a plain model of block_table.rs:5-58 (free
//     list [N-1 .. 0], pop from the end, release appends in table order);
//   * planner: executing every plan's chains in order, each with its held
//     copy, moves exactly the requested blocks (destination d holds what
//     source s held, every other block keeps its bytes), no block is in two
//     chains (chains run concurrently on the GPU), plan size within the
//     capacity bound, bad inputs refused;
//   * scheduler: block accounting (free + blocks held by live sequences ==
//     pool), plan arrays within the pool, one token per producing row.
// Exit status 0 when every check passed.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "../../ai-engine_amd/csrc/compact_plan.h"
#include "../../include/pagedkv.h"

namespace {

int g_fail = 0;
// activity, so that a run that exercised nothing does not pass
long g_rows = 0, g_forks = 0, g_compact_moves = 0, g_chains = 0, g_cycles = 0;
long g_bad_plans_caught = 0;
#define CHECK(c, ...)                                  \
  do {                                                 \
    if (!(c)) {                                        \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);               \
      std::fprintf(stderr, "\n");                      \
      if (++g_fail > 20) std::exit(1);                 \
    }                                                  \
  } while (0)

struct Rng {  // splitmix64
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  int below(int n) { return n > 0 ? (int)(next() % (uint64_t)n) : 0; }
};

// ---- allocator against a model -------------------------------------------
void check_allocator(uint64_t seed) {
  Rng r(seed);
  const size_t N = 1 + r.below(300), BS = (size_t)1 << r.below(6);
  pkv_allocator* a = pkv_allocator_new(N, BS);
  CHECK(a, "allocator_new");
  std::vector<uint32_t> free_list;
  for (size_t i = 0; i < N; ++i) free_list.push_back((uint32_t)(N - 1 - i));
  std::vector<pkv_table*> tabs;
  std::vector<std::vector<uint32_t>> model;
  for (int step = 0; step < 400; ++step) {
    const int op = r.below(10);
    if (op < 2 || tabs.empty()) {
      tabs.push_back(pkv_table_new());
      model.emplace_back();
      continue;
    }
    const int t = r.below((int)tabs.size());
    if (op < 7) {  // ensure capacity for a longer sequence
      const size_t tokens = model[t].size() * BS + r.below((int)(3 * BS + 40));
      const size_t need = (tokens + BS - 1) / BS;
      const size_t want = need > model[t].size() ? need - model[t].size() : 0;
      CHECK(pkv_allocator_blocks_for(a, tokens) == need, "blocks_for");
      const int rc = pkv_allocator_ensure_capacity(a, tabs[t], tokens);
      if (want > free_list.size()) {
        CHECK(rc == PKV_ERR_CAPACITY, "expected capacity error, got %d", rc);
      } else {
        CHECK(rc == PKV_OK, "ensure_capacity rc %d", rc);
        for (size_t k = 0; k < want; ++k) {
          model[t].push_back(free_list.back());
          free_list.pop_back();
        }
      }
    } else if (op < 9) {  // release
      pkv_allocator_release(a, tabs[t]);
      for (uint32_t b : model[t]) free_list.push_back(b);
      model[t].clear();
    } else {  // locate every position and one past the end
      const size_t len = model[t].size() * BS;
      for (size_t pos = 0; pos <= len && pos < 4 * BS + 3; ++pos) {
        uint32_t blk = 0;
        size_t slot = 0;
        const int rc = pkv_allocator_locate(a, tabs[t], pos, &blk, &slot);
        if (pos < len) {
          CHECK(rc == PKV_OK && blk == model[t][pos / BS] && slot == pos % BS,
                "locate %zu", pos);
        } else {
          CHECK(rc == PKV_ERR_INVALID, "locate past the end rc %d", rc);
        }
      }
    }
    CHECK(pkv_allocator_free_count(a) == free_list.size(), "free_count");
    CHECK(pkv_table_len(tabs[t]) == model[t].size(), "table len");
    const uint32_t* bl = pkv_table_blocks(tabs[t]);
    for (size_t k = 0; k < model[t].size(); ++k) CHECK(bl[k] == model[t][k], "table block %zu", k);
  }
  for (pkv_table* t : tabs) {
    pkv_allocator_release(a, t);
    pkv_table_free(t);
  }
  CHECK(pkv_allocator_free_count(a) == N, "all blocks back");
  pkv_allocator_free(a);
}

// ---- compaction planner by simulation ------------------------------------
// Runs the plan's chains in order, each with its held copy, on blocks that
// hold their own ids; true when every destination holds its source's id,
// every block neither moved from nor to keeps its own, and no block is in
// two chains.
bool plan_moves_correctly(int N, const std::vector<int32_t>& src, const std::vector<int32_t>& dst,
                          const std::vector<int32_t>& ops, const std::vector<int32_t>& starts,
                          std::string* err) {
  char buf[200];
  auto no = [&](const char* what, long a, long b) {
    std::snprintf(buf, sizeof buf, "%s (%ld, %ld)", what, a, b);
    *err = buf;
    return false;
  };
  std::vector<uint64_t> mem(N), want(N);
  for (int i = 0; i < N; ++i) mem[i] = want[i] = 0x1000 + i;
  for (size_t i = 0; i < src.size(); ++i) want[dst[i]] = 0x1000 + src[i];
  std::vector<char> vacated(N, 0);
  for (int32_t x : src) vacated[x] = 1;
  for (int32_t x : dst) vacated[x] = 0;
  std::vector<int> owner(N, -1);
  if (starts.empty() || starts.back() * 2 != (int)ops.size()) return no("end marker", 0, 0);
  for (size_t c = 0; c + 1 < starts.size(); ++c) {
    uint64_t held = 0;
    bool have = false;
    if (starts[c] > starts[c + 1]) return no("starts out of order", (long)c, starts[c]);
    for (int k = starts[c]; k < starts[c + 1]; ++k) {
      const int32_t s = ops[2 * k], d = ops[2 * k + 1];
      for (int32_t b : {s, d}) {
        if (b < 0) continue;
        if (b >= N) return no("block out of range", b, N);
        if (owner[b] != -1 && owner[b] != (int)c) return no("block in two chains", b, owner[b]);
        owner[b] = (int)c;
      }
      if (s < 0 && d < 0) return no("op with neither side", (long)c, k);
      if (s < 0 && !have) return no("held copy read before it was parked", (long)c, k);
      const uint64_t v = s < 0 ? held : mem[s];
      if (d < 0) {
        held = v;
        have = true;
      } else {
        mem[d] = v;
      }
    }
  }
  for (int i = 0; i < N; ++i)
    if (!vacated[i] && mem[i] != want[i]) return no("block holds the wrong bytes", i, (long)mem[i]);
  return true;
}

void check_planner(uint64_t seed) {
  Rng r(seed);
  const int N = 1 + r.below(400);
  // a random injective move set: some live blocks move to random distinct
  // targets (chains, cycles, self moves all occur)
  std::vector<int32_t> perm(N), tgt(N);
  for (int i = 0; i < N; ++i) perm[i] = tgt[i] = i;
  for (int i = N - 1; i > 0; --i) std::swap(perm[i], perm[r.below(i + 1)]);
  for (int i = N - 1; i > 0; --i) std::swap(tgt[i], tgt[r.below(i + 1)]);
  const int n = r.below(N + 1);
  std::vector<int32_t> src(perm.begin(), perm.begin() + n), dst(tgt.begin(), tgt.begin() + n);
  if (r.below(4) == 0) {  // a pure permutation of a subset: cycles only
    dst = src;
    for (int i = n - 1; i > 0; --i) std::swap(dst[i], dst[r.below(i + 1)]);
  }
  std::vector<int32_t> ops, starts;
  std::string why;
  CHECK(pkv::plan_compaction(N, src.data(), dst.data(), n, ops, starts, why), "plan: %s",
        why.c_str());
  CHECK(ops.size() * sizeof(int32_t) + starts.size() * sizeof(int32_t) <=
            pkv::plan_capacity_bytes((size_t)N),
        "plan larger than its capacity bound");
  std::string err;
  CHECK(plan_moves_correctly(N, src, dst, ops, starts, &err), "%s", err.c_str());
  for (size_t c = 0; c + 1 < starts.size(); ++c) {
    ++g_chains;
    if (ops[2 * starts[c] + 1] < 0) ++g_cycles;
  }
  // the simulation is not vacuous: a chain with its first two moves swapped
  // (a block overwritten before it is read) is caught
  for (size_t c = 0; c + 1 < starts.size(); ++c) {
    if (starts[c + 1] - starts[c] < 2) continue;
    std::vector<int32_t> bad = ops;
    std::swap(bad[2 * starts[c]], bad[2 * starts[c] + 2]);
    std::swap(bad[2 * starts[c] + 1], bad[2 * starts[c] + 3]);
    CHECK(!plan_moves_correctly(N, src, dst, bad, starts, &err), "corrupted plan passed");
    ++g_bad_plans_caught;
    break;
  }
  // refused inputs
  if (n >= 2) {
    std::vector<int32_t> s2 = src, d2 = dst;
    s2[1] = s2[0];
    CHECK(!pkv::plan_compaction(N, s2.data(), dst.data(), n, ops, starts, why), "dup src");
    d2[1] = d2[0];
    CHECK(!pkv::plan_compaction(N, src.data(), d2.data(), n, ops, starts, why), "dup dst");
  }
  if (n >= 1) {
    std::vector<int32_t> s3 = src;
    s3[0] = N;
    CHECK(!pkv::plan_compaction(N, s3.data(), dst.data(), n, ops, starts, why), "range");
    s3[0] = -1;
    CHECK(!pkv::plan_compaction(N, s3.data(), dst.data(), n, ops, starts, why), "negative");
  }
}

// ---- scheduler step machine ----------------------------------------------
void check_sched(uint64_t seed) {
  Rng r(seed);
  pkv_sched_config cfg{};
  cfg.max_num_seqs = 1 + r.below(8);
  cfg.block_size = 1 << (2 + r.below(4));
  cfg.kv_cache_blocks = 4 + r.below(120);
  cfg.max_seq = 16 + r.below(600);
  cfg.eos_token_id = 7;
  cfg.prefill_chunk = r.below(2) ? 0 : 1 + r.below(64);
  cfg.step_token_budget = cfg.prefill_chunk && r.below(2) ? 1 + r.below(96) : 0;
  pkv_sched* s = nullptr;
  CHECK(pkv_sched_create(&s, &cfg) == PKV_OK && s, "sched_create: %s", pkv_sched_last_error());
  if (!s) return;
  std::vector<int64_t> ids;
  std::vector<int32_t> csrc(cfg.kv_cache_blocks), cdst(cfg.kv_cache_blocks);
  for (int it = 0; it < 300; ++it) {
    const int op = r.below(12);
    if (op < 3) {
      int64_t id = -1;
      const int rc = pkv_sched_submit(s, r.below(cfg.max_seq + 40), r.below(40), &id);
      if (rc == PKV_OK) ids.push_back(id);
      continue;
    }
    if (op == 3 && !ids.empty()) {  // fork (refused unless the parent is decoding)
      int64_t child = -1;
      if (pkv_sched_fork(s, ids[r.below((int)ids.size())], r.below(20), &child) == PKV_OK) {
        ids.push_back(child);
        ++g_forks;
      }
      continue;
    }
    if (op == 4) {
      int n = -1;
      const int rc = pkv_sched_compact(s, csrc.data(), cdst.data(), (int)csrc.size(), &n);
      CHECK(rc == PKV_OK && n >= 0 && n <= (int)csrc.size(), "sched_compact rc %d n %d", rc, n);
      if (rc == PKV_OK) {  // the moves are a plan the planner accepts
        g_compact_moves += n;
        std::vector<int32_t> ops, starts;
        std::string why;
        CHECK(pkv::plan_compaction(cfg.kv_cache_blocks, csrc.data(), cdst.data(), n, ops, starts,
                                   why),
              "scheduler moves refused by the planner: %s", why.c_str());
      }
      continue;
    }
    pkv_sched_plan plan{};
    if (pkv_sched_step(s, &plan) != PKV_OK) continue;
    CHECK(plan.n_rows == plan.n_prefill + plan.n_decode, "rows");
    int producing = 0;
    for (int i = 0; i < plan.n_rows; ++i) {
      producing += plan.produces[i] ? 1 : 0;
      CHECK(plan.context_lens[i] >= 1, "context length %d", plan.context_lens[i]);
      for (int k = 0; k < plan.max_blocks; ++k) {
        const int32_t b = plan.block_tables[(size_t)i * plan.max_blocks + k];
        CHECK(b >= 0 && b < cfg.kv_cache_blocks, "table entry %d", b);
      }
    }
    for (int i = 0; i < plan.n_tokens; ++i)
      CHECK(plan.slot_mapping[i] >= 0 &&
                plan.slot_mapping[i] < cfg.kv_cache_blocks * cfg.block_size,
            "slot %d", plan.slot_mapping[i]);
    for (int i = 0; i < plan.n_copies; ++i)
      CHECK(plan.copy_src[i] != plan.copy_dst[i], "copy onto itself");
    if (plan.n_rows == 0) continue;
    g_rows += plan.n_rows;
    std::vector<int32_t> toks(producing);
    for (auto& t : toks) t = r.below(10) == 0 ? cfg.eos_token_id : 100 + r.below(1000);
    const bool fail = r.below(25) == 0;
    CHECK(pkv_sched_complete(s, toks.data(), producing, fail ? "forward: injected" : nullptr) ==
              PKV_OK,
          "complete: %s", pkv_sched_last_error());
    pkv_sched_event ev;
    while (pkv_sched_poll(s, &ev) == 1) {
      CHECK(ev.kind == PKV_EV_TOKEN || ev.kind == PKV_EV_FINISHED || ev.kind == PKV_EV_ERROR,
            "event kind %d", ev.kind);
      CHECK(std::memchr(ev.message, 0, sizeof ev.message) != nullptr, "message not terminated");
    }
    // block accounting
    int running = 0, waiting = 0, free_blocks = 0;
    CHECK(pkv_sched_counts(s, &running, &waiting, &free_blocks) == PKV_OK, "counts");
    std::set<uint32_t> held;
    for (int64_t id : ids) {
      const uint32_t* bl = nullptr;
      int nb = 0, pos = 0;
      if (pkv_sched_table(s, id, &bl, &nb, &pos) == PKV_OK && bl)
        for (int k = 0; k < nb; ++k) held.insert(bl[k]);
    }
    CHECK(free_blocks + (int)held.size() <= cfg.kv_cache_blocks, "free %d + held %zu > %d",
          free_blocks, held.size(), cfg.kv_cache_blocks);
  }
  pkv_sched_destroy(s);
}

}  // namespace

int main(int argc, char** argv) {
  const int rounds = argc > 1 ? std::atoi(argv[1]) : 200;
  for (int i = 0; i < rounds; ++i) {
    check_allocator(1000 + i);
    check_planner(2000 + i);
    check_sched(3000 + i);
  }
  std::printf("host_check: %d rounds, %d failures; scheduler rows %ld, forks %ld, compaction "
              "moves %ld; planner chains %ld (cycles %ld), corrupted plans caught %ld\n",
              rounds, g_fail, g_rows, g_forks, g_compact_moves, g_chains, g_cycles,
              g_bad_plans_caught);
  const bool exercised = g_rows > 0 && g_forks > 0 && g_compact_moves > 0 && g_cycles > 0 &&
                         g_bad_plans_caught > 0;
  if (!exercised) std::printf("host_check: a path was not exercised\n");
  return g_fail || !exercised ? 1 : 0;
}
