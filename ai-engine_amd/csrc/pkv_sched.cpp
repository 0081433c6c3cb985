// pkv_sched.cpp -- continuous-batching scheduler: the block bookkeeping of
// the reference's engine thread (crates/ai-engine-candle/src/paged/engine.rs:
// run_loop :62-180, prefill :182-237) as a step machine around the caller's
// model forward, plus chunked prefill, forks with copy-on-write blocks and
// compaction (no reference counterpart).  Pure host code.
//
// Allocator semantics are the reference's BlockAllocator (block_table.rs):
// free list [N-1 .. 0] popped from the back, ensure_capacity all-or-nothing,
// release appending the table's blocks in table order.  With forks a block
// carries a reference count and returns to the free list when the last table
// holding it releases it; without forks every count is 1 and the free list
// evolves exactly as the reference's.
#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <deque>
#include <new>
#include <string>
#include <vector>

#include "../../include/pagedkv.h"

namespace {

struct Request {
  int64_t id;
  int prompt_len;
  int max_tokens;
};

struct Seq {             // engine.rs:20-28
  int64_t id = 0;
  std::vector<uint32_t> table;
  int prompt_len = 0;
  int prefilled = 0;     // prompt tokens already written (chunked prefill)
  int pos = 0;           // tokens in the cache = position of the next write
  int produced = 0;
  int max_tokens = 0;
  int32_t next_token = 0;
  bool decoding = false; // prompt done and first token sampled
};

enum Phase { kAdmit = 0, kDecode = 1 };

struct Row {
  size_t seq;            // index into running
  bool prefill;
  int q_start, q_len;
  bool produces;
};

}  // namespace

struct pkv_sched {
  pkv_sched_config cfg{};
  std::deque<Request> queue;
  std::vector<Seq> running;             // the reference's running Vec, in order
  std::vector<uint32_t> free;           // LIFO, back() handed out next
  std::vector<int32_t> refs;            // per block
  std::deque<pkv_sched_event> events;
  int64_t next_id = 1;
  Phase phase = kAdmit;
  bool plan_open = false;
  // the open plan
  std::vector<Row> rows;
  std::vector<int64_t> row_seq;
  std::vector<int32_t> tables, ctx_lens, cu, q_start, slots, positions, copy_src, copy_dst;
  std::vector<int8_t> produces;
  int max_blocks = 0;

  void event(int64_t seq, int kind, int32_t token, const char* fmt = nullptr, ...) {
    pkv_sched_event ev{};
    ev.seq = seq;
    ev.kind = kind;
    ev.token = token;
    if (fmt) {
      va_list ap;
      va_start(ap, fmt);
      vsnprintf(ev.message, sizeof ev.message, fmt, ap);
      va_end(ap);
    }
    events.push_back(ev);
  }
  size_t blocks_for(size_t n) const { return (n + cfg.block_size - 1) / cfg.block_size; }
  // block_table.rs:32-47: all or nothing.
  bool ensure_capacity(Seq& s, size_t n_tokens) {
    size_t need = blocks_for(n_tokens);
    if (need <= s.table.size()) return true;
    size_t extra = need - s.table.size();
    if (extra > free.size()) return false;
    for (size_t i = 0; i < extra; ++i) {
      uint32_t b = free.back();
      free.pop_back();
      refs[b] = 1;
      s.table.push_back(b);
    }
    return true;
  }
  // block_table.rs:49-52, with reference counts.
  void release(Seq& s) {
    for (uint32_t b : s.table)
      if (--refs[b] == 0) free.push_back(b);
    s.table.clear();
  }
  // The block about to receive position pos must be private: a shared block
  // is first copied to a fresh one (recorded for the caller).
  bool make_private(Seq& s, int pos) {
    size_t j = (size_t)pos / cfg.block_size;
    uint32_t b = s.table[j];
    if (refs[b] <= 1) return true;
    if (free.empty()) return false;
    uint32_t nb = free.back();
    free.pop_back();
    refs[nb] = 1;
    --refs[b];
    s.table[j] = nb;
    copy_src.push_back((int32_t)b);
    copy_dst.push_back((int32_t)nb);
    return true;
  }
  int32_t slot(const Seq& s, int pos) const {
    return (int32_t)(s.table[(size_t)pos / cfg.block_size] * cfg.block_size + pos % cfg.block_size);
  }
  // engine.rs:77-100 + prefill() guards :189-206.  Admitted sequences join
  // `running` with their whole prompt's blocks allocated.
  int admit() {
    int admitted = 0;
    while ((int)running.size() < cfg.max_num_seqs && !queue.empty()) {
      Request r = queue.front();
      queue.pop_front();
      if (r.max_tokens == 0) {  // :190-192, nothing is sent
        event(r.id, PKV_EV_FINISHED, 0);
        continue;
      }
      if (r.prompt_len > cfg.max_seq) {  // :194-201
        event(r.id, PKV_EV_ERROR, 0, "prompt exceeds max context (%d > %d)", r.prompt_len,
              cfg.max_seq);
        continue;
      }
      Seq s;
      s.id = r.id;
      s.prompt_len = r.prompt_len;
      s.max_tokens = r.max_tokens;
      if (!ensure_capacity(s, (size_t)r.prompt_len)) {  // :203-206
        event(r.id, PKV_EV_ERROR, 0, "KV cache exhausted at admission");
        continue;
      }
      running.push_back(std::move(s));
      ++admitted;
    }
    return admitted;
  }
  // engine.rs:102-128: context guard, then capacity for the new token;
  // failures end the sequence and free its blocks.  Returns true if any
  // sequence was evicted.
  bool capacity_pass() {
    bool evicted = false;
    std::vector<Seq> keep;
    keep.reserve(running.size());
    for (Seq& s : running) {
      if (!s.decoding) {
        keep.push_back(std::move(s));
        continue;
      }
      if (s.pos + 1 > cfg.max_seq) {
        event(s.id, PKV_EV_ERROR, 0, "sequence exceeded max context (%d > %d)", s.pos + 1,
              cfg.max_seq);
        release(s);
        evicted = true;
        continue;
      }
      if (!ensure_capacity(s, (size_t)s.pos + 1) || !make_private(s, s.pos)) {
        event(s.id, PKV_EV_ERROR, 0, "KV cache exhausted");
        release(s);
        evicted = true;
        continue;
      }
      keep.push_back(std::move(s));
    }
    running.swap(keep);
    return evicted;
  }
  void clear_plan() {
    rows.clear();
    row_seq.clear();
    tables.clear();
    ctx_lens.clear();
    cu.clear();
    q_start.clear();
    slots.clear();
    positions.clear();
    produces.clear();
    copy_src.clear();
    copy_dst.clear();
    max_blocks = 0;
  }
  void finish_plan() {
    // rows are prefill rows then decode rows (built in that order)
    int n_tok = 0;
    cu.push_back(0);
    for (const Row& r : rows) {
      const Seq& s = running[r.seq];
      row_seq.push_back(s.id);
      int ctx = r.prefill ? r.q_start + r.q_len : s.pos + 1;
      ctx_lens.push_back(ctx);
      max_blocks = std::max(max_blocks, (int)blocks_for((size_t)ctx));
      produces.push_back(r.produces ? 1 : 0);
      if (r.prefill) {
        q_start.push_back(r.q_start);
        for (int i = 0; i < r.q_len; ++i) {
          slots.push_back(slot(s, r.q_start + i));
          positions.push_back(r.q_start + i);
        }
        n_tok += r.q_len;
        cu.push_back(n_tok);
      } else {
        slots.push_back(slot(s, s.pos));
        positions.push_back(s.pos);
      }
    }
    max_blocks = std::max(max_blocks, 1);
    tables.assign(rows.size() * (size_t)max_blocks, 0);
    for (size_t i = 0; i < rows.size(); ++i) {
      const Seq& s = running[rows[i].seq];
      size_t nb = std::min(s.table.size(), (size_t)max_blocks);
      for (size_t j = 0; j < nb; ++j) tables[i * max_blocks + j] = (int32_t)s.table[j];
    }
  }
  void remove_ended(const std::vector<bool>& ended) {
    std::vector<Seq> keep;
    for (size_t i = 0; i < running.size(); ++i)
      if (!ended[i]) keep.push_back(std::move(running[i]));
    running.swap(keep);
  }
};

namespace {

thread_local std::string g_sched_error;

int sfail(int code, const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_sched_error = buf;
  return code;
}

void fill_plan(const pkv_sched* s, pkv_sched_plan* p) {
  int np = 0;
  for (const Row& r : s->rows) np += r.prefill ? 1 : 0;
  p->n_prefill = np;
  p->n_decode = (int)s->rows.size() - np;
  p->n_rows = (int)s->rows.size();
  p->max_blocks = s->max_blocks;
  p->n_tokens = (int)s->slots.size();
  p->n_copies = (int)s->copy_src.size();
  p->row_seq = s->row_seq.data();
  p->block_tables = s->tables.data();
  p->context_lens = s->ctx_lens.data();
  p->cu_q_lens = s->cu.data();
  p->q_start = s->q_start.data();
  p->slot_mapping = s->slots.data();
  p->positions = s->positions.data();
  p->produces = s->produces.data();
  p->copy_src = s->copy_src.data();
  p->copy_dst = s->copy_dst.data();
}

}  // namespace

extern "C" {

const char* pkv_sched_last_error(void) { return g_sched_error.c_str(); }

int pkv_sched_create(pkv_sched** out, const pkv_sched_config* cfg) {
  if (!out || !cfg) return sfail(PKV_ERR_INVALID, "NULL argument");
  *out = nullptr;
  if (cfg->max_num_seqs <= 0 || cfg->block_size <= 0 || cfg->kv_cache_blocks <= 0 ||
      cfg->max_seq <= 0 || cfg->prefill_chunk < 0 || cfg->step_token_budget < 0)
    return sfail(PKV_ERR_INVALID, "scheduler config out of range");
  pkv_sched* s = new (std::nothrow) pkv_sched();
  if (!s) return sfail(PKV_ERR_OOM, "host allocation failed");
  try {
    s->cfg = *cfg;
    s->free.resize((size_t)cfg->kv_cache_blocks);
    for (int i = 0; i < cfg->kv_cache_blocks; ++i)  // block_table.rs:17-21
      s->free[i] = (uint32_t)(cfg->kv_cache_blocks - 1 - i);
    s->refs.assign((size_t)cfg->kv_cache_blocks, 0);
  } catch (...) {
    delete s;
    return sfail(PKV_ERR_OOM, "host allocation failed");
  }
  *out = s;
  return PKV_OK;
}

void pkv_sched_destroy(pkv_sched* s) { delete s; }

int pkv_sched_submit(pkv_sched* s, int prompt_len, int max_tokens, int64_t* id) {
  if (!s || prompt_len <= 0 || max_tokens < 0)
    return sfail(PKV_ERR_INVALID, "submit: prompt_len %d, max_tokens %d", prompt_len, max_tokens);
  int64_t rid = s->next_id++;
  s->queue.push_back(Request{rid, prompt_len, max_tokens});
  if (id) *id = rid;
  return PKV_OK;
}

int pkv_sched_step(pkv_sched* s, pkv_sched_plan* plan) {
  if (!s || !plan) return sfail(PKV_ERR_INVALID, "NULL argument");
  if (s->plan_open) return sfail(PKV_ERR_INVALID, "step: the previous plan is not completed");
  std::memset(plan, 0, sizeof *plan);
  s->clear_plan();
  const bool chunked = s->cfg.prefill_chunk > 0;
  for (int guard = 0; guard < 1 << 20; ++guard) {
    if (!chunked && s->phase == kAdmit) {
      // An iteration opens with admission; admitted prompts are prefilled
      // whole in a plan of their own (engine.rs:77-100,182-237).
      s->admit();
      for (size_t i = 0; i < s->running.size(); ++i)
        if (!s->running[i].decoding)
          s->rows.push_back(Row{i, true, 0, s->running[i].prompt_len, true});
      s->phase = kDecode;
      if (!s->rows.empty()) break;
    }
    if (chunked) s->admit();
    if (s->running.empty()) {  // nothing runnable (engine.rs:101-112)
      s->phase = kAdmit;
      break;
    }
    bool evicted = s->capacity_pass();
    if (chunked) {
      int budget = s->cfg.step_token_budget > 0 ? s->cfg.step_token_budget : 1 << 30;
      for (size_t i = 0; i < s->running.size() && budget > 0; ++i) {
        Seq& q = s->running[i];
        if (q.decoding) continue;
        int len = std::min({s->cfg.prefill_chunk, q.prompt_len - q.prefilled, budget});
        budget -= len;
        s->rows.push_back(Row{i, true, q.prefilled, len, q.prefilled + len == q.prompt_len});
      }
    }
    for (size_t i = 0; i < s->running.size(); ++i)
      if (s->running[i].decoding) s->rows.push_back(Row{i, false, 0, 1, true});
    if (s->rows.empty() && evicted && !s->queue.empty()) {
      // engine.rs:125-127: all evicted -> next iteration admits again
      s->phase = kAdmit;
      continue;
    }
    if (s->rows.empty()) s->phase = kAdmit;
    break;
  }
  if (s->rows.empty()) {
    s->clear_plan();
    return PKV_OK;
  }
  // prefill rows before decode rows
  std::stable_partition(s->rows.begin(), s->rows.end(), [](const Row& r) { return r.prefill; });
  s->finish_plan();
  s->plan_open = true;
  fill_plan(s, plan);
  return PKV_OK;
}

int pkv_sched_complete(pkv_sched* s, const int32_t* tokens, int n, const char* error) {
  if (!s) return sfail(PKV_ERR_INVALID, "NULL scheduler");
  if (!s->plan_open) return sfail(PKV_ERR_INVALID, "complete: no plan is open");
  int want = 0;
  for (const Row& r : s->rows) want += r.produces ? 1 : 0;
  if (!error && (n != want || (want > 0 && !tokens)))
    return sfail(PKV_ERR_INVALID, "complete: %d tokens for %d producing rows", n, want);
  const bool chunked = s->cfg.prefill_chunk > 0;
  std::vector<bool> ended(s->running.size(), false);
  if (error) {
    // engine.rs:134-141 (forward) and :207-215 (prefill): every sequence of
    // the failed forward ends with Err and frees its blocks.
    for (const Row& r : s->rows) {
      Seq& q = s->running[r.seq];
      if (ended[r.seq]) continue;
      s->event(q.id, PKV_EV_ERROR, 0, "%s: %s", r.prefill ? "prefill" : "forward", error);
      s->release(q);
      ended[r.seq] = true;
    }
  } else {
    int k = 0;
    for (const Row& r : s->rows) {
      Seq& q = s->running[r.seq];
      if (r.prefill) {
        q.prefilled = r.q_start + r.q_len;
        if (!r.produces) continue;
        // prefill() sends its sampled token unconditionally (:226-227)
        int32_t t = tokens[k++];
        s->event(q.id, PKV_EV_TOKEN, t);
        q.next_token = t;
        q.pos = q.prompt_len;
        q.produced = 1;
        q.decoding = true;
        continue;
      }
      // engine.rs:160-178
      int32_t next = tokens[k++];
      q.pos += 1;
      q.produced += 1;
      bool eos = next == s->cfg.eos_token_id;
      bool at_limit = q.produced >= q.max_tokens;
      if (!eos) s->event(q.id, PKV_EV_TOKEN, next);
      if (eos || at_limit) {
        s->release(q);
        s->event(q.id, PKV_EV_FINISHED, 0);
        ended[r.seq] = true;
      } else {
        q.next_token = next;
      }
    }
  }
  s->remove_ended(ended);
  // Reference mode: a completed prefill plan is followed by the same
  // iteration's decode step (also when some prefills failed, as a failed
  // prefill() only drops its request); a completed decode plan ends the
  // iteration.
  bool had_decode = false;
  for (const Row& r : s->rows) had_decode |= !r.prefill;
  if (!chunked) s->phase = had_decode ? kAdmit : kDecode;
  s->plan_open = false;
  s->clear_plan();
  return PKV_OK;
}

int pkv_sched_poll(pkv_sched* s, pkv_sched_event* ev) {
  if (!s || !ev || s->events.empty()) return 0;
  *ev = s->events.front();
  s->events.pop_front();
  return 1;
}

int pkv_sched_fork(pkv_sched* s, int64_t parent, int max_tokens, int64_t* child) {
  if (!s || max_tokens < 0) return sfail(PKV_ERR_INVALID, "fork: bad argument");
  if (s->plan_open) return sfail(PKV_ERR_INVALID, "fork: a plan is open");
  size_t i = 0;
  while (i < s->running.size() && s->running[i].id != parent) ++i;
  if (i == s->running.size() || !s->running[i].decoding)
    return sfail(PKV_ERR_INVALID, "fork: sequence %lld is not decoding", (long long)parent);
  if ((int)s->running.size() >= s->cfg.max_num_seqs)
    return sfail(PKV_ERR_CAPACITY, "fork: max_num_seqs reached");
  Seq c = s->running[i];
  c.id = s->next_id++;
  c.max_tokens = max_tokens;
  for (uint32_t b : c.table) ++s->refs[b];
  s->running.push_back(std::move(c));
  if (child) *child = s->running.back().id;
  return PKV_OK;
}

int pkv_sched_compact(pkv_sched* s, int32_t* src, int32_t* dst, int cap, int* n) {
  if (!s || !n) return sfail(PKV_ERR_INVALID, "compact: NULL argument");
  if (s->plan_open) return sfail(PKV_ERR_INVALID, "compact: a plan is open");
  const int N = s->cfg.kv_cache_blocks;
  int live = 0;
  for (int b = 0; b < N; ++b) live += s->refs[b] > 0 ? 1 : 0;
  // fewest moves: live blocks at ids >= live fill the free ids below live
  std::vector<int32_t> holes, movers;
  for (int b = 0; b < live; ++b)
    if (s->refs[b] == 0) holes.push_back(b);
  for (int b = live; b < N; ++b)
    if (s->refs[b] > 0) movers.push_back(b);
  if ((int)movers.size() > cap)
    return sfail(PKV_ERR_INVALID, "compact: %zu moves exceed capacity %d", movers.size(), cap);
  std::vector<uint32_t> remap((size_t)N);
  for (int b = 0; b < N; ++b) remap[b] = (uint32_t)b;
  for (size_t i = 0; i < movers.size(); ++i) {
    remap[movers[i]] = (uint32_t)holes[i];
    s->refs[holes[i]] = s->refs[movers[i]];
    s->refs[movers[i]] = 0;
    if (src) src[i] = movers[i];
    if (dst) dst[i] = holes[i];
  }
  for (Seq& q : s->running)
    for (uint32_t& b : q.table) b = remap[b];
  s->free.clear();  // pops hand out live, live + 1, ... (block_table.rs:17-21)
  for (int b = N - 1; b >= live; --b) s->free.push_back((uint32_t)b);
  *n = (int)movers.size();
  return PKV_OK;
}

int pkv_sched_counts(const pkv_sched* s, int* running, int* waiting, int* free_blocks) {
  if (!s) return sfail(PKV_ERR_INVALID, "NULL scheduler");
  if (running) *running = (int)s->running.size();
  if (waiting) *waiting = (int)s->queue.size();
  if (free_blocks) *free_blocks = (int)s->free.size();
  return PKV_OK;
}

int pkv_sched_table(const pkv_sched* s, int64_t seq, const uint32_t** blocks, int* n_blocks,
                    int* pos) {
  if (!s) return sfail(PKV_ERR_INVALID, "NULL scheduler");
  for (const Seq& q : s->running)
    if (q.id == seq) {
      if (blocks) *blocks = q.table.empty() ? nullptr : q.table.data();
      if (n_blocks) *n_blocks = (int)q.table.size();
      if (pos) *pos = q.decoding ? q.pos : q.prefilled;
      return PKV_OK;
    }
  if (blocks) *blocks = nullptr;
  if (n_blocks) *n_blocks = 0;
  return sfail(PKV_ERR_INVALID, "sequence %lld is not live", (long long)seq);
}

}  // extern "C"
