// block_table.cpp -- host-side block bookkeeping, the C++ counterpart of the
// reference's BlockAllocator / BlockTable
// (crates/ai-engine-candle/src/paged/block_table.rs:5-58), exported through
// the C ABI (pkv_allocator_*, pkv_table_*).  Pure host code: it never touches
// the GPU, so it is usable (and tested) on machines without one.
#include <cstdint>
#include <cstdio>
#include <new>
#include <string>
#include <vector>

#include "../../include/pagedkv.h"

struct pkv_table {
  std::vector<uint32_t> blocks;  // block_table.rs:12-14
};

struct pkv_allocator {
  size_t block_size = 0;
  std::vector<uint32_t> free;  // LIFO; back() is handed out next
};

extern "C" {

pkv_allocator* pkv_allocator_new(size_t num_blocks, size_t block_size) {
  if (block_size == 0 || num_blocks > UINT32_MAX) return nullptr;
  pkv_allocator* a = new (std::nothrow) pkv_allocator();
  if (!a) return nullptr;
  a->block_size = block_size;
  // block_table.rs:17-21: (0..num_blocks).rev() so pops yield 0, 1, 2, ...
  try {
    a->free.resize(num_blocks);
  } catch (...) {
    delete a;
    return nullptr;
  }
  for (size_t i = 0; i < num_blocks; ++i)
    a->free[i] = (uint32_t)(num_blocks - 1 - i);
  return a;
}

void pkv_allocator_free(pkv_allocator* a) { delete a; }

size_t pkv_allocator_free_count(const pkv_allocator* a) {  // :23-25
  return a ? a->free.size() : 0;
}

size_t pkv_allocator_blocks_for(const pkv_allocator* a, size_t n_tokens) {  // :27-30
  if (!a || a->block_size == 0) return 0;
  return (n_tokens + a->block_size - 1) / a->block_size;
}

int pkv_allocator_ensure_capacity(pkv_allocator* a, pkv_table* t, size_t n_tokens) {  // :32-47
  if (!a || !t) return PKV_ERR_INVALID;
  size_t need = pkv_allocator_blocks_for(a, n_tokens);
  if (need <= t->blocks.size()) return PKV_OK;
  size_t extra = need - t->blocks.size();
  if (extra > a->free.size()) return PKV_ERR_CAPACITY;  // nothing allocated
  try {
    t->blocks.reserve(need);
  } catch (...) {
    return PKV_ERR_OOM;
  }
  for (size_t i = 0; i < extra; ++i) {
    t->blocks.push_back(a->free.back());
    a->free.pop_back();
  }
  return PKV_OK;
}

void pkv_allocator_release(pkv_allocator* a, pkv_table* t) {  // :49-52
  if (!a || !t) return;
  a->free.insert(a->free.end(), t->blocks.begin(), t->blocks.end());
  t->blocks.clear();
}

int pkv_allocator_locate(const pkv_allocator* a, const pkv_table* t, size_t pos,
                         uint32_t* block_id, size_t* slot) {  // :54-58
  if (!a || !t) return PKV_ERR_INVALID;
  size_t bi = pos / a->block_size;
  if (bi >= t->blocks.size()) return PKV_ERR_INVALID;  // the reference panics
  if (block_id) *block_id = t->blocks[bi];
  if (slot) *slot = pos % a->block_size;
  return PKV_OK;
}

pkv_table* pkv_table_new(void) { return new (std::nothrow) pkv_table(); }

void pkv_table_free(pkv_table* t) { delete t; }

size_t pkv_table_len(const pkv_table* t) { return t ? t->blocks.size() : 0; }

const uint32_t* pkv_table_blocks(const pkv_table* t) {
  return (t && !t->blocks.empty()) ? t->blocks.data() : nullptr;
}

}  // extern "C"
