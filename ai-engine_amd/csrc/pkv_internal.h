// pkv_internal.h -- definitions shared by the C-ABI host code and the HIP
// kernels of libpagedkv (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "../../include/pagedkv.h"

// One handle = the reference's Vec<KvPool> (engine.rs:70-72).  Device memory
// is a single slab laid out [layer][K|V][num_blocks][block_size][n_kv][hd].
struct pkv_pool {
  int n_layers = 0;
  int num_blocks = 0;
  int block_size = 0;
  int n_kv_head = 0;
  int head_dim = 0;
  int dtype = 0;
  int device = 0;
  size_t elem_bytes = 0;
  size_t row_bytes = 0;    // one (slot, kv head) row: head_dim * elem_bytes
  size_t block_bytes = 0;  // one block of one layer's K (or V)
  size_t layer_bytes = 0;  // one layer's K (or V): num_blocks * block_bytes
  char* base = nullptr;    // device slab
  uint32_t* err = nullptr; // device error word, bit set by kernels
  // workspace: split-context partials (m, l, O) of decode and split prefill;
  // buffers replaced by a larger one wait in ws_retired until the device is
  // known to be done with them
  char* ws = nullptr;
  size_t ws_bytes = 0;
  std::vector<char*> ws_retired;
  size_t ws_retired_bytes = 0;
  // this device's copy of the static scratch array of
  // pkv_decode_attention_noalloc (looked up at pool creation)
  char* scratch = nullptr;
  // compute units of the device (workgroup placement of the prefill kernel)
  int n_cu = 0;
  // compaction plan (chains of block moves), kept between calls: device
  // buffer and its pinned host staging copy
  char* plan = nullptr;
  char* plan_host = nullptr;
  size_t plan_bytes = 0;
  // recorded by each compaction after its plan upload (the staging copy may
  // be rewritten once it has completed) and after its kernel (the device
  // plan may be rewritten once it has completed)
  hipEvent_t plan_uploaded = nullptr;
  hipEvent_t plan_consumed = nullptr;
  bool plan_pending = false;
  // main-kernel timing events (pkv_pool_profile)
  bool prof_on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_events;
  size_t prof_used = 0;
  std::string last_error;

  char* layer_k(int layer) const {
    return base + (size_t)layer * 2 * layer_bytes;
  }
  char* layer_v(int layer) const { return layer_k(layer) + layer_bytes; }
};

// RoPE tables (Rope::new) in device memory.
struct pkv_rope {
  int rope_dim = 0;
  int max_seq = 0;
  int device = 0;
  float* cos = nullptr;     // [max_seq][rope_dim / 2]
  float* sin = nullptr;
  uint32_t* err = nullptr;  // device error word of pkv_rope_apply
};

// Device error bits (pkv_pool::err, pkv_rope::err).
enum : uint32_t {
  PKV_EBIT_SLOT = 1u,      // append/gather slot out of range
  PKV_EBIT_BLOCK = 2u,     // block table entry out of range
  PKV_EBIT_LENGTH = 4u,    // context length beyond max_context_len / table
  PKV_EBIT_POSITION = 8u,  // RoPE position outside the table, or a negative query position
};

namespace pkv {

inline size_t dtype_bytes(int dt) { return dt == PKV_F32 ? 4 : 2; }

// Token selection (pkv_sample.hip): the fixed draw r of a seed, and the
// launcher of the per-row argmax / sample kernel.
float sample_draw(uint64_t seed);
hipError_t launch_sample(const void* logits, int dtype, long long row_stride, int batch,
                         int vocab, const float* temperatures, int top_k, float top_p,
                         float r, int32_t* tokens, hipStream_t stream);
// The bit-exact variant (the reference's f32 arithmetic; top_p NaN = None;
// routes, when not null, gets per row the kernel that selected it), and the
// exp it uses.
hipError_t launch_sample_exact(const void* logits, int dtype, long long row_stride, int batch,
                               int vocab, const float* temperatures, int top_k, float top_p,
                               float r, int32_t* tokens, int32_t* routes, hipStream_t stream);
hipError_t launch_expf_glibc(const float* in, float* out, long long n, hipStream_t stream);

// Launchers (defined in the .hip files).  They validate nothing that the
// C-ABI layer already validated, return hipError_t and enqueue on `stream`.
hipError_t launch_append(const pkv_pool* p, int layer, const void* k,
                         const void* v, const int32_t* slots, int n,
                         hipStream_t stream);
hipError_t launch_gather(const pkv_pool* p, int layer, const int32_t* table,
                         int len, void* out_k, void* out_v,
                         hipStream_t stream);
hipError_t launch_gather_varlen(const pkv_pool* p, int layer, const int32_t* tables, int mbps,
                                const int32_t* cu_lens, int batch, int total_rows, void* out_k,
                                void* out_v, hipStream_t stream);
hipError_t launch_copy_blocks(const pkv_pool* p, const int32_t* src,
                              const int32_t* dst, int n, hipStream_t stream);
// Compaction: ops[] holds (src, dst) pairs executed in order within each
// chain; chain c is ops[chain_start[c] .. chain_start[c+1]).  src == -1
// reads the chain's held copy, dst == -1 stores into it (cycles).
hipError_t launch_compact(const pkv_pool* p, const int32_t* ops,
                          const int32_t* chain_start, int n_chains,
                          hipStream_t stream);
hipError_t launch_fill_normal(const pkv_pool* p, uint64_t seed,
                              hipStream_t stream);
// Adds to *count the 16-byte chunks of blocks[i] (every layer, K and V) that
// differ from what launch_fill_normal(seed) wrote into block origin[i].
hipError_t launch_verify_normal(const pkv_pool* p, uint64_t seed, const int32_t* blocks,
                                const int32_t* origin, int n, unsigned long long* count,
                                hipStream_t stream);

// Adds the 32-bit words of blocks[i] (every layer, K and V) into *sum
// (device, mod 2^64): a read-only stream of the blocks.
hipError_t launch_read_blocks(const pkv_pool* p, const int32_t* blocks, int n,
                              unsigned long long* sum, hipStream_t stream);

// Host computation of the RoPE tables (Rope::new, rope.rs:14-23).
void rope_tables_host(int rope_dim, float freq_base, int max_seq, float* cos_t,
                      float* sin_t);
hipError_t launch_rope_apply(const pkv_rope* r, const void* x, int in_dtype,
                             void* out, int out_dtype, const int32_t* positions,
                             int n_tokens, int n_head, hipStream_t stream);
hipError_t launch_append_rope(const pkv_pool* p, int layer, const pkv_rope* r,
                              const int32_t* positions, int in_dtype, const void* k,
                              const void* v, const int32_t* slots, int n_tokens,
                              const void* q, void* q_out, int n_head, hipStream_t stream);

struct DecodeArgs {
  const void* q;
  void* out;
  int out_dtype;
  const int32_t* block_tables;
  int max_blocks_per_seq;
  const int32_t* context_lens;
  int max_context_len;
  int batch;
  int n_head;
  float scale;
  const void* k_new;
  const void* v_new;
  // RoPE inside the kernel (rope_cos == nullptr: q and k_new are final)
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int rope_max = 0;
  const int32_t* positions = nullptr;
  int in_f32 = 0;  // q, k_new, v_new are f32 (else the pool dtype)
};

// A 1-D launch of `blocks` workgroups of `threads` work-items: HIP counts a
// grid's work-items in 32 bits, so launchers refuse larger ones
// (hipErrorInvalidValue) instead of letting the grid size wrap.
inline bool grid_fits(long long blocks, int threads) {
  return blocks >= 0 && blocks * (long long)threads <= 0xFFFFFFFFLL;
}

// Longest max_context_len / max_q_len the attention calls accept (tokens):
// the planners' length arithmetic stays within 32-bit ints below it.
constexpr int kMaxLen = 1 << 30;

// Partition length (tokens), the length of the parts a context's last
// part_tokens are cut into, and the most partitions of a sequence, for a
// decode launch; all are functions of the pool shape and the arguments only.
void decode_plan(const pkv_pool* p, int batch, int n_head, int max_context_len,
                 int* part_tokens, int* max_parts, int* sub_tokens = nullptr);
size_t decode_workspace_bytes(const pkv_pool* p, int batch, int n_head,
                              int max_context_len);
bool decode_supported(const pkv_pool* p, int n_head);
// The split-context partials go to `partials` (decode_workspace_bytes of the
// launch).  ev_begin / ev_end (may be null) are recorded on `stream` right
// before and right after the main partition kernel.
hipError_t launch_decode(const pkv_pool* p, int layer, const DecodeArgs& a,
                         char* partials, hipStream_t stream, hipEvent_t ev_begin = nullptr,
                         hipEvent_t ev_end = nullptr);
// Bytes of the static scratch array of pkv_decode_attention_noalloc, and the
// address of the current device's copy (looked up once per device).
size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch(int device, char** ptr);

struct PrefillArgs {
  const void* q;
  void* out;
  int out_dtype;
  const int32_t* cu_q_lens;
  const int32_t* context_lens;
  const int32_t* block_tables;
  int max_blocks_per_seq;
  int n_seqs;
  int max_q_len;
  int max_context_len;
  int n_head;
  float scale;
  // fused store of the prompt's K/V ([total_q][n_kv][hd], pool dtype), or null
  const void* k_new = nullptr;
  const void* v_new = nullptr;
};
bool prefill_supported(const pkv_pool* p, int n_head);
// Split of long key ranges for launches with few row blocks: keys per part,
// parts per row block at most, and the workspace the partials need (0: no
// split).
void prefill_plan(const pkv_pool* p, int n_seqs, int n_head, int max_q_len, int max_context_len,
                  int* part_keys, int* max_parts, size_t* ws_bytes);
hipError_t launch_prefill(const pkv_pool* p, int layer, const PrefillArgs& a,
                          hipStream_t stream, hipEvent_t ev_begin = nullptr,
                          hipEvent_t ev_end = nullptr);

// One launch for a layer's prefill batch and decode batch (pkv_mixed.hip):
// same results as launch_prefill then launch_decode, with the decode
// partials at decode_partials and the prefill split partials at
// prefill_partials (disjoint).  ev_begin / ev_end bracket the combined
// kernel.  hipErrorNotSupported, with nothing enqueued, for shapes without a
// combined kernel (mixed_supported false, or different n_head).
bool mixed_supported(const pkv_pool* p, int n_head, bool rope);
hipError_t launch_mixed(const pkv_pool* p, int layer, const PrefillArgs& pa,
                        const DecodeArgs& da, char* decode_partials, char* prefill_partials,
                        hipStream_t stream, hipEvent_t ev_begin = nullptr,
                        hipEvent_t ev_end = nullptr);

}  // namespace pkv
