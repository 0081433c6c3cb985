//! ffi.rs -- Rust declarations of libpagedkv's C ABI (include/pagedkv.h), the
//! file a maintainer adds as `crates/ai-engine-candle/src/paged/ffi.rs` to run
//! the `engine = "paged"` path on the MI355X library.  Every `extern "C"`
//! function, constant and `#[repr(C)]` struct of the header appears here with
//! the same names, argument order and types; `tests/test_rust_binding.py`
//! parses both files and fails when they differ.  Device pointers are raw
//! pointers; a HIP stream is a `*mut c_void` (null = the default stream).
#![allow(non_camel_case_types, dead_code)]

use std::ffi::{c_char, c_int, c_longlong, c_void, CStr};

// ---- status codes
pub const PKV_OK: c_int = 0;
pub const PKV_ERR_INVALID: c_int = -1;
pub const PKV_ERR_OOM: c_int = -2;
pub const PKV_ERR_HIP: c_int = -3;
pub const PKV_ERR_UNSUPPORTED: c_int = -4;
pub const PKV_ERR_CAPACITY: c_int = -5;
pub const PKV_ERR_DEVICE_DATA: c_int = -6;

// ---- element types and pool selectors
pub const PKV_F32: c_int = 0;
pub const PKV_F16: c_int = 1;
pub const PKV_BF16: c_int = 2;
pub const PKV_K: c_int = 0;
pub const PKV_V: c_int = 1;

// ---- scheduler event kinds
pub const PKV_EV_TOKEN: c_int = 0;
pub const PKV_EV_FINISHED: c_int = 1;
pub const PKV_EV_ERROR: c_int = 2;

/// Bytes of the static scratch array of pkv_decode_attention_noalloc.
pub const PKV_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

// ---- opaque handles
#[repr(C)] pub struct PkvPool { _p: [u8; 0] }
#[repr(C)] pub struct PkvRope { _p: [u8; 0] }
#[repr(C)] pub struct PkvAllocator { _p: [u8; 0] }
#[repr(C)] pub struct PkvTable { _p: [u8; 0] }
#[repr(C)] pub struct PkvSched { _p: [u8; 0] }

// ---- argument structs
#[repr(C)]
pub struct PkvPrefillBatch {
    pub q: *const c_void,
    pub out: *mut c_void,
    pub out_dtype: c_int,
    pub cu_q_lens: *const i32,
    pub context_lens: *const i32,
    pub block_tables: *const i32,
    pub max_blocks_per_seq: c_int,
    pub n_seqs: c_int,
    pub max_q_len: c_int,
    pub max_context_len: c_int,
    pub k_new: *const c_void,
    pub v_new: *const c_void,
}

#[repr(C)]
pub struct PkvDecodeBatch {
    pub q: *const c_void,
    pub out: *mut c_void,
    pub out_dtype: c_int,
    pub block_tables: *const i32,
    pub max_blocks_per_seq: c_int,
    pub context_lens: *const i32,
    pub max_context_len: c_int,
    pub batch: c_int,
    pub k_new: *const c_void,
    pub v_new: *const c_void,
}

#[repr(C)]
pub struct PkvSchedConfig {
    pub max_num_seqs: c_int,
    pub block_size: c_int,
    pub kv_cache_blocks: c_int,
    pub max_seq: c_int,
    pub eos_token_id: i32,
    pub prefill_chunk: c_int,
    pub step_token_budget: c_int,
}

#[repr(C)]
pub struct PkvSchedEvent {
    pub seq: i64,
    pub kind: c_int,
    pub token: i32,
    pub message: [c_char; 120],
}

#[repr(C)]
pub struct PkvSchedPlan {
    pub n_prefill: c_int,
    pub n_decode: c_int,
    pub n_rows: c_int,
    pub max_blocks: c_int,
    pub n_tokens: c_int,
    pub n_copies: c_int,
    pub row_seq: *const i64,
    pub block_tables: *const i32,
    pub context_lens: *const i32,
    pub cu_q_lens: *const i32,
    pub q_start: *const i32,
    pub slot_mapping: *const i32,
    pub positions: *const i32,
    pub produces: *const i8,
    pub copy_src: *const i32,
    pub copy_dst: *const i32,
}

#[link(name = "pagedkv")]
extern "C" {
    // ---- status and pool handle (KvPool::new, attention.rs:39-55)
    pub fn pkv_version() -> *const c_char;
    pub fn pkv_last_error(pool: *const PkvPool) -> *const c_char;
    pub fn pkv_pool_create(
        out: *mut *mut PkvPool, n_layers: c_int, num_blocks: c_int, block_size: c_int,
        n_kv_head: c_int, head_dim: c_int, dtype: c_int, device: c_int
    ) -> c_int;
    pub fn pkv_pool_destroy(pool: *mut PkvPool) -> c_int;
    pub fn pkv_pool_shape(
        pool: *const PkvPool, n_layers: *mut c_int, num_blocks: *mut c_int, block_size: *mut c_int,
        n_kv_head: *mut c_int, head_dim: *mut c_int, dtype: *mut c_int
    ) -> c_int;
    pub fn pkv_pool_layer_bytes(pool: *const PkvPool) -> usize;
    pub fn pkv_pool_layer_ptrs(
        pool: *const PkvPool, layer: c_int, k: *mut *mut c_void, v: *mut *mut c_void
    ) -> c_int;
    pub fn pkv_pool_read(
        pool: *mut PkvPool, layer: c_int, which: c_int, byte_offset: usize, nbytes: usize,
        host_dst: *mut c_void
    ) -> c_int;
    pub fn pkv_pool_write(
        pool: *mut PkvPool, layer: c_int, which: c_int, byte_offset: usize,
        host_src: *const c_void, nbytes: usize
    ) -> c_int;
    pub fn pkv_pool_check(pool: *mut PkvPool) -> c_int;

    // ---- KV append / scatter (KvPool::write, attention.rs:57-83)
    pub fn pkv_append(
        pool: *mut PkvPool, layer: c_int, k: *const c_void, v: *const c_void,
        slot_mapping: *const i32, n_tokens: c_int, stream: *mut c_void
    ) -> c_int;

    // ---- gather (KvPool::gather_seq, attention.rs:85-97) and its batched form
    pub fn pkv_gather_seq(
        pool: *mut PkvPool, layer: c_int, block_table: *const i32, len: c_int, out_k: *mut c_void,
        out_v: *mut c_void, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_gather_varlen(
        pool: *mut PkvPool, layer: c_int, block_tables: *const i32, max_blocks_per_seq: c_int,
        cu_lens: *const i32, batch: c_int, total_rows: c_int, out_k: *mut c_void,
        out_v: *mut c_void, stream: *mut c_void
    ) -> c_int;

    // ---- fork / copy-on-write and compaction (no reference counterpart)
    pub fn pkv_copy_blocks(
        pool: *mut PkvPool, src: *const i32, dst: *const i32, n: c_int, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_compact(
        pool: *mut PkvPool, src_host: *const i32, dst_host: *const i32, n: c_int,
        stream: *mut c_void
    ) -> c_int;

    // ---- decode attention (transformer.rs:271-292, attention.rs:11-28,100-136)
    pub fn pkv_decode_attention(
        pool: *mut PkvPool, layer: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        block_tables: *const i32, max_blocks_per_seq: c_int, context_lens: *const i32,
        max_context_len: c_int, batch: c_int, n_head: c_int, scale: f32, k_new: *const c_void,
        v_new: *const c_void, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_decode_workspace_bytes(
        pool: *const PkvPool, batch: c_int, n_head: c_int, max_context_len: c_int
    ) -> usize;
    pub fn pkv_pool_reserve_decode(
        pool: *mut PkvPool, batch: c_int, n_head: c_int, max_context_len: c_int
    ) -> c_int;
    pub fn pkv_decode_attention_positions(
        pool: *mut PkvPool, layer: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        block_tables: *const i32, max_blocks_per_seq: c_int, context_lens: *const i32,
        positions: *const i32, max_context_len: c_int, batch: c_int, n_head: c_int, scale: f32,
        k_new: *const c_void, v_new: *const c_void, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_decode_attention_noalloc(
        pool: *mut PkvPool, layer: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        block_tables: *const i32, max_blocks_per_seq: c_int, context_lens: *const i32,
        max_context_len: c_int, batch: c_int, n_head: c_int, scale: f32, k_new: *const c_void,
        v_new: *const c_void, stream: *mut c_void
    ) -> c_int;

    // ---- chunked-prefill attention (transformer.rs:139-196)
    pub fn pkv_prefill_attention(
        pool: *mut PkvPool, layer: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        cu_q_lens: *const i32, context_lens: *const i32, block_tables: *const i32,
        max_blocks_per_seq: c_int, n_seqs: c_int, max_q_len: c_int, max_context_len: c_int,
        n_head: c_int, scale: f32, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_prefill_attention_append(
        pool: *mut PkvPool, layer: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        cu_q_lens: *const i32, context_lens: *const i32, block_tables: *const i32,
        max_blocks_per_seq: c_int, n_seqs: c_int, max_q_len: c_int, max_context_len: c_int,
        n_head: c_int, scale: f32, k_new: *const c_void, v_new: *const c_void, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_prefill_workspace_bytes(
        pool: *const PkvPool, n_seqs: c_int, n_head: c_int, max_q_len: c_int,
        max_context_len: c_int
    ) -> usize;
    pub fn pkv_pool_reserve_prefill(
        pool: *mut PkvPool, n_seqs: c_int, n_head: c_int, max_q_len: c_int, max_context_len: c_int
    ) -> c_int;

    // ---- a layer's prefill batch and decode batch in one launch
    pub fn pkv_mixed_attention(
        pool: *mut PkvPool, layer: c_int, prefill: *const PkvPrefillBatch,
        decode: *const PkvDecodeBatch, n_head: c_int, scale: f32, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_mixed_workspace_bytes(
        pool: *const PkvPool, n_head: c_int, prefill: *const PkvPrefillBatch,
        decode: *const PkvDecodeBatch
    ) -> usize;

    // ---- rotary embedding (rope.rs:14-42, transformer.rs:160-174,252-269)
    pub fn pkv_rope_tables_host(
        rope_dim: c_int, freq_base: f32, max_seq: c_int, cos_host: *mut f32, sin_host: *mut f32
    ) -> c_int;
    pub fn pkv_rope_create(
        out: *mut *mut PkvRope, rope_dim: c_int, freq_base: f32, max_seq: c_int, device: c_int
    ) -> c_int;
    pub fn pkv_rope_destroy(rope: *mut PkvRope) -> c_int;
    pub fn pkv_rope_tables(
        rope: *const PkvRope, cos_dev: *mut *const f32, sin_dev: *mut *const f32
    ) -> c_int;
    pub fn pkv_rope_apply(
        rope: *mut PkvRope, x: *const c_void, in_dtype: c_int, out: *mut c_void, out_dtype: c_int,
        positions: *const i32, n_tokens: c_int, n_head: c_int, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_rope_check(rope: *mut PkvRope) -> c_int;
    pub fn pkv_decode_attention_rope(
        pool: *mut PkvPool, layer: c_int, rope: *const PkvRope, positions: *const i32,
        in_dtype: c_int, q: *const c_void, out: *mut c_void, out_dtype: c_int,
        block_tables: *const i32, max_blocks_per_seq: c_int, context_lens: *const i32,
        max_context_len: c_int, batch: c_int, n_head: c_int, scale: f32, k_new: *const c_void,
        v_new: *const c_void, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_append_rope(
        pool: *mut PkvPool, layer: c_int, rope: *const PkvRope, positions: *const i32,
        in_dtype: c_int, k: *const c_void, v: *const c_void, slot_mapping: *const i32,
        n_tokens: c_int, q: *const c_void, q_out: *mut c_void, n_head: c_int, stream: *mut c_void
    ) -> c_int;

    // ---- token selection (sample.rs:12-55, engine.rs:145-162)
    pub fn pkv_sample(
        logits: *const c_void, dtype: c_int, row_stride: c_longlong, batch: c_int, vocab: c_int,
        temperatures: *const f32, top_k: c_int, top_p: f32, seed: u64, tokens: *mut i32,
        stream: *mut c_void
    ) -> c_int;
    pub fn pkv_sample_exact(
        logits: *const c_void, dtype: c_int, row_stride: c_longlong, batch: c_int, vocab: c_int,
        temperatures: *const f32, top_k: c_int, top_p: f32, seed: u64, tokens: *mut i32,
        stream: *mut c_void
    ) -> c_int;
    pub fn pkv_sample_exact_routes(
        logits: *const c_void, dtype: c_int, row_stride: c_longlong, batch: c_int, vocab: c_int,
        temperatures: *const f32, top_k: c_int, top_p: f32, seed: u64, tokens: *mut i32,
        routes: *mut i32, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_sample_expf(
        in: *const f32, out: *mut f32, n: c_longlong, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_sample_draw(seed: u64) -> f32;

    // ---- block allocator and tables (block_table.rs:5-58)
    pub fn pkv_allocator_new(num_blocks: usize, block_size: usize) -> *mut PkvAllocator;
    pub fn pkv_allocator_free(a: *mut PkvAllocator);
    pub fn pkv_allocator_free_count(a: *const PkvAllocator) -> usize;
    pub fn pkv_allocator_blocks_for(a: *const PkvAllocator, n_tokens: usize) -> usize;
    pub fn pkv_allocator_ensure_capacity(
        a: *mut PkvAllocator, t: *mut PkvTable, n_tokens: usize
    ) -> c_int;
    pub fn pkv_allocator_release(a: *mut PkvAllocator, t: *mut PkvTable);
    pub fn pkv_allocator_locate(
        a: *const PkvAllocator, t: *const PkvTable, pos: usize, block_id: *mut u32,
        slot: *mut usize
    ) -> c_int;
    pub fn pkv_table_new() -> *mut PkvTable;
    pub fn pkv_table_free(t: *mut PkvTable);
    pub fn pkv_table_len(t: *const PkvTable) -> usize;
    pub fn pkv_table_blocks(t: *const PkvTable) -> *const u32;

    // ---- engine step machine (engine.rs:62-237 run_loop bookkeeping)
    pub fn pkv_sched_last_error() -> *const c_char;
    pub fn pkv_sched_create(out: *mut *mut PkvSched, cfg: *const PkvSchedConfig) -> c_int;
    pub fn pkv_sched_destroy(s: *mut PkvSched);
    pub fn pkv_sched_submit(
        s: *mut PkvSched, prompt_len: c_int, max_tokens: c_int, id: *mut i64
    ) -> c_int;
    pub fn pkv_sched_step(s: *mut PkvSched, plan: *mut PkvSchedPlan) -> c_int;
    pub fn pkv_sched_complete(
        s: *mut PkvSched, tokens: *const i32, n: c_int, error: *const c_char
    ) -> c_int;
    pub fn pkv_sched_poll(s: *mut PkvSched, ev: *mut PkvSchedEvent) -> c_int;
    pub fn pkv_sched_fork(
        s: *mut PkvSched, parent: i64, max_tokens: c_int, child: *mut i64
    ) -> c_int;
    pub fn pkv_sched_compact(
        s: *mut PkvSched, src: *mut i32, dst: *mut i32, cap: c_int, n: *mut c_int
    ) -> c_int;
    pub fn pkv_sched_counts(
        s: *const PkvSched, running: *mut c_int, waiting: *mut c_int, free_blocks: *mut c_int
    ) -> c_int;
    pub fn pkv_sched_table(
        s: *const PkvSched, seq: i64, blocks: *mut *const u32, n_blocks: *mut c_int,
        pos: *mut c_int
    ) -> c_int;

    // ---- benchmark and test helpers (no reference counterpart)
    pub fn pkv_pool_fill_normal(pool: *mut PkvPool, seed: u64, stream: *mut c_void) -> c_int;
    pub fn pkv_pool_verify_normal(
        pool: *mut PkvPool, seed: u64, blocks: *const i32, origin: *const i32, n: c_int,
        mismatches: *mut u64, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_pool_read_blocks(
        pool: *mut PkvPool, blocks: *const i32, n: c_int, sum: *mut u64, stream: *mut c_void
    ) -> c_int;
    pub fn pkv_pool_profile(pool: *mut PkvPool, enable: c_int) -> c_int;
    pub fn pkv_pool_profile_read(
        pool: *mut PkvPool, total_ms: *mut f64, launches: *mut c_int
    ) -> c_int;
}

/// A status as the reference's error type on this path (candle_core::Error,
/// attention.rs:39-97): Ok for PKV_OK, else the pool's last error message
/// (the calling thread's when `pool` is null).
pub fn check(rc: c_int, pool: *const PkvPool) -> candle_core::Result<()> {
    if rc == PKV_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(pkv_last_error(pool)) }.to_string_lossy().into_owned();
    Err(candle_core::Error::Msg(format!("pagedkv [{rc}]: {msg}")))
}
