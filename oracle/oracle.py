"""CPU oracle for the paged-KV path (test infrastructure only).

Numpy/ctypes front end of ``pagedkv_oracle.c``.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use this
module, and only as the checker or as the timed CPU baseline; the product
path (``libpagedkv.so``) never calls it.

Each wrapper names the reference function it restates (paths relative to the
reference repository).  How each one is pinned is listed at the top of
``pagedkv_oracle.c`` and exercised by ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liborc.so")

F32, F16, BF16 = 0, 1, 2

_lib = None


def build() -> str:
    """Compile the oracle with gcc (make)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


def _declare(L: ctypes.CDLL) -> None:
    L.orc_kv_write.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _P, _P, _SZ]
    L.orc_kv_write.restype = ctypes.c_int
    L.orc_gather_seq.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _P, _P]
    L.orc_gather_seq.restype = ctypes.c_int
    L.orc_build_mask.argtypes = [_P, _P, _SZ, _SZ, _P]
    L.orc_build_mask.restype = None
    L.orc_sdpa_f32.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P]
    L.orc_sdpa_f32.restype = None
    L.orc_decode_step_f32.argtypes = [_P, _P, _SZ, _SZ, _SZ, _P, _SZ, _P, _P, _P, _P, _P,
                                      _SZ, _SZ, ctypes.c_float, _P]
    L.orc_decode_step_f32.restype = ctypes.c_int
    L.orc_decode_step_faithful_f32.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _P, _P, _P,
                                               _P, _P, _SZ, _SZ, ctypes.c_float, _P]
    L.orc_decode_step_faithful_f32.restype = ctypes.c_int
    L.orc_prefill_chunk_faithful_f32.argtypes = [_P, _P, _SZ, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _SZ,
                                                 _SZ, _P, _P, _P, _SZ, ctypes.c_float, _P]
    L.orc_prefill_chunk_faithful_f32.restype = ctypes.c_int
    L.orc_paged_attention_f64.argtypes = [_P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _P, _SZ, _P, _P,
                                          _SZ, _SZ, ctypes.c_double, _P]
    L.orc_paged_attention_f64.restype = None
    L.orc_prefill_attention_f64.argtypes = [_P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _P, _SZ, _P, _P,
                                            _SZ, _P, _SZ, ctypes.c_double, _P]
    L.orc_prefill_attention_f64.restype = None
    L.orc_prefill_seq_f32.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P]
    L.orc_prefill_seq_f32.restype = None
    L.orc_copy_blocks.argtypes = [_P, _SZ, _SZ, _SZ, _P, _P, _SZ]
    L.orc_copy_blocks.restype = None
    L.orc_compact.argtypes = [_P, _SZ, _SZ, _SZ, _P, _P, _SZ]
    L.orc_compact.restype = ctypes.c_int
    L.orc_decode_inplace.argtypes = [_P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _P, _SZ, _P, _P, _P, _P,
                                     _SZ, _SZ, ctypes.c_float, _P, ctypes.c_int]
    L.orc_decode_inplace.restype = None
    L.orc_prefill_inplace.argtypes = [_P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _P, _SZ, _P, _P, _SZ,
                                      _P, _P, _P, _SZ, ctypes.c_float, _P, ctypes.c_int]
    L.orc_prefill_inplace.restype = None
    L.orc_rope_table.argtypes = [_SZ, ctypes.c_float, _SZ, _P, _P]
    L.orc_rope_table.restype = None
    L.orc_rope_apply.argtypes = [_P, _P, _SZ, _SZ, _SZ, _P, _P, _P]
    L.orc_rope_apply.restype = None
    L.orc_pcg32_output.argtypes = [ctypes.c_uint64]
    L.orc_pcg32_output.restype = ctypes.c_uint32
    L.orc_chacha_block.argtypes = [_P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, _P]
    L.orc_chacha_block.restype = None
    L.orc_seed_from_u64.argtypes = [ctypes.c_uint64, _P]
    L.orc_seed_from_u64.restype = None
    L.orc_sample_draw.argtypes = [ctypes.c_uint64]
    L.orc_sample_draw.restype = ctypes.c_float
    L.orc_argmax.argtypes = [_P, _SZ]
    L.orc_argmax.restype = ctypes.c_int64
    L.orc_sample.argtypes = [_P, _SZ, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                             ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    L.orc_sample.restype = ctypes.c_int64
    L.orc_threads.argtypes = [ctypes.c_int]
    L.orc_threads.restype = ctypes.c_int
    L.orc_expf_host.argtypes = [_P, _P, _SZ]
    L.orc_expf_host.restype = None
    L.orc_expf_glibc.argtypes = [ctypes.c_float]
    L.orc_expf_glibc.restype = ctypes.c_float
    L.orc_exp2_tab_entry.argtypes = [ctypes.c_int]
    L.orc_exp2_tab_entry.restype = ctypes.c_uint64
    L.orc_expf_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_uint32)]
    L.orc_expf_mismatches.restype = ctypes.c_int64


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def widen(a: np.ndarray, dtype: int) -> np.ndarray:
    """Exact widening of stored f16/bf16 bits (uint16) or f32 to float32."""
    if dtype == F32:
        return np.ascontiguousarray(a, dtype=np.float32)
    if dtype == F16:
        return np.ascontiguousarray(a).view(np.float16).astype(np.float32)
    u = np.ascontiguousarray(a).view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


# --------------------------------------------------------------------------
# byte-moving functions (bit-exact)
# --------------------------------------------------------------------------
def kv_write(k_pool: np.ndarray, v_pool: np.ndarray, block_size: int,
             blocks: np.ndarray, start_pos: int, k: np.ndarray, v: np.ndarray) -> None:
    """KvPool::write (attention.rs:57-83) on pools shaped
    (num_blocks, block_size, n_kv, hd); k, v: (n_new, n_kv, hd)."""
    n_kv, hd = k_pool.shape[2], k_pool.shape[3]
    blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
    k = np.ascontiguousarray(k, dtype=k_pool.dtype)
    v = np.ascontiguousarray(v, dtype=v_pool.dtype)
    rc = lib().orc_kv_write(_p(k_pool), _p(v_pool), k_pool.itemsize, block_size, n_kv, hd,
                            _p(blocks), blocks.size, start_pos, _p(k), _p(v), k.shape[0])
    if rc != 0:
        raise IndexError("position beyond block table (the reference panics here)")


def gather_seq(k_pool: np.ndarray, v_pool: np.ndarray, block_size: int,
               blocks: np.ndarray, length: int) -> tuple[np.ndarray, np.ndarray]:
    """KvPool::gather_seq (attention.rs:85-97) -> (len, n_kv, hd) each."""
    n_kv, hd = k_pool.shape[2], k_pool.shape[3]
    blocks = np.ascontiguousarray(blocks, dtype=np.uint32)
    ok = np.empty((length, n_kv, hd), dtype=k_pool.dtype)
    ov = np.empty((length, n_kv, hd), dtype=v_pool.dtype)
    rc = lib().orc_gather_seq(_p(k_pool), _p(v_pool), k_pool.itemsize, block_size, n_kv, hd,
                              _p(blocks), blocks.size, length, _p(ok), _p(ov))
    if rc != 0:
        raise IndexError("position beyond block table (the reference panics here)")
    return ok, ov


def build_mask(seq_lens, q_positions, kv_len: int) -> np.ndarray:
    """build_mask (attention.rs:11-28) -> (batch, 1, 1, kv_len) float32."""
    sl = np.ascontiguousarray(seq_lens, dtype=np.int64)
    qp = np.ascontiguousarray(q_positions, dtype=np.int64)
    out = np.empty((sl.size, kv_len), dtype=np.float32)
    lib().orc_build_mask(_p(sl), _p(qp), sl.size, kv_len, _p(out))
    return out.reshape(sl.size, 1, 1, kv_len)


def copy_blocks(pool: np.ndarray, n_layers: int, block_bytes: int, src, dst) -> None:
    """Closed form of block copy over [n_layers][2][pool bytes] (uint8 array)."""
    src = np.ascontiguousarray(src, dtype=np.int32)
    dst = np.ascontiguousarray(dst, dtype=np.int32)
    layer_bytes = pool.nbytes // (n_layers * 2)
    lib().orc_copy_blocks(_p(pool), n_layers, layer_bytes, block_bytes, _p(src), _p(dst), src.size)


def compact(pool: np.ndarray, n_layers: int, block_bytes: int, src, dst) -> None:
    """Closed form of compaction: new[dst[i]] = old[src[i]], out of place."""
    src = np.ascontiguousarray(src, dtype=np.int32)
    dst = np.ascontiguousarray(dst, dtype=np.int32)
    layer_bytes = pool.nbytes // (n_layers * 2)
    if lib().orc_compact(_p(pool), n_layers, layer_bytes, block_bytes, _p(src), _p(dst), src.size):
        raise MemoryError("oracle compact: host allocation failed")


# --------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------
def sdpa_f32(q, k, v, mask, n_head: int, n_kv_head: int, scale: float | None = None) -> np.ndarray:
    """sdpa (attention.rs:100-136) in f32.  q: (B,H,Lq,hd); k,v: (B,KVH,kv,hd);
    mask: (B,1,Lq,kv).  Returns (B, Lq, H*hd)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    mask = np.ascontiguousarray(mask, dtype=np.float32)
    B, H, Lq, hd = q.shape
    kv = k.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty((B, Lq, H * hd), dtype=np.float32)
    lib().orc_sdpa_f32(_p(q), _p(k), _p(v), _p(mask), B, H, n_kv_head, Lq, kv, hd,
                       float(scale), _p(out))
    return out


def decode_step_faithful_f32(k_pool, v_pool, block_size: int, tables, seq_lens, positions,
                             q, k_new, v_new, scale: float | None = None) -> np.ndarray:
    """decode_step_f32 with the reference's cost: every appended row copies
    the whole K and V pool first (slice_assign, attention.rs:73-80)."""
    assert k_pool.dtype == np.float32 and v_pool.dtype == np.float32
    NB, KVH, hd = k_pool.shape[0], k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.uint32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int64)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_new = np.ascontiguousarray(k_new, dtype=np.float32)
    v_new = np.ascontiguousarray(v_new, dtype=np.float32)
    B, H = q.shape[0], q.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty((B, H * hd), dtype=np.float32)
    rc = lib().orc_decode_step_faithful_f32(_p(k_pool), _p(v_pool), NB, block_size, KVH, hd,
                                            _p(tables), tables.shape[1], _p(sl), _p(pos), _p(q),
                                            _p(k_new), _p(v_new), B, H, float(scale), _p(out))
    if rc:
        raise IndexError("position beyond block table" if rc == -1 else "allocation failed")
    return out


def prefill_chunk_faithful_f32(k_pool, v_pool, block_size: int, table, prior: int, q, k_new,
                               v_new, scale: float | None = None,
                               n_copies: int | None = None) -> np.ndarray:
    """The reference's cost model for one prompt chunk on f32 pools: a full K
    and V pool copy before each of the first n_copies token writes (default:
    every token; slice_assign, attention.rs:73-80), the sequence's rows
    gathered, dense masked sdpa over all prior + C keys per query
    (transformer.rs:139-196).  q: (C, H, hd); k_new/v_new: (C, KVH, hd).
    Pools are modified (the writes).  Returns (C, H*hd)."""
    assert k_pool.dtype == np.float32 and v_pool.dtype == np.float32
    NB, KVH, hd = k_pool.shape[0], k_pool.shape[2], k_pool.shape[3]
    table = np.ascontiguousarray(table, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_new = np.ascontiguousarray(k_new, dtype=np.float32)
    v_new = np.ascontiguousarray(v_new, dtype=np.float32)
    C, H = q.shape[0], q.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    if n_copies is None:
        n_copies = C
    out = np.empty((C, H * hd), dtype=np.float32)
    rc = lib().orc_prefill_chunk_faithful_f32(_p(k_pool), _p(v_pool), NB, block_size, KVH, hd,
                                              _p(table), table.size, int(prior), C, int(n_copies),
                                              _p(q), _p(k_new), _p(v_new), H, float(scale),
                                              _p(out))
    if rc:
        raise IndexError("position beyond block table" if rc == -1 else "allocation failed")
    return out


def decode_step_f32(k_pool, v_pool, block_size: int, tables, seq_lens, positions,
                    q, k_new, v_new, scale: float | None = None) -> np.ndarray:
    """Transformer::decode_step attention slice (transformer.rs:271-292) in f32.
    Pools (num_blocks, bs, KVH, hd) float32 are modified (append).
    tables: (B, max_nb); q: (B, H, hd); k_new/v_new: (B, KVH, hd).
    Returns (B, H*hd)."""
    assert k_pool.dtype == np.float32 and v_pool.dtype == np.float32
    KVH, hd = k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.uint32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int64)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    k_new = np.ascontiguousarray(k_new, dtype=np.float32)
    v_new = np.ascontiguousarray(v_new, dtype=np.float32)
    B, H = q.shape[0], q.shape[1]
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty((B, H * hd), dtype=np.float32)
    rc = lib().orc_decode_step_f32(_p(k_pool), _p(v_pool), block_size, KVH, hd, _p(tables),
                                   tables.shape[1], _p(sl), _p(pos), _p(q), _p(k_new),
                                   _p(v_new), B, H, float(scale), _p(out))
    if rc:
        raise IndexError("position beyond block table")
    return out


def paged_attention_f64(k_pool, v_pool, dtype: int, block_size: int, tables, ctx_lens,
                        q, scale: float) -> np.ndarray:
    """Closed-form fp64 paged decode attention.  Pools hold stored elements
    (uint16 bits for f16/bf16); q: (B, H, hd) float32.  Returns (B, H*hd) f64."""
    KVH, hd = k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.uint32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, H = q.shape[0], q.shape[1]
    out = np.empty((B, H * hd), dtype=np.float64)
    lib().orc_paged_attention_f64(_p(np.ascontiguousarray(k_pool)), _p(np.ascontiguousarray(v_pool)),
                                  dtype, block_size, KVH, hd, _p(tables), tables.shape[1],
                                  _p(cl), _p(q), B, H, float(scale), _p(out))
    return out


def prefill_attention_f64(k_pool, v_pool, dtype: int, block_size: int, tables, cu_q_lens,
                          ctx_lens, q, scale: float) -> np.ndarray:
    """Closed-form fp64 chunked-prefill attention.  q: (T, H, hd) float32.
    Returns (T, H*hd) f64."""
    KVH, hd = k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.uint32)
    cu = np.ascontiguousarray(cu_q_lens, dtype=np.int64)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int64)
    q = np.ascontiguousarray(q, dtype=np.float32)
    T, H = q.shape[0], q.shape[1]
    out = np.empty((T, H * hd), dtype=np.float64)
    lib().orc_prefill_attention_f64(_p(np.ascontiguousarray(k_pool)), _p(np.ascontiguousarray(v_pool)),
                                    dtype, block_size, KVH, hd, _p(tables), tables.shape[1],
                                    _p(cu), _p(cl), cl.size, _p(q), H, float(scale), _p(out))
    return out


def prefill_seq_f32(q, k, v, n_kv_head: int, scale: float | None = None) -> np.ndarray:
    """prefill_seq attention slice (transformer.rs:139-196) in f32.
    q: (H, N, hd); k, v: (KVH, N, hd).  Returns (N, H*hd)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    H, N, hd = q.shape
    if scale is None:
        scale = 1.0 / np.sqrt(hd)
    out = np.empty((N, H * hd), dtype=np.float32)
    lib().orc_prefill_seq_f32(_p(q), _p(k), _p(v), H, n_kv_head, N, hd, float(scale), _p(out))
    return out


def decode_inplace(k_pool, v_pool, dtype: int, block_size: int, tables, ctx_lens, q,
                   k_new, v_new, scale: float, n_threads: int = 0) -> np.ndarray:
    """CPU baseline: reference decode math, in place, ragged, OpenMP.
    Pools/q/k_new/v_new hold stored elements of `dtype`.  Returns (B, H*hd) f32."""
    KVH, hd = k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    B, H = q.shape[0], q.shape[1]
    out = np.empty((B, H * hd), dtype=np.float32)
    kn = _p(k_new) if k_new is not None else None
    vn = _p(v_new) if v_new is not None else None
    lib().orc_decode_inplace(_p(k_pool), _p(v_pool), dtype, block_size, KVH, hd, _p(tables),
                             tables.shape[1], _p(cl), _p(q), kn, vn, B, H, float(scale),
                             _p(out), int(n_threads))
    return out


def prefill_inplace(k_pool, v_pool, dtype: int, block_size: int, tables, cu_q_lens, ctx_lens,
                    q, k_new, v_new, scale: float, n_threads: int = 0) -> np.ndarray:
    """CPU baseline: reference prefill math (f32, causal) over a prior
    context, chunk K/V stored first, in place, OpenMP.  Pools/q/k_new/v_new
    hold stored elements of `dtype`; q (T, H, hd).  Returns (T, H*hd) f32."""
    KVH, hd = k_pool.shape[2], k_pool.shape[3]
    tables = np.ascontiguousarray(tables, dtype=np.int32)
    cu = np.ascontiguousarray(cu_q_lens, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    T, H = q.shape[0], q.shape[1]
    out = np.empty((T, H * hd), dtype=np.float32)
    kn = _p(k_new) if k_new is not None else None
    vn = _p(v_new) if v_new is not None else None
    lib().orc_prefill_inplace(_p(k_pool), _p(v_pool), dtype, block_size, KVH, hd, _p(tables),
                              tables.shape[1], _p(cu), _p(cl), cl.size, _p(q), kn, vn, H,
                              float(scale), _p(out), int(n_threads))
    return out


def rope_table(rope_dim: int, freq_base: float, max_seq: int):
    """Rope::new (rope.rs:14-23): f32 cos/sin tables (max_seq, rope_dim/2)."""
    half = rope_dim // 2
    c = np.zeros((max_seq, half), np.float32)
    s = np.zeros((max_seq, half), np.float32)
    lib().orc_rope_table(rope_dim, freq_base, max_seq, _p(c), _p(s))
    return c, s


def rope_apply(x, cos_t, sin_t, positions) -> np.ndarray:
    """apply_rope (rope.rs:38-42) on x (n_tokens, n_head, d) float32, each
    token at its own position (transformer.rs:252-269)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, h, d = x.shape
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    assert pos.shape == (n,) and cos_t.shape[1] * 2 == d
    assert pos.min(initial=0) >= 0 and pos.max(initial=0) < cos_t.shape[0]
    out = np.empty_like(x)
    lib().orc_rope_apply(_p(x), _p(out), n, h, d, _p(np.ascontiguousarray(cos_t)),
                         _p(np.ascontiguousarray(sin_t)), _p(pos))
    return out


def threads(requested: int = 0) -> int:
    return int(lib().orc_threads(int(requested)))


# ---------------------------------------------------------------------------
# token selection (crates/ai-engine-runtime/src/sample.rs:12-55)
# ---------------------------------------------------------------------------
def pcg32_output(state: int) -> int:
    return int(lib().orc_pcg32_output(state))


def chacha_block(key, counter: int, stream: int, rounds: int) -> np.ndarray:
    k = np.ascontiguousarray(key, dtype=np.uint32)
    assert k.size == 8
    out = np.zeros(16, np.uint32)
    lib().orc_chacha_block(_p(k), counter, stream, rounds, _p(out))
    return out


def seed_from_u64(seed: int) -> np.ndarray:
    out = np.zeros(8, np.uint32)
    lib().orc_seed_from_u64(seed, _p(out))
    return out


def sample_draw(seed: int) -> float:
    """StdRng::seed_from_u64(seed).gen::<f32>() (sample.rs:41-42)."""
    return float(lib().orc_sample_draw(seed))


def argmax(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_argmax(_p(x), x.size))


def sample(logits, temperature: float, top_k: int | None = None, top_p: float | None = None,
           seed: int = 42, precise: bool = False) -> tuple[int, float]:
    """sample() of sample.rs:12-48 -> (token, margin of the decisive sums).
    precise=False: the reference's f32 arithmetic; True: the same steps with
    exp, normalisation and running sums in double."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    m = ctypes.c_double()
    tok = lib().orc_sample(_p(x) if x.size else None, x.size, temperature, top_k or 0,
                           0 if top_p is None else 1, 0.0 if top_p is None else top_p, seed,
                           1 if precise else 0, ctypes.byref(m))
    return int(tok), float(m.value)


def expf_host(x) -> np.ndarray:
    """The host C library's expf, element by element (what the reference's
    f32::exp calls); numpy's float32 exp is a different implementation."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_expf_host(_p(x), _p(out), x.size)
    return out


def expf_glibc(x: float) -> float:
    """The device's restatement of glibc's expf, evaluated on the host."""
    return float(lib().orc_expf_glibc(x))


def exp2_tab_entry(i: int) -> int:
    return int(lib().orc_exp2_tab_entry(i))


def expf_mismatches(lo: int, hi: int, step: int = 1) -> tuple[int, int]:
    """(count, first bit pattern) of inputs lo, lo + step, ... <= hi (float
    bit patterns) where the restatement and the host expf differ."""
    f = ctypes.c_uint32()
    n = lib().orc_expf_mismatches(lo, hi, step, ctypes.byref(f))
    return int(n), int(f.value)
