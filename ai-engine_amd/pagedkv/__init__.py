"""pagedkv -- Python front end of libpagedkv, the MI355X paged-KV engine.

Mirrors the reference's host API of the candle `engine = "paged"` path
(crates/ai-engine-candle/src/paged/{block_table,attention}.rs) on top of the
C ABI in include/pagedkv.h:

  BlockAllocator / BlockTable   block_table.rs:5-58 (C++ host code)
  PagedKvCache                  the reference's Vec<KvPool> (engine.rs:70-72)
  PagedKvCache.layer(l) -> KvPool  KvPool::{write, gather_seq} (attention.rs:39-97)
  KvPool.decode_attention       build_mask + sdpa of the decode step
                                (attention.rs:11-28,100-136, transformer.rs:271-292)
  KvPool.prefill_attention      prefill_seq's attention (transformer.rs:139-196)

torch tensors are used only as device memory and for the current stream.
"""
from __future__ import annotations

import ctypes
import sys
import math
from typing import Sequence

from ._lib import (BF16, F16, F32, K, V, CapacityError, PagedKvError, check, lib,
                   LIB_PATH)

__all__ = [
    "BlockAllocator", "BlockTable", "PagedKvCache", "KvPool", "Rope", "rope_tables_host",
    "CapacityError",
    "PagedKvError", "F32", "F16", "BF16", "lib", "LIB_PATH", "torch_dtype",
    "pkv_dtype",
]


# ---------------------------------------------------------------------------
# host block bookkeeping (C++), block_table.rs:5-58
# ---------------------------------------------------------------------------
class BlockTable:
    """One sequence's ordered physical block ids (block_table.rs:10-14)."""

    def __init__(self) -> None:
        self._h = lib().pkv_table_new()
        if not self._h:
            raise MemoryError("pkv_table_new")

    def __del__(self, _finalizing=sys.is_finalizing) -> None:
        h = getattr(self, "_h", None)
        if h and not _finalizing():
            lib().pkv_table_free(h)
            self._h = None

    @property
    def blocks(self) -> list[int]:
        n = lib().pkv_table_len(self._h)
        if n == 0:
            return []
        ptr = lib().pkv_table_blocks(self._h)
        return [ptr[i] for i in range(n)]

    def __len__(self) -> int:
        return int(lib().pkv_table_len(self._h))


class BlockAllocator:
    """Fixed-size block pool with a LIFO free list (block_table.rs:16-58)."""

    def __init__(self, num_blocks: int, block_size: int) -> None:
        self._h = lib().pkv_allocator_new(num_blocks, block_size)
        if not self._h:
            raise ValueError("pkv_allocator_new: bad arguments or out of memory")
        self.block_size = block_size

    def __del__(self, _finalizing=sys.is_finalizing) -> None:
        h = getattr(self, "_h", None)
        if h and not _finalizing():
            lib().pkv_allocator_free(h)
            self._h = None

    def free_count(self) -> int:
        return int(lib().pkv_allocator_free_count(self._h))

    def blocks_for(self, n_tokens: int) -> int:
        return int(lib().pkv_allocator_blocks_for(self._h, n_tokens))

    def ensure_capacity(self, table: BlockTable, n_tokens: int) -> None:
        """Raises CapacityError (nothing allocated) when the pool is short."""
        check(lib().pkv_allocator_ensure_capacity(self._h, table._h, n_tokens))

    def release(self, table: BlockTable) -> None:
        lib().pkv_allocator_release(self._h, table._h)

    def locate(self, table: BlockTable, pos: int) -> tuple[int, int]:
        blk = ctypes.c_uint32()
        slot = ctypes.c_size_t()
        rc = lib().pkv_allocator_locate(self._h, table._h, pos, ctypes.byref(blk),
                                        ctypes.byref(slot))
        if rc != 0:
            raise IndexError(f"position {pos} beyond the block table")
        return int(blk.value), int(slot.value)

    def slot(self, table: BlockTable, pos: int) -> int:
        b, s = self.locate(table, pos)
        return b * self.block_size + s


# ---------------------------------------------------------------------------
# device pool
# ---------------------------------------------------------------------------
def pkv_dtype(t) -> int:
    import torch
    m = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
    if t not in m:
        raise TypeError(f"unsupported dtype {t}")
    return m[t]


def torch_dtype(d: int):
    import torch
    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[d]


def _stream_ptr(stream) -> int | None:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream) or None


def _dev_ptr(t) -> int:
    return int(t.data_ptr())


def _i32(x, device):
    import torch
    if isinstance(x, torch.Tensor):
        t = x.to(device=device, dtype=torch.int32)
    else:
        t = torch.as_tensor(x, dtype=torch.int32).to(device)
    return t.contiguous()


def rope_tables_host(rope_dim: int, freq_base: float, max_seq: int):
    """Rope::new's cos/sin tables (rope.rs:14-23) computed by the library on
    the host: two float32 arrays (max_seq, rope_dim // 2)."""
    import numpy as np
    c = np.zeros((max_seq, rope_dim // 2), np.float32)
    s = np.zeros_like(c)
    check(lib().pkv_rope_tables_host(rope_dim, freq_base, max_seq, c.ctypes.data,
                                     s.ctypes.data), None)
    return c, s


def sample_draw(seed: int = 42) -> float:
    """StdRng::seed_from_u64(seed).gen::<f32>() (sample.rs:41-42), the fixed
    draw that sample() compares the cumulative probabilities with."""
    return float(lib().pkv_sample_draw(seed))


def sample(logits, temperatures=None, top_k: int | None = None, top_p: float | None = None,
           seed: int = 42, out=None, stream=None, exact: bool = True, routes=None):
    """Token per logits row on the device: argmax / sample() of sample.rs:12-55.
    logits: (batch, vocab) f32/f16/bf16 with unit stride along vocab;
    temperatures: (batch,) float32 on the device (None: all greedy).
    exact=True (pkv_sample_exact, the default since the engine needs the
    reference's tokens): the reference's f32 arithmetic bit for bit, so the
    token is the reference's on every row.  It allocates its scratch on the
    stream for each call (hipMallocAsync, freed in stream order after the
    launch): 1 MiB per row for 16-bit logits (the row's runs of equal
    values); for f32 logits 8 bytes per logit (1 MiB per 128k-entry row),
    rows taken in rounds of at most 512 MiB.  top_p=None is the reference's
    None (no cut; passed as NaN), which differs from Some(1.0): with f32
    sums, 1.0 cuts where the running sum first reaches 1.0.
    exact=False (pkv_sample): faster, allocates only for rows split over
    several workgroups; sums the probabilities exactly, so a row can differ
    where the reference's f32 running sum lands within its rounding of r or
    top_p (top_p=None is 1.0 there, the same as no cut in exact sums).
    routes (exact=True only): a (batch,) int32 device tensor that receives
    the kernel that selected each row (pkv_sample_exact_routes: 0 argmax,
    1 buckets of f32 logits, 2 runs of equal 16-bit values, 3 radix sort).
    Returns (batch,) int32 on the device."""
    import torch
    if logits.dim() != 2 or (logits.shape[1] > 1 and logits.stride(1) != 1):
        raise ValueError("logits must be (batch, vocab) with unit stride along vocab")
    B, V = logits.shape
    dev = logits.device
    # The kernels run on `stream`: it first waits for the work queued so far
    # on the current stream (which produced the logits), and the temporaries
    # made here are allocated on it, so they are neither read early nor
    # reused before the launch has run.
    cur = torch.cuda.current_stream(dev)
    s = cur if stream is None else stream
    if s != cur:
        s.wait_stream(cur)
    if routes is not None and not exact:
        raise ValueError("routes are reported by the exact path only")
    if exact:  # top_p None is NaN; any other value is Some(top_p)
        fn, tp = lib().pkv_sample_exact, float("nan") if top_p is None else float(top_p)
    else:      # top_p None is 1.0 (no cut in exact arithmetic)
        fn, tp = lib().pkv_sample, 1.0 if top_p is None else float(top_p)
    extra = ()
    if routes is not None:
        if routes.dtype != torch.int32 or routes.numel() != B or not routes.is_contiguous():
            raise ValueError("routes must be a contiguous int32 tensor of one entry per row")
        fn, extra = lib().pkv_sample_exact_routes, (_dev_ptr(routes),)
    with torch.cuda.stream(s):
        if out is None:
            out = torch.empty(B, dtype=torch.int32, device=dev)
        t = None
        if temperatures is not None:
            t = torch.as_tensor(temperatures, dtype=torch.float32).to(dev).contiguous()
            if t.numel() != B:
                raise ValueError("temperatures must have one value per row")
        check(fn(_dev_ptr(logits) if V else None, pkv_dtype(logits.dtype),
                 logits.stride(0) if B > 1 else V, B, V,
                 _dev_ptr(t) if t is not None else None, top_k or 0, tp, seed, _dev_ptr(out),
                 *extra, _stream_ptr(s)), None)
    return out


def sample_expf(x):
    """expf as the exact sampler computes it (glibc's algorithm) for a float32
    device tensor; returns a new tensor."""
    import torch
    x = x.contiguous()
    if x.dtype != torch.float32:
        raise ValueError("float32 input expected")
    out = torch.empty_like(x)
    check(lib().pkv_sample_expf(_dev_ptr(x), _dev_ptr(out), x.numel(),
                                _stream_ptr(torch.cuda.current_stream(x.device))), None)
    return out


class Rope:
    """The reference's Rope (rope.rs:6-33): cos/sin tables in device memory;
    apply() is apply_rope (rope.rs:38-42) with per-token positions."""

    def __init__(self, rope_dim: int, freq_base: float, max_seq: int, device: int = 0) -> None:
        import torch
        h = ctypes.c_void_p()
        check(lib().pkv_rope_create(ctypes.byref(h), rope_dim, freq_base, max_seq, device), None)
        self._h = h
        self.rope_dim, self.freq_base, self.max_seq = rope_dim, freq_base, max_seq
        self.device = torch.device("cuda", device)

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h:
            lib().pkv_rope_destroy(h)
            self._h = None

    def __del__(self, _finalizing=sys.is_finalizing) -> None:
        # at interpreter exit the module's globals may already be gone; the
        # process end releases the device memory
        if not _finalizing():
            self.close()

    def apply(self, x, positions, out_dtype=None, out=None, stream=None):
        """x: (n_tokens, n_head, rope_dim) f32/f16/bf16 on the device;
        positions: (n_tokens,) int32.  Returns the rotated rows."""
        import torch
        if x.dim() != 3 or x.shape[2] != self.rope_dim:
            raise ValueError(f"x must be (n, heads, {self.rope_dim})")
        xx = x.contiguous()
        if out is None:
            out = torch.empty(xx.shape, dtype=out_dtype or xx.dtype, device=xx.device)
        pos = _i32(positions, xx.device)
        check(lib().pkv_rope_apply(self._h, _dev_ptr(xx), pkv_dtype(xx.dtype), _dev_ptr(out),
                                   pkv_dtype(out.dtype), _dev_ptr(pos), xx.shape[0],
                                   xx.shape[1], _stream_ptr(stream)), None)
        return out

    def check(self) -> None:
        check(lib().pkv_rope_check(self._h), None)


class PagedKvCache:
    """K/V pools of every layer on one GPU (the reference's Vec<KvPool>,
    engine.rs:70-72; KvPool::new, attention.rs:39-55).  Zero-initialised,
    layout [layer][K|V][num_blocks][block_size][n_kv_head][head_dim]."""

    def __init__(self, n_layers: int, num_blocks: int, block_size: int, n_kv_head: int,
                 head_dim: int, dtype=None, device: int = 0) -> None:
        import torch
        if dtype is None:
            dtype = torch.float32
        self.dtype = dtype
        self.n_layers, self.num_blocks, self.block_size = n_layers, num_blocks, block_size
        self.n_kv_head, self.head_dim, self.device_index = n_kv_head, head_dim, device
        self.device = torch.device("cuda", device)
        h = ctypes.c_void_p()
        rc = lib().pkv_pool_create(ctypes.byref(h), n_layers, num_blocks, block_size,
                                   n_kv_head, head_dim, pkv_dtype(dtype), device)
        check(rc, None)
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h:
            lib().pkv_pool_destroy(h)
            self._h = None

    def __del__(self, _finalizing=sys.is_finalizing) -> None:
        # at interpreter exit the module's globals may already be gone; the
        # process end releases the device memory
        if not _finalizing():
            self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def layer(self, l: int) -> "KvPool":
        if not 0 <= l < self.n_layers:
            raise IndexError(l)
        return KvPool(self, l)

    @property
    def layer_bytes(self) -> int:
        return int(lib().pkv_pool_layer_bytes(self._h))

    @property
    def block_bytes(self) -> int:
        return self.layer_bytes // self.num_blocks

    def fill_normal(self, seed: int, stream=None) -> None:
        check(lib().pkv_pool_fill_normal(self._h, seed, _stream_ptr(stream)), self._h)

    def verify_normal(self, seed: int, blocks, origin, stream=None) -> int:
        """16-byte chunks of blocks[i] (all layers, K and V) that differ from
        what fill_normal(seed) wrote into block origin[i] (synchronous)."""
        b = _i32(blocks, self.device)
        o = _i32(origin, self.device)
        if b.numel() != o.numel():
            raise ValueError("blocks and origin must have the same length")
        n = ctypes.c_uint64()
        check(lib().pkv_pool_verify_normal(self._h, seed, _dev_ptr(b), _dev_ptr(o), b.numel(),
                                           ctypes.byref(n), _stream_ptr(stream)), self._h)
        return int(n.value)

    def read_blocks(self, blocks, out=None, stream=None):
        """Reads every byte of blocks[i] (all layers, K and V) on the device
        and adds their 32-bit words (mod 2^64) into out, a device int64
        tensor of one element holding the unsigned sum's bits (zeroed here
        unless given); returns out.  Asynchronous."""
        import torch
        b = _i32(blocks, self.device)
        if out is None:
            out = torch.zeros(1, dtype=torch.int64, device=self.device)
        if out.dtype != torch.int64 or out.numel() < 1 or not out.is_cuda:
            raise ValueError("out must be a device int64 tensor")
        check(lib().pkv_pool_read_blocks(self._h, _dev_ptr(b), b.numel(), _dev_ptr(out),
                                         _stream_ptr(stream)), self._h)
        return out

    def copy_blocks(self, src, dst, stream=None) -> None:
        """Copy-on-write: block dst[i] <- src[i] in every layer, K and V."""
        s = _i32(src, self.device)
        d = _i32(dst, self.device)
        if s.numel() != d.numel():
            raise ValueError("src/dst length mismatch")
        check(lib().pkv_copy_blocks(self._h, _dev_ptr(s), _dev_ptr(d), s.numel(),
                                    _stream_ptr(stream)), self._h)

    def compact(self, src: Sequence[int], dst: Sequence[int], stream=None) -> None:
        """In-place block moves src[i] -> dst[i] (sets may overlap)."""
        import numpy as np
        s = np.ascontiguousarray(src, dtype=np.int32)
        d = np.ascontiguousarray(dst, dtype=np.int32)
        if s.size != d.size:
            raise ValueError("src/dst length mismatch")
        P = ctypes.POINTER(ctypes.c_int32)
        check(lib().pkv_compact(self._h, s.ctypes.data_as(P), d.ctypes.data_as(P), s.size,
                                _stream_ptr(stream)), self._h)

    def check(self) -> None:
        """Raise if a kernel met an out-of-range id or length since last check."""
        check(lib().pkv_pool_check(self._h), self._h)

    def profile(self, enable: bool) -> None:
        """Record HIP events around every decode call's main kernel."""
        check(lib().pkv_pool_profile(self._h, 1 if enable else 0), self._h)

    def profile_read(self) -> tuple[float, int]:
        """(summed main-kernel ms, launches) since the last read."""
        ms = ctypes.c_double()
        n = ctypes.c_int()
        check(lib().pkv_pool_profile_read(self._h, ctypes.byref(ms), ctypes.byref(n)), self._h)
        return float(ms.value), int(n.value)

    def decode_workspace_bytes(self, batch: int, n_head: int, max_context_len: int) -> int:
        return int(lib().pkv_decode_workspace_bytes(self._h, batch, n_head, max_context_len))

    def reserve_decode(self, batch: int, n_head: int, max_context_len: int) -> None:
        check(lib().pkv_pool_reserve_decode(self._h, batch, n_head, max_context_len), self._h)

    def prefill_workspace_bytes(self, n_seqs: int, n_head: int, max_q_len: int,
                                max_context_len: int) -> int:
        return int(lib().pkv_prefill_workspace_bytes(self._h, n_seqs, n_head, max_q_len,
                                                     max_context_len))

    def reserve_prefill(self, n_seqs: int, n_head: int, max_q_len: int,
                        max_context_len: int) -> None:
        check(lib().pkv_pool_reserve_prefill(self._h, n_seqs, n_head, max_q_len,
                                             max_context_len), self._h)

    # raw byte access (synchronous), for tests and checkpoints
    def read_bytes(self, layer: int, which: int, offset: int = 0, nbytes: int | None = None):
        import numpy as np
        if nbytes is None:
            nbytes = self.layer_bytes - offset
        buf = np.empty(nbytes, dtype=np.uint8)
        check(lib().pkv_pool_read(self._h, layer, which, offset, nbytes, buf.ctypes.data), self._h)
        return buf

    def write_bytes(self, layer: int, which: int, data, offset: int = 0) -> None:
        import numpy as np
        a = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        check(lib().pkv_pool_write(self._h, layer, which, offset, a.ctypes.data, a.size), self._h)


class KvPool:
    """One layer of a PagedKvCache: the reference's KvPool (attention.rs:30-98)."""

    def __init__(self, cache: PagedKvCache, layer: int) -> None:
        self.cache = cache
        self.layer_index = layer

    @property
    def _h(self):
        return self.cache.handle

    # -- KvPool::write (attention.rs:57-83) --------------------------------
    def write(self, alloc: BlockAllocator, table: BlockTable, start_pos: int, k, v,
              stream=None) -> None:
        n_new = int(k.shape[0])
        slots = [alloc.slot(table, start_pos + i) for i in range(n_new)]
        self.append(k, v, slots, stream)

    def append(self, k, v, slot_mapping, stream=None) -> None:
        """Scatter k, v (n, n_kv, hd) to the given slots (int32, -1 = skip)."""
        c = self.cache
        self._check_rows(k, "k")
        self._check_rows(v, "v")
        sm = _i32(slot_mapping, c.device)
        if sm.numel() != k.shape[0] or v.shape[0] != k.shape[0]:
            raise ValueError("slot_mapping / k / v lengths differ")
        check(lib().pkv_append(self._h, self.layer_index, _dev_ptr(k), _dev_ptr(v),
                               _dev_ptr(sm), k.shape[0], _stream_ptr(stream)), self._h)

    def append_rope(self, rope: "Rope", k, v, slot_mapping, positions, q=None, q_out=None,
                    stream=None):
        """prefill_seq's glue (transformer.rs:160-174) in one launch: rotate k
        (n, n_kv, hd) by `positions`, store it and v at `slot_mapping`, and,
        with q (n, H, hd), return q rotated into the pool dtype (into q_out if
        given).  k, v, q share one dtype: float32 or the pool dtype."""
        import torch
        c = self.cache
        n = int(k.shape[0])
        if q is not None and q.dtype != k.dtype:
            raise TypeError("q must have k's dtype")
        if k.dtype not in (torch.float32, c.dtype) or v.dtype != k.dtype:
            raise TypeError("k and v must be float32 or the pool dtype, and equal")
        for t, name in ((k, "k"), (v, "v")):
            if t.shape != (n, c.n_kv_head, c.head_dim) or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous ({n}, {c.n_kv_head}, {c.head_dim})")
        sm = _i32(slot_mapping, c.device)
        pos = _i32(positions, c.device)
        if sm.numel() != n or pos.numel() != n:
            raise ValueError("slot_mapping / positions / k lengths differ")
        H = 0
        if q is not None:
            if q.dim() != 3 or q.shape[0] != n or q.shape[2] != c.head_dim:
                raise ValueError(f"q must be ({n}, H, {c.head_dim})")
            q = q.contiguous()
            H = int(q.shape[1])
            if q_out is None:
                q_out = torch.empty(q.shape, dtype=c.dtype, device=c.device)
            if q_out.dtype != c.dtype or q_out.shape != q.shape or not q_out.is_contiguous():
                raise ValueError("q_out must be contiguous, q's shape, in the pool dtype")
        check(lib().pkv_append_rope(
            self._h, self.layer_index, rope.handle, _dev_ptr(pos), pkv_dtype(k.dtype),
            _dev_ptr(k), _dev_ptr(v), _dev_ptr(sm), n,
            _dev_ptr(q) if q is not None else None,
            _dev_ptr(q_out) if q is not None else None, H, _stream_ptr(stream)), self._h)
        return q_out if q is not None else None

    # -- KvPool::gather_seq (attention.rs:85-97) ----------------------------
    def gather_seq(self, table, length: int, stream=None):
        import torch
        c = self.cache
        blocks = table.blocks if isinstance(table, BlockTable) else list(table)
        need = -(-length // c.block_size)
        if need > len(blocks):
            raise IndexError("length beyond the block table")
        tb = _i32(blocks[:max(need, 1)] if blocks else [0], c.device)
        ok = torch.empty((length, c.n_kv_head, c.head_dim), dtype=c.dtype, device=c.device)
        ov = torch.empty_like(ok)
        check(lib().pkv_gather_seq(self._h, self.layer_index, _dev_ptr(tb), length,
                                   _dev_ptr(ok), _dev_ptr(ov), _stream_ptr(stream)), self._h)
        return ok, ov

    def gather_varlen(self, block_tables, lengths, stream=None):
        """Several sequences' K/V in one launch: rows of sequence b at
        cu[b] .. cu[b+1]-1 of the returned (total, n_kv, hd) K and V, where
        cu = [0, cumsum(lengths)]; returns (k, v, cu) with cu on the device."""
        import numpy as np
        import torch
        c = self.cache
        lens = np.asarray(lengths, np.int64)
        cu_np = np.zeros(lens.size + 1, np.int32)
        cu_np[1:] = np.cumsum(lens)
        total = int(cu_np[-1])
        bt = _i32(block_tables, c.device)
        cu = torch.from_numpy(cu_np).to(c.device)
        ok = torch.empty((total, c.n_kv_head, c.head_dim), dtype=c.dtype, device=c.device)
        ov = torch.empty_like(ok)
        if total:
            check(lib().pkv_gather_varlen(self._h, self.layer_index, _dev_ptr(bt), bt.shape[1],
                                          _dev_ptr(cu), lens.size, total, _dev_ptr(ok),
                                          _dev_ptr(ov), _stream_ptr(stream)), self._h)
        return ok, ov, cu

    # -- decode attention ---------------------------------------------------
    def decode_attention(self, q, block_tables, context_lens, max_context_len: int | None = None,
                         k_new=None, v_new=None, scale: float | None = None, out_dtype=None,
                         out=None, stream=None, rope: "Rope | None" = None, positions=None):
        """q: (B, H, hd); block_tables: (B, max_nb) int32 device; context_lens:
        (B,) int32 device = keys attended (seq_lens + 1).  With k_new/v_new
        (B, n_kv, hd) the new token is stored at position context_lens-1 first.
        With `rope`, q and k_new are the projections before rotation (f32 or
        the pool dtype) and the kernel applies the rotary embedding at
        `positions` (default context_lens - 1).  Given, `positions` ((B,)
        int32 device) also bound the keys attended: k <= positions[b]
        (build_mask's second bound; pkv_decode_attention_positions without
        rope).  Returns (B, H*hd)."""
        if rope is not None:
            return self._decode_attention_rope(q, block_tables, context_lens, max_context_len,
                                               k_new, v_new, scale, out_dtype, out, stream,
                                               rope, positions)
        import torch
        c = self.cache
        B, H, hd = q.shape
        if hd != c.head_dim:
            raise ValueError("head_dim mismatch")
        if out_dtype is None:
            out_dtype = q.dtype
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        bt = _i32(block_tables, c.device)
        cl = _i32(context_lens, c.device)
        if max_context_len is None:
            max_context_len = int(cl.max().item()) if B else 1
        if out is None:
            out = torch.empty((B, H * hd), dtype=out_dtype, device=c.device)
        if k_new is not None:
            self._check_rows(k_new, "k_new")
            self._check_rows(v_new, "v_new")
        qq = q.contiguous()
        if qq.dtype != c.dtype:
            raise TypeError("q must have the pool dtype")
        kv = (_dev_ptr(k_new) if k_new is not None else None,
              _dev_ptr(v_new) if v_new is not None else None, _stream_ptr(stream))
        if positions is not None:
            pos = _i32(positions, c.device)
            check(lib().pkv_decode_attention_positions(
                self._h, self.layer_index, _dev_ptr(qq), _dev_ptr(out), pkv_dtype(out.dtype),
                _dev_ptr(bt), bt.shape[1], _dev_ptr(cl), _dev_ptr(pos), int(max_context_len), B,
                H, float(scale), *kv), self._h)
            return out
        check(lib().pkv_decode_attention(
            self._h, self.layer_index, _dev_ptr(qq), _dev_ptr(out), pkv_dtype(out.dtype),
            _dev_ptr(bt), bt.shape[1], _dev_ptr(cl), int(max_context_len), B, H, float(scale),
            *kv), self._h)
        return out

    def _decode_attention_rope(self, q, block_tables, context_lens, max_context_len, k_new,
                               v_new, scale, out_dtype, out, stream, rope, positions):
        import torch
        c = self.cache
        B, H, hd = q.shape
        if hd != c.head_dim:
            raise ValueError("head_dim mismatch")
        if q.dtype not in (torch.float32, c.dtype):
            raise TypeError("q must be float32 or the pool dtype")
        for t, name in ((k_new, "k_new"), (v_new, "v_new")):
            if t is not None and (t.dtype != q.dtype or t.shape != (B, c.n_kv_head, hd)):
                raise ValueError(f"{name} must be ({B}, {c.n_kv_head}, {hd}) in q's dtype")
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        bt = _i32(block_tables, c.device)
        cl = _i32(context_lens, c.device)
        if max_context_len is None:
            max_context_len = int(cl.max().item()) if B else 1
        if out is None:
            out = torch.empty((B, H * hd), dtype=out_dtype or c.dtype, device=c.device)
        pos = _i32(positions, c.device) if positions is not None else None
        qq = q.contiguous()
        kk = k_new.contiguous() if k_new is not None else None
        vv = v_new.contiguous() if v_new is not None else None
        check(lib().pkv_decode_attention_rope(
            self._h, self.layer_index, rope.handle, _dev_ptr(pos) if pos is not None else None,
            pkv_dtype(qq.dtype), _dev_ptr(qq), _dev_ptr(out), pkv_dtype(out.dtype), _dev_ptr(bt),
            bt.shape[1], _dev_ptr(cl), int(max_context_len), B, H, float(scale),
            _dev_ptr(kk) if kk is not None else None, _dev_ptr(vv) if vv is not None else None,
            _stream_ptr(stream)), self._h)
        return out

    # -- chunked prefill attention -------------------------------------------
    def prefill_attention(self, q, cu_q_lens, context_lens, block_tables, max_q_len: int,
                          max_context_len: int, scale: float | None = None, out_dtype=None,
                          out=None, stream=None, k_new=None, v_new=None):
        """Causal attention of prompt chunks over prior context + chunk.  With
        k_new / v_new (total_q, n_kv, hd), the chunk's K/V are stored in the
        same launch (pkv_prefill_attention_append); without, they must
        already be in the pool."""
        import torch
        c = self.cache
        T, H, hd = q.shape
        if out_dtype is None:
            out_dtype = q.dtype
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        cu = _i32(cu_q_lens, c.device)
        cl = _i32(context_lens, c.device)
        bt = _i32(block_tables, c.device)
        if out is None:
            out = torch.empty((T, H * hd), dtype=out_dtype, device=c.device)
        args = [self._h, self.layer_index, _dev_ptr(q.contiguous()), _dev_ptr(out),
                pkv_dtype(out.dtype), _dev_ptr(cu), _dev_ptr(cl), _dev_ptr(bt), bt.shape[1],
                cl.numel(), int(max_q_len), int(max_context_len), H, float(scale)]
        if k_new is not None or v_new is not None:
            self._check_rows(k_new, "k_new")
            self._check_rows(v_new, "v_new")
            check(lib().pkv_prefill_attention_append(*args, _dev_ptr(k_new), _dev_ptr(v_new),
                                                     _stream_ptr(stream)), self._h)
        else:
            check(lib().pkv_prefill_attention(*args, _stream_ptr(stream)), self._h)
        return out

    # -- a layer's mixed batch -------------------------------------------------
    def mixed_attention(self, prefill: dict, decode: dict, scale: float | None = None,
                        stream=None):
        """pkv_mixed_attention: the prefill batch (keys of prefill_attention:
        q, cu_q_lens, context_lens, block_tables, max_q_len, max_context_len,
        optional k_new, v_new, out_dtype, out) and the decode batch (keys of
        decode_attention: q, block_tables, context_lens, optional
        max_context_len, k_new, v_new, out_dtype, out) of one layer in one
        call; results identical to the two calls.  Returns (prefill out,
        decode out)."""
        import torch
        c = self.cache
        pq, dq = prefill["q"].contiguous(), decode["q"].contiguous()
        H, hd = pq.shape[1], pq.shape[2]
        if dq.shape[1:] != (H, hd) or hd != c.head_dim:
            raise ValueError("prefill and decode q must be (n, n_head, head_dim) of the pool")
        if pq.dtype != c.dtype or dq.dtype != c.dtype:
            raise TypeError("q must have the pool dtype")
        if scale is None:
            scale = 1.0 / math.sqrt(hd)
        keep = []  # tensors the structs point into, alive until the call returns

        def dev(t):
            keep.append(t)
            return _dev_ptr(t)

        rows = {}
        for side, d in (("prefill", prefill), ("decode", decode)):
            for key in ("k_new", "v_new"):
                if d.get(key) is not None:
                    self._check_rows(d[key], key)
            n = (d["q"].shape[0])
            out = d.get("out")
            if out is None:
                out = torch.empty((n, H * hd), dtype=d.get("out_dtype") or c.dtype,
                                  device=c.device)
            rows[side] = out
        pcu = _i32(prefill["cu_q_lens"], c.device)
        pcl = _i32(prefill["context_lens"], c.device)
        pbt = _i32(prefill["block_tables"], c.device)
        dcl = _i32(decode["context_lens"], c.device)
        dbt = _i32(decode["block_tables"], c.device)
        dmax = decode.get("max_context_len")
        if dmax is None:
            dmax = int(dcl.max().item()) if dcl.numel() else 1
        pk, pv = prefill.get("k_new"), prefill.get("v_new")
        dk, dv = decode.get("k_new"), decode.get("v_new")
        pb = _lib.PrefillBatch(dev(pq), dev(rows["prefill"]), pkv_dtype(rows["prefill"].dtype),
                               dev(pcu), dev(pcl), dev(pbt), pbt.shape[1], pcl.numel(),
                               int(prefill["max_q_len"]), int(prefill["max_context_len"]),
                               dev(pk) if pk is not None else None,
                               dev(pv) if pv is not None else None)
        db = _lib.DecodeBatch(dev(dq), dev(rows["decode"]), pkv_dtype(rows["decode"].dtype),
                              dev(dbt), dbt.shape[1], dev(dcl), int(dmax), dcl.numel(),
                              dev(dk) if dk is not None else None,
                              dev(dv) if dv is not None else None)
        check(lib().pkv_mixed_attention(self._h, self.layer_index, ctypes.byref(pb),
                                        ctypes.byref(db), H, float(scale),
                                        _stream_ptr(stream)), self._h)
        return rows["prefill"], rows["decode"]

    def _check_rows(self, t, name: str) -> None:
        c = self.cache
        if t.dtype != c.dtype:
            raise TypeError(f"{name} must have the pool dtype {c.dtype}")
        if t.dim() != 3 or t.shape[1] != c.n_kv_head or t.shape[2] != c.head_dim:
            raise ValueError(f"{name} must be (n, {c.n_kv_head}, {c.head_dim})")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
