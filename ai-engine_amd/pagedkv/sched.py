"""Python front end of the continuous-batching scheduler (pkv_sched_*, the
block bookkeeping of the reference's engine thread,
crates/ai-engine-candle/src/paged/engine.rs:62-237)."""
from __future__ import annotations

import ctypes
import sys
import dataclasses

import numpy as np

from ._lib import PagedKvError, lib

TOKEN, FINISHED, ERROR = 0, 1, 2


class _Config(ctypes.Structure):
    _fields_ = [("max_num_seqs", ctypes.c_int), ("block_size", ctypes.c_int),
                ("kv_cache_blocks", ctypes.c_int), ("max_seq", ctypes.c_int),
                ("eos_token_id", ctypes.c_int32), ("prefill_chunk", ctypes.c_int),
                ("step_token_budget", ctypes.c_int)]


class _Event(ctypes.Structure):
    _fields_ = [("seq", ctypes.c_int64), ("kind", ctypes.c_int), ("token", ctypes.c_int32),
                ("message", ctypes.c_char * 120)]


_I32P = ctypes.POINTER(ctypes.c_int32)


class _Plan(ctypes.Structure):
    _fields_ = [("n_prefill", ctypes.c_int), ("n_decode", ctypes.c_int), ("n_rows", ctypes.c_int),
                ("max_blocks", ctypes.c_int), ("n_tokens", ctypes.c_int),
                ("n_copies", ctypes.c_int), ("row_seq", ctypes.POINTER(ctypes.c_int64)),
                ("block_tables", _I32P), ("context_lens", _I32P), ("cu_q_lens", _I32P),
                ("q_start", _I32P), ("slot_mapping", _I32P), ("positions", _I32P),
                ("produces", ctypes.POINTER(ctypes.c_int8)), ("copy_src", _I32P),
                ("copy_dst", _I32P)]


def _arr(ptr, n, dtype):
    if n <= 0:
        return np.zeros(0, dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


@dataclasses.dataclass
class Plan:
    """One forward's work (copied out of the library)."""
    n_prefill: int
    n_decode: int
    row_seq: np.ndarray
    block_tables: np.ndarray     # (rows, max_blocks) int32
    context_lens: np.ndarray
    cu_q_lens: np.ndarray
    q_start: np.ndarray
    slot_mapping: np.ndarray
    positions: np.ndarray
    produces: np.ndarray
    copy_src: np.ndarray
    copy_dst: np.ndarray

    @property
    def n_rows(self) -> int:
        return self.n_prefill + self.n_decode

    @property
    def n_producing(self) -> int:
        return int(self.produces.sum())

    @property
    def n_copies(self) -> int:
        return int(self.copy_src.size)


def _check(rc: int) -> None:
    if rc != 0:
        raise PagedKvError(rc, lib().pkv_sched_last_error().decode(errors="replace"))


class Scheduler:
    """Step machine of run_loop: step() -> Plan, complete(tokens), events()."""

    def __init__(self, max_num_seqs: int, block_size: int, kv_cache_blocks: int, max_seq: int,
                 eos_token_id: int, prefill_chunk: int = 0, step_token_budget: int = 0) -> None:
        cfg = _Config(max_num_seqs, block_size, kv_cache_blocks, max_seq, eos_token_id,
                      prefill_chunk, step_token_budget)
        h = ctypes.c_void_p()
        _check(lib().pkv_sched_create(ctypes.byref(h), ctypes.byref(cfg)))
        self._h = h
        self.block_size = block_size
        self.kv_cache_blocks = kv_cache_blocks

    def __del__(self, _finalizing=sys.is_finalizing) -> None:
        h = getattr(self, "_h", None)
        if h and not _finalizing():
            lib().pkv_sched_destroy(h)
            self._h = None

    def submit(self, prompt_len: int, max_tokens: int) -> int:
        i = ctypes.c_int64()
        _check(lib().pkv_sched_submit(self._h, prompt_len, max_tokens, ctypes.byref(i)))
        return int(i.value)

    def step(self) -> Plan:
        p = _Plan()
        _check(lib().pkv_sched_step(self._h, ctypes.byref(p)))
        rows = p.n_rows
        return Plan(p.n_prefill, p.n_decode, _arr(p.row_seq, rows, np.int64),
                    _arr(p.block_tables, rows * p.max_blocks, np.int32).reshape(rows, -1)
                    if rows else np.zeros((0, 1), np.int32),
                    _arr(p.context_lens, rows, np.int32),
                    _arr(p.cu_q_lens, p.n_prefill + 1 if rows else 0, np.int32),
                    _arr(p.q_start, p.n_prefill, np.int32),
                    _arr(p.slot_mapping, p.n_tokens, np.int32),
                    _arr(p.positions, p.n_tokens, np.int32),
                    _arr(p.produces, rows, np.int8), _arr(p.copy_src, p.n_copies, np.int32),
                    _arr(p.copy_dst, p.n_copies, np.int32))

    def complete(self, tokens, error: str | None = None) -> None:
        t = np.ascontiguousarray(tokens if tokens is not None else [], dtype=np.int32)
        _check(lib().pkv_sched_complete(self._h, t.ctypes.data if t.size else None, t.size,
                                        error.encode() if error is not None else None))

    def events(self) -> list[tuple]:
        out, ev = [], _Event()
        while lib().pkv_sched_poll(self._h, ctypes.byref(ev)):
            payload = (ev.token if ev.kind == TOKEN else
                       ev.message.decode() if ev.kind == ERROR else None)
            out.append((int(ev.seq), int(ev.kind), payload))
        return out

    def fork(self, parent: int, max_tokens: int) -> int:
        c = ctypes.c_int64()
        _check(lib().pkv_sched_fork(self._h, parent, max_tokens, ctypes.byref(c)))
        return int(c.value)

    def compact(self):
        """Renumber live blocks to [0, live) -> (src, dst) moves for pkv_compact."""
        n_cap = max(1, self.kv_cache_blocks)  # at most one move per block
        src = np.zeros(n_cap, np.int32)
        dst = np.zeros(n_cap, np.int32)
        n = ctypes.c_int()
        _check(lib().pkv_sched_compact(self._h, src.ctypes.data, dst.ctypes.data, n_cap,
                                       ctypes.byref(n)))
        return src[:n.value].copy(), dst[:n.value].copy()

    def counts(self) -> tuple[int, int, int]:
        r, w, f = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(lib().pkv_sched_counts(self._h, ctypes.byref(r), ctypes.byref(w),
                                      ctypes.byref(f)))
        return r.value, w.value, f.value

    def table(self, seq: int) -> tuple[list[int], int]:
        blk = ctypes.POINTER(ctypes.c_uint32)()
        n, pos = ctypes.c_int(), ctypes.c_int()
        _check(lib().pkv_sched_table(self._h, seq, ctypes.byref(blk), ctypes.byref(n),
                                     ctypes.byref(pos)))
        return [blk[i] for i in range(n.value)], pos.value
