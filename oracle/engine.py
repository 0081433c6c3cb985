"""Pure-Python restatement of the reference engine thread (test infrastructure).

Follows crates/ai-engine-candle/src/paged/engine.rs run_loop (:62-180) and
prefill (:182-237) statement by statement, with the model forward and the
sampler replaced by a callback, so that the product's step-machine scheduler
(``pkv_sched_*`` in libpagedkv) can be checked against the reference's
control flow: the same requests and the same sampled tokens must produce the
same channel traffic (Ok(token) / Err(message) / closed) and the same block
allocations.  Only tests/ use this module.
"""
from __future__ import annotations

import dataclasses
from collections import deque

from block_table import BlockAllocator, BlockTable, CapacityError

TOKEN, FINISHED, ERROR = 0, 1, 2


@dataclasses.dataclass
class Request:          # GenRequest, engine.rs:13-18 (the channel is the id)
    id: int
    prompt_len: int
    max_tokens: int


@dataclasses.dataclass
class Seq:              # engine.rs:20-28
    id: int
    table: BlockTable
    next_token: int
    pos: int
    produced: int
    max_tokens: int


@dataclasses.dataclass
class Config:           # EngineConfig, engine.rs:30-36
    max_num_seqs: int
    block_size: int
    kv_cache_blocks: int
    max_seq: int
    eos_token_id: int


class ForwardError(Exception):
    pass


def run_loop(cfg: Config, requests, sample, fail_at=None):
    """Runs the engine over `requests` (all submitted before the loop, the
    sender then dropped) until it returns.  sample(seq_id, produced) -> the
    token the model would sample next; fail_at(kind, iteration) -> an error
    message to inject into that prefill ("prefill") or decode step
    ("forward"), or None.  Returns (events, allocator, decode_steps, trace)
    where trace lists, per decode step, the (seq id, block table, position)
    of every sequence that runs it (taken right before the step,
    engine.rs:130-133)."""
    alloc = BlockAllocator(cfg.kv_cache_blocks, cfg.block_size)
    queue = deque(requests)
    running: list[Seq] = []
    events: list[tuple] = []
    trace: list[list[tuple]] = []
    it = 0

    def send(seq_id, kind, payload=None):
        events.append((seq_id, kind, payload))

    def prefill(req: Request):                               # :182-237
        if req.max_tokens == 0:                              # :190-192
            send(req.id, FINISHED)
            return None
        if req.prompt_len > cfg.max_seq:                     # :194-201
            send(req.id, ERROR, f"prompt exceeds max context ({req.prompt_len} > {cfg.max_seq})")
            return None
        table = BlockTable()
        try:                                                 # :203-206
            alloc.ensure_capacity(table, req.prompt_len)
        except CapacityError:
            send(req.id, ERROR, "KV cache exhausted at admission")
            return None
        msg = fail_at("prefill", it) if fail_at else None
        if msg is not None:                                  # :207-215
            send(req.id, ERROR, f"prefill: {msg}")
            alloc.release(table)
            return None
        nxt = sample(req.id, 0)                              # :226
        send(req.id, TOKEN, nxt)                             # :227
        return Seq(req.id, table, nxt, req.prompt_len, 1, req.max_tokens)

    while True:
        while len(running) < cfg.max_num_seqs:               # :77-90
            if queue:
                seq = prefill(queue.popleft())
                if seq is not None:
                    running.append(seq)
            else:                                            # Disconnected
                if not running:
                    return events, alloc, it, trace
                break
        if not running:                                      # :91-100
            if not queue:
                return events, alloc, it, trace
            seq = prefill(queue.popleft())
            if seq is not None:
                running.append(seq)
            continue
        evicted = False                                      # :102-128
        survivors = []
        for s in running:
            if s.pos + 1 > cfg.max_seq:
                send(s.id, ERROR, f"sequence exceeded max context ({s.pos + 1} > {cfg.max_seq})")
                alloc.release(s.table)
                evicted = True
                continue
            try:
                alloc.ensure_capacity(s.table, s.pos + 1)
            except CapacityError:
                send(s.id, ERROR, "KV cache exhausted")
                alloc.release(s.table)
                evicted = True
                continue
            survivors.append(s)
        running = survivors
        if evicted and not running:
            continue
        trace.append([(s.id, tuple(s.table.blocks), s.pos) for s in running])
        msg = fail_at("forward", it) if fail_at else None    # :134-141
        it += 1
        if msg is not None:
            for s in running:
                send(s.id, ERROR, f"forward: {msg}")
            for s in running:
                alloc.release(s.table)
            running = []
            continue
        keep = []                                            # :160-178
        for s in running:
            nxt = sample(s.id, s.produced)
            s.pos += 1
            s.produced += 1
            eos = nxt == cfg.eos_token_id
            at_limit = s.produced >= s.max_tokens
            if not eos:
                send(s.id, TOKEN, nxt)
            if eos or at_limit:
                alloc.release(s.table)
                send(s.id, FINISHED)
            else:
                s.next_token = nxt
                keep.append(s)
        running = keep
