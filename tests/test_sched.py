"""CPU tests of the continuous-batching scheduler (pkv_sched_*), the block
bookkeeping of the reference's engine thread
(crates/ai-engine-candle/src/paged/engine.rs:62-237).

Reference mode is checked against oracle/engine.py, a statement-by-statement
restatement of run_loop/prefill: on randomised workloads both must send the
same events (Ok(token) / Err(message) / closed) and run every decode step
over the same block tables.  Chunked prefill, forks (copy-on-write) and
compaction have no reference counterpart; they are checked by invariants."""
import random

import numpy as np
import pytest

import engine as ref_engine
from pagedkv.sched import ERROR, FINISHED, TOKEN, Scheduler

EOS = 2


def sampler(seed):
    """Deterministic 'model': the token a sequence samples after `produced`
    tokens; EOS with probability ~1/12."""
    def sample(seq_id, produced):
        h = (seq_id * 1000003 + produced * 7919 + seed * 104729) % 2147483647
        h = (h * 48271) % 2147483647
        return EOS if h % 12 == 0 else 3 + h % 1000
    return sample


def drive(s: Scheduler, sample, fail_forward=None, on_plan=None):
    """Runs the scheduler to completion the way the engine thread would:
    returns (events, decode-step trace)."""
    produced = {}
    events, trace = [], []
    forward_it = 0
    while True:
        p = s.step()
        if p.n_rows == 0:
            events += s.events()
            break
        if on_plan:
            on_plan(p)
        if p.n_decode:
            rows = []
            for r in range(p.n_prefill, p.n_rows):
                sid = int(p.row_seq[r])
                tbl, pos = s.table(sid)
                rows.append((sid, tuple(tbl), pos))
            trace.append(rows)
        msg = None
        if p.n_decode and fail_forward is not None:
            msg = fail_forward(forward_it)
        if p.n_decode:
            forward_it += 1
        if msg is not None:
            s.complete(None, error=msg)
        else:
            toks = []
            for r in range(p.n_rows):
                if not p.produces[r]:
                    continue
                sid = int(p.row_seq[r])
                k = produced.get(sid, 0)
                toks.append(sample(sid, k))
                produced[sid] = k + 1
            s.complete(toks)
        events += s.events()
    return events, trace


def per_seq(events):
    """Each request has its own channel in the reference (engine.rs:13-18):
    only the order within one sequence is observable."""
    out = {}
    for sid, kind, payload in events:
        out.setdefault(sid, []).append((kind, payload))
    return out


def random_case(seed):
    rnd = random.Random(seed)
    cfg = ref_engine.Config(max_num_seqs=rnd.randint(1, 6), block_size=rnd.choice([4, 16]),
                            kv_cache_blocks=rnd.randint(3, 30), max_seq=rnd.randint(20, 90),
                            eos_token_id=EOS)
    reqs = [ref_engine.Request(i + 1, rnd.randint(1, cfg.max_seq + 8),
                               rnd.choice([0, 1, 2, 3, 5, 8, 13, 40, 90]))
            for i in range(rnd.randint(1, 25))]
    fail = rnd.randint(0, 30) if seed % 3 == 0 else None
    return cfg, reqs, fail


@pytest.mark.parametrize("seed", range(60))
def test_reference_mode_matches_run_loop(seed):
    cfg, reqs, fail = random_case(seed)
    sample = sampler(seed)
    fail_at = (lambda kind, it: "boom" if kind == "forward" and it == fail else None)
    ev_ref, alloc, _, trace_ref = ref_engine.run_loop(cfg, reqs, sample, fail_at)
    s = Scheduler(cfg.max_num_seqs, cfg.block_size, cfg.kv_cache_blocks, cfg.max_seq, EOS)
    for r in reqs:
        assert s.submit(r.prompt_len, r.max_tokens) == r.id
    ev, trace = drive(s, sample, (lambda it: "boom" if it == fail else None))
    assert per_seq(ev) == per_seq(ev_ref)
    assert trace == trace_ref
    running, waiting, free = s.counts()
    assert (running, waiting, free) == (0, 0, alloc.free_count()) == (0, 0, cfg.kv_cache_blocks)


def test_engine_guards_and_messages():
    # engine.rs:190-206 admission guards, :110-120 decode guards
    s = Scheduler(4, 16, 3, 40, EOS)
    a = s.submit(10, 0)      # max_tokens == 0: nothing sent
    b = s.submit(41, 5)      # prompt > max_seq
    c = s.submit(30, 50)     # 2 blocks
    d = s.submit(20, 5)      # needs 2 blocks, 1 left: exhausted at admission
    p = s.step()
    assert p.n_prefill == 1 and list(p.row_seq) == [c]
    ev = s.events()
    assert (a, FINISHED, None) in ev
    assert (b, ERROR, "prompt exceeds max context (41 > 40)") in ev
    assert (d, ERROR, "KV cache exhausted at admission") in ev
    s.complete([7])
    for _ in range(2):       # positions 30, 31 fit the 2 blocks
        p = s.step()
        s.complete([9])
    p = s.step()             # position 32 needs a third block: granted (1 free)
    assert p.n_decode == 1 and p.context_lens[0] == 33
    s.complete([9])
    for _ in range(7):
        p = s.step()
        s.complete([9])
    p = s.step()             # position 40: 41 > max_seq
    assert p.n_rows == 0
    assert (c, ERROR, "sequence exceeded max context (41 > 40)") in s.events()
    assert s.counts() == (0, 0, 3)


def test_kv_exhausted_mid_decode_releases():
    s = Scheduler(2, 4, 3, 100, EOS)
    a = s.submit(4, 10)
    b = s.submit(4, 10)      # 1 block each, 1 free
    s.step()
    s.complete([5, 6])
    p = s.step()             # both need a 2nd block: a gets it, b is evicted
    assert list(p.row_seq) == [a]
    assert (b, ERROR, "KV cache exhausted") in s.events()
    s.complete([7])
    assert s.counts() == (1, 0, 1)


def test_prefill_token_always_sent_and_max_tokens_one_quirk():
    # prefill() sends its token even when it is EOS (:226-227) and the
    # sequence keeps decoding; with max_tokens == 1 the first decode step
    # still sends its token before at_limit ends the sequence (:160-178).
    s = Scheduler(2, 16, 8, 100, EOS)
    a = s.submit(5, 1)
    s.step()
    s.complete([EOS])
    assert s.events() == [(a, TOKEN, EOS)]
    p = s.step()
    assert p.n_decode == 1
    s.complete([11])
    assert s.events() == [(a, TOKEN, 11), (a, FINISHED, None)]


def test_prefill_failure_drops_request_then_decodes():
    s = Scheduler(4, 16, 16, 100, EOS)
    a = s.submit(5, 4)
    s.step()
    s.complete([10])
    p = s.step()             # the first iteration's decode step
    assert p.n_decode == 1
    s.complete([11])
    assert s.events() == [(a, TOKEN, 10), (a, TOKEN, 11)]
    b = s.submit(7, 4)
    p = s.step()             # next iteration: b's prefill
    assert p.n_prefill == 1 and list(p.row_seq) == [b]
    s.complete(None, error="bad")
    assert s.events() == [(b, ERROR, "prefill: bad")]
    p = s.step()             # the same iteration's decode step for a
    assert p.n_decode == 1 and list(p.row_seq) == [a]
    s.complete([12])


@pytest.mark.parametrize("seed", range(12))
def test_chunked_prefill_invariants_and_same_streams(seed):
    rnd = random.Random(100 + seed)
    bs, chunk, budget = rnd.choice([4, 16]), rnd.choice([3, 16, 64]), rnd.choice([0, 40, 100])
    reqs = [(rnd.randint(1, 150), rnd.randint(1, 9)) for _ in range(rnd.randint(1, 12))]
    sample = sampler(seed)

    def streams(s, chunked):
        ids = [s.submit(pl, mt) for pl, mt in reqs]
        seen = {}

        def check(p):
            assert p.cu_q_lens[-1] == int((p.context_lens[:p.n_prefill] - p.q_start).sum())
            if budget:
                assert p.cu_q_lens[-1] <= budget
            for r in range(p.n_prefill):
                n = p.cu_q_lens[r + 1] - p.cu_q_lens[r]
                assert 1 <= n <= chunk
                sid = int(p.row_seq[r])
                assert p.q_start[r] == seen.get(sid, 0)   # chunks in order, no gap
                seen[sid] = p.q_start[r] + n
                assert p.produces[r] == (seen[sid] == reqs[ids.index(sid)][0])
            for t in range(p.slot_mapping.size):          # slot = locate(table, pos)
                r = np.searchsorted(p.cu_q_lens, t, side="right") - 1 if t < p.cu_q_lens[-1] \
                    else p.n_prefill + (t - p.cu_q_lens[-1])
                pos = p.positions[t]
                assert p.slot_mapping[t] == p.block_tables[r, pos // bs] * bs + pos % bs
        ev, _ = drive(s, sample, on_plan=check if chunked else None)
        return per_seq(ev)

    ref = streams(Scheduler(4, bs, 4096, 4096, EOS), False)
    got = streams(Scheduler(4, bs, 4096, 4096, EOS, prefill_chunk=chunk, step_token_budget=budget),
                  True)
    assert got == ref   # ample blocks: chunking changes timing, not streams


def test_fork_copy_on_write_and_release():
    s = Scheduler(4, 4, 32, 1000, EOS)
    a = s.submit(6, 20)           # blocks for positions 0..5 (2 blocks)
    s.step()
    s.complete([10])
    p = s.step()                  # a writes position 6 (block 1)
    s.complete([11])
    tbl_a, pos = s.table(a)
    assert pos == 7 and len(tbl_a) == 2
    c = s.fork(a, 20)
    assert s.table(c) == (tbl_a, 7)
    free0 = s.counts()[2]
    p = s.step()                  # both write position 7 in shared block 1
    assert p.n_decode == 2 and p.copy_src.tolist() == [tbl_a[1]]
    new = p.copy_dst.tolist()[0]
    assert s.table(a)[0] == [tbl_a[0], new] and s.table(c)[0] == tbl_a
    assert p.slot_mapping.tolist() == [new * 4 + 3, tbl_a[1] * 4 + 3]
    assert s.counts()[2] == free0 - 1
    s.complete([12, 13])
    p = s.step()                  # position 8: each gets its own fresh block
    assert p.n_copies == 0
    s.complete([EOS, 14])         # a ends: shared block 0 stays for c
    assert (a, FINISHED, None) in s.events()
    assert tbl_a[0] in s.table(c)[0]
    for _ in range(30):
        p = s.step()
        if p.n_rows == 0:
            break
        s.complete([15] * p.n_producing)
    assert s.counts() == (0, 0, 32)


def test_compact_moves_live_blocks_to_prefix():
    rnd = random.Random(5)
    s = Scheduler(8, 4, 64, 1000, EOS)
    ids = [s.submit(rnd.randint(1, 30), 50) for _ in range(8)]
    s.step()
    s.complete([20] * 8)
    content = {}                  # block id -> content tag (what the pool holds)
    for sid in ids:
        for j, b in enumerate(s.table(sid)[0]):
            content[b] = (sid, j)
    for sid in ids[::2]:          # free some sequences' blocks
        p = s.step()
        s.complete([EOS if int(x) == sid else 21 for x in p.row_seq])
        content = {}
        for x in p.row_seq:
            x = int(x)
            if x != sid:
                for j, b in enumerate(s.table(x)[0]):
                    content[b] = (x, j)
    live = sorted(content)
    src, dst = s.compact()
    assert all(b >= len(live) for b in src) and all(b < len(live) for b in dst)
    assert len(set(dst.tolist())) == len(dst)
    moved = dict(content)
    for a, b in zip(src.tolist(), dst.tolist()):
        moved[b] = content[a]
        del moved[a]
    for sid in ids:
        try:
            tbl = s.table(sid)[0]
        except Exception:
            continue
        assert all(b < len(live) for b in tbl)
        assert [moved[b] for b in tbl] == [(sid, j) for j in range(len(tbl))]
    # the free list hands out live, live + 1, ... next
    n_free = s.counts()[2]
    assert n_free == 64 - len(live)
    nid = s.submit(4, 3)
    p = s.step()
    while p.n_prefill == 0:
        s.complete([30] * p.n_producing)
        p = s.step()
    assert s.table(nid)[0] == [len(live)]


def test_api_misuse_is_reported():
    from pagedkv import PagedKvError
    with pytest.raises(PagedKvError):
        Scheduler(0, 16, 8, 100, EOS)             # no sequences allowed
    s = Scheduler(2, 16, 8, 100, EOS)
    with pytest.raises(PagedKvError):
        s.complete([1])                           # no plan is open
    with pytest.raises(PagedKvError):
        s.submit(-1, 4)
    a = s.submit(5, 4)
    p = s.step()
    with pytest.raises(PagedKvError):
        s.step()                                  # the open plan must be completed first
    with pytest.raises(PagedKvError):
        s.fork(a, 3)                              # not while a plan is open
    with pytest.raises(PagedKvError):
        s.complete([1, 2])                        # one token per producing row
    s.complete([9] * p.n_producing)
    with pytest.raises(PagedKvError):
        s.fork(12345, 3)                          # not a live sequence
    b = s.fork(a, 3)
    with pytest.raises(PagedKvError):
        s.fork(a, 3)                              # max_num_seqs reached
    with pytest.raises(PagedKvError):
        s.table(999)
    assert s.counts()[0] == 2 and b != a
