"""End to end on the GPU: the scheduler's plans (pkv_sched_*) drive the
kernels the way the reference's engine thread drives its forward
(crates/ai-engine-candle/src/paged/engine.rs:62-237, transformer.rs
prefill/decode_step): per step, copy-on-write block copies, then per layer the
prompt chunks' K/V appended by slot mapping and prefill attention, and decode
attention with the new token's K/V appended inside the kernel (or, in the
mixed runs, both batches of a layer in one pkv_mixed_attention call); every
so often the pool is compacted.  Each attention output is checked against the fp64
closed form over the sequence's own K/V history kept on the host (so a wrong
block table, slot, copy or move shows up as a wrong attention row).
Tolerance: |gpu - ref| <= 1e-3 + 2e-3 |ref|."""
import math
import random

import numpy as np
import pytest
import torch

import pagedkv
from pagedkv import workload as wl
from pagedkv.sched import ERROR, FINISHED, Scheduler

pytestmark = pytest.mark.gpu

EOS = 2
ATOL, RTOL = 1e-3, 2e-3


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def _attention_f64(q, k, v, q_pos, scale):
    """q (n, H, hd) at positions q_pos attends keys 0..q_pos of k/v (L, KVH, hd)."""
    n, H, hd = q.shape
    R = H // k.shape[1]
    kk = np.repeat(k.astype(np.float64), R, axis=1)          # (L, H, hd)
    vv = np.repeat(v.astype(np.float64), R, axis=1)
    s = np.einsum("nhd,lhd->nhl", q.astype(np.float64), kk) * scale
    mask = np.arange(k.shape[0])[None, :] > np.asarray(q_pos)[:, None]
    s[np.broadcast_to(mask[:, None, :], s.shape)] = -np.inf
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=2, keepdims=True)
    return np.einsum("nhl,lhd->nhd", p, vv).reshape(n, H * hd)


class Model:
    """Stands in for the transformer: per layer, fresh bf16 q/k/v rows for
    every token a plan runs, a K/V history per live sequence, and a sampler
    that ends a sequence now and then."""

    def __init__(self, gpu, n_layers, H, KVH, hd, bs, blocks, seed):
        self.gpu, self.L, self.H, self.KVH, self.hd, self.bs = gpu, n_layers, H, KVH, hd, bs
        self.cache = pagedkv.PagedKvCache(n_layers, blocks, bs, KVH, hd, torch.bfloat16)
        self.cache.fill_normal(seed)        # stale contents in every free block
        self.rng = np.random.default_rng(seed)
        self.hist = {}                      # seq -> [layer] -> (k list, v list) of f32 rows
        self.scale = 1 / math.sqrt(hd)
        self.checked = 0

    def rows(self, n, heads):
        x = self.rng.standard_normal((n, heads, self.hd)) * 0.5
        st = wl.to_storage(x, wl.BF16).reshape(n, heads, self.hd)
        return st, wl.widen(st, wl.BF16)

    def history(self, seq):
        return self.hist.setdefault(seq, [([], []) for _ in range(self.L)])

    def check(self, got, ref, what):
        err = np.abs(got.astype(np.float64) - ref)
        bad = err > ATOL + RTOL * np.abs(ref)
        assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} off, max err {err.max():.3g}"
        self.checked += got.shape[0]

    def forward(self, p, mixed=False):
        """One plan's forward.  mixed: a step with both prompt chunks and
        decode rows runs each layer's attention as one pkv_mixed_attention
        call (the chunk's K/V stored by the call) instead of pkv_append,
        pkv_prefill_attention and pkv_decode_attention."""
        g, bs = self.gpu, self.bs
        if p.n_copies:
            self.cache.copy_blocks(p.copy_src, p.copy_dst)
        T = int(p.cu_q_lens[-1]) if p.n_prefill else 0
        D = p.n_decode
        for l in range(self.L):
            pool = self.cache.layer(l)
            if T:
                pk, pkf = self.rows(T, self.KVH)
                pv, pvf = self.rows(T, self.KVH)
                pq, pqf = self.rows(T, self.H)
                pre = dict(q=_dev(pq, g), cu_q_lens=p.cu_q_lens,
                           context_lens=p.context_lens[:p.n_prefill],
                           block_tables=np.ascontiguousarray(p.block_tables[:p.n_prefill]),
                           max_q_len=int(np.diff(p.cu_q_lens).max()),
                           max_context_len=int(p.context_lens[:p.n_prefill].max()),
                           out_dtype=torch.float32)
            if D:
                dk, dkf = self.rows(D, self.KVH)
                dv, dvf = self.rows(D, self.KVH)
                dq, dqf = self.rows(D, self.H)
                cl = p.context_lens[p.n_prefill:]
                dec = dict(q=_dev(dq, g), block_tables=np.ascontiguousarray(p.block_tables[p.n_prefill:]),
                           context_lens=cl, k_new=_dev(dk, g), v_new=_dev(dv, g),
                           out_dtype=torch.float32)
            if mixed and T and D:
                po, do = pool.mixed_attention(dict(pre, k_new=_dev(pk, g), v_new=_dev(pv, g)), dec)
                pout, dout = po.cpu().numpy(), do.cpu().numpy()
            else:
                if T:
                    pool.append(_dev(pk, g), _dev(pv, g), p.slot_mapping[:T])
                    a = dict(pre)
                    pout = pool.prefill_attention(a.pop("q"), a.pop("cu_q_lens"),
                                                  a.pop("context_lens"), a.pop("block_tables"),
                                                  **a).cpu().numpy()
                if D:
                    a = dict(dec)
                    dout = pool.decode_attention(a.pop("q"), a.pop("block_tables"),
                                                 a.pop("context_lens"), **a).cpu().numpy()
            for r in range(p.n_prefill if T else 0):
                a, b = int(p.cu_q_lens[r]), int(p.cu_q_lens[r + 1])
                hk, hv = self.history(int(p.row_seq[r]))[l]
                assert len(hk) == int(p.q_start[r])
                hk.extend(pkf[a:b])
                hv.extend(pvf[a:b])
                ref = _attention_f64(pqf[a:b], np.stack(hk), np.stack(hv),
                                     np.arange(int(p.q_start[r]), len(hk)), self.scale)
                self.check(pout[a:b], ref, f"prefill layer {l} seq {int(p.row_seq[r])}")
            for i in range(D):
                hk, hv = self.history(int(p.row_seq[p.n_prefill + i]))[l]
                assert len(hk) == int(cl[i]) - 1
                hk.append(dkf[i])
                hv.append(dvf[i])
                ref = _attention_f64(dqf[i:i + 1], np.stack(hk), np.stack(hv),
                                     [len(hk) - 1], self.scale)
                self.check(dout[i:i + 1], ref, f"decode layer {l} seq {int(p.row_seq[p.n_prefill + i])}")
        torch.cuda.synchronize()
        self.cache.check()
        return bool(mixed and T and D)


@pytest.mark.parametrize("chunk,budget,seed,mixed", [(0, 0, 1, False), (48, 160, 2, False),
                                                    (16, 0, 3, False), (48, 160, 4, True),
                                                    (16, 0, 5, True)])
def test_engine_end_to_end(gpu, chunk, budget, seed, mixed):
    rnd = random.Random(seed)
    bs, blocks = 16, 72
    m = Model(gpu, 2, 8, 2, 128, bs, blocks, seed)
    s = Scheduler(5, bs, blocks, 700, EOS, prefill_chunk=chunk, step_token_budget=budget)
    live = set()
    for _ in range(14):
        live.add(s.submit(rnd.randint(1, 260), rnd.randint(1, 40)))
    steps = forks = compactions = copies = mixed_steps = 0
    while True:
        p = s.step()
        if p.n_rows == 0:
            break
        mixed_steps += m.forward(p, mixed)
        copies += p.n_copies
        toks = [EOS if rnd.random() < 0.04 else 100 + rnd.randrange(1000)
                for _ in range(p.n_producing)]
        s.complete(toks)
        for sid, kind, _ in s.events():
            if kind in (FINISHED, ERROR):
                live.discard(sid)
                m.hist.pop(sid, None)
        steps += 1
        decoding = [int(x) for x in p.row_seq[p.n_prefill:] if int(x) in live]
        if decoding and steps % 9 == 0 and s.counts()[0] < 5:
            parent = rnd.choice(decoding)
            child = s.fork(parent, rnd.randint(2, 30))
            m.hist[child] = [(list(k), list(v)) for k, v in m.history(parent)]
            live.add(child)
            forks += 1
        if steps % 13 == 0:
            src, dst = s.compact()
            if src.size:
                m.cache.compact(src, dst)
                compactions += 1
    assert s.counts() == (0, 0, blocks)
    assert forks > 0 and copies > 0 and compactions > 0 and m.checked > 0
    assert mixed_steps > 0 or not mixed
    m.cache.check()
    m.cache.close()
