"""pkv_mixed_attention: a layer's prefill batch and decode batch in one
call.  Every output row and every stored K/V byte must equal, bit for bit,
the two separate calls (pkv_prefill_attention(_append), then
pkv_decode_attention), which the prefill and decode tests pin against the
oracle; covered for the shapes with a combined kernel and for shapes that
fall back to the two launches, with split prefill and split decode
partials sharing the workspace, and under HIP graph replay."""
import math

import numpy as np
import pytest
import torch

import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}


class Mix:
    """Two identical pools (fill_normal) and one mixed batch over them."""

    def __init__(self, gpu, dt, H, KVH, hd, bs, priors, chunks, dctx, seed, fused=True):
        self.gpu, self.dt, self.H, self.KVH, self.hd, self.bs = gpu, dt, H, KVH, hd, bs
        priors, chunks, dctx = (np.asarray(x, np.int64) for x in (priors, chunks, dctx))
        pneed = -(-(priors + chunks) // bs)
        dneed = -(-(dctx + 1) // bs)
        nb = int(pneed.sum() + dneed.sum()) + 7
        perm = wl.permutation(seed, nb).astype(np.int32)
        o = 0

        def tables(need):
            nonlocal o
            t = np.zeros((len(need), max(int(need.max()), 1)), np.int32)
            for i, n in enumerate(need):
                t[i, :n] = perm[o:o + n]
                o += int(n)
            return t

        ptab, dtab = tables(pneed), tables(dneed)
        self.caches = [pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt]) for _ in range(2)]
        for c in self.caches:
            c.fill_normal(seed)
        g = torch.Generator(device=gpu)
        g.manual_seed(seed)
        tdt = TD[dt]

        def rnd(*shp, sc=1.0):
            return (torch.randn(shp, generator=g, device=gpu) * sc).to(tdt)

        T, B = int(chunks.sum()), len(dctx)
        sc = 1 / math.sqrt(hd)
        cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
        self.prefill = dict(q=rnd(T, H, hd, sc=sc), cu_q_lens=torch.from_numpy(cu).to(gpu),
                            context_lens=torch.from_numpy((priors + chunks).astype(np.int32)).to(gpu),
                            block_tables=torch.from_numpy(ptab).to(gpu),
                            max_q_len=int(chunks.max()), max_context_len=int((priors + chunks).max()))
        self.decode = dict(q=rnd(B, H, hd, sc=sc), block_tables=torch.from_numpy(dtab).to(gpu),
                           context_lens=torch.from_numpy((dctx + 1).astype(np.int32)).to(gpu),
                           max_context_len=int(dctx.max()) + 1)
        if fused:
            self.prefill.update(k_new=rnd(T, KVH, hd), v_new=rnd(T, KVH, hd))
            self.decode.update(k_new=rnd(B, KVH, hd), v_new=rnd(B, KVH, hd))
        self.scale = sc

    def separate(self, out_dtype):
        pool = self.caches[0].layer(0)
        pa = {k: v for k, v in self.prefill.items()}
        op = pool.prefill_attention(pa.pop("q"), pa.pop("cu_q_lens"), pa.pop("context_lens"),
                                    pa.pop("block_tables"), scale=self.scale,
                                    out_dtype=out_dtype, **pa)
        od = pool.decode_attention(self.decode["q"], self.decode["block_tables"],
                                   self.decode["context_lens"],
                                   max_context_len=self.decode["max_context_len"],
                                   k_new=self.decode.get("k_new"), v_new=self.decode.get("v_new"),
                                   scale=self.scale, out_dtype=out_dtype)
        torch.cuda.synchronize()
        self.caches[0].check()
        return op, od

    def mixed(self, out_dtype, cache=1):
        pool = self.caches[cache].layer(0)
        op, od = pool.mixed_attention(dict(self.prefill, out_dtype=out_dtype),
                                      dict(self.decode, out_dtype=out_dtype), scale=self.scale)
        torch.cuda.synchronize()
        self.caches[cache].check()
        return op, od

    def pools_equal(self):
        a, b = self.caches
        return all(np.array_equal(a.read_bytes(0, w), b.read_bytes(0, w))
                   for w in (pagedkv.K, pagedkv.V))

    def close(self):
        for c in self.caches:
            c.close()


def _same(x, y):
    return torch.equal(x.view(torch.int16) if x.element_size() == 2 else x.view(torch.int32),
                       y.view(torch.int16) if y.element_size() == 2 else y.view(torch.int32))


@pytest.mark.parametrize("dt,hd,R,combined", [
    (wl.F16, 64, 8, True), (wl.BF16, 128, 4, True), (wl.BF16, 64, 4, True),
    (wl.F16, 128, 8, True), (wl.BF16, 128, 8, True), (wl.F16, 64, 4, True),
    (wl.F16, 128, 4, False), (wl.F32, 64, 4, False), (wl.BF16, 128, 2, False),
    (wl.BF16, 64, 7, False)])
@pytest.mark.parametrize("fused", [True, False])
def test_mixed_equals_separate_calls(gpu, dt, hd, R, combined, fused):
    KVH = 4
    priors = [0, 37, 300, 1024, 15, 700]
    chunks = [40, 128, 1, 256, 17, 64]
    dctx = list(wl.randint(hd + R, 40, 0, 2000)) + [0, 15, 16]
    m = Mix(gpu, dt, R * KVH, KVH, hd, 16, priors, chunks, dctx, seed=hd + R + dt, fused=fused)
    c = m.caches[0]
    assert pagedkv.lib().pkv_mixed_workspace_bytes(c.handle, R * KVH, None, None) == 0
    od = torch.float32 if dt == wl.F32 else TD[dt]
    sp, sd = m.separate(od)
    mp, md = m.mixed(od)
    assert _same(sp, mp), "prefill rows differ"
    assert _same(sd, md), "decode rows differ"
    assert m.pools_equal()
    m.close()


def test_mixed_split_partials_share_the_workspace(gpu):
    # two long-prior prompts (the prefill splits its key ranges) and a few
    # long decodes (split-context partitions): both merges read partials from
    # one workspace, side by side
    m = Mix(gpu, wl.BF16, 32, 8, 128, 16, priors=[6000, 9000], chunks=[64, 100],
            dctx=[7000, 30, 12000], seed=5)
    c = m.caches[0]
    assert c.prefill_workspace_bytes(2, 32, 100, 9100) > 0
    assert c.decode_workspace_bytes(3, 32, 12001) > 256
    sp, sd = m.separate(torch.float32)
    mp, md = m.mixed(torch.float32)
    assert _same(sp, mp) and _same(sd, md) and m.pools_equal()
    m.close()


def test_mixed_with_split_last_partitions(gpu):
    # a decode half of 128 sequences x 8 kv heads up to 4096 tokens, whose
    # plan cuts each context's last 1024 tokens in two, beside two prompt
    # chunks: the one-launch result equals the two calls bit for bit
    dctx = [int(x) for x in wl.randint(17, 128, 1, 4095)]
    dctx[0] = 4095
    m = Mix(gpu, wl.BF16, 32, 8, 128, 16, priors=[700, 30], chunks=[64, 200], dctx=dctx, seed=17)
    c = m.caches[0]
    assert c.decode_workspace_bytes(128, 32, 4096) == (
        -(-128 * 8 * 5 * 32 * 4 // 256) * 256 + 128 * 8 * 5 * 4 * 128 * 4)
    sp, sd = m.separate(torch.float32)
    mp, md = m.mixed(torch.float32)
    assert _same(sp, mp) and _same(sd, md) and m.pools_equal()
    m.close()


def test_mixed_cfg2_shape_and_graph_replay(gpu):
    # the TinyLlama continuous-batching mix: 8 chunks of 256 over priors
    # U[0, 1024] and 56 decodes over U[256, 2048]; replayed from a HIP graph
    pri = list(wl.randint(3, 8, 0, 1024))
    m = Mix(gpu, wl.F16, 32, 4, 64, 16, pri, [256] * 8, list(wl.randint(4, 56, 256, 2048)),
            seed=11)
    sp, sd = m.separate(torch.float16)
    mp, md = m.mixed(torch.float16)
    assert _same(sp, mp) and _same(sd, md) and m.pools_equal()
    pool = m.caches[1].layer(0)
    outp, outd = torch.empty_like(mp), torch.empty_like(md)
    stream = torch.cuda.Stream(gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        pool.mixed_attention(dict(m.prefill, out=outp), dict(m.decode, out=outd), scale=m.scale,
                             stream=torch.cuda.current_stream(gpu))
    for _ in range(3):
        outp.zero_()
        outd.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert _same(outp, mp) and _same(outd, md)
    m.caches[1].check()
    m.close()


def test_mixed_one_side_empty(gpu):
    m = Mix(gpu, wl.BF16, 32, 8, 128, 16, [100], [50], [300, 20], seed=2)
    sp, sd = m.separate(torch.float32)
    pool = m.caches[1].layer(0)
    empty_p = dict(m.prefill, cu_q_lens=m.prefill["cu_q_lens"][:1],
                   context_lens=m.prefill["context_lens"][:0],
                   block_tables=m.prefill["block_tables"][:0])
    _, md = pool.mixed_attention(dict(empty_p, out_dtype=torch.float32),
                                 dict(m.decode, out_dtype=torch.float32), scale=m.scale)
    torch.cuda.synchronize()
    assert _same(sd, md)
    m.close()


def test_mixed_rejects_bad_arguments(gpu):
    m = Mix(gpu, wl.BF16, 32, 8, 128, 16, [100], [50], [300, 20], seed=3)
    pool = m.caches[1].layer(0)
    with pytest.raises(pagedkv.PagedKvError):
        pool.mixed_attention(dict(m.prefill, max_context_len=0), m.decode, scale=m.scale)
    with pytest.raises(pagedkv.PagedKvError):
        pool.mixed_attention(m.prefill, dict(m.decode, out_dtype=torch.float16), scale=m.scale)
    torch.cuda.synchronize()
    assert m.pools_equal()  # neither batch stored its rows
    m.close()


def test_mixed_rejection_enqueues_neither_call(gpu):
    # a shape the one-launch kernel does not take (f32 pool) runs the two
    # calls in sequence; a bad decode batch still stops the prefill's stores
    m = Mix(gpu, wl.F32, 16, 4, 64, 16, [100], [50], [300, 20], seed=4)
    pool = m.caches[1].layer(0)
    with pytest.raises(pagedkv.PagedKvError):
        pool.mixed_attention(m.prefill, dict(m.decode, out_dtype=torch.float16), scale=m.scale)
    torch.cuda.synchronize()
    assert m.pools_equal()
    sp, sd = m.separate(torch.float32)
    mp, md = m.mixed(torch.float32)
    assert _same(sp, mp) and _same(sd, md) and m.pools_equal()
    m.close()


@pytest.mark.parametrize("dt", [wl.F32, wl.BF16])
@pytest.mark.parametrize("side", ["prefill", "decode"])
def test_mixed_negative_count_enqueues_neither_call(gpu, monkeypatch, dt, side):
    # a negative n_seqs or batch in either struct is refused before the
    # other batch is enqueued, on the two-call path (f32) and the one-launch
    # path (bf16): no chunk row is stored
    m = Mix(gpu, dt, 16, 4, 64, 16, [100], [50], [300, 20], seed=5, fused=True)
    pool = m.caches[1].layer(0)
    base = pagedkv._lib.PrefillBatch if side == "prefill" else pagedkv._lib.DecodeBatch
    field = "n_seqs" if side == "prefill" else "batch"

    class Negative(base):
        def __init__(self, *args):
            super().__init__(*args)
            setattr(self, field, -1)

    monkeypatch.setattr(pagedkv._lib, base.__name__, Negative)
    with pytest.raises(pagedkv.PagedKvError, match="< 0"):
        pool.mixed_attention(m.prefill, m.decode, scale=m.scale)
    monkeypatch.undo()
    torch.cuda.synchronize()
    assert m.pools_equal()
    m.close()
