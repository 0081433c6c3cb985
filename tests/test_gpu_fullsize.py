"""GPU checks at the benchmark's full cfg3 and cfg4 shapes (Llama-3-8B KV,
bf16, 256 sequences with contexts U[512, 4096]; Llama-3-70B stage, 128
sequences with contexts U[2048, 8192]; pools 1.2x the live tokens; one
layer), through properties that do not depend on size:
  * moving every live block to another place with in-place compaction
    (pkv_compact) and remapping the tables leaves every decode output bit
    for bit unchanged (attention reads blocks only through the table);
  * permuting the batch permutes the output rows bit for bit (a row's
    result does not depend on its batch mates, paged_batching.rs:40-51);
  * sampled rows equal the fp64 oracle within the north-star tolerance
    (|gpu - ref| <= 1e-3 + 2e-3 |ref|), their K/V read back through
    pkv_gather_seq."""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-3


@pytest.mark.parametrize("shape,B,lo,hi", [(wl.CFG3, 256, 512, 4096), (wl.CFG4, 128, 2048, 8192),
                                           (wl.CFG3, 128, 512, 4096)],
                         ids=["cfg3", "cfg4", "cfg3-B128-split-last-partition"])
def test_full_shape_relocation_permutation_and_oracle(gpu, shape, B, lo, hi):
    batch = wl.decode_batch(shape, B, lo, hi, seed=1234)
    H, KVH, hd, bs = shape.n_head, shape.n_kv_head, shape.head_dim, shape.block_size
    print(f"[fullsize] {shape.name}: B={B}, num_blocks={batch.num_blocks}", flush=True)
    cache = pagedkv.PagedKvCache(1, batch.num_blocks, bs, KVH, hd, torch.bfloat16)
    try:
        cache.fill_normal(77)
        pool = cache.layer(0)
        g = torch.Generator(device="cpu").manual_seed(5)
        q = (torch.randn((B, H, hd), generator=g) / math.sqrt(hd)).to(torch.bfloat16).to(gpu)
        tables = np.where(batch.tables < 0, 0, batch.tables).astype(np.int32)
        cl = torch.from_numpy(batch.context_lens).to(gpu)
        mcl = int(batch.context_lens.max())

        def decode(qq, tb, ll):
            out = pool.decode_attention(qq, torch.from_numpy(np.ascontiguousarray(tb)).to(gpu), ll,
                                        max_context_len=mcl, out_dtype=torch.float32)
            torch.cuda.synchronize()
            cache.check()
            return out

        out = decode(q, tables, cl)

        # batch permutation
        perm = wl.permutation(9, B)
        pt = torch.from_numpy(perm).to(gpu)
        out_p = decode(q[pt], tables[perm], cl[pt])
        assert torch.equal(out_p, out[pt]), "permuted batch changed some row"

        # relocation of every live block (chains and cycles inside the pool)
        live = np.unique(np.concatenate([batch.tables[b, :-(-int(c) // bs)]
                                         for b, c in enumerate(batch.context_lens)]))
        dst = wl.permutation(10, batch.num_blocks)[:live.size].astype(np.int64)
        remap = np.arange(batch.num_blocks, dtype=np.int64)
        remap[live] = dst
        cache.compact(live.tolist(), dst.tolist())
        torch.cuda.synchronize()
        moved_tables = remap[tables].astype(np.int32)
        out_m = decode(q, moved_tables, cl)
        assert torch.equal(out_m, out), "relocated blocks changed some output"

        # sampled rows against the fp64 oracle (K/V read back per sequence)
        qh = q.float().cpu().numpy()
        got = out.cpu().numpy()
        for b in (0, 77, B // 2 + 3, B - 1):
            n = int(batch.context_lens[b])
            k, v = pool.gather_seq(moved_tables[b].tolist(), n)
            nb = -(-n // bs)
            kp = np.zeros((nb * bs, KVH, hd), np.uint16)
            vp = np.zeros_like(kp)
            kp[:n] = k.view(torch.int16).cpu().numpy().view(np.uint16)
            vp[:n] = v.view(torch.int16).cpu().numpy().view(np.uint16)
            ref = oracle.paged_attention_f64(kp.reshape(nb, bs, KVH, hd), vp.reshape(nb, bs, KVH, hd),
                                             wl.BF16, bs, np.arange(nb, dtype=np.uint32)[None],
                                             np.array([n]), qh[b:b + 1], 1.0 / math.sqrt(hd))
            err = np.abs(got[b] - ref[0])
            assert (err <= ATOL + RTOL * np.abs(ref[0])).all(), (
                f"row {b}: max err {err.max():.3g}")
    finally:
        cache.close()


def test_full_shape_positions_bound_equals_shorter_context(gpu):
    # build_mask's second bound at the full cfg3 shape: attention with
    # positions (k <= positions[b], attention.rs:22) equals plain decode over
    # min(context_lens, positions + 1) keys bit for bit -- both lay the
    # partitions out over that bounded length; positions at, below and past
    # each context
    shape, B = wl.CFG3, 256
    batch = wl.decode_batch(shape, B, 512, 4096, seed=1234)
    H, KVH, hd, bs = shape.n_head, shape.n_kv_head, shape.head_dim, shape.block_size
    print(f"[fullsize] positions bound: B={B}, num_blocks={batch.num_blocks}", flush=True)
    cache = pagedkv.PagedKvCache(1, batch.num_blocks, bs, KVH, hd, torch.bfloat16)
    try:
        cache.fill_normal(78)
        pool = cache.layer(0)
        g = torch.Generator(device="cpu").manual_seed(6)
        q = (torch.randn((B, H, hd), generator=g) / math.sqrt(hd)).to(torch.bfloat16).to(gpu)
        tables = torch.from_numpy(np.where(batch.tables < 0, 0, batch.tables).astype(np.int32)).to(gpu)
        cl = batch.context_lens.astype(np.int64)
        r = np.random.default_rng(11)
        pos = np.where(np.arange(B) % 4 == 0, cl - 1,                     # the engine's own position
                       np.where(np.arange(B) % 4 == 1, cl + r.integers(0, 900, B),  # past the context
                                r.integers(0, cl)))                        # somewhere before it
        mcl = int(cl.max())
        out_p = pool.decode_attention(q, tables, torch.from_numpy(cl.astype(np.int32)).to(gpu),
                                      max_context_len=mcl, out_dtype=torch.float32,
                                      positions=torch.from_numpy(pos.astype(np.int32)).to(gpu))
        short = np.minimum(cl, pos + 1).astype(np.int32)
        out_s = pool.decode_attention(q, tables, torch.from_numpy(short).to(gpu),
                                      max_context_len=mcl, out_dtype=torch.float32)
        torch.cuda.synchronize()
        cache.check()
        assert torch.equal(out_p, out_s), "positions bound differs from the shorter context"
    finally:
        cache.close()
