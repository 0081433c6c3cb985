"""The reference's own parity shape through every attention path of the
engine: Qwen2-0.5B's attention (14 query heads over 2 kv heads, a GQA ratio
of 7; head_dim 64; rope_freq_base 1e6) with the engine settings of the
reference's correctness gate (crates/ai-engine-candle/tests/paged_parity.rs:
58-68: block_size 16, kv_cache_blocks 256).

Three prompts are prefilled in one chunked launch (RoPE and the K/V store
either in pkv_append_rope or in the attention launch itself), then decoded
for several steps with the rotary embedding and the append fused into the
decode kernel, block tables grown by the BlockAllocator as the engine does
(engine.rs:102-133, 203-206).  Every output is checked against the fp64
closed form over the oracle's own pool (tolerance 1e-3 + 2e-3 |ref|), and
the pool bytes at the end against the oracle's writes, bit for bit.  The
pool dtypes are f32 (the reference's KvPool dtype) and bf16."""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}
H, KVH, HD, BS, NBLOCKS, BASE = 14, 2, 64, 16, 256, 1000000.0
RTOL, ATOL = 2e-3, 1e-3


def _close(got, ref, what):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} outside tolerance, max err {err.max():.3g}"


def _padded(tables):
    w = max(len(t.blocks) for t in tables)
    out = np.zeros((len(tables), w), np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t.blocks)] = t.blocks
    return out


@pytest.mark.parametrize("dt", [wl.F32, wl.BF16])
@pytest.mark.parametrize("store", ["append_rope", "fused"])
def test_qwen2_prompts_then_decode(gpu, dt, store):
    max_seq = 4096
    scale = 1.0 / math.sqrt(HD)
    rope = pagedkv.Rope(HD, BASE, max_seq)
    cs, sn = oracle.rope_table(HD, BASE, max_seq)
    cache = pagedkv.PagedKvCache(1, NBLOCKS, BS, KVH, HD, TD[dt])
    alloc = pagedkv.BlockAllocator(NBLOCKS, BS)
    nd = np.float32 if dt == wl.F32 else np.uint16
    kp = np.zeros((NBLOCKS, BS, KVH, HD), nd)   # KvPool::new: zeros
    vp = np.zeros_like(kp)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)

    # ---- prefill: three prompts in one launch ----
    prompts = [6, 23, 40]
    tables = [pagedkv.BlockTable() for _ in prompts]
    for t, n in zip(tables, prompts):
        alloc.ensure_capacity(t, n)
    T = sum(prompts)
    k = wl.normal_storage(11, (T, KVH, HD), wl.F32)   # the f32 projections
    v = wl.normal_storage(12, (T, KVH, HD), wl.F32)
    q = wl.normal_storage(13, (T, H, HD), wl.F32)
    pos = np.concatenate([np.arange(n) for n in prompts]).astype(np.int32)
    slots = np.array([alloc.slot(t, p) for t, n in zip(tables, prompts) for p in range(n)],
                     np.int32)
    cu = np.concatenate([[0], np.cumsum(prompts)]).astype(np.int32)
    ctx = np.asarray(prompts, np.int32)
    tb = _padded(tables)
    pool = cache.layer(0)
    if store == "append_rope":
        q_rot = pool.append_rope(rope, dev(k), dev(v), dev(slots), dev(pos), q=dev(q))
        out = pool.prefill_attention(q_rot, dev(cu), dev(ctx), dev(tb), max_q_len=max(prompts),
                                     max_context_len=max(prompts), scale=scale,
                                     out_dtype=torch.float32)
    else:
        pd = dev(pos)
        q_rot = rope.apply(dev(q), pd, out_dtype=TD[dt])
        k_rot = rope.apply(dev(k), pd, out_dtype=TD[dt])
        out = pool.prefill_attention(q_rot, dev(cu), dev(ctx), dev(tb), max_q_len=max(prompts),
                                     max_context_len=max(prompts), scale=scale,
                                     out_dtype=torch.float32, k_new=k_rot,
                                     v_new=dev(v).to(TD[dt]))
    torch.cuda.synchronize()
    cache.check()
    kr = wl.to_storage(oracle.rope_apply(k, cs, sn, pos), dt)
    vr = wl.to_storage(v, dt)
    qr = wl.to_storage(oracle.rope_apply(q, cs, sn, pos), dt)
    for s, t in enumerate(tables):
        rows = slice(int(cu[s]), int(cu[s + 1]))
        oracle.kv_write(kp, vp, BS, np.asarray(t.blocks, np.uint32), 0, kr[rows], vr[rows])
    ref = oracle.prefill_attention_f64(kp, vp, dt, BS, tb.astype(np.uint32), cu, ctx,
                                       wl.widen(qr, dt), scale)
    _close(out.cpu().numpy(), ref, f"prefill dt={dt} store={store}")

    # ---- decode: the RoPE and the append fused into the attention launch ----
    lens = list(prompts)
    for step in range(7):
        for t, n in zip(tables, lens):
            alloc.ensure_capacity(t, n + 1)   # engine.rs:116 before the step
        tb = _padded(tables)
        B = len(lens)
        qd = wl.normal_storage(100 + step, (B, H, HD), wl.F32)
        kd = wl.normal_storage(200 + step, (B, KVH, HD), wl.F32)
        vd = wl.normal_storage(300 + step, (B, KVH, HD), wl.F32)
        cl = (np.asarray(lens) + 1).astype(np.int32)
        got = pool.decode_attention(dev(qd), dev(tb), dev(cl), k_new=dev(kd), v_new=dev(vd),
                                    rope=rope, scale=scale, out_dtype=torch.float32)
        torch.cuda.synchronize()
        cache.check()
        p = np.asarray(lens, np.int32)   # positions == seq_lens (engine.rs:130-133)
        kr = wl.to_storage(oracle.rope_apply(kd, cs, sn, p), dt)
        qr = wl.to_storage(oracle.rope_apply(qd, cs, sn, p), dt)
        vr = wl.to_storage(vd, dt)
        for b, t in enumerate(tables):
            oracle.kv_write(kp, vp, BS, np.asarray(t.blocks, np.uint32), lens[b],
                            kr[b:b + 1], vr[b:b + 1])
        ref = oracle.paged_attention_f64(kp, vp, dt, BS, tb.astype(np.uint32), cl,
                                         wl.widen(qr, dt), scale)
        _close(got.cpu().numpy(), ref, f"decode step {step} dt={dt}")
        lens = [n + 1 for n in lens]

    assert np.array_equal(cache.read_bytes(0, pagedkv.K), kp.view(np.uint8).reshape(-1))
    assert np.array_equal(cache.read_bytes(0, pagedkv.V), vp.view(np.uint8).reshape(-1))
    cache.close()
    rope.close()


@pytest.mark.parametrize("dt", [wl.F32, wl.BF16])
def test_qwen2_batched_equals_solo(gpu, dt):
    # paged_batching.rs:40-51 at the attention level, Qwen2 shape: a row's
    # output bits do not depend on its batch mates
    ctx = [5, 130, 777, 2047]
    need = [-(-(c + 1) // BS) for c in ctx]
    nb = sum(need) + 4
    perm = wl.permutation(9, nb)
    tb = np.zeros((len(ctx), max(need)), np.int32)
    o = 0
    for b, n in enumerate(need):
        tb[b, :n] = perm[o:o + n]
        o += n
    cache = pagedkv.PagedKvCache(1, nb, BS, KVH, HD, TD[dt])
    cache.write_bytes(0, pagedkv.K, wl.normal_storage(1, (nb, BS, KVH, HD), dt))
    cache.write_bytes(0, pagedkv.V, wl.normal_storage(2, (nb, BS, KVH, HD), dt))
    q = wl.normal_storage(3, (len(ctx), H, HD), dt, scale=1 / math.sqrt(HD))
    qd = torch.from_numpy(q.view(np.int16) if dt != wl.F32 else q).to(gpu)
    if dt != wl.F32:
        qd = qd.view(TD[dt])
    cl = torch.tensor([c + 1 for c in ctx], dtype=torch.int32, device=gpu)
    tbd = torch.from_numpy(tb).to(gpu)
    full = cache.layer(0).decode_attention(qd, tbd, cl, max_context_len=max(ctx) + 1,
                                           out_dtype=torch.float32).cpu()
    for b in range(len(ctx)):
        solo = cache.layer(0).decode_attention(qd[b:b + 1], tbd[b:b + 1], cl[b:b + 1],
                                               max_context_len=max(ctx) + 1,
                                               out_dtype=torch.float32).cpu()
        assert torch.equal(solo[0], full[b])
    cache.close()
