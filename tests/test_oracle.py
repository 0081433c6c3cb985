"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each oracle function is checked against something it does not share code
with: the reference's own known-answer tests (block_table.rs:65-116,
attention.rs:142-156), an independent library routine (torch float64
scaled_dot_product_attention), closed forms computed with numpy indexing,
special cases whose answer is fixed by the mathematics, and mutation checks
showing that a plausible mistake (wrong GQA mapping, missing scale, wrong
slot formula, off-by-one causal mask) would be caught.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from block_table import BlockAllocator, BlockTable, CapacityError
from pagedkv import workload as wl


# ---------------------------------------------------------------------------
# reference KATs
# ---------------------------------------------------------------------------
def test_build_mask_kat():
    # attention.rs:142-156
    m = oracle.build_mask([3, 1], [2, 0], 4)
    assert m.shape == (2, 1, 1, 4)
    v = m.reshape(-1)
    assert v[0] == 0.0 and v[1] == 0.0 and v[2] == 0.0
    assert np.isneginf(v[3])
    assert v[4] == 0.0
    assert np.isneginf(v[5]) and np.isneginf(v[6]) and np.isneginf(v[7])


def test_allocator_kat_blocks_for_rounds_up():  # block_table.rs:65-72
    a = BlockAllocator(10, 16)
    assert [a.blocks_for(n) for n in (0, 1, 16, 17)] == [0, 1, 1, 2]


def test_allocator_kat_ensure_capacity_allocates_and_reuses():  # :74-85
    a = BlockAllocator(4, 16)
    t = BlockTable()
    a.ensure_capacity(t, 1)
    assert t.blocks == [0]
    a.ensure_capacity(t, 16)
    assert t.blocks == [0]
    a.ensure_capacity(t, 17)
    assert t.blocks == [0, 1]
    assert a.free_count() == 2


def test_allocator_kat_release_returns_blocks():  # :87-96
    a = BlockAllocator(4, 16)
    t = BlockTable()
    a.ensure_capacity(t, 40)
    assert a.free_count() == 1
    a.release(t)
    assert a.free_count() == 4
    assert t.blocks == []


def test_allocator_kat_oom_no_partial():  # :98-105
    a = BlockAllocator(2, 16)
    t = BlockTable()
    with pytest.raises(CapacityError):
        a.ensure_capacity(t, 48)
    assert t.blocks == []
    assert a.free_count() == 2


def test_allocator_kat_locate():  # :107-116
    a = BlockAllocator(4, 16)
    t = BlockTable()
    a.ensure_capacity(t, 32)
    assert a.locate(t, 0) == (0, 0)
    assert a.locate(t, 15) == (0, 15)
    assert a.locate(t, 16) == (1, 0)
    assert a.locate(t, 31) == (1, 15)


def test_allocator_lifo_reuse_order():
    # release appends in table order; the next pop is the table's last block
    a = BlockAllocator(8, 16)
    t1, t2 = BlockTable(), BlockTable()
    a.ensure_capacity(t1, 48)  # [0, 1, 2]
    a.release(t1)
    a.ensure_capacity(t2, 32)
    assert t2.blocks == [2, 1]


# ---------------------------------------------------------------------------
# scatter / gather: closed form with numpy indexing
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_kv_write_and_gather_closed_form(dtype):
    rng = np.random.default_rng(1)
    nb, bs, kvh, hd = 9, 16, 3, 8
    kp = rng.integers(0, 60000, size=(nb, bs, kvh, hd)).astype(dtype)
    vp = rng.integers(0, 60000, size=(nb, bs, kvh, hd)).astype(dtype)
    kp0, vp0 = kp.copy(), vp.copy()
    blocks = np.array([7, 2, 5], dtype=np.uint32)
    start, n = 13, 20
    k = rng.integers(0, 60000, size=(n, kvh, hd)).astype(dtype)
    v = rng.integers(0, 60000, size=(n, kvh, hd)).astype(dtype)
    oracle.kv_write(kp, vp, bs, blocks, start, k, v)
    exp_k, exp_v = kp0.reshape(nb * bs, kvh, hd).copy(), vp0.reshape(nb * bs, kvh, hd).copy()
    pos = np.arange(start, start + n)
    slots = blocks[pos // bs].astype(np.int64) * bs + pos % bs
    exp_k[slots] = k
    exp_v[slots] = v
    assert np.array_equal(kp.reshape(nb * bs, kvh, hd), exp_k)  # and nothing else changed
    assert np.array_equal(vp.reshape(nb * bs, kvh, hd), exp_v)
    gk, gv = oracle.gather_seq(kp, vp, bs, blocks, start + n)
    allpos = np.arange(start + n)
    s2 = blocks[allpos // bs].astype(np.int64) * bs + allpos % bs
    assert np.array_equal(gk, exp_k[s2]) and np.array_equal(gv, exp_v[s2])
    with pytest.raises(IndexError):
        oracle.gather_seq(kp, vp, bs, blocks, 3 * bs + 1)


def test_kv_write_mutation_slot_formula_detected():
    # A slot formula that forgot the block indirection (pos instead of
    # blocks[pos/bs]*bs + pos%bs) gives a different pool.
    nb, bs, kvh, hd = 6, 16, 1, 4
    kp = np.zeros((nb, bs, kvh, hd), np.float32)
    vp = np.zeros_like(kp)
    blocks = np.array([4, 1], np.uint32)
    k = np.ones((3, kvh, hd), np.float32)
    oracle.kv_write(kp, vp, bs, blocks, 0, k, k)
    wrong = np.zeros_like(kp).reshape(nb * bs, kvh, hd)
    wrong[0:3] = 1
    assert not np.array_equal(kp.reshape(nb * bs, kvh, hd), wrong)
    assert kp[4, 0:3].sum() == 3 * hd


# ---------------------------------------------------------------------------
# sdpa: torch float64 as the independent library routine
# ---------------------------------------------------------------------------
def _torch_sdpa64(q, k, v, mask, n_head, n_kv, scale, gqa="consecutive"):
    q = torch.from_numpy(np.asarray(q, np.float64))
    k = torch.from_numpy(np.asarray(k, np.float64))
    v = torch.from_numpy(np.asarray(v, np.float64))
    r = n_head // n_kv
    if gqa == "consecutive":
        k = k.repeat_interleave(r, dim=1)
        v = v.repeat_interleave(r, dim=1)
    else:  # the plausible mistake: head h -> kv head h % n_kv
        k = k.repeat(1, r, 1, 1)
        v = v.repeat(1, r, 1, 1)
    m = torch.from_numpy(np.asarray(mask, np.float64))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=m, scale=scale)
    B, H, Lq, hd = o.shape
    return o.transpose(1, 2).reshape(B, Lq, H * hd).numpy()


@pytest.mark.parametrize("B,H,KVH,Lq,kv,hd", [(2, 4, 2, 1, 37, 16), (1, 8, 1, 3, 20, 8),
                                                (3, 4, 4, 1, 5, 32), (2, 8, 2, 2, 64, 64),
                                                (2, 14, 2, 1, 40, 16), (1, 9, 3, 2, 21, 8),
                                                (2, 12, 2, 1, 33, 16), (1, 20, 1, 1, 17, 8)])
def test_sdpa_f32_matches_torch_float64(B, H, KVH, Lq, kv, hd):
    rng = np.random.default_rng(B * 100 + kv)
    q = rng.standard_normal((B, H, Lq, hd)).astype(np.float32)
    k = rng.standard_normal((B, KVH, kv, hd)).astype(np.float32)
    v = rng.standard_normal((B, KVH, kv, hd)).astype(np.float32)
    lens = rng.integers(1, kv + 1, size=B)
    pos = np.array([l - 1 for l in lens])
    mask = np.repeat(oracle.build_mask(lens, pos, kv), Lq, axis=2)
    scale = 1.0 / math.sqrt(hd)
    got = oracle.sdpa_f32(q, k, v, mask, H, KVH)
    ref = _torch_sdpa64(q, k, v, mask, H, KVH, scale)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)
    if 1 < KVH < H:  # the wrong GQA mapping is distinguishable
        bad = _torch_sdpa64(q, k, v, mask, H, KVH, scale, gqa="modulo")
        assert np.abs(got - bad).max() > 1e-2
    # a missing scale is distinguishable
    noscale = _torch_sdpa64(q, k, v, mask, H, KVH, 1.0)
    assert np.abs(got - noscale).max() > 1e-3


def test_sdpa_special_cases():
    rng = np.random.default_rng(7)
    hd = 16
    # one key -> that V row exactly
    q = rng.standard_normal((1, 2, 1, hd)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, hd)).astype(np.float32)
    v = rng.standard_normal((1, 1, 1, hd)).astype(np.float32)
    out = oracle.sdpa_f32(q, k, v, np.zeros((1, 1, 1, 1), np.float32), 2, 1)
    assert np.array_equal(out.reshape(2, hd), np.repeat(v.reshape(1, hd), 2, 0))
    # identical keys -> mean of V
    n = 9
    k = np.repeat(rng.standard_normal((1, 1, 1, hd)).astype(np.float32), n, axis=2)
    v = rng.standard_normal((1, 1, n, hd)).astype(np.float32)
    out = oracle.sdpa_f32(q, k, v, np.zeros((1, 1, 1, n), np.float32), 2, 1)
    np.testing.assert_allclose(out.reshape(2, hd), np.repeat(v[0, 0].mean(0, keepdims=True), 2, 0),
                               rtol=1e-5, atol=1e-6)
    # one dominant score -> that V row
    k = rng.standard_normal((1, 1, n, hd)).astype(np.float32) * 0.01
    k[0, 0, 4] = q[0, 0, 0] * 100.0
    out = oracle.sdpa_f32(q[:, :1], k, v, np.zeros((1, 1, 1, n), np.float32), 1, 1)
    np.testing.assert_allclose(out.reshape(hd), v[0, 0, 4], rtol=1e-5, atol=1e-5)
    # padding invariance: zero keys/values behind -inf mask add nothing
    k2 = np.concatenate([k, np.zeros((1, 1, 5, hd), np.float32)], axis=2)
    v2 = np.concatenate([v, np.zeros((1, 1, 5, hd), np.float32)], axis=2)
    m2 = oracle.build_mask([n], [n - 1], n + 5)
    out2 = oracle.sdpa_f32(q[:, :1], k2, v2, m2, 1, 1)
    assert np.array_equal(out, out2)


# ---------------------------------------------------------------------------
# decode step: reference op order (gather/pad/mask/sdpa) vs ragged closed form
# ---------------------------------------------------------------------------
def _random_paged(seed, B, KVH, hd, bs, ctx_hi, dtype=wl.F32):
    ctx = wl.randint(seed, B, 0, ctx_hi)
    need = -(-(ctx + 1) // bs)
    nb = int(need.sum()) + 3
    perm = wl.permutation(seed + 1, nb)
    tables = np.zeros((B, int(need.max())), np.uint32)
    o = 0
    for b in range(B):
        tables[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    kp = wl.normal_storage(seed + 2, (nb, bs, KVH, hd), dtype)
    vp = wl.normal_storage(seed + 3, (nb, bs, KVH, hd), dtype)
    return ctx, tables, kp, vp


@pytest.mark.parametrize("B,H,KVH,hd,bs", [(3, 8, 2, 16, 16), (4, 4, 4, 8, 16), (2, 8, 1, 32, 32),
                                           (3, 14, 2, 16, 16), (2, 15, 5, 8, 16)])
def test_decode_step_f32_matches_closed_form(B, H, KVH, hd, bs):
    ctx, tables, kp, vp = _random_paged(11 + B, B, KVH, hd, bs, 70)
    rng = np.random.default_rng(3)
    q = rng.standard_normal((B, H, hd)).astype(np.float32)
    kn = rng.standard_normal((B, KVH, hd)).astype(np.float32)
    vn = rng.standard_normal((B, KVH, hd)).astype(np.float32)
    kp_ref, vp_ref = kp.copy(), vp.copy()
    out = oracle.decode_step_f32(kp, vp, bs, tables, ctx, ctx, q, kn, vn)
    # the append happened at seq_lens[b]
    for b in range(B):
        s = tables[b, ctx[b] // bs] * bs + ctx[b] % bs
        kp_ref.reshape(-1, KVH, hd)[s] = kn[b]
        vp_ref.reshape(-1, KVH, hd)[s] = vn[b]
    assert np.array_equal(kp, kp_ref) and np.array_equal(vp, vp_ref)
    ref = oracle.paged_attention_f64(kp, vp, wl.F32, bs, tables, ctx + 1, q, 1 / math.sqrt(hd))
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_decode_step_faithful_equals_in_place():
    # the reference-faithful cost model (a full pool copy per appended row)
    # leaves the same pool bytes and output bits as the in-place restatement
    B, H, KVH, hd, bs = 4, 8, 2, 16, 16
    ctx, tables, kp, vp = _random_paged(21, B, KVH, hd, bs, 90)
    rng = np.random.default_rng(8)
    q = rng.standard_normal((B, H, hd)).astype(np.float32)
    kn = rng.standard_normal((B, KVH, hd)).astype(np.float32)
    vn = rng.standard_normal((B, KVH, hd)).astype(np.float32)
    k2, v2 = kp.copy(), vp.copy()
    a = oracle.decode_step_f32(kp, vp, bs, tables, ctx, ctx, q, kn, vn)
    b = oracle.decode_step_faithful_f32(k2, v2, bs, tables, ctx, ctx, q, kn, vn)
    assert np.array_equal(a, b)
    assert np.array_equal(kp, k2) and np.array_equal(vp, v2)


def test_prefill_chunk_faithful_matches_closed_form():
    # the reference's cost model for a chunk (full pool copy per token, dense
    # masked attention over all prior + C keys): the same pool bytes as the
    # plain writes, outputs equal to the fp64 closed form, and with no prior
    # the reference's prefill_seq attention
    H, KVH, hd, bs = 14, 2, 16, 16
    for P, C, copies in ((29, 21, None), (0, 37, 5), (40, 1, 0)):
        tb, kp, vp, q = _prefill_setup(61 + P, P, C, H, KVH, hd, bs)
        rng = np.random.default_rng(P + C)
        kn = rng.standard_normal((C, KVH, hd)).astype(np.float32)
        vn = rng.standard_normal((C, KVH, hd)).astype(np.float32)
        k2, v2 = kp.copy(), vp.copy()
        got = oracle.prefill_chunk_faithful_f32(kp, vp, bs, tb, P, q[P:], kn, vn,
                                                n_copies=copies)
        oracle.kv_write(k2, v2, bs, tb, P, kn, vn)
        assert np.array_equal(kp, k2) and np.array_equal(vp, v2)
        ref = oracle.prefill_attention_f64(kp, vp, wl.F32, bs, tb[None], [0, C], [P + C], q[P:],
                                           1 / math.sqrt(hd))
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
        if P == 0:
            gk, gv = oracle.gather_seq(kp, vp, bs, tb, C)
            seq = oracle.prefill_seq_f32(q.transpose(1, 0, 2), gk.transpose(1, 0, 2),
                                         gv.transpose(1, 0, 2), KVH)
            np.testing.assert_allclose(got, seq, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("H,KVH", [(8, 2), (14, 2), (6, 2), (21, 3)])
def test_paged_attention_f64_matches_torch_on_gathered(H, KVH):
    B, hd, bs = 3, 16, 16
    ctx, tables, kp, vp = _random_paged(5, B, KVH, hd, bs, 50, wl.BF16)
    q = wl.widen(wl.normal_storage(9, (B, H, hd), wl.BF16), wl.BF16)
    got = oracle.paged_attention_f64(kp, vp, wl.BF16, bs, tables, ctx + 1, q, 0.25)
    kf, vf = wl.widen(kp, wl.BF16), wl.widen(vp, wl.BF16)
    for b in range(B):
        n = int(ctx[b]) + 1
        gk, gv = oracle.gather_seq(kf, vf, bs, tables[b], n)
        ref = _torch_sdpa64(q[b][None, :, None], gk.transpose(1, 0, 2)[None],
                            gv.transpose(1, 0, 2)[None], np.zeros((1, 1, 1, n)), H, KVH, 0.25)
        np.testing.assert_allclose(got[b], ref.reshape(-1), rtol=1e-10, atol=1e-12)


def test_decode_inplace_baseline_matches_closed_form():
    B, H, KVH, hd, bs = 5, 8, 2, 32, 16
    ctx, tables, kp, vp = _random_paged(21, B, KVH, hd, bs, 90, wl.BF16)
    q = wl.normal_storage(22, (B, H, hd), wl.BF16)
    kn = wl.normal_storage(23, (B, KVH, hd), wl.BF16)
    vn = wl.normal_storage(24, (B, KVH, hd), wl.BF16)
    cl = (ctx + 1).astype(np.int32)
    kp2, vp2 = kp.copy(), vp.copy()
    out = oracle.decode_inplace(kp2, vp2, wl.BF16, bs, tables.astype(np.int32), cl, q, kn, vn,
                                1 / math.sqrt(hd), n_threads=2)
    ref = oracle.paged_attention_f64(kp2, vp2, wl.BF16, bs, tables, cl, wl.widen(q, wl.BF16),
                                     1 / math.sqrt(hd))
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# prefill: reductions and chunk invariance
# ---------------------------------------------------------------------------
def _prefill_setup(seed, P, C, H, KVH, hd, bs):
    n = P + C
    nb = -(-n // bs) + 2
    tb = wl.permutation(seed, nb)[: -(-n // bs)].astype(np.uint32)
    kp = wl.normal_storage(seed + 1, (nb, bs, KVH, hd), wl.F32)
    vp = wl.normal_storage(seed + 2, (nb, bs, KVH, hd), wl.F32)
    q = wl.normal(seed + 3, n * H * hd).reshape(n, H, hd).astype(np.float32)
    return tb, kp, vp, q


@pytest.mark.parametrize("H,KVH", [(4, 2), (14, 2), (9, 3)])
def test_prefill_reduces_to_reference_prefill_seq(H, KVH):
    # prior context 0: the reference's one-shot causal prefill attention
    hd, bs, N = 16, 16, 37
    tb, kp, vp, q = _prefill_setup(31, 0, N, H, KVH, hd, bs)
    got = oracle.prefill_attention_f64(kp, vp, wl.F32, bs, tb[None], [0, N], [N], q,
                                       1 / math.sqrt(hd))
    gk, gv = oracle.gather_seq(kp, vp, bs, tb, N)
    ref = oracle.prefill_seq_f32(q.transpose(1, 0, 2), gk.transpose(1, 0, 2), gv.transpose(1, 0, 2),
                                 KVH)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    # an off-by-one causal mask (j >= i masked) would differ
    wrong_first = gv[0]  # query 0 attends key 0 only
    np.testing.assert_allclose(got[0].reshape(H, hd)[0], wrong_first[0], rtol=1e-6, atol=1e-6)


def test_prefill_chunking_invariance_and_decode_reduction():
    H, KVH, hd, bs = 8, 2, 16, 16
    P, C = 29, 21
    n = P + C
    tb, kp, vp, q = _prefill_setup(41, P, C, H, KVH, hd, bs)
    scale = 1 / math.sqrt(hd)
    full = oracle.prefill_attention_f64(kp, vp, wl.F32, bs, tb[None], [0, n], [n], q, scale)
    chunk = oracle.prefill_attention_f64(kp, vp, wl.F32, bs, tb[None], [0, C], [n], q[P:], scale)
    np.testing.assert_allclose(chunk, full[P:], rtol=1e-12, atol=1e-14)
    # one query at position n-1 is the decode case
    dec = oracle.paged_attention_f64(kp, vp, wl.F32, bs, tb[None], [n], q[n - 1:n], scale)
    np.testing.assert_allclose(dec, full[n - 1:n], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("H,KVH", [(2, 1), (6, 2), (7, 1)])
def test_prefill_brute_force_tiny(H, KVH):
    hd, bs = 4, 16
    P, C = 3, 2
    tb, kp, vp, q = _prefill_setup(51, P, C, H, KVH, hd, bs)
    got = oracle.prefill_attention_f64(kp, vp, wl.F32, bs, tb[None], [0, C], [P + C], q[P:], 0.5)
    kf, vf = oracle.gather_seq(kp, vp, bs, tb, P + C)
    for i in range(C):
        for h in range(H):
            g = h // (H // KVH)   # query head h reads kv head h / (H / KVH)
            s = [0.5 * float(np.dot(q[P + i, h].astype(np.float64), kf[j, g])) for j in range(P + i + 1)]
            w = np.exp(np.array(s) - max(s))
            w /= w.sum()
            o = (w[:, None] * vf[: P + i + 1, g].astype(np.float64)).sum(0)
            np.testing.assert_allclose(got[i, h * hd:(h + 1) * hd], o, rtol=1e-12, atol=1e-14)


def test_prefill_inplace_baseline_matches_closed_form():
    # the CPU baseline's chunked prefill (f32, stored chunk K/V first) against
    # the fp64 closed form over the same pool, two sequences with priors
    H, KVH, hd, bs = 8, 2, 32, 16
    priors, chunks = np.array([0, 45]), np.array([37, 20])
    lens = priors + chunks
    need = -(-lens // bs)
    nb = int(need.sum()) + 2
    perm = wl.permutation(61, nb)
    tables = np.zeros((2, int(need.max())), np.int32)
    tables[0, :need[0]] = perm[:need[0]]
    tables[1, :need[1]] = perm[need[0]:need[0] + need[1]]
    kp = wl.normal_storage(62, (nb, bs, KVH, hd), wl.F16)
    vp = wl.normal_storage(63, (nb, bs, KVH, hd), wl.F16)
    T = int(chunks.sum())
    q = wl.normal_storage(64, (T, H, hd), wl.F16, scale=1 / math.sqrt(hd))
    kn = wl.normal_storage(65, (T, KVH, hd), wl.F16)
    vn = wl.normal_storage(66, (T, KVH, hd), wl.F16)
    cu = np.array([0, chunks[0], T], np.int32)
    kp2, vp2 = kp.copy(), vp.copy()
    out = oracle.prefill_inplace(kp2, vp2, wl.F16, bs, tables, cu, lens.astype(np.int32), q, kn, vn,
                                 1 / math.sqrt(hd), n_threads=3)
    # the chunk store is the closed-form scatter
    kp3, vp3 = kp.copy(), vp.copy()
    for s_ in range(2):
        tb = tables[s_].astype(np.uint32)
        oracle.kv_write(kp3, vp3, bs, tb, int(priors[s_]), kn[cu[s_]:cu[s_ + 1]], vn[cu[s_]:cu[s_ + 1]])
    assert np.array_equal(kp2, kp3) and np.array_equal(vp2, vp3)
    ref = oracle.prefill_attention_f64(kp2, vp2, wl.F16, bs, tables.astype(np.uint32), cu, lens,
                                       wl.widen(q, wl.F16), 1 / math.sqrt(hd))
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# block copy / compaction closed forms
# ---------------------------------------------------------------------------
def test_copy_and_compact_closed_form():
    rng = np.random.default_rng(5)
    L, nb, bb = 3, 12, 32
    pool = rng.integers(0, 255, size=L * 2 * nb * bb).astype(np.uint8)
    p0 = pool.copy().reshape(L * 2, nb, bb)
    oracle.copy_blocks(pool, L, bb, [1, 4], [7, 9])
    exp = p0.copy()
    exp[:, 7] = p0[:, 1]
    exp[:, 9] = p0[:, 4]
    assert np.array_equal(pool.reshape(L * 2, nb, bb), exp)
    # compaction with overlapping src/dst (a cycle 0<->3 and a chain 5->0? no: dst distinct)
    src = [3, 0, 8, 10]
    dst = [0, 3, 1, 8]
    p1 = pool.copy().reshape(L * 2, nb, bb)
    oracle.compact(pool, L, bb, src, dst)
    exp = p1.copy()
    for s, d in zip(src, dst):
        exp[:, d] = p1[:, s]
    assert np.array_equal(pool.reshape(L * 2, nb, bb), exp)


# ---------------------------------------------------------------------------
# committed golden vectors (regression pin of the oracle itself)
# ---------------------------------------------------------------------------
def test_golden_vectors_reproduce():
    import glob
    import os
    here = os.path.join(os.path.dirname(__file__), "golden")
    files = sorted(glob.glob(os.path.join(here, "decode_*.npz")))
    assert files, "golden fixtures missing (tests/golden/make_golden.py)"
    for f in files:
        z = np.load(f, allow_pickle=False)
        dt = int(z["dtype"])
        got = oracle.paged_attention_f64(z["k_pool"], z["v_pool"], dt, int(z["block_size"]),
                                         z["tables"], z["context_lens"],
                                         wl.widen(z["q"], dt), float(z["scale"]))
        np.testing.assert_allclose(got, z["out"], rtol=1e-12, atol=1e-14, err_msg=f)
