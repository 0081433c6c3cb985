"""GPU parity of the byte-moving kernels (append/scatter, gather, block copy,
compaction) against the CPU oracle: bit-exact, and no other byte changes."""
import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}
ND = {wl.F32: np.float32, wl.F16: np.uint16, wl.BF16: np.uint16}


def _host_pool(cache, layer):
    """Layer's K and V as (num_blocks, bs, kvh, hd) storage arrays."""
    nd = ND[pagedkv.pkv_dtype(cache.dtype)]
    shp = (cache.num_blocks, cache.block_size, cache.n_kv_head, cache.head_dim)
    k = cache.read_bytes(layer, pagedkv.K).view(nd).reshape(shp)
    v = cache.read_bytes(layer, pagedkv.V).view(nd).reshape(shp)
    return k, v


def _to_dev(a, dt, device):
    """Storage array (float32 or uint16 bits) -> device tensor of dtype dt."""
    a = np.ascontiguousarray(a)
    if dt == wl.F32:
        return torch.from_numpy(a).to(device)
    return torch.from_numpy(a.view(np.int16)).view(TD[dt]).to(device)


def _fill(cache, seed):
    dt = pagedkv.pkv_dtype(cache.dtype)
    shp = (cache.num_blocks, cache.block_size, cache.n_kv_head, cache.head_dim)
    for l in range(cache.n_layers):
        cache.write_bytes(l, pagedkv.K, wl.normal_storage(seed + 2 * l, shp, dt))
        cache.write_bytes(l, pagedkv.V, wl.normal_storage(seed + 2 * l + 1, shp, dt))


@pytest.mark.parametrize("dt", [wl.BF16, wl.F16, wl.F32])
@pytest.mark.parametrize("hd,kvh,bs", [(128, 8, 16), (64, 4, 32), (256, 2, 16)])
def test_append_bit_exact_and_untouched(gpu, dt, hd, kvh, bs):
    cache = pagedkv.PagedKvCache(2, 40, bs, kvh, hd, TD[dt])
    _fill(cache, 100)
    k0, v0 = _host_pool(cache, 1)
    n = 37
    rng = np.random.default_rng(hd + bs)
    slots = rng.choice(40 * bs, size=n, replace=False).astype(np.int32)
    slots[[3, 11]] = -1  # padding tokens are skipped
    k = wl.normal_storage(7, (n, kvh, hd), dt)
    v = wl.normal_storage(8, (n, kvh, hd), dt)
    cache.layer(1).append(_to_dev(k, dt, gpu), _to_dev(v, dt, gpu), slots)
    cache.check()
    k1, v1 = _host_pool(cache, 1)
    ek = k0.reshape(-1, kvh, hd).copy()
    ev = v0.reshape(-1, kvh, hd).copy()
    keep = slots >= 0
    ek[slots[keep]] = k[keep]
    ev[slots[keep]] = v[keep]
    assert np.array_equal(k1.reshape(-1, kvh, hd).view(np.uint8), ek.view(np.uint8))
    assert np.array_equal(v1.reshape(-1, kvh, hd).view(np.uint8), ev.view(np.uint8))
    # layer 0 untouched
    a0, b0 = _host_pool(cache, 0)
    assert np.array_equal(a0, wl.normal_storage(100, a0.shape, dt))
    cache.close()


def test_append_out_of_range_slot_is_reported_not_written(gpu):
    cache = pagedkv.PagedKvCache(1, 8, 16, 2, 64, torch.bfloat16)
    k0, _ = _host_pool(cache, 0)
    k = torch.ones((2, 2, 64), dtype=torch.bfloat16, device=gpu)
    cache.layer(0).append(k, k, [5, 8 * 16])  # second slot is one past the pool
    with pytest.raises(pagedkv.PagedKvError) as e:
        cache.check()
    assert e.value.code == pagedkv._lib.PKV_ERR_DEVICE_DATA
    k1, _ = _host_pool(cache, 0)
    diff = np.nonzero((k1 != k0).reshape(8 * 16, -1).any(1))[0]
    assert diff.tolist() == [5]
    cache.check()  # cleared
    cache.close()


def test_kvpool_write_matches_reference_write(gpu):
    # KvPool::write(alloc, table, start_pos, k, v) -- attention.rs:57-83
    dt, bs, kvh, hd = wl.BF16, 16, 4, 128
    cache = pagedkv.PagedKvCache(1, 12, bs, kvh, hd, TD[dt])
    alloc = pagedkv.BlockAllocator(12, bs)
    t = pagedkv.BlockTable()
    alloc.ensure_capacity(t, 50)
    kp, vp = _host_pool(cache, 0)
    kp, vp = kp.copy(), vp.copy()
    k = wl.normal_storage(1, (20, kvh, hd), dt)
    v = wl.normal_storage(2, (20, kvh, hd), dt)
    cache.layer(0).write(alloc, t, 30, _to_dev(k, dt, gpu), _to_dev(v, dt, gpu))
    oracle.kv_write(kp, vp, bs, np.array(t.blocks, np.uint32), 30, k, v)
    k1, v1 = _host_pool(cache, 0)
    assert np.array_equal(k1, kp) and np.array_equal(v1, vp)
    gk, gv = cache.layer(0).gather_seq(t, 50)
    ok, ov = oracle.gather_seq(kp, vp, bs, np.array(t.blocks, np.uint32), 50)
    gkn = gk.cpu().view(torch.int16).numpy().view(np.uint16)
    gvn = gv.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(gkn, ok) and np.array_equal(gvn, ov)
    cache.close()


@pytest.mark.parametrize("dt", [wl.F16, wl.F32])
def test_gather_bit_exact(gpu, dt):
    bs, kvh, hd = 32, 2, 64
    cache = pagedkv.PagedKvCache(1, 30, bs, kvh, hd, TD[dt])
    _fill(cache, 5)
    kp, vp = _host_pool(cache, 0)
    table = wl.permutation(3, 30)[:9].astype(np.uint32)
    for length in (1, 31, 32, 33, 9 * 32):
        gk, gv = cache.layer(0).gather_seq(table.tolist(), length)
        ok, ov = oracle.gather_seq(kp, vp, bs, table, length)
        if dt == wl.F32:
            assert np.array_equal(gk.cpu().numpy(), ok) and np.array_equal(gv.cpu().numpy(), ov)
        else:
            assert np.array_equal(gk.cpu().view(torch.int16).numpy().view(np.uint16), ok)
            assert np.array_equal(gv.cpu().view(torch.int16).numpy().view(np.uint16), ov)
    cache.close()


@pytest.mark.parametrize("dt,bs", [(wl.BF16, 16), (wl.F32, 32)])
def test_gather_varlen_equals_per_sequence_gathers(gpu, dt, bs):
    # several sequences in one launch: each sequence's rows equal its own
    # gather_seq and the oracle's, bit for bit; empty sequences and a ragged
    # last block included
    kvh, hd, nb = 4, 128, 200
    cache = pagedkv.PagedKvCache(2, nb, bs, kvh, hd, TD[dt])
    _fill(cache, 8)
    kp, vp = _host_pool(cache, 1)
    lens = [0, 1, bs - 1, bs, bs + 1, 5 * bs + 3, 0, 17 * bs]
    need = [-(-n // bs) for n in lens]
    mbps = max(need)
    perm = wl.permutation(4, nb)
    tables = np.zeros((len(lens), mbps), np.int32)
    o = 0
    for b, k in enumerate(need):
        tables[b, :k] = perm[o:o + k]
        o += k
    pool = cache.layer(1)
    gk, gv, cu = pool.gather_varlen(torch.from_numpy(tables).to(gpu), lens)
    torch.cuda.synchronize()
    cache.check()
    assert cu.cpu().tolist() == [0] + list(np.cumsum(lens))
    view = (lambda t: t.cpu().numpy()) if dt == wl.F32 else (
        lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16))
    c = cu.cpu().numpy()
    for b, n in enumerate(lens):
        if n == 0:
            continue
        ok, ov = oracle.gather_seq(kp, vp, bs, tables[b].astype(np.uint32), n)
        assert np.array_equal(view(gk[c[b]:c[b + 1]]), ok)
        assert np.array_equal(view(gv[c[b]:c[b + 1]]), ov)
        sk, sv = pool.gather_seq(tables[b, :need[b]].tolist(), n)
        assert torch.equal(sk, gk[c[b]:c[b + 1]]) and torch.equal(sv, gv[c[b]:c[b + 1]])
    cache.close()


def test_gather_varlen_bad_block_reported(gpu):
    cache = pagedkv.PagedKvCache(1, 8, 16, 2, 64, torch.float16)
    _fill(cache, 3)
    tables = torch.tensor([[0, 1], [2, 99]], dtype=torch.int32, device=gpu)
    gk, gv, _ = cache.layer(0).gather_varlen(tables, [20, 20])
    torch.cuda.synchronize()
    with pytest.raises(pagedkv.PagedKvError):
        cache.check()
    assert torch.count_nonzero(gk[36:]) == 0        # rows 16..19 of sequence 1: block 99
    assert torch.count_nonzero(gv[36:]) == 0
    assert bool((gk[:36] != 0).any(dim=(1, 2)).all())   # every valid row holds data
    cache.check()                                   # the error was cleared
    cache.close()


def _all_bytes(cache):
    return np.concatenate([np.concatenate([cache.read_bytes(l, pagedkv.K), cache.read_bytes(l, pagedkv.V)])
                           for l in range(cache.n_layers)])


def test_copy_blocks_bit_exact(gpu):
    cache = pagedkv.PagedKvCache(3, 50, 16, 8, 128, torch.bfloat16)
    _fill(cache, 9)
    before = _all_bytes(cache)
    src = [3, 3, 17, 40, 0]
    dst = [10, 11, 49, 2, 1]
    cache.copy_blocks(src, dst)
    cache.check()
    after = _all_bytes(cache)
    exp = before.copy()
    oracle.copy_blocks(exp, 3, cache.block_bytes, src, dst)
    assert np.array_equal(after, exp)
    cache.close()


@pytest.mark.parametrize("case", ["prefix", "cycles", "mixed"])
def test_compact_in_place_bit_exact(gpu, case):
    N = 96
    cache = pagedkv.PagedKvCache(2, N, 16, 4, 128, torch.bfloat16)
    _fill(cache, 77)
    rng = np.random.default_rng({"prefix": 1, "cycles": 2, "mixed": 3}[case])
    if case == "prefix":  # survivors -> contiguous prefix under a random remap
        surv = np.sort(rng.choice(N, size=40, replace=False))
        dst = rng.permutation(40)
        src = surv
    elif case == "cycles":  # a pure permutation of a subset (cycles only)
        src = rng.choice(N, size=30, replace=False)
        dst = rng.permutation(src)
    else:  # chains + cycles + identity moves
        src = np.array([5, 6, 7, 20, 21, 30, 31, 32, 50, 60], np.int32)
        dst = np.array([6, 7, 8, 21, 20, 31, 32, 30, 50, 0], np.int32)
    before = _all_bytes(cache)
    cache.compact(src, dst)
    cache.check()
    after = _all_bytes(cache)
    exp = before.copy()
    oracle.compact(exp, 2, cache.block_bytes, src, dst)
    assert np.array_equal(after, exp)
    cache.close()


def test_compact_long_chains_forward_and_back(gpu):
    # 1,400 of 2,048 blocks gathered into a prefix under a random remap (long
    # chains and cycles), then moved back: both calls bit-exact against the
    # oracle, and the round trip restores every moved block (blocks of the
    # prefix that were free keep what the first call wrote there)
    N = 2048
    cache = pagedkv.PagedKvCache(2, N, 16, 2, 64, torch.float16)
    _fill(cache, 123)
    rng = np.random.default_rng(44)
    src = np.sort(rng.choice(N, size=1400, replace=False)).astype(np.int32)
    dst = rng.permutation(1400).astype(np.int32)
    before = _all_bytes(cache)
    cache.compact(src, dst)
    cache.check()
    exp = before.copy()
    oracle.compact(exp, 2, cache.block_bytes, src, dst)
    assert np.array_equal(_all_bytes(cache), exp)
    cache.compact(dst, src)
    cache.check()
    oracle.compact(exp, 2, cache.block_bytes, dst, src)
    got = _all_bytes(cache)
    assert np.array_equal(got, exp)
    bb = cache.block_bytes
    for layer_kv in range(4):                   # 2 layers x K/V slabs
        slab = slice(layer_kv * N * bb, (layer_kv + 1) * N * bb)
        g, b = got[slab].reshape(N, bb), before[slab].reshape(N, bb)
        assert np.array_equal(g[src], b[src])
    cache.close()


def test_compact_rejects_duplicates(gpu):
    cache = pagedkv.PagedKvCache(1, 8, 16, 2, 64, torch.float16)
    with pytest.raises(pagedkv.PagedKvError):
        cache.compact([1, 2], [3, 3])
    with pytest.raises(pagedkv.PagedKvError):
        cache.compact([1, 1], [3, 4])
    cache.close()


def test_fill_normal_deterministic_and_standard(gpu):
    cache = pagedkv.PagedKvCache(1, 64, 16, 8, 128, torch.bfloat16)
    cache.fill_normal(123)
    a = cache.read_bytes(0, pagedkv.K).view(np.uint16)
    cache.fill_normal(123)
    b = cache.read_bytes(0, pagedkv.K).view(np.uint16)
    assert np.array_equal(a, b)
    x = wl.widen(a, wl.BF16)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1) < 0.01
    cache.close()


def test_cfg5_geometry_churn_against_oracle(gpu):
    # BASELINE configs[4]'s block geometry (8 kv heads, head_dim 128, bf16,
    # block_size 16: 32 KiB per block and slab) on a 2-layer pool of 6,144
    # blocks (768 MiB): 60 % occupancy, copy-on-write of 300 blocks into
    # fresh ones, eviction, then the survivors gathered into a prefix under a
    # random remap (long chains and cycles, in place).  Every byte of the pool
    # equals the oracle's closed form after each step; the device
    # recomputation of the fill (pkv_pool_verify_normal) agrees with it.
    N, L, seed = 6144, 2, 505
    cache = pagedkv.PagedKvCache(L, N, 16, 8, 128, torch.bfloat16)
    cache.fill_normal(seed)
    pool = _all_bytes(cache)
    rng = np.random.default_rng(5)
    perm = rng.permutation(N).astype(np.int32)
    live = perm[: int(0.6 * N)]
    free = perm[int(0.6 * N):]
    src = rng.choice(live, size=300, replace=False).astype(np.int32)
    dst = free[:300].copy()
    cache.copy_blocks(src, dst)
    cache.check()
    oracle.copy_blocks(pool, L, cache.block_bytes, src, dst)
    assert np.array_equal(_all_bytes(cache), pool)
    origin = np.arange(N, dtype=np.int32)
    origin[dst] = origin[src]
    held = np.concatenate([live, dst])
    assert cache.verify_normal(seed, held, origin[held]) == 0
    # evict a quarter, gather the rest into [0, n) under a random remap
    surv = rng.permutation(held)[: int(0.75 * held.size)].astype(np.int32)
    remap = rng.permutation(surv.size).astype(np.int32)
    cache.compact(surv, remap)
    cache.check()
    oracle.compact(pool, L, cache.block_bytes, surv, remap)
    assert np.array_equal(_all_bytes(cache), pool)
    assert cache.verify_normal(seed, remap, origin[surv]) == 0
    cache.close()


def test_verify_normal_counts_planted_differences(gpu):
    # the check is not vacuous: a changed byte, a wrong origin and a wrong
    # seed are all counted, chunk by chunk
    cache = pagedkv.PagedKvCache(3, 40, 16, 8, 128, torch.bfloat16)
    cache.fill_normal(77)
    ids = np.arange(40, dtype=np.int32)
    assert cache.verify_normal(77, ids, ids) == 0
    slabs, block_chunks = 2 * 3, cache.block_bytes // 16
    assert cache.verify_normal(78, ids[:5], ids[:5]) == 5 * slabs * block_chunks
    assert cache.verify_normal(77, ids[:3], ids[1:4]) == 3 * slabs * block_chunks
    off = 7 * cache.block_bytes + 100           # layer 1's V, block 7: flip one byte
    byte = cache.read_bytes(1, pagedkv.V, off, 1)
    cache.write_bytes(1, pagedkv.V, byte ^ np.uint8(0xFF), offset=off)
    assert cache.verify_normal(77, ids, ids) == 1
    cache.close()


def test_copy_blocks_contract_checked_in_debug_mode(gpu, monkeypatch):
    # PKV_DEBUG: a destination that is also a source, a repeated destination
    # or an id out of range is refused before anything is copied
    cache = pagedkv.PagedKvCache(1, 16, 16, 2, 64, torch.float16)
    _fill(cache, 3)
    before = _all_bytes(cache)
    monkeypatch.setenv("PKV_DEBUG", "1")
    for src, dst, what in (([1, 2], [3, 1], b"also a source"), ([1, 2], [5, 5], b"twice"),
                           ([1, 2], [5, 16], b"out of range")):
        with pytest.raises(pagedkv.PagedKvError, match=what.decode()):
            cache.copy_blocks(src, dst)
    assert np.array_equal(_all_bytes(cache), before)
    cache.copy_blocks([1, 2], [5, 6])   # a valid call still copies
    exp = before.copy()
    oracle.copy_blocks(exp, 1, cache.block_bytes, [1, 2], [5, 6])
    assert np.array_equal(_all_bytes(cache), exp)
    cache.close()


def test_compactions_back_to_back_on_two_streams(gpu):
    # pkv_compact returns once the moves are enqueued; a second call on
    # another stream reuses the plan buffers only after the first call's
    # kernel (a device-side wait), so both plans apply in order
    N = 1024
    cache = pagedkv.PagedKvCache(2, N, 16, 4, 128, torch.bfloat16)
    _fill(cache, 8)
    exp = _all_bytes(cache)
    rng = np.random.default_rng(9)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    plans = []
    for k in range(4):
        src = rng.choice(N, size=600, replace=False).astype(np.int32)
        dst = rng.permutation(src).astype(np.int32)   # cycles only
        plans.append((src, dst))
    for k, (src, dst) in enumerate(plans):
        cache.compact(src, dst, stream=s1 if k % 2 == 0 else s2)
    torch.cuda.synchronize()
    cache.check()
    for src, dst in plans:
        oracle.compact(exp, 2, cache.block_bytes, src, dst)
    assert np.array_equal(_all_bytes(cache), exp)
    cache.close()


@pytest.mark.parametrize("dt", [wl.BF16, wl.F32])
def test_read_blocks_sums_every_word_of_the_listed_blocks(gpu, dt):
    # the read-ceiling stream: its sum equals the numpy sum of the 32-bit
    # words of blocks[i] over every layer's K and V (ids may repeat); an id
    # out of range is skipped and reported, the others still summed
    L, nb, bs, kvh, hd = 3, 300, 16, 4, 64
    cache = pagedkv.PagedKvCache(L, nb, bs, kvh, hd, {wl.BF16: torch.bfloat16,
                                                       wl.F32: torch.float32}[dt])
    cache.fill_normal(41)
    blocks = np.concatenate([wl.permutation(42, nb)[:170], [5, 5, 299, 0]]).astype(np.int32)
    want = 0
    for layer in range(L):
        for which in (pagedkv.K, pagedkv.V):
            w = cache.read_bytes(layer, which).view(np.uint32).reshape(nb, -1).astype(np.uint64)
            want += int(w[blocks].sum())
    got = cache.read_blocks(torch.from_numpy(blocks))
    torch.cuda.synchronize()
    assert int(got.cpu().numpy().view(np.uint64)[0]) == want % (1 << 64)
    cache.check()
    bad = np.concatenate([blocks, [nb, -1]]).astype(np.int32)
    got = cache.read_blocks(torch.from_numpy(bad))
    torch.cuda.synchronize()
    assert int(got.cpu().numpy().view(np.uint64)[0]) == want % (1 << 64)
    with pytest.raises(pagedkv.PagedKvError):
        cache.check()
    cache.close()
