"""GPU parity of paged decode attention (+ fused KV append) against the CPU
oracle.  Tolerance: |gpu - ref| <= 1e-3 + 2e-3 |ref|,
fp32 accumulation; the reference output is the fp64 closed form over the
same stored (dtype-rounded) inputs."""
import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}
ND = {wl.F32: np.float32, wl.F16: np.uint16, wl.BF16: np.uint16}
RTOL, ATOL = 2e-3, 1e-3


def _to_dev(a, dt, device):
    a = np.ascontiguousarray(a)
    if dt == wl.F32:
        return torch.from_numpy(a).to(device)
    return torch.from_numpy(a.view(np.int16)).view(TD[dt]).to(device)


def _host_pool(cache, layer):
    nd = ND[pagedkv.pkv_dtype(cache.dtype)]
    shp = (cache.num_blocks, cache.block_size, cache.n_kv_head, cache.head_dim)
    return (cache.read_bytes(layer, pagedkv.K).view(nd).reshape(shp),
            cache.read_bytes(layer, pagedkv.V).view(nd).reshape(shp))


def _close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref)
    bound = ATOL + RTOL * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance; "
                           f"max err {err.max():.3g}, worst excess {(err - bound).max():.3g}")


class Case:
    """A one-layer pool with a random decode batch on it."""

    def __init__(self, gpu, dt, H, KVH, hd, bs, ctx, seed, fused=False, pool_factor=1.3):
        self.dt, self.H, self.KVH, self.hd, self.bs = dt, H, KVH, hd, bs
        B = len(ctx)
        self.ctx = np.asarray(ctx, np.int64)
        need = -(-(self.ctx + 1) // bs)
        nb = max(int(math.ceil(pool_factor * need.sum())), int(need.sum()) + 1)
        perm = wl.permutation(seed, nb)
        tables = np.zeros((B, max(int(need.max()), 1)), np.int32)
        o = 0
        for b in range(B):
            tables[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        self.tables = tables
        self.cache = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt])
        shp = (nb, bs, KVH, hd)
        self.kp = wl.normal_storage(seed + 1, shp, dt)
        self.vp = wl.normal_storage(seed + 2, shp, dt)
        self.cache.write_bytes(0, pagedkv.K, self.kp)
        self.cache.write_bytes(0, pagedkv.V, self.vp)
        self.q = wl.normal_storage(seed + 3, (B, H, hd), dt, scale=1 / math.sqrt(hd))
        self.kn = wl.normal_storage(seed + 4, (B, KVH, hd), dt)
        self.vn = wl.normal_storage(seed + 5, (B, KVH, hd), dt)
        self.scale = 1 / math.sqrt(hd)
        self.gpu = gpu
        self.fused = fused

    @property
    def context_lens(self):
        return (self.ctx + 1).astype(np.int32)

    def run(self, out_dtype=None, max_context_len=None, positions=None, check=True):
        pool = self.cache.layer(0)
        kn = _to_dev(self.kn, self.dt, self.gpu) if self.fused else None
        vn = _to_dev(self.vn, self.dt, self.gpu) if self.fused else None
        pos = None if positions is None else torch.from_numpy(
            np.asarray(positions, np.int32)).to(self.gpu)
        out = pool.decode_attention(_to_dev(self.q, self.dt, self.gpu),
                                    torch.from_numpy(self.tables).to(self.gpu),
                                    torch.from_numpy(self.context_lens).to(self.gpu),
                                    max_context_len=max_context_len or int(self.context_lens.max()),
                                    k_new=kn, v_new=vn, scale=self.scale,
                                    out_dtype=out_dtype or torch.float32, positions=pos)
        torch.cuda.synchronize()
        if check:
            self.cache.check()
        return out.float().cpu().numpy()

    def reference(self, positions=None):
        """fp64 closed form after the oracle's append of the new rows at
        seq_lens; with positions, the keys are bounded by build_mask's
        k <= positions[b] too (attention.rs:22)."""
        kp, vp = self.kp.copy(), self.vp.copy()
        lens = self.context_lens
        if positions is not None:
            pos = np.asarray(positions, np.int64)
            lens = np.where(pos < 0, 0, np.minimum(lens, pos + 1)).astype(np.int32)
        if self.fused:
            for b in range(len(self.ctx)):
                if positions is None or positions[b] >= 0:
                    oracle.kv_write(kp, vp, self.bs, self.tables[b].astype(np.uint32),
                                    int(self.ctx[b]), self.kn[b:b + 1], self.vn[b:b + 1])
        ref = oracle.paged_attention_f64(kp, vp, self.dt, self.bs, self.tables.astype(np.uint32),
                                         lens, wl.widen(self.q, self.dt), self.scale)
        return ref, kp, vp

    def close(self):
        self.cache.close()


# ---------------------------------------------------------------------------
def test_golden_fixtures(gpu):
    import glob
    import os
    files = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "decode_*.npz")))
    assert files
    for f in files:
        z = np.load(f, allow_pickle=False)
        dt = int(z["dtype"])
        kp, vp = z["k_pool"], z["v_pool"]
        nb, bs, kvh, hd = kp.shape
        H = int(z["n_head"])
        cache = pagedkv.PagedKvCache(1, nb, bs, kvh, hd, TD[dt])
        cache.write_bytes(0, pagedkv.K, kp)
        cache.write_bytes(0, pagedkv.V, vp)
        for od in ([torch.float32] + ([TD[dt]] if dt != wl.F32 else [])):
            out = cache.layer(0).decode_attention(
                _to_dev(z["q"], dt, gpu), torch.from_numpy(z["tables"]).to(gpu),
                torch.from_numpy(z["context_lens"]).to(gpu), scale=float(z["scale"]),
                out_dtype=od)
            torch.cuda.synchronize()
            _close(out.float().cpu().numpy(), z["out"], f"{os.path.basename(f)} out={od}")
        cache.check()
        cache.close()


@pytest.mark.parametrize("dt", [wl.BF16, wl.F16, wl.F32])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("R", [1, 2, 3, 4, 5, 6, 7, 8, 16])
def test_decode_matches_oracle(gpu, dt, hd, R):
    # any GQA ratio n_head / n_kv_head (repeat_kv, attention.rs:113,128-136):
    # ratios other than 1, 2, 4, 8, 16 run on the next wider kernel with the
    # extra query rows zero and unstored
    KVH = 2
    ctx = [0, 1, 14, 15, 16, 63, 64, 200, 257, 700]
    c = Case(gpu, dt, R * KVH, KVH, hd, 16, ctx, seed=hd * 10 + R + dt)
    got = c.run()
    ref, _, _ = c.reference()
    _close(got, ref, f"dt={dt} hd={hd} R={R}")
    c.close()


@pytest.mark.parametrize("dt,hd,R", [(wl.BF16, 64, 4), (wl.F16, 64, 8), (wl.BF16, 128, 4),
                                     (wl.BF16, 128, 8), (wl.F16, 256, 2), (wl.F32, 128, 4),
                                     (wl.BF16, 128, 7), (wl.F16, 64, 6), (wl.F32, 64, 5),
                                     (wl.BF16, 128, 3), (wl.BF16, 64, 16), (wl.F32, 256, 12)])
def test_many_partitions_merge(gpu, dt, hd, R):
    # a small batch with long contexts: 64-token partitions, up to ~150 per
    # sequence, so the merge covers several (m, l) lane groups and unrolled
    # partial-row loads, plus a sequence with exactly one partition
    ctx = [9500, 4096, 63, 4097, 1500]
    c = Case(gpu, dt, 2 * R, 2, hd, 16, ctx, seed=hd + R, fused=True)
    got = c.run(out_dtype=torch.float32 if dt == wl.F32 else TD[dt])
    ref, _, _ = c.reference()
    _close(got, ref, f"many partitions dt={dt} hd={hd} R={R}")
    c.close()


def _partials_bytes(pairs, parts, width, hd):
    # (m, l) of an item's heads in one 128-byte line, then the partial rows
    ml = -(-pairs * parts * 32 * 4 // 256) * 256
    return ml + pairs * parts * width * hd * 4


@pytest.mark.parametrize("dt,hd,R,bs,fused", [(wl.BF16, 128, 4, 16, True), (wl.F16, 64, 8, 32, False),
                                              (wl.BF16, 128, 4, 256, True), (wl.F32, 128, 2, 16, True),
                                              (wl.BF16, 64, 3, 64, True)])
def test_split_last_partition(gpu, dt, hd, R, bs, fused):
    # 128 sequences x 8 kv heads with contexts up to 4096: a work list of
    # 4096 items of 1024 tokens, short enough that the kernel cuts each
    # context's last 1024 tokens in two (5 partitions at most; so does the
    # 8192-item list of 256 sequences, against 4 for the 16384-item list of
    # 512); lengths on and around every 512-token edge, the rest random
    edges = [1, 2, 511, 512, 513, 1023, 1024, 1025, 1536, 1537, 2048, 2049, 2560, 2561,
             3072, 3073, 3584, 3585, 4095, 4096]
    cl = edges + [int(x) for x in wl.randint(hd + R + bs, 128 - len(edges), 1, 4096)]
    c = Case(gpu, dt, 8 * R, 8, hd, bs, [x - 1 for x in cl], seed=hd * R + bs, fused=fused)
    L = pagedkv.lib()
    w = 1 << (R - 1).bit_length()
    assert L.pkv_decode_workspace_bytes(c.cache.handle, 128, 8 * R, 4096) == \
        _partials_bytes(128 * 8, 5, w, hd)
    assert L.pkv_decode_workspace_bytes(c.cache.handle, 256, 8 * R, 4096) == \
        _partials_bytes(256 * 8, 5, w, hd)
    assert L.pkv_decode_workspace_bytes(c.cache.handle, 512, 8 * R, 4096) == \
        _partials_bytes(512 * 8, 4, w, hd)
    got = c.run()
    ref, _, _ = c.reference()
    _close(got, ref, f"split last partition dt={dt} hd={hd} R={R} bs={bs}")
    c.close()


def test_split_layout_with_a_loose_length_bound(gpu):
    # max_context_len 4096 (the plan cuts every context's last 1024 tokens
    # in two) while most contexts are far shorter: items past a sequence's
    # partitions exit, the merge reads only the partitions it has
    ctx = [0, 1, 100, 511, 512, 513, 1023, 1024, 1500, 2049] + [int(x) for x in wl.randint(91, 118, 1, 800)]
    c = Case(gpu, wl.BF16, 32, 8, 128, 16, ctx, seed=91, fused=True)
    assert pagedkv.lib().pkv_decode_workspace_bytes(c.cache.handle, 128, 32, 4096) == \
        _partials_bytes(128 * 8, 5, 4, 128)
    got = c.run(max_context_len=4096)
    ref, _, _ = c.reference()
    _close(got, ref, "split layout, loose bound")
    c.close()


@pytest.mark.parametrize("bs", [16, 32, 64, 256])
def test_decode_block_sizes(gpu, bs):
    c = Case(gpu, wl.BF16, 8, 2, 128, bs, [0, bs - 2, bs - 1, bs, 3 * bs + 5, 1000], seed=bs)
    _close(c.run(), c.reference()[0], f"bs={bs}")
    c.close()


@pytest.mark.parametrize("bs", [1, 2, 4, 8])
@pytest.mark.parametrize("dt,H,KVH,hd", [(wl.BF16, 32, 8, 128), (wl.F16, 32, 4, 64),
                                         (wl.F32, 4, 2, 64), (wl.BF16, 2, 2, 256),
                                         (wl.F16, 14, 2, 64)])
def test_decode_small_block_sizes(gpu, bs, dt, H, KVH, hd):
    # block_size below 16 (the reference's config takes any size): a K
    # sub-tile of 16 tokens spans 16 / bs blocks and each lane reads its
    # token's block id.  Contexts around block and partition edges (the
    # planner's partitions are at most 64 blocks: 64 * bs tokens), with the
    # fused append bit-exact into the pool
    ctx = [0, 1, bs - 1, bs, bs + 1, 15, 16, 17, 64 * bs - 1, 64 * bs, 64 * bs + 3, 700, 1500]
    c = Case(gpu, dt, H, KVH, hd, bs, ctx, seed=100 * bs + hd + H, fused=True)
    got = c.run()
    ref, kp, vp = c.reference()
    _close(got, ref, f"bs={bs} dt={dt} H={H}/{KVH} hd={hd}")
    k1, v1 = _host_pool(c.cache, 0)
    assert np.array_equal(k1.view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(v1.view(np.uint8), vp.view(np.uint8))
    c.close()


@pytest.mark.parametrize("dt", [wl.BF16, wl.F16, wl.F32])
def test_fused_append_writes_pool_and_attends(gpu, dt):
    c = Case(gpu, dt, 16, 4, 128, 16, [0, 5, 15, 16, 31, 255, 256, 300, 1023, 2047], seed=77 + dt,
             fused=True)
    got = c.run()
    ref, kp, vp = c.reference()
    _close(got, ref, "fused")
    k1, v1 = _host_pool(c.cache, 0)  # the append is bit-exact, nothing else changed
    assert np.array_equal(k1.view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(v1.view(np.uint8), vp.view(np.uint8))
    c.close()


def test_fused_equals_separate_append(gpu):
    # write-then-attend in one launch == KvPool::write then attention
    dt = wl.BF16
    ctx = list(wl.randint(5, 24, 0, 1500))
    c = Case(gpu, dt, 32, 8, 128, 16, ctx, seed=5, fused=True)
    fused = c.run()
    d = Case(gpu, dt, 32, 8, 128, 16, ctx, seed=5, fused=False)
    slots = d.tables[np.arange(len(ctx)), d.ctx // 16].astype(np.int64) * 16 + d.ctx % 16
    d.cache.layer(0).append(_to_dev(d.kn, dt, gpu), _to_dev(d.vn, dt, gpu), slots.astype(np.int32))
    sep = d.run()
    assert np.array_equal(fused, sep)
    c.close()
    d.close()


def test_zero_context_gives_zero_row(gpu):
    c = Case(gpu, wl.BF16, 8, 2, 128, 16, [10, 0, 3], seed=9)
    c.context_lens_override = None
    pool = c.cache.layer(0)
    cl = torch.tensor([11, 0, 4], dtype=torch.int32, device=gpu)
    out = pool.decode_attention(_to_dev(c.q, wl.BF16, gpu), torch.from_numpy(c.tables).to(gpu), cl,
                                max_context_len=11, out_dtype=torch.float32)
    o = out.cpu().numpy()
    assert np.all(o[1] == 0) and np.abs(o[0]).sum() > 0
    c.close()


def test_reference_f32_op_order(gpu):
    # f32 pool: compare with the restatement of the reference's own op order
    # (write -> gather -> pad -> build_mask -> sdpa, transformer.rs:271-292)
    B, H, KVH, hd, bs = 6, 16, 4, 64, 16
    ctx = [3, 40, 17, 100, 0, 64]
    c = Case(gpu, wl.F32, H, KVH, hd, bs, ctx, seed=3, fused=True)
    got = c.run()
    kp, vp = c.kp.copy(), c.vp.copy()
    ref = oracle.decode_step_f32(kp, vp, bs, c.tables.astype(np.uint32), c.ctx, c.ctx,
                                 c.q, c.kn, c.vn, c.scale)
    _close(got, ref.astype(np.float64), "reference op order")
    c.close()


def test_out_of_range_block_id_reported(gpu):
    c = Case(gpu, wl.BF16, 8, 2, 128, 16, [40, 20], seed=4)
    c.tables[0, 1] = c.cache.num_blocks + 7
    c.run_ok = False
    with pytest.raises(pagedkv.PagedKvError):
        c.run()
    c.close()


@pytest.mark.parametrize("B,max_cl,rc_name,msg", [
    (1024, (1 << 31) - 1, "PKV_ERR_INVALID", b"2^30"),
    (4096, 1 << 30, "PKV_ERR_UNSUPPORTED", b"2^26")])
def test_refuses_lengths_beyond_the_planners_range(gpu, B, max_cl, rc_name, msg):
    # max_context_len above 2^30, and B x 8 kv heads x 2^20 partitions of
    # 1024 tokens (more 64-lane waves than a grid's 32-bit count): both
    # refused by the argument checks, before anything is allocated or
    # enqueued (were the second not, its partials' workspace of several TB
    # would fail to allocate before any launch)
    cache = pagedkv.PagedKvCache(1, 64, 16, 8, 128, torch.bfloat16)
    H, hd = 32, 128
    q = torch.zeros((B, H, hd), dtype=torch.bfloat16, device=gpu)
    out = torch.zeros((B, H * hd), dtype=torch.float32, device=gpu)
    tables = torch.zeros((B, 1), dtype=torch.int32, device=gpu)
    cl = torch.ones(B, dtype=torch.int32, device=gpu)
    L = pagedkv.lib()
    rc = L.pkv_decode_attention(cache.handle, 0, q.data_ptr(), out.data_ptr(), pagedkv.F32,
                                tables.data_ptr(), 1, cl.data_ptr(), max_cl, B, H,
                                ctypes.c_float(0.1), None, None, None)
    assert rc == getattr(pagedkv._lib, rc_name)
    assert msg in L.pkv_last_error(cache.handle)
    assert L.pkv_decode_workspace_bytes(cache.handle, B, H, (1 << 31) - 1) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
    cache.close()


@pytest.mark.parametrize("cfg,B,lo,hi", [(wl.CFG1, 8, 128, 1024), (wl.CFG2, 56, 256, 2048),
                                         (wl.CFG3, 32, 512, 4096), (wl.CFG4, 6, 2048, 8192)])
def test_config_shapes(gpu, cfg, B, lo, hi):
    ctx = wl.randint(cfg.n_layers * 7 + B, B, lo, hi)
    c = Case(gpu, cfg.dtype, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.block_size, ctx,
             seed=cfg.n_head + B, fused=True)
    got = c.run(out_dtype=TD[cfg.dtype])
    ref, _, _ = c.reference()
    _close(got, ref, cfg.name)
    c.close()


def test_batched_equals_solo(gpu):
    # the reference's batched_matches_solo (paged_batching.rs:40-51) at the
    # attention level: a row's result does not depend on its batch mates
    ctx = list(wl.randint(12, 10, 1, 3000))
    c = Case(gpu, wl.BF16, 32, 8, 128, 16, ctx, seed=12)
    full = c.run()
    pool = c.cache.layer(0)
    for b in (0, 3, 9):
        out = pool.decode_attention(_to_dev(c.q[b:b + 1], wl.BF16, gpu),
                                    torch.from_numpy(c.tables[b:b + 1]).to(gpu),
                                    torch.from_numpy(c.context_lens[b:b + 1]).to(gpu),
                                    max_context_len=int(c.context_lens.max()), scale=c.scale,
                                    out_dtype=torch.float32)
        assert np.array_equal(out.cpu().numpy()[0], full[b])  # identical, as the reference demands
    c.close()


def test_workspace_grows_under_queued_work(gpu):
    # Calls queued back to back without synchronising, each needing a larger
    # workspace than the last: the growth replaces the buffer while earlier
    # launches may still read the old one, which must stay valid until the
    # reserve call frees it.  Every call's rows match the oracle.
    ctx = list(wl.randint(41, 24, 200, 6000))
    c = Case(gpu, wl.F16, 32, 8, 64, 16, ctx, seed=41)
    ref = c.reference()[0]
    pool = c.cache.layer(0)
    q = _to_dev(c.q, c.dt, gpu)
    tables = torch.from_numpy(c.tables).to(gpu)
    lens = torch.from_numpy(c.context_lens).to(gpu)
    outs = []
    for n, mcl in ((2, 1000), (8, 3000), (24, int(c.context_lens.max()))):
        sub = torch.from_numpy(np.minimum(c.context_lens[:n], mcl)).to(gpu)
        outs.append((n, mcl, pool.decode_attention(q[:n], tables[:n], sub, max_context_len=mcl,
                                                   scale=c.scale, out_dtype=torch.float32)))
    c.cache.reserve_decode(24, 32, 8192)  # frees the replaced buffers after a device sync
    torch.cuda.synchronize()
    c.cache.check()
    for n, mcl, out in outs:
        if mcl >= int(c.context_lens[:n].max()):
            _close(out.cpu().numpy(), ref[:n], f"batch {n}")
        else:  # rows clamped to mcl keys: compare with the oracle over those keys
            kp, vp = c.kp, c.vp
            r = oracle.paged_attention_f64(kp, vp, c.dt, c.bs, c.tables[:n].astype(np.uint32),
                                           np.minimum(c.context_lens[:n], mcl).astype(np.int32),
                                           wl.widen(c.q[:n], c.dt), c.scale)
            _close(out.cpu().numpy(), r, f"batch {n} clamped to {mcl}")
    c.close()


def test_profile_hook_times_main_kernel(gpu):
    c = Case(gpu, wl.BF16, 32, 8, 128, 16, list(wl.randint(3, 16, 100, 2000)), seed=31)
    c.cache.profile(True)
    for _ in range(3):
        c.run()
    ms, n = c.cache.profile_read()
    assert n == 3 and ms > 0
    c.cache.profile(False)
    c.run()
    assert c.cache.profile_read() == (0.0, 0)
    c.close()


@pytest.mark.parametrize("dt,hd,R", [(wl.BF16, 128, 20), (wl.F32, 64, 33), (wl.F16, 64, 17),
                                     (wl.BF16, 256, 32)])
def test_ratio_above_sixteen_in_head_slices(gpu, dt, hd, R):
    # ratios above 16 run as launches over slices of at most 16 query heads of
    # every group (each reads the group's K/V); the first slice stores the new
    # token and every slice attends to it
    KVH = 2
    c = Case(gpu, dt, R * KVH, KVH, hd, 16, [0, 3, 700, 2100, 64], seed=hd + R, fused=True)
    got = c.run()
    ref, kp, vp = c.reference()
    _close(got, ref, f"R={R} dt={dt} hd={hd}")
    k1, v1 = _host_pool(c.cache, 0)
    assert np.array_equal(k1.view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(v1.view(np.uint8), vp.view(np.uint8))
    c.close()


@pytest.mark.parametrize("R", [3, 6, 7, 12])
def test_fused_equals_separate_append_any_ratio(gpu, R):
    # the fused new token (taken from the launch's own copy of the stored
    # row) gives the same bits as KvPool::write followed by attention
    dt, KVH, hd = wl.BF16, 2, 128
    ctx = list(wl.randint(50 + R, 9, 0, 2500))
    c = Case(gpu, dt, R * KVH, KVH, hd, 16, ctx, seed=50 + R, fused=True)
    fused = c.run()
    d = Case(gpu, dt, R * KVH, KVH, hd, 16, ctx, seed=50 + R, fused=False)
    slots = d.tables[np.arange(len(ctx)), d.ctx // 16].astype(np.int64) * 16 + d.ctx % 16
    d.cache.layer(0).append(_to_dev(d.kn, dt, gpu), _to_dev(d.vn, dt, gpu), slots.astype(np.int32))
    assert np.array_equal(fused, d.run())
    k1, _ = _host_pool(c.cache, 0)
    k2, _ = _host_pool(d.cache, 0)
    assert np.array_equal(k1, k2)
    c.close()
    d.close()


def test_positions_bound_of_build_mask(gpu):
    # build_mask's second bound k <= positions[b] (attention.rs:22) with
    # positions different from seq_lens: the reference's decode-step order
    # (write at seq_lens, gather seq_lens + 1, mask with both bounds, sdpa)
    # equals pkv_append at seq_lens plus attention over
    # min(seq_lens + 1, positions + 1) keys
    B, H, KVH, hd, bs = 5, 14, 2, 64, 16
    ctx = [3, 40, 17, 100, 64]
    pos = [1, 40, 5, 99, 0]   # <= seq_lens
    c = Case(gpu, wl.F32, H, KVH, hd, bs, ctx, seed=19)
    kp, vp = c.kp.copy(), c.vp.copy()
    ref = oracle.decode_step_f32(kp, vp, bs, c.tables.astype(np.uint32), c.ctx, pos, c.q, c.kn,
                                 c.vn, c.scale)
    slots = c.tables[np.arange(B), c.ctx // bs].astype(np.int64) * bs + c.ctx % bs
    pool = c.cache.layer(0)
    pool.append(_to_dev(c.kn, wl.F32, gpu), _to_dev(c.vn, wl.F32, gpu), slots.astype(np.int32))
    cl = np.minimum(c.ctx + 1, np.asarray(pos) + 1).astype(np.int32)
    got = pool.decode_attention(_to_dev(c.q, wl.F32, gpu), torch.from_numpy(c.tables).to(gpu),
                                torch.from_numpy(cl).to(gpu), max_context_len=int(c.ctx.max()) + 1,
                                scale=c.scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    c.cache.check()
    _close(got.cpu().numpy(), ref.astype(np.float64), "positions bound")
    # and the bound matters: attention over seq_lens + 1 keys differs
    full = oracle.paged_attention_f64(kp, vp, wl.F32, bs, c.tables.astype(np.uint32),
                                      (c.ctx + 1).astype(np.int32), c.q, c.scale)
    assert np.abs(full - ref).max() > 1e-2
    c.close()


def _positions(ctx, seed):
    # per row: the reference's own position (== seq_len), one below it, a
    # random earlier one, 0, or one past the context (no effect)
    r = np.random.default_rng(seed)
    pos = []
    for i, c in enumerate(ctx):
        k = i % 5
        pos.append([c, max(c - 1, 0), int(r.integers(0, c + 1)), 0, c + int(r.integers(1, 5000))][k])
    return pos


@pytest.mark.parametrize("dt,H,KVH,hd,bs", [(wl.BF16, 32, 8, 128, 16), (wl.F16, 32, 4, 64, 16),
                                           (wl.F32, 16, 8, 64, 16), (wl.BF16, 32, 8, 128, 4),
                                           (wl.BF16, 28, 4, 64, 32)])
def test_decode_positions_bound(gpu, dt, H, KVH, hd, bs):
    # pkv_decode_attention_positions: both build_mask bounds with the new
    # row stored at seq_lens (attended only when positions >= seq_lens), on
    # contexts that span several partitions (the merge uses the bounded
    # lengths too)
    ctx = [0, 1, 15, 16, 17, 40, 700, 1023, 1024, 1025, 2100, 3000] + \
        [int(x) for x in wl.randint(hd + bs, 28, 1, 3000)]
    pos = _positions(ctx, hd + bs)
    c = Case(gpu, dt, H, KVH, hd, bs, ctx, seed=hd + H + bs, fused=True)
    got = c.run(max_context_len=3001, positions=pos)
    ref, kp, vp = c.reference(pos)
    _close(got, ref, f"positions bound dt={dt} hd={hd} bs={bs}")
    k1, v1 = _host_pool(c.cache, 0)
    assert np.array_equal(k1, kp) and np.array_equal(v1, vp)
    c.close()


def test_decode_positions_bound_work_list(gpu):
    # 200 sequences x 4 kv heads x 3 partitions: a work-list launch (items
    # ordered from the bounded lengths, the last 1024 tokens split in two)
    ctx = [0, 1023, 1024, 2047, 2048, 2999] + [int(x) for x in wl.randint(7, 194, 1, 3000)]
    pos = _positions(ctx, 7)
    c = Case(gpu, wl.BF16, 16, 4, 64, 16, ctx, seed=7, fused=True)
    got = c.run(max_context_len=3001, positions=pos)
    ref, kp, vp = c.reference(pos)
    _close(got, ref, "positions bound, work list")
    k1, v1 = _host_pool(c.cache, 0)
    assert np.array_equal(k1, kp) and np.array_equal(v1, vp)
    c.close()


def test_decode_positions_equal_seq_lens_is_plain_decode(gpu):
    # positions == seq_lens (the reference's engine, engine.rs:130-133):
    # bit for bit pkv_decode_attention
    ctx = [3, 500, 1500, 2500, 77]
    a = Case(gpu, wl.BF16, 32, 8, 128, 16, ctx, seed=3, fused=True)
    b = Case(gpu, wl.BF16, 32, 8, 128, 16, ctx, seed=3, fused=True)
    x = a.run()
    y = b.run(positions=ctx)
    assert np.array_equal(x, y)
    ka, va = _host_pool(a.cache, 0)
    kb, vb = _host_pool(b.cache, 0)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.close()
    b.close()


def test_decode_negative_position_reported(gpu):
    ctx = [30, 40, 50]
    pos = [30, -1, 20]
    c = Case(gpu, wl.BF16, 32, 8, 128, 16, ctx, seed=5, fused=True)
    got = c.run(positions=pos, check=False)
    with pytest.raises(pagedkv.PagedKvError):
        c.cache.check()
    ref, kp, vp = c.reference(pos)
    assert np.all(got[1] == 0.0)
    _close(got, ref, "negative position")
    k1, v1 = _host_pool(c.cache, 0)
    assert np.array_equal(k1, kp) and np.array_equal(v1, vp)  # row 1 stored nothing
    c.close()


def test_decode_positions_refuses_null(gpu):
    c = Case(gpu, wl.BF16, 32, 8, 128, 16, [10, 20], seed=1)
    L = pagedkv.lib()
    q = _to_dev(c.q, c.dt, gpu)
    out = torch.empty((2, 32 * 128), dtype=torch.float32, device=gpu)
    t = torch.from_numpy(c.tables).to(gpu)
    cl = torch.from_numpy(c.context_lens).to(gpu)
    rc = L.pkv_decode_attention_positions(c.cache.handle, 0, q.data_ptr(), out.data_ptr(),
                                          pagedkv.F32, t.data_ptr(), t.shape[1], cl.data_ptr(),
                                          None, 64, 2, 32, c.scale, None, None, None)
    assert rc == pagedkv._lib.PKV_ERR_INVALID
    c.close()
