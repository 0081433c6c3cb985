"""GPU parity of chunked-prefill attention over the paged pool against the
CPU oracle (fp64 closed form; the reference's prefill_seq op order for an
empty prior context).  Tolerance: |gpu - ref| <= 1e-3 + 2e-3 |ref|."""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}
RTOL, ATOL = 2e-3, 1e-3


def _to_dev(a, dt, device):
    a = np.ascontiguousarray(a)
    if dt == wl.F32:
        return torch.from_numpy(a).to(device)
    return torch.from_numpy(a.view(np.int16)).view(TD[dt]).to(device)


def _close(got, ref, what=""):
    got = np.asarray(got, np.float64)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} outside tolerance, max err {err.max():.3g}"


class PCase:
    """Sequences with (prior, chunk) token counts; the chunk's K/V are in the
    pool already (random pool contents for every position)."""

    def __init__(self, gpu, dt, H, KVH, hd, bs, priors, chunks, seed):
        self.dt, self.H, self.KVH, self.hd, self.bs = dt, H, KVH, hd, bs
        self.priors = np.asarray(priors, np.int64)
        self.chunks = np.asarray(chunks, np.int64)
        ctx = self.priors + self.chunks
        need = -(-ctx // bs)
        nb = int(need.sum()) + 3
        perm = wl.permutation(seed, nb)
        self.tables = np.zeros((len(ctx), max(int(need.max()), 1)), np.int32)
        o = 0
        for s in range(len(ctx)):
            self.tables[s, :need[s]] = perm[o:o + need[s]]
            o += need[s]
        self.cache = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt])
        self.kp = wl.normal_storage(seed + 1, (nb, bs, KVH, hd), dt)
        self.vp = wl.normal_storage(seed + 2, (nb, bs, KVH, hd), dt)
        self.cache.write_bytes(0, pagedkv.K, self.kp)
        self.cache.write_bytes(0, pagedkv.V, self.vp)
        self.cu = np.concatenate([[0], np.cumsum(self.chunks)]).astype(np.int32)
        T = int(self.cu[-1])
        self.q = wl.normal_storage(seed + 3, (T, H, hd), dt, scale=1 / math.sqrt(hd))
        self.ctx = ctx.astype(np.int32)
        self.scale = 1 / math.sqrt(hd)
        self.gpu = gpu

    def run(self, out_dtype=torch.float32, q=None, cu=None, ctx=None):
        q = self.q if q is None else q
        cu = self.cu if cu is None else cu
        ctx = self.ctx if ctx is None else ctx
        qlens = np.diff(cu)
        out = self.cache.layer(0).prefill_attention(
            _to_dev(q, self.dt, self.gpu), torch.from_numpy(np.ascontiguousarray(cu)).to(self.gpu),
            torch.from_numpy(np.ascontiguousarray(ctx)).to(self.gpu),
            torch.from_numpy(self.tables).to(self.gpu), max_q_len=int(max(qlens.max(), 1)),
            max_context_len=int(ctx.max()), scale=self.scale, out_dtype=out_dtype)
        torch.cuda.synchronize()
        self.cache.check()
        return out.float().cpu().numpy()

    def reference(self):
        return oracle.prefill_attention_f64(self.kp, self.vp, self.dt, self.bs,
                                            self.tables.astype(np.uint32), self.cu, self.ctx,
                                            wl.widen(self.q, self.dt), self.scale)

    def close(self):
        self.cache.close()


@pytest.mark.parametrize("dt", [wl.BF16, wl.F16, wl.F32])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("R", [1, 2, 3, 4, 5, 6, 7, 8, 16])
def test_prefill_matches_oracle(gpu, dt, hd, R):
    # any GQA ratio: rows are (token, head) pairs, so with R not dividing a
    # row block's 128 (64) rows a token's heads straddle two row blocks
    KVH = 2
    priors = [0, 0, 37, 300, 5]
    chunks = [1, 45, 16, 70, 33]
    c = PCase(gpu, dt, R * KVH, KVH, hd, 16, priors, chunks, seed=hd + 10 * R + dt)
    _close(c.run(), c.reference(), f"dt={dt} hd={hd} R={R}")
    c.close()


@pytest.mark.parametrize("bs", [16, 32, 128])
def test_prefill_block_sizes(gpu, bs):
    c = PCase(gpu, wl.BF16, 16, 2, 128, bs, [0, bs - 1, 3 * bs], [bs + 3, 20, 64], seed=bs)
    _close(c.run(), c.reference(), f"bs={bs}")
    c.close()


@pytest.mark.parametrize("bs", [1, 2, 4, 8])
@pytest.mark.parametrize("dt,hd,R", [(wl.BF16, 128, 4), (wl.F16, 64, 8), (wl.F32, 64, 2),
                                     (wl.F32, 256, 1), (wl.BF16, 64, 7)])
def test_prefill_small_block_sizes(gpu, bs, dt, hd, R):
    # block_size below 16: where it is below the keys one wave's share of a
    # tile load spans (64 / (row bytes / 16), twice that for f32 V), each
    # lane reads its key's block id; at or above it, the uniform-id kernel
    # runs.  Priors and chunks starting and ending mid-block, a prior long
    # enough for the split into parts
    KVH = 2
    priors = [0, bs - 1, 37, 300, 2100]
    chunks = [bs + 3, 1, 45, 70, 16]
    c = PCase(gpu, dt, R * KVH, KVH, hd, bs, priors, chunks, seed=bs + hd + R)
    _close(c.run(), c.reference(), f"bs={bs} dt={dt} hd={hd} R={R}")
    c.close()


def test_prefill_out_dtype_pool(gpu):
    c = PCase(gpu, wl.F16, 32, 4, 64, 16, [10, 100], [40, 90], seed=3)
    _close(c.run(out_dtype=torch.float16), c.reference(), "f16 out")
    c.close()


def test_empty_prior_is_reference_prefill_seq(gpu):
    # prior context 0 == Transformer::prefill_seq's attention (transformer.rs:139-196),
    # restated in the reference's op order (mask, GQA expand, sdpa) in f32
    H, KVH, hd, bs, N = 16, 4, 64, 16, 53
    c = PCase(gpu, wl.F32, H, KVH, hd, bs, [0], [N], seed=8)
    got = c.run()
    gk, gv = oracle.gather_seq(c.kp, c.vp, bs, c.tables[0].astype(np.uint32), N)
    ref = oracle.prefill_seq_f32(c.q.transpose(1, 0, 2), gk.transpose(1, 0, 2),
                                 gv.transpose(1, 0, 2), KVH, c.scale)
    _close(got, ref.astype(np.float64), "prefill_seq op order")
    c.close()


def test_chunked_equals_one_shot(gpu):
    # queries attend the same keys whether the prompt is split or not: each
    # row's arithmetic is identical, so the outputs are bit-identical
    H, KVH, hd, bs = 32, 8, 128, 16
    n, split = 150, 61
    c = PCase(gpu, wl.BF16, H, KVH, hd, bs, [0], [n], seed=21)
    full = c.run()
    part2 = c.run(q=c.q[split:], cu=np.array([0, n - split], np.int32), ctx=np.array([n], np.int32))
    part1 = c.run(q=c.q[:split], cu=np.array([0, split], np.int32), ctx=np.array([split], np.int32))
    assert np.array_equal(np.concatenate([part1, part2]), full)
    c.close()


def test_one_query_matches_decode(gpu):
    H, KVH, hd, bs = 32, 8, 128, 16
    priors = [0, 15, 200, 1000]
    c = PCase(gpu, wl.BF16, H, KVH, hd, bs, priors, [1, 1, 1, 1], seed=4)
    pre = c.run()
    dec = c.cache.layer(0).decode_attention(
        _to_dev(c.q, wl.BF16, gpu), torch.from_numpy(c.tables).to(gpu),
        torch.from_numpy(c.ctx).to(gpu), scale=c.scale, out_dtype=torch.float32)
    np.testing.assert_allclose(pre, dec.cpu().numpy(), rtol=1e-4, atol=5e-5)
    c.close()


def test_append_then_prefill_end_to_end(gpu):
    # the prompt's K/V stored with KvPool::write (one append), then attended
    H, KVH, hd, bs, N = 32, 4, 64, 16, 77
    dt = wl.F16
    cache = pagedkv.PagedKvCache(1, 20, bs, KVH, hd, TD[dt])
    alloc = pagedkv.BlockAllocator(20, bs)
    t = pagedkv.BlockTable()
    alloc.ensure_capacity(t, N)
    k = wl.normal_storage(1, (N, KVH, hd), dt)
    v = wl.normal_storage(2, (N, KVH, hd), dt)
    q = wl.normal_storage(3, (N, H, hd), dt, scale=1 / math.sqrt(hd))
    cache.layer(0).write(alloc, t, 0, _to_dev(k, dt, gpu), _to_dev(v, dt, gpu))
    tb = np.array([t.blocks], np.int32)
    out = cache.layer(0).prefill_attention(
        _to_dev(q, dt, gpu), torch.tensor([0, N], dtype=torch.int32, device=gpu),
        torch.tensor([N], dtype=torch.int32, device=gpu), torch.from_numpy(tb).to(gpu),
        max_q_len=N, max_context_len=N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle.prefill_seq_f32(wl.widen(q, dt).transpose(1, 0, 2), wl.widen(k, dt).transpose(1, 0, 2),
                                 wl.widen(v, dt).transpose(1, 0, 2), KVH)
    _close(out.cpu().numpy(), ref.astype(np.float64), "append + prefill")
    cache.close()


def test_tinyllama_chunked_prefill_shape(gpu):
    # BASELINE configs[1] prefill part: 256-token chunks over a prior context
    # (32 q / 4 kv heads, hd 64, f16); four sequences keep the fp64 oracle fast
    priors = wl.randint(77, 4, 0, 1024)
    c = PCase(gpu, wl.F16, 32, 4, 64, 16, priors, [256] * 4, seed=77)
    _close(c.run(out_dtype=torch.float16), c.reference(), "tinyllama prefill")
    c.close()


@pytest.mark.parametrize("dt,hd,R", [(wl.F16, 64, 8), (wl.BF16, 128, 4), (wl.BF16, 256, 2),
                                     (wl.F32, 64, 4), (wl.F32, 128, 1), (wl.BF16, 64, 2),
                                     (wl.BF16, 128, 7), (wl.F32, 256, 3), (wl.F16, 64, 12)])
def test_long_prior_split_into_parts(gpu, dt, hd, R):
    # Priors beyond the part length split a row block's keys into parts run
    # by separate workgroups and merged afterwards (launches with few row
    # blocks); parts end on the prior, so the causal diagonal stays in the
    # last part.  Priors on and next to part boundaries, one-token chunks,
    # chunks of several row blocks, and a short sequence that is not split.
    KVH = 2
    priors = [4100, 1023, 1024, 2048, 1500, 20, 2600]
    chunks = [37, 1, 130, 64, 7, 90, 1]
    c = PCase(gpu, dt, R * KVH, KVH, hd, 16, priors, chunks, seed=hd + R + dt)
    pool_bytes = c.cache.prefill_workspace_bytes(len(priors), R * KVH, max(chunks),
                                                 int(c.ctx.max()))
    assert pool_bytes > 0  # this launch is split
    out_dtype = torch.float32 if dt == wl.F32 else TD[dt]
    _close(c.run(out_dtype=out_dtype), c.reference(), f"split dt={dt} hd={hd} R={R}")
    c.close()


def test_split_workspace_reserved_up_front(gpu):
    # a reserved workspace is used as is (no growth inside the call), and a
    # launch with many row blocks is not split at all
    c = PCase(gpu, wl.BF16, 8, 2, 128, 16, [3000, 700], [50, 20], seed=3)
    need = c.cache.prefill_workspace_bytes(2, 8, 50, int(c.ctx.max()))
    c.cache.reserve_prefill(2, 8, 50, int(c.ctx.max()))
    _close(c.run(), c.reference(), "reserved split")
    assert c.cache.prefill_workspace_bytes(512, 8, 2048, 8192) == 0
    assert need > 0
    c.close()


# -- the chunk's K/V stored in the same launch (pkv_prefill_attention_append) --
def _slots(case):
    """Pool slots of every chunk token (positions prior + i), in token order."""
    out = []
    for s in range(len(case.chunks)):
        for i in range(int(case.chunks[s])):
            pos = int(case.priors[s]) + i
            out.append(int(case.tables[s, pos // case.bs]) * case.bs + pos % case.bs)
    return np.asarray(out, np.int32)


@pytest.mark.parametrize("dt,hd,R,bs", [(wl.F16, 64, 8, 16), (wl.BF16, 128, 4, 16),
                                        (wl.BF16, 64, 1, 32), (wl.F32, 128, 2, 16),
                                        (wl.BF16, 256, 2, 64), (wl.F16, 128, 8, 128),
                                        (wl.BF16, 64, 7, 16), (wl.F16, 128, 3, 32),
                                        (wl.F32, 256, 6, 16), (wl.BF16, 128, 20, 16),
                                        (wl.F16, 64, 8, 4), (wl.BF16, 128, 4, 1),
                                        (wl.F32, 64, 2, 8), (wl.BF16, 64, 3, 2)])
def test_fused_store_equals_append_then_prefill(gpu, dt, hd, R, bs):
    # same attention output and same pool bytes, bit for bit, as pkv_append
    # followed by pkv_prefill_attention; chunks that start and end mid-block,
    # an empty prior, a one-token chunk and a prior long enough to split
    KVH = 2
    priors, chunks = [0, 37, 300, 1, 4100], [45, 130, 1, 64, 20]
    a = PCase(gpu, dt, R * KVH, KVH, hd, bs, priors, chunks, seed=hd + R + bs)
    b = PCase(gpu, dt, R * KVH, KVH, hd, bs, priors, chunks, seed=hd + R + bs)
    T = int(a.cu[-1])
    kn = wl.normal_storage(hd + 91, (T, KVH, hd), dt)
    vn = wl.normal_storage(hd + 92, (T, KVH, hd), dt)
    knd, vnd = _to_dev(kn, dt, gpu), _to_dev(vn, dt, gpu)
    args = dict(max_q_len=int(max(chunks)), max_context_len=int(a.ctx.max()), scale=a.scale,
                out_dtype=torch.float32)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    qd = _to_dev(a.q, dt, gpu)
    a.cache.layer(0).append(knd, vnd, _slots(a))
    ref = a.cache.layer(0).prefill_attention(qd, dev(a.cu), dev(a.ctx), dev(a.tables), **args)
    got = b.cache.layer(0).prefill_attention(qd, dev(b.cu), dev(b.ctx), dev(b.tables), **args,
                                             k_new=knd, v_new=vnd)
    torch.cuda.synchronize()
    a.cache.check()
    b.cache.check()
    assert torch.equal(got, ref)
    for which in (pagedkv.K, pagedkv.V):
        assert np.array_equal(a.cache.read_bytes(0, which), b.cache.read_bytes(0, which))
    a.close()
    b.close()


def test_fused_store_matches_oracle(gpu):
    # the fused call against the fp64 closed form over the pool with the
    # chunk stored by the oracle's KvPool::write restatement
    dt, KVH, R, hd, bs = wl.F16, 4, 8, 64, 16
    case = PCase(gpu, dt, R * KVH, KVH, hd, bs, [900, 29, 0], [256, 256, 100], seed=61)
    T = int(case.cu[-1])
    kn = wl.normal_storage(71, (T, KVH, hd), dt)
    vn = wl.normal_storage(72, (T, KVH, hd), dt)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)
    got = case.cache.layer(0).prefill_attention(
        _to_dev(case.q, dt, gpu), dev(case.cu), dev(case.ctx), dev(case.tables),
        max_q_len=256, max_context_len=int(case.ctx.max()), scale=case.scale,
        out_dtype=torch.float32, k_new=_to_dev(kn, dt, gpu), v_new=_to_dev(vn, dt, gpu))
    torch.cuda.synchronize()
    case.cache.check()
    for s in range(3):   # the oracle's write of each sequence's chunk
        rows = slice(int(case.cu[s]), int(case.cu[s + 1]))
        oracle.kv_write(case.kp, case.vp, bs, case.tables[s].astype(np.uint32),
                        int(case.priors[s]), kn[rows], vn[rows])
    _close(got.cpu().numpy(), case.reference(), "fused store vs oracle")
    assert np.array_equal(case.cache.read_bytes(0, pagedkv.K), case.kp.view(np.uint8).reshape(-1))
    case.close()
