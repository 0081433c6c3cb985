"""GPU parity of the rotary embedding (rope.rs, transformer.rs:252-269):
pkv_rope_apply and pkv_decode_attention_rope against the CPU oracle.  The
rotation is f32 with every product rounded, so the rotated rows are bit-exact;
the attention then follows pkv_decode_attention (tolerance 1e-3 + 2e-3 |ref|
against the fp64 closed form)."""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}


def _dev(a, dt, device):
    a = np.ascontiguousarray(a)
    if dt == wl.F32:
        return torch.from_numpy(a.astype(np.float32)).to(device)
    return torch.from_numpy(a.view(np.int16)).view(TD[dt]).to(device)


def _bits(t):
    t = t.contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("in_dt,out_dt", [(wl.F32, wl.F32), (wl.F32, wl.BF16), (wl.F32, wl.F16),
                                          (wl.BF16, wl.BF16), (wl.F16, wl.F32)])
@pytest.mark.parametrize("dim", [64, 128, 256])
def test_rope_apply_bit_exact(gpu, in_dt, out_dt, dim):
    rope = pagedkv.Rope(dim, 500000.0, 4096)
    c, s = oracle.rope_table(dim, 500000.0, 4096)
    n, h = 37, 5
    x = wl.normal_storage(dim + in_dt, (n, h, dim), in_dt)
    pos = wl.randint(dim, n, 0, 4095).astype(np.int32)
    pos[0] = 0
    got = rope.apply(_dev(x, in_dt, gpu), torch.from_numpy(pos).to(gpu), out_dtype=TD[out_dt])
    torch.cuda.synchronize()
    rope.check()
    ref = wl.to_storage(oracle.rope_apply(wl.widen(x, in_dt), c, s, pos), out_dt)
    assert np.array_equal(_bits(got), ref.view(np.uint32 if out_dt == wl.F32 else np.uint16))
    rope.close()


def test_rope_apply_in_place_and_bad_position(gpu):
    rope = pagedkv.Rope(128, 10000.0, 100)
    x = torch.randn((4, 2, 128), device=gpu)
    keep = x.clone()
    pos = torch.tensor([1, 100, -1, 3], dtype=torch.int32, device=gpu)
    rope.apply(x, pos, out=x)
    torch.cuda.synchronize()
    with pytest.raises(pagedkv.PagedKvError):
        rope.check()
    assert torch.equal(x[1], keep[1]) and torch.equal(x[2], keep[2])  # not written
    assert not torch.equal(x[0], keep[0])
    rope.check()  # the error was cleared
    rope.close()


class RopeCase:
    def __init__(self, gpu, dt, in_dt, H, KVH, hd, ctx, seed, positions=None, max_seq=9000):
        self.gpu, self.dt, self.in_dt, self.H, self.KVH, self.hd = gpu, dt, in_dt, H, KVH, hd
        self.ctx = np.asarray(ctx, np.int64)
        B, bs = len(ctx), 16
        need = -(-(self.ctx + 1) // bs)
        nb = int(need.sum()) + 7
        perm = wl.permutation(seed, nb)
        self.tables = np.zeros((B, int(need.max())), np.int32)
        o = 0
        for b in range(B):
            self.tables[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        self.nb, self.bs = nb, bs
        shp = (nb, bs, KVH, hd)
        self.kp = wl.normal_storage(seed + 1, shp, dt)
        self.vp = wl.normal_storage(seed + 2, shp, dt)
        self.q = wl.normal_storage(seed + 3, (B, H, hd), in_dt)   # before rotation
        self.kn = wl.normal_storage(seed + 4, (B, KVH, hd), in_dt)
        self.vn = wl.normal_storage(seed + 5, (B, KVH, hd), in_dt)
        self.pos = (self.ctx.astype(np.int32) if positions is None
                    else np.asarray(positions, np.int32))
        self.explicit = positions is not None
        self.max_seq = max_seq
        self.cos, self.sin = oracle.rope_table(hd, 500000.0, max_seq)

    def cache(self):
        c = pagedkv.PagedKvCache(1, self.nb, self.bs, self.KVH, self.hd, TD[self.dt])
        c.write_bytes(0, pagedkv.K, self.kp)
        c.write_bytes(0, pagedkv.V, self.vp)
        return c

    def rotated(self):
        """The oracle's rotated q, k_new (pool dtype storage) and v_new."""
        q = wl.to_storage(oracle.rope_apply(wl.widen(self.q, self.in_dt), self.cos, self.sin,
                                            self.pos), self.dt)
        k = wl.to_storage(oracle.rope_apply(wl.widen(self.kn, self.in_dt), self.cos, self.sin,
                                            self.pos), self.dt)
        v = wl.to_storage(wl.widen(self.vn, self.in_dt), self.dt)
        return q, k, v

    def run_fused(self, rope):
        c = self.cache()
        g = self.gpu
        out = c.layer(0).decode_attention(
            _dev(self.q, self.in_dt, g), torch.from_numpy(self.tables).to(g),
            torch.from_numpy((self.ctx + 1).astype(np.int32)).to(g),
            k_new=_dev(self.kn, self.in_dt, g), v_new=_dev(self.vn, self.in_dt, g),
            rope=rope, positions=torch.from_numpy(self.pos).to(g) if self.explicit else None,
            out_dtype=torch.float32)
        torch.cuda.synchronize()
        c.check()
        return c, out.cpu().numpy()


@pytest.mark.parametrize("dt,in_dt,hd,R", [(wl.BF16, wl.F32, 128, 4), (wl.BF16, wl.BF16, 128, 4),
                                           (wl.F16, wl.F32, 64, 8), (wl.F32, wl.F32, 128, 2),
                                           (wl.BF16, wl.F32, 256, 2), (wl.F16, wl.F16, 64, 4)])
def test_decode_attention_rope_matches_oracle(gpu, dt, in_dt, hd, R):
    KVH = 2
    ctx = [0, 1, 15, 16, 300, 1100, 2500]
    case = RopeCase(gpu, dt, in_dt, R * KVH, KVH, hd, ctx, seed=hd + R + dt)
    rope = pagedkv.Rope(hd, 500000.0, case.max_seq)
    cache, got = case.run_fused(rope)
    q, k, v = case.rotated()
    # the appended rows are the oracle's rotated k and the converted v, bit for bit
    kp, vp = case.kp.copy(), case.vp.copy()
    for b in range(len(ctx)):
        oracle.kv_write(kp, vp, case.bs, case.tables[b].astype(np.uint32), int(case.ctx[b]),
                        k[b:b + 1], v[b:b + 1])
    nd = np.float32 if dt == wl.F32 else np.uint16
    k1 = cache.read_bytes(0, pagedkv.K).view(nd).reshape(kp.shape)
    v1 = cache.read_bytes(0, pagedkv.V).view(nd).reshape(vp.shape)
    assert np.array_equal(k1.view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(v1.view(np.uint8), vp.view(np.uint8))
    # attention: the fp64 closed form over the rotated q and the updated pool
    ref = oracle.paged_attention_f64(kp, vp, dt, case.bs, case.tables.astype(np.uint32),
                                     (case.ctx + 1).astype(np.int32), wl.widen(q, dt),
                                     1 / math.sqrt(hd))
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-3 + 2e-3 * np.abs(ref)), err.max()
    # and the plain kernel fed the oracle's rotated rows gives the same output
    c2 = case.cache()
    out2 = c2.layer(0).decode_attention(
        _dev(q, dt, gpu), torch.from_numpy(case.tables).to(gpu),
        torch.from_numpy((case.ctx + 1).astype(np.int32)).to(gpu), k_new=_dev(k, dt, gpu),
        v_new=_dev(v, dt, gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(out2.cpu().numpy(), got)
    cache.close()
    c2.close()
    rope.close()


def test_decode_attention_rope_explicit_positions(gpu):
    # positions need not equal seq_lens (decode_step takes them separately)
    ctx = [40, 700, 1200]
    case = RopeCase(gpu, wl.BF16, wl.F32, 16, 4, 128, ctx, seed=21, positions=[5, 8000, 1199])
    rope = pagedkv.Rope(128, 500000.0, case.max_seq)
    cache, got = case.run_fused(rope)
    q, k, v = case.rotated()
    kp, vp = case.kp.copy(), case.vp.copy()
    for b in range(len(ctx)):
        oracle.kv_write(kp, vp, case.bs, case.tables[b].astype(np.uint32), int(case.ctx[b]),
                        k[b:b + 1], v[b:b + 1])
    ref = oracle.paged_attention_f64(kp, vp, wl.BF16, case.bs, case.tables.astype(np.uint32),
                                     (case.ctx + 1).astype(np.int32), wl.widen(q, wl.BF16),
                                     1 / math.sqrt(128))
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-3 + 2e-3 * np.abs(ref)), err.max()
    cache.close()
    rope.close()


def test_decode_attention_rope_bad_position_reported(gpu):
    case = RopeCase(gpu, wl.BF16, wl.F32, 8, 2, 128, [30, 40], seed=5, positions=[3, 50],
                    max_seq=50)
    rope = pagedkv.Rope(128, 500000.0, 50)
    with pytest.raises(pagedkv.PagedKvError):
        case.run_fused(rope)
    rope.close()


def test_decode_attention_rope_rejects_mismatch(gpu):
    rope = pagedkv.Rope(64, 10000.0, 64)
    c = pagedkv.PagedKvCache(1, 8, 16, 2, 128, torch.bfloat16)
    q = torch.zeros((1, 4, 128), dtype=torch.float32, device=gpu)
    with pytest.raises(pagedkv.PagedKvError):   # rope_dim != head_dim
        c.layer(0).decode_attention(q, torch.zeros((1, 1), dtype=torch.int32, device=gpu),
                                    torch.ones(1, dtype=torch.int32, device=gpu), rope=rope)
    c.close()
    rope.close()
