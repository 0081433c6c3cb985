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
    def __init__(self, gpu, dt, in_dt, H, KVH, hd, ctx, seed, positions=None, max_seq=9000,
                 bs=16):
        self.gpu, self.dt, self.in_dt, self.H, self.KVH, self.hd = gpu, dt, in_dt, H, KVH, hd
        self.ctx = np.asarray(ctx, np.int64)
        B = len(ctx)
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
                                           (wl.BF16, wl.F32, 256, 2), (wl.F16, wl.F16, 64, 4),
                                           (wl.BF16, wl.F32, 128, 7), (wl.F32, wl.F32, 64, 7),
                                           (wl.BF16, wl.F32, 128, 5), (wl.BF16, wl.F32, 64, 20)])
def test_decode_attention_rope_matches_oracle(gpu, dt, in_dt, hd, R):
    _rope_decode_check(gpu, dt, in_dt, hd, R, 2, [0, 1, 15, 16, 300, 1100, 2500], hd + R + dt)


def test_decode_attention_rope_split_last_partition(gpu):
    # 300 sequences x 2 kv heads with max_context_len 4096 (2,400 work items
    # of 1024 tokens): the plan cuts each context's last 1024 tokens in two,
    # with RoPE applied in the same launch; most contexts are short so the
    # host-side pool stays small
    ctx = [0, 511, 512, 1023, 1024, 1535, 1536, 4095] + [int(x) for x in wl.randint(33, 292, 1, 40)]
    _rope_decode_check(gpu, wl.BF16, wl.F32, 128, 4, 2, ctx, 33)


@pytest.mark.parametrize("bs", [1, 2, 4, 8])
@pytest.mark.parametrize("dt,in_dt,hd,R", [(wl.BF16, wl.F32, 128, 4), (wl.F16, wl.F16, 64, 8),
                                           (wl.F32, wl.F32, 64, 2)])
def test_decode_attention_rope_small_block_sizes(gpu, dt, in_dt, hd, R, bs):
    # blocks of fewer than 16 tokens: each lane of a 16-token sub-tile looks
    # up its own block id, and the appended rotated row lands in block
    # ctx // bs at slot ctx % bs
    _rope_decode_check(gpu, dt, in_dt, hd, R, 2, [0, 1, bs - 1, bs, 15, 16, 300, 64 * bs + 3],
                       hd + R + bs, bs=bs)


def _rope_decode_check(gpu, dt, in_dt, hd, R, KVH, ctx, seed, bs=16):
    case = RopeCase(gpu, dt, in_dt, R * KVH, KVH, hd, ctx, seed=seed, bs=bs)
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
    # up to f32 summation order (the two kernels tile the context
    # differently): within a twentieth of the tolerance against the oracle
    c2 = case.cache()
    out2 = c2.layer(0).decode_attention(
        _dev(q, dt, gpu), torch.from_numpy(case.tables).to(gpu),
        torch.from_numpy((case.ctx + 1).astype(np.int32)).to(gpu), k_new=_dev(k, dt, gpu),
        v_new=_dev(v, dt, gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    diff = np.abs(out2.cpu().numpy().astype(np.float64) - got)
    assert np.all(diff <= 5e-5 + 1e-4 * np.abs(ref)), diff.max()
    cache.close()
    c2.close()
    rope.close()


def test_decode_attention_rope_explicit_positions(gpu):
    # positions need not equal seq_lens (decode_step takes them separately):
    # they rotate q and k and bound the keys attended (build_mask's
    # k <= positions[b], attention.rs:22); the new row is stored at seq_lens
    ctx = [40, 700, 1200]
    case = RopeCase(gpu, wl.BF16, wl.F32, 16, 4, 128, ctx, seed=21, positions=[5, 8000, 1199])
    rope = pagedkv.Rope(128, 500000.0, case.max_seq)
    cache, got = case.run_fused(rope)
    q, k, v = case.rotated()
    kp, vp = case.kp.copy(), case.vp.copy()
    for b in range(len(ctx)):
        oracle.kv_write(kp, vp, case.bs, case.tables[b].astype(np.uint32), int(case.ctx[b]),
                        k[b:b + 1], v[b:b + 1])
    lens = np.minimum(case.ctx + 1, case.pos.astype(np.int64) + 1).astype(np.int32)  # [6, 701, 1200]
    ref = oracle.paged_attention_f64(kp, vp, wl.BF16, case.bs, case.tables.astype(np.uint32),
                                     lens, wl.widen(q, wl.BF16), 1 / math.sqrt(128))
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-3 + 2e-3 * np.abs(ref)), err.max()
    k1 = cache.read_bytes(0, pagedkv.K).view(np.uint16).reshape(kp.shape)
    v1 = cache.read_bytes(0, pagedkv.V).view(np.uint16).reshape(vp.shape)
    assert np.array_equal(k1, kp) and np.array_equal(v1, vp)
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


# -- prefill glue: pkv_append_rope (transformer.rs:160-174) --------------------
def _slot_case(seed, n, nb, bs):
    slots = wl.permutation(seed, nb * bs)[:n].astype(np.int32)
    slots[::7] = -1                                        # padding tokens
    return slots


@pytest.mark.parametrize("dt,in_dt,hd,KVH,R", [(wl.BF16, wl.F32, 128, 8, 4),
                                               (wl.BF16, wl.BF16, 128, 8, 4),
                                               (wl.F16, wl.F32, 64, 4, 8),
                                               (wl.F16, wl.F16, 64, 2, 1),
                                               (wl.F32, wl.F32, 256, 2, 2),
                                               (wl.BF16, wl.F32, 256, 1, 8),
                                               (wl.F32, wl.F32, 64, 2, 7),
                                               (wl.BF16, wl.F32, 64, 2, 7)])
def test_append_rope_bit_exact(gpu, dt, in_dt, hd, KVH, R):
    n, nb, bs, H, max_seq = 203, 40, 16, KVH * R, 3000
    seed = hd + KVH + R + 3 * dt + in_dt
    kp0 = wl.normal_storage(seed + 1, (nb, bs, KVH, hd), dt)
    vp0 = wl.normal_storage(seed + 2, (nb, bs, KVH, hd), dt)
    k = wl.normal_storage(seed + 3, (n, KVH, hd), in_dt)
    v = wl.normal_storage(seed + 4, (n, KVH, hd), in_dt)
    q = wl.normal_storage(seed + 5, (n, H, hd), in_dt)
    slots = _slot_case(seed, n, nb, bs)
    pos = wl.randint(seed + 6, n, 0, max_seq - 1).astype(np.int32)
    pos[:3] = [0, max_seq - 1, 1]
    c = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt])
    c.write_bytes(0, pagedkv.K, kp0)
    c.write_bytes(0, pagedkv.V, vp0)
    rope = pagedkv.Rope(hd, 500000.0, max_seq)
    qo = c.layer(0).append_rope(rope, _dev(k, in_dt, gpu), _dev(v, in_dt, gpu),
                                torch.from_numpy(slots).to(gpu), torch.from_numpy(pos).to(gpu),
                                q=_dev(q, in_dt, gpu))
    torch.cuda.synchronize()
    c.check()
    cs, sn = oracle.rope_table(hd, 500000.0, max_seq)
    kr = wl.to_storage(oracle.rope_apply(wl.widen(k, in_dt), cs, sn, pos), dt)
    vr = wl.to_storage(wl.widen(v, in_dt), dt)
    qr = wl.to_storage(oracle.rope_apply(wl.widen(q, in_dt), cs, sn, pos), dt)
    kp, vp = kp0.copy().reshape(nb * bs, KVH, hd), vp0.copy().reshape(nb * bs, KVH, hd)
    live = slots >= 0
    kp[slots[live]] = kr[live]
    vp[slots[live]] = vr[live]
    assert np.array_equal(c.read_bytes(0, pagedkv.K), kp.view(np.uint8).reshape(-1))
    assert np.array_equal(c.read_bytes(0, pagedkv.V), vp.view(np.uint8).reshape(-1))
    nd = np.uint32 if dt == wl.F32 else np.uint16
    assert np.array_equal(_bits(qo), qr.view(nd))
    c.close()
    rope.close()


def test_append_rope_equals_separate_passes(gpu):
    # one launch == rope_apply(k) + pkv_append + rope_apply(q), byte for byte
    n, nb, bs, KVH, hd, H = 96, 12, 16, 4, 128, 32
    k = torch.randn((n, KVH, hd), device=gpu)
    v = torch.randn((n, KVH, hd), device=gpu)
    q = torch.randn((n, H, hd), device=gpu)
    slots = torch.from_numpy(_slot_case(9, n, nb, bs)).to(gpu)
    pos = torch.arange(500, 500 + n, dtype=torch.int32, device=gpu)
    rope = pagedkv.Rope(hd, 500000.0, 1024)
    a = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, torch.bfloat16)
    b = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, torch.bfloat16)
    qa = a.layer(0).append_rope(rope, k, v, slots, pos, q=q)
    kb = rope.apply(k, pos, out_dtype=torch.bfloat16)
    b.layer(0).append(kb, v.to(torch.bfloat16), slots)
    qb = rope.apply(q, pos, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for which in (pagedkv.K, pagedkv.V):
        assert np.array_equal(a.read_bytes(0, which), b.read_bytes(0, which))
    assert torch.equal(qa.view(torch.int16), qb.view(torch.int16))
    a.close()
    b.close()
    rope.close()


def test_append_rope_in_place_q_and_no_q(gpu):
    n, nb, bs, KVH, hd, H = 20, 4, 16, 2, 64, 4
    rope = pagedkv.Rope(hd, 10000.0, 256)
    c = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, torch.float16)
    k = torch.randn((n, KVH, hd), device=gpu).half()
    v = torch.randn((n, KVH, hd), device=gpu).half()
    q = torch.randn((n, H, hd), device=gpu).half()
    ref_q = rope.apply(q, torch.arange(n, dtype=torch.int32, device=gpu))
    slots = torch.arange(n, dtype=torch.int32, device=gpu)
    pos = torch.arange(n, dtype=torch.int32, device=gpu)
    out = c.layer(0).append_rope(rope, k, v, slots, pos, q=q, q_out=q)
    assert out is q
    assert c.layer(0).append_rope(rope, k, v, slots, pos) is None
    torch.cuda.synchronize()
    assert torch.equal(q, ref_q)
    kg, vg = c.layer(0).gather_seq(list(range(nb)), n)
    assert torch.equal(kg, rope.apply(k, pos))
    assert torch.equal(vg, v)
    c.close()
    rope.close()


def test_append_rope_bad_position_and_slot(gpu):
    n, nb, bs, KVH, hd, H = 4, 2, 16, 2, 128, 4
    rope = pagedkv.Rope(hd, 10000.0, 100)
    c = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, torch.bfloat16)
    k = torch.randn((n, KVH, hd), device=gpu)
    v = torch.randn((n, KVH, hd), device=gpu)
    q = torch.randn((n, H, hd), device=gpu)
    qo = torch.zeros((n, H, hd), dtype=torch.bfloat16, device=gpu)
    before_k = c.read_bytes(0, pagedkv.K)
    slots = torch.tensor([0, 1, 2, nb * bs], dtype=torch.int32, device=gpu)
    pos = torch.tensor([0, 100, 5, 6], dtype=torch.int32, device=gpu)
    c.layer(0).append_rope(rope, k, v, slots, pos, q=q, q_out=qo)
    torch.cuda.synchronize()
    with pytest.raises(pagedkv.PagedKvError):
        c.check()
    row = KVH * hd * 2
    after_k = c.read_bytes(0, pagedkv.K)
    assert np.array_equal(after_k[row:2 * row], before_k[row:2 * row])   # position 100: unwritten
    assert not np.array_equal(after_k[:row], before_k[:row])
    assert torch.count_nonzero(qo[1]) == 0 and torch.count_nonzero(qo[0]) > 0
    c.check()   # cleared
    # at the C boundary: q without q_out is rejected before any launch
    rc = pagedkv.lib().pkv_append_rope(c.handle, 0, rope.handle, pos.data_ptr(), pagedkv.F32,
                                       k.data_ptr(), v.data_ptr(), slots.data_ptr(), n,
                                       q.data_ptr(), None, H, None)
    assert rc != 0 and b"q_out" in pagedkv.lib().pkv_last_error(c.handle)
    with pytest.raises(ValueError):
        c.layer(0).append_rope(rope, k, v, slots[:3], pos)
    c.close()
    rope.close()
