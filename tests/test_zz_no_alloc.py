"""pkv_decode_attention_noalloc (no reference counterpart: the decode entry
point for callers that cannot allocate) against pkv_decode_attention,
through the C ABI: identical output bits and identical pool bytes after the
fused append, on two calls in a row, the second with a smaller input; the
call allocates no device memory; a launch whose partials exceed the static
scratch array is refused before anything is enqueued."""
import ctypes
import math

import numpy as np
import pytest
import torch

import pagedkv
from pagedkv import workload as wl

pytestmark = pytest.mark.gpu

TD = {wl.F32: torch.float32, wl.F16: torch.float16, wl.BF16: torch.bfloat16}


def _dev(a, dt, gpu):
    a = np.ascontiguousarray(a)
    if dt == wl.F32:
        return torch.from_numpy(a).to(gpu)
    return torch.from_numpy(a.view(np.int16)).view(TD[dt]).to(gpu)


def _batch(seed, dt, H, KVH, hd, bs, ctx, nb, gpu):
    """Random q / new rows and disjoint block tables over nb blocks."""
    ctx = np.asarray(ctx, np.int64)
    need = -(-(ctx + 1) // bs)
    perm = wl.permutation(seed, nb)
    tables = np.zeros((len(ctx), int(need.max())), np.int32)
    o = 0
    for b in range(len(ctx)):
        tables[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    assert o <= nb
    B = len(ctx)
    return dict(
        q=_dev(wl.normal_storage(seed + 3, (B, H, hd), dt, scale=1 / math.sqrt(hd)), dt, gpu),
        kn=_dev(wl.normal_storage(seed + 4, (B, KVH, hd), dt), dt, gpu),
        vn=_dev(wl.normal_storage(seed + 5, (B, KVH, hd), dt), dt, gpu),
        tables=torch.from_numpy(tables).to(gpu),
        cl=torch.from_numpy((ctx + 1).astype(np.int32)).to(gpu),
        max_cl=int(ctx.max()) + 1, B=B, H=H)


def _call(fn, cache, x, out, stream):
    L = pagedkv.lib()
    rc = getattr(L, fn)(cache.handle, 0, x["q"].data_ptr(), out.data_ptr(), pagedkv.F32,
                        x["tables"].data_ptr(), x["tables"].shape[1], x["cl"].data_ptr(),
                        x["max_cl"], x["B"], x["H"], ctypes.c_float(1 / math.sqrt(out.shape[1] // x["H"])),
                        x["kn"].data_ptr(), x["vn"].data_ptr(), stream)
    assert rc == 0, L.pkv_last_error(cache.handle)


@pytest.mark.parametrize("dt,H,KVH,hd", [(wl.BF16, 32, 8, 128), (wl.F32, 14, 2, 64),
                                         (wl.F16, 40, 2, 128)])
def test_noalloc_equals_decode_attention_twice(gpu, dt, H, KVH, hd):
    bs, nb = 16, 3000
    fill = [wl.normal_storage(1, (nb, bs, KVH, hd), dt), wl.normal_storage(2, (nb, bs, KVH, hd), dt)]
    ref = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt])
    new = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, TD[dt])
    for c in (ref, new):
        c.write_bytes(0, pagedkv.K, fill[0])
        c.write_bytes(0, pagedkv.V, fill[1])
    stream = torch.cuda.current_stream().cuda_stream or None
    # first call: long contexts (split partitions and a merge), then a
    # smaller batch with shorter contexts
    for seed, ctx in ((10, [4000, 17, 2500, 1023, 1024, 9, 3100, 600]), (20, [300, 5, 1900])):
        x = _batch(seed, dt, H, KVH, hd, bs, ctx, nb, gpu)
        o_ref = torch.empty((x["B"], H * hd), dtype=torch.float32, device=gpu)
        o_new = torch.full_like(o_ref, float("nan"))
        _call("pkv_decode_attention", ref, x, o_ref, stream)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        _call("pkv_decode_attention_noalloc", new, x, o_new, stream)
        torch.cuda.synchronize()
        if seed == 20:  # kernels loaded by the first call: nothing may be allocated
            assert torch.cuda.mem_get_info()[0] == free0
        ref.check()
        new.check()
        assert torch.equal(o_new, o_ref)
        for which in (pagedkv.K, pagedkv.V):
            assert np.array_equal(new.read_bytes(0, which), ref.read_bytes(0, which))
    ref.close()
    new.close()


def test_noalloc_refuses_partials_beyond_the_array(gpu):
    H, KVH, hd, bs = 32, 8, 128, 16
    cache = pagedkv.PagedKvCache(1, 64, bs, KVH, hd, torch.bfloat16)
    B, max_cl = 256, 32768
    need = pagedkv.lib().pkv_decode_workspace_bytes(cache.handle, B, H, max_cl)
    assert need > (64 << 20)
    q = torch.zeros((B, H, hd), dtype=torch.bfloat16, device=gpu)
    out = torch.zeros((B, H * hd), dtype=torch.float32, device=gpu)
    tables = torch.zeros((B, 1), dtype=torch.int32, device=gpu)
    cl = torch.ones(B, dtype=torch.int32, device=gpu)
    L = pagedkv.lib()
    rc = L.pkv_decode_attention_noalloc(cache.handle, 0, q.data_ptr(), out.data_ptr(),
                                        pagedkv.F32, tables.data_ptr(), 1, cl.data_ptr(), max_cl,
                                        B, H, ctypes.c_float(0.1), None, None, None)
    assert rc == pagedkv._lib.PKV_ERR_UNSUPPORTED
    assert b"static scratch" in L.pkv_last_error(cache.handle)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0   # nothing was enqueued
    cache.close()
