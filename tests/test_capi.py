"""CPU-side tests of libpagedkv's C ABI: the library loads, exports every
symbol include/pagedkv.h declares, and the C++ host allocator behaves like
the reference's BlockAllocator (block_table.rs:16-116).  No GPU compute."""
import os
import re
import subprocess

import numpy as np
import pytest

import pagedkv
from pagedkv import _lib
import block_table as oracle_bt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pagedkv.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared, "no functions parsed from pagedkv.h"
    assert sorted(_lib.SIGNATURES) == declared


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", pagedkv.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (pkv_[a-z0-9_]+)$", out, flags=re.M))
    missing = [f for f in _declared_functions() if f not in exported]
    assert not missing, f"not exported: {missing}"
    L = pagedkv.lib()
    for f in _declared_functions():
        assert hasattr(L, f)
    assert b"gfx950" in L.pkv_version()


def test_library_holds_gfx950_code_object():
    out = subprocess.run(["/opt/rocm/bin/roc-obj-ls", pagedkv.LIB_PATH],
                         capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("roc-obj-ls unavailable")
    assert "gfx950" in out.stdout


# -- reference KATs through the product allocator (block_table.rs:65-116) --
def test_blocks_for_rounds_up():
    a = pagedkv.BlockAllocator(10, 16)
    assert [a.blocks_for(n) for n in (0, 1, 16, 17)] == [0, 1, 1, 2]


def test_ensure_capacity_allocates_and_reuses():
    a = pagedkv.BlockAllocator(4, 16)
    t = pagedkv.BlockTable()
    a.ensure_capacity(t, 1)
    assert t.blocks == [0]
    a.ensure_capacity(t, 16)
    assert t.blocks == [0]
    a.ensure_capacity(t, 17)
    assert t.blocks == [0, 1]
    assert a.free_count() == 2


def test_release_returns_blocks():
    a = pagedkv.BlockAllocator(4, 16)
    t = pagedkv.BlockTable()
    a.ensure_capacity(t, 40)
    assert a.free_count() == 1
    a.release(t)
    assert a.free_count() == 4
    assert t.blocks == []


def test_oom_returns_err_without_partial_alloc():
    a = pagedkv.BlockAllocator(2, 16)
    t = pagedkv.BlockTable()
    with pytest.raises(pagedkv.CapacityError):
        a.ensure_capacity(t, 48)
    assert t.blocks == []
    assert a.free_count() == 2


def test_locate_maps_position_to_block_and_slot():
    a = pagedkv.BlockAllocator(4, 16)
    t = pagedkv.BlockTable()
    a.ensure_capacity(t, 32)
    assert a.locate(t, 0) == (0, 0)
    assert a.locate(t, 15) == (0, 15)
    assert a.locate(t, 16) == (1, 0)
    assert a.locate(t, 31) == (1, 15)
    with pytest.raises(IndexError):  # the reference panics here
        a.locate(t, 32)


def test_allocator_random_ops_match_oracle():
    rng = np.random.default_rng(1234)
    N, bs = 64, 16
    a = pagedkv.BlockAllocator(N, bs)
    o = oracle_bt.BlockAllocator(N, bs)
    tabs = [(pagedkv.BlockTable(), oracle_bt.BlockTable()) for _ in range(6)]
    lens = [0] * len(tabs)
    for _ in range(3000):
        i = int(rng.integers(len(tabs)))
        t, ot = tabs[i]
        if rng.random() < 0.15:
            a.release(t)
            o.release(ot)
            lens[i] = 0
        else:
            n = lens[i] + int(rng.integers(0, 40))
            err_a = err_o = False
            try:
                a.ensure_capacity(t, n)
            except pagedkv.CapacityError:
                err_a = True
            try:
                o.ensure_capacity(ot, n)
            except oracle_bt.CapacityError:
                err_o = True
            assert err_a == err_o
            if not err_a:
                lens[i] = n
        assert t.blocks == ot.blocks
        assert a.free_count() == o.free_count()
        if lens[i]:
            pos = int(rng.integers(lens[i]))
            assert a.locate(t, pos) == o.locate(ot, pos)


def test_pool_create_validates_before_touching_device():
    import ctypes
    h = ctypes.c_void_p()
    L = pagedkv.lib()
    rc = L.pkv_pool_create(ctypes.byref(h), 1, 16, 12, 2, 128, pagedkv.BF16, 0)
    assert rc == _lib.PKV_ERR_UNSUPPORTED and not h.value
    assert b"block_size" in L.pkv_last_error(None)
    rc = L.pkv_pool_create(ctypes.byref(h), 1, 16, 16, 2, 96, pagedkv.BF16, 0)
    assert rc == _lib.PKV_ERR_UNSUPPORTED
    rc = L.pkv_pool_create(ctypes.byref(h), 0, 16, 16, 2, 128, pagedkv.BF16, 0)
    assert rc == _lib.PKV_ERR_INVALID
    # shapes whose byte counts would overflow the kernels' 32-bit chunk
    # counts or wrap the slab's size: refused before any device call
    for n_layers, nb, bs, kvh, hd in ((1, 16, 16, 2048, 128), (1000, 1 << 30, 256, 1024, 256),
                                      (1 << 22, 1 << 30, 16, 1, 64)):
        rc = L.pkv_pool_create(ctypes.byref(h), n_layers, nb, bs, kvh, hd, pagedkv.F32, 0)
        assert rc == _lib.PKV_ERR_UNSUPPORTED and not h.value
        assert b"pool shape" in L.pkv_last_error(None)
    assert L.pkv_pool_destroy(None) == 0
    assert L.pkv_append(None, 0, None, None, None, 1, None) == _lib.PKV_ERR_INVALID
