"""Writes the committed decode golden vectors (tests/golden/decode_*.npz).

Inputs come from the seeded workload generator (pagedkv.workload); expected
outputs from the oracle's fp64 closed form (oracle.paged_attention_f64),
whose agreement with torch float64 SDPA and the reference's own KATs is
checked in tests/test_oracle.py.  Run from the repository root:
    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "ai-engine_amd"), os.path.join(ROOT, "oracle")]

import oracle  # noqa: E402
from pagedkv import workload as wl  # noqa: E402

CASES = [
    # name, dtype, H, KVH, hd, bs, B, ctx_lo, ctx_hi
    ("bf16_h128_r4", wl.BF16, 8, 2, 128, 16, 3, 0, 200),
    ("f16_h64_r8", wl.F16, 16, 2, 64, 16, 3, 1, 200),
    ("f32_h64_r1", wl.F32, 4, 4, 64, 32, 2, 0, 100),
    ("bf16_h256_r2", wl.BF16, 4, 2, 256, 16, 2, 5, 90),
]


def make(name, dt, H, KVH, hd, bs, B, lo, hi, seed):
    shape = wl.Shape(name, 1, H, KVH, hd, bs, dt)
    batch = wl.decode_batch(shape, B, lo, hi, seed, pool_factor=1.5)
    nb = batch.num_blocks
    kp = wl.normal_storage(seed + 1, (nb, bs, KVH, hd), dt)
    vp = wl.normal_storage(seed + 2, (nb, bs, KVH, hd), dt)
    q = wl.normal_storage(seed + 3, (B, H, hd), dt, scale=1 / math.sqrt(hd))
    scale = 1 / math.sqrt(hd)
    tables = np.where(batch.tables < 0, 0, batch.tables).astype(np.int32)
    cl = batch.context_lens
    out = oracle.paged_attention_f64(kp, vp, dt, bs, tables.astype(np.uint32), cl,
                                     wl.widen(q, dt), scale)
    np.savez_compressed(os.path.join(os.path.dirname(__file__), f"decode_{name}.npz"),
                        k_pool=kp, v_pool=vp, tables=tables, context_lens=cl, q=q,
                        scale=np.float64(scale), block_size=np.int64(bs), dtype=np.int64(dt),
                        n_head=np.int64(H), out=out)


if __name__ == "__main__":
    for i, c in enumerate(CASES):
        make(*c, seed=1000 + 17 * i)
        print("wrote", c[0])
