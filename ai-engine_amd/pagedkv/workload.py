"""Seeded synthetic workloads of the benchmark shapes (host side, numpy).

Generator: SplitMix64 (Steele, Lea, Flood, OOPSLA 2014) in counter mode,
x_i = mix(seed + (i + 1) * 0x9E3779B97F4A7C15); uniforms u = (x >> 11) 2^-53;
N(0,1) by Box-Muller in fp64 (r = sqrt(-2 ln(1 - u1)), n = r cos(2 pi u2));
then rounded to nearest-even to f32, and from f32 to nearest-even f16/bf16.
The same bytes feed the GPU and the CPU oracle.

Context lengths are uniform integers in the stated inclusive range (tokens
already cached, i.e. the reference's seq_lens[b], transformer.rs:215-217);
block tables are a Fisher-Yates permutation of [0, num_blocks), sequence b
taking the next ceil((ctx_b + 1) / block_size) ids.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

F32, F16, BF16 = 0, 1, 2


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int) -> np.ndarray:
    """n samples of N(0,1) in fp64."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    t = 2.0 * np.pi * u[1::2]
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n]


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16, as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    return (u >> np.uint64(16)).astype(np.uint16)


def to_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """fp64 -> storage elements: float32, or uint16 bit patterns of f16/bf16."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == F32:
        return x32
    if dtype == F16:
        return x32.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(x32)


def widen(a: np.ndarray, dtype: int) -> np.ndarray:
    """Storage elements -> float32 (exact)."""
    if dtype == F32:
        return np.asarray(a, dtype=np.float32)
    if dtype == F16:
        return np.asarray(a).view(np.float16).astype(np.float32)
    return (np.asarray(a).view(np.uint16).astype(np.uint32) << 16).view(np.float32)


def normal_storage(seed: int, shape, dtype: int, scale: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return to_storage(normal(seed, n) * scale, dtype).reshape(shape)


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Uniform integers in [lo, hi] inclusive."""
    span = np.uint64(hi - lo + 1)
    return (splitmix64(seed, n) % span).astype(np.int64) + lo


def permutation(seed: int, n: int) -> np.ndarray:
    """Fisher-Yates shuffle of [0, n)."""
    r = splitmix64(seed, max(n - 1, 0))
    p = np.arange(n, dtype=np.int64)
    for k, i in enumerate(range(n - 1, 0, -1)):
        j = int(r[k] % np.uint64(i + 1))
        p[i], p[j] = p[j], p[i]
    return p


@dataclasses.dataclass(frozen=True)
class Shape:
    name: str
    n_layers: int
    n_head: int
    n_kv_head: int
    head_dim: int
    block_size: int
    dtype: int


# BASELINE.json configs (model shapes).
CFG1 = Shape("llama-3.2-1b", 16, 32, 8, 64, 16, F16)
CFG2 = Shape("tinyllama-1.1b", 22, 32, 4, 64, 16, F16)
CFG3 = Shape("llama-3-8b", 32, 32, 8, 128, 16, BF16)
CFG4 = Shape("llama-3-70b-stage0", 40, 64, 8, 128, 16, BF16)
CFG5 = Shape("llama-3-8b-churn", 32, 32, 8, 128, 16, BF16)


@dataclasses.dataclass
class DecodeBatch:
    """One decode step of B sequences: contexts (tokens already cached),
    block tables, and the pool size."""
    shape: Shape
    ctx: np.ndarray          # (B,) int64, seq_lens
    tables: np.ndarray       # (B, max_nb) int32, -1 padded
    num_blocks: int

    @property
    def batch(self) -> int:
        return int(self.ctx.size)

    @property
    def context_lens(self) -> np.ndarray:
        """Keys attended after the append: seq_lens + 1."""
        return (self.ctx + 1).astype(np.int32)

    @property
    def max_blocks(self) -> int:
        return int(self.tables.shape[1])

    def slot_of_new(self) -> np.ndarray:
        bs = self.shape.block_size
        pos = self.ctx
        return (self.tables[np.arange(self.batch), pos // bs].astype(np.int64) * bs + pos % bs)


def decode_batch(shape: Shape, batch: int, ctx_lo: int, ctx_hi: int, seed: int,
                 num_blocks: int | None = None, pool_factor: float = 1.2) -> DecodeBatch:
    """Contexts U[ctx_lo, ctx_hi]; pool = ceil(pool_factor * live / bs) unless given."""
    bs = shape.block_size
    ctx = randint(seed, batch, ctx_lo, ctx_hi)
    need = -(-(ctx + 1) // bs)
    live = int((ctx + 1).sum())
    if num_blocks is None:
        num_blocks = max(int(math.ceil(pool_factor * live / bs)), int(need.sum()))
    if int(need.sum()) > num_blocks:
        raise ValueError("pool too small for the batch")
    perm = permutation(seed ^ 0x5EED, num_blocks)
    max_nb = int(need.max())
    tables = np.full((batch, max_nb), -1, dtype=np.int32)
    o = 0
    for b in range(batch):
        tables[b, :need[b]] = perm[o:o + need[b]]
        o += int(need[b])
    return DecodeBatch(shape, ctx, tables, num_blocks)


def decode_bytes(shape: Shape, ctx: np.ndarray, n_layers: int | None = None) -> int:
    """Algorithmic HBM bytes of one decode step (append + attention) summed
    over layers: per layer and sequence, K and V reads of (ctx+1) rows,
    new K/V read + write, Q read + O write, table, length and slot."""
    L = shape.n_layers if n_layers is None else n_layers
    e = 4 if shape.dtype == F32 else 2
    kvh, hd, H = shape.n_kv_head, shape.head_dim, shape.n_head
    c1 = ctx.astype(np.int64) + 1
    per = (c1 * kvh * hd * 2 * e + 2 * kvh * hd * e * 2 + 2 * H * hd * e
           + 4 * (-(-c1 // shape.block_size)) + 12)
    return int(per.sum()) * L


@dataclasses.dataclass
class MixBatch:
    """One continuous-batching step: `prior`/`chunk` of the sequences in
    chunked prefill, `ctx` of the decoding ones, and one block table per
    sequence (prefill sequences first) over a shared pool."""
    shape: Shape
    prior: np.ndarray        # (Sp,) int64 tokens cached before the chunk
    chunk: np.ndarray        # (Sp,) int64 chunk tokens appended this step
    ctx: np.ndarray          # (Sd,) int64 seq_lens of decoding sequences
    tables: np.ndarray       # (Sp + Sd, max_nb) int32, -1 padded
    num_blocks: int

    @property
    def n_prefill(self) -> int:
        return int(self.prior.size)

    @property
    def cu_q_lens(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.chunk)]).astype(np.int32)

    def chunk_slots(self) -> np.ndarray:
        """Slot (block * bs + offset) of every chunk token, in cu_q_lens order."""
        bs = self.shape.block_size
        out = []
        for s in range(self.n_prefill):
            pos = np.arange(self.prior[s], self.prior[s] + self.chunk[s])
            out.append(self.tables[s, pos // bs].astype(np.int64) * bs + pos % bs)
        return np.concatenate(out).astype(np.int32)


def mix_batch(shape: Shape, n_prefill: int, chunk: int, prior_lo: int, prior_hi: int,
              n_decode: int, ctx_lo: int, ctx_hi: int, seed: int,
              pool_factor: float = 1.2) -> MixBatch:
    """Priors U[prior_lo, prior_hi], decode contexts U[ctx_lo, ctx_hi];
    pool = ceil(pool_factor * live / bs); tables from one permutation."""
    bs = shape.block_size
    prior = randint(seed, n_prefill, prior_lo, prior_hi)
    ctx = randint(seed + 1, n_decode, ctx_lo, ctx_hi)
    lens = np.concatenate([prior + chunk, ctx + 1])
    need = -(-lens // bs)
    num_blocks = max(int(math.ceil(pool_factor * int(lens.sum()) / bs)), int(need.sum()))
    perm = permutation(seed ^ 0x5EED, num_blocks)
    tables = np.full((lens.size, int(need.max())), -1, dtype=np.int32)
    o = 0
    for s in range(lens.size):
        tables[s, :need[s]] = perm[o:o + need[s]]
        o += int(need[s])
    return MixBatch(shape, prior, np.full(n_prefill, chunk, np.int64), ctx, tables, num_blocks)


def prefill_bytes(shape: Shape, prior: np.ndarray, chunk: np.ndarray) -> int:
    """Algorithmic HBM bytes of one layer's prefill attention: K and V reads
    of prior + chunk rows, Q read and O write of the chunk (the chunk's K/V
    store is the append's, counted there)."""
    e = 4 if shape.dtype == F32 else 2
    kvh, hd, H = shape.n_kv_head, shape.head_dim, shape.n_head
    p, c = prior.astype(np.int64), chunk.astype(np.int64)
    return int(((p + c) * kvh * hd * 2 * e + 2 * c * H * hd * e).sum())


def prefill_flops(shape: Shape, prior: np.ndarray, chunk: np.ndarray) -> int:
    """Algorithmic flops of one layer's causal prefill attention: QK^T and
    PV over the unmasked (query, key) pairs, 2 flops per multiply-add."""
    p, c = prior.astype(np.int64), chunk.astype(np.int64)
    pairs = c * p + c * (c + 1) // 2
    return int((4 * shape.head_dim * shape.n_head * pairs).sum())
