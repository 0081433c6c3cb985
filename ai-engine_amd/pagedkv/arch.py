"""Model shape of the paged path, from GGUF metadata.

Restates `ArchConfig::from_gguf` and `supported_arch`
(crates/ai-engine-candle/src/paged/arch.rs:8-90): the engine sizes its KV
pools from `block_count`, `head_count_kv` and `head_dim` (engine.rs:68-71)
and its RoPE tables from `rope_dim`, `rope_freq_base` and `context_length`
(transformer.rs:113, engine.rs:45-47).  The metadata arrives as a plain
mapping from GGUF keys to values (reading the GGUF file itself belongs to
the model loader, outside this library).  Pure host code.
"""
from __future__ import annotations

import dataclasses
from typing import Any, Mapping

SUPPORTED = ("llama", "qwen2", "qwen3")


class ArchError(ValueError):
    """Unsupported architecture or missing metadata (the reference's bail!)."""


def supported_arch(arch: str) -> str:
    """arch.rs:27-36: the allowlist; anything else is an error."""
    if arch in SUPPORTED:
        return arch
    raise ArchError(f"paged engine: unsupported architecture '{arch}' "
                    f"(supported: {', '.join(SUPPORTED)})")


@dataclasses.dataclass(frozen=True)
class ArchConfig:
    """arch.rs:8-24."""
    arch: str
    block_count: int
    embedding_length: int
    head_count: int
    head_count_kv: int
    head_dim: int
    rope_dim: int
    rope_freq_base: float
    rms_norm_eps: float
    qkv_bias: bool
    qk_norm: bool
    context_length: int

    @classmethod
    def from_metadata(cls, meta: Mapping[str, Any]) -> "ArchConfig":
        """arch.rs:39-90.  Required keys raise ArchError naming the key;
        optional ones take the reference's fallbacks: head_dim =
        `attention.key_length` else embedding_length / head_count (integer
        division), rope_dim = `rope.dimension_count` else that head_dim,
        rope_freq_base 10000, context_length 4096."""
        if "general.architecture" not in meta:
            raise ArchError("gguf missing general.architecture")
        arch = supported_arch(str(meta["general.architecture"]))

        def req(key: str):
            full = f"{arch}.{key}"
            if full not in meta:
                raise ArchError(f"gguf missing {full}")
            return meta[full]

        def opt(key: str, default):
            return meta.get(f"{arch}.{key}", default)

        head_count = int(req("attention.head_count"))
        head_count_kv = int(req("attention.head_count_kv"))
        block_count = int(req("block_count"))
        embedding_length = int(req("embedding_length"))
        head_dim = int(opt("attention.key_length", embedding_length // head_count))
        rope_dim = int(opt("rope.dimension_count", head_dim))
        rms_norm_eps = float(req("attention.layer_norm_rms_epsilon"))
        return cls(arch=arch, block_count=block_count, embedding_length=embedding_length,
                   head_count=head_count, head_count_kv=head_count_kv, head_dim=head_dim,
                   rope_dim=rope_dim, rope_freq_base=float(opt("rope.freq_base", 10000.0)),
                   rms_norm_eps=rms_norm_eps, qkv_bias=arch == "qwen2", qk_norm=arch == "qwen3",
                   context_length=int(opt("context_length", 4096)))

    def pool_shape(self, kv_cache_blocks: int, block_size: int) -> dict:
        """Arguments of PagedKvCache for this model (engine.rs:68-72: one
        pool per layer of (blocks, block_size, head_count_kv, head_dim))."""
        return dict(n_layers=self.block_count, num_blocks=kv_cache_blocks,
                    block_size=block_size, n_kv_head=self.head_count_kv,
                    head_dim=self.head_dim)

    def rope_shape(self) -> dict:
        """Arguments of Rope for this model (transformer.rs:113; the table
        covers context_length positions, engine.rs:45-47)."""
        return dict(rope_dim=self.rope_dim, freq_base=self.rope_freq_base,
                    max_seq=self.context_length)
