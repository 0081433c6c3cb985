"""CPU checks of the model-shape rule (pagedkv.arch), which restates
ArchConfig::from_gguf / supported_arch (crates/ai-engine-candle/src/paged/
arch.rs:8-90): the reference's own tests (arch.rs:113-127) and metadata of
three public model families, each exercising one fallback."""
import pytest

from pagedkv.arch import ArchConfig, ArchError, supported_arch


def test_reference_kat_supported_arch_allowlist():
    # arch.rs:113-119
    assert supported_arch("llama") == "llama"
    assert supported_arch("qwen2") == "qwen2"
    assert supported_arch("qwen3") == "qwen3"
    with pytest.raises(ArchError, match="unsupported architecture 'gemma'"):
        supported_arch("gemma")


def _meta(arch, **kw):
    base = {"general.architecture": arch, f"{arch}.attention.head_count": 32,
            f"{arch}.attention.head_count_kv": 8, f"{arch}.block_count": 32,
            f"{arch}.embedding_length": 4096, f"{arch}.attention.layer_norm_rms_epsilon": 1e-5}
    base.update({f"{arch}.{k.replace('__', '.')}": v for k, v in kw.items()})
    return base


@pytest.mark.parametrize("arch,qkv,qkn", [("llama", False, False), ("qwen2", True, False),
                                          ("qwen3", False, True)])
def test_reference_kat_flags_match_family(arch, qkv, qkn):
    # arch.rs:121-127
    c = ArchConfig.from_metadata(_meta(arch))
    assert (c.qkv_bias, c.qk_norm) == (qkv, qkn)


def test_llama3_8b_shape_derives_head_dim():
    # no attention.key_length: head_dim = embedding_length / head_count
    c = ArchConfig.from_metadata(_meta("llama", rope__dimension_count=128, rope__freq_base=500000.0,
                                       context_length=8192))
    assert (c.head_dim, c.rope_dim, c.head_count_kv, c.block_count) == (128, 128, 8, 32)
    assert (c.rope_freq_base, c.context_length) == (500000.0, 8192)
    assert c.pool_shape(4096, 16) == dict(n_layers=32, num_blocks=4096, block_size=16,
                                          n_kv_head=8, head_dim=128)
    assert c.rope_shape() == dict(rope_dim=128, freq_base=500000.0, max_seq=8192)


def test_qwen3_explicit_key_length_wins():
    # Qwen3-0.6B: embedding 1024 / 16 heads = 64, but key_length says 128
    m = _meta("qwen3", attention__key_length=128)
    m.update({"qwen3.embedding_length": 1024, "qwen3.attention.head_count": 16})
    c = ArchConfig.from_metadata(m)
    assert c.head_dim == 128
    assert c.rope_dim == 128  # no rope.dimension_count: falls back to key_length


def test_qwen2_rope_dim_falls_back_to_derived_head_dim():
    # Qwen2-0.5B: 896 / 14 = 64, no key_length, no rope.dimension_count
    m = _meta("qwen2", rope__freq_base=1000000.0)
    m.update({"qwen2.embedding_length": 896, "qwen2.attention.head_count": 14,
              "qwen2.attention.head_count_kv": 2, "qwen2.block_count": 24})
    c = ArchConfig.from_metadata(m)
    assert (c.head_dim, c.rope_dim, c.head_count_kv) == (64, 64, 2)
    assert c.rope_freq_base == 1000000.0


def test_defaults_and_integer_division():
    m = _meta("llama")
    m["llama.embedding_length"] = 4100  # not a multiple of head_count: integer division
    c = ArchConfig.from_metadata(m)
    assert c.head_dim == 4100 // 32
    assert (c.rope_freq_base, c.context_length) == (10000.0, 4096)


@pytest.mark.parametrize("key", ["attention.head_count", "attention.head_count_kv", "block_count",
                                 "embedding_length", "attention.layer_norm_rms_epsilon"])
def test_missing_required_key_is_named(key):
    m = _meta("llama")
    del m[f"llama.{key}"]
    with pytest.raises(ArchError, match=f"gguf missing llama.{key}"):
        ArchConfig.from_metadata(m)


def test_missing_architecture():
    with pytest.raises(ArchError, match="general.architecture"):
        ArchConfig.from_metadata({})
    with pytest.raises(ArchError, match="unsupported"):
        ArchConfig.from_metadata(_meta("gemma"))
