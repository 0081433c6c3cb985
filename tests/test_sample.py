"""CPU checks of token selection: the oracle's restatement of sample() and
argmax() (crates/ai-engine-runtime/src/sample.rs:12-55) pinned by the
reference's four KATs (crates/ai-engine-runtime/tests/sample.rs), closed
forms and the public test vectors of the random-number primitives; and the
library's host-side draw checked against it; and the restatement of glibc's
expf that the device's exact sampler uses, checked against the host libm on
every float <= 0."""
import math
import struct

import numpy as np
import pytest

import oracle
import pagedkv

R42 = oracle.sample_draw(42)


# -- the reference's own tests (ai-engine-runtime/tests/sample.rs) ----------
def test_reference_kat_greedy_picks_argmax():
    assert oracle.sample([0.1, 5.0, 2.0, -1.0], 0.0, seed=42)[0] == 1


def test_reference_kat_temperature_zero_is_greedy():
    for _ in range(20):
        assert oracle.sample([1.0, 5.0, 2.0], 0.0, seed=0)[0] == 1


def test_reference_kat_top_k_one_picks_largest():
    for _ in range(20):
        assert oracle.sample([1.0, 1.0, 1.0, 1.0, 100.0], 1.0, top_k=1, seed=0)[0] == 4


def test_reference_kat_top_p_nucleus_concentrates_mass():
    for _ in range(20):
        assert oracle.sample([1.0, 1.0, 100.0, 1.0], 1.0, top_p=0.5, seed=0)[0] == 2


# -- random-number primitives: public test vectors ---------------------------
def test_chacha_block_public_vectors():
    # all-zero key, counter and nonce: the ChaCha20 keystream of RFC 8439
    # appendix A.1 test vector #1, and the 12-round keystream of the
    # ChaCha test-vector draft (TC1), as little-endian words
    z = np.zeros(8, np.uint32)
    c20 = oracle.chacha_block(z, 0, 0, 20)
    assert [hex(w) for w in c20[:8]] == ["0xade0b876", "0x903df1a0", "0xe56a5d40", "0x28bd8653",
                                         "0xb819d2bd", "0x1aed8da0", "0xccef36a8", "0xc70d778b"]
    c12 = oracle.chacha_block(z, 0, 0, 12).astype("<u4").tobytes()
    assert c12[:32].hex() == "9bf49a6a0755f953811fce125f2683d50429c3bb49e074147e0089a52eae155f"


def test_pcg32_output_demo_vector():
    # pcg32-demo of the PCG reference implementation: srandom(42, 54), then
    # each output is XSH-RR of the state before the step
    mul, m64 = 6364136223846793005, (1 << 64) - 1
    inc = (54 << 1) | 1
    st = 0
    st = (st * mul + inc) & m64
    st = (st + 42) & m64
    st = (st * mul + inc) & m64
    out = []
    for _ in range(6):
        out.append(oracle.pcg32_output(st))
        st = (st * mul + inc) & m64
    assert out == [0xa15c02b7, 0x7b47f409, 0xba1d3330, 0x83d2f293, 0xbfa4784b, 0xcbed606e]


def test_draw_composition_and_range():
    # the draw is the top 24 bits of ChaCha12 block 0, word 0, under the
    # seed_from_u64 key; a different seed gives a different value
    key = oracle.seed_from_u64(42)
    w0 = int(oracle.chacha_block(key, 0, 0, 12)[0])
    assert R42 == (w0 >> 8) * 2.0 ** -24
    assert 0.0 <= R42 < 1.0
    assert oracle.sample_draw(0) != R42


def test_library_draw_equals_oracle():
    for seed in (0, 1, 42, 2 ** 63 + 5, 2 ** 64 - 1):
        assert pagedkv.sample_draw(seed) == oracle.sample_draw(seed)


# -- closed forms --------------------------------------------------------------
@pytest.mark.parametrize("V", [10, 100, 1000, 4096])
def test_uniform_logits_pick_floor_r_v(V):
    # equal values keep index order; each p = 1/V, so the first index whose
    # cumulative mass reaches r is floor(r V) (r V is far from an integer here)
    assert abs(R42 * V - round(R42 * V)) > 1e-3
    assert oracle.sample(np.zeros(V), 1.0)[0] == math.floor(R42 * V)
    assert oracle.sample(np.full(V, 3.5), 0.6)[0] == math.floor(R42 * V)


def test_uniform_top_k_and_top_p_renormalise():
    # top_k = 10: the first ten indices, p = 1/10 -> floor(10 r)
    assert oracle.sample(np.zeros(1000), 1.0, top_k=10)[0] == math.floor(10 * R42)
    # top_p = 0.5: the first ~500 indices, renormalised -> floor(500 r)
    assert oracle.sample(np.zeros(1000), 1.0, top_p=0.5)[0] == math.floor(500 * R42)


@pytest.mark.parametrize("a,b,T", [(0.0, 2.0, 1.0), (1.0, -1.0, 0.5), (3.0, 3.5, 2.0),
                                   (0.0, 5.0, 1.0), (2.0, 0.0, -1.0)])
def test_two_tokens_logistic(a, b, T):
    # sorted by a/T and b/T; the larger one is picked iff r <= its p
    ya, yb = a / T, b / T
    top, other = (0, 1) if ya >= yb else (1, 0)
    p_top = 1.0 / (1.0 + math.exp(-abs(ya - yb)))
    expect = top if R42 <= p_top else other
    tok, margin = oracle.sample([a, b], T)
    assert margin > 1e-4
    assert tok == expect


def test_argmax_rules():
    assert oracle.argmax([1.0, 5.0, 5.0, 2.0]) == 1          # first maximum
    assert oracle.argmax([math.nan, 1.0, 3.0]) == 2          # NaN never chosen
    assert oracle.argmax([-math.inf, -math.inf]) == 0        # fold starts at (0, -inf)
    assert oracle.argmax([math.nan, -math.inf, math.nan]) == 0
    assert oracle.argmax([]) == 0
    assert oracle.sample([7.0], 2.0)[0] == 0                  # one logit: argmax path


def test_sample_mutations_detected():
    # a different draw or a reversed tie order changes the uniform pick
    V = 1000
    assert math.floor(oracle.sample_draw(0) * V) != math.floor(R42 * V)
    assert V - 1 - math.floor(R42 * V) != oracle.sample(np.zeros(V), 1.0)[0]


def test_f32_rounding_is_the_only_difference_from_exact_arithmetic():
    # The reference's f32 running sums (sorted order) approximate the exact
    # cumulative mass; over a vocabulary of tens of thousands they drift by up
    # to ~5e-5, enough to move the pick inside a run of near-equal
    # probabilities.  Where the f32 and float64 restatements disagree, the
    # exact running sum must sit that close to its threshold.
    rng = np.random.default_rng(11)
    disagree = 0
    for t in range(160):
        V = int(rng.choice([7, 1000, 32000]))
        if t % 2:
            x = rng.integers(-3, 3, V).astype(np.float32)
        else:
            x = rng.standard_normal(V).astype(np.float32) * 3
        T = float(rng.choice([0.3, 0.7, 1.0, -1.0]))
        k = int(rng.choice([0, 40]))
        p = [None, 0.9][t % 3 == 0]
        a, _ = oracle.sample(x, T, top_k=k, top_p=p)
        b, m64 = oracle.sample(x, T, top_k=k, top_p=p, precise=True)
        if a != b:
            disagree += 1
            assert m64 < 1e-4, (t, V, a, b, m64)
    assert disagree < 40


def test_vocab_of_two_to_the_24_is_refused():
    # masses are 2^-40 fixed point summed in 64 bits: a flat row of 2^24
    # tokens would total 2^64 and wrap, so the call refuses it before any
    # device work (2^24 - 1 passes validation)
    import pagedkv
    from pagedkv import _lib
    L = pagedkv.lib()
    rc = L.pkv_sample(None, pagedkv.F32, 1 << 24, 1, 1 << 24, None, 0, 1.0, 42, None, None)
    assert rc == _lib.PKV_ERR_INVALID
    assert b"2^24" in L.pkv_last_error(None)


# -- expf: the reference's f32::exp is the host C library's expf ------------
def test_exp2_table_is_two_to_the_i_over_32():
    # the restatement's table: 2^(i/32) rounded to double, minus i << 47
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    for i in range(32):
        d = float((Decimal(i) / 32 * ln2).exp())  # correctly rounded
        bits = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert oracle.exp2_tab_entry(i) == (bits - (i << 47)) % (1 << 64), i


def test_expf_restatement_equals_host_libm_on_every_nonpositive_float():
    # all 2^31 - 2^23 + 1 patterns from -0.0 to -inf: the sampler only
    # evaluates exp(y - max) <= 0
    n, first = oracle.expf_mismatches(0x80000000, 0xFF800000)
    assert n == 0, hex(first)
    # positive finite arguments, every 61st pattern
    n, first = oracle.expf_mismatches(0, 0x7F7FFFFF, 61)
    assert n == 0, hex(first)


def test_expf_reduction_is_one_fused_multiply_add():
    # the one non-positive input where computing r = x N / ln2 - k from the
    # rounded product instead (an unfused build) rounds the result the other
    # way: the host libm gives 0x1.f45326p-92, the correctly rounded value
    # is 0x1.f45324p-92
    x = struct.unpack("<f", struct.pack("<I", 0xC27C65D9))[0]
    host = float(oracle.expf_host(np.array([x], np.float32))[0])
    assert host == float.fromhex("0x1.f45326p-92") == oracle.expf_glibc(x)


def test_flat_rows_where_f32_rounding_moves_the_pick():
    # Equal logits: p = 1 each, the sum is V, each probability fl(1/V), and
    # the f32 running sum drifts from (k + 1) / V.  The oracle's f32 pick
    # equals numpy's sequential float32 cumulative sum; the exact pick is
    # ceil(r V) - 1.  These rows tell the reference's arithmetic apart.
    r = np.float32(R42)
    for V, f32_pick, exact_pick in ((2616, 349, 348), (3493, 465, 466),
                                    (128256, 17114, 17110), (139990, 18673, 18676)):
        acc = np.add.accumulate(np.full(V, np.float32(1) / np.float32(V), np.float32),
                                dtype=np.float32)
        assert int(np.argmax(acc >= r)) == f32_pick
        assert math.ceil(float(r) * V) - 1 == exact_pick
        x = np.full(V, 1.25, np.float32)
        assert oracle.sample(x, 1.0)[0] == f32_pick
        assert oracle.sample(x, 1.0, precise=True)[0] == exact_pick
