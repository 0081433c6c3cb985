"""CPU checks of token selection: the oracle's restatement of sample() and
argmax() (crates/ai-engine-runtime/src/sample.rs:12-55) pinned by the
reference's four KATs (crates/ai-engine-runtime/tests/sample.rs), closed
forms and the public test vectors of the random-number primitives; and the
library's host-side draw checked against it."""
import math

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
