"""CPU checks of the rotary embedding: the oracle's restatement of Rope::new /
apply_rope (crates/ai-engine-candle/src/paged/rope.rs) pinned by the
reference's KAT and by what the mathematics fixes, and the library's host
table builder checked against it bit for bit."""
import math

import numpy as np
import pytest

import oracle
import pagedkv


def test_reference_kat_gather_picks_rows():
    # rope.rs:49-63: Rope::new(8, 10000, 512); gather([0, 200]) has dims
    # (2, 4) and its rows equal table rows 0 and 200.
    c, s = oracle.rope_table(8, 10000.0, 512)
    pos = np.array([0, 200])
    gc, gs = c[pos], s[pos]
    assert gc.shape == (2, 4) and gs.shape == (2, 4)
    assert np.array_equal(gc[0], c[0]) and np.array_equal(gc[1], c[200])


@pytest.mark.parametrize("dim,base,max_seq", [(64, 10000.0, 2048), (128, 500000.0, 8192),
                                              (128, 10000.0, 4096), (256, 1000000.0, 1024)])
def test_table_closed_form(dim, base, max_seq):
    c, s = oracle.rope_table(dim, base, max_seq)
    half = dim // 2
    # position 0 is the identity rotation, exactly
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # theta_0 = 1, so column 0 is cos/sin of the position itself
    p = np.arange(max_seq, dtype=np.float32).astype(np.float64)
    assert np.all(np.abs(c[:, 0] - np.cos(p)) <= 2e-7)
    assert np.all(np.abs(s[:, 0] - np.sin(p)) <= 2e-7)
    # every entry: cos/sin of p * base^(-2i/dim) up to the f32 rounding of
    # theta (relative 2^-23) and of the angle (half an ulp of p * theta)
    i = np.arange(half, dtype=np.float64)
    theta = base ** (-2.0 * i / dim)
    ang = p[:, None] * theta[None, :]
    tol = ang * 2.0 ** -22 + np.spacing(ang.astype(np.float32)).astype(np.float64) + 2e-7
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    assert np.all(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1) < 1e-6)


def test_table_formula_mutations_detected():
    # plausible mistakes (2i/(d-1) exponent, i/d exponent) break the closed form
    c, _ = oracle.rope_table(128, 10000.0, 256)
    i = np.arange(64, dtype=np.float64)
    p = np.arange(256, dtype=np.float64)[:, None]
    for wrong in (10000.0 ** (-2.0 * i / 127), 10000.0 ** (-i / 128)):
        assert np.abs(c - np.cos(p * wrong)).max() > 1e-2


@pytest.mark.parametrize("dim,base,max_seq", [(64, 10000.0, 300), (128, 500000.0, 5000),
                                              (256, 10000.0, 100)])
def test_library_host_tables_equal_oracle(dim, base, max_seq):
    c, s = oracle.rope_table(dim, base, max_seq)
    lc, ls = pagedkv.rope_tables_host(dim, base, max_seq)
    assert np.array_equal(c.view(np.uint32), lc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), ls.view(np.uint32))


def test_library_host_tables_reject_bad_shape():
    with pytest.raises(pagedkv.PagedKvError):
        pagedkv.rope_tables_host(12, 10000.0, 8)   # not a multiple of 8
    with pytest.raises(pagedkv.PagedKvError):
        pagedkv.rope_tables_host(64, -1.0, 8)


def _rotate_f64(x, c, s, pos):
    half = x.shape[2] // 2
    x = x.astype(np.float64)
    cc = c[pos].astype(np.float64)[:, None, :]
    ss = s[pos].astype(np.float64)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cc - x2 * ss, x1 * ss + x2 * cc], axis=-1)


def test_apply_identity_norm_and_float64():
    rng = np.random.default_rng(3)
    c, s = oracle.rope_table(128, 500000.0, 4096)
    x = rng.standard_normal((9, 4, 128)).astype(np.float32)
    pos = np.array([0, 1, 2, 17, 511, 512, 2047, 4000, 4095], np.int32)
    y = oracle.rope_apply(x, c, s, pos)
    assert np.array_equal(y[0], x[0])                       # position 0: identity, exactly
    n_in = x[..., :64].astype(np.float64) ** 2 + x[..., 64:].astype(np.float64) ** 2
    n_out = y[..., :64].astype(np.float64) ** 2 + y[..., 64:].astype(np.float64) ** 2
    assert np.all(np.abs(n_out - n_in) <= 1e-5 * (n_in + 1e-3))  # a rotation of each pair
    ref = _rotate_f64(x, c, s, pos)
    assert np.all(np.abs(y - ref) <= 4e-7 * (np.abs(ref) + 1))
    # the rotate-half convention (not interleaved pairs, not the inverse
    # rotation): a sign or pairing mistake is far off the float64 rotation
    half = 64
    inv = np.concatenate([x[..., :half] * c[pos][:, None] + x[..., half:] * s[pos][:, None],
                          -x[..., :half] * s[pos][:, None] + x[..., half:] * c[pos][:, None]], -1)
    assert np.abs(inv[1:] - ref[1:]).max() > 1e-2


def test_apply_relative_position_invariance():
    # <rope(q, p), rope(k, p + d)> depends on d only (rotations compose)
    rng = np.random.default_rng(4)
    c, s = oracle.rope_table(128, 10000.0, 4096)
    q = rng.standard_normal((1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128)).astype(np.float32)
    for d in (0, 5, 100):
        dots = []
        for p in (0, 7, 300, 2000):
            qr = oracle.rope_apply(q, c, s, np.array([p], np.int32))
            kr = oracle.rope_apply(k, c, s, np.array([p + d], np.int32))
            dots.append(float(np.dot(qr.ravel().astype(np.float64), kr.ravel())))
        assert max(dots) - min(dots) <= 2e-3 * (1 + abs(dots[0]))
