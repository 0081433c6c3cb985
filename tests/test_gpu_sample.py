"""GPU parity of token selection against the CPU oracle's restatement of
sample() / argmax() (crates/ai-engine-runtime/src/sample.rs:12-55).

pkv_sample_exact (pagedkv.sample, the default): the token equals the
oracle's f32 restatement -- the reference's own arithmetic -- on every row.

pkv_sample (exact=False): greedy rows are exact; the kernel sums probability
mass exactly (integers), so sampled rows are compared with the oracle's
restatement in exact arithmetic (float64 exp and running sums over the
reference's f32 values): the token must be equal unless that restatement's
running sum lies within 1e-6 of r or top_p.  Against the f32 restatement, a
row may differ only where that rounding alone moves the pick, i.e. where the
f32 and float64 restatements differ."""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
AMBIGUOUS = 1e-6


def _logits(rng, kind, V):
    if kind == "normal":
        return rng.standard_normal(V).astype(np.float32) * rng.choice([0.5, 3.0, 10.0])
    if kind == "ties":
        return rng.integers(-3, 3, V).astype(np.float32)
    if kind == "flat":
        return np.full(V, 1.25, np.float32)
    x = (rng.standard_normal(V) * 4).astype(np.float32)   # a few dominant tokens
    x[rng.integers(0, V, 3)] = 9.0
    return x


def _check_rows(x32, temps, top_k, top_p, got, seed=42):
    """Returns the rows where the kernel and the f32 restatement differ."""
    differ = []
    for b in range(x32.shape[0]):
        t = float(temps[b])
        exact, margin = oracle.sample(x32[b], t, top_k=top_k, top_p=top_p, seed=seed,
                                      precise=True)
        ref32, _ = oracle.sample(x32[b], t, top_k=top_k, top_p=top_p, seed=seed)
        g = int(got[b])
        if g != exact:
            assert margin < AMBIGUOUS, (b, exact, g, margin)
        if g != ref32:
            assert ref32 != exact or margin < AMBIGUOUS, (b, ref32, exact, g)
            differ.append(b)
    return differ


@pytest.mark.parametrize("exact", [True, False])
def test_reference_kats_on_device(gpu, exact):
    cases = [([0.1, 5.0, 2.0, -1.0], 0.0, None, None, 1),
             ([1.0, 5.0, 2.0], 0.0, None, None, 1),
             ([1.0, 1.0, 1.0, 1.0, 100.0], 1.0, 1, None, 4),
             ([1.0, 1.0, 100.0, 1.0], 1.0, None, 0.5, 2)]
    for x, t, k, p, want in cases:
        lg = torch.tensor([x], dtype=torch.float32, device=gpu)
        tok = pagedkv.sample(lg, torch.tensor([t]), top_k=k, top_p=p, seed=0, exact=exact)
        assert int(tok.item()) == want


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [2, 7, 1000, 32000, 128256])
@pytest.mark.parametrize("top_k,top_p", [(None, None), (40, None), (None, 0.9), (5, 0.5)])
def test_sample_matches_oracle(gpu, dt, V, top_k, top_p):
    rng = np.random.default_rng(V + 7 * (top_k or 0) + int(100 * (top_p or 0)))
    kinds = ["normal", "ties", "flat", "spiky"]
    B = 24
    x = np.stack([_logits(rng, kinds[b % 4], V) for b in range(B)])
    lg = torch.from_numpy(x).to(gpu).to(TD[dt])
    x32 = lg.float().cpu().numpy()          # the values the kernel sees
    temps = np.array([[0.0, 0.7, 1.0, 1.6, -1.0, 0.3][b % 6] for b in range(B)], np.float32)
    got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), top_k=top_k, top_p=top_p, exact=False)
    torch.cuda.synchronize()
    _check_rows(x32, temps, top_k, top_p, got.cpu().numpy())


def test_uniform_rows_closed_form(gpu):
    # equal logits keep index order: the pick is floor(r V)
    r = pagedkv.sample_draw(42)
    for V in (10, 100, 1000, 4096, 50000):
        lg = torch.zeros((3, V), dtype=torch.bfloat16, device=gpu)
        tok = pagedkv.sample(lg, torch.tensor([1.0, 0.5, 2.0]), exact=False)
        assert tok.cpu().tolist() == [math.floor(r * V)] * 3
    lg = torch.zeros((1, 1000), device=gpu)
    assert int(pagedkv.sample(lg, torch.tensor([1.0]), top_k=10, exact=False).item()) == math.floor(10 * r)
    assert int(pagedkv.sample(lg, torch.tensor([1.0]), top_p=0.5, exact=False).item()) == math.floor(500 * r)


@pytest.mark.parametrize("exact", [True, False])
def test_greedy_rules_on_device(gpu, exact):
    nan, inf = math.nan, math.inf
    rows = [[1.0, 5.0, 5.0, 2.0], [nan, 1.0, 3.0, 3.0], [-inf, -inf, -inf, -inf],
            [nan, -inf, nan, nan], [2.0, nan, 2.0, 9.0]]
    lg = torch.tensor(rows, device=gpu)
    tok = pagedkv.sample(lg, exact=exact)    # no temperatures: every row greedy
    assert tok.cpu().tolist() == [oracle.argmax(r) for r in rows] == [1, 2, 0, 0, 3]
    # one logit: argmax even when sampling; no logits: token 0
    one = torch.tensor([[4.0]], device=gpu)
    assert int(pagedkv.sample(one, torch.tensor([1.0]), exact=exact).item()) == 0
    assert int(pagedkv.sample(torch.zeros((1, 0), device=gpu), exact=exact).item()) == 0
    # a large greedy row: first maximum by index
    x = torch.randn((4, 128256), device=gpu)
    x[:, 77777] = 50.0
    x[:, 99999] = 50.0
    assert pagedkv.sample(x, exact=exact).cpu().tolist() == [77777] * 4


def test_strided_rows_and_determinism(gpu):
    rng = np.random.default_rng(3)
    big = torch.from_numpy(rng.standard_normal((16, 40000)).astype(np.float32)).to(gpu)
    lg = big[:, 1000:33000]                  # row stride 40000, vocab 32000
    temps = torch.full((16,), 0.8)
    a = pagedkv.sample(lg, temps, exact=False)
    b = pagedkv.sample(lg, temps, exact=False)
    assert torch.equal(a, b)
    _check_rows(lg.cpu().numpy(), temps.numpy(), None, None, a.cpu().numpy())


def test_seed_changes_draw(gpu):
    lg = torch.zeros((1, 1000), device=gpu)
    for seed in (0, 1, 42, 12345):
        tok = int(pagedkv.sample(lg, torch.tensor([1.0]), seed=seed, exact=False).item())
        assert tok == math.floor(pagedkv.sample_draw(seed) * 1000)


@pytest.mark.parametrize("exact", [True, False])
def test_invalid_arguments(gpu, exact):
    lg = torch.zeros((2, 10), device=gpu)
    with pytest.raises(pagedkv.PagedKvError):
        pagedkv.sample(lg, torch.ones(2), top_k=-1, exact=exact)


# -- batches of at most 128 rows split each row over several workgroups --------
def _rows(rng, B, V):
    kinds = ["normal", "ties", "flat", "spiky"]
    return np.stack([_logits(rng, kinds[b % 4], V) for b in range(B)])


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_split_rows_equal_one_workgroup_rows(gpu, dt):
    # 16 rows go through the split path; the same rows repeated to 256 rows
    # (one workgroup per row) must give the same tokens, bit for bit: both
    # add the same integer masses
    rng = np.random.default_rng(5)
    V, B = 128256, 16
    x = _rows(rng, B, V)
    temps = np.array([[0.0, 0.7, 1.0, 1.6, -1.0, 0.3, 0.8, 2.0][b % 8] for b in range(B)],
                     np.float32)
    lg = torch.from_numpy(x).to(gpu).to(TD[dt])
    small = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), exact=False)
    big = pagedkv.sample(lg.repeat(16, 1), torch.from_numpy(np.tile(temps, 16)).to(gpu),
                         exact=False)
    torch.cuda.synchronize()
    assert torch.equal(big.view(16, B), small.view(1, B).expand(16, B))
    _check_rows(lg.float().cpu().numpy(), temps, None, None, small.cpu().numpy())


@pytest.mark.parametrize("B", [1, 3, 8, 64, 128])
def test_split_ragged_vocab_and_strides(gpu, B):
    # a vocabulary that is not a multiple of the 16-byte vector, rows at an
    # odd stride (element loads), and batch sizes on both sides of the limit
    rng = np.random.default_rng(B)
    V = 50001
    big = torch.from_numpy(_rows(rng, B, V + 3)).to(gpu).to(torch.bfloat16)
    lg = big[:, 1:V + 1]                       # row stride V + 3, misaligned start
    temps = np.array([[0.9, 0.0, 1.3, 0.6][b % 4] for b in range(B)], np.float32)
    got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), exact=False)
    torch.cuda.synchronize()
    _check_rows(lg.float().cpu().numpy(), temps, None, None, got.cpu().numpy())


@pytest.mark.parametrize("with_temps", [False, True])
def test_split_greedy_rows(gpu, with_temps):
    # greedy rows: without temperatures (one launch) and with zero
    # temperatures (the split path's per-chunk maxima); first maximum by
    # index across chunk borders
    B, V = 6, 128256
    x = torch.randn((B, V), device=gpu)
    for b, pos in enumerate([0, 4095, 4096, 65000, 128255, 100]):
        x[b, pos] = 40.0
    x[5, 90000] = 40.0                         # a later equal maximum loses
    temps = torch.zeros(B, device=gpu) if with_temps else None
    assert pagedkv.sample(x, temps, exact=False).cpu().tolist() == [0, 4095, 4096, 65000, 128255, 100]


def test_split_path_replays_in_a_graph(gpu):
    # captured in a HIP graph (the split path's stream-ordered allocation and
    # its five launches become graph nodes) and replayed several times, with
    # eager work between the replays: every replay gives the eager tokens
    rng = np.random.default_rng(9)
    B, V = 8, 128256
    lg = torch.from_numpy(_rows(rng, B, V)).to(gpu).to(torch.bfloat16)
    temps = torch.full((B,), 0.9, device=gpu)
    ref = pagedkv.sample(lg, temps, exact=False).clone()
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):               # warm-up on a side stream
        pagedkv.sample(lg, temps, out=out, exact=False)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pagedkv.sample(lg, temps, out=out, exact=False)
    for i in range(4):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        eager = pagedkv.sample(lg[:3], temps[:3], exact=False)
        torch.cuda.synchronize()
        assert torch.equal(eager, ref[:3])


# -- pkv_sample_exact: the reference's f32 arithmetic, bit for bit -----------
def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_expf_on_device_equals_host_libm(gpu):
    # every 64th float from -0.0 to -104 (the exact sampler's arguments are
    # y - max <= 0; below -103.97 the result is 0), every float in [-2^-20,
    # 0] and around the input where an unfused reduction rounds differently,
    # and the special values
    pats = [np.arange(0x80000000, 0xC2D00000, 64, dtype=np.uint64),
            np.arange(0x80000000, 0xB5800000, 977, dtype=np.uint64),
            np.arange(0xC27C65D9 - 4096, 0xC27C65D9 + 4096, dtype=np.uint64),
            np.array([0x00000000, 0x80000000, 0xFF800000, 0xC2CFF1B4, 0xC2CFF1B5], np.uint64)]
    x = np.concatenate(pats).astype(np.uint32).view(np.float32)
    want = oracle.expf_host(x)
    got = pagedkv.sample_expf(torch.from_numpy(x).to(gpu)).cpu().numpy()
    bad = np.flatnonzero(_bits(got) != _bits(want))
    assert bad.size == 0, [(hex(int(_bits(x)[i])), float(got[i]), float(want[i])) for i in bad[:5]]
    assert math.isnan(float(pagedkv.sample_expf(torch.tensor([math.nan], device=gpu)).item()))


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("V", [2, 7, 1000, 32000, 128256])
@pytest.mark.parametrize("top_k,top_p", [(None, None), (40, None), (None, 0.9), (5, 0.5),
                                         (None, 1.0)])
def test_exact_equals_reference_f32(gpu, dt, V, top_k, top_p):
    # every row's token is the f32 restatement's (top_p 1.0 is Some(1.0):
    # it truncates where the f32 running sum reaches 1)
    rng = np.random.default_rng(V + 7 * (top_k or 0) + int(100 * (top_p or 0)))
    kinds = ["normal", "ties", "flat", "spiky"]
    B = 24
    x = np.stack([_logits(rng, kinds[b % 4], V) for b in range(B)])
    lg = torch.from_numpy(x).to(gpu).to(TD[dt])
    x32 = lg.float().cpu().numpy()
    temps = np.array([[0.0, 0.7, 1.0, 1.6, -1.0, 0.3][b % 6] for b in range(B)], np.float32)
    got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), top_k=top_k, top_p=top_p)
    torch.cuda.synchronize()
    want = [oracle.sample(x32[b], float(temps[b]), top_k=top_k, top_p=top_p)[0]
            for b in range(B)]
    assert got.cpu().tolist() == want


def test_exact_follows_f32_rounding_on_flat_rows(gpu):
    # equal logits: the reference's f32 running sum drifts from (k + 1) / V,
    # which moves its pick off the exact-arithmetic one (ceil(r V) - 1); the
    # exact path takes the reference's token, the fast path the other
    for V, f32_pick, exact_pick in ((2616, 349, 348), (3493, 465, 466),
                                    (128256, 17114, 17110), (139990, 18673, 18676)):
        for dt in (torch.float32, torch.bfloat16):
            lg = torch.full((3, V), 1.25, dtype=dt, device=gpu)
            temps = torch.tensor([1.0, 0.5, 3.0], device=gpu)
            assert pagedkv.sample(lg, temps).cpu().tolist() == [f32_pick] * 3, (V, dt)
            assert pagedkv.sample(lg, temps, exact=False).cpu().tolist() == [exact_pick] * 3


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_exact_spiky_and_tied_rows_with_cuts(gpu, dt):
    # a few dominant tokens over a flat or tied tail, with top_k cutting
    # inside a tie group and top_p thresholds the f32 running sum reaches
    # early; every row against the f32 restatement (f32 logits take the
    # radix sort, 16-bit logits the runs of equal values)
    rng = np.random.default_rng(21)
    V, B = 50000, 16
    x = rng.integers(-2, 2, (B, V)).astype(np.float32)
    for b in range(B):
        x[b, rng.integers(0, V, 1 + b % 5)] = 6.0 + (b % 3)
    temps = np.array([0.5, 1.0, 2.0, 4.0] * 4, np.float32)
    lg = torch.from_numpy(x).to(gpu).to(TD[dt])
    x32 = lg.float().cpu().numpy()
    for top_k, top_p in ((None, None), (3, None), (20000, None), (None, 0.5), (None, 0.999),
                         (100, 0.8), (None, 1.0)):
        got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), top_k=top_k, top_p=top_p)
        want = [oracle.sample(x32[b], float(temps[b]), top_k=top_k, top_p=top_p)[0]
                for b in range(B)]
        assert got.cpu().tolist() == want, (top_k, top_p)


def test_exact_batch_over_several_launches(gpu):
    # at most 512 MB of scratch per launch: f32 rows of 2^20 logits take
    # 8 MB each (64 rows per launch), 16-bit rows 1 MB each (512 per launch)
    rng = np.random.default_rng(4)
    B, V = 70, 1 << 20
    lg = torch.randn((B, V), device=gpu) * 2
    temps = torch.from_numpy(rng.choice([0.0, 0.8, 1.0, 1.5], B).astype(np.float32)).to(gpu)
    got = pagedkv.sample(lg, temps).cpu().tolist()
    x32 = lg.cpu().numpy()
    t = temps.cpu().numpy()
    for b in (0, 1, 62, 63, 64, 65, 69):
        assert got[b] == oracle.sample(x32[b], float(t[b]))[0], b
    B, V = 600, 3000
    lg = (torch.randn((B, V), device=gpu) * 2).to(torch.bfloat16)
    temps = torch.from_numpy(rng.choice([0.0, 0.8, 1.0, 1.5], B).astype(np.float32)).to(gpu)
    got = pagedkv.sample(lg, temps).cpu().tolist()
    x32 = lg.float().cpu().numpy()
    t = temps.cpu().numpy()
    for b in (0, 1, 510, 511, 512, 513, 599):
        assert got[b] == oracle.sample(x32[b], float(t[b]))[0], b


def test_exact_f32_rows_of_bf16_values(gpu):
    # f32 logits that are bf16 values (a bf16 model's logits upcast) and
    # genuine f32 logits in one call (buckets first, runs of equal values or
    # the radix sort for the rows they leave): every row equals the f32
    # restatement, and the bf16-valued rows equal the same logits passed as
    # bf16; batches over several launches keep each row's result (70 rows of
    # 2^20: 64 rows per launch)
    rng = np.random.default_rng(17)
    for B, V in ((24, 128256), (70, 1 << 20)):
        x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
        lg = torch.from_numpy(x).to(gpu)
        as_bf16 = lg.to(torch.bfloat16)
        exact_rows = [b for b in range(B) if b % 3 != 1]
        lg[exact_rows] = as_bf16[exact_rows].float()
        if B > 24:
            lg[65, 12345] = 0.1  # one logit with low bits: that row takes the sort
        temps = torch.from_numpy(rng.choice([0.0, 0.7, 1.0, -1.3], B).astype(np.float32)).to(gpu)
        got = pagedkv.sample(lg, temps, top_p=0.95).cpu().tolist()
        x32 = lg.cpu().numpy()
        t = temps.cpu().numpy()
        check = range(B) if B <= 24 else (0, 1, 2, 63, 64, 65, 66, 69)
        for b in check:
            assert got[b] == oracle.sample(x32[b], float(t[b]), top_p=0.95)[0], (B, b)
        via16 = pagedkv.sample(as_bf16, temps, top_p=0.95).cpu().tolist()
        for b in exact_rows:
            if B > 24 and b == 65:
                continue
            assert got[b] == via16[b], (B, b)


def test_exact_16bit_edge_values(gpu):
    # signed zeros (one key), subnormal and largest finite f16 values, and
    # every value of a row equal except one; T < 0 reverses the order
    rows = [[0.0, -0.0, 0.0, -0.0, 1e-7, -1e-7] * 50,
            [65504.0, -65504.0, 6e-8, -6e-8, 0.0] * 40,
            [3.0] * 999 + [3.0009765625]]
    for dt in (torch.float16, torch.bfloat16):
        for T in (1.0, -0.7, 1e-3):
            for r in rows:
                lg = torch.tensor([r], dtype=dt, device=gpu)
                got = int(pagedkv.sample(lg, torch.tensor([T])).item())
                want = oracle.sample(lg.float().cpu().numpy()[0], T)[0]
                assert got == want, (dt, T, r[:6])


def test_exact_replays_in_a_graph(gpu):
    # the stream-ordered scratch allocation and the launch as graph nodes,
    # replayed with eager work in between: every replay gives the eager tokens
    rng = np.random.default_rng(10)
    B, V = 8, 128256
    lg = torch.from_numpy(_rows(rng, B, V)).to(gpu).to(torch.bfloat16)
    temps = torch.full((B,), 0.9, device=gpu)
    ref = pagedkv.sample(lg, temps).clone()
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pagedkv.sample(lg, temps, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pagedkv.sample(lg, temps, out=out)
    for i in range(3):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        eager = pagedkv.sample(lg[:3], temps[:3])
        torch.cuda.synchronize()
        assert torch.equal(eager, ref[:3])
    x32 = lg.float().cpu().numpy()
    assert ref.cpu().tolist() == [oracle.sample(x32[b], 0.9)[0] for b in range(B)]


# -- f32 logits on buckets of y (sample_bucket_kernel) -------------------------
ROUTE_ARGMAX, ROUTE_BUCKETS, ROUTE_RUNS, ROUTE_SORT = 0, 1, 2, 3


def _sample_routes(lg, temps, **kw):
    routes = torch.full((lg.shape[0],), -1, dtype=torch.int32, device=lg.device)
    tok = pagedkv.sample(lg, temps, routes=routes, **kw)
    return tok.cpu().tolist(), routes.cpu().tolist()


def _f32_rows(rng, B, V):
    """Genuine f32 logits (low bits set) of several shapes."""
    rows = []
    for b in range(B):
        kind = b % 7
        if kind == 0:
            x = rng.standard_normal(V) * [0.5, 3.0, 10.0][(b // 7) % 3]
        elif kind == 1:  # a language model's: a flat bulk and a few strong tokens
            x = rng.standard_normal(V) * 2.5
            x[rng.integers(0, V, 5)] = rng.uniform(15, 25, 5)
        elif kind == 2:  # one very low logit stretches the range
            x = rng.standard_normal(V) * 3
            x[rng.integers(0, V)] = -1e4
        elif kind == 3:  # half the vocabulary masked
            x = rng.standard_normal(V) * 3
            x[rng.permutation(V)[:V // 2]] = -np.inf
        elif kind == 4:  # a narrow range
            x = rng.uniform(-1, 1, V)
        elif kind == 5:  # heavy tail towards the top
            x = rng.gumbel(0, 2, V)
        else:            # few distinct values: ties inside buckets
            x = rng.integers(-40, 40, V) * 0.173
        rows.append(x.astype(np.float32))
    return np.stack(rows)


def _expected_routes(temps):
    # greedy rows: argmax; half the vocabulary at -inf (row kind 3) with T < 0:
    # max y is +inf, left to the sort; every other row: the buckets
    return [ROUTE_ARGMAX if t == 0 else ROUTE_SORT if b % 7 == 3 and t < 0 else ROUTE_BUCKETS
            for b, t in enumerate(temps)]


@pytest.mark.parametrize("top_k,top_p", [(None, None), (50, None), (3000, None), (None, 0.9),
                                         (None, 0.3), (200, 0.95), (None, 1.0), (1, None)])
def test_exact_f32_buckets_equal_reference(gpu, top_k, top_p):
    # every sampled f32 row is selected by the bucket kernel (none left to the
    # sort), and each token is the f32 restatement's
    rng = np.random.default_rng(31 + (top_k or 0) + int(100 * (top_p or 0)))
    B, V = 28, 128256
    x = _f32_rows(rng, B, V)
    temps = np.array([[0.8, 1.0, 0.3, -1.1, 1.7, 0.0, 5.0, 0.05][b % 8] for b in range(B)],
                     np.float32)
    lg = torch.from_numpy(x).to(gpu)
    got, routes = _sample_routes(lg, torch.from_numpy(temps).to(gpu), top_k=top_k, top_p=top_p)
    want = [oracle.sample(x[b], float(temps[b]), top_k=top_k, top_p=top_p)[0] for b in range(B)]
    assert got == want
    expect = _expected_routes(temps)
    assert routes == expect, [(b, routes[b], expect[b]) for b in range(B) if routes[b] != expect[b]]


@pytest.mark.parametrize("V", [2, 3, 7, 64, 1000, 4097, 50000])
def test_exact_f32_buckets_small_vocab(gpu, V):
    rng = np.random.default_rng(V)
    B = 21
    x = _f32_rows(rng, B, V)
    temps = np.array([[0.8, 1.0, 0.3, -1.1, 1.7, 5.0, 0.05][b % 7] for b in range(B)], np.float32)
    lg = torch.from_numpy(x).to(gpu)
    for top_k, top_p in ((None, None), (2, None), (None, 0.5)):
        got, routes = _sample_routes(lg, torch.from_numpy(temps).to(gpu), top_k=top_k,
                                     top_p=top_p)
        want = [oracle.sample(x[b], float(temps[b]), top_k=top_k, top_p=top_p)[0]
                for b in range(B)]
        assert got == want, (top_k, top_p)
        assert routes == _expected_routes(temps), routes


def test_exact_f32_rows_the_buckets_leave(gpu):
    # rows the bucket kernel leaves to the later kernels, with the reference's
    # tokens: all logits equal (one bucket of 60,000), a dense cluster of
    # 10,000 distinct values at the top (a top bucket above the 4,096 logits
    # kept in LDS), the same cluster of bf16 values (runs of equal values),
    # and a NaN (outside the contract: a token in range, from the sort); a
    # cluster of 3,000 stays on the buckets
    rng = np.random.default_rng(5)
    V = 60000
    flat = np.full(V, 0.7310585, np.float32)
    cluster = (rng.standard_normal(V) * 3).astype(np.float32)
    cluster[:10000] = (20.0 + rng.uniform(0, 1e-3, 10000)).astype(np.float32)
    cl16 = torch.from_numpy(cluster).to(torch.bfloat16).float().numpy()
    cl16[:10000] = 20.0
    small = cluster.copy()
    small[3000:10000] = (rng.standard_normal(7000) * 3).astype(np.float32)
    nanrow = (rng.standard_normal(V) * 3).astype(np.float32)
    nanrow[123] = np.nan
    x = np.stack([flat, cluster, cl16, nanrow, small])
    temps = torch.tensor([1.0, 0.9, 0.9, 1.0, 0.9], device=gpu)
    got, routes = _sample_routes(torch.from_numpy(x).to(gpu), temps)
    assert routes == [ROUTE_SORT, ROUTE_SORT, ROUTE_RUNS, ROUTE_SORT, ROUTE_BUCKETS], routes
    for b in (0, 1, 2, 4):
        assert got[b] == oracle.sample(x[b], float(temps[b]))[0], b
    assert 0 <= got[3] < V


def test_exact_f32_buckets_agree_with_the_sort_on_shuffled_rows(gpu):
    # the same logits in another order give the token at the same sorted
    # position (positions of equal logits aside): bucket scatter order and
    # atomics do not leak into the result
    rng = np.random.default_rng(8)
    V, B = 128256, 8
    base = (rng.standard_normal(V) * 3).astype(np.float32)
    perms = [rng.permutation(V) for _ in range(B)]
    x = np.stack([base[p] for p in perms])
    temps = torch.full((B,), 0.8, device=gpu)
    got, routes = _sample_routes(torch.from_numpy(x).to(gpu), temps, top_p=0.9)
    assert set(routes) == {ROUTE_BUCKETS}
    picked = {float(base[perms[b][got[b]]]) for b in range(B)}
    assert len(picked) == 1, picked
    assert got == [oracle.sample(x[b], 0.8, top_p=0.9)[0] for b in range(B)]
