"""GPU parity of token selection (pkv_sample) against the CPU oracle's
restatement of sample() / argmax() (crates/ai-engine-runtime/src/sample.rs:
12-55).  Greedy rows are exact.  The kernel sums probability mass exactly
(integers), so sampled rows are compared with the oracle's restatement in
exact arithmetic (float64 exp and running sums over the reference's f32
values): the token must be equal unless that restatement's running sum lies
within 1e-6 of r or top_p.  Against the oracle's f32 restatement (the
reference's own rounding), a row may differ only where that rounding alone
moves the pick, i.e. where the f32 and float64 restatements differ."""
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


def test_reference_kats_on_device(gpu):
    cases = [([0.1, 5.0, 2.0, -1.0], 0.0, None, None, 1),
             ([1.0, 5.0, 2.0], 0.0, None, None, 1),
             ([1.0, 1.0, 1.0, 1.0, 100.0], 1.0, 1, None, 4),
             ([1.0, 1.0, 100.0, 1.0], 1.0, None, 0.5, 2)]
    for x, t, k, p, want in cases:
        lg = torch.tensor([x], dtype=torch.float32, device=gpu)
        tok = pagedkv.sample(lg, torch.tensor([t]), top_k=k, top_p=p, seed=0)
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
    got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu), top_k=top_k, top_p=top_p)
    torch.cuda.synchronize()
    _check_rows(x32, temps, top_k, top_p, got.cpu().numpy())


def test_uniform_rows_closed_form(gpu):
    # equal logits keep index order: the pick is floor(r V)
    r = pagedkv.sample_draw(42)
    for V in (10, 100, 1000, 4096, 50000):
        lg = torch.zeros((3, V), dtype=torch.bfloat16, device=gpu)
        tok = pagedkv.sample(lg, torch.tensor([1.0, 0.5, 2.0]))
        assert tok.cpu().tolist() == [math.floor(r * V)] * 3
    lg = torch.zeros((1, 1000), device=gpu)
    assert int(pagedkv.sample(lg, torch.tensor([1.0]), top_k=10).item()) == math.floor(10 * r)
    assert int(pagedkv.sample(lg, torch.tensor([1.0]), top_p=0.5).item()) == math.floor(500 * r)


def test_greedy_rules_on_device(gpu):
    nan, inf = math.nan, math.inf
    rows = [[1.0, 5.0, 5.0, 2.0], [nan, 1.0, 3.0, 3.0], [-inf, -inf, -inf, -inf],
            [nan, -inf, nan, nan], [2.0, nan, 2.0, 9.0]]
    lg = torch.tensor(rows, device=gpu)
    tok = pagedkv.sample(lg)                 # no temperatures: every row greedy
    assert tok.cpu().tolist() == [oracle.argmax(r) for r in rows] == [1, 2, 0, 0, 3]
    # one logit: argmax even when sampling; no logits: token 0
    assert int(pagedkv.sample(torch.tensor([[4.0]], device=gpu), torch.tensor([1.0])).item()) == 0
    assert int(pagedkv.sample(torch.zeros((1, 0), device=gpu)).item()) == 0
    # a large greedy row: first maximum by index
    x = torch.randn((4, 128256), device=gpu)
    x[:, 77777] = 50.0
    x[:, 99999] = 50.0
    assert pagedkv.sample(x).cpu().tolist() == [77777] * 4


def test_strided_rows_and_determinism(gpu):
    rng = np.random.default_rng(3)
    big = torch.from_numpy(rng.standard_normal((16, 40000)).astype(np.float32)).to(gpu)
    lg = big[:, 1000:33000]                  # row stride 40000, vocab 32000
    temps = torch.full((16,), 0.8)
    a = pagedkv.sample(lg, temps)
    b = pagedkv.sample(lg, temps)
    assert torch.equal(a, b)
    _check_rows(lg.cpu().numpy(), temps.numpy(), None, None, a.cpu().numpy())


def test_seed_changes_draw(gpu):
    lg = torch.zeros((1, 1000), device=gpu)
    for seed in (0, 1, 42, 12345):
        tok = int(pagedkv.sample(lg, torch.tensor([1.0]), seed=seed).item())
        assert tok == math.floor(pagedkv.sample_draw(seed) * 1000)


def test_invalid_arguments(gpu):
    lg = torch.zeros((2, 10), device=gpu)
    with pytest.raises(pagedkv.PagedKvError):
        pagedkv.sample(lg, torch.ones(2), top_k=-1)


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
    small = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu))
    big = pagedkv.sample(lg.repeat(16, 1), torch.from_numpy(np.tile(temps, 16)).to(gpu))
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
    got = pagedkv.sample(lg, torch.from_numpy(temps).to(gpu))
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
    assert pagedkv.sample(x, temps).cpu().tolist() == [0, 4095, 4096, 65000, 128255, 100]


def test_split_path_replays_in_a_graph(gpu):
    # captured in a HIP graph (the split path's stream-ordered allocation and
    # its five launches become graph nodes) and replayed several times, with
    # eager work between the replays: every replay gives the eager tokens
    rng = np.random.default_rng(9)
    B, V = 8, 128256
    lg = torch.from_numpy(_rows(rng, B, V)).to(gpu).to(torch.bfloat16)
    temps = torch.full((B,), 0.9, device=gpu)
    ref = pagedkv.sample(lg, temps).clone()
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):               # warm-up on a side stream
        pagedkv.sample(lg, temps, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pagedkv.sample(lg, temps, out=out)
    for i in range(4):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        eager = pagedkv.sample(lg[:3], temps[:3])
        torch.cuda.synchronize()
        assert torch.equal(eager, ref[:3])
