"""Token scoring, deterministic top-k and gather attention vs the CPU oracle.

Scores and attention outputs: north_star tolerance (fp32 scores compared to
1e-3 absolute); top-k indices: bit-exact against the oracle run on the same
fp32 scores.
"""
import math

import pytest
import torch

from bytes_amd import sparse as SP
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
SCORE_TOL = 1e-3
pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


@pytest.mark.parametrize("B,Hq,Hk,S,D", [(2, 8, 2, 1000, 128), (1, 24, 8, 4099, 128), (2, 4, 4, 300, 64),
                                          (1, 40, 2, 777, 128)])
def test_score_per_head(dev, B, Hq, Hk, S, D):
    x = W.dense(B, Hq, Hk, D, S, seed=S)
    s = SP.sparse_score_scalar(x["q"].to(dev), x["k"].to(dev), 0.088)
    ref = R.sparse_score_scalar(x["q"], x["k"], 0.088)
    assert s.shape == (B, Hq, S) and s.dtype == torch.float32
    assert (s.cpu() - ref).abs().max() <= SCORE_TOL


@pytest.mark.parametrize("B,Hq,Hk,S", [(2, 24, 8, 5000), (1, 4, 1, 129), (1, 32, 2, 1024)])
def test_group_scores(dev, B, Hq, Hk, S):
    x = W.dense(B, Hq, Hk, 128, S, seed=S + 1)
    s = SP.group_scores(x["q"].to(dev), x["k"].to(dev), 0.088)
    ref = R.group_scores(x["q"], x["k"], 0.088)
    assert s.shape == (B, Hk, S)
    assert (s.cpu() - ref).abs().max() <= SCORE_TOL


def test_group_scores_long_ragged(dev):
    """A cache long enough that each wave of the score pass runs several
    iterations and stores whole batches of group sums, with a ragged last
    range (S = 200003), plain and with the fused selection histogram of the
    top-k pipeline: scores against the oracle, the pipeline's selection
    bit-exact against the oracle's top-k on the same scores."""
    B, Hq, Hk, S = 2, 24, 8, 200003
    x = W.dense(B, Hq, Hk, 128, S, seed=5)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    s = SP.group_scores(q, k, 0.088)
    ref = R.group_scores(x["q"], x["k"], 0.088)
    assert (s.cpu() - ref).abs().max() <= SCORE_TOL
    _, idx = SP.token_topk_decode(q, k, v, 1024, 0.088)
    assert torch.equal(idx.cpu().long(), R.topk_indices(s.cpu(), 1024, sorted_by_score=False))


@pytest.mark.parametrize("fp8,D", [(True, 128), (False, 64)])
def test_score_per_head_full_lds_buffer(dev, fp8, D):
    """Per-head scores (16 query heads on one KV head) on a row long enough
    that, on 256 CUs, each score workgroup's token range is the largest its
    LDS score buffer holds for 16 head rows (768 tokens for fp8 keys and for
    D = 64), with a ragged end: slices at the start, across workgroup
    boundaries and at the end against the oracle (fp8 keys widened to bf16,
    which is exact)."""
    B, Hq, Hk = 1, 16, 1
    S = 2048 * 768 + 555
    g = torch.Generator(device=dev).manual_seed(17)
    q = torch.randn(B, Hq, 1, D, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(B, Hk, S, D, device=dev, generator=g, dtype=torch.bfloat16)
    if fp8:
        k = k.to(torch.float8_e4m3fn)
    s = SP.sparse_score_scalar(q, k, 0.088, score_bits=8 if fp8 else 16)
    assert s.shape == (B, Hq, S)
    qc = q.cpu()
    for a, b in ((0, 2000), (768 - 300, 768 + 300), (7 * 768 - 200, 7 * 768 + 200), (S - 3000, S)):
        ks = k[:, :, a:b].cpu()
        ref = R.sparse_score_scalar(qc, ks.to(torch.bfloat16) if fp8 else ks, 0.088)
        d = (s[:, :, a:b].cpu() - ref).abs().max().item()
        print(f"tokens {a}..{b}: max-abs {d:.3e}", flush=True)
        assert d <= SCORE_TOL, (a, b)
    del k, s
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fp8", [False, True])
def test_group_scores_full_lds_buffer(dev, fp8):
    """Rows long enough that, on 256 CUs, each score workgroup's token range
    is the largest its LDS score buffer holds (6144 tokens with bf16 keys,
    8192 with fp8), with a ragged end: group sums at the start, across
    workgroup boundaries and at the end of every row against the oracle on
    those key slices (fp8 keys widened to bf16, which is exact)."""
    B, Hq, Hk, D = 1, 24, 8, 128
    cap = 8192 if fp8 else 6144
    S = 2048 * cap // Hk + 1001
    g = torch.Generator(device=dev).manual_seed(11)
    q = torch.randn(B, Hq, 1, D, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(B, Hk, S, D, device=dev, generator=g, dtype=torch.bfloat16)
    if fp8:
        k = k.to(torch.float8_e4m3fn)
    s = SP.group_scores(q, k, 0.088)
    assert s.shape == (B, Hk, S)
    qc = q.cpu()
    for a, b in ((0, 3000), (cap - 700, cap + 700), (5 * cap - 300, 5 * cap + 300), (S - 4000, S)):
        ks = k[:, :, a:b].cpu()
        ref = R.group_scores(qc, ks.to(torch.bfloat16) if fp8 else ks, 0.088)
        d = (s[:, :, a:b].cpu() - ref).abs().max().item()
        print(f"tokens {a}..{b}: max-abs {d:.3e}", flush=True)
        assert d <= SCORE_TOL, (a, b)
    del k, s
    torch.cuda.empty_cache()


def _tie_heavy(rows, n, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.randint(-8, 8, (rows, n), generator=g).float() * 0.25      # many exact ties
    s[0, ::7] = 0.0
    s[0, 1::7] = -0.0
    if rows > 1:
        s[1, 5] = float("nan")
        s[1, 9] = float("-nan")
        s[1, 11] = float("inf")
        s[1, 12] = float("-inf")
    return s


@pytest.mark.parametrize("sorted_out", [True, False])
@pytest.mark.parametrize("rows,n,k", [(3, 1000, 1), (3, 1000, 17), (4, 4096, 256), (2, 1001, 1001),
                                      (5, 333, 100), (28, 2048, 128), (2, 20000, 8192), (3, 70000, 3000),
                                      (1100, 17000, 100)])
def test_topk_bit_exact_with_ties(dev, rows, n, k, sorted_out):
    s = _tie_heavy(rows, n, seed=n + k)
    got = SP.topk_indices(s.to(dev), k, sorted=sorted_out).cpu()
    ref = R.topk_indices(s, k, sorted_by_score=sorted_out)
    assert got.dtype == torch.int32
    assert torch.equal(got.long(), ref)


@pytest.mark.parametrize("rows,n,k", [(3, 40000, 10000), (2, 65536, 16384), (2, 9000, 9000), (130, 20000, 12000),
                                      (2, 131072, 32768), (3, 20000, 8193)])
def test_topk_large_k(dev, rows, n, k):
    """k above 8192: the same set by ascending index (sorted=False), and in the
    total order (sorted=True: blocks of 8192 sorted in LDS, merged by rank),
    both bit-exact against the oracle on tie-heavy rows."""
    s = _tie_heavy(rows, n, seed=n + k)
    got = SP.topk_indices(s.to(dev), k, sorted=False).cpu()
    assert torch.equal(got.long(), R.topk_indices(s, k, sorted_by_score=False))
    got_s = SP.topk_indices(s.to(dev), k, sorted=True).cpu()
    assert torch.equal(got_s.long(), R.topk_indices(s, k, sorted_by_score=True))


@pytest.mark.parametrize("k", [8193, 13107, 32768, 65536, 131071])
def test_topk_large_k_c5_rows(dev, k):
    """k above 8192 on the C5 row shape (64 x 131072): threshold-digit
    candidates, per-row selection and per-slice ordered writes, with a tied
    block at the threshold, a row of rounded (heavily tied) scores and a row
    whose keys share one top digit (the whole-row exact fallback)."""
    g = torch.Generator().manual_seed(k)
    s = torch.randn(64, 131072, generator=g)
    s[3, 1000:1100] = 5.0
    s[5, :] = s[5, :].round()
    s[7, :] = 1.0 + torch.rand(131072, generator=g) * 0.2    # one top digit for every key
    got = SP.topk_indices(s.to(dev), k, sorted=False).cpu().long()
    assert torch.equal(got, R.topk_indices(s, k, sorted_by_score=False))


def test_topk_large_k_row_batches(dev):
    """More rows than one launch group (1024) with k above 8192."""
    s = _tie_heavy(1100, 20000, seed=1)
    got = SP.topk_indices(s.to(dev), 9000, sorted=False).cpu().long()
    assert torch.equal(got, R.topk_indices(s, 9000, sorted_by_score=False))


@pytest.mark.parametrize("sorted_out", [True, False])
@pytest.mark.parametrize("rows,n,k", [(600, 2048, 128), (600, 1000, 1), (300, 4096, 256), (700, 2051, 17),
                                      (260, 64, 64), (1000, 4095, 200)])
def test_topk_many_short_rows(dev, rows, n, k, sorted_out):
    """More rows than CUs with n <= 4096 and k <= 256: the one-wave-per-row
    selection (ties, +-0, NaN, +-inf and all-equal rows included)."""
    s = _tie_heavy(rows, n, seed=n + k + rows)
    s[2] = 0.5                                             # an all-equal row
    s[3, : n // 2] = float("inf")                          # more infinities than k
    got = SP.topk_indices(s.to(dev), k, sorted=sorted_out).cpu()
    assert torch.equal(got.long(), R.topk_indices(s, k, sorted_by_score=sorted_out))


@pytest.mark.parametrize("rows,n,k", [(1, 1, 1), (1, 3, 2), (5, 64, 64), (28, 2048, 1024), (3, 4096, 4096),
                                      (4, 4096, 1024), (2, 3000, 2000), (280, 1500, 512), (7, 4095, 1)])
def test_topk_small_rows(dev, rows, n, k):
    """Rows of at most 4096 elements outside the one-wave path: one 256-thread
    workgroup per row (sorted output up to k = 1024; larger sorted k takes the
    whole-row sort)."""
    s = _tie_heavy(rows, n, seed=3 * n + k)
    if rows > 3:
        s[2] = -1.5                                          # an all-equal row
        s[3, : n // 2] = float("-inf")
        s[3, n // 2:] = float("inf")
    for so in (True, False):
        got = SP.topk_indices(s.to(dev), k, sorted=so).cpu()
        assert torch.equal(got.long(), R.topk_indices(s, k, sorted_by_score=so)), so
    big = torch.zeros(rows * n + 1)
    big[1:] = s.reshape(-1)
    view = big.to(dev)[1:].reshape(rows, n)                  # rows not 16-byte aligned
    assert torch.equal(SP.topk_indices(view, k, sorted=False).cpu().long(),
                       R.topk_indices(s, k, sorted_by_score=False))


@pytest.mark.parametrize("rows,n,k,shift", [(16, 3000, 150, 0.0), (16, 3000, 750, 0.0), (28, 2048, 128, 0.0),
                                            (4, 1000, 999, 0.0), (28, 2048, 128, 40.0), (8, 4096, 1, 0.0)])
def test_topk_small_rows_continuous(dev, rows, n, k, shift):
    """Rows of distinct continuous scores (and the same shifted far from zero,
    as page bounds sit): the digit pass that reaches a crossing bin of a few
    keys ranks those keys directly; the result must equal the oracle's."""
    g = torch.Generator().manual_seed(rows * n + k)
    s = torch.randn(rows, n, generator=g) + shift
    for so in (True, False):
        got = SP.topk_indices(s.to(dev), k, sorted=so).cpu()
        assert torch.equal(got.long(), R.topk_indices(s, k, sorted_by_score=so)), so


@pytest.mark.parametrize("rows,n,k", [(300, 2048, 128), (28, 2048, 128), (280, 4096, 600), (5, 1000, 17)])
def test_topk_narrow_range_rows(dev, rows, n, k):
    """Scores in a narrow range (every key shares its top bits; the digit
    passes start below them), with exact ties and an all-equal row, on the
    one-wave path (more rows than CUs, k <= 256) and the workgroup path."""
    g = torch.Generator().manual_seed(rows + n + k)
    s = 3.0 + torch.rand(rows, n, generator=g) * 0.5
    s[0, 10:40] = 3.25                                       # a block of exact ties
    s[1] = 3.125                                             # an all-equal row
    if n > 100:
        s[2, :5] = 3.0 + 2.0 ** -20                          # keys one ulp-scale apart
    for so in (True, False):
        got = SP.topk_indices(s.to(dev), k, sorted=so).cpu()
        assert torch.equal(got.long(), R.topk_indices(s, k, sorted_by_score=so)), so


def test_topk_many_short_rows_unaligned(dev):
    s = _tie_heavy(400, 1500, seed=11)
    big = torch.zeros(400 * 1500 + 1)
    big[1:] = s.reshape(-1)
    view = big.to(dev)[1:].reshape(400, 1500)              # rows not 16-byte aligned
    for srt in (True, False):
        assert torch.equal(SP.topk_indices(view, 100, sorted=srt).cpu().long(),
                           R.topk_indices(s, 100, sorted_by_score=srt))


def test_topk_unaligned_rows(dev):
    s = _tie_heavy(6, 2051, seed=3)
    big = torch.zeros(6 * 2051 + 1)
    big[1:] = s.reshape(-1)
    view = big.to(dev)[1:].reshape(6, 2051)                # rows not 16-byte aligned
    assert torch.equal(SP.topk_indices(view, 300).cpu().long(), R.topk_indices(s, 300))


@pytest.mark.parametrize("case", ["narrow", "all_equal"])
def test_topk_crowded_digit_rows(dev, case):
    """Every key of a row shares its top 11 bits: the candidate list overflows and
    the whole-row exact selection runs."""
    g = torch.Generator().manual_seed(5)
    if case == "narrow":
        s = 1.0 + torch.rand(3, 20000, generator=g) * 0.2
        s[1, 7777] = 1.1                                      # plus exact ties
        s[1, 7778] = 1.1
    else:
        s = torch.full((3, 20000), 0.5)
    for k in (1, 100, 8192):
        for so in (True, False):
            got = SP.topk_indices(s.to(dev), k, sorted=so).cpu().long()
            assert torch.equal(got, R.topk_indices(s, k, sorted_by_score=so)), (case, k, so)


@pytest.mark.parametrize("k", [256, 1024, 4096])
def test_topk_c5_rows(dev, k):
    """64 rows x 131072 fp32 (BASELINE C5 selection shape)."""
    g = torch.Generator().manual_seed(k)
    s = torch.randn(64, 131072, generator=g)
    s[3, 1000:1100] = 5.0                                   # a tied block straddling the boundary
    s[5, :] = s[5, :].round()                               # heavy ties at the threshold
    for so in (True, False):
        got = SP.topk_indices(s.to(dev), k, sorted=so).cpu().long()
        assert torch.equal(got, R.topk_indices(s, k, sorted_by_score=so)), so


def _gather_case(dev, B, Hq, Hk, S, D, kb, per_head, seed, chunk=0):
    x = W.dense(B, Hq, Hk, D, S, seed=seed)
    g = torch.Generator().manual_seed(seed)
    H = Hq if per_head else Hk
    idx = torch.randint(0, S, (B, H, kb), generator=g)
    idx[..., ::13] = -1                                     # masked entries
    idx[..., 1::29] = S                                     # sentinel (unfilled slot)
    if kb > 4:
        idx[..., 2] = idx[..., 4]                           # a repeated row counts twice
    out = SP.sparse_gather_attn(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), idx.to(dev), 0.09, chunk=chunk)
    ref = R.sparse_gather_attn(x["q"], x["k"], x["v"], idx, 0.09)
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.bfloat16
    _check(out, ref, f"gather B{B} Hq{Hq} Hk{Hk} S{S} D{D} kb{kb} per_head{per_head} chunk{chunk}")


@pytest.mark.parametrize("B,Hq,Hk,S,D,kb", [(2, 8, 2, 2000, 128, 100), (1, 24, 8, 5000, 128, 1000),
                                             (1, 7, 1, 300, 64, 31), (2, 28, 4, 4096, 128, 2048)])
@pytest.mark.parametrize("per_head", [1, 0])
def test_gather_matches_oracle(dev, B, Hq, Hk, S, D, kb, per_head):
    _gather_case(dev, B, Hq, Hk, S, D, kb, per_head, seed=kb + per_head)


@pytest.mark.parametrize("chunk", [128, 1024])
def test_gather_split_counts(dev, chunk):
    _gather_case(dev, 1, 8, 2, 40000, 128, 37000, 0, seed=7, chunk=chunk)     # 290 / 37 splits


def test_gather_single_valid_row(dev):
    x = W.dense(1, 4, 1, 128, 64, seed=1)
    idx = torch.full((1, 1, 40), -1)
    idx[0, 0, 17] = 5
    out = SP.sparse_gather_attn(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), idx.to(dev), 0.1)
    # one row survives the mask: the output is that value row for every head
    assert torch.allclose(out.cpu().float()[0, :, 0], x["v"][0, 0, 5].float().expand(4, -1), atol=1e-2)


@pytest.mark.parametrize("frac", [0.05, 0.25])
def test_sparse_decode_scalar_pipeline(dev, frac):
    x = W.dense(2, 8, 2, 128, 3000, seed=11)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    sc = 1 / math.sqrt(128)
    out = SP.sparse_decode_scalar(q, k, None, None, k, v, frac, sc, score_bits=16)
    ref = R.sparse_decode_scalar(x["q"], x["k"], x["k"], x["v"], frac, sc)
    _check(out, ref, f"sparse_decode_scalar frac {frac}")
    # selection is bit-exact given the same fp32 scores
    s = SP.sparse_score_scalar(q, k, sc)
    kb = SP.budget(frac, 3000)
    assert torch.equal(SP.topk_indices(s, kb).cpu().long(), R.topk_indices(s.cpu(), kb))


@pytest.mark.parametrize("kb", [256, 1024, 4096, 32768])
def test_token_topk_c5_full(dev, kb):
    """BASELINE C5 at full size: B8 Hq24 Hkv8 D128 L131072."""
    x = W.c5_topk(seed=0, device=dev)
    q, k, v = x["q"], x["k"], x["v"]
    sc = x["scale"]
    out, idx = SP.token_topk_decode(q, k, v, kb, sc)
    # scores of batch 0 against the oracle
    s = SP.group_scores(q, k, sc)
    ref_s0 = R.group_scores(q[:1].cpu(), k[:1].cpu(), sc)
    assert (s[:1].cpu() - ref_s0).abs().max() <= SCORE_TOL
    # selection bit-exact on the same scores (the pipeline returns the set by ascending index)
    ref_idx = R.topk_indices(s.cpu(), kb, sorted_by_score=False)
    assert torch.equal(idx.cpu().long(), ref_idx)
    # attention over the selected rows: dense oracle on the gathered rows
    B, Hk = k.shape[:2]
    gi = idx.long().unsqueeze(-1).expand(B, Hk, kb, k.shape[-1])
    ks, vs = torch.gather(k, 2, gi).cpu(), torch.gather(v, 2, gi).cpu()
    _check(out, R.decode_attn(q.cpu(), ks, vs, scale=sc), f"C5 kb{kb}")
