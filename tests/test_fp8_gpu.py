"""OCP float8_e4m3fn paths vs the CPU oracle: dense fp8 decode, fp8 score keys,
fp8 gathered values, and the fp8 two-pass sparse decode."""
import math

import pytest
import torch

from bytes_amd import attention_kernels as AK
from bytes_amd import sparse as SP
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
SCORE_TOL = 1e-3
F8 = torch.float8_e4m3fn
pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


@pytest.mark.parametrize("B,Hq,Hk,S,D,scale", [
    (2, 8, 2, 128, 64, 1.0),              # benchmarks/test_correctness.py:82-115 shape, no scale
    (1, 14, 2, 8192, 64, 0.125),          # C1 shape
    (4, 28, 4, 16384, 128, 1 / math.sqrt(128)),
    (1, 7, 1, 77, 128, 0.3),              # ragged
])
def test_decode_attn_fp8(dev, B, Hq, Hk, S, D, scale):
    x = W.dense(B, Hq, Hk, D, S, seed=S)
    k8, v8 = x["k"].to(F8), x["v"].to(F8)
    out = AK.decode_attn_fp8(x["q"].to(dev), k8.to(dev), v8.to(dev), scale)
    assert out.dtype == torch.bfloat16 and out.shape == (B, Hq, 1, D)
    _check(out, R.decode_attn(x["q"], k8, v8, scale=scale, out_dtype=torch.bfloat16), f"fp8 S{S}")


def test_fp8_every_code_scores_exactly(dev):
    """Each of the 254 finite e4m3fn codes as a key entry: the score equals the
    fp32 product computed on the CPU (the widening to bf16 is exact)."""
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[~torch.isnan(codes.view(F8).float())]
    n = codes.numel()
    k = torch.zeros(1, 1, n, 128, dtype=torch.uint8)
    k[0, 0, :, 5] = codes
    q = torch.zeros(1, 1, 1, 128, dtype=torch.bfloat16)
    q[0, 0, 0, 5] = 1.0
    s = SP.sparse_score_scalar(q.to(dev), k.view(F8).to(dev), 1.0, score_bits=8).cpu()
    assert torch.equal(s[0, 0], codes.view(F8).float())


@pytest.mark.parametrize("B,Hq,Hk,S,D", [(2, 8, 2, 1000, 128), (1, 24, 8, 4099, 128), (2, 4, 4, 300, 64)])
def test_fp8_scores(dev, B, Hq, Hk, S, D):
    x = W.dense(B, Hq, Hk, D, S, seed=S)
    k8 = x["k"].to(F8)
    s = SP.sparse_score_scalar(x["q"].to(dev), k8.to(dev), 0.088, score_bits=8)
    assert (s.cpu() - R.sparse_score_scalar(x["q"], k8, 0.088)).abs().max() <= SCORE_TOL
    g = SP.group_scores(x["q"].to(dev), k8.to(dev), 0.088)
    assert (g.cpu() - R.group_scores(x["q"], k8, 0.088)).abs().max() <= SCORE_TOL


@pytest.mark.parametrize("per_head", [1, 0])
def test_fp8_gather(dev, per_head):
    x = W.dense(1, 24, 8, 128, 5000, seed=9)
    k8, v8 = x["k"].to(F8), x["v"].to(F8)
    g = torch.Generator().manual_seed(9)
    idx = torch.randint(0, 5000, (1, 24 if per_head else 8, 700), generator=g)
    idx[..., ::17] = -1
    out = SP.sparse_gather_attn(x["q"].to(dev), k8.to(dev), v8.to(dev), idx.to(dev), 0.09)
    assert out.dtype == torch.bfloat16
    _check(out, R.sparse_gather_attn(x["q"], k8, v8, idx, 0.09), f"fp8 gather per_head={per_head}")


@pytest.mark.parametrize("frac", [0.05, 0.25])
def test_sparse_decode_fp8_scores(dev, frac):
    """The two-pass path with fp8 score keys and bf16 values
    (benchmarks/test_correctness.py:740-800, bits = 8)."""
    x = W.dense(2, 8, 2, 128, 3000, seed=12)
    k8 = x["k"].to(F8)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    sc = 1 / math.sqrt(128)
    out = SP.sparse_decode_scalar(q, k8.to(dev), None, None, k, v, frac, sc, score_bits=8)
    s = SP.sparse_score_scalar(q, k8.to(dev), sc, score_bits=8)
    kb = SP.budget(frac, 3000)
    idx = SP.topk_indices(s, kb, sorted=False)
    assert torch.equal(idx.cpu().long(), R.topk_indices(s.cpu(), kb, sorted_by_score=False))
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], idx.cpu().long(), sc), f"fp8-score decode {frac}")
