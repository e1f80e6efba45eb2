"""Outlier-aware (asymmetric) PQ-LUT decode, the paged PQ decodes, LUT+outlier
scoring and the PQ sparse decode vs the CPU oracle
(src/attention_kernels.py:505-984, :1062-1074; shapes of
benchmarks/test_correctness.py:393-594)."""
import math

import pytest
import torch

from bytes_amd import pq as PQ
from bytes_amd import sparse as SP
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
F8 = torch.float8_e4m3fn
pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


def _asym_inputs(B, Hq, Hk, S, D, C, K, seed, v_dtype=torch.bfloat16):
    """LUT from a random codebook (the test's einsum), random codes, outlier
    channels an order of magnitude larger than the rest, bf16/fp8 values."""
    g = torch.Generator().manual_seed(seed)
    M = D // 8
    cb = torch.randn(M, K, 8, generator=g)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    lut = R.pq_build_lut(q, cb, 1.0 / math.sqrt(D))
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g, dtype=torch.uint8)
    k_out = ((torch.randn(B, Hk, S, C, generator=g) + 3.0) * 2.0).to(torch.bfloat16)
    q_out = (torch.randn(B, Hq, C, generator=g) * 0.2).to(torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g).to(v_dtype)
    return lut, k_idx, k_out, q_out, v


@pytest.mark.parametrize("B,Hq,Hk,S,D,C,v_dtype", [
    (2, 8, 2, 128, 64, 2, torch.bfloat16),        # benchmarks/test_correctness.py:403-408 cases
    (2, 8, 2, 128, 64, 2, F8),
    (1, 4, 1, 64, 128, 1, F8),
    (2, 16, 1, 256, 128, 2, torch.bfloat16),
    (1, 28, 4, 32768, 128, 4, torch.bfloat16),    # C3 shape with outliers
    (2, 8, 2, 1000, 128, 0, F8),                  # no outliers, ragged S
    (1, 7, 1, 77, 64, 16, torch.bfloat16),        # the maximum outlier count
])
@pytest.mark.parametrize("K", [8, 256])
def test_decode_attn_pq_lut_asym(dev, B, Hq, Hk, S, D, C, v_dtype, K):
    lut, k_idx, k_out, q_out, v = _asym_inputs(B, Hq, Hk, S, D, C, K, seed=S + C + K, v_dtype=v_dtype)
    out = PQ.decode_attn_pq_lut_asym(lut.to(dev), k_idx.to(dev), k_out.to(dev), q_out.to(dev), v.to(dev))
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.bfloat16
    _check(out, R.decode_attn_pq_lut_asym(lut, k_idx, k_out, q_out, v), f"asym S{S} D{D} C{C} K{K} {v_dtype}")


def _paginate(x, lens, bs, seed, nblocks_extra=3):
    """Contiguous [B, H, S, ...] -> (paged [blocks, H, bs, ...], block_table with -1
    padding, shuffled block order and spare blocks)."""
    g = torch.Generator().manual_seed(seed)
    B = x[0].shape[0]
    nb = [(n + bs - 1) // bs for n in lens]
    total = sum(nb) + nblocks_extra
    perm = torch.randperm(total, generator=g)
    table = torch.full((B, max(nb) + 1), -1, dtype=torch.int32)
    c = 0
    for b in range(B):
        for i in range(nb[b]):
            table[b, i] = int(perm[c])
            c += 1
    outs = []
    for t_ in x:
        p = torch.zeros(total, t_.shape[1], bs, *t_.shape[3:], dtype=t_.dtype)
        for b in range(B):
            for t in range(lens[b]):
                p[table[b, t // bs], :, t % bs] = t_[b, :, t]
        outs.append(p)
    return outs, table


@pytest.mark.parametrize("B,Hq,Hk,D,C,bs,lens,v_dtype", [
    (2, 8, 2, 64, 2, 16, [45, 78], torch.bfloat16),     # benchmarks/test_correctness.py:484-489 cases
    (2, 8, 2, 64, 2, 16, [45, 78], F8),
    (1, 4, 1, 128, 1, 32, [55], F8),
    (4, 28, 4, 128, 4, 16, [5000, 1, 4096, 2047], torch.bfloat16),
])
def test_paged_attn_pq_lut_asym(dev, B, Hq, Hk, D, C, bs, lens, v_dtype):
    S = max(lens)
    lut, k_idx, k_out, q_out, v = _asym_inputs(B, Hq, Hk, S, D, C, 8, seed=S + bs, v_dtype=v_dtype)
    (kp, kop, vp), table = _paginate([k_idx, k_out, v], lens, bs, seed=bs)
    cl = torch.tensor(lens, dtype=torch.int32)
    out = PQ.paged_attn_pq_lut_asym(lut.to(dev), kp.to(dev), kop.to(dev), q_out.to(dev), vp.to(dev), table.to(dev),
                                    cl.to(dev), block_size=bs)
    ref = R.paged_attn_pq_lut_asym(lut, kp, kop, q_out, vp, table, cl, bs)
    _check(out, ref, f"paged asym lens {lens} bs {bs} {v_dtype}")
    # each sequence equals the contiguous decode over its own length
    b = 0
    n = lens[b]
    solo = PQ.decode_attn_pq_lut_asym(lut[b:b + 1].to(dev), k_idx[b:b + 1, :, :n].to(dev),
                                      k_out[b:b + 1, :, :n].to(dev), q_out[b:b + 1].to(dev), v[b:b + 1, :, :n].to(dev))
    _check(out[b:b + 1], solo.cpu(), "paged == contiguous, sequence 0")


@pytest.mark.parametrize("lens,bs,K", [([45, 78], 16, 256), ([3000, 17, 1024], 16, 64), ([55], 32, 8)])
def test_paged_attn_pq_lut_kv(dev, lens, bs, K):
    B, Hq, Hk, D = len(lens), 8, 2, 128
    S = max(lens)
    g = torch.Generator().manual_seed(S)
    M = D // 8
    cb = torch.randn(M, K, 8, generator=g).half()
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    lut = R.pq_build_lut(q, cb.float(), 1.0 / math.sqrt(D))
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g, dtype=torch.uint8)
    v_idx = torch.randint(0, K, (B, Hk, S, M), generator=g, dtype=torch.uint8)
    (kp, vp), table = _paginate([k_idx, v_idx], lens, bs, seed=S)
    cl = torch.tensor(lens, dtype=torch.int32)
    out = PQ.paged_attn_pq_lut_kv(lut.to(dev), kp.to(dev), vp.to(dev), cb.to(dev), table.to(dev), cl.to(dev),
                                  block_size=bs)
    assert out.dtype == torch.float16
    _check(out, R.paged_attn_pq_lut_kv(lut, kp, vp, cb, table, cl, bs), f"paged lut-kv lens {lens}")


@pytest.mark.parametrize("B,Hq,Hk,S,D,C,K", [(2, 8, 2, 1000, 128, 2, 8), (1, 28, 4, 32768, 128, 4, 256),
                                            (2, 4, 4, 77, 64, 0, 16)])
def test_sparse_score_pq_lut_asym(dev, B, Hq, Hk, S, D, C, K):
    lut, k_idx, k_out, q_out, _ = _asym_inputs(B, Hq, Hk, S, D, C, K, seed=S)
    s = PQ.sparse_score_pq_lut_asym(lut.to(dev), k_idx.to(dev), k_out.to(dev), q_out.to(dev)).cpu()
    ref = R.pq_asym_scores(lut, k_idx, k_out, q_out)
    assert (s - ref).abs().max() <= 1e-4 * max(1.0, float(ref.abs().max()))


def test_sparse_decode_pq_lut_pipeline(dev):
    B, Hq, Hk, S, D, C = 2, 8, 2, 3000, 128, 2
    lut, k_idx, k_out, q_out, v = _asym_inputs(B, Hq, Hk, S, D, C, 256, seed=5)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    sc = 1 / math.sqrt(D)
    args = [t.to(dev) for t in (lut, k_idx, k_out, q_out, q, k, v)]
    out = PQ.sparse_decode_pq_lut(*args, 0.05, sc)
    s = PQ.sparse_score_pq_lut_asym(*args[:4])
    kb = SP.budget(0.05, S)
    idx = R.topk_indices(s.cpu(), kb)
    assert torch.equal(SP.topk_indices(s, kb).cpu().long(), idx)
    _check(out, R.sparse_gather_attn(q, k, v, idx, sc), "sparse_decode_pq_lut")


def test_asym_argument_errors(dev):
    lut, k_idx, k_out, q_out, v = _asym_inputs(1, 4, 1, 64, 128, 2, 8, seed=1)
    args = [t.to(dev) for t in (lut, k_idx, k_out, q_out, v)]
    with pytest.raises(ValueError):
        PQ.decode_attn_pq_lut_asym(*args[:4], args[4].half())                         # fp16 values
    with pytest.raises(ValueError):
        PQ.decode_attn_pq_lut_asym(args[0], args[1], torch.zeros(1, 1, 64, 17, device=dev),
                                   torch.zeros(1, 4, 17, device=dev), args[4])          # 17 outlier channels
    with pytest.raises(ValueError):
        PQ.decode_attn_pq_lut_asym(args[0], args[1], args[2], args[3][:, :2], args[4])  # q_out heads
