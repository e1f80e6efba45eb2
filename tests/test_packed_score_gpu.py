"""Packed 4/2-bit score keys vs the CPU oracle: the quantize/pack kernel
(bit-exact), the packed score kernel, and the packed two-pass sparse decode
(src/attention_kernels.py:1136-1263; benchmarks/test_correctness.py:704-721)."""
import math

import pytest
import torch

from bytes_amd import attention_kernels as AK
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


def _keys(B, Hk, S, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, Hk, S, D, generator=g) * 1.5
    k[0, 0, 0] = 0.75                                   # constant groups: scale = 1e-8/(levels-1), codes 0
    if S > 2:
        k[0, 0, 1, 3] = 40.0                            # one outlier per group
        k[0, 0, 2] = -k[0, 0, 2].abs()                  # all-negative row
    return k.to(dtype)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,Hk,S,D", [(2, 2, 300, 128), (1, 8, 77, 64), (1, 1, 1, 128)])
def test_pack_bit_exact(dev, bits, dtype, B, Hk, S, D):
    k = _keys(B, Hk, S, D, dtype, seed=S + D)
    p, s, z = AK.quantize_and_pack_score_keys(k.to(dev), bits, 32)
    rp, rs, rz = R.quantize_and_pack_score_keys(k, bits, 32)
    assert p.dtype == torch.uint8 and s.dtype == dtype and z.dtype == dtype
    assert torch.equal(p.cpu(), rp), f"packed codes differ ({bits}-bit, {dtype})"
    assert torch.equal(s.cpu(), rs) and torch.equal(z.cpu(), rz), f"scale/min differ ({bits}-bit, {dtype})"


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("D", [128, 64])
def test_every_position_scores_exactly(dev, bits, D):
    """One-hot queries pick one key element each: the score is code*scale + min,
    one rounding of an exact value in fp32 (an 8-bit by <= 4-bit product plus
    min), so it must equal the oracle's dequantized key bit for bit.  Pins the code
    layout (element c at bits ((c % (8/bits)) * bits) of byte c // (8/bits))
    and the group of each scale/min."""
    S = 256
    g = torch.Generator().manual_seed(bits * 1000 + D)
    packed = torch.randint(0, 256, (1, 1, S, D * bits // 8), generator=g, dtype=torch.uint8)
    scale = (torch.rand(1, 1, S, D // 32, generator=g) * 0.5).to(torch.bfloat16)
    z = torch.randn(1, 1, S, D // 32, generator=g)
    zero = (z.sign() * (z.abs() + 0.05)).to(torch.bfloat16)      # |min| >= 0.05: min - 128*scale is exact in fp32
    q = torch.eye(D, dtype=torch.bfloat16).reshape(1, D, 1, D)
    s = AK.sparse_score_packed(q.to(dev), packed.to(dev), scale.to(dev), zero.to(dev), 1.0, score_bits=bits)
    ref = R.sparse_score_packed(q, packed, scale, zero, 1.0, score_bits=bits)
    assert torch.equal(s.cpu(), ref)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("B,Hq,Hk,S,D", [(2, 8, 2, 1000, 128), (1, 24, 8, 4099, 128), (2, 4, 4, 300, 64),
                                         (1, 7, 1, 1, 128)])
def test_packed_scores(dev, bits, B, Hq, Hk, S, D):
    x = W.dense(B, Hq, Hk, D, S, seed=S + bits)
    p, s, z = R.quantize_and_pack_score_keys(x["k"], bits, 32)
    out = AK.sparse_score_packed(x["q"].to(dev), p.to(dev), s.to(dev), z.to(dev), 0.088, score_bits=bits)
    ref = R.sparse_score_packed(x["q"], p, s, z, 0.088, score_bits=bits)
    d = (out.cpu() - ref).abs().max()
    print(f"packed scores {bits}-bit B{B} Hq{Hq} Hk{Hk} S{S} D{D}: max-abs {d:.3e}", flush=True)
    assert d <= SCORE_TOL


def test_packed_scores_strided_cache(dev):
    """Views into a larger cache (row strides above the packed row width)."""
    x = W.dense(1, 8, 2, 128, 600, seed=3)
    p, s, z = R.quantize_and_pack_score_keys(x["k"], 4, 32)
    big_p = torch.zeros(1, 2, 1024, 64, dtype=torch.uint8)
    big_s = torch.zeros(1, 2, 1024, 4, dtype=torch.bfloat16)
    big_z = torch.zeros_like(big_s)
    big_p[:, :, :600], big_s[:, :, :600], big_z[:, :, :600] = p, s, z
    bp, bs, bz = big_p.to(dev), big_s.to(dev), big_z.to(dev)
    out = AK.sparse_score_packed(x["q"].to(dev), bp[:, :, :600], bs[:, :, :600], bz[:, :, :600], 0.1, score_bits=4)
    assert (out.cpu() - R.sparse_score_packed(x["q"], p, s, z, 0.1, score_bits=4)).abs().max() <= SCORE_TOL


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("frac", [0.05, 0.25])
def test_sparse_decode_packed_pipeline(dev, bits, frac):
    """Two-pass decode on packed score keys: GPU pack -> packed scores -> top-kb
    -> gather attention over the exact bf16 keys/values."""
    x = W.dense(2, 8, 2, 128, 3000, seed=21)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    sc = 1 / math.sqrt(128)
    p, s, z = AK.quantize_and_pack_score_keys(k, bits, 32)
    out = AK.sparse_decode_scalar(q, p, s, z, k, v, frac, sc, score_bits=bits, group_size=32)
    scores = AK.sparse_score_packed(q, p, s, z, sc, score_bits=bits)
    rscores = R.sparse_score_packed(x["q"], p.cpu(), s.cpu(), z.cpu(), sc, score_bits=bits)
    assert (scores.cpu() - rscores).abs().max() <= SCORE_TOL
    kb = SP.budget(frac, 3000)
    # selection bit-exact given the same fp32 scores; attention over it within tolerance
    idx = R.topk_indices(scores.cpu(), kb)
    assert torch.equal(SP.topk_indices(scores, kb).cpu().long(), idx)
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], idx, sc), f"packed {bits}-bit decode frac {frac}")
    # the oracle's own selection (on its scores) agrees except at near-ties
    ridx = R.topk_indices(rscores, kb)
    same = sum(len(set(a.tolist()) & set(b.tolist())) for a, b in zip(idx.reshape(-1, kb), ridx.reshape(-1, kb)))
    assert same >= 0.99 * idx.numel()


def test_packed_argument_errors(dev):
    q = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16, device=dev)
    p = torch.zeros(1, 1, 10, 64, dtype=torch.uint8, device=dev)
    s = torch.zeros(1, 1, 10, 4, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        AK.sparse_score_packed(q, p, s, s, 1.0, score_bits=4, group_size=64)
    with pytest.raises(ValueError):
        AK.sparse_score_packed(q, p, s, s, 1.0, score_bits=2)          # 64 bytes are 256 2-bit codes
    with pytest.raises(ValueError):
        AK.sparse_score_packed(q, p, s[..., :2], s, 1.0, score_bits=4)
    with pytest.raises(ValueError):
        AK.quantize_and_pack_score_keys(torch.zeros(1, 1, 4, 128, device=dev, dtype=torch.bfloat16), 3, 32)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("B,Hq,Hk,S,kb,D", [(2, 6, 2, 4096, 256, 128), (1, 24, 8, 3001, 100, 128),
                                            (17, 24, 8, 1024, 64, 128), (2, 32, 2, 2000, 128, 64)])
def test_token_topk_packed_score_keys(dev, bits, B, Hq, Hk, S, kb, D):
    """Group-shared token top-k with packed selection keys: group-summed scores
    against the oracle on the dequantized keys, indices bit-exact given the same
    scores, attention over the exact bf16 cache (B*Hk = 136 rows, above the
    fused-histogram limit of 128, takes the separate histogram pass)."""
    x = W.dense(B, Hq, Hk, D, S, seed=S + bits)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    p, s, z = AK.quantize_and_pack_score_keys(k, bits, 32)
    out, idx = SP.token_topk_decode(q, k, v, kb, x["scale"], k_score=p, score_scale=s, score_zero=z,
                                    score_bits=bits)
    g = SP._score(q, p, x["scale"], group_sum=True, packed=(s, z, bits)).cpu()
    kd = R.score_keys_dequant(p.cpu(), s.cpu(), z.cpu(), bits, 32)
    assert (g - R.group_scores(x["q"], kd, x["scale"])).abs().max() <= SCORE_TOL
    ridx = R.topk_indices(g, kb, sorted_by_score=False)
    assert torch.equal(idx.cpu().long(), ridx)
    gi = ridx.unsqueeze(-1).expand(B, Hk, kb, D)
    _check(out, R.decode_attn(x["q"], torch.gather(x["k"], 2, gi), torch.gather(x["v"], 2, gi), scale=x["scale"]),
           f"token top-k {bits}-bit score keys B{B} S{S} kb{kb} D{D}")


@pytest.mark.parametrize("bits", [4, 2])
def test_packed_group_scores_full_lds_buffer(dev, bits):
    """Packed selection keys on rows long enough that, on 256 CUs, each score
    workgroup's token range is the largest the host plans (the LDS score
    buffer's capacity: 8192 tokens with 4-bit keys, 4096 with 2-bit), with
    a ragged end: group sums at the start,
    across workgroup boundaries and at the end against the oracle on those
    slices of the dequantized keys."""
    B, Hq, Hk, D = 1, 24, 8, 128
    S = 2048 * 8192 // Hk + 777
    g = torch.Generator(device=dev).manual_seed(13)
    q = torch.randn(B, Hq, 1, D, device=dev, generator=g, dtype=torch.bfloat16)
    k = torch.randn(B, Hk, S, D, device=dev, generator=g, dtype=torch.bfloat16)
    p, s, z = AK.quantize_and_pack_score_keys(k, bits, 32)
    del k
    out = SP._score(q, p, 0.088, group_sum=True, packed=(s, z, bits))
    assert out.shape == (B, Hk, S)
    qc = q.cpu()
    for a, b in ((0, 3000), (8192 - 700, 8192 + 700), (5 * 8192 - 300, 5 * 8192 + 300), (S - 4000, S)):
        kd = R.score_keys_dequant(p[:, :, a:b].cpu(), s[:, :, a:b].cpu(), z[:, :, a:b].cpu(), bits, 32)
        d = (out[:, :, a:b].cpu() - R.group_scores(qc, kd, 0.088)).abs().max().item()
        print(f"{bits}-bit tokens {a}..{b}: max-abs {d:.3e}", flush=True)
        assert d <= SCORE_TOL, (a, b)
    del p, s, z, out
    torch.cuda.empty_cache()

