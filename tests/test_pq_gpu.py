"""PQ decode (LUT-KV, LUT, dequant), LUT build, encode, k-means vs the CPU oracle.

Encode and decode_vectors: bit-exact.  LUT: fp32, 1e-5 relative.  Attention
outputs: north_star tolerance.  k-means values depend on the RNG stream and
are treated as inputs (parity given identical codebooks); the update step is
checked against the mean formula.
"""
import pytest
import torch

from bytes_amd import pq as PQ
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


def _rand_cb(shape, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


@pytest.mark.parametrize("per_head", [True, False])
def test_lut_build(dev, per_head):
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 8, 1, 128, generator=g).to(torch.bfloat16)
    cb = _rand_cb((2, 16, 256, 8) if per_head else (16, 256, 8), 2, torch.float16 if per_head else torch.float32)
    if not per_head:
        cb = cb.half().float()                       # values exactly representable in fp16
    lut = PQ.pq_build_lut(q.to(dev), cb.to(dev), 0.088)
    ref = R.pq_build_lut(q, cb, 0.088)
    assert lut.shape == (2, 8, 16, 256)
    assert torch.allclose(lut.cpu(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_encode_bit_exact(dev, dtype):
    g = torch.Generator().manual_seed(3)
    cb = _rand_cb((16, 256, 8), 4, torch.float32)
    cb[:, 7] = cb[:, 3]                                   # duplicate codewords: the first index wins
    x = torch.randn(1000, 128, generator=g).to(dtype)
    x[5] = cb[torch.arange(16), 200].reshape(-1).to(dtype)   # exact codewords
    got = PQ.pq_encode(x.to(dev), cb.to(dev)).cpu()
    ref = R.pq_encode(x, cb)
    assert got.dtype == torch.uint8 and torch.equal(got.long(), ref)
    # per-head fp16 codebooks
    cbh = _rand_cb((3, 8, 64, 8), 5)
    xh = torch.randn(3, 500, 64, generator=g).to(dtype)
    goth = PQ.pq_encode(xh.to(dev), cbh.to(dev)).cpu().long()
    refh = torch.stack([R.pq_encode(xh[h], cbh[h].float()) for h in range(3)])
    assert torch.equal(goth, refh)


def test_decode_vectors_exact(dev):
    cb = _rand_cb((16, 256, 8), 6, torch.float32)
    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, 256, (3, 77, 16), generator=g)
    got = PQ.pq_decode(idx.to(dev), cb.to(dev)).cpu()
    assert torch.equal(got, R.pq_decode(idx, cb))


def test_lut_kv_reference_shape(dev):
    """benchmarks/test_correctness.py:237-297 shape: B2 Hq8 Hk2 S128 D64, d_sub 8, 3-bit (K=8)."""
    g = torch.Generator().manual_seed(8)
    q = torch.randn(2, 8, 1, 64, generator=g).to(torch.bfloat16)
    kcb, vcb = _rand_cb((8, 8, 8), 9, torch.float32), _rand_cb((8, 8, 8), 10, torch.float32)
    k_idx = torch.randint(0, 8, (2, 2, 128, 8), generator=g).to(torch.uint8)
    v_idx = torch.randint(0, 8, (2, 2, 128, 8), generator=g).to(torch.uint8)
    lut = R.pq_build_lut(q, kcb)
    out = PQ.decode_attn_pq_lut_kv(lut.to(dev), k_idx.to(dev), v_idx.to(dev), vcb.to(dev))
    assert out.dtype == torch.float32 and out.shape == (2, 8, 1, 64)
    _check(out, R.decode_attn_pq_lut_kv(lut, k_idx, v_idx, vcb), "pq_lut_kv K=8")


@pytest.mark.parametrize("B,Hq,Hk,S,D,K", [(1, 7, 1, 1000, 128, 256), (2, 8, 2, 333, 64, 16),
                                          (1, 28, 4, 4096, 128, 256)])
def test_lut_modes_match_oracle(dev, B, Hq, Hk, S, D, K):
    g = torch.Generator().manual_seed(S)
    M = D // 8
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    kcb, vcb = _rand_cb((Hk, M, K, 8), S + 1), _rand_cb((Hk, M, K, 8), S + 2)
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    v_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    lut = R.pq_build_lut(q, kcb, 0.1)
    d = {n: t.to(dev) for n, t in dict(q=q, v=v, kcb=kcb, vcb=vcb, k_idx=k_idx, v_idx=v_idx, lut=lut).items()}
    o0 = PQ.decode_attn_pq_lut_kv(d["lut"], d["k_idx"], d["v_idx"], d["vcb"])
    assert o0.dtype == torch.float16
    _check(o0, R.decode_attn_pq_lut_kv(lut, k_idx, v_idx, vcb), f"lut_kv S{S}")
    o1 = PQ.decode_attn_pq_lut(d["lut"], d["k_idx"], d["v"])
    _check(o1, R.decode_attn_pq_lut(lut, k_idx, v), f"lut S{S}")
    kcb_small = (kcb.float() * 0.1).half()             # keep q . k_hat in a softmax-friendly range
    o2 = PQ.decode_attn_dequant(d["q"], d["k_idx"], kcb_small.to(dev), d["v"])
    _check(o2, R.decode_attn_dequant(q, k_idx, kcb_small, v), f"dequant S{S}")


@pytest.mark.parametrize("chunk", [128, 4096])
def test_lut_kv_split_counts(dev, chunk):
    g = torch.Generator().manual_seed(11)
    q = torch.randn(1, 8, 1, 128, generator=g).to(torch.bfloat16)
    kcb, vcb = _rand_cb((2, 16, 256, 8), 12), _rand_cb((2, 16, 256, 8), 13)
    k_idx = torch.randint(0, 256, (1, 2, 40000, 16), generator=g).to(torch.uint8)
    v_idx = torch.randint(0, 256, (1, 2, 40000, 16), generator=g).to(torch.uint8)
    lut = R.pq_build_lut(q, kcb, 0.088)
    out = PQ.decode_attn_pq_lut_kv(lut.to(dev), k_idx.to(dev), v_idx.to(dev), vcb.to(dev), chunk=chunk)
    _check(out, R.decode_attn_pq_lut_kv(lut, k_idx, v_idx, vcb), f"lut_kv chunk {chunk}")


@pytest.mark.parametrize("G,S,D,chunk", [(1, 777, 128, 0), (2, 2049, 64, 0), (3, 100, 128, 0), (5, 4100, 128, 64),
                                         (8, 1500, 128, 0), (7, 5000, 128, 512), (7, 5000, 128, 544),
                                         (9, 1200, 128, 0), (16, 640, 64, 0)])
def test_lut_kv_group_sizes(dev, G, S, D, chunk):
    """Query groups of 1..16 heads per KV head, quantized values: all G heads
    in one workgroup (G <= 8, chunks of <= 512 tokens) or groups of four
    (G > 8, or a longer chunk), against the oracle.  The fused call scores
    from q and the key codebook (on MFMA in the grouped kernel, through an
    in-kernel LUT in the general one): within the attention tolerance of the
    caller-LUT call, and bit for bit where the general kernel runs."""
    B, Hk, K = 2, 2, 256
    M = D // 8
    g = torch.Generator().manual_seed(G * 1000 + S)
    q = torch.randn(B, Hk * G, 1, D, generator=g).to(torch.bfloat16)
    kcb, vcb = _rand_cb((Hk, M, K, 8), S + 5), _rand_cb((Hk, M, K, 8), S + 6)
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    v_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    d = {n: t.to(dev) for n, t in dict(q=q, kcb=kcb, vcb=vcb, k_idx=k_idx, v_idx=v_idx).items()}
    scale = D ** -0.5
    lut = PQ.pq_build_lut(d["q"], d["kcb"], scale)
    two = PQ.decode_attn_pq_lut_kv(lut, d["k_idx"], d["v_idx"], d["vcb"], chunk=chunk)
    fused = PQ.decode_attn_pq_kv_fused(d["q"], d["kcb"], d["k_idx"], d["v_idx"], d["vcb"], scale, chunk=chunk)
    grouped = G <= 8 and chunk <= 512
    if grouped:
        _check(fused, two.cpu(), f"fused vs two calls G{G} S{S} D{D} chunk {chunk}")
    else:
        assert torch.equal(fused, two)
    ref = R.decode_attn_pq_lut_kv(R.pq_build_lut(q, kcb, scale), k_idx, v_idx, vcb)
    _check(two, ref, f"lut_kv G{G} S{S} D{D} chunk {chunk}")
    _check(fused, ref, f"fused G{G} S{S} D{D} chunk {chunk}")


def test_c3_full(dev):
    """BASELINE C3: B1 Hq28 Hkv4 D128 L32768, 16 x 8-dim subspaces, 256 fp16 codewords per head."""
    x = W.c3_pq(seed=0, device=dev)
    c = {n: (t.cpu() if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    assert x["k_idx"].shape == (1, 4, 32768, 16) and x["k_cb"].shape == (4, 16, 256, 8)
    # setup parity: LUT and codes from the GPU equal the oracle's on the same codebooks
    assert torch.allclose(c["lut"], R.pq_build_lut(c["q"], c["k_cb"], c["scale"]), rtol=1e-5, atol=1e-6)
    for h in range(4):
        assert torch.equal(c["k_idx"][0, h].long(), R.pq_encode(c["k"][0, h], c["k_cb"][h].float())), h
    out = PQ.decode_attn_pq_lut_kv(x["lut"], x["k_idx"], x["v_idx"], x["v_cb"])
    _check(out, R.decode_attn_pq_lut_kv(c["lut"], c["k_idx"], c["v_idx"], c["v_cb"]), "C3 pq_lut_kv")
    out1 = PQ.decode_attn_pq_lut(x["lut"], x["k_idx"], x["v"])
    _check(out1, R.decode_attn_pq_lut(c["lut"], c["k_idx"], c["v"]), "C3 pq_lut")
    out2 = PQ.decode_attn_dequant((x["q"].float() * c["scale"]).to(torch.bfloat16), x["k_idx"], x["k_cb"], x["v"])
    qs = (c["q"].float() * c["scale"]).to(torch.bfloat16)
    _check(out2, R.decode_attn_dequant(qs, c["k_idx"], c["k_cb"], c["v"]), "C3 dequant")


@pytest.mark.parametrize("B,Hq,Hk,S,D,K,per_head", [(1, 28, 4, 32768, 128, 256, True),   # C3
                                                   (1, 7, 1, 1000, 128, 256, True),
                                                   (2, 8, 2, 333, 64, 16, False),
                                                   (2, 12, 2, 5000, 128, 64, True)])
def test_fused_matches_two_calls(dev, B, Hq, Hk, S, D, K, per_head):
    """decode_attn_pq_kv_fused against pq_build_lut + decode_attn_pq_lut_kv and
    the oracle: within the attention tolerance (scores q . k_hat on MFMA from
    the codebook rows, exact products summed in fp32, instead of summed LUT
    entries), deterministic from call to call."""
    g = torch.Generator().manual_seed(S + K)
    M = D // 8
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    shp = (Hk, M, K, 8) if per_head else (M, K, 8)
    kcb, vcb = _rand_cb(shp, S + 3), _rand_cb(shp, S + 4)
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    v_idx = torch.randint(0, K, (B, Hk, S, M), generator=g).to(torch.uint8)
    d = {n: t.to(dev) for n, t in dict(q=q, kcb=kcb, vcb=vcb, k_idx=k_idx, v_idx=v_idx).items()}
    scale = D ** -0.5
    lut = PQ.pq_build_lut(d["q"], d["kcb"], scale)
    two = PQ.decode_attn_pq_lut_kv(lut, d["k_idx"], d["v_idx"], d["vcb"])
    fused = PQ.decode_attn_pq_kv_fused(d["q"], d["kcb"], d["k_idx"], d["v_idx"], d["vcb"], scale)
    assert fused.shape == two.shape and fused.dtype == two.dtype
    again = PQ.decode_attn_pq_kv_fused(d["q"], d["kcb"], d["k_idx"], d["v_idx"], d["vcb"], scale)
    assert torch.equal(fused, again)
    _check(fused, two.cpu(), f"fused vs two calls B{B} Hq{Hq} Hk{Hk} S{S} D{D} K{K}")
    ref = R.decode_attn_pq_lut_kv(R.pq_build_lut(q, kcb, scale), k_idx, v_idx, vcb)
    _check(fused, ref, f"fused B{B} Hq{Hq} Hk{Hk} S{S} D{D} K{K}")


def test_kmeans_update_and_determinism(dev):
    g = torch.Generator().manual_seed(13)
    H, N, D, K = 2, 3000, 64, 32
    X = torch.randn(H, N, D, generator=g)
    X[:, :10] = X[:, :1]                                  # repeated points
    a = PQ.kmeans(X.to(dev), K, 3, generator=torch.Generator().manual_seed(5)).cpu()
    b = PQ.kmeans(X.to(dev), K, 3, generator=torch.Generator().manual_seed(5)).cpu()
    assert a.shape == (H, 8, K, 8) and torch.equal(a, b)
    # one update from the seeded initial codewords, replayed on the CPU with the
    # same draws: exact nearest-codeword labels, then per-cluster fp32 means
    # (an empty cluster takes its re-seed point)
    init = PQ.kmeans(X.to(dev), K, 0, generator=torch.Generator().manual_seed(5)).cpu()
    one = PQ.kmeans(X.to(dev), K, 1, generator=torch.Generator().manual_seed(5)).cpu()
    gg = torch.Generator().manual_seed(5)
    for _ in range(H * 8):
        torch.randperm(N, generator=gg)
    reseed = torch.randint(0, N, (H, 8, K), generator=gg)
    for h in range(H):
        for j in range(8):
            xs = X[h, :, j * 8:(j + 1) * 8]
            lab = R.pq_encode(xs, init[h, j:j + 1])[:, 0]
            for c in range(K):
                m = lab == c
                exp = xs[m].mean(0) if m.any() else xs[reseed[h, j, c]]
                assert torch.allclose(one[h, j, c], exp, rtol=1e-6, atol=1e-6), (h, j, c)
    # quantization error drops from the initial codewords to the fitted ones
    err = lambda cb: (PQ.pq_decode(PQ.pq_encode(X.to(dev), cb.to(dev)), cb.to(dev)).cpu() - X).pow(2).mean()  # noqa
    assert err(a) < err(init)


def test_kmeans_pytorch_drop_in_shapes(dev):
    """src/quantization.py:102-132 signature: X [N, d_sub] -> [k, d_sub] in X's
    dtype, padding with zero rows when N <= k; other d_sub raise."""
    g = torch.Generator().manual_seed(3)
    X = torch.randn(500, 8, generator=g).to(dev)
    cb = PQ.kmeans_pytorch(X, 16, 4, generator=torch.Generator().manual_seed(1))
    assert cb.shape == (16, 8) and cb.dtype == X.dtype
    assert torch.equal(cb, PQ.kmeans(X, 16, 4, generator=torch.Generator().manual_seed(1))[0])
    small = torch.randn(5, 8, generator=g).to(dev).to(torch.bfloat16)
    pad = PQ.kmeans_pytorch(small, 8, 2)
    assert pad.shape == (8, 8) and pad.dtype == torch.bfloat16
    assert torch.equal(pad[:5], small) and not pad[5:].any()
    with pytest.raises(ValueError):
        PQ.kmeans_pytorch(torch.randn(100, 4, device=dev), 8)


def test_product_quantizer_round_trip(dev):
    pq = PQ.ProductQuantizer(64, 8, bits=4, device=dev)
    g = torch.Generator().manual_seed(21)
    X = torch.randn(2000, 64, generator=g)
    pq.fit(X, num_iters=5, generator=torch.Generator().manual_seed(1))
    codes = pq.quantize(X)
    assert codes.dtype == torch.int64 and codes.shape == (2000, 8)
    rec = pq.dequantize(codes)
    assert torch.equal(pq.quantize(rec), codes)            # codewords encode to their own index
