"""Harness microkernels (gather-reduce, staged packed-score probe) on the GPU
against the oracle's restatements of benchmarks/bench_access_pattern.py:25-52
and benchmarks/bench_unpack_ablation.py:19-53."""
import pytest
import torch

from bytes_amd.harness import kernels as HK
from bytes_amd.sparse import quantize_and_pack_score_keys
from oracle import reference as R

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("pattern", ["contiguous", "random", "paged"])
def test_gather_reduce_matches_oracle(dev, D, pattern):
    g = torch.Generator().manual_seed(D)
    H, S = 6, 3000
    K = 2100 if pattern != "paged" else 1600
    v = torch.randn(H, S, D, generator=g).half()
    if pattern == "contiguous":
        idx = torch.arange(K).expand(H, K).to(torch.int32)
    elif pattern == "random":
        idx = torch.stack([torch.randperm(S, generator=g)[:K] for _ in range(H)]).to(torch.int32)
    else:
        starts = torch.randint(0, S // 16, (H, K // 16), generator=g) * 16
        idx = (starts[..., None] + torch.arange(16)).reshape(H, K).to(torch.int32)
    out = HK.gather_reduce(v.to(dev), idx.to(dev)).cpu()
    ref = R.gather_reduce(v, idx)
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-3), (out - ref).abs().max()


def test_gather_reduce_long_list_and_duplicates(dev):
    """Index lists longer than one staged segment (16384) and repeated rows."""
    g = torch.Generator().manual_seed(5)
    H, S, D = 3, 20000, 64
    v = torch.randn(H, S, D, generator=g).half()
    idx = torch.randint(0, S, (H, 40000), generator=g).to(torch.int32)
    out = HK.gather_reduce(v.to(dev), idx.to(dev)).cpu()
    assert torch.allclose(out, R.gather_reduce(v, idx), rtol=1e-5, atol=2e-3)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("D", [64, 128])
def test_packed_stages_match_oracle(dev, bits, D):
    g = torch.Generator().manual_seed(bits * D)
    B, Hq, Hk, S = 2, 8, 2, 1000
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    p, s, z = quantize_and_pack_score_keys(k.to(dev), bits, 32)
    for stage in range(4):
        out = HK.stage_score(q.to(dev), p, s, z, bits, stage).cpu()
        ref = R.packed_stage(q, p.cpu(), s.cpu(), z.cpu(), bits, stage)
        if stage < 2:                                   # integer sums: exact in fp32
            assert torch.equal(out, ref), stage
        else:
            assert torch.allclose(out, ref, rtol=1e-4, atol=1e-3), (stage, (out - ref).abs().max())


@pytest.mark.parametrize("nontemporal", [False, True])
def test_stream_read_folds_every_word(dev, nontemporal):
    """The floor probe reads each 16-byte word of its slice exactly once:
    thread t of workgroup g folds (XOR) the words of vectors t + 256*i of
    each 2048-vector block of slice g (plain and non-temporal loads alike)."""
    import numpy as np
    wgs, vec_per_wg = 4, 4096
    g = torch.Generator().manual_seed(7)
    words = torch.randint(0, 2**31 - 1, (wgs * vec_per_wg * 4,), generator=g, dtype=torch.int64).to(torch.int32)
    out = HK.stream_read(words.to(dev), wgs, nontemporal=nontemporal).cpu()
    w = words.numpy().view(np.uint32).reshape(wgs, vec_per_wg // 2048, 8, 256, 4)
    want = np.bitwise_xor.reduce(w, axis=(1, 2, 4)).reshape(-1).astype(np.float32)
    assert np.array_equal(out.numpy(), want)
    HK.empty_launch(8, dev)
    torch.cuda.synchronize()
