"""Dense bf16 decode attention: HIP kernel vs the CPU oracle (north_star tolerance)."""
import math

import pytest
import torch

from bytes_amd import attention_kernels as AK
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


@pytest.mark.parametrize("B,Hq,Hk,S,D,scale", [
    (2, 8, 2, 128, 64, 1.0),          # benchmarks/test_correctness.py:50-80 shape, no scale
    (1, 14, 2, 8192, 64, 0.125),      # BASELINE C1
    (2, 4, 4, 1000, 128, 0.1),        # G = 1 (MHA), ragged S
    (1, 40, 2, 333, 64, 0.2),         # G = 20: two head blocks
    (1, 7, 1, 1, 128, 1.0),           # single token
    (1, 8, 1, 31, 64, 1.0),           # shorter than one tile
])
def test_dense_matches_oracle(dev, B, Hq, Hk, S, D, scale):
    x = W.dense(B, Hq, Hk, D, S, seed=S + Hq)
    out = AK.decode_attn_bf16(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), scale)
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.bfloat16
    ref = R.decode_attn(x["q"], x["k"], x["v"], scale=scale)
    _check(out, ref, f"dense B{B} Hq{Hq} Hk{Hk} S{S} D{D}")


@pytest.mark.parametrize("chunk", [128, 256, 1024, 1 << 20])
def test_dense_split_counts_agree(dev, chunk):
    x = W.dense(2, 28, 4, 128, 3000, seed=5)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    out = AK.decode_attn_bf16(q, k, v, 1 / math.sqrt(128), chunk=chunk)
    ref = R.decode_attn(x["q"], x["k"], x["v"], scale=1 / math.sqrt(128))
    _check(out, ref, f"chunk {chunk}")


def test_dense_strided_views_and_determinism(dev):
    x = W.dense(1, 8, 2, 64, 700, seed=11)
    big_k = torch.zeros(1, 2, 1024, 64, dtype=torch.bfloat16)
    big_k[:, :, 100:800] = x["k"]
    k_view = big_k.to(dev)[:, :, 100:800]                      # non-contiguous in S/B
    v_t = x["v"].to(dev).transpose(1, 2).contiguous().transpose(1, 2)   # [B,S,H,D] storage
    q = x["q"].to(dev)
    a = AK.decode_attn_bf16(q, k_view, v_t, 0.125)
    b = AK.decode_attn_bf16(q, k_view, v_t, 0.125)
    assert torch.equal(a, b)
    _check(a, R.decode_attn(x["q"], x["k"], x["v"], scale=0.125), "strided")


def test_dense_large_l16k(dev):
    x = W.dense_16k(seed=0)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    out = AK.decode_attn_bf16(q, k, v, x["scale"])
    _check(out, R.decode_attn(x["q"], x["k"], x["v"], scale=x["scale"]), "dense 16K")
    # softmax invariant at full size: uniform V rows give back that row exactly-ish
    vv = torch.ones_like(v) * 0.5
    o2 = AK.decode_attn_bf16(q, k, vv, x["scale"])
    assert torch.all(o2 == 0.5)


def test_dense_rejects_bad_input(dev):
    q = torch.zeros(1, 6, 1, 64, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 4, 16, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        AK.decode_attn_bf16(q, k, k)                               # 6 % 4 != 0
    with pytest.raises(ValueError):
        AK.decode_attn_bf16(q.float(), k[:, :2], k[:, :2])          # dtype
    with pytest.raises(ValueError):
        AK.decode_attn_bf16(q, k[:, :2, :0], k[:, :2, :0])          # empty cache


def test_dense_back_to_back_calls_share_the_workspace(dev):
    """Consecutive calls (same plan, then a different plan) on the shared
    workspace each match the oracle."""
    for seed, (B, Hq, Hk, S) in enumerate([(2, 28, 4, 5000), (2, 28, 4, 5000), (3, 16, 2, 2900),
                                           (2, 28, 4, 5000)]):
        x = W.dense(B, Hq, Hk, 128, S, seed=100 + seed)
        out = AK.decode_attn_bf16(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), 0.09)
        _check(out, R.decode_attn(x["q"], x["k"], x["v"], scale=0.09), f"call {seed} B{B} S{S}")


def test_dense_many_splits_use_the_merge_kernel(dev):
    # chunk 128 over 40000 tokens: 313 splits, several blocks of the merge kernel
    x = W.dense(1, 8, 1, 128, 40000, seed=9)
    out = AK.decode_attn_bf16(x["q"].to(dev), x["k"].to(dev), x["v"].to(dev), 0.09, chunk=128)
    _check(out, R.decode_attn(x["q"], x["k"], x["v"], scale=0.09), "313 splits")


def test_dense_graph_replays(dev):
    """Captured once, replayed with new input contents (eager copies and syncs in
    between): every replay equals the eager call on the same inputs."""
    x = W.dense(2, 14, 2, 64, 3000, seed=21)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    AK.decode_attn_bf16(q, k, v, 0.125)                      # sizes the workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = AK.decode_attn_bf16(q, k, v, 0.125)
    torch.cuda.synchronize()
    for it in range(3):
        y = W.dense(2, 14, 2, 64, 3000, seed=30 + it)
        q.copy_(y["q"].to(dev)); k.copy_(y["k"].to(dev)); v.copy_(y["v"].to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = AK.decode_attn_bf16(q, k, v, 0.125)
        assert torch.equal(out, eager), f"replay {it}"
        _check(out, R.decode_attn(y["q"], y["k"], y["v"], scale=0.125), f"replay {it}")


def test_workspace_growth_after_capture(dev):
    """A graph captured with the split-K workspace at one size keeps working
    after a larger eager call has replaced that workspace: the superseded
    buffer is never released, so the replay still writes memory nothing else
    owns and its output equals the eager result."""
    from bytes_amd import _lib
    key = (dev.index or 0, "splitk")
    if key in _lib._ws:                         # start from a fresh workspace, as a new process does
        _lib._retired.append(_lib._ws.pop(key))
    x = W.dense(1, 14, 2, 64, 700, seed=41)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    AK.decode_attn_bf16(q, k, v, 0.125)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = AK.decode_attn_bf16(q, k, v, 0.125)
    torch.cuda.synchronize()
    before = _lib._ws[key].data_ptr()
    S = 65536
    assert _lib.size_query("bytes_decode_attn_bf16_workspace_size", 4, 28, 4, S, 128, 64) > _lib._ws[key].numel()
    bq = torch.randn((4, 28, 1, 128), device=dev).to(torch.bfloat16)
    bk = torch.zeros((4, 4, S, 128), dtype=torch.bfloat16, device=dev)
    filler = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=dev) for _ in range(8)]
    AK.decode_attn_bf16(bq, bk, bk, 0.1, chunk=64)
    torch.cuda.synchronize()
    assert _lib._ws[key].data_ptr() != before
    for it in range(2):
        y = W.dense(1, 14, 2, 64, 700, seed=50 + it)
        q.copy_(y["q"].to(dev)); k.copy_(y["k"].to(dev)); v.copy_(y["v"].to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, AK.decode_attn_bf16(q, k, v, 0.125)), f"replay {it}"
        _check(out, R.decode_attn(y["q"], y["k"], y["v"], scale=0.125), f"grown replay {it}")
    assert all(int(f[0]) == 7 and int(f[-1]) == 7 for f in filler)


def test_workspace_growth_during_capture_raises(dev):
    """Growing the workspace inside a capture would take the buffer from the
    graph's pool with its zero fill deferred to replay; the wrapper refuses."""
    from bytes_amd import _lib
    key = (dev.index or 0, "splitk")
    have = _lib.workspace(dev, 1).numel()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="graph capture"):
        with torch.cuda.graph(g):
            _lib.workspace(dev, have + 1)
    torch.cuda.synchronize()
    assert _lib._ws[key].numel() == have
