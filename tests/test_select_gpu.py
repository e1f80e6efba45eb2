"""select_topk / _quest_select / attend_topk over query chunks (Qc >= 1) on the
GPU against the oracle's restatement of benchmarks/sparse_attention.py:226-387:
indices bit-exact given the same fp32 scores, attention within the north_star
tolerance."""
import pytest
import torch

from bytes_amd import sparse as SP
from bytes_amd import sparse_attention as SA
from oracle import reference as R

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


def _inputs(B, Hq, Hk, Qc, S, D, seed, integer=False):
    g = torch.Generator().manual_seed(seed)
    if integer:
        q = torch.randint(-2, 3, (B, Hq, Qc, D), generator=g).to(torch.bfloat16)
        k = torch.randint(-2, 3, (B, Hk, S, D), generator=g).to(torch.bfloat16)
    else:
        q = torch.randn(B, Hq, Qc, D, generator=g).to(torch.bfloat16)
        k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,Hq,Hk,Qc,S,D,kb,local_w,expanded", [
    (1, 4, 2, 4, 600, 64, 48, 0, False),       # rows at 100..599: partial chunks, GQA keys
    (2, 8, 2, 3, 1000, 128, 64, 16, True),     # GQA-expanded keys as the reference passes them
    (1, 4, 4, 5, 300, 64, 200, 8, False),      # early rows hold fewer causal keys than kb: sentinels
    (1, 28, 4, 2, 4096, 128, 256, 0, False),   # G = 7
])
def test_select_topk_exact_matches_oracle(dev, B, Hq, Hk, Qc, S, D, kb, local_w, expanded):
    q, k, _ = _inputs(B, Hq, Hk, Qc, S, D, seed=S + Qc)
    pos = torch.linspace(S // 6, S - 1, Qc).long()
    keys = R.repeat_kv(k, Hq // Hk) if expanded else k
    got = SA.select_topk("exact", q.to(dev), keys.to(dev), pos, S, kb, 4096 // 4, 0.125, local_w=local_w)
    assert got.dtype == torch.int64 and got.shape == (B, Hq, Qc, kb)
    # the oracle ranks the GPU's own fp32 scores (the contract: identical scores)
    max_key = int(pos.max()) + 1
    s = SP.sparse_score_scalar(q.reshape(B, Hq * Qc, 1, D).to(dev), keys[:, :, :max_key].to(dev), 0.125).cpu()
    ref_s = R.sparse_score_scalar(q.reshape(B, Hq * Qc, 1, D), keys[:, :, :max_key], 0.125)
    assert (s - ref_s).abs().max() < 1e-3
    want = R.select_topk_from_scores(s.reshape(B, Hq, Qc, max_key), pos, S, kb, 1000, local_w)
    assert torch.equal(got.cpu(), want)
    if local_w == 0 and kb > int(pos.min()) + 1:
        assert (got[:, :, 0] == S).any(), "the first row must hold sentinel fillers"


def test_select_topk_exact_integer_scores_end_to_end(dev):
    """Integer-valued q and keys: every fp32 score is exact, so the GPU result
    equals the oracle's own scoring and selection, ties included."""
    B, Hq, Hk, Qc, S, D = 1, 8, 2, 6, 777, 64
    q, k, _ = _inputs(B, Hq, Hk, Qc, S, D, seed=5, integer=True)
    pos = torch.tensor([0, 15, 100, 401, 700, 776])
    for kb, lw in ((32, 0), (100, 24), (1, 0)):
        got = SA.select_topk("exact", q.to(dev), k.to(dev), pos.to(dev), S, kb, 128, 0.5, local_w=lw)
        want = R.select_topk_exact(q, k, pos, S, kb, 128, 0.5, lw)
        assert torch.equal(got.cpu(), want), (kb, lw)


def test_select_topk_large_budget(dev):
    """kb above 8192 over several key chunks: the running list is longer than a
    chunk, the last merge sorts more than 8192 entries; score order as the
    oracle's."""
    B, Hq, Hk, Qc, S, D = 1, 2, 1, 2, 20000, 64
    q, k, _ = _inputs(B, Hq, Hk, Qc, S, D, seed=9)
    pos = torch.tensor([12000, 19999])
    got = SA.select_topk("exact", q.to(dev), k.to(dev), pos, S, 10000, 4096, 0.125)
    s = SP.sparse_score_scalar(q.reshape(B, Hq * Qc, 1, D).to(dev), k.to(dev), 0.125).cpu()
    want = R.select_topk_from_scores(s.reshape(B, Hq, Qc, S), pos, S, 10000, 4096)
    assert torch.equal(got.cpu(), want)


def _soft_keys(selector, k, g):
    """The selection keys the reference's make_selection_keys builds for a
    selector (benchmarks/sparse_attention.py:127-150, without the RoPE, which
    is the caller's): per-token asymmetric fake-quantization over head_dim
    with 16 / 4 levels (int4 / int2), an fp8 e4m3fn round trip (fp8, also
    passed as the fp8 tensor itself), a perturbed copy (approx)."""
    if selector in ("int4", "int2"):
        codes, scale, xmin = R.asym_quant_codes(k.float(), 16 if selector == "int4" else 4, -1)
        return (codes.float() * scale + xmin).to(k.dtype)
    if selector == "fp8":
        return k.to(torch.float8_e4m3fn).to(k.dtype)
    if selector == "fp8_native":
        return k.to(torch.float8_e4m3fn)
    return (k.float() + 0.05 * torch.randn(k.shape, generator=g)).to(k.dtype)


@pytest.mark.parametrize("selector", ["approx", "int4", "int2", "fp8", "fp8_native"])
@pytest.mark.parametrize("Qc,S,kb,k_chunk,local_w", [
    (4, 600, 48, 100, 0),        # six chunks, the last partial
    (5, 700, 200, 64, 8),        # running list longer than a chunk; early rows with sentinels; recent window
    (3, 1000, 1, 333, 0),        # kb = 1
])
def test_select_topk_soft_selectors_stream(dev, selector, Qc, S, kb, k_chunk, local_w):
    """Every SOFT_SELECTOR the reference routes through the same streaming
    top-k (:35, :287-309) over the keys the caller passes: bit-exact against
    the oracle's streaming selection on the GPU's own fp32 scores, with a
    partial last chunk, sentinels and the recent window."""
    B, Hq, Hk, D = 1, 14, 2, 128
    q, k, _ = _inputs(B, Hq, Hk, Qc, S, D, seed=S + kb)
    g = torch.Generator().manual_seed(kb)
    sk = _soft_keys(selector, k, g)
    pos = torch.linspace(S // 8, S - 1, Qc).long()
    name = "fp8" if selector == "fp8_native" else selector
    got = SA.select_topk(name, q.to(dev), sk.to(dev), pos, S, kb, k_chunk, 0.088, local_w=local_w)
    assert got.dtype == torch.int64 and got.shape == (B, Hq, Qc, kb)
    max_key = int(pos.max()) + 1
    bits = 8 if sk.dtype == torch.float8_e4m3fn else 16
    s = SP.sparse_score_scalar(q.reshape(B, Hq * Qc, 1, D).to(dev), sk[:, :, :max_key].to(dev), 0.088,
                               score_bits=bits).cpu()
    want = R.select_topk_from_scores(s.reshape(B, Hq, Qc, max_key), pos, S, kb, k_chunk, local_w)
    assert torch.equal(got.cpu(), want)


def test_select_topk_recent(dev):
    B, Hq, Hk, Qc, S, D = 2, 6, 2, 4, 500, 64
    q, k, _ = _inputs(B, Hq, Hk, Qc, S, D, seed=21)
    pos = torch.tensor([0, 5, 130, 499])
    for kb in (1, 16, 200):
        got = SA.select_topk("recent", q.to(dev), k.to(dev), pos, S, kb, 128, 0.1)
        assert got.dtype == torch.int64
        assert torch.equal(got.cpu(), R.select_recent(B, Hq, pos, kb)), kb


def test_select_topk_memory_is_bounded_by_the_chunk(dev):
    """benchmarks/test_sparse_eval.py:60-83 at its shape (Hq 8, Hk 1, D 64,
    q_chunk 256, k_chunk 2048, frac 0.1): every query chunk of a prefill
    window selected and attended; peak memory grows by less than 3x when S
    doubles.  Then the selection alone at a fixed budget: its scratch does
    not grow with the context (O(Qc * (k_chunk + kb)), :477), where a
    one-shot selection would hold Hq * Qc * S fp32 scores."""
    Hq, Hk, D, qc, kc = 8, 1, 64, 256, 2048
    peaks = {}
    for S in (4096, 8192, 16384):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        g = torch.Generator().manual_seed(S)
        q = torch.randn(1, Hq, S, D, generator=g).to(torch.bfloat16).to(dev)
        k = torch.randn(1, Hk, S, D, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(1, Hk, S, D, generator=g).to(torch.bfloat16).to(dev)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        kb = max(1, round(0.1 * S))
        for q0 in range(0, S, qc):
            blk = q[:, :, q0:q0 + qc]
            p = torch.arange(q0, q0 + blk.shape[2])
            idx = SA.select_topk("exact", blk, k, p, S, kb, kc, D ** -0.5)
            SA.attend_topk(blk, k, v, idx, p, D ** -0.5)
        torch.cuda.synchronize()
        peaks[S] = torch.cuda.max_memory_allocated()
        del q, k, v
    print(f"peak MB {({S: round(p / 1e6, 1) for S, p in peaks.items()})}", flush=True)
    assert peaks[8192] / peaks[4096] < 3.0 and peaks[16384] / peaks[8192] < 3.0

    extra = {}
    kb = 512
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, Hq, qc, D, generator=g).to(torch.bfloat16).to(dev)
    for S in (8192, 32768, 131072):
        k = torch.randn(1, Hk, S, D, generator=g).to(torch.bfloat16).to(dev)
        p = torch.arange(S - qc, S)
        SA.select_topk("exact", q, k, p, S, kb, kc, D ** -0.5)        # workspaces at their size
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        idx = SA.select_topk("exact", q, k, p, S, kb, kc, D ** -0.5)
        torch.cuda.synchronize()
        extra[S] = torch.cuda.max_memory_allocated() - base
        del k, idx
    one_shot = Hq * qc * 131072 * 4
    print(f"selection scratch MB {({S: round(e / 1e6, 1) for S, e in extra.items()})}; one-shot scores at "
          f"S=131072: {one_shot / 1e6:.0f} MB", flush=True)
    assert extra[131072] <= 1.1 * extra[8192] and extra[131072] < one_shot / 4


def test_selectors_outside_the_hot_path_raise(dev):
    q, k, _ = _inputs(1, 2, 1, 1, 64, 64, seed=1)
    for sel in ("h2o", "snapkv", "signvq", "sparq", "random"):
        with pytest.raises(ValueError):
            SA.select_topk(sel, q.to(dev), k.to(dev), torch.tensor([63]), 64, 8, 64, 0.1)
