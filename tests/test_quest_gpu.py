"""Quest page selection: metadata and page bounds bit-exact, page ids bit-exact,
attention over the selected pages within the north_star tolerance."""
import math

import pytest
import torch

from bytes_amd import quest as Q
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
pytestmark = pytest.mark.gpu


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


@pytest.mark.parametrize("B,H,S,D,page", [(1, 4, 32768, 128, 16), (2, 3, 1000, 64, 16), (1, 2, 77, 128, 8)])
def test_page_minmax_bit_exact(dev, B, H, S, D, page):
    x = W.dense(B, H, H, D, S, seed=S)
    kmin, kmax = Q.quest_page_minmax(x["k"].to(dev), page)
    rmin, rmax = R.quest_page_minmax(x["k"], page)
    assert torch.equal(kmin.cpu().view(torch.int16), rmin.view(torch.int16))
    assert torch.equal(kmax.cpu().view(torch.int16), rmax.view(torch.int16))


@pytest.mark.parametrize("B,Hq,Hk,S,D,scale", [(1, 28, 4, 32768, 128, 1 / math.sqrt(128)), (2, 8, 8, 3000, 64, 1.0),
                                                (1, 32, 2, 4096, 128, 0.3)])
def test_page_scores_bit_exact(dev, B, Hq, Hk, S, D, scale):
    x = W.dense(B, Hq, Hk, D, S, seed=S + 1)
    rmin, rmax = R.quest_page_minmax(x["k"], 16)
    got = Q.quest_page_scores(x["q"].to(dev), rmin.to(dev), rmax.to(dev), scale)
    ref = R.quest_page_scores(x["q"], rmin, rmax, scale)
    assert torch.equal(got.cpu(), ref)


def test_page_scores_nonfinite_keys_bit_exact(dev):
    """Keys with +-inf / NaN entries: the bound follows torch.maximum(q*kmin,
    q*kmax) (benchmarks/sparse_attention.py:344), e.g. q_d < 0 with kmax_d = +inf
    gives the finite q_d*kmin_d, and q_d = 0 next to an infinity gives NaN."""
    x = W.dense(1, 8, 2, 128, 1024, seed=11)
    k = x["k"].clone()
    k[0, 0, 5, 3] = float("inf")          # page 0
    k[0, 0, 40, 7] = float("-inf")        # page 2
    k[0, 1, 100, 9] = float("nan")        # page 6 of head 1
    k[0, 1, 300, 0] = float("inf")
    k[0, 1, 301, 0] = float("-inf")       # page 18: both infinities at one d
    q = x["q"].clone()
    q[0, 0, 0, 3] = 0.0                   # q_d = 0 against the infinity of page 0
    q[0, 1, 0, 7] = -0.0
    rmin, rmax = R.quest_page_minmax(k, 16)
    got = Q.quest_page_scores(q.to(dev), rmin.to(dev), rmax.to(dev), 0.5).cpu()
    ref = R.quest_page_scores(q, rmin, rmax, 0.5)
    same = (got == ref) | (got.isnan() & ref.isnan())
    assert bool(same.all()), (got[~same], ref[~same])
    assert bool(ref.isnan().any()) and bool(torch.isfinite(ref[0, 2:4, 0]).all())


def test_page_scores_causal_and_recent_window(dev):
    x = W.dense(1, 8, 2, 128, 1000, seed=2)
    rmin, rmax = R.quest_page_minmax(x["k"], 16)
    pos, local_w = 500, 40
    got = Q.quest_page_scores(x["q"].to(dev), rmin.to(dev), rmax.to(dev), 0.1, pos=pos, local_w=local_w).cpu()
    ref = R.quest_page_scores(x["q"], rmin, rmax, 0.1)
    pg = torch.arange(ref.shape[-1])
    ref = torch.where(pg * 16 <= pos, ref, torch.full_like(ref, float("-inf")))     # :346-348
    lo, hi = max(pos - local_w + 1, 0) // 16, pos // 16
    ref = torch.where((pg >= lo) & (pg <= hi), torch.full_like(ref, float("inf")), ref)   # :349-355
    assert torch.equal(got, ref)


def test_quest_c4_full_pages_bit_exact(dev):
    """BASELINE C4: B1 Hq28 Hkv4 D128 L32768, 64 needles, 2048-token budget (128 pages)."""
    x = W.c4_quest(seed=0)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    sc = x["scale"]
    out, pid = Q.quest_decode(q, k, v, 2048, sc, return_pages=True)
    rpid, rtok, rbound = R.quest_select(x["q"], x["k"], 2048, 16, sc)
    assert pid.shape == (1, 28, 128)
    assert torch.equal(pid.cpu().long(), rpid)                              # bit-exact page ids
    tok = Q._quest_select(q, k, torch.tensor([32767]), 32768, 2048, 16, sc)
    assert torch.equal(tok.cpu()[:, :, 0], rtok)
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], rtok, sc), "C4 quest decode")
    # Quest upper bound at full size: each needle page's bound >= the needle's exact score
    needles = x["needles"][0]                                               # [Hk, 64]
    exact = R.sparse_score_scalar(x["q"], x["k"], sc)[0]                   # [Hq, S]
    bound = rbound[0]                                                       # [Hq, np]
    for h in range(28):
        t = needles[h // 7]
        assert torch.all(bound[h, t // 16] >= exact[h, t] - 1e-4), h
    sel = pid.cpu().long()[0]
    recall = sum(torch.isin(needles[h // 7] // 16, sel[h]).float().mean().item() for h in range(28)) / 28
    print(f"C4 needle-page recall at 128 pages: {recall:.3f}", flush=True)


@pytest.mark.parametrize("S,kb", [(1000, 100), (777, 64), (50, 2048)])
def test_quest_decode_ragged(dev, S, kb):
    """Partial last page (clamped, repeated row S-1) and a budget above the cache."""
    x = W.dense(1, 8, 2, 128, S, seed=S)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    out, pid = Q.quest_decode(q, k, v, kb, 0.09, return_pages=True)
    rpid, rtok, _ = R.quest_select(x["q"], x["k"], kb, 16, 0.09)
    assert torch.equal(pid.cpu().long(), rpid)
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], rtok, 0.09), f"quest S{S} kb{kb}")


def test_quest_decode_causal_position(dev):
    x = W.dense(1, 8, 2, 128, 2000, seed=4)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    pos = 1234
    out = Q.quest_decode(q, k, v, 256, 0.09, pos=pos)
    # restatement: bounds with causal page mask -> top pages -> attend rows <= pos
    rmin, rmax = R.quest_page_minmax(x["k"], 16)
    b = R.quest_page_scores(x["q"], rmin, rmax, 0.09)
    pg = torch.arange(b.shape[-1])
    b = torch.where(pg * 16 <= pos, b, torch.full_like(b, float("-inf")))
    pidx = R.topk_indices(b, 16)
    tok = (pidx.unsqueeze(-1) * 16 + torch.arange(16)).reshape(1, 8, -1).clamp(max=1999)
    tok = torch.where(tok <= pos, tok, torch.full_like(tok, -1))
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], tok, 0.09), "quest pos 1234")


@pytest.mark.parametrize("B,Hq,Hk,np_,npick,page,S,lim", [
    (1, 8, 2, 64, 8, 16, 1000, 1000),        # np = one wave's 64 lanes
    (2, 6, 3, 777, 100, 8, 6200, 5000),      # ragged np, rows past limit masked
    (1, 4, 1, 2048, 128, 16, 32768, 32768),  # the C4 page count
    (1, 4, 4, 3000, 1, 16, 48000, 47000),    # np above 2048 (64 bounds per lane), one page
    (1, 2, 1, 4096, 4096, 4, 16384, 16384),  # every page
])
def test_quest_gather_selects_like_topk_then_gather(dev, B, Hq, Hk, np_, npick, page, S, lim):
    """The in-kernel page selection equals bytes_topk (unsorted) + gather bit for
    bit, on integer-valued bounds (many ties) with -inf and +inf entries."""
    from bytes_amd.sparse import sparse_gather_attn, topk_indices
    g = torch.Generator().manual_seed(np_ + npick)
    x = W.dense(B, Hq, Hk, 128, S, seed=np_)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    bound = torch.randint(-20, 20, (B, Hq, np_), generator=g).float()
    bound[..., 5::17] = float("-inf")
    bound[..., 3::29] = float("inf")
    bound = bound.to(dev)
    got = Q.quest_gather_attn(q, k, v, bound, npick, 0.09, page=page, limit=lim)
    pid = topk_indices(bound, npick, sorted=False)
    assert torch.equal(pid.cpu().long(), R.topk_indices(bound.cpu(), npick).sort(-1).values)
    want = sparse_gather_attn(q, k, v, pid, 0.09, page=page, limit=lim)
    assert got.shape == want.shape and torch.equal(got, want)


def test_quest_decode_fused_path_c4(dev):
    """BASELINE C4 through the default (fused) path: the same output as the
    unfused pipeline with ascending page ids, bit for bit, and the oracle's
    within tolerance."""
    from bytes_amd.sparse import sparse_gather_attn
    x = W.c4_quest(seed=0)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    sc = x["scale"]
    meta = Q.quest_page_minmax(k, 16)
    out = Q.quest_decode(q, k, v, 2048, sc, meta=meta)
    pid = Q.quest_select_pages(q, meta[0], meta[1], 32768, 2048, 16, sc, sorted=False)
    assert torch.equal(out, sparse_gather_attn(q, k, v, pid, sc, page=16))
    rpid, rtok, _ = R.quest_select(x["q"], x["k"], 2048, 16, sc)
    assert torch.equal(pid.cpu().long(), rpid.sort(-1).values)
    _check(out, R.sparse_gather_attn(x["q"], x["k"], x["v"], rtok, sc), "C4 quest decode (fused)")
