"""Quest page-sparse decode: page metadata, page bounds, page top-k, gather.

Keeps the call surface of benchmarks/sparse_attention.py:328-387
(`_quest_select`, then `attend_topk` over the selected keys) for one decode
query, with every step on a gfx950 HIP kernel: page min/max metadata, fp32
page bounds (bit-identical to a sequential fp32 sum over d), the
deterministic top-k over pages (bound descending, lowest page first on ties)
and gather attention that expands page ids to rows while staging them.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _checks as C
from ._lib import call, ptr, size_query, stream_of, workspace
from .sparse import _qk_shapes, sparse_gather_attn, topk_indices


def quest_page_minmax(k: torch.Tensor, page: int = 16) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-page elementwise min/max of k [B,H,S,D] bf16 over pages of `page`
    tokens, the last partial page padded with the last key
    (benchmarks/sparse_attention.py:336-341).  Returns (kmin, kmax)
    [B,H,ceil(S/page),D] bf16 (exact: min/max of bf16 values)."""
    C.cuda_tensors(k)
    C.ndim(k, 4, "k")
    C.dtype_in(k, "k", torch.bfloat16)
    B, H, S, D = k.shape
    if S == 0 or page < 1 or D % 8 != 0:
        raise ValueError(f"bad shape/page: k {tuple(k.shape)}, page {page}")
    k = C.rows16(k)
    np_ = (S + page - 1) // page
    kmin = torch.empty((B, H, np_, D), dtype=k.dtype, device=k.device)
    kmax = torch.empty_like(kmin)
    call("bytes_quest_page_minmax", ptr(k), ptr(kmin), ptr(kmax), B, H, S, D, int(page),
         k.stride(0), k.stride(1), k.stride(2), stream_of(k))
    return kmin, kmax


def quest_page_scores(q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor, scaling: float = 1.0, *,
                      page: int = 16, pos: Optional[int] = None, local_w: int = 0) -> torch.Tensor:
    """bound[b,h,p] = scaling * sum_d max(q_d*kmin_d, q_d*kmax_d) in fp32
    (benchmarks/sparse_attention.py:342-345), -inf for pages starting after
    `pos` (default: the last cached token) and +inf for pages overlapping the
    `local_w` most recent tokens (:346-355).  q [B,H_q,1,D] bf16;
    kmin/kmax [B,H_k,np,D] bf16.  Returns [B,H_q,np] fp32."""
    C.cuda_tensors(q, kmin, kmax)
    C.ndim(q, 4, "q")
    C.dtype_in(q, "q", torch.bfloat16)
    C.dtype_in(kmin, "kmin", torch.bfloat16)
    C.dtype_in(kmax, "kmax", torch.bfloat16)
    B, Hq, one, D = q.shape
    _, Hk, np_, Dm = kmin.shape
    if one != 1 or Dm != D or tuple(kmax.shape) != tuple(kmin.shape) or kmin.shape[0] != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, kmin {tuple(kmin.shape)}, kmax {tuple(kmax.shape)}")
    if Hq % Hk != 0:
        raise ValueError(f"H_q={Hq} is not a multiple of H_k={Hk}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    kmin, kmax = kmin.contiguous(), kmax.contiguous()
    qs = C.rows16(q.squeeze(2))
    if pos is None:
        pos = np_ * page - 1
    bound = torch.empty((B, Hq, np_), dtype=torch.float32, device=q.device)
    call("bytes_quest_page_scores", ptr(qs), ptr(kmin), ptr(kmax), ptr(bound), B, Hq, Hk, np_, D, int(page),
         int(pos), int(local_w), qs.stride(0), qs.stride(1), bound.stride(0), bound.stride(1), float(scaling),
         stream_of(q))
    return bound


def _npick(kb: int, page: int, np_: int) -> int:
    return min(max(1, (kb + page - 1) // page), np_)        # benchmarks/sparse_attention.py:356-357


def quest_select_pages(q, kmin, kmax, S: int, kb: int, page: int, scaling: float, *, pos: Optional[int] = None,
                       local_w: int = 0, sorted: bool = True) -> torch.Tensor:
    """Page ids [B,H_q,npick] int32 of the top ceil(kb/page) page bounds, ordered
    by bound descending with the lowest page first among equal bounds
    (sorted=False: the same pages by ascending page id)."""
    bound = quest_page_scores(q, kmin, kmax, scaling, page=page, pos=S - 1 if pos is None else pos,
                              local_w=local_w)
    return topk_indices(bound, _npick(kb, page, bound.shape[-1]), sorted=sorted)


def _quest_select(q_blk, k_r, pos, S, kb, page, scaling, local_w=0):
    """Drop-in for benchmarks/sparse_attention.py:328-364 for Qc >= 1 query
    rows (see bytes_amd.sparse_attention._quest_select): returns token ids
    [B,H_q,Qc,npick*page] int64 of the selected pages, clamped to S-1."""
    from .sparse_attention import _quest_select as qs
    return qs(q_blk, k_r, pos, S, kb, page, scaling, local_w)


_SELECT_IN_GATHER_MAX = 4096        # page-bound rows the gather kernel selects from itself


def quest_gather_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bound: torch.Tensor, npick: int,
                      scaling: float, *, page: int = 16, limit: Optional[int] = None, chunk: int = 0) -> torch.Tensor:
    """The top `npick` pages of each query head's bound row (bound [B,H_q,np]
    fp32; exact: bound descending, lowest page first on equal bounds), attended
    over in one gather launch that selects the pages itself: equal bit for bit
    to topk_indices(bound, npick, sorted=False) followed by
    sparse_gather_attn(..., page=page, limit=limit)
    (benchmarks/sparse_attention.py:356-387).  np <= 4096."""
    B, Hq, Hk, S, D = _qk_shapes(q, k)
    C.cuda_tensors(q, v, bound)
    C.dtype_in(k, "k", torch.bfloat16, torch.float8_e4m3fn)
    C.dtype_in(v, "v", k.dtype)
    C.dtype_in(bound, "bound", torch.float32)
    if tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"shape mismatch: k {tuple(k.shape)}, v {tuple(v.shape)}")
    if bound.dim() != 3 or tuple(bound.shape[:2]) != (B, Hq):
        raise ValueError(f"bound must be [B, H_q, np]; got {tuple(bound.shape)}")
    np_ = bound.shape[-1]
    if not 0 < npick <= np_ or np_ > _SELECT_IN_GATHER_MAX or page < 1:
        raise ValueError(f"npick={npick}, np={np_}, page={page} (need 0 < npick <= np <= {_SELECT_IN_GATHER_MAX})")
    lim = S if limit is None else int(limit)
    if not 0 <= lim <= S:
        raise ValueError(f"limit={limit} outside [0, S]")
    if bound.stride(-1) != 1:
        bound = bound.contiguous()
    qs = C.rows16(q.squeeze(2))
    k, v = C.rows16(k), C.rows16(v)
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=q.device)
    kb = npick * page
    ws = workspace(q.device, size_query("bytes_gather_attn_workspace_size", B, Hq, Hk, kb, D, 1, int(chunk)))
    call("bytes_quest_gather_attn", ptr(qs), ptr(k), ptr(v), int(k.dtype == torch.float8_e4m3fn), ptr(bound),
         bound.stride(0), bound.stride(1), np_, int(npick), ptr(out), B, Hq, Hk, S, D, int(page), lim,
         qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2),
         out.stride(0), out.stride(1), float(scaling), int(chunk), ptr(ws), ws.numel(), stream_of(q))
    return out.unsqueeze(2)


def quest_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kb: int, scaling: float, *, page: int = 16,
                 meta: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, pos: Optional[int] = None,
                 local_w: int = 0, return_pages: bool = False):
    """Quest decode step: page bounds from (kmin, kmax) metadata (computed from k
    when `meta` is None), the top ceil(kb/page) pages per query head, exact
    attention over their rows (rows past `pos` masked, as attend_topk,
    benchmarks/sparse_attention.py:367-387).  q [B,H_q,1,D]; k, v [B,H_k,S,D]
    bf16.  Returns out [B,H_q,1,D] bf16 (and the page ids, ordered by bound
    descending, if return_pages).  Up to 4096 pages, the gather kernel selects
    the pages itself (two launches and the split merge); return_pages and
    longer caches run the page top-k as a launch of its own."""
    S = k.shape[2]
    if meta is None:
        meta = quest_page_minmax(k, page)
    p = S - 1 if pos is None else int(pos)
    if not return_pages and meta[0].shape[2] <= _SELECT_IN_GATHER_MAX:
        bound = quest_page_scores(q, meta[0], meta[1], scaling, page=page, pos=p, local_w=local_w)
        return quest_gather_attn(q, k, v, bound, _npick(kb, page, bound.shape[-1]), scaling, page=page,
                                 limit=p + 1)
    pid = quest_select_pages(q, meta[0], meta[1], S, kb, page, scaling, pos=p, local_w=local_w,
                             sorted=return_pages)
    out = sparse_gather_attn(q, k, v, pid, scaling, page=page, limit=p + 1)
    return (out, pid) if return_pages else out
