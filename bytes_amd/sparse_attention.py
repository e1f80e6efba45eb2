"""Selection and attention over query chunks: drop-ins for the functions of
benchmarks/sparse_attention.py that the chunked sparse-attention driver
(`sparse_attention_chunked`, :463-496) calls for each block of Qc >= 1 query
rows.

- `select_topk(selector, ...)` (:226-325) for the "exact"/"approx" selectors
  (exact fp32 scores of the keys the caller passes) and "quest";
- `_quest_select(...)` (:328-364);
- `attend_topk(...)` (:367-387).

Row (h, qc) of a chunk is run as query head h*Qc + qc of the same KV head
(h // G), so the single-query kernels serve every row: the score kernel, the
Quest bound kernel, the deterministic top-k and the gather-attention kernel,
with the per-row causal mask, forced recent window and sentinel rule applied
by the select kernels (csrc/select.hip).  Positions `q_pos` may be a host or
device tensor; the host needs max(q_pos) (as the reference does, :295).

Differences from the reference, each deliberate:
- ties rank by lowest index (the reference's torch.topk tie order is
  unspecified); a slot a row cannot fill holds the sentinel S, also where the
  reference's tie order could name a masked future key;
- `k_chunk` is accepted and does not change the result: the streaming merge
  of :301-309 selects the same set as one selection over all keys under a
  total order, so the scores of a whole chunk of rows are ranked at once
  (memory B*Hq*Qc*max(q_pos) fp32 scores);
- outputs are ordered by score (descending) when k <= 8192, else by
  ascending index;
- attend_topk accumulates its weighted sum in fp32 (the reference casts the
  weights to v's dtype first).
"""
from __future__ import annotations

import torch

from . import _checks as C
from ._lib import call, ptr, stream_of
from .quest import quest_page_minmax, quest_page_scores
from .sparse import TOPK_MAX, _score, sparse_gather_attn, topk_indices

SELECTORS = ("exact", "approx", "quest")


def _positions(q_pos, Qc: int, device):
    """(int64 positions on `device` [Qc], max position) from an int, a sequence
    or a tensor of Qc positions."""
    if isinstance(q_pos, torch.Tensor):
        p = q_pos.reshape(-1)
        if p.numel() == 1 and Qc > 1:
            raise ValueError(f"q_pos holds 1 position for Qc={Qc} query rows")
        host = p if p.device.type == "cpu" else None
        p = p.to(device=device, dtype=torch.int64)
    else:
        vals = [int(x) for x in (q_pos if isinstance(q_pos, (list, tuple)) else [q_pos])]
        host = torch.tensor(vals, dtype=torch.int64)
        p = host.to(device)
    if p.numel() != Qc:
        raise ValueError(f"q_pos holds {p.numel()} positions for Qc={Qc} query rows")
    pmax = int((host if host is not None else p).max().item())
    pmin = int((host if host is not None else p).min().item())
    if pmin < 0:
        raise ValueError("negative query position")
    return p.contiguous(), pmax


def _fold(q_blk: torch.Tensor) -> torch.Tensor:
    C.cuda_tensors(q_blk)
    C.ndim(q_blk, 4, "q_blk")
    B, Hq, Qc, D = q_blk.shape
    return q_blk.reshape(B, Hq * Qc, 1, D)


def _mask(s: torch.Tensor, pos: torch.Tensor, Qc: int, unit: int, local_w: int) -> None:
    n = s.shape[-1]
    call("bytes_select_mask", ptr(s), s.numel() // n, n, n, ptr(pos), Qc, int(unit), int(local_w), stream_of(s))


def _fill(idx: torch.Tensor, pos: torch.Tensor, Qc: int, S: int, k_out: int, dtype) -> torch.Tensor:
    """idx [..., k_in] -> [..., k_out]: entries that are negative, >= S or past
    their row's position become S; slots past k_in are S."""
    k_in = idx.shape[-1]
    src = idx.reshape(-1, k_in)
    if src.dtype not in (torch.int32, torch.int64):
        src = src.to(torch.int64)
    if src.stride(-1) != 1:
        src = src.contiguous()
    rows = src.shape[0]
    out = torch.empty((rows, k_out), dtype=dtype, device=idx.device)
    call("bytes_select_fill", ptr(src), int(src.dtype == torch.int64), src.stride(0), k_in, ptr(out),
         int(dtype == torch.int64), out.stride(0), k_out, rows, ptr(pos), Qc, int(S), stream_of(idx))
    return out.reshape(*idx.shape[:-1], k_out)


def select_topk(selector, q_blk, sel_keys, q_pos, S, kb, k_chunk, scaling, page=16, generator=None, local_w=0):
    """Top-kb causal key indices per query row (benchmarks/sparse_attention.py:226-325).

    q_blk [B,Hq,Qc,D] bf16; sel_keys [B,Hq,S,D] (GQA-expanded, as the
    reference passes them) or [B,Hk,S,D] bf16 / float8_e4m3fn: the keys of
    the selector's score space; q_pos [Qc] positions.  "exact" / "approx":
    fp32 scores (q . k) * scaling of keys 0..max(q_pos), keys past a row's
    position masked, the `local_w` most recent forced in; returns int64
    [B,Hq,Qc,kb], slots a row cannot fill hold S.  "quest": `_quest_select`.
    Other selectors raise ValueError."""
    if selector == "quest":
        return _quest_select(q_blk, sel_keys, q_pos, S, kb, page, scaling, local_w)
    if selector not in SELECTORS:
        raise ValueError(f"selector {selector!r} not supported ({', '.join(SELECTORS)})")
    if kb < 1:
        raise ValueError(f"kb={kb} must be >= 1")
    qf = _fold(q_blk)
    B, Hq, Qc, D = q_blk.shape
    pos, pmax = _positions(q_pos, Qc, q_blk.device)
    max_key = min(pmax + 1, int(S), sel_keys.shape[2])
    s = _score(qf, sel_keys[:, :, :max_key], scaling, group_sum=False)      # [B, Hq*Qc, max_key]
    _mask(s, pos, Qc, 1, local_w)
    kk = min(int(kb), max_key)
    sel = topk_indices(s, kk, sorted=kk <= TOPK_MAX)
    return _fill(sel, pos, Qc, S, int(kb), torch.int64).reshape(B, Hq, Qc, int(kb))


def _quest_select(q_blk, k_r, pos, S, kb, page, scaling, local_w=0):
    """Quest page selection for Qc >= 1 query rows
    (benchmarks/sparse_attention.py:328-364).

    q_blk [B,Hq,Qc,D] bf16; k_r [B,Hq,S,D] (GQA-expanded, as the reference
    passes it) or [B,Hk,S,D] bf16; pos [Qc] positions.  Page bounds
    sum_d max(q_d*kmin_d, q_d*kmax_d) * scaling in fp32 over pages of `page`
    tokens (the last padded with the last key), pages starting after a row's
    position at -inf, pages overlapping its `local_w` most recent tokens at
    +inf, the top ceil(kb/page) pages per row (lowest page first on ties),
    expanded to token ids clamped to S-1.  Returns int64 [B,Hq,Qc,npick*page]."""
    qf = _fold(q_blk)
    B, Hq, Qc, D = q_blk.shape
    p, _ = _positions(pos, Qc, q_blk.device)
    S = int(S)
    kmin, kmax = quest_page_minmax(k_r[:, :, :S], page)
    np_ = kmin.shape[2]
    bound = quest_page_scores(qf, kmin, kmax, scaling, page=page, pos=np_ * page, local_w=0)
    _mask(bound, p, Qc, page, local_w)
    npick = min(max(1, (int(kb) + page - 1) // page), np_)
    pid = topk_indices(bound, npick, sorted=npick <= TOPK_MAX).contiguous()
    tok = torch.empty((B, Hq, Qc, npick * page), dtype=torch.int64, device=q_blk.device)
    call("bytes_select_pages", ptr(pid), pid.numel() // npick, npick, int(page), S, ptr(tok), stream_of(pid))
    return tok


def attend_topk(q_blk, k_r, v, idx, q_pos, scaling):
    """Exact attention of each query row over its selected keys
    (benchmarks/sparse_attention.py:367-387).

    q_blk [B,Hq,Qc,D] bf16; k_r, v [B,Hq,S,D] or [B,Hk,S,D] bf16 (or
    float8_e4m3fn); idx [B,Hq,Qc,ksel] integer; q_pos [Qc].  Entries past the
    row's position, negative or >= S take no part.  Returns [B,Hq,Qc,D] bf16."""
    qf = _fold(q_blk)
    B, Hq, Qc, D = q_blk.shape
    if idx.dim() != 4 or tuple(idx.shape[:3]) != (B, Hq, Qc):
        raise ValueError(f"idx must be [B, Hq, Qc, ksel] = [{B}, {Hq}, {Qc}, .]; got {tuple(idx.shape)}")
    C.cuda_tensors(idx)
    pos, _ = _positions(q_pos, Qc, q_blk.device)
    S = k_r.shape[2]
    rows = _fill(idx, pos, Qc, S, idx.shape[-1], torch.int32).reshape(B, Hq * Qc, idx.shape[-1])
    out = sparse_gather_attn(qf, k_r, v, rows, scaling)
    return out.reshape(B, Hq, Qc, D)
