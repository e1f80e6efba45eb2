"""Selection and attention over query chunks: drop-ins for the functions of
benchmarks/sparse_attention.py that the chunked sparse-attention driver
(`sparse_attention_chunked`, :463-496) calls for each block of Qc >= 1 query
rows.

- `select_topk(selector, ...)` (:226-325): "exact", "approx", "int4", "int2"
  and "fp8" (the streaming top-k over the fp32 scores of whatever keys the
  caller passes, as the reference runs every one of them), "recent"
  (:261-265) and "quest";
- `_quest_select(...)` (:328-364);
- `attend_topk(...)` (:367-387).

Row (h, qc) of a chunk is run as query head h*Qc + qc of the same KV head
(h // G), so the single-query kernels serve every row: the score kernel, the
Quest bound kernel, the deterministic top-k and the gather-attention kernel,
with the per-row causal mask, forced recent window, streaming merge and
sentinel rule applied by the select kernels (csrc/select.hip).  Positions
`q_pos` may be a host or device tensor; the host needs max(q_pos) (as the
reference does, :295).

The streaming top-k keeps the reference's memory bound (:286-309, stated at
:477): keys are scored k_chunk at a time into a buffer that holds the running
list of kb (score, index) pairs followed by the chunk, the top kb of it
become the next running list, so the extra memory is
O(B * Hq * Qc * (k_chunk + kb)) whatever the context length.

Differences from the reference, each deliberate:
- ties rank by lowest index (the reference's torch.topk tie order is
  unspecified); a slot a row cannot fill holds the sentinel S, also where the
  reference's tie order could name a masked future key;
- attend_topk accumulates its weighted sum in fp32 (the reference casts the
  weights to v's dtype first).
"""
from __future__ import annotations

import torch

from . import _checks as C
from ._lib import call, ptr, stream_of
from .quest import quest_page_minmax, quest_page_scores
from .sparse import _score, _topk, sparse_gather_attn, topk_indices

# selectors that rank by exact fp32 scores of the keys passed in (the
# reference's "exact" and its SOFT_SELECTORS other than "signvq", :35, which
# all reach the same streaming top-k over the sel_keys they are given)
SCORE_SELECTORS = ("exact", "approx", "int4", "int2", "fp8")
SELECTORS = SCORE_SELECTORS + ("recent", "quest")


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


def _stream_select(qf, sel_keys, pos, Qc: int, S: int, kb: int, k_chunk: int, scaling: float, max_key: int,
                   local_w: int) -> torch.Tensor:
    """The streaming top-k of benchmarks/sparse_attention.py:286-309 over folded
    rows qf [B, Hq*Qc, 1, D]: int32 key indices [B*Hq*Qc, kb] ordered by
    (score desc, index asc), fillers (-inf, S) where a row has fewer than kb
    candidates.

    Each chunk of k_chunk keys is scored into cand[:, kbp:], masked (causal,
    recent window) with its key offset, and the top kb of the row's running
    list (cand[:, kbp - kb:kbp]) plus the chunk become the next running list,
    written to the other buffer.  The running list comes first in each row, so
    the top-k's lowest-position tie rule keeps the lowest key index on equal
    scores; the last merge orders the list by score."""
    B, R1 = qf.shape[0], qf.shape[1]
    rows = B * R1
    dev = qf.device
    kc = max(1, min(int(k_chunk), max_key))
    kbp = (kb + 63) // 64 * 64
    W = kbp + (kc + 63) // 64 * 64
    cand = [torch.empty((rows, W), dtype=torch.float32, device=dev) for _ in range(2)]
    ridx = [torch.empty((rows, kb), dtype=torch.int32, device=dev) for _ in range(2)]
    cur, nrun = 0, 0
    st = stream_of(qf)
    for kc0 in range(0, max_key, kc):
        kc1 = min(kc0 + kc, max_key)
        n = kc1 - kc0
        last = kc1 == max_key
        buf = cand[cur]
        _score(qf, sel_keys[:, :, kc0:kc1], scaling, group_sum=False,
               out=buf.view(B, R1, W)[:, :, kbp:kbp + n])
        call("bytes_select_mask_at", ptr(buf) + 4 * kbp, rows, n, W, kc0, ptr(pos), Qc, 1, int(local_w), st)
        off = kbp - nrun
        ksel = min(kb, nrun + n)
        sel = _topk(buf[:, off:off + nrun + n], ksel, sorted=last)
        nxt = 1 - cur
        call("bytes_select_merge", ptr(buf), W, off, nrun, ptr(ridx[cur]), kb, ptr(sel), sel.stride(0), ksel, kc0,
             int(S), rows, None if last else ptr(cand[nxt]), W, kbp - kb, ptr(ridx[nxt]), kb, kb, st)
        cur, nrun = nxt, kb
    return ridx[cur]


def select_topk(selector, q_blk, sel_keys, q_pos, S, kb, k_chunk, scaling, page=16, generator=None, local_w=0):
    """Top-kb causal key indices per query row (benchmarks/sparse_attention.py:226-325).

    q_blk [B,Hq,Qc,D] bf16; sel_keys [B,Hq,S,D] (GQA-expanded, as the
    reference passes them) or [B,Hk,S,D] bf16 / float8_e4m3fn: the keys of
    the selector's score space; q_pos [Qc] positions.
    "exact" / "approx" / "int4" / "int2" / "fp8": fp32 scores (q . k) * scaling
    of keys 0..max(q_pos), keys past a row's position masked, the `local_w`
    most recent forced in, selected by a streaming top-k over chunks of
    k_chunk keys; returns int64 [B,Hq,Qc,kb] ordered by score (descending,
    lowest index first on ties), slots a row cannot fill hold S.
    "recent": positions pos - j for j < kb, clamped at 0 (:261-265).
    "quest": `_quest_select`.  Other selectors raise ValueError."""
    if selector == "quest":
        return _quest_select(q_blk, sel_keys, q_pos, S, kb, page, scaling, local_w)
    if selector not in SELECTORS:
        raise ValueError(f"selector {selector!r} not supported ({', '.join(SELECTORS)})")
    if kb < 1:
        raise ValueError(f"kb={kb} must be >= 1")
    if k_chunk < 1:
        raise ValueError(f"k_chunk={k_chunk} must be >= 1")
    qf = _fold(q_blk)
    B, Hq, Qc, D = q_blk.shape
    pos, pmax = _positions(q_pos, Qc, q_blk.device)
    kb = int(kb)
    if selector == "recent":
        out = torch.empty((B, Hq, Qc, kb), dtype=torch.int64, device=q_blk.device)
        call("bytes_select_recent", ptr(pos), Qc, B * Hq * Qc, kb, ptr(out), stream_of(q_blk))
        return out
    max_key = min(pmax + 1, int(S), sel_keys.shape[2])
    sel = _stream_select(qf, sel_keys, pos, Qc, int(S), kb, int(k_chunk), scaling, max_key, local_w)
    return _fill(sel, pos, Qc, S, kb, torch.int64).reshape(B, Hq, Qc, kb)


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
    pid = topk_indices(bound, npick, sorted=True).contiguous()
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
