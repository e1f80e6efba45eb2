"""Token-level sparse decode: scoring, deterministic top-k, gather attention.

Drop-in replacements for the reference's two-pass sparse decode
(src/attention_kernels.py:987-1263) plus the group-shared token top-k
pipeline: every score, selection and attention step is a gfx950 HIP kernel
launched through the C ABI on the current stream.  The top-k is
deterministic: score descending, lowest index first among equal scores.
"""
from __future__ import annotations

import torch

from . import _checks as C
from ._lib import HIP_ERROR_NOT_SUPPORTED, call, lib, ptr, size_query, stream_of, workspace

TOPK_HIST_ROWS = 1024         # rows whose digit histogram fits the top-k workspace's fixed region


def _qk_shapes(q: torch.Tensor, k: torch.Tensor, k_dim: int = None):
    """Shapes of q [B,H_q,1,D] against keys [B,H_k,S,D]; k_dim overrides the
    keys' last extent (packed codes store D*bits/8 bytes per row)."""
    C.cuda_tensors(q, k)
    C.ndim(q, 4, "q"), C.ndim(k, 4, "k")
    C.dtype_in(q, "q", torch.bfloat16)
    B, Hq, one, D = q.shape
    Bk, Hk, S, Dk = k.shape
    if k_dim is not None:
        Dk = k_dim
    if one != 1 or Dk != D or Bk != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}")
    if Hq % Hk != 0:
        raise ValueError(f"H_q={Hq} is not a multiple of H_k={Hk}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    if S == 0:
        raise ValueError("empty KV cache (S == 0)")
    return B, Hq, Hk, S, D


def _score(q, k_score, scaling, group_sum: bool, hist=None, packed=None, out=None) -> torch.Tensor:
    """Launch the score kernel. packed = (scale, zero, bits) marks k_score as
    uint8 4/2-bit codes along head_dim with bf16 per-32-dim scale/min.  out:
    an fp32 [B, H, S] destination (unit stride along S, any other strides),
    else a new tensor."""
    if packed is None:
        B, Hq, Hk, S, D = _qk_shapes(q, k_score)
        if k_score.dtype not in (torch.bfloat16, torch.float8_e4m3fn):
            raise ValueError(f"k_score: dtype {k_score.dtype} not supported (bf16 or float8_e4m3fn)")
        mode = int(k_score.dtype == torch.float8_e4m3fn)
        sc = zr = None
        m_strides = (0, 0, 0)
    else:
        scale, zero, bits = packed
        if bits not in (4, 2):
            raise ValueError(f"score_bits={bits}: packed keys are 4 or 2 bits")
        C.dtype_in(k_score, "k_packed", torch.uint8)
        nb = k_score.shape[-1]
        if (nb * 8) % bits:
            raise ValueError(f"k_packed last dim {nb} does not hold whole {bits}-bit codes")
        B, Hq, Hk, S, D = _qk_shapes(q, k_score, k_dim=nb * 8 // bits)
        for name, t in (("scale", scale), ("zero", zero)):
            C.cuda_tensors(q, t)
            C.dtype_in(t, name, torch.bfloat16)
            if tuple(t.shape) != (B, Hk, S, D // 32):
                raise ValueError(f"{name}: expected shape {(B, Hk, S, D // 32)}, got {tuple(t.shape)}")
        mode = 2 if bits == 4 else 3
        sc = C.rows16(scale, D // 32 * 2)
        zr = C.rows16(zero, D // 32 * 2)
        if sc.stride() != zr.stride():
            sc, zr = sc.contiguous(), zr.contiguous()
        m_strides = (sc.stride(0), sc.stride(1), sc.stride(2))
    if group_sum and Hq // Hk > 16:
        raise ValueError("group-summed scores support query groups of at most 16 heads")
    qs = C.rows16(q.squeeze(2))
    k = C.rows16(k_score)
    H = Hk if group_sum else Hq
    if out is None:
        out = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != (B, H, S) or out.stride(-1) != 1:
        raise ValueError(f"out: expected fp32 {(B, H, S)} with unit stride along S")
    call("bytes_sparse_score", ptr(qs), ptr(k), mode, ptr(sc) if sc is not None else None,
         ptr(zr) if zr is not None else None, ptr(out), B, Hq, Hk, S, D, int(group_sum),
         qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2), *m_strides,
         out.stride(0), out.stride(1), float(scaling), hist, stream_of(q))
    return out


def sparse_score_scalar(q: torch.Tensor, k_score: torch.Tensor, scaling: float, *, score_bits: int = 16,
                        BLOCK_N: int = 128) -> torch.Tensor:
    """Pass 1: fp32 scores[b, h, t] = (q[b, h] . k[b, h // G, t]) * scaling.

    Replaces src/attention_kernels.py:1113-1133.  q [B,H_q,1,D] bf16;
    k_score [B,H_k,S,D] bf16 (score_bits=16) or float8_e4m3fn (score_bits=8).
    Returns [B,H_q,S] fp32.
    """
    want = {16: torch.bfloat16, 8: torch.float8_e4m3fn}.get(score_bits)
    if want is None or k_score.dtype != want:
        raise ValueError(f"score_bits={score_bits} with k_score {k_score.dtype}: use 16 with bf16 or 8 with "
                         "float8_e4m3fn keys (packed 4/2-bit keys: sparse_score_packed)")
    return _score(q, k_score, scaling, group_sum=False)


def sparse_score_packed(q: torch.Tensor, k_packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor,
                        scaling: float, *, score_bits: int = 4, group_size: int = 32,
                        BLOCK_N: int = 128) -> torch.Tensor:
    """Pass 1 on packed keys: fp32 scores[b, h, t] = (q[b, h] . k_hat[b, h // G, t]) * scaling
    with k_hat = code * scale + zero per 32-dim group.

    Replaces src/attention_kernels.py:1199-1222.  q [B,H_q,1,D] bf16;
    k_packed uint8 [B,H_k,S,D*score_bits/8] (layout of
    quantize_and_pack_score_keys); scale, zero bf16 [B,H_k,S,D/32] (the
    dtype the packer gives bf16 keys).
    group_size must be 32 (every reference caller's value).  Returns
    [B,H_q,S] fp32."""
    if group_size != 32:
        raise ValueError(f"group_size={group_size} not supported (32)")
    return _score(q, k_packed, scaling, group_sum=False, packed=(scale, zero, score_bits))


def quantize_and_pack_score_keys(k: torch.Tensor, score_bits: int, group_size: int):
    """Asymmetric min/max quantization of keys along head_dim in groups of 32,
    packed to uint8 (element c at bits score_bits*(c % (8/score_bits)) of byte
    c // (8/score_bits)).  Replaces src/attention_kernels.py:1225-1249:
    k [B,H_k,S,D] bf16/fp16/fp32 -> (packed uint8 [B,H_k,S,D*score_bits/8],
    scale [B,H_k,S,D/32], zero [B,H_k,S,D/32]) in k's dtype."""
    C.cuda_tensors(k)
    C.ndim(k, 4, "k")
    if score_bits not in (4, 2):
        raise ValueError("Unsupported score_bits")
    if group_size != 32:
        raise ValueError(f"group_size={group_size} not supported (32)")
    dt = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}.get(k.dtype)
    if dt is None:
        raise ValueError(f"k: dtype {k.dtype} not supported (bf16, fp16 or fp32)")
    B, Hk, S, D = k.shape
    if D % 32:
        raise ValueError(f"head_dim {D} is not a multiple of 32")
    x = k.reshape(-1, D)
    if x.stride(-1) != 1:
        x = x.contiguous()
    rows = x.shape[0]
    packed = torch.empty((B, Hk, S, D * score_bits // 8), dtype=torch.uint8, device=k.device)
    scale = torch.empty((B, Hk, S, D // 32), dtype=k.dtype, device=k.device)
    zero = torch.empty_like(scale)
    call("bytes_score_keys_pack", ptr(x), dt, rows, D, x.stride(0) if rows else D, score_bits, ptr(packed),
         ptr(scale), ptr(zero), stream_of(k))
    return packed, scale, zero


def group_scores(q: torch.Tensor, k: torch.Tensor, scaling: float) -> torch.Tensor:
    """Selection score of each KV head, summed over its query group:
    s[b, hk, t] = sum_{g < G} (q[b, hk*G + g] . k[b, hk, t]) * scaling.
    Returns [B,H_k,S] fp32."""
    return _score(q, k, scaling, group_sum=True)


def topk_indices(scores: torch.Tensor, k: int, *, sorted: bool = True) -> torch.Tensor:
    """Indices of the k largest scores per row of [..., n] fp32 under one total
    order: score descending, lowest index first among equal scores (+0 == -0;
    NaN ranks above +inf).  sorted=True orders the result by that order, like
    `scores.topk(k).indices` (src/attention_kernels.py:1262) with a
    deterministic tie rule, for any k (above 8192 the selection is sorted in
    blocks of 8192 and merged by rank); sorted=False returns the same set by
    ascending index (cheaper: no sort).  Returns int32 [..., k]."""
    return _topk(scores, k, sorted=sorted)


def _topk_workspace(device, rows: int, n: int, k: int) -> torch.Tensor:
    return workspace(device, size_query("bytes_topk_workspace_size", rows, n, int(k)), "topk")


def _topk(scores: torch.Tensor, k: int, *, sorted: bool, ws=None, hist_ready: bool = False) -> torch.Tensor:
    C.cuda_tensors(scores)
    C.dtype_in(scores, "scores", torch.float32)
    n = scores.shape[-1]
    if not 1 <= k <= n:
        raise ValueError(f"k={k} outside [1, {n}]")
    s = scores.reshape(-1, n)
    if s.stride(-1) != 1:
        s = s.contiguous()
    rows = s.shape[0]
    out = torch.empty((rows, k), dtype=torch.int32, device=scores.device)
    if ws is None:
        ws = _topk_workspace(scores.device, rows, n, k)
    call("bytes_topk", ptr(s), rows, n, s.stride(0), int(k), int(bool(sorted)), int(bool(hist_ready)), ptr(out),
         out.stride(0), ptr(ws), ws.numel(), stream_of(scores))
    return out.reshape(*scores.shape[:-1], k)


def sparse_gather_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor, scaling: float,
                       BLOCK_K: int = 64, *, chunk: int = 0, page: int = 1, limit=None) -> torch.Tensor:
    """Pass 2: exact attention over the gathered rows.

    Replaces src/attention_kernels.py:1037-1059.  q [B,H_q,1,D] bf16; k, v
    [B,H_k,S,D] bf16 or float8_e4m3fn; idx [B,H_q,kb] (per query head, the
    reference layout) or [B,H_k,kb] (one selection per KV head, shared by its
    query group), any integer dtype.  Entries outside [0, S) are masked
    (sentinel rule of benchmarks/sparse_attention.py:376).  Returns
    [B,H_q,1,D] bf16 (also for fp8 values, :1044).

    page > 1: idx holds page ids, each standing for rows p*page .. p*page+page-1
    clamped to S-1 (the Quest expansion, benchmarks/sparse_attention.py:360-363).
    limit: rows at or past it are masked (the causal bound pos+1; default S).
    """
    page = int(page)
    if page < 1:
        raise ValueError(f"page={page} must be >= 1")
    if limit is not None and not 0 <= int(limit) <= k.shape[2]:
        raise ValueError(f"limit={limit} outside [0, S]")
    B, Hq, Hk, S, D = _qk_shapes(q, k)
    C.cuda_tensors(q, v, idx)
    C.dtype_in(k, "k", torch.bfloat16, torch.float8_e4m3fn)
    C.dtype_in(v, "v", k.dtype)
    if tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"shape mismatch: k {tuple(k.shape)}, v {tuple(v.shape)}")
    if idx.dim() != 3 or idx.shape[0] != B or idx.shape[1] not in (Hq, Hk):
        raise ValueError(f"idx must be [B, H_q or H_k, kb]; got {tuple(idx.shape)}")
    kb = idx.shape[-1]
    if kb == 0:
        raise ValueError("empty index list")
    per_head = 1 if idx.shape[1] == Hq else 0
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    qs = C.rows16(q.squeeze(2))
    k, v = C.rows16(k), C.rows16(v)
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=q.device)
    if page == 1:
        page = 0                                    # plain row indices
    nbytes = size_query("bytes_gather_attn_workspace_size", B, Hq, Hk, kb * max(page, 1), D, per_head, int(chunk))
    ws = workspace(q.device, nbytes)
    call("bytes_gather_attn", ptr(qs), ptr(k), ptr(v), int(k.dtype == torch.float8_e4m3fn), ptr(idx), ptr(out),
         B, Hq, Hk, S, D, kb * max(page, 1),
         per_head, page, S if limit is None else int(limit), qs.stride(0), qs.stride(1),
         k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2),
         idx.stride(0), idx.stride(1), out.stride(0), out.stride(1), float(scaling), int(chunk), ptr(ws),
         ws.numel(), stream_of(q))
    return out.unsqueeze(2)


def budget(frac: float, S: int) -> int:
    """kb = max(1, round(frac * S)), as src/attention_kernels.py:1261."""
    return max(1, int(round(frac * S)))


def sparse_decode_scalar(q, k_score_or_packed, scale, zero, k_val, v_val, frac, scaling, *, score_bits,
                         group_size=32, BLOCK_N=128, BLOCK_K=64):
    """Two-pass sparse decode: score every key, keep the top kb = max(1, round(frac*S))
    per query head, attend exactly over them.  Replaces
    src/attention_kernels.py:1252-1263: bf16 (score_bits=16) or fp8
    (score_bits=8) score keys, or packed 4/2-bit keys with their `scale` and
    `zero` (score_bits=4/2, group_size=32).  Returns [B,H_q,1,D] bf16."""
    if score_bits in (16, 8):
        scores = sparse_score_scalar(q, k_score_or_packed, scaling, score_bits=score_bits)
    else:
        scores = sparse_score_packed(q, k_score_or_packed, scale, zero, scaling, score_bits=score_bits,
                                     group_size=group_size)
    kb = budget(frac, scores.shape[-1])
    idx = topk_indices(scores, kb, sorted=False)      # attention does not depend on the order
    return sparse_gather_attn(q, k_val, v_val, idx, scaling)


def token_topk_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kb: int, scaling: float, *,
                      k_score: torch.Tensor = None, score_scale: torch.Tensor = None,
                      score_zero: torch.Tensor = None, score_bits: int = None):
    """Group-shared token top-k decode: group-summed fp32 scores per KV head,
    the kb best tokens per (b, KV head), attention of every query head of the
    group over them.  `k_score` (default k) holds the keys the selection scores
    use: a float8_e4m3fn copy of the cache, or packed 4/2-bit codes (uint8,
    with score_scale, score_zero and score_bits as quantize_and_pack_score_keys
    gives them).  Returns (out [B,H_q,1,D] bf16, idx [B,H_k,kb] int32 by
    ascending token index)."""
    ks = k if k_score is None else k_score
    packed = None
    if ks.dtype == torch.uint8:
        if score_bits not in (4, 2) or score_scale is None or score_zero is None:
            raise ValueError("packed score keys need score_bits 4 or 2 with score_scale and score_zero")
        packed = (score_scale, score_zero, score_bits)
        B, Hq, Hk, S, D = _qk_shapes(q, ks, k_dim=ks.shape[-1] * 8 // score_bits)
        if tuple(ks.shape[:3]) != tuple(k.shape[:3]) or D != k.shape[-1]:
            raise ValueError(f"packed score keys {tuple(ks.shape)} do not match k {tuple(k.shape)}")
    else:
        B, Hq, Hk, S, D = _qk_shapes(q, ks)
        if tuple(ks.shape) != tuple(k.shape):
            raise ValueError(f"k_score {tuple(ks.shape)} does not match k {tuple(k.shape)}")
    if B * Hk <= TOPK_HIST_ROWS:
        # the score kernel also counts the top-k digit histogram, in the top-k workspace
        ws = _topk_workspace(q.device, B * Hk, S, kb)
        s = _score(q, ks, scaling, group_sum=True, hist=ptr(ws), packed=packed)
        idx = _topk(s, kb, sorted=False, ws=ws, hist_ready=True)
    else:
        s = _score(q, ks, scaling, group_sum=True, packed=packed)
        idx = topk_indices(s, kb, sorted=False)
    return sparse_gather_attn(q, k, v, idx, scaling), idx
