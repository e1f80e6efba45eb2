"""Product-quantized KV decode attention and the PQ setup path.

Keeps the call surface of src/attention_kernels.py (`decode_attn_pq_lut_kv`
:471, `decode_attn_pq_lut` :365, `decode_attn_dequant` :267) and
src/quantization.py (`kmeans_pytorch` :102, `ProductQuantizer` :134), with
every step on a gfx950 HIP kernel through the C ABI: the LUT build, the three
decode variants, nearest-codeword encoding (bit-exact argmin) and the k-means
centroid update.

Codebooks: the reference keeps one [M, K, d_sub] codebook per quantizer
(src/quantization.py:145); BASELINE C3 uses one per KV head.  Both layouts
are accepted ([M,K,8] shared or [H_k,M,K,8]); the kernels read fp16 codebooks
and other dtypes are converted once per call.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _checks as C
from ._lib import call, dtype_code, ptr, size_query, stream_of, workspace

D_SUB = 8


def _codebook16(cb: torch.Tensor, Hk: int, name: str):
    """-> (fp16 contiguous codebook, head stride in elements, M, K)."""
    if cb.dim() == 3:
        M, K, ds = cb.shape
        sh = 0
    elif cb.dim() == 4:
        if cb.shape[0] != Hk:
            raise ValueError(f"{name}: per-head codebook needs {Hk} heads, got {tuple(cb.shape)}")
        _, M, K, ds = cb.shape
        sh = M * K * ds
    else:
        raise ValueError(f"{name}: expected [M,K,d_sub] or [H_k,M,K,d_sub], got {tuple(cb.shape)}")
    if ds != D_SUB:
        raise ValueError(f"{name}: d_sub={ds} not supported (8)")
    if not (0 < K <= 256 and K % 4 == 0):
        raise ValueError(f"{name}: K={K} codewords not supported (multiple of 4, <= 256)")
    cb16 = cb.to(torch.float16).contiguous()
    return cb16, sh, M, K


def _codes(idx: torch.Tensor, name: str) -> torch.Tensor:
    """uint8 codes whose token rows are M contiguous bytes on an M-byte boundary
    (the kernels read one token's codes with one 8- or 16-byte load)."""
    if idx.dtype != torch.uint8:
        idx = idx.to(torch.uint8)
    M = idx.shape[-1]
    if idx.stride(-1) != 1 or idx.stride(-2) != M or idx.data_ptr() % 16 != 0:
        idx = idx.contiguous()
    return idx


def _decode(mode: int, *, lut=None, q=None, kcb=None, k_idx, v_idx=None, vcb=None, v=None, out_dtype, B, Hq, Hk,
            S, D, K, dev, chunk=0, scale=1.0):
    out = torch.empty((B, Hq, D), dtype=out_dtype, device=dev)
    nbytes = size_query("bytes_pq_decode_workspace_size", B, Hq, Hk, S, D, int(chunk))
    ws = workspace(dev, nbytes)
    z = lambda t, i: t.stride(i) if t is not None else 0    # noqa: E731
    p = lambda t: ptr(t) if t is not None else None          # noqa: E731
    kcb16, kcb_sh = kcb if kcb is not None else (None, 0)
    vcb16, vcb_sh = vcb if vcb is not None else (None, 0)
    call("bytes_pq_decode_attn", mode, p(lut), p(q), p(kcb16), ptr(k_idx), p(v_idx), p(vcb16), p(v), ptr(out),
         dtype_code(out), B, Hq, Hk, S, D, K, z(lut, 0), z(lut, 1), z(q, 0), z(q, 1), kcb_sh,
         k_idx.stride(0), k_idx.stride(1), k_idx.stride(2), z(v_idx, 0), z(v_idx, 1), z(v_idx, 2), vcb_sh,
         z(v, 0), z(v, 1), z(v, 2), out.stride(0), out.stride(1), float(scale), int(chunk), ptr(ws), ws.numel(),
         stream_of(k_idx))
    return out.unsqueeze(2)


def _lut_checks(lut, k_idx):
    C.cuda_tensors(lut, k_idx)
    C.ndim(lut, 4, "lut"), C.ndim(k_idx, 4, "k_idx")
    if lut.dtype != torch.float32:
        lut = lut.float()
    B, Hq, M, K = lut.shape
    Bk, Hk, S, Mk = k_idx.shape
    if Bk != B or Mk != M or Hq % Hk != 0 or S == 0:
        raise ValueError(f"shape mismatch: lut {tuple(lut.shape)}, k_idx {tuple(k_idx.shape)}")
    if M * D_SUB not in (64, 128):
        raise ValueError(f"M={M} subspaces: head_dim {M * D_SUB} not supported (64 or 128)")
    if not (0 < K <= 256 and K % 4 == 0):
        raise ValueError(f"K={K} codewords not supported (multiple of 4, <= 256)")
    if lut.stride(-1) != 1 or lut.stride(-2) != K or lut.data_ptr() % 16 != 0:
        lut = lut.contiguous()
    return lut, B, Hq, Hk, S, M, K


def decode_attn_pq_lut_kv(lut: torch.Tensor, k_idx: torch.Tensor, v_idx: torch.Tensor, v_centroids: torch.Tensor,
                          d_sub_v: int = 8, *, chunk: int = 0) -> torch.Tensor:
    """LUT-scored keys and codebook-reconstructed values.

    Replaces src/attention_kernels.py:471-500: score_t = sum_j lut[b,h,j,k_idx[t,j]]
    (no scale inside: fold it into the LUT), out = softmax(score) . concat_j
    v_centroids[j, v_idx[t,j]].  lut [B,H_q,M,K] fp32; k_idx, v_idx
    [B,H_k,S,M] integer codes; v_centroids [M,K,8] or [H_k,M,K,8].
    Returns [B,H_q,1,D] in v_centroids' dtype (:484)."""
    if d_sub_v != D_SUB:
        raise ValueError(f"d_sub_v={d_sub_v} not supported (8)")
    lut, B, Hq, Hk, S, M, K = _lut_checks(lut, k_idx)
    C.cuda_tensors(lut, v_idx, v_centroids)
    if tuple(v_idx.shape[:3]) != (B, Hk, S):
        raise ValueError(f"v_idx {tuple(v_idx.shape)} does not match k_idx {tuple(k_idx.shape)}")
    vcb16, vsh, Mv, Kv = _codebook16(v_centroids, Hk, "v_centroids")
    if Mv != M or v_idx.shape[-1] != Mv or Kv != K:
        raise ValueError("value codebook / codes must use the key's subspace and codeword counts")
    return _decode(0, lut=lut, k_idx=_codes(k_idx, "k_idx"), v_idx=_codes(v_idx, "v_idx"), vcb=(vcb16, vsh),
                   out_dtype=v_centroids.dtype, B=B, Hq=Hq, Hk=Hk, S=S, D=M * D_SUB, K=K, dev=lut.device,
                   chunk=chunk)


def decode_attn_pq_kv_fused(q: torch.Tensor, k_centroids: torch.Tensor, k_idx: torch.Tensor, v_idx: torch.Tensor,
                            v_centroids: torch.Tensor, scale: float = 1.0, d_sub_v: int = 8, *,
                            chunk: int = 0) -> torch.Tensor:
    """pq_build_lut(q, k_centroids, scale) followed by decode_attn_pq_lut_kv
    (benchmarks/test_correctness.py:272-273, then src/attention_kernels.py:
    471-500), in one launch that forms no LUT in HBM.  With at most 8 query
    heads per KV head the scores are scale * (q . k_hat) on MFMA, k_hat the
    codebook rows the key codes select (exact products, fp32 sums); with more,
    each workgroup builds its heads' LUTs in LDS entry for entry as
    pq_build_lut and the result is bit-identical to the two calls.  Either way
    it agrees with the two calls within the attention tolerance.  q
    [B,H_q,1,D] bf16; k_centroids, v_centroids [M,K,8] or [H_k,M,K,8]; k_idx,
    v_idx [B,H_k,S,M].  Returns [B,H_q,1,D] in v_centroids' dtype."""
    if d_sub_v != D_SUB:
        raise ValueError(f"d_sub_v={d_sub_v} not supported (8)")
    C.cuda_tensors(q, k_centroids, k_idx, v_idx, v_centroids)
    C.ndim(q, 4, "q"), C.ndim(k_idx, 4, "k_idx")
    C.dtype_in(q, "q", torch.bfloat16)
    B, Hq, one, D = q.shape
    Bk, Hk, S, M = k_idx.shape
    if one != 1 or Bk != B or M * D_SUB != D or Hq % Hk != 0 or S == 0:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k_idx {tuple(k_idx.shape)}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    if tuple(v_idx.shape[:3]) != (B, Hk, S):
        raise ValueError(f"v_idx {tuple(v_idx.shape)} does not match k_idx {tuple(k_idx.shape)}")
    kcb16, ksh, Mk, K = _codebook16(k_centroids, Hk, "k_centroids")
    vcb16, vsh, Mv, Kv = _codebook16(v_centroids, Hk, "v_centroids")
    if Mk != M or Mv != M or v_idx.shape[-1] != M or Kv != K:
        raise ValueError("codebooks / codes must share the subspace and codeword counts")
    if not (0 < K <= 256 and K % 4 == 0):
        raise ValueError(f"K={K} codewords not supported (multiple of 4, <= 256)")
    qs = C.rows16(q.squeeze(2))
    return _decode(3, q=qs, kcb=(kcb16, ksh), k_idx=_codes(k_idx, "k_idx"), v_idx=_codes(v_idx, "v_idx"),
                   vcb=(vcb16, vsh), out_dtype=v_centroids.dtype, B=B, Hq=Hq, Hk=Hk, S=S, D=D, K=K, dev=q.device,
                   chunk=chunk, scale=scale)


def decode_attn_pq_lut(lut: torch.Tensor, k_idx: torch.Tensor, v: torch.Tensor, *, chunk: int = 0) -> torch.Tensor:
    """LUT-scored keys, dense V.  Replaces src/attention_kernels.py:365-392.
    v [B,H_k,S,D] bf16; returns [B,H_q,1,D] in v's dtype (:375)."""
    lut, B, Hq, Hk, S, M, K = _lut_checks(lut, k_idx)
    C.cuda_tensors(lut, v)
    C.dtype_in(v, "v", torch.bfloat16)
    if tuple(v.shape) != (B, Hk, S, M * D_SUB):
        raise ValueError(f"v {tuple(v.shape)} does not match k_idx {tuple(k_idx.shape)}")
    v = C.rows16(v)
    return _decode(1, lut=lut, k_idx=_codes(k_idx, "k_idx"), v=v, out_dtype=v.dtype, B=B, Hq=Hq, Hk=Hk, S=S,
                   D=M * D_SUB, K=K, dev=lut.device, chunk=chunk)


def decode_attn_dequant(q: torch.Tensor, k_idx: torch.Tensor, centroids: torch.Tensor, v: torch.Tensor,
                        d_sub: int = 8, *, chunk: int = 0) -> torch.Tensor:
    """Codebook-reconstructed keys, dense V, no scale.  Replaces
    src/attention_kernels.py:267-296.  q [B,H_q,1,D] bf16; k_idx [B,H_k,S,M];
    centroids [M,K,8] or [H_k,M,K,8]; v [B,H_k,S,D] bf16.  Returns
    [B,H_q,1,D] in q's dtype (:278)."""
    if d_sub != D_SUB:
        raise ValueError(f"d_sub={d_sub} not supported (8)")
    C.cuda_tensors(q, k_idx, centroids, v)
    C.ndim(q, 4, "q"), C.ndim(k_idx, 4, "k_idx"), C.ndim(v, 4, "v")
    C.dtype_in(q, "q", torch.bfloat16)
    C.dtype_in(v, "v", torch.bfloat16)
    B, Hq, one, D = q.shape
    Bk, Hk, S, M = k_idx.shape
    if one != 1 or Bk != B or M * D_SUB != D or tuple(v.shape) != (B, Hk, S, D) or Hq % Hk != 0 or S == 0:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k_idx {tuple(k_idx.shape)}, v {tuple(v.shape)}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    kcb16, ksh, Mk, K = _codebook16(centroids, Hk, "centroids")
    if Mk != M:
        raise ValueError("codebook subspaces do not match k_idx")
    qs = C.rows16(q.squeeze(2))
    return _decode(2, q=qs, kcb=(kcb16, ksh), k_idx=_codes(k_idx, "k_idx"), v=C.rows16(v), out_dtype=q.dtype,
                   B=B, Hq=Hq, Hk=Hk, S=S, D=D, K=K, dev=q.device, chunk=chunk)


# ---------------------------------------------------------------------------
# outlier-aware (asymmetric) and paged variants
# ---------------------------------------------------------------------------
OUTLIER_MAX = 16
_F8 = torch.float8_e4m3fn


def _outliers(k_out: torch.Tensor, q_out: torch.Tensor, lead: tuple, B: int, Hq: int):
    """-> (k_out rows with unit stride along C, q_out, C); C = 0 passes no pointers."""
    C.cuda_tensors(k_out, q_out)
    C.ndim(k_out, 4, "k_out"), C.ndim(q_out, 3, "q_out")
    Cn = k_out.shape[-1]
    if tuple(k_out.shape[:3]) != lead:
        raise ValueError(f"k_out {tuple(k_out.shape)} does not match the key codes' {lead}")
    if tuple(q_out.shape) != (B, Hq, Cn):
        raise ValueError(f"q_out {tuple(q_out.shape)} must be [B, H_q, C] = {(B, Hq, Cn)}")
    if Cn > OUTLIER_MAX:
        raise ValueError(f"C={Cn} outlier channels above the supported {OUTLIER_MAX}")
    for t, n in ((k_out, "k_out"), (q_out, "q_out")):
        C.dtype_in(t, n, torch.bfloat16, torch.float16, torch.float32)
    if Cn and k_out.stride(-1) != 1:
        k_out = k_out.contiguous()
    if Cn and q_out.stride(-1) != 1:
        q_out = q_out.contiguous()
    return k_out, q_out, Cn


def _paging(block_table: torch.Tensor, context_lens: torch.Tensor, B: int, block_size: int, nblocks: int):
    C.cuda_tensors(block_table, context_lens)
    if block_table.dim() != 2 or block_table.shape[0] != B or context_lens.shape != (B,):
        raise ValueError(f"block_table must be [B, max_blocks] and context_lens [B]; got "
                         f"{tuple(block_table.shape)}, {tuple(context_lens.shape)}")
    if block_size <= 0 or nblocks <= 0:
        raise ValueError("empty paged cache")
    bt = block_table.to(torch.int32)
    if bt.stride(-1) != 1:
        bt = bt.contiguous()
    return bt, context_lens.to(torch.int32).contiguous(), block_table.shape[1] * block_size


def _lut_decode(lut, k_idx, *, v_idx=None, vcb=None, v=None, k_out=None, q_out=None, Cn=0, paging=None,
                out_dtype, Hk, S, K, chunk=0):
    B, Hq, M, _ = lut.shape
    D = M * D_SUB
    dev = lut.device
    out = torch.empty((B, Hq, D), dtype=out_dtype, device=dev)
    ws = workspace(dev, size_query("bytes_pq_decode_workspace_size", B, Hq, Hk, S, D, int(chunk)))
    z = lambda t, i: t.stride(i) if t is not None else 0    # noqa: E731
    p = lambda t: ptr(t) if t is not None else None          # noqa: E731
    vcb16, vcb_sh = vcb if vcb is not None else (None, 0)
    ko = k_out if Cn else None
    qo = q_out if Cn else None
    bt, cl, bs, nblk = paging if paging is not None else (None, None, 0, 0)
    call("bytes_pq_lut_decode_attn", ptr(lut), lut.stride(0), lut.stride(1),
         ptr(k_idx), k_idx.stride(0), k_idx.stride(1), k_idx.stride(2),
         p(v_idx), z(v_idx, 0), z(v_idx, 1), z(v_idx, 2), p(vcb16), vcb_sh,
         p(v), int(v is not None and v.dtype == _F8), z(v, 0), z(v, 1), z(v, 2),
         p(ko), dtype_code(ko) if ko is not None else 0, z(ko, 0), z(ko, 1), z(ko, 2),
         p(qo), dtype_code(qo) if qo is not None else 0, z(qo, 0), z(qo, 1), int(Cn),
         p(bt), z(bt, 0), p(cl), int(bs), int(nblk),
         ptr(out), dtype_code(out), out.stride(0), out.stride(1),
         B, Hq, Hk, S, D, K, 1.0, int(chunk), ptr(ws), ws.numel(), stream_of(lut))
    return out.unsqueeze(2)


def _dense_values(v: torch.Tensor, lead: tuple, D: int) -> torch.Tensor:
    C.dtype_in(v, "v", torch.bfloat16, _F8)
    if tuple(v.shape) != (*lead, D):
        raise ValueError(f"v {tuple(v.shape)} does not match the key codes: expected {(*lead, D)}")
    return C.rows16(v)


def decode_attn_pq_lut_asym(lut: torch.Tensor, k_idx: torch.Tensor, k_out: torch.Tensor, q_out: torch.Tensor,
                            v: torch.Tensor, BLOCK_N: int = 256, *, chunk: int = 0) -> torch.Tensor:
    """LUT-scored keys plus exact outlier channels, dense V.

    Replaces src/attention_kernels.py:713-753: score_t = sum_j lut[b,h,j,k_idx[t,j]]
    + sum_c q_out[b,h,c] * k_out[b,h//G,t,c], softmax without a scale inside
    (fold it into the LUT and q_out).  lut [B,H_q,M,K] fp32; k_idx [B,H_k,S,M];
    k_out [B,H_k,S,C] and q_out [B,H_q,C] (C <= 16; C = 0 allowed); v
    [B,H_k,S,D] bf16 or float8_e4m3fn.  Returns [B,H_q,1,D] in v's dtype, bf16
    for fp8 values (:735)."""
    lut, B, Hq, Hk, S, M, K = _lut_checks(lut, k_idx)
    C.cuda_tensors(lut, v)
    k_out, q_out, Cn = _outliers(k_out, q_out, (B, Hk, S), B, Hq)
    v = _dense_values(v, (B, Hk, S), M * D_SUB)
    od = torch.bfloat16 if v.dtype == _F8 else v.dtype
    return _lut_decode(lut, _codes(k_idx, "k_idx"), v=v, k_out=k_out, q_out=q_out, Cn=Cn, out_dtype=od, Hk=Hk,
                       S=S, K=K, chunk=chunk)


def _paged_lut_checks(lut, k_idx_paged):
    C.cuda_tensors(lut, k_idx_paged)
    C.ndim(lut, 4, "lut"), C.ndim(k_idx_paged, 4, "k_idx_paged")
    if lut.dtype != torch.float32:
        lut = lut.float()
    B, Hq, M, K = lut.shape
    nblk, Hk, bs, Mk = k_idx_paged.shape
    if Mk != M or Hq % Hk != 0:
        raise ValueError(f"shape mismatch: lut {tuple(lut.shape)}, k_idx_paged {tuple(k_idx_paged.shape)}")
    if M * D_SUB not in (64, 128):
        raise ValueError(f"M={M} subspaces: head_dim {M * D_SUB} not supported (64 or 128)")
    if not (0 < K <= 256 and K % 4 == 0):
        raise ValueError(f"K={K} codewords not supported (multiple of 4, <= 256)")
    if lut.stride(-1) != 1 or lut.stride(-2) != K or lut.data_ptr() % 16 != 0:
        lut = lut.contiguous()
    return lut, B, Hq, Hk, nblk, bs, M, K


def paged_attn_pq_lut_kv(lut: torch.Tensor, k_idx_paged: torch.Tensor, v_idx_paged: torch.Tensor,
                         v_centroids: torch.Tensor, block_table: torch.Tensor, context_lens: torch.Tensor,
                         block_size: int = 16, *, chunk: int = 0) -> torch.Tensor:
    """The LUT-KV decode over a paged cache.  Replaces
    src/attention_kernels.py:588-622: k_idx_paged, v_idx_paged
    [num_blocks,H_k,block_size,M]; block_table [B,max_blocks] (entries past a
    sequence's blocks unused, e.g. -1); context_lens [B].  Returns
    [B,H_q,1,D] in v_centroids' dtype."""
    lut, B, Hq, Hk, nblk, bs, M, K = _paged_lut_checks(lut, k_idx_paged)
    if bs != block_size:
        raise ValueError(f"k_idx_paged rows per block {bs} != block_size {block_size}")
    C.cuda_tensors(lut, v_idx_paged, v_centroids)
    if tuple(v_idx_paged.shape[:3]) != (nblk, Hk, bs):
        raise ValueError(f"v_idx_paged {tuple(v_idx_paged.shape)} does not match k_idx_paged")
    vcb16, vsh, Mv, Kv = _codebook16(v_centroids, Hk, "v_centroids")
    if Mv != M or v_idx_paged.shape[-1] != Mv or Kv != K:
        raise ValueError("value codebook / codes must use the key's subspace and codeword counts")
    bt, cl, S = _paging(block_table, context_lens, B, block_size, nblk)
    return _lut_decode(lut, _codes(k_idx_paged, "k_idx_paged"), v_idx=_codes(v_idx_paged, "v_idx_paged"),
                       vcb=(vcb16, vsh), paging=(bt, cl, block_size, nblk), out_dtype=v_centroids.dtype, Hk=Hk,
                       S=S, K=K, chunk=chunk)


def paged_attn_pq_lut_asym(lut: torch.Tensor, k_idx_paged: torch.Tensor, k_out_paged: torch.Tensor,
                           q_out: torch.Tensor, v_paged: torch.Tensor, block_table: torch.Tensor,
                           context_lens: torch.Tensor, block_size: int = 16, BLOCK_N: int = 256, *,
                           chunk: int = 0) -> torch.Tensor:
    """The outlier-aware LUT decode over a paged cache.  Replaces
    src/attention_kernels.py:858-906: k_idx_paged [num_blocks,H_k,block_size,M],
    k_out_paged [num_blocks,H_k,block_size,C], v_paged [num_blocks,H_k,block_size,D]
    bf16 or float8_e4m3fn, q_out [B,H_q,C].  Returns [B,H_q,1,D] in v's dtype,
    bf16 for fp8 values."""
    lut, B, Hq, Hk, nblk, bs, M, K = _paged_lut_checks(lut, k_idx_paged)
    if bs != block_size:
        raise ValueError(f"k_idx_paged rows per block {bs} != block_size {block_size}")
    C.cuda_tensors(lut, v_paged)
    k_out_paged, q_out, Cn = _outliers(k_out_paged, q_out, (nblk, Hk, bs), B, Hq)
    v_paged = _dense_values(v_paged, (nblk, Hk, bs), M * D_SUB)
    bt, cl, S = _paging(block_table, context_lens, B, block_size, nblk)
    od = torch.bfloat16 if v_paged.dtype == _F8 else v_paged.dtype
    return _lut_decode(lut, _codes(k_idx_paged, "k_idx_paged"), v=v_paged, k_out=k_out_paged, q_out=q_out, Cn=Cn,
                       paging=(bt, cl, block_size, nblk), out_dtype=od, Hk=Hk, S=S, K=K, chunk=chunk)


def sparse_score_pq_lut_asym(lut: torch.Tensor, k_idx: torch.Tensor, k_out: torch.Tensor, q_out: torch.Tensor,
                             BLOCK_N: int = 256) -> torch.Tensor:
    """Per-key LUT + outlier scores [B,H_q,S] fp32 (no softmax).  Replaces
    src/attention_kernels.py:960-984."""
    lut, B, Hq, Hk, S, M, K = _lut_checks(lut, k_idx)
    k_out, q_out, Cn = _outliers(k_out, q_out, (B, Hk, S), B, Hq)
    k_idx = _codes(k_idx, "k_idx")
    out = torch.empty((B, Hq, S), dtype=torch.float32, device=lut.device)
    ko = k_out if Cn else None
    qo = q_out if Cn else None
    z = lambda t, i: t.stride(i) if t is not None else 0    # noqa: E731
    call("bytes_pq_lut_scores", ptr(lut), lut.stride(0), lut.stride(1), ptr(k_idx), k_idx.stride(0),
         k_idx.stride(1), k_idx.stride(2), ptr(ko) if Cn else None, dtype_code(ko) if Cn else 0, z(ko, 0), z(ko, 1),
         z(ko, 2), ptr(qo) if Cn else None, dtype_code(qo) if Cn else 0, z(qo, 0), z(qo, 1), int(Cn), ptr(out),
         out.stride(0), out.stride(1), B, Hq, Hk, S, M * D_SUB, K, stream_of(lut))
    return out


def sparse_decode_pq_lut(lut: torch.Tensor, k_idx: torch.Tensor, k_out: torch.Tensor, q_out: torch.Tensor,
                         q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, frac: float, scaling: float,
                         BLOCK_N: int = 256, BLOCK_K: int = 64) -> torch.Tensor:
    """LUT + outlier scores over every key -> the kb = max(1, round(frac*S))
    best per query head (ties to the lowest index) -> exact gathered attention
    over k, v.  Replaces src/attention_kernels.py:1062-1074.  Returns
    [B,H_q,1,D] bf16."""
    from .sparse import budget, sparse_gather_attn, topk_indices
    s = sparse_score_pq_lut_asym(lut, k_idx, k_out, q_out)
    kb = budget(frac, s.shape[-1])
    idx = topk_indices(s, kb, sorted=False)
    return sparse_gather_attn(q, k, v, idx, scaling)


def pq_build_lut(q: torch.Tensor, centroids: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """lut[b,h,j,c] = scale * sum_e q[b,h,8j+e] * centroids[h//G][j][c][e] (fp32):
    the reference's LUT precompute (benchmarks/test_correctness.py:272-273,
    einsum("bhmd,mkd->bhmk")) with the softmax scale folded in.  q [B,H_q,1,D]
    or [B,H_q,D] bf16; centroids [M,K,8] or [H_k,M,K,8].  Returns [B,H_q,M,K]."""
    C.cuda_tensors(q, centroids)
    C.dtype_in(q, "q", torch.bfloat16)
    qs = q.squeeze(2) if q.dim() == 4 else q
    B, Hq, D = qs.shape
    Hk = centroids.shape[0] if centroids.dim() == 4 else 1
    if Hq % Hk != 0 or D % D_SUB != 0:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, centroids {tuple(centroids.shape)}")
    cb16, sh, M, K = _codebook16(centroids, Hk, "centroids")
    if M * D_SUB != D:
        raise ValueError("codebook subspaces do not cover head_dim")
    qs = C.rows16(qs)
    lut = torch.empty((B, Hq, M, K), dtype=torch.float32, device=q.device)
    call("bytes_pq_build_lut", ptr(qs), ptr(cb16), ptr(lut), B, Hq, Hk, D, K, qs.stride(0), qs.stride(1), sh,
         float(scale), stream_of(q))
    return lut


def _x_code(x: torch.Tensor) -> int:
    return {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}[x.dtype]


def pq_encode(x: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """Nearest codeword per subspace: idx[..., j] = argmin_c sum_e (x[8j+e] - c[e])^2
    in fp32 (e ascending, separate multiply and add), first index on ties -
    the CPU rule of src/quantization.py:203-211 (cdist + argmin).
    x [..., D] (or [H_k, ..., D] with per-head [H_k,M,K,8] centroids).
    Returns uint8 [..., M]."""
    C.cuda_tensors(x, centroids)
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"x: dtype {x.dtype} not supported")
    D = x.shape[-1]
    per_head = centroids.dim() == 4
    heads = centroids.shape[0] if per_head else 1
    if per_head and x.shape[0] != heads:
        raise ValueError(f"per-head centroids: x's first dim must be {heads}")
    f32 = centroids.dtype == torch.float32
    cb = centroids.contiguous() if f32 else centroids.to(torch.float16).contiguous()
    M, K, ds = cb.shape[-3:]
    if ds != D_SUB or M * D_SUB != D or M > 16 or not 0 < K <= 256:
        raise ValueError(f"centroids {tuple(centroids.shape)} do not fit head_dim {D}")
    xf = x.reshape(-1, D)
    if xf.stride(-1) != 1:
        xf = xf.contiguous()
    rows = xf.shape[0] // heads
    idx = torch.empty((xf.shape[0], M), dtype=torch.uint8, device=x.device)
    call("bytes_pq_encode", ptr(xf), _x_code(xf), heads, rows, xf.stride(0), D, ptr(cb), int(f32),
         M * K * D_SUB if per_head else 0, K, ptr(idx), stream_of(x))
    return idx.reshape(*x.shape[:-1], M)


def pq_decode(idx: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """Codes [..., M] -> fp32 vectors [..., M*8] (src/quantization.py:213-226);
    per-head centroids [H_k,M,K,8] take idx [H_k, ..., M]."""
    C.cuda_tensors(idx, centroids)
    per_head = centroids.dim() == 4
    heads = centroids.shape[0] if per_head else 1
    f32 = centroids.dtype == torch.float32
    cb = centroids.contiguous() if f32 else centroids.to(torch.float16).contiguous()
    M, K, ds = cb.shape[-3:]
    flat = idx.reshape(-1, M).to(torch.uint8).contiguous()
    out = torch.empty((flat.shape[0], M * ds), dtype=torch.float32, device=idx.device)
    call("bytes_pq_decode_vectors", ptr(flat), heads, flat.shape[0] // heads, M * ds, ptr(cb), int(f32),
         M * K * ds if per_head else 0, K, ptr(out), stream_of(idx))
    return out.reshape(*idx.shape[:-1], M * ds)


def kmeans(X: torch.Tensor, k: int, num_iters: int = 20, generator: Optional[torch.Generator] = None,
           d_sub: int = D_SUB) -> torch.Tensor:
    """k-means codebooks for every subspace of X [H, N, D] (or [N, D]) on the GPU.

    Follows src/quantization.py:102-132 per subspace: random distinct points as
    initial centroids, assignment to the nearest centroid (the encode kernel),
    mean update, empty clusters re-seeded from a random point (drawn from
    `generator`, a CPU generator, so runs are reproducible).
    Returns fp32 centroids [H, M, k, d_sub] (or [M, k, d_sub] for 2-D X).
    """
    if d_sub != D_SUB:
        raise ValueError("d_sub must be 8")
    C.cuda_tensors(X)
    squeeze = X.dim() == 2
    Xh = (X.unsqueeze(0) if squeeze else X).float().contiguous()
    H, N, D = Xh.shape
    M = D // d_sub
    if N <= k:                          # src/quantization.py:111-114: pad with zeros
        cb = torch.zeros(H, M, k, d_sub, device=X.device)
        cb[:, :, :N] = Xh.reshape(H, N, M, d_sub).permute(0, 2, 1, 3)
        return cb[0] if squeeze else cb
    g = generator if generator is not None else torch.Generator().manual_seed(0)
    init = torch.stack([torch.stack([torch.randperm(N, generator=g)[:k] for _ in range(M)]) for _ in range(H)])
    init = init.to(X.device)                                              # [H, M, k]
    xs = Xh.reshape(H, N, M, d_sub)
    cb32 = torch.stack([torch.stack([xs[h, init[h, j], j] for j in range(M)]) for h in range(H)]).contiguous()
    cb16 = cb32.to(torch.float16)
    labels = torch.empty((H, N, M), dtype=torch.uint8, device=X.device)
    for _ in range(num_iters):
        call("bytes_pq_encode", ptr(Xh), 2, H, N, D, D, ptr(cb32), 1, M * k * d_sub, k, ptr(labels),
             stream_of(Xh))
        reseed = torch.randint(0, N, (H, M, k), generator=g).to(X.device)
        call("bytes_pq_kmeans_update", ptr(Xh), H, N, D, k, ptr(labels), ptr(reseed), ptr(cb16), ptr(cb32),
             stream_of(Xh))
    return cb32[0] if squeeze else cb32


def kmeans_pytorch(X: torch.Tensor, k: int, num_iters: int = 20,
                   generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """Drop-in for src/quantization.py:102-132: X [N, d_sub] -> centroids
    [k, d_sub] in X's dtype, fitted on the GPU by `kmeans`.

    d_sub must be 8, the subspace width of the encode kernel and of every PQ
    caller on the decode path (BASELINE C3, test_correctness.py:33).  N <= k
    returns the points followed by zero rows, as the reference does.
    """
    if X.dim() != 2:
        raise ValueError(f"X must be [N, d_sub], got {tuple(X.shape)}")
    if X.shape[1] != D_SUB:
        raise ValueError(f"d_sub {X.shape[1]} not supported (8)")
    return kmeans(X, k, num_iters, generator)[0].to(X.dtype)


class ProductQuantizer:
    """Drop-in for src/quantization.py:134-226 on the GPU kernels: `fit` runs
    k-means per subspace, `quantize` the bit-exact nearest-codeword encoder
    (returns long codes, as the reference), `dequantize` the codebook gather."""

    def __init__(self, d: int, d_sub: int, bits: int = 3, device="cuda"):
        if d % d_sub != 0:
            raise ValueError(f"d ({d}) must be divisible by d_sub ({d_sub})")
        self.d, self.d_sub, self.bits, self.k = d, d_sub, bits, 2 ** bits
        self.M = d // d_sub
        self.device = device
        self.centroids = torch.zeros((self.M, self.k, self.d_sub), device=device)

    def fit(self, X: torch.Tensor, num_iters: int = 20, generator: Optional[torch.Generator] = None):
        self.centroids = kmeans(X.to(self.device).reshape(-1, self.d), self.k, num_iters, generator, self.d_sub)

    def quantize(self, X: torch.Tensor) -> torch.Tensor:
        return pq_encode(X.to(self.device), self.centroids).long()

    def dequantize(self, indices: torch.Tensor) -> torch.Tensor:
        return pq_decode(indices.to(self.device), self.centroids).to(self.centroids.dtype)
