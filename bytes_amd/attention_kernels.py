"""Drop-in decode-attention operators (src/attention_kernels.py surface).

Each function keeps the reference's name, argument meaning and output
layout/dtype, launches a hand-written gfx950 HIP kernel through the C ABI on
the current stream (no host sync), and allocates only its output (plus a
cached, zero-initialised split-K workspace).  BLOCK_* arguments of the
reference are tuning hints for Triton and are accepted and ignored.
"""
from __future__ import annotations

import torch

from . import _checks as C
from ._lib import call, ptr, size_query, stream_of, workspace


def decode_attn_bf16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = 1.0,
                     *, chunk: int = 0) -> torch.Tensor:
    """softmax(scale * q.K^T) V for one query per (b, h_q); GQA h_k = h_q // G.

    Replaces src/attention_kernels.py:65-92.  q [B,H_q,1,D] bf16; k, v
    [B,H_k,S,D] bf16 (any strides; a copy is made if rows are not 16-byte
    aligned with unit stride in D).  Returns [B,H_q,1,D] in q's dtype.
    The reference applies no scale (:42): `scale` defaults to 1.0; pass
    1/sqrt(D) for standard attention.  `chunk` forces the split-K chunk
    length in tokens (0 = automatic).
    """
    C.cuda_tensors(q, k, v)
    C.ndim(q, 4, "q"), C.ndim(k, 4, "k"), C.ndim(v, 4, "v")
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        C.dtype_in(t, n, torch.bfloat16)
    B, Hq, one, D = q.shape
    _, Hk, S, Dk = k.shape
    if one != 1 or Dk != D or tuple(v.shape) != tuple(k.shape) or k.shape[0] != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if Hq % Hk != 0:
        raise ValueError(f"H_q={Hq} is not a multiple of H_k={Hk}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    if S == 0:
        raise ValueError("empty KV cache (S == 0)")
    qs = C.rows16(q.squeeze(2))
    k, v = C.rows16(k), C.rows16(v)
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    nbytes = size_query("bytes_decode_attn_bf16_workspace_size", B, Hq, Hk, S, D, int(chunk))
    ws = workspace(q.device, nbytes)
    call("bytes_decode_attn_bf16", ptr(qs), ptr(k), ptr(v), ptr(out), B, Hq, Hk, S, D,
         qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2),
         v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1),
         float(scale), int(chunk), ptr(ws), ws.numel(), stream_of(q))
    return out.unsqueeze(2)


NOALLOC_SCRATCH_BYTES = 16 << 20      # BYTES_NOALLOC_SCRATCH_BYTES of include/bytes_amd.h


def decode_attn_bf16_noalloc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                             scale: float = 1.0, *, chunk: int = 0) -> torch.Tensor:
    """decode_attn_bf16 for callers that cannot allocate: writes `out`
    [B,H_q,1,D] (or [B,H_q,D]) bf16 and allocates nothing, on the device or
    through torch.  The split-K partials go to a 16 MiB device-resident scratch
    shared by every call on the device (calls that overlap on one device
    race).  Inputs must already have unit stride in D and 16-byte-aligned rows
    (no copy is made).  Raises ValueError when the call's partials exceed the
    scratch (larger B*H_k*splits); a larger `chunk` needs fewer splits."""
    C.cuda_tensors(q, k, v, out)
    C.ndim(q, 4, "q"), C.ndim(k, 4, "k"), C.ndim(v, 4, "v")
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out")):
        C.dtype_in(t, n, torch.bfloat16)
    B, Hq, one, D = q.shape
    _, Hk, S, Dk = k.shape
    if one != 1 or Dk != D or tuple(v.shape) != tuple(k.shape) or k.shape[0] != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if Hq % Hk != 0 or D not in (64, 128) or S == 0:
        raise ValueError(f"unsupported shape: q {tuple(q.shape)}, k {tuple(k.shape)}")
    o3 = out.reshape(B, Hq, D) if out.dim() == 4 else out
    if tuple(o3.shape) != (B, Hq, D):
        raise ValueError(f"out must be [B,H_q,1,D] or [B,H_q,D]; got {tuple(out.shape)}")
    qs = q.squeeze(2)
    for t, n in ((qs, "q"), (k, "k"), (v, "v"), (o3, "out")):
        if C.rows16(t) is not t:
            raise ValueError(f"{n} needs unit stride in D and 16-byte-aligned rows (no copy is made)")
    need = size_query("bytes_decode_attn_bf16_workspace_size", B, Hq, Hk, S, D, int(chunk))
    if need > NOALLOC_SCRATCH_BYTES:
        raise ValueError(f"split-K partials need {need} bytes, above the {NOALLOC_SCRATCH_BYTES}-byte scratch")
    call("bytes_decode_attn_bf16_noalloc", ptr(qs), ptr(k), ptr(v), ptr(o3), B, Hq, Hk, S, D,
         qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2),
         v.stride(0), v.stride(1), v.stride(2), o3.stride(0), o3.stride(1),
         float(scale), int(chunk), stream_of(q))
    return out


def decode_attn_fp8(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = 1.0,
                    *, chunk: int = 0) -> torch.Tensor:
    """softmax(scale * q.K^T) V with OCP float8_e4m3fn K and V.

    Replaces src/attention_kernels.py:156-182: q [B,H_q,1,D] bf16; k, v
    [B,H_k,S,D] float8_e4m3fn, widened to bf16 exactly inside the kernel; fp32
    softmax and accumulation; no scale in the reference (`scale` defaults to
    1.0).  Returns [B,H_q,1,D] in q's dtype (:171)."""
    C.cuda_tensors(q, k, v)
    C.ndim(q, 4, "q"), C.ndim(k, 4, "k"), C.ndim(v, 4, "v")
    C.dtype_in(q, "q", torch.bfloat16)
    C.dtype_in(k, "k", torch.float8_e4m3fn)
    C.dtype_in(v, "v", torch.float8_e4m3fn)
    B, Hq, one, D = q.shape
    _, Hk, S, Dk = k.shape
    if one != 1 or Dk != D or tuple(v.shape) != tuple(k.shape) or k.shape[0] != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if Hq % Hk != 0:
        raise ValueError(f"H_q={Hq} is not a multiple of H_k={Hk}")
    if D not in (64, 128):
        raise ValueError(f"head_dim {D} not supported (64 or 128)")
    if S == 0:
        raise ValueError("empty KV cache (S == 0)")
    qs = C.rows16(q.squeeze(2))
    k, v = C.rows16(k), C.rows16(v)
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    nbytes = size_query("bytes_decode_attn_bf16_workspace_size", B, Hq, Hk, S, D, int(chunk))
    ws = workspace(q.device, nbytes)
    call("bytes_decode_attn_fp8", ptr(qs), ptr(k), ptr(v), ptr(out), B, Hq, Hk, S, D,
         qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2),
         v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1),
         float(scale), int(chunk), ptr(ws), ws.numel(), stream_of(q))
    return out.unsqueeze(2)


# Sparse decode operators of the same module (src/attention_kernels.py:1037-1263).
from .sparse import (quantize_and_pack_score_keys, sparse_decode_scalar, sparse_gather_attn,  # noqa: E402,F401
                     sparse_score_packed, sparse_score_scalar, topk_indices)
from .pq import (decode_attn_dequant, decode_attn_pq_lut, decode_attn_pq_lut_asym,  # noqa: E402,F401
                 decode_attn_pq_lut_kv, paged_attn_pq_lut_asym, paged_attn_pq_lut_kv, sparse_decode_pq_lut,
                 sparse_score_pq_lut_asym)
