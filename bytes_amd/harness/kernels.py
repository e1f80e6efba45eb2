"""Python surface of the harness microkernels (csrc/harness.hip).

- `gather_reduce(v, idx)`: replaces `gather_reduce` of
  benchmarks/bench_access_pattern.py:44-52: v fp16 [H, S, D] (D in 8 .. 256,
  a power of two), idx int32 [H, K] -> fp32 [H, D], out[h] = sum_k v[h, idx[h, k]].
- `stage_score(q, packed, scale, zero, bits, stage)`: replaces `stage_score`
  of benchmarks/bench_unpack_ablation.py:56-66: the cumulative stages
  0 (load), 1 (+ unpack), 2 (+ dequant), 3 (+ dot with q) of the packed-key
  score pass, fp32 [B, H_q, S].
"""
from __future__ import annotations

import torch

from .. import _checks as C
from .._lib import call, ptr, stream_of


def gather_reduce(v: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    C.cuda_tensors(v, idx)
    C.ndim(v, 3, "v"), C.ndim(idx, 2, "idx")
    C.dtype_in(v, "v", torch.float16)
    H, S, D = v.shape
    if idx.shape[0] != H or idx.shape[1] == 0:
        raise ValueError(f"idx must be [H={H}, K>0]; got {tuple(idx.shape)}")
    if D not in (8, 16, 32, 64, 128, 256):
        raise ValueError(f"row width D={D} not supported (8 .. 256, a power of two)")
    v = C.rows16(v)
    idx = idx.to(torch.int32)
    if idx.stride(-1) != 1:
        idx = idx.contiguous()
    out = torch.empty((H, D), dtype=torch.float32, device=v.device)
    call("bytes_gather_reduce", ptr(v), v.stride(0), v.stride(1), ptr(idx), idx.stride(0), ptr(out), H, S,
         idx.shape[1], D, stream_of(v))
    return out


def stage_score(q: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, bits: int,
                stage: int) -> torch.Tensor:
    C.cuda_tensors(q, packed, scale, zero)
    C.dtype_in(q, "q", torch.bfloat16)
    C.dtype_in(packed, "packed", torch.uint8)
    C.dtype_in(scale, "scale", torch.bfloat16)
    C.dtype_in(zero, "zero", torch.bfloat16)
    if bits not in (4, 2) or stage not in (0, 1, 2, 3):
        raise ValueError(f"bits={bits}, stage={stage}: bits 4 or 2, stage 0 .. 3")
    B, Hq, one, D = q.shape
    _, Hk, S, nb = packed.shape
    if one != 1 or nb * 8 // bits != D or Hq % Hk or tuple(scale.shape) != (B, Hk, S, D // 32):
        raise ValueError(f"shapes: q {tuple(q.shape)}, packed {tuple(packed.shape)}, scale {tuple(scale.shape)}")
    if tuple(zero.shape) != tuple(scale.shape):
        raise ValueError("scale and zero shapes differ")
    qs = q.squeeze(2).contiguous()
    packed = C.rows16(packed)
    scale, zero = scale.contiguous(), zero.contiguous()
    out = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    call("bytes_packed_stage", ptr(qs), qs.stride(0), qs.stride(1), ptr(packed), packed.stride(0), packed.stride(1),
         packed.stride(2), ptr(scale), ptr(zero), scale.stride(0), scale.stride(1), scale.stride(2), ptr(out),
         out.stride(0), out.stride(1), B, Hq, Hk, S, D, bits, stage, stream_of(q))
    return out


def stream_read(src: torch.Tensor, wgs: int, out: torch.Tensor = None, nontemporal: bool = False) -> torch.Tensor:
    """Floor probe: `wgs` workgroups of 256 threads read src (a contiguous
    device tensor whose byte size is a multiple of 16 * wgs) in 16-byte loads,
    one contiguous slice each (with the non-temporal hint if `nontemporal`);
    returns the fp32 fold [wgs * 256]."""
    C.cuda_tensors(src)
    if not src.is_contiguous():
        raise ValueError("src must be contiguous")
    nbytes = src.numel() * src.element_size()
    if wgs <= 0 or nbytes % (16 * wgs) != 0 or src.data_ptr() % 16 != 0:
        raise ValueError(f"{nbytes} bytes do not split into {wgs} slices of 16-byte words")
    if out is None:
        out = torch.empty(wgs * 256, dtype=torch.float32, device=src.device)
    call("bytes_stream_read", ptr(src), nbytes, int(wgs), int(bool(nontemporal)), ptr(out), stream_of(src))
    return out


def empty_launch(wgs: int, device: torch.device) -> None:
    """Floor probe: a launch of `wgs` workgroups of 256 threads that do nothing."""
    call("bytes_empty_launch", int(wgs), torch.cuda.current_stream(device).cuda_stream)
