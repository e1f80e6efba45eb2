"""Drop-in KIVI operators (benchmarks/kivi_latency.py surface) on gfx950 kernels.

Cache layout is the reference's: codes packed 32/bits per int32 along the last
dim (element i of word w at bits [i*bits, (i+1)*bits)), fp16 scale/zero per
group of `group_size` consecutive last-dim elements.  Keys are packed from the
transposed cache [B,Hk,D,Sq] (per-channel groups of tokens), values from
[B,Hk,Sq,D] (per-token groups of channels).
"""
from __future__ import annotations

import math

import torch

from . import _checks as C
from ._lib import call, dtype_code, ptr, size_query, stream_of, workspace


def quantize_and_pack_along_last_dim(data: torch.Tensor, group_size: int, bit: int):
    """Asymmetric min/max quantize along the last dim in groups and pack into int32.

    Replaces KIVI's `triton_quantize_and_pack_along_last_dim(data, group_size, bit)`
    as called at benchmarks/kivi_latency.py:123,127 (KIVI is not vendored in the
    reference; the arithmetic is src/quantization.py:432-442 in fp32, scale and
    zero rounded to fp16).  data [..., T] fp16/bf16/fp32 ->
    (code int32 [..., T*bit/32], scale fp16 [..., T/group_size], mn fp16 [..., T/group_size]).
    """
    C.cuda_tensors(data)
    if bit not in (2, 4):
        raise ValueError(f"bit must be 2 or 4, got {bit}")
    T = data.shape[-1]
    fpi = 32 // bit
    if T % group_size != 0 or group_size % fpi != 0:
        raise ValueError(f"last dim {T} must be a multiple of group_size {group_size} (itself a multiple of {fpi})")
    x = data if data.stride(-1) == 1 else data.contiguous()
    x2 = x.reshape(-1, T) if x.is_contiguous() else x.contiguous().reshape(-1, T)
    rows = x2.shape[0]
    lead = tuple(data.shape[:-1])
    code = torch.empty(lead + (T // fpi,), dtype=torch.int32, device=data.device)
    scale = torch.empty(lead + (T // group_size,), dtype=torch.float16, device=data.device)
    mn = torch.empty_like(scale)
    call("bytes_kivi_quantize_pack", ptr(x2), dtype_code(x2), rows, T, x2.stride(0), group_size, bit,
         ptr(code), ptr(scale), ptr(mn), stream_of(data))
    return code, scale, mn


# KIVI's own name for the same operator (the reference harness imports it by this name).
triton_quantize_and_pack_along_last_dim = quantize_and_pack_along_last_dim


def _dequant_last_dim(code, scale, mn, group_size, bits, out_dtype, fp16_math):
    C.cuda_tensors(code, scale, mn)
    fpi = 32 // bits
    T = code.shape[-1] * fpi
    code = code.contiguous()
    scale = scale.to(torch.float16).contiguous()
    mn = mn.to(torch.float16).contiguous()
    rows = code.numel() // code.shape[-1]
    if scale.numel() != rows * (T // group_size) or mn.numel() != scale.numel():
        raise ValueError(f"scale/mn shape {tuple(scale.shape)} does not match codes {tuple(code.shape)}")
    out = torch.empty(tuple(code.shape[:-1]) + (T,), dtype=out_dtype, device=code.device)
    call("bytes_kivi_dequant", ptr(code), ptr(scale), ptr(mn), rows, T, group_size, bits, int(fp16_math),
         ptr(out), dtype_code(out), stream_of(code))
    return out


def unpack_tensor_last_dim(code: torch.Tensor, bits: int) -> torch.Tensor:
    """int32 words -> fp16 codes along the last dim (benchmarks/kivi_latency.py:26-35)."""
    fpi = 32 // bits
    T = code.shape[-1] * fpi
    ones = torch.ones(tuple(code.shape[:-1]) + (1,), dtype=torch.float16, device=code.device)
    return _dequant_last_dim(code, ones, torch.zeros_like(ones), T, bits, torch.float16, True)


def dequant_k(Kq, K_scale, K_mn, group_size: int, bits: int) -> torch.Tensor:
    """[B,H,D,Sq*bits/32] -> [B,H,Sq,D] fp16 (benchmarks/kivi_latency.py:37-46, fp16 arithmetic)."""
    kd = _dequant_last_dim(Kq, K_scale, K_mn, group_size, bits, torch.float16, True)
    return kd.transpose(2, 3).contiguous()


def dequant_v(Vq, V_scale, V_mn, group_size: int, bits: int) -> torch.Tensor:
    """[B,H,Sq,D*bits/32] -> [B,H,Sq,D] fp16 (benchmarks/kivi_latency.py:48-57, fp16 arithmetic)."""
    return _dequant_last_dim(Vq, V_scale, V_mn, group_size, bits, torch.float16, True)


def kivi_decode_attn(Q, Kq, K_scale, K_mn, K_residual, Vq, V_scale, V_mn, V_residual, bits: int,
                     group_size: int = 32, *, scale: float | None = None, chunk: int = 0):
    """softmax([Q.K_dq^T, Q.K_res^T]/sqrt(D)) . [V_dq; V_res] in one fused kernel.

    Replaces benchmarks/kivi_latency.py:59-90 (`kivi_decode_attn`; semantics of
    `kivi_decode_attn_ref` :92-100).  Q [B,Hq,1,D] bf16; Kq [B,Hk,D,Sq*bits/32]
    int32; K_scale/K_mn [B,Hk,D,Sq/32] fp16; K_residual [B,Hk,R,D] bf16;
    Vq [B,Hk,Sq,D*bits/32]; V_scale/V_mn [B,Hk,Sq,D/32]; V_residual [B,Hk,R,D].
    Returns [B,Hq,1,D] in Q's dtype.  `scale` defaults to 1/sqrt(D) (:76).
    `chunk` (a tuning hint, default 0 = automatic): > 0 sets the split length
    in tokens of the two-half / streaming kernels; < 0 runs D = 128 caches
    (Sq a multiple of 64, at least 1024) on the pipelined kernel with splits
    of -chunk 256-token granules.
    """
    C.cuda_tensors(Q, K_residual, V_residual)
    C.dtype_in(Q, "Q", torch.bfloat16)
    C.dtype_in(K_residual, "K_residual", torch.bfloat16)
    C.dtype_in(V_residual, "V_residual", torch.bfloat16)
    if bits not in (2, 4):
        raise ValueError(f"bits must be 2 or 4, got {bits}")
    if group_size != 32:
        raise ValueError("the fused KIVI kernel implements group_size=32 (the reference's setting)")
    B, Hq, one, D = Q.shape
    Hk, R = K_residual.shape[1], K_residual.shape[2]
    fpi = 32 // bits
    Sq = Kq.shape[-1] * fpi if Kq is not None and Kq.numel() else 0
    if one != 1 or Hq % Hk or D not in (64, 128):
        raise ValueError(f"bad Q shape {tuple(Q.shape)} for H_k={Hk}")
    if tuple(V_residual.shape) != (B, Hk, R, D):
        raise ValueError("K_residual / V_residual shapes differ")
    if Sq:
        C.cuda_tensors(Kq, K_scale, K_mn, Vq, V_scale, V_mn)
        exp = {"Kq": (B, Hk, D, Sq // fpi), "K_scale": (B, Hk, D, Sq // 32), "K_mn": (B, Hk, D, Sq // 32),
               "Vq": (B, Hk, Sq, D // fpi), "V_scale": (B, Hk, Sq, D // 32), "V_mn": (B, Hk, Sq, D // 32)}
        got = {"Kq": Kq, "K_scale": K_scale, "K_mn": K_mn, "Vq": Vq, "V_scale": V_scale, "V_mn": V_mn}
        for n, shp in exp.items():
            if tuple(got[n].shape) != shp:
                raise ValueError(f"{n}: expected shape {shp}, got {tuple(got[n].shape)}")
    if Sq + R == 0:
        raise ValueError("empty KV cache")
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if Sq % 32 != 0:
        raise ValueError(f"quantized length {Sq} is not a whole number of 32-token key groups")
    q3 = C.rows16(Q.squeeze(2))
    kr, vr = C.rows16(K_residual), C.rows16(V_residual)
    t = [x.contiguous() if x is not None else None for x in (Kq, K_scale, K_mn, Vq, V_scale, V_mn)]
    if Sq:
        t[1], t[2], t[4], t[5] = (x.to(torch.float16) for x in (t[1], t[2], t[4], t[5]))
    out = torch.empty((B, Hq, D), dtype=Q.dtype, device=Q.device)
    nbytes = size_query("bytes_kivi_decode_workspace_size", B, Hq, Hk, Sq, R, D, bits, int(chunk))
    ws = workspace(Q.device, nbytes)
    pz = [ptr(x) if (x is not None and Sq) else None for x in t]
    call("bytes_kivi_decode_attn", ptr(q3), pz[0], pz[1], pz[2], ptr(kr) if R else None,
         pz[3], pz[4], pz[5], ptr(vr) if R else None, ptr(out),
         B, Hq, Hk, Sq, R, D, bits, q3.stride(0), q3.stride(1),
         kr.stride(0), kr.stride(1), kr.stride(2), vr.stride(0), vr.stride(1), vr.stride(2),
         out.stride(0), out.stride(1), sc, int(chunk), ptr(ws), ws.numel(), stream_of(Q))
    return out.unsqueeze(2)
