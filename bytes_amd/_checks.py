"""Argument validation shared by the operator wrappers.

The reference wrappers do no validation (shape errors surface as Triton
compile errors or silent out-of-bounds reads); these wrappers raise
ValueError for bad shapes/dtypes/devices before anything is launched.
"""
from __future__ import annotations

import torch


def cuda_tensors(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(f"bytes_amd operators run on the GPU; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def dtype_in(t: torch.Tensor, name: str, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: dtype {t.dtype} not supported (expected one of {dtypes})")


def rows16(t: torch.Tensor, align: int = 16) -> torch.Tensor:
    """Unit stride on the last dim, every row start `align`-byte aligned (16 by
    default: 128-bit row loads); copies on the GPU when the given layout does
    not allow that."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % align == 0
    if ok:
        for d in range(t.dim() - 1):
            if t.size(d) > 1 and (t.stride(d) * es) % align != 0:
                ok = False
                break
    if ok:
        return t
    c = t.contiguous()
    if c.data_ptr() % align != 0:
        raise ValueError(f"tensor storage is not {align}-byte aligned")
    return c


def ndim(t: torch.Tensor, n: int, name: str) -> None:
    if t.dim() != n:
        raise ValueError(f"{name}: expected {n} dims, got shape {tuple(t.shape)}")
