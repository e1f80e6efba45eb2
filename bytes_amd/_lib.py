"""ctypes binding of libbytes_amd.so, the C ABI over the gfx950 kernels.

Every exported function takes device pointers, shape ints, int64 element
strides, a workspace pointer/size and a hipStream_t, and returns 0 or a
hipError_t.  This module maps a non-zero return to RuntimeError.  There is no
fallback: if the library is missing, every operator raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, List, Tuple

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libbytes_amd.so")

c_int, c_i64, c_f32, c_sz, c_vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
c_szp = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes (restype is always c_int unless listed in _RESTYPES)
SIGNATURES: Dict[str, Tuple] = {
    "bytes_abi_version": (),
    "bytes_error_string": (c_int,),
    "bytes_set_kernel_events": (c_int, c_vp, c_vp),
    "bytes_decode_attn_bf16_workspace_size": (c_int, c_int, c_int, c_int, c_int, c_int, c_szp),
    "bytes_decode_attn_bf16": (
        c_vp, c_vp, c_vp, c_vp,                       # q, k, v, out
        c_int, c_int, c_int, c_int, c_int,            # B, Hq, Hk, S, D
        c_i64, c_i64,                                 # q strides (b, h)
        c_i64, c_i64, c_i64,                          # k strides (b, h, s)
        c_i64, c_i64, c_i64,                          # v strides (b, h, s)
        c_i64, c_i64,                                 # out strides (b, h)
        c_f32, c_int, c_vp, c_sz, c_vp),              # scale, chunk, workspace, bytes, stream
    "bytes_decode_attn_bf16_noalloc": (
        c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int,
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
        c_f32, c_int, c_vp),                          # scale, chunk, stream
    "bytes_decode_attn_fp8": (
        c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int,
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
        c_f32, c_int, c_vp, c_sz, c_vp),
    "bytes_kivi_quantize_pack": (c_vp, c_int, c_i64, c_int, c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp),
    "bytes_kivi_dequant": (c_vp, c_vp, c_vp, c_i64, c_int, c_int, c_int, c_int, c_vp, c_int, c_vp),
    "bytes_kivi_decode_workspace_size": (c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_szp),
    "bytes_kivi_decode_attn": (
        c_vp, c_vp, c_vp, c_vp, c_vp,                 # q, kq, k_scale, k_mn, k_res
        c_vp, c_vp, c_vp, c_vp, c_vp,                 # vq, v_scale, v_mn, v_res, out
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,   # B, Hq, Hk, Sq, R, D, bits
        c_i64, c_i64,                                 # q strides
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,     # k_res / v_res strides
        c_i64, c_i64,                                 # out strides
        c_f32, c_int, c_vp, c_sz, c_vp),
    "bytes_sparse_score": (
        c_vp, c_vp, c_int, c_vp, c_vp, c_vp,          # q, k, key mode, k scale, k min, out
        c_int, c_int, c_int, c_int, c_int, c_int,     # B, Hq, Hk, S, D, group_sum
        c_i64, c_i64, c_i64, c_i64, c_i64,            # q (b, h), k (b, h, s) strides
        c_i64, c_i64, c_i64,                          # scale / min strides (b, h, s)
        c_i64, c_i64,                                 # out strides (b, h)
        c_f32, c_vp, c_vp),                           # scaling, histogram (or None), stream
    "bytes_score_keys_pack": (c_vp, c_int, c_i64, c_int, c_i64, c_int, c_vp, c_vp, c_vp, c_vp),
    "bytes_topk_workspace_size": (c_i64, c_int, c_int, c_szp),
    "bytes_topk": (c_vp, c_i64, c_int, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_sz, c_vp),
    "bytes_gather_attn_workspace_size": (c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_szp),
    "bytes_gather_attn": (
        c_vp, c_vp, c_vp, c_int, c_vp, c_vp,          # q, k, v, k/v are fp8, idx, out
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,   # B, Hq, Hk, S, D, kb, per_head
        c_int, c_int,                                 # page, limit
        c_i64, c_i64,                                 # q strides
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,     # k, v strides (b, h, s)
        c_i64, c_i64,                                 # idx strides (b, h)
        c_i64, c_i64,                                 # out strides
        c_f32, c_int, c_vp, c_sz, c_vp),              # scaling, chunk, workspace, bytes, stream
    "bytes_quest_gather_attn": (
        c_vp, c_vp, c_vp, c_int, c_vp, c_i64, c_i64,  # q, k, v, k/v are fp8, bound, bound strides (b, h)
        c_int, c_int, c_vp,                           # np, npick, out
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,   # B, Hq, Hk, S, D, page, limit
        c_i64, c_i64,                                 # q strides
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,     # k, v strides (b, h, s)
        c_i64, c_i64,                                 # out strides
        c_f32, c_int, c_vp, c_sz, c_vp),              # scaling, chunk, workspace, bytes, stream
    "bytes_stream_read": (c_vp, c_i64, c_int, c_int, c_vp, c_vp),
    "bytes_empty_launch": (c_int, c_vp),
    "bytes_quest_page_minmax": (c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_vp),
    "bytes_quest_page_scores": (
        c_vp, c_vp, c_vp, c_vp,                       # q, kmin, kmax, bound
        c_int, c_int, c_int, c_int, c_int, c_int,     # B, Hq, Hk, np, D, page
        c_int, c_int,                                 # pos, local_w
        c_i64, c_i64, c_i64, c_i64,                   # q strides, bound strides
        c_f32, c_vp),                                 # scale, stream
    "bytes_pq_decode_workspace_size": (c_int, c_int, c_int, c_int, c_int, c_int, c_szp),
    "bytes_pq_decode_attn": (
        c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,   # mode, lut, q, kcb, kidx, vidx, vcb, v, out
        c_int, c_int, c_int, c_int, c_int, c_int, c_int,         # out_dtype, B, Hq, Hk, S, D, K
        c_i64, c_i64, c_i64, c_i64, c_i64,                       # lut (b, h), q (b, h), kcb head stride
        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,         # kidx (b, h, s), vidx (b, h, s), vcb head stride
        c_i64, c_i64, c_i64, c_i64, c_i64,                       # v (b, h, s), out (b, h)
        c_f32, c_int, c_vp, c_sz, c_vp),                         # scale, chunk, workspace, bytes, stream
    "bytes_pq_lut_decode_attn": (
        c_vp, c_i64, c_i64,                                      # lut, strides (b, h)
        c_vp, c_i64, c_i64, c_i64,                               # kidx, strides (batch|block, h, row)
        c_vp, c_i64, c_i64, c_i64, c_vp, c_i64,                  # vidx + strides, vcb, vcb head stride
        c_vp, c_int, c_i64, c_i64, c_i64,                        # v, v is fp8, strides
        c_vp, c_int, c_i64, c_i64, c_i64,                        # k_out, dtype, strides
        c_vp, c_int, c_i64, c_i64, c_int,                        # q_out, dtype, strides (b, h), C
        c_vp, c_i64, c_vp, c_int, c_int,                         # block table, row stride, lengths, bs, blocks
        c_vp, c_int, c_i64, c_i64,                               # out, dtype, strides (b, h)
        c_int, c_int, c_int, c_int, c_int, c_int,                # B, Hq, Hk, S, D, K
        c_f32, c_int, c_vp, c_sz, c_vp),                         # scale, chunk, workspace, bytes, stream
    "bytes_pq_lut_scores": (
        c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64,           # lut + strides, kidx + strides
        c_vp, c_int, c_i64, c_i64, c_i64,                        # k_out, dtype, strides
        c_vp, c_int, c_i64, c_i64, c_int,                        # q_out, dtype, strides, C
        c_vp, c_i64, c_i64,                                      # out [B, Hq, S], strides (b, h)
        c_int, c_int, c_int, c_int, c_int, c_int, c_vp),         # B, Hq, Hk, S, D, K, stream
    "bytes_pq_build_lut": (c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_f32, c_vp),
    "bytes_pq_encode": (c_vp, c_int, c_int, c_i64, c_i64, c_int, c_vp, c_int, c_i64, c_int, c_vp, c_vp),
    "bytes_pq_decode_vectors": (c_vp, c_int, c_i64, c_int, c_vp, c_int, c_i64, c_int, c_vp, c_vp),
    "bytes_pq_kmeans_update": (c_vp, c_int, c_i64, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp),
    "bytes_gather_reduce": (c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_int, c_int, c_int, c_int, c_vp),
    "bytes_packed_stage": (
        c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64,          # q + strides, packed keys + strides
        c_vp, c_vp, c_i64, c_i64, c_i64,                        # scale, zero, their strides
        c_vp, c_i64, c_i64,                                     # out + strides (b, h)
        c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_vp),  # B, Hq, Hk, S, D, bits, stage, stream
    "bytes_select_mask": (c_vp, c_i64, c_int, c_i64, c_vp, c_int, c_int, c_int, c_vp),
    "bytes_select_fill": (c_vp, c_int, c_i64, c_int, c_vp, c_int, c_i64, c_int, c_i64, c_vp, c_int, c_i64, c_vp),
    "bytes_select_pages": (c_vp, c_i64, c_int, c_int, c_i64, c_vp, c_vp),
    "bytes_select_mask_at": (c_vp, c_i64, c_int, c_i64, c_i64, c_vp, c_int, c_int, c_int, c_vp),
    "bytes_select_merge": (c_vp, c_i64, c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_int, c_int, c_int, c_i64, c_vp,
                           c_i64, c_int, c_vp, c_i64, c_int, c_vp),
    "bytes_select_recent": (c_vp, c_int, c_i64, c_int, c_vp, c_vp),
}
_RESTYPES = {"bytes_error_string": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()


def lib():
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"bytes_amd: {LIB_PATH} is missing; build it with "
                    "`python -m bytes_amd.build` (there is no CPU fallback)")
            h = ctypes.CDLL(LIB_PATH)
            for name, argt in SIGNATURES.items():
                fn = getattr(h, name)
                fn.argtypes = list(argt)
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = h
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = lib().bytes_error_string(rc)
        raise RuntimeError(f"bytes_amd.{name}: {msg.decode() if msg else 'error'} (hipError {rc})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


# ---------------------------------------------------------------------------
# Workspaces: zero-initialised byte buffers, one per (device, family).  The
# split-K decode kernels (dense, KIVI, gather, PQ) share the "splitk" family
# for their per-split partials.  The top-k kernels keep a histogram and list
# counters that they leave at zero when they finish, in a buffer of their own
# ("topk").  A buffer is cleared only when it is
# (re)allocated; it grows on demand, and the usual warm-up call before a graph
# capture sizes it.  Calls that share a buffer must be ordered on one stream
# (the reference harness runs everything on the current stream).
#
# A graph captured earlier keeps the address of the buffer it was captured
# with, so a buffer that has been replaced by a larger one is never released:
# it stays in _retired until the process ends, still zero at rest, and old
# graphs keep replaying into memory that nothing else owns.  A buffer cannot
# be created or grown while the current stream is capturing (the allocation
# would come from the graph's pool and its zero fill would only run at
# replay); that raises, and a warm-up call before the capture avoids it.
# ---------------------------------------------------------------------------
_ws: Dict[Tuple[int, str], torch.Tensor] = {}
_retired: List[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int, family: str = "splitk") -> torch.Tensor:
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), family)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"bytes_amd: the {family!r} workspace on cuda:{key[0]} needs {int(nbytes)} bytes "
                f"(has {0 if buf is None else buf.numel()}) during graph capture; make one eager call "
                "of the same shape before capturing")
        size = max(int(nbytes), 1 << 20)
        if buf is not None:
            _retired.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=dev)
        _ws[key] = buf
    return buf


def dtype_code(t: torch.Tensor) -> int:
    """0 bf16, 1 fp16, 2 fp32 (the OutDtype / input-dtype codes of the C ABI)."""
    codes = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
    if t.dtype not in codes:
        raise ValueError(f"dtype {t.dtype} not supported (bf16, fp16, fp32)")
    return codes[t.dtype]


HIP_ERROR_NOT_SUPPORTED = 801


def size_query(name: str, *args) -> int:
    out = ctypes.c_size_t(0)
    call(name, *args, ctypes.byref(out))
    return int(out.value)
