"""The no-allocation dense decode entry point (bytes_decode_attn_bf16_noalloc),
called through the C ABI, equals the workspace entry point bit for bit on two
calls in a row, the second with a smaller input; sizes beyond its scratch are
refused."""
import ctypes

import pytest
import torch

from bytes_amd import _lib
from bytes_amd import attention_kernels as AK
from bytes_amd import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu


def _args(q, k, v, out):
    B, Hq, _, D = q.shape
    _, Hk, S, _ = k.shape
    qs = q.squeeze(2)
    return ([qs.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hk, S, D,
             qs.stride(0), qs.stride(1), k.stride(0), k.stride(1), k.stride(2),
             v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1)],
            (B, Hq, Hk, S, D))


def _noalloc(q, k, v, scale, chunk=0):
    out = torch.full((q.shape[0], q.shape[1], q.shape[3]), float("nan"), dtype=torch.bfloat16, device=q.device)
    a, _ = _args(q, k, v, out)
    rc = _lib.lib().bytes_decode_attn_bf16_noalloc(*a, ctypes.c_float(scale), chunk,
                                                  torch.cuda.current_stream().cuda_stream)
    return rc, out


def _with_workspace(q, k, v, scale, chunk=0):
    out = torch.empty((q.shape[0], q.shape[1], q.shape[3]), dtype=torch.bfloat16, device=q.device)
    a, (B, Hq, Hk, S, D) = _args(q, k, v, out)
    n = _lib.size_query("bytes_decode_attn_bf16_workspace_size", B, Hq, Hk, S, D, chunk)
    ws = torch.zeros(max(n, 1), dtype=torch.uint8, device=q.device)
    rc = _lib.lib().bytes_decode_attn_bf16(*a, ctypes.c_float(scale), chunk, ws.data_ptr(), ws.numel(),
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    return out


@pytest.mark.parametrize("first,second", [
    ((4, 28, 4, 128, 16384), (1, 14, 2, 64, 8192)),     # dense L16K point, then BASELINE C1
    ((2, 14, 2, 64, 3000), (1, 7, 1, 128, 700)),
])
def test_noalloc_equals_workspace_entry_point(dev, first, second):
    for i, shape in enumerate((first, second)):
        x = W.dense(*shape, seed=60 + i)
        q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
        rc, got = _noalloc(q, k, v, x["scale"])
        assert rc == 0, _lib.lib().bytes_error_string(rc)
        want = _with_workspace(q, k, v, x["scale"])
        torch.cuda.synchronize()
        print(f"noalloc call {i} {shape}: equal={torch.equal(got, want)}", flush=True)
        assert torch.equal(got, want), f"call {i} {shape}"
        if shape[-1] <= 8192:
            d = (got.float().cpu() - R.decode_attn(x["q"], x["k"], x["v"], scale=x["scale"]).squeeze(2).float()).abs()
            assert d.max() <= 2e-2 and d.mean() <= 2e-3


def test_noalloc_refuses_partials_beyond_its_scratch(dev):
    q = torch.zeros((64, 64, 1, 128), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((64, 64, 256, 128), dtype=torch.bfloat16, device=dev)
    need = _lib.size_query("bytes_decode_attn_bf16_workspace_size", 64, 64, 64, 256, 128, 128)
    assert need > AK.NOALLOC_SCRATCH_BYTES                # 4096 units x 2 splits of partials
    rc, _ = _noalloc(q, k, k, 0.1, chunk=128)
    assert rc == 2                                   # hipErrorOutOfMemory
    with pytest.raises(ValueError, match="scratch"):
        AK.decode_attn_bf16_noalloc(q, k, k, torch.empty((64, 64, 128), dtype=torch.bfloat16, device=dev),
                                    0.1, chunk=128)


def test_noalloc_python_wrapper_writes_out(dev):
    x = W.dense(1, 14, 2, 64, 8192, seed=70)
    q, k, v = (x[n].to(dev) for n in ("q", "k", "v"))
    out = torch.empty((1, 14, 1, 64), dtype=torch.bfloat16, device=dev)
    assert AK.decode_attn_bf16_noalloc(q, k, v, out, x["scale"]) is out
    assert torch.equal(out, AK.decode_attn_bf16(q, k, v, x["scale"]))
