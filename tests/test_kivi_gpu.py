"""KIVI pack (bit-exact) and fused decode (north_star tolerance) vs the CPU oracle."""
import pytest
import torch

from bytes_amd import kivi as K
from bytes_amd import workloads as W
from oracle import reference as R

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
pytestmark = pytest.mark.gpu


def _to(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _check(out, ref, tag):
    d = (out.float().cpu() - ref.float()).abs()
    print(f"{tag}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, tag


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_pack_bit_exact(dev, bits, dtype):
    g = torch.Generator().manual_seed(bits)
    x = (torch.randn(3, 5, 256, generator=g) * 3).to(dtype)
    x[0, 0, :32] = 1.25                                  # constant group -> scale = 1e-8/levels
    x[0, 1, 32:64] = torch.arange(32) * 0.5              # exact grid -> half-way rounding cases
    code, scale, mn = K.quantize_and_pack_along_last_dim(x.to(dev), 32, bits)
    rc, rs, rm = R.kivi_quantize_and_pack_last_dim(x, 32, bits)
    assert torch.equal(code.cpu(), rc)
    assert torch.equal(scale.cpu().view(torch.int16), rs.view(torch.int16))
    assert torch.equal(mn.cpu().view(torch.int16), rm.view(torch.int16))


@pytest.mark.parametrize("bits", [2, 4])
def test_unpack_and_dequant(dev, bits):
    g = torch.Generator().manual_seed(10 + bits)
    codes = torch.randint(0, 2 ** bits, (2, 3, 4, 128), generator=g)
    words = R.kivi_pack_last_dim(codes, bits)
    un = K.unpack_tensor_last_dim(words.to(dev), bits)
    assert un.dtype == torch.float16 and torch.equal(un.cpu().long(), codes)
    sc = (torch.rand(2, 3, 4, 4, generator=g) + 0.1).half()
    mn = (torch.rand(2, 3, 4, 4, generator=g) - 0.5).half()
    dk = K.dequant_k(words.to(dev), sc.to(dev), mn.to(dev), 32, bits)
    ref = R.kivi_dequant_k(words, sc, mn, 32, bits, fp16_math=True)
    assert torch.equal(dk.cpu(), ref.half())
    dv = K.dequant_v(words.to(dev), sc.to(dev), mn.to(dev), 32, bits)
    assert torch.equal(dv.cpu(), R.kivi_dequant_v(words, sc, mn, 32, bits, fp16_math=True).half())


def _decode_case(dev, bits, B, Hq, Hk, D, L, Rw, seed=0, chunk=0):
    raw = W.kivi_raw(B, Hq, Hk, D, L, Rw, seed=seed)
    cpu = W.kivi_pack_inputs(raw, R.kivi_quantize_and_pack_last_dim, bits)
    gpu = _to(cpu, dev)
    args = [gpu[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale", "V_mn", "V_residual")]
    out = K.kivi_decode_attn(*args, bits, 32, chunk=chunk)
    ref = R.kivi_decode_attn(*[cpu[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale",
                                                 "V_mn", "V_residual")], bits, 32)
    assert out.shape == (B, Hq, 1, D) and out.dtype == torch.bfloat16
    _check(out, ref, f"kivi{bits} B{B} Hq{Hq} Hk{Hk} D{D} L{L} R{Rw} chunk{chunk}")
    return out


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("B,Hq,Hk,D,L,Rw", [
    (2, 8, 2, 128, 256 + 128, 128),     # kivi_latency.py integrity-gate shape (:104-110)
    (1, 7, 1, 128, 2048 + 64, 64),
    (2, 4, 4, 64, 1024 + 32, 32),       # D = 64, G = 1
    (1, 20, 1, 128, 640, 0),            # no residual, two head blocks
    (1, 4, 2, 128, 128, 128),           # residual only (Sq = 0)
    (1, 4, 2, 128, 300, 300),           # residual only, three 128-token residual splits, ragged end
    (1, 7, 1, 128, 1024 + 200, 200),    # residual pieces of 64 tokens (two tiles) on the last splits
    (2, 8, 2, 128, 256 + 384, 384),     # more residual than four 128-token pieces hold: own splits
    (1, 7, 1, 128, 2080 + 128, 128),    # Sq = 2080, an odd number of key groups: the streaming kernel
    (2, 4, 4, 64, 1056 + 32, 32),       # the same at D = 64, G = 1
    (8, 8, 8, 64, 2048 + 32, 32),       # 64 units x two 1024-token chunks: eight-wave workgroups at D = 64
    (4, 28, 4, 128, 2048 + 96, 96),     # 16 units, four-wave workgroups over a short cache, ragged residual
])
def test_decode_small(dev, bits, B, Hq, Hk, D, L, Rw):
    _decode_case(dev, bits, B, Hq, Hk, D, L, Rw, seed=L + bits)


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_odd_group_count(dev, bits):
    # Sq = 96: three 32-token key groups (2-bit key rows are 24 bytes: 8-byte key pieces)
    _decode_case(dev, bits, 1, 4, 2, 128, 96 + 16, 16, seed=3)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("extra", [0, 32])
@pytest.mark.parametrize("chunk", [64, 256, 512, 1280, 2304])
def test_decode_split_counts(dev, bits, extra, chunk):
    """Forced split lengths on both kernels: Sq = 4096 (an even number of key
    groups: the two-half kernel) and Sq = 4128 (odd: the streaming kernel,
    whose splits of 1280 and 2304 tokens run five and five phases, the second
    phase group padded with an empty phase, and whose 4128-token cache ends
    in a half tile)."""
    _decode_case(dev, bits, 1, 7, 1, 128, 4096 + extra + 128, 128, seed=4, chunk=chunk)


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_c2_odd_group_count_runs_fused(dev, bits):
    """C2 with 32 more packed tokens (Sq = 16288, an odd number of key groups)
    runs in the fused decode kernel (its launch is seen by the kernel timing
    hook) and matches the oracle."""
    from bytes_amd import _lib
    raw = W.kivi_raw(L=16288 + 128, seed=9)
    cpu = W.kivi_pack_inputs(raw, R.kivi_quantize_and_pack_last_dim, bits)
    g = _to(cpu, dev)
    names = ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale", "V_mn", "V_residual")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    t_before = e0.elapsed_time(e1)
    lib = _lib.lib()
    assert lib.bytes_set_kernel_events(2, e0.cuda_event, e1.cuda_event) == 0
    try:
        out = K.kivi_decode_attn(*[g[n] for n in names], bits)
    finally:
        lib.bytes_set_kernel_events(0, None, None)
    torch.cuda.synchronize()
    assert e0.elapsed_time(e1) != t_before and e0.elapsed_time(e1) > 0, "the fused KIVI kernel did not launch"
    _check(out, R.kivi_decode_attn(*[cpu[n] for n in names], bits), f"C2+32 kivi{bits}")


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_c2_full(dev, bits):
    """BASELINE C2: B=4, Hq=28, Hkv=4, D=128, L=16384, residual 128, outlier key channels x8."""
    raw = W.kivi_raw(seed=0)
    g = _to(W.kivi_pack_inputs(_to(raw, dev), K.quantize_and_pack_along_last_dim, bits), dev)
    out = K.kivi_decode_attn(*[g[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale",
                                              "V_mn", "V_residual")], bits)
    cpu = _to(g, "cpu")
    ref = R.kivi_decode_attn(*[cpu[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale",
                                                 "V_mn", "V_residual")], bits)
    _check(out, ref, f"C2 kivi{bits}")
    # the GPU pack of the full cache is bit-identical to the oracle's
    ref_pack = W.kivi_pack_inputs(raw, R.kivi_quantize_and_pack_last_dim, bits)
    for n in ("Kq", "Vq"):
        assert torch.equal(cpu[n], ref_pack[n]), n
    for n in ("K_scale", "K_mn", "V_scale", "V_mn"):
        assert torch.equal(cpu[n].view(torch.int16), ref_pack[n].view(torch.int16)), n
    # deterministic
    out2 = K.kivi_decode_attn(*[g[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale",
                                               "V_mn", "V_residual")], bits)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("B,Hq,Hk,D,L,Rw", [
    (2, 8, 4, 64, 16256 + 128, 128),      # two-half kernel, eight-wave workgroups
    (1, 14, 2, 128, 65536 + 64, 64),      # two-half kernel, residual pieces on the last splits
    (2, 8, 2, 128, 65536 + 200, 200),     # two-half kernel, two residual tiles per piece
    (2, 8, 4, 64, 16288 + 128, 128),      # streaming kernel, D = 64
    (1, 14, 2, 128, 65568 + 64, 64),      # streaming kernel: about 19 phases per split (phase-group loop)
])
def test_decode_long_contexts(dev, bits, B, Hq, Hk, D, L, Rw):
    _decode_case(dev, bits, B, Hq, Hk, D, L, Rw, seed=L + bits)


@pytest.mark.parametrize("Rw", [40, 64, 100, 128])
def test_decode_residual_lengths_eight_wave_grid(dev, Rw):
    """Eight-wave grid with 512-token splits (B=2, Hk=4, Sq=16256, 2-bit): the
    residual window, whole and ragged, rides in pieces on the last splits."""
    _decode_case(dev, 2, 2, 8, 4, 128, 16256 + Rw, Rw, seed=70 + Rw)


@pytest.mark.parametrize("Rw", [72, 128])
def test_decode_residual_lengths_c2_grid(dev, Rw):
    """The C2 grid (16 units of 1024-token splits, the last holding 896 tokens)
    with G = 2 and a whole or ragged residual window."""
    _decode_case(dev, 2, 2, 16, 8, 128, 16256 + Rw, Rw, seed=90 + Rw)


def test_decode_back_to_back_calls(dev):
    """Consecutive calls with new data, and a different split plan in between,
    reuse the shared split-K workspace: each call's partials overwrite the
    previous call's, and every result matches the oracle."""
    for i, (B, Hq, Hk, L, Rw) in enumerate([(2, 8, 2, 4096 + 128, 128), (2, 8, 2, 4096 + 128, 128),
                                            (1, 7, 1, 8192 + 64, 64), (2, 8, 2, 4096 + 128, 128)]):
        _decode_case(dev, 2 + 2 * (i % 2), B, Hq, Hk, 128, L, Rw, seed=50 + i)


def test_decode_many_splits_use_the_merge_kernel(dev):
    # chunk 256 over 69120 packed tokens: 270 splits, several blocks of the merge kernel
    _decode_case(dev, 2, 1, 7, 1, 128, 69120 + 32, 32, seed=6, chunk=256)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("B,Hq,Hk,L,Rw,gps", [
    (1, 7, 1, 4096 + 128, 128, 3),      # splits of 3 granules, the last one granule long
    (2, 8, 2, 4160 + 72, 72, 2),        # a last granule with one 64-token tile, ragged residual
    (1, 20, 1, 1024, 0, 8),             # four granules in one split, no residual, two head blocks
    (2, 32, 2, 5184 + 100, 100, 5),     # G = 16 (a full head block), Sq = 64 (mod 128)
    (1, 7, 1, 2048 + 300, 300, 1),      # one granule per split, three residual splits
])
def test_decode_pipelined(dev, bits, B, Hq, Hk, L, Rw, gps):
    """The pipelined kernel (D = 128, 2- and 4-bit) forced with splits of
    `gps` 256-token granules: partial last granules and splits, residual
    splits, head blocks of 16 and fewer columns."""
    _decode_case(dev, bits, B, Hq, Hk, 128, L, Rw, seed=L + gps + bits, chunk=-gps)


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_pipelined_long_cache_automatic(dev, bits):
    """A long cache (B=4, Hk=4, Sq=32768: four-granule splits fill two
    workgroups per CU) takes the pipelined kernel by default."""
    _decode_case(dev, bits, 4, 28, 4, 128, 32768 + 128, 128, seed=11 + bits)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("Sq,chunk,amp,vamp", [(16256, 512, 1800.0, 1000.0), (16288, 4096, 900.0, 1000.0),
                                               (16256, 512, 1800.0, 12000.0), (16288, 4096, 900.0, 12000.0),
                                               (16256, -8, 1800.0, 12000.0)])
def test_decode_rising_scores_large_values(dev, bits, Sq, chunk, amp, vamp):
    """Scores that climb by many octaves along the cache up to its middle (a
    bump along head 0's query in every key) and values of magnitude ~vamp
    (2-bit value scales up to a few thousand at 1000, about 8K to 20K at
    12000), on splits long enough that each wave runs several tiles: the
    two-half kernel (Sq = 16256, 512-token splits: a wave's two tiles 256
    tokens, ~7.7 octaves, apart), the streaming kernel (Sq = 16288,
    4096-token splits: eight phases per wave, 512 tokens and ~7.7 octaves
    apart) and the pipelined kernel (chunk -8: 2048-token splits,
    eight tiles per wave 256 tokens apart).  The running maximum moves on many tiles, and probabilities
    times value scales must stay finite in fp16 for any finite fp16 scale.
    Error bound relative to the output's magnitude."""
    B, Hq, Hk, D, Rw = 1, 7, 1, 128, 64
    raw = W.kivi_raw(B, Hq, Hk, D, Sq + Rw, Rw, seed=Sq + bits)
    q = raw["q"].float()
    t = torch.arange(Sq + Rw, dtype=torch.float32)
    bump = (1.0 - (t - Sq / 2).abs() / (Sq / 2)).clamp(min=0.0)
    qdir = q[0, 0, 0] / q[0, 0, 0].pow(2).sum()
    k = raw["k"].float() + (bump[:, None] * amp) * qdir
    raw["k"] = k.to(torch.bfloat16)
    raw["v"] = (raw["v"].float() * vamp).to(torch.bfloat16)
    cpu = W.kivi_pack_inputs(raw, R.kivi_quantize_and_pack_last_dim, bits)
    vs_max = cpu["V_scale"].float().max().item()
    print(f"kivi{bits} value scales up to {vs_max:.0f}", flush=True)
    if vamp > 1000.0 and bits == 2:
        assert vs_max > 8000.0
    gpu = _to(cpu, dev)
    names = ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale", "V_mn", "V_residual")
    out = K.kivi_decode_attn(*[gpu[n] for n in names], bits, 32, chunk=chunk)
    ref = R.kivi_decode_attn(*[cpu[n] for n in names], bits, 32)
    assert torch.isfinite(out.float()).all()
    d = (out.float().cpu() - ref.float()).abs()
    mag = ref.float().abs().max()
    print(f"kivi{bits} Sq{Sq} chunk{chunk} vamp{vamp:.0f} rising: max-abs {d.max():.3e} of |ref| max {mag:.3e}", flush=True)
    assert d.max() <= 2e-2 * mag and d.mean() <= 2e-3 * mag
