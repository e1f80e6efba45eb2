"""Pins the CPU oracle against brute force, closed forms and invariants.

Each check is chosen so that a plausible slip in the oracle (dropped term,
wrong index or sign, transposed operand, wrong tie rule) fails it.  CPU only.
"""
import itertools
import math

import pytest
import torch

from oracle import reference as R


def _bf16(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


# ---------------------------------------------------------------- GQA / dense
def test_repeat_kv_matches_index_rule():
    x = torch.arange(2 * 3 * 4 * 5, dtype=torch.float32).reshape(2, 3, 4, 5)
    y = R.repeat_kv(x, 4)
    assert y.shape == (2, 12, 4, 5)
    for h in range(12):
        assert torch.equal(y[:, h], x[:, h // 4])


def _attn_bruteforce(q, k, v, scale):
    """float64 per-(b, h_q) loop with explicit exp/sum (test_correctness.py:64-75 form)."""
    B, Hq, _, D = q.shape
    Hk, S = k.shape[1], k.shape[2]
    G = Hq // Hk
    out = torch.zeros(B, Hq, 1, D, dtype=torch.float64)
    for b in range(B):
        for h in range(Hq):
            qq = q[b, h, 0].double()
            kk = k[b, h // G].double()
            vv = v[b, h // G].double()
            s = [float((qq * kk[t]).sum()) * scale for t in range(S)]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            out[b, h, 0] = sum(e[t] / z * vv[t] for t in range(S))
    return out


@pytest.mark.parametrize("B,Hq,Hk,S,D", [(2, 8, 2, 37, 16), (1, 3, 3, 20, 8), (1, 6, 1, 9, 4)])
def test_decode_attn_bruteforce(B, Hq, Hk, S, D):
    q, k, v = _bf16(B, Hq, 1, D, seed=1), _bf16(B, Hk, S, D, seed=2), _bf16(B, Hk, S, D, seed=3)
    ref = _attn_bruteforce(q, k, v, 0.37)
    out = R.decode_attn(q, k, v, scale=0.37, out_dtype=torch.float32)
    assert (out.double() - ref).abs().max() < 1e-5


def test_decode_attn_invariants():
    q, k = _bf16(1, 4, 1, 8, seed=4), _bf16(1, 2, 50, 8, seed=5)
    row = _bf16(8, seed=6)
    v = row.expand(1, 2, 50, 8).contiguous()
    out = R.decode_attn(q, k, v, out_dtype=torch.float32)        # uniform V -> V row
    assert torch.allclose(out[0, :, 0], row.float().expand(4, 8), atol=1e-6)
    ones = torch.ones(1, 2, 50, 8)
    assert torch.allclose(R.decode_attn(q, k, ones, out_dtype=torch.float32), torch.ones(1, 4, 1, 8), atol=1e-6)
    # head h_q reads kv head h_q // G: swapping kv heads swaps query-head groups
    v2 = _bf16(1, 2, 50, 8, seed=7)
    a = R.decode_attn(q, k, v2, out_dtype=torch.float32)
    b = R.decode_attn(q[:, [2, 3, 0, 1]], k.flip(1), v2.flip(1), out_dtype=torch.float32)
    assert torch.allclose(a[:, [2, 3, 0, 1]], b, atol=1e-6)


# ---------------------------------------------------------------- KIVI layout
@pytest.mark.parametrize("bits", [2, 4])
def test_kivi_pack_unpack_exhaustive(bits):
    fpi = 32 // bits
    vals = list(range(2 ** bits))
    # every code value in every slot of a word
    codes = torch.tensor([[c if i == s else 0 for i in range(fpi)]
                          for s in range(fpi) for c in vals], dtype=torch.int64)
    words = R.kivi_pack_last_dim(codes, bits)
    assert words.dtype == torch.int32 and words.shape == (len(codes), 1)
    for row, w in zip(codes.tolist(), words[:, 0].tolist()):
        expect = sum(c << (i * bits) for i, c in enumerate(row))
        assert (w & 0xFFFFFFFF) == expect
    assert torch.equal(R.kivi_unpack_last_dim(words, bits), codes)


def test_kivi_unpack_hand_word():
    # bits=2: logical positions 0..15 of word 0 at bits 2i; 0xE4 = codes 0,1,2,3
    w = torch.tensor([[0xE4, -1]], dtype=torch.int32)
    c = R.kivi_unpack_last_dim(w, 2)
    assert c[0, :4].tolist() == [0, 1, 2, 3] and c[0, 4:16].tolist() == [0] * 12
    assert c[0, 16:].tolist() == [3] * 16
    c4 = R.kivi_unpack_last_dim(torch.tensor([[0x76543210]], dtype=torch.int32), 4)
    assert c4[0].tolist() == list(range(8))


def test_asym_quant_closed_form():
    x = torch.tensor([[-1.0, 0.0, 0.5, 2.0], [3.0, 3.0, 3.0, 3.0]])
    codes, scale, xmin = R.asym_quant_codes(x, 4, dim=-1)
    assert codes[0].tolist() == [0, 1, 2, 3]          # (x+1)/1: 0, 1, 1.5 -> 2, 3
    # round half to even: (1.5+1)/1 = 2.5 -> 2 (not 3); (0.5+1)/1 = 1.5 -> 2
    codes2, _, _ = R.asym_quant_codes(torch.tensor([[-1.0, 1.5, 0.5, 2.0]]), 4, dim=-1)
    assert codes2[0].tolist() == [0, 2, 2, 3]
    assert codes[1].tolist() == [0, 0, 0, 0]           # constant group
    assert float(scale[1, 0]) == float(torch.tensor(1e-8) / 3)   # clamp(min=1e-8) in fp32
    assert float(scale[0, 0]) == 1.0 and float(xmin[0, 0]) == -1.0


@pytest.mark.parametrize("bits", [2, 4])
def test_kivi_quantize_pack_roundtrip(bits):
    x = _bf16(2, 3, 64, seed=8).to(torch.float16)
    code, scale, mn = R.kivi_quantize_and_pack_last_dim(x, 32, bits)
    assert code.shape == (2, 3, 64 * bits // 32) and scale.shape == (2, 3, 2) and mn.dtype == torch.float16
    c = R.kivi_unpack_last_dim(code, bits)
    # the codes are those of the fp32 fake-quant closed form
    g = x.float().reshape(2, 3, 2, 32)
    lo, hi = g.amin(-1, keepdim=True), g.amax(-1, keepdim=True)
    s = (hi - lo).clamp(min=1e-8) / (2 ** bits - 1)
    expect = torch.clamp(torch.round((g - lo) / s), 0, 2 ** bits - 1).reshape(2, 3, 64)
    assert torch.equal(c, expect.long())
    # min element -> code 0, max element -> top code, in every group
    cg = c.reshape(2, 3, 2, 32)
    assert torch.equal(torch.gather(cg, -1, g.argmin(-1, keepdim=True)), torch.zeros(2, 3, 2, 1, dtype=torch.long))
    assert torch.equal(torch.gather(cg, -1, g.argmax(-1, keepdim=True)),
                       torch.full((2, 3, 2, 1), 2 ** bits - 1, dtype=torch.long))


def test_kivi_dequant_layouts():
    bits, gs = 2, 32
    B, H, D, Sq = 1, 2, 4, 64
    codes = torch.randint(0, 4, (B, H, D, Sq), generator=torch.Generator().manual_seed(0))
    Kq = R.kivi_pack_last_dim(codes, bits)
    sc = torch.rand(B, H, D, Sq // gs, generator=torch.Generator().manual_seed(1)).half() + 0.5
    mn = torch.rand(B, H, D, Sq // gs, generator=torch.Generator().manual_seed(2)).half() - 0.5
    kd = R.kivi_dequant_k(Kq, sc, mn, gs, bits)
    assert kd.shape == (B, H, Sq, D)
    for d, t in itertools.product(range(D), [0, 31, 32, 63]):
        e = codes[0, 1, d, t] * sc[0, 1, d, t // gs].float() + mn[0, 1, d, t // gs].float()
        assert float(kd[0, 1, t, d]) == pytest.approx(float(e), abs=1e-6)
    # values: per-token groups of 32 channels along the last dim
    vc = torch.randint(0, 4, (B, H, 3, 64), generator=torch.Generator().manual_seed(3))
    vs = torch.rand(B, H, 3, 2, generator=torch.Generator().manual_seed(4)).half() + 0.5
    vm = torch.rand(B, H, 3, 2, generator=torch.Generator().manual_seed(5)).half() - 0.5
    vd = R.kivi_dequant_v(R.kivi_pack_last_dim(vc, bits), vs, vm, gs, bits)
    assert vd.shape == (B, H, 3, 64)
    for t, d in itertools.product(range(3), [0, 31, 32, 63]):
        e = vc[0, 1, t, d] * vs[0, 1, t, d // gs].float() + vm[0, 1, t, d // gs].float()
        assert float(vd[0, 1, t, d]) == pytest.approx(float(e), abs=1e-6)


def test_kivi_decode_matches_dense_on_dequantized_cache():
    bits, gs, R_ = 4, 32, 16
    B, Hq, Hk, D, Sq = 1, 4, 2, 64, 64
    k, v, q = _bf16(B, Hk, Sq + R_, D, seed=9), _bf16(B, Hk, Sq + R_, D, seed=10), _bf16(B, Hq, 1, D, seed=11)
    Kq, Ks, Km = R.kivi_quantize_and_pack_last_dim(k[:, :, :Sq].transpose(2, 3).half(), gs, bits)
    Vq, Vs, Vm = R.kivi_quantize_and_pack_last_dim(v[:, :, :Sq].half(), gs, bits)
    out = R.kivi_decode_attn(q, Kq, Ks, Km, k[:, :, Sq:], Vq, Vs, Vm, v[:, :, Sq:], bits, gs)
    kd = torch.cat([R.kivi_dequant_k(Kq, Ks, Km, gs, bits), k[:, :, Sq:].float()], 2)
    vd = torch.cat([R.kivi_dequant_v(Vq, Vs, Vm, gs, bits), v[:, :, Sq:].float()], 2)
    ref = _attn_bruteforce(q, kd, vd, 1 / math.sqrt(D))
    assert (out.double() - ref).abs().max() < 1e-2   # bf16 output rounding
    # 4-bit dequant error is bounded by half a step of each group
    err = (R.kivi_dequant_k(Kq, Ks, Km, gs, bits) - k[:, :, :Sq].float()).abs()
    assert float(err.max()) <= float(Ks.float().max()) * 0.5 + 1e-2


# ---------------------------------------------------------------- PQ
def test_pq_encode_bruteforce():
    g = torch.Generator().manual_seed(3)
    cb = torch.randn(4, 16, 8, generator=g)
    x = torch.randn(50, 32, generator=g)
    idx = R.pq_encode(x, cb)
    for j in range(4):
        d = torch.cdist(x[:, j * 8:(j + 1) * 8].double(), cb[j].double())
        assert torch.equal(idx[:, j], d.argmin(1))
    exact = torch.stack([cb[j, 5] for j in range(4)]).reshape(1, 32)
    assert R.pq_encode(exact, cb).tolist() == [[5, 5, 5, 5]]
    dup = cb.clone()
    dup[:, 9] = dup[:, 2]                                 # tie -> first index
    assert R.pq_encode(torch.stack([dup[j, 2] for j in range(4)]).reshape(1, 32), dup).tolist() == [[2] * 4]


def test_pq_lut_scores_loop_and_dequant_equivalence():
    g = torch.Generator().manual_seed(4)
    B, Hq, Hk, S, M, K, ds = 1, 4, 2, 12, 4, 8, 8
    cb = torch.randn(M, K, ds, generator=g)
    q = torch.randn(B, Hq, 1, M * ds, generator=g).to(torch.bfloat16)
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g)
    v = torch.randn(B, Hk, S, M * ds, generator=g)
    lut = R.pq_build_lut(q, cb)
    sc = R.pq_lut_scores(lut, k_idx)
    for h, t in itertools.product(range(Hq), range(S)):
        e = sum(float(lut[0, h, j, k_idx[0, h // 2, t, j]]) for j in range(M))
        assert float(sc[0, h, t]) == pytest.approx(e, abs=1e-5)
    a = R.decode_attn_pq_lut(lut, k_idx, v)
    b = R.decode_attn_dequant(q.float(), k_idx, cb, v)          # fp32 out (out dtype = q dtype)
    assert (a - b).abs().max() < 1e-4                      # LUT path == dequant path
    # per-head codebooks that are all equal == shared codebook
    cbh = cb.unsqueeze(0).expand(Hk, M, K, ds).contiguous()
    assert torch.allclose(R.pq_build_lut(q, cbh), lut)
    vi = torch.randint(0, K, (B, Hk, S, M), generator=g)
    o1 = R.decode_attn_pq_lut_kv(lut, k_idx, vi, cb)
    o2 = R.decode_attn_pq_lut(lut, k_idx, torch.stack([R.pq_decode(vi[:, h], cb) for h in range(Hk)], 1))
    assert (o1 - o2).abs().max() < 1e-5


# ---------------------------------------------------------------- top-k
def _topk_brute(row, k):
    def key(i):
        x = row[i]
        if math.isnan(x):
            return (0, 0.0, i)
        return (1, -x if x != 0 else 0.0, i)
    return sorted(range(len(row)), key=key)[:k]


def test_topk_bruteforce_with_ties():
    g = torch.Generator().manual_seed(5)
    pool = torch.tensor([0.0, -0.0, 1.0, -1.0, 2.5, float("inf"), float("-inf"), float("nan")])
    for trial in range(40):
        n = int(torch.randint(1, 40, (1,), generator=g))
        row = pool[torch.randint(0, len(pool), (n,), generator=g)]
        for k in {1, n // 2 or 1, n}:
            got = R.topk_indices(row, k).tolist()
            assert got == _topk_brute(row.tolist(), k)


def test_topk_matches_torch_without_ties():
    x = torch.randperm(1000, generator=torch.Generator().manual_seed(6)).float().reshape(4, 250) * 0.37
    for k in (1, 17, 250):
        assert torch.equal(R.topk_indices(x, k), x.topk(k, dim=-1).indices)
        assert torch.equal(R.topk_indices(x, k, sorted_by_score=False),
                           torch.sort(x.topk(k, dim=-1).indices, -1).values)


def test_streaming_topk_equals_global():
    g = torch.Generator().manual_seed(7)
    x = torch.randint(-5, 5, (3, 300), generator=g).float()      # heavy ties
    for k, chunk in [(10, 64), (64, 64), (100, 17), (300, 1000)]:
        assert torch.equal(R.streaming_topk(x, k, chunk), R.topk_indices(x, k))


# ---------------------------------------------------------------- Quest
def test_quest_bound_is_upper_bound():
    B, Hq, Hk, S, D, page = 1, 4, 2, 50, 16, 16
    q, k = _bf16(B, Hq, 1, D, seed=12), _bf16(B, Hk, S, D, seed=13)
    kmin, kmax = R.quest_page_minmax(k, page)
    assert kmin.shape == (B, Hk, 4, D)
    bound = R.quest_page_scores(q, kmin, kmax)
    s = R.sparse_score_scalar(q, k, 1.0)
    for p in range(4):
        hi = min(S, (p + 1) * page)
        assert torch.all(bound[..., p] >= s[..., p * page:hi].amax(-1) - 1e-4)
    # single-token pages: the bound is the exact score
    k1min, k1max = R.quest_page_minmax(k, 1)
    assert torch.allclose(R.quest_page_scores(q, k1min, k1max), s, atol=1e-4)
    # last partial page is padded with the last key
    assert torch.equal(kmin[:, :, 3], k[:, :, 48:50].amin(2))


def test_quest_select_expansion():
    B, Hq, Hk, S, D = 1, 2, 1, 40, 8
    q, k = _bf16(B, Hq, 1, D, seed=14), _bf16(B, Hk, S, D, seed=15)
    pidx, tok, bound = R.quest_select(q, k, budget_tokens=20, page=16)
    assert pidx.shape == (1, 2, 2) and tok.shape == (1, 2, 32)
    assert tok.max() <= S - 1
    for h in range(2):
        assert pidx[0, h].tolist() == _topk_brute(bound[0, h].tolist(), 2)


# ---------------------------------------------------------------- scores / gather
def test_group_scores_and_gather():
    B, Hq, Hk, S, D = 1, 6, 2, 30, 16
    q, k, v = _bf16(B, Hq, 1, D, seed=16), _bf16(B, Hk, S, D, seed=17), _bf16(B, Hk, S, D, seed=18)
    s = R.sparse_score_scalar(q, k, 0.25)
    gs = R.group_scores(q, k, 0.25)
    for h in range(Hk):
        assert torch.allclose(gs[0, h], s[0, 3 * h] + s[0, 3 * h + 1] + s[0, 3 * h + 2], atol=1e-5)
    full = torch.arange(S).expand(B, Hq, S)
    a = R.sparse_gather_attn(q, k, v, full, 0.25)
    d = R.decode_attn(q, k, v, scale=0.25)
    assert (a.float() - d.float()).abs().max() < 1e-2
    # sentinel / out-of-range entries are masked
    padded = torch.cat([full, torch.full((B, Hq, 3), S), torch.full((B, Hq, 1), -1)], -1)
    assert torch.equal(R.sparse_gather_attn(q, k, v, padded, 0.25), a)
    # per-KV-head idx shared by the group == repeated per-q-head idx
    idx_kv = torch.randint(0, S, (B, Hk, 7), generator=torch.Generator().manual_seed(1))
    assert torch.equal(R.sparse_gather_attn(q, k, v, idx_kv, 0.25),
                       R.sparse_gather_attn(q, k, v, idx_kv.repeat_interleave(3, 1), 0.25))


@pytest.mark.parametrize("bits", [4, 2])
def test_score_keys_pack_exhaustive(bits):
    """Every code in every slot of a byte survives pack -> unpack, and a hand
    byte decodes as the reference loop (test_correctness.py:708-718) reads it."""
    per = 8 // bits
    codes = torch.cartesian_prod(*[torch.arange(2 ** bits)] * per).reshape(-1, per)
    packed = R.score_keys_pack(codes, bits)
    assert packed.shape == (codes.shape[0], 1)
    assert torch.equal(R.score_keys_unpack(packed, bits), codes)
    if bits == 4:
        assert R.score_keys_pack(torch.tensor([[3, 12]]), 4).item() == 3 | (12 << 4)
    else:
        assert R.score_keys_pack(torch.tensor([[1, 2, 3, 0]]), 2).item() == 1 | (2 << 2) | (3 << 4)


def test_quantize_and_pack_score_keys_closed_form():
    g = torch.Generator().manual_seed(2)
    k = torch.randn(2, 3, 5, 64, generator=g).to(torch.bfloat16)
    k[0, 0, 0, :32] = 0.75                                   # constant group
    for bits in (4, 2):
        packed, sc, zr = R.quantize_and_pack_score_keys(k, bits, 32)
        assert packed.dtype == torch.uint8 and packed.shape == (2, 3, 5, 64 * bits // 8)
        assert sc.dtype == torch.bfloat16 and sc.shape == (2, 3, 5, 2)
        codes = R.score_keys_unpack(packed, bits).reshape(2, 3, 5, 2, 32)
        kf = k.float().reshape(2, 3, 5, 2, 32)
        lo, hi = kf.amin(-1), kf.amax(-1)
        # each group's extremes quantize to the end codes (non-constant groups)
        for b_, h_, s_, gi in [(1, 2, 4, 1), (0, 1, 2, 0)]:
            row = codes[b_, h_, s_, gi]
            assert row[kf[b_, h_, s_, gi].argmin()] == 0
            assert row[kf[b_, h_, s_, gi].argmax()] == 2 ** bits - 1
        assert torch.all(codes[0, 0, 0, 0] == 0)
        assert torch.equal(zr, lo.to(torch.bfloat16))
        exp_scale = ((hi - lo).clamp(min=1e-8) / (2 ** bits - 1)).to(torch.bfloat16)
        assert torch.equal(sc, exp_scale)
        # dequantized keys are within half a step of the originals, plus what the
        # bf16 rounding of scale (times the code) and of the minimum adds
        dq = R.score_keys_dequant(packed, sc, zr, bits, 32)
        step = sc.float().repeat_interleave(32, -1)
        lvl = 2 ** bits - 1
        bound = 0.5 * step + lvl * step * 2 ** -8 + 2 ** -8 * lo.repeat_interleave(32, -1).abs() + 1e-6
        assert torch.all((dq - k.float()).abs() <= bound)


# ---------------------------------------------------------------- PQ asym / paged
def test_pq_asym_scores_loop_and_full_width():
    """Per-token loop (benchmarks/test_correctness.py:455-466 form) and, with a
    LUT built from the key codebook, equality with q . [k_hat, k_out]."""
    g = torch.Generator().manual_seed(7)
    B, Hq, Hk, S, M, K, C = 2, 4, 2, 9, 8, 8, 2
    cb = torch.randn(M, K, 8, generator=g)
    q = torch.randn(B, Hq, 1, M * 8, generator=g).to(torch.bfloat16)
    k_idx = torch.randint(0, K, (B, Hk, S, M), generator=g, dtype=torch.uint8)
    k_out = torch.randn(B, Hk, S, C, generator=g).to(torch.bfloat16)
    q_out = torch.randn(B, Hq, C, generator=g).to(torch.bfloat16)
    lut = R.pq_build_lut(q, cb)
    s = R.pq_asym_scores(lut, k_idx, k_out, q_out)
    G = Hq // Hk
    for b in range(B):
        for h in range(Hq):
            for t in range(S):
                ref = sum(float(lut[b, h, j, int(k_idx[b, h // G, t, j])]) for j in range(M))
                ref += sum(float(q_out[b, h, c]) * float(k_out[b, h // G, t, c]) for c in range(C))
                assert abs(float(s[b, h, t]) - ref) < 1e-4
    khat = torch.stack([R.pq_decode(k_idx[:, h], cb) for h in range(Hk)], 1)          # [B,Hk,S,D]
    qf = torch.cat([q.float(), q_out.float().unsqueeze(2)], -1)
    kf = torch.cat([khat, k_out.float()], -1)
    full = torch.matmul(qf.reshape(B, Hk, G, -1), kf.transpose(-1, -2)).reshape(B, Hq, S)
    assert torch.allclose(s, full, atol=1e-4)
    # C = 0 reduces to the LUT decode
    v = torch.randn(B, Hk, S, M * 8, generator=g).to(torch.bfloat16)
    a = R.decode_attn_pq_lut_asym(lut, k_idx, k_out[..., :0], q_out[..., :0], v)
    assert torch.equal(a, R.decode_attn_pq_lut(lut, k_idx, v))


def test_paged_rows_follow_the_block_table():
    """A cache split into shuffled blocks and read back through the table
    (src/attention_kernels.py:536-545 rule) reproduces the contiguous rows, so
    the paged decodes equal the contiguous ones per sequence."""
    g = torch.Generator().manual_seed(3)
    Hk, bs, M, K = 2, 16, 8, 8
    lens = [45, 78]
    nb = [(n + bs - 1) // bs for n in lens]
    perm = torch.randperm(sum(nb), generator=g)
    table = torch.full((2, max(nb)), -1, dtype=torch.int32)
    k_idx = torch.randint(0, K, (2, Hk, max(lens), M), generator=g, dtype=torch.uint8)
    v_idx = torch.randint(0, K, (2, Hk, max(lens), M), generator=g, dtype=torch.uint8)
    kp = torch.zeros(sum(nb), Hk, bs, M, dtype=torch.uint8)
    vp = torch.zeros_like(kp)
    c = 0
    for b in range(2):
        for i in range(nb[b]):
            table[b, i] = int(perm[c])
            c += 1
        for t in range(lens[b]):
            kp[table[b, t // bs], :, t % bs] = k_idx[b, :, t]
            vp[table[b, t // bs], :, t % bs] = v_idx[b, :, t]
    for b in range(2):
        assert torch.equal(R.paged_rows(kp, table, b, lens[b], bs)[0], k_idx[b, :, :lens[b]])
    cb = torch.randn(M, K, 8, generator=g)
    lut = torch.randn(2, 4, M, K, generator=g)
    out = R.paged_attn_pq_lut_kv(lut, kp, vp, cb, table, torch.tensor(lens), bs)
    for b in range(2):
        ref = R.decode_attn_pq_lut_kv(lut[b:b + 1], k_idx[b:b + 1, :, :lens[b]], v_idx[b:b + 1, :, :lens[b]], cb)
        assert torch.equal(out[b:b + 1], ref)


# ---------------------------------------------------------------------------
# k-means (src/quantization.py:102-132), pinned by a brute-force Lloyd replay
# ---------------------------------------------------------------------------
def _lloyd_bruteforce(pts, cent, draw):
    """One Lloyd step over Python lists: squared distances summed coordinate by
    coordinate, the first centroid on ties, then cluster i (in index order)
    becomes the mean of its points or, when empty, the point draw() names."""
    labels = []
    for p in pts:
        best, bi = None, 0
        for i, c in enumerate(cent):
            dist = sum((a - b) ** 2 for a, b in zip(p, c))
            if best is None or dist < best:
                best, bi = dist, i
        labels.append(bi)
    new = []
    for i in range(len(cent)):
        members = [p for p, l in zip(pts, labels) if l == i]
        if members:
            new.append([sum(col) / len(members) for col in zip(*members)])
        else:
            new.append(list(pts[draw()]))
    return new, labels


def _sse(pts, cent):
    return sum(min(sum((a - b) ** 2 for a, b in zip(p, c)) for c in cent) for p in pts)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_kmeans_one_step_bruteforce(seed):
    g = torch.Generator().manual_seed(100 + seed)
    X = torch.randn(37, 3, generator=g)
    pts = X.tolist()
    k = 5
    out = R.kmeans(X, k, 1, torch.Generator().manual_seed(seed))
    rng = torch.Generator().manual_seed(seed)
    init = [pts[i] for i in torch.randperm(37, generator=rng)[:k].tolist()]
    want, _ = _lloyd_bruteforce(pts, init, lambda: int(torch.randint(0, 37, (1,), generator=rng)))
    assert torch.allclose(out, torch.tensor(want), atol=1e-5, rtol=0)


def test_kmeans_empty_cluster_takes_drawn_point():
    # two distinct values: any three initial centroids repeat one, the repeat
    # loses every tie to the lower index, and its cluster is re-seeded
    X = torch.tensor([[0.0, 0.0]] * 6 + [[5.0, 5.0]] * 4)
    pts = X.tolist()
    for seed in range(6):
        out = R.kmeans(X, 3, 1, torch.Generator().manual_seed(seed))
        rng = torch.Generator().manual_seed(seed)
        init = [pts[i] for i in torch.randperm(10, generator=rng)[:3].tolist()]
        draws = []

        def draw():
            draws.append(int(torch.randint(0, 10, (1,), generator=rng)))
            return draws[-1]
        want, labels = _lloyd_bruteforce(pts, init, draw)
        assert len(set(labels)) < 3 and draws, "the data must leave a cluster empty"
        assert torch.equal(out, torch.tensor(want)), f"seed {seed}"


def test_kmeans_sse_does_not_increase():
    g = torch.Generator().manual_seed(7)
    centers = torch.randn(4, 2, generator=g) * 6
    X = (centers.repeat_interleave(30, 0) + torch.randn(120, 2, generator=g))
    pts = X.tolist()
    prev = None
    for it in range(0, 7):
        cent = R.kmeans(X, 4, it, torch.Generator().manual_seed(3)).tolist()
        _, labels = _lloyd_bruteforce(pts, cent, lambda: 0)
        assert len(set(labels)) == 4            # no empty cluster: Lloyd's descent holds
        sse = _sse(pts, cent)
        if prev is not None:
            assert sse <= prev * (1 + 1e-6) + 1e-6, f"iteration {it}: {sse} > {prev}"
        prev = sse


def test_kmeans_pads_when_points_do_not_exceed_k():
    X = torch.randn(5, 8)
    out = R.kmeans(X, 8, 10, torch.Generator().manual_seed(0))
    assert out.shape == (8, 8)
    assert torch.equal(out[:5], X) and torch.equal(out[5:], torch.zeros(3, 8))
    same = R.kmeans(X, 5, 10, torch.Generator().manual_seed(0))
    assert torch.equal(same, X)


# ---------------------------------------------------------------------------
# select_topk / _quest_select / attend_topk over query chunks (Qc >= 1)
# ---------------------------------------------------------------------------
def _brute_select(scores, pos, S, kb, local_w):
    """Per row: the causal keys (t <= pos), recent ones forced to +inf, ranked
    by Python's sorted() on (-score, t); slots past the causal count hold S."""
    out = []
    for row, p in zip(scores, pos):
        cands = []
        for t, s in enumerate(row):
            if t > p:
                continue
            if local_w > 0 and p - local_w < t <= p:
                s = math.inf
            cands.append((-s, t))
        picked = [t for _, t in sorted(cands)[:kb]]
        out.append(picked + [S] * (kb - len(picked)))
    return out


@pytest.mark.parametrize("local_w", [0, 3])
def test_select_topk_from_scores_bruteforce(local_w):
    g = torch.Generator().manual_seed(11)
    Qc, S = 5, 40
    pos = torch.tensor([2, 9, 17, 31, 39])
    max_key = int(pos.max()) + 1
    scores = torch.randint(-3, 4, (2, 3, Qc, max_key), generator=g).float()   # many ties
    for kb in (1, 4, 8, 12):
        want = [[_brute_select(scores[b, h].tolist(), pos.tolist(), S, kb, local_w) for h in range(3)]
                for b in range(2)]
        for chunk in (1, 5, 16, max_key):
            got = R.select_topk_from_scores(scores, pos, S, kb, chunk, local_w)
            assert got.tolist() == want, (kb, chunk)


def test_select_topk_exact_integer_keys():
    """Integer-valued q and keys give exact fp32 scores (and many ties), so the
    full selection equals the brute-force ranking of Python dot products."""
    g = torch.Generator().manual_seed(12)
    B, Hq, Hk, Qc, S, D = 1, 4, 2, 3, 30, 8
    q = torch.randint(-2, 3, (B, Hq, Qc, D), generator=g).to(torch.bfloat16)
    k = torch.randint(-2, 3, (B, Hk, S, D), generator=g).to(torch.bfloat16)
    pos = torch.tensor([5, 20, 29])
    got = R.select_topk_exact(q, k, pos, S, 9, 7, 0.5)
    for h in range(Hq):
        sc = [[sum(float(q[0, h, r, d]) * float(k[0, h // 2, t, d]) for d in range(D)) * 0.5 for t in range(30)]
              for r in range(Qc)]
        assert got[0, h].tolist() == _brute_select(sc, pos.tolist(), S, 9, 0), h
    kr = R.repeat_kv(k, 2)                                   # GQA-expanded keys give the same ids
    assert torch.equal(R.select_topk_exact(q, kr, pos, S, 9, 7, 0.5), got)


def test_select_recent_is_the_most_recent_causal_window():
    pos = torch.tensor([0, 3, 9, 40])
    for kb in (1, 4, 10, 16):
        got = R.select_recent(2, 3, pos, kb)
        assert got.shape == (2, 3, 4, kb) and got.dtype == torch.int64
        for r, p in enumerate(pos.tolist()):
            m = min(kb, p + 1)
            row = got[1, 2, r].tolist()
            assert row[:m] == sorted(range(p + 1))[::-1][:m]          # the newest m positions, newest first
            assert set(row[:m]) == set(range(p + 1 - m, p + 1))
            assert all(x == 0 for x in row[m:])                        # clamp at 0 past the first key


@pytest.mark.parametrize("local_w", [0, 20])
def test_quest_select_rows_bruteforce(local_w):
    g = torch.Generator().manual_seed(13)
    B, Hq, Hk, Qc, S, D, page = 1, 4, 2, 3, 70, 8, 16
    q = torch.randint(-2, 3, (B, Hq, Qc, D), generator=g).to(torch.bfloat16)
    k = torch.randint(-3, 4, (B, Hk, S, D), generator=g).to(torch.bfloat16)
    pos = torch.tensor([10, 40, 69])
    kb = 35                                                  # ceil(35/16) = 3 pages
    got = R.quest_select_rows(q, k, pos, S, kb, page, 0.25, local_w)
    np_ = 5
    for h in range(Hq):
        for r in range(Qc):
            p = int(pos[r])
            cands = []
            for pg in range(np_):
                rows = [min(t, S - 1) for t in range(pg * page, pg * page + page)]
                bnd = sum(max(float(q[0, h, r, d]) * min(float(k[0, h // 2, t, d]) for t in rows),
                              float(q[0, h, r, d]) * max(float(k[0, h // 2, t, d]) for t in rows))
                          for d in range(D)) * 0.25
                if pg * page > p:
                    bnd = -math.inf
                if local_w and max(p - local_w + 1, 0) // page <= pg <= p // page:
                    bnd = math.inf
                cands.append((-bnd, pg))
            pages = [pg for _, pg in sorted(cands)[:3]]
            want = [min(pg * page + o, S - 1) for pg in pages for o in range(page)]
            assert got[0, h, r].tolist() == want, (h, r)
    # one row at the last position equals the decode-step selection
    one = R.quest_select_rows(q[:, :, 2:3], k, pos[2:3], S, kb, page, 0.25)
    _, tok, _ = R.quest_select(q[:, :, 2:3], k, kb, page, 0.25)
    assert torch.equal(one.squeeze(2), tok)


def test_attend_topk_bruteforce_and_causal_dense():
    g = torch.Generator().manual_seed(14)
    B, Hq, Hk, Qc, S, D = 1, 4, 2, 3, 24, 16
    q = torch.randn(B, Hq, Qc, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g).to(torch.float32)
    pos = torch.tensor([3, 12, 23])
    idx = torch.randint(-2, S + 3, (B, Hq, Qc, 10), generator=g)
    idx[..., 0] = 0                                          # every row keeps one valid entry
    out = R.attend_topk(q, k, v, idx, pos, 0.3)
    for h in range(Hq):
        for r in range(Qc):
            sel = [int(t) for t in idx[0, h, r] if 0 <= int(t) < S and int(t) <= int(pos[r])]
            sc = [sum(float(q[0, h, r, d]) * float(k[0, h // 2, t, d]) for d in range(D)) * 0.3 for t in sel]
            m = max(sc)
            w = [math.exp(s - m) for s in sc]
            want = [sum(wi * float(v[0, h // 2, t, d]) for wi, t in zip(w, sel)) / sum(w) for d in range(D)]
            assert torch.allclose(out[0, h, r], torch.tensor(want), atol=1e-5), (h, r)
    # every position 0..S-1 selected: causal dense attention of each row
    allidx = torch.arange(S).expand(B, Hq, Qc, S)
    full = R.attend_topk(q, k, v, allidx, pos, 0.3)
    for r in range(Qc):
        p = int(pos[r])
        dense = R.decode_attn(q[:, :, r:r + 1], k[:, :, :p + 1], v[:, :, :p + 1], scale=0.3)
        assert torch.allclose(full[:, :, r], dense.squeeze(2).float(), atol=5e-3)   # bf16 output of decode_attn


# ---------------------------------------------------------------------------
# harness microkernels: gather-reduce and the staged packed-score probe
# ---------------------------------------------------------------------------
def test_gather_reduce_closed_forms():
    g = torch.Generator().manual_seed(21)
    H, S, D = 3, 50, 16
    v = torch.randn(H, S, D, generator=g).half()
    full = torch.arange(S).expand(H, S)
    assert torch.allclose(R.gather_reduce(v, full), v.float().sum(1), atol=1e-4)
    perm = torch.stack([torch.randperm(S, generator=g) for _ in range(H)])
    assert torch.allclose(R.gather_reduce(v, perm), v.float().sum(1), atol=1e-4)
    one = torch.tensor([[7], [0], [S - 1]])
    assert torch.equal(R.gather_reduce(v, one), torch.stack([v[0, 7], v[1, 0], v[2, S - 1]]).float())
    twice = torch.tensor([[4, 4, 9]] * H)
    assert torch.allclose(R.gather_reduce(v, twice), 2 * v[:, 4].float() + v[:, 9].float(), atol=1e-4)


@pytest.mark.parametrize("bits", [4, 2])
def test_packed_stage_closed_forms(bits):
    g = torch.Generator().manual_seed(22)
    B, Hq, Hk, S, D = 1, 4, 2, 9, 64
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
    p, s, z = R.quantize_and_pack_score_keys(k, bits, 32)
    st = [R.packed_stage(q, p, s, z, bits, i) for i in range(4)]
    ex = lambda t: R.repeat_kv(t, 2)  # noqa: E731  per-KV-head sums seen by every query head of the group
    assert torch.equal(st[0], ex((8 // bits) * p.long().sum(-1, keepdim=True).float()).squeeze(-1))
    assert torch.equal(st[1], ex(R.score_keys_unpack(p, bits).sum(-1, keepdim=True).float()).squeeze(-1))
    deq = R.score_keys_dequant(p, s, z, bits, 32)
    assert torch.allclose(st[2], ex(deq.sum(-1, keepdim=True)).squeeze(-1), atol=1e-4)
    assert torch.allclose(st[3], R.sparse_score_packed(q, p, s, z, 1.0, bits, 32), atol=1e-4)
