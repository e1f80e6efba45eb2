"""CPU restatement of the saifmb0/bytes decode-attention hot path (the oracle).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker; never by the product path.

Every function cites the reference file:line it restates (paths relative to
the saifmb0/bytes checkout).  All arithmetic is plain torch on the CPU in
fp32 unless a function says otherwise; integer/bit work is exact.

Pinning (how each function is checked independently of its own formula) is
listed in each docstring as "Pinned by:"; the tests in tests/test_oracle*.py
carry those checks.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

NEG_INF = float("-inf")


# ---------------------------------------------------------------------------
# GQA helpers
# ---------------------------------------------------------------------------
def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B,Hk,S,D] -> [B,Hk*n_rep,S,D]; query head h reads KV head h // n_rep.

    Restates benchmarks/sparse_attention.py:85-90 (same as
    benchmarks/kivi_latency.py:20-24).
    Pinned by: test_repeat_kv_matches_index_rule (h -> h // G by brute force).
    """
    if n_rep == 1:
        return x
    B, H, S, D = x.shape
    return x[:, :, None, :, :].expand(B, H, n_rep, S, D).reshape(B, H * n_rep, S, D)


def _softmax_attend(scores: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """fp32 softmax over the last dim of scores, then weights @ v (fp32)."""
    p = torch.softmax(scores.float(), dim=-1)
    return torch.matmul(p, v.float())


# ---------------------------------------------------------------------------
# a1: dense decode attention
# ---------------------------------------------------------------------------
def decode_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                scale: float = 1.0, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Single-query GQA attention: softmax(scale * q.K^T) V per (b, h_q).

    Restates src/attention_kernels.py:8-92 (`_decode_attn_bf16_kernel`,
    `decode_attn_bf16`): fp32 scores and online softmax, fp32 accumulation,
    output cast to q's dtype (:77).  The reference applies no softmax scale
    (:42); ``scale`` (default 1.0) multiplies the fp32 scores.  The fp8 form
    (:97-182) is the same with K/V upcast from float8_e4m3fn.
    Loop reference: benchmarks/test_correctness.py:64-75.

    q [B,Hq,1,D]; k, v [B,Hk,S,D] -> [B,Hq,1,D].
    Pinned by: per-head brute-force loop, uniform-V invariant, G=1 == MHA,
    softmax rows summing to one (tests/test_oracle.py).
    """
    B, Hq, _, D = q.shape
    Hk = k.shape[1]
    G = Hq // Hk
    qf = q.float().reshape(B, Hk, G, D)
    s = torch.matmul(qf, k.float().transpose(-1, -2)) * scale       # [B,Hk,G,S]
    o = _softmax_attend(s, v)                                         # [B,Hk,G,D]
    od = out_dtype if out_dtype is not None else q.dtype
    return o.reshape(B, Hq, 1, D).to(od)


# ---------------------------------------------------------------------------
# a2/a3: KIVI pack / unpack / dequant (int32 words, codes along the last dim)
# ---------------------------------------------------------------------------
def kivi_unpack_last_dim(code: torch.Tensor, bits: int) -> torch.Tensor:
    """int32 words -> integer codes along the last dim (int64 result).

    Restates benchmarks/kivi_latency.py:26-35 (`unpack_tensor_last_dim`):
    logical position w*(32/bits)+i is held in word w at bits [i*bits,(i+1)*bits).
    (The reference returns the codes as fp16; the values are identical.)
    Pinned by: exhaustive round trip with kivi_pack_last_dim over every code
    value in every slot, and a hand-built word (tests/test_oracle.py).
    """
    fpi = 32 // bits
    mask = (1 << bits) - 1
    c = code.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(fpi, dtype=torch.int64) * bits
    vals = (c.unsqueeze(-1) >> shifts) & mask                         # [..., W, fpi]
    return vals.reshape(*code.shape[:-1], code.shape[-1] * fpi)


def kivi_pack_last_dim(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Integer codes [..., N] -> int32 words [..., N*bits/32]; inverse of
    kivi_unpack_last_dim (the bit layout read by kivi_latency.py:26-35)."""
    fpi = 32 // bits
    N = codes.shape[-1]
    assert N % fpi == 0
    c = codes.to(torch.int64).reshape(*codes.shape[:-1], N // fpi, fpi)
    shifts = torch.arange(fpi, dtype=torch.int64) * bits
    w = (c << shifts).sum(-1)                                         # < 2^32, exact
    w = torch.where(w >= 2 ** 31, w - 2 ** 32, w)
    return w.to(torch.int32)


def asym_quant_codes(x: torch.Tensor, levels: int, dim: int):
    """Asymmetric min/max uniform quantization: returns (codes, scale, xmin) in fp32.

    Restates src/quantization.py:432-442 (`_asym_uniform_fakequant`) without
    the final dequant: scale = max(max-min, 1e-8)/(levels-1),
    code = clamp(round_half_even((x-min)/scale), 0, levels-1).
    Pinned by: codes reproduce the fake-quant values of the closed form,
    endpoints map to 0 and levels-1, constant groups give code 0.
    """
    xf = x.float()
    xmin = xf.amin(dim=dim, keepdim=True)
    xmax = xf.amax(dim=dim, keepdim=True)
    scale = (xmax - xmin).clamp(min=1e-8) / (levels - 1)
    q = torch.clamp(torch.round((xf - xmin) / scale), 0, levels - 1)
    return q.to(torch.int64), scale, xmin


def kivi_quantize_and_pack_last_dim(x: torch.Tensor, group_size: int, bits: int):
    """Group-wise asym quantize along the last dim and pack (KIVI layout).

    Restates the call contract of KIVI's `triton_quantize_and_pack_along_last_dim`
    (called at benchmarks/kivi_latency.py:123,127): groups of `group_size`
    consecutive elements of the last dim share fp16 (scale, mn); codes are
    packed 32/bits per int32 in the layout of kivi_latency.py:26-35.  The
    arithmetic is src/quantization.py:432-442 in fp32; scale and mn are
    rounded to fp16 after the codes are chosen.  KIVI's own kernel is not in
    the reference checkout, so its exact rounding is parity unpinned; this
    function is the build's definition (bit-exact target for the GPU pack).

    x [..., T] (T % group_size == 0, group_size % (32/bits) == 0)
    -> (code int32 [..., T*bits/32], scale fp16 [..., T/group_size], mn fp16 same)
    """
    T = x.shape[-1]
    assert T % group_size == 0
    xg = x.reshape(*x.shape[:-1], T // group_size, group_size)
    codes, scale, xmin = asym_quant_codes(xg, 2 ** bits, dim=-1)
    code = kivi_pack_last_dim(codes.reshape(*x.shape[:-1], T), bits)
    return code, scale.squeeze(-1).to(torch.float16), xmin.squeeze(-1).to(torch.float16)


def kivi_dequant_k(Kq, K_scale, K_mn, group_size: int, bits: int, fp16_math: bool = False):
    """Packed per-channel keys [B,H,D,Sq*bits/32] -> dequantized [B,H,Sq,D].

    Restates benchmarks/kivi_latency.py:37-46 (`dequant_k`).  With
    fp16_math=True the arithmetic is the reference's fp16 (c*scale rounded,
    then +mn rounded); otherwise c*scale+mn in fp32 (the build's kernels).
    """
    B, H, D, _ = Kq.shape
    c = kivi_unpack_last_dim(Kq, bits)                                # [B,H,D,Sq]
    Sq = c.shape[-1]
    ng = Sq // group_size
    c = c.reshape(B, H, D, ng, group_size)
    if fp16_math:
        kd = c.to(torch.float16) * K_scale.unsqueeze(-1) + K_mn.unsqueeze(-1)
    else:
        kd = c.float() * K_scale.float().unsqueeze(-1) + K_mn.float().unsqueeze(-1)
    return kd.reshape(B, H, D, Sq).transpose(2, 3).contiguous()


def kivi_dequant_v(Vq, V_scale, V_mn, group_size: int, bits: int, fp16_math: bool = False):
    """Packed per-token values [B,H,Sq,D*bits/32] -> dequantized [B,H,Sq,D].

    Restates benchmarks/kivi_latency.py:48-57 (`dequant_v`); fp16_math as in
    kivi_dequant_k.
    """
    B, H, Sq, _ = Vq.shape
    c = kivi_unpack_last_dim(Vq, bits)                                # [B,H,Sq,D]
    D = c.shape[-1]
    ng = D // group_size
    c = c.reshape(B, H, Sq, ng, group_size)
    if fp16_math:
        vd = c.to(torch.float16) * V_scale.unsqueeze(-1) + V_mn.unsqueeze(-1)
    else:
        vd = c.float() * V_scale.float().unsqueeze(-1) + V_mn.float().unsqueeze(-1)
    return vd.reshape(B, H, Sq, D)


def kivi_decode_attn(Q, Kq, K_scale, K_mn, K_residual, Vq, V_scale, V_mn, V_residual,
                     bits: int, group_size: int = 32, scale: Optional[float] = None):
    """softmax([Q.K_dq^T, Q.K_res^T] * scale) . [V_dq; V_res] per query head.

    Restates the semantics of benchmarks/kivi_latency.py:59-100
    (`kivi_decode_attn` == `kivi_decode_attn_ref` over `dequant_k`/`dequant_v`);
    scale defaults to 1/sqrt(D) (:76).  The dequantized cache is c*scale+mn in
    fp32, the softmax and accumulation are fp32 (the reference rounds
    intermediate scores/weights to Q's dtype); output is Q's dtype.
    Pinned by: equals decode_attn() on the explicitly dequantized and
    concatenated cache; with bits-only codes at scale 1 / mn 0 it reduces to
    attention on integer keys (tests/test_oracle.py).
    """
    D = Q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    Kd = kivi_dequant_k(Kq, K_scale, K_mn, group_size, bits)
    Vd = kivi_dequant_v(Vq, V_scale, V_mn, group_size, bits)
    K = torch.cat([Kd, K_residual.float()], dim=2)
    V = torch.cat([Vd, V_residual.float()], dim=2)
    return decode_attn(Q, K, V, scale=scale, out_dtype=Q.dtype)


# ---------------------------------------------------------------------------
# a5/a6: product quantization
# ---------------------------------------------------------------------------
def _per_head_codebook(cb: torch.Tensor, Hk: int) -> torch.Tensor:
    """Shared [M,K,dsub] (reference layout, src/quantization.py:145) or per-head
    [Hk,M,K,dsub] codebooks -> [Hk,M,K,dsub]."""
    if cb.dim() == 3:
        return cb.unsqueeze(0).expand(Hk, *cb.shape)
    assert cb.dim() == 4 and cb.shape[0] == Hk
    return cb


def pq_encode(x: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """Nearest-codeword indices: argmin_c sum_e (x_e - c_e)^2, first index on ties.

    Restates src/quantization.py:203-211 (CPU path of ProductQuantizer.quantize:
    cdist + argmin).  The squared distance is accumulated in fp32 in element
    order e = 0..dsub-1 with separate multiply and add (no fused multiply-add),
    the order the GPU encode kernel uses, so indices are bit-exact.
    x [..., M*dsub]; centroids [M,K,dsub] -> uint8/int64 [..., M].
    Pinned by: brute force against torch.cdist argmin on tie-free inputs;
    exact codewords encode to their own index (tests/test_oracle.py).
    """
    M, K, dsub = centroids.shape
    xs = x.float().reshape(-1, M, dsub)
    c = centroids.float()
    dist = torch.zeros(xs.shape[0], M, K)
    for e in range(dsub):
        d = xs[:, :, e].unsqueeze(-1) - c[:, :, e].unsqueeze(0)      # [N,M,K]
        dist = dist + d * d
    idx = torch.argmin(dist, dim=-1)                                   # first min
    return idx.reshape(*x.shape[:-1], M)


def pq_decode(idx: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """Codes [..., M] -> vectors [..., M*dsub] (src/quantization.py:213-226)."""
    M, K, dsub = centroids.shape
    flat = idx.reshape(-1, M).long()
    out = torch.stack([centroids[j][flat[:, j]] for j in range(M)], dim=1)
    return out.reshape(*idx.shape[:-1], M * dsub)


def kmeans(X: torch.Tensor, k: int, num_iters: int, generator: torch.Generator) -> torch.Tensor:
    """Codebook fitting (setup only, not on the timed path).

    Restates src/quantization.py:102-132 (`kmeans_pytorch`) step for step:
    - N <= k: the points followed by k - N zero rows (:111-114);
    - initial centroids: the first k points of one randperm(N) (:117-118);
    - each iteration assigns every point to argmin of cdist (first index on
      ties, :122-123), then updates the clusters in index order (:126-130):
      a non-empty cluster takes the mean of its points, an empty one the point
      X[randint(0, N, (1,))], drawn in that order from the same generator.
    The reference draws from torch's global RNG; here the generator is
    explicit.  Arithmetic is fp32 (X is converted first).
    """
    N, d = X.shape
    X = X.float()
    if N <= k:
        return torch.cat([X.clone(), torch.zeros(k - N, d)], 0)
    perm = torch.randperm(N, generator=generator)
    cent = X[perm[:k]].clone()
    for _ in range(num_iters):
        labels = torch.argmin(torch.cdist(X, cent), dim=1)
        for i in range(k):
            members = labels == i
            if bool(members.any()):
                cent[i] = X[members].mean(dim=0)
            else:
                cent[i] = X[torch.randint(0, N, (1,), generator=generator)]
    return cent


def pq_build_lut(q: torch.Tensor, centroids: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """LUT[b,h,j,c] = scale * sum_e q[b,h,j*dsub+e] * cb[h//G, j, c, e]  (fp32).

    Restates the LUT precompute of benchmarks/test_correctness.py:181-182 and
    :272-273 (`einsum("bhmd,mkd->bhmk")`), with optional per-KV-head codebooks
    [Hk,M,K,dsub] (BASELINE C3) and the softmax scale folded in.
    q [B,Hq,1,D] or [B,Hq,D] -> [B,Hq,M,K].
    """
    if q.dim() == 4:
        q = q.squeeze(2)
    B, Hq, D = q.shape
    if centroids.dim() == 3:
        M, K, dsub = centroids.shape
        qs = q.float().reshape(B, Hq, M, dsub)
        lut = torch.einsum("bhmd,mkd->bhmk", qs, centroids.float())
    else:
        Hk, M, K, dsub = centroids.shape
        G = Hq // Hk
        qs = q.float().reshape(B, Hk, G, M, dsub)
        lut = torch.einsum("bhgmd,hmkd->bhgmk", qs, centroids.float()).reshape(B, Hq, M, K)
    return lut * scale


def pq_lut_scores(lut: torch.Tensor, k_idx: torch.Tensor) -> torch.Tensor:
    """scores[b,h,t] = sum_j lut[b,h,j,k_idx[b,h//G,t,j]] (fp32, j ascending).

    Restates the score loop of src/attention_kernels.py:330-341 / :425-435.
    Pinned by: per-token Python loop (benchmarks/test_correctness.py:282-291
    form) at small shapes.
    """
    B, Hq, M, K = lut.shape
    Hk = k_idx.shape[1]
    G = Hq // Hk
    idx = repeat_kv(k_idx.long(), G)                                   # [B,Hq,S,M]
    s = torch.zeros(B, Hq, idx.shape[2])
    for j in range(M):
        s = s + torch.gather(lut[:, :, j, :].float(), 2, idx[..., j])
    return s


def decode_attn_pq_lut_kv(lut, k_idx, v_idx, v_centroids, d_sub_v: int = 8):
    """LUT-scored keys + codebook-reconstructed values.

    Restates src/attention_kernels.py:397-500 (`decode_attn_pq_lut_kv`): no
    scale inside (fold it into the LUT); output dtype = v_centroids.dtype (:484).
    v_centroids [M_v,K_v,dsub] (reference) or [Hk,M_v,K_v,dsub] (per head).
    """
    B, Hq, M, K = lut.shape
    Hk = k_idx.shape[1]
    G = Hq // Hk
    s = pq_lut_scores(lut, k_idx)                                      # [B,Hq,S]
    cb = _per_head_codebook(v_centroids, Hk).float()                   # [Hk,Mv,Kv,dsub]
    Mv = cb.shape[1]
    vh = torch.stack([cb[h][torch.arange(Mv)[None, :], v_idx[:, h].long()]
                      for h in range(Hk)], dim=1)                      # [B,Hk,S,Mv,dsub]
    vh = vh.reshape(B, Hk, v_idx.shape[2], -1)
    o = _softmax_attend(s.reshape(B, Hk, G, -1), vh)                  # [B,Hk,G,D]
    return o.reshape(B, Hq, 1, -1).to(v_centroids.dtype)


def decode_attn_pq_lut(lut, k_idx, v):
    """LUT-scored keys, dense V.  Restates src/attention_kernels.py:301-392;
    output dtype = v.dtype (:375)."""
    B, Hq, M, K = lut.shape
    Hk = k_idx.shape[1]
    G = Hq // Hk
    s = pq_lut_scores(lut, k_idx)
    o = _softmax_attend(s.reshape(B, Hk, G, -1), v)
    return o.reshape(B, Hq, 1, -1).to(v.dtype)


def decode_attn_dequant(q, k_idx, centroids, v, d_sub: int = 8):
    """Codebook-reconstructed keys, dense V, no scale.

    Restates src/attention_kernels.py:187-296 (`decode_attn_dequant`); output
    dtype = q.dtype (:278).  Loop reference benchmarks/test_correctness.py:142-150.
    """
    Hk = k_idx.shape[1]
    cb = _per_head_codebook(centroids, Hk).float()
    kh = torch.stack([pq_decode(k_idx[:, h], cb[h]) for h in range(Hk)], dim=1)
    return decode_attn(q, kh, v, scale=1.0, out_dtype=q.dtype)


def pq_asym_scores(lut, k_idx, k_out, q_out) -> torch.Tensor:
    """LUT scores plus the exact outlier channels:
    s[b,h,t] = sum_j lut[b,h,j,k_idx[t,j]] + sum_c q_out[b,h,c] * k_out[b,h//G,t,c] (fp32).

    Restates paths A and B of src/attention_kernels.py:660-685 (decode) and
    :943-955 (`sparse_score_pq_lut_asym`).  Pinned by: per-token Python loop
    (benchmarks/test_correctness.py:455-466 form) and equality with full-width
    q.k when the LUT comes from the same codebook.
    """
    s = pq_lut_scores(lut, k_idx)
    C = k_out.shape[-1]
    if C > 0:
        G = lut.shape[1] // k_idx.shape[1]
        ko = repeat_kv(k_out.float(), G)                                   # [B,Hq,S,C]
        s = s + (ko * q_out.float()[:, :, None, :]).sum(-1)
    return s


def decode_attn_pq_lut_asym(lut, k_idx, k_out, q_out, v):
    """LUT + outlier scores, dense bf16 or float8_e4m3fn V, no scale inside.

    Restates src/attention_kernels.py:625-753 (`decode_attn_pq_lut_asym`);
    output dtype = v.dtype, bf16 for fp8 values (:735)."""
    B, Hq, M, K = lut.shape
    Hk = k_idx.shape[1]
    G = Hq // Hk
    s = pq_asym_scores(lut, k_idx, k_out, q_out)
    o = _softmax_attend(s.reshape(B, Hk, G, -1), v.float())
    od = torch.bfloat16 if v.dtype == torch.float8_e4m3fn else v.dtype
    return o.reshape(B, Hq, 1, -1).to(od)


def paged_rows(x_paged: torch.Tensor, block_table: torch.Tensor, b: int, n: int, block_size: int) -> torch.Tensor:
    """Rows 0..n-1 of sequence b from a paged cache [blocks, H, block_size, ...]:
    token t is row t % block_size of block block_table[b, t // block_size]
    (src/attention_kernels.py:536-545 / :813-819).  Returns [1, H, n, ...]."""
    t = torch.arange(n)
    blk = block_table[b, t // block_size].long()
    return x_paged[blk, :, t % block_size].transpose(0, 1).unsqueeze(0)


def paged_attn_pq_lut_kv(lut, k_idx_paged, v_idx_paged, v_centroids, block_table, context_lens, block_size=16):
    """Restates src/attention_kernels.py:505-622: the LUT-KV decode of each
    sequence over its context_lens[b] tokens gathered through the block table."""
    outs = []
    for b in range(lut.shape[0]):
        n = int(context_lens[b])
        ki = paged_rows(k_idx_paged, block_table, b, n, block_size)
        vi = paged_rows(v_idx_paged, block_table, b, n, block_size)
        outs.append(decode_attn_pq_lut_kv(lut[b:b + 1], ki, vi, v_centroids))
    return torch.cat(outs, 0)


def paged_attn_pq_lut_asym(lut, k_idx_paged, k_out_paged, q_out, v_paged, block_table, context_lens,
                           block_size=16):
    """Restates src/attention_kernels.py:756-906: the asymmetric PQ-LUT decode
    of each sequence over its context_lens[b] tokens gathered through the
    block table."""
    outs = []
    for b in range(lut.shape[0]):
        n = int(context_lens[b])
        ki = paged_rows(k_idx_paged, block_table, b, n, block_size)
        ko = paged_rows(k_out_paged, block_table, b, n, block_size)
        vv = paged_rows(v_paged, block_table, b, n, block_size)
        outs.append(decode_attn_pq_lut_asym(lut[b:b + 1], ki, ko, q_out[b:b + 1], vv))
    return torch.cat(outs, 0)


def sparse_decode_pq_lut(lut, k_idx, k_out, q_out, q, k, v, frac: float, scaling: float):
    """LUT + outlier scores -> top-kb per query head (ties to the lowest
    index) -> exact gathered attention.  Restates
    src/attention_kernels.py:1062-1074 with the build's deterministic top-k."""
    s = pq_asym_scores(lut, k_idx, k_out, q_out)
    kb = budget(frac, s.shape[-1])
    return sparse_gather_attn(q, k, v, topk_indices(s, kb), scaling)


# ---------------------------------------------------------------------------
# a10: deterministic top-k (total order: score desc, index asc)
# ---------------------------------------------------------------------------
def canonical_scores(s: torch.Tensor) -> torch.Tensor:
    """Canonicalise fp32 scores for ranking: -0 -> +0, every NaN -> +NaN.

    The build's total order ranks NaN above +inf (as torch.topk does) and
    treats +0/-0 as equal so the lowest index wins their tie."""
    s = s.float()
    s = torch.where(s == 0, torch.zeros_like(s), s)
    return s


def order_key(s: torch.Tensor) -> torch.Tensor:
    """Monotone int64 key of canonical fp32 scores (larger score -> larger key;
    NaN -> largest).  Used to make ranking a pure integer sort."""
    s = canonical_scores(s)
    nan = torch.isnan(s)
    bits = s.view(torch.int32).to(torch.int64)
    key = torch.where(bits < 0, -(bits & 0x7FFFFFFF) - 1, bits)        # order-preserving
    return torch.where(nan, torch.full_like(key, 2 ** 40), key)


def topk_indices(scores: torch.Tensor, k: int, sorted_by_score: bool = True) -> torch.Tensor:
    """Indices of the k largest entries per row under the total order
    (score descending, index ascending on ties).

    Replaces `scores.topk(kb, dim=-1).indices` (src/attention_kernels.py:1262,
    benchmarks/sparse_attention.py:307,358) whose tie order is unspecified;
    the lowest-index tie rule is the BASELINE contract.  With
    sorted_by_score=True the result is ordered like torch.topk(sorted=True);
    otherwise by ascending index.  Returns int64 [..., k].
    Pinned by: brute force with Python's sorted() on tiny rows, equality with
    torch.topk on tie-free rows, chunked streaming merge == global selection.
    """
    key = order_key(scores)
    n = key.shape[-1]
    idx = torch.arange(n, dtype=torch.int64).expand_as(key)
    # composite key: primary -key (desc), secondary index (asc).  Stable sort on
    # -key keeps ascending index among equal keys.
    order = torch.sort(-key, dim=-1, stable=True).indices
    sel = order[..., :k]
    if not sorted_by_score:
        sel = torch.sort(sel, dim=-1).values
    del idx
    return sel


def streaming_topk(scores: torch.Tensor, k: int, chunk: int) -> torch.Tensor:
    """Chunked streaming top-k with running candidate merge, as in
    benchmarks/sparse_attention.py:287-309 (`select_topk`, sentinel idx = S for
    unfilled slots, :292-293), under the build's total order.  Returns indices
    ordered like topk_indices(sorted_by_score=True)."""
    S = scores.shape[-1]
    lead = scores.shape[:-1]
    run_s = torch.full((*lead, k), NEG_INF)
    run_i = torch.full((*lead, k), S, dtype=torch.int64)
    for c0 in range(0, S, chunk):
        c1 = min(c0 + chunk, S)
        cs = torch.cat([run_s, scores[..., c0:c1].float()], -1)
        ci = torch.cat([run_i, torch.arange(c0, c1).expand(*lead, c1 - c0)], -1)
        # rank candidates by (score desc, index asc); sentinels (index S) lose ties
        key = order_key(cs)
        o = torch.sort(ci, dim=-1, stable=True).indices                 # index asc
        o2 = torch.sort(-torch.gather(key, -1, o), dim=-1, stable=True).indices
        perm = torch.gather(o, -1, o2)[..., :k]
        run_s = torch.gather(cs, -1, perm)
        run_i = torch.gather(ci, -1, perm)
    return run_i


# ---------------------------------------------------------------------------
# a8/a9: scoring and gather attention
# ---------------------------------------------------------------------------
def sparse_score_scalar(q: torch.Tensor, k: torch.Tensor, scaling: float) -> torch.Tensor:
    """fp32 scores[b,h,t] = (q[b,h] . k[b,h//G,t]) * scaling.

    Restates src/attention_kernels.py:1077-1133 (`sparse_score_scalar`; bf16
    or float8_e4m3fn keys upcast to fp32).  Loop reference
    benchmarks/test_correctness.py:694-700.
    """
    B, Hq, _, D = q.shape
    Hk = k.shape[1]
    G = Hq // Hk
    qf = q.float().reshape(B, Hk, G, D)
    s = torch.matmul(qf, k.float().transpose(-1, -2)) * scaling
    return s.reshape(B, Hq, -1)


def group_scores(q: torch.Tensor, k: torch.Tensor, scaling: float) -> torch.Tensor:
    """Per-KV-head scores summed over the query group:
    s[b,h,t] = sum_{g<G} score(q[b,h*G+g], k[b,h,t]) (g ascending, fp32).

    BASELINE C5's group-summed selection score, built on the per-head score of
    src/attention_kernels.py:1077-1110 and the chunked scoring of
    benchmarks/sparse_attention.py:208-223.
    """
    B, Hq, _, D = q.shape
    Hk = k.shape[1]
    G = Hq // Hk
    s = sparse_score_scalar(q, k, scaling).reshape(B, Hk, G, -1)
    acc = s[:, :, 0]
    for g in range(1, G):
        acc = acc + s[:, :, g]
    return acc


def sparse_gather_attn(q, k, v, idx, scaling: float):
    """Exact fp32 attention over the gathered rows idx (per query head).

    Restates src/attention_kernels.py:987-1059 (`sparse_gather_attn`) and the
    torch semantics of benchmarks/sparse_attention.py:367-387 (`attend_topk`):
    index entries outside [0, S) are masked (sentinel rule, :376).  idx is
    [B,Hq,kb] or per-KV-head [B,Hk,kb] (shared by the query group).  Output
    dtype bf16 if v is float8_e4m3fn else v.dtype (:1044).
    """
    B, Hq, _, D = q.shape
    Hk, S = k.shape[1], k.shape[2]
    G = Hq // Hk
    if idx.shape[1] == Hk and Hk != Hq:
        idx = idx.repeat_interleave(G, dim=1)
    idx = idx.long()
    valid = (idx >= 0) & (idx < S)
    gi = idx.clamp(0, S - 1)
    kr = repeat_kv(k.float(), G)
    vr = repeat_kv(v.float(), G)
    kb = idx.shape[-1]
    ks = torch.gather(kr, 2, gi.unsqueeze(-1).expand(B, Hq, kb, D))
    vs = torch.gather(vr, 2, gi.unsqueeze(-1).expand(B, Hq, kb, D))
    sc = (q.float().reshape(B, Hq, 1, D) * ks).sum(-1) * scaling        # [B,Hq,kb]
    sc = torch.where(valid, sc, torch.full_like(sc, NEG_INF))
    p = torch.softmax(sc, dim=-1)
    o = (p.unsqueeze(-1) * vs).sum(2)
    od = torch.bfloat16 if v.dtype == torch.float8_e4m3fn else v.dtype
    return o.reshape(B, Hq, 1, D).to(od)


def score_keys_pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [..., D] (ints < 2^bits) -> uint8 [..., D*bits/8]: element c of a
    row at bits ((c % (8/bits)) * bits) of byte c // (8/bits), the layout of
    src/attention_kernels.py:1239-1245 (4-bit: lo | hi << 4; 2-bit: 4 per byte)."""
    per = 8 // bits
    c = codes.long().reshape(*codes.shape[:-1], -1, per)
    out = torch.zeros(c.shape[:-1], dtype=torch.int64)
    for i in range(per):
        out |= (c[..., i] & ((1 << bits) - 1)) << (i * bits)
    return out.to(torch.uint8)


def score_keys_unpack(packed: torch.Tensor, bits: int) -> torch.Tensor:
    """Inverse of score_keys_pack (the unpack loop of benchmarks/test_correctness.py:708-718)."""
    per = 8 // bits
    p = packed.long()
    parts = [(p >> (i * bits)) & ((1 << bits) - 1) for i in range(per)]
    return torch.stack(parts, dim=-1).reshape(*packed.shape[:-1], -1)


def quantize_and_pack_score_keys(k: torch.Tensor, score_bits: int, group_size: int):
    """Asym min/max quantization of the keys along head_dim in groups, packed to
    uint8; scale and min rounded to k's dtype after the codes are formed.
    Restates src/attention_kernels.py:1225-1249.  k [B,H,S,D] ->
    (packed [B,H,S,D*bits/8] uint8, scale [B,H,S,D/g], zero [B,H,S,D/g])."""
    B, H, S, D = k.shape
    ng = D // group_size
    kr = k.reshape(B, H, S, ng, group_size)
    codes, scale, xmin = asym_quant_codes(kr, 2 ** score_bits, dim=-1)
    packed = score_keys_pack(codes.reshape(B, H, S, D), score_bits)
    return packed, scale.reshape(B, H, S, ng).to(k.dtype), xmin.reshape(B, H, S, ng).to(k.dtype)


def score_keys_dequant(packed, scale, zero, score_bits: int, group_size: int) -> torch.Tensor:
    """k_hat = code * scale + zero in fp32 (src/attention_kernels.py:1170-1187)."""
    codes = score_keys_unpack(packed, score_bits).float()
    B, H, S, D = codes.shape
    s = scale.float().repeat_interleave(group_size, dim=-1)
    z = zero.float().repeat_interleave(group_size, dim=-1)
    return codes * s + z


def sparse_score_packed(q, packed, scale, zero, scaling: float, score_bits: int = 4, group_size: int = 32):
    """fp32 scores against dequantized packed keys (src/attention_kernels.py:1136-1222)."""
    return sparse_score_scalar(q, score_keys_dequant(packed, scale, zero, score_bits, group_size), scaling)


def budget(frac: float, S: int) -> int:
    """kb = max(1, round(frac*S)) with Python's round (src/attention_kernels.py:1261)."""
    return max(1, int(round(frac * S)))


def sparse_decode_scalar(q, k_score, k_val, v_val, frac: float, scaling: float):
    """Two-pass sparse decode, per query head: score -> top-kb -> gather attend.

    Restates src/attention_kernels.py:1252-1263 for score_bits 16/8 with the
    build's deterministic top-k (ties to the lowest index)."""
    s = sparse_score_scalar(q, k_score, scaling)
    kb = budget(frac, s.shape[-1])
    idx = topk_indices(s, kb)
    return sparse_gather_attn(q, k_val, v_val, idx, scaling)


def token_topk_decode(q, k, v, kb: int, scaling: float):
    """BASELINE C5 pipeline: group-summed fp32 scores per KV head, top-kb per
    (b, kv head), gathered attention for every query head of the group.
    Returns (out [B,Hq,1,D], idx [B,Hk,kb] ordered by score desc, index asc)."""
    s = group_scores(q, k, scaling)
    idx = topk_indices(s, kb)
    return sparse_gather_attn(q, k, v, idx, scaling), idx


# ---------------------------------------------------------------------------
# a7: Quest page selection
# ---------------------------------------------------------------------------
def quest_page_minmax(k: torch.Tensor, page: int):
    """Per-page elementwise min/max of the keys; the last partial page is padded
    with the last key.  Restates benchmarks/sparse_attention.py:336-344
    (`_quest_select`) / benchmarks/eval_ppl.py:56-63 (`_quest_mask`).
    k [B,H,S,D] -> (kmin, kmax) [B,H,ceil(S/page),D] in k's dtype (exact)."""
    B, H, S, D = k.shape
    np_ = (S + page - 1) // page
    pad = np_ * page - S
    kp = k
    if pad:
        kp = torch.cat([k, k[:, :, -1:, :].expand(B, H, pad, D)], dim=2)
    kp = kp.reshape(B, H, np_, page, D)
    return kp.amin(dim=3), kp.amax(dim=3)


def quest_page_scores(q: torch.Tensor, kmin: torch.Tensor, kmax: torch.Tensor,
                      scale: float = 1.0) -> torch.Tensor:
    """bound[b,h,p] = scale * sum_d max(q_d*kmin_d, q_d*kmax_d)  (fp32).

    Restates benchmarks/sparse_attention.py:342-345 (fp32 via `_scast`).  The
    products are exact in fp32 (bf16 x bf16); the sum over d is accumulated
    in ascending d so the GPU kernel can match it bit for bit.  At decode
    (query at position S-1) every page is causally valid (:347-349).
    q [B,Hq,1,D]; kmin/kmax [B,Hk,np,D] -> [B,Hq,np].
    Pinned by: the bound is >= max_t q.k_t over each page (Quest upper bound)
    and equals it for single-token pages (tests/test_oracle.py).
    """
    B, Hq, _, D = q.shape
    Hk = kmin.shape[1]
    G = Hq // Hk
    qf = q.float().reshape(B, Hk, G, 1, D)
    a = qf * kmin.float().unsqueeze(2)
    b = qf * kmax.float().unsqueeze(2)
    m = torch.maximum(a, b)                                             # [B,Hk,G,np,D]
    acc = m[..., 0]
    for d in range(1, D):
        acc = acc + m[..., d]
    out = acc.reshape(B, Hq, -1)
    return out * scale if scale != 1.0 else out


def quest_select(q, k, budget_tokens: int, page: int = 16, scale: float = 1.0):
    """Quest decode selection: page bounds -> top ceil(kb/page) pages (score
    desc, index asc) -> token ids clamped to S-1.

    Restates benchmarks/sparse_attention.py:328-364 (`_quest_select`) for one
    decode query.  Returns (page_ids [B,Hq,npick] int64, token_ids
    [B,Hq,npick*page] int64, bounds [B,Hq,np] fp32).
    """
    S = k.shape[2]
    kmin, kmax = quest_page_minmax(k, page)
    bound = quest_page_scores(q, kmin, kmax, scale)
    np_ = bound.shape[-1]
    npick = min(max(1, (budget_tokens + page - 1) // page), np_)
    pidx = topk_indices(bound, npick)
    tok = (pidx.unsqueeze(-1) * page + torch.arange(page)).reshape(*pidx.shape[:-1], -1)
    return pidx, tok.clamp(max=S - 1), bound


# ---------------------------------------------------------------------------
# Query chunks of Qc >= 1 rows: select_topk / _quest_select / attend_topk
# ---------------------------------------------------------------------------
def _fold_rows(q_blk: torch.Tensor) -> torch.Tensor:
    """[B,Hq,Qc,D] -> [B,Hq*Qc,1,D]: row (h, qc) becomes query head h*Qc + qc,
    which reads KV head h // G as every row of query head h does."""
    B, Hq, Qc, D = q_blk.shape
    return q_blk.reshape(B, Hq * Qc, 1, D)


def selection_mask(s: torch.Tensor, q_pos: torch.Tensor, unit: int = 1, local_w: int = 0) -> torch.Tensor:
    """Causal mask and forced recent window over candidate t (position t*unit)
    of query row qc: -inf where t*unit > pos[qc], then +inf where local_w > 0 and
    max(pos-local_w+1, 0)//unit <= t <= pos//unit.  s [..., Qc, n].
    Restates benchmarks/sparse_attention.py:248-256 with :298-300 (tokens,
    unit 1) and :346-355 (pages, unit = page size)."""
    n = s.shape[-1]
    pos = q_pos.reshape(-1).long()
    t = torch.arange(n)
    valid = (t[None, :] * unit) <= pos[:, None]                           # [Qc, n]
    out = torch.where(valid, s.float(), torch.full_like(s.float(), NEG_INF))
    if local_w > 0:
        lo = (pos - local_w + 1).clamp(min=0) // unit
        hi = pos // unit
        rec = (t[None, :] >= lo[:, None]) & (t[None, :] <= hi[:, None])
        out = torch.where(rec, torch.full_like(out, float("inf")), out)
    return out


def select_topk_from_scores(scores: torch.Tensor, q_pos: torch.Tensor, S: int, kb: int, k_chunk: int,
                            local_w: int = 0) -> torch.Tensor:
    """The streaming selection of benchmarks/sparse_attention.py:286-309 over
    precomputed fp32 scores [..., Qc, max_key] (max_key = max(q_pos) + 1):
    a running list of kb (score, index) pairs starting as (-inf, S) sentinels
    (:291-292) is merged with each k_chunk-key tile (causal mask and recent
    window applied, :297-300) and cut back to kb under the total order (score
    descending, index ascending).  Keys past a row's position never enter the
    list (they rank below the sentinels), so every slot a row cannot fill
    holds the sentinel S - the purpose the reference states at :288-293.
    Returns int64 [..., Qc, kb] ordered by that order."""
    max_key = scores.shape[-1]
    lead = scores.shape[:-1]
    run_s = torch.full((*lead, kb), NEG_INF)
    run_i = torch.full((*lead, kb), S, dtype=torch.int64)
    pos = q_pos.reshape(-1).long()
    for c0 in range(0, max_key, k_chunk):
        c1 = min(c0 + k_chunk, max_key)
        sc = selection_mask(scores[..., c0:c1], pos - c0, 1, 0)           # causal on this tile
        if local_w > 0:
            kp = torch.arange(c0, c1)
            rec = (kp[None, :] > (pos[:, None] - local_w)) & (kp[None, :] <= pos[:, None])
            sc = torch.where(rec, torch.full_like(sc, float("inf")), sc)
        kp = torch.arange(c0, c1).expand(*lead, c1 - c0)
        causal = kp <= pos.reshape(*([1] * (len(lead) - 1)), -1, 1)
        ci_tile = torch.where(causal, kp, S + 1 + kp)                      # masked keys lose to sentinels
        cs = torch.cat([run_s, sc], -1)
        ci = torch.cat([run_i, ci_tile], -1)
        key = order_key(cs)
        o = torch.sort(ci, dim=-1, stable=True).indices                    # index ascending
        o2 = torch.sort(-torch.gather(key, -1, o), dim=-1, stable=True).indices
        perm = torch.gather(o, -1, o2)[..., :kb]
        run_s = torch.gather(cs, -1, perm)
        run_i = torch.gather(ci, -1, perm)
    return torch.where(run_i > S, torch.full_like(run_i, S), run_i)


def select_recent(B: int, Hq: int, q_pos: torch.Tensor, kb: int) -> torch.Tensor:
    """select_topk(selector="recent") of benchmarks/sparse_attention.py:261-265:
    the kb most recent causal positions of each query row, pos, pos-1, ...,
    clamped at 0 (so a row at position p < kb - 1 repeats key 0), for every
    (b, h).  Returns int64 [B,Hq,Qc,kb].
    Pinned by: the set of the first min(kb, p+1) entries equals the last
    min(kb, p+1) positions of range(p+1), in descending order, and every
    later entry is 0 (tests/test_oracle.py)."""
    pos = q_pos.reshape(-1).long()
    idx = (pos[:, None] - torch.arange(kb)[None, :]).clamp(min=0)
    return idx[None, None].expand(B, Hq, pos.numel(), kb).contiguous()


def select_topk_exact(q_blk, sel_keys, q_pos, S: int, kb: int, k_chunk: int, scaling: float,
                      local_w: int = 0) -> torch.Tensor:
    """select_topk(selector="exact"/"approx") of benchmarks/sparse_attention.py:226-325:
    fp32 scores (q . k) * scaling of every key before max(q_pos) + 1 (:208-210,
    :294-296), then the streaming selection above.  q_blk [B,Hq,Qc,D];
    sel_keys [B,Hq,S,D] (GQA-expanded, as the reference passes them) or
    [B,Hk,S,D].  Returns int64 [B,Hq,Qc,kb]."""
    B, Hq, Qc, D = q_blk.shape
    max_key = int(q_pos.max()) + 1
    s = sparse_score_scalar(_fold_rows(q_blk), sel_keys[:, :, :max_key], scaling)   # [B,Hq*Qc,max_key]
    return select_topk_from_scores(s.reshape(B, Hq, Qc, max_key), q_pos, S, kb, k_chunk, local_w)


def quest_select_rows(q_blk, k_r, q_pos, S: int, kb: int, page: int, scaling: float,
                      local_w: int = 0) -> torch.Tensor:
    """_quest_select of benchmarks/sparse_attention.py:328-364 for Qc >= 1 query
    rows: page metadata, fp32 bounds * scaling, causal page validity and
    forced recent pages per row, the top ceil(kb/page) pages under the total
    order, expanded to token ids clamped to S - 1.  Returns int64
    [B,Hq,Qc,npick*page] (pages in bound-descending order)."""
    B, Hq, Qc, D = q_blk.shape
    kmin, kmax = quest_page_minmax(k_r[:, :, :S], page)
    bound = quest_page_scores(_fold_rows(q_blk), kmin, kmax, scaling).reshape(B, Hq, Qc, -1)
    bound = selection_mask(bound, q_pos, page, local_w)
    np_ = bound.shape[-1]
    npick = min(max(1, (kb + page - 1) // page), np_)
    pidx = topk_indices(bound, npick)
    tok = (pidx.unsqueeze(-1) * page + torch.arange(page)).reshape(B, Hq, Qc, npick * page)
    return tok.clamp(max=S - 1)


def attend_topk(q_blk, k_r, v, idx, q_pos, scaling: float) -> torch.Tensor:
    """Exact attention of each query row over its selected keys.

    Restates benchmarks/sparse_attention.py:367-387: an entry takes part iff
    it is at or before the row's position and below S (:376; negative entries
    are masked too, the sentinel rule of sparse_gather_attn); fp32 scores and
    softmax; the weights are cast to v's dtype and the weighted sum is taken
    in v's dtype, as the reference does (:386-387).  q_blk [B,Hq,Qc,D];
    k_r, v [B,Hq,S,D] or [B,Hk,S,D]; idx [B,Hq,Qc,ksel]."""
    B, Hq, Qc, D = q_blk.shape
    Hs, S = k_r.shape[1], k_r.shape[2]
    G = Hq // Hs
    ksel = idx.shape[-1]
    pos = q_pos.reshape(-1).long()
    idx = idx.long()
    valid = (idx >= 0) & (idx < S) & (idx <= pos[None, None, :, None])
    gi = idx.clamp(0, S - 1)
    kr = repeat_kv(k_r, G).float()
    vr = repeat_kv(v, G)
    ks = torch.gather(kr.unsqueeze(2).expand(B, Hq, Qc, S, D), 3, gi.unsqueeze(-1).expand(B, Hq, Qc, ksel, D))
    vs = torch.gather(vr.unsqueeze(2).expand(B, Hq, Qc, S, D), 3, gi.unsqueeze(-1).expand(B, Hq, Qc, ksel, D))
    sc = (q_blk.float().unsqueeze(3) * ks).sum(-1) * scaling
    sc = torch.where(valid, sc, torch.full_like(sc, NEG_INF))
    w = torch.softmax(sc, dim=-1).to(v.dtype)
    return (w.unsqueeze(-1) * vs).sum(3)


# ---------------------------------------------------------------------------
# f2/f4 study-harness microkernels
# ---------------------------------------------------------------------------
def gather_reduce(v: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """out[h, d] = sum_k v[h, idx[h, k], d] in fp32.

    Restates `_gather_reduce_kernel` / `gather_reduce` of
    benchmarks/bench_access_pattern.py:25-52 (v [H,S,D] fp16, idx [H,K]).
    Pinned by: the full contiguous list equals v.sum(1); a permutation of
    the list gives the same sums; one-hot rows (tests/test_oracle.py)."""
    H, S, D = v.shape
    gi = idx.long().unsqueeze(-1).expand(H, idx.shape[1], D)
    return torch.gather(v.float(), 1, gi).sum(1)


def packed_stage(q, packed, scale, zero, bits: int, stage: int) -> torch.Tensor:
    """The four cumulative stages of benchmarks/bench_unpack_ablation.py:19-53
    (`_packed_stage_kernel`) per (b, query head) and key row, in fp32:
    0 sum over columns of each column's packed byte, 1 sum of the codes,
    2 sum of code*scale+zero, 3 sum of (code*scale+zero)*q.
    q [B,Hq,1,D]; packed [B,Hk,S,D*bits/8]; scale/zero [B,Hk,S,D/32].
    Returns [B,Hq,S].  Pinned by: stage 0 = (8/bits) * sum of the bytes,
    stage 1 = sum of score_keys_unpack, stage 2 = sum of score_keys_dequant,
    stage 3 = sparse_score_packed at scaling 1 (tests/test_oracle.py)."""
    B, Hq, _, D = q.shape
    Hk = packed.shape[1]
    G = Hq // Hk
    epb = 8 // bits
    cols = torch.arange(D)
    p = packed.long()[..., cols // epb]                                   # [B,Hk,S,D]: the byte of each column
    if stage == 0:
        vals = p.float()
    else:
        vals = ((p >> ((cols % epb) * bits)) & ((1 << bits) - 1)).float()
        if stage >= 2:
            vals = vals * scale.float().repeat_interleave(32, -1) + zero.float().repeat_interleave(32, -1)
    if stage == 3:
        vr = repeat_kv(vals, G)                                            # [B,Hq,S,D]
        return (vr * q.float().reshape(B, Hq, 1, D)).sum(-1)
    return repeat_kv(vals.sum(-1, keepdim=True), G).squeeze(-1)
