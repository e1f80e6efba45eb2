"""Seeded synthetic inputs for the BASELINE.json decode-attention configs.

All tensors are drawn on the CPU from a torch.Generator seeded per config
(default seed 0), then moved to `device`.  Shapes and distributions follow
BASELINE.json `configs`; choices the config leaves open are fixed here and
recorded in the returned dict under "meta".
"""
from __future__ import annotations

import math
from typing import Dict

import torch

# name -> (B, Hq, Hk, D, L)
SHAPES = {
    "c1_dense": (1, 14, 2, 64, 8192),
    "dense_16k": (4, 28, 4, 128, 16384),     # the L>=16K dense bandwidth point
    "c2_kivi": (4, 28, 4, 128, 16384),
    "c3_pq": (1, 28, 4, 128, 32768),
    "c4_quest": (1, 28, 4, 128, 32768),
    "c5_topk": (8, 24, 8, 128, 131072),
}


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn_bf16(shape, g: torch.Generator) -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(torch.bfloat16)


def dense(B: int, Hq: int, Hk: int, D: int, L: int, seed: int = 0, device="cpu") -> Dict:
    """q, K, V i.i.d. N(0,1) as bf16 (BASELINE C1 and the dense L>=16K point)."""
    g = _gen(seed)
    q = randn_bf16((B, Hq, 1, D), g)
    k = randn_bf16((B, Hk, L, D), g)
    v = randn_bf16((B, Hk, L, D), g)
    return {"q": q.to(device), "k": k.to(device), "v": v.to(device),
            "scale": 1.0 / math.sqrt(D),
            "meta": {"seed": seed, "shape": (B, Hq, Hk, D, L)}}


def c1_dense(seed: int = 0, device="cpu") -> Dict:
    return dense(*SHAPES["c1_dense"], seed=seed, device=device)


def dense_16k(seed: int = 0, device="cpu", L: int = 16384) -> Dict:
    B, Hq, Hk, D, _ = SHAPES["dense_16k"]
    return dense(B, Hq, Hk, D, L, seed=seed, device=device)


def kivi_raw(B: int = 4, Hq: int = 28, Hk: int = 4, D: int = 128, L: int = 16384, R: int = 128,
             seed: int = 0, device="cpu", n_outlier: int = 4, outlier_scale: float = 8.0) -> Dict:
    """BASELINE C2 raw tensors: bf16 K, V ~ N(0,1); `n_outlier` key channels chosen
    by a seeded randperm(D) (the same for every b, h) are multiplied by
    `outlier_scale`; q ~ N(0,1) bf16.  The last R tokens form the bf16 residual
    window; the first L - R are to be packed (keys transposed per channel)."""
    g = _gen(seed)
    q = randn_bf16((B, Hq, 1, D), g)
    k = torch.randn(B, Hk, L, D, generator=g)
    v = torch.randn(B, Hk, L, D, generator=g)
    ch = torch.randperm(D, generator=g)[:n_outlier]
    k[..., ch] *= outlier_scale
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    Sq = L - R
    return {"q": q.to(device), "k": k.to(device), "v": v.to(device), "Sq": Sq, "R": R,
            "scale": 1.0 / math.sqrt(D),
            "meta": {"seed": seed, "outlier_channels": ch.tolist(), "shape": (B, Hq, Hk, D, L, R)}}


def kivi_pack_inputs(raw: Dict, pack_fn, bits: int, group_size: int = 32) -> Dict:
    """Pack a kivi_raw() cache with `pack_fn(x, group_size, bits)` the way the
    reference harness does (benchmarks/kivi_latency.py:121-128): keys transposed
    to [B,Hk,D,Sq] and cast to fp16, values cast to fp16."""
    Sq = raw["Sq"]
    k, v = raw["k"], raw["v"]
    kq, ks, km = pack_fn(k[:, :, :Sq].transpose(2, 3).contiguous().to(torch.float16), group_size, bits)
    vq, vs, vm = pack_fn(v[:, :, :Sq].contiguous().to(torch.float16), group_size, bits)
    return {"Q": raw["q"], "Kq": kq, "K_scale": ks, "K_mn": km, "K_residual": k[:, :, Sq:],
            "Vq": vq, "V_scale": vs, "V_mn": vm, "V_residual": v[:, :, Sq:], "bits": bits,
            "group_size": group_size}


def c5_topk(seed: int = 0, device="cpu", B: int = 8, Hq: int = 24, Hk: int = 8, D: int = 128,
            L: int = 131072) -> Dict:
    """BASELINE C5 inputs: q, K, V ~ N(0,1) bf16.  Drawn on `device` from a
    generator seeded there (the full-size cache is 2 GiB per tensor, so it is
    generated where it is used)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g, device=device, dtype=torch.bfloat16)
    k = torch.randn(B, Hk, L, D, generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn(B, Hk, L, D, generator=g, device=device, dtype=torch.bfloat16)
    return {"q": q, "k": k, "v": v, "scale": 1.0 / math.sqrt(D),
            "meta": {"seed": seed, "shape": (B, Hq, Hk, D, L), "generator": str(torch.device(device))}}


def c4_quest(seed: int = 0, device="cpu", B: int = 1, Hq: int = 28, Hk: int = 4, D: int = 128, L: int = 32768,
             n_needle: int = 64, needle_scale: float = 4.0, noise: float = 0.1) -> Dict:
    """BASELINE C4 inputs: q, K, V ~ N(0,1) bf16, plus `n_needle` needle tokens
    per (b, KV head) at seeded random positions whose keys are set to
    needle_scale * q_dir + noise * N(0,1), q_dir being the unit vector of the sum
    of the group's query vectors (so every head of the group sees them)."""
    g = _gen(seed)
    q = torch.randn(B, Hq, 1, D, generator=g)
    k = torch.randn(B, Hk, L, D, generator=g)
    v = torch.randn(B, Hk, L, D, generator=g)
    G = Hq // Hk
    qdir = q.reshape(B, Hk, G, D).sum(2)
    qdir = qdir / qdir.norm(dim=-1, keepdim=True)
    pos = torch.stack([torch.randperm(L, generator=g)[:n_needle] for _ in range(B * Hk)]).reshape(B, Hk, n_needle)
    for b in range(B):
        for h in range(Hk):
            k[b, h, pos[b, h]] = needle_scale * qdir[b, h] + noise * torch.randn(n_needle, D, generator=g)
    return {"q": q.to(torch.bfloat16).to(device), "k": k.to(torch.bfloat16).to(device),
            "v": v.to(torch.bfloat16).to(device), "scale": 1.0 / math.sqrt(D), "needles": pos,
            "meta": {"seed": seed, "shape": (B, Hq, Hk, D, L), "n_needle": n_needle}}


def c3_pq(seed: int = 0, device="cuda", B: int = 1, Hq: int = 28, Hk: int = 4, D: int = 128, L: int = 32768,
          K: int = 256, n_train: int = 16384, iters: int = 10) -> Dict:
    """BASELINE C3 inputs: q, K, V ~ N(0,1) bf16; per KV head, 16 subspaces of 8
    dims with a K-entry fp16 codebook each for keys and for values, fitted by
    k-means (`iters` iterations, seeded) on `n_train` fresh N(0,1) bf16 training
    vectors per head; uint8 codes of K and V; the fp32 LUT of q against the key
    codebooks with 1/sqrt(D) folded in.  Codebook fitting and encoding run on
    the GPU kernels of bytes_amd.pq (setup, not part of a decode step)."""
    from . import pq as PQ
    g = _gen(seed)
    q = randn_bf16((B, Hq, 1, D), g).to(device)
    k = randn_bf16((B, Hk, L, D), g).to(device)
    v = randn_bf16((B, Hk, L, D), g).to(device)
    tk = randn_bf16((Hk, n_train, D), g).to(device)
    tv = randn_bf16((Hk, n_train, D), g).to(device)
    kcb = PQ.kmeans(tk, K, iters, generator=g).to(torch.float16)          # [Hk, M, K, 8]
    vcb = PQ.kmeans(tv, K, iters, generator=g).to(torch.float16)
    k_idx = PQ.pq_encode(k.transpose(0, 1).contiguous(), kcb).transpose(0, 1).contiguous()   # [B,Hk,L,M]
    v_idx = PQ.pq_encode(v.transpose(0, 1).contiguous(), vcb).transpose(0, 1).contiguous()
    scale = 1.0 / math.sqrt(D)
    lut = PQ.pq_build_lut(q, kcb, scale)
    return {"q": q, "k": k, "v": v, "k_cb": kcb, "v_cb": vcb, "k_idx": k_idx, "v_idx": v_idx, "lut": lut,
            "scale": scale, "meta": {"seed": seed, "shape": (B, Hq, Hk, D, L), "K": K, "n_train": n_train,
                                     "kmeans_iters": iters}}
