"""Sparse-vs-dense decode crossover on MI355X.

Port of benchmarks/bench_sparse_crossover.py:62-224: for every cell of a
context-length x budget grid at the headline shape B=32, H_q=64, H_k=8, D=128,
time (ms per decode step, graph replays) dense bf16 and fp8 decode, KIVI-4 and
KIVI-2 decode (residual window 128), and the two-pass sparse decode with bf16,
fp8, packed int4 and packed int2 score keys; for int2 also its stages (score
pass, top-k, gather).  Writes JSON rows {S, frac, lat_ms, stages, winner} and
prints the int2 / KIVI-4 latency ratio grid of the reference's heatmap.

    python -m bytes_amd.harness.crossover [--quick] [--output-json PATH]

--c5 runs BASELINE C5's own sweep instead: at B=8, H_q=24, H_k=8, D=128,
L=131072, the group-shared token top-k decode (score pass + top-k + gather,
with bf16, fp8 and packed int2 score keys) at budgets of 1 / 2 / 5 / 10 / 25 /
50 % of L against dense bf16 and fp8 decode of the same cache, and names the
budget where each sparse variant stops beating dense bf16.
"""
from __future__ import annotations

import argparse
import json
import math
import os

import torch

from .timing import HBM_PEAK_GBS, clones, copies_for, graph_ms

S_GRID = [4096, 8192, 16384, 32768, 65536]
FRAC_GRID = [0.01, 0.02, 0.05, 0.10, 0.25]


def _time(fn, inp, nbytes, runs):
    inps = clones(inp, copies_for(nbytes))
    ms = graph_ms(fn, inps, warmup=5, runs=runs)
    del inps
    return ms


def run_cell(B, Hq, Hk, D, S, frac, seed, runs, dev):
    from .. import attention_kernels as AK
    from .. import kivi as KV
    from ..sparse import budget, sparse_gather_attn, topk_indices

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn(B, Hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(B, Hk, S, D, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g, device=dev, dtype=torch.bfloat16)
    scaling = 1.0 / math.sqrt(D)
    kb = budget(frac, S)
    kvb = B * Hk * S * D * 2
    lat, stages = {}, {}

    lat["bf16"] = _time(lambda x: AK.decode_attn_bf16(x["q"], x["k"], x["v"]), {"q": q, "k": k, "v": v}, 2 * kvb,
                        runs)
    k8, v8 = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
    lat["fp8"] = _time(lambda x: AK.decode_attn_fp8(x["q"], x["k"], x["v"]), {"q": q, "k": k8, "v": v8}, kvb, runs)

    R = 128
    Sq = S - R
    for bits in (4, 2):
        kq, ks, km = KV.quantize_and_pack_along_last_dim(k[:, :, :Sq].transpose(2, 3).contiguous().half(), 32, bits)
        vq, vs, vm = KV.quantize_and_pack_along_last_dim(v[:, :, :Sq].contiguous().half(), 32, bits)
        x = {"Q": q, "Kq": kq, "K_scale": ks, "K_mn": km, "K_res": k[:, :, Sq:].contiguous(), "Vq": vq,
             "V_scale": vs, "V_mn": vm, "V_res": v[:, :, Sq:].contiguous()}
        nb = sum(t.numel() * t.element_size() for t in x.values())
        lat[f"kivi{bits}"] = _time(lambda x, b=bits: KV.kivi_decode_attn(
            x["Q"], x["Kq"], x["K_scale"], x["K_mn"], x["K_res"], x["Vq"], x["V_scale"], x["V_mn"], x["V_res"],
            b, 32), x, nb, runs)
        del x, kq, ks, km, vq, vs, vm

    gather_b = 2 * B * Hq * kb * D * 2
    sx = {"q": q, "k": k, "v": v}
    lat["sparse_bf16"] = _time(lambda x: AK.sparse_decode_scalar(x["q"], x["k"], None, None, x["k"], x["v"], frac,
                                                                 scaling, score_bits=16), sx, kvb + gather_b, runs)
    sx8 = {"q": q, "k8": k8, "k": k, "v": v}
    lat["sparse_fp8"] = _time(lambda x: AK.sparse_decode_scalar(x["q"], x["k8"], None, None, x["k"], x["v"], frac,
                                                                scaling, score_bits=8), sx8, kvb // 2 + gather_b, runs)
    del k8, v8, sx8
    for bits in (4, 2):
        p, sc, zr = AK.quantize_and_pack_score_keys(k, bits, 32)
        xp = {"q": q, "p": p, "s": sc, "z": zr, "k": k, "v": v}
        nb = p.numel() + 2 * sc.numel() * 2
        lat[f"sparse_int{bits}"] = _time(lambda x, b=bits: AK.sparse_decode_scalar(
            x["q"], x["p"], x["s"], x["z"], x["k"], x["v"], frac, scaling, score_bits=b, group_size=32), xp,
            nb + gather_b, runs)
        if bits == 2:
            stages["score_pass_ms"] = _time(lambda x: AK.sparse_score_packed(x["q"], x["p"], x["s"], x["z"], scaling,
                                                                             score_bits=2), xp, nb, runs)
            scores = AK.sparse_score_packed(q, p, sc, zr, scaling, score_bits=2)
            stages["topk_only_ms"] = _time(lambda x: topk_indices(x["s"], kb, sorted=False), {"s": scores},
                                           scores.numel() * 4, runs)
            idx = topk_indices(scores, kb, sorted=False)
            stages["gather_only_ms"] = _time(lambda x: sparse_gather_attn(x["q"], x["k"], x["v"], x["i"], scaling),
                                             {"q": q, "k": k, "v": v, "i": idx}, gather_b, runs)
            del scores, idx
        del xp, p, sc, zr
    del q, k, v, sx
    torch.cuda.empty_cache()
    return {"S": S, "frac": frac, "kb": kb, "lat_ms": lat, "stages": stages,
            "winner": min(lat, key=lat.get),
            "dense_bf16_hbm_frac": (2 * kvb / (lat["bf16"] * 1e-3)) / (HBM_PEAK_GBS * 1e9)}


C5_FRACS = [0.01, 0.02, 0.05, 0.10, 0.25, 0.50]


def c5_sweep(runs, seed, dev, B=8, Hq=24, Hk=8, D=128, L=131072):
    from .. import attention_kernels as AK
    from ..sparse import quantize_and_pack_score_keys, token_topk_decode
    from ..workloads import c5_topk
    x = c5_topk(seed=seed, device=dev, B=B, Hq=Hq, Hk=Hk, D=D, L=L)
    q, k, v, sc = x["q"], x["k"], x["v"], x["scale"]
    kvb = B * Hk * L * D * 2
    rows = {"dense_bf16": _time(lambda z: AK.decode_attn_bf16(z["q"], z["k"], z["v"], sc), {"q": q, "k": k, "v": v},
                                2 * kvb, runs)}
    k8, v8 = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
    rows["dense_fp8"] = _time(lambda z: AK.decode_attn_fp8(z["q"], z["k"], z["v"], sc), {"q": q, "k": k8, "v": v8},
                              kvb, runs)
    del v8
    p2, s2, z2 = quantize_and_pack_score_keys(k, 2, 32)
    keys = {"bf16": {}, "fp8": {"ks": k8}, "int2": {"ks": p2, "ksc": s2, "kzr": z2, "bits": 2}}
    sparse = {}
    for name, extra in keys.items():
        sparse[name] = []
        for frac in C5_FRACS:
            kb = max(1, int(round(frac * L)))
            inp = {"q": q, "k": k, "v": v, **{n: t for n, t in extra.items() if n != "bits"}}
            fn = (lambda z, kb=kb, bits=extra.get("bits"):
                  token_topk_decode(z["q"], z["k"], z["v"], kb, sc, k_score=z.get("ks"), score_scale=z.get("ksc"),
                                    score_zero=z.get("kzr"), score_bits=bits))
            ms = graph_ms(fn, [inp], warmup=3, runs=runs)
            sparse[name].append({"frac": frac, "kb": kb, "ms": ms, "vs_dense_bf16": ms / rows["dense_bf16"]})
            print(f"C5 {name:5s} score keys, k = {100 * frac:4.1f}% of L ({kb:6d}): {ms * 1e3:8.1f} us "
                  f"({ms / rows['dense_bf16']:.3f} x dense bf16)", flush=True)
    cross = {}
    for name, pts in sparse.items():
        beaten = [p for p in pts if p["ms"] >= rows["dense_bf16"]]
        cross[name] = beaten[0]["frac"] if beaten else None
    return {"shape": {"B": B, "H_q": Hq, "H_k": Hk, "D": D, "L": L}, "dense_ms": rows, "sparse": sparse,
            "first_budget_not_faster_than_dense_bf16": cross}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--quick", action="store_true", help="3 x 3 grid (S 4K/16K/64K, frac 1%%/5%%/25%%)")
    ap.add_argument("--c5", action="store_true", help="BASELINE C5's budget sweep against dense at its own shape")
    ap.add_argument("--B", type=int, default=32)
    ap.add_argument("--Hq", type=int, default=64)
    ap.add_argument("--Hk", type=int, default=8)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--output-json", default="harness_out/sparse_crossover.json")
    a = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    if a.c5:
        res = c5_sweep(a.runs, a.seed, dev)
        print("dense: " + " ".join(f"{n} {ms * 1e3:.1f} us" for n, ms in res["dense_ms"].items()))
        print("first budget (k/L) not faster than dense bf16: " + ", ".join(
            f"{n} keys {('%.0f%%' % (100 * f)) if f is not None else 'none (sparse faster at every budget)'}"
            for n, f in res["first_budget_not_faster_than_dense_bf16"].items()))
        os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
        with open(a.output_json, "w") as f:
            json.dump({"schema": "c5_crossover_v1", "gpu": torch.cuda.get_device_name(0), "seed": a.seed, **res}, f,
                      indent=2)
        print(f"saved {a.output_json}")
        return
    s_grid = [4096, 16384, 65536] if a.quick else S_GRID
    f_grid = [0.01, 0.05, 0.25] if a.quick else FRAC_GRID
    rows = []
    print(f"crossover sweep B={a.B} H_q={a.Hq} H_k={a.Hk} D=128 on {torch.cuda.get_device_name(0)}", flush=True)
    for S in s_grid:
        for frac in f_grid:
            r = run_cell(a.B, a.Hq, a.Hk, 128, S, frac, a.seed, a.runs, dev)
            rows.append(r)
            lat = " ".join(f"{k}={v:.3f}" for k, v in r["lat_ms"].items())
            print(f"S={S} frac={frac}: {lat} | int2 stages " +
                  " ".join(f"{k}={v:.3f}" for k, v in r["stages"].items()) + f" | winner {r['winner']}", flush=True)
    print("\nsparse_int2 / kivi4 latency (rows: frac, columns: S)")
    print("frac   " + " ".join(f"{S:>8}" for S in s_grid))
    for frac in f_grid:
        cells = [r for r in rows if r["frac"] == frac]
        print(f"{frac:<6} " + " ".join(f"{c['lat_ms']['sparse_int2'] / c['lat_ms']['kivi4']:>8.2f}" for c in cells))
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump({"schema": "sparse_crossover_v1", "gpu": torch.cuda.get_device_name(0), "B": a.B, "H_q": a.Hq,
                   "H_k": a.Hk, "D": 128, "seed": a.seed, "rows": rows}, f, indent=2)
    print(f"saved {a.output_json}")


if __name__ == "__main__":
    main()
