"""Achieved bandwidth of gathered attention by token pattern on MI355X.

Port of benchmarks/bench_access_pattern.py:103-159, measured on this build's
gather-attention kernel itself rather than a stand-alone gather: for budgets
of 1 / 2 / 5 / 10 / 25 / 100 % of S, one selection of kb tokens per (b, KV
head) is attended by every query head of its group, with the selection drawn
as
  contiguous     tokens 0 .. kb-1
  random         kb distinct tokens in random order
  sorted_random  the same set in ascending order
  paged          random 16-token pages (vLLM-style)
The bytes read (2 * B * H_k * kb * D * 2: the selected K and V rows) are the
same for every pattern, so GB/s differences come from the pattern alone; the
peak is MI355X's 8 TB/s (the reference hard-codes 360 GB/s, :22).

It also runs the reference's own probe, the gather-reduce microkernel
(:25-52, csrc/harness.hip): per (b, KV head) the fp32 sum of the listed fp16
value rows, over the same budgets and patterns (reads B * H_k * kb * D * 2
bytes), and the granularity sweep of :136-156: a full gather (every row once,
so no cache reuse) in random against contiguous order at row widths of
16 .. 512 bytes (D = 8 .. 256 fp16), which shows where a scatter penalty would
begin.

    python -m bytes_amd.harness.access_pattern [--B 32 --Hk 8 --S 16384]
"""
from __future__ import annotations

import argparse
import json
import os

import torch

from .timing import HBM_PEAK_GBS, clones, copies_for, graph_ms


def make_idx(pattern, rows, S, kb, page, g, dev):
    if pattern == "contiguous":
        return torch.arange(kb, device=dev, dtype=torch.int32).expand(rows, kb).contiguous()
    if pattern in ("random", "sorted_random"):
        idx = torch.stack([torch.randperm(S, generator=g, device=dev)[:kb] for _ in range(rows)]).to(torch.int32)
        return torch.sort(idx, dim=-1).values if pattern == "sorted_random" else idx
    if pattern == "paged":
        n = (kb + page - 1) // page
        starts = torch.randint(0, S // page, (rows, n), generator=g, device=dev) * page
        offs = (starts[..., None] + torch.arange(page, device=dev)).reshape(rows, -1)
        return offs[:, :kb].to(torch.int32).contiguous()
    raise ValueError(pattern)


def main(argv=None):
    from ..sparse import sparse_gather_attn
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--B", type=int, default=32)
    ap.add_argument("--Hq", type=int, default=64)
    ap.add_argument("--Hk", type=int, default=8)
    ap.add_argument("--S", type=int, default=16384)
    ap.add_argument("--D", type=int, default=128)
    ap.add_argument("--page", type=int, default=16)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--output-json", default="harness_out/access_pattern.json")
    a = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(a.seed)
    q = torch.randn(a.B, a.Hq, 1, a.D, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(a.B, a.Hk, a.S, a.D, generator=g, device=dev, dtype=torch.bfloat16)
    v = torch.randn(a.B, a.Hk, a.S, a.D, generator=g, device=dev, dtype=torch.bfloat16)
    scaling = a.D ** -0.5
    rows_out = []
    budgets = [("1%", max(a.page, int(0.01 * a.S))), ("2%", int(0.02 * a.S)), ("5%", int(0.05 * a.S)),
               ("10%", int(0.10 * a.S)), ("25%", int(0.25 * a.S)), ("full", a.S)]
    print(f"gather attention B={a.B} H_q={a.Hq} H_k={a.Hk} S={a.S} D={a.D} page={a.page}; peak {HBM_PEAK_GBS} GB/s")
    print(f"{'budget':>6} {'kb':>6} {'pattern':>13} {'us':>9} {'GB/s':>8} {'%peak':>7}")
    for tag, kb in budgets:
        pats = ["contiguous", "random", "sorted_random", "paged"] if kb < a.S else ["contiguous", "random",
                                                                                   "sorted_random"]
        for pat in pats:
            idx = make_idx(pat, a.B * a.Hk, a.S, kb, a.page, g, dev).reshape(a.B, a.Hk, kb)
            nbytes = 2 * a.B * a.Hk * kb * a.D * 2
            x = {"q": q, "k": k, "v": v, "i": idx}
            # rotate whole K/V copies only when the selected rows could stay cached
            inps = clones(x, copies_for(nbytes)) if nbytes < (512 << 20) else [x]
            ms = graph_ms(lambda z: sparse_gather_attn(z["q"], z["k"], z["v"], z["i"], scaling), inps, 5, a.runs)
            del inps
            gbs = nbytes / (ms * 1e-3) / 1e9
            rows_out.append({"budget": tag, "kb": kb, "pattern": pat, "us": ms * 1e3, "gbs": gbs,
                             "pct_peak": 100 * gbs / HBM_PEAK_GBS})
            print(f"{tag:>6} {kb:>6} {pat:>13} {ms * 1e3:>9.1f} {gbs:>8.0f} {100 * gbs / HBM_PEAK_GBS:>6.1f}%",
                  flush=True)
    del q, k
    # ---- the reference's gather-reduce probe over the same budgets and patterns ----
    from .kernels import gather_reduce
    H = a.B * a.Hk
    vh = v.reshape(H, a.S, a.D).to(torch.float16)
    del v
    torch.cuda.empty_cache()
    probe = []
    print(f"\ngather-reduce probe H={H} S={a.S} D={a.D} (fp16 rows)")
    print(f"{'budget':>6} {'kb':>6} {'pattern':>13} {'us':>9} {'GB/s':>8} {'%peak':>7}")
    for tag, kb in budgets:
        pats = ["contiguous", "random", "sorted_random", "paged"] if kb < a.S else ["contiguous", "random",
                                                                                   "sorted_random"]
        for pat in pats:
            idx = make_idx(pat, H, a.S, kb, a.page, g, dev)
            nbytes = H * kb * a.D * 2
            x = {"v": vh, "i": idx}
            inps = clones(x, copies_for(nbytes)) if nbytes < (512 << 20) else [x]
            ms = graph_ms(lambda z: gather_reduce(z["v"], z["i"]), inps, 5, a.runs)
            del inps
            gbs = nbytes / (ms * 1e-3) / 1e9
            probe.append({"budget": tag, "kb": kb, "pattern": pat, "us": ms * 1e3, "gbs": gbs,
                          "pct_peak": 100 * gbs / HBM_PEAK_GBS})
            print(f"{tag:>6} {kb:>6} {pat:>13} {ms * 1e3:>9.1f} {gbs:>8.0f} {100 * gbs / HBM_PEAK_GBS:>6.1f}%",
                  flush=True)
    del vh
    torch.cuda.empty_cache()
    # ---- granularity sweep: full gather, random vs contiguous, by row width ----
    print(f"\n{'D':>5} {'rowB':>6} {'contig%pk':>10} {'rand%pk':>9} {'rand/contig':>12}")
    gsweep = []
    for D in (8, 16, 32, 64, 128, 256):
        vd = torch.randn(H, a.S, D, generator=g, device=dev, dtype=torch.float16)
        nbytes = H * a.S * D * 2
        res = {}
        for pat in ("contiguous", "random"):
            idx = make_idx(pat, H, a.S, a.S, a.page, g, dev)
            x = {"v": vd, "i": idx}
            inps = clones(x, copies_for(nbytes)) if nbytes < (512 << 20) else [x]
            ms = graph_ms(lambda z: gather_reduce(z["v"], z["i"]), inps, 5, a.runs)
            del inps
            res[pat] = (ms * 1e3, 100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
        gsweep.append({"D": D, "row_bytes": D * 2, "contig_us": res["contiguous"][0], "rand_us": res["random"][0],
                       "contig_pct": res["contiguous"][1], "rand_pct": res["random"][1],
                       "ratio": res["random"][1] / res["contiguous"][1]})
        print(f"{D:>5} {D * 2:>6} {res['contiguous'][1]:>9.1f}% {res['random'][1]:>8.1f}% "
              f"{res['random'][1] / res['contiguous'][1]:>11.3f}", flush=True)
        del vd
        torch.cuda.empty_cache()
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump({"schema": "access_pattern_v2", "gpu": torch.cuda.get_device_name(0), "peak_gbs": HBM_PEAK_GBS,
                   "B": a.B, "H_q": a.Hq, "H_k": a.Hk, "S": a.S, "D": a.D, "page": a.page, "rows": rows_out,
                   "gather_reduce": probe, "granularity_sweep": gsweep}, f, indent=2)
    print(f"saved {a.output_json}")


if __name__ == "__main__":
    main()
