"""Score-pass latency per key format on MI355X.

Port of the question benchmarks/bench_unpack_ablation.py:63-103 asks: do
fewer key bytes give a faster score pass?  For S in {8192, 16384} and
D in {64, 128} at B=32, H_q=64, H_k=8, times the per-head score pass
(graph replays) with bf16 keys, fp8 e4m3fn keys, and packed int4 and int2
keys (bf16 scale/min per 32 dims), and reports the bytes each reads and the
achieved bandwidth against MI355X's 8 TB/s.

    python -m bytes_amd.harness.score_ablation
"""
from __future__ import annotations

import argparse
import json
import math
import os

import torch

from .timing import HBM_PEAK_GBS, clones, copies_for, graph_ms


def main(argv=None):
    from .. import attention_kernels as AK
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--B", type=int, default=32)
    ap.add_argument("--Hq", type=int, default=64)
    ap.add_argument("--Hk", type=int, default=8)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--output-json", default="harness_out/score_ablation.json")
    a = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    rows = []
    for S in (8192, 16384):
        for D in (64, 128):
            q = torch.randn(a.B, a.Hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
            k = torch.randn(a.B, a.Hk, S, D, generator=g, device=dev, dtype=torch.bfloat16)
            sc = 1 / math.sqrt(D)
            out_b = a.B * a.Hq * S * 4
            row = {"S": S, "D": D, "us": {}, "bytes": {}, "gbs": {}}
            cases = [("bf16_dot", {"q": q, "k": k}, lambda x: AK.sparse_score_scalar(x["q"], x["k"], sc),
                      k.numel() * 2),
                     ("fp8_dot", {"q": q, "k": k.to(torch.float8_e4m3fn)},
                      lambda x: AK.sparse_score_scalar(x["q"], x["k"], sc, score_bits=8), k.numel())]
            for bits in (4, 2):
                p, s, z = AK.quantize_and_pack_score_keys(k, bits, 32)
                cases.append((f"int{bits}_full_dot", {"q": q, "p": p, "s": s, "z": z},
                               lambda x, b=bits: AK.sparse_score_packed(x["q"], x["p"], x["s"], x["z"], sc,
                                                                        score_bits=b),
                               p.numel() + 2 * s.numel() * 2))
            for name, x, fn, kb in cases:
                nbytes = kb + out_b
                ms = graph_ms(fn, clones(x, copies_for(nbytes)), 5, a.runs)
                row["us"][name] = ms * 1e3
                row["bytes"][name] = nbytes
                row["gbs"][name] = nbytes / (ms * 1e-3) / 1e9
            rows.append(row)
            print(f"S={S} D={D}: " + " ".join(f"{n} {row['us'][n]:.1f} us ({row['gbs'][n]:.0f} GB/s)"
                                              for n in row["us"]), flush=True)
            del q, k, cases
            torch.cuda.empty_cache()
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump({"schema": "score_ablation_v1", "gpu": torch.cuda.get_device_name(0), "peak_gbs": HBM_PEAK_GBS,
                   "B": a.B, "H_q": a.Hq, "H_k": a.Hk, "rows": rows}, f, indent=2)
    print(f"saved {a.output_json}")


if __name__ == "__main__":
    main()
