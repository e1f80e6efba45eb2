"""Where the packed-key score pass spends its time, stage by stage, on MI355X.

Port of benchmarks/bench_unpack_ablation.py:63-103.  For S in {8192, 16384}
and D in {64, 128} at B=32, H_q=64, H_k=8 it times, per query head over
every key (graph replays, inputs rotated past the Infinity Cache):
  fp8_dot             the production score pass on fp8 e4m3fn keys
  intN_load_reduce    stage 0: load the packed bytes, sum them
  intN_unpack_reduce  stage 1: + unpack the codes
  intN_dequant_reduce stage 2: + code * scale + zero (bf16 per 32 dims)
  intN_valu_dot       stage 3: + the dot with q, all on the vector ALUs
  intN_full_dot       the production packed score pass (MFMA, csrc/score.hip)
for N = 4 and 2, with the stages run by the probe kernel of csrc/harness.hip.
The reference's D = 256 has no production kernel here (head_dim 64 or 128).

    python -m bytes_amd.harness.unpack_ablation
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
    from .kernels import stage_score
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--B", type=int, default=32)
    ap.add_argument("--Hq", type=int, default=64)
    ap.add_argument("--Hk", type=int, default=8)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--output-json", default="harness_out/unpack_ablation.json")
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
            row = {"S": S, "D": D, "B": a.B, "H_q": a.Hq, "H_k": a.Hk, "us": {}, "bytes": {}, "gbs": {}}
            fp8 = k.to(torch.float8_e4m3fn)
            cases = [("fp8_dot", {"q": q, "k": fp8}, lambda x: AK.sparse_score_scalar(x["q"], x["k"], sc,
                                                                                      score_bits=8),
                      fp8.numel())]
            for bits in (4, 2):
                p, s, z = AK.quantize_and_pack_score_keys(k, bits, 32)
                x = {"q": q, "p": p, "s": s, "z": z}
                meta = 2 * s.numel() * 2
                for stage, label in enumerate(("load_reduce", "unpack_reduce", "dequant_reduce", "valu_dot")):
                    cases.append((f"int{bits}_{label}", x,
                                  lambda x, b=bits, st=stage: stage_score(x["q"], x["p"], x["s"], x["z"], b, st),
                                  p.numel() + (meta if stage >= 2 else 0)))
                cases.append((f"int{bits}_full_dot", x,
                               lambda x, b=bits: AK.sparse_score_packed(x["q"], x["p"], x["s"], x["z"], sc,
                                                                        score_bits=b),
                               p.numel() + meta))
            for name, x, fn, kb in cases:
                nbytes = kb + out_b
                ms = graph_ms(fn, clones(x, copies_for(nbytes)), 5, a.runs)
                row["us"][name] = ms * 1e3
                row["bytes"][name] = nbytes
                row["gbs"][name] = nbytes / (ms * 1e-3) / 1e9
            rows.append(row)
            print(f"S={S} D={D}: " + " ".join(f"{n} {row['us'][n]:.1f} us ({row['gbs'][n]:.0f} GB/s)"
                                              for n in row["us"]), flush=True)
            del q, k, fp8, cases
            torch.cuda.empty_cache()
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump({"schema": "unpack_ablation_v1", "gpu": torch.cuda.get_device_name(0), "peak_gbs": HBM_PEAK_GBS,
                   "rows": rows}, f, indent=2)
    print(f"saved {a.output_json}")


if __name__ == "__main__":
    main()
