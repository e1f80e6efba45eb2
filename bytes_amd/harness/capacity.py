"""Largest decode batch whose cache fits on one MI355X, per storage format.

Port of benchmarks/bench_sparse_capacity.py:8-111.  The reference allocates
growing batches until an out-of-memory error; here the cache bytes per
sequence come from the layouts themselves (the same tensors the reference
allocates), the largest batch that fits in the device's free memory is
computed, and that batch is then allocated once to confirm it (--verify).

  BF16         K, V bf16 [B, H_k, S, D]
  FP8          K, V float8_e4m3fn
  KIVI-4       4-bit codes (keys per channel, values per token), fp16 scale/min
               per 32, residual window of 128 bf16 tokens
  Sparse-INT2  packed 2-bit score keys + bf16 scale/min per 32 dims, plus the
               bf16 K, V the gather reads

    python -m bytes_amd.harness.capacity [--verify]
"""
from __future__ import annotations

import argparse
import json
import os

import torch

REF_BATCHES = [1, 2, 4, 8, 16, 32, 64, 128, 256, 384, 512]


def per_sequence_bytes(method: str, Hk: int, S: int, D: int) -> int:
    if method == "BF16":
        return 2 * Hk * S * D * 2
    if method == "FP8":
        return 2 * Hk * S * D
    if method == "KIVI-4":
        R = 128
        Sq = S - R
        codes = Hk * D * (Sq // 8) * 4 + Hk * Sq * (D // 8) * 4
        meta = 2 * Hk * D * (Sq // 32) * 2 + 2 * Hk * Sq * (D // 32) * 2
        return codes + meta + 2 * Hk * R * D * 2
    if method == "Sparse-INT2":
        return Hk * S * (D // 4) + 2 * Hk * S * (D // 32) * 2 + 2 * Hk * S * D * 2
    raise ValueError(method)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--Hk", type=int, default=8)
    ap.add_argument("--D", type=int, default=128)
    ap.add_argument("--verify", action="store_true", help="allocate the computed batch once")
    ap.add_argument("--output-json", default="harness_out/sparse_capacity.json")
    a = ap.parse_args(argv)
    free, total = torch.cuda.mem_get_info(0)
    res = {"gpu": torch.cuda.get_device_name(0), "free_bytes": free, "total_bytes": total}
    for S in (16384, 32768):
        res[str(S)] = {}
        for m in ("BF16", "FP8", "KIVI-4", "Sparse-INT2"):
            per = per_sequence_bytes(m, a.Hk, S, a.D)
            bmax = free // per
            ref_b = max([b for b in REF_BATCHES if b <= bmax], default=0)
            ok = None
            if a.verify and bmax > 0:
                try:
                    buf = torch.empty(bmax * per, dtype=torch.uint8, device="cuda:0")
                    ok = True
                    del buf
                except RuntimeError:
                    ok = False
                torch.cuda.empty_cache()
            res[str(S)][m] = {"bytes_per_sequence": per, "max_batch": int(bmax), "max_batch_in_reference_list": ref_b,
                              "cache_gb_at_max": round(bmax * per / 2 ** 30, 2), "verified": ok}
            print(f"S={S} {m:12s} {per / 2 ** 20:9.1f} MiB/seq  max batch {bmax:5d} "
                  f"(reference list: {ref_b})" + ("" if ok is None else f" verified={ok}"), flush=True)
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump(res, f, indent=2)
    print(f"saved {a.output_json}")


if __name__ == "__main__":
    main()
