"""What any decode step on MI355X is bounded by: the fixed cost of a launch,
the first HBM round trip, and the streaming-read ceiling at a given grid.

The decode kernels' roofline fractions are quoted against HBM's 8 TB/s peak;
this probe measures what plain reads reach on the same GPU, with the same
graph-replay timing and Infinity Cache rotation as the harnesses and
bench.py (csrc/harness.hip: stream_read_kernel, empty_kernel):
  empty      a graph-replayed launch of W workgroups that do nothing
  first_rt   W workgroups each reading one 16-byte word per thread (a single
             dependent HBM round trip after launch)
  stream     W workgroups reading N bytes in total, contiguous slices, eight
             16-byte loads per thread in flight
  stream_nt  the same reads with the non-temporal hint (the decode kernels
             stream their K/V rows so)
for W in {256, 512, 1024, 2048} and N from 4 MB to 1 GB.

    python -m bytes_amd.harness.floor
"""
from __future__ import annotations

import argparse
import json
import os

import torch

from .timing import HBM_PEAK_GBS, copies_for, graph_ms


def main(argv=None):
    from .kernels import empty_launch, stream_read
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--output-json", default="harness_out/floor.json")
    a = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    rows = []

    def emit(kind, wgs, nbytes, ms):
        us = ms * 1e3
        gbs = nbytes / (ms * 1e-3) / 1e9 if nbytes else 0.0
        rows.append({"kind": kind, "wgs": wgs, "bytes": nbytes, "us": round(us, 3), "GBps": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)})
        print(f"{kind:9s} W={wgs:5d} {nbytes / 2**20:8.1f} MiB  {us:9.3f} us  {gbs:8.1f} GB/s", flush=True)

    for wgs in (256, 1024):
        emit("empty", wgs, 0, graph_ms(lambda _x, w=wgs: empty_launch(w, dev), [None], runs=a.runs))
    for wgs in (256, 1024):
        nbytes = wgs * 256 * 16
        bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(copies_for(nbytes))]
        outs = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
        emit("first_rt", wgs, nbytes, graph_ms(lambda x, w=wgs: stream_read(x, w, outs), bufs, runs=a.runs))
        del bufs
    for nbytes in (4 << 20, 32 << 20, 128 << 20, 512 << 20, 1 << 30):
        bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(copies_for(nbytes))]
        for nt in (False, True):
            for wgs in (256, 512, 1024, 2048):
                outs = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
                emit("stream_nt" if nt else "stream", wgs, nbytes,
                     graph_ms(lambda x, w=wgs, n=nt: stream_read(x, w, outs, nontemporal=n), bufs,
                              runs=max(5, a.runs // (1 + nbytes // (128 << 20)))))
        del bufs
        torch.cuda.empty_cache()
    os.makedirs(os.path.dirname(a.output_json) or ".", exist_ok=True)
    with open(a.output_json, "w") as f:
        json.dump({"schema": 1, "gpu": torch.cuda.get_device_name(dev), "rows": rows}, f, indent=1)
    print(f"wrote {a.output_json}", flush=True)


if __name__ == "__main__":
    main()
