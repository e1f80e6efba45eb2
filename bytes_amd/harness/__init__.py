"""Study harnesses of the reference, re-pointed at MI355X.

Each module runs as ``python -m bytes_amd.harness.<name>`` and writes JSON:

  crossover       sparse decode (bf16 / fp8 / int4 / int2 score keys) vs dense
                  bf16 / fp8 and KIVI-4 / KIVI-2 over context length and budget
                  (benchmarks/bench_sparse_crossover.py)
  access_pattern  achieved bandwidth of the gather-attention kernel for
                  contiguous, random, sorted-random and paged token sets
                  (benchmarks/bench_access_pattern.py)
  capacity        largest batch whose cache fits in device memory per storage
                  format (benchmarks/bench_sparse_capacity.py)
  score_ablation  score-pass latency per key format: bf16, fp8, packed int4 and
                  int2 keys (benchmarks/bench_unpack_ablation.py)

Timing follows benchmarks/timing.py (warm-up, one graph capture, event-timed
replays) with the inputs rotated across copies larger than the 256 MiB
Infinity Cache, so every replay streams from HBM.
"""
