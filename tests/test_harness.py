"""CPU checks of the study harnesses: they import, and the capacity model
counts exactly the bytes of the tensors the reference's capacity study
allocates (benchmarks/bench_sparse_capacity.py:46-83)."""
import torch

from bytes_amd.harness import access_pattern, capacity, crossover, floor, kernels, score_ablation, timing, unpack_ablation  # noqa: F401,E501


def _nbytes(*shapes_dtypes):
    return sum(torch.empty(s, dtype=d, device="meta").numel() * torch.empty((), dtype=d).element_size()
               for s, d in shapes_dtypes)


def test_capacity_bytes_match_reference_tensors():
    Hk, D = 8, 128
    for S in (16384, 32768):
        Sq = S - 128
        ref = {
            "BF16": _nbytes(((1, Hk, S, D), torch.bfloat16), ((1, Hk, S, D), torch.bfloat16)),
            "FP8": _nbytes(((1, Hk, S, D), torch.float8_e4m3fn), ((1, Hk, S, D), torch.float8_e4m3fn)),
            "KIVI-4": _nbytes(((1, Hk, D, Sq // 8), torch.int32), ((1, Hk, D, Sq // 32), torch.float16),
                              ((1, Hk, D, Sq // 32), torch.float16), ((1, Hk, Sq, D // 8), torch.int32),
                              ((1, Hk, Sq, D // 32), torch.float16), ((1, Hk, Sq, D // 32), torch.float16),
                              ((1, Hk, 128, D), torch.bfloat16), ((1, Hk, 128, D), torch.bfloat16)),
            "Sparse-INT2": _nbytes(((1, Hk, S, D // 4), torch.uint8), ((1, Hk, S, D // 32), torch.bfloat16),
                                   ((1, Hk, S, D // 32), torch.bfloat16), ((1, Hk, S, D), torch.bfloat16),
                                   ((1, Hk, S, D), torch.bfloat16)),
        }
        for m, b in ref.items():
            assert capacity.per_sequence_bytes(m, Hk, S, D) == b, (m, S)


def test_copies_cover_the_infinity_cache():
    for n in (1 << 20, 100 << 20, 300 << 20):
        assert timing.copies_for(n) * n >= 2 * timing.MALL_BYTES
    assert timing.copies_for(1 << 30) == 1
