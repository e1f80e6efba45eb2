#!/usr/bin/env python3
"""MI355X decode-attention benchmark (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--only] [--all] [--no-cpu]

One "step" is one decode-attention call of a configuration over one batch of
synthetic inputs already resident in HBM.  W untimed warm-up steps run
first; then exactly K steps are captured into one hipGraph (each step on its
own copy of the inputs, rotating through enough copies to exceed 2x the
256 MB Infinity Cache, so every step streams from HBM) and the graph replay
is timed with HIP events on the capture's stream, between two device
synchronisations.  The step's dominant kernel is then timed on its own: at
least 60 more (eager) steps, each with a HIP event pair that the library
records on the kernel's stream right around that launch, and the median pair;
the steps are queued behind a spin kernel in chunks, so they run back to
back as the graph-replayed ones do.

Before a config is timed, one step on its own inputs is checked against the
CPU oracle (test infrastructure, oracle/, used only as the checker): outside
the attention tolerance (max-abs 2e-2, mean-abs 2e-3) the run stops and no
JSON line is printed; each config's `gate` records the differences.

`value` is the headline config (BASELINE C2, KIVI 2-bit) in us/step;
`roofline` is its dominant kernel's algorithmic bytes over that kernel's
median duration (`step_frac` the same over the whole step).  `per_config`
holds the same figures for every other BASELINE config (C1, C2 4-bit, the
dense and KIVI L>=16K points, C3, C4, C5 at k = 256/1024/4096; --all adds
more).  Each config's cpu_baseline times the CPU oracle on the whole step,
or on a stated sample where the whole step would take minutes (C5).  Rank 0
prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
import time

import torch

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
MALL_BYTES = 256 << 20     # Infinity Cache


# ---------------------------------------------------------------------------
# Cases
# ---------------------------------------------------------------------------
class Case:
    name = ""
    workload = ""
    dtype = "bf16"
    kernel = ""            # kernel symbol (substring) that dominates the step
    family = 0             # its family in the library's kernel timing hook (bytes_set_kernel_events)

    def bytes_per_step(self) -> int:
        raise NotImplementedError

    def kernel_bytes(self) -> int:
        """Algorithmic bytes of one launch of the dominant kernel."""
        return self.bytes_per_step()

    def make(self, dev):
        raise NotImplementedError

    def step(self, inp):
        raise NotImplementedError

    def cpu_sample(self):
        """-> (description, fn running the oracle on the sample, full/sample work ratio);
        the sample is the whole step (ratio 1) wherever the oracle runs it in
        seconds."""
        raise NotImplementedError

    def reference(self, inp, out):
        """Parity gate: (GPU output, oracle output) on the CPU for the step's
        own inputs `inp` and output `out`; where the oracle's fp32 copies of
        the whole cache would not fit host memory, batch row 0 of both.  None:
        no gate (not a decode step)."""
        raise NotImplementedError


class DenseCase(Case):
    kernel = "dense_decode_kernel"
    family = 1

    def __init__(self, name, B, Hq, Hk, D, L):
        self.name, self.shape = name, (B, Hq, Hk, D, L)
        self.workload = f"dense bf16 GQA decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L}"

    def bytes_per_step(self):
        B, Hq, Hk, D, L = self.shape
        return 2 * B * Hk * L * D * 2 + 2 * B * Hq * D * 2

    def make(self, dev):
        from bytes_amd import workloads as W
        B, Hq, Hk, D, L = self.shape
        if B * Hk * L * D > (1 << 28):       # multi-GiB caches are drawn on the device
            x = W.c5_topk(seed=0, device=dev, B=B, Hq=Hq, Hk=Hk, D=D, L=L)
            return {"q": x["q"], "k": x["k"], "v": x["v"], "scale": x["scale"]}
        x = W.dense(*self.shape, seed=0, device="cpu")
        return {"q": x["q"].to(dev), "k": x["k"].to(dev), "v": x["v"].to(dev), "scale": x["scale"]}

    def step(self, inp):
        from bytes_amd.attention_kernels import decode_attn_bf16
        return decode_attn_bf16(inp["q"], inp["k"], inp["v"], inp["scale"])

    def cpu_sample(self):
        from bytes_amd import workloads as W
        from oracle import reference as R
        B, Hq, Hk, D, L = self.shape
        if B * Hk * L * D > (1 << 28):                     # multi-GiB caches: one (b, kv-head) unit
            x = W.dense(1, Hq // Hk, 1, D, L, seed=0)
            units = B * Hk
            return (f"one (b, kv-head) unit of {units}: q [1,{Hq // Hk},1,{D}], K/V [1,1,{L},{D}]",
                    lambda: R.decode_attn(x["q"], x["k"], x["v"], scale=x["scale"]), units)
        x = W.dense(*self.shape, seed=0)
        return (f"the whole step: oracle decode_attn on q [{B},{Hq},1,{D}], K/V [{B},{Hk},{L},{D}]",
                lambda: R.decode_attn(x["q"], x["k"], x["v"], scale=x["scale"]), 1)

    def reference(self, inp, out):
        from oracle import reference as R
        B, Hq, Hk, D, L = self.shape
        rows = slice(0, 1) if B * Hk * L * D > (1 << 28) else slice(0, B)
        q, k, v = (inp[n][rows].cpu() for n in ("q", "k", "v"))
        return out[rows].cpu(), R.decode_attn(q, k, v, scale=inp["scale"])


class DenseFp8Case(DenseCase):
    kernel = "dense_decode_kernel"
    dtype = "fp8 e4m3fn K/V, bf16 q"

    def __init__(self, name, B, Hq, Hk, D, L):
        super().__init__(name, B, Hq, Hk, D, L)
        self.workload = f"fp8 (e4m3fn) GQA decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L}"

    def bytes_per_step(self):
        B, Hq, Hk, D, L = self.shape
        return 2 * B * Hk * L * D + 2 * B * Hq * D * 2

    def make(self, dev):
        x = super().make(dev)
        x["k"], x["v"] = x["k"].to(torch.float8_e4m3fn), x["v"].to(torch.float8_e4m3fn)
        return x

    def step(self, inp):
        from bytes_amd.attention_kernels import decode_attn_fp8
        return decode_attn_fp8(inp["q"], inp["k"], inp["v"], inp["scale"])

    def cpu_sample(self):
        desc, fn, ratio = super().cpu_sample()
        return desc + " (fp8 K/V as the oracle's fp32 values)", fn, ratio


class KiviCase(Case):
    kernel = "kivi_decode_kernel"
    family = 2

    def __init__(self, name, bits, B=4, Hq=28, Hk=4, D=128, L=16384, R=128, kernel="kivi_decode_kernel"):
        self.name, self.bits, self.shape = name, bits, (B, Hq, Hk, D, L, R)
        self.kernel = kernel   # the library's choice for this shape on MI355X (256 CUs)
        self.dtype = f"u{bits}+fp16 meta+bf16"
        self.workload = (f"KIVI-{bits} decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L} "
                         f"(Sq={L - R} packed, residual {R} bf16, group 32)")

    def bytes_per_step(self):
        B, Hq, Hk, D, L, R = self.shape
        Sq = L - R
        codes = 2 * B * Hk * D * Sq * self.bits // 8
        kmeta = B * Hk * D * (Sq // 32) * 4
        vmeta = B * Hk * Sq * (D // 32) * 4
        resid = 2 * B * Hk * R * D * 2
        return codes + kmeta + vmeta + resid + 2 * B * Hq * D * 2

    def make(self, dev):
        from bytes_amd import workloads as W
        from bytes_amd.kivi import quantize_and_pack_along_last_dim
        B, Hq, Hk, D, L, R = self.shape
        raw = W.kivi_raw(B, Hq, Hk, D, L, R, seed=0)
        raw = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in raw.items()}
        x = W.kivi_pack_inputs(raw, quantize_and_pack_along_last_dim, self.bits)
        x["K_residual"] = x["K_residual"].contiguous()
        x["V_residual"] = x["V_residual"].contiguous()
        return x

    def step(self, x):
        from bytes_amd.kivi import kivi_decode_attn
        return kivi_decode_attn(x["Q"], x["Kq"], x["K_scale"], x["K_mn"], x["K_residual"], x["Vq"],
                                x["V_scale"], x["V_mn"], x["V_residual"], self.bits, 32)

    def cpu_sample(self):
        from bytes_amd import workloads as W
        from oracle import reference as R
        B, Hq, Hk, D, L, Rw = self.shape
        raw = W.kivi_raw(B, Hq, Hk, D, L, Rw, seed=0)
        x = W.kivi_pack_inputs(raw, R.kivi_quantize_and_pack_last_dim, self.bits)
        args = [x[n] for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale", "V_mn", "V_residual")]
        return (f"the whole step: oracle kivi_decode_attn on Q [{B},{Hq},1,{D}], "
                f"Sq={L - Rw} packed + {Rw} residual",
                lambda: R.kivi_decode_attn(*args, self.bits, 32), 1)

    def reference(self, inp, out):
        from oracle import reference as R
        args = [inp[n].cpu() for n in ("Q", "Kq", "K_scale", "K_mn", "K_residual", "Vq", "V_scale", "V_mn",
                                       "V_residual")]
        return out.cpu(), R.kivi_decode_attn(*args, self.bits, 32)


class TopkCase(Case):
    """BASELINE C5: group-summed fp32 scores per KV head over the whole cache,
    deterministic top-k per (b, KV head), gathered bf16 attention for every
    query head of the group.  One step = score + top-k + gather."""
    kernel = "score_kernel"
    family = 5

    def __init__(self, name, kb, B=8, Hq=24, Hk=8, D=128, L=131072, score_bits=16):
        self.name, self.kb, self.shape, self.score_bits = name, kb, (B, Hq, Hk, D, L), score_bits
        keys = {16: "", 8: " on fp8 e4m3fn score keys", 4: " on packed 4-bit score keys",
                2: " on packed 2-bit score keys"}[score_bits]
        self.workload = f"token top-k decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L} k={kb} (group-summed scores{keys})"
        if score_bits != 16:
            self.dtype = {8: "bf16 (fp8 score keys)", 4: "bf16 (int4 score keys)", 2: "bf16 (int2 score keys)"}[
                score_bits]

    def key_bytes(self):
        """Bytes of score keys the score pass reads: codes plus, for packed keys,
        the bf16 scale and min of every 32-dim group."""
        B, Hq, Hk, D, L = self.shape
        rows = B * Hk * L
        if self.score_bits in (16, 8):
            return rows * D * self.score_bits // 8
        return rows * (D * self.score_bits // 8 + (D // 32) * 2 * 2)

    def bytes_per_step(self):
        B, Hq, Hk, D, L = self.shape
        scores = B * Hk * L * 4 * 2               # fp32 scores written, read by the top-k
        gather = 2 * B * Hk * self.kb * D * 2     # selected K and V rows
        return self.key_bytes() + scores + gather + 2 * B * Hq * D * 2

    def kernel_bytes(self):
        B, Hq, Hk, D, L = self.shape
        return self.key_bytes() + B * Hk * L * 4 + B * Hq * D * 2

    def make(self, dev):
        from bytes_amd import workloads as W
        from bytes_amd.sparse import quantize_and_pack_score_keys
        B, Hq, Hk, D, L = self.shape
        x = W.c5_topk(seed=0, device=dev, B=B, Hq=Hq, Hk=Hk, D=D, L=L)
        d = {"q": x["q"], "k": x["k"], "v": x["v"], "scale": x["scale"]}
        if self.score_bits == 8:
            d["ks"] = x["k"].to(torch.float8_e4m3fn)
        elif self.score_bits in (4, 2):
            d["ks"], d["ksc"], d["kzr"] = quantize_and_pack_score_keys(x["k"], self.score_bits, 32)
        return d

    def step(self, inp):
        from bytes_amd.sparse import token_topk_decode
        return token_topk_decode(inp["q"], inp["k"], inp["v"], self.kb, inp["scale"], k_score=inp.get("ks"),
                                 score_scale=inp.get("ksc"), score_zero=inp.get("kzr"),
                                 score_bits=self.score_bits if self.score_bits in (4, 2) else None)

    def cpu_sample(self):
        from bytes_amd import workloads as W
        from oracle import reference as R
        B, Hq, Hk, D, L = self.shape
        x = W.dense(1, Hq, Hk, D, L, seed=0)
        return (f"one batch row of {B} (the oracle's fp32 copies of the whole 4 GiB cache would need "
                f"tens of GiB): oracle group scores + top-{self.kb} + gather, q [1,{Hq},1,{D}], "
                f"K/V [1,{Hk},{L},{D}]; x {B} to a full step",
                lambda: R.token_topk_decode(x["q"], x["k"], x["v"], self.kb, x["scale"]), B)

    def reference(self, inp, out):
        from oracle import reference as R
        q, k, v = (inp[n][0:1].cpu() for n in ("q", "k", "v"))
        if self.score_bits == 16:
            ks = k
        elif self.score_bits == 8:
            ks = inp["ks"][0:1].cpu().float()
        else:
            ks = R.score_keys_dequant(inp["ks"][0:1].cpu(), inp["ksc"][0:1].cpu(), inp["kzr"][0:1].cpu(),
                                      self.score_bits, 32)
        idx = R.topk_indices(R.group_scores(q, ks, inp["scale"]), self.kb)
        o = out[0] if isinstance(out, tuple) else out              # (output, selected indices)
        return o[0:1].cpu(), R.sparse_gather_attn(q, k, v, idx, inp["scale"])


class QuestCase(Case):
    """BASELINE C4: Quest page bounds from the per-page min/max metadata, top
    ceil(2048/16) = 128 pages per query head, attention over their rows.  The
    metadata is a property of the cache (built once, outside the step)."""
    kernel = "gather_decode_kernel"
    family = 4

    def __init__(self, name, budget=2048, page=16, B=1, Hq=28, Hk=4, D=128, L=32768):
        self.name, self.budget, self.page, self.shape = name, budget, page, (B, Hq, Hk, D, L)
        self.workload = (f"Quest page-sparse decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L} page {page} "
                         f"budget {budget} tokens (64 needles)")

    def bytes_per_step(self):
        B, Hq, Hk, D, L = self.shape
        np_ = L // self.page
        meta = 2 * B * Hk * np_ * D * 2                    # kmin + kmax read by the bound kernel
        bounds = B * Hq * np_ * 4 * 2                      # written, then read by the top-k
        rows = 2 * B * Hq * self.budget * D * 2            # gathered K and V rows (per query head)
        return meta + bounds + rows + 2 * B * Hq * D * 2

    def kernel_bytes(self):
        B, Hq, Hk, D, L = self.shape
        return 2 * B * Hq * self.budget * D * 2 + 2 * B * Hq * D * 2

    def make(self, dev):
        from bytes_amd import quest as Q
        from bytes_amd import workloads as W
        x = W.c4_quest(seed=0)
        k = x["k"].to(dev)
        return {"q": x["q"].to(dev), "k": k, "v": x["v"].to(dev), "meta": Q.quest_page_minmax(k, self.page),
                "scale": x["scale"]}

    def step(self, inp):
        from bytes_amd.quest import quest_decode
        return quest_decode(inp["q"], inp["k"], inp["v"], self.budget, inp["scale"], page=self.page,
                            meta=inp["meta"])

    def cpu_sample(self):
        from bytes_amd import workloads as W
        from oracle import reference as R
        x = W.c4_quest(seed=0)
        B, Hq, Hk, D, L = self.shape

        def run():
            _, tok, _ = R.quest_select(x["q"], x["k"], self.budget, self.page, x["scale"])
            return R.sparse_gather_attn(x["q"], x["k"], x["v"], tok, x["scale"])
        return (f"the whole step: oracle page metadata + bounds + page top-k + gather "
                f"(B{B} Hq{Hq} L{L})", run, 1)

    def reference(self, inp, out):
        from oracle import reference as R
        q, k, v = (inp[n].cpu() for n in ("q", "k", "v"))
        _, tok, _ = R.quest_select(q, k, self.budget, self.page, inp["scale"])
        return out.cpu(), R.sparse_gather_attn(q, k, v, tok, inp["scale"])


class PqCase(Case):
    """BASELINE C3: PQ-LUT decode with quantized keys and values.  Scoring q
    against the key codebooks is part of the step, fused into the decode launch
    (decode_attn_pq_kv_fused: q . k_hat on MFMA from the codebook rows, within
    the attention tolerance of pq_build_lut followed by decode_attn_pq_lut_kv);
    codebook fitting and encoding are setup."""
    kernel = "pq_wave_kernel"
    family = 3

    def __init__(self, name, B=1, Hq=28, Hk=4, D=128, L=32768, K=256):
        self.name, self.shape, self.K = name, (B, Hq, Hk, D, L), K
        self.dtype = "u8 codes+fp16 codebooks+fp32 LUT"
        self.workload = f"PQ-LUT KV decode B{B} Hq{Hq} Hkv{Hk} D{D} L{L} (16 x 8-dim subspaces, K={K})"

    def bytes_per_step(self):
        B, Hq, Hk, D, L = self.shape
        M = D // 8
        codes = 2 * B * Hk * L * M
        cbs = 2 * Hk * M * self.K * 8 * 2
        return codes + cbs + B * Hq * D * 2 + B * Hq * D * 2

    def make(self, dev):
        from bytes_amd import workloads as W
        x = W.c3_pq(seed=0, device=dev)
        return {n: x[n] for n in ("q", "k_cb", "v_cb", "k_idx", "v_idx", "scale")}

    def step(self, x):
        from bytes_amd.pq import decode_attn_pq_kv_fused
        return decode_attn_pq_kv_fused(x["q"], x["k_cb"], x["k_idx"], x["v_idx"], x["v_cb"], x["scale"])

    def cpu_sample(self):
        from oracle import reference as R
        B, Hq, Hk, D, L = self.shape
        g = torch.Generator().manual_seed(0)
        M = D // 8
        q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16)
        kcb = torch.randn(Hk, M, self.K, 8, generator=g).half()
        vcb = torch.randn(Hk, M, self.K, 8, generator=g).half()
        ki = torch.randint(0, self.K, (B, Hk, L, M), generator=g).to(torch.uint8)
        vi = torch.randint(0, self.K, (B, Hk, L, M), generator=g).to(torch.uint8)

        def run():
            lut = R.pq_build_lut(q, kcb, 1.0 / D ** 0.5)
            return R.decode_attn_pq_lut_kv(lut, ki, vi, vcb)
        return (f"the whole step: oracle LUT build + pq_lut_kv, B{B} Hq{Hq} Hkv{Hk} L{L} (seeded random "
                f"codes and codebooks of the C3 shape)", run, 1)

    def reference(self, inp, out):
        from oracle import reference as R
        x = {n: inp[n].cpu() for n in ("q", "k_cb", "v_cb", "k_idx", "v_idx")}
        lut = R.pq_build_lut(x["q"], x["k_cb"], inp["scale"])
        return out.cpu(), R.decode_attn_pq_lut_kv(lut, x["k_idx"], x["v_idx"], x["v_cb"])


class CopyCase(Case):
    """Plain device copy of known size: the calibration point for HBM byte counters
    (FETCH_SIZE / WRITE_SIZE of this kernel vs its exact 2 x nbytes traffic)."""
    kernel = "elementwise_kernel"
    dtype = "u8"

    def __init__(self, name, nbytes):
        self.name, self.nbytes = name, nbytes
        self.workload = f"device copy {nbytes >> 20} MiB (counter calibration)"

    def bytes_per_step(self):
        return 2 * self.nbytes

    def make(self, dev):
        return {"src": torch.randint(0, 255, (self.nbytes,), dtype=torch.uint8, device=dev),
                "dst": torch.empty(self.nbytes, dtype=torch.uint8, device=dev)}

    def step(self, inp):
        return inp["dst"].copy_(inp["src"])

    def cpu_sample(self):
        src = torch.randint(0, 255, (self.nbytes // 16,), dtype=torch.uint8)
        dst = torch.empty_like(src)
        return f"copy of {self.nbytes // 16} bytes", lambda: dst.copy_(src), 16

    def reference(self, inp, out):
        return None


def cases():
    from bytes_amd import workloads as W
    return {
        "copy_calib": CopyCase("copy_calib", 256 << 20),
        "c2_kivi2": KiviCase("c2_kivi2", 2),
        "c2_kivi4": KiviCase("c2_kivi4", 4),
        "c1_dense": DenseCase("c1_dense", *W.SHAPES["c1_dense"]),
        "dense_16k": DenseCase("dense_16k", *W.SHAPES["dense_16k"]),
        "dense_32k": DenseCase("dense_32k", 4, 28, 4, 128, 32768),
        "c2_kivi2_64k": KiviCase("c2_kivi2_64k", 2, L=65536, kernel="kivi_pipe_kernel"),
        "c2_kivi4_64k": KiviCase("c2_kivi4_64k", 4, L=65536, kernel="kivi_pipe_kernel"),
        "c3_pq": PqCase("c3_pq"),
        "c4_quest": QuestCase("c4_quest"),
        "c5_topk256": TopkCase("c5_topk256", 256),
        "c5_topk1024": TopkCase("c5_topk1024", 1024),
        "c5_topk4096": TopkCase("c5_topk4096", 4096),
        "c5_dense": DenseCase("c5_dense", *W.SHAPES["c5_topk"]),
        "c5_topk1024_fp8s": TopkCase("c5_topk1024_fp8s", 1024, score_bits=8),
        "c5_topk1024_int4s": TopkCase("c5_topk1024_int4s", 1024, score_bits=4),
        "c5_topk1024_int2s": TopkCase("c5_topk1024_int2s", 1024, score_bits=2),
        "dense_16k_fp8": DenseFp8Case("dense_16k_fp8", *W.SHAPES["dense_16k"]),
    }


HEADLINE = "c2_kivi2"


def measured_traffic(name: str):
    """HBM bytes per launch of the config's dominant kernel, measured by the
    FETCH_SIZE / WRITE_SIZE counter passes recorded in profiles/traffic.json
    (each scaled by the same counter's reading for a copy of known size)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
def clone_inputs(inp, copies):
    out = [inp]
    for _ in range(copies - 1):
        out.append({k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()})
    return out


def time_step(case: Case, inps, steps: int) -> float:
    """ms per step: `steps` steps captured in one hipGraph, replay timed with
    HIP events on the capture's stream between two device synchronisations."""
    copies = len(inps)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            case.step(inps[i % copies])
    torch.cuda.synchronize()
    g.replay()                       # untimed: uploads the graph
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del g
    return ms


def time_kernel(case: Case, inps, steps: int) -> float:
    """Duration (ms) of the step's dominant kernel: the library records a HIP
    event pair on the kernel's own stream right before and after that launch
    (bytes_set_kernel_events), one pair per step, over at least 60 steps; the
    median of the pairs (a single pair is perturbed now and then by the host's
    launch timing).  The steps are launched in chunks of 20 queued behind a
    spin kernel, so they run back to back as the graph-replayed steps do: a
    launch onto an idle GPU starts its XCDs up to ~2 us apart (measured with
    per-wave timestamps), which would otherwise land in the pair."""
    from bytes_amd import _lib
    if case.family == 0:                  # not a library kernel: the step is the kernel
        return time_step(case, inps, steps)
    steps = max(steps, 60)
    lib = _lib.lib()
    copies = len(inps)
    s = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in evs:                # create the events
        e0.record(s)
        e1.record(s)
    torch.cuda.synchronize()
    chunk, spin = 20, 4_000_000
    try:
        for c0 in range(0, steps, chunk):
            while True:
                torch.cuda._sleep(spin)   # holds the queue while the chunk is launched
                for i in range(c0, min(c0 + chunk, steps)):
                    e0, e1 = evs[i]
                    _lib.check(lib.bytes_set_kernel_events(case.family, e0.cuda_event, e1.cuda_event),
                               "bytes_set_kernel_events")
                    case.step(inps[i % copies])
                caught_up = evs[c0][0].query()   # the GPU reached the chunk before it was all queued
                torch.cuda.synchronize()
                if not caught_up or spin >= 256_000_000:
                    break
                spin *= 2
    finally:
        lib.bytes_set_kernel_events(0, None, None)
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)


GATE_MAX_ABS, GATE_MEAN_ABS = 2e-2, 2e-3      # north_star attention tolerance


class GateFailure(RuntimeError):
    pass


def parity_gate(case: Case, base, dev):
    """One step on the config's own inputs checked against the CPU oracle
    (the checker, as in the tests) before anything is timed; a step outside
    the attention tolerance raises GateFailure, so no figure is reported
    for it."""
    out = case.step(base)
    torch.cuda.synchronize()
    pair = case.reference(base, out)
    if pair is None:
        return None
    got, ref = pair
    d = (got.float() - ref.float()).abs()
    g = {"max_abs": float(d.max()), "mean_abs": float(d.mean()), "tolerance": [GATE_MAX_ABS, GATE_MEAN_ABS],
         "checked": list(got.shape)}
    if not (torch.isfinite(got.float()).all() and g["max_abs"] <= GATE_MAX_ABS and g["mean_abs"] <= GATE_MEAN_ABS):
        raise GateFailure(f"{case.name}: step output differs from the oracle (max-abs {g['max_abs']:.3e}, "
                          f"mean-abs {g['mean_abs']:.3e}); not timed")
    return {k: (round(v, 7) if isinstance(v, float) else v) for k, v in g.items()}


def measure(case: Case, steps: int, warmup: int, dev, gate: bool = True) -> dict:
    base = case.make(dev)
    gate_r = parity_gate(case, base, dev) if gate else None
    nbytes = case.bytes_per_step()
    copies = max(2, math.ceil(2 * MALL_BYTES / max(nbytes, 1)) + 1)
    inps = clone_inputs(base, copies)
    for i in range(warmup):
        case.step(inps[i % copies])
    torch.cuda.synchronize()
    ms = time_step(case, inps, steps)
    kms = time_kernel(case, inps, steps)
    del inps, base
    torch.cuda.empty_cache()
    step_bps = nbytes / (ms * 1e-3)
    kern_bps = case.kernel_bytes() / (kms * 1e-3)
    return {"ms_per_step": ms, "copies": copies, "bytes_per_step": nbytes, "kernel_ms": kms,
            "kernel_bytes": case.kernel_bytes(), "step_Bps": step_bps, "kernel_Bps": kern_bps, "gate": gate_r}


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cpu(case: Case, budget_s: float = 10.0) -> dict:
    """The CPU oracle (oracle/, test infrastructure) on the same workload:
    median of at least 5 timed runs (3 when one run takes over a second) after
    one warm-up, with every host thread torch offers."""
    desc, fn, ratio = case.cpu_sample()
    torch.set_num_threads(os.cpu_count() or 1)
    fn()                                            # warm-up
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        need = 3 if times[0] > 1.0 else 5
        if len(times) >= need and (time.perf_counter() - t_start > budget_s / 4 or len(times) >= 30):
            break
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    med = statistics.median(times)
    return {"value": round(med * ratio * 1e6, 1), "unit": "us/step", "cores": torch.get_num_threads(),
            "host_cpus": os.cpu_count(), "cpu_model": cpu_model(), "kind": "port",
            "sample": f"{desc}; median of {len(times)} runs" + (f" x {ratio}" if ratio != 1 else "")}


# C1, C2 (2-bit headline and 4-bit), the dense and
# KIVI L>=16K points the north_star bar is judged at (dense B4 L16K and L32K,
# KIVI-2/-4 at L64K), C3, C4 and C5 at its three budgets.
DEFAULT_CONFIGS = ["c1_dense", "c2_kivi4", "dense_16k", "dense_32k", "c2_kivi2_64k", "c2_kivi4_64k", "c3_pq",
                   "c4_quest", "c5_topk256", "c5_topk1024", "c5_topk4096"]
EXTRA_CONFIGS = ["dense_16k_fp8", "c5_dense", "c5_topk1024_fp8s", "c5_topk1024_int4s", "c5_topk1024_int2s"]


def entry(case: Case, r: dict, cpu) -> dict:
    e = {"workload": case.workload, "us_per_step": round(r["ms_per_step"] * 1e3, 3),
         "GBps": round(r["step_Bps"] / 1e9, 1), "hbm_frac": round(r["step_Bps"] / HBM_PEAK, 4),
         "bytes": r["bytes_per_step"], "kernel": case.kernel, "kernel_us": round(r["kernel_ms"] * 1e3, 3),
         "kernel_bytes": r["kernel_bytes"], "kernel_GBps": round(r["kernel_Bps"] / 1e9, 1),
         "kernel_frac": round(r["kernel_Bps"] / HBM_PEAK, 4), "traffic": None, "gate": r["gate"]}
    tr = measured_traffic(case.name)
    if tr is not None:
        e["traffic"] = tr["traffic_bytes"]
        e["traffic_source"] = tr["source"]
    if cpu is not None:
        e["cpu_baseline"] = cpu
    return e


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # defaults: at least 200 timed steps after 20 warm-up steps, as the
    # baseline's measurement rules ask
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default=HEADLINE)
    ap.add_argument("--only", action="store_true", help="time the named config alone (no per_config)")
    ap.add_argument("--all", action="store_true", help="add the extra configs to per_config")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline legs")
    ap.add_argument("--no-gate", action="store_true", help="skip the parity gate against the CPU oracle")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only: every configuration is one GPU's share "
              "of the work (units of (batch, KV head) split across GPUs, no cross-GPU traffic in the "
              "step). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    allc = cases()
    if args.config not in allc:
        print(f"unknown config {args.config}; known: {sorted(allc)}", file=sys.stderr)
        sys.exit(2)
    head = allc[args.config]
    t0 = time.perf_counter()
    try:
        r = measure(head, args.steps, args.warmup, dev, gate=not args.no_gate)
    except GateFailure as ex:
        print(f"bench.py: parity gate failed: {ex}", file=sys.stderr)
        sys.exit(1)
    print(f"[bench] {head.name}: {r['ms_per_step'] * 1e3:.3f} us/step, kernel {r['kernel_ms'] * 1e3:.3f} us "
          f"({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    us = r["ms_per_step"] * 1e3
    line = {
        "metric": "decode-attn us/step & % of HBM peak BW (BF16/KIVI/PQ/top-k), 1 MI355X",
        "value": round(us, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.dtype,
        "data": "synthetic (seeded N(0,1), BASELINE.json configs)",
        "config": {"workload": head.workload, "name": head.name, "mall_rotation_copies": r["copies"]},
        "gate": r["gate"],
        "roofline": {"bound": "hbm", "achieved": round(r["kernel_Bps"] / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(r["kernel_Bps"] / HBM_PEAK, 4), "traffic": None,
                     "kernel": head.kernel, "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                     "algorithmic_bytes": r["kernel_bytes"],
                     "step_GBps": round(r["step_Bps"] / 1e9, 1), "step_frac": round(r["step_Bps"] / HBM_PEAK, 4)},
    }
    tr = measured_traffic(head.name)
    if tr is not None:
        line["roofline"]["traffic"] = tr["traffic_bytes"]
        line["roofline"]["traffic_source"] = tr["source"]
    if not args.no_cpu:
        line["cpu_baseline"] = time_cpu(head)
    if not args.only:
        per = {}
        names = DEFAULT_CONFIGS + (EXTRA_CONFIGS if args.all else [])
        for name in names:
            if name == head.name:
                continue
            c = allc[name]
            t1 = time.perf_counter()
            try:
                rr = measure(c, args.steps, args.warmup, dev, gate=not args.no_gate)
            except GateFailure as ex:
                print(f"bench.py: parity gate failed: {ex}", file=sys.stderr)
                sys.exit(1)
            cpu = None if args.no_cpu else time_cpu(c)
            per[name] = entry(c, rr, cpu)
            print(f"[bench] {name}: {rr['ms_per_step'] * 1e3:.3f} us/step, kernel {rr['kernel_ms'] * 1e3:.3f} us "
                  f"({time.perf_counter() - t1:.1f} s)", file=sys.stderr, flush=True)
        line["per_config"] = per
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
