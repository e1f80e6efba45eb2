"""bytes_amd: MI355X (gfx950) decode-attention hot path of the saifmb0/bytes study.

Drop-in operators keep the reference's Python call surface:

* ``bytes_amd.attention_kernels`` - src/attention_kernels.py operators
* ``bytes_amd.kivi``              - benchmarks/kivi_latency.py operators (KIVI pack/dequant/decode)
* ``bytes_amd.sparse``            - token scoring, deterministic top-k, gather attention
* ``bytes_amd.quest``             - Quest page metadata, page bounds, page selection and decode
* ``bytes_amd.pq``                - product-quantized decode (LUT / LUT-KV / dequant), LUT build,
                                    encode, k-means, ProductQuantizer
* ``bytes_amd.workloads``         - seeded BASELINE.json synthetic inputs

Every operator runs a hand-written HIP kernel from ``libbytes_amd.so``
(built in-tree by ``python -m bytes_amd.build``); there is no CPU fallback.
"""
from . import attention_kernels, kivi, pq, quest, sparse, workloads  # noqa: F401
from .attention_kernels import decode_attn_bf16  # noqa: F401

__all__ = ["attention_kernels", "kivi", "pq", "quest", "sparse", "workloads", "decode_attn_bf16"]
