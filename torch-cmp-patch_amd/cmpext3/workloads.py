"""The five attention workloads this build is measured and checked on (plus a
grouped-query decode step, outside BASELINE's list), and their seeded
synthetic inputs.

Inputs follow one recipe everywhere (bench, tests, smoke): a CPU
torch.Generator seeded per workload draws fp32 N(0,1) for Q, then K, then V;
K and V are multiplied by `kv_std`; the three are cast to the workload dtype
and only then moved to the device.  The GPU kernel and the CPU oracle
therefore see bit-identical (dtype-rounded) inputs.

FLOP convention: 4*B*H*Sq*Sk*D (two GEMMs, the reference's own count,
tools/dev_flash_attn.py:29); causal counts only visible (query, key) pairs.
Bytes: one read of Q, K, V and one write of O.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


@dataclass(frozen=True)
class Workload:
    name: str
    dtype: str
    B: int
    H: int
    Sq: int
    Sk: int
    D: int
    causal: bool = False
    scale: Optional[float] = None
    kv_std: float = 1.0
    seed: int = 0
    note: str = field(default="", compare=False)
    Hkv: Optional[int] = None  # K/V heads (grouped-query); None = H

    @property
    def torch_dtype(self) -> torch.dtype:
        return DTYPES[self.dtype]

    @property
    def eff_scale(self) -> float:
        return self.scale if self.scale is not None else 1.0 / math.sqrt(self.D)

    def visible_pairs(self) -> int:
        """(query, key) pairs that enter the softmax, per (batch, head)."""
        if not self.causal:
            return self.Sq * self.Sk
        n = min(self.Sq, self.Sk)  # rows i < Sk see i + 1 keys, the rest see all Sk
        return n * (n + 1) // 2 + max(0, self.Sq - self.Sk) * self.Sk

    def flops(self) -> int:
        return 4 * self.B * self.H * self.visible_pairs() * self.D

    @property
    def kv_heads(self) -> int:
        return self.H if self.Hkv is None else self.Hkv

    def bytes(self) -> int:
        es = torch.tensor([], dtype=self.torch_dtype).element_size()
        return es * self.B * self.D * (2 * self.H * self.Sq + 2 * self.kv_heads * self.Sk)

    def shapes(self):
        return (self.B, self.H, self.Sq, self.D), (self.B, self.kv_heads, self.Sk, self.D)

    def make_inputs(self, device="cpu", seed: Optional[int] = None, layout: str = "bhsd"):
        """(q, k, v) with the recipe in the module docstring.  layout="bshd" returns
        [B,H,S,D] views of [B,S,H,D] memory (the diffusers/webui layout)."""
        g = torch.Generator().manual_seed(self.seed if seed is None else seed)
        qs, ks = self.shapes()
        q = torch.randn(*qs, generator=g, dtype=torch.float32)
        k = torch.randn(*ks, generator=g, dtype=torch.float32) * self.kv_std
        v = torch.randn(*ks, generator=g, dtype=torch.float32) * self.kv_std
        out = []
        for t in (q, k, v):
            t = t.to(self.torch_dtype)
            if layout == "bshd":
                t = t.transpose(1, 2).contiguous().to(device).transpose(1, 2)
            else:
                t = t.to(device)
            out.append(t)
        return tuple(out)


# BASELINE.json "configs", in order (cfg1 .. cfg5).
WORKLOADS = [
    Workload("cpu_ref_fp32", "fp32", 1, 8, 1024, 1024, 64, seed=1,
             note="CPU reference path: non-causal fp32, default scale"),
    Workload("sdxl_self_fp16", "fp16", 2, 10, 4096, 4096, 64, scale=1 / 8, seed=2,
             note="SDXL UNet self-attention (64x64 latent), CFG pair"),
    Workload("sdxl_cross_fp16", "fp16", 2, 10, 4096, 77, 64, scale=1 / 8, kv_std=0.5, seed=3,
             note="SDXL UNet cross-attention, 77 text tokens, K/V std 0.5"),
    Workload("qwen3_prefill_bf16", "bf16", 4, 16, 2048, 2048, 128, causal=True,
             scale=1 / math.sqrt(128), seed=4,
             note="Qwen3-0.6B-style causal prefill, KV heads repeat_interleaved 8->16"),
    Workload("sd15_self_fp32", "fp32", 2, 8, 4096, 4096, 40, scale=1 / math.sqrt(40), seed=5,
             note="SD1.5 UNet self-attention on the fp32 path, D=40"),
]
# Measured beside BASELINE's configs (bench.py --workload NAME), not part of them.
EXTRA_WORKLOADS = [
    Workload("qwen3_decode_bf16", "bf16", 16, 16, 1, 4096, 128, scale=1 / math.sqrt(128), seed=6,
             Hkv=8, note="Qwen3-0.6B-style decode step: 16 query heads over 8 K/V heads "
                         "(native GQA), 4096-token KV cache, non-causal"),
    # head dims that are not a whole number of 16-byte chunks: run in place on
    # the element-granular kernel variants (one kernel per call, no copies)
    Workload("odd_dim_fp16", "fp16", 1, 8, 2048, 2048, 100, seed=7,
             note="head dim 100 (not a multiple of 8 halves), fp16, non-causal"),
    Workload("odd_dim_fp32", "fp32", 1, 8, 1024, 1024, 33, seed=8,
             note="head dim 33 (not a multiple of 4 floats), fp32, non-causal"),
    # head dims above 128 (one workgroup per CU): grouped-query decode steps
    # whose few blocks are key-split and whose query heads are packed per K/V head
    Workload("gqa_decode_d160_bf16", "bf16", 16, 16, 1, 4096, 160, seed=9, Hkv=8,
             note="decode step at the reference's largest tabled head dim (160): "
                  "16 query heads over 8 K/V heads, 4096-token KV cache"),
    Workload("long_decode_d256_bf16", "bf16", 1, 16, 1, 16384, 256, seed=10, Hkv=8,
             note="single-sequence decode, head dim 256, 16 query heads over 8 K/V "
                  "heads, 16384-token KV cache"),
    Workload("prefill_d256_bf16", "bf16", 1, 16, 4096, 4096, 256, causal=True, seed=11, Hkv=8,
             note="causal prefill at head dim 256: 16 query heads over 8 K/V heads, "
                  "4096 tokens (the training pair's head-dim > 128 buckets with --backward)"),
]
BY_NAME = {w.name: w for w in WORKLOADS + EXTRA_WORKLOADS}

# The workload the headline metric is quoted on.
HEADLINE = BY_NAME["sdxl_self_fp16"]

# MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s).
PEAK_TFLOPS = {"fp16": 2516.6, "bf16": 2516.6, "fp32": 157.3}
PEAK_HBM_GBS = 8000.0
