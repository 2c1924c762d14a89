#!/usr/bin/env python3
"""Writes tests/golden/sdpa_golden.npz: small SDPA known-answer vectors.

The reference ships no golden vectors for attention (its numeric checks are
GPU-only cosine thresholds, tests_hardware/test_attention_causal.py:103-110),
so these are produced from PyTorch alone: torch's MATH backend of
F.scaled_dot_product_attention in float64 on the CPU, on seeded inputs
rounded to each case's dtype.  Nothing from the reference is imported or run.

Each case stores q, k, v (the dtype-rounded values, as float32), the scale,
the causal flag and the float64 expected output.

Run: python tests/golden/make_golden.py   (deterministic; overwrites the file)
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sdpa_golden.npz")

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}

# name, dtype, B, H, Sq, Sk, D, causal, scale (None = 1/sqrt(D)), kv_std
CASES = [
    ("f32_q67_k67_d40", "fp32", 1, 2, 67, 67, 40, False, None, 1.0),
    ("f16_q64_k77_d64_cross", "fp16", 1, 2, 64, 77, 64, False, 0.125, 0.5),
    ("bf16_q96_k96_d128_causal", "bf16", 1, 2, 96, 96, 128, True, None, 1.0),
    ("f16_q40_k90_d32_causal_sq_lt_sk", "fp16", 1, 1, 40, 90, 32, True, None, 1.0),
    ("bf16_q90_k40_d32_causal_sq_gt_sk", "bf16", 1, 1, 90, 40, 32, True, None, 1.0),
    ("f16_q5_k1_d64_single_key", "fp16", 2, 1, 5, 1, 64, False, None, 1.0),
    ("f32_q33_k50_d24_negscale", "fp32", 1, 2, 33, 50, 24, False, -0.3, 1.0),
    ("f16_q17_k17_d16_zero_scale_causal", "fp16", 1, 1, 17, 17, 16, True, 0.0, 1.0),
]


def make_case(dtype, B, H, Sq, Sk, D, causal, scale, kv_std, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g)
    k = torch.randn(B, H, Sk, D, generator=g) * kv_std
    v = torch.randn(B, H, Sk, D, generator=g) * kv_std
    q, k, v = (t.to(DT[dtype]).to(torch.float64) for t in (q, k, v))
    s = scale if scale is not None else 1.0 / math.sqrt(D)
    with sdpa_kernel(SDPBackend.MATH):
        o = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=s)
    return q, k, v, s, o


def main() -> None:
    arrays = {}
    for i, (name, dtype, B, H, Sq, Sk, D, causal, scale, kv_std) in enumerate(CASES):
        q, k, v, s, o = make_case(dtype, B, H, Sq, Sk, D, causal, scale, kv_std, seed=1000 + i)
        arrays[f"{name}/q"] = q.numpy().astype(np.float32)
        arrays[f"{name}/k"] = k.numpy().astype(np.float32)
        arrays[f"{name}/v"] = v.numpy().astype(np.float32)
        arrays[f"{name}/o"] = o.numpy()
        arrays[f"{name}/meta"] = np.array([s, float(causal)], dtype=np.float64)
        arrays[f"{name}/dtype"] = np.array(dtype)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(CASES)} cases, {os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
