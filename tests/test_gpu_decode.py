"""GPU parity of the decode kernel (attn_fwd_decode16.hip).

Decode-shaped launches (non-causal, unmasked inference with at most 16 query
rows per K/V head once grouped query heads are packed) run on a kernel whose
waves each stream their own 16-key tiles: at D = 160, 192, 224, 256 always,
at D = 64, 96, 128 when the (batch, K/V head) units fill less than half of
the CUs.  The oracle is float64 SDPA on the CPU over
K/V repeated per query head, with the usual bar (max abs error <= 1e-2 fp16,
2e-2 bf16).  Covers ragged key counts (one key, fewer than a tile, a tile
and one), 1 to 16 rows, grouped and multi-query K/V, negative and zero
scales, [B,S,H,D] views, the key split against the unsplit launch,
bit-identical reruns of the split, and the two-level merge of deep splits
(up to 128 parts, a last group shorter than the others).
"""
from __future__ import annotations

import math

import pytest
import torch

from cmpext3 import abi
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE


def _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed, layout="bhsd"):
    q = W.Workload("dq", dtype, B, H, Sq, Sk, D, seed=seed).make_inputs("cuda", layout=layout)[0]
    _, k, v = W.Workload("dk", dtype, B, Hkv, Sq, Sk, D, seed=seed + 1).make_inputs("cuda", layout=layout)
    return q, k, v


def _oracle(q, k, v, scale):
    g = q.shape[1] // k.shape[1]
    return orc.sdpa_np(q.cpu(), k.cpu().repeat_interleave(g, dim=1), v.cpu().repeat_interleave(g, dim=1),
                       scale, False)


CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D
    ("bf16", 1, 16, 8, 1, 16384, 256),   # long single-sequence decode (bench workload)
    ("bf16", 16, 16, 8, 1, 4096, 160),   # batched grouped-query decode (bench workload)
    ("fp16", 2, 8, 8, 1, 1000, 192),     # multi-head, ragged key count
    ("fp16", 1, 4, 1, 4, 77, 224),       # multi-query, 4 positions x 4 heads = 16 rows
    ("bf16", 3, 6, 2, 5, 33, 256),       # 15 rows, two tiles and one key
    ("fp16", 1, 2, 2, 16, 1, 160),       # one key
    ("fp16", 1, 2, 2, 1, 15, 256),       # fewer keys than a tile
    ("bf16", 1, 8, 8, 16, 5000, 192),    # 16 rows without grouping
    ("fp16", 4, 32, 4, 2, 2048, 256),    # G = 8, 2 positions
    ("bf16", 1, 32, 8, 4, 8192, 128),    # D = 128, 8 units of 16 rows (speculative block)
    ("fp16", 2, 16, 4, 1, 20000, 64),    # D = 64, 8 units, long cache
    ("fp16", 1, 12, 12, 3, 777, 96),     # D = 96, 12 units of 3 rows
]


def _describe(case):
    dtype, B, H, Hkv, Sq, Sk, D = case
    return abi.describe(abi.dtype_code(getattr(torch, {"fp16": "float16", "bf16": "bfloat16"}[dtype])),
                        B, Hkv, Sq * (H // Hkv), Sk, D)[1]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-b{c[1]}h{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}" for c in CASES])
def test_decode_parity(case):
    dtype, B, H, Hkv, Sq, Sk, D = case
    assert "decode16" in _describe(case)
    print(f"decode parity {case}", flush=True)
    q, k, v = _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=Sk + D)
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, False)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, scale)) <= TOL[dtype]


@pytest.mark.parametrize("scale", [-0.11, 0.0, 0.9])
def test_decode_scales(scale):
    q, k, v = _inputs("fp16", 2, 8, 2, 1, 3000, 256, seed=5)
    out = abi.attn_fwd(q, k, v, scale, False)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, scale)) <= TOL["fp16"]


def test_decode_bshd_views():
    """Q, K, V and O as [B,H,S,D] views of [B,S,H,D] memory: no copies."""
    q, k, v = _inputs("bf16", 2, 8, 4, 3, 2500, 192, seed=7, layout="bshd")
    assert not k.is_contiguous() and not q.is_contiguous()
    out = torch.empty(2, 3, 8, 192, dtype=torch.bfloat16, device="cuda").transpose(1, 2)
    rc = abi.attn_fwd_raw(q, k, v, out, 0.07, False)
    torch.cuda.synchronize()
    assert rc == 0
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, 0.07)) <= TOL["bf16"]


@pytest.mark.parametrize("D", [160, 256])
def test_decode_split_matches_unsplit_and_reruns_bit_identical(D):
    B, H, Hkv, Sq, Sk = 1, 8, 4, 1, 8192
    dt = abi.dtype_code(torch.float16)
    assert abi.plan(dt, B, H, Hkv, Sq, Sk, D, abi.workspace_size(dt, B, H, Hkv, Sq, Sk, D))[1] >= 2
    q, k, v = _inputs("fp16", B, H, Hkv, Sq, Sk, D, seed=11)
    split1 = torch.empty_like(q)
    split2 = torch.empty_like(q)
    whole = torch.empty_like(q)
    assert abi.attn_fwd_raw(q, k, v, split1, 0.1, False) == 0
    assert abi.attn_fwd_raw(q, k, v, split2, 0.1, False) == 0
    assert abi.attn_fwd_raw(q, k, v, whole, 0.1, False, workspace=False) == 0
    torch.cuda.synchronize()
    assert torch.equal(split1, split2)
    want = _oracle(q, k, v, 0.1)
    assert orc.max_abs_err(split1.cpu(), want) <= TOL["fp16"]
    assert orc.max_abs_err(whole.cpu(), want) <= TOL["fp16"]


DEEP = [
    # dtype, B, H, Hkv, Sq, Sk, D, merge groups: deep splits of many rows
    ("bf16", 1, 32, 4, 1, 65536, 256, 8),    # 4 units x 64 parts of 8 rows
    ("fp16", 1, 16, 1, 1, 65536, 256, 12),   # 1 unit x 128 parts (the most) of 16 rows, last group 8
    ("bf16", 5, 8, 1, 1, 20000, 256, 8),     # 5 units x 52 parts: a last group of 4, ragged keys
]


@pytest.mark.parametrize("case", DEEP, ids=[f"{c[0]}-b{c[1]}h{c[2]}of{c[3]}-k{c[5]}d{c[6]}" for c in DEEP])
def test_decode_two_level_merge(case):
    """Deep splits merge per group of parts, then over the groups: the output
    meets the oracle, a rerun is bit-identical (fixed groups and order, whichever
    part arrives last), and the unsplit launch agrees within the same bar."""
    dtype, B, H, Hkv, Sq, Sk, D, groups = case
    desc = _describe(case[:7])
    assert f"merged in groups of {groups}" in desc, desc
    print(f"decode two-level merge {case}", flush=True)
    q, k, v = _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=D + B)
    scale = 1.0 / math.sqrt(D)
    split1, split2, whole = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    assert abi.attn_fwd_raw(q, k, v, split1, scale, False) == 0
    assert abi.attn_fwd_raw(q, k, v, split2, scale, False) == 0
    assert abi.attn_fwd_raw(q, k, v, whole, scale, False, workspace=False) == 0
    torch.cuda.synchronize()
    assert torch.equal(split1, split2)
    want = _oracle(q, k, v, scale)
    assert orc.max_abs_err(split1.cpu(), want) <= TOL[dtype]
    assert orc.max_abs_err(whole.cpu(), want) <= TOL[dtype]


def test_seventeen_rows_stay_on_the_prefill_kernel():
    dt = abi.dtype_code(torch.bfloat16)
    assert "decode16" not in abi.describe(dt, 1, 8, 17, 4096, 256)[1]
    assert "decode16" not in abi.describe(dt, 16, 16, 1, 4096, 128)[1]  # 256 units: pipelined
    q, k, v = _inputs("bf16", 1, 8, 8, 17, 1500, 256, seed=13)
    out = abi.attn_fwd(q, k, v, 0.0625, False)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, 0.0625)) <= TOL["bf16"]
