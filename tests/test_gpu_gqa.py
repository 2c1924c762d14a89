"""GPU parity of grouped-query attention (K/V with fewer heads than Q).

cmpext3_attn_fwd_gqa reads K/V head h / (H / H_kv) for query head h, torch's
scaled_dot_product_attention(..., enable_gqa=True) semantics.  The oracle is
float64 SDPA on the CPU over K/V repeated per query head
(repeat_interleave on the head dim), with the usual bar: max abs error
<= 1e-2 fp16, 2e-2 bf16, 1e-4 fp32.  Covers all three kernels (short key
sweeps and fp32 on their own kernels, long ones on the pipelined kernel,
with and without the key split), causal masking, strided K/V and the
drop-in path through F.scaled_dot_product_attention.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import cmpext3
from cmpext3 import abi
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE


def _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed):
    q = W.Workload("gq", dtype, B, H, Sq, Sk, D, seed=seed).make_inputs("cuda")[0]
    _, k, v = W.Workload("gk", dtype, B, Hkv, Sq, Sk, D, seed=seed + 1).make_inputs("cuda")
    return q, k, v


def _oracle(q, k, v, scale, causal):
    g = q.shape[1] // k.shape[1]
    kr = k.cpu().repeat_interleave(g, dim=1)
    vr = v.cpu().repeat_interleave(g, dim=1)
    return orc.sdpa_np(q.cpu(), kr, vr, scale, causal)


CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D
    ("fp16", 2, 8, 2, 100, 90, 64),      # short keys: v2 kernel
    ("fp16", 1, 8, 1, 200, 600, 64),     # multi-query, pipelined kernel, key split
    ("bf16", 2, 6, 3, 150, 700, 128),
    ("bf16", 1, 16, 8, 256, 2048, 128),  # Qwen-like grouping, key split
    ("fp16", 1, 4, 2, 64, 300, 160),     # head dim above 128: v2 kernel
    ("fp32", 1, 8, 4, 67, 130, 40),      # fp32 kernel
    ("fp32", 2, 4, 1, 129, 64, 64),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}" for c in CASES])
def test_gqa_parity(case, causal):
    dtype, B, H, Hkv, Sq, Sk, D = case
    q, k, v = _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=Sq + Sk)
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, causal)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, scale, causal)) <= TOL[dtype]


def test_gqa_strided_kv():
    """K/V sliced out of longer, head-interleaved buffers ([B,S,Hkv,D] memory)."""
    B, H, Hkv, S, D = 1, 8, 2, 400, 64
    q = W.Workload("gq", "fp16", B, H, S, S, D, seed=3).make_inputs("cuda")[0]
    big_k = torch.randn(B, S + 64, Hkv, D, dtype=torch.float16, device="cuda")
    big_v = torch.randn(B, S + 64, Hkv, D, dtype=torch.float16, device="cuda")
    k = big_k[:, 32:32 + S].transpose(1, 2)
    v = big_v[:, 32:32 + S].transpose(1, 2)
    assert not k.is_contiguous()
    out = abi.attn_fwd(q, k, v, 0.125, True)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, 0.125, True)) <= TOL["fp16"]


def test_gqa_through_patched_sdpa(patched):
    """F.scaled_dot_product_attention(..., enable_gqa=True) stays on the native
    kernel and matches torch's own GQA result on the same inputs."""
    q, k, v = _gqa_inputs("bf16", 1, 8, 2, 128, 512, 64, seed=11)
    calls = {"n": 0}
    real = cmpext3._C

    class Counting:
        @staticmethod
        def attention(*args):
            calls["n"] += 1
            return real.attention(*args)

    old = cmpext3._C
    cmpext3._C = Counting
    try:
        with torch.inference_mode():
            out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    finally:
        cmpext3._C = old
    torch.cuda.synchronize()
    assert calls["n"] == 1
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, None, True)) <= TOL["bf16"]


def test_mismatched_heads_without_gqa_still_raise(patched):
    q, k, v = _gqa_inputs("fp16", 1, 4, 2, 32, 32, 64, seed=1)
    with pytest.raises(RuntimeError):
        F.scaled_dot_product_attention(q, k, v)


PACKED = [
    # dtype, B, H, Hkv, Sq, Sk, D: short query sweeps, packed G query heads per K/V head
    ("bf16", 4, 32, 8, 1, 4096, 128),    # decode step, key split
    ("fp16", 2, 16, 2, 5, 700, 64),      # ragged rows per head, 8 heads per group
    ("fp16", 1, 8, 4, 64, 333, 64),      # the largest packed Sq
    ("bf16", 1, 12, 3, 7, 2048, 96),     # head dim below its bucket
    ("bf16", 1, 32, 8, 1, 32768, 128),   # long-context decode: 64 key parts, 3 of 4 waves rowless
]


@pytest.mark.parametrize("case", PACKED, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}" for c in PACKED])
def test_gqa_packed_query_heads(case):
    """Grouped-query launches with short query sweeps pack each group's query
    heads into the rows of one problem (K/V streamed once per group)."""
    dtype, B, H, Hkv, Sq, Sk, D = case
    q, k, v = _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=Sq * 3 + Sk)
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, False)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), _oracle(q, k, v, scale, False)) <= TOL[dtype]


def test_gqa_packed_strided_query_and_output():
    """Packed rows with [B,S,H,D]-memory query and output views."""
    B, H, Hkv, Sq, Sk, D = 2, 8, 2, 3, 640, 64
    g = torch.Generator().manual_seed(17)
    q = torch.randn(B, Sq, H, D, generator=g).half().cuda().transpose(1, 2)
    k = torch.randn(B, Hkv, Sk, D, generator=g).half().cuda()
    v = torch.randn(B, Hkv, Sk, D, generator=g).half().cuda()
    o = torch.empty(B, Sq, H, D, dtype=torch.float16, device="cuda").transpose(1, 2)
    assert abi.attn_fwd_raw(q, k, v, o, 0.125, False) == abi.OK
    torch.cuda.synchronize()
    assert orc.max_abs_err(o.cpu(), _oracle(q, k, v, 0.125, False)) <= TOL["fp16"]


MASKED = [
    # dtype, B, H, Hkv, Sq, Sk, D, mask shape (None = full [B, H, Sq, Sk])
    ("fp16", 2, 6, 2, 150, 260, 64, None),
    ("bf16", 1, 8, 2, 40, 1500, 128, (1, 8, 40, 1500)),   # short query sweep: masks are never packed
    ("fp16", 1, 4, 1, 96, 900, 64, (96, 900)),            # 2-D mask, multi-query, key split
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", MASKED, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}" for c in MASKED])
def test_gqa_with_attention_mask(case, causal):
    """Grouped-query K/V together with an attention mask: the mask indexes
    query heads, K/V head h / (H / H_kv) serves query head h."""
    dtype, B, H, Hkv, Sq, Sk, D, mshape = case
    q, k, v = _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=Sq * 3 + Sk)
    g = torch.Generator().manual_seed(D + Sk)
    if mshape is None:
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.25
        m[..., 0] = True
    else:
        m = (torch.randn(*mshape, generator=g) * 1.5).to(q.dtype)
        m[..., 2::7] = -math.inf
    m = m.cuda()
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, causal, attn_mask=m)
    torch.cuda.synchronize()
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    want = orc.sdpa_np(q.cpu(), kr, vr, scale, causal, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), want) <= TOL[dtype]
