"""GPU parity of attention with an explicit attn_mask (torch SDPA semantics).

A bool mask keeps the (query, key) pairs where it is True; a float mask
(f16/bf16/f32) is added to scale * Q K^T, -inf dropping the pair; masks
broadcast to [B, H, Sq, Sk]; a row whose keys are all dropped gives zeros.
Checked through the C ABI (cmpext3_attn_fwd_masked) and through
F.scaled_dot_product_attention against the float64 oracle with the same mask
(oracle/sdpa_oracle.py sdpa_np, pinned to torch in tests/test_oracle.py), at
the usual bar: max abs error <= 1e-2 fp16, 2e-2 bf16.

Shapes cover short key sweeps (the pipelined kernel takes every masked call),
odd tile counts, the key split (parts of a row merge masked partials, some of
them empty), grouped-query K/V, head dims below their bucket, and mask
layouts the ABI cannot read in place (transposed, key count not a multiple
of 4), which the bindings copy.  With is_causal a pair must be causally
visible and kept by the mask (torch's CPU rule; the oracle is pinned to it in
tests/test_oracle.py).  fp32 calls run the fp32 kernel's mask path and head
dims above 128 the wide kernel's (bar 1e-4 for fp32).
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
TDT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _inputs(dtype, B, H, Sq, Sk, D, seed, Hkv=None):
    q = W.Workload("mq", dtype, B, H, Sq, Sk, D, seed=seed).make_inputs("cuda")[0]
    _, k, v = W.Workload("mk", dtype, B, Hkv or H, Sq, Sk, D, seed=seed + 1).make_inputs("cuda")
    return q, k, v


def _mask(kind, dtype, B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool_pad":                    # key padding, [B,1,1,Sk]
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 1 - (17 * (b + 1)) % Sk:] = False
    elif kind == "bool_full":                 # per (b, h, query), one row fully dropped
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
        m[0, 0, min(5, Sq - 1)] = False
    elif kind == "add_heads":                 # additive, per head, query dtype, some -inf
        m = (torch.randn(1, H, Sq, Sk, generator=g) * 2).to(TDT[dtype])
        m[..., ::7] = -math.inf
    elif kind == "add_2d_f32":                # additive fp32 [Sq, Sk], causal-like -inf band
        m = torch.randn(Sq, Sk, generator=g)
        m = m.masked_fill(torch.ones(Sq, Sk, dtype=torch.bool).triu(Sk // 2 + 1), -math.inf)
    else:
        raise ValueError(kind)
    return m.cuda()


CASES = [
    # dtype, B, H, Sq, Sk, D
    ("fp16", 2, 3, 100, 77, 64),      # short keys
    ("bf16", 1, 2, 130, 300, 128),    # odd tile count
    ("fp16", 1, 2, 256, 2048, 64),    # key split, 8 parts
    ("bf16", 2, 2, 200, 1000, 40),    # D below its bucket, key split
    ("fp32", 2, 3, 100, 77, 64),      # fp32 kernel, short keys
    ("fp32", 1, 2, 130, 300, 40),     # fp32, the SD1.5 head dim
    ("fp32", 1, 2, 256, 2048, 64),    # fp32 key split
    ("fp16", 1, 2, 130, 300, 160),    # head dims above 128
    ("bf16", 1, 2, 64, 2048, 256),    # above 128, key split merged by the whole workgroup
    ("bf16", 2, 2, 200, 700, 192),
]
KINDS = ["bool_pad", "bool_full", "add_heads", "add_2d_f32"]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}" for c in CASES])
def test_mask_parity(case, kind, causal):
    dtype, B, H, Sq, Sk, D = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk)
    m = _mask(kind, dtype, B, H, Sq, Sk, seed=D)
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, causal, attn_mask=m)
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), scale, causal=causal, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


BCAST = [
    # dtype, B, H, Sq, Sk, D, causal, mask: masks that are the same for every
    # query row (key padding, per-head biases, a single query row) and are
    # read in whole runs: their tile slices ride the pipelined kernel's LDS
    # ring (D = 32/64/128 buckets)
    ("fp16", 2, 3, 300, 1000, 64, False, "pad_bool"),
    ("bf16", 1, 4, 200, 777, 128, True, "head_bias_bf16"),     # [1,H,1,Sk] expanded, ragged Sk
    ("fp16", 2, 2, 130, 2056, 32, False, "pad_f32"),           # additive fp32, key split
    ("bf16", 2, 4, 1, 4096, 128, False, "row_bool"),           # one query row, [B,H,1,Sk]
    ("fp16", 1, 2, 96, 520, 80, True, "pad_bool"),             # 96 bucket: register-staged loads
]


@pytest.mark.parametrize("case", BCAST, ids=[f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}{'c' if c[6] else ''}-{c[7]}"
                                             for c in BCAST])
def test_query_broadcast_masks(case):
    dtype, B, H, Sq, Sk, D, causal, kind = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk + D)
    g = torch.Generator().manual_seed(Sk)
    if kind == "pad_bool":
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 37 * (b + 1):] = False
            m[b, ..., 3] = False
    elif kind == "head_bias_bf16":
        m = (torch.randn(1, H, 1, Sk, generator=g) * 3).bfloat16()
        m[..., 5::7] = -math.inf
        m = m.expand(B, H, Sq, Sk)
    elif kind == "pad_f32":
        m = torch.zeros(B, 1, 1, Sk)
        m[..., -100:] = -math.inf
        m[0, ..., :40] = -2.5
    else:
        m = torch.rand(B, H, 1, Sk, generator=g) > 0.5
        m[..., 0] = True
    m = m.cuda()
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, causal, attn_mask=m)
    again = abi.attn_fwd(q, k, v, scale, causal, attn_mask=m)
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), scale, causal=causal, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]
    assert torch.equal(out, again)


def test_fully_masked_rows_are_zero():
    q, k, v = _inputs("fp16", 1, 2, 64, 600, 64, seed=3)
    m = torch.ones(1, 2, 64, 600, dtype=torch.bool, device="cuda")
    m[:, :, 10] = False                    # whole row dropped (every key-split part empty)
    m[:, 1, 20, :300] = False              # first half dropped: one part empty, one not
    out = abi.attn_fwd(q, k, v, 0.125, False, attn_mask=m)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[:, :, 10]) == 0
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["fp16"]


def test_mask_with_grouped_query_heads():
    q, k, v = _inputs("bf16", 1, 8, 128, 512, 64, seed=9, Hkv=2)
    m = _mask("bool_full", "bf16", 1, 8, 128, 512, seed=4)
    out = abi.attn_fwd(q, k, v, 0.125, False, attn_mask=m)
    torch.cuda.synchronize()
    kr, vr = k.cpu().repeat_interleave(4, dim=1), v.cpu().repeat_interleave(4, dim=1)
    ref = orc.sdpa_np(q.cpu(), kr, vr, 0.125, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["bf16"]


NARROW = [
    # dtype, B, H, Sq, Sk, D, layout
    ("fp16", 2, 10, 256, 77, 64, "pad"),     # [B,1,1,77] bool text padding (SDXL cross-attention)
    ("bf16", 1, 4, 100, 300, 128, "rows"),   # [1,1,Sq,300] additive bf16, rows 600 bytes apart
    ("fp32", 2, 2, 70, 123, 40, "offset"),   # additive f32 starting one element into its buffer
    ("fp16", 1, 2, 64, 999, 256, "pad"),     # head dim above 128
    ("fp32", 1, 2, 40, 45, 64, "pad"),       # fp32, bool padding
]


def _narrow_mask(layout, dtype, B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    if layout == "pad":
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 1 - (13 * (b + 1)) % Sk:] = False
        return m.cuda()
    if layout == "rows":
        return (torch.randn(1, 1, Sq, Sk, generator=g) * 2).to(TDT[dtype]).cuda()
    buf = torch.randn(Sq * Sk + 1, generator=g)
    buf[1::5] = -math.inf
    return buf.cuda()[1:].view(1, 1, Sq, Sk)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", NARROW, ids=[f"{c[0]}-{c[6]}-k{c[4]}d{c[5]}" for c in NARROW])
def test_masks_read_in_place_element_by_element(case, causal, run_without_copies):
    """Masks whose rows are not whole runs of 8 keys (a key count that is not
    a multiple of 8, row strides or a base off 16 bytes) are read in place,
    element by element: the binding makes no copy, and nothing past the last
    key of a row is read."""
    dtype, B, H, Sq, Sk, D, layout = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sk + D)
    m = _narrow_mask(layout, dtype, B, H, Sq, Sk, seed=D)
    out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, 0.1, causal, m))
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.1, causal=causal, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


NARROW_ROWS = [
    # dtype, B, H, Sq, Sk, D: rows of 4- or 8-byte pieces, not whole 16-byte chunks
    ("fp16", 2, 3, 150, 500, 100),   # 200-byte rows: 8-byte pieces, pipelined kernel
    ("bf16", 1, 4, 96, 333, 70),     # 140-byte rows: 4-byte pieces
    ("fp16", 1, 2, 80, 700, 132),    # above 128: the wide kernel's narrow rows
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", NARROW_ROWS, ids=[f"{c[0]}-d{c[5]}" for c in NARROW_ROWS])
def test_masked_rows_of_narrow_pieces_run_in_place(case, causal, run_without_copies):
    """Masked f16/bf16 calls whose head dim is not whole 16-byte chunks run on
    the narrow-row kernels in place (no padded copy of Q, K, V or O)."""
    dtype, B, H, Sq, Sk, D = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=D + Sk)
    m = _mask("bool_full", dtype, B, H, Sq, Sk, seed=D)
    out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, 0.09, causal, m))
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.09, causal=causal, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


def test_mask_layouts_that_need_a_copy():
    """A transposed mask view (key stride not 1) and a key count that is not
    a multiple of 4."""
    q, k, v = _inputs("fp16", 1, 2, 96, 301, 64, seed=12)
    base = torch.randn(2, 301, 96, device="cuda").to(torch.float16)
    m = base.transpose(1, 2)[None]           # [1, 2, 96, 301], key stride 96
    assert m.stride(-1) != 1
    out = abi.attn_fwd(q, k, v, 0.125, False, attn_mask=m)
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["fp16"]


@pytest.mark.parametrize("dtype,D", [("fp32", 64), ("fp16", 256)])
def test_fully_masked_rows_are_zero_on_every_kernel(dtype, D):
    q, k, v = _inputs(dtype, 1, 2, 64, 600, D, seed=4)
    m = torch.ones(1, 2, 64, 600, dtype=torch.bool, device="cuda")
    m[:, :, 10] = False
    m[:, 1, 20, :300] = False
    out = abi.attn_fwd(q, k, v, 0.1, False, attn_mask=m)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[:, :, 10]) == 0
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.1, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_masked_sdpa_runs_native(patched, dtype):
    q, k, v = _inputs(dtype, 2, 4, 200, 333, 64, seed=21)
    m = _mask("bool_pad", dtype, 2, 4, 200, 333, seed=1)
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
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=m)
    finally:
        cmpext3._C = old
    torch.cuda.synchronize()
    assert calls["n"] == 1
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), None, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


def test_fp32_masked_sdpa_runs_native(patched):
    """fp32 with a mask goes to the native op (one call) and meets the fp32 bar."""
    q, k, v = (torch.randn(1, 2, 50, 64, device="cuda") for _ in range(3))
    m = torch.rand(50, 50, device="cuda") > 0.5
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
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=m)
    finally:
        cmpext3._C = old
    torch.cuda.synchronize()
    assert calls["n"] == 1
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), None, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["fp32"]