"""GPU parity of the training pair at head dims above 128: the forward that
keeps the row log-sum-exp (cmpext3_attn_fwd_lse, in its 192 and 256 buckets:
the pipelined kernel for prefills of more than 64 rows and 256+ keys, key
split included, else the head-dim > 128 kernel) and the backward
(cmpext3_attn_bwd, gradient kernels in the 192 and 256 buckets at one wave per
SIMD), through the C ABI, plus the autograd Function and the SDPA route.

Oracle and bars as in test_gpu_backward.py: float64 restatements in
oracle/sdpa_oracle.py; forward output and log-sum-exp max abs error <= 1e-2
fp16 / 2e-2 bf16; each gradient's max abs error <= the same numbers times
max |oracle| of that gradient (at least 1e-3).  Head dims below a bucket (136,
160, 200) check the zero-padded columns; ragged sequence lengths, one query
row, one key, negative and zero scales, causal with Sq < Sk and Sq > Sk,
grouped-query K/V, masks and [B,S,H,D] views are covered.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import cmpext3
from cmpext3 import abi
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = {"fp16": 1e-2, "bf16": 2e-2}
TDT = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _t(dtype, B, H, S, D, g, amp=1.0):
    return (torch.randn(B, H, S, D, generator=g) * amp).to(TDT[dtype]).cuda()


def _rel_err(got, want):
    want = torch.as_tensor(want)
    return orc.max_abs_err(got.cpu(), want) / max(float(want.abs().max()), 1e-3)


def _check(dtype, q, k, v, do, out, lse, grads, s, causal, mask=None):
    """Compare (out, lse, dq, dk, dv) with the oracle on K/V repeated per query
    head (dK/dV of a K/V head sum its query heads' contributions)."""
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    qc, dc = q.cpu(), do.cpu()
    mc = None if mask is None else mask.cpu()
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kr, vr, s, causal, attn_mask=mc)) <= TOL[dtype]
    assert orc.max_abs_err(lse.cpu(), orc.sdpa_lse_np(qc, kr, s, causal, attn_mask=mc)) <= TOL[dtype]
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(qc, kr, vr, dc, s, causal, attn_mask=mc)
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, ref in zip(("dq", "dk", "dv"), grads, (dq_r, dk_r, dv_r)):
        assert _rel_err(got, ref) <= TOL[dtype], name


CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D, causal, scale (None = 1/sqrt(D))
    ("bf16", 1, 2, 2, 200, 300, 256, False, None),
    ("fp16", 2, 2, 2, 130, 257, 160, True, None),     # ragged, causal Sq < Sk, 192 bucket
    ("bf16", 1, 1, 1, 300, 130, 192, True, None),     # causal Sq > Sk
    ("fp16", 1, 2, 2, 64, 1000, 136, False, None),    # D = 136 (192 bucket), many key blocks
    ("bf16", 2, 1, 1, 1, 33, 256, False, None),       # one query row
    ("fp16", 1, 1, 1, 37, 1, 200, True, None),        # one key, D = 200 (256 bucket)
    ("fp16", 1, 2, 2, 96, 160, 256, False, -0.07),    # negative scale
    ("bf16", 1, 2, 2, 100, 200, 192, False, 0.0),     # scale 0: uniform P, no score gradient
    ("bf16", 1, 8, 2, 150, 260, 256, True, None),     # grouped-query K/V
    ("fp16", 1, 4, 1, 100, 300, 160, False, None),    # multi-query
    ("bf16", 1, 4, 4, 1024, 1024, 256, True, None),   # a long causal sweep
    ("fp16", 1, 2, 2, 512, 4096, 200, False, None),   # pipelined forward, key split (8 blocks x 16 parts)
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}{'c' if c[7] else ''}"
                                             f"{'' if c[8] is None else 's' + str(c[8])}" for c in CASES])
def test_wide_training_pair(case):
    dtype, B, H, Hkv, Sq, Sk, D, causal, scale = case
    print(f"wide training pair {case}", flush=True)
    g = torch.Generator().manual_seed(Sq * 7 + Sk + D)
    q, k, v, do = _t(dtype, B, H, Sq, D, g), _t(dtype, B, Hkv, Sk, D, g), _t(dtype, B, Hkv, Sk, D, g), \
        _t(dtype, B, H, Sq, D, g)
    s = D ** -0.5 if scale is None else scale
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal)
    grads = abi.attn_bwd(q, k, v, out, do, lse, s, causal)
    torch.cuda.synchronize()
    _check(dtype, q, k, v, do, out, lse, grads, s, causal)


def test_wide_training_forward_matches_inference_forward():
    """The training forward's output is the inference forward's within the
    forward bar (different buckets and plans, same attention)."""
    g = torch.Generator().manual_seed(21)
    q, k, v = (_t("bf16", 1, 8, 512, 160, g) for _ in range(3))
    out, _ = abi.attn_fwd_lse(q, k, v, 0.08, False)
    ref = abi.attn_fwd(q, k, v, 0.08, False)
    torch.cuda.synchronize()
    assert float((out.float() - ref.float()).abs().max()) <= TOL["bf16"]


def test_wide_bwd_is_deterministic():
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (_t("fp16", 2, 2, 300, 256, g) for _ in range(4))
    out, lse = abi.attn_fwd_lse(q, k, v, 0.0625, True)
    first = abi.attn_bwd(q, k, v, out, do, lse, 0.0625, True)
    second = abi.attn_bwd(q, k, v, out, do, lse, 0.0625, True)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_wide_bwd_strided_views():
    """[B,S,H,D] memory viewed as [B,H,S,D] for every operand and gradient."""
    B, S, H, D = 1, 192, 3, 192
    g = torch.Generator().manual_seed(3)
    mk = lambda: torch.randn(B, S, H, D, generator=g).half().cuda().transpose(1, 2)
    q, k, v, do = mk(), mk(), mk(), mk()
    assert not q.is_contiguous()
    out, lse = abi.attn_fwd_lse(q, k, v, 0.07, True)
    dq, dk, dv = (torch.empty(B, S, H, D, dtype=torch.float16, device="cuda").transpose(1, 2)
                  for _ in range(3))
    delta = torch.empty(B, H, S, device="cuda")
    assert abi.attn_bwd_raw(q, k, v, out, do, lse, dq, dk, dv, delta, 0.07, True) == abi.OK
    torch.cuda.synchronize()
    _check("fp16", q, k, v, do, out, lse, (dq, dk, dv), 0.07, True)


def _mask(kind, B, H, Sq, Sk, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool_pad":                    # key padding [B,1,1,Sk]
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 1 - (11 * (b + 1)) % Sk:] = False
    elif kind == "bool_full":                 # per (b, h, query), key 0 kept
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
        m[..., 0] = True
    else:                                     # additive in the query dtype, -inf entries
        m = (torch.randn(1, H, Sq, Sk, generator=g) * 2).to(TDT[dtype])
        m[..., 1::5] = -math.inf
    return m.cuda()


MASK_CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D, kind
    ("bf16", 2, 2, 2, 160, 300, 256, "bool_pad"),
    ("fp16", 1, 2, 2, 300, 2048, 192, "add_heads"),   # pipelined forward, key split when non-causal
    ("fp16", 1, 4, 2, 120, 264, 192, "bool_full"),
    ("bf16", 1, 2, 1, 90, 200, 160, "add_heads"),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", MASK_CASES, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}-{c[7]}"
                                                  for c in MASK_CASES])
def test_wide_masked_training_pair(case, causal):
    dtype, B, H, Hkv, Sq, Sk, D, kind = case
    print(f"wide masked training pair {case} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(H * Sq + Sk + D)
    q, k, v, do = _t(dtype, B, H, Sq, D, g), _t(dtype, B, Hkv, Sk, D, g), _t(dtype, B, Hkv, Sk, D, g), \
        _t(dtype, B, H, Sq, D, g)
    m = _mask(kind, B, H, Sq, Sk, dtype, seed=Sk)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal, attn_mask=m)
    grads = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m)
    torch.cuda.synchronize()
    _check(dtype, q, k, v, do, out, lse, grads, s, causal, mask=m)


def test_wide_sdpa_training_route(patched):
    """enable_backward(): SDPA with live autograd at D = 256 (grouped-query,
    causal) runs the native pair; the gradients match the oracle."""
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 8, 160, 256, generator=g).bfloat16().cuda().requires_grad_(True)
    k = torch.randn(1, 2, 160, 256, generator=g).bfloat16().cuda().requires_grad_(True)
    v = torch.randn(1, 2, 160, 256, generator=g).bfloat16().cuda().requires_grad_(True)
    do = torch.randn(1, 8, 160, 256, generator=g).bfloat16().cuda()
    was = cmpext3.backward_enabled()
    cmpext3.enable_backward(True)
    try:
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
        assert out.grad_fn is not None and "_Attention" in type(out.grad_fn).__name__
        out.backward(do)
    finally:
        cmpext3.enable_backward(was)
    torch.cuda.synchronize()
    kr, vr = (t.detach().cpu().repeat_interleave(4, dim=1) for t in (k, v))
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(q.detach().cpu(), kr, vr, do.cpu(), None, True)
    assert _rel_err(q.grad, dq_r) <= TOL["bf16"]
    assert _rel_err(k.grad, dk_r.reshape(1, 2, 4, 160, 256).sum(axis=2)) <= TOL["bf16"]
    assert _rel_err(v.grad, dv_r.reshape(1, 2, 4, 160, 256).sum(axis=2)) <= TOL["bf16"]


def test_wide_autograd_function_with_odd_head_dim():
    """D = 129 (not whole chunks): the binding pads to 136 and the kernels run
    the 192 bucket; gradients come back at D = 129."""
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 2, 150, 129, generator=g).half().cuda().requires_grad_(True) for _ in range(3))
    do = torch.randn(1, 2, 150, 129, generator=g).half().cuda()
    out = cmpext3.attention(q, k, v, None, True)
    out.backward(do)
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), do.cpu(), None, True)
    for got, ref in zip((q.grad, k.grad, v.grad), want):
        assert got.shape == (1, 2, 150, 129)
        assert _rel_err(got, ref) <= TOL["fp16"]
