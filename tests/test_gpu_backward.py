"""GPU parity of the training pair: the forward that keeps the row
log-sum-exp (cmpext3_attn_fwd_lse) and the backward (cmpext3_attn_bwd), both
through the C ABI, plus the autograd Function and the opt-in SDPA route.

Oracle: float64 restatements in oracle/sdpa_oracle.py (sdpa_np, sdpa_lse_np,
sdpa_bwd_np), pinned to torch autograd, finite differences and closed forms in
tests/test_oracle_bwd.py.  Bars, written here:
  * forward output: max abs error <= 1e-2 fp16, 2e-2 bf16 (the forward's bar);
  * log-sum-exp: max abs error <= 1e-2 fp16, 2e-2 bf16 (natural log);
  * gradients: max abs error <= 1e-2 (fp16) / 2e-2 (bf16) times max |oracle|
    of that gradient (at least 1e-3), i.e. the same numbers relative to each
    gradient's own scale (gradients, unlike attention outputs, are not bounded
    by the values of V; the floor covers gradients that are exactly zero, such
    as dQ and dK with a single key).
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


def _inputs(dtype, B, H, Sq, Sk, D, seed, amp=1.0):
    g = torch.Generator().manual_seed(seed)
    mk = lambda S: (torch.randn(B, H, S, D, generator=g) * amp).to(TDT[dtype]).cuda()
    q, k, v = mk(Sq), mk(Sk), mk(Sk)
    do = torch.randn(B, H, Sq, D, generator=g).to(TDT[dtype]).cuda()
    return q, k, v, do


def _rel_err(got, want):
    want = torch.as_tensor(want)
    return orc.max_abs_err(got.cpu(), want) / max(float(want.abs().max()), 1e-3)


CASES = [
    # dtype, B, H, Sq, Sk, D, causal, scale (None = 1/sqrt(D))
    ("fp16", 1, 2, 128, 128, 64, False, None),
    ("fp16", 2, 2, 200, 300, 64, True, None),     # ragged, causal Sq < Sk
    ("bf16", 1, 2, 300, 130, 64, True, None),     # causal Sq > Sk
    ("fp16", 1, 2, 256, 77, 128, False, None),    # short keys, D = 128
    ("bf16", 1, 3, 333, 257, 96, False, None),    # D below its 128 bucket
    ("fp16", 1, 1, 100, 500, 40, True, None),     # D = 40 (padded to 48 by the binding)
    ("fp16", 1, 2, 64, 1024, 64, False, -0.2),    # negative scale, key split in the forward
    ("bf16", 2, 1, 1, 33, 128, False, None),      # one query row
    ("fp16", 1, 1, 37, 1, 64, True, None),        # one key
    ("fp16", 1, 2, 100, 200, 64, False, 0.0),     # scale 0: uniform P, no score gradient
    ("bf16", 1, 1, 64, 96, 64, True, 1e-39),      # denormal scale (the kernel's c is floored)
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-q{c[3]}k{c[4]}d{c[5]}{'c' if c[6] else ''}"
                                             f"{'' if c[7] is None else 's' + str(c[7])}" for c in CASES])
def test_fwd_lse_and_bwd_parity(case):
    dtype, B, H, Sq, Sk, D, causal, scale = case
    q, k, v, do = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq * 7 + Sk)
    s = D ** -0.5 if scale is None else scale
    if D % 8 == 0:   # the C ABI itself (the binding pads other head dims)
        out, lse = abi.attn_fwd_lse(q, k, v, s, causal)
        dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, s, causal)
    else:
        out, lse = cmpext3.ops.attention_fwd_lse(q, k, v, s, causal)
        dq, dk, dv = cmpext3.ops.attention_bwd(q, k, v, out, do, lse, s, causal)
    torch.cuda.synchronize()
    qc, kc, vc, dc = (t.cpu() for t in (q, k, v, do))
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kc, vc, s, causal)) <= TOL[dtype]
    assert orc.max_abs_err(lse.cpu(), orc.sdpa_lse_np(qc, kc, s, causal)) <= TOL[dtype]
    want = orc.sdpa_bwd_np(qc, kc, vc, dc, s, causal)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert _rel_err(got, ref) <= TOL[dtype], name


def test_bwd_wide_scores():
    """Scores spread over tens of log2 units: P spans many orders of magnitude."""
    q, k, v, do = _inputs("fp16", 1, 2, 160, 700, 64, seed=5, amp=2.5)
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, False)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, 0.125, False)
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.cpu(), k.cpu(), v.cpu(), do.cpu(), 0.125, False)
    for got, ref in zip((dq, dk, dv), want):
        assert _rel_err(got, ref) <= TOL["fp16"]


def test_bwd_is_deterministic():
    q, k, v, do = _inputs("bf16", 2, 2, 300, 600, 64, seed=9)
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, True)
    first = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True)
    second = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D", [64, 128])
def test_bwd_strided_views(D):
    """[B,S,H,D] memory viewed as [B,H,S,D] for every operand and gradient
    (D = 128: the dK/dV kernel's V operands parked in LDS)."""
    B, S, H = 1, 192, 4
    g = torch.Generator().manual_seed(3)
    mk = lambda: torch.randn(B, S, H, D, generator=g).half().cuda().transpose(1, 2)
    q, k, v, do = mk(), mk(), mk(), mk()
    assert not q.is_contiguous()
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, True)
    dq, dk, dv = (torch.empty(B, S, H, D, dtype=torch.float16, device="cuda").transpose(1, 2)
                  for _ in range(3))
    delta = torch.empty(B, H, S, device="cuda")
    assert abi.attn_bwd_raw(q, k, v, out, do, lse, dq, dk, dv, delta, 0.125, True) == abi.OK
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.cpu(), k.cpu(), v.cpu(), do.cpu(), 0.125, True)
    for got, ref in zip((dq, dk, dv), want):
        assert _rel_err(got, ref) <= TOL["fp16"]


def test_bwd_headline_shape_heads_and_identities():
    """SDXL self-attention shape [2,10,4096,64] fp16: two heads against the
    oracle, and over every head the identities the mathematics fixes (the dK
    rows sum to zero, the dV rows sum to the dO rows)."""
    q, k, v, do = _inputs("fp16", 2, 10, 4096, 4096, 64, seed=1)
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, False)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, 0.125, False)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (1, 9)):
        sl = lambda t: t[b:b + 1, h:h + 1].cpu()
        want = orc.sdpa_bwd_np(sl(q), sl(k), sl(v), sl(do), 0.125, False)
        for got, ref in zip((dq, dk, dv), want):
            assert _rel_err(sl(got), ref) <= TOL["fp16"]
    # each identity's violation relative to the L1 mass of the summed rows
    # (rounding noise leaves ~1e-3; a wrong Delta or P transpose leaves O(1))
    dk64, dv64, do64 = dk.double(), dv.double(), do.double()
    assert float((dk64.sum(dim=2).abs() / dk64.abs().sum(dim=2)).max()) <= 1e-2
    assert float(((dv64.sum(dim=2) - do64.sum(dim=2)).abs() / dv64.abs().sum(dim=2)).max()) <= 1e-2


def test_autograd_function_matches_oracle():
    q, k, v, do = _inputs("bf16", 1, 2, 150, 220, 64, seed=4)
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = cmpext3.attention(q, k, v, None, True)
    out.backward(do)
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), do.cpu(), None, True)
    for got, ref in zip((q.grad, k.grad, v.grad), want):
        assert _rel_err(got, ref) <= TOL["bf16"]


def test_sdpa_training_route(patched):
    """With enable_backward(), SDPA with live autograd runs the native pair;
    without it, stock (the reference's behaviour)."""
    q, k, v, do = _inputs("fp16", 2, 2, 128, 256, 64, seed=6)
    calls = {"fwd": 0, "bwd": 0}
    real = cmpext3._C

    class Counting:
        attention = staticmethod(real.attention)

        @staticmethod
        def attention_fwd_lse(*a):
            calls["fwd"] += 1
            return real.attention_fwd_lse(*a)

        @staticmethod
        def attention_bwd(*a):
            calls["bwd"] += 1
            return real.attention_bwd(*a)

    old, was = cmpext3._C, cmpext3.backward_enabled()
    cmpext3._C = Counting
    try:
        for flag in (False, True):
            cmpext3.enable_backward(flag)
            qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
            out = F.scaled_dot_product_attention(qq, kk, vv, is_causal=True)
            out.backward(do)
            torch.cuda.synchronize()
            assert calls == ({"fwd": 1, "bwd": 1} if flag else {"fwd": 0, "bwd": 0})
            want = orc.sdpa_bwd_np(q.cpu(), k.cpu(), v.cpu(), do.cpu(), None, True)
            for got, ref in zip((qq.grad, kk.grad, vv.grad), want):
                assert _rel_err(got, ref) <= TOL["fp16"]
    finally:
        cmpext3._C = old
        cmpext3.enable_backward(was)


GQA_CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D, causal
    ("fp16", 1, 8, 2, 256, 256, 64, False),
    ("bf16", 2, 6, 3, 300, 200, 128, True),
    ("fp16", 1, 4, 1, 130, 700, 64, True),    # multi-query, causal Sq < Sk
    ("fp16", 1, 8, 2, 256, 384, 128, False),  # D = 128 non-causal: V operands parked in LDS
]


@pytest.mark.parametrize("case", GQA_CASES, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}"
                                                 f"{'c' if c[7] else ''}" for c in GQA_CASES])
def test_bwd_grouped_query(case):
    """K/V with fewer heads: dK/dV sum every query head of the group; the
    oracle runs on K/V repeated per query head and sums the repeats."""
    dtype, B, H, Hkv, Sq, Sk, D, causal = case
    g = torch.Generator().manual_seed(H * Sq + Sk)
    mk = lambda h, S: torch.randn(B, h, S, D, generator=g).to(TDT[dtype]).cuda()
    q, k, v, do = mk(H, Sq), mk(Hkv, Sk), mk(Hkv, Sk), mk(H, Sq)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, s, causal)
    torch.cuda.synchronize()
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    qc, dc = q.cpu(), do.cpu()
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kr, vr, s, causal)) <= TOL[dtype]
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(qc, kr, vr, dc, s, causal)
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), (dq_r, dk_r, dv_r)):
        assert _rel_err(got, ref) <= TOL[dtype], name


def test_sdpa_training_route_grouped_query(patched):
    """enable_gqa=True with live autograd stays native under enable_backward()."""
    g = torch.Generator().manual_seed(8)
    q = torch.randn(1, 8, 192, 64, generator=g).half().cuda().requires_grad_(True)
    k = torch.randn(1, 2, 192, 64, generator=g).half().cuda().requires_grad_(True)
    v = torch.randn(1, 2, 192, 64, generator=g).half().cuda().requires_grad_(True)
    do = torch.randn(1, 8, 192, 64, generator=g).half().cuda()
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
    assert _rel_err(q.grad, dq_r) <= TOL["fp16"]
    assert _rel_err(k.grad, dk_r.reshape(1, 2, 4, 192, 64).sum(axis=2)) <= TOL["fp16"]
    assert _rel_err(v.grad, dv_r.reshape(1, 2, 4, 192, 64).sum(axis=2)) <= TOL["fp16"]


def test_double_backward_is_refused():
    q, k, v, do = _inputs("fp16", 1, 1, 64, 64, 64, seed=2)
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = cmpext3.attention(q, k, v)
    (gq,) = torch.autograd.grad(out, q, do, create_graph=True)
    with pytest.raises(RuntimeError):
        gq.sum().backward()


def _train_mask(kind, B, H, Sq, Sk, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool_pad":                    # key padding [B,1,1,Sk]
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 1 - (13 * (b + 1)) % Sk:] = False
    elif kind == "bool_full":                 # per (b, h, query), key 0 kept
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
        m[..., 0] = True
    elif kind == "add_heads":                 # additive in the query dtype, -inf entries
        m = (torch.randn(1, H, Sq, Sk, generator=g) * 2).to(TDT[dtype])
        m[..., 1::5] = -math.inf
    else:                                     # additive fp32 [Sq, Sk]
        m = torch.randn(Sq, Sk, generator=g)
    return m.cuda()


MASK_TRAIN = [
    # dtype, B, H, Sq, Sk, D
    ("fp16", 2, 2, 160, 300, 64),
    ("bf16", 1, 2, 200, 1100, 128),   # forward key split
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", ["bool_pad", "bool_full", "add_heads", "add_2d_f32"])
@pytest.mark.parametrize("case", MASK_TRAIN, ids=[f"{c[0]}-q{c[3]}k{c[4]}d{c[5]}" for c in MASK_TRAIN])
def test_masked_training_pair(case, kind, causal):
    dtype, B, H, Sq, Sk, D = case
    q, k, v, do = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk + D)
    m = _train_mask(kind, B, H, Sq, Sk, dtype, seed=D)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal, attn_mask=m)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m)
    torch.cuda.synchronize()
    qc, kc, vc, dc, mc = (t.cpu() for t in (q, k, v, do, m))
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kc, vc, s, causal, attn_mask=mc)) <= TOL[dtype]
    assert orc.max_abs_err(lse.cpu(), orc.sdpa_lse_np(qc, kc, s, causal, attn_mask=mc)) <= TOL[dtype]
    want = orc.sdpa_bwd_np(qc, kc, vc, dc, s, causal, attn_mask=mc)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert _rel_err(got, ref) <= TOL[dtype], name


MASK_GQA_TRAIN = [
    # dtype, B, H, Hkv, Sq, Sk, D, kind
    ("fp16", 2, 6, 2, 150, 260, 64, "bool_full"),
    ("bf16", 1, 4, 1, 100, 1100, 128, "add_heads"),   # multi-query, forward key split when non-causal
    ("fp16", 1, 8, 2, 64, 500, 64, "add_2d_f32"),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", MASK_GQA_TRAIN, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}-{c[7]}"
                                                      for c in MASK_GQA_TRAIN])
def test_masked_grouped_query_training_pair(case, causal):
    """Masks and grouped-query K/V together: the dK/dV sweep over a group's
    query heads reads each query head's own mask rows."""
    dtype, B, H, Hkv, Sq, Sk, D, kind = case
    g = torch.Generator().manual_seed(H * Sq + Sk + D)
    mk = lambda h, S: torch.randn(B, h, S, D, generator=g).to(TDT[dtype]).cuda()
    q, k, v, do = mk(H, Sq), mk(Hkv, Sk), mk(Hkv, Sk), mk(H, Sq)
    m = _train_mask(kind, B, H, Sq, Sk, dtype, seed=Sk)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal, attn_mask=m)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m)
    torch.cuda.synchronize()
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    qc, dc, mc = q.cpu(), do.cpu(), m.cpu()
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kr, vr, s, causal, attn_mask=mc)) <= TOL[dtype]
    assert orc.max_abs_err(lse.cpu(), orc.sdpa_lse_np(qc, kr, s, causal, attn_mask=mc)) <= TOL[dtype]
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(qc, kr, vr, dc, s, causal, attn_mask=mc)
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), (dq_r, dk_r, dv_r)):
        assert _rel_err(got, ref) <= TOL[dtype], name


def test_masked_training_dead_rows():
    """Rows whose keys are all dropped: output 0, lse -inf, no gradient."""
    q, k, v, do = _inputs("fp16", 1, 2, 96, 200, 64, seed=77)
    m = torch.ones(1, 2, 96, 200, dtype=torch.bool, device="cuda")
    m[:, :, 7] = False
    m[:, 1, 40, :100] = False
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, False, attn_mask=m)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, 0.125, False, attn_mask=m)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[:, :, 7]) == 0
    assert bool(torch.isneginf(lse[:, :, 7]).all())
    assert torch.count_nonzero(dq[:, :, 7]) == 0
    want = orc.sdpa_bwd_np(q.cpu(), k.cpu(), v.cpu(), do.cpu(), 0.125, False, attn_mask=m.cpu())
    for got, ref in zip((dq, dk, dv), want):
        assert _rel_err(got, ref) <= TOL["fp16"]


def test_sdpa_training_route_with_mask(patched):
    """enable_backward(): a masked SDPA call with live autograd stays native."""
    q, k, v, do = _inputs("bf16", 2, 2, 128, 192, 64, seed=13)
    m = _train_mask("bool_pad", 2, 2, 128, 192, "bf16", seed=2)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    was = cmpext3.backward_enabled()
    cmpext3.enable_backward(True)
    try:
        out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=m, is_causal=True)
        assert "_Attention" in type(out.grad_fn).__name__
        out.backward(do)
    finally:
        cmpext3.enable_backward(was)
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.cpu(), k.cpu(), v.cpu(), do.cpu(), None, True, attn_mask=m.cpu())
    for got, ref in zip((qq.grad, kk.grad, vv.grad), want):
        assert _rel_err(got, ref) <= TOL["bf16"]
