"""GPU parity of the fp32 training pair: the fp32 forward that keeps the row
log-sum-exp (cmpext3_attn_fwd_lse on the fp32 kernel, key-split on small grids) and the
fp32 backward (cmpext3_attn_bwd: attn_bwd32_delta / _dkdv / _dq on 16x16x4
fp32 MFMAs), through the C ABI, plus the autograd Function and the SDPA route.

Oracle: float64 restatements in oracle/sdpa_oracle.py (sdpa_np, sdpa_lse_np,
sdpa_bwd_np), pinned to torch autograd, finite differences and closed forms in
tests/test_oracle_bwd.py.  Bars, written here (fp32 products are exact and
accumulate in fp32, so the bars are the forward's fp32 bar):
  * forward output and natural-log log-sum-exp: max abs error <= 1e-4;
  * gradients: max abs error <= 1e-4 times max |oracle| of that gradient (at
    least 0.1: a gradient that is exactly zero, dQ and dK with one key, where
    dP = Delta in exact arithmetic, keeps the fp32 cancellation of dP - Delta,
    ~1e-7 of terms of order sqrt(D), summed over the queries: ~1e-6);
  * rows with no visible key: lse -inf exactly where the oracle's is.
Covered: head dims 8..256 across the buckets (32, 40, 64, 96, 128, 192, 256,
zero columns past D), ragged lengths, one query row, one key, negative and
zero scales, causal with Sq < Sk and Sq > Sk, grouped-query K/V, four mask
kinds, [B,S,H,D] views, bit-identical reruns, the SD1.5 fp32 shape.
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

TOL = 1e-4


def _t(B, H, S, D, g, amp=1.0):
    return (torch.randn(B, H, S, D, generator=g, dtype=torch.float32) * amp).cuda()


def _rel_err(got, want):
    want = torch.as_tensor(want)
    return orc.max_abs_err(got.cpu(), want) / max(float(want.abs().max()), 0.1)


def _check(q, k, v, do, out, lse, grads, s, causal, mask=None):
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    qc, dc = q.cpu(), do.cpu()
    mc = None if mask is None else mask.cpu()
    assert orc.max_abs_err(out.cpu(), orc.sdpa_np(qc, kr, vr, s, causal, attn_mask=mc)) <= TOL
    want_lse = torch.as_tensor(orc.sdpa_lse_np(qc, kr, s, causal, attn_mask=mc))
    dead = torch.isneginf(want_lse)
    assert torch.equal(torch.isneginf(lse.cpu()), dead)
    assert orc.max_abs_err(lse.cpu()[~dead], want_lse[~dead]) <= TOL
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(qc, kr, vr, dc, s, causal, attn_mask=mc)
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, ref in zip(("dq", "dk", "dv"), grads, (dq_r, dk_r, dv_r)):
        assert _rel_err(got, ref) <= TOL, name


CASES = [
    # B, H, Hkv, Sq, Sk, D, causal, scale (None = 1/sqrt(D))
    (1, 2, 2, 128, 128, 64, False, None),
    (2, 2, 2, 200, 300, 40, True, None),       # SD1.5 head dim, ragged, causal Sq < Sk
    (1, 1, 1, 300, 130, 64, True, None),       # causal Sq > Sk
    (1, 2, 2, 64, 1000, 128, False, -0.2),     # negative scale, many key tiles
    (2, 1, 1, 1, 33, 96, False, None),         # one query row
    (1, 1, 1, 37, 1, 32, True, None),          # one key
    (1, 2, 2, 100, 200, 256, False, 0.0),      # scale 0: uniform P, no score gradient
    (1, 1, 1, 77, 150, 8, False, None),        # D = 8 (32 bucket)
    (1, 2, 2, 90, 120, 192, True, None),       # D = 192
    (1, 2, 2, 70, 90, 100, False, None),       # D = 100 (128 bucket)
    (1, 2, 2, 130, 70, 36, True, 0.3),         # D = 36 (40 bucket)
    (1, 8, 2, 150, 260, 64, True, None),       # grouped-query K/V
    (1, 4, 1, 100, 300, 40, False, None),      # multi-query
]


@pytest.mark.parametrize("case", CASES, ids=[f"H{c[1]}of{c[2]}-q{c[3]}k{c[4]}d{c[5]}{'c' if c[6] else ''}"
                                             f"{'' if c[7] is None else 's' + str(c[7])}" for c in CASES])
def test_fp32_training_pair(case):
    B, H, Hkv, Sq, Sk, D, causal, scale = case
    print(f"fp32 training pair {case}", flush=True)
    g = torch.Generator().manual_seed(Sq * 7 + Sk + D)
    q, k, v, do = _t(B, H, Sq, D, g), _t(B, Hkv, Sk, D, g), _t(B, Hkv, Sk, D, g), _t(B, H, Sq, D, g)
    s = D ** -0.5 if scale is None else scale
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal)
    grads = abi.attn_bwd(q, k, v, out, do, lse, s, causal)
    torch.cuda.synchronize()
    _check(q, k, v, do, out, lse, grads, s, causal)


def test_fp32_training_forward_matches_inference_forward():
    """Unsplit training forward against the key-split inference forward of
    the same problem ([1,8,1024,1024,64]: 128 blocks x 4 parts)."""
    g = torch.Generator().manual_seed(12)
    q, k, v = (_t(1, 8, 1024, 64, g) for _ in range(3))
    out, _ = abi.attn_fwd_lse(q, k, v, 0.125, False)
    ref = abi.attn_fwd(q, k, v, 0.125, False)
    torch.cuda.synchronize()
    assert float((out - ref).abs().max()) <= TOL


def test_fp32_bwd_is_deterministic():
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (_t(2, 2, 300, 64, g) for _ in range(4))
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, True)
    first = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True)
    second = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_fp32_bwd_strided_views():
    """[B,S,H,D] memory viewed as [B,H,S,D] for every operand and gradient."""
    B, S, H, D = 1, 192, 4, 64
    g = torch.Generator().manual_seed(3)
    mk = lambda: torch.randn(B, S, H, D, generator=g).cuda().transpose(1, 2)
    q, k, v, do = mk(), mk(), mk(), mk()
    assert not q.is_contiguous()
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, True)
    dq, dk, dv = (torch.empty(B, S, H, D, device="cuda").transpose(1, 2) for _ in range(3))
    delta = torch.empty(B, H, S, device="cuda")
    assert abi.attn_bwd_raw(q, k, v, out, do, lse, dq, dk, dv, delta, 0.125, True) == abi.OK
    torch.cuda.synchronize()
    _check(q, k, v, do, out, lse, (dq, dk, dv), 0.125, True)


def test_fp32_bwd_sd15_shape_heads_and_identities():
    """SD1.5 self-attention shape [2,8,4096,4096,40] fp32: two heads against
    the oracle, and over every head the identities the mathematics fixes (dK
    rows sum to zero, dV rows sum to the dO rows)."""
    g = torch.Generator().manual_seed(5)
    q, k, v, do = (_t(2, 8, 4096, 40, g) for _ in range(4))
    s = 40 ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, False)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, s, False)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (1, 7)):
        sl = lambda t: t[b:b + 1, h:h + 1].cpu()
        want = orc.sdpa_bwd_np(sl(q), sl(k), sl(v), sl(do), s, False)
        for got, ref in zip((dq, dk, dv), want):
            assert _rel_err(sl(got), ref) <= TOL
    dk64, dv64, do64 = dk.double(), dv.double(), do.double()
    assert float((dk64.sum(dim=2).abs() / dk64.abs().sum(dim=2)).max()) <= 1e-4
    assert float(((dv64.sum(dim=2) - do64.sum(dim=2)).abs() / dv64.abs().sum(dim=2)).max()) <= 1e-4


def _mask(kind, B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool_pad":                    # key padding [B,1,1,Sk]
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        for b in range(B):
            m[b, ..., Sk - 1 - (13 * (b + 1)) % Sk:] = False
    elif kind == "bool_full":                 # per (b, h, query), key 0 kept
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
        m[..., 0] = True
    elif kind == "add_heads":                 # additive fp32 per head, -inf entries
        m = torch.randn(1, H, Sq, Sk, generator=g) * 2
        m[..., 1::5] = -math.inf
    else:                                     # additive bf16 [Sq, Sk]
        m = torch.randn(Sq, Sk, generator=g).bfloat16()
    return m.cuda()


MASK_CASES = [
    # B, H, Hkv, Sq, Sk, D
    (2, 2, 2, 160, 300, 40),
    (1, 4, 2, 120, 264, 128),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", ["bool_pad", "bool_full", "add_heads", "add_2d_bf16"])
@pytest.mark.parametrize("case", MASK_CASES, ids=[f"H{c[1]}of{c[2]}-q{c[3]}k{c[4]}d{c[5]}" for c in MASK_CASES])
def test_fp32_masked_training_pair(case, kind, causal):
    B, H, Hkv, Sq, Sk, D = case
    g = torch.Generator().manual_seed(H * Sq + Sk + D)
    q, k, v, do = _t(B, H, Sq, D, g), _t(B, Hkv, Sk, D, g), _t(B, Hkv, Sk, D, g), _t(B, H, Sq, D, g)
    m = _mask(kind, B, H, Sq, Sk, seed=Sk)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal, attn_mask=m)
    grads = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m)
    torch.cuda.synchronize()
    _check(q, k, v, do, out, lse, grads, s, causal, mask=m)


def test_fp32_masked_training_dead_rows():
    """Rows whose keys are all dropped: output 0, lse -inf, no gradient."""
    g = torch.Generator().manual_seed(77)
    q, k, v, do = (_t(1, 2, 96 if i in (0, 3) else 200, 64, g) for i in range(4))
    m = torch.ones(1, 2, 96, 200, dtype=torch.bool, device="cuda")
    m[:, :, 7] = False
    m[:, 1, 40, :100] = False
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, False, attn_mask=m)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, 0.125, False, attn_mask=m)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[:, :, 7]) == 0
    assert bool(torch.isneginf(lse[:, :, 7]).all())
    assert torch.count_nonzero(dq[:, :, 7]) == 0
    _check(q, k, v, do, out, lse, (dq, dk, dv), 0.125, False, mask=m)


def test_fp32_sdpa_training_route_with_mask(patched):
    """enable_backward(): a masked fp32 SDPA call with live autograd runs the
    native pair."""
    g = torch.Generator().manual_seed(13)
    q, k, v, do = (_t(2, 2, 128, 40, g) if i != 1 and i != 2 else _t(2, 2, 192, 40, g) for i in range(4))
    m = _mask("bool_pad", 2, 2, 128, 192, seed=2)
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
        assert _rel_err(got, ref) <= TOL


def test_fp32_autograd_function_with_odd_head_dim():
    """D = 41 (not whole 16-byte chunks): the binding pads to 44 and the
    kernels run the 64 bucket; gradients come back at D = 41."""
    g = torch.Generator().manual_seed(4)
    q, k, v = (_t(1, 2, 150, 41, g).requires_grad_(True) for _ in range(3))
    do = _t(1, 2, 150, 41, g)
    out = cmpext3.attention(q, k, v, None, True)
    out.backward(do)
    torch.cuda.synchronize()
    want = orc.sdpa_bwd_np(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), do.cpu(), None, True)
    for got, ref in zip((q.grad, k.grad, v.grad), want):
        assert got.shape == (1, 2, 150, 41)
        assert _rel_err(got, ref) <= TOL


def test_fp32_training_forward_key_split():
    """Grids of few query blocks key-split the fp32 training forward too: the
    merging part writes the log-sum-exp of the merged (m, l).  BASELINE config
    1's shape (128 blocks, 4 parts) and a masked ragged one: output and lse
    meet the oracle, agree with the unsplit launch, and reruns are
    bit-identical."""
    dt = abi.DTYPE_F32
    for B, H, Sq, Sk, D, masked in ((1, 8, 1024, 1024, 64, False), (1, 2, 100, 700, 40, True)):
        ws = abi.workspace_size(dt, B, H, H, Sq, Sk, D, abi.DTYPE_BOOL if masked else -1, False, with_lse=True)
        assert abi.plan(dt, B, H, H, Sq, Sk, D, ws, abi.DTYPE_BOOL if masked else -1, False, with_lse=True)[1] >= 2
        g = torch.Generator().manual_seed(Sk + D)
        q, k, v = _t(B, H, Sq, D, g), _t(B, H, Sk, D, g), _t(B, H, Sk, D, g)
        m = None
        if masked:
            m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
            m[..., Sk - 150:] = False
            m = m.cuda()
        s = D ** -0.5
        o1, l1 = abi.attn_fwd_lse(q, k, v, s, False, attn_mask=m)
        o2, l2 = abi.attn_fwd_lse(q, k, v, s, False, attn_mask=m)
        ow, lw = abi.attn_fwd_lse(q, k, v, s, False, attn_mask=m, workspace=False)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
        mc = None if m is None else m.cpu()
        qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
        want_o = orc.sdpa_np(qc, kc, vc, s, False, attn_mask=mc)
        want_l = orc.sdpa_lse_np(qc, kc, s, False, attn_mask=mc)
        for o, l in ((o1, l1), (ow, lw)):
            assert orc.max_abs_err(o.cpu(), want_o) <= TOL
            assert orc.max_abs_err(l.cpu(), want_l) <= TOL
