"""GPU parity of the fused attention forward, called through the C ABI.

Bar (north star): max |kernel - oracle| <= 1e-2 (fp16), 2e-2 (bf16), 1e-4 (fp32),
where the oracle is float64 SDPA on the CPU over the same dtype-rounded inputs
(oracle/sdpa_oracle.py: sdpa_np for large shapes, the C restatement sdpa_c
for the small sweep).

Covers the five BASELINE configs at full size, then edge cases the reference
exercises or that the tiling makes risky: ragged Sq/Sk (tile tails), Sk=1,
cross-attention, causal with Sq <, =, > Sk (top-left), every head-dim bucket
including non-power-of-two D, negative / zero / large scale, [B,S,H,D]-memory
views and other strided inputs, and bitwise determinism across reruns.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cmpext3 import abi
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE


def _run(q, k, v, scale, causal):
    out = abi.attn_fwd(q, k, v, scale, causal)
    torch.cuda.synchronize()
    return out


def _inputs(dtype, B, H, Sq, Sk, D, seed=0, kv_std=1.0, device="cuda"):
    wl = W.Workload("case", dtype, B, H, Sq, Sk, D, kv_std=kv_std, seed=seed)
    return wl.make_inputs(device)


@pytest.mark.parametrize("wl", W.WORKLOADS, ids=[w.name for w in W.WORKLOADS])
def test_baseline_config_full_size(wl):
    q, k, v = wl.make_inputs("cuda")
    out = _run(q, k, v, wl.eff_scale, wl.causal)
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), wl.eff_scale, wl.causal)
    err = orc.max_abs_err(out.cpu(), ref)
    print(f"{wl.name}: max abs err {err:.3e} (tol {TOL[wl.dtype]:.0e})", flush=True)
    assert err <= TOL[wl.dtype]


SMALL = [
    # dtype, B, H, Sq, Sk, D, causal
    ("fp16", 1, 1, 1, 1, 64, False),
    ("fp16", 1, 2, 7, 1, 64, False),
    ("fp16", 2, 3, 100, 77, 64, False),
    ("fp16", 1, 2, 129, 300, 40, False),
    ("fp16", 1, 1, 257, 65, 80, False),
    ("fp16", 2, 2, 128, 128, 128, True),
    ("fp16", 1, 2, 200, 333, 64, True),     # causal Sq < Sk
    ("fp16", 1, 2, 333, 200, 64, True),     # causal Sq > Sk
    ("bf16", 1, 2, 77, 77, 128, True),
    ("bf16", 2, 2, 300, 129, 64, False),
    ("bf16", 1, 1, 1, 513, 128, False),
    ("bf16", 1, 3, 190, 190, 96, True),
    ("fp32", 1, 2, 67, 67, 40, False),
    ("fp32", 2, 2, 130, 70, 64, False),
    ("fp32", 1, 2, 129, 129, 64, True),
    ("fp32", 1, 1, 50, 300, 128, True),
    ("fp32", 1, 1, 300, 50, 32, True),
]


@pytest.mark.parametrize("case", SMALL, ids=[
    f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}{'-causal' if c[6] else ''}" for c in SMALL])
def test_small_shapes(case):
    dtype, B, H, Sq, Sk, D, causal = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq * 7 + Sk)
    scale = 1.0 / math.sqrt(D)
    out = _run(q, k, v, scale, causal)
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("D", [8, 16, 24, 40, 48, 56, 64, 72, 80, 96, 112, 128, 136, 160, 192,
                               200, 256])
def test_head_dim_buckets(dtype, D):
    if dtype == "fp32" and D % 4:
        pytest.skip("fp32 needs D % 4 == 0")
    q, k, v = _inputs(dtype, 1, 2, 70, 90, D, seed=D)
    scale = 1.0 / math.sqrt(D)
    out = _run(q, k, v, scale, False)
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, False)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [8, 24, 32, 40, 56, 64, 72, 80, 96, 112, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_buckets_long_keys(dtype, D, causal):
    """Key sweeps of 256+ keys take the software-pipelined kernel for head-dim
    buckets up to 128; Sk = 275 gives an odd number of 32-key tiles (the loop
    runs a masked padding tile) and a ragged last tile."""
    q, k, v = _inputs(dtype, 1, 2, 70, 275, D, seed=D + 1000 * causal)
    text = abi.describe(abi.dtype_code(q.dtype), 1, 2, 70, 275, D, causal)[1]
    assert "pipe16" in text
    scale = 1.0 / math.sqrt(D)
    out = _run(q, k, v, scale, causal)
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("scale", [-0.125, 0.0, 0.5, 1e-3, 1.0, -2.0])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sk", [80, 300])
def test_scale_values(dtype, scale, causal, Sk):
    q, k, v = _inputs(dtype, 1, 2, 96, Sk, 64, seed=11)
    out = _run(q, k, v, scale, causal)
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("S", [150, 300])
def test_bshd_views_and_strided_kv(dtype, S):
    wl = W.Workload("v", dtype, 2, 5, S, S, 64, seed=21)
    q, k, v = wl.make_inputs("cuda", layout="bshd")   # [B,H,S,D] views of [B,S,H,D]
    assert not q.is_contiguous()
    # K/V sliced out of a longer sequence: seq stride larger than D
    big_k = torch.randn(2, 5, S + 250, 64, dtype=q.dtype, device="cuda")
    big_v = torch.randn(2, 5, S + 250, 64, dtype=q.dtype, device="cuda")
    k2, v2 = big_k[:, :, 100:100 + S], big_v[:, :, 100:100 + S]
    for kk, vv in ((k, v), (k2, v2)):
        for causal in (False, True):
            out = _run(q, kk, vv, 0.125, causal)
            ref = orc.sdpa_np(q.cpu(), kk.cpu(), vv.cpu(), 0.125, causal)
            assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


def test_output_stride_is_honoured():
    q, k, v = _inputs("fp16", 2, 4, 64, 64, 64, seed=3)
    o = torch.full((2, 64, 4, 64), float("nan"), dtype=q.dtype, device="cuda").transpose(1, 2)
    rc = abi.attn_fwd_raw(q, k, v, o, 0.125, False)
    torch.cuda.synchronize()
    assert rc == abi.OK
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, False)
    assert orc.max_abs_err(o.cpu(), ref) <= TOL["fp16"]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_deterministic_rerun(dtype):
    """Same input twice -> bitwise identical output (an LDS race would show here)."""
    q, k, v = _inputs(dtype, 2, 4, 500, 500, 64, seed=9)
    a = _run(q, k, v, 0.125, True)
    b = _run(q, k, v, 0.125, True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_wide_score_range(dtype, causal):
    """Scores spanning tens of log2 units: the running exp2 offset must move
    (and O, l be rescaled) many times, in both directions of the key sweep."""
    Sk = 300 if causal else 333
    q, k, v = _inputs(dtype, 1, 2, 200, Sk, 64, seed=5)
    q = (q.float() * 12).to(q.dtype)
    out = _run(q, k, v, 0.125, causal)
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, causal)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("order", ["rising", "falling"])
def test_monotone_scores(dtype, order):
    """Scores rising by ~9 log2 units per 32 keys force a rescale on every key
    tile; falling scores never rescale after the first and underflow later
    tiles' probabilities."""
    Sk, D = 1000, 64
    j = torch.arange(Sk, dtype=torch.float32)
    if order == "falling":
        j = j.flip(0)
    kf = (0.05 * j)[:, None].expand(Sk, D)
    k = kf.to(getattr(torch, {"fp16": "float16", "bf16": "bfloat16"}[dtype]))[None, None].repeat(1, 2, 1, 1)
    q = torch.full((1, 2, 64, D), 0.5, dtype=k.dtype)
    v = torch.randn(1, 2, Sk, D, generator=torch.Generator().manual_seed(3)).to(k.dtype)
    q, k, v = q.cuda(), k.cuda(), v.cuda()
    out = _run(q, k, v, 0.125, False)
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, False)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL[dtype]


def test_huge_kv_row_stride_falls_back():
    """K/V rows further apart than the pipelined kernel's 32-bit buffer offsets
    reach ((Sk + 32) * stride * 2 bytes >= 2^31): the other fp16 kernel runs."""
    Sk, D, stride = 40, 64, 15_000_000
    gen = torch.Generator(device="cuda").manual_seed(4)
    base_k = torch.empty(Sk, stride, dtype=torch.float16, device="cuda")
    base_v = torch.empty(Sk, stride, dtype=torch.float16, device="cuda")
    base_k[:, :D] = torch.randn(Sk, D, generator=gen, device="cuda").half()
    base_v[:, :D] = torch.randn(Sk, D, generator=gen, device="cuda").half()
    k = base_k[:, :D][None, None]
    v = base_v[:, :D][None, None]
    assert k.stride(2) == stride
    q = torch.randn(1, 1, 50, D, generator=gen, device="cuda").half()
    out = _run(q, k, v, 0.125, False)
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, False)
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["fp16"]
    del base_k, base_v


def test_causal_differs_from_noncausal():
    """Reference check tests_hardware/test_attention_causal.py:113-130: the causal
    flag must actually reach the kernel."""
    q, k, v = _inputs("fp16", 1, 4, 256, 256, 128, seed=0)
    a = _run(q, k, v, 128 ** -0.5, True)
    b = _run(q, k, v, 128 ** -0.5, False)
    assert (a.float() - b.float()).abs().max().item() > 1e-3


def test_empty_and_rejected_inputs_launch_nothing():
    q, k, v = _inputs("fp16", 1, 2, 64, 64, 64)
    o = torch.empty_like(q)
    empty_q = q[:, :, :0]
    assert abi.attn_fwd_raw(empty_q, k, v, o[:, :, :0], 0.125) == abi.OK
    assert abi.attn_fwd_raw(q, k[:, :, :0], v[:, :, :0], o, 0.125) == abi.E_EMPTY_KEYS
    # an odd head dim, and a 2-byte offset view (rows of 2-byte pieces), are
    # refused with a mask (which needs 4-byte pieces) ...
    odd = torch.randn(1, 2, 64, 35, dtype=torch.float16, device="cuda")
    keep = torch.ones(1, 1, 64, 64, dtype=torch.bool, device="cuda")
    assert abi.attn_fwd_raw(odd, odd, odd, torch.empty_like(odd), 0.125, attn_mask=keep) == abi.E_HEAD_DIM
    mis = torch.randn(1, 2, 64 * 64 + 1, dtype=torch.float16, device="cuda")[..., 1:]
    mis = mis.view(1, 2, 64, 64)
    assert abi.attn_fwd_raw(mis, k, v, o, 0.125, attn_mask=keep) == abi.E_ALIGN
    # (an even head dim that is not whole 16-byte chunks runs with the mask)
    even = torch.randn(1, 2, 64, 36, dtype=torch.float16, device="cuda")
    oe = torch.empty_like(even)
    assert abi.attn_fwd_raw(even, even, even, oe, 0.125, attn_mask=keep) == abi.OK
    assert orc.max_abs_err(oe.cpu(), orc.sdpa_np(even.cpu(), even.cpu(), even.cpu(), 0.125)) <= TOL["fp16"]
    # ... and run in place without one (element-granular rows)
    oo = torch.empty_like(odd)
    assert abi.attn_fwd_raw(odd, odd, odd, oo, 0.125) == abi.OK
    assert orc.max_abs_err(oo.cpu(), orc.sdpa_np(odd.cpu(), odd.cpu(), odd.cpu(), 0.125)) <= TOL["fp16"]
    assert abi.attn_fwd_raw(mis, k, v, o, 0.125) == abi.OK
    assert orc.max_abs_err(o.cpu(), orc.sdpa_np(mis.cpu(), k.cpu(), v.cpu(), 0.125)) <= TOL["fp16"]
