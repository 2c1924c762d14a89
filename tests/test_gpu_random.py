"""Seeded random sweep over what the forward and training entry points accept.

Each case draws dtype, batch, query heads and K/V heads (grouped-query when
they differ), query and key lengths (decode-like, short-key, ragged, long),
head dim 1..256, causal, scale (default, positive, zero or negative), the
tensor layout (contiguous [B,H,S,D], a [B,S,H,D] view, or rows one element
off 16-byte alignment inside wider rows) and, where the ABI takes one, an
attention mask (bool or additive, broadcast or full); a further set of
causal cases of one sequence with 1024-2600 queries and keys drives the
causal key-split plans.  The cases are fixed by the seed below, so a
failure names a case that reruns identically.

Forward cases run through the C ABI (cmpext3_attn_fwd / _gqa / _masked) into
an output that is a view inside a larger buffer filled with a sentinel: the
output must match the float64 oracle (oracle/sdpa_oracle.py sdpa_np, pinned
to torch in tests/test_oracle.py) at the usual bar (max abs error <= 1e-2
fp16, 2e-2 bf16, 1e-4 fp32), and every buffer element outside the output's
own elements must still hold the sentinel (no stray writes from tail tiles,
key-split merges or narrow-row stores).  Cases without K/V grouping or mask
also run through the torch binding (ops.attention).

Training cases (fp16/bf16/fp32, D <= 256 in whole 16-byte chunks, contiguous or
[B,S,H,D] views, grouped-query K/V, masks) run cmpext3_attn_fwd_lse and then
cmpext3_attn_bwd against sdpa_np / sdpa_lse_np / sdpa_bwd_np (pinned to torch
autograd in tests/test_oracle_bwd.py), at the bars of
tests/test_gpu_backward.py: output and natural-log lse within 1e-2 fp16 /
2e-2 bf16 / 1e-4 fp32 (rows with no visible key must give lse -inf exactly), each
gradient within that fraction of its own largest oracle magnitude (floor
1e-3; 0.1 for fp32); grouped dK/dV are the oracle's per-query-head gradients summed over
each group.

Contract the draws stay inside (include/cmpext3_attn.h): any head dim 1..256
and element-aligned strides for the unmasked entry points; masks for every
dtype and head dim with rows in whole 16-byte chunks (the masks themselves in
any layout with unit key stride: key counts that are not a multiple of 8 are
read element by element).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import cmpext3
from cmpext3 import abi
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE
TDT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
SEED = 20261202
NCASES = 192
NTRAIN = 96
NLONG = 24   # extra causal cases of few blocks and long sweeps (key-split causal plans)
SENTINEL = -4096.0  # exact in fp16, bf16 and fp32; never an attention output here
# oracle work bound (B * H * Sq * Sk * D) so that every case checks in about a second
MAX_WORK = 1.2e9
MAX_WORK_TRAIN = 2.5e8


def _draw(rng):
    dtype = rng.choice(["fp16", "bf16", "fp32"], p=[0.4, 0.4, 0.2])
    B = int(rng.integers(1, 4))
    hkv = int(rng.integers(1, 4))
    group = int(rng.choice([1, 1, 2, 4]))
    H = hkv * group
    r = rng.random()
    Sq = int(rng.integers(1, 17) if r < 0.2 else rng.integers(17, 300) if r < 0.6 else rng.integers(300, 1100))
    Sk = int(rng.integers(1, 129) if rng.random() < 0.3 else rng.integers(129, 2100))
    D = int(rng.choice([8, 16, 32, 40, 64, 64, 80, 96, 128, 128, 160, 192, 256]) if rng.random() < 0.7
            else rng.integers(1, 257))
    causal = bool(rng.random() < 0.5)
    r = rng.random()
    scale = None if r < 0.5 else 0.0 if r < 0.55 else float(rng.uniform(-0.3, 0.6))
    layout = str(rng.choice(["bhsd", "bshd", "offset"], p=[0.45, 0.35, 0.2]))
    mask = "none"
    if D % (4 if dtype == "fp32" else 8) == 0 and layout != "offset" and rng.random() < 0.35:
        mask = str(rng.choice(["bool_keys", "bool_full", "add_heads", "add_f32"]))
    while B * H * Sq * Sk * D > MAX_WORK:
        if Sq > 64:
            Sq //= 2
        elif Sk > 64:
            Sk //= 2
        else:
            B = 1
            break
    return dict(dtype=str(dtype), B=B, H=H, Hkv=hkv, Sq=Sq, Sk=Sk, D=D, causal=causal, scale=scale,
                layout=layout, mask=mask, seed=int(rng.integers(1, 2**31 - 1)))


def _draw_train(rng):
    dtype = str(rng.choice(["fp16", "bf16", "fp32"], p=[0.4, 0.4, 0.2]))
    B = int(rng.integers(1, 3))
    hkv = int(rng.integers(1, 4))
    H = hkv * int(rng.choice([1, 1, 2, 3]))
    Sq = int(rng.integers(1, 17) if rng.random() < 0.15 else rng.integers(17, 600))
    Sk = int(rng.integers(1, 129) if rng.random() < 0.3 else rng.integers(129, 1200))
    D = int(8 * rng.integers(1, 33))
    causal = bool(rng.random() < 0.5)
    r = rng.random()
    scale = None if r < 0.5 else 0.0 if r < 0.55 else float(rng.uniform(-0.3, 0.5))
    layout = str(rng.choice(["bhsd", "bshd"]))
    mask = "none" if rng.random() < 0.65 else str(rng.choice(["bool_keys", "bool_full", "add_heads", "add_f32"]))
    while B * H * Sq * Sk * D > MAX_WORK_TRAIN:
        if Sq > 64:
            Sq //= 2
        elif Sk > 64:
            Sk //= 2
        else:
            B = 1
            break
    return dict(dtype=dtype, B=B, H=H, Hkv=hkv, Sq=Sq, Sk=Sk, D=D, causal=causal, scale=scale,
                layout=layout, mask=mask, seed=int(rng.integers(1, 2**31 - 1)))


def _draw_long_causal(rng):
    """Causal grids of few blocks with long sweeps: the launches that cut
    every block's keys into parts (whose rows may see none of a part's keys)."""
    c = _draw(rng)
    c.update(causal=True, B=1, Sq=int(rng.integers(1024, 2600)), Sk=int(rng.integers(1024, 2600)))
    c["H"] = c["Hkv"] * int(rng.choice([1, 2]))
    while c["H"] * c["Sq"] * c["Sk"] * c["D"] > MAX_WORK:
        c["Sq"] = max(1024, c["Sq"] // 2)
        c["D"] = max(8, c["D"] // 2)
    return c


_rng = np.random.default_rng(SEED)
CASES = [_draw(_rng) for _ in range(NCASES)]
_rng_long = np.random.default_rng(SEED + 2)
CASES += [_draw_long_causal(_rng_long) for _ in range(NLONG)]
_rng_train = np.random.default_rng(SEED + 1)
TRAIN_CASES = [_draw_train(_rng_train) for _ in range(NTRAIN)]


def _case_id(c):
    sc = "def" if c["scale"] is None else f"{c['scale']:.3g}"
    return (f"{c['dtype']}-B{c['B']}H{c['H']}kv{c['Hkv']}-q{c['Sq']}k{c['Sk']}d{c['D']}"
            f"-{'c' if c['causal'] else 'n'}-s{sc}-{c['layout']}-{c['mask']}")


def _laid_out(x, layout, fill=None):
    """Copy of [B,H,S,D] tensor x in the given layout, as a view of a larger
    buffer (returned too).  fill: value of the buffer outside the view."""
    B, H, S, D = x.shape
    if layout == "bhsd":
        buf = torch.empty(B * H * S * D + 64, dtype=x.dtype, device=x.device)
        view = buf[32:32 + B * H * S * D].view(B, H, S, D)
    elif layout == "bshd":
        buf = torch.empty(B * S * H * D + 64, dtype=x.dtype, device=x.device)
        view = buf[32:32 + B * S * H * D].view(B, S, H, D).transpose(1, 2)
    else:  # rows of D + 1 elements, the view starting one element in
        buf = torch.empty(B * H * S * (D + 1) + 64, dtype=x.dtype, device=x.device)
        view = buf[32:32 + B * H * S * (D + 1)].view(B, H, S, D + 1)[..., 1:]
    if fill is not None:
        buf.fill_(fill)
    view.copy_(x)
    return view, buf


def _mask(kind, dtype, B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "bool_keys":      # key padding [B,1,1,Sk], at least key 0 kept
        m = torch.rand(B, 1, 1, Sk, generator=g) > 0.4
        m[..., 0] = True
    elif kind == "bool_full":    # [B,H,Sq,Sk], some rows fully dropped
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.5
        m[:, :, ::5] = False
    elif kind == "add_heads":    # additive [1,H,Sq,Sk] in the query dtype, some -inf
        m = (torch.randn(1, H, Sq, Sk, generator=g) * 3).to(TDT[dtype])
        m[..., 1::3] = -math.inf
    else:                        # additive fp32 [Sq, Sk]
        m = torch.randn(Sq, Sk, generator=g) * 2
    return m.cuda()


@pytest.mark.parametrize("case", CASES, ids=[_case_id(c) for c in CASES])
def test_random_case(case):
    c = case
    dtype, B, H, Hkv, Sq, Sk, D = c["dtype"], c["B"], c["H"], c["Hkv"], c["Sq"], c["Sk"], c["D"]
    print(f"random case: {_case_id(c)} seed={c['seed']}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    t = TDT[dtype]
    q0 = torch.randn(B, H, Sq, D, generator=g).to(t)
    k0 = torch.randn(B, Hkv, Sk, D, generator=g).to(t)
    v0 = torch.randn(B, Hkv, Sk, D, generator=g).to(t)
    q, _ = _laid_out(q0.cuda(), c["layout"])
    k, _ = _laid_out(k0.cuda(), c["layout"])
    v, _ = _laid_out(v0.cuda(), c["layout"])
    o, obuf = _laid_out(torch.zeros(B, H, Sq, D, dtype=t, device="cuda"), c["layout"], fill=SENTINEL)
    m = None if c["mask"] == "none" else _mask(c["mask"], dtype, B, H, Sq, Sk, c["seed"] + 1)
    scale = D ** -0.5 if c["scale"] is None else c["scale"]

    rc = abi.attn_fwd_raw(q, k, v, o, scale, c["causal"], attn_mask=m)
    torch.cuda.synchronize()
    assert rc == abi.OK, abi.strerror(rc)

    # nothing outside the output's elements was written
    touched = torch.zeros(obuf.numel(), dtype=torch.bool, device="cuda")
    torch.as_strided(touched, o.shape, o.stride(), o.storage_offset()).fill_(True)
    outside = obuf[~touched]
    assert bool((outside == SENTINEL).all()), "write outside the output view"

    kx = k0.repeat_interleave(H // Hkv, dim=1)
    vx = v0.repeat_interleave(H // Hkv, dim=1)
    want = orc.sdpa_np(q0, kx, vx, scale, c["causal"], attn_mask=None if m is None else m.cpu())
    got = o.float().cpu().numpy()
    err = orc.max_abs_err(got, want)
    assert err <= TOL[dtype], f"max abs err {err:.3g} > {TOL[dtype]}"

    if Hkv == H and m is None:
        out = cmpext3.ops.attention(q, k, v, scale, c["causal"])
        err2 = orc.max_abs_err(out.float().cpu().numpy(), want)
        assert err2 <= TOL[dtype], f"ops.attention: max abs err {err2:.3g} > {TOL[dtype]}"


def _rel_err(got, want, floor=1e-3):
    return orc.max_abs_err(got, want) / max(float(np.abs(want).max()) if want.size else 0.0, floor)


@pytest.mark.parametrize("case", TRAIN_CASES, ids=[_case_id(c) for c in TRAIN_CASES])
def test_random_training_case(case):
    c = case
    dtype, B, H, Hkv, Sq, Sk, D = c["dtype"], c["B"], c["H"], c["Hkv"], c["Sq"], c["Sk"], c["D"]
    print(f"random training case: {_case_id(c)} seed={c['seed']}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    t = TDT[dtype]
    q0 = torch.randn(B, H, Sq, D, generator=g).to(t)
    k0 = torch.randn(B, Hkv, Sk, D, generator=g).to(t)
    v0 = torch.randn(B, Hkv, Sk, D, generator=g).to(t)
    do0 = torch.randn(B, H, Sq, D, generator=g).to(t)
    q, k, v, do = (_laid_out(x.cuda(), c["layout"])[0] for x in (q0, k0, v0, do0))
    m = None if c["mask"] == "none" else _mask(c["mask"], dtype, B, H, Sq, Sk, c["seed"] + 1)
    scale = D ** -0.5 if c["scale"] is None else c["scale"]

    out, lse = abi.attn_fwd_lse(q, k, v, scale, c["causal"], attn_mask=m)
    dq, dk, dv = abi.attn_bwd(q, k, v, out, do, lse, scale, c["causal"], attn_mask=m)
    torch.cuda.synchronize()

    grp = H // Hkv
    kx, vx = k0.repeat_interleave(grp, dim=1), v0.repeat_interleave(grp, dim=1)
    mc = None if m is None else m.cpu()
    want_o = orc.sdpa_np(q0, kx, vx, scale, c["causal"], attn_mask=mc)
    assert orc.max_abs_err(out.float().cpu().numpy(), want_o) <= TOL[dtype], "output"
    want_lse = orc.sdpa_lse_np(q0, kx, scale, c["causal"], attn_mask=mc)
    got_lse = lse.double().cpu().numpy()
    dead = np.isneginf(want_lse)
    assert np.array_equal(np.isneginf(got_lse), dead), "rows without a visible key"
    assert orc.max_abs_err(got_lse[~dead], want_lse[~dead]) <= TOL[dtype], "lse"
    dq_r, dk_r, dv_r = orc.sdpa_bwd_np(q0, kx, vx, do0, scale, c["causal"], attn_mask=mc)
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), (dq_r, dk_r, dv_r)):
        # fp32: a gradient that is exactly zero (one key) keeps ~1e-6 of the
        # cancellation of dP - Delta
        err = _rel_err(got.float().cpu().numpy(), ref, 0.1 if dtype == "fp32" else 1e-3)
        assert err <= TOL[dtype], f"{name}: relative error {err:.3g}"
