"""GPU parity of the split gradient sweeps of the backward (cmpext3_attn_bwd_ws).

With too few blocks for the CUs (one or two sequences, grouped-query K/V,
causal sweeps whose length runs from one tile to all of them) the dK/dV sweep
of a key block over (query head of the group, query tile), and the dQ sweep
of a query block over key tiles, are cut into up to 8 contiguous parts whose
fp32 partials a further kernel sums in part order; non-causal f16/bf16 grids
past one round split only the blocks of their last, partial round (split
tails, block-indexed partials).
Oracle: float64 sdpa_bwd_np on K/V repeated per query head, the repeats'
gradients summed; bar: max abs error <= 1e-2 (fp16) / 2e-2 (bf16) / 1e-4
(fp32) times the gradient's largest oracle magnitude (at least 1e-3; 0.1 for
fp32, as in test_gpu_backward32.py), as for the unsplit backward.  Also: the split launch agrees with the unsplit one (no workspace)
within the same bar, reruns are bit-identical, and a workspace below the
size query runs unsplit.  The plan itself (which problems split) is a CPU test in
test_abi.py.
"""
from __future__ import annotations

import pytest
import torch

from cmpext3 import abi
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = {"fp16": 1e-2, "bf16": 2e-2, "fp32": 1e-4}
TDT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _rel_err(got, want, dtype):
    want = torch.as_tensor(want)
    return orc.max_abs_err(got.cpu(), want) / max(float(want.abs().max()), 0.1 if dtype == "fp32" else 1e-3)


CASES = [
    # dtype, B, H, Hkv, Sq, Sk, D, causal, mask
    ("bf16", 1, 8, 2, 1024, 1024, 128, True, None),     # grouped-query causal, 8 parts
    ("fp16", 1, 4, 4, 1000, 777, 64, False, None),      # ragged non-causal, dQ split too
    ("fp16", 2, 8, 1, 300, 1500, 64, True, None),       # multi-query, causal Sq < Sk (empty parts)
    ("bf16", 1, 4, 2, 700, 300, 128, True, None),       # causal Sq > Sk
    ("bf16", 1, 4, 2, 600, 900, 256, True, None),       # D = 256 bucket, one wave per SIMD
    ("fp16", 1, 2, 1, 333, 520, 160, False, None),      # D = 160 in the 192 bucket
    ("fp16", 2, 4, 2, 500, 700, 64, False, "pad"),      # key-padding mask
    ("bf16", 1, 4, 2, 400, 400, 128, True, "full"),     # per-row bool mask with causal
    ("fp16", 1, 2, 2, 260, 200, 64, False, None),       # short sweeps: 2 parts of 4 and 5 tiles
    ("fp16", 1, 36, 36, 2048, 2048, 64, False, None),   # split tails: 512 whole + 64 x 4 parts
    ("fp16", 1, 36, 36, 2048, 2048, 64, False, "pad"),  # a dK/dV split tail with a mask
    ("bf16", 1, 20, 20, 2048, 2048, 128, False, None),  # split tails at two workgroups per CU
    ("bf16", 1, 40, 20, 2048, 2048, 128, False, None),  # a dK/dV split tail, grouped-query K/V
    ("fp32", 1, 8, 8, 1024, 1024, 64, False, None),     # BASELINE config 1 shape: 6 + 8 parts
    ("fp32", 1, 4, 2, 700, 500, 40, True, None),        # SD1.5 head dim, grouped-query causal
    ("fp32", 1, 2, 1, 300, 400, 128, True, "pad"),      # masked causal D = 128
]


def _mask(kind, B, H, Sq, Sk, seed):
    if kind is None:
        return None
    g = torch.Generator().manual_seed(seed)
    if kind == "pad":
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        m[..., Sk - Sk // 5:] = False
    else:
        m = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
        m[..., 0] = True
    return m.cuda()


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-b{c[1]}h{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}"
                                             f"{'c' if c[7] else ''}{'-' + c[8] if c[8] else ''}" for c in CASES])
def test_split_backward(case):
    dtype, B, H, Hkv, Sq, Sk, D, causal, mk = case
    dt = abi.dtype_code(TDT[dtype])
    mdt = -1 if mk is None else abi.DTYPE_BOOL
    assert abi.bwd_workspace_size(dt, B, H, Hkv, Sq, Sk, D, mdt, causal) > 0
    print(f"split backward {case}", flush=True)
    g = torch.Generator().manual_seed(Sq + Sk + D)
    rnd = lambda h, S: torch.randn(B, h, S, D, generator=g).to(TDT[dtype]).cuda()
    q, k, v, do = rnd(H, Sq), rnd(Hkv, Sk), rnd(Hkv, Sk), rnd(H, Sq)
    m = _mask(mk, B, H, Sq, Sk, seed=D)
    s = D ** -0.5
    out, lse = abi.attn_fwd_lse(q, k, v, s, causal, attn_mask=m)
    split1 = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m, workspace=True)
    split2 = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m, workspace=True)
    whole = abi.attn_bwd(q, k, v, out, do, lse, s, causal, attn_mask=m, workspace=None)
    torch.cuda.synchronize()
    for a, b in zip(split1, split2):
        assert torch.equal(a, b)
    grp = H // Hkv
    kr, vr = (t.cpu().repeat_interleave(grp, dim=1) for t in (k, v))
    want = orc.sdpa_bwd_np(q.cpu(), kr, vr, do.cpu(), s, causal, attn_mask=None if m is None else m.cpu())
    dq_r, dk_r, dv_r = want
    dk_r = dk_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    dv_r = dv_r.reshape(B, Hkv, grp, Sk, D).sum(axis=2)
    for name, got, alt, ref in zip(("dq", "dk", "dv"), split1, whole, (dq_r, dk_r, dv_r)):
        assert _rel_err(got, ref, dtype) <= TOL[dtype], name
        assert _rel_err(alt, ref, dtype) <= TOL[dtype], name
        assert _rel_err(got, alt.cpu(), dtype) <= TOL[dtype], name


def test_workspace_smaller_than_asked_runs_unsplit():
    """A sweep whose partials do not fit the workspace runs unsplit (dK/dV's
    take the workspace first, then dQ's): with a few bytes short of the size
    query only dK/dV split, so dQ is bit for bit the unsplit launch's; with a
    tiny workspace nothing splits and all three gradients are."""
    B, H, Hkv, Sq, Sk, D = 1, 4, 2, 512, 512, 64
    dt = abi.dtype_code(torch.float16)
    need = abi.bwd_workspace_size(dt, B, H, Hkv, Sq, Sk, D, -1, True)
    assert need > 0
    g = torch.Generator().manual_seed(3)
    rnd = lambda h, S: torch.randn(B, h, S, D, generator=g).half().cuda()
    q, k, v, do = rnd(H, Sq), rnd(Hkv, Sk), rnd(Hkv, Sk), rnd(H, Sq)
    out, lse = abi.attn_fwd_lse(q, k, v, 0.125, True)
    short = torch.empty(need - 16, dtype=torch.uint8, device="cuda")
    tiny = torch.empty(1024, dtype=torch.uint8, device="cuda")
    a = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True, workspace=short)
    t = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True, workspace=tiny)
    w = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True, workspace=None)
    full = abi.attn_bwd(q, k, v, out, do, lse, 0.125, True, workspace=True)
    torch.cuda.synchronize()
    assert torch.equal(a[0], w[0])
    assert not torch.equal(full[0], w[0])  # the full workspace splits dQ too
    for x, y in zip(t, w):
        assert torch.equal(x, y)
