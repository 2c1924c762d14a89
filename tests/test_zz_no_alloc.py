"""GPU test of the allocation-free forward, cmpext3_attn_fwd_noalloc.

The entry point runs the same kernels as cmpext3_attn_fwd_ws; only the key
split's exchange differs (a fixed per-device array in the library instead of
the caller's workspace).  It must behave exactly like cmpext3_attn_fwd_ws
given a workspace of the array's size (CMPEXT3_NOALLOC_SCRATCH_BYTES): same
plan, so the results are equal bit for bit, and both must lie within the
north-star tolerance of the float64 oracle.  Calls run back to back, each
one smaller than the one before, and the first is repeated at the end: the
shared counters must be back at zero after every merge, or the repeat would
differ.
"""
from __future__ import annotations

import pytest
import torch

from cmpext3 import abi
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE

# name, dtype, B, H, H_kv, Sq, Sk, D, mask; in call order, largest first
CALLS = [
    # the headline: its stream-K plan needs more than the array holds, so the
    # last 128 of its 640 blocks are cut in 2 key ranges (9.4 MB of exchange)
    ("headline_fp16", "fp16", 2, 10, 10, 4096, 4096, 64, False),
    # grouped-query decode step: packed rows, one exchanging wave per block, 4 parts
    ("decode_bf16_gqa", "bf16", 16, 16, 8, 1, 4096, 128, False),
    # 4 blocks cut in 8 parts each, with a bool key-padding mask
    ("short_fp16_masked", "fp16", 1, 2, 2, 256, 2048, 64, True),
]


def _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed):
    wl = W.Workload("noalloc", dtype, B, H, Sq, Sk, D, seed=seed, Hkv=Hkv)
    return wl.make_inputs("cuda")


def _mask(B, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    keep = torch.rand(B, 1, 1, Sk, generator=g) > 0.3
    keep[..., 0] = True
    return keep.to("cuda")


def _call(raw, q, k, v, scale, mask):
    o = torch.full(q.shape, float("nan"), dtype=q.dtype, device=q.device)
    rc = raw(q, k, v, o, scale, False, attn_mask=mask)
    assert rc == abi.OK, abi.strerror(rc)
    return o


def _oracle_check(name, dtype, q, k, v, out, scale, mask, heads=2):
    """float64 oracle on the first `heads` query heads (K/V repeated per group)."""
    G = q.shape[1] // k.shape[1]
    hq = min(heads, q.shape[1])
    kk = k.repeat_interleave(G, dim=1)[:, :hq]
    vv = v.repeat_interleave(G, dim=1)[:, :hq]
    m = None if mask is None else mask.cpu()
    ref = orc.sdpa_np(q[:, :hq].cpu(), kk.cpu(), vv.cpu(), scale, False, attn_mask=m)
    err = orc.max_abs_err(out[:, :hq].cpu(), ref)
    assert err <= TOL[dtype], f"{name}: max abs err {err:.3e} > {TOL[dtype]}"


def test_noalloc_matches_the_workspace_entry_point_on_calls_in_a_row():
    results = {}
    ws = torch.zeros(abi.NOALLOC_SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    for seed, (name, dtype, B, H, Hkv, Sq, Sk, D, masked) in enumerate(CALLS):
        print(f"noalloc call {name}: {dtype} B={B} H={H}/{Hkv} Sq={Sq} Sk={Sk} D={D} mask={masked}",
              flush=True)
        q, k, v = _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed)
        mask = _mask(B, Sk, seed) if masked else None
        scale = D ** -0.5
        got = _call(abi.attn_fwd_noalloc_raw, q, k, v, scale, mask)
        want = _call(lambda *a, **kw: abi.attn_fwd_raw(*a[:6], attn_mask=kw["attn_mask"], workspace=ws),
                     q, k, v, scale, mask)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name}: differs from cmpext3_attn_fwd_ws"
        _oracle_check(name, dtype, q, k, v, got, scale, mask)
        results[name] = (q, k, v, scale, mask, got)
    # the first (largest) call again, after the smaller ones: bit for bit
    q, k, v, scale, mask, first = results[CALLS[0][0]]
    again = _call(abi.attn_fwd_noalloc_raw, q, k, v, scale, mask)
    torch.cuda.synchronize()
    assert torch.equal(again, first), "repeat of the first call differs"


def test_noalloc_passes_argument_checks_like_the_masked_entry_point():
    q, k, v = _inputs("fp16", 1, 2, 2, 64, 300, 64, 0)
    o = torch.empty_like(q)
    # a masked call whose rows are 2-byte pieces (odd head dim)
    bad = q[..., :59]
    keep = torch.ones(1, 1, 64, 300, dtype=torch.bool, device="cuda")
    assert abi.attn_fwd_noalloc_raw(bad, k[..., :59], v[..., :59], o[..., :59], 0.1,
                                    attn_mask=keep) == abi.E_HEAD_DIM
    # fp32 with a mask: the same result as the workspace entry point
    m = torch.rand(1, 1, 64, 300, device="cuda") > 0.3
    qf, kf, vf = (t.float() for t in (q, k, v))
    got, want = torch.empty_like(qf), torch.empty_like(qf)
    assert abi.attn_fwd_noalloc_raw(qf, kf, vf, got, 0.1, attn_mask=m) == abi.OK
    assert abi.attn_fwd_raw(qf, kf, vf, want, 0.1, attn_mask=m) == abi.OK
    torch.cuda.synchronize()
    assert torch.equal(got, want)


# Plans larger than the fixed scratch: cut to fewer key ranges inside the
# allocation-free entry point (the allocating plan differs, so these are
# checked against the float64 oracle and against a rerun, not against the
# workspace entry point).
OVERSIZED = [
    # 128 blocks x 4 parts of 4.7 MB partials: 18.9 MB, cut to 3 parts
    ("fp16_128x4_cut", "fp16", 1, 16, 16, 1024, 8192, 64),
    # fp32, D = 128: 128 blocks x 4 parts of 4.7 MB, cut to 3 parts
    ("fp32_128x4_cut", "fp32", 1, 8, 8, 1024, 2048, 128),
]


@pytest.mark.parametrize("case", OVERSIZED, ids=[c[0] for c in OVERSIZED])
def test_noalloc_cuts_plans_larger_than_its_scratch(case):
    name, dtype, B, H, Hkv, Sq, Sk, D = case
    print(f"noalloc oversized {name}: {dtype} B={B} H={H} Sq={Sq} Sk={Sk} D={D}", flush=True)
    q, k, v = _inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=7)
    scale = D ** -0.5
    got = _call(abi.attn_fwd_noalloc_raw, q, k, v, scale, None)
    again = _call(abi.attn_fwd_noalloc_raw, q, k, v, scale, None)
    torch.cuda.synchronize()
    assert torch.equal(got, again), f"{name}: rerun differs"
    _oracle_check(name, dtype, q, k, v, got, scale, None)
