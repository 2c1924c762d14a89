"""GPU parity of the key-split launches of the pipelined fp16/bf16 kernel
(and of the fp32 kernel's plans at one to two query blocks per CU, and of the
split and grouped-query row packing of the head-dim > 128 kernel).

When the query blocks do not fill whole rounds of the chip, the blocks past the
last whole round run as several workgroups over disjoint key ranges, and the
last one of a block to finish merges the partial (O, m, l) of the others.
These cases drive that path (describe() must name the split) with the same
bar as every other parity test: max |kernel - oracle| <= 1e-2 fp16, 2e-2 bf16,
oracle = float64 SDPA on the CPU over the same rounded inputs.

Shapes: fewer blocks than CUs (every block split, up to 8 parts), causal
grids of few blocks (every block cut into the same number of parts), one
whole round plus a remainder, ragged key counts whose parts get odd tile counts
(a masked padding tile inside a part), scores spread over tens of log2 units
(parts settle on different offsets before the merge), back-to-back
launches of different plans (the per-wave counters must come back to zero),
and HIP graph capture (under capture every launch runs unsplit: nothing is
allocated or cleared in the graph and it holds no workspace, so
replays on another stream beside eager split launches stay correct; replays
equal each other bit for bit and match the oracle).
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


def _inputs(dtype, B, H, Sq, Sk, D, seed=0):
    return W.Workload("split", dtype, B, H, Sq, Sk, D, seed=seed).make_inputs("cuda")


def _split_text(q, B, H, Sq, Sk, D, causal=False):
    return abi.describe(abi.dtype_code(q.dtype), B, H, Sq, Sk, D, causal)[1]


def _splits(text):
    """Does the plan cut query blocks' keys over workgroups (a key split of the
    last blocks, or a stream-K plan of equal shares)?"""
    return "key-split" in text or "stream-K" in text


def _check(q, k, v, scale, causal, dtype):
    out = abi.attn_fwd(q, k, v, scale, causal)
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"
    return out


SPLIT = [
    # dtype, B, H, Sq, Sk, D: blocks of 128 queries, 32-key tiles
    ("fp16", 1, 2, 256, 2048, 64),    # 4 blocks, 8 parts each
    ("bf16", 1, 2, 256, 2048, 64),
    ("fp16", 1, 1, 100, 1024, 128),   # one ragged block, 4 parts
    ("bf16", 2, 3, 130, 2000, 96),    # ragged Sq and Sk: parts of 15 and 16 tiles
    ("fp16", 1, 3, 64, 777, 40),      # D below the bucket, odd Sk
    ("fp16", 1, 17, 2048, 512, 64),   # one whole round + 16 blocks in 2 parts
    ("bf16", 1, 17, 2048, 512, 128),
]


@pytest.mark.parametrize("case", SPLIT, ids=[f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}" for c in SPLIT])
def test_split_parity(case):
    dtype, B, H, Sq, Sk, D = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk + D)
    text = _split_text(q, B, H, Sq, Sk, D)
    assert _splits(text), text
    _check(q, k, v, 1.0 / math.sqrt(D), False, dtype)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_split_wide_scores(dtype):
    """Q scaled by 6 (scores with a standard deviation near 9 log2 units):
    each part rescales on its own and ends on its own offset; the merge must
    bring them to a common one."""
    B, H, Sq, Sk, D = 1, 2, 200, 1500, 64
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=77)
    q = (q.float() * 6).to(q.dtype)
    assert _splits(_split_text(q, B, H, Sq, Sk, D))
    _check(q, k, v, 0.125, False, dtype)


def test_split_back_to_back_plans():
    """Different split plans in a row on one stream share the workspace;
    a rerun of the first must reproduce it bit for bit."""
    a = _inputs("fp16", 1, 2, 256, 2048, 64, seed=1)
    b = _inputs("fp16", 1, 17, 2048, 512, 64, seed=2)
    c = _inputs("bf16", 1, 1, 100, 1024, 128, seed=3)
    out_a1 = _check(*a, 0.125, False, "fp16")
    _check(*b, 0.125, False, "fp16")
    _check(*c, 128 ** -0.5, False, "bf16")
    out_a2 = _check(*a, 0.125, False, "fp16")
    assert torch.equal(out_a1, out_a2)


def test_split_bshd_views():
    """[B,S,H,D]-memory views through the split path."""
    wl = W.Workload("v", "fp16", 1, 3, 200, 1200, 64, seed=8)
    q, k, v = wl.make_inputs("cuda", layout="bshd")
    assert not q.is_contiguous()
    assert _splits(_split_text(q, 1, 3, 200, 1200, 64))
    _check(q, k, v, 0.125, False, "fp16")


def test_causal_and_whole_rounds_do_not_split():
    q = torch.empty(1, dtype=torch.float16)
    # causal sweeps too short for two parts of 16 tiles
    assert not _splits(_split_text(q, 1, 2, 256, 2048, 64, causal=True))
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        # 2 x 12 x 32 blocks = one whole round at three workgroups per CU
        assert not _splits(_split_text(q, 2, 12, 4096, 4096, 64))
        # 640 blocks (SDXL): the last 128 split; 256 blocks (one per CU):
        # equal shares of the block-tile sequence for all 768 slots
        assert "key-split: 512 whole + 128 x 2 parts" in _split_text(q, 2, 10, 4096, 4096, 64)
        assert "stream-K: 768 workgroups x 42 tiles of 256 blocks" in _split_text(q, 2, 4, 4096, 4096, 64)


CAUSAL_SPLIT = [
    # dtype, B, H, Sq, Sk, D, parts: causal grids filling at most half the
    # slots with long sweeps, or leaving most CUs without a block
    ("fp16", 1, 8, 1024, 1024, 64, 2),     # 64 blocks
    ("bf16", 1, 2, 4096, 4096, 128, 4),    # 64 blocks, 4 parts: the count-in merge
    ("bf16", 1, 8, 4096, 4096, 128, 2),    # 256 blocks of up to 128 tiles
    ("fp16", 1, 4, 1000, 3000, 64, 2),     # Sq < Sk (top-left): keys past the last query unseen
    ("fp16", 1, 4, 3000, 1000, 64, 2),     # Sq > Sk: later blocks see every key
    ("bf16", 1, 8, 2048, 2048, 256, 2),    # head dim 256, one wave per SIMD
    ("bf16", 1, 4, 2048, 2048, 192, 4),    # causal D = 192 on the head-dim > 128 kernel
    ("fp32", 1, 8, 1024, 1024, 64, 2),     # the fp32 kernel's 64-row blocks
    ("fp32", 1, 8, 1024, 1024, 256, 4),    # fp32, 16-key tiles
    ("fp32", 1, 4, 4096, 4096, 128, 2),    # fp32, 256 blocks of long sweeps
]


@pytest.mark.parametrize("case", CAUSAL_SPLIT, ids=[f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}"
                                                     for c in CAUSAL_SPLIT])
def test_causal_split_parity(case):
    """Causal blocks cut into key ranges: a part's rows either see a key in
    its first tile or none of its keys (no weight in the merge); the merged
    output meets the oracle, a rerun is bit-identical, and the training
    forward's log-sum-exp (the merging part's offset and row sum) too."""
    dtype, B, H, Sq, Sk, D, parts = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk + D)
    text = _split_text(q, B, H, Sq, Sk, D, causal=True)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert f"x {parts} parts" in text, text
    s = 1.0 / math.sqrt(D)
    out = _check(q, k, v, s, True, dtype)
    again = abi.attn_fwd(q, k, v, s, True)
    o2, lse = abi.attn_fwd_lse(q, k, v, s, True)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    qc, kc = q.cpu(), k.cpu()
    assert orc.max_abs_err(o2.cpu(), orc.sdpa_np(qc, kc, v.cpu(), s, True)) <= TOL[dtype]
    assert orc.max_abs_err(lse.cpu(), orc.sdpa_lse_np(qc, kc, s, True)) <= TOL[dtype]


def test_causal_split_with_mask():
    """A key-padding mask and causal together on a split causal grid."""
    B, H, Sq, Sk, D = 1, 8, 1024, 1024, 64
    q, k, v = _inputs("fp16", B, H, Sq, Sk, D, seed=5)
    m = torch.ones(B, 1, 1, Sk, dtype=torch.bool, device="cuda")
    m[..., 900:] = False
    out = abi.attn_fwd(q, k, v, 0.125, True, attn_mask=m)
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125, True, attn_mask=m.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= TOL["fp16"]


def test_fewer_blocks_than_cus_take_two_parts_per_cu():
    """With no whole round each CU holds two parts at once: a packed decode
    step (128 blocks of 4096 keys) is cut in 4 key ranges per block, and the
    result still matches the oracle."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("plan checked for a 256-CU MI355X")
    q, k, v = _inputs("bf16", 16, 8, 2, 4096, 128, seed=5)
    assert "key-split: 0 whole + 128 x 4 parts" in _split_text(q, 16, 8, 2, 4096, 128)
    _check(q, k, v, 128 ** -0.5, False, "bf16")


# fp32 key split: fewer query blocks (64 rows) than CUs, non-causal
SPLIT32 = [
    # B, H, Sq, Sk, D
    (1, 8, 1024, 1024, 64),   # 128 blocks, 4 parts of 8 tiles
    (1, 2, 100, 700, 40),     # 4 ragged blocks, parts of 4-5 tiles (odd counts), D = 40
    (1, 1, 20, 2000, 64),     # one short block: only 2 waves hold rows and exchange
    (1, 3, 64, 777, 96),      # D below its bucket, ragged Sk
]


@pytest.mark.parametrize("case", SPLIT32, ids=[f"fp32-B{c[0]}H{c[1]}-q{c[2]}k{c[3]}d{c[4]}" for c in SPLIT32])
def test_split_parity_fp32(case):
    B, H, Sq, Sk, D = case
    q, k, v = _inputs("fp32", B, H, Sq, Sk, D, seed=Sq + Sk + D)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _splits(_split_text(q, B, H, Sq, Sk, D)), _split_text(q, B, H, Sq, Sk, D)
    out = _check(q, k, v, 1.0 / math.sqrt(D), False, "fp32")
    # every part merges in part order: a rerun is bit-identical
    assert torch.equal(out, _check(q, k, v, 1.0 / math.sqrt(D), False, "fp32"))


def test_split_fp32_wide_scores_and_causal_unsplit():
    """Scores over tens of log2 units (each part settles on its own offset),
    and a causal fp32 launch of short sweeps, which stays whole."""
    q, k, v = _inputs("fp32", 1, 2, 128, 1500, 64, seed=31)
    q = q * 6
    _check(q, k, v, 0.125, False, "fp32")
    assert not _splits(_split_text(q, 1, 2, 128, 1500, 64, causal=True))
    _check(q, k, v, 0.125, True, "fp32")


def _replays(g, out, reps=4):
    """Replay a captured graph with eager work (and a sync) between replays."""
    results = []
    for _ in range(reps):
        g.replay()
        torch.randn(4096, device="cuda").mul_(2).sum().item()   # eager work in between
        torch.cuda.synchronize()
        results.append(out.clone())
    return results


def test_graph_capture_on_a_fresh_stream_runs_unsplit():
    """Under capture the binding takes no workspace (nothing allocated, no
    memset node): a split-eligible launch on a stream it has not seen runs
    unsplit, and every replay matches the oracle and the first replay."""
    q, k, v = _inputs("fp16", 1, 2, 256, 2048, 64, seed=21)
    assert _splits(_split_text(q, 1, 2, 256, 2048, 64))
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125)
    import cmpext3
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = cmpext3.ops.attention(q, k, v, 0.125, False)
    res = _replays(g, out)
    for r in res:
        assert orc.max_abs_err(r.cpu(), ref) <= TOL["fp16"]
        assert torch.equal(r, res[0])


def test_graph_capture_never_carries_a_streams_exchange_buffer():
    """A stream that already owns a workspace still records its launch
    unsplit under capture, so the graph holds no buffer address.  Replays on a
    second stream, running beside eager split launches on the capturing
    stream, equal each other bit for bit and match the oracle, and so do the
    eager results."""
    q, k, v = _inputs("bf16", 1, 3, 256, 2048, 64, seed=22)
    assert _splits(_split_text(q, 1, 3, 256, 2048, 64))
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125)
    import cmpext3
    s, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s):
        eager = cmpext3.ops.attention(q, k, v, 0.125, False)   # s now owns a workspace
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = cmpext3.ops.attention(q, k, v, 0.125, False)
    torch.cuda.synchronize()
    replays, eagers = [], []
    for _ in range(4):
        with torch.cuda.stream(s2):
            g.replay()
            replays.append(out.clone())
        with torch.cuda.stream(s):
            eagers.append(cmpext3.ops.attention(q, k, v, 0.125, False))
    torch.cuda.synchronize()
    for r in replays:
        assert torch.equal(r, replays[0])
        assert orc.max_abs_err(r.cpu(), ref) <= TOL["bf16"]
    for e in eagers:
        assert torch.equal(e, eager)
    assert orc.max_abs_err(eager.cpu(), ref) <= TOL["bf16"]


FP32_PLANS = [
    # B, H, Sq, Sk, D, causal, plan that describe() names on a 256-CU device
    (2, 8, 1024, 1024, 64, False, ("key-split: 256 x 2 parts", "BK=64")),   # one block per CU
    (2, 8, 1000, 1500, 128, False, ("key-split: 256 x 2 parts", "BK=32")),  # ragged, D = 128
    (1, 8, 2048, 2048, 40, False, ("key-split: 256 x 2 parts", "BK=64")),   # the D = 40 bucket
    (2, 10, 1024, 1000, 64, False, ("BK=64",)),                             # 320 blocks: unsplit
    (2, 8, 1024, 1024, 64, True, ("BK=32",)),                               # causal, short sweeps: whole
]


@pytest.mark.parametrize("case", FP32_PLANS,
                         ids=[f"B{c[0]}H{c[1]}-q{c[2]}k{c[3]}d{c[4]}{'c' if c[5] else ''}" for c in FP32_PLANS])
def test_fp32_plans_at_one_to_two_blocks_per_cu(case):
    """fp32 launches of at most one block per CU split their keys in two; up
    to two blocks per CU they run unsplit on 64-key tiles (D <= 64).  Each
    plan against the oracle at 1e-4, and a rerun bit-identical."""
    B, H, Sq, Sk, D, causal, plan = case
    q, k, v = _inputs("fp32", B, H, Sq, Sk, D, seed=Sq + Sk + D)
    text = _split_text(q, B, H, Sq, Sk, D, causal)
    print(f"fp32 plan: {text}", flush=True)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        for part in plan:
            assert part in text, text
        if len(plan) == 1:
            assert "key-split" not in text, text
    scale = D ** -0.5
    out = _check(q, k, v, scale, causal, "fp32")
    again = abi.attn_fwd(q, k, v, scale, causal)
    torch.cuda.synchronize()
    assert torch.equal(out, again)


BIG_D = [
    # dtype, B, H, Hkv, Sq, Sk, D, scale (None = 1/sqrt(D)): head dims above
    # 128 run the mfma16 kernel, one workgroup per CU; fewer blocks than CUs split
    ("fp16", 1, 16, 8, 1, 16384, 256, None),    # long-context decode: packed rows, 8 blocks x 32 parts
    ("bf16", 16, 16, 8, 1, 4096, 256, None),    # batched decode: 128 blocks x 2 parts
    ("bf16", 2, 16, 4, 5, 3000, 160, None),     # 5 query rows x 4 heads packed per K/V head, ragged Sk, 23 parts
    ("fp16", 1, 4, 4, 512, 4096, 160, None),    # prefill-like, 16 blocks x 16 parts
    ("bf16", 1, 4, 4, 100, 3000, 192, -0.07),   # ragged rows and keys, negative scale, 8 parts
    ("fp16", 1, 2, 2, 70, 2000, 199, None),     # odd head dim: element-granular rows, 15 parts
]


def _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed):
    return W.Workload("bigd", dtype, B, H, Sq, Sk, D, seed=seed, Hkv=Hkv).make_inputs("cuda")


@pytest.mark.parametrize("case", BIG_D, ids=[f"{c[0]}-B{c[1]}H{c[2]}kv{c[3]}-q{c[4]}k{c[5]}d{c[6]}" for c in BIG_D])
def test_large_head_dim_split_and_packed_rows(case):
    """Head dims above 128 with fewer query blocks than CUs: each block's keys
    are cut into parts and merged by the last part; grouped-query launches with
    few query rows pack a K/V head's query heads into one problem.  Against the
    oracle on K/V repeated per query head, and a rerun bit-identical."""
    dtype, B, H, Hkv, Sq, Sk, D, scale = case
    q, k, v = _gqa_inputs(dtype, B, H, Hkv, Sq, Sk, D, seed=Sq + Sk + D)
    print(f"large-D split: {case}", flush=True)
    if Hkv == H and torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _splits(_split_text(q, B, H, Sq, Sk, D)), _split_text(q, B, H, Sq, Sk, D)
    s = D ** -0.5 if scale is None else scale
    out = abi.attn_fwd(q, k, v, s)
    again = abi.attn_fwd(q, k, v, s)
    torch.cuda.synchronize()
    g = H // Hkv
    kx, vx = (t.cpu().repeat_interleave(g, dim=1) for t in (k, v))
    err = orc.max_abs_err(out.cpu(), orc.sdpa_np(q.cpu(), kx, vx, s))
    assert err <= TOL[dtype], f"max abs err {err:.3e}"
    assert torch.equal(out, again)


def test_large_head_dim_split_without_allocation():
    """The allocation-free entry point runs the same split through the
    library's fixed scratch (this plan's 2.1 MB fits it): bit for bit the
    workspace entry point's output."""
    q, k, v = _gqa_inputs("bf16", 1, 16, 8, 1, 16384, 256, seed=21)
    s = 256 ** -0.5
    want = abi.attn_fwd(q, k, v, s)
    got = torch.empty_like(q)
    assert abi.attn_fwd_noalloc_raw(q, k, v, got, s) == abi.OK
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_large_head_dim_split_under_graph_capture():
    """Head dims above 128 follow the same graph rules: through the binding
    a launch captured on a stream that already owns a workspace records
    unsplit (replays on a second stream beside eager split
    launches on the first stay bit-identical and match the oracle), and the
    allocation-free entry point records its split through the fixed scratch,
    whose replays equal its eager result bit for bit."""
    import cmpext3
    q, k, v = _gqa_inputs("fp16", 1, 4, 4, 1, 8192, 256, seed=23)
    assert "key-split: 4 x 32 parts" in _split_text(q, 1, 4, 1, 8192, 256) or \
        torch.cuda.get_device_properties(0).multi_processor_count != 256
    s_ = 256 ** -0.5
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), s_)
    s, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s):
        eager = cmpext3.ops.attention(q, k, v, s_, False)   # s now owns a workspace
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = cmpext3.ops.attention(q, k, v, s_, False)
    torch.cuda.synchronize()
    replays, eagers = [], []
    for _ in range(4):
        with torch.cuda.stream(s2):
            g.replay()
            replays.append(out.clone())
        with torch.cuda.stream(s):
            eagers.append(cmpext3.ops.attention(q, k, v, s_, False))
    torch.cuda.synchronize()
    for r in replays:
        assert torch.equal(r, replays[0])
        assert orc.max_abs_err(r.cpu(), ref) <= TOL["fp16"]
    for e in eagers:
        assert torch.equal(e, eager)
    assert orc.max_abs_err(eager.cpu(), ref) <= TOL["fp16"]

    # allocation-free: eager first (the scratch's address is set up outside
    # capture), then the captured split, replayed with eager work between
    want = torch.empty_like(q)
    assert abi.attn_fwd_noalloc_raw(q, k, v, want, s_) == abi.OK
    torch.cuda.synchronize()
    got = torch.empty_like(q)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        rc = abi.attn_fwd_noalloc_raw(q, k, v, got, s_, stream=s)
    assert rc == abi.OK
    for r in _replays(g2, got):
        assert torch.equal(r, want)


def test_binding_takes_its_workspace_from_torch():
    """The torch binding runs the key split through a workspace from torch's
    caching allocator (one per stream, counted by memory_allocated), and its
    output equals the C ABI's workspace entry point bit for bit; the plain
    entry point (no workspace) runs unsplit and stays within tolerance."""
    import cmpext3
    q, k, v = _inputs("fp16", 2, 10, 4096, 4096, 64, seed=31)
    need = abi.workspace_size(abi.DTYPE_F16, 2, 10, 10, 4096, 4096, 64)
    assert need > 0
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        before = torch.cuda.memory_allocated()
        out = cmpext3.ops.attention(q, k, v, 0.125, False)
        grown = torch.cuda.memory_allocated() - before
        held = cmpext3.ops.workspace_bytes(0)
    s.synchronize()
    print(f"workspace need {need} B, held {held} B, memory_allocated grew {grown} B", flush=True)
    assert held >= need
    assert grown >= need  # the output tensor plus the workspace
    via_abi = torch.empty_like(q)
    with torch.cuda.stream(s):
        assert abi.attn_fwd_raw(q, k, v, via_abi, 0.125) == abi.OK
        again = cmpext3.ops.attention(q, k, v, 0.125, False)
    s.synchronize()
    assert torch.equal(out, via_abi)
    assert torch.equal(out, again)
    plain = torch.empty_like(q)
    assert abi.attn_fwd_raw(q, k, v, plain, 0.125, workspace=False) == abi.OK
    torch.cuda.synchronize()
    ref = orc.sdpa_np(q[:, :2].cpu(), k[:, :2].cpu(), v[:, :2].cpu(), 0.125)
    assert orc.max_abs_err(plain[:, :2].cpu(), ref) <= TOL["fp16"]
    assert orc.max_abs_err(out[:, :2].cpu(), ref) <= TOL["fp16"]


def test_short_workspace_cuts_the_plan():
    """A workspace with room for fewer key ranges than the plan asks runs
    that many (here 5 of 8), within tolerance and bit-identical on rerun."""
    q, k, v = _inputs("fp16", 1, 2, 256, 2048, 64, seed=32)
    need = abi.workspace_size(abi.DTYPE_F16, 1, 2, 2, 256, 2048, 64)
    ctr = 65536
    part = (need - ctr) // 8
    rc, parts = abi.plan(abi.DTYPE_F16, 1, 2, 2, 256, 2048, 64, ctr + 5 * part)
    assert (rc, parts) == (abi.OK, 5) or torch.cuda.get_device_properties(0).multi_processor_count != 256
    import ctypes
    ws = torch.zeros(ctr + 5 * part, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        o = torch.empty_like(q)
        st = [(ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2)) for t in (q, k, v, o)]
        rc = abi.lib().cmpext3_attn_fwd_ws(
            *(ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, o)), abi.DTYPE_F16, 1, 2, 2, 256, 2048, 64,
            *st, ctypes.c_void_p(0), -1, st[0], ctypes.c_float(0.125), 0, ctypes.c_void_p(ws.data_ptr()),
            ws.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == abi.OK
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert int(ws[:ctr].count_nonzero()) == 0   # counters back at zero
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), 0.125)
    assert orc.max_abs_err(outs[0].cpu(), ref) <= TOL["fp16"]


STREAMK = [
    # dtype, B, H, Sq, Sk, D: one block per CU (256), two per CU (512),
    # bf16 D = 128 with a last round a quarter full (640 on 512 slots), and a
    # ragged key count whose shares end inside tiles of different blocks
    ("fp16", 2, 4, 4096, 4096, 64),
    ("fp16", 2, 8, 2048, 3000, 64),
    ("bf16", 2, 10, 4096, 4096, 128),
    ("bf16", 2, 4, 4000, 2500, 64),
]


@pytest.mark.parametrize("case", STREAMK, ids=[f"{c[0]}-B{c[1]}H{c[2]}-q{c[3]}k{c[4]}d{c[5]}" for c in STREAMK])
def test_streamk_parity(case):
    """Stream-K launches (equal shares of the block-tile sequence; a block cut
    between two or three workgroups merges in part order): the oracle on the
    first and last heads, every head within tolerance of the unsplit launch,
    a rerun bit-identical, and the workspace's counters back at zero."""
    dtype, B, H, Sq, Sk, D = case
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk + H)
    text = _split_text(q, B, H, Sq, Sk, D)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert "stream-K" in text, text
    s = D ** -0.5
    need = abi.workspace_size(abi.dtype_code(q.dtype), B, H, H, Sq, Sk, D)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = []
    for w in (ws, ws, False):
        o = torch.empty_like(q)
        assert abi.attn_fwd_raw(q, k, v, o, s, workspace=w) == abi.OK
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert int(ws[:abi.WORKSPACE_COUNTER_BYTES].count_nonzero()) == 0
    assert (outs[0].float() - outs[2].float()).abs().max().item() <= TOL[dtype]
    for h in (0, H - 1):
        ref = orc.sdpa_np(q[:, h:h + 1].cpu(), k[:, h:h + 1].cpu(), v[:, h:h + 1].cpu(), s)
        err = orc.max_abs_err(outs[0][:, h:h + 1].cpu(), ref)
        assert err <= TOL[dtype], f"head {h}: max abs err {err:.3e}"
