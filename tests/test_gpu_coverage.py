"""GPU parity of routes the product serves beyond the BASELINE shapes.

Same bar as tests/test_gpu_parity.py (max |kernel - oracle| <= 1e-2 fp16,
2e-2 bf16, 1e-4 fp32; oracle = float64 SDPA on the CPU over the same rounded
inputs):

  * head dims that are not a whole number of 16-byte chunks, for every
    dtype, through the torch binding (ops.attention), causal and not, run
    in place (the call allocates nothing but its output);
    the reference's fp32 kernel takes any D <= 128
    (src/cuda/fp32_attention.cu:200-204);
  * head dims 160, 192 and 256 over long key sweeps (>= 1024 keys, many
    tiles, scores wide enough to force offset rescales), causal and not; the
    reference serves D = 160 at any key length
    (src/cuda/fp16_flash_attention_hfma2.cu:278-285); prefills above 128 on
    the pipelined kernel (head dims below their bucket, ragged tiles,
    grouped-query K/V, views, a key split, reruns bit-identical) and the one
    case kept on the plain kernel;
  * the reference's production sequence length S = 17402
    (cmpext3/__init__.py:16-20, tests_hardware/test_attention_bf16_routing.py:240-243),
    bf16 [1, 4, 17402, 64], causal and not: ragged in every tiling here
    (17402 = 135 * 128 + 122 = 543 * 32 + 26).  The kernel runs the whole
    problem; the oracle checks a sample of query rows that includes the first
    rows, the ragged last tile and rows spread over the sweep.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import cmpext3
from cmpext3 import abi
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu

TOL = orc.TOLERANCE


def _inputs(dtype, B, H, Sq, Sk, D, seed):
    return W.Workload("cov", dtype, B, H, Sq, Sk, D, seed=seed).make_inputs("cuda")



@pytest.mark.parametrize("dtype,D", [("fp32", 33), ("fp32", 36), ("fp32", 100), ("fp32", 3),
                                     ("bf16", 36), ("bf16", 100), ("bf16", 2),
                                     ("fp16", 33), ("fp16", 100), ("fp16", 50)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk", [(70, 50), (129, 300)])
def test_odd_head_dims_every_dtype(dtype, D, causal, Sq, Sk, run_without_copies):
    q, k, v = _inputs(dtype, 1, 2, Sq, Sk, D, seed=D * 31 + Sk)
    print(f"odd D: {dtype} D={D} Sq={Sq} Sk={Sk} causal={causal}", flush=True)
    if dtype != "fp32" and D % 2:
        # 16-bit rows of an odd element count: the binding pads them (faster
        # than the in-place 2-byte path, which test_two_byte_rows_through_the_abi covers)
        out = cmpext3.ops.attention(q, k, v, None, causal)
    else:
        out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, None, causal))
    assert out.shape == q.shape and out.dtype == q.dtype
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), None, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype,D,layout,scale,causal,shape", [
    ("fp16", 36, "bhsd", None, False, (1, 2, 256, 2048)),  # key split, 8-byte pieces
    ("bf16", 100, "bshd", None, True, (2, 3, 300, 300)),   # [B,S,H,D] view: row stride H*D
    ("fp16", 60, "bhsd", 0.0, False, (1, 2, 130, 700)),    # scale 0, ragged tiles
    ("fp16", 50, "bshd", None, False, (1, 4, 77, 77)),     # short keys, 4-byte pieces (v2 kernel)
    ("bf16", 90, "bhsd", 1.0, False, (1, 2, 200, 1000)),   # 4-byte pieces, wide scores (rescales)
])
def test_narrow_rows_in_place(dtype, D, layout, scale, causal, shape, run_without_copies):
    """Narrow-row variants (head dims that are not whole 16-byte chunks) on
    the pipelined kernel (8- and 4-byte pieces, Sk >= 256) and the v2 kernel
    (short sweeps), with the key split, BSHD views, scale 0 and scores wide
    enough to move the running offset."""
    B, H, Sq, Sk = shape
    wl = W.Workload("narrow", dtype, B, H, Sq, Sk, D, seed=D + Sq)
    q, k, v = wl.make_inputs("cuda", layout=layout)
    print(f"narrow rows: {dtype} D={D} {layout} scale={scale} causal={causal} {shape}", flush=True)
    out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, scale, causal))
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"
    assert out.stride() == q.stride() if layout == "bshd" else out.is_contiguous()


@pytest.mark.parametrize("dtype,D,offset,causal,Sq,Sk", [
    ("fp16", 33, 0, True, 200, 300),    # odd head dim: 66-byte rows
    ("bf16", 64, 1, False, 130, 77),    # 2-byte offset views of aligned rows
    ("fp16", 161, 0, False, 96, 1100),  # odd D above 128 (the v2 kernel's only path)
])
def test_two_byte_rows_through_the_abi(dtype, D, offset, causal, Sq, Sk):
    """Rows the C ABI reads in 2-byte pieces (the v2 kernel's narrow variant):
    in place, caller-allocated output, against the oracle."""
    B, H = 1, 2
    g = torch.Generator().manual_seed(D + Sk)
    dt = W.DTYPES[dtype]

    def make(S):
        flat = torch.randn(B * H * S * D + offset, generator=g).to(dt).cuda()
        return flat[offset:].view(B, H, S, D)
    q, k, v = make(Sq), make(Sk), make(Sk)
    o = make(Sq)
    print(f"2-byte rows: {dtype} D={D} offset={offset} causal={causal} Sq={Sq} Sk={Sk}", flush=True)
    scale = D ** -0.5
    assert abi.attn_fwd_raw(q, k, v, o, scale, causal) == abi.OK
    torch.cuda.synchronize()
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    err = orc.max_abs_err(o.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [160, 192, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk,scale", [(160, 1100, None), (1024, 1024, None), (96, 2049, 1.0)])
def test_large_head_dims_long_key_sweeps(dtype, D, causal, Sq, Sk, scale):
    """Many key tiles per query block on the D > 128 kernel; scale 1 spreads
    the scores over tens of log2 units, so the running offset rises on
    later tiles (rescales of O and l)."""
    q, k, v = _inputs(dtype, 1, 2, Sq, Sk, D, seed=D + Sk)
    print(f"large D: {dtype} D={D} Sq={Sq} Sk={Sk} causal={causal} scale={scale}", flush=True)
    eff = 1.0 / math.sqrt(D) if scale is None else scale
    out = abi.attn_fwd(q, k, v, eff, causal)
    torch.cuda.synchronize()
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), eff, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


WIDE_PREFILL = [
    # dtype, B, H, Hkv, Sq, Sk, D, causal, layout: head dims above 128 on the
    # pipelined kernel (unmasked inference, at least three waves of rows,
    # 256+ keys), D below its bucket (zeroed K columns), ragged tiles,
    # grouped-query K/V, [B,S,H,D] views, a key split (fewer blocks than CUs)
    ("bf16", 1, 4, 4, 300, 1000, 256, False, "bhsd"),
    ("fp16", 2, 4, 2, 257, 257, 136, True, "bhsd"),
    ("bf16", 1, 8, 2, 65, 700, 200, False, "bhsd"),     # three waves of rows
    ("fp16", 1, 2, 2, 512, 4096, 248, False, "bshd"),   # key split
    ("fp16", 1, 3, 3, 200, 333, 192, True, "bshd"),     # fp16 pre-scaled causal 192: pipelined
    ("bf16", 1, 2, 2, 130, 900, 160, True, "bhsd"),
]


@pytest.mark.parametrize("case", WIDE_PREFILL, ids=[f"{c[0]}-H{c[2]}of{c[3]}-q{c[4]}k{c[5]}d{c[6]}"
                                                    f"{'c' if c[7] else ''}-{c[8]}" for c in WIDE_PREFILL])
def test_wide_prefill_on_the_pipelined_kernel(case):
    dtype, B, H, Hkv, Sq, Sk, D, causal, layout = case
    text = abi.describe(abi.dtype_code(W.DTYPES[dtype]), B, H, Sq, Sk, D, causal)[1]
    assert "pipe16" in text and f"DK={(160 if D <= 160 else 192 if D <= 192 else 256)}" in text, text
    print(f"wide prefill {case}", flush=True)
    q = W.Workload("wq", dtype, B, H, Sq, Sk, D, seed=Sq + D).make_inputs("cuda", layout=layout)[0]
    _, k, v = W.Workload("wk", dtype, B, Hkv, Sq, Sk, D, seed=Sk + D).make_inputs("cuda", layout=layout)
    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(q, k, v, scale, causal)
    again = abi.attn_fwd(q, k, v, scale, causal)
    torch.cuda.synchronize()
    g = H // Hkv
    kx, vx = (t.cpu().repeat_interleave(g, dim=1) for t in (k, v))
    err = orc.max_abs_err(out.cpu(), orc.sdpa_np(q.cpu(), kx, vx, scale, causal))
    assert err <= TOL[dtype], f"max abs err {err:.3e}"
    assert torch.equal(out, again)


def test_wide_prefill_exception_stays_on_the_plain_kernel():
    """Causal bf16 launches of the 192 bucket keep the plain head-dim > 128
    kernel (two waves per SIMD there); its output matches the oracle."""
    assert "mfma16" in abi.describe(abi.dtype_code(torch.bfloat16), 1, 4, 300, 1000, 192, True)[1]
    q, k, v = _inputs("bf16", 1, 2, 300, 1000, 192, seed=5)
    out = abi.attn_fwd(q, k, v, 0.07, True)
    torch.cuda.synchronize()
    assert orc.max_abs_err(out.cpu(), orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), 0.07, True)) <= TOL["bf16"]


@pytest.mark.parametrize("Sk", [1, 17, 48, 49, 64, 65, 77, 80, 81, 100, 112, 113, 128])
@pytest.mark.parametrize("dtype,D", [("fp16", 64), ("bf16", 40)])
def test_short_key_slices(Sk, dtype, D):
    """The short-key kernel at every 16-key slice count (3..8 slices: the
    exponentials and PV MFMAs of slices past Sk are skipped), keys ragged
    inside a slice and at slice edges."""
    rc, text = abi.describe(abi.dtype_code(W.DTYPES[dtype]), 1, 3, 200, Sk, D)
    assert rc == abi.OK and "short16" in text and f"keys<={16 * max(3, (Sk + 15) // 16)}" in text, text
    q, k, v = _inputs(dtype, 1, 3, 200, Sk, D, seed=Sk)
    print(f"short keys: {dtype} D={D} Sk={Sk}", flush=True)
    out = abi.attn_fwd(q, k, v, D ** -0.5, False)
    torch.cuda.synchronize()
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), D ** -0.5, False)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype,D,layout,scale,shape", [
    ("fp16", 40, "bshd", None, (2, 3, 130, 77)),    # [B,S,H,D] view, D below its bucket
    ("bf16", 64, "bshd", -0.125, (1, 4, 257, 50)),  # negative scale
    ("fp16", 64, "bhsd", 0.0, (1, 2, 100, 33)),     # scale 0: uniform weights
    ("fp16", 96, "bshd", 0.5, (1, 2, 31, 128)),     # fewer rows than one wave holds
    ("bf16", 128, "bhsd", None, (1, 3, 4096, 120)),  # a long sweep of query blocks
])
def test_short_keys_layouts_and_scales(dtype, D, layout, scale, shape, run_without_copies):
    """The short-key kernel's buffer loads and stores of Q and O: row strides
    of [B,S,H,D] views (the chunks past a head dim below its bucket hold the
    next head's values, which must be neither used nor overwritten), rows past
    Sq, negative and zero scales."""
    B, H, Sq, Sk = shape
    rc, text = abi.describe(abi.dtype_code(W.DTYPES[dtype]), B, H, Sq, Sk, D)
    assert rc == abi.OK and "short16" in text, text
    wl = W.Workload("short", dtype, B, H, Sq, Sk, D, seed=D + Sk)
    q, k, v = wl.make_inputs("cuda", layout=layout)
    print(f"short keys: {dtype} D={D} {layout} scale={scale} {shape}", flush=True)
    out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, scale, False))
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), scale, False)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


@pytest.mark.parametrize("dtype,B,H,Sq,Sk,D,scale", [
    ("fp16", 2, 4, 17, 4096, 64, None),    # decode-like block: three waves hold no rows
    ("bf16", 1, 3, 33, 1000, 128, None),   # two rowless waves, ragged Sk
    ("fp16", 1, 2, 64, 777, 96, 1.0),      # exactly two rowless waves, D below its bucket, wide scores
    ("bf16", 2, 2, 80, 600, 64, None),     # one rowless wave: the ordinary variant
    ("fp16", 1, 3, 5, 3000, 40, None),     # D below its bucket (K columns zeroed by the loaders)
    ("bf16", 1, 2, 50, 513, 32, None),     # 128 chunks per K tile over 128 loader threads
    ("fp16", 2, 2, 1, 900, 72, 1.0),       # DP above DK, odd tile count
])
def test_short_query_blocks_with_rowless_waves(dtype, B, H, Sq, Sk, D, scale):
    """A single query block whose last waves hold no rows: those waves are
    the only K/V loaders (a register ring two or four tiles ahead) and leave
    before the key-split exchange; the waves with rows only compute."""
    rc, text = abi.describe(abi.dtype_code(W.DTYPES[dtype]), B, H, Sq, Sk, D)
    assert rc == abi.OK and "pipe16" in text, text
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=Sq + Sk)
    eff = 1.0 / math.sqrt(D) if scale is None else scale
    print(f"rowless waves: {dtype} B={B} H={H} Sq={Sq} Sk={Sk} D={D} scale={eff}", flush=True)
    out = abi.attn_fwd(q, k, v, eff, False)
    torch.cuda.synchronize()
    ref = orc.sdpa_c(q.cpu(), k.cpu(), v.cpu(), eff, False)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"


def _sample_rows(S, n_spread=200, seed=0):
    rng = np.random.default_rng(seed)
    tail = range(S - 150, S)                       # the ragged last block and tile
    head = range(0, 40)
    spread = rng.choice(S, size=n_spread, replace=False)
    return np.unique(np.concatenate([np.fromiter(head, int), spread, np.fromiter(tail, int)]))


@pytest.mark.parametrize("causal", [False, True])
def test_production_length_17402(causal):
    S, D = 17402, 64
    q, k, v = _inputs("bf16", 1, 4, S, S, D, seed=17402 + causal)
    print(f"S=17402 bf16 causal={causal}", flush=True)
    out = cmpext3.ops.attention(q, k, v, None, causal)
    torch.cuda.synchronize()
    rows = _sample_rows(S, seed=causal)
    qs = q.cpu()[:, :, rows]
    mask = None
    if causal:  # row r of the sample is query position rows[r]: keys 0..rows[r]
        mask = torch.from_numpy(np.arange(S)[None, :] <= rows[:, None]).view(1, 1, len(rows), S)
    ref = orc.sdpa_np(qs, k.cpu(), v.cpu(), 1.0 / math.sqrt(D), False, attn_mask=mask)
    err = orc.max_abs_err(out.cpu()[:, :, rows], ref)
    assert err <= TOL["bf16"], f"max abs err {err:.3e}"
    assert bool(torch.isfinite(out).all())


@pytest.mark.parametrize("dtype,D,bucket", [("fp16", 120, 128), ("bf16", 120, 128), ("bf16", 56, 64),
                                            ("fp16", 24, 32)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 2, 300, 300), (1, 2, 256, 2048)])
def test_head_dim_below_bucket_with_nan_past_d(dtype, D, bucket, causal, B, H, Sq, Sk):
    """Q/K/V as views of rows `bucket` elements wide whose columns past D
    hold NaN: the pipelined kernel loads whole 16-byte chunks of its bucket
    straight into LDS, and the K chunks past D must arrive as zeros (an
    out-of-range load offset), never as the NaN behind them, or 0 * NaN
    would reach every score of the row.  V chunks past D only feed output
    columns that are never stored.  The (1, 2, 256, 2048) shape also takes
    the key split when not causal."""
    q, k, v = _inputs(dtype, B, H, Sq, Sk, D, seed=D + Sk + causal)
    print(f"D below bucket: {dtype} D={D} bucket={bucket} {B}x{H}x{Sq}x{Sk} causal={causal}", flush=True)

    def wide(t):
        w = torch.full(t.shape[:-1] + (bucket,), float("nan"), dtype=t.dtype, device=t.device)
        w[..., :D] = t
        return w[..., :D]

    scale = 1.0 / math.sqrt(D)
    out = abi.attn_fwd(wide(q), wide(k), wide(v), scale, causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), scale, causal)
    err = orc.max_abs_err(out.cpu(), ref)
    assert err <= TOL[dtype], f"max abs err {err:.3e}"
