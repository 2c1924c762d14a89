"""C ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad arguments before touching the device."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from cmpext3 import abi

REPO = Path(__file__).resolve().parents[1]


def _declared_functions():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:int|size_t|const char\*|void)\s+(cmpext3_\w+)\s*\(", text, re.M))
    return names


def test_header_declares_what_the_binding_lists():
    assert _declared_functions() == set(abi.SYMBOLS)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = _declared_functions() - exported
    assert not missing, missing
    lib = abi.lib()
    for name in _declared_functions():
        assert hasattr(lib, name)


def test_version_and_messages():
    assert abi.lib().cmpext3_attn_abi_version() == 9
    for code in range(10):
        assert abi.strerror(code) and abi.strerror(code) != "unknown error code"
    assert abi.strerror(99) == "unknown error code"


@pytest.mark.parametrize("dtype,D,expect", [
    (abi.DTYPE_F16, 64, abi.OK), (abi.DTYPE_BF16, 128, abi.OK), (abi.DTYPE_F32, 40, abi.OK),
    (abi.DTYPE_F16, 36, abi.OK), (abi.DTYPE_F32, 6, abi.OK), (abi.DTYPE_BF16, 1, abi.OK),
    (abi.DTYPE_F16, 264, abi.E_HEAD_DIM), (abi.DTYPE_F32, 0, abi.E_HEAD_DIM), (7, 64, abi.E_DTYPE),
])
def test_describe_classifies(dtype, D, expect):
    rc, text = abi.describe(dtype, 2, 10, 4096, 4096, D)
    assert rc == expect
    if rc == abi.OK:
        assert "mfma" in text
        # a head dim that is not whole 16-byte chunks runs in place on a
        # narrow-row variant
        es = 4 if dtype == abi.DTYPE_F32 else 2
        assert ("narrow rows" in text) == (D * es % 16 != 0)


def test_describe_baseline_configs():
    from cmpext3 import workloads as W
    for w in W.WORKLOADS:
        rc, text = abi.describe(abi.dtype_code(w.torch_dtype), w.B, w.H, w.Sq, w.Sk, w.D, w.causal)
        assert rc == abi.OK, text
        assert ("causal" in text) == w.causal


def test_describe_key_split_plan():
    """Without a visible device the plan assumes MI355X's 256 CUs.  SDXL
    self-attention: 640 blocks of 128 queries = 2 whole rounds + 128 blocks
    cut in 2 key ranges (one part per CU); 2*4*32 = 256 blocks fill whole
    rounds; causal launches of many blocks and short key sweeps never split;
    4 blocks of
    2048 keys (64 tiles) get 8 parts of 8 tiles.  With no whole round every
    CU holds two parts: 128 blocks of 4096 keys (a packed decode step) get
    4 parts each, 200 blocks get 2."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("plan depends on the visible device's CU count")
    f16, bf16 = abi.DTYPE_F16, abi.DTYPE_BF16
    assert "key-split: 512 whole + 128 x 2 parts" in abi.describe(f16, 2, 10, 4096, 4096, 64)[1]
    # whole CUs but a partial round of the 3 x 256 slots (one or two blocks per
    # CU, nothing left to split): stream-K, equal shares of the block-tile
    # sequence; also a last round at most half full at two workgroups per CU
    assert "stream-K: 768 workgroups x 42 tiles of 256 blocks" in abi.describe(f16, 2, 4, 4096, 4096, 64)[1]
    assert "stream-K: 768 workgroups x 85 tiles of 512 blocks" in abi.describe(f16, 2, 8, 4096, 4096, 64)[1]
    assert "stream-K: 1024 workgroups x 80 tiles of 640 blocks" in abi.describe(bf16, 2, 10, 4096, 4096, 128)[1]
    for H in (12, 16):  # one whole round; 1024 blocks past one round at three per CU
        assert "stream-K" not in abi.describe(f16, 2, H, 4096, 4096, 64)[1]
        assert "key-split" not in abi.describe(f16, 2, H, 4096, 4096, 64)[1]
    # shares under 8 tiles: the classic plan (16 blocks past one round in 2 parts)
    assert "key-split: 256 whole + 16 x 2 parts" in abi.describe(f16, 1, 17, 2048, 512, 64)[1]
    assert "key-split" not in abi.describe(f16, 2, 10, 4096, 4096, 64, True)[1]
    # causal grids of few blocks: every block in the same number of parts,
    # where they leave most CUs without a block or sweep long key ranges
    assert "key-split: 0 whole + 64 x 2 parts" in abi.describe(f16, 1, 8, 1024, 1024, 64, True)[1]
    assert "key-split: 0 whole + 256 x 2 parts" in abi.describe(bf16, 1, 8, 4096, 4096, 128, True)[1]
    assert "key-split" not in abi.describe(bf16, 1, 32, 1024, 1024, 128, True)[1]
    assert "key-split" not in abi.describe(bf16, 4, 16, 2048, 2048, 128, True)[1]
    assert "key-split" not in abi.describe(f16, 1, 2, 256, 300, 64)[1]
    assert "key-split: 0 whole + 4 x 8 parts" in abi.describe(f16, 1, 2, 256, 2048, 64)[1]
    bf16 = abi.DTYPE_BF16
    assert "key-split: 0 whole + 128 x 4 parts" in abi.describe(bf16, 16, 8, 2, 4096, 128)[1]
    assert "key-split: 0 whole + 200 x 2 parts" in abi.describe(f16, 1, 200, 100, 4096, 64)[1]
    # fp32: 64-row blocks, split only with at most one block per CU (about
    # two parts per CU, at least 4 tiles of 32 keys each), never causal
    f32 = abi.DTYPE_F32
    assert "key-split: 128 x 4 parts" in abi.describe(f32, 1, 8, 1024, 1024, 64)[1]
    assert "key-split: 256 x 2 parts" in abi.describe(f32, 2, 8, 1024, 1024, 64)[1]
    assert "key-split: 256 x 2 parts" in abi.describe(f32, 2, 8, 1024, 1024, 128)[1]
    assert "key-split" not in abi.describe(f32, 2, 10, 1024, 1024, 64)[1]
    # split launches of D <= 64 take 64-key tiles where that keeps the part
    # count, and so do unsplit non-causal ones of one to two blocks per CU
    assert "BK=64" in abi.describe(f32, 1, 8, 1024, 1024, 64)[1]
    assert "BK=64" in abi.describe(f32, 2, 8, 1024, 1024, 64)[1]
    assert "BK=32" in abi.describe(f32, 2, 8, 1024, 1024, 128)[1]
    assert "BK=64" in abi.describe(f32, 2, 10, 1024, 1024, 64)[1]
    assert "BK=64" in abi.describe(f32, 2, 16, 1024, 1024, 64)[1]
    assert "BK=32" in abi.describe(f32, 2, 17, 1024, 1024, 64)[1]
    assert "BK=32" in abi.describe(f32, 2, 10, 1024, 1024, 64, True)[1]
    assert "BK=32" in abi.describe(f32, 1, 2, 100, 700, 40)[1]
    assert "BK=32" in abi.describe(f32, 2, 8, 4096, 4096, 64)[1]
    # causal fp32: every block in the same number of parts where most CUs
    # idle (128 blocks of up to 32 tiles: 2 parts) or sweeps are long
    assert "key-split: 128 x 2 parts" in abi.describe(f32, 1, 8, 1024, 1024, 64, True)[1]
    assert "key-split" not in abi.describe(f32, 1, 12, 2048, 2048, 64, True)[1]   # 384 blocks
    assert "key-split" not in abi.describe(f32, 2, 8, 4096, 4096, 40)[1]
    assert "key-split: 4 x 5 parts" in abi.describe(f32, 1, 2, 100, 700, 40)[1]
    # decode steps (at most 16 rows per head) at head dims above 128 run the
    # decode kernel: units (batch x heads) x parts fill the CUs' workgroup
    # slots, each wave keeping at least 4 tiles of 16 keys
    assert "decode16" in abi.describe(f16, 1, 16, 1, 16384, 256)[1]
    assert "key-split: 16 x 16 parts" in abi.describe(f16, 1, 16, 1, 16384, 256)[1]
    assert "key-split: 8 x 32 parts" in abi.describe(f16, 1, 8, 1, 32768, 160)[1]
    assert "merged in groups" not in abi.describe(f16, 1, 8, 1, 32768, 160)[1]
    # deep splits of many rows merge in two levels of about sqrt(parts)
    assert "key-split: 4 x 64 parts, merged in groups of 8" in abi.describe(bf16, 1, 4, 8, 65536, 256)[1]
    assert "key-split: 1 x 128 parts, merged in groups of 12" in abi.describe(f16, 1, 1, 16, 65536, 256)[1]
    assert "key-split" not in abi.describe(bf16, 64, 8, 1, 4096, 256)[1]   # 512 units: unsplit
    assert "decode16" in abi.describe(bf16, 1, 8, 16, 4096, 64)[1]         # 8 units at D = 64
    assert "decode16" not in abi.describe(bf16, 16, 8, 1, 4096, 128)[1]    # 128 units: pipelined
    assert "decode16" not in abi.describe(bf16, 1, 8, 17, 4096, 256)[1]    # 17 rows
    # prefills at head dims above 128 (rows in at least three waves of a
    # block, 256+ keys) run the pipelined kernel at one workgroup per CU:
    # fewer blocks than CUs split into up to CUs / n parts of at least 8
    # tiles of 32 keys; causal into parts of at least 16 tiles of the last
    # block's sweep (1024 keys: 2 parts)
    assert "key-split: 0 whole + 64 x 4 parts" in abi.describe(f16, 1, 8, 1024, 4096, 160)[1]
    assert "key-split: 0 whole + 4 x 11 parts" in abi.describe(bf16, 1, 4, 100, 3000, 192)[1]
    assert "key-split: 0 whole + 2 x 11 parts" in abi.describe(bf16, 1, 2, 70, 3000, 160)[1]
    assert "key-split: 0 whole + 64 x 2 parts" in abi.describe(f16, 1, 8, 1024, 4096, 160, True)[1]
    assert "key-split" not in abi.describe(f16, 2, 10, 1024, 1024, 160)[1]
    assert "pipe16" in abi.describe(f16, 1, 4, 300, 1000, 192, True)[1]
    # causal bf16 192 keeps the plain kernel (two waves per SIMD fit there),
    # and so do blocks with rows in at most two waves: up to CUs / n parts of
    # at least 4 tiles (at most 32; 8 from the 192 bucket up when every wave
    # of a block holds rows)
    assert "mfma16" in abi.describe(bf16, 1, 4, 300, 1000, 192, True)[1]
    assert "mfma16" in abi.describe(bf16, 1, 4, 40, 3000, 192)[1]
    assert "key-split: 4 x 23 parts" in abi.describe(bf16, 1, 4, 40, 3000, 192)[1]


def _call(q=16, k=16, v=16, o=16, dtype=abi.DTYPE_F16, B=1, H=1, Sq=8, Sk=8, D=64,
          strides=(512, 512, 64), scale=0.125):
    st = (ctypes.c_int64 * 3)(*strides)
    return abi.lib().cmpext3_attn_fwd(ctypes.c_void_p(q), ctypes.c_void_p(k), ctypes.c_void_p(v),
                                      ctypes.c_void_p(o), dtype, B, H, Sq, Sk, D, st, st, st, st,
                                      ctypes.c_float(scale), 0, None)


# Fake device addresses: every case below must be rejected before any launch.
# (Odd head dims and 2-byte aligned rows are accepted by the unmasked entry
# points, so they appear here only with a mask, which needs 4-byte pieces.)
def test_rejections_before_launch():
    assert _call(dtype=5) == abi.E_DTYPE
    assert _call(B=-1) == abi.E_INVALID
    assert _call(D=0) == abi.E_HEAD_DIM
    assert _call(D=257) == abi.E_HEAD_DIM
    assert _call(Sk=0) == abi.E_EMPTY_KEYS
    assert _call(q=0) == abi.E_INVALID
    assert _call(q=25) == abi.E_ALIGN                      # not element-aligned
    assert _call(dtype=abi.DTYPE_F32, o=18) == abi.E_ALIGN  # fp32 needs 4 bytes
    assert _call(strides=(512, 512, -64)) == abi.E_INVALID
    assert _call(scale=float("inf")) == abi.E_INVALID
    assert _call(scale=float("nan")) == abi.E_INVALID
    # masked f16/bf16 calls run rows of 4- or 8-byte pieces in place; 2-byte
    # pieces (odd head dim, pointer or stride) are refused
    assert _call_masked_layout(D=13) == abi.E_HEAD_DIM
    assert _call_masked_layout(q=18) == abi.E_ALIGN
    assert _call_masked_layout(strides=(512, 512, 61)) == abi.E_ALIGN
    # masks: any layout with element-aligned rows (read element by element
    # unless they allow runs of 8 keys), but not a misaligned element, a
    # negative stride, or a mask without runs for the training entry points
    assert _call_masked_layout(mask=17, mask_dtype=abi.DTYPE_F16) == abi.E_ALIGN
    assert _call_masked_layout(mask=18, mask_dtype=abi.DTYPE_F32) == abi.E_ALIGN
    assert _call_masked_layout(mask_str=(0, -8, 0)) == abi.E_ALIGN
    assert _call_masked(Sk=64, lse=16, mask_str=(0, 0, 66)) == abi.E_ALIGN      # row stride % 4


def _call_masked_layout(q=16, D=64, strides=(512, 512, 64), mask=16, mask_dtype=abi.DTYPE_BOOL,
                        mask_str=(0, 0, 0)):
    st = (ctypes.c_int64 * 3)(*strides)
    ms = (ctypes.c_int64 * 3)(*mask_str)
    return abi.lib().cmpext3_attn_fwd_masked(ctypes.c_void_p(q), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                             ctypes.c_void_p(16), abi.DTYPE_F16, 1, 1, 1, 8, 8, D, st, st,
                                             st, st, ctypes.c_void_p(mask), mask_dtype, ms,
                                             ctypes.c_float(0.125), 0, None)


def test_empty_problem_is_a_noop_even_without_pointers():
    assert _call(q=0, k=0, v=0, o=0, Sq=0) == abi.OK
    assert _call(q=0, k=0, v=0, o=0, B=0) == abi.OK


def _call_gqa(H=4, H_kv=2, q=16, dtype=abi.DTYPE_F16, B=1, Sq=8, Sk=8, D=64):
    st = (ctypes.c_int64 * 3)(2048, 512, 64)
    return abi.lib().cmpext3_attn_fwd_gqa(ctypes.c_void_p(q), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                          ctypes.c_void_p(16), dtype, B, H, H_kv, Sq, Sk, D,
                                          st, st, st, st, ctypes.c_float(0.125), 0, None)


def test_gqa_head_counts_are_checked_before_launch():
    """K/V head count must divide the query head count; checked after the
    shape checks and before any launch (fake addresses, no GPU touched)."""
    assert _call_gqa(H=4, H_kv=3, q=0) == abi.E_INVALID
    assert _call_gqa(H=4, H_kv=3) == abi.E_INVALID
    assert _call_gqa(H=4, H_kv=0) == abi.E_INVALID
    assert _call_gqa(H=4, H_kv=8) == abi.E_INVALID
    assert _call_gqa(H=4, H_kv=-1) == abi.E_INVALID
    assert _call_gqa(H=4, H_kv=2, dtype=9) == abi.E_DTYPE
    assert _call_gqa(H=4, H_kv=2, Sq=0, q=0) == abi.OK   # empty problem


def _call_lse(lse=16, dtype=abi.DTYPE_F16, D=64, q=16, Sq=8, Sk=8, scale=0.125):
    st = (ctypes.c_int64 * 3)(512, 512, 64)
    vp = ctypes.c_void_p
    return abi.lib().cmpext3_attn_fwd_lse(vp(q), vp(16), vp(16), vp(16), vp(lse), dtype, 1, 1, 1, Sq, Sk,
                                          D, st, st, st, st, vp(0), -1, st, ctypes.c_float(scale), 0,
                                          vp(0), 0, None)


def _call_bwd(delta=16, lse=16, dtype=abi.DTYPE_F16, D=64, dq=16, Sq=8, Sk=8, scale=0.125,
              strides=(512, 512, 64), H=1, H_kv=1, mask=0, mask_dtype=-1, mask_str=(0, 0, 0)):
    st = (ctypes.c_int64 * 3)(*strides)
    vp = ctypes.c_void_p
    return abi.lib().cmpext3_attn_bwd(vp(16), vp(16), vp(16), vp(16), vp(16), vp(lse), vp(dq), vp(16),
                                      vp(16), vp(delta), dtype, 1, H, H_kv, Sq, Sk, D,
                                      *([st] * 8), vp(mask), mask_dtype, (ctypes.c_int64 * 3)(*mask_str),
                                      ctypes.c_float(scale), 1, None)


def test_training_entry_points_reject_before_launch():
    """Fake device addresses: each case must be turned down on the host."""
    assert _call_lse(dtype=abi.DTYPE_F32, D=66) == abi.E_HEAD_DIM   # fp32 training: D a multiple of 4
    assert _call_lse(D=264) == abi.E_HEAD_DIM
    assert _call_lse(lse=0) == abi.E_INVALID
    assert _call_lse(lse=18) == abi.E_INVALID
    assert _call_lse(q=24) == abi.E_ALIGN
    assert _call_lse(D=36) == abi.E_HEAD_DIM               # training needs whole chunks
    assert _call_lse(Sk=0) == abi.E_EMPTY_KEYS
    assert _call_lse(lse=0, q=0, Sq=0) == abi.OK          # empty problem
    assert _call_bwd(dtype=abi.DTYPE_F32, D=62) == abi.E_HEAD_DIM
    assert _call_bwd(dtype=abi.DTYPE_F32, strides=(512, 512, 66)) == abi.E_ALIGN
    assert _call_bwd(D=260) == abi.E_HEAD_DIM
    assert _call_bwd(D=36) == abi.E_HEAD_DIM
    assert _call_bwd(delta=0) == abi.E_INVALID
    assert _call_bwd(lse=0) == abi.E_INVALID
    assert _call_bwd(delta=18) == abi.E_ALIGN
    assert _call_bwd(dq=24) == abi.E_ALIGN
    assert _call_bwd(strides=(512, 512, 60)) == abi.E_ALIGN
    assert _call_bwd(scale=float("nan")) == abi.E_INVALID
    assert _call_bwd(strides=(1 << 40, 1 << 40, 1 << 26)) == abi.E_TOO_LARGE
    assert _call_bwd(delta=0, Sq=0) == abi.OK
    assert _call_bwd(H=4, H_kv=3) == abi.E_INVALID
    assert _call_bwd(H=4, H_kv=0) == abi.E_INVALID
    assert _call_bwd(mask=0, mask_dtype=abi.DTYPE_BOOL) == abi.E_INVALID
    assert _call_bwd(mask=16, mask_dtype=7) == abi.E_DTYPE
    assert _call_bwd(mask=24, mask_dtype=abi.DTYPE_BOOL) == abi.E_ALIGN
    assert _call_bwd(mask=16, mask_dtype=abi.DTYPE_BOOL, mask_str=(0, 0, 6)) == abi.E_ALIGN


def test_training_plans():
    """Short-query training forwards above D = 128 (f16, bf16; the
    head-dim > 128 kernel) run unsplit (no workspace), masked or not; the fp32
    training forward key-splits small non-causal grids like the inference
    forward (the merging part writes the log-sum-exp), causal ones by the
    causal plan of the inference forward."""
    for dt in (abi.DTYPE_F16, abi.DTYPE_BF16):
        for D in (136, 160, 192, 200, 256):
            for mdt in (-1, abi.DTYPE_BOOL):
                assert abi.workspace_size(dt, 1, 8, 8, 16, 8192, D, mdt, with_lse=True) == 0
                assert abi.plan(dt, 1, 8, 8, 16, 8192, D, 1 << 30, mdt, with_lse=True) == (abi.OK, 1)
    for D in (8, 40, 64, 100, 128, 256):
        for mdt in (-1, abi.DTYPE_F32):
            train = abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, D, 1 << 30, mdt, with_lse=True)
            assert train == abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, D, 1 << 30, mdt)
            assert train[0] == abi.OK and train[1] >= 2
            assert abi.workspace_size(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, D, mdt, with_lse=True) > 0
            assert abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, D, 1 << 30, mdt, True, with_lse=True) == \
                abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, D, 1 << 30, mdt, True)
    # BASELINE config 1's shape: 128 blocks x 4 parts, training or not
    assert abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, 64, 1 << 30) == (abi.OK, 4)
    assert abi.plan(abi.DTYPE_F32, 1, 8, 8, 1024, 1024, 64, 1 << 30, with_lse=True) == (abi.OK, 4)
    # f16/bf16 training prefills above D = 128 take the pipelined kernel,
    # which splits small grids like the inference launch (64 blocks x 4 parts)
    need = abi.workspace_size(abi.DTYPE_BF16, 1, 8, 8, 1024, 4096, 256, with_lse=True)
    assert need > 0
    assert abi.plan(abi.DTYPE_BF16, 1, 8, 8, 1024, 4096, 256, need, with_lse=True) == (abi.OK, 4)


def _call_masked(k_row=64, q_row=64, o_row=64, Sk=1 << 17, Sq=1, mask_str=(0, 0, 0), lse=0,
                 mask_dtype=abi.DTYPE_BOOL):
    """A masked (or training) call whose K/V rows sit k_row elements apart:
    fake, aligned device addresses, so only the host checks may run."""
    vp = ctypes.c_void_p
    q_st = (ctypes.c_int64 * 3)(q_row * Sq, q_row * Sq, q_row)
    kv_st = (ctypes.c_int64 * 3)(k_row * Sk, k_row * Sk, k_row)
    o_st = (ctypes.c_int64 * 3)(o_row * Sq, o_row * Sq, o_row)
    m_st = (ctypes.c_int64 * 3)(*mask_str)
    if lse:
        return abi.lib().cmpext3_attn_fwd_lse(vp(16), vp(16), vp(16), vp(16), vp(lse), abi.DTYPE_F16, 1,
                                              1, 1, Sq, Sk, 64, q_st, kv_st, kv_st, o_st, vp(16),
                                              mask_dtype, m_st, ctypes.c_float(0.125), 0, vp(0), 0, None)
    return abi.lib().cmpext3_attn_fwd_masked(vp(16), vp(16), vp(16), vp(16), abi.DTYPE_F16, 1, 1, 1, Sq,
                                             Sk, 64, q_st, kv_st, kv_st, o_st, vp(16), mask_dtype, m_st,
                                             ctypes.c_float(0.125), 0, None)


def test_mask_is_never_dropped_for_wide_kv_rows():
    """Only the pipelined kernel applies masks, and it addresses the whole
    key sweep with 32-bit offsets.  A long masked sweep over K/V rows of a
    packed QKV buffer (row stride 3 * 16 heads * 64) exceeds that: the call
    must be refused (so the binding falls back to stock), not run unmasked."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("fake device addresses: host-side checks only")
    wide = 3 * 32 * 128  # 131072 keys of 24 KiB rows: 3.2 GB past the first row
    assert _call_masked(k_row=wide, Sk=1 << 17) == abi.E_TOO_LARGE
    assert _call_masked(k_row=wide, Sk=1 << 17, mask_dtype=abi.DTYPE_F32) == abi.E_TOO_LARGE
    assert _call_masked(k_row=wide, Sk=1 << 17, lse=16, mask_dtype=-1) == abi.E_TOO_LARGE


def test_training_forward_refuses_what_its_backward_would():
    """The backward addresses Q and dO (laid out like O) with 32-bit tile
    offsets; the training forward checks the same, so a step never passes
    the forward and then fails in the backward (where autograd has no stock
    fallback)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("fake device addresses: host-side checks only")
    wide, Sq = 3 * 32 * 128, 1 << 17
    # the backward refuses Q or dO rows this wide (one stride for all operands here)
    assert _call_bwd(strides=(wide * Sq, wide * Sq, wide), Sq=Sq, Sk=64) == abi.E_TOO_LARGE
    for q_row, o_row in ((wide, 64), (64, wide)):
        fwd = _call_masked(q_row=q_row, o_row=o_row, Sq=Sq, Sk=64, lse=16, mask_dtype=-1)
        assert fwd == abi.E_TOO_LARGE


def test_workspace_size_and_plan():
    """The workspace a problem's full key-split plan takes (64 KiB of counters,
    then one 1 KiB vector per lane set for every (split block, part, wave)),
    and the plan a launch takes with a given workspace: none -> unsplit, too
    little -> fewer key ranges or none, enough -> the full plan.  Host-only
    dry runs of the launch's own dispatch (256 CUs without a device)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("plan depends on the visible device's CU count")
    f16, bf16, f32 = abi.DTYPE_F16, abi.DTYPE_BF16, abi.DTYPE_F32
    ctr, vec = 65536, 64 * 16
    # SDXL self-attention: 128 split blocks x 2 parts x 4 waves x (64/8 + 1) vectors
    need = abi.workspace_size(f16, 2, 10, 10, 4096, 4096, 64)
    assert need == ctr + 128 * 2 * 4 * 9 * vec
    assert abi.plan(f16, 2, 10, 10, 4096, 4096, 64, 0) == (abi.OK, 1)          # null workspace: unsplit
    assert abi.plan(f16, 2, 10, 10, 4096, 4096, 64, need) == (abi.OK, 2)
    assert abi.plan(f16, 2, 10, 10, 4096, 4096, 64, need - 1) == (abi.OK, 1)   # less than 2 parts fit
    assert abi.plan(f16, 2, 10, 10, 4096, 4096, 64, 1 << 40) == (abi.OK, 2)
    # one block per CU, stream-K: 256 blocks x (128 / 42 + 2 = 5) part slots;
    # without room for it the classic plan, which leaves such a grid unsplit
    need = abi.workspace_size(f16, 2, 4, 4, 4096, 4096, 64)
    assert need == ctr + 256 * 5 * 4 * 9 * vec
    assert abi.plan(f16, 2, 4, 4, 4096, 4096, 64, need) == (abi.OK, 5)
    assert abi.plan(f16, 2, 4, 4, 4096, 4096, 64, need - 1) == (abi.OK, 1)
    # 4 blocks of 2048 keys, 8 parts; a workspace for 5 of them gets 5
    need = abi.workspace_size(f16, 1, 2, 2, 256, 2048, 64)
    assert need == ctr + 4 * 8 * 4 * 9 * vec
    assert abi.plan(f16, 1, 2, 2, 256, 2048, 64, ctr + 4 * 5 * 4 * 9 * vec) == (abi.OK, 5)
    # masked, and the training forward: the same plan and size
    assert abi.workspace_size(f16, 1, 2, 2, 256, 2048, 64, mask_dtype=abi.DTYPE_BOOL) == need
    assert abi.workspace_size(f16, 1, 2, 2, 256, 2048, 64, with_lse=True) == need
    assert abi.plan(f16, 1, 2, 2, 256, 2048, 64, need, with_lse=True) == (abi.OK, 8)
    # grouped-query decode (packed rows: one exchanging wave per block), D = 128
    need = abi.workspace_size(bf16, 16, 16, 8, 1, 4096, 128)
    assert need == ctr + 128 * 4 * 1 * 17 * vec
    assert abi.plan(bf16, 16, 16, 8, 1, 4096, 128, need) == (abi.OK, 4)
    # fp32 config 1: 128 blocks x 4 parts x 4 waves x (4 + 1) vectors
    need = abi.workspace_size(f32, 1, 8, 8, 1024, 1024, 64)
    assert need == ctr + 128 * 4 * 4 * 5 * vec
    assert abi.plan(f32, 1, 8, 8, 1024, 1024, 64, need) == (abi.OK, 4)
    assert abi.plan(f32, 1, 8, 8, 1024, 1024, 64, 0) == (abi.OK, 1)
    # head dim 256 decode on the decode kernel: 16 units x 16 parts
    assert abi.plan(f16, 1, 16, 16, 1, 16384, 256, 1 << 30) == (abi.OK, 16)
    # never split: causal grids of many blocks, whole rounds, short keys
    for args in ((f16, 2, 10, 10, 4096, 4096, 64, -1, True), (f16, 2, 12, 12, 4096, 4096, 64),
                 (f16, 2, 10, 10, 4096, 77, 64)):
        assert abi.workspace_size(*args) == 0
    # errors: the size is 0 and the plan reports the code
    assert abi.workspace_size(f16, 1, 1, 1, 8, 8, 300) == 0
    assert abi.plan(f16, 1, 1, 1, 8, 8, 300, 0) == (abi.E_HEAD_DIM, 0)
    assert abi.plan(f32, 1, 1, 1, 8, 8, 64, 0, mask_dtype=abi.DTYPE_BOOL) == (abi.OK, 1)  # fp32 masks run
    assert abi.plan(f16, 1, 4, 3, 8, 8, 64, 0) == (abi.E_INVALID, 0)


def test_workspace_alignment_is_checked_before_launch():
    st = (ctypes.c_int64 * 3)(512, 512, 64)
    vp = ctypes.c_void_p
    rc = abi.lib().cmpext3_attn_fwd_ws(vp(16), vp(16), vp(16), vp(16), abi.DTYPE_F16, 1, 1, 1, 8, 8, 64,
                                       st, st, st, st, vp(0), -1, st, ctypes.c_float(0.125), 0,
                                       vp(24), 1 << 20, None)
    assert rc == abi.E_ALIGN


def test_bwd_workspace_plan():
    """The backward splits a gradient sweep only with too few blocks for the
    CU slots (256 CUs without a visible device): a split dK/dV sweep asks for
    ns x B x H_kv x Sk x D x 2 fp32 partials, a split dQ sweep for
    ns_q x B x H x Sq x D; the Qwen3 and SDXL training shapes and invalid
    arguments ask for nothing."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("plan depends on the visible device's CU count")
    f16, bf16, f32 = abi.DTYPE_F16, abi.DTYPE_BF16, abi.DTYPE_F32
    kv = lambda ns, B, Hkv, Sk, D: ns * B * Hkv * Sk * D * 2 * 4
    dq = lambda ns, B, H, Sq, D: ns * B * H * Sq * D * 4
    assert abi.bwd_workspace_size(bf16, 4, 16, 16, 2048, 2048, 128, -1, True) == 0     # Qwen3 shape
    # SDXL shape: 640 blocks at three per CU, the last 128 in 2 parts (split
    # tails: block-indexed partials of 128 rows)
    tail = lambda ns, nsb, D: ns * nsb * 128 * D * 4
    assert abi.bwd_workspace_size(f16, 2, 10, 10, 4096, 4096, 64, -1, False) == \
        2 * tail(2, 128, 64) + tail(2, 128, 64)
    assert abi.bwd_workspace_size(f16, 2, 12, 12, 4096, 4096, 64, -1, False) == 0      # whole rounds
    # fp32: 64-row blocks; BASELINE config 1's 128 key blocks (3 workgroups per
    # CU) take 6 parts and its 128 query blocks (4 per CU) 8; SD1.5's none
    assert abi.bwd_workspace_size(f32, 1, 8, 8, 1024, 1024, 64, -1, False) == \
        kv(6, 1, 8, 1024, 64) + dq(8, 1, 8, 1024, 64)
    assert abi.bwd_workspace_size(f32, 2, 8, 8, 4096, 4096, 40, -1, False) == 0
    assert abi.bwd_workspace_size(bf16, 1, 32, 7, 4096, 4096, 128, -1, True) == 0      # 7 does not divide 32
    assert abi.bwd_workspace_size(bf16, 1, 32, 8, 4096, 4096, 128, -1, True) == kv(4, 1, 8, 4096, 128)
    assert abi.bwd_workspace_size(bf16, 1, 32, 8, 4096, 4096, 129, -1, True) == 0      # rows off 16 bytes
    # grouped-query K/V: only the dK/dV grid is small (the dQ grid has every
    # query head); causal: two rounds of the 512 slots (2 waves per SIMD at
    # D = 128), non-causal one
    assert abi.bwd_workspace_size(bf16, 2, 32, 8, 4096, 4096, 128, -1, True) == kv(2, 2, 8, 4096, 128)
    assert abi.bwd_workspace_size(bf16, 1, 32, 8, 4096, 4096, 128, -1, False) == kv(2, 1, 8, 4096, 128)
    # one wave per SIMD: D = 256, and masked causal D = 128
    assert abi.bwd_workspace_size(bf16, 1, 16, 8, 4096, 4096, 256, -1, True) == kv(2, 1, 8, 4096, 256)
    assert abi.bwd_workspace_size(bf16, 2, 32, 8, 4096, 4096, 128, 3, True) == 0
    # few sequences and heads: both sweeps split, at most 8 parts each, each
    # part at least 4 tiles of the longest sweep
    assert abi.bwd_workspace_size(f16, 1, 2, 2, 4096, 4096, 64, -1, False) == \
        kv(8, 1, 2, 4096, 64) + dq(8, 1, 2, 4096, 64)
    assert abi.bwd_workspace_size(f16, 1, 2, 2, 260, 200, 64, -1, False) == kv(2, 1, 2, 200, 64)
    assert abi.bwd_workspace_size(f16, 1, 2, 2, 260, 700, 64, -1, False) == \
        kv(2, 1, 2, 700, 64) + dq(5, 1, 2, 260, 64)
    assert abi.bwd_workspace_size(f16, 1, 2, 2, 100, 200, 64, -1, False) == 0
