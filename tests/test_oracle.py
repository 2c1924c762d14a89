"""Pins the CPU oracle (oracle/sdpa_oracle.{c,py}) before it is trusted as the checker.

Each restatement (numpy, C, pure-Python loops) is held against things that do
not share its code:
  * torch's MATH backend of F.scaled_dot_product_attention in float64, and the
    explicit fp32 matmul -> softmax -> matmul form of the reference's own
    ground truth (tests_hardware/test_attention_causal.py:44-53);
  * the committed golden fixtures (tests/golden/sdpa_golden.npz, torch-made);
  * closed forms: a single key returns that value row; scale 0 returns the
    mean of the visible values; causal row 0 returns V[0]; with Sq == Sk the
    causal last row equals the non-causal last row;
  * invariants: permuting K and V rows together leaves non-causal O unchanged;
    adding a constant to every score of a row (via an extra Q coordinate
    paired with a constant K coordinate) leaves O unchanged.
A last test plants plausible mistakes in a copy of the oracle (dropped scale,
transposed causal mask, off-by-one diagonal, K/V rows not paired, softmax over
the wrong axis) and checks that these pins reject every one of them.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import sdpa_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "sdpa_golden.npz")


def _rand(B, H, Sq, Sk, D, seed, Dv=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, Sk, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, Sk, Dv or D, generator=g, dtype=torch.float64)
    return q, k, v


def _torch_math(q, k, v, scale, causal):
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale).numpy()


SHAPES = [
    (1, 1, 1, 1, 8), (1, 2, 7, 13, 16), (2, 3, 33, 33, 40), (1, 2, 65, 17, 64),
    (1, 1, 17, 65, 24), (2, 1, 129, 100, 128),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_numpy_and_c_match_torch_math(shape, causal):
    B, H, Sq, Sk, D = shape
    q, k, v = _rand(B, H, Sq, Sk, D, seed=sum(shape))
    scale = 0.37
    want = _torch_math(q, k, v, scale, causal)
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, scale, causal), want) < 1e-12
    assert orc.max_abs_err(orc.sdpa_c(q, k, v, scale, causal), want) < 1e-12


def test_value_head_dim_may_differ():
    q, k, v = _rand(1, 2, 9, 11, 16, seed=3, Dv=24)
    want = _torch_math(q, k, v, 0.25, False)
    assert orc.max_abs_err(orc.sdpa_c(q, k, v, 0.25), want) < 1e-12
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.25), want) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_pure_python_brute_force_agrees(causal):
    q, k, v = _rand(1, 2, 5, 6, 4, seed=7)
    a = orc.sdpa_loops(q, k, v, None, causal)
    assert orc.max_abs_err(a, orc.sdpa_c(q, k, v, None, causal)) < 1e-12
    assert orc.max_abs_err(a, orc.sdpa_np(q, k, v, None, causal)) < 1e-12
    assert orc.max_abs_err(a, _torch_math(q, k, v, 0.5, causal)) < 1e-12  # 1/sqrt(4)


def test_reference_fp32_matmul_form():
    """The reference's ground truth: fp32 matmul, triu(diagonal=1) -> -inf, softmax,
    matmul (tests_hardware/test_attention_causal.py:44-53)."""
    q, k, v = _rand(1, 4, 128, 128, 64, seed=0)
    q32, k32, v32 = q.float(), k.float(), v.float()
    scores = torch.matmul(q32, k32.transpose(-2, -1)) * 0.125
    mask = torch.triu(torch.ones(128, 128, dtype=torch.bool), diagonal=1)
    want = torch.matmul(torch.softmax(scores.masked_fill(mask, float("-inf")), -1), v32)
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.125, True), want) < 1e-5


def _golden_cases():
    data = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


def test_golden_file_present():
    data, names = _golden_cases()
    assert len(names) >= 8


@pytest.mark.parametrize("name", _golden_cases()[1])
def test_golden_vectors(name):
    data, _ = _golden_cases()
    q, k, v, want = (data[f"{name}/{x}"] for x in ("q", "k", "v", "o"))
    scale, causal = data[f"{name}/meta"]
    for fn in (orc.sdpa_np, orc.sdpa_c):
        got = fn(q, k, v, float(scale), bool(causal))
        assert orc.max_abs_err(got, want) < 1e-12, fn.__name__


@pytest.mark.parametrize("fn", [orc.sdpa_np, orc.sdpa_c, orc.sdpa_loops])
def test_single_key_returns_value_row(fn):
    q, k, v = _rand(2, 2, 6, 1, 8, seed=5)
    got = fn(q, k, v, 0.9, False)
    assert np.allclose(got, np.broadcast_to(v.numpy(), got.shape), atol=1e-14)


@pytest.mark.parametrize("fn", [orc.sdpa_np, orc.sdpa_c])
def test_zero_scale_is_mean_of_visible_values(fn):
    q, k, v = _rand(1, 2, 9, 9, 8, seed=6)
    vn = v.numpy()
    assert np.allclose(fn(q, k, v, 0.0, False), vn.mean(axis=2, keepdims=True).repeat(9, 2),
                       atol=1e-13)
    prefix = np.cumsum(vn, axis=2) / np.arange(1, 10)[None, None, :, None]
    assert np.allclose(fn(q, k, v, 0.0, True), prefix, atol=1e-13)


@pytest.mark.parametrize("fn", [orc.sdpa_np, orc.sdpa_c])
def test_causal_row_identities(fn):
    q, k, v = _rand(1, 3, 20, 20, 16, seed=8)
    c = fn(q, k, v, None, True)
    n = fn(q, k, v, None, False)
    assert np.allclose(c[:, :, 0], v.numpy()[:, :, 0], atol=1e-14)
    assert np.allclose(c[:, :, -1], n[:, :, -1], atol=1e-13)
    assert np.abs(c - n).max() > 1e-3


@pytest.mark.parametrize("fn", [orc.sdpa_np, orc.sdpa_c])
def test_joint_kv_permutation_invariance(fn):
    q, k, v = _rand(1, 2, 10, 30, 16, seed=9)
    perm = torch.randperm(30, generator=torch.Generator().manual_seed(1))
    a = fn(q, k, v, 0.3, False)
    b = fn(q, k[:, :, perm], v[:, :, perm], 0.3, False)
    assert orc.max_abs_err(a, b) < 1e-12


def test_row_shift_invariance():
    """Adding the same constant to every score of a row leaves softmax unchanged."""
    q, k, v = _rand(1, 1, 8, 12, 8, seed=10)
    q2 = torch.cat([q, torch.full((1, 1, 8, 1), 3.0, dtype=q.dtype)], -1)
    k2 = torch.cat([k, torch.ones(1, 1, 12, 1, dtype=k.dtype)], -1)
    a = orc.sdpa_np(q, k, v, 0.5, False)
    b = orc.sdpa_np(q2, k2, v, 0.5, False)
    assert orc.max_abs_err(a, b) < 1e-12


def test_empty_key_sequence_gives_zeros_like_torch():
    q, k, v = _rand(1, 1, 3, 0, 4, seed=0)
    want = _torch_math(q, k, v, 0.5, False)
    assert np.array_equal(orc.sdpa_np(q, k, v, 0.5), want)
    assert np.array_equal(orc.sdpa_c(q, k, v, 0.5), want)


# ---------------------------------------------------------------------------
# Planted mistakes: each mutant must fail at least one of the pins above.
# ---------------------------------------------------------------------------

def _mutant(kind):
    def f(q, k, v, scale=None, causal=False):
        q, k, v = (np.asarray(orc._as_f64(t)) for t in (q, k, v))
        D = q.shape[-1]
        s_ = orc.default_scale(D) if scale is None else scale
        if kind == "no_scale":
            s_ = 1.0
        s = np.einsum("bhid,bhjd->bhij", q, k) * s_
        Sq, Sk = s.shape[-2:]
        if causal:
            if kind == "mask_transposed":
                vis = np.triu(np.ones((Sq, Sk), bool))
            elif kind == "diag_off_by_one":
                vis = np.tril(np.ones((Sq, Sk), bool), k=-1) | (np.arange(Sk)[None] == 0)
            else:
                vis = np.tril(np.ones((Sq, Sk), bool))
            s = np.where(vis, s, -np.inf)
        axis = -2 if kind == "softmax_wrong_axis" else -1
        e = np.exp(s - s.max(axis=axis, keepdims=True))
        p = e / e.sum(axis=axis, keepdims=True)
        vv = v[:, :, ::-1] if kind == "kv_unpaired" else v
        return p @ vv
    return f


def _pins_pass(fn) -> bool:
    """The cheap subset of the pins above, applied to an arbitrary oracle."""
    checks = []
    for causal in (False, True):
        q, k, v = _rand(1, 2, 12, 12, 8, seed=21)
        checks.append(orc.max_abs_err(fn(q, k, v, 0.4, causal), _torch_math(q, k, v, 0.4, causal)) < 1e-10)
    q, k, v = _rand(1, 1, 6, 6, 8, seed=22)
    checks.append(np.allclose(fn(q, k, v, None, True)[:, :, 0], v.numpy()[:, :, 0]))
    return all(checks)


@pytest.mark.parametrize("kind", ["no_scale", "mask_transposed", "diag_off_by_one",
                                  "softmax_wrong_axis", "kv_unpaired"])
def test_planted_mistakes_are_caught(kind):
    assert _pins_pass(_mutant("none"))          # the unmutated restatement passes
    assert not _pins_pass(_mutant(kind))


# ---------------------------------------------------------------------------
# attn_mask (torch's SDPA rule: bool keeps where True, float is added to the
# scaled scores; broadcast to [B, H, Sq, Sk]; rows with no visible key -> 0).
# ---------------------------------------------------------------------------

def _torch_math_masked(q, k, v, scale, mask):
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale).numpy()


def _masks(B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    full = torch.rand(B, H, Sq, Sk, generator=g) > 0.4
    full[0, 0, 1] = False                                   # one row sees no key at all
    pad = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
    pad[..., Sk // 2:] = False                              # key-padding mask
    add = torch.randn(1, H, Sq, Sk, generator=g, dtype=torch.float64) * 3
    add[..., 0] = -math.inf                                 # -inf entries in a float mask
    rows = torch.randn(Sq, Sk, generator=g, dtype=torch.float64)
    return {"bool_full": full, "bool_pad": pad, "float_heads": add, "float_2d": rows}


@pytest.mark.parametrize("kind", ["bool_full", "bool_pad", "float_heads", "float_2d"])
def test_masked_oracle_matches_torch_math(kind):
    q, k, v = _rand(2, 3, 9, 13, 8, seed=41)
    mask = _masks(2, 3, 9, 13, seed=42)[kind]
    want = _torch_math_masked(q, k, v, 0.3, mask)
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.3, attn_mask=mask), want) < 1e-12
    assert orc.max_abs_err(orc.sdpa_loops(q, k, v, 0.3, attn_mask=mask), want) < 1e-12


@pytest.mark.parametrize("kind", ["bool_full", "bool_pad", "float_heads", "float_2d"])
def test_masked_causal_oracle_matches_torch_cpu(kind):
    """attn_mask with is_causal: torch's CPU SDPA (default dispatch; its MATH
    backend refuses the pair) uses a (query, key) pair only if it is causally
    visible and the mask keeps it (bool) / adds the mask to the visible pairs
    (float).  Sq < Sk and Sq > Sk both checked."""
    for sq, sk in ((9, 13), (13, 9)):
        q, k, v = _rand(2, 3, sq, sk, 8, seed=43)
        mask = _masks(2, 3, sq, sk, seed=44)[kind]
        mask = mask if kind != "bool_full" else mask.clone()
        if kind == "bool_full":
            mask[..., 0] = True          # torch's CPU path gives NaN for rows with no visible key
        want = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=True, scale=0.3).numpy()
        assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.3, causal=True, attn_mask=mask), want) < 1e-12
        assert orc.max_abs_err(orc.sdpa_loops(q, k, v, 0.3, causal=True, attn_mask=mask), want) < 1e-12


def test_fully_masked_rows_give_zeros_like_torch():
    q, k, v = _rand(1, 1, 4, 6, 8, seed=5)
    mask = torch.ones(4, 6, dtype=torch.bool)
    mask[2] = False
    out = orc.sdpa_np(q, k, v, 0.5, attn_mask=mask)
    assert np.array_equal(out[0, 0, 2], np.zeros(8))
    assert np.array_equal(out[0, 0, 2], _torch_math_masked(q, k, v, 0.5, mask)[0, 0, 2])


def test_mask_identities():
    """An all-True bool mask or an all-zero float mask changes nothing; a mask
    that keeps only key j returns V[j]; a constant added to a row's float mask
    changes nothing."""
    q, k, v = _rand(1, 2, 5, 7, 8, seed=6)
    base = orc.sdpa_np(q, k, v, 0.4)
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.4, attn_mask=torch.ones(5, 7, dtype=torch.bool)), base) < 1e-14
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.4, attn_mask=torch.zeros(5, 7)), base) < 1e-14
    only3 = torch.zeros(5, 7, dtype=torch.bool)
    only3[:, 3] = True
    got = orc.sdpa_np(q, k, v, 0.4, attn_mask=only3)
    assert np.allclose(got, np.broadcast_to(v.numpy()[:, :, 3:4], got.shape), atol=1e-14)
    shift = torch.randn(5, 1, dtype=torch.float64) * 10
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.4, attn_mask=shift.expand(5, 7)), base) < 1e-12


def test_planted_mask_polarity_mistake_is_caught():
    """Applying a bool mask inverted (keeping where False) fails the torch pin."""
    q, k, v = _rand(1, 2, 6, 9, 8, seed=8)
    mask = _masks(1, 2, 6, 9, seed=9)["bool_full"]
    want = _torch_math_masked(q, k, v, 0.3, mask)
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.3, attn_mask=mask), want) < 1e-12
    assert orc.max_abs_err(orc.sdpa_np(q, k, v, 0.3, attn_mask=~mask), want) > 1e-3
