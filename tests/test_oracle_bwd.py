"""Pins for the oracle's backward restatement (oracle/sdpa_oracle.py
sdpa_bwd_np, sdpa_lse_np), CPU only.

The reference has no backward (its patch sends calls with live autograd to
stock torch, cmpext3/__init__.py:115-125), so the gradients are pinned by
what the mathematics fixes:
  * torch autograd through math SDPA in float64 (independent implementation);
  * central finite differences of sum(O * dO) on tiny shapes;
  * closed forms: one key (O = V[0] for every query), scale 0 (uniform P);
  * identities: each row of dS sums to zero, so dQ is unchanged when every
    key row is shifted by one vector and the dK rows sum to zero; P's rows sum
    to one, so the dV rows sum to the dO rows;
  * planted mistakes (no Delta term, no scale on dK, P untransposed in dV)
    each fail the autograd comparison.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sdpa_oracle as orc

SHAPES = [
    # B, H, Sq, Sk, D, causal
    (1, 2, 17, 17, 8, False),
    (2, 1, 9, 23, 16, True),     # causal, Sq < Sk (top-left)
    (1, 2, 31, 12, 40, True),    # causal, Sq > Sk
    (1, 1, 40, 33, 24, False),
]


def _rand(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def _inputs(B, H, Sq, Sk, D, seed=0):
    return (_rand((B, H, Sq, D), seed), _rand((B, H, Sk, D), seed + 1),
            _rand((B, H, Sk, D), seed + 2), _rand((B, H, Sq, D), seed + 3))


def _torch_grads(q, k, v, do, scale, causal):
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale)
    o.backward(do)
    return q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("shape", SHAPES, ids=[f"q{s[2]}k{s[3]}d{s[4]}{'c' if s[5] else ''}" for s in SHAPES])
def test_bwd_matches_torch_autograd_f64(shape):
    B, H, Sq, Sk, D, causal = shape
    q, k, v, do = _inputs(B, H, Sq, Sk, D, seed=Sq)
    scale = 0.3
    got = orc.sdpa_bwd_np(q, k, v, do, scale, causal, block=7)   # odd block: rows split across blocks
    want = _torch_grads(q, k, v, do, scale, causal)
    for g, w in zip(got, want):
        assert np.abs(g - w).max() <= 1e-10


def test_lse_matches_torch_logsumexp():
    q, k, _, _ = _inputs(1, 2, 19, 25, 16, seed=4)
    for causal in (False, True):
        s = (q @ k.transpose(-1, -2)) * 0.25
        if causal:
            s = s.masked_fill(~torch.ones(19, 25, dtype=torch.bool).tril(), -torch.inf)
        want = torch.logsumexp(s, dim=-1).numpy()
        assert np.abs(orc.sdpa_lse_np(q, k, 0.25, causal, block=5) - want).max() <= 1e-12


def test_bwd_finite_differences():
    B, H, Sq, Sk, D = 1, 1, 5, 7, 4
    q, k, v, do = _inputs(B, H, Sq, Sk, D, seed=11)
    scale, eps = 0.7, 1e-6
    grads = orc.sdpa_bwd_np(q, k, v, do, scale, True)
    loss = lambda qq, kk, vv: float((orc.sdpa_np(qq, kk, vv, scale, True) * do.numpy()).sum())
    base = [q.numpy(), k.numpy(), v.numpy()]
    rng = np.random.default_rng(0)
    for which in range(3):
        for _ in range(3):
            dirn = rng.standard_normal(base[which].shape)
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which] += eps * dirn
            minus[which] -= eps * dirn
            fd = (loss(*plus) - loss(*minus)) / (2 * eps)
            an = float((grads[which] * dirn).sum())
            assert abs(fd - an) <= 1e-7 * max(1.0, abs(an))


def test_bwd_closed_forms():
    q, k, v, do = _inputs(1, 2, 6, 1, 8, seed=2)
    dq, dk, dv = orc.sdpa_bwd_np(q, k, v, do, 0.5, False)
    # one key: O_i = V_0 whatever the scores, so only V gets a gradient (dP and
    # Delta are the same dot product, summed in different orders)
    assert np.abs(dq).max() <= 1e-12 and np.abs(dk).max() <= 1e-12
    assert np.allclose(dv[:, :, 0], do.numpy().sum(axis=2), atol=1e-12)
    # scale 0: P uniform over the keys, no gradient through the scores
    q, k, v, do = _inputs(1, 1, 5, 4, 8, seed=3)
    dq, dk, dv = orc.sdpa_bwd_np(q, k, v, do, 0.0, False)
    assert np.abs(dq).max() == 0 and np.abs(dk).max() == 0
    want = np.broadcast_to(do.numpy().sum(axis=2, keepdims=True) / 4, dv.shape)
    assert np.allclose(dv, want, atol=1e-12)


def test_bwd_identities():
    q, k, v, do = _inputs(2, 1, 13, 11, 8, seed=5)
    for causal in (False, True):
        dq, dk, dv = orc.sdpa_bwd_np(q, k, v, do, 0.4, causal)
        assert np.abs(dk.sum(axis=2)).max() <= 1e-10
        assert np.abs(dv.sum(axis=2) - do.numpy().sum(axis=2)).max() <= 1e-10
        shift = k + _rand((1, 1, 1, 8), 9)        # same vector added to every key row
        dq2, _, _ = orc.sdpa_bwd_np(q, shift, v, do, 0.4, causal)
        assert np.abs(dq2 - dq).max() <= 1e-10


def _bwd_with_mistake(q, k, v, do, scale, mistake):
    q, k, v, do = (t.numpy() for t in (q, k, v, do))
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = p @ v
    dv = (np.swapaxes(p, -1, -2) if mistake != "p_untransposed" else p) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    delta = (do * o).sum(-1, keepdims=True)
    ds = p * (dp - delta) if mistake != "no_delta" else p * dp
    dq = scale * ds @ k
    dk = (scale if mistake != "dk_no_scale" else 1.0) * np.swapaxes(ds, -1, -2) @ q
    return dq, dk, dv


@pytest.mark.parametrize("mistake", ["none", "no_delta", "dk_no_scale", "p_untransposed"])
def test_planted_mistakes_fail(mistake):
    q, k, v, do = _inputs(1, 1, 12, 12, 8, seed=7)
    want = _torch_grads(q, k, v, do, 0.5, False)
    got = _bwd_with_mistake(q, k, v, do, 0.5, mistake)
    err = max(np.abs(g - w).max() for g, w in zip(got, want))
    if mistake == "none":
        assert err <= 1e-10
    else:
        assert err > 1e-3


def _masks(B, H, Sq, Sk, seed):
    g = torch.Generator().manual_seed(seed)
    keep = torch.rand(B, H, Sq, Sk, generator=g) > 0.3
    keep[..., 0] = True                       # every row keeps key 0 (no dead rows for torch)
    pad = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
    pad[..., Sk - 3:] = False
    add = torch.randn(1, H, Sq, Sk, generator=g, dtype=torch.float64) * 2
    add[..., 1::4] = -torch.inf
    return {"bool": keep, "pad": pad, "add": add}


@pytest.mark.parametrize("kind", ["bool", "pad", "add"])
@pytest.mark.parametrize("causal", [False, True])
def test_masked_bwd_matches_torch_autograd_f64(kind, causal):
    B, H, Sq, Sk, D = 2, 2, 11, 14, 8
    q, k, v, do = _inputs(B, H, Sq, Sk, D, seed=31)
    mask = _masks(B, H, Sq, Sk, seed=32)[kind]
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, is_causal=causal, scale=0.4)
    o.backward(do)
    got = orc.sdpa_bwd_np(q, k, v, do, 0.4, causal, block=5, attn_mask=mask)
    for g, w in zip(got, (qq.grad, kk.grad, vv.grad)):
        assert np.abs(g - w.numpy()).max() <= 1e-10
    s = (q @ k.transpose(-1, -2)) * 0.4
    if causal:
        s = s.masked_fill(~torch.ones(Sq, Sk, dtype=torch.bool).tril(), -torch.inf)
    s = s.masked_fill(~mask, -torch.inf) if mask.dtype == torch.bool else s + mask
    want_lse = torch.logsumexp(s, dim=-1).numpy()
    assert np.abs(orc.sdpa_lse_np(q, k, 0.4, causal, block=5, attn_mask=mask) - want_lse).max() <= 1e-12


def test_masked_bwd_dead_rows_pass_no_gradient():
    """A row whose keys are all dropped has O = 0 (torch's result): it adds
    nothing to dK/dV and its dQ is zero; lse is -inf there."""
    q, k, v, do = _inputs(1, 1, 6, 9, 8, seed=33)
    keep = torch.ones(1, 1, 6, 9, dtype=torch.bool)
    keep[0, 0, 2] = False
    dq, dk, dv = orc.sdpa_bwd_np(q, k, v, do, 0.5, False, attn_mask=keep)
    assert np.abs(dq[0, 0, 2]).max() == 0
    rows = [i for i in range(6) if i != 2]
    dq2, dk2, dv2 = orc.sdpa_bwd_np(q[:, :, rows], k, v, do[:, :, rows], 0.5, False)
    assert np.abs(dk - dk2).max() <= 1e-12 and np.abs(dv - dv2).max() <= 1e-12
    assert orc.sdpa_lse_np(q, k, 0.5, attn_mask=keep)[0, 0, 2] == -np.inf
