"""CPU oracle for the fused attention forward.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only to CHECK the HIP path (or to time a CPU baseline); the
product path (the cmpext3 package) never imports it.

Three restatements of O = softmax(scale * Q K^T [causal]) V:

  sdpa_np    numpy float64, blocked over query rows (fast enough for the full
             BASELINE shapes through BLAS);
  sdpa_c     the C restatement in sdpa_oracle.c, float64, one row at a time
             (small shapes; built by `make -C oracle`);
  sdpa_loops pure-Python loops, for tiny brute-force cases only.

Reference behaviour restated (WifiLast/torch-cmp-patch):
  - math: tests_hardware/test_attention_bf16_routing.py:47-53 (fp32 matmul ->
    softmax -> matmul) and tests_hardware/test_attention_causal.py:44-53
    (causal = triu(diagonal=1) masked to -inf);
  - default scale 1/sqrt(D): src/main.cpp:1700-1703;
  - causal for Sq != Sk is top-left aligned (key j visible to query i iff
    j <= i), which is torch's is_causal convention;
  - max-abs error bar and the fp32-upcast oracle: tools/dev_flash_attn.py:24-27.
Rows with no visible key (Sk == 0, or every key masked out) give zeros, as
torch's math SDPA does (torch 2.10 CPU, pinned in tests/test_oracle.py).

attn_mask (sdpa_np, sdpa_loops): torch's scaled_dot_product_attention rule --
a bool mask keeps the (query, key) pairs where it is True, a float mask is
added to scale * Q K^T; either broadcasts to [B, H, Sq, Sk].  The reference
never ran masks natively (cmpext3/__init__.py:624 sends them to stock torch),
so the restated behaviour is torch's.

Backward (sdpa_lse_np, sdpa_bwd_np): the gradient of the same forward.  The
reference is forward-only (its patch sends every call with live autograd to
stock torch, cmpext3/__init__.py:115-125), so there is no reference code to
follow; the restatement is the calculus of softmax attention, with
P = softmax(S), S = scale * Q K^T (causal: invisible pairs at -inf):
  dV = P^T dO,  dP = dO V^T,  Delta_i = sum_d dO_id O_id = sum_j P_ij dP_ij,
  dS = P * (dP - Delta),  dQ = scale * dS K,  dK = scale * dS^T Q,
and lse_i = log sum_j exp(S_ij) (natural log).  attn_mask / causal act on S
as in the forward (invisible pairs at -inf, float masks added); a row with no
visible key has P = 0.  Pinned in tests/test_oracle_bwd.py against torch
autograd in float64 (masks included), central finite differences and closed
forms.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsdpa_oracle.so")
_lib = None


def default_scale(d: int) -> float:
    """1/sqrt(D), the scale SDPA uses when none is given (src/main.cpp:1700-1703)."""
    return 1.0 / math.sqrt(d)


def _as_f64(x) -> np.ndarray:
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", torch.float64).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(x, dtype=np.float64)


def causal_visible(sq: int, sk: int) -> np.ndarray:
    """[sq, sk] bool: key j visible to query i iff j <= i (top-left aligned)."""
    return np.tril(np.ones((sq, sk), dtype=bool))


def _mask_4d(mask, B, H, Sq, Sk):
    """attn_mask as a read-only [B, H, Sq, Sk] view: bool (keep where True) or
    float64 (additive), broadcast like torch's SDPA."""
    if mask is None:
        return None
    try:
        import torch
        if isinstance(mask, torch.Tensor):
            mask = (mask.detach().cpu().numpy() if mask.dtype == torch.bool
                    else mask.detach().to("cpu", torch.float64).numpy())
    except ImportError:  # pragma: no cover
        pass
    mask = np.asarray(mask)
    if mask.dtype != np.bool_:
        mask = mask.astype(np.float64)
    return np.broadcast_to(mask, (B, H, Sq, Sk))


def _apply_mask(s, m):
    """scores s with mask slice m (bool keep / float additive)."""
    if m is None:
        return s
    if m.dtype == np.bool_:
        return np.where(m, s, -np.inf)
    return s + m


def sdpa_np(q, k, v, scale: Optional[float] = None, causal: bool = False,
            block: int = 512, attn_mask=None) -> np.ndarray:
    """float64 SDPA over [B, H, S, D] arrays or tensors, blocked over query rows."""
    q, k, v = _as_f64(q), _as_f64(k), _as_f64(v)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    Dv = v.shape[3]
    if scale is None:
        scale = default_scale(D)
    out = np.empty((B, H, Sq, Dv), dtype=np.float64)
    if Sk == 0:
        out[...] = 0.0
        return out
    mask = _mask_4d(attn_mask, B, H, Sq, Sk)
    for b in range(B):
        for h in range(H):
            kt = k[b, h].T
            for i0 in range(0, Sq, block):
                i1 = min(Sq, i0 + block)
                s = (q[b, h, i0:i1] @ kt) * scale
                if causal:
                    vis = causal_visible(Sq, Sk)[i0:i1]
                    s = np.where(vis, s, -np.inf)
                if mask is not None:
                    s = _apply_mask(s, mask[b, h, i0:i1])
                m = s.max(axis=1, keepdims=True)
                dead = ~np.isfinite(m) & (m < 0)          # no visible key in the row
                m = np.where(dead, 0.0, m)
                with np.errstate(invalid="ignore"):
                    e = np.exp(s - m)
                    z = e.sum(axis=1, keepdims=True)
                    o = (e @ v[b, h]) / np.where(dead, 1.0, z)
                out[b, h, i0:i1] = np.where(dead, 0.0, o)
    return out


def sdpa_lse_np(q, k, scale: Optional[float] = None, causal: bool = False,
                block: int = 512, attn_mask=None) -> np.ndarray:
    """float64 [B, H, Sq] natural-log logsumexp over keys of scale * Q K^T
    (causal / attn_mask: visible keys only, float masks added; a row with no
    visible key gives -inf)."""
    q, k = _as_f64(q), _as_f64(k)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if scale is None:
        scale = default_scale(D)
    mask = _mask_4d(attn_mask, B, H, Sq, Sk)
    out = np.empty((B, H, Sq), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kt = k[b, h].T
            for i0 in range(0, Sq, block):
                i1 = min(Sq, i0 + block)
                s = (q[b, h, i0:i1] @ kt) * scale
                if causal:
                    s = np.where(causal_visible(Sq, Sk)[i0:i1], s, -np.inf)
                if mask is not None:
                    s = _apply_mask(s, mask[b, h, i0:i1])
                m = s.max(axis=1, keepdims=True)
                dead = ~np.isfinite(m) & (m < 0)
                m = np.where(dead, 0.0, m)
                with np.errstate(divide="ignore"):
                    lse = m + np.log(np.exp(s - m).sum(axis=1, keepdims=True))
                out[b, h, i0:i1] = np.where(dead, -np.inf, lse)[:, 0]
    return out


def sdpa_bwd_np(q, k, v, do, scale: Optional[float] = None, causal: bool = False,
                block: int = 512, attn_mask=None):
    """float64 gradients (dq, dk, dv) of sum(O * dO) for O = sdpa(q, k, v),
    blocked over query rows.  attn_mask as in sdpa_np; a row with no visible
    key has O = 0 and passes no gradient."""
    q, k, v, do = _as_f64(q), _as_f64(k), _as_f64(v), _as_f64(do)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if scale is None:
        scale = default_scale(D)
    mask = _mask_4d(attn_mask, B, H, Sq, Sk)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        for h in range(H):
            kt = k[b, h].T
            for i0 in range(0, Sq, block):
                i1 = min(Sq, i0 + block)
                s = (q[b, h, i0:i1] @ kt) * scale
                if causal:
                    s = np.where(causal_visible(Sq, Sk)[i0:i1], s, -np.inf)
                if mask is not None:
                    s = _apply_mask(s, mask[b, h, i0:i1])
                m = s.max(axis=1, keepdims=True)
                dead = ~np.isfinite(m) & (m < 0)                    # no visible key
                m = np.where(dead, 0.0, m)
                e = np.exp(s - m)
                z = e.sum(axis=1, keepdims=True)
                p = np.where(dead, 0.0, e / np.where(dead, 1.0, z))  # [rows, Sk]
                g = do[b, h, i0:i1]
                o = p @ v[b, h]
                dv[b, h] += p.T @ g
                dp = g @ v[b, h].T
                delta = (g * o).sum(axis=1, keepdims=True)
                ds = p * (dp - delta)
                dq[b, h, i0:i1] = scale * (ds @ k[b, h])
                dk[b, h] += scale * (ds.T @ q[b, h, i0:i1])
    return dq, dk, dv


def _load_c():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise FileNotFoundError(f"{_LIB_PATH} not built; run `make -C oracle`")
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.POINTER(ctypes.c_double)
        i64 = ctypes.c_int64
        lib.sdpa_oracle_f64.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64,
                                        ctypes.c_double, ctypes.c_int]
        lib.sdpa_oracle_f64.restype = ctypes.c_int
        _lib = lib
    return _lib


def c_available() -> bool:
    try:
        _load_c()
        return True
    except (OSError, FileNotFoundError):
        return False


def sdpa_c(q, k, v, scale: Optional[float] = None, causal: bool = False) -> np.ndarray:
    """float64 SDPA through the C restatement (sdpa_oracle.c)."""
    lib = _load_c()
    q = np.ascontiguousarray(_as_f64(q))
    k = np.ascontiguousarray(_as_f64(k))
    v = np.ascontiguousarray(_as_f64(v))
    B, H, Sq, D = q.shape
    Sk, Dv = k.shape[2], v.shape[3]
    if scale is None:
        scale = default_scale(D)
    out = np.empty((B, H, Sq, Dv), dtype=np.float64)
    p = ctypes.POINTER(ctypes.c_double)
    rc = lib.sdpa_oracle_f64(q.ctypes.data_as(p), k.ctypes.data_as(p), v.ctypes.data_as(p),
                             out.ctypes.data_as(p), B, H, Sq, Sk, D, Dv, float(scale),
                             1 if causal else 0)
    if rc != 0:
        raise RuntimeError(f"sdpa_oracle_f64 failed with code {rc}")
    return out


def sdpa_loops(q, k, v, scale: Optional[float] = None, causal: bool = False,
               attn_mask=None) -> np.ndarray:
    """Pure-Python brute force (tiny inputs only)."""
    q, k, v = _as_f64(q), _as_f64(k), _as_f64(v)
    B, H, Sq, D = q.shape
    Sk, Dv = k.shape[2], v.shape[3]
    if scale is None:
        scale = default_scale(D)
    mask = _mask_4d(attn_mask, B, H, Sq, Sk)
    out = np.empty((B, H, Sq, Dv), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for i in range(Sq):
                def add(j):
                    if mask is None or mask.dtype == np.bool_:
                        return 0.0
                    return float(mask[b, h, i, j])
                keys = [j for j in range(Sk) if (not causal or j <= i)
                        and (mask is None or mask.dtype != np.bool_ or bool(mask[b, h, i, j]))
                        and add(j) != -math.inf]
                if not keys:
                    out[b, h, i, :] = 0.0
                    continue
                s = [scale * sum(float(q[b, h, i, d]) * float(k[b, h, j, d]) for d in range(D)) + add(j)
                     for j in keys]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                z = sum(w)
                for e in range(Dv):
                    out[b, h, i, e] = sum(w[t] * float(v[b, h, j, e])
                                          for t, j in enumerate(keys)) / z
    return out


def max_abs_err(got, want) -> float:
    """max |got - want| over all elements (NaN anywhere -> inf)."""
    g, w = _as_f64(got), _as_f64(want)
    if g.shape != w.shape:
        raise ValueError(f"shape {g.shape} vs {w.shape}")
    if g.size == 0:
        return 0.0
    d = np.abs(g - w)
    if not np.all(np.isfinite(d)):
        return math.inf
    return float(d.max())


# North-star tolerances (max abs error vs the fp32/f64 CPU oracle).
TOLERANCE = {"fp16": 1e-2, "bf16": 2e-2, "fp32": 1e-4}
