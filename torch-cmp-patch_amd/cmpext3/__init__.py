"""cmpext3 (MI355X build) -- routes torch.nn.functional.scaled_dot_product_attention
through a hand-written gfx950 fused attention forward.

Drop-in for the SDPA path of WifiLast/torch-cmp-patch's ``cmpext3`` package
(cmpext3/__init__.py there): the same import-time patch, the same
``enable()/disable()/is_enabled()/autoselect_report()`` controls, the same
``ops`` handle on the native module, the same environment knobs
(``CMPEXT3_AUTOPATCH``, ``CMPEXT3_DISABLE_OPS`` with the ``attention`` alias,
``CMPEXT3_AUTOSELECT*``, ``CMPEXT3_VERBOSE``) and the same fallback rules.

    import cmpext3          # patches F.scaled_dot_product_attention on import
    cmpext3.disable()       # stock SDPA again
    cmpext3.enable()

What runs where:
  * fp16 / bf16 [B,H,S,D] on the GPU: MFMA kernel (bf16 natively, no cast);
  * fp32 on the GPU: fp32-MFMA kernel (causal included);
  * causal (top-left, torch convention) and cross-attention (Sq != Sk) for
    every dtype; head dims up to 256; ``attn_mask`` (bool or additive) for
    every dtype, where the reference always fell back
    (cmpext3/__init__.py:624 there);
  * stock torch for ``dropout_p != 0``, non-4D inputs, live autograd, CPU
    tensors and any other dtype -- the cases where the reference itself
    falls back (cmpext3/__init__.py:624-628 there) -- and for any argument
    the native op rejects (RuntimeError/TypeError), e.g. GQA head counts or
    an empty key sequence.

Training (no counterpart in the reference, which is forward-only): with
``CMPEXT3_BACKWARD=1`` in the environment, or after ``enable_backward()``,
SDPA calls with live autograd on fp16/bf16/fp32 GPU tensors with D <= 256, equal
head counts (or grouped-query K/V under enable_gqa=True), an optional
attn_mask that needs no gradient, and no dropout run the native forward and
backward
kernels (``attention`` below, a torch.autograd.Function); everything else
with live autograd still goes to stock.  Off by default, so the default
behaviour is the reference's.

Only the attention op of the reference is in this package: its other patched
ops (linear, conv, norms, activations, ...) and its NVML clock/power side
effect are deliberately absent.
"""
from __future__ import annotations

import os
from typing import Any, Callable

import torch
import torch.nn.functional as F

try:
    from . import _native as _C
except ImportError as exc:  # the product path never runs without its kernels
    raise ImportError(
        "cmpext3 native extension not built (cmpext3/_native*.so and "
        "libcmpext3_attn.so). Build it with: python torch-cmp-patch_amd/build.py"
    ) from exc

# Raw, unpatched access to the native op(s): ops.attention(q, k, v, scale=None,
# causal=False).  Same role as the reference's `ops = _C` (cmpext3/__init__.py:216).
ops = _C

from . import autoselect  # noqa: E402

__all__ = ["enable", "disable", "is_enabled", "autoselect_report", "ops", "autoselect",
           "attention", "enable_backward", "backward_enabled"]

_SUPPORTED_DTYPES = (torch.float16, torch.float32, torch.bfloat16)
_ORIGINALS: dict[tuple[Any, str], Callable] = {}
_ENABLED = False



def _names_from_env(var: str) -> frozenset:
    """A comma-separated environment list as a set of names (blanks dropped)."""
    names = (name.strip() for name in os.environ.get(var, "").split(","))
    return frozenset(name for name in names if name)


# CMPEXT3_DISABLE_OPS=attention (or =scaled_dot_product_attention) keeps SDPA
# stock; read once at import, as the reference does (cmpext3/__init__.py:258-261).
_OP_ALIASES = {"scaled_dot_product_attention": "attention"}
_DISABLED_OPS = _names_from_env("CMPEXT3_DISABLE_OPS")


def _grad_safe(*tensors: Any) -> bool:
    """True when a forward-only kernel cannot break autograd for these tensors:
    inference mode, grad mode off, or no tensor argument requires grad."""
    if torch.is_inference_mode_enabled() or not torch.is_grad_enabled():
        return True
    return not any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


def _usable(*tensors: Any) -> bool:
    """True when every tensor argument is a GPU fp16/fp32/bf16 tensor.
    Non-tensor arguments are ignored."""
    for t in tensors:
        if isinstance(t, torch.Tensor) and (not t.is_cuda or t.dtype not in _SUPPORTED_DTYPES):
            return False
    return True


def _install(target: Any, name: str, wrapper: Callable) -> None:
    """Put `wrapper` in place of target.<name> unless the op is pinned to stock
    by CMPEXT3_DISABLE_OPS (under its own name or its alias).  The stock
    callable is remembered the first time only, so enabling twice never
    records the wrapper as the original (reference: cmpext3/__init__.py:322-329)."""
    if not _DISABLED_OPS.isdisjoint((name, _OP_ALIASES.get(name, name))):
        return
    stock = _ORIGINALS.setdefault((target, name), getattr(target, name))
    _keep_scriptable(wrapper, stock)
    setattr(target, name, wrapper)


def _keep_scriptable(wrapper: Callable, original: Callable) -> None:
    """Let torch.jit.script keep resolving the patched name to the stock op.

    TorchScript maps builtins by object identity; a Python wrapper in place of
    F.scaled_dot_product_attention would otherwise make any scripted caller
    try (and fail) to compile the wrapper.  Registering the wrapper as an
    alias of the original's aten builtin keeps scripted code on stock while
    eager calls go through the wrapper (same contract as the reference,
    cmpext3/__init__.py:332-346).
    """
    from torch.jit import _builtins
    op = _builtins._find_builtin(original)
    if op is not None:
        _builtins._register_builtin(wrapper, op)


_DTYPE_TAG = {torch.float16: "fp16", torch.float32: "fp32", torch.bfloat16: "bf16"}
# attn_mask dtypes the native op takes (bool keeps, floats are added)
_MASK_DTYPES = (torch.bool, torch.float16, torch.bfloat16, torch.float32)


_TRAIN_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_BACKWARD = os.environ.get("CMPEXT3_BACKWARD", "0") == "1"


def enable_backward(flag: bool = True) -> None:
    """Send SDPA calls with live autograd to the native forward/backward pair
    (where it applies) instead of stock torch."""
    global _BACKWARD
    _BACKWARD = bool(flag)


def backward_enabled() -> bool:
    return _BACKWARD


class _Attention(torch.autograd.Function):
    """softmax(scale * Q K^T [causal]) V with the native backward: the forward
    keeps the row log-sum-exp, the backward recomputes P from it (three
    kernels: Delta, dK/dV, dQ; no atomics)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, attn_mask):
        if attn_mask is None:
            out, lse = _C.attention_fwd_lse(q, k, v, scale, causal)
        else:
            out, lse = _C.attention_fwd_lse(q, k, v, scale, causal, attn_mask)
        ctx.save_for_backward(q, k, v, out, lse, attn_mask)
        ctx.scale, ctx.causal = scale, causal
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        q, k, v, out, lse, attn_mask = ctx.saved_tensors
        if attn_mask is None:
            dq, dk, dv = _C.attention_bwd(q, k, v, out, grad_out, lse, ctx.scale, ctx.causal)
        else:
            dq, dk, dv = _C.attention_bwd(q, k, v, out, grad_out, lse, ctx.scale, ctx.causal, attn_mask)
        return dq, dk, dv, None, None, None


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
              scale: float | None = None, causal: bool = False,
              attn_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Differentiable native attention (fp16/bf16/fp32 GPU tensors [B, H, S, D],
    D <= 256; K/V may hold fewer heads than Q when that count divides H, with
    torch's enable_gqa meaning; attn_mask as in SDPA, bool or additive, no
    gradient taken for it).  Raises RuntimeError for anything else."""
    return _Attention.apply(query, key, value, scale, causal, attn_mask)


def _training_applies(query, key, value, attn_mask, dropout_p, enable_gqa) -> bool:
    mask_ok = attn_mask is None or (isinstance(attn_mask, torch.Tensor) and attn_mask.is_cuda
                                    and attn_mask.dtype in _MASK_DTYPES and not attn_mask.requires_grad)
    if not (_BACKWARD and mask_ok and dropout_p == 0.0
            and all(isinstance(t, torch.Tensor) and t.is_cuda and t.dim() == 4
                    and t.dtype == query.dtype for t in (query, key, value))
            and query.dtype in _TRAIN_DTYPES):
        return False
    hq, hkv = query.shape[1], key.shape[1]
    heads_ok = hkv == hq or (enable_gqa and hkv >= 1 and hq % hkv == 0)
    return (heads_ok and key.shape[0] == query.shape[0] and key.shape[3] == query.shape[3]
            and value.shape == key.shape and 1 <= query.shape[3] <= 256 and key.shape[2] > 0)


def _dispatch(op: str, ref: torch.Tensor, key: tuple,
              native_call: Callable, stock_call: Callable) -> Any:
    """Serve one call from the native kernel or stock torch
    (reference: cmpext3/__init__.py:376-399).

    Autoselect on and a hashable signature: autoselect.choose measures the
    choice once per signature (correctness first, then speed).  Otherwise
    (autoselect off, or a signature that cannot key its table): the native
    kernel, and stock only when it raises RuntimeError or TypeError.
    """
    if autoselect.enabled() and _hashable(key):
        tag = _DTYPE_TAG.get(ref.dtype, ref.dtype)
        return autoselect.choose(f"{op} {tag}", key, native_call, stock_call)
    try:
        return native_call()
    except (RuntimeError, TypeError):
        return stock_call()


def _hashable(key: tuple) -> bool:
    try:
        hash(key)
    except TypeError:
        return False
    return True


def _patched_sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                  scale=None, **kwargs):
    """F.scaled_dot_product_attention replacement (reference: cmpext3/__init__.py:609-633).

    Bails to stock for dropout, non-4D query, live autograd and non-GPU /
    unsupported dtypes.  Extra keyword arguments reach only the stock call;
    the native op sees (q, k, v, scale, is_causal) positionally (plus the mask
    as a sixth argument when one is given) and rejects what it does not
    support.  Grouped-query calls (K/V with fewer heads than Q) run natively
    only under enable_gqa=True, as torch requires; without it they go to
    stock, which raises torch's own error.  An attn_mask (bool or float
    tensor) runs natively, also together with is_causal (a pair must pass
    both, torch's rule).
    """
    orig = _ORIGINALS[(F, "scaled_dot_product_attention")]

    def stock():
        return orig(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                    is_causal=is_causal, scale=scale, **kwargs)

    if (isinstance(query, torch.Tensor) and not _grad_safe(query, key, value, attn_mask)
            and _training_applies(query, key, value, attn_mask, dropout_p,
                                  bool(kwargs.get("enable_gqa", False)))):
        try:
            return _Attention.apply(query, key, value, scale, is_causal, attn_mask)
        except (RuntimeError, TypeError):
            return stock()
    if (dropout_p != 0.0
            or not isinstance(query, torch.Tensor) or query.dim() != 4
            or not _grad_safe(query, key, value, attn_mask)
            or not _usable(query, key, value)):
        return stock()
    if (isinstance(key, torch.Tensor) and key.dim() == 4 and key.shape[1] != query.shape[1]
            and not kwargs.get("enable_gqa", False)):
        return stock()
    if attn_mask is None:
        return _dispatch("attention", query,
                         (query.shape, query.dtype, key.shape, value.shape, scale, is_causal),
                         lambda: _C.attention(query, key, value, scale, is_causal),
                         stock)
    if not isinstance(attn_mask, torch.Tensor) or attn_mask.dtype not in _MASK_DTYPES:
        return stock()
    return _dispatch("attention", query,
                     (query.shape, query.dtype, key.shape, value.shape, scale, is_causal,
                      tuple(attn_mask.shape), attn_mask.dtype, attn_mask.stride()),
                     lambda: _C.attention(query, key, value, scale, is_causal, attn_mask),
                     stock)


def enable() -> None:
    """Patch F.scaled_dot_product_attention (idempotent)."""
    global _ENABLED
    if not _ENABLED and hasattr(F, "scaled_dot_product_attention"):
        _install(F, "scaled_dot_product_attention", _patched_sdpa)
    _ENABLED = True


def disable() -> None:
    """Put every patched function back to stock (no-op when not enabled)."""
    global _ENABLED
    while _ORIGINALS:
        (target, name), stock = _ORIGINALS.popitem()
        setattr(target, name, stock)
    _ENABLED = False


def is_enabled() -> bool:
    return _ENABLED


def autoselect_report() -> str:
    """Every native-vs-stock decision made so far, as printable text."""
    return autoselect.format_report()


if os.environ.get("CMPEXT3_AUTOPATCH", "1") != "0":
    enable()
