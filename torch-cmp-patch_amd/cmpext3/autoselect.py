"""Per-signature choice between the native kernel and stock torch, made at run time.

Same contract as the reference's chooser (cmpext3/autoselect.py there,
choose/_probe/_mismatch/_time at :200-364):

  * the first call with a new signature runs BOTH implementations once
    (untimed: this also pays module load / first-launch costs);
  * correctness gate before speed: if the native output's shape differs, it
    holds NaN/Inf, or max|native - stock| / max|stock| exceeds the dtype's
    tolerance, stock is used for that signature from then on (with a one-time
    warning);
  * otherwise both are timed and the faster one is cached for the signature;
    the loser never runs again for it;
  * a native RuntimeError/TypeError at probe time is a permanent "stock here";
    at steady state it serves that one call from stock and keeps the decision;
  * an out-of-memory during the probe serves the call from stock and records
    nothing (the probe holds two outputs at once);
  * after 64 probed signatures of one op, new signatures are not probed but
    inherit the majority verdict of that op.

Knobs (read at import): CMPEXT3_AUTOSELECT=0 (always native, stock only on an
exception), CMPEXT3_VERBOSE=1 (print decisions to stderr),
CMPEXT3_AUTOSELECT_BUDGET_MS (timing budget per candidate, default 20, min 1),
CMPEXT3_AUTOSELECT_TOLERANCE (one relative tolerance for every dtype).
"""
from __future__ import annotations

import math
import os
import sys
import time
from typing import Any, Callable

import torch


def _flag(name: str, default: str) -> bool:
    return os.environ.get(name, default) not in ("0", "", "false", "False")


_ENABLED = _flag("CMPEXT3_AUTOSELECT", "1")
_VERBOSE = _flag("CMPEXT3_VERBOSE", "0")

try:
    _BUDGET_S = max(1.0, float(os.environ.get("CMPEXT3_AUTOSELECT_BUDGET_MS", "20"))) / 1000.0
except ValueError:
    _BUDGET_S = 0.020

_MAX_SIGNATURES_PER_OP = 64
_MAX_TIMED_ITERS = 50

# Relative (to max|stock|) disagreement above which the native output is
# rejected.  Loose on purpose: this catches a wrong kernel, not rounding.
_TOLERANCE = {
    torch.float32: 1e-3,
    torch.float16: 3e-2,
    torch.bfloat16: 5e-2,
}

_TOLERANCE_OVERRIDE: float | None
try:
    _TOLERANCE_OVERRIDE = (float(os.environ["CMPEXT3_AUTOSELECT_TOLERANCE"])
                           if os.environ.get("CMPEXT3_AUTOSELECT_TOLERANCE") else None)
except ValueError:
    _TOLERANCE_OVERRIDE = None

_CHUNK = 1 << 22  # elements compared per step: bounds the fp32 copies the gate makes


class Decision:
    """Which implementation serves one signature, and why."""

    __slots__ = ("op", "use_native", "native_ms", "stock_ms", "note")

    def __init__(self, op: str, use_native: bool, native_ms: float | None = None,
                 stock_ms: float | None = None, note: str = ""):
        self.op = op
        self.use_native = use_native
        self.native_ms = native_ms  # seconds per call, despite the name (as in the reference)
        self.stock_ms = stock_ms
        self.note = note

    @property
    def speedup(self) -> float | None:
        if self.native_ms and self.stock_ms:
            return self.stock_ms / self.native_ms
        return None

    def _who(self) -> str:
        return "cmpext3" if self.use_native else "stock"

    def __repr__(self) -> str:
        if self.native_ms is not None and self.stock_ms is not None:
            return (f"<{self.op}: {self._who()} ({self.native_ms * 1e3:.3f}ms vs "
                    f"{self.stock_ms * 1e3:.3f}ms stock)>")
        return f"<{self.op}: {self._who()} ({self.note})>"


_decisions: dict[Any, Decision] = {}
_probe_counts: dict[str, int] = {}
_warned: set[str] = set()


def enabled() -> bool:
    return _ENABLED


def reset() -> None:
    """Forget all decisions (the next call of each signature probes again)."""
    _decisions.clear()
    _probe_counts.clear()
    _warned.clear()


def report() -> list[Decision]:
    """All decisions, lowest native speedup first."""
    return sorted(_decisions.values(), key=lambda d: d.speedup or 0.0)


def format_report() -> str:
    if not _decisions:
        return "cmpext3: no kernel decisions made yet (no eligible op has run)."
    out = [f"cmpext3: {len(_decisions)} kernel decision(s), slowest native first:"]
    for d in report():
        who = "cmpext3" if d.use_native else "stock  "
        if d.native_ms is not None and d.stock_ms is not None:
            out.append(f"  {who}  {d.op:<24} {d.native_ms * 1e3:9.3f} ms vs "
                       f"{d.stock_ms * 1e3:9.3f} ms stock ({d.speedup:.2f}x)")
        else:
            out.append(f"  {who}  {d.op:<24} {d.note}")
    return "\n".join(out)


def _log(msg: str) -> None:
    if _VERBOSE:
        sys.stderr.write(f"[cmpext3] {msg}\n")
        sys.stderr.flush()


def _warn_once(tag: str, msg: str) -> None:
    if tag not in _warned:
        _warned.add(tag)
        sys.stderr.write(f"[cmpext3] {msg}\n")
        sys.stderr.flush()


def _sync() -> None:
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def _time(fn: Callable) -> tuple[float, Any]:
    """(seconds per call, last result).  One synced call sizes the loop: a call
    that already used the whole budget is measured once, a fast one is repeated
    up to 50 times within the budget."""
    _sync()
    t0 = time.perf_counter()
    result = fn()
    _sync()
    once = time.perf_counter() - t0
    if once <= 0.0 or once >= _BUDGET_S:
        return once, result
    n = min(_MAX_TIMED_ITERS, max(1, int(_BUDGET_S / once)))
    t0 = time.perf_counter()
    for _ in range(n):
        result = fn()
    _sync()
    return (time.perf_counter() - t0) / n, result


def _mismatch(native_out: Any, stock_out: Any) -> str | None:
    """None when the outputs agree, else a short reason."""
    if not isinstance(native_out, torch.Tensor) or not isinstance(stock_out, torch.Tensor):
        return None  # nothing to judge
    if tuple(native_out.shape) != tuple(stock_out.shape):
        return f"shape {tuple(native_out.shape)} vs stock {tuple(stock_out.shape)}"
    a_all = native_out.detach().reshape(-1)
    b_all = stock_out.detach().reshape(-1)
    worst = 0.0
    peak = 0.0
    for lo in range(0, a_all.numel(), _CHUNK):
        a = a_all[lo:lo + _CHUNK].float()
        b = b_all[lo:lo + _CHUNK].float()
        if not bool(torch.isfinite(a).all()):
            return "native output contains NaN/Inf"
        worst = max(worst, float((a - b).abs_().max()))
        peak = max(peak, float(b.abs_().max()))
    if not math.isfinite(worst):
        return "native output contains NaN/Inf"
    rel = worst / peak if peak > 0.0 else worst
    tol = _TOLERANCE_OVERRIDE if _TOLERANCE_OVERRIDE is not None else \
        _TOLERANCE.get(stock_out.dtype, 1e-3)
    if rel > tol:
        return f"max relative difference {rel:.2e} exceeds {tol:.0e}"
    return None


def _fallback_verdict(op: str) -> bool:
    """Majority verdict of the signatures already measured for `op` (native on a tie
    or when none were measured)."""
    votes = [d.use_native for d in _decisions.values() if d.op == op]
    if not votes:
        return True
    return 2 * sum(votes) >= len(votes)


def _record(key: Any, op: str, use_native: bool, native_ms: float | None = None,
            stock_ms: float | None = None, note: str = "") -> Decision:
    d = Decision(op, use_native, native_ms, stock_ms, note)
    _decisions[key] = d
    if native_ms is not None and stock_ms is not None:
        why = f"{native_ms * 1e3:.3f} ms vs {stock_ms * 1e3:.3f} ms stock"
    else:
        why = note
    _log(f"{op}: using {'the cmpext3 kernel' if use_native else 'stock'} -- {why}")
    return d


def _native_or_stock(native_call: Callable, stock_call: Callable) -> Any:
    try:
        return native_call()
    except (RuntimeError, TypeError):
        return stock_call()


def choose(op: str, key: Any, native_call: Callable, stock_call: Callable) -> Any:
    """Serve this call with the implementation chosen for `key`, probing first
    if the signature is new.  `stock_call` must always succeed."""
    d = _decisions.get(key)
    if d is not None:
        # cached: the winner only; a one-off native failure does not flip it
        return _native_or_stock(native_call, stock_call) if d.use_native else stock_call()

    if _probe_counts.get(op, 0) >= _MAX_SIGNATURES_PER_OP:
        use_native = _fallback_verdict(op)
        _record(key, op, use_native,
                note=f"not probed ({_MAX_SIGNATURES_PER_OP} signatures already measured "
                     f"for {op}; following that majority)")
        return _native_or_stock(native_call, stock_call) if use_native else stock_call()

    try:
        return _probe(op, key, native_call, stock_call)
    except torch.OutOfMemoryError:
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        _probe_counts[op] = max(0, _probe_counts.get(op, 0) - 1)
        return stock_call()


def _probe(op: str, key: Any, native_call: Callable, stock_call: Callable) -> Any:
    _probe_counts[op] = _probe_counts.get(op, 0) + 1
    try:
        native_out = native_call()
    except torch.OutOfMemoryError:
        raise
    except (RuntimeError, TypeError) as exc:
        _record(key, op, False, note=f"native kernel raised {type(exc).__name__}: {exc}")
        return stock_call()
    stock_out = stock_call()

    reason = _mismatch(native_out, stock_out)
    if reason is not None:
        _record(key, op, False, note=f"output mismatch -- {reason}")
        _warn_once(f"mismatch:{op}",
                   f"{op}: native output disagrees with stock ({reason}); using stock for "
                   f"this shape. This is a kernel bug -- please report the shape.")
        return stock_out

    native_s, native_out = _time(native_call)
    stock_s, stock_out = _time(stock_call)
    use_native = native_s < stock_s
    _record(key, op, use_native, native_s, stock_s)
    return native_out if use_native else stock_out
