"""Run-time arbitration between the native kernel and stock torch.

Every eligible call carries a signature (the caller builds it: shapes, dtype,
scale, causal flag, mask layout).  The first call of a signature is a *trial*:
the native kernel and stock torch both serve it, their outputs are compared,
and, if the kernel's output is acceptable, both are timed.  The verdict is
kept for the signature and later calls run only the winner.  Behaviour
contract (reference: cmpext3/autoselect.py:200-364, choose/_probe/_time):

  * acceptance comes before speed: a kernel whose output has another shape,
    holds NaN/Inf, or differs from stock by more than the dtype's tolerance
    (max|native - stock| / max|stock|: fp32 1e-3, fp16 3e-2, bf16 5e-2)
    loses the signature for good, with one warning per op;
  * a kernel that raises RuntimeError/TypeError during the trial loses the
    signature; once a signature has gone native, a later exception serves
    only that call from stock and the verdict stands;
  * running out of memory during a trial (it holds both outputs) serves the
    call from stock and leaves no trace: the signature is tried again later
    and does not count toward the cap;
  * at most 64 trials per op; later signatures take the op's majority
    verdict so far (native on a tie or with no verdicts) without a trial.

Knobs, read at import: CMPEXT3_AUTOSELECT=0 (no trials: native, stock only
when the kernel raises), CMPEXT3_VERBOSE=1 (verdicts to stderr),
CMPEXT3_AUTOSELECT_BUDGET_MS (timing budget per implementation per trial,
default 20, at least 1), CMPEXT3_AUTOSELECT_TOLERANCE (one tolerance for
every dtype).

The names the reference's tests reach into are kept: choose, _time (patched
by tests to fake timings), _decisions, _probe_counts, _MAX_SIGNATURES_PER_OP,
Decision.use_native/native_ms/stock_ms/note/speedup.
"""
from __future__ import annotations

import dataclasses
import math
import os
import sys
import time
from typing import Any, Callable

import torch

_OFF_VALUES = ("0", "", "false", "False")


def _env_float(name: str, default: float | None) -> float | None:
    raw = os.environ.get(name)
    if not raw:
        return default
    try:
        return float(raw)
    except ValueError:
        return default


_ENABLED = os.environ.get("CMPEXT3_AUTOSELECT", "1") not in _OFF_VALUES
_VERBOSE = os.environ.get("CMPEXT3_VERBOSE", "0") not in _OFF_VALUES
_BUDGET_S = max(1.0, _env_float("CMPEXT3_AUTOSELECT_BUDGET_MS", 20.0)) * 1e-3
_TOLERANCE_OVERRIDE = _env_float("CMPEXT3_AUTOSELECT_TOLERANCE", None)

_MAX_SIGNATURES_PER_OP = 64
_MAX_TIMED_CALLS = 64      # per implementation per trial
_COMPARE_SLICE = 1 << 22   # elements upcast to fp32 at a time by the output check

# max|native - stock| / max|stock| above which a kernel's output is refused:
# loose enough for reduced-precision accumulation, tight enough for a bug.
_TOLERANCE = {torch.float32: 1e-3, torch.float16: 3e-2, torch.bfloat16: 5e-2}


@dataclasses.dataclass
class Decision:
    """The verdict for one signature.  Times are milliseconds per call (None
    when nothing was timed); `note` says why when there was no race."""

    op: str
    use_native: bool
    native_ms: float | None = None
    stock_ms: float | None = None
    note: str = ""

    @property
    def speedup(self) -> float | None:
        """Stock time over native time (> 1: the kernel is faster)."""
        if not self.native_ms or not self.stock_ms:
            return None
        return self.stock_ms / self.native_ms

    @property
    def winner(self) -> str:
        return "native" if self.use_native else "stock"

    def __str__(self) -> str:
        if self.speedup is None:
            return f"{self.op} -> {self.winner}: {self.note}"
        return (f"{self.op} -> {self.winner}: native {self.native_ms:.3f} ms, "
                f"stock {self.stock_ms:.3f} ms ({self.speedup:.2f}x)")


# signature -> Decision; op -> number of completed trials; op -> [native, stock] verdict counts
_decisions: dict[Any, Decision] = {}
_probe_counts: dict[str, int] = {}
_tally: dict[str, list[int]] = {}
_warned_ops: set[str] = set()


def enabled() -> bool:
    return _ENABLED


def reset() -> None:
    """Forget every verdict; each signature gets a new trial on its next call."""
    _decisions.clear()
    _probe_counts.clear()
    _tally.clear()
    _warned_ops.clear()


def report() -> list[Decision]:
    """Every verdict, the ones least favourable to the kernel first (verdicts
    without timings, i.e. refusals and inherited ones, lead)."""
    return sorted(_decisions.values(), key=lambda d: d.speedup or 0.0)


def format_report() -> str:
    if not _decisions:
        return "cmpext3 autoselect: no kernel decisions recorded (no eligible call seen yet)"
    lines = [f"cmpext3 autoselect: {len(_decisions)} signature(s), least favourable to the kernel first"]
    lines.extend(f"  {d}" for d in report())
    return "\n".join(lines)


def _say(msg: str) -> None:
    sys.stderr.write(f"cmpext3 autoselect: {msg}\n")
    sys.stderr.flush()


def _device_sync() -> None:
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def _time(fn: Callable) -> tuple[float, Any]:
    """Seconds per call of `fn`, and its last output.

    Calls run in synchronised batches of 1, 2, 4, ... until the budget is
    spent or the next batch would pass _MAX_TIMED_CALLS; the result is the
    fastest batch's mean, which discards batches that met a clock ramp or a
    stray host stall.  A call slower than the whole budget runs once.
    """
    best = math.inf
    spent = 0.0
    calls = 0
    batch = 1
    out = None
    while True:
        _device_sync()
        t0 = time.perf_counter()
        for _ in range(batch):
            out = fn()
        _device_sync()
        elapsed = time.perf_counter() - t0
        best = min(best, elapsed / batch)
        spent += elapsed
        calls += batch
        batch *= 2
        if spent >= _BUDGET_S or calls + batch > _MAX_TIMED_CALLS:
            return best, out


def _tolerance(dtype: torch.dtype) -> float:
    if _TOLERANCE_OVERRIDE is not None:
        return _TOLERANCE_OVERRIDE
    return _TOLERANCE.get(dtype, _TOLERANCE[torch.float32])


def _disagreement(got: Any, want: Any) -> str | None:
    """Why the kernel's output is not acceptable next to stock's, or None.

    The error and the scale are reduced on the outputs' device slice by slice
    (bounded fp32 temporaries) and read back once."""
    if not isinstance(got, torch.Tensor) or not isinstance(want, torch.Tensor):
        return None
    if got.shape != want.shape:
        return f"shape {tuple(got.shape)} where stock gives {tuple(want.shape)}"
    if want.numel() == 0:
        return None
    g_flat = got.detach().reshape(-1)
    w_flat = want.detach().reshape(-1)
    err = torch.zeros((), dtype=torch.float32, device=want.device)
    scale = torch.zeros((), dtype=torch.float32, device=want.device)
    finite = torch.ones((), dtype=torch.bool, device=want.device)
    for g, w in zip(g_flat.split(_COMPARE_SLICE), w_flat.split(_COMPARE_SLICE)):
        g32 = g.float()
        finite &= torch.isfinite(g32).all()
        err = torch.maximum(err, (g32 - w.float()).abs().max())
        scale = torch.maximum(scale, w.float().abs().max())
    if not bool(finite):
        return "NaN/Inf in the kernel's output"
    err_v, scale_v = float(err), float(scale)
    rel = err_v / scale_v if scale_v > 0.0 else err_v
    limit = _tolerance(want.dtype)
    if not rel <= limit:
        return f"relative error {rel:.3g} over the {want.dtype} limit {limit:.3g}"
    return None


def _settle(op: str, key: Any, verdict: Decision, counted: bool) -> Decision:
    _decisions[key] = verdict
    votes = _tally.setdefault(op, [0, 0])
    votes[0 if verdict.use_native else 1] += 1
    if counted:
        _probe_counts[op] = _probe_counts.get(op, 0) + 1
    if _VERBOSE:
        _say(str(verdict))
    return verdict


def _trial(op: str, native_call: Callable, stock_call: Callable) -> tuple[Decision, Any]:
    """Run both implementations for a new signature; return the verdict and
    the output that serves this call.  OutOfMemoryError propagates."""
    try:
        native_out = native_call()
    except torch.OutOfMemoryError:
        raise
    except (RuntimeError, TypeError) as exc:
        return Decision(op, False, note=f"kernel refused: {type(exc).__name__}: {exc}"), stock_call()
    stock_out = stock_call()
    flaw = _disagreement(native_out, stock_out)
    if flaw is not None:
        if op not in _warned_ops:
            _warned_ops.add(op)
            _say(f"{op}: kernel output mismatch against stock ({flaw}); stock serves this "
                 f"signature. Please report the call's shapes: this is a kernel bug.")
        return Decision(op, False, note=f"output mismatch: {flaw}"), stock_out
    native_s, native_out = _time(native_call)
    stock_s, stock_out = _time(stock_call)
    verdict = Decision(op, native_s < stock_s, native_s * 1e3, stock_s * 1e3)
    return verdict, (native_out if verdict.use_native else stock_out)


def _inherited(op: str) -> Decision:
    n_native, n_stock = _tally.get(op, (0, 0))
    return Decision(op, n_native >= n_stock,
                    note=f"not probed: {op} reached its {_MAX_SIGNATURES_PER_OP}-trial cap; "
                         f"majority verdict ({n_native} native / {n_stock} stock)")


def _serve(verdict: Decision, native_call: Callable, stock_call: Callable) -> Any:
    if not verdict.use_native:
        return stock_call()
    try:
        return native_call()
    except (RuntimeError, TypeError) as exc:
        if _VERBOSE:
            _say(f"{verdict.op}: kernel raised {type(exc).__name__} on one call; stock served it")
        return stock_call()


def choose(op: str, key: Any, native_call: Callable, stock_call: Callable) -> Any:
    """Serve one call of `op` whose signature is `key` (hashable).

    `native_call` and `stock_call` take no arguments; `stock_call` must not
    fail.  A new signature gets a trial (or, past the op's cap, the op's
    majority verdict); a known one runs its winner.
    """
    verdict = _decisions.get(key)
    if verdict is not None:
        return _serve(verdict, native_call, stock_call)
    if _probe_counts.get(op, 0) >= _MAX_SIGNATURES_PER_OP:
        return _serve(_settle(op, key, _inherited(op), counted=False), native_call, stock_call)
    try:
        verdict, out = _trial(op, native_call, stock_call)
    except torch.OutOfMemoryError:
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        return stock_call()
    _settle(op, key, verdict, counted=True)
    return out
