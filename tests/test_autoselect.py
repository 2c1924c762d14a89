"""The run-time native-vs-stock arbiter (cmpext3/autoselect.py), CPU only.

Covers the behaviour contract of the reference's chooser
(cmpext3/autoselect.py:200-364 there; its tests address choose, _time,
_decisions, _probe_counts, _MAX_SIGNATURES_PER_OP and Decision's fields):
acceptance before speed, sticky verdicts, refusal on exceptions, no trace
after an out-of-memory trial, and the per-op trial cap.  Wall-clock timing is
replaced by a table (`fake_clock`) so verdicts are deterministic; the real
timer is tested on its own with a counting callable.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import cmpext3
from conftest import STOCK_SDPA, force_eligible


class Impl:
    """A scripted implementation: returns `value` (or raises `error`) and
    counts its calls.  Hashable, so a timing table can key on it."""

    def __init__(self, value=None, error=None):
        self.value = torch.zeros(4) if value is None else value
        self.error = error
        self.calls = 0

    def __call__(self):
        self.calls += 1
        if self.error is not None:
            raise self.error
        return self.value.clone()


@pytest.fixture
def fake_clock(monkeypatch, autoselecting):
    """Install a timing table {impl: seconds per call} as autoselect._time."""
    table: dict = {}

    def timed(fn):
        return table[fn], fn()

    monkeypatch.setattr(autoselecting, "_time", timed)
    return table


def test_faster_kernel_wins_and_stock_is_not_run_again(autoselecting, fake_clock):
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.002, stock: 0.008})
    autoselecting.choose("op", ("sig",), kern, stock)
    verdict = autoselecting._decisions[("sig",)]
    assert verdict.use_native
    assert verdict.speedup == pytest.approx(4.0)
    stock_calls = stock.calls
    for _ in range(5):
        autoselecting.choose("op", ("sig",), kern, stock)
    assert stock.calls == stock_calls


def test_times_are_kept_in_milliseconds(autoselecting, fake_clock):
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.0015, stock: 0.0030})
    autoselecting.choose("op", ("sig",), kern, stock)
    verdict = autoselecting._decisions[("sig",)]
    assert verdict.native_ms == pytest.approx(1.5)
    assert verdict.stock_ms == pytest.approx(3.0)


def test_slower_kernel_loses_and_is_not_run_again(autoselecting, fake_clock):
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.009, stock: 0.003})
    out = autoselecting.choose("op", ("sig",), kern, stock)
    assert torch.equal(out, torch.zeros(4))
    assert autoselecting._decisions[("sig",)].use_native is False
    kern_calls = kern.calls
    for _ in range(5):
        autoselecting.choose("op", ("sig",), kern, stock)
    assert kern.calls == kern_calls


def test_wrong_output_is_refused_before_any_timing(autoselecting, fake_clock):
    kern, stock = Impl(torch.arange(4.0)), Impl(torch.ones(4))
    fake_clock.update({kern: 0.001, stock: 1.0})  # a wrong kernel may be fast
    out = autoselecting.choose("op", ("sig",), kern, stock)
    verdict = autoselecting._decisions[("sig",)]
    assert not verdict.use_native
    assert "mismatch" in verdict.note
    assert verdict.native_ms is None and verdict.speedup is None
    assert torch.equal(out, torch.ones(4))  # the call is served by stock
    assert kern.calls == 1


def test_mismatch_warns_once_per_op(autoselecting, fake_clock, capsys):
    for i in range(3):
        autoselecting.choose("op", ("sig", i), Impl(torch.ones(4)), Impl(torch.zeros(4)))
    assert capsys.readouterr().err.count("mismatch") == 1


def test_rounding_noise_is_accepted(autoselecting, fake_clock):
    kern, stock = Impl(torch.full((6,), 2.0 + 1e-6)), Impl(torch.full((6,), 2.0))
    fake_clock.update({kern: 0.001, stock: 0.002})
    autoselecting.choose("op", ("sig",), kern, stock)
    assert autoselecting._decisions[("sig",)].use_native


@pytest.mark.parametrize("dtype,rel,accepted", [
    (torch.float32, 5e-4, True), (torch.float32, 3e-3, False),
    (torch.float16, 2e-2, True), (torch.float16, 6e-2, False),
    (torch.bfloat16, 4e-2, True), (torch.bfloat16, 1e-1, False),
])
def test_the_limit_depends_on_the_dtype(autoselecting, fake_clock, dtype, rel, accepted):
    # the error is measured against the largest stock magnitude (here 4)
    want = torch.tensor([1.0, -4.0, 2.0, 0.5]).to(dtype)
    got = (want.float() + torch.tensor([0.0, 0.0, 4.0 * rel, 0.0])).to(dtype)
    kern, stock = Impl(got), Impl(want)
    fake_clock.update({kern: 0.001, stock: 0.002})
    autoselecting.choose("op", ("sig",), kern, stock)
    assert autoselecting._decisions[("sig",)].use_native is accepted


def test_tolerance_override(autoselecting, fake_clock, monkeypatch):
    monkeypatch.setattr(autoselecting, "_TOLERANCE_OVERRIDE", 0.5)
    kern, stock = Impl(torch.full((4,), 1.4)), Impl(torch.ones(4))
    fake_clock.update({kern: 0.001, stock: 0.002})
    autoselecting.choose("op", ("sig",), kern, stock)
    assert autoselecting._decisions[("sig",)].use_native


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_non_finite_output_is_refused(autoselecting, fake_clock, bad):
    got = torch.zeros(4)
    got[2] = bad
    autoselecting.choose("op", ("sig",), Impl(got), Impl())
    verdict = autoselecting._decisions[("sig",)]
    assert not verdict.use_native and "NaN/Inf" in verdict.note


def test_output_of_another_shape_is_refused(autoselecting, fake_clock):
    autoselecting.choose("op", ("sig",), Impl(torch.zeros(2, 2)), Impl(torch.zeros(4)))
    verdict = autoselecting._decisions[("sig",)]
    assert not verdict.use_native and "shape" in verdict.note


def test_large_outputs_are_compared_slice_by_slice(autoselecting, fake_clock, monkeypatch):
    monkeypatch.setattr(autoselecting, "_COMPARE_SLICE", 7)
    want = torch.linspace(-3.0, 3.0, 50)
    got = want.clone()
    got[45] += 1.0  # in the last slice
    autoselecting.choose("op", ("sig",), Impl(got), Impl(want))
    assert "mismatch" in autoselecting._decisions[("sig",)].note


def test_kernel_that_raises_in_its_trial_loses_for_good(autoselecting):
    kern, stock = Impl(error=RuntimeError("head dim not supported")), Impl(torch.ones(4))
    for _ in range(4):
        assert torch.equal(autoselecting.choose("op", ("sig",), kern, stock), torch.ones(4))
    assert kern.calls == 1
    verdict = autoselecting._decisions[("sig",)]
    assert not verdict.use_native
    assert "RuntimeError" in verdict.note and "head dim" in verdict.note


def test_type_error_in_the_trial_also_loses(autoselecting):
    kern = Impl(error=TypeError("bad argument"))
    autoselecting.choose("op", ("sig",), kern, Impl())
    assert "TypeError" in autoselecting._decisions[("sig",)].note


def test_a_failure_after_a_native_verdict_serves_only_that_call(autoselecting, fake_clock):
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.001, stock: 0.004})
    autoselecting.choose("op", ("sig",), kern, stock)
    settled = stock.calls
    kern.error = RuntimeError("one bad call")
    autoselecting.choose("op", ("sig",), kern, stock)
    assert stock.calls == settled + 1
    assert autoselecting._decisions[("sig",)].use_native
    kern.error = None
    autoselecting.choose("op", ("sig",), kern, stock)
    assert stock.calls == settled + 1


def test_out_of_memory_in_a_trial_leaves_no_trace(autoselecting, fake_clock):
    kern = Impl(torch.ones(4), error=torch.OutOfMemoryError("trial holds two outputs"))
    stock = Impl(torch.ones(4))
    fake_clock.update({kern: 0.001, stock: 0.002})
    assert torch.equal(autoselecting.choose("op", ("sig",), kern, stock), torch.ones(4))
    assert ("sig",) not in autoselecting._decisions
    assert autoselecting._probe_counts.get("op", 0) == 0
    kern.error = None  # memory is back: the next call holds a full trial
    autoselecting.choose("op", ("sig",), kern, stock)
    assert autoselecting._decisions[("sig",)].use_native
    assert autoselecting._probe_counts["op"] == 1


def test_out_of_memory_in_stock_during_the_trial_leaves_no_trace(autoselecting, fake_clock):
    class StockOomOnce(Impl):
        def __call__(self):
            self.calls += 1
            if self.calls == 1:
                raise torch.OutOfMemoryError("second output did not fit")
            return self.value.clone()

    kern, stock = Impl(), StockOomOnce()
    fake_clock.update({kern: 0.001, stock: 0.002})
    autoselecting.choose("op", ("sig",), kern, stock)
    assert ("sig",) not in autoselecting._decisions
    assert autoselecting._probe_counts.get("op", 0) == 0


def test_trials_stop_at_the_cap_and_later_signatures_follow_the_majority(autoselecting, fake_clock):
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.001, stock: 0.003})
    cap = autoselecting._MAX_SIGNATURES_PER_OP
    for i in range(cap):
        autoselecting.choose("op", ("sig", i), kern, stock)
    assert autoselecting._probe_counts["op"] == cap
    calls = (kern.calls, stock.calls)
    autoselecting.choose("op", ("sig", "late"), kern, stock)
    late = autoselecting._decisions[("sig", "late")]
    assert late.use_native and "not probed" in late.note
    assert (kern.calls, stock.calls) == (calls[0] + 1, calls[1])  # served, not tried
    assert autoselecting._probe_counts["op"] == cap


def test_past_the_cap_a_stock_majority_is_inherited(autoselecting, fake_clock, monkeypatch):
    monkeypatch.setattr(autoselecting, "_MAX_SIGNATURES_PER_OP", 3)
    kern, stock = Impl(), Impl()
    fake_clock.update({kern: 0.005, stock: 0.001})
    for i in range(3):
        autoselecting.choose("op", ("sig", i), kern, stock)
    autoselecting.choose("op", ("sig", "late"), kern, stock)
    assert not autoselecting._decisions[("sig", "late")].use_native
    # the cap is per op: another op still gets trials
    autoselecting.choose("other", ("sig", "x"), kern, stock)
    assert "not probed" not in autoselecting._decisions[("sig", "x")].note


def test_timer_runs_doubling_batches_within_the_call_cap(autoselecting, monkeypatch):
    monkeypatch.setattr(autoselecting, "_BUDGET_S", 10.0)  # never the limit here
    fn = Impl()
    per_call, out = autoselecting._time(fn)
    assert fn.calls == 1 + 2 + 4 + 8 + 16 + 32  # the next batch (64) would pass the cap
    assert fn.calls <= autoselecting._MAX_TIMED_CALLS
    assert per_call > 0.0 and torch.equal(out, torch.zeros(4))


def test_timer_runs_a_slow_call_once(autoselecting, monkeypatch):
    monkeypatch.setattr(autoselecting, "_BUDGET_S", 0.0)
    fn = Impl()
    autoselecting._time(fn)
    assert fn.calls == 1


def test_autoselect_off_runs_the_kernel_without_a_trial(monkeypatch):
    from cmpext3 import autoselect
    monkeypatch.setattr(autoselect, "_ENABLED", False)
    kern, stock = Impl(), Impl(torch.ones(4))
    got = cmpext3._dispatch("op", torch.zeros(4), ("sig",), kern, stock)
    assert torch.equal(got, torch.zeros(4)) and stock.calls == 0
    assert autoselect._decisions == {}
    kern.error = RuntimeError("unsupported")
    assert torch.equal(cmpext3._dispatch("op", torch.zeros(4), ("sig",), kern, stock), torch.ones(4))


def test_unhashable_signature_skips_the_trial(autoselecting):
    """A signature that cannot key the decision table is served as with
    autoselect off: the kernel, no measurement, nothing recorded."""
    kern, stock = Impl(), Impl(torch.ones(4))
    got = cmpext3._dispatch("op", torch.zeros(4), ("sig", [1, 2]), kern, stock)
    assert torch.equal(got, torch.zeros(4)) and kern.calls == 1 and stock.calls == 0
    assert autoselecting._decisions == {}


def test_sdpa_signature_and_report(autoselecting, patched, native, monkeypatch):
    force_eligible(monkeypatch)
    q, k, v = torch.randn(1, 2, 5, 8), torch.randn(1, 2, 6, 8), torch.randn(1, 2, 6, 8)
    native.attention.side_effect = lambda *a: STOCK_SDPA(q, k, v, scale=0.25)
    F.scaled_dot_product_attention(q, k, v, scale=0.25)
    assert list(autoselecting._decisions) == [(q.shape, q.dtype, k.shape, v.shape, 0.25, False)]
    text = cmpext3.autoselect_report()
    assert "1 signature" in text and "attention fp32" in text


def test_report_lists_least_favourable_first(autoselecting, fake_clock):
    fast, slow, stock = Impl(), Impl(), Impl()
    fake_clock.update({fast: 0.001, slow: 0.002, stock: 0.004})
    autoselecting.choose("op", ("fast",), fast, stock)
    autoselecting.choose("op", ("slow",), slow, stock)
    autoselecting.choose("op", ("refused",), Impl(error=RuntimeError("no")), stock)
    order = [d.speedup for d in autoselecting.report()]
    assert order[0] is None and order[1:] == pytest.approx([2.0, 4.0])
    lines = autoselecting.format_report().splitlines()
    assert "refused" in lines[1] and "2.00x" in lines[2] and "4.00x" in lines[3]


def test_report_when_nothing_ran(autoselecting):
    assert "no kernel decisions" in cmpext3.autoselect_report()
