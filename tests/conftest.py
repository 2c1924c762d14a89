"""Shared pytest setup.

* Puts the repo root (oracle/, __graft_entry__) and torch-cmp-patch_amd/
  (the cmpext3 package) on sys.path.
* Forces CMPEXT3_AUTOPATCH=0 before cmpext3 is imported, so collecting the
  tests never patches torch as a side effect; tests opt in via `patched`.
* Builds the native library, the torch binding and the C oracle once if they
  are missing (a fresh checkout has no .so files).
* `gpu` marks tests that need an MI355X; they are skipped when no GPU is
  visible.

The dispatch tests mirror the reference's mock-based suite
(tests/conftest.py and tests/test_cmpext3_monkeypatch.py there): the native
module is swapped for a fake whose `attention` is a MagicMock, and
force_eligible() bypasses the GPU/dtype gate so plain CPU tensors reach the
native branch.
"""
from __future__ import annotations

import os
import subprocess
import sys
import types
from pathlib import Path
from unittest.mock import MagicMock

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "torch-cmp-patch_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("CMPEXT3_AUTOPATCH", "0")


def _ensure_built() -> None:
    import sysconfig
    pkg = PKG_ROOT / "cmpext3"
    native = pkg / ("_native" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not (pkg / "libcmpext3_attn.so").exists() or not native.exists():
        subprocess.run([sys.executable, str(PKG_ROOT / "build.py")], check=True)
    if not (REPO / "oracle" / "libsdpa_oracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(REPO / "oracle")], check=True)


_ensure_built()

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402
import cmpext3  # noqa: E402

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def no_autoselect():
    """Runtime native-vs-stock selection OFF by default: with it off, dispatch is
    'native, stock only on exception', which is what the routing tests assert.
    The `autoselecting` fixture turns it back on."""
    from cmpext3 import autoselect
    prev = autoselect._ENABLED
    autoselect._ENABLED = False
    autoselect.reset()
    try:
        yield
    finally:
        autoselect._ENABLED = prev
        autoselect.reset()


@pytest.fixture
def autoselecting():
    from cmpext3 import autoselect
    autoselect._ENABLED = True
    autoselect.reset()
    try:
        yield autoselect
    finally:
        autoselect._ENABLED = False
        autoselect.reset()


@pytest.fixture
def native(monkeypatch):
    """A fake native module whose `attention` is a MagicMock, installed as both
    cmpext3._C (what the wrappers call) and cmpext3.ops."""
    fake = types.ModuleType("cmpext3._native_fake")
    fake.attention = MagicMock(name="attention")
    monkeypatch.setattr(cmpext3, "_C", fake)
    monkeypatch.setattr(cmpext3, "ops", fake)
    return fake


@pytest.fixture
def patched():
    """cmpext3.enable() for the duration of the test, always reverted."""
    assert not cmpext3.is_enabled(), "a previous test left cmpext3 enabled"
    cmpext3.enable()
    try:
        yield cmpext3
    finally:
        cmpext3.disable()


@pytest.fixture
def run_without_copies():
    """run(fn): call fn() (one attention call on the GPU) and check that the
    only device memory it took from torch's allocator is its output, i.e. no
    padded or contiguous copy of Q, K or V was made (the allocator rounds
    every block up to 512 bytes).  A key-split workspace the binding makes
    for the stream (kept for later calls) is not a copy: fn() runs once
    first, unmeasured, so that the measured call finds the workspace in
    place (a new workspace may also take a larger cached block of the
    allocator whole, which would blur the count)."""
    def run(fn):
        fn()  # the workspace, if the call takes one, is made here
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        before = torch.cuda.memory_allocated()
        ws_before = cmpext3.ops.workspace_bytes(torch.cuda.current_device())
        out = fn()
        torch.cuda.synchronize()
        grew = torch.cuda.max_memory_allocated() - before
        assert cmpext3.ops.workspace_bytes(torch.cuda.current_device()) == ws_before
        nbytes = out.untyped_storage().nbytes()
        assert grew <= (nbytes + 511) // 512 * 512, f"{grew} bytes allocated for a {nbytes}-byte output"
        return out
    return run


def force_eligible(monkeypatch):
    """Make the GPU/dtype and grad gates pass so CPU tensors reach the native branch."""
    monkeypatch.setattr(cmpext3, "_usable", lambda *a, **k: True)
    monkeypatch.setattr(cmpext3, "_grad_safe", lambda *a, **k: True)


STOCK_SDPA = F.scaled_dot_product_attention
