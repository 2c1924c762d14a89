"""Dispatch-layer tests of the cmpext3 SDPA patch (CPU only, no GPU).

Mirrors the reference's mock-based suite for this path
(tests/test_cmpext3_monkeypatch.py there: the grad and device gates,
TestEnableDisable :91-180, TestScaledDotProductAttention :857-926),
written against this package: the
native module is a fake whose `attention` is a MagicMock (`native` fixture),
and force_eligible() lets CPU tensors through the GPU/dtype gate.
"""
from __future__ import annotations

import contextlib
import os
import subprocess
import sys

import pytest
import torch
import torch.nn.functional as F

import cmpext3
from conftest import PKG_ROOT, STOCK_SDPA, force_eligible


def _called_once_with_tensors(mock_fn, *expected):
    assert mock_fn.call_count == 1, f"expected 1 call, got {mock_fn.call_count}"
    args, kwargs = mock_fn.call_args
    assert kwargs == {}
    assert len(args) == len(expected)
    for got, want in zip(args, expected):
        if isinstance(want, torch.Tensor):
            assert isinstance(got, torch.Tensor) and torch.equal(got, want)
        else:
            assert got == want


def _qkv(*shape):
    return torch.randn(*shape), torch.randn(*shape), torch.randn(*shape)


def _leaf(needs_grad: bool = False) -> torch.Tensor:
    return torch.randn(3, requires_grad=needs_grad)


# (what the call looks like, arguments, context it runs in, expected answer)
_GRAD_CASES = [
    ("only non-tensors", lambda: (7, "name", None), contextlib.nullcontext, True),
    ("tensors without grad", lambda: (_leaf(), _leaf()), contextlib.nullcontext, True),
    ("one tensor needs grad", lambda: (_leaf(), _leaf(True)), contextlib.nullcontext, False),
    ("grad tensor beside non-tensors", lambda: (None, _leaf(True), 1.5), contextlib.nullcontext,
     False),
    ("grad tensor under no_grad", lambda: (_leaf(True),), torch.no_grad, True),
    ("grad tensor in inference mode", lambda: (_leaf(True),), torch.inference_mode, True),
]


@pytest.mark.parametrize("what,make_args,context,want", _GRAD_CASES,
                         ids=[case[0] for case in _GRAD_CASES])
def test_grad_safe(what, make_args, context, want):
    args = make_args()
    with context():
        assert cmpext3._grad_safe(*args) is want, what


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16,
                                   torch.float64, torch.int64, torch.int8])
@pytest.mark.parametrize("on_gpu", [True, False])
def test_usable_accepts_only_gpu_tensors_of_the_three_dtypes(monkeypatch, dtype, on_gpu):
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: on_gpu))
    t = torch.zeros(2, dtype=dtype)
    want = on_gpu and dtype in (torch.float16, torch.float32, torch.bfloat16)
    assert cmpext3._usable(t) is want
    # non-tensor arguments never change the answer
    assert cmpext3._usable(None, t, 3, "x") is want
    assert cmpext3._usable(None, 3, "x") is True


def test_usable_needs_every_tensor_to_pass(monkeypatch):
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: self.dtype != torch.int32))
    good = torch.zeros(2, dtype=torch.float16)
    assert cmpext3._usable(good, good) is True
    assert cmpext3._usable(good, torch.zeros(2, dtype=torch.int32)) is False


class TestEnableDisable:
    def test_enable_installs_sdpa(self, patched):
        assert cmpext3.is_enabled() is True
        assert F.scaled_dot_product_attention is cmpext3._patched_sdpa

    def test_disable_restores_original(self, patched):
        orig = cmpext3._ORIGINALS[(F, "scaled_dot_product_attention")]
        cmpext3.disable()
        assert F.scaled_dot_product_attention is orig is STOCK_SDPA
        assert cmpext3.is_enabled() is False
        cmpext3.enable()  # keep the fixture's teardown meaningful

    def test_enable_is_idempotent(self, patched):
        first = cmpext3._ORIGINALS[(F, "scaled_dot_product_attention")]
        cmpext3.enable()
        assert cmpext3._ORIGINALS[(F, "scaled_dot_product_attention")] is first
        assert F.scaled_dot_product_attention is cmpext3._patched_sdpa

    def test_disable_without_enable_is_noop(self):
        assert cmpext3.is_enabled() is False
        cmpext3.disable()
        assert cmpext3.is_enabled() is False
        assert F.scaled_dot_product_attention is STOCK_SDPA

    @pytest.mark.parametrize("names", [{"attention"}, {"scaled_dot_product_attention"}])
    def test_disable_ops_pins_attention_to_stock(self, monkeypatch, names):
        monkeypatch.setattr(cmpext3, "_DISABLED_OPS", frozenset(names))
        cmpext3.enable()
        try:
            assert F.scaled_dot_product_attention is STOCK_SDPA
        finally:
            cmpext3.disable()

    def test_ops_alias_is_native_module(self, native):
        assert cmpext3.ops is native

    def test_torchscript_still_sees_stock_sdpa(self, patched):
        @torch.jit.script
        def f(q, k, v):
            return F.scaled_dot_product_attention(q, k, v)
        q = torch.randn(1, 1, 4, 8)
        assert torch.allclose(f(q, q, q), STOCK_SDPA(q, q, q))

    def test_import_patches_unless_autopatch_is_zero(self):
        code = ("import torch.nn.functional as F, cmpext3; "
                "print(F.scaled_dot_product_attention is cmpext3._patched_sdpa)")
        for env_val, want in (("1", "True"), ("0", "False")):
            env = dict(os.environ, CMPEXT3_AUTOPATCH=env_val, PYTHONPATH=str(PKG_ROOT))
            out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                                 text=True, timeout=300)
            assert out.returncode == 0, out.stderr
            assert out.stdout.strip().splitlines()[-1] == want

    def test_disable_ops_env_var_is_read_at_import(self):
        code = ("import torch.nn.functional as F, cmpext3; "
                "print(F.scaled_dot_product_attention is cmpext3._patched_sdpa)")
        env = dict(os.environ, CMPEXT3_AUTOPATCH="1", CMPEXT3_DISABLE_OPS="conv2d, attention",
                   PYTHONPATH=str(PKG_ROOT))
        out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                             text=True, timeout=300)
        assert out.returncode == 0, out.stderr
        assert out.stdout.strip().splitlines()[-1] == "False"


class TestScaledDotProductAttention:
    def test_calls_native_when_eligible(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        native.attention.return_value = "native-result"
        assert F.scaled_dot_product_attention(q, k, v) == "native-result"
        _called_once_with_tensors(native.attention, q, k, v, None, False)

    def test_passes_scale_and_is_causal_positionally(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        native.attention.return_value = "native-result"
        assert F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.3) == "native-result"
        _called_once_with_tensors(native.attention, q, k, v, 0.3, True)

    def test_attn_mask_goes_native_as_sixth_argument(self, patched, native, monkeypatch):
        """The reference sent every attn_mask to stock (its cmpext3/__init__.py:624);
        here bool/float masks without is_causal reach the kernel, positionally."""
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        mask = torch.zeros(3, 3, dtype=torch.bool)
        native.attention.return_value = "native-result"
        assert F.scaled_dot_product_attention(q, k, v, attn_mask=mask) == "native-result"
        _called_once_with_tensors(native.attention, q, k, v, None, False, mask)

    def test_mask_with_causal_goes_native(self, patched, native, monkeypatch):
        """attn_mask together with is_causal reaches the kernel (a pair must
        pass both rules, torch's CPU behaviour)."""
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        mask = torch.ones(3, 3, dtype=torch.bool)
        native.attention.return_value = "native-result"
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=True)
        assert out == "native-result"
        _called_once_with_tensors(native.attention, q, k, v, None, True, mask)

    def test_falls_back_for_unsupported_mask_dtype(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        mask = torch.zeros(3, 3, dtype=torch.float64)
        try:
            F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        except RuntimeError:
            pass   # stock's own error for a float64 mask on float32 q
        native.attention.assert_not_called()

    def test_falls_back_when_dropout_nonzero(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        q, k, v = _qkv(1, 2, 3, 4)
        F.scaled_dot_product_attention(q, k, v, dropout_p=0.1)
        native.attention.assert_not_called()

    def test_falls_back_on_non_4d_query(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        q, k, v = _qkv(2, 3, 4)
        F.scaled_dot_product_attention(q, k, v)
        native.attention.assert_not_called()

    def test_falls_back_when_not_gpu(self, patched, native):
        q, k, v = _qkv(1, 2, 3, 4)
        out = F.scaled_dot_product_attention(q, k, v)
        native.attention.assert_not_called()
        assert torch.allclose(out, STOCK_SDPA(q, k, v))

    def test_falls_back_when_autograd_is_live(self, patched, native, monkeypatch):
        monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
        q = torch.randn(1, 2, 3, 4, requires_grad=True)
        k, v = torch.randn(1, 2, 3, 4), torch.randn(1, 2, 3, 4)
        monkeypatch.setattr(cmpext3, "_ORIGINALS",
                            {**cmpext3._ORIGINALS, (F, "scaled_dot_product_attention"):
                             lambda *a, **kw: "stock"})
        assert F.scaled_dot_product_attention(q, k, v) == "stock"
        native.attention.assert_not_called()

    def test_falls_back_on_native_runtime_error(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        native.attention.side_effect = RuntimeError("boom")
        q, k, v = _qkv(1, 2, 3, 4)
        out = F.scaled_dot_product_attention(q, k, v)
        native.attention.assert_called_once()
        assert torch.allclose(out, STOCK_SDPA(q, k, v))

    def test_falls_back_on_native_type_error(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        native.attention.side_effect = TypeError("bad args")
        q, k, v = _qkv(1, 2, 3, 4)
        assert F.scaled_dot_product_attention(q, k, v).shape == q.shape

    def test_gqa_runs_native_only_with_enable_gqa(self, patched, native, monkeypatch):
        """K/V with fewer heads than Q: native (positional call, the kernel reads
        the grouping from the shapes) under enable_gqa=True; stock otherwise,
        where torch raises its own head-count error."""
        force_eligible(monkeypatch)
        q = torch.randn(1, 4, 3, 8)
        k, v = torch.randn(1, 2, 3, 8), torch.randn(1, 2, 3, 8)
        native.attention.return_value = "native-result"
        assert F.scaled_dot_product_attention(q, k, v, enable_gqa=True) == "native-result"
        _called_once_with_tensors(native.attention, q, k, v, None, False)
        native.attention.reset_mock()
        with pytest.raises(RuntimeError):
            F.scaled_dot_product_attention(q, k, v)
        native.attention.assert_not_called()

    def test_extra_kwargs_reach_only_stock(self, patched, native, monkeypatch):
        force_eligible(monkeypatch)
        native.attention.side_effect = RuntimeError("gqa head count")
        q = torch.randn(1, 4, 3, 8)
        k, v = torch.randn(1, 2, 3, 8), torch.randn(1, 2, 3, 8)
        out = F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
        _called_once_with_tensors(native.attention, q, k, v, None, False)
        assert torch.allclose(out, STOCK_SDPA(q, k, v, enable_gqa=True))


def test_missing_native_extension_fails_loudly(tmp_path):
    """The product path must not import without its HIP library."""
    import shutil
    dst = tmp_path / "cmpext3"
    shutil.copytree(PKG_ROOT / "cmpext3", dst, ignore=shutil.ignore_patterns("*.so", "__pycache__"))
    env = dict(os.environ, PYTHONPATH=str(tmp_path), CMPEXT3_AUTOPATCH="0")
    out = subprocess.run([sys.executable, "-c", "import cmpext3"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode != 0 and "native extension not built" in out.stderr


def test_product_package_never_imports_the_oracle():
    src = PKG_ROOT / "cmpext3"
    for path in src.glob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
        assert "sdpa_oracle" not in text, path
