"""End-to-end drop-in checks on the GPU: F.scaled_dot_product_attention after
cmpext3.enable() reaches the native kernel (no silent stock path), produces
oracle-accurate results, honours the caller's stream and layout, and falls
back to stock exactly where the reference does (cmpext3/__init__.py:624-628
there) or where the native op rejects the input."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import cmpext3
from cmpext3 import workloads as W
from oracle import sdpa_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture
def counting_native(monkeypatch):
    real = cmpext3._C
    calls = {"n": 0}

    class Counting:
        @staticmethod
        def attention(*args):
            calls["n"] += 1
            return real.attention(*args)

    monkeypatch.setattr(cmpext3, "_C", Counting)
    return calls


@pytest.mark.parametrize("dtype,causal,D", [("fp16", False, 64), ("bf16", True, 128),
                                            ("fp32", True, 40), ("fp16", True, 80)])
def test_patched_sdpa_runs_native_and_matches_oracle(patched, counting_native, dtype, causal, D):
    wl = W.Workload("e2e", dtype, 2, 3, 200, 200, D, causal=causal, seed=4)
    q, k, v = wl.make_inputs("cuda")
    with torch.inference_mode():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    torch.cuda.synchronize()
    assert counting_native["n"] == 1
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), None, causal)
    assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE[dtype]


def test_bshd_query_gets_bshd_output(patched):
    wl = W.Workload("bshd", "fp16", 2, 4, 130, 130, 64, seed=5)
    q, k, v = wl.make_inputs("cuda", layout="bshd")
    out = cmpext3.ops.attention(q, k, v, None, False)
    assert out.shape == q.shape and out.stride() == q.stride()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["fp16"]


@pytest.mark.parametrize("D", [4, 12, 36, 100])
def test_odd_head_dims_run_in_place(D, run_without_copies):
    wl = W.Workload("odd", "fp16", 1, 2, 70, 50, D, seed=D)
    q, k, v = wl.make_inputs("cuda")
    out = run_without_copies(lambda: cmpext3.ops.attention(q, k, v, None, True))
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), None, True)
    assert out.shape == q.shape
    assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["fp16"]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sk", [64, 300])
def test_misaligned_storage(causal, Sk, run_without_copies):
    """A 4-byte offset view runs in place (4-byte pieces); a 2-byte offset
    view is repacked by the binding (faster than 2-byte pieces)."""
    k = torch.randn(1, 2, Sk, 64, dtype=torch.float16, device="cuda")
    for off in (2, 1):
        base = torch.randn(1 * 2 * 64 * 64 + off, dtype=torch.float16, device="cuda")
        q = base[off:].view(1, 2, 64, 64)
        if off == 2:
            out = run_without_copies(lambda: cmpext3.ops.attention(q, k, k, 0.2, causal))
        else:
            out = cmpext3.ops.attention(q, k, k, 0.2, causal)
        ref = orc.sdpa_np(q.cpu(), k.cpu(), k.cpu(), 0.2, causal)
        assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["fp16"]


def test_odd_head_dim_with_a_mask_is_repacked():
    """Masked calls need whole 16-byte chunks: the binding repacks those."""
    wl = W.Workload("oddmask", "bf16", 1, 2, 70, 300, 36, seed=3)
    q, k, v = wl.make_inputs("cuda")
    keep = torch.rand(1, 1, 70, 300, device="cuda") > 0.3
    out = cmpext3.ops.attention(q, k, v, None, False, keep)
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu(), None, False, attn_mask=keep.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["bf16"]


def test_runs_on_the_callers_stream():
    wl = W.Workload("stream", "bf16", 1, 4, 300, 300, 64, seed=6)
    q, k, v = wl.make_inputs("cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = cmpext3.ops.attention(q, k, v, None, False)
    s.synchronize()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu())
    assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["bf16"]


def test_reference_fallbacks_do_not_reach_native(patched, counting_native):
    """Dropout and live autograd stay on stock (attn_mask calls, with or
    without is_causal, run natively: tests/test_gpu_mask.py)."""
    q, k, v = W.Workload("fb", "fp16", 1, 2, 64, 64, 64).make_inputs("cuda")
    F.scaled_dot_product_attention(q, k, v, dropout_p=0.5)
    qg = q.clone().requires_grad_(True)
    F.scaled_dot_product_attention(qg, k, v)
    assert counting_native["n"] == 0


def test_native_rejections_fall_back_to_correct_stock_results(patched):
    q = torch.randn(1, 4, 32, 64, dtype=torch.float16, device="cuda")
    k = torch.randn(1, 4, 32, 64, dtype=torch.float16, device="cuda")
    v32 = torch.randn(1, 4, 32, 32, dtype=torch.float16, device="cuda")
    with torch.inference_mode():
        out = F.scaled_dot_product_attention(q, k, v32)                     # Dv != D
        want = cmpext3._ORIGINALS[(F, "scaled_dot_product_attention")](q, k, v32)
        assert torch.equal(out, want)
        empty = torch.randn(1, 4, 0, 64, dtype=torch.float16, device="cuda")
        out = F.scaled_dot_product_attention(q, empty, empty)                # Sk = 0
        assert torch.count_nonzero(out) == 0


def test_autoselect_probe_on_gpu(patched, autoselecting):
    q, k, v = W.Workload("as", "fp16", 2, 4, 512, 512, 64, seed=7).make_inputs("cuda")
    with torch.inference_mode():
        a = F.scaled_dot_product_attention(q, k, v)
        b = F.scaled_dot_product_attention(q, k, v)
    torch.cuda.synchronize()
    (d,) = autoselecting._decisions.values()
    assert "mismatch" not in d.note and d.native_ms is not None
    assert "attention fp16" in cmpext3.autoselect_report()
    ref = orc.sdpa_np(q.cpu(), k.cpu(), v.cpu())
    for out in (a, b):
        assert orc.max_abs_err(out.cpu(), ref) <= orc.TOLERANCE["fp16"]


def test_describe_names_the_kernel():
    text = cmpext3.ops.describe(0, 2, 10, 4096, 4096, 64, False)
    assert "pipe16" in text and "DK=64" in text
    # SDXL cross-attention (77 keys): all of K/V in LDS, one pass per row
    assert "short16" in cmpext3.ops.describe(0, 2, 10, 4096, 77, 64, False)
    assert "short16" not in cmpext3.ops.describe(0, 2, 10, 4096, 77, 64, True)
    # head dims above 128: prefills on the pipelined kernel, one wave per SIMD
    assert "pipe16" in cmpext3.ops.describe(0, 2, 10, 4096, 4096, 256, False)
    assert "mfma16" in cmpext3.ops.describe(0, 2, 10, 64, 4096, 256, False)  # two waves of rows
    assert "mfma32" in cmpext3.ops.describe(2, 2, 8, 4096, 4096, 40, False)
