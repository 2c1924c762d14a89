#!/usr/bin/env python3
"""Attention-forward benchmark on one MI355X (the BASELINE.json metric).

A step is one fused attention forward over one batch of synthetic input of the
headline workload (SDXL self-attention fp16
[2,10,4096,64], scale 1/8), called through the drop-in native op
cmpext3.ops.attention with Q/K/V already resident in HBM.  W untimed warmup
steps, then exactly K timed steps between synchronisations; prints ONE JSON
line.

  value        TFLOP/s over the K timed steps, FLOPs = 4*B*H*Sq*Sk*D
  roofline     dominant kernel: FLOPs per launch / average launch duration,
               measured with HIP events on the launch stream, vs the 2516.6
               TFLOP/s dense fp16 MFMA peak; traffic = HBM bytes per launch
               from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
               (null if absent)
  cpu_baseline stock torch SDPA on the host CPU (what the reference runs for CPU
               tensors), same workload and dtype, bounded to ~10 s; with the
               host's CPU model, torch version and thread counts
  configs      every BASELINE config: the same kernel timing, stock torch SDPA
               on the host CPU in the config's dtype (time, TFLOP/s, GPU
               speedup), and the GPU output's max abs error against torch's CPU
               math SDPA on fp32-upcast inputs, with the north-star tolerance

--backward times a training step instead: the forward that keeps the row
log-sum-exp plus the backward (Delta, dK/dV and dQ kernels), FLOPs counted as
4*B*H*Sq*Sk*D forward + 2.5x that backward (the five matrix products of the
gradient; the kernels recompute S and dP once more, which is not counted);
causal workloads count the visible pairs only.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                       [--no-cpu-baseline] [--no-configs] [--backward]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "torch-cmp-patch_amd"))
sys.path.insert(0, REPO)
os.environ.setdefault("CMPEXT3_AUTOPATCH", "0")


def _ensure_built() -> None:
    import sysconfig
    pkg = os.path.join(REPO, "torch-cmp-patch_amd", "cmpext3")
    native = os.path.join(pkg, "_native" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not (os.path.exists(os.path.join(pkg, "libcmpext3_attn.so")) and os.path.exists(native)):
        import subprocess
        subprocess.run([sys.executable, os.path.join(REPO, "torch-cmp-patch_amd", "build.py")],
                       check=True)


def _traffic_from_profile(workload: str):
    """HBM bytes per launch from profiles/<kernel>_<workload>_hbm.txt, if committed."""
    path = os.path.join(REPO, "profiles", f"attn_fwd_{workload}_hbm.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"^hbm_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def time_kernel(fn, steps: int, warmup: int):
    """(wall seconds for `steps` calls, mean per-call device seconds).

    The device time comes from one pair of HIP events on the launching stream
    around the `steps` back-to-back launches (the op launches on torch's
    current stream), divided by `steps`: an event pair around every launch
    would add a marker packet and its dispatch gap to each measurement, which
    the profiler's per-kernel duration does not contain.
    """
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev = start.elapsed_time(end) / steps / 1e3
    return wall, dev


def host_info() -> dict:
    """The host the CPU baseline ran on: CPU model (lscpu "Model name"), the
    torch version, and the thread count torch uses."""
    import subprocess
    import torch
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.split(":")[0].strip() == "Model name":
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return {"cpu_model": model, "torch_version": torch.__version__,
            "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}


def config_cpu_and_error(wl, out_gpu, budget_s: float = 4.0) -> dict:
    """Per-config CPU figures: stock torch SDPA on the host CPU in the
    config's own dtype (1 warmup + timed calls, ~budget_s; the reference's
    own CPU figures are quoted this way), and the GPU output's max abs error
    against torch's CPU math SDPA on the fp32-upcast inputs (the reference's
    accuracy check)."""
    import torch
    import torch.nn.functional as F
    torch.set_num_threads(os.cpu_count() or 1)
    q, k, v = wl.make_inputs("cpu")
    gqa = wl.kv_heads != wl.H
    call = lambda a, b, c: F.scaled_dot_product_attention(  # noqa: E731
        a, b, c, is_causal=wl.causal, scale=wl.eff_scale, enable_gqa=gqa)
    t0 = time.perf_counter()
    call(q, k, v)
    one = time.perf_counter() - t0
    n = max(1, min(10, int(budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        call(q, k, v)
    dt = (time.perf_counter() - t0) / n
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel(SDPBackend.MATH):
        ref = call(q.float(), k.float(), v.float())
    err = float((out_gpu.float().cpu() - ref).abs().max())
    tol = {"fp16": 1e-2, "bf16": 2e-2, "fp32": 1e-4}[wl.dtype]
    return {"cpu_ms": round(dt * 1e3, 3), "cpu_tflops": round(wl.flops() / dt / 1e12, 5),
            "cpu_calls": n, "max_abs_err_vs_cpu_fp32_math": err, "tolerance": tol,
            "within_tolerance": err <= tol}


def cpu_baseline(wl, budget_s: float = 10.0):
    import torch
    import torch.nn.functional as F
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k, v = wl.make_inputs("cpu")
    gqa = wl.kv_heads != wl.H
    t0 = time.perf_counter()
    F.scaled_dot_product_attention(q, k, v, is_causal=wl.causal, scale=wl.eff_scale, enable_gqa=gqa)
    one = time.perf_counter() - t0
    n = max(1, min(20, int(budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        F.scaled_dot_product_attention(q, k, v, is_causal=wl.causal, scale=wl.eff_scale, enable_gqa=gqa)
    dt = (time.perf_counter() - t0) / n
    return {
        "value": round(wl.flops() / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (f"stock torch.nn.functional.scaled_dot_product_attention on host CPU tensors "
                   f"(the reference's path for CPU inputs), full {wl.name} workload "
                   f"{list(wl.shapes()[0])} {wl.dtype}, 1 warmup + {n} timed calls, "
                   f"{dt * 1e3:.1f} ms/call, os.cpu_count()={os.cpu_count()}"),
        **host_info(),
    }


def cpu_baseline_training(wl, budget_s: float = 20.0):
    """Stock torch SDPA forward + backward on host CPU tensors (fp32 when the
    CPU kernels reject the workload dtype), bounded to ~budget_s."""
    import torch
    import torch.nn.functional as F
    torch.set_num_threads(os.cpu_count() or 1)
    q, k, v = wl.make_inputs("cpu")
    dt_used = wl.dtype

    def step(q, k, v):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        out = F.scaled_dot_product_attention(qq, kk, vv, is_causal=wl.causal, scale=wl.eff_scale,
                                             enable_gqa=wl.kv_heads != wl.H)
        out.backward(torch.ones_like(out))

    try:
        t0 = time.perf_counter()
        step(q, k, v)
    except RuntimeError:
        q, k, v = (t.float() for t in (q, k, v))
        dt_used = "fp32"
        t0 = time.perf_counter()
        step(q, k, v)
    one = time.perf_counter() - t0
    n = max(1, min(5, int(budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        step(q, k, v)
    dt = (time.perf_counter() - t0) / n
    return {
        "value": round(3.5 * wl.flops() / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (f"stock torch SDPA forward+backward on host CPU tensors, full {wl.name} workload "
                   f"{list(wl.shapes()[0])} {dt_used}, 1 warmup + {n} timed steps, "
                   f"{dt * 1e3:.1f} ms/step"),
    }


def bench_training(wl, args) -> dict:
    import torch
    import cmpext3
    g = torch.Generator().manual_seed(1)
    q, k, v = wl.make_inputs("cuda")
    do = torch.randn(q.shape, generator=g).to(q.dtype).to("cuda")
    ops, sc, ca = cmpext3.ops, wl.eff_scale, wl.causal
    out, lse = ops.attention_fwd_lse(q, k, v, sc, ca)
    fwd = lambda: ops.attention_fwd_lse(q, k, v, sc, ca)  # noqa: E731
    bwd = lambda: ops.attention_bwd(q, k, v, out, do, lse, sc, ca)  # noqa: E731

    def step():
        fwd()
        bwd()

    wall, dev_step = time_kernel(step, args.steps, args.warmup)
    _, dev_fwd = time_kernel(fwd, args.steps, 3)
    _, dev_bwd = time_kernel(bwd, args.steps, 3)
    f_fwd, f_bwd = wl.flops(), 2.5 * wl.flops()
    peak = 2516.6 if wl.dtype in ("fp16", "bf16") else 157.3
    return {
        "metric": "attention training step (fwd with lse + bwd) TFLOP/s, % of MI355X MFMA peak",
        "value": round((f_fwd + f_bwd) * args.steps / wall / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[wl.dtype],
        "data": "synthetic (seeded N(0,1) Q/K/V/dO, CPU generator -> device)",
        "config": {"workload": wl.name, "B": wl.B, "H": wl.H, "Sq": wl.Sq, "Sk": wl.Sk, "D": wl.D,
                   "causal": wl.causal, "scale": sc,
                   "entry": "cmpext3.ops.attention_fwd_lse + attention_bwd -> cmpext3_attn_fwd_lse, "
                            "cmpext3_attn_bwd_ws"},
        "roofline": {"bound": "mfma", "achieved": round(f_bwd / dev_bwd / 1e12, 3), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(f_bwd / dev_bwd / 1e12 / peak, 4), "traffic": None,
                     "kernel_us": round(dev_bwd * 1e6, 3), "flops_per_launch": f_bwd,
                     "what": "backward call (Delta + dK/dV + dQ kernels) as one unit"},
        "forward_lse": {"kernel_us": round(dev_fwd * 1e6, 3),
                        "tflops": round(f_fwd / dev_fwd / 1e12, 3)},
        "step_device_us": round(dev_step * 1e6, 3),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_training(wl),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true")
    ap.add_argument("--backward", action="store_true",
                    help="time a training step (forward with lse + backward) instead")
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="after the timed loop, run 3 plain elementwise copies (fp32, out = in*1) "
                         "of this many MiB: the known-traffic kernel that scales rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE readings")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (attention forward shards per "
              "(batch, head) with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    _ensure_built()
    import torch
    import cmpext3
    from cmpext3 import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    wl = W.BY_NAME[args.workload] if args.workload else W.HEADLINE
    torch.manual_seed(0)
    if args.backward:
        print(json.dumps(bench_training(wl, args)), flush=True)
        return 0
    q, k, v = wl.make_inputs("cuda")
    fn = lambda: cmpext3.ops.attention(q, k, v, wl.eff_scale, wl.causal)  # noqa: E731

    wall, dev = time_kernel(fn, args.steps, args.warmup)
    ms = wall / args.steps * 1e3
    value = wl.flops() * args.steps / wall / 1e12
    peak = W.PEAK_TFLOPS[wl.dtype]
    traffic = _traffic_from_profile(wl.name)
    # below the ridge point (peak FLOP/s over peak HBM bytes/s) HBM bounds the kernel
    hbm_bound = wl.flops() / wl.bytes() < peak * 1e12 / (W.PEAK_HBM_GBS * 1e9)
    if hbm_bound:
        roofline = {"bound": "hbm", "achieved": round(wl.bytes() / dev / 1e9, 1), "peak": W.PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(wl.bytes() / dev / 1e9 / W.PEAK_HBM_GBS, 4),
                    "traffic": traffic, "kernel_us": round(dev * 1e6, 3), "bytes_per_launch": wl.bytes()}
    else:
        achieved = wl.flops() / dev / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": peak,
                    "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
                    "kernel_us": round(dev * 1e6, 3), "flops_per_launch": wl.flops()}

    if args.calibrate_copy_mb > 0:
        n = args.calibrate_copy_mb * (1 << 20) // 4
        src = torch.rand(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

    configs = {}
    if not args.no_configs:
        for other in W.WORKLOADS:
            qo, ko, vo = other.make_inputs("cuda")
            f2 = lambda: cmpext3.ops.attention(qo, ko, vo, other.eff_scale, other.causal)  # noqa
            _, d2 = time_kernel(f2, 20, 5)
            entry = {
                "us_per_launch": round(d2 * 1e6, 2),
                "tflops": round(other.flops() / d2 / 1e12, 2),
                "pct_fp16_mfma_peak": round(100 * other.flops() / d2 / 1e12 / 2516.6, 2),
                "pct_dtype_peak": round(100 * other.flops() / d2 / 1e12 / W.PEAK_TFLOPS[other.dtype], 2),
                "hbm_gbs_algorithmic": round(other.bytes() / d2 / 1e9, 1),
            }
            if not args.no_cpu_baseline:
                out = f2()
                torch.cuda.synchronize()
                entry.update(config_cpu_and_error(other, out))
                entry["gpu_speedup_vs_cpu"] = round(entry["cpu_ms"] / (d2 * 1e3), 1)
            configs[other.name] = entry
            del qo, ko, vo

    line = {
        "metric": "attention fwd TFLOP/s and % of MI355X fp16/bf16 MFMA peak; x vs host-CPU SDPA",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "f16", "bf16": "bf16", "fp32": "f32"}[wl.dtype],
        "data": "synthetic (seeded N(0,1) Q/K/V, CPU generator -> device)",
        "config": {"workload": wl.name, "B": wl.B, "H": wl.H, "Hkv": wl.kv_heads, "Sq": wl.Sq,
                   "Sk": wl.Sk, "D": wl.D, "causal": wl.causal, "scale": wl.eff_scale,
                   "entry": "cmpext3.ops.attention -> cmpext3_attn_fwd_ws"},
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(wl),
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
