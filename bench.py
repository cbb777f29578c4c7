"""Benchmark of the MI355X conv3d hot path (one JSON line on stdout).

Headline workload (the north-star conv target):
conv3d 3x3x3, stride 1, padding 1, +bias, NDHWC fp32, N=1, 64^3 voxels,
Cin = Cout = 64; 57.98 GFLOP per step.  One step = the full operator
(input pack + implicit-GEMM kernel) on inputs already resident in HBM.

``roofline`` is the GEMM kernel alone, timed live with HIP events on the
stream it is launched on, against the FP32 MFMA peak (157.3 TFLOP/s).
``cpu_baseline`` is the same conv via PyTorch CPU (the op the reference's
parity tests compare against), timed on this host's cores.
``secondary`` reports the other configs' GPU numbers (config 1 residual
block, config 2 resolution-change convs, bf16 variant of config 0).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]
"""

from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

FP32_PEAK = 157.3e12
BF16_PEAK = 2516.6e12
HBM_PEAK = 8.0e12


def conv_flops(n, d, h, w, cin, cout, taps=27):
    return 2.0 * n * d * h * w * cin * cout * taps


def _events_ms(fn, iters):
    import torch

    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def _wall_ms(fn, steps):
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def gemm_only(pkg, x, w, b, dtype_code):
    """A closure launching only the implicit-GEMM stage on a pre-packed input."""
    import torch

    L, ops = pkg._lib, pkg.ops
    cin, cout = int(x.shape[-1]), int(w.shape[0])
    desc = ops.make_desc(tuple(x.shape), cout, 3, 1, L.MODE_PLAIN, 0, dtype_code, 0)
    ws_bytes = L.workspace_bytes(desc)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    packed_w = ops.pack_weight(w, cin, cout, 3, L.MODE_PLAIN, dtype_code)
    y = torch.empty((*x.shape[:-1], cout), device=x.device, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    lib = L.lib()
    L.check(lib.ctmr_conv3d_pack(ctypes.byref(desc), x.data_ptr(), None, ws.data_ptr(), ws_bytes, stream),
            "ctmr_conv3d_pack")

    def run():
        lib.ctmr_conv3d_gemm(ctypes.byref(desc), x.data_ptr(), packed_w.data_ptr(), b.data_ptr(), None,
                             y.data_ptr(), ws.data_ptr(), ws_bytes, stream)

    run()
    L.check(lib.ctmr_conv3d_gemm(ctypes.byref(desc), x.data_ptr(), packed_w.data_ptr(), b.data_ptr(), None,
                                 y.data_ptr(), ws.data_ptr(), ws_bytes, stream), "ctmr_conv3d_gemm")
    return run, (ws, packed_w, y)


def cpu_baseline(budget_s=20.0):
    """Config 0 conv via PyTorch CPU fp32 (oracle.cpu_baseline), best of layouts."""
    from oracle import cpu_baseline as cb

    return cb.time_config0_conv(budget_s=budget_s)


def secondary(pkg, dev, steps):
    """Config 1 (VAE residual block at 128^3 x 128) and config 2 GPU numbers."""
    import numpy as np
    import torch

    f = pkg.fast_fp32
    out = {}
    rng = np.random.default_rng(1)
    c, s = 128, 128
    x = torch.from_numpy(rng.standard_normal((1, s, s, s, c), dtype=np.float32)).to(dev)
    mk = lambda cout, cin, k=3: torch.from_numpy(
        (rng.standard_normal((cout, cin, k, k, k)) / np.sqrt(k**3 * cin)).astype(np.float32)).to(dev)
    w1, w2 = mk(c, c), mk(c, c)
    b1 = torch.from_numpy((0.01 * rng.standard_normal(c)).astype(np.float32)).to(dev)
    b2 = torch.from_numpy((0.01 * rng.standard_normal(c)).astype(np.float32)).to(dev)
    g = torch.ones(c, device=dev)
    z = torch.zeros(c, device=dev)

    def block():
        return f.vae_resblock([x], (w1, b1), (w2, b2), (g, z), (g, z), None, num_groups=32, eps=1e-6)

    for _ in range(2):
        block()
    ms = _wall_ms(block, max(2, steps // 4))
    flops = 2 * conv_flops(1, s, s, s, c, c)
    out["config1_vae_resblock_128c_128^3"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 2),
                                              "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    del x
    # config 2a: stride-2 conv 64->128, 128^3 -> 64^3
    xa = torch.from_numpy(rng.standard_normal((1, 128, 128, 128, 64), dtype=np.float32)).to(dev)
    wa, ba = mk(128, 64), torch.zeros(128, device=dev)
    run = lambda: f.conv3d(xa, wa, ba, padding=1, stride=2)
    run()
    ms = _wall_ms(run, steps)
    flops = conv_flops(1, 64, 64, 64, 64, 128)
    out["config2a_down_s2_64to128"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 2),
                                       "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    del xa
    # config 2b: nearest-2x + conv 256->128, 64^3 -> 128^3 (8-tap parity fold)
    xb = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 256), dtype=np.float32)).to(dev)
    wb, bb = mk(128, 256), torch.zeros(128, device=dev)
    run = lambda: f.norm_conv3d(xb, wb, bb, norm=None, num_groups=1, eps=1e-6, apply_silu=False, upsample=True)
    run()
    ms = _wall_ms(run, max(2, steps // 2))
    flops = conv_flops(8, 64, 64, 64, 256, 128, taps=8)
    out["config2b_nearest_up_256to128"] = {"ms": round(ms, 3), "tflops_folded": round(flops / ms / 1e9, 2),
                                           "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    del xb
    # config 2c: 1x1x1 128 -> 256 at 64^3
    xc = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 128), dtype=np.float32)).to(dev)
    wc, bc = mk(256, 128, 1), torch.zeros(256, device=dev)
    run = lambda: f.pointwise_conv(xc, wc, bc)
    run()
    ms = _wall_ms(run, steps)
    flops = 2.0 * 64**3 * 128 * 256
    nbytes = 4.0 * 64**3 * (128 + 256)
    out["config2c_pointwise_128to256"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                                          "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4),
                                          "hbm_GBps": round(nbytes / ms / 1e6, 1),
                                          "frac_hbm": round(nbytes / ms / 1e-3 / HBM_PEAK, 4)}
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip the config 1/2 measurements")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM-counter scale reference for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (N=1); multi-GPU runs are not part of it",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy:
        src = torch.ones(1 << 28, device="cuda:0")  # 1 GiB fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                          "launches": 3}), flush=True)
        return 0

    pkg = importlib.import_module("mlx-generate-ctmr_amd")
    f = pkg.fast_fp32
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    n, s, cin, cout = 1, 64, 64, 64
    x = torch.from_numpy(rng.standard_normal((n, s, s, s, cin), dtype=np.float32)).to(dev)
    w = torch.from_numpy((rng.standard_normal((cout, cin, 3, 3, 3)) / np.sqrt(27 * cin)).astype(np.float32)).to(dev)
    b = torch.from_numpy((0.01 * rng.standard_normal(cout)).astype(np.float32)).to(dev)
    flops = conv_flops(n, s, s, s, cin, cout)

    step = lambda: f.conv3d(x, w, b, padding=1)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    value = flops / (ms * 1e-3) / 1e12

    # dominant kernel (implicit GEMM) alone, HIP events on its stream
    run_gemm, _keep = gemm_only(pkg, x, w, b, pkg._lib.DT_F32)
    for _ in range(3):
        run_gemm()
    gemm_ms = _events_ms(run_gemm, max(args.steps, 10))
    achieved = flops / (gemm_ms * 1e-3)
    # bf16 variant of the same layer (secondary)
    run_bf16, _keep16 = gemm_only(pkg, x, w, b, pkg._lib.DT_BF16)
    for _ in range(3):
        run_bf16()
    bf16_ms = _events_ms(run_bf16, max(args.steps, 10))

    result = {
        "metric": "conv3d fp32 TFLOP/s (implicit GEMM, FP32 MFMA)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy default_rng(0) Gaussian input/weights, bias N(0,0.01))",
        "config": {"workload": "config0: conv3d 3x3x3 s1 p1 +bias, NDHWC fp32, N=1, 64^3, Cin=Cout=64",
                   "flop_per_step": flops, "step": "input pack + implicit-GEMM conv"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 3), "peak": FP32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK, 4), "traffic": None,
                     "kernel": "conv_kernel<f32> (implicit GEMM)", "kernel_ms": round(gemm_ms, 4)},
    }
    # HBM bytes per GEMM launch from the committed rocprofv3 --pmc passes
    # (FETCH_SIZE x read scale + WRITE_SIZE x write scale, copy-calibrated).
    traffic_file = REPO / "profiles" / "conv3d_config0_traffic.json"
    if traffic_file.exists():
        result["roofline"]["traffic"] = json.loads(traffic_file.read_text())["traffic_bytes"]
        result["roofline"]["traffic_source"] = "profiles/conv3d_config0_traffic.json"
    sec = {"config0_bf16_gemm": {"ms": round(bf16_ms, 4), "tflops": round(flops / bf16_ms / 1e9, 2),
                                 "frac_bf16_peak": round(flops / (bf16_ms * 1e-3) / BF16_PEAK, 4)}}
    if not args.no_secondary:
        sec.update(secondary(pkg, dev, args.steps))
    result["secondary"] = sec
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
