"""CPU baseline timing for bench.py — TEST/BENCH INFRASTRUCTURE ONLY.

The reference's CPU path cannot run here (MLX is Darwin-arm64 only,
pyproject.toml:44), so the baseline is the operation its parity tests compare
against: PyTorch's fp32 ``conv3d`` on the CPU (tests/test_maisi_mlx_blocks.py,
tests/_torch.py of the reference), timed in both the channels-last-3d and the
contiguous NCDHW layout; the faster is reported.
"""

from __future__ import annotations

import os
import platform
import time


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_config0_conv(budget_s: float = 20.0) -> dict:
    """Time config 0 (64^3 x 64 -> 64 conv3d, 57.98 GFLOP) on the host cores."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 64), dtype=np.float32)).permute(0, 4, 1, 2, 3)
    w = torch.from_numpy((rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32))
    b = torch.from_numpy((0.01 * rng.standard_normal(64)).astype(np.float32))
    flops = 2.0 * 64**3 * 64 * 64 * 27
    best = {}
    deadline = time.perf_counter() + budget_s
    for layout in ("channels_last_3d", "contiguous"):
        fmt = torch.channels_last_3d if layout == "channels_last_3d" else torch.contiguous_format
        xi, wi = x.contiguous(memory_format=fmt), w.contiguous(memory_format=fmt)
        with torch.no_grad():
            F.conv3d(xi, wi, b, padding=1)  # warm-up
            times = []
            while len(times) < 3 or (len(times) < 10 and time.perf_counter() < deadline):
                t0 = time.perf_counter()
                F.conv3d(xi, wi, b, padding=1)
                times.append(time.perf_counter() - t0)
                if time.perf_counter() > deadline + budget_s:
                    break
        best[layout] = float(np.median(times))
    layout = min(best, key=best.get)
    sec = best[layout]
    return {
        "value": round(flops / sec / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"full config-0 conv3d (57.98 GFLOP) via torch.nn.functional.conv3d fp32 on CPU, "
                   f"{layout} layout (faster of channels_last_3d/contiguous), median of >=3 runs, "
                   f"{sec * 1e3:.1f} ms/conv; torch {torch.__version__}; {_cpu_model()}"),
    }
