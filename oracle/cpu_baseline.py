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


def cores() -> int:
    return len(os.sched_getaffinity(0))


def median_seconds(fn, reps: int = 3, warmup: int = 1) -> float:
    """Median wall-clock seconds of ``fn()`` over ``reps`` runs after ``warmup`` untimed ones."""
    import numpy as np

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def _cl(t):
    import torch

    return t.contiguous(memory_format=torch.channels_last_3d)


def config_legs(reps: int = 3) -> dict:
    """PyTorch CPU fp32 timings of configs 1, 2a, 2b and 2c (the reference's CPU-path ops, all host
    cores, channels-last), median of ``reps`` after one warm-up: milliseconds per operation."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    torch.set_num_threads(cores())
    rng = np.random.default_rng(1)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    w = lambda o, i, k=3: _cl(t(rng.standard_normal((o, i, k, k, k)) / np.sqrt(k ** 3 * i)))
    out = {}
    with torch.no_grad():
        x1 = _cl(t(rng.standard_normal((1, 128, 128, 128, 128))).permute(0, 4, 1, 2, 3))
        w1, w2, b = w(128, 128), w(128, 128), torch.zeros(128)
        g, z = torch.ones(128), torch.zeros(128)

        def block():
            h = F.conv3d(_cl(F.silu(F.group_norm(x1, 32, g, z, 1e-6))), w1, b, padding=1)
            h = F.conv3d(_cl(F.silu(F.group_norm(h, 32, g, z, 1e-6))), w2, b, padding=1)
            return x1 + h

        out["config1"] = median_seconds(block, reps) * 1e3
        del x1
        xa = _cl(t(rng.standard_normal((1, 128, 128, 128, 64))).permute(0, 4, 1, 2, 3))
        wa = w(128, 64)
        out["config2a"] = median_seconds(lambda: F.conv3d(xa, wa, torch.zeros(128), padding=1, stride=2), reps) * 1e3
        del xa
        xb = _cl(t(rng.standard_normal((1, 64, 64, 64, 256))).permute(0, 4, 1, 2, 3))
        wb = w(128, 256)
        out["config2b"] = median_seconds(
            lambda: F.conv3d(_cl(F.interpolate(xb, scale_factor=2, mode="nearest")), wb, torch.zeros(128), padding=1),
            reps) * 1e3
        del xb
        xc = _cl(t(rng.standard_normal((1, 64, 64, 64, 128))).permute(0, 4, 1, 2, 3))
        wc = w(256, 128, 1)
        out["config2c"] = median_seconds(lambda: F.conv3d(xc, wc, torch.zeros(256)), reps) * 1e3
    return out


def vae_decode_seconds(weights_host: dict, constructor: dict, z, roi, overlap: float) -> float:
    """One full sliding-window decode on the CPU (PyTorch fp32, the restated MAISI decoder and
    Gaussian blend of decode.py:104-245, then the int16 conversion of image.py:85-87): seconds of
    one run after a warm-up on a 1/8-size window (the full decode takes tens of seconds)."""
    import torch

    from . import maisi_torch as mt

    torch.set_num_threads(cores())
    w = mt.to_torch(weights_host, dtype=torch.float32, strip="")
    zt = torch.from_numpy(z).permute(0, 4, 1, 2, 3).contiguous()
    with torch.no_grad():
        mt.vae_decode(zt[:, :, :10, :32, :32].contiguous(), w, constructor)
        t0 = time.perf_counter()
        y = mt.sliding_window_decode(zt, w, constructor, roi, overlap, scale_factor=1.0)
        torch.clamp(y * 1000.0, min=0.0).to(torch.int16)
        return time.perf_counter() - t0
