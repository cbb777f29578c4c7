"""Seeded random sweep of the conv operator against the float64 oracle.

Each case draws a shape and option set (fp32 / bf16, 3x3x3 / 1x1x1, stride 2,
nearest-2x / trilinear-2x upsampling, GN affine (+ SiLU) staging, residual,
per-channel / per-batch bias, batch 1-2, ragged extents and channel counts
from 1 to 128), so the library's shape-driven routing (LDS-staged or
streaming GEMM, direct reads or packed copy, K splits, pointwise, im2col and
tap-expanded layouts) is exercised on shapes no hand-written case names.
Every case must meet the per-layer bar of its dtype against the float64
restatement and repeat bit for bit.  Sizes stay small enough for the float64
oracle to take well under a second per case (96 cases: about 1 s of oracle
time in all).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
BF16_REL = 2e-2
CIN = (1, 3, 4, 8, 16, 24, 32, 48, 64, 96, 128)
COUT = (1, 3, 4, 8, 16, 20, 32, 64, 96, 128)


def _draw_cases(count: int, seed: int) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        bf16 = bool(rng.random() < 0.3)
        ksize = 1 if rng.random() < 0.15 else 3
        mode, stride = "plain", 1
        if ksize == 3:
            r = rng.random()
            mode = "nearest" if r < 0.2 else ("trilinear" if r < 0.4 else "plain")
            if mode == "plain" and rng.random() < 0.25:
                stride = 2
        up = mode != "plain"
        hi = 7 if up else 13
        spatial = tuple(int(v) for v in rng.integers(1, hi, size=3))
        n = int(rng.integers(1, 3))
        cin, cout = int(rng.choice(CIN)), int(rng.choice(COUT))
        affine = mode != "trilinear" and bool(rng.random() < 0.4)
        silu = affine and bool(rng.random() < 0.8)
        residual = bool(rng.random() < 0.3)
        bias = ("none", "channel", "batch")[int(rng.integers(0, 3))]
        cases.append(dict(id=f"case{i:02d}", bf16=bf16, ksize=ksize, mode=mode, stride=stride, n=n,
                          spatial=spatial, cin=cin, cout=cout, affine=affine, silu=silu, residual=residual,
                          bias=bias, seed=seed * 1000 + i))
    return cases


CASES = _draw_cases(96, 2024)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_random_conv_matches_float64(ctmr, dev, case):
    print(f"sweep {case}", flush=True)
    f = ctmr.fast_fp32
    rng = np.random.default_rng(case["seed"])
    n, cin, cout, k = case["n"], case["cin"], case["cout"], case["ksize"]
    x = (2 * rng.standard_normal((n, *case["spatial"], cin)) + 0.3).astype(np.float32)
    w = (rng.standard_normal((cout, cin, k, k, k)) / np.sqrt(cin * k ** 3)).astype(np.float32)
    bias = None
    if case["bias"] == "channel":
        bias = rng.standard_normal(cout).astype(np.float32)
    elif case["bias"] == "batch":
        bias = rng.standard_normal((n, cout)).astype(np.float32)
    affine = None
    if case["affine"]:
        affine = np.stack([1 + 0.2 * rng.standard_normal((n, cin)), 0.2 * rng.standard_normal((n, cin))],
                          axis=-1).astype(np.float32)

    prepared = x.astype(np.float64)
    if affine is not None:
        prepared = rm.apply_affine(prepared, affine, case["silu"])
    if case["mode"] == "nearest":
        prepared = rm.upsample_nearest(prepared)
    elif case["mode"] == "trilinear":
        prepared = rm.upsample_trilinear(prepared)
    expected = rm.conv3d(prepared, w, bias, stride=case["stride"])
    residual = None
    if case["residual"]:
        residual = rng.standard_normal(expected.shape).astype(np.float32)
        expected = expected + residual

    dtype = "bf16" if case["bf16"] else "fp32"
    wt = _t(w, dev)
    packed = f.pack_upsample_weight(wt, dtype=dtype) if case["mode"] == "nearest" else f.pack_weight(wt, dtype=dtype)
    kw = dict(cout=cout, ksize=k, affine=None if affine is None else _t(affine, dev), silu=case["silu"],
              stride=case["stride"], upsample=case["mode"] == "nearest", trilinear=case["mode"] == "trilinear",
              residual=None if residual is None else _t(residual, dev))
    xt = _t(x, dev)
    bt = None if bias is None else _t(bias, dev)
    y = f.implicit_gemm_conv3d(xt, packed, bt, **kw)
    got = y.detach().cpu().numpy().astype(np.float64)
    assert got.shape == expected.shape, (got.shape, expected.shape)
    assert np.isfinite(got).all()
    err = rm.max_rel_error(got, expected)
    bound = BF16_REL if case["bf16"] else FP32_REL
    print(f"{case['id']}: max rel error {err:.3e} (bound {bound:g})", flush=True)
    assert err <= bound
    assert torch.equal(f.implicit_gemm_conv3d(xt, packed, bt, **kw), y), "not bit-identical run to run"
