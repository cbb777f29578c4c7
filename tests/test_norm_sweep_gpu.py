"""Seeded random sweep of the group-norm kernels against the float64 oracle.

Cases draw batch 1-3, ragged extents (1 to 24 per axis, plus two volumes of a few
million elements that take many partial chunks), channel counts from 4 to 512
with every group count from 1 to 32 that divides them, an offset mean (the
one-pass fp64 variance must not cancel), eps and SiLU on or off.  The (N, C, 2)
affine of ``ctmr_gn_affine`` and the applied norm (+ SiLU) must match
tests/test_fast_fp32.py:41-48's float64 group norm (biased variance) within 1e-6
relative, and repeat bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

REL = 1e-6
CHANNELS = (4, 8, 16, 32, 48, 64, 96, 128, 256, 320, 512)


def _draw_cases(count: int, seed: int) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        c = int(rng.choice(CHANNELS))
        groups = int(rng.choice([g for g in (1, 2, 4, 8, 16, 32) if c % g == 0]))
        if i < 2:  # large volumes: many partial chunks per group
            spatial, n = ((40, 40, 40), 1) if i == 0 else ((24, 32, 48), 2)
            c, groups = (64, 32) if i == 0 else (32, 8)
        else:
            spatial, n = tuple(int(v) for v in rng.integers(1, 25, size=3)), int(rng.integers(1, 4))
        cases.append(dict(id=f"gn{i:02d}", n=n, spatial=spatial, c=c, groups=groups,
                          eps=float(rng.choice([1e-6, 1e-5])), silu=bool(rng.random() < 0.5),
                          mean=float(rng.uniform(-4, 4)), seed=seed * 1000 + i))
    return cases


CASES = _draw_cases(40, 77)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_random_group_norm_matches_float64(ctmr, dev, case):
    print(f"gn sweep {case}", flush=True)
    f = ctmr.fast_fp32
    rng = np.random.default_rng(case["seed"])
    n, c, groups, eps = case["n"], case["c"], case["groups"], case["eps"]
    x = (rng.uniform(0.5, 3.0) * rng.standard_normal((n, *case["spatial"], c)) + case["mean"]).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    xt, gt, bt = _t(x, dev), _t(gamma, dev), _t(beta, dev)

    aff = f.group_norm_affine(xt, gt, bt, groups=groups, eps=eps)
    err = rm.max_rel_error(aff.cpu().numpy(), rm.group_norm_affine(x, gamma, beta, groups, eps))
    print(f"{case['id']}: affine max rel error {err:.3e}", flush=True)
    assert err <= REL

    y = f.group_norm(xt, gt, bt, num_groups=groups, eps=eps, apply_silu=case["silu"])
    expected = rm.group_norm(x, gamma, beta, groups, eps, apply_silu=case["silu"])
    err = rm.max_rel_error(y.cpu().numpy(), expected)
    print(f"{case['id']}: norm max rel error {err:.3e}", flush=True)
    assert err <= REL
    assert torch.equal(f.group_norm(xt, gt, bt, num_groups=groups, eps=eps, apply_silu=case["silu"]), y)


@pytest.mark.parametrize(("shape", "silu"), [
    ((2, 64, 64, 32, 64), True),    # UNet top-level down block input
    ((1, 9, 7, 11, 48), True),      # odd extents: the last plane, row and column are dropped
    ((2, 6, 4, 8, 6), False),       # channels not a multiple of 4 (scalar path)
])
def test_gn_avgpool_equals_gn_apply_then_pool(ctmr, dev, shape, silu):
    """``ctmr_gn_avgpool`` (the down-sampling residual block's norm + SiLU + pool and the pool of its
    input, from one read) equals ``gn_apply`` followed by the average pool, and the pool of the input,
    bit for bit; both within the float64 bar."""
    print(f"gn_avgpool {shape} silu={silu}", flush=True)
    ops = ctmr.ops
    g = torch.Generator(device=dev).manual_seed(sum(shape))
    x = 1.5 * torch.randn(*shape, device=dev, generator=g) + 0.25
    n, c = shape[0], shape[-1]
    affine = torch.stack([1 + 0.2 * torch.randn(n, c, device=dev, generator=g),
                          0.3 * torch.randn(n, c, device=dev, generator=g)], dim=-1).contiguous()
    y, y_skip = ops.gn_avgpool(x, affine, silu)
    assert torch.equal(y, ops.resample(ops.gn_apply(x, affine, silu), ctmr._lib.AVGPOOL2))
    assert torch.equal(y_skip, ops.resample(x, ctmr._lib.AVGPOOL2))
    y2, _ = ops.gn_avgpool(x, affine, silu)
    assert torch.equal(y, y2)
    xh, ah = x.double().cpu().numpy(), affine.double().cpu().numpy()
    t = xh * ah[:, None, None, None, :, 0] + ah[:, None, None, None, :, 1]
    if silu:
        t = t / (1 + np.exp(-t))
    d2, h2, w2 = (v // 2 for v in shape[1:4])
    pool = lambda a: a[:, :2 * d2, :2 * h2, :2 * w2].reshape(n, d2, 2, h2, 2, w2, 2, c).mean(axis=(2, 4, 6))
    assert rm.max_rel_error(y.cpu().numpy(), pool(t)) <= REL
    assert rm.max_rel_error(y_skip.cpu().numpy(), pool(xh)) <= REL
