"""Group-norm statistics written by the convolution epilogues (``ctmr_conv3d_gn``).

For every GEMM form (register-streaming, LDS-staged, K split through the
reduction, nearest-2x parity phases, im2col, trilinear, stride 2, bf16) the
fused call must
* store the same output bits as ``ctmr_conv3d``;
* hold partials whose per-(batch item, group) totals equal float64 sums of the
  stored output (a wrong tile or group slot changes a total);
* give the affine of ``ctmr_gn_affine`` on that output (both fp64 statistics,
  different summation orders: max relative difference 1e-6);
* repeat bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

AFFINE_REL = 1e-6  # two fp64 statistics of the same fp32 values, rounded to fp32
TOTAL_REL = 1e-12  # float64 totals of the same values in different orders


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


CASES = [
    # (name, x shape NDHWC, cout, groups, keyword arguments)
    ("streaming", (2, 8, 16, 16, 64), 64, 32, {"split": 1, "stream_gemm": True}),
    ("streaming ragged", (1, 7, 9, 13, 48), 64, 8, {"split": 1}),
    ("streaming 2x2 waves", (1, 16, 16, 32, 64), 256, 32, {"split": 1, "stream_gemm": True}),
    ("streaming 128-wide groups", (1, 16, 16, 32, 32), 256, 2, {"split": 1}),
    ("lds fused", (2, 8, 16, 16, 128), 128, 32, {"split": 1, "fused": True}),
    ("lds ragged", (1, 7, 16, 15, 128), 64, 16, {"split": 1}),
    ("lds split", (1, 4, 8, 8, 512), 512, 32, {"split": 8}),
    ("streaming split", (2, 4, 8, 8, 256), 256, 32, {"stream_gemm": True, "fused": True}),
    ("nearest-2x phases", (1, 4, 8, 8, 64), 64, 32, {"upsample": True, "split": 1}),
    ("nearest-2x split", (2, 4, 4, 4, 128), 128, 32, {"upsample": True}),
    ("im2col", (2, 8, 8, 8, 4), 64, 32, {"split": 1}),
    ("trilinear", (1, 4, 8, 8, 32), 32, 8, {"trilinear": True, "split": 1}),
    ("stride 2", (1, 8, 16, 16, 32), 64, 16, {"stride": 2, "split": 1}),
    ("bf16", (2, 8, 16, 16, 64), 64, 32, {"bf16": True, "split": 1}),
    ("bf16 split", (2, 8, 16, 16, 64), 64, 32, {"bf16": True}),
    ("bf16 nearest-2x LDS parities", (2, 4, 8, 8, 64), 64, 32, {"bf16": True, "upsample": True, "split": 1}),
    ("bf16 nearest-2x LDS fused ragged", (1, 7, 16, 15, 64), 128, 16,
     {"bf16": True, "upsample": True, "split": 1, "fused": True}),
]


@pytest.mark.parametrize(("name", "shape", "cout", "groups", "kw"), CASES, ids=[c[0] for c in CASES])
def test_epilogue_statistics_match_a_separate_pass(ctmr, dev, name, shape, cout, groups, kw):
    print(f"case {name}: {shape} -> {cout}, {groups} groups, {kw}", flush=True)
    f, ops, L = ctmr.fast_fp32, ctmr.ops, ctmr._lib
    kw = dict(kw)
    fused, bf16 = kw.pop("fused", False), kw.pop("bf16", False)
    rng = np.random.default_rng(sum(shape) + cout + groups)
    n, c = shape[0], shape[-1]
    x = (2 * rng.standard_normal(shape) + 0.5).astype(np.float32)
    w = (rng.standard_normal((cout, c, 3, 3, 3)) / np.sqrt(27 * c)).astype(np.float32)
    bias = rng.standard_normal((n, cout)).astype(np.float32)
    dtype = "bf16" if bf16 else "fp32"
    wt = _t(w, dev)
    packed = f.pack_upsample_weight(wt, dtype=dtype) if kw.get("upsample") else f.pack_weight(wt, dtype=dtype)
    xt = _t(x, dev)
    affine = residual = None
    if fused:
        gw = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
        gb = (0.1 * rng.standard_normal(c)).astype(np.float32)
        affine = f.group_norm_affine(xt, _t(gw, dev), _t(gb, dev), groups=8, eps=1e-6)
    call = dict(cout=cout, affine=affine, silu=fused, **kw)
    plain = f.implicit_gemm_conv3d(xt, packed, _t(bias, dev), residual=None, **call)
    if fused:
        residual = _t(rng.standard_normal(tuple(plain.shape)).astype(np.float32), dev)
        plain = f.implicit_gemm_conv3d(xt, packed, _t(bias, dev), residual=residual, **call)
    y = f.implicit_gemm_conv3d(xt, packed, _t(bias, dev), residual=residual, gn_groups=groups, **call)
    stats = f.conv_output_stats(y, groups)
    assert stats is not None, "this shape should produce epilogue statistics"
    assert stats.dtype == torch.float64 and stats.shape[0] == n and stats.shape[2:] == (groups, 2)
    assert torch.equal(y, plain), "the fused-statistics call changed the output"

    yh = y.cpu().numpy().astype(np.float64).reshape(n, -1, groups, cout // groups)
    totals = stats.cpu().numpy().sum(axis=1)
    expected = np.stack([yh.sum(axis=(1, 3)), (yh * yh).sum(axis=(1, 3))], axis=-1)
    err = rm.max_rel_error(totals, expected)
    print(f"{name}: partial totals max rel error {err:.3e}", flush=True)
    assert err <= TOTAL_REL

    gamma = (1 + 0.1 * rng.standard_normal(cout)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(cout)).astype(np.float32)
    a_stats = f.group_norm_affine(y, _t(gamma, dev), _t(beta, dev), groups=groups, eps=1e-6)
    a_pass = ops.gn_affine(plain, _t(gamma, dev), _t(beta, dev), groups, 1e-6)
    err = rm.max_rel_error(a_stats.cpu().numpy(), a_pass.cpu().numpy())
    print(f"{name}: affine from partials vs separate pass {err:.3e}", flush=True)
    assert err <= AFFINE_REL

    y2 = f.implicit_gemm_conv3d(xt, packed, _t(bias, dev), residual=residual, gn_groups=groups, **call)
    assert torch.equal(y2, y)
    assert torch.equal(f.conv_output_stats(y2, groups), stats)
    assert L.F_STREAM  # the flag table is loaded


def test_statistics_are_dropped_after_an_in_place_change(ctmr, dev):
    f, ops = ctmr.fast_fp32, ctmr.ops
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 8, 8, 8, 64)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3, 3)) / 40).astype(np.float32)
    y = f.conv3d(_t(x, dev), _t(w, dev), None, padding=1, gn_groups=32)
    assert f.conv_output_stats(y, 32) is not None
    assert f.conv_output_stats(y, 16) is None  # other group counts use the separate pass
    y.mul_(3.0).add_(1.0)
    assert f.conv_output_stats(y, 32) is None
    gamma, beta = torch.ones(64, device=dev), torch.zeros(64, device=dev)
    got = f.group_norm_affine(y, gamma, beta, groups=32, eps=1e-6)
    assert torch.equal(got, ops.gn_affine(y, gamma, beta, 32, 1e-6))


def test_shapes_without_statistics_fall_back(ctmr, dev):
    """cout <= 4 (tap sum) and groups that do not fit the tile compute without partials."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(4)
    x = _t(rng.standard_normal((1, 6, 6, 6, 64)).astype(np.float32), dev)
    w1 = _t((rng.standard_normal((1, 64, 3, 3, 3)) / 40).astype(np.float32), dev)
    y = f.conv3d(x, w1, None, padding=1, gn_groups=1)
    assert f.conv_output_stats(y, 1) is None
    assert torch.equal(y, f.conv3d(x, w1, None, padding=1))


FINER_CASES = [
    # (name, x shape NDHWC, cout, stat groups written by the conv, norm groups, keyword arguments)
    ("per channel lds", (2, 8, 16, 16, 64), 64, 64, 32, {"split": 1}),
    ("per channel streaming", (2, 8, 16, 16, 64), 64, 64, 32, {"split": 1, "stream_gemm": True}),
    ("per channel split", (1, 4, 8, 8, 512), 512, 512, 32, {"split": 8}),
    ("per channel nearest-2x", (1, 4, 8, 8, 64), 64, 64, 32, {"upsample": True, "split": 1}),
    ("finer groups", (2, 8, 16, 16, 128), 128, 32, 8, {"split": 1}),
]


def _count_read_passes(monkeypatch, ops):
    """Counts ``ops.gn_affine`` calls (statistics read passes) by the number of sources."""
    calls = {"one": 0, "cat": 0}
    real = ops.gn_affine

    def counted(x, gamma, beta, groups, eps, x2=None):
        calls["one" if x2 is None else "cat"] += 1
        return real(x, gamma, beta, groups, eps, x2)

    monkeypatch.setattr(ops, "gn_affine", counted)
    return calls, real


@pytest.mark.parametrize(("name", "shape", "cout", "sgroups", "groups", "kw"), FINER_CASES,
                         ids=[c[0] for c in FINER_CASES])
def test_norm_from_finer_epilogue_statistics(ctmr, dev, monkeypatch, name, shape, cout, sgroups, groups, kw):
    """A group norm over a conv output whose epilogue wrote statistics at a finer grouping (per channel
    for the up path's concatenations) reads no pass and gives the separate pass's affine."""
    print(f"case {name}: {shape} -> {cout}, stats {sgroups}, norm {groups}, {kw}", flush=True)
    f, ops = ctmr.fast_fp32, ctmr.ops
    rng = np.random.default_rng(sum(shape) + cout + sgroups)
    n, c = shape[0], shape[-1]
    x = (2 * rng.standard_normal(shape) + 0.5).astype(np.float32)
    w = (rng.standard_normal((cout, c, 3, 3, 3)) / np.sqrt(27 * c)).astype(np.float32)
    wt = _t(w, dev)
    packed = f.pack_upsample_weight(wt) if kw.get("upsample") else f.pack_weight(wt)
    y = f.implicit_gemm_conv3d(_t(x, dev), packed, None, cout=cout, gn_groups=sgroups, **kw)
    stats = f.conv_output_stats(y, sgroups)
    assert stats is not None and stats.shape[2] == sgroups
    yh = y.cpu().numpy().astype(np.float64).reshape(n, -1, sgroups, cout // sgroups)
    expected = np.stack([yh.sum(axis=(1, 3)), (yh * yh).sum(axis=(1, 3))], axis=-1)
    assert rm.max_rel_error(stats.cpu().numpy().sum(axis=1), expected) <= TOTAL_REL

    gamma = _t((1 + 0.1 * rng.standard_normal(cout)).astype(np.float32), dev)
    beta = _t((0.1 * rng.standard_normal(cout)).astype(np.float32), dev)
    calls, real = _count_read_passes(monkeypatch, ops)
    got = f.group_norm_affine(y, gamma, beta, groups=groups, eps=1e-6)
    assert calls == {"one": 0, "cat": 0}, "the norm read its input although finer statistics were attached"
    ref = real(y, gamma, beta, groups, 1e-6)
    err = rm.max_rel_error(got.cpu().numpy(), ref.cpu().numpy())
    print(f"{name}: affine from finer partials vs separate pass {err:.3e}", flush=True)
    assert err <= AFFINE_REL
    assert torch.equal(f.group_norm_affine(y, gamma, beta, groups=groups, eps=1e-6), got)  # run to run


CAT_CASES = [
    # (name, hidden channels, hidden stat groups, skip channels, skip stat groups, norm groups, reads a pass)
    ("64+64 per channel", 64, 64, 64, 64, 32, False),
    ("256+128 straddling, per channel", 256, 256, 128, 128, 32, False),
    ("256+128 straddling, 4-channel stat groups", 256, 64, 128, 32, 32, False),
    ("256+128 straddling, hidden at the norm's 8-channel groups", 256, 32, 128, 128, 32, True),
    ("128+64, skip without statistics", 128, 128, 64, 0, 32, True),
]


@pytest.mark.parametrize(("name", "c1", "sg1", "c2", "sg2", "groups", "reads"), CAT_CASES,
                         ids=[c[0] for c in CAT_CASES])
def test_concatenation_norm_from_both_halves_statistics(ctmr, dev, monkeypatch, name, c1, sg1, c2, sg2, groups,
                                                        reads):
    """The up path's norm1 over cat([hidden, skip]) (unet.py:444) from the two producers' partials:
    equal to the two-source read pass within the fp64-statistics bar, and to float64 statistics of
    the concatenation; groupings that do not tile the norm's groups (or a half without statistics)
    fall back to the read pass."""
    print(f"case {name}", flush=True)
    f, ops = ctmr.fast_fp32, ctmr.ops
    rng = np.random.default_rng(c1 + 3 * c2 + sg1 + sg2)
    shape = (2, 8, 8, 16)

    def produce(cout, sg):
        x = (rng.standard_normal((*shape, 32)) + 0.3).astype(np.float32)
        w = (rng.standard_normal((cout, 32, 3, 3, 3)) / np.sqrt(27 * 32)).astype(np.float32)
        return f.conv3d(_t(x, dev), _t(w, dev), None, padding=1, gn_groups=sg)

    hidden, skip = produce(c1, sg1), produce(c2, sg2)
    gamma = _t((1 + 0.1 * rng.standard_normal(c1 + c2)).astype(np.float32), dev)
    beta = _t((0.1 * rng.standard_normal(c1 + c2)).astype(np.float32), dev)
    calls, real = _count_read_passes(monkeypatch, ops)
    got = f.group_norm_affine(f.concat_channels(hidden, skip), gamma, beta, groups=groups, eps=1e-6)
    assert calls == {"one": 0, "cat": 1 if reads else 0}
    ref = real(hidden, gamma, beta, groups, 1e-6, skip)
    err = rm.max_rel_error(got.cpu().numpy(), ref.cpu().numpy())
    cat = np.concatenate([hidden.cpu().numpy(), skip.cpu().numpy()], -1).astype(np.float64).reshape(2, -1, groups,
                                                                                                   (c1 + c2) // groups)
    mean, var = cat.mean(axis=(1, 3)), cat.var(axis=(1, 3))
    scale = gamma.cpu().numpy()[None].astype(np.float64) / np.repeat(np.sqrt(var + 1e-6), (c1 + c2) // groups, -1)
    offset = beta.cpu().numpy()[None] - np.repeat(mean, (c1 + c2) // groups, -1) * scale
    err64 = rm.max_rel_error(got.cpu().numpy(), np.stack([scale, offset], -1))
    print(f"{name}: vs two-source pass {err:.3e}, vs float64 {err64:.3e}", flush=True)
    assert err <= AFFINE_REL and err64 <= AFFINE_REL


def test_add_with_statistics(ctmr, dev, monkeypatch):
    """``add_with_stats`` (the ControlNet residual added to a skip, the attention residual): the sum's
    bits equal ``a + b``, its per-channel partials total the float64 sums, and a norm of the sum, alone
    or concatenated, reads no pass."""
    f, ops = ctmr.fast_fp32, ctmr.ops
    rng = np.random.default_rng(21)
    a = _t(rng.standard_normal((2, 6, 10, 12, 128)).astype(np.float32), dev)
    b = _t((0.5 * rng.standard_normal((2, 6, 10, 12, 128)) + 0.2).astype(np.float32), dev)
    y = f.add_with_stats(a, b)
    assert torch.equal(y, a + b)
    stats = f.conv_output_stats(y, 128)
    assert stats is not None
    yh = y.cpu().numpy().astype(np.float64).reshape(2, -1, 128)
    expected = np.stack([yh.sum(axis=1), (yh * yh).sum(axis=1)], axis=-1)
    assert rm.max_rel_error(stats.cpu().numpy().sum(axis=1), expected) <= TOTAL_REL
    gamma, beta = torch.ones(128, device=dev), torch.zeros(128, device=dev)
    calls, real = _count_read_passes(monkeypatch, ops)
    got = f.group_norm_affine(y, gamma, beta, groups=32, eps=1e-6)
    other = f.add_with_stats(b, a)
    got_cat = f.group_norm_affine(f.concat_channels(y, other), torch.ones(256, device=dev),
                                  torch.zeros(256, device=dev), groups=32, eps=1e-6)
    assert calls == {"one": 0, "cat": 0}
    assert rm.max_rel_error(got.cpu().numpy(), real(y, gamma, beta, 32, 1e-6).cpu().numpy()) <= AFFINE_REL
    ref_cat = real(y, torch.ones(256, device=dev), torch.zeros(256, device=dev), 32, 1e-6, other)
    assert rm.max_rel_error(got_cat.cpu().numpy(), ref_cat.cpu().numpy()) <= AFFINE_REL
    # broadcasting sums and channel counts the kernel does not take are plain sums without statistics
    z = f.add_with_stats(a, b[:1])
    assert torch.equal(z, a + b[:1]) and f.conv_output_stats(z, 128) is None
    y.add_(1.0)
    assert f.conv_output_stats(y, 128) is None
