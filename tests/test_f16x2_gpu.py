"""GPU parity of the split-fp16 convolution (``CTMR_F16X2``, ``precision("f16x2")``): the reference's
"exact" mode for fp32 tensors (``_nax_conv.py:27-35``) on fp16 MFMA.

Bars: the reference's own kernel-test tolerance ``max|y - ref| <= 2e-6 * max|ref|`` against float64
(``tests/test_fast_fp32.py:16-18``) at every route of the split GEMM (plain, nearest-2x parity fold,
trilinear-2x, GN affine + SiLU staging, per-batch bias and residual, K splits, two-tensor inputs,
inputs far from unit scale); bitwise repeat runs; the packed operands checked against the split's
definition (hi + lo reproduces the fp32 value to 2^-22, halos and pad channels zero); shapes the
split GEMM does not take run the FP32 GEMM bit for bit.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

REF_REL = 2e-6


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _assert_rel(actual, expected, bound, what):
    expected = np.asarray(expected, np.float64)
    actual = np.asarray(actual, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.isfinite(actual).all(), f"{what}: non-finite output"
    err = rm.max_rel_error(actual, expected)
    print(f"{what}: max rel error {err:.3e} (bound {bound:g})", flush=True)
    assert err <= bound, f"{what}: max rel error {err:.3e} > {bound:g}"


# name, NDHWC input shape, cout, options
CASES = [
    ("plain_64", (2, 8, 16, 16, 64), 64, {}),
    ("plain_ragged", (1, 7, 12, 13, 48), 64, {}),
    ("norm_silu_batchbias_residual", (2, 4, 8, 8, 64), 128, {"norm": True, "batch_bias": True, "residual": True}),
    ("deep_split_512", (2, 8, 8, 4, 512), 512, {}),
    ("forced_split_3", (1, 8, 8, 8, 96), 64, {"split": 3}),
    ("nearest2x", (2, 4, 8, 8, 64), 64, {"upsample": True}),
    ("nearest2x_norm_residual", (1, 4, 4, 8, 128), 64, {"upsample": True, "norm": True, "residual": True}),
    ("trilinear2x", (1, 4, 6, 8, 32), 64, {"trilinear": True}),
    ("cat_two_tensors", (2, 4, 8, 8, 64), 64, {"cat": 32, "norm": True}),
    ("small_inputs_1e-3", (1, 4, 8, 8, 64), 64, {"scale": 1e-3}),
    ("large_inputs_1e3", (1, 4, 8, 8, 64), 64, {"scale": 1e3}),
]


def _case_inputs(shape, cout, opts, seed):
    rng = np.random.default_rng(seed)
    n, d, h, w, c = shape
    x = (opts.get("scale", 1.0) * rng.standard_normal(shape)).astype(np.float32)
    wt = (rng.standard_normal((cout, c, 3, 3, 3)) / np.sqrt(27 * c)).astype(np.float32)
    b = rng.standard_normal((n, cout) if opts.get("batch_bias") else cout).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(c)).astype(np.float32)
    s = 2 if (opts.get("upsample") or opts.get("trilinear")) else 1
    res = rng.standard_normal((n, s * d, s * h, s * w, cout)).astype(np.float32) if opts.get("residual") else None
    return x, wt, b, gamma, beta, res


def _expected(x, wt, b, gamma, beta, res, opts, groups):
    src = rm.group_norm(x, gamma, beta, groups, 1e-6, apply_silu=True) if opts.get("norm") else x
    if opts.get("upsample"):
        src = rm.upsample_nearest(src)
    if opts.get("trilinear"):
        src = rm.upsample_trilinear(src)
    bias = b if b.ndim == 1 else None
    y = rm.conv3d(src, wt, bias)
    if b.ndim == 2:
        y = y + b[:, None, None, None, :].astype(np.float64)
    if res is not None:
        y = y + res
    return y


def _run(ctmr, dev, x, wt, b, gamma, beta, res, opts, groups):
    f = ctmr.fast_fp32
    xg, wg, bg = _t(x, dev), _t(wt, dev), _t(b, dev)
    rg = None if res is None else _t(res, dev)
    if opts.get("cat"):
        c1 = opts["cat"]
        xg = f.ChannelCat(xg[..., :c1].contiguous(), xg[..., c1:].contiguous())
    if opts.get("trilinear"):
        packed = f.pack_weight(wg, dtype="f16x2")
        return f.implicit_gemm_conv3d(xg, packed, bg, cout=int(wt.shape[0]), trilinear=True)
    if opts.get("split"):
        affine = f.group_norm_affine(xg, _t(gamma, dev), _t(beta, dev), groups=groups, eps=1e-6) \
            if opts.get("norm") else None
        packed = f.pack_weight(wg, dtype="f16x2")
        return f.implicit_gemm_conv3d(xg, packed, bg, cout=int(wt.shape[0]), affine=affine,
                                      silu=bool(opts.get("norm")), residual=rg, split=opts["split"])
    norm = (_t(gamma, dev), _t(beta, dev)) if opts.get("norm") else None
    return f.norm_conv3d(xg, wg, bg, norm=norm, num_groups=groups, eps=1e-6, apply_silu=bool(opts.get("norm")),
                         upsample=bool(opts.get("upsample")), residual=rg)


@pytest.mark.parametrize(("name", "shape", "cout", "opts"), CASES, ids=[c[0] for c in CASES])
def test_f16x2_matches_float64(ctmr, dev, name, shape, cout, opts):
    """Every route option of the split-fp16 GEMM against float64 at the reference's 2e-6 bar; the
    route is the split GEMM; repeat runs are bit-identical."""
    L, f = ctmr._lib, ctmr.fast_fp32
    groups = 8
    x, wt, b, gamma, beta, res = _case_inputs(shape, cout, opts, seed=sum(map(ord, name)))
    mode = L.MODE_NEAREST2X if opts.get("upsample") else (L.MODE_TRILINEAR2X if opts.get("trilinear")
                                                          else L.MODE_PLAIN)
    c2 = shape[-1] - opts["cat"] if opts.get("cat") else 0
    xs = (*shape[:-1], shape[-1] - c2)
    desc = ctmr.ops.make_desc(xs, cout, 3, 1, mode, 0, L.DT_F16X2, opts.get("split", 0), c2)
    route = L.conv_kernel(desc)
    print(f"f16x2 case {name}: {shape}->{cout} route {route} split {L.conv_split(desc)}", flush=True)
    assert route == "lds_f16x2"
    with f.precision("f16x2"):
        y = _run(ctmr, dev, x, wt, b, gamma, beta, res, opts, groups)
        y2 = _run(ctmr, dev, x, wt, b, gamma, beta, res, opts, groups)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), f"{name}: repeat run differs"
    _assert_rel(_h(y), _expected(x, wt, b, gamma, beta, res, opts, groups), REF_REL, f"f16x2 {name}")


def test_f16x2_epilogue_group_norm_statistics(ctmr, dev):
    """The split GEMM's epilogue statistics (``gn_groups``) give the output's group-norm affine to
    float64 precision, as the fp32 GEMMs' do."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(81)
    x = rng.standard_normal((2, 8, 8, 16, 64)).astype(np.float32)
    wt = (rng.standard_normal((128, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(128)).astype(np.float32)
    with f.precision("f16x2"):
        y = f.conv3d(_t(x, dev), _t(wt, dev), _t(b, dev), padding=1, gn_groups=32)
    assert f.conv_output_stats(y, 32) is not None
    aff = _h(f.group_norm_affine(y, _t(gamma, dev), _t(beta, dev), groups=32, eps=1e-6))
    ref = rm.group_norm_affine(_h(y), gamma, beta, 32, 1e-6)
    _assert_rel(aff, ref, 1e-6, "f16x2 epilogue GN affine")


@pytest.mark.parametrize("mode", ["plain", "nearest"])
def test_f16x2_packed_weight_is_the_split_of_the_scaled_weight(ctmr, dev, mode):
    """Packed split weights, read back: per (phase, tap, 16-channel block, column) hi, hi * 2^-11 and lo
    of the column-scaled weight w * 2^k, 2^-k the column's power-of-two scale (largest scaled
    magnitude in [2^14, 2^15)); hi + lo equals the scaled (folded, for nearest-2x) weight to 2^-22
    relative; pad channels are zero."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(82)
    cin, cout = 40, 64
    col_scale = np.geomspace(1e-3, 2.0, cout)[:, None, None, None, None]
    wt = (rng.standard_normal((cout, cin, 3, 3, 3)) * col_scale).astype(np.float32)
    wg = _t(wt, dev)
    if mode == "nearest":
        packed = f.pack_upsample_weight(wg, dtype="f16x2")
        folded = rm.fold_upsample_weight(wt)  # (8, O, C, 2, 2, 2), float64
        want = folded.reshape(8, cout, cin, 8).transpose(0, 3, 2, 1)  # (phase, tap, cin, cout)
        phases, taps, bound = 8, 8, 2.0 ** -20  # the kernel folds in fp32
    else:
        packed = f.pack_weight(wg, dtype="f16x2")
        want = wt.astype(np.float64).reshape(cout, cin, 27).transpose(2, 1, 0)[None]
        phases, taps, bound = 1, 27, 2.0 ** -21
    kb, npc = 3, 64
    raw = packed.view(torch.int16).cpu().numpy().view(np.uint16)
    nblk = phases * taps * kb * npc * 48
    assert raw.size == nblk + 2 * npc
    halves = raw[:nblk].view(np.float16).astype(np.float64).reshape(phases, taps, kb, npc, 3, 16)
    scale = raw[nblk:].view(np.float32).astype(np.float64)
    k = -np.log2(scale)
    assert np.all(k == np.round(k)), "column scales are powers of two"
    hi, hi_s, lo = halves[..., 0, :], halves[..., 1, :], halves[..., 2, :]
    # hi * 2^-11 is exact where it is a normal fp16 (|hi| >= 2^-3); below, within half a subnormal step
    normal = np.abs(hi) >= 2.0 ** -3
    np.testing.assert_array_equal(hi_s[normal], hi[normal] * 2.0 ** -11)
    assert np.all(np.abs(hi_s - hi * 2.0 ** -11)[~normal] <= 2.0 ** -25)
    full = (hi + lo).transpose(0, 1, 2, 4, 3).reshape(phases, taps, kb * 16, npc)
    assert np.all(full[:, :, cin:] == 0), "pad channels are zero"
    ws = full[:, :, :cin, :cout]
    colmax = np.abs(ws).reshape(-1, cout).max(axis=0)
    assert np.all((colmax >= 2.0 ** 14) & (colmax < 2.0 ** 15))
    scaled = want / scale[None, None, None, :cout]
    err = np.abs(ws - scaled).max(axis=(0, 1, 2)) / np.abs(scaled).max(axis=(0, 1, 2))
    print(f"packed weight {mode}: hi + lo vs scaled weight, worst column rel {err.max():.3e}", flush=True)
    assert err.max() <= bound


def test_f16x2_packed_input_is_the_split_of_the_transformed_input(ctmr, dev):
    """``ctmr_conv3d_pack`` with ``CTMR_F16X2``: per padded voxel and 16-channel block [hi | lo], hi +
    lo * 2^-11 equals GN affine + SiLU of x to 2^-22 relative; halo voxels and pad channels are zero
    bit for bit."""
    L, ops = ctmr._lib, ctmr.ops
    rng = np.random.default_rng(83)
    n, d, h, w, c = 1, 4, 8, 5, 40  # bricks half full: the split route
    x = rng.standard_normal((n, d, h, w, c)).astype(np.float32)
    aff = np.stack([1 + 0.2 * rng.standard_normal((n, c)), 0.3 * rng.standard_normal((n, c))], -1).astype(np.float32)
    desc = ops.make_desc((n, d, h, w, c), 64, 3, 1, L.MODE_PLAIN, L.F_AFFINE | L.F_SILU, L.DT_F16X2, 0)
    ws_bytes = L.workspace_bytes(desc)
    cp = 48
    assert ws_bytes >= n * (d + 2) * (h + 2) * (w + 2) * cp * 4
    xg, ag = _t(x, dev), _t(aff, dev)
    ws = torch.full((ws_bytes // 2,), 7, dtype=torch.int16, device=dev)
    rc = L.lib().ctmr_conv3d_pack(ctypes.byref(desc), xg.data_ptr(), ag.data_ptr(), ws.data_ptr(), ws_bytes,
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == L.OK, L.last_error()
    torch.cuda.synchronize()
    raw = ws.cpu().numpy().view(np.uint16)[: n * (d + 2) * (h + 2) * (w + 2) * cp * 2]
    blocks = raw.view(np.float16).astype(np.float64).reshape(n, d + 2, h + 2, w + 2, cp // 16, 2, 16)
    val = blocks[..., 0, :] + blocks[..., 1, :] * 2.0 ** -11  # (..., block, channel)
    val = val.reshape(n, d + 2, h + 2, w + 2, cp)
    t = x.astype(np.float64) * aff[:, None, None, None, :, 0] + aff[:, None, None, None, :, 1]
    want = t / (1 + np.exp(-t))
    inner = val[:, 1:-1, 1:-1, 1:-1, :c]
    err = np.abs(inner - want).max() / np.abs(want).max()
    print(f"packed input: hi + lo vs GN+SiLU(x) rel {err:.3e}", flush=True)
    assert err <= 4e-7  # 2^-22 split, plus the SiLU's 1e-6-relative evaluation rounded into hi
    halo = np.ones((d + 2, h + 2, w + 2), bool)
    halo[1:-1, 1:-1, 1:-1] = False
    vox = raw.reshape(n, d + 2, h + 2, w + 2, cp * 2)
    assert np.all(vox[:, halo] == 0), "halo voxels must be +0 bit for bit"
    padc = blocks[:, 1:-1, 1:-1, 1:-1, 2, :, 8:]  # block 2 holds channels 32..47: 40..47 are padding
    assert np.all(padc == 0)


def test_f16x2_falls_back_to_fp32_where_the_split_gemm_does_not_apply(ctmr, dev):
    """Under ``precision("f16x2")``, convs the split GEMM does not take (stride 2, cout not a multiple
    of 64, 1x1x1, 4 input channels) run the FP32 GEMMs: bit-identical to ``precision("fp32")``."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(84)
    cases = [((1, 8, 8, 8, 64), 64, 3, 2), ((1, 4, 8, 8, 64), 48, 3, 1), ((1, 4, 8, 8, 64), 128, 1, 1),
             ((2, 8, 8, 8, 4), 64, 3, 1)]
    for shape, cout, k, stride in cases:
        x = _t(rng.standard_normal(shape).astype(np.float32), dev)
        wt = _t((rng.standard_normal((cout, shape[-1], k, k, k)) / np.sqrt(k ** 3 * shape[-1])).astype(np.float32), dev)
        b = _t(rng.standard_normal(cout).astype(np.float32), dev)
        with f.precision("f16x2"):
            y = f.conv3d(x, wt, b, padding=k // 2, stride=stride)
        y32 = f.conv3d(x, wt, b, padding=k // 2, stride=stride)
        assert torch.equal(y, y32), (shape, cout, k, stride)


def test_f16x2_rejects_unsupported_descriptors(ctmr):
    """The C ABI refuses CTMR_F16X2 where the split GEMM cannot run, before any launch."""
    L, ops = ctmr._lib, ctmr.ops
    for shape, cout, k, stride in [((1, 8, 8, 8, 64), 64, 3, 2), ((1, 8, 8, 8, 64), 48, 3, 1),
                                   ((1, 8, 8, 8, 64), 64, 1, 1), ((1, 2, 2, 2, 64), 64, 3, 1)]:
        desc = ops.make_desc(shape, cout, k, stride, L.MODE_PLAIN, 0, L.DT_F16X2, 0)
        assert L.lib().ctmr_conv3d_kernel(ctypes.byref(desc)) == L.E_UNSUPPORTED
