"""GPU parity at the exact shapes ``bench.py`` times: BASELINE.json configs 0, 1, 2a, 2b, 2c and 4.

Every test runs the same operator call the benchmark times, on the same shapes, and checks:

* the whole output volume against PyTorch's fp32 convolution on the CPU (the op the reference's
  tests compare against, ``tests/test_fast_fp32.py`` / ``tests/_torch.py``): max relative error
  ``max|y - ref| / max|ref|`` <= 1e-5 per layer (north-star FP32 bar), 1e-4 for a whole block or
  decoder window;
* every corner, edge and face of the output plus random interior voxels against the float64
  oracle (``oracle/reference_math.conv3d_points``), <= 1e-5;
* group-norm statistics over the configs' 8.4M-element groups against float64, <= 1e-6;
* the GEMM formulation the shape takes (``ctmr_conv3d_kernel``) and bit-identical repeats.

Method follows the reference's ``test_nax_conv_matches_float64`` (test_fast_fp32.py:59-88).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import maisi_torch as mt
from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
BLOCK_REL = 1e-4
GN_REL = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _cpu_threads():
    """The CPU references use the host's cores (at most 16, the GPU box's share)."""
    before = torch.get_num_threads()
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    yield
    torch.set_num_threads(before)


def _g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(t):
    return t.detach().cpu().numpy()


def _check(actual, expected, bound, what):
    assert np.isfinite(actual).all(), f"{what}: non-finite output"
    err = rm.max_rel_error(actual, expected)
    print(f"{what}: max rel error {err:.3e} (bound {bound:g})", flush=True)
    assert err <= bound, f"{what}: max rel error {err:.3e} > {bound:g}"


def _route(ctmr, x_shape, cout, *, stride=1, mode=0, flags=0, ksize=3):
    L = ctmr._lib
    desc = ctmr.ops.make_desc(tuple(x_shape), cout, ksize, stride, mode, flags, L.DT_F32, 0)
    return L.conv_kernel(desc), L.conv_split(desc), L.workspace_bytes(desc)


def _torch_conv_cpu(x_ndhwc, w, b, *, stride=1, padding=1, upsample=False):
    """PyTorch CPU fp32 conv3d of an NDHWC host array (channels-last 3d), NDHWC result."""
    t = torch.from_numpy(x_ndhwc).permute(0, 4, 1, 2, 3)  # a channels_last_3d view
    if upsample:
        t = F.interpolate(t, scale_factor=2, mode="nearest").contiguous(memory_format=torch.channels_last_3d)
    with torch.no_grad():
        y = F.conv3d(t, torch.from_numpy(w).contiguous(memory_format=torch.channels_last_3d),
                     torch.from_numpy(b), stride=stride, padding=padding)
    return y.permute(0, 2, 3, 4, 1).numpy()


def test_config0_conv_full_volume(ctmr, dev):
    """Config 0, bench.py's headline step: conv3d 64^3 x 64 -> 64, +bias, on the LDS-staged GEMM
    (one launch, no split, no workspace) -- both as the operator and as the two C-ABI stages the
    roofline line times."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(0)  # bench.py's draw order
    x = rng.standard_normal((1, 64, 64, 64, 64), dtype=np.float32)
    w = (rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    b = (0.01 * rng.standard_normal(64)).astype(np.float32)
    assert _route(ctmr, x.shape, 64) == ("lds", 1, 0)
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    y = f.conv3d(xg, wg, bg, padding=1)
    assert torch.equal(y, f.conv3d(xg, wg, bg, padding=1))
    import bench  # the roofline leg's two-stage call (ctmr_conv3d_pack + ctmr_conv3d_gemm)

    pack, gemm, keep = bench.staged_op(ctmr, xg, wg, bg, ctmr._lib.DT_F32)
    pack()
    gemm()
    torch.cuda.synchronize()
    assert torch.equal(keep[2], y)
    y = _h(y)
    pts = rm.boundary_points(1, (64, 64, 64), 4096, seed=0)
    _check(rm.gather_points(y, pts), rm.conv3d_points(x, w, b, pts), FP32_REL, "config0 points vs float64")
    _check(y, _torch_conv_cpu(x, w, b), FP32_REL, "config0 whole volume vs torch CPU fp32")


def test_config0_conv_full_volume_f16x2(ctmr, dev):
    """Config 0 under ``precision("f16x2")`` (the reference's exact mode: split fp16 on fp16 MFMA, the
    LDS-staged 16-bit GEMM over the packed hi/lo copy) -- the step bench.py reports as the split
    variant -- against PyTorch CPU fp32 and float64 points at the fp32 bar, and as the two C-ABI
    stages its roofline times."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 64, 64, 64, 64), dtype=np.float32)
    w = (rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    b = (0.01 * rng.standard_normal(64)).astype(np.float32)
    desc = ctmr.ops.make_desc(x.shape, 64, 3, 1, ctmr._lib.MODE_PLAIN, 0, ctmr._lib.DT_F16X2, 0)
    assert ctmr._lib.conv_kernel(desc) == "lds_f16x2" and ctmr._lib.conv_split(desc) == 1
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    with f.precision("f16x2"):
        y = f.conv3d(xg, wg, bg, padding=1)
        assert torch.equal(y, f.conv3d(xg, wg, bg, padding=1))
    import bench

    pack, gemm, keep = bench.staged_op(ctmr, xg, wg, bg, ctmr._lib.DT_F16X2)
    pack()
    gemm()
    torch.cuda.synchronize()
    assert torch.equal(keep[2], y)
    y = _h(y)
    pts = rm.boundary_points(1, (64, 64, 64), 4096, seed=0)
    _check(rm.gather_points(y, pts), rm.conv3d_points(x, w, b, pts), FP32_REL, "config0 f16x2 points vs float64")
    _check(y, _torch_conv_cpu(x, w, b), FP32_REL, "config0 f16x2 whole volume vs torch CPU fp32")


def test_config1_vae_resblock_full_size(ctmr, dev):
    """Config 1 at 128^3 x 128: GN(32) + SiLU + conv 128->128, twice, + identity skip (bench.py's
    ``vae_resblock`` call), checked per stage: the input's GN statistics (groups of 8.4M values)
    and those conv1's epilogue writes for norm2 against float64, conv1 and conv2 (+skip) on
    sampled voxels against float64, the whole block against PyTorch CPU fp32."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(1)  # bench.py's draw order for x, w1, w2, b1, b2
    c, s, groups, eps = 128, 128, 32, 1e-6
    x = rng.standard_normal((1, s, s, s, c), dtype=np.float32)
    mk = lambda: (rng.standard_normal((c, c, 3, 3, 3)) / np.sqrt(27 * c)).astype(np.float32)
    w1, w2 = mk(), mk()
    b1 = (0.01 * rng.standard_normal(c)).astype(np.float32)
    b2 = (0.01 * rng.standard_normal(c)).astype(np.float32)
    # non-trivial norm affines so a swapped scale/offset cannot pass
    g1, be1, g2, be2 = ((1 + 0.1 * rng.standard_normal(c)).astype(np.float32) if i % 2 == 0 else
                        (0.1 * rng.standard_normal(c)).astype(np.float32) for i in range(4))
    L = ctmr._lib
    assert _route(ctmr, x.shape, c, flags=L.F_AFFINE | L.F_SILU)[:2] == ("lds", 1)
    xg = _g(x, dev)
    t = lambda a: _g(a, dev)
    aff1 = _h(f.group_norm_affine(xg, t(g1), t(be1), groups=groups, eps=eps))
    ref_aff1 = rm.group_norm_affine(x, g1, be1, groups, eps)
    for k, name in ((0, "scale"), (1, "offset")):
        _check(aff1[..., k], ref_aff1[..., k], GN_REL, f"config1 GN1 {name} (8.4M-value groups)")
    shifted = _h(f.group_norm_affine(xg + 3.0, t(g1), t(be1), groups=groups, eps=eps))
    ref_shift = rm.group_norm_affine(x.astype(np.float64) + 3.0, g1, be1, groups, eps)
    for k, name in ((0, "scale"), (1, "offset")):
        _check(shifted[..., k], ref_shift[..., k], GN_REL, f"config1 GN1 {name}, mean 3")
    h1g = f.norm_conv3d(xg, t(w1), t(b1), norm=(t(g1), t(be1)), num_groups=groups, eps=eps, apply_silu=True,
                        out_gn_groups=groups)
    assert f.conv_output_stats(h1g, groups) is not None  # norm2's statistics come from the epilogue
    h1 = _h(h1g)
    pts = rm.boundary_points(1, (s, s, s), 2048, seed=1)
    _check(rm.gather_points(h1, pts), rm.conv3d_points(x, w1, b1, pts, affine=ref_aff1, apply_silu=True),
           FP32_REL, "config1 conv1 points vs float64")
    aff2 = _h(f.group_norm_affine(h1g, t(g2), t(be2), groups=groups, eps=eps))
    ref_aff2 = rm.group_norm_affine(h1, g2, be2, groups, eps)
    for k, name in ((0, "scale"), (1, "offset")):
        _check(aff2[..., k], ref_aff2[..., k], GN_REL, f"config1 GN2 {name} from conv1's epilogue")
    del h1g
    block = lambda: f.vae_resblock([xg], (t(w1), t(b1)), (t(w2), t(b2)), (t(g1), t(be1)), (t(g2), t(be2)), None,
                                   num_groups=groups, eps=eps)
    yg = block()
    assert torch.equal(yg, block())
    y = _h(yg)
    del yg
    conv2 = rm.conv3d_points(h1, w2, b2, pts, affine=ref_aff2, apply_silu=True) + rm.gather_points(x, pts)
    _check(rm.gather_points(y, pts), conv2, FP32_REL, "config1 conv2 + skip points vs float64")
    del h1
    with torch.no_grad():
        xc = torch.from_numpy(x).permute(0, 4, 1, 2, 3)
        hc = F.silu(F.group_norm(xc, groups, torch.from_numpy(g1), torch.from_numpy(be1), eps))
        hc = F.conv3d(hc.contiguous(memory_format=torch.channels_last_3d),
                      torch.from_numpy(w1).contiguous(memory_format=torch.channels_last_3d), torch.from_numpy(b1),
                      padding=1)
        hc = F.silu(F.group_norm(hc, groups, torch.from_numpy(g2), torch.from_numpy(be2), eps))
        hc = F.conv3d(hc.contiguous(memory_format=torch.channels_last_3d),
                      torch.from_numpy(w2).contiguous(memory_format=torch.channels_last_3d), torch.from_numpy(b2),
                      padding=1)
        ref = (xc + hc).permute(0, 2, 3, 4, 1).numpy()
    _check(y, ref, BLOCK_REL, "config1 block vs torch CPU fp32")


def test_config2a_stride2_full_size(ctmr, dev):
    """Config 2a: conv3d 3x3x3 stride 2, 64 -> 128, 128^3 -> 64^3 (bench.py's call)."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(21)
    x = rng.standard_normal((1, 128, 128, 128, 64), dtype=np.float32)
    w = (rng.standard_normal((128, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    b = (0.01 * rng.standard_normal(128)).astype(np.float32)
    assert _route(ctmr, x.shape, 128, stride=2)[:2] == ("stream_direct", 1)
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    yg = f.conv3d(xg, wg, bg, padding=1, stride=2)
    assert tuple(yg.shape) == (1, 64, 64, 64, 128)
    assert torch.equal(yg, f.conv3d(xg, wg, bg, padding=1, stride=2))
    y = _h(yg)
    pts = rm.boundary_points(1, (64, 64, 64), 2048, seed=2)
    _check(rm.gather_points(y, pts), rm.conv3d_points(x, w, b, pts, stride=2), FP32_REL, "config2a points vs float64")
    _check(y, _torch_conv_cpu(x, w, b, stride=2), FP32_REL, "config2a whole volume vs torch CPU fp32")


def test_config2b_nearest_up_full_size(ctmr, dev):
    """Config 2b: nearest-2x upsampling + conv3d 256 -> 128, 64^3 -> 128^3, as the parity-folded
    8-tap GEMM (bench.py's call), against the conv of the materialized upsampling."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(22)
    x = rng.standard_normal((1, 64, 64, 64, 256), dtype=np.float32)
    w = (rng.standard_normal((128, 256, 3, 3, 3)) / np.sqrt(27 * 256)).astype(np.float32)
    b = (0.01 * rng.standard_normal(128)).astype(np.float32)
    assert _route(ctmr, x.shape, 128, mode=ctmr._lib.MODE_NEAREST2X)[:2] == ("stream", 1)
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    run = lambda: f.norm_conv3d(xg, wg, bg, norm=None, num_groups=1, eps=1e-6, apply_silu=False, upsample=True)
    yg = run()
    assert tuple(yg.shape) == (1, 128, 128, 128, 128)
    assert torch.equal(yg, run())
    y = _h(yg)
    del yg
    pts = rm.boundary_points(1, (128, 128, 128), 2048, seed=3)
    _check(rm.gather_points(y, pts), rm.conv3d_points(x, w, b, pts, upsample=True), FP32_REL,
           "config2b points vs float64")
    _check(y, _torch_conv_cpu(x, w, b, upsample=True), FP32_REL, "config2b whole volume vs torch CPU fp32")


def test_config2c_pointwise_full_volume(ctmr, dev):
    """Config 2c: 1x1x1 conv 128 -> 256 at 64^3 on the persistent pointwise GEMM, every output
    against a float64 matmul."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(23)
    x = rng.standard_normal((1, 64, 64, 64, 128), dtype=np.float32)
    w = (rng.standard_normal((256, 128, 1, 1, 1)) / np.sqrt(128)).astype(np.float32)
    b = (0.01 * rng.standard_normal(256)).astype(np.float32)
    assert _route(ctmr, x.shape, 256, ksize=1) == ("pointwise", 1, 0)
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    yg = f.pointwise_conv(xg, wg, bg)
    assert torch.equal(yg, f.pointwise_conv(xg, wg, bg))
    ref = x.reshape(-1, 128).astype(np.float64) @ w[:, :, 0, 0, 0].T.astype(np.float64) + b
    _check(_h(yg).reshape(-1, 256), ref, FP32_REL, "config2c whole volume vs float64")


def _decoder(ctmr, dev):
    m = ctmr.maisi
    ctor = m.PRODUCTION_VAE_CONSTRUCTOR
    host = m.random_weights(m.vae_decoder_weight_shapes(ctor), seed=11)  # bench.py's seed
    return ctor, host, {k: _g(v, dev) for k, v in host.items()}


BF16_REL = 2e-2  # north-star per-layer bar of the bf16-in / fp32-accumulate variant


@pytest.fixture(scope="module")
def cpu_window(ctmr):
    """bench.py's first config-4 window (latent 20x64x64x4) and its PyTorch CPU fp32 decode (NDHWC),
    computed once for the fp32 and bf16 window checks."""
    m = ctmr.maisi
    ctor = m.PRODUCTION_VAE_CONSTRUCTOR
    host = m.random_weights(m.vae_decoder_weight_shapes(ctor), seed=11)  # bench.py's seed
    z = np.random.default_rng(4).standard_normal((1, 64, 64, 64, 4), dtype=np.float32)  # bench.py's latent
    window = np.ascontiguousarray(z[:, 0:20])
    with torch.no_grad():
        _, ref = mt.vae_decode(torch.from_numpy(np.moveaxis(window, -1, 1).copy()),
                               mt.to_torch(host, dtype=torch.float32, strip=""), ctor)
    return window, np.moveaxis(ref.numpy(), 1, -1)


def test_config4_full_window_matches_cpu_oracle(ctmr, dev, cpu_window):
    """One full config-4 window (latent 20x64x64x4 -> 80x256x256, production decoder, random init):
    the top level convolves 5.2M voxels x 64 channels and normalizes groups of 10.5M values.  The
    window bench.py decodes first, against the PyTorch CPU fp32 decoder, <= 1e-4."""
    m = ctmr.maisi
    ctor, _, w = _decoder(ctmr, dev)
    window, ref = cpu_window
    post, y = m.decode_vae(_g(window, dev), w, constructor=ctor)
    assert tuple(y.shape) == (1, 80, 256, 256, 1)
    y = _h(y)
    del post
    _check(y, ref, BLOCK_REL, "config4 window vs torch CPU fp32 decoder")


def test_config4_full_window_bf16_matches_cpu_oracle(ctmr, dev, cpu_window):
    """The same window decoded under ``precision("bf16")`` -- the variant bench.py times as
    ``config4 ... bf16_s`` (3x3x3 convs on bf16 MFMA with fp32 accumulation, the LDS-staged bf16
    GEMM, its nearest/trilinear packs) -- against the PyTorch CPU fp32 decoder, <= 2e-2, and
    bit-identical run to run."""
    m, f = ctmr.maisi, ctmr.fast_fp32
    ctor, _, w = _decoder(ctmr, dev)
    window, ref = cpu_window
    with f.precision("bf16"):
        _, y = m.decode_vae(_g(window, dev), w, constructor=ctor)
        _, y2 = m.decode_vae(_g(window, dev), w, constructor=ctor)
    assert tuple(y.shape) == (1, 80, 256, 256, 1)
    assert torch.equal(y, y2)
    _check(_h(y), ref, BF16_REL, "config4 window bf16 vs torch CPU fp32 decoder")


def test_config4_full_window_f16x2_matches_cpu_oracle(ctmr, dev, cpu_window):
    """The window under ``precision("f16x2")`` against the PyTorch CPU fp32 decoder at the fp32 bar,
    1e-4 (the decoder's 3x3x3 convs with 64 or more output channels on the split-fp16 GEMM, the
    64 -> 1 output conv and the 1x1 shortcuts on FP32)."""
    m, f = ctmr.maisi, ctmr.fast_fp32
    ctor, _, w = _decoder(ctmr, dev)
    window, ref = cpu_window
    with f.precision("f16x2"):
        _, y = m.decode_vae(_g(window, dev), w, constructor=ctor)
    _check(_h(y), ref, BLOCK_REL, "config4 window f16x2 vs torch CPU fp32 decoder")


def _check_256_decode(ctmr, dev, tag):
    """bench.py's config-4 decode under the active precision: finite; equal, at every voxel, to the
    float64 Gaussian blend of the four windows decoded separately; int16 = truncation, in range."""
    m = ctmr.maisi
    ctor, _, w = _decoder(ctmr, dev)
    z = np.random.default_rng(4).standard_normal((1, 64, 64, 64, 4), dtype=np.float32)
    zg = _g(z, dev)
    roi = (20, 64, 64)
    y = m.sliding_window_decode(zg, w, constructor=ctor, roi=roi, overlap=0.25, scale_factor=1.0)
    assert tuple(y.shape) == (1, 256, 256, 256, 1)
    img = _h(torch.clamp(y * 1000.0, min=0.0).to(torch.int16))
    y = _h(y)
    assert np.isfinite(y).all()
    windows = m.dense_patch_slices((64, 64, 64), roi, m.scan_interval((64, 64, 64), roi, 0.25))
    starts = [sd.start for sd, _, _ in windows]
    assert starts == [0, 15, 30, 44]
    gw = np.asarray(_h(m.gaussian_importance(roi, 0.125)), np.float64)
    gw = gw.repeat(4, 0).repeat(4, 1).repeat(4, 2)
    num = np.zeros((256, 256, 256), np.float64)
    den = np.zeros((256, 256, 256), np.float64)
    for a in starts:
        pred = _h(m.decode_vae(_g(np.ascontiguousarray(z[:, a:a + 20]), dev), w, constructor=ctor)[1])
        num[4 * a:4 * a + 80] += pred[0, ..., 0].astype(np.float64) * gw
        den[4 * a:4 * a + 80] += gw
    blend = num / den
    _check(y[0, ..., 0], blend, GN_REL, f"config4 256^3 {tag} decode vs float64 blend of its windows")
    for a in starts[1:]:  # the rows either side of each window start
        seam = slice(4 * a - 2, 4 * a + 2)
        _check(y[0, seam, ..., 0], blend[seam], GN_REL, f"config4 {tag} seam at depth {4 * a}")
    scaled = np.maximum(y.astype(np.float64) * 1000.0, 0.0)
    assert scaled.max() < 32767.0, f"MR-scaled intensities overflow int16: max {scaled.max():.1f}"
    np.testing.assert_array_equal(img, np.trunc(np.maximum(y * np.float32(1000.0), 0)).astype(np.int16))
    ct = m.output_intensities(y, configuration="ct")
    assert ct.dtype == np.int16 and ct.min() >= -1000 and ct.max() <= 1000


def test_config4_256_decode_blend_and_int16(ctmr, dev):
    """bench.py's config-4 decode (64^3 latent, roi 20x64x64, overlap 0.25 -> 4 windows along D,
    256^3 output, int16): finite; equal, at every voxel, to the Gaussian blend of the four windows
    decoded separately recomputed in float64 (so continuous across each seam); the int16 image
    is the truncation of max(1000 x, 0) with no value outside the int16 range."""
    _check_256_decode(ctmr, dev, "fp32")


def test_config4_256_decode_f16x2_blend_and_int16(ctmr, dev):
    """The split-fp16 variant of the same 256^3 decode: blend, seam and int16 checks."""
    with ctmr.fast_fp32.precision("f16x2"):
        _check_256_decode(ctmr, dev, "f16x2")


def test_config4_256_decode_bf16_blend_and_int16(ctmr, dev):
    """The bf16 variant of the same 256^3 decode (the one bench.py times as ``bf16_s``): the same
    blend, seam and int16 checks, with every window decoded under ``precision("bf16")`` (each
    window itself is checked against the fp32 CPU decoder, <= 2e-2, above)."""
    with ctmr.fast_fp32.precision("bf16"):
        _check_256_decode(ctmr, dev, "bf16")


def test_outputs_beyond_2gib(ctmr, dev):
    """A conv whose output exceeds 2 GiB (1x80x256x256x64 -> 128 channels: 2.68 GB) on the fp32 LDS-staged
    GEMM, the fp32 streaming GEMM and the bf16 LDS-staged GEMM. Their epilogues store through buffer
    descriptors based at each brick's first output plane (LDS GEMMs) or each wave's first output row
    (streaming GEMM), so byte offsets stay within 32 bits; checked on every corner, edge and face of the
    volume (its last planes, 2.6 GB past the start, included) and interior voxels against float64."""
    f, L = ctmr.fast_fp32, ctmr._lib
    rng = np.random.default_rng(5)
    shape, cout = (1, 80, 256, 256, 64), 128
    x = rng.standard_normal(shape, dtype=np.float32)
    w = (rng.standard_normal((cout, shape[-1], 3, 3, 3)) / np.sqrt(27 * shape[-1])).astype(np.float32)
    b = (0.01 * rng.standard_normal(cout)).astype(np.float32)
    assert np.prod(shape[:-1]) * cout * 4 > 2**31
    pts = rm.boundary_points(1, shape[1:4], 1024, seed=5)
    expected = rm.conv3d_points(x, w, b, pts)
    xg, wg, bg = _g(x, dev), _g(w, dev), _g(b, dev)
    idx = tuple(torch.from_numpy(pts[:, a]).to(dev) for a in range(4))
    for name, dtype, stream, route, bound in (("fp32 LDS GEMM", "fp32", False, "lds", FP32_REL),
                                              ("fp32 streaming GEMM", "fp32", True, "stream", FP32_REL),
                                              ("bf16 LDS GEMM", "bf16", False, "lds_bf16", 2e-2)):
        desc = ctmr.ops.make_desc(shape, cout, 3, 1, L.MODE_PLAIN, L.F_STREAM if stream else 0,
                                  L.DT_BF16 if dtype == "bf16" else L.DT_F32, 0)
        assert L.conv_kernel(desc) in (route, route + "_direct"), (name, L.conv_kernel(desc))
        print(f"case {name}: route {L.conv_kernel(desc)}", flush=True)
        y = f.implicit_gemm_conv3d(xg, f.pack_weight(wg, dtype=dtype), bg, cout=cout, stream_gemm=stream)
        got = _h(y[idx])
        del y
        torch.cuda.empty_cache()
        _check(got, expected, bound, f"{name}, output beyond 2 GiB, points vs float64")


@pytest.mark.parametrize(("name", "shape", "cout", "mode", "dtype", "route", "bound"), [
    ("fp32 LDS GEMM, 4 planes of 256x256x1984", (1, 8, 256, 256, 64), 1984, "plain", "fp32", "lds", FP32_REL),
    ("bf16 nearest-2x LDS GEMM, 8 planes of 256x256x960", (1, 8, 128, 128, 64), 960, "nearest", "bf16", "lds_bf16",
     2e-2),
])
def test_brick_output_span_near_2gib(ctmr, dev, name, shape, cout, mode, dtype, route, bound):
    """Brick epilogues store at 32-bit byte offsets from the brick's first output plane, and the library
    keeps a brick route only while a brick's output planes (4; 8 for the nearest-2x phases) span under
    2 GiB. Here that span is 1.94-1.88 GiB (outputs 4.2 / 4.0 GB): the far corners of each brick, the
    last channel of the volume's last voxel among them, against float64."""
    f, L = ctmr.fast_fp32, ctmr._lib
    rng = np.random.default_rng(11)
    n, d, h, w, c = shape
    up = mode == "nearest"
    s = 2 if up else 1
    span = 4 * s * (s * h) * (s * w) * cout * 4
    assert 0.9 * 2**31 < span < 2**31, span
    x = rng.standard_normal(shape, dtype=np.float32)
    wt = (rng.standard_normal((cout, c, 3, 3, 3)) / np.sqrt(27 * c)).astype(np.float32)
    b = (0.01 * rng.standard_normal(cout)).astype(np.float32)
    out_sp = (s * d, s * h, s * w)
    pts = rm.boundary_points(1, out_sp, 512, seed=11)
    last = np.array([[0, s * d - 1 - dz, s * h - 1, s * w - 1] for dz in range(4 * s)])  # a brick's far corners
    pts = np.concatenate([pts, last])
    expected = rm.conv3d_points(x, wt, b, pts, upsample=up)
    m = L.MODE_NEAREST2X if up else L.MODE_PLAIN
    desc = ctmr.ops.make_desc(shape, cout, 3, 1, m, 0, L.DT_BF16 if dtype == "bf16" else L.DT_F32, 0)
    assert L.conv_kernel(desc) == route, (name, L.conv_kernel(desc))
    print(f"case {name}: route {route}, brick span {span / 2**30:.3f} GiB", flush=True)
    packed = (f.pack_upsample_weight if up else f.pack_weight)(_g(wt, dev), dtype=dtype)
    y = f.implicit_gemm_conv3d(_g(x, dev), packed, _g(b, dev), cout=cout, upsample=up)
    idx = tuple(torch.from_numpy(pts[:, a]).to(dev) for a in range(4))
    got = _h(y[idx])
    del y
    torch.cuda.empty_cache()
    _check(got, expected, bound, f"{name}, points vs float64")
