"""The arithmetic-module surface (CPU): fast_fp32 provides every method of the reference's
arithmetic protocols with the same parameter names, so it can be returned from
``unet_arithmetic()`` / ``vae_arithmetic()`` (reference _types.py:216-286, fast_fp32.py:30-68)."""

from __future__ import annotations

import inspect

import pytest
import torch

# protocol method -> keyword parameters the reference's callers pass by name
PROTOCOLS = {
    "MlpArithmetic": {"linear": ["mx"], "silu": ["mx"]},
    "ConvArithmetic": {
        "silu": ["mx"],
        "group_norm_ncdhw": ["num_groups", "eps", "mx"],
        "conv3d_ncdhw": ["padding", "mx", "stride"],
    },
    "VaeArithmetic": {"upsample_trilinear_ncdhw": ["mx", "scale"]},
    "ResidualArithmetic": {"avg_pool3d_ncdhw": ["mx"], "upsample_nearest_ncdhw": ["mx"]},
    "AttentionArithmetic": {"attention_projection": ["mx"], "attention": ["scale", "mx"]},
    "UnetArithmetic": {"sinusoidal_timestep_embedding": ["mx", "max_period"]},
}
# other module-level names the reference's networks use from fast_fp32 (fast_fp32.py:30-68, 102-406)
EXTRA = ["norm_conv3d_ncdhw", "pointwise_conv_ncdhw", "residual_block_ncdhw", "vae_resblock_ncdhw",
         "trilinear_conv3d_ncdhw", "self_attention_tokens", "flash_attention", "flash_eligible",
         "pack_weight", "pack_upsample_weight", "drop_packed_weights", "group_norm_affine", "nax_conv3d",
         "nax_available"]


@pytest.mark.parametrize("protocol", sorted(PROTOCOLS))
def test_fast_fp32_satisfies_reference_protocols(ctmr, protocol):
    ff = ctmr.fast_fp32
    for name, keywords in PROTOCOLS[protocol].items():
        fn = getattr(ff, name, None)
        assert callable(fn), f"{protocol}.{name} missing"
        params = inspect.signature(fn).parameters
        for kw in keywords:
            assert kw in params, f"{protocol}.{name} lacks keyword {kw!r}"


def test_fast_fp32_exports_reference_names(ctmr):
    missing = [n for n in EXTRA if not callable(getattr(ctmr.fast_fp32, n, None))]
    assert not missing, missing


def test_operators_reject_cpu_tensors_without_fallback(ctmr):
    import torch

    x = torch.zeros(1, 4, 4, 4, 4)
    w = torch.zeros(4, 4, 3, 3, 3)
    with pytest.raises(ValueError, match="GPU"):
        ctmr.fast_fp32.conv3d_ncdhw(x, w, None, padding=1)
    with pytest.raises(ValueError, match="GPU"):
        ctmr.fast_fp32.flash_attention(torch.zeros(1, 8, 32), torch.zeros(1, 8, 32), torch.zeros(1, 8, 32),
                                       heads=1, scale=1.0)


def test_unet_graph_rejects_cpu_inputs(ctmr):
    import torch

    with pytest.raises(ValueError, match="CUDA"):
        ctmr.maisi.UNetGraph(torch.zeros(1, 4, 4, 4, 4), torch.zeros(1), None, None, {}, constructor={})


def test_output_intensities_default_and_configurations(ctmr):
    """image.py:68-87: the default configuration is CT; MR and MR-Brain share ``max(1000 x, 0)``
    with no upper clip; any other name raises (the reference's InvalidInputError)."""
    import numpy as np

    m = ctmr.maisi
    x = np.array([-0.2, 0.0, 0.25, 0.5004, 1.7], np.float32)
    np.testing.assert_array_equal(m.output_intensities(x), [-1000, -1000, -500, 0, 1000])
    np.testing.assert_array_equal(m.output_intensities(x, configuration="ct"), m.output_intensities(x))
    for name in ("mr", "mr-brain"):
        np.testing.assert_array_equal(m.output_intensities(x, configuration=name), [0, 0, 250, 500, 1700])
    for bad in ("CT", "mri", "", None):
        with pytest.raises(ValueError, match="configuration must be"):
            m.output_intensities(x, configuration=bad)
    with pytest.raises(ValueError, match="finite"):
        m.output_intensities(np.array([np.nan], np.float32))


@pytest.mark.parametrize(("kw", "message"), [
    ({"roi": (4, 4)}, "roi must be three"),
    ({"roi": (4, 0, 4)}, "roi must be three"),
    ({"overlap": 1.0}, "overlap must be"),
    ({"overlap": -0.1}, "overlap must be"),
    ({"mode": "constant"}, "mode"),
    ({"z_scale": 2}, "z_scale"),
])
def test_sliding_window_argument_validation(ctmr, kw, message):
    """decode.py:132-146, 336-351: window arguments are checked before any window is decoded."""
    import torch

    args = {"roi": (4, 4, 4), "overlap": 0.25}
    args.update(kw)
    called = []
    with pytest.raises(ValueError, match=message):
        ctmr.maisi.sliding_window(torch.zeros(1, 8, 8, 8, 4), lambda t: called.append(t), **args)
    assert not called


def test_window_helpers_validate(ctmr):
    m = ctmr.maisi
    with pytest.raises(ValueError, match="overlap"):
        m.scan_interval((8, 8, 8), (4, 4, 4), 1.5)
    with pytest.raises(ValueError, match="image_size"):
        m.scan_interval((8, 8), (4, 4, 4), 0.5)
    with pytest.raises(ValueError, match="interval"):
        m.dense_patch_slices((8, 8, 8), (4, 4, 4), (0, 1, 1))
    with pytest.raises(ValueError, match="sigma_scale"):
        m.gaussian_importance((4, 4, 4), 0.0)
    with pytest.raises(ValueError, match="roi"):
        m.sliding_window_decode(None, {}, constructor={}, roi=(1, 2))
    assert m.scan_interval((64, 64, 64), (20, 64, 64), 0.25) == (15, 64, 64)


def test_channel_cat_validation(ctmr):
    """ChannelCat takes two fp32 GPU NDHWC tensors on the same voxels with channel counts that are
    multiples of 16; concat_channels falls back to torch.cat otherwise (CPU-side checks only)."""
    f = ctmr.fast_fp32
    a = torch.zeros(1, 2, 2, 2, 16)
    with pytest.raises(ValueError, match="GPU"):
        f.ChannelCat(a, a)
    with pytest.raises(ValueError, match="torch.Tensor"):
        f.ChannelCat(a.numpy(), a)
    out = f.concat_channels(torch.zeros(1, 2, 2, 2, 8), torch.ones(1, 2, 2, 2, 8))
    assert isinstance(out, torch.Tensor) and tuple(out.shape) == (1, 2, 2, 2, 16)


@pytest.mark.parametrize(("shape", "keeps"), [
    ((64, 64, 3, 3, 3), False),   # UNet / VAE 3x3x3 convs: bf16 under precision("bf16")
    ((128, 256, 3, 3, 3), False),
    ((64, 4, 3, 3, 3), True),     # 4-channel input conv: fp32 LDS-staged im2col GEMM
    ((32, 8, 3, 3, 3), True),     # 8-channel condition-encoder conv
    ((64, 16, 3, 3, 3), False),   # 16 input channels: bf16
    ((4, 64, 3, 3, 3), True),     # UNet output conv (cout 4): fp32 direct conv
    ((1, 64, 3, 3, 3), True),     # VAE output conv
    ((5, 64, 3, 3, 3), False),
    ((256, 128, 1, 1, 1), True),  # 1x1 skip projections
])
def test_bf16_precision_keeps_small_convs_fp32(ctmr, shape, keeps):
    """Which convs keep fp32 operands under ``precision("bf16")`` (a function of the weight shape only):
    1x1 convs, at most 8 input channels, at most 4 output channels."""
    assert ctmr.fast_fp32._keeps_fp32(torch.empty(shape)) is keeps


def test_derived_cache_accepts_inference_tensors(ctmr):
    """The derived-weight cache keys on each source's version counter; inference tensors (made under
    ``torch.inference_mode``) have none, and must still build once and then hit (CPU: host logic
    only; the build function stands in for a pack)."""
    import threading

    f = ctmr.fast_fp32
    cache, lock, builds = {}, threading.Lock(), []

    def build():
        builds.append(1)
        return torch.zeros(3)

    with torch.inference_mode():
        w = torch.ones(4)
    assert w.is_inference()
    first = f.cached_derived(cache, lock, ("k",), (w,), build)
    second = f.cached_derived(cache, lock, ("k",), (w,), build)
    assert first is second and len(builds) == 1
    v = torch.ones(4)  # an ordinary tensor: an in-place change still forces a rebuild
    f.cached_derived(cache, lock, ("v",), (v,), build)
    v.add_(1)
    f.cached_derived(cache, lock, ("v",), (v,), build)
    assert len(builds) == 3


def test_python_kernel_constants_match_header(ctmr):
    """Every ``CTMR_K_*`` route of include/ctmr.h has its Python constant, in enum order."""
    import re

    L = ctmr._lib
    text = L.HEADER_PATH.read_text()
    names = re.findall(r"CTMR_K_(\w+)\s*=\s*(\d+)", text)
    assert len(names) == len(L.KERNEL_NAMES)
    for name, value in names:
        assert getattr(L, "K_" + name) == int(value), name


def test_custom_operators_are_registered_and_trace(ctmr):
    """Every ``ctmr::*`` operator is a registered custom op with a fake implementation: under a
    FakeTensorMode (tracing) the call goes through the dispatcher to the fake and launches nothing; an
    eager call on plain tensors (and only that) bypasses the dispatcher."""
    from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

    ops = ctmr.ops
    names = ["pack_weight", "conv3d", "conv3d_gn", "gn_affine_from_stats", "gn_affine_from_stats2", "add_gn",
             "gn_affine", "gn_apply", "silu", "resample", "gn_avgpool", "flash_attention"]
    for name in names:
        wrapper = getattr(ops, name)
        assert hasattr(torch.ops.ctmr, name) and type(wrapper.op).__name__ == "CustomOpDef", name
        assert callable(wrapper.fn) and wrapper.__doc__
    x = torch.zeros(2, 4, 4, 4, 64)
    assert ops._direct((x, 3, None))
    assert not ops._direct((x.requires_grad_(),))
    with torch.no_grad():
        assert ops._direct((x,))  # autograd records nothing here
    x = x.detach()
    with FakeTensorMode():
        assert not ops._direct((3,))
        fx = torch.empty(2, 4, 4, 4, 64)
        a = ops.gn_affine(fx, torch.empty(64), torch.empty(64), 32, 1e-6)
        y, st = ops.add_gn(fx, fx)
        s2 = ops.gn_affine_from_stats2(st, 64, torch.empty(128), torch.empty(128), 32, 100, 1e-6, st)
    assert isinstance(a, FakeTensor) and tuple(a.shape) == (2, 64, 2)
    assert tuple(y.shape) == tuple(x.shape) and st.dtype == torch.float64 and st.shape[2:] == (64, 2)
    assert tuple(s2.shape) == (2, 128, 2)


def test_depth_slab_plan(ctmr):
    """The depth-slab plan (descriptors only, no GPU work): every input plane is kept by exactly one slab,
    each slab reads a one-plane halo inside the volume, and each slab's descriptor selects the whole
    volume's kernel and split; budgets too small for any such slab depth give no plan (the conv then runs
    whole)."""
    f, L, ops = ctmr.fast_fp32, ctmr._lib, ctmr.ops
    for shape, cout, code, stream in (((2, 20, 64, 64, 64), 64, L.DT_F32, False),  # fp32 LDS-staged GEMM
                                      ((1, 18, 32, 32, 64), 64, L.DT_F32, True),  # four-wave split form
                                      ((1, 16, 32, 32, 64), 64, L.DT_F16X2, False)):
        x = torch.empty(shape, device="meta")
        flags = L.F_AFFINE | L.F_SILU | (L.F_STREAM if stream else 0)
        whole = ops.make_desc(shape, cout, 3, 1, 0, flags, code, 0)
        per_plane = max(1, L.workspace_bytes(whole) // shape[1])
        plans = 0
        for depth in range(1, 9):
            out = f._slabs(x, None, cout=cout, ksize=3, mode=0, flags=flags, code=code, split=0,
                           budget=per_plane * (depth + 2))
            if out is None:
                continue
            plans += 1
            split, plan, extra = out
            assert split == L.conv_split(whole)
            assert extra == (L.F_SPLIT_WAVES if L.conv_kernel(whole) == "split_waves" else 0)
            assert [p for a, b, s0, s1 in plan for p in range(s0, s1)] == list(range(shape[1]))
            assert max(s1 - s0 for a, b, s0, s1 in plan) <= depth
            for a, b, s0, s1 in plan:
                assert a == max(s0 - 1, 0) and b == min(s1 + 1, shape[1])
                desc = ops.make_desc((shape[0], b - a, *shape[2:]), cout, 3, 1, 0, flags | extra, code, split)
                assert L.conv_kernel(desc) == L.conv_kernel(whole) and L.conv_split(desc) == split
        assert plans > 0, shape


def test_split_waves_flag_host_checks(ctmr, native_loaded):
    """``CTMR_F_SPLIT_WAVES`` selects the four-wave split form with the caller's split, and is refused
    where that form does not apply (no split, a split over taps * K blocks / 32, 1x1x1, 16-bit LDS GEMMs)."""
    import ctypes

    L = ctmr._lib
    d = L.conv_desc(1, 18, 32, 32, 64, 64, flags=L.F_SPLIT_WAVES, split=2)
    assert L.conv_kernel(d) == "split_waves" and L.conv_split(d) == 2
    for kw, status in (({"split": 0}, L.E_INVALID), ({"split": 4}, L.E_INVALID), ({"split": 2, "ksize": 1}, L.E_INVALID),
                       ({"split": 2, "dtype": L.DT_F16X2}, L.E_UNSUPPORTED)):  # split fp16: the LDS GEMM only
        args = dict(flags=L.F_SPLIT_WAVES)
        args.update(kw)
        rc = native_loaded.ctmr_conv3d_kernel(ctypes.byref(L.conv_desc(1, 18, 32, 32, 64, 64, **args)))
        assert rc == status, kw
