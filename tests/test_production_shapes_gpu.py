"""The reference's other production grids (configurations.json of the reference; README.md:26-28):

* general MR, 128x256x256 output (latent 32x64x64), guidance 15 (batched CFG, batch 2);
* MR-Brain and CT, 256x256x128 output (latent 64x64x32): MR-Brain guided at batch 2 is config 3's
  UNet step itself; CT from a 256x256x128 mask runs the ControlNet and the UNet at batch 1
  (from_mask.py:101-118 accepts 256x256x128 and 256^3).

Checked here: the MR UNet step at its latent (batch 2) against the PyTorch-CPU oracle (<= 1e-4, fp32 and
split fp16) and the guided velocity formed from it; two ControlNet-conditioned rflow steps from a
256x256x128 mask against the oracle's sampler (<= 1e-4); and the windowed decode with the reference's
default window (roi 48x48x64 latent, overlap 0.6666): both grids' latents are smaller than that window,
so they decode in one pass, checked against the PyTorch-CPU decoder at 256x256x128.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import maisi_torch as mt
from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

STEP_REL = 1e-4  # north-star bar of a UNet step


def _g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(t):
    return t.detach().cpu().numpy()


def _weights(m, shapes, seed, dev):
    host = m.random_weights(shapes, seed=seed)
    return host, {k: torch.from_numpy(v).to(dev) for k, v in host.items()}


def _threads():
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))


@pytest.fixture(scope="module")
def unet(ctmr, dev):
    m = ctmr.maisi
    return _weights(m, m.unet_weight_shapes(m.PRODUCTION_UNET_CONSTRUCTOR), 7, dev)


@pytest.fixture(scope="module")
def mr_step_reference(ctmr, unet):
    """The oracle's batch-2 (conditional, unconditional) UNet output at the general-MR latent."""
    m = ctmr.maisi
    host, _ = unet
    rng = np.random.default_rng(61)
    x = rng.standard_normal((1, 32, 64, 64, 4)).astype(np.float32)
    t = np.float32(rng.uniform(0, 1000))
    spacing = np.asarray([[1.25, 1.0, 1.0]], np.float64)
    sp16 = (spacing * 100).astype(np.float16).astype(np.float32)  # spacing_tensor's rounding
    xx = np.concatenate([x, x])
    _threads()
    with torch.no_grad():
        _, ref = mt.unet(torch.from_numpy(np.moveaxis(xx, -1, 1).copy()), torch.full((2,), float(t)),
                         torch.tensor([9, 0]), torch.from_numpy(np.repeat(sp16, 2, 0)),
                         mt.to_torch(host, dtype=torch.float32, strip=""), m.PRODUCTION_UNET_CONSTRUCTOR)
    return x, float(t), spacing[0], np.moveaxis(ref.numpy(), 1, -1)


@pytest.mark.parametrize("precision", ["fp32", "f16x2"])
def test_general_mr_guided_step_matches_cpu_oracle(ctmr, dev, unet, mr_step_reference, precision):
    """General MR (128x256x256 output): the batched-CFG UNet pass at latent 32x64x64 (batch 2: class 9
    and the unconditional class 0) within 1e-4 of the oracle; ``guided_velocity`` at the MR guidance
    scale (15) is uncond + 15 (cond - uncond) of exactly that pass."""
    m = ctmr.maisi
    _, w = unet
    x, t, spacing, ref = mr_step_reference
    ctor = m.PRODUCTION_UNET_CONSTRUCTOR
    sp = m.spacing_tensor(list(spacing), device=dev)
    xg = _g(x, dev)
    with ctmr.fast_fp32.precision(precision):
        _, y = m.denoise_unet(torch.cat([xg, xg]), torch.full((2,), t, device=dev), torch.tensor([9, 0], device=dev),
                              torch.cat([sp, sp]), w, constructor=ctor)
        v = m.guided_velocity(xg, t, class_labels=torch.tensor([9], device=dev), spacing=sp, weights=w,
                              constructor=ctor, guidance_scale=15.0)
    err = rm.max_rel_error(_h(y), ref)
    print(f"general MR step ({precision}) vs CPU oracle: {err:.3e}", flush=True)
    assert err <= STEP_REL
    expect = y[1:] + 15.0 * (y[:1] - y[1:])
    assert torch.equal(v, expect)


def test_ct_from_256x256x128_mask_matches_cpu_oracle(ctmr, dev, unet):
    """CT from a 256x256x128 label map: the condition encoded at full resolution, then two ControlNet +
    UNet rflow steps at latent 64x64x32 (batch 1), fp32 and split fp16, against the oracle's sampler."""
    m = ctmr.maisi
    uh, uw = unet
    uc, cc = m.PRODUCTION_UNET_CONSTRUCTOR, m.PRODUCTION_CONTROLNET_CONSTRUCTOR
    ch, cw = _weights(m, m.controlnet_weight_shapes(cc), 13, dev)
    rng = np.random.default_rng(62)
    label = rng.choice(np.array(sorted(m.VALID_LABELS)), size=(1, 1, 256, 256, 128)).astype(np.int16)
    label[0, 0, :, :, :16] = 0
    z0 = rng.standard_normal((1, 64, 64, 32, 4)).astype(np.float32)
    spacing_mm, steps = (1.7, 1.7, 2.0), 2
    m.require_supported_production_shape(label.shape[2:])
    got = {}
    for precision in ("fp32", "f16x2"):
        with ctmr.fast_fp32.precision(precision):
            lat, _ = m.sample_ct_latent(label, spacing_mm, unet_weights=uw, controlnet_weights=cw,
                                        unet_constructor=uc, controlnet_constructor=cc, scale_factor=1.0,
                                        latent=_g(z0, dev), num_inference_steps=steps, drop_weights=False)
        got[precision] = _h(lat)
    times, _ = m.set_timesteps_rflow(num_inference_steps=steps, input_img_size_numel=64 * 64 * 32)
    _threads()
    with torch.no_grad():
        cond = mt.binarize_labels(torch.from_numpy(label.astype(np.int64)))
        sp = torch.tensor([[v * 100.0 for v in spacing_mm]], dtype=torch.float32)  # from-mask: not rounded
        ref = mt.ct_sample(torch.from_numpy(np.moveaxis(z0, -1, 1).copy()), cond, sp, torch.tensor([1]),
                           mt.to_torch(uh, dtype=torch.float32, strip=""),
                           mt.to_torch(ch, dtype=torch.float32, strip=""), uc, cc, [float(v) for v in times])
    ref = np.moveaxis(ref.numpy(), 1, -1)
    for precision, lat in got.items():
        err = rm.max_rel_error(lat, ref)
        print(f"CT 256x256x128 from mask ({precision}), {steps} steps: latent vs CPU oracle {err:.3e}", flush=True)
        assert err <= STEP_REL


@pytest.fixture(scope="module")
def brain_decode_reference(ctmr):
    """The PyTorch-CPU decoder's output for a 64x64x32 latent (256x256x128 image)."""
    m = ctmr.maisi
    ctor = m.PRODUCTION_VAE_CONSTRUCTOR
    host = m.random_weights(m.vae_decoder_weight_shapes(ctor), seed=11)
    z = np.random.default_rng(63).standard_normal((1, 64, 64, 32, 4)).astype(np.float32)
    _threads()
    with torch.no_grad():
        _, ref = mt.vae_decode(torch.from_numpy(np.moveaxis(z, -1, 1).copy()),
                               mt.to_torch(host, dtype=torch.float32, strip=""), ctor)
    return z, np.moveaxis(ref.numpy(), 1, -1)


@pytest.mark.parametrize(("name", "latent"), [("general MR 128x256x256", (32, 64, 64)),
                                              ("MR-Brain / CT 256x256x128", (64, 64, 32))])
@pytest.mark.parametrize("precision", ["fp32", "f16x2"])
def test_production_grid_decode_is_one_pass(ctmr, dev, brain_decode_reference, name, latent, precision):
    """Both grids' latents hold fewer voxels than the default window (48 x 48 x 64 = 147,456 latent
    voxels), so the windowed decode takes its one-pass branch (decode.py:187-245): the whole latent
    through the decoder, bit-identical to ``decode_vae``; the 256x256x128 image within 1e-4 of the
    PyTorch-CPU decoder."""
    m = ctmr.maisi
    print(f"case {name} ({precision})", flush=True)
    ctor = m.PRODUCTION_VAE_CONSTRUCTOR
    _, w = _weights(m, m.vae_decoder_weight_shapes(ctor), 11, dev)
    assert np.prod(latent) <= np.prod(m.DEFAULT_ROI_SIZE)
    if latent == (64, 64, 32):
        z, ref = brain_decode_reference
    else:
        z, ref = np.random.default_rng(64).standard_normal((1, *latent, 4)).astype(np.float32), None
    with ctmr.fast_fp32.precision(precision):
        y = m.sliding_window_decode(_g(z, dev), w, constructor=ctor)
        whole = m.decode_vae(_g(z, dev), w, constructor=ctor)[1]
    assert tuple(y.shape) == (1, *(4 * s for s in latent), 1)
    assert torch.equal(y, whole)
    y = _h(y)
    assert np.isfinite(y).all()
    if ref is not None:
        err = rm.max_rel_error(y, ref)
        print(f"{name} ({precision}): one-pass decode vs CPU decoder {err:.3e}", flush=True)
        assert err <= STEP_REL
