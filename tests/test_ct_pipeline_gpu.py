"""CT from a label mask through the HIP path (from_mask.py:121-338 of the reference) against the
PyTorch-CPU oracle at a reduced size: production ControlNet, UNet and VAE decoder (random init),
a 32^3 label map (8^3 latent), three rflow steps, a tiled decode (roi 4^3, overlap 0.5) and the
label-masked HU conversion.  Bars: latent and decoded image <= 1e-4 relative (the UNet-step bar),
HU within 2000 x that."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import maisi_torch as mt
from oracle import reference_math as rm

pytestmark = pytest.mark.gpu


def _weights(m, shapes, seed, dev):
    host = m.random_weights(shapes, seed=seed)
    return host, {k: torch.from_numpy(v).to(dev) for k, v in host.items()}


def test_ct_from_mask_matches_cpu_oracle(ctmr, dev):
    m = ctmr.maisi
    uc, cc, vc = m.PRODUCTION_UNET_CONSTRUCTOR, m.PRODUCTION_CONTROLNET_CONSTRUCTOR, m.PRODUCTION_VAE_CONSTRUCTOR
    uh, uw = _weights(m, m.unet_weight_shapes(uc), 7, dev)
    ch, cw = _weights(m, m.controlnet_weight_shapes(cc), 13, dev)
    vh, vw = _weights(m, m.vae_decoder_weight_shapes(vc), 11, dev)
    rng = np.random.default_rng(40)
    ids = np.array(sorted(m.VALID_LABELS))
    label = rng.choice(ids, size=(1, 1, 32, 32, 32)).astype(np.int16)
    label[0, 0, :4] = 0  # background slab
    label[0, 0, 4:8] = 200
    z0 = rng.standard_normal((1, 8, 8, 8, 4)).astype(np.float32)
    spacing_mm = (0.75, 0.75, 1.5)
    steps, roi, overlap, scale = 3, (4, 4, 4), 0.5, 1.3
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    res = m.sample_ct_from_mask(label, spacing_mm, unet_weights=uw, controlnet_weights=cw, vae_weights=vw,
                                unet_constructor=uc, controlnet_constructor=cc, vae_constructor=vc, scale_factor=scale,
                                latent=torch.from_numpy(z0).to(dev), num_inference_steps=steps, roi=roi,
                                overlap=overlap)
    assert res.seam_audit == "tiled" and res.num_inference_steps == steps
    assert set(res.stage_timings_s) == {"rflow_controlnet_unet", "vae_decode", "hu_postprocess",
                                        "total_synchronized_inference"}
    t32 = lambda h: mt.to_torch(h, dtype=torch.float32, strip="")
    times, _ = m.set_timesteps_rflow(num_inference_steps=steps, input_img_size_numel=8 ** 3)
    with torch.no_grad():
        lab = torch.from_numpy(label.astype(np.int64))
        cond = mt.binarize_labels(lab)
        spacing = torch.tensor([[75.0, 75.0, 150.0]])
        ref_lat = mt.ct_sample(torch.from_numpy(np.moveaxis(z0, -1, 1).copy()), cond, spacing, torch.tensor([1]),
                               t32(uh), t32(ch), uc, cc, [float(t) for t in times])
        ref_dec = mt.sliding_window_decode(ref_lat, t32(vh), vc, roi=roi, overlap=overlap, scale_factor=scale)
        ref_hu = mt.to_hu(ref_dec, lab)
    to_nd = lambda t: np.moveaxis(t.numpy(), 1, -1)
    lat_err = rm.max_rel_error(res.latent.cpu().numpy(), to_nd(ref_lat))
    dec_err = rm.max_rel_error(res.decoded.cpu().numpy(), to_nd(ref_dec))
    hu_abs = np.abs(res.hu.cpu().numpy() - to_nd(ref_hu)).max()
    print(f"CT from mask: latent {lat_err:.3e}, decoded {dec_err:.3e}, HU max abs {hu_abs:.3e}", flush=True)
    assert lat_err <= 1e-4 and dec_err <= 1e-4
    assert hu_abs <= 2000.0 * 1e-4 * np.abs(to_nd(ref_dec)).max() + 1e-3
    hu = res.hu.cpu().numpy()
    assert (hu[0, :4] == -1000.0).all() and hu.min() >= -1000.0 and hu.max() <= 1000.0
