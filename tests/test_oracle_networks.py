"""Pin the network-level CPU oracle (oracle/maisi_torch.py) on the reference goldens.

Goldens are MONAI 1.6.0 / Torch CPU recordings (tests/golden); tolerances are
the reference's own (maisi_mlx_feasibility.py:11-29 of the reference):
residual 1e-5/1e-6, UNet and VAE 1e-4/1e-5.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from golden_util import load_boundary, load_fixture
from oracle import maisi_torch as mt

UNET_RTOL, UNET_ATOL = 1e-4, 1e-5
VAE_RTOL, VAE_ATOL = 1e-4, 1e-5
RES_RTOL, RES_ATOL = 1e-5, 1e-6
D = torch.float64


def _t(a, dtype=D):
    return torch.from_numpy(np.asarray(a)).to(dtype)


def test_residual_block_golden():
    manifest, a = load_boundary("residual")
    w = mt.to_torch(a)
    c = manifest["constructor"]
    y = mt.residual_block(_t(a["x"]), _t(a["emb"]), w, c["norm_num_groups"], c["norm_eps"])
    np.testing.assert_allclose(y.numpy(), a["y"], rtol=RES_RTOL, atol=RES_ATOL)


def test_planted_missing_skip_fails_residual_golden():
    """Dropping the skip path must fail the golden.  (The time-embedding bias is
    not a usable plant here: with 32 groups over 32 channels, GroupNorm removes
    any per-channel constant, so this golden cannot see it; the UNet goldens,
    with 2 channels per group, do.)"""
    manifest, a = load_boundary("residual")
    w = mt.to_torch(a)
    c = manifest["constructor"]
    x = _t(a["x"])
    y = mt.residual_block(x, _t(a["emb"]), w, c["norm_num_groups"], c["norm_eps"]) - x
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(y.numpy(), a["y"], rtol=RES_RTOL, atol=RES_ATOL)


def test_unet_diffusion_boundary_golden():
    manifest, a = load_boundary("diffusion")
    weights = mt.to_torch(load_fixture("unet.npz"))
    t_emb, y = mt.unet(_t(a["x"]), _t(a["timesteps"]), torch.from_numpy(a["class_labels"]), _t(a["spacing"]),
                       weights, manifest["constructor"])
    np.testing.assert_allclose(t_emb.numpy(), a["t_emb"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(y.numpy(), a["y"], rtol=UNET_RTOL, atol=UNET_ATOL)


def test_unet_fixture_golden():
    f = load_fixture("unet.npz")
    meta = f["__metadata__"]
    _, y = mt.unet(_t(f["input.x"]), _t(f["input.timesteps"]), torch.from_numpy(f["input.class_labels"]),
                   _t(f["input.spacing"]), mt.to_torch(f), meta["constructor"])
    np.testing.assert_allclose(y.numpy(), f["output.velocity"], rtol=UNET_RTOL, atol=UNET_ATOL)


def test_vae_decode_and_tiled_golden():
    f = load_fixture("vae.npz")
    ctor = f["__metadata__"]["constructor"]
    w = mt.to_torch(f)
    _, decoded = mt.vae_decode(_t(f["input.z"]), w, ctor)
    np.testing.assert_allclose(decoded.numpy(), f["output.decoded"], rtol=VAE_RTOL, atol=VAE_ATOL)
    tiled = mt.sliding_window_decode(_t(f["input.z"]), w, ctor, roi=(2, 2, 2), overlap=0.5, scale_factor=1.25)
    np.testing.assert_allclose(tiled.numpy(), f["output.tiled"], rtol=VAE_RTOL, atol=VAE_ATOL)


def test_vae_boundary_golden():
    _, a = load_boundary("vae")
    f = load_fixture("vae.npz")
    post, decoded = mt.vae_decode(_t(a["z"]), mt.to_torch(f), f["__metadata__"]["constructor"])
    np.testing.assert_allclose(post.numpy(), a["post_quant"], rtol=VAE_RTOL, atol=VAE_ATOL)
    np.testing.assert_allclose(decoded.numpy(), a["decoded"], rtol=VAE_RTOL, atol=VAE_ATOL)


@pytest.mark.parametrize("name", ["mr.npz", "mr-brain.npz"])
def test_mr_pipeline_golden(name):
    """The reference's only end-to-end golden of the fast path (test_mr.py:181-242):
    CFG velocity batch at t=1000, the 30-step latent, the decode and the int16 image."""
    f = load_fixture(name)
    meta = f["__metadata__"]
    ctor = meta["constructor"]
    unet_w = mt.to_torch(f, strip="weight.unet.")
    vae_w = mt.to_torch(f, strip="weight.vae.")
    x = _t(f["input.latent"])
    modality = int(meta["modality"])
    spacing = _t(f["output.spacing"])
    classes = torch.tensor([modality, 0])
    _, vb = mt.unet(torch.cat([x, x]), _t([1000.0, 1000.0]), classes, spacing.repeat(2, 1), unet_w, ctor["unet"])
    np.testing.assert_allclose(vb.numpy(), f["output.velocity_batch"], rtol=UNET_RTOL, atol=UNET_ATOL)
    steps = mt.rflow_timesteps(int(meta["num_inference_steps"]), int(np.prod(x.shape[2:])))
    np.testing.assert_array_equal(steps, f["output.timesteps"])
    g = float(meta["guidance_scale"])
    z = x
    nxt = np.concatenate([steps[1:], [0.0]])
    for t, tn in zip(steps.tolist(), nxt.tolist()):
        _, v = mt.unet(torch.cat([z, z]), _t([t, t]), classes, spacing.repeat(2, 1), unet_w, ctor["unet"])
        v = v[1:] + g * (v[:1] - v[1:])
        z = z + v * ((t - int(tn)) / 1000.0)
    np.testing.assert_allclose(z.numpy(), f["output.latent"], rtol=UNET_RTOL, atol=UNET_ATOL)
    decoded = mt.sliding_window_decode(_t(f["output.latent"]), vae_w, ctor["vae"], roi=(80, 80, 80), overlap=0.4,
                                       scale_factor=1.25)
    np.testing.assert_allclose(decoded.numpy(), f["output.decoded"], rtol=VAE_RTOL, atol=VAE_ATOL)
    image = np.clip(f["output.decoded"].astype(np.float32) * 1000.0, 0.0, None).astype(np.int16)
    np.testing.assert_array_equal(image, f["output.image"])


@pytest.mark.parametrize(("name", "key"), [("unet.npz", None), ("vae.npz", None), ("mr.npz", "unet"), ("mr.npz", "vae")])
def test_weight_catalogs_match_recorded_recipes(ctmr, name, key):
    """The product's state-dict catalogs (names, shapes) equal the reference recipes'."""
    f = load_fixture(name)
    meta = f["__metadata__"]
    ctor = meta["constructor"][key] if key else meta["constructor"]
    prefix = "weight." + (f"{key}." if key else "")
    recorded = {n[len(prefix):]: tuple(s) for n, s in meta["weight_recipe"]["shapes"] if n.startswith(prefix)}
    if "vae" in (key or name):
        recorded = {k: v for k, v in recorded.items() if k.startswith(("decoder.", "post_quant"))}
        mine = dict(ctmr.maisi.vae_decoder_weight_shapes(ctor))
    else:
        mine = dict(ctmr.maisi.unet_weight_shapes(ctor))
    assert mine == recorded


def test_rflow_schedule_and_step(ctmr):
    f = load_fixture("rflow.npz")
    m = ctmr.maisi
    times, nxt = m.set_timesteps_rflow(num_inference_steps=7, input_img_size_numel=64)
    np.testing.assert_allclose(times, f["output.timesteps"], rtol=1e-6)
    np.testing.assert_allclose(nxt, f["output.next_timesteps"], rtol=1e-6)
    x = torch.from_numpy(f["input.x"])
    step, origin, dt = m.step_rflow(x, x * 0.125, float(times[1]), float(nxt[1]))
    np.testing.assert_allclose(step.numpy(), f["output.step"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(origin.numpy(), f["output.origin"], rtol=1e-5, atol=1e-6)
    assert dt == (float(times[1]) - int(float(nxt[1]))) / 1000.0
    sample = m.sample_rflow(x, lambda cur, t: cur * 0.125 + t * 0.0001, times)
    np.testing.assert_allclose(sample.numpy(), f["output.sample"], rtol=1e-5, atol=1e-6)


def test_controlnet_oracle_identity_invariant(ctmr):
    """With identity 1x1 zero convs and a zero conditioning encoder, the ControlNet's down
    residuals are the UNet encoder's skips (golden-pinned blocks) and its mid residual is the
    mid-block output; the 3x down-blocks and mid block are the UNet's own, so this ties the
    ControlNet composition to the UNet goldens.  (No recorded ControlNet outputs ship with
    the reference, so this is the available pin.)"""
    f = load_fixture("controlnet.npz")
    ctor = f["__metadata__"]["constructor"]
    w = mt.to_torch(f)
    for k in list(w):
        if k.startswith("controlnet_down_blocks.") or k.startswith("controlnet_mid_block."):
            if k.endswith("weight"):
                c = w[k].shape[0]
                w[k] = torch.eye(c, dtype=D).reshape(c, c, 1, 1, 1)
            else:
                w[k] = torch.zeros_like(w[k])
        if k == "controlnet_cond_embedding.conv_out.conv.weight" or k == "controlnet_cond_embedding.conv_out.conv.bias":
            w[k] = torch.zeros_like(w[k])
    x = _t(f["input.x"])
    cond = torch.from_numpy(np.random.default_rng(2).standard_normal((1, 8, 16, 16, 16)))
    t = _t(f["input.timesteps"])
    labels = torch.from_numpy(f["input.class_labels"])
    down, mid = mt.controlnet(x, t, labels, cond, w, ctor)
    emb = mt._mlp(mt.timestep_embedding(t, ctor["num_channels"][0]), w, "time_embed") + w["class_embedding.weight"][labels.long()]
    h = torch.nn.functional.conv3d(x, w["conv_in.conv.weight"], w["conv_in.conv.bias"], padding=1)
    h, skips = mt.down_path(h, emb, w, ctor)
    assert len(down) == len(skips)
    for d, s in zip(down, skips):
        np.testing.assert_allclose(d.numpy(), s.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mid.numpy(), mt.mid_block(h, emb, w, ctor).numpy(), rtol=1e-12, atol=1e-12)


def test_controlnet_catalog_matches_recorded_recipe(ctmr):
    f = load_fixture("controlnet.npz")
    meta = f["__metadata__"]
    recorded = {n[len("weight."):]: tuple(s) for n, s in meta["weight_recipe"]["shapes"]}
    assert dict(ctmr.maisi.controlnet_weight_shapes(meta["constructor"])) == recorded


def test_controlnet_rejects_bad_condition_shapes(ctmr):
    """Host-side validation runs before any kernel: cond channels and the 4x spatial ratio."""
    f = load_fixture("controlnet.npz")
    ctor = f["__metadata__"]["constructor"]
    x = torch.zeros(1, 4, 4, 4, 4)
    with pytest.raises(ValueError, match="cond channels"):
        ctmr.maisi.encode_controlnet_condition(torch.zeros(1, 16, 16, 16, 3), {}, constructor=ctor)
    with pytest.raises(ValueError, match="4x latent"):
        ctmr.maisi.controlnet_residuals(x, torch.zeros(1), torch.zeros(1, dtype=torch.long),
                                        torch.zeros(1, 8, 8, 8, 8), {}, constructor=ctor)
    with pytest.raises(ValueError, match="ddpm-ct"):
        ctmr.maisi.controlnet_residuals(x, None, None, x, {}, constructor={**ctor, "resblock_updown": False})


def test_attention_oracle_golden():
    """Residual spatial self-attention (attention.py:92-160) against the recorded MONAI block."""
    manifest, a = load_boundary("attention")
    c = manifest["constructor"]
    y = mt.attention(_t(a["x"]), mt.to_torch(a), c["norm_num_groups"], c["norm_eps"], c["num_head_channels"],
                     c["include_fc"])
    np.testing.assert_allclose(y.numpy(), a["y"], rtol=RES_RTOL, atol=RES_ATOL)


def test_planted_unscaled_scores_fail_attention_golden():
    """Dropping the 1/sqrt(head_dim) score scale (head_dim 1 -> scale 1) must fail the golden."""
    manifest, a = load_boundary("attention")
    c = manifest["constructor"]
    w = mt.to_torch(a)
    x = _t(a["x"])
    n = x.shape[0]
    h = torch.nn.functional.group_norm(x, c["norm_num_groups"], w["norm.weight"], w["norm.bias"], c["norm_eps"])
    tok = h.reshape(n, x.shape[1], -1).transpose(1, 2)
    q, k, v = (torch.nn.functional.linear(tok, w[f"attn.to_{m}.weight"], w[f"attn.to_{m}.bias"]) for m in "qkv")
    out = torch.softmax(q @ k.transpose(1, 2), dim=-1) @ v
    out = torch.nn.functional.linear(out, w["attn.out_proj.weight"], w["attn.out_proj.bias"])
    y = x + out.transpose(1, 2).reshape(x.shape)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(y.numpy(), a["y"], rtol=RES_RTOL, atol=RES_ATOL)
