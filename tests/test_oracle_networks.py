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


# --- ControlNet: closed-form pins of the conditioning encoder and the conditioning scale -------------
def _encoder_brute_force(cond_ndhwc, w, ctor, *, strides=(1, 2), silu_mask=None):
    """Conditioning encoder (controlnet.py:194-249) composed layer by layer from the float64 NumPy
    oracle (oracle/reference_math, pinned on the recorded conv/SiLU goldens): conv_in + SiLU, per
    level a conv of stride ``strides[0]`` + SiLU and one of ``strides[1]`` + SiLU, conv_out.
    ``silu_mask`` (one flag per SiLU) plants a dropped SiLU."""
    from oracle import reference_math as rm

    p = "controlnet_cond_embedding"
    get = lambda k: w[k].numpy()
    flags = iter(silu_mask or [True] * 99)
    act = lambda v: rm.silu(v) if next(flags) else v
    h = act(rm.conv3d(cond_ndhwc, get(f"{p}.conv_in.conv.weight"), get(f"{p}.conv_in.conv.bias")))
    block = 0
    for _ in range(len(ctor["conditioning_embedding_num_channels"]) - 1):
        for stride in strides:
            h = act(rm.conv3d(h, get(f"{p}.blocks.{block}.conv.weight"), get(f"{p}.blocks.{block}.conv.bias"),
                              stride=stride))
            block += 1
    return rm.conv3d(h, get(f"{p}.conv_out.conv.weight"), get(f"{p}.conv_out.conv.bias"))


def _controlnet_fixture():
    f = load_fixture("controlnet.npz")
    ctor = f["__metadata__"]["constructor"]
    cond = np.random.default_rng(21).integers(0, 2, (1, 16, 16, 16, 8)).astype(np.float64)
    return f, ctor, mt.to_torch(f), cond


def test_controlnet_encoder_matches_brute_force_and_planted_mistakes_fail():
    """The oracle's encoder (torch F.conv3d) equals the NumPy layer-by-layer composition on the recorded
    recipe network with a non-zero conv_out; swapping each level's stride order, or dropping the SiLU
    after a stride-2 conv, changes the embedding beyond the comparison tolerance."""
    _, ctor, w, cond = _controlnet_fixture()
    got = mt.controlnet_condition(torch.from_numpy(np.moveaxis(cond, -1, 1).copy()), w, ctor)
    got = np.moveaxis(got.numpy(), 1, -1)
    assert np.abs(got).max() > 1e-3  # conv_out is live
    np.testing.assert_allclose(got, _encoder_brute_force(cond, w, ctor), rtol=1e-10, atol=1e-12)
    scale = np.abs(got).max()
    with pytest.raises(AssertionError):  # stride-2 first, then stride-1
        np.testing.assert_allclose(got, _encoder_brute_force(cond, w, ctor, strides=(2, 1)), rtol=0,
                                   atol=1e-6 * scale)
    with pytest.raises(AssertionError):  # SiLU dropped after the first stride-2 conv
        np.testing.assert_allclose(got, _encoder_brute_force(cond, w, ctor, silu_mask=[True, True, False, True, True]),
                                   rtol=0, atol=1e-6 * scale)


def test_controlnet_first_residual_is_conv_in_plus_embedding():
    """With identity zero convs, the first down residual is the skip taken before any block:
    conv_in(x) + encoder(cond) (controlnet.py:119-131) -- so the embedding joins right after conv_in.
    Closed form from the NumPy oracle."""
    from oracle import reference_math as rm

    f, ctor, w, cond = _controlnet_fixture()
    for k in list(w):
        if k.startswith("controlnet_down_blocks.") or k.startswith("controlnet_mid_block."):
            if k.endswith("weight"):
                c = w[k].shape[0]
                w[k] = torch.eye(c, dtype=D).reshape(c, c, 1, 1, 1)
            else:
                w[k] = torch.zeros_like(w[k])
    x = np.asarray(f["input.x"], np.float64)
    down, _ = mt.controlnet(torch.from_numpy(x), _t(f["input.timesteps"]), torch.from_numpy(f["input.class_labels"]),
                            torch.from_numpy(np.moveaxis(cond, -1, 1).copy()), w, ctor)
    x_nd = np.moveaxis(x, 1, -1)
    expected = rm.conv3d(x_nd, w["conv_in.conv.weight"].numpy(), w["conv_in.conv.bias"].numpy()) + \
        _encoder_brute_force(cond, w, ctor)
    np.testing.assert_allclose(np.moveaxis(down[0].numpy(), 1, -1), expected, rtol=1e-10, atol=1e-12)


def test_controlnet_conditioning_scale_multiplies_zero_conv_outputs():
    """``conditioning_scale`` multiplies every zero-conv output, bias included, down and mid alike
    (controlnet.py:160-163): with zero 1x1 weights each residual is exactly ``scale * bias``; with the
    recipe weights the residuals are exactly linear in the scale."""
    f, ctor, w, cond = _controlnet_fixture()
    args = (_t(f["input.x"]), _t(f["input.timesteps"]), torch.from_numpy(f["input.class_labels"]),
            torch.from_numpy(np.moveaxis(cond, -1, 1).copy()))
    base_down, base_mid = mt.controlnet(*args, w, ctor)
    down, mid = mt.controlnet(*args, w, ctor, scale=-0.375)
    for a, b in zip(down + [mid], base_down + [base_mid]):
        np.testing.assert_allclose(a.numpy(), -0.375 * b.numpy(), rtol=1e-12, atol=1e-15)
    zw = dict(w)
    biases = {}
    for k in list(zw):
        if (k.startswith("controlnet_down_blocks.") or k.startswith("controlnet_mid_block.")) and k.endswith("weight"):
            zw[k] = torch.zeros_like(zw[k])
        elif k.startswith("controlnet_down_blocks.") or k.startswith("controlnet_mid_block."):
            biases[k] = zw[k]
    down, mid = mt.controlnet(*args, zw, ctor, scale=2.5)
    keys = [k for k in sorted(biases, key=lambda s: (s.startswith("controlnet_mid"),
                                                     int(s.split(".")[1]) if s.startswith("controlnet_down") else 0))]
    for res, key in zip(down + [mid], keys):
        expected = 2.5 * biases[key].numpy().reshape(1, -1, 1, 1, 1) * np.ones(res.shape)
        np.testing.assert_allclose(res.numpy(), expected, rtol=1e-15, atol=0)


# --- CT from mask: label bits, HU, sampling loop ------------------------------------------------------
def test_binarize_labels_recomposes_every_id(ctmr):
    """Both restatements of condition.py:20-43 (the product's bit masks, the oracle's halving) give
    channels whose weighted sum sum_k 2^k c_k is the label id, for every valid MAISI id."""
    ids = np.array(sorted(ctmr.maisi.VALID_LABELS), np.int64)
    lab = ids.reshape(1, 1, 1, 1, -1)
    ora = mt.binarize_labels(torch.from_numpy(lab)).numpy()  # (1, 8, 1, 1, L)
    prod = ctmr.maisi.binarize_labels(torch.from_numpy(lab[:, 0])).numpy()  # (1, 1, 1, L, 8)
    weights = 2.0 ** np.arange(8)
    np.testing.assert_array_equal((ora[0, :, 0, 0, :] * weights[:, None]).sum(0), ids)
    np.testing.assert_array_equal(np.moveaxis(ora, 1, -1)[0, 0], prod[0, 0])
    assert set(np.unique(prod)) <= {0.0, 1.0} and prod.dtype == np.float32


def test_to_hu_closed_form(ctmr):
    img = torch.tensor([-0.5, 0.0, 0.25, 0.5, 1.0, 1.5]).reshape(1, 1, 1, 6, 1)  # NDHWC
    lab = torch.tensor([1, 1, 200, 0, 5, 1]).reshape(1, 1, 1, 6)
    expected = [-1000.0, -1000.0, -500.0, -1000.0, 1000.0, 1000.0]
    np.testing.assert_array_equal(ctmr.maisi.to_hu(img, lab).reshape(-1).numpy(), expected)
    np.testing.assert_array_equal(mt.to_hu(img.reshape(1, 1, 1, 1, 6), lab.reshape(1, 1, 1, 1, 6)).reshape(-1).numpy(),
                                  expected)


def test_ct_label_validation(ctmr):
    m = ctmr.maisi
    ok = np.full((1, 1, 8, 8, 8), 200, np.int16)
    m.require_ct_label(ok)
    with pytest.raises(ValueError, match="1 channel"):
        m.require_ct_label(ok[:, 0])
    with pytest.raises(ValueError, match="integer"):
        m.require_ct_label(ok.astype(np.float32))
    bad = ok.copy()
    bad[0, 0, 0, 0, 0] = 150
    with pytest.raises(ValueError, match="outside 0..132"):
        m.require_ct_label(bad)
    with pytest.raises(ValueError, match="body-envelope"):
        m.require_ct_label(np.zeros((1, 1, 8, 8, 8), np.int32))
    with pytest.raises(ValueError, match="multiples of 4"):
        m.require_ct_label(np.full((1, 1, 8, 8, 6), 200, np.int32))
    with pytest.raises(ValueError, match="scale_factor"):
        m.require_scale_factor(float("nan"))
    with pytest.raises(ValueError, match="not production-proven"):
        m.require_supported_production_shape((128, 128, 128))
    assert m.require_supported_production_shape([256, 256, 128]) == (256, 256, 128)
    with pytest.raises(ValueError, match="finite and > 0"):
        m.ct_spacing_tensor([1.0, 0.0, 1.0])
    np.testing.assert_array_equal(m.ct_spacing_tensor([0.703125, 0.703125, 1.25]).numpy(), [[70.3125, 70.3125, 125.0]])


def test_ct_sampling_oracle_euler_identity():
    """With every zero conv and the UNet's output conv set to zero except the output bias ``b``,
    the velocity is the constant ``b``; the sampler then moves the latent by ``b * sum(dt)`` with
    ``dt = (t - int(t_next)) / 1000`` (rflow.py:100-119)."""
    f, ctor, w, _ = _controlnet_fixture()
    uf = load_fixture("unet.npz")
    uctor = uf["__metadata__"]["constructor"]
    uw = mt.to_torch(uf)
    uw["out.2.conv.weight"] = torch.zeros_like(uw["out.2.conv.weight"])
    b = uw["out.2.conv.bias"]
    z0 = torch.from_numpy(np.random.default_rng(3).standard_normal((1, 4, 4, 4, 4)))
    cond = mt.binarize_labels(torch.full((1, 1, 16, 16, 16), 200, dtype=torch.int64)).to(D)
    times = mt.rflow_timesteps(3, 64)
    ctor_u = dict(uctor)
    z = mt.ct_sample(z0, cond, _t(uf["input.spacing"]), torch.tensor([1]), uw, w, ctor_u, ctor, times)
    total = sum((float(t) - int(float(tn))) / 1000.0 for t, tn in zip(times, list(times[1:]) + [0.0]))
    np.testing.assert_allclose(z.numpy(), z0.numpy() + total * b.numpy().reshape(1, -1, 1, 1, 1), rtol=1e-12,
                               atol=1e-12)
