"""Checkpoint format and weight inventories (CPU).

The production inventories are pinned on the reference's released-checkpoint
catalog (tests/golden/from_mask_catalog.json, extracted by make_golden.py from
the reference's maisi_mlx_from_mask_weight_catalog.json); the loader follows
weights.py:102-166 of the reference (channels-last conv weights on disk,
catalog validation, the UNet's scale_factor).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from golden_util import load_fixture

CATALOG = json.loads((Path(__file__).parent / "golden" / "from_mask_catalog.json").read_text())["networks"]


@pytest.mark.parametrize("network", ["unet", "controlnet", "vae"])
def test_production_inventories_match_released_catalog(ctmr, network):
    mine = dict(ctmr.weights.production_catalog(network))
    ref = {name: tuple(shape) for name, shape, _ in CATALOG[network]}
    if network == "vae":
        ref = {k: v for k, v in ref.items() if k.startswith(("decoder.", "post_quant"))}
    assert mine == ref


@pytest.mark.parametrize("network", ["unet", "controlnet", "vae"])
def test_stored_layouts_match_catalog(ctmr, network):
    """conv3d_w tensors are exactly the rank-5 weights (stored channels-last)."""
    for name, shape, layout in CATALOG[network]:
        assert (layout == "conv3d_w") == (len(shape) == 5 and name.endswith(".weight")), name
        stored = ctmr.weights.stored_shape(name, shape)
        if layout == "conv3d_w":
            assert stored == (shape[0], shape[2], shape[3], shape[4], shape[1])
        else:
            assert stored == tuple(shape)


def _tiny_unet(seed=5):
    f = load_fixture("unet.npz")
    w = {k[len("weight."):]: torch.from_numpy(np.asarray(v, np.float32)) for k, v in f.items()
         if k.startswith("weight.")}
    shapes = [(k, tuple(v.shape)) for k, v in w.items()]
    return w, shapes


def test_round_trip_restores_torch_layout(ctmr, tmp_path):
    w, shapes = _tiny_unet()
    path = tmp_path / "unet.safetensors"
    ctmr.weights.save_network(path, w, scale_factor=0.875)
    from safetensors.numpy import load_file

    raw = load_file(str(path))
    conv = "conv_in.conv.weight"
    assert raw[conv].shape == (4, 3, 3, 3, 4)  # (O, kD, kH, kW, I) on disk
    assert raw[conv][1, 2, 0, 1, 3] == w[conv][1, 3, 2, 0, 1]
    loaded, scale = ctmr.weights.load_network(path, network="unet", device="cpu", catalog=shapes)
    assert scale == 0.875
    assert sorted(loaded) == sorted(w)
    for k in w:
        assert torch.equal(loaded[k], w[k]), k


def test_consolidated_file_uses_network_prefixes(ctmr, tmp_path):
    w, shapes = _tiny_unet()
    path = ctmr.weights.network_file(tmp_path)
    ctmr.weights.save_network(path, w, scale_factor=1.5, prefix="unet.")
    loaded, scale = ctmr.weights.load_network(path, network="unet", device="cpu", catalog=shapes)
    assert scale == 1.5 and torch.equal(loaded["out.2.conv.weight"], w["out.2.conv.weight"])


def _expect(ctmr, path, shapes, match, network="unet"):
    with pytest.raises(ctmr.weights.InvalidInputError, match=match):
        ctmr.weights.load_network(path, network=network, device="cpu", catalog=shapes)


def test_loader_rejects_bad_files(ctmr, tmp_path):
    w, shapes = _tiny_unet()
    save = ctmr.weights.save_network
    p = tmp_path / "a.safetensors"
    save(p, w)
    _expect(ctmr, p, shapes, "missing scale_factor")
    save(p, w, scale_factor=0.0)
    _expect(ctmr, p, shapes, "non-zero")
    save(p, w, scale_factor=1.0)
    _expect(ctmr, p, shapes, "must not contain scale_factor", network="controlnet")
    save(p, {k: v for k, v in w.items() if k != "conv_in.conv.bias"}, scale_factor=1.0)
    _expect(ctmr, p, shapes, "missing conv_in.conv.bias")
    save(p, {**w, "extra.weight": torch.zeros(2)}, scale_factor=1.0)
    _expect(ctmr, p, shapes, "unexpected tensor extra.weight")
    bad = dict(w)
    bad["conv_in.conv.bias"] = torch.full_like(w["conv_in.conv.bias"], float("nan"))
    save(p, bad, scale_factor=1.0)
    _expect(ctmr, p, shapes, "finite float32")
    bad["conv_in.conv.bias"] = torch.zeros(5)
    save(p, bad, scale_factor=1.0)
    _expect(ctmr, p, shapes, "shape")
    _expect(ctmr, tmp_path / "a.pt", shapes, "must be a safetensors file")
    _expect(ctmr, p, shapes, "unknown network", network="mask_vae")


def test_vae_file_skips_encoder_tensors(ctmr, tmp_path):
    """The released VAE file holds the encoder too; the decoder path validates and skips it."""
    f = load_fixture("vae.npz")
    w = {k[len("weight."):]: torch.from_numpy(np.asarray(v, np.float32)) for k, v in f.items()
         if k.startswith("weight.")}
    dec = {k: v for k, v in w.items() if k.startswith(("decoder.", "post_quant"))}
    assert len(dec) < len(w)
    p = tmp_path / "vae.safetensors"
    ctmr.weights.save_network(p, w)
    loaded, scale = ctmr.weights.load_network(p, network="vae", device="cpu",
                                              catalog=[(k, tuple(v.shape)) for k, v in dec.items()])
    assert scale is None and sorted(loaded) == sorted(dec)
