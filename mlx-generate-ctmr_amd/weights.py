"""Native safetensors checkpoints for the MAISI networks on this path.

Counterpart of the reference's ``weights.load_network`` (``weights.py:38-73``
and ``_load_with_catalog``, ``:102-166``): one ``.safetensors`` file holds one
network's float32 tensors (or all three in ``model.safetensors`` under
``<network>.`` prefixes), 3D convolution weights are stored channels-last as
``(O, kD, kH, kW, I)`` (``maisi_mlx_weights.py:123-133``) and come back in the
Torch ``(O, I, kD, kH, kW)`` layout the kernels take, every tensor is checked
for name, shape, dtype and finiteness against the network's catalog, and the
UNet's file carries the latent ``scale_factor``.

The catalogs are this package's own (``maisi.unet_weight_shapes`` and friends
over the production constructors).  The VAE file also holds the encoder and
the quantisation convolutions, which this path never runs: they are validated
as finite float32 and skipped.  Files are read only through ``safetensors``,
which executes nothing from the file.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from pathlib import Path
from typing import Optional, Union

import numpy as np
import torch
from torch import Tensor

from . import maisi

NETWORKS = ("unet", "controlnet", "vae")
# VAE tensors outside the decoder (vae.py:29-62 builds the full autoencoder).
_VAE_UNUSED_PREFIXES = ("encoder.", "quant_conv_mu.", "quant_conv_log_sigma.")


class InvalidInputError(ValueError):
    """A checkpoint that does not match its network's catalog."""


def network_file(directory: Union[str, Path]) -> Path:
    """The consolidated weights file of a checkpoint directory (``weights.py:33-35``)."""
    return Path(directory) / "model.safetensors"


def production_catalog(network: str) -> list[tuple[str, tuple[int, ...]]]:
    """Torch-layout ``(name, shape)`` inventory of a production network."""
    if network == "unet":
        return maisi.unet_weight_shapes(maisi.PRODUCTION_UNET_CONSTRUCTOR)
    if network == "controlnet":
        return maisi.controlnet_weight_shapes(maisi.PRODUCTION_CONTROLNET_CONSTRUCTOR)
    if network == "vae":
        return maisi.vae_decoder_weight_shapes(maisi.PRODUCTION_VAE_CONSTRUCTOR)
    raise InvalidInputError(f"unknown network {network!r}")


def stored_shape(name: str, torch_shape: Sequence[int]) -> tuple[int, ...]:
    """On-disk shape: rank-5 ``.weight`` tensors are channels-last ``(O, kD, kH, kW, I)``."""
    shape = tuple(int(s) for s in torch_shape)
    if len(shape) == 5 and name.endswith(".weight"):
        return (shape[0], *shape[2:], shape[1])
    return shape


def _require_scale(array: np.ndarray) -> float:
    if array.size != 1:
        raise InvalidInputError(f"scale_factor must be a scalar; got {list(array.shape)}")
    value = float(array.reshape(()))
    if not np.isfinite(value) or value == 0.0:
        raise InvalidInputError("scale_factor must be a finite non-zero checkpoint value")
    return value


def load_network(
    path: Union[str, Path],
    *,
    network: str,
    device: Union[str, torch.device] = "cuda",
    catalog: Optional[Sequence[tuple[str, Sequence[int]]]] = None,
) -> tuple[dict[str, Tensor], Optional[float]]:
    """Load one network (``"unet"``, ``"controlnet"`` or ``"vae"``) from ``path``.

    Returns ``(weights, scale_factor)``: float32 tensors on ``device`` in Torch
    layouts keyed by state-dict name, and the UNet's latent scale (``None`` for
    the other networks).  ``catalog`` overrides the production inventory
    (``(name, torch_shape)`` pairs), e.g. for the small test networks.

    Raises:
        InvalidInputError: wrong suffix, unknown network, a missing, unexpected,
            mis-shaped, non-float32 or non-finite tensor, or a missing/extra
            ``scale_factor``.
    """
    from safetensors import safe_open

    path = Path(path)
    if network not in NETWORKS:
        raise InvalidInputError(f"unknown network {network!r}")
    if path.suffix != ".safetensors":
        raise InvalidInputError(f"{path.name} must be a safetensors file")
    specs = {n: tuple(int(s) for s in shape) for n, shape in (catalog or production_catalog(network))}
    prefix = network + "." if path.name == "model.safetensors" else ""
    weights: dict[str, Tensor] = {}
    scale: Optional[float] = None
    with safe_open(str(path), framework="np") as tensors:
        selected = {k[len(prefix):]: k for k in tensors.keys() if k.startswith(prefix)}
        skipped = set()
        for name in selected:
            if name == "scale_factor" or name in specs:
                continue
            if network == "vae" and name.startswith(_VAE_UNUSED_PREFIXES):
                skipped.add(name)
                continue
            raise InvalidInputError(f"{path.name} has unexpected tensor {name}")
        missing = [n for n in specs if n not in selected]
        if missing:
            raise InvalidInputError(f"{path.name} is missing {missing[0]}")
        if network == "unet":
            if "scale_factor" not in selected:
                raise InvalidInputError(f"{path.name} is missing scale_factor")
            scale = _require_scale(tensors.get_tensor(selected["scale_factor"]))
        elif "scale_factor" in selected:
            raise InvalidInputError(f"{path.name} must not contain scale_factor")
        for name, stored in selected.items():
            if name == "scale_factor":
                continue
            array = tensors.get_tensor(stored)
            if name in skipped:
                if array.dtype != np.float32 or not np.isfinite(array).all():
                    raise InvalidInputError(f"{path.name} tensor {name} must be finite float32")
                continue
            expected = stored_shape(name, specs[name])
            if array.shape != expected or array.dtype != np.float32 or not np.isfinite(array).all():
                raise InvalidInputError(f"{path.name} tensor {name} must be finite float32 with shape "
                                        f"{expected}; got {array.dtype} {array.shape}")
            if array.ndim == 5 and name.endswith(".weight"):
                array = np.transpose(array, (0, 4, 1, 2, 3))
            weights[name] = torch.from_numpy(np.ascontiguousarray(array)).to(device)
            del array
    return weights, scale


def save_network(path: Union[str, Path], weights: Mapping[str, Union[Tensor, np.ndarray]], *,
                 scale_factor: Optional[float] = None, prefix: str = "") -> None:
    """Write Torch-layout weights in the on-disk layout ``load_network`` reads (conv weights
    channels-last), e.g. to hand random-init or converted weights to the loader."""
    from safetensors.numpy import save_file

    out = {}
    for name, value in weights.items():
        array = value.detach().cpu().numpy() if isinstance(value, Tensor) else np.asarray(value)
        array = np.asarray(array, dtype=np.float32)
        if array.ndim == 5 and name.endswith(".weight"):
            array = np.transpose(array, (0, 2, 3, 4, 1))
        out[prefix + name] = np.ascontiguousarray(array)
    if scale_factor is not None:
        out[prefix + "scale_factor"] = np.asarray(scale_factor, dtype=np.float32)
    save_file(out, str(path))
