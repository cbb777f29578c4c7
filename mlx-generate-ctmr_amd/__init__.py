"""ctmr_amd — MI355X-native conv3d + GroupNorm/SiLU hot path of mlx-generate-ctmr.

Modules:
  fast_fp32  the reference's fast-FP32 arithmetic surface (NDHWC-native plus
             ``*_ncdhw`` adapters with the reference's names)
  maisi      UNet / ControlNet / VAE decoder / sliding-window decode / rflow
             sampler composed over fast_fp32 (the callers of the hot path)
  weights    safetensors checkpoints (channels-last conv weights on disk)
  ops        ``torch.library`` custom ops (``ctmr::*``) over the C ABI
  _lib       ctypes binding of ``libctmr_hip.so`` (``include/ctmr.h``)
  _build     hipcc build of the HIP sources for gfx950

The directory name is not a Python identifier; load the package with
``importlib.import_module("mlx-generate-ctmr_amd")`` from the repository root.
"""

from . import _lib, fast_fp32, maisi, ops, weights  # noqa: F401

__all__ = ["_lib", "fast_fp32", "maisi", "ops", "weights"]
