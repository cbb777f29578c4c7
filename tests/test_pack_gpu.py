"""The packed input copy itself (``ctmr_conv3d_pack``) against the float64 oracle.

The pack stage writes the zero-padded NDHWC copy the streaming and bf16 GEMMs read: the source, or its
trilinear-2x upsampling, with the optional group-norm affine and SiLU, rounded to bf16 for bf16 GEMMs.
The host picks one of three kernels for it: the plane-batched pack (channels a multiple of 4, the
affine table 16-byte aligned), the trilinear pack (channels a multiple of 4; runs of 8 cells along z on
large grids, one cell per thread on small ones), and the general per-item pack (everything else).
Each case here checks, on the copy read back from the workspace:

* the interior against ``oracle/reference_math`` (``apply_affine``, ``upsample_trilinear``) in float64:
  fp32 copies within 2e-6 of the volume's largest magnitude; bf16 copies within half a bf16 ulp of the
  value (round to nearest) plus the same fp32 margin;
* the one-voxel halo and the channels past the source's exactly zero (the workspace is filled with a
  non-zero byte pattern first);
* bit-identical repeats, and the general kernel (reached through a misaligned affine table) equal to
  the plane-batched one bit for bit.
"""

from __future__ import annotations

import ctypes
import zlib

import numpy as np
import pytest
import torch

from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

FP32_ABS = 2e-6  # times max |expected|
BF16_REL = 2.0 ** -8  # one bf16 ulp of the value bounds round-to-nearest plus the fp32 margin

CASES = [
    # (name, x shape NDHWC, stride, mode, flags, dtype)
    ("bf16 GN + SiLU, planes batched across batch items", (3, 5, 7, 3, 36), 1, "plain", "affine_silu", "bf16"),
    ("bf16 plain", (2, 9, 10, 11, 64), 1, "plain", "", "bf16"),
    ("bf16 GN, 256 channels", (1, 6, 8, 10, 256), 1, "plain", "affine", "bf16"),
    ("fp32 stride-2 GN + SiLU", (2, 9, 12, 10, 48), 2, "plain", "affine_silu", "fp32"),
    ("fp32 GN + SiLU, 18 channels (general pack)", (2, 6, 7, 5, 18), 2, "plain", "affine_silu", "fp32"),
    ("fp32 trilinear, ragged, one cell per thread", (2, 5, 7, 9, 36), 1, "trilinear", "", "fp32"),
    ("bf16 trilinear, faces only (h 3, w 2)", (1, 17, 3, 2, 44), 1, "trilinear", "", "bf16"),
    ("bf16 trilinear, runs of 8 cells", (2, 22, 62, 62, 64), 1, "trilinear", "", "bf16"),
    ("fp32 trilinear, runs of 8 cells", (1, 30, 62, 62, 64), 1, "trilinear", "", "fp32"),
    ("fp32 trilinear, one cell per thread", (1, 12, 20, 22, 64), 1, "trilinear", "", "fp32"),
]


def _bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def _pack(ctmr, dev, shape, stride, mode, flags, dtype, x, affine_t, offset_floats=0):
    """Run ctmr_conv3d_pack; return the padded copy as float32 NDHWC (cp channels)."""
    L = ctmr._lib
    n, d, h, w, c = shape
    m = L.MODE_TRILINEAR2X if mode == "trilinear" else L.MODE_PLAIN
    f = (L.F_AFFINE if "affine" in flags else 0) | (L.F_SILU if "silu" in flags else 0)
    dt = L.DT_BF16 if dtype == "bf16" else L.DT_F32
    desc = ctmr.ops.make_desc(shape, 64, 3, stride, m, f, dt, 0)
    ws_bytes = L.workspace_bytes(desc)
    ws = torch.full((ws_bytes,), 0x5A, dtype=torch.uint8, device=dev)
    aff_ptr = None
    if f & L.F_AFFINE:
        buf = torch.zeros(affine_t.numel() + 4, device=dev)
        buf[offset_floats:offset_floats + affine_t.numel()] = affine_t.reshape(-1)
        aff_ptr = buf.data_ptr() + 4 * offset_floats
    stream = torch.cuda.current_stream().cuda_stream
    L.check(L.lib().ctmr_conv3d_pack(ctypes.byref(desc), x.data_ptr(), aff_ptr, ws.data_ptr(), ws_bytes, stream),
            "ctmr_conv3d_pack")
    torch.cuda.synchronize()
    s = 2 if mode == "trilinear" else 1
    unit = 32 if dtype == "bf16" else 16
    cp = -(-c // unit) * unit
    dims = (n, s * d + 2, s * h + 2, s * w + 2, cp)
    count = int(np.prod(dims))
    assert ws_bytes >= count * (2 if dtype == "bf16" else 4), "route keeps no packed copy"
    raw = ws.cpu().numpy()
    if dtype == "bf16":
        out = _bf16_to_f32(raw[:2 * count].view(np.uint16))
    else:
        out = raw[:4 * count].view(np.float32).copy()
    return out.reshape(dims), raw[:(2 if dtype == "bf16" else 4) * count].copy()


@pytest.mark.parametrize(("name", "shape", "stride", "mode", "flags", "dtype"), CASES, ids=[c[0] for c in CASES])
def test_packed_copy_matches_oracle(ctmr, dev, name, shape, stride, mode, flags, dtype):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    n, d, h, w, c = shape
    xn = (2 * rng.standard_normal(shape) + 0.5).astype(np.float32)
    affn = np.stack([rng.uniform(0.5, 1.5, (n, c)), rng.standard_normal((n, c))], axis=-1).astype(np.float32)
    x = torch.from_numpy(xn).to(dev)
    affine_t = torch.from_numpy(affn).to(dev)
    got, raw = _pack(ctmr, dev, shape, stride, mode, flags, dtype, x, affine_t)
    _, raw2 = _pack(ctmr, dev, shape, stride, mode, flags, dtype, x, affine_t)
    assert np.array_equal(raw, raw2), f"{name}: repeat differs"

    src = rm.upsample_trilinear(xn) if mode == "trilinear" else np.asarray(xn, np.float64)
    if "affine" in flags:
        src = rm.apply_affine(src, affn, "silu" in flags)
    interior = got[:, 1:-1, 1:-1, 1:-1, :c]
    assert interior.shape == src.shape
    scale = float(np.abs(src).max())
    err = np.abs(interior.astype(np.float64) - src)
    if dtype == "bf16":
        bound = BF16_REL * np.abs(src) + FP32_ABS * scale
    else:
        bound = FP32_ABS * scale
    worst = float((err - bound).max())
    assert worst <= 0.0, f"{name}: packed copy off the oracle by {worst:.3e} beyond the bound"

    halo = got.copy()
    halo[:, 1:-1, 1:-1, 1:-1, :c] = 0.0
    assert not np.any(halo), f"{name}: halo or padding channels not zero"

    if "affine" in flags:
        # a table off 16-byte alignment takes the general per-item pack: same bits
        _, raw_general = _pack(ctmr, dev, shape, stride, mode, flags, dtype, x, affine_t, offset_floats=1)
        assert np.array_equal(raw, raw_general), f"{name}: general pack differs from the plane-batched one"
