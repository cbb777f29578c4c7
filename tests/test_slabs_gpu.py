"""Depth-slab execution (``fast_fp32.SLAB_WORKSPACE_BYTES``): a conv whose workspace exceeds the budget runs
in depth slabs with the whole volume's kernel and K split and returns the whole volume's bits -- the
reference's contract for its slabbed packs (``_nax_conv.py:571-573,667-684``), pinned by its
``tests/test_fast_fp32.py:153-216`` (fused norm + SiLU + residual, trilinear packing, a small grid with a
tap split), restated here over this library's routes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


CASES = [
    # (name, x shape, second-source channels, cout, keyword arguments, dtype, slabbed)
    ("fp32 LDS GEMM, GN + SiLU + residual + per-batch bias", (2, 20, 64, 64, 64), 0, 64,
     {"fused": True, "batch_bias": True}, "fp32", True),
    ("fp32 streaming GEMM over the packed copy", (1, 18, 32, 32, 64), 0, 64,
     {"fused": True, "stream_gemm": True}, "fp32", True),
    ("trilinear-2x packing", (1, 10, 8, 8, 32), 0, 32, {"trilinear": True}, "fp32", True),
    ("small grid with a K split", (1, 8, 8, 8, 256), 0, 256, {"fused": True}, "fp32", None),
    ("bf16 LDS GEMM", (1, 16, 32, 32, 64), 0, 64, {"fused": True, "batch_bias": True}, "bf16", True),
    ("split fp16 LDS GEMM", (1, 16, 32, 32, 64), 0, 64, {"fused": True}, "f16x2", True),
    ("two-source input", (2, 16, 32, 32, 64), 32, 64, {"fused": True}, "fp32", True),
    ("1x1x1 over a GN + SiLU pack", (1, 16, 32, 32, 128), 0, 64, {"fused": True, "ksize": 1}, "fp32", True),
]


@pytest.mark.parametrize(("name", "shape", "cin2", "cout", "kw", "dtype", "slabbed"), CASES,
                         ids=[c[0] for c in CASES])
def test_depth_slabs_match_whole_volume(ctmr, dev, monkeypatch, name, shape, cin2, cout, kw, dtype, slabbed):
    print(f"case {name}: {shape} + {cin2} -> {cout}, {kw}, {dtype}", flush=True)
    f, ops = ctmr.fast_fp32, ctmr.ops
    kw = dict(kw)
    fused, batch_bias, ksize = kw.pop("fused", False), kw.pop("batch_bias", False), kw.pop("ksize", 3)
    trilinear = kw.get("trilinear", False)
    rng = np.random.default_rng(sum(shape) + cout)
    n, d = shape[0], shape[1]
    x = _t((3 * rng.standard_normal(shape) + 1).astype(np.float32), dev)
    x2 = _t(rng.standard_normal((*shape[:-1], cin2)).astype(np.float32), dev) if cin2 else None
    cin = shape[-1] + cin2
    w = _t((rng.standard_normal((cout, cin, ksize, ksize, ksize)) / np.sqrt(ksize ** 3 * cin)).astype(np.float32), dev)
    bias = _t(rng.standard_normal((n, cout) if batch_bias else cout).astype(np.float32), dev)
    affine = residual = None
    scale = 2 if trilinear else 1
    if fused:
        gamma = _t((1 + 0.1 * rng.standard_normal(cin)).astype(np.float32), dev)
        beta = _t((0.1 * rng.standard_normal(cin)).astype(np.float32), dev)
        xin = f.ChannelCat(x, x2) if x2 is not None else x
        affine = f.group_norm_affine(xin, gamma, beta, groups=8, eps=1e-6)
        out_shape = (n, scale * d, *(scale * v for v in shape[2:4]), cout)
        residual = _t(rng.standard_normal(out_shape).astype(np.float32), dev)
    packed = f.pack_weight(w, dtype=dtype)
    xin = f.ChannelCat(x, x2) if x2 is not None else x
    call = dict(cout=cout, ksize=ksize, affine=affine, silu=fused, residual=residual, **kw)

    monkeypatch.setattr(f, "SLAB_WORKSPACE_BYTES", None)
    whole = f.implicit_gemm_conv3d(xin, packed, bias, **call)
    flags = ops._flags(affine is not None, fused, batch_bias, residual is not None)
    flags |= ctmr._lib.F_STREAM if kw.get("stream_gemm") else 0
    desc = ops.make_desc(tuple(x.shape), cout, ksize, 1, ctmr._lib.MODE_TRILINEAR2X if trilinear else 0, flags,
                         f._PACKED_DTYPES[packed.dtype], 0, cin2)
    ws = ctmr._lib.workspace_bytes(desc)
    assert ws > 0
    # a budget for slabs of about four input planes
    monkeypatch.setattr(f, "SLAB_WORKSPACE_BYTES", max(1, ws // d * 6))
    calls = {"n": 0}
    real = ops.conv3d

    def counted(*args, **kwargs):
        calls["n"] += 1
        return real(*args, **kwargs)

    monkeypatch.setattr(ops, "conv3d", counted)
    slabs = f.implicit_gemm_conv3d(xin, packed, bias, **call)
    print(f"{name}: route {ctmr._lib.conv_kernel(desc)}, split {ctmr._lib.conv_split(desc)}, "
          f"{calls['n']} slab launches", flush=True)
    if slabbed:
        assert calls["n"] > 1, "the budget should have split this conv into slabs"
    assert tuple(slabs.shape) == tuple(whole.shape)
    assert torch.equal(slabs, whole), "a slabbed conv must return the whole volume's bits"
