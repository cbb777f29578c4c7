"""GPU parity of the split-fp16 flash attention (``ctmr_flash_attention_f16x2``), the
reference's matrix-unit kernel (``_flash_attention.py:140-290``, chosen at :336-350), which
``fast_fp32`` runs under ``precision("f16x2")``.

References: float64 softmax(Q K^T s) V on the CPU (bar 1e-5, the FP32 per-layer tolerance),
the oracle's restatement of the reference's split arithmetic
(``oracle.reference_math.flash_attention_split_f16``: the same fp16 halves and the same three
products per multiply-add, summed in float64; bar 1e-6, which a dropped cross term or an
unsplit operand misses by two orders of magnitude), and the float64 CPU oracle of the
production attention blocks.  Different query tilings are bit-identical.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import maisi_torch as mt
from oracle import reference_math as rm
from test_attention_gpu import _case, _ref_attention, _sweep_cases

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5
SPLIT_REL = 1e-6


def _flash(ctmr, dev, q, k, v, heads, scale, tiles, mode="f16x2"):
    with ctmr.fast_fp32.precision(mode):
        out = ctmr.fast_fp32.flash_attention(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                             torch.from_numpy(v).to(dev), heads=heads, scale=scale,
                                             query_tiles=tiles)
    return out.cpu().numpy()


@pytest.mark.parametrize(
    ("seed", "n", "lq", "lk", "heads", "q_gain"),
    [
        (0, 1, 64, 64, 1, 1.0),      # one 32-wide head, two key blocks
        (1, 2, 256, 256, 16, 1.0),   # production deep level (8x8x4 latent, 512 channels)
        (2, 2, 2048, 2048, 8, 1.0),  # production level 2 (16x16x8 latent, 256 channels): two key parts
        (3, 1, 100, 77, 3, 1.0),     # ragged query and key counts (zero-padded, masked last key block)
        (4, 2, 33, 130, 2, 8.0),     # cross lengths, large scores (max subtraction)
        (5, 1, 1, 1, 1, 1.0),        # single key
    ],
)
def test_split_attention_matches_float64_and_reference_arithmetic(ctmr, dev, seed, n, lq, lk, heads, q_gain):
    print(f"case seed={seed} n={n} lq={lq} lk={lk} heads={heads}", flush=True)
    q, k, v = _case(seed, n, lq, lk, heads, q_gain)
    scale = 32 ** -0.5
    ref = _ref_attention(q, k, v, heads, scale)
    split_ref = rm.flash_attention_split_f16(q, k, v, heads, scale)
    outs = []
    for tiles in (1, 2):
        outs.append(_flash(ctmr, dev, q, k, v, heads, scale, tiles))
        err, err_split = rm.max_rel_error(outs[-1], ref), rm.max_rel_error(outs[-1], split_ref)
        print(f"query_tiles={tiles} vs float64 {err:.3e}, vs the split arithmetic {err_split:.3e}", flush=True)
        assert err <= FP32_REL
        assert err_split <= SPLIT_REL
    np.testing.assert_array_equal(outs[0], outs[1])
    if lk >= 64:
        # the split kernel ran, not the FP32 one
        assert not np.array_equal(outs[1], _flash(ctmr, dev, q, k, v, heads, scale, 2, mode="fp32"))


@pytest.mark.parametrize(("seed", "n", "lq", "lk", "heads", "q_gain"), _sweep_cases(24, 23),
                         ids=[f"sweep{i:02d}" for i in range(24)])
def test_split_attention_random_shapes(ctmr, dev, seed, n, lq, lk, heads, q_gain):
    """Seeded sweep around the block boundaries (full or ragged last key block, one or two key parts,
    both query tilings, cross lengths, large score ranges)."""
    test_split_attention_matches_float64_and_reference_arithmetic(ctmr, dev, seed, n, lq, lk, heads, q_gain)


def test_split_attention_through_c_abi(ctmr, dev, native_loaded):
    """The entry point on fused-projection views (row stride 3C) with a caller workspace of exactly the
    queried size equals the operator's output; one byte less is refused on the host."""
    rng = np.random.default_rng(5)
    n, length, heads = 2, 300, 4
    c = heads * 32
    qkv = torch.from_numpy(rng.standard_normal((n, length, 3 * c)).astype(np.float32)).to(dev)
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    with ctmr.fast_fp32.precision("f16x2"):
        expected = ctmr.fast_fp32.flash_attention(q, k, v, heads=heads, scale=0.2)
    d = ctmr._lib.AttnDesc(n, length, length, heads, 32, 0, 3 * c, 3 * c, 3 * c, c, 0.2)
    nbytes = native_loaded.ctmr_flash_attention_f16x2_workspace_bytes(ctypes.byref(d))
    lkp = (length + 31) // 32 * 32
    assert nbytes == 2 * 2 * n * heads * 32 * (length + 2 * lkp)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty((n, length, c), device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = (ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr())
    assert native_loaded.ctmr_flash_attention_f16x2(*args, nbytes - 1, stream) == -1
    assert "workspace" in ctmr._lib.last_error()
    assert native_loaded.ctmr_flash_attention_f16x2(*args, nbytes, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, expected)
    ref = _ref_attention(*(np.ascontiguousarray(t.cpu().numpy()) for t in (q, k, v)), heads, 0.2)
    assert rm.max_rel_error(out.cpu().numpy(), ref) <= FP32_REL


def test_bf16_precision_keeps_fp32_attention(ctmr, dev):
    """Under ``precision("bf16")`` attention stays on the FP32 kernel (same bits as fp32)."""
    q, k, v = _case(7, 2, 200, 200, 4)
    scale = 32 ** -0.5
    np.testing.assert_array_equal(_flash(ctmr, dev, q, k, v, 4, scale, 0, mode="bf16"),
                                  _flash(ctmr, dev, q, k, v, 4, scale, 0, mode="fp32"))


@pytest.mark.parametrize(("shape", "groups"), [((2, 8, 8, 4, 512), 32), ((2, 16, 16, 8, 256), 32)])
def test_split_spatial_attention_production_shapes_match_oracle(ctmr, dev, shape, groups):
    """The production UNet's attention blocks under ``precision("f16x2")`` against the float64 oracle."""
    rng = np.random.default_rng(sum(shape) + 1)
    c = shape[-1]
    x = rng.standard_normal(shape).astype(np.float32)
    w = {"norm.weight": 1.0 + 0.1 * rng.standard_normal(c), "norm.bias": 0.1 * rng.standard_normal(c)}
    for m in ("q", "k", "v", "out_proj"):
        prefix = f"attn.{m}" if m == "out_proj" else f"attn.to_{m}"
        w[f"{prefix}.weight"] = rng.standard_normal((c, c)) / np.sqrt(c)
        w[f"{prefix}.bias"] = 0.01 * rng.standard_normal(c)
    wg = {k: torch.from_numpy(np.asarray(v, dtype=np.float32)).to(dev) for k, v in w.items()}
    with ctmr.fast_fp32.precision("f16x2"):
        y = ctmr.maisi.spatial_attention(torch.from_numpy(x).to(dev), wg, num_groups=groups, eps=1e-6,
                                         num_head_channels=32, include_fc=True)
    ref = mt.attention(torch.from_numpy(x).double().permute(0, 4, 1, 2, 3),
                       {k: torch.from_numpy(np.asarray(v, dtype=np.float32)).double() for k, v in w.items()},
                       groups, 1e-6, 32, True).permute(0, 2, 3, 4, 1).numpy()
    err = rm.max_rel_error(y.cpu().numpy(), ref)
    print(f"split spatial attention {shape}: max rel error {err:.3e}", flush=True)
    assert err <= FP32_REL
