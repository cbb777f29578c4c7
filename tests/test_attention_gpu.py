"""GPU parity of the HIP flash-attention kernel (``ctmr_flash_attention``).

References: float64 softmax(Q K^T s) V on the CPU for the kernel itself, the
recorded MONAI attention block (tests/golden/maisi/attention.*) for the
residual spatial-attention composition, and the float64 CPU oracle
(oracle/maisi_torch.attention) at the production UNet's attention shapes.
Bar: max relative error (max |a - b| / max |b|) within 1e-5, the FP32
per-layer tolerance; different query tilings are bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_util import load_boundary
from oracle import maisi_torch as mt
from oracle import reference_math as rm

pytestmark = pytest.mark.gpu

FP32_REL = 1e-5


def _ref_attention(q, k, v, heads, scale):
    """float64 multi-head softmax(q k^T * scale) v on (B, L, heads*dh) arrays."""
    n, lq, c = q.shape
    dh = c // heads

    def split(t):
        return torch.from_numpy(t).double().reshape(n, -1, heads, dh).transpose(1, 2)

    s = split(q) @ split(k).transpose(-1, -2) * scale
    out = torch.softmax(s, dim=-1) @ split(v)
    return out.transpose(1, 2).reshape(n, lq, c).numpy()


def _case(seed, n, lq, lk, heads, q_gain=1.0):
    rng = np.random.default_rng(seed)
    c = heads * 32
    q = (rng.standard_normal((n, lq, c)) * q_gain).astype(np.float32)
    k = rng.standard_normal((n, lk, c)).astype(np.float32)
    v = rng.standard_normal((n, lk, c)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize(
    ("seed", "n", "lq", "lk", "heads", "q_gain"),
    [
        (0, 1, 64, 64, 1, 1.0),      # the golden block's shape
        (1, 2, 256, 256, 16, 1.0),   # production deep level (8x8x4 latent, 512 channels)
        (2, 2, 2048, 2048, 8, 1.0),  # production level 2 (16x16x8 latent, 256 channels)
        (3, 1, 100, 77, 3, 1.0),     # ragged query and key counts (masked last key block)
        (4, 2, 33, 130, 2, 8.0),     # cross lengths, large scores (max subtraction)
        (5, 1, 1, 1, 1, 1.0),        # single key
    ],
)
def test_flash_attention_matches_float64(ctmr, dev, seed, n, lq, lk, heads, q_gain):
    print(f"case seed={seed} n={n} lq={lq} lk={lk} heads={heads}", flush=True)
    q, k, v = _case(seed, n, lq, lk, heads, q_gain)
    scale = 32 ** -0.5
    ref = _ref_attention(q, k, v, heads, scale)
    outs = []
    for tiles in (1, 2):
        out = ctmr.fast_fp32.flash_attention(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                             torch.from_numpy(v).to(dev), heads=heads, scale=scale,
                                             query_tiles=tiles)
        outs.append(out.cpu().numpy())
        err = rm.max_rel_error(outs[-1], ref)
        print(f"query_tiles={tiles} max rel error {err:.3e}", flush=True)
        assert err <= FP32_REL
    np.testing.assert_array_equal(outs[0], outs[1])


def _sweep_cases(count, seed):
    """Random shapes around the kernel's block boundaries: key counts that leave the last 32-key block
    full or ragged, an odd or even number of blocks per key part, one or two key parts (at least 128
    keys and a small grid), both query tilings, cross lengths and large score ranges."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        lk = int(rng.choice([int(rng.integers(1, 97)), 32 * int(rng.integers(1, 12)) + int(rng.integers(-1, 2)),
                             int(rng.integers(128, 700))]))
        lk = max(lk, 1)
        lq = int(rng.integers(1, 300))
        cases.append((1000 + i, int(rng.integers(1, 3)), lq, lk, int(rng.integers(1, 6)),
                      float(rng.choice([0.5, 1.0, 4.0]))))
    return cases


@pytest.mark.parametrize(("seed", "n", "lq", "lk", "heads", "q_gain"), _sweep_cases(40, 11),
                         ids=[f"sweep{i:02d}" for i in range(40)])
def test_flash_attention_random_shapes(ctmr, dev, seed, n, lq, lk, heads, q_gain):
    """Seeded sweep: every shape within the FP32 bar of float64 and both query tilings bit-identical."""
    test_flash_attention_matches_float64(ctmr, dev, seed, n, lq, lk, heads, q_gain)


def test_flash_attention_on_fused_projection_views(ctmr, dev):
    """q/k/v as column slices of one (B, L, 3C) projection (row stride 3C), as the UNet calls it."""
    rng = np.random.default_rng(9)
    n, length, heads = 2, 300, 4
    c = heads * 32
    qkv = rng.standard_normal((n, length, 3 * c)).astype(np.float32)
    g = torch.from_numpy(qkv).to(dev)
    out = ctmr.fast_fp32.flash_attention(g[..., :c], g[..., c:2 * c], g[..., 2 * c:], heads=heads, scale=0.2)
    ref = _ref_attention(np.ascontiguousarray(qkv[..., :c]), np.ascontiguousarray(qkv[..., c:2 * c]),
                         np.ascontiguousarray(qkv[..., 2 * c:]), heads, 0.2)
    assert rm.max_rel_error(out.cpu().numpy(), ref) <= FP32_REL
    again = ctmr.fast_fp32.flash_attention(g[..., :c], g[..., c:2 * c], g[..., 2 * c:], heads=heads, scale=0.2)
    assert torch.equal(out, again)


def test_spatial_attention_golden(ctmr, dev):
    """Residual spatial self-attention on the recorded MONAI block (one 32-wide head, 64 tokens)."""
    manifest, a = load_boundary("attention")
    c = manifest["constructor"]
    w = {k[len("weight."):]: torch.from_numpy(v).to(dev) for k, v in a.items() if k.startswith("weight.")}
    x = ctmr.fast_fp32.to_ndhwc(torch.from_numpy(a["x"]).to(dev))
    y = ctmr.maisi.spatial_attention(x, w, num_groups=c["norm_num_groups"], eps=c["norm_eps"],
                                     num_head_channels=c["num_head_channels"], include_fc=c["include_fc"])
    y = ctmr.fast_fp32.to_ncdhw(y).cpu().numpy()
    np.testing.assert_allclose(y, a["y"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize(("shape", "groups"), [((2, 8, 8, 4, 512), 32), ((2, 16, 16, 8, 256), 32)])
def test_spatial_attention_production_shapes_match_oracle(ctmr, dev, shape, groups):
    """The production UNet's attention blocks (32-wide heads) against the float64 oracle."""
    rng = np.random.default_rng(sum(shape))
    c = shape[-1]
    x = rng.standard_normal(shape).astype(np.float32)
    w = {"norm.weight": 1.0 + 0.1 * rng.standard_normal(c), "norm.bias": 0.1 * rng.standard_normal(c)}
    for m in ("q", "k", "v", "out_proj"):
        prefix = f"attn.{m}" if m == "out_proj" else f"attn.to_{m}"
        w[f"{prefix}.weight"] = rng.standard_normal((c, c)) / np.sqrt(c)
        w[f"{prefix}.bias"] = 0.01 * rng.standard_normal(c)
    wg = {k: torch.from_numpy(np.asarray(v, dtype=np.float32)).to(dev) for k, v in w.items()}
    y = ctmr.maisi.spatial_attention(torch.from_numpy(x).to(dev), wg, num_groups=groups, eps=1e-6,
                                     num_head_channels=32, include_fc=True)
    ref = mt.attention(torch.from_numpy(x).double().permute(0, 4, 1, 2, 3),
                       {k: torch.from_numpy(np.asarray(v, dtype=np.float32)).double() for k, v in w.items()},
                       groups, 1e-6, 32, True).permute(0, 2, 3, 4, 1).numpy()
    err = rm.max_rel_error(y.cpu().numpy(), ref)
    print(f"spatial attention {shape}: max rel error {err:.3e}", flush=True)
    assert err <= FP32_REL


@pytest.mark.parametrize(("b", "h", "lq", "lk", "d"), [(2, 4, 96, 80, 32), (1, 2, 40, 40, 16)])
def test_attention_protocol_on_head_major_inputs(ctmr, dev, b, h, lq, lk, d):
    """``fast_fp32.attention`` on (B, H, L, D) heads (the AttentionArithmetic surface): 32-wide heads
    through the flash kernel, other widths through PyTorch's attention, both against float64."""
    rng = np.random.default_rng(b * 100 + d)
    q = rng.standard_normal((b, h, lq, d)).astype(np.float32)
    k = rng.standard_normal((b, h, lk, d)).astype(np.float32)
    v = rng.standard_normal((b, h, lk, d)).astype(np.float32)
    scale = d ** -0.5
    out = ctmr.fast_fp32.attention(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                   torch.from_numpy(v).to(dev), scale=scale)
    s = torch.from_numpy(q).double() @ torch.from_numpy(k).double().transpose(-1, -2).contiguous() * scale
    ref = (torch.softmax(s, dim=-1) @ torch.from_numpy(v).double()).numpy()
    assert rm.max_rel_error(out.cpu().numpy(), ref) <= FP32_REL
    assert ctmr.fast_fp32.kernels_available()
