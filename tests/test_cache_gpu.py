"""GPU tests of the derived-weight caches (packed conv weights, fused Q/K/V, stacked time
projections) and of what a recorded UNet graph holds on to.

The reference keys its packed-weight cache by ``id`` with weak-reference eviction and drops it
after sampling (fast_fp32.py:70-91, from_mask.py:240).  Torch tensors, unlike MLX arrays, change
in place, so here every cache entry is also validated on each source tensor's ``_version``.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from golden_util import load_boundary, load_fixture
from oracle import maisi_torch as mt
from oracle import reference_math as rm

pytestmark = pytest.mark.gpu


def _g(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dtype)


def _h(t):
    return t.detach().cpu().numpy()


def test_inplace_weight_update_repacks(ctmr, dev):
    """A conv weight changed in place (``copy_``) is packed again: the output follows the new weight."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(50)
    x = rng.standard_normal((1, 6, 8, 8, 64)).astype(np.float32)
    w1 = (rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    w2 = (rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    xg, wg, bg = _g(x, dev), _g(w1, dev), _g(b, dev)
    y1 = _h(f.conv3d(xg, wg, bg, padding=1))
    assert rm.max_rel_error(y1, rm.conv3d(x, w1, b)) <= 1e-5
    wg.copy_(_g(w2, dev))
    y2 = _h(f.conv3d(xg, wg, bg, padding=1))
    assert rm.max_rel_error(y2, rm.conv3d(x, w2, b)) <= 1e-5
    with f.precision("bf16"):  # the bf16 packing is its own entry, built from the current values
        y3 = _h(f.conv3d(xg, wg, bg, padding=1))
    assert rm.max_rel_error(y3, rm.conv3d(x, w2, b)) <= 2e-2


def test_inplace_qkv_bias_update_refuses_stale_fusion(ctmr, dev):
    """The fused Q/K/V projection includes the biases: q and v biases changed in place are fused again."""
    manifest, a = load_boundary("attention")
    c = manifest["constructor"]
    weights = {k[len("weight."):]: _g(v, dev) for k, v in a.items() if k.startswith("weight.")}
    m = ctmr.maisi
    x = m.ff.to_ndhwc(_g(a["x"], dev))
    run = lambda: _h(m.ff.to_ncdhw(m.spatial_attention(x, weights, num_groups=c["norm_num_groups"],
                                                        eps=c["norm_eps"], num_head_channels=c["num_head_channels"],
                                                        include_fc=c.get("include_fc", True))))
    np.testing.assert_allclose(run(), a["y"], rtol=1e-4, atol=1e-5)
    host = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in
            ((k[len("weight."):], v) for k, v in a.items() if k.startswith("weight."))}
    for key, delta in (("attn.to_q.bias", 2.0), ("attn.to_v.bias", 0.5)):
        weights[key].add_(delta)
        host[key] = host[key] + delta
    with torch.no_grad():
        ref = mt.attention(torch.from_numpy(np.asarray(a["x"], np.float64)), host, c["norm_num_groups"], c["norm_eps"],
                           c["num_head_channels"], c.get("include_fc", True)).numpy()
    got = run()
    assert np.abs(got - a["y"]).max() > 1e-3  # the update changed the output
    assert rm.max_rel_error(got, ref) <= 1e-5


def test_inplace_time_projection_bias_update(ctmr, dev):
    """The stacked time projections fold in ``time_emb_proj.bias`` and ``conv1.conv.bias``: both are
    sources of the cache entry, so in-place updates reach the UNet output (tiny golden UNet)."""
    m = ctmr.maisi
    manifest, a = load_boundary("diffusion")
    ctor = manifest["constructor"]
    f = load_fixture("unet.npz")
    w = {k[len("weight."):]: _g(v, dev) for k, v in f.items() if k.startswith("weight.")}
    host = {k[len("weight."):]: torch.from_numpy(np.asarray(v, np.float64)) for k, v in f.items()
            if k.startswith("weight.")}
    args = (_g(a["x"], dev), _g(a["timesteps"], dev), _g(a["class_labels"], dev, torch.int64), _g(a["spacing"], dev))
    y0 = _h(m.denoise_unet_ncdhw(*args, w, constructor=ctor)[1])
    # per-channel deltas (a uniform shift of every channel of a group is removed by norm2)
    for name, lo, hi in (("down_blocks.0.resnets.0.time_emb_proj.bias", -0.5, 0.75),
                         ("down_blocks.0.resnets.0.conv1.conv.bias", 0.6, -0.4)):
        delta = np.linspace(lo, hi, int(w[name].numel()))
        w[name].add_(torch.from_numpy(delta.astype(np.float32)).to(dev))
        host[name] = host[name] + torch.from_numpy(delta)
    y1 = _h(m.denoise_unet_ncdhw(*args, w, constructor=ctor)[1])
    with torch.no_grad():
        _, ref = mt.unet(torch.from_numpy(np.asarray(a["x"], np.float64)),
                         torch.from_numpy(np.asarray(a["timesteps"], np.float64)), torch.from_numpy(a["class_labels"]),
                         torch.from_numpy(np.asarray(a["spacing"], np.float64)), host, ctor)
    assert np.abs(y1 - y0).max() > 1e-4
    assert rm.max_rel_error(y1, ref.numpy()) <= 1e-4


def test_drop_packed_weights_and_eviction(ctmr, dev):
    """``drop_packed_weights`` removes every entry derived from the given weights (a later call packs
    again, same bits); a weight that is collected is evicted by its weak reference."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(51)
    x = _g(rng.standard_normal((1, 4, 8, 8, 32)).astype(np.float32), dev)
    w = _g((rng.standard_normal((32, 32, 3, 3, 3)) / np.sqrt(27 * 32)).astype(np.float32), dev)
    b = _g(rng.standard_normal(32).astype(np.float32), dev)
    before = f.cache_size()
    y = f.conv3d(x, w, b, padding=1)
    assert f.cache_size() == before + 1
    f.conv3d(x, w, b, padding=1)  # a hit: no new entry
    assert f.cache_size() == before + 1
    f.drop_packed_weights([w])
    assert f.cache_size() == before
    assert torch.equal(f.conv3d(x, w, b, padding=1), y)
    assert f.cache_size() == before + 1
    del w
    gc.collect()
    assert f.cache_size() == before


def test_graph_keeps_cached_weights_after_drop(ctmr, dev):
    """A recorded UNet pass keeps references to the cached tensors its kernels read: after
    ``drop_packed_weights`` on every weight, ``empty_cache`` and new allocations filled with other
    data, replays still equal the eager pass bit for bit."""
    m, f = ctmr.maisi, ctmr.fast_fp32
    uc = m.PRODUCTION_UNET_CONSTRUCTOR
    host = m.random_weights(m.unet_weight_shapes(uc), seed=7)
    w = {k: _g(v, dev) for k, v in host.items()}
    rng = np.random.default_rng(52)
    x = _g(rng.standard_normal((2, 16, 16, 16, 4)).astype(np.float32), dev)
    t = torch.tensor([300.0, 300.0], device=dev)
    cls = torch.tensor([9, 0], device=dev)
    sp = m.spacing_tensor([1.0, 1.0, 1.2], device=dev).repeat(2, 1)
    graph = m.UNetGraph(x, t, cls, sp, w, constructor=uc)
    _, eager = m.denoise_unet(x, t, cls, sp, w, constructor=uc)
    eager = eager.clone()
    f.drop_packed_weights(list(w.values()))
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 22,), float(i) + 0.5, device=dev) for i in range(64)]  # reuse freed blocks
    torch.cuda.synchronize()
    for _ in range(3):
        _, y = graph(x, t, cls, sp)
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    del junk


def test_inference_mode_weights_and_residual_block(ctmr, dev):
    """Weights created under ``torch.inference_mode`` (inference tensors have no version counter)
    pack and cache; a residual block run under inference mode (its outputs are inference tensors,
    so no epilogue statistics ride on them and each group norm makes its own pass) matches the same
    block run outside it."""
    f = ctmr.fast_fp32
    rng = np.random.default_rng(58)
    c = 64
    x = _g(rng.standard_normal((1, 6, 8, 8, c)).astype(np.float32), dev)
    emb = _g(rng.standard_normal((1, 32)).astype(np.float32), dev)
    arrays = {
        "norm1.weight": 1 + 0.1 * rng.standard_normal(c), "norm1.bias": 0.1 * rng.standard_normal(c),
        "norm2.weight": 1 + 0.1 * rng.standard_normal(c), "norm2.bias": 0.1 * rng.standard_normal(c),
        "conv1.conv.weight": rng.standard_normal((c, c, 3, 3, 3)) / np.sqrt(27 * c),
        "conv1.conv.bias": 0.01 * rng.standard_normal(c),
        "conv2.conv.weight": rng.standard_normal((c, c, 3, 3, 3)) / np.sqrt(27 * c),
        "conv2.conv.bias": 0.01 * rng.standard_normal(c),
        "time_emb_proj.weight": rng.standard_normal((c, 32)) / np.sqrt(32),
        "time_emb_proj.bias": 0.01 * rng.standard_normal(c),
    }
    plain = {k: _g(v.astype(np.float32), dev) for k, v in arrays.items()}
    want = f.residual_block(x, emb, plain, num_groups=32, eps=1e-6)
    with torch.inference_mode():
        inf = {k: _g(v.astype(np.float32), dev) for k, v in arrays.items()}
        assert all(t.is_inference() for t in inf.values())
        got = f.residual_block(x, emb, inf, num_groups=32, eps=1e-6)
        again = f.residual_block(x, emb, inf, num_groups=32, eps=1e-6)  # cache hits on inference tensors
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    scale = float(want.abs().max())
    assert float((got - want).abs().max()) <= 1e-6 * scale
