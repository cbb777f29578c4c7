"""Float64 NumPy restatement of the reference's conv / norm / split-attention math — test
infrastructure only.

Layout: activations NDHWC ``(N, D, H, W, C)`` (the reference is NCDHW; the
math is layout-independent), conv weights Torch ``(O, C, k, k, k)``.
Every function returns float64.
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def conv3d(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None, *, stride: int = 1,
           padding: int | None = None) -> np.ndarray:
    """Cross-correlation of NDHWC ``x`` with ``(O, C, k, k, k)`` weight, float64.

    Follows the reference's float64 test conv (tests/test_fast_fp32.py:21-38):
    pad by ``padding`` (default k // 2), then for each tap (kd, kh, kw) add the
    strided window times ``w[:, :, kd, kh, kw]``.  Output extent per axis is
    ``(n + 2p - k) // stride + 1``.
    """
    x = np.asarray(x, F64)
    w = np.asarray(w, F64)
    k = w.shape[2]
    p = k // 2 if padding is None else padding
    n, d, h, wd, c = x.shape
    xp = np.pad(x, [(0, 0), (p, p), (p, p), (p, p), (0, 0)])
    od, oh, ow = ((s + 2 * p - k) // stride + 1 for s in (d, h, wd))
    out = np.zeros((n, od, oh, ow, w.shape[0]), F64)
    for kd in range(k):
        for kh in range(k):
            for kw in range(k):
                win = xp[:, kd : kd + stride * od : stride, kh : kh + stride * oh : stride,
                         kw : kw + stride * ow : stride, :]
                out += win @ w[:, :, kd, kh, kw].T
    if b is not None:
        b = np.asarray(b, F64)
        out += b.reshape(b.shape[0], 1, 1, 1, -1) if b.ndim == 2 else b
    return out


def conv3d_points(x: np.ndarray, w: np.ndarray, b: np.ndarray | None, points: np.ndarray, *,
                  stride: int = 1, upsample: bool = False, affine: np.ndarray | None = None,
                  apply_silu: bool = False, chunk: int = 512) -> np.ndarray:
    """The padding-``k // 2`` conv of ``conv3d`` evaluated only at output voxels ``points``.

    ``points`` is ``(P, 4)`` integer ``(n, d, h, w)`` output coordinates; the
    result is ``(P, O)`` float64.  The conv input is ``x`` after the optional
    prologue of the reference's pack kernel (_nax_conv.py:174-197):
    ``silu?(x * scale + offset)`` with ``(N, C, 2)`` pairs ``affine``, then the
    optional nearest-2x upsampling (output voxel ``u`` of an axis reads source
    voxel ``u // 2``, test_fast_fp32.py:123-125); the zero padding lies outside
    the transformed (and upsampled) volume.  Used to check full-size volumes
    whose complete float64 convolution would take too long on the CPU.
    """
    x = np.asarray(x)
    w = np.asarray(w, F64)
    pts = np.asarray(points, np.int64)
    k = w.shape[2]
    p = k // 2
    n_, d_, h_, w_, c = x.shape
    extent = np.array([d_, h_, w_]) * (2 if upsample else 1)
    offs = np.arange(k) - p
    out = np.zeros((len(pts), w.shape[0]), F64)
    wk = w.transpose(2, 3, 4, 1, 0).reshape(k * k * k * c, w.shape[0])  # (tap * C + c, O)
    for lo in range(0, len(pts), chunk):
        blk = pts[lo:lo + chunk]
        # (P, k) coordinates per axis on the (upsampled) conv-input grid
        coords = [stride * blk[:, 1 + a, None] + offs[None, :] for a in range(3)]
        valid = [(cc >= 0) & (cc < extent[a]) for a, cc in enumerate(coords)]
        src = [np.clip(cc, 0, extent[a] - 1) // (2 if upsample else 1) for a, cc in enumerate(coords)]
        nn = blk[:, 0, None, None, None]
        patch = np.asarray(x[nn, src[0][:, :, None, None], src[1][:, None, :, None], src[2][:, None, None, :]],
                           F64)  # (P, k, k, k, C)
        if affine is not None:
            a = np.asarray(affine, F64)[blk[:, 0]]  # (P, C, 2)
            patch = patch * a[:, None, None, None, :, 0] + a[:, None, None, None, :, 1]
        if apply_silu:
            patch = silu(patch)
        mask = valid[0][:, :, None, None] & valid[1][:, None, :, None] & valid[2][:, None, None, :]
        patch = patch * mask[..., None]
        out[lo:lo + chunk] = patch.reshape(len(blk), -1) @ wk
    if b is not None:
        b = np.asarray(b, F64)
        out += b[pts[:, 0]] if b.ndim == 2 else b
    return out


def boundary_points(n: int, spatial: tuple[int, int, int], count: int, seed: int) -> np.ndarray:
    """``(P, 4)`` output coordinates covering every corner, the 12 edges and 6 faces of each batch
    item's output volume (three points per edge, eight per face) plus ``count`` random voxels."""
    rng = np.random.default_rng(seed)
    ext = [int(s) for s in spatial]
    picks = []
    for item in range(n):
        for corner in np.ndindex(2, 2, 2):
            picks.append((item, *[(ext[a] - 1) * corner[a] for a in range(3)]))
        for free in range(3):  # edges: one free axis, the others at 0 or max
            for fixed in np.ndindex(2, 2):
                for v in (0, ext[free] // 2, ext[free] - 1):
                    pt, j = [0, 0, 0], 0
                    for a in range(3):
                        if a == free:
                            pt[a] = v
                        else:
                            pt[a] = (ext[a] - 1) * fixed[j]
                            j += 1
                    picks.append((item, *pt))
        for axis in range(3):  # faces
            for side in (0, ext[axis] - 1):
                for _ in range(8):
                    pt = [int(rng.integers(0, e)) for e in ext]
                    pt[axis] = side
                    picks.append((item, *pt))
    rand = np.stack([rng.integers(0, n, count)] + [rng.integers(0, e, count) for e in ext], axis=1)
    return np.concatenate([np.asarray(picks, np.int64), rand.astype(np.int64)])


def gather_points(y: np.ndarray, points: np.ndarray) -> np.ndarray:
    """``(P, C)`` rows of NDHWC ``y`` at ``points``."""
    p = np.asarray(points, np.int64)
    return np.asarray(y[p[:, 0], p[:, 1], p[:, 2], p[:, 3]])


def upsample_nearest(x: np.ndarray) -> np.ndarray:
    """Nearest 2x upsampling of NDHWC ``x`` (repeat each voxel 2x per axis;
    the reference test materializes it the same way, test_fast_fp32.py:123-125)."""
    x = np.asarray(x, F64)
    return x.repeat(2, 1).repeat(2, 2).repeat(2, 3)


def _tri_axis(n_in: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Half-pixel 2x source indices and upper weight per output index:
    src = max(0, o/2 - 1/4), i0 = floor(src), i1 = min(i0 + 1, n - 1)
    (_nax_conv.py:122-128)."""
    o = np.arange(2 * n_in, dtype=F64)
    src = np.maximum(0.0, 0.5 * o - 0.25)
    i0 = np.floor(src).astype(np.int64)
    i1 = np.minimum(i0 + 1, n_in - 1)
    return i0, i1, src - i0


def upsample_trilinear(x: np.ndarray) -> np.ndarray:
    """Trilinear 2x upsampling, align_corners=False, clamped upper neighbours
    (source_vae.upsample_trilinear_ncdhw; formula at _nax_conv.py:115-142)."""
    y = np.asarray(x, F64)
    for axis in (1, 2, 3):
        i0, i1, l1 = _tri_axis(y.shape[axis])
        shape = [1] * y.ndim
        shape[axis] = -1
        l1 = l1.reshape(shape)
        y = np.take(y, i0, axis=axis) * (1.0 - l1) + np.take(y, i1, axis=axis) * l1
    return y


def avg_pool(x: np.ndarray) -> np.ndarray:
    """2x2x2 mean pooling with stride 2 (medmlx_core avg_pool3d_ncdhw as used at
    fast_fp32.py:251-255 and residual.py:93-95)."""
    x = np.asarray(x, F64)
    n, d, h, w, c = x.shape
    x = x[:, : d // 2 * 2, : h // 2 * 2, : w // 2 * 2]
    return x.reshape(n, d // 2, 2, h // 2, 2, w // 2, 2, c).mean(axis=(2, 4, 6))


def fold_upsample_weight(w: np.ndarray) -> np.ndarray:
    """Nearest-2x parity fold of a 3x3x3 weight (_nax_conv.pack_upsample_weight, :407-445).

    Returns ``(8, O, C, 2, 2, 2)``: parity ``pd*4 + ph*2 + pw``, taps ``(td, th, tw)``.
    Per axis, parity 0 taps are ``(k0, k1 + k2)`` and parity 1 taps ``(k0 + k1, k2)``.
    """
    w = np.asarray(w, F64)
    sets = {(0, 0): [0], (0, 1): [1, 2], (1, 0): [0, 1], (1, 1): [2]}
    out = np.zeros((8, w.shape[0], w.shape[1], 2, 2, 2), F64)
    for pd in range(2):
        for ph in range(2):
            for pw in range(2):
                for td in range(2):
                    for th in range(2):
                        for tw in range(2):
                            acc = 0.0
                            for kd in sets[(pd, td)]:
                                for kh in sets[(ph, th)]:
                                    for kw in sets[(pw, tw)]:
                                        acc = acc + w[:, :, kd, kh, kw]
                            out[pd * 4 + ph * 2 + pw, :, :, td, th, tw] = acc
    return out


def conv3d_upsample_folded(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """Conv of the nearest-2x upsampling computed with the parity-folded 2x2x2 filters.

    Output voxel ``2m + p`` (per axis) is the 2x2x2 conv of the zero-padded
    source over padded offsets ``m + p + t``, t in {0, 1} (_nax_conv.py:218-233).
    """
    x = np.asarray(x, F64)
    folded = fold_upsample_weight(w)
    n, d, h, wd, _ = x.shape
    xp = np.pad(x, [(0, 0), (1, 1), (1, 1), (1, 1), (0, 0)])
    out = np.zeros((n, 2 * d, 2 * h, 2 * wd, w.shape[0]), F64)
    for pd in range(2):
        for ph in range(2):
            for pw in range(2):
                f = folded[pd * 4 + ph * 2 + pw]
                acc = np.zeros((n, d, h, wd, w.shape[0]), F64)
                for td in range(2):
                    for th in range(2):
                        for tw in range(2):
                            win = xp[:, pd + td : pd + td + d, ph + th : ph + th + h, pw + tw : pw + tw + wd, :]
                            acc += win @ f[:, :, td, th, tw].T
                out[:, pd::2, ph::2, pw::2, :] = acc
    if b is not None:
        b = np.asarray(b, F64)
        out += b.reshape(b.shape[0], 1, 1, 1, -1) if b.ndim == 2 else b
    return out


def group_norm_affine(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, groups: int,
                      eps: float) -> np.ndarray:
    """``(N, C, 2)`` per-channel (scale, offset) of a group norm of NDHWC ``x``.

    Mean and biased variance per (n, group) over (C/G channels) x voxels
    (tests/test_fast_fp32.py:41-48); scale = gamma / sqrt(var + eps),
    offset = beta - mean * scale (the pair layout of _nax_conv.py:502-504).
    """
    x = np.asarray(x, F64)
    n, c = x.shape[0], x.shape[-1]
    g = x.reshape(n, -1, groups, c // groups)
    mean = g.mean(axis=(1, 3))
    var = g.var(axis=(1, 3))
    rstd = 1.0 / np.sqrt(var + eps)
    scale = np.asarray(gamma, F64)[None, :] * np.repeat(rstd, c // groups, axis=1)
    offset = np.asarray(beta, F64)[None, :] - np.repeat(mean, c // groups, axis=1) * scale
    return np.stack([scale, offset], axis=-1)


def silu(x: np.ndarray) -> np.ndarray:
    """``x / (1 + exp(-x))`` (_nax_conv.py:177)."""
    x = np.asarray(x, F64)
    return x / (1.0 + np.exp(-x))


def group_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, groups: int, eps: float,
               apply_silu: bool = False) -> np.ndarray:
    """Group norm (+ SiLU) of NDHWC ``x`` (tests/test_fast_fp32.py:41-48)."""
    return apply_affine(x, group_norm_affine(x, gamma, beta, groups, eps), apply_silu)


def apply_affine(x: np.ndarray, affine: np.ndarray, apply_silu: bool) -> np.ndarray:
    """``silu?(x * scale + offset)`` with ``(N, C, 2)`` pairs."""
    x = np.asarray(x, F64)
    a = np.asarray(affine, F64)
    n, c = x.shape[0], x.shape[-1]
    y = x * a[..., 0].reshape(n, 1, 1, 1, c) + a[..., 1].reshape(n, 1, 1, 1, c)
    return silu(y) if apply_silu else y


def split_f16(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The reference's split of fp32 values into fp16 halves (_flash_attention.py:314-317, the
    same split as _nax_conv.py:27-35): ``hi = fp16(x)``, ``lo = fp16((x - hi) * 2^11)``, both
    rounded to nearest even; returned as float64 (``x ~ hi + lo * 2^-11``)."""
    x = np.asarray(x, np.float32)
    hi = x.astype(np.float16)
    lo = ((x - hi.astype(np.float32)) * np.float32(2048.0)).astype(np.float16)
    return hi.astype(F64), lo.astype(F64)


def flash_attention_split_f16(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int,
                              scale: float) -> np.ndarray:
    """The reference's split-fp16 multi-head attention (_flash_attention.py:140-290 on the
    operands prepared at :336-350), with exact (float64) sums of its products.

    ``q * (scale * log2 e)`` (an fp32 product), ``k`` and ``v`` are split by ``split_f16``;
    scores are ``qh kh + (qh kl + ql kh) * 2^-11`` in log2 units; ``P = 2^(S - max)`` is
    rounded to fp32 and split the same way, and the output is
    ``(Ph Vh + (Ph Vl + Pl Vh) * 2^-11) / sum(P)`` per head.  ``(B, L, heads * dh)`` arrays.
    """
    q32 = np.asarray(q, np.float32) * np.float32(scale * 1.4426950408889634)
    n, lq, c = q32.shape
    dh = c // heads

    def per_head(t: np.ndarray) -> np.ndarray:
        return t.reshape(n, -1, heads, dh).transpose(0, 2, 1, 3)

    qh, ql = (per_head(t) for t in split_f16(q32))
    kh, kl = (per_head(t).transpose(0, 1, 3, 2) for t in split_f16(k))
    vh, vl = (per_head(t) for t in split_f16(v))
    s = qh @ kh + (qh @ kl + ql @ kh) * 2.0**-11
    p = np.exp2(s - s.max(axis=-1, keepdims=True)).astype(np.float32)
    ph, pl = split_f16(p)
    o = (ph @ vh + (ph @ vl + pl @ vh) * 2.0**-11) / p.astype(F64).sum(axis=-1, keepdims=True)
    return o.transpose(0, 2, 1, 3).reshape(n, lq, c)


def ncdhw_to_ndhwc(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.moveaxis(np.asarray(x), 1, -1))


def ndhwc_to_ncdhw(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(np.moveaxis(np.asarray(x), -1, 1))


def max_rel_error(actual: np.ndarray, expected: np.ndarray) -> float:
    """``max|actual - expected| / max|expected|`` (the per-layer error measure)."""
    expected = np.asarray(expected, F64)
    return float(np.abs(np.asarray(actual, F64) - expected).max() / max(np.abs(expected).max(), 1e-300))
