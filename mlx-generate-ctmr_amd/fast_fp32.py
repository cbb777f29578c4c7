"""Fast FP32 arithmetic for the MAISI UNet, ControlNet and VAE decoder on MI355X.

Drop-in counterpart of the reference's arithmetic plug-in
``src/mlx_generate_ctmr/fast_fp32.py`` (entry points at :102-349) and of the
kernel orchestrator ``_nax_conv.nax_conv3d`` (``_nax_conv.py:475-684``), with
tensors held by PyTorch-ROCm on the GPU and every hot operation running in the
hand-written HIP kernels of ``libctmr_hip.so``:

* padding-1 3x3x3 convolutions (stride 1/2, nearest-2x folded into parity
  weights, trilinear-2x computed while packing the input) and 1x1x1
  convolutions are implicit GEMMs on FP32 MFMA (or bf16 MFMA with fp32
  accumulation inside ``precision("bf16")``, or split fp16 -- the reference's
  "exact" mode for fp32 tensors, _nax_conv.py:27-35 -- on fp16 MFMA inside
  ``precision("f16x2")``);
* a preceding group norm + SiLU is applied while packing the convolution
  input; bias, the residual block's per-batch time-embedding bias and the
  residual join the fp32 sum before the single store;
* group-norm statistics are a deterministic fp64 reduction.

The native activation layout is NDHWC (``(N, D, H, W, C)`` contiguous).  The
reference's NCDHW entry points (``*_ncdhw``, same names and keywords; the
``mx`` argument is accepted and ignored) permute to NDHWC and back.
Weights keep the Torch layouts the reference uses: conv ``(O, C, k, k, k)``,
linear ``(O, I)``.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
import math
import threading
import weakref
from collections.abc import Iterable, Iterator, Mapping
from contextvars import ContextVar
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib, ops

# ---------------------------------------------------------------------------
# precision selection (the reference's request-scoped arithmetic switch,
# arithmetic_mode.py:28-60, reduced to the MFMA variants of this path)
# ---------------------------------------------------------------------------
PRECISIONS = ("fp32", "bf16", "f16x2")
_DTYPE_CODES = {"fp32": _lib.DT_F32, "bf16": _lib.DT_BF16, "f16x2": _lib.DT_F16X2}
_PACKED_DTYPES = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16X2}
_precision: ContextVar[str] = ContextVar("ctmr_precision", default="fp32")


@contextlib.contextmanager
def precision(mode: str) -> Iterator[None]:
    """Select ``"fp32"`` (FP32 MFMA), ``"bf16"`` (bf16 MFMA, fp32 accumulate) or ``"f16x2"`` convs.

    ``"f16x2"`` is the reference's exact mode for fp32 tensors (``_nax_conv.py:27-35``): each fp32
    value is split into an fp16 high half and an fp16 low half scaled by 2^11, weights are scaled per
    output column by a power of two, and every product is summed as hi*hi + lo*hi + hi*lo on fp16
    MFMA with fp32 accumulation (about 2^-22 relative per product).  It applies to the stride-1
    3x3x3 convs the LDS-staged 16-bit GEMM takes (cout a multiple of 64, at least 16 input
    channels) and to flash attention (the reference's split-fp16 kernel, ``_flash_attention.py:
    140-290``); every other conv runs on FP32 MFMA.  Values must stay below 65504 in magnitude."""
    if mode not in PRECISIONS:
        raise ValueError(f"precision must be one of {PRECISIONS}; got {mode!r}")
    token = _precision.set(mode)
    try:
        yield
    finally:
        _precision.reset(token)


def active_precision() -> str:
    return _precision.get()


def _dtype_code() -> int:
    return _DTYPE_CODES[_precision.get()]


# ---------------------------------------------------------------------------
# validation helpers
# ---------------------------------------------------------------------------
def _require(x: Tensor, name: str, ndim: int = 5) -> Tensor:
    if not isinstance(x, Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if x.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D; got shape {tuple(x.shape)}")
    if x.dtype != torch.float32:
        raise ValueError(f"{name} must be float32; got {x.dtype}")
    if x.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (there is no CPU path); got {x.device}")
    return x.contiguous()


class ChannelCat:
    """The channel concatenation of two NDHWC fp32 tensors on the same voxels, never materialised.

    The up path of the diffusion UNet concatenates its hidden state with a skip before every residual
    block (``unet.py:444``); the block's group norm, 3x3x3 conv and 1x1x1 skip projection read each
    channel block from its own tensor instead (``ctmr_gn_affine_cat``, ``ctmr_conv3d_cat``), with the
    same values in the same order, so the results equal those on ``torch.cat`` bit for bit.  Both
    channel counts must be multiples of 16; ``materialize()`` returns the concatenated tensor for
    consumers that need one.
    """

    __slots__ = ("first", "second")

    def __init__(self, first: Tensor, second: Tensor):
        first, second = _require(first, "first"), _require(second, "second")
        if tuple(first.shape[:-1]) != tuple(second.shape[:-1]):
            raise ValueError(f"concatenated tensors differ in voxels: {tuple(first.shape)} vs {tuple(second.shape)}")
        if first.device != second.device:
            raise ValueError("concatenated tensors are on different devices")
        if int(first.shape[-1]) % 16 or int(second.shape[-1]) % 16:
            raise ValueError("concatenated channel counts must be multiples of 16; got "
                             f"{int(first.shape[-1])} and {int(second.shape[-1])}")
        self.first, self.second = first, second

    @property
    def shape(self) -> torch.Size:
        return torch.Size((*self.first.shape[:-1], int(self.first.shape[-1]) + int(self.second.shape[-1])))

    @property
    def device(self) -> torch.device:
        return self.first.device

    def materialize(self) -> Tensor:
        return torch.cat([self.first, self.second], dim=-1)


def concat_channels(first: Tensor, second: Tensor):
    """``ChannelCat(first, second)`` when both channel counts are multiples of 16 (the two-source
    kernels' channel blocks), else the materialised ``torch.cat``."""
    if int(first.shape[-1]) % 16 == 0 and int(second.shape[-1]) % 16 == 0:
        return ChannelCat(first, second)
    return torch.cat([first, second], dim=-1)


def _split_input(x, name: str = "x") -> tuple[Tensor, Optional[Tensor]]:
    """``(x, None)`` for a tensor, ``(first, second)`` for a ``ChannelCat``."""
    if isinstance(x, ChannelCat):
        return x.first, x.second
    return _require(x, name), None


def _vec(t: Optional[Tensor], n: int, name: str, device: torch.device) -> Optional[Tensor]:
    if t is None:
        return None
    t = t.to(device=device, dtype=torch.float32).contiguous()
    if t.shape[-1] != n:
        raise ValueError(f"{name} last axis {t.shape[-1]} != {n}")
    return t


# ---------------------------------------------------------------------------
# derived-weight caches (fast_fp32.py:70-91): keyed by the ids of every source
# tensor (weights and biases) plus the mode/dtype; an entry is valid while weak
# references to the same source objects are alive and each source's
# ``_version`` is what it was when the entry was built (torch tensors, unlike
# MLX arrays, can change in place: ``copy_`` or an in-place reload bumps it).
# ---------------------------------------------------------------------------
_packed: dict[tuple, tuple[tuple[weakref.ref, ...], tuple[int, ...], Tensor]] = {}
_packed_lock = threading.RLock()  # re-entrant: a weakref eviction may run inside a locked section
_retained = threading.local()


def _version(t: Tensor) -> int:
    """``t._version``, or -1 for an inference tensor (created under ``torch.inference_mode``), which
    has no version counter; such a tensor cannot be modified in place outside inference mode."""
    return -1 if t.is_inference() else t._version


def _sources_match(refs: tuple[weakref.ref, ...], versions: tuple[int, ...], sources: tuple[Tensor, ...]) -> bool:
    return all(r() is t and v == _version(t) for r, v, t in zip(refs, versions, sources))


def _note_use(*derived: Optional[Tensor]) -> None:
    """Record derived tensors handed to a kernel while ``retain_cached`` is active."""
    sink = getattr(_retained, "sink", None)
    if sink is not None:
        sink.extend(t for t in derived if t is not None)


@contextlib.contextmanager
def retain_cached(sink: list) -> Iterator[list]:
    """Collect into ``sink`` every cached derived tensor (packed conv weights, fused Q/K/V
    projections, stacked time projections) used on this thread while the context is active.
    A recorded HIP graph keeps such a list so its kernels' weight addresses stay valid even
    after ``drop_packed_weights`` or a cache refresh releases the cache's own reference."""
    previous = getattr(_retained, "sink", None)
    _retained.sink = sink
    try:
        yield sink
    finally:
        _retained.sink = previous


def cached_derived(cache: dict, lock: threading.Lock, key: tuple, sources: tuple[Tensor, ...], build):
    """The cache entry for ``key`` built from ``sources`` by ``build()``, rebuilt when a source was
    collected, replaced or modified in place since.  ``build`` returns a tensor or a tuple whose
    tensors are the derived data (recorded for ``retain_cached``)."""
    with lock:
        hit = cache.get(key)
        if hit is not None and _sources_match(hit[0], hit[1], sources):
            _note_use(*(hit[2] if isinstance(hit[2], tuple) else (hit[2],)))
            return hit[2]
    value = build()

    def _evict(_ref, key=key):
        with lock:
            cache.pop(key, None)

    with lock:
        cache[key] = (tuple(weakref.ref(t, _evict) for t in sources), tuple(_version(t) for t in sources), value)
    _note_use(*(value if isinstance(value, tuple) else (value,)))
    return value


def pack_weight(weight: Tensor, *, dtype: Optional[str] = None) -> Tensor:
    """Packed ``(O, C, k, k, k)`` weight for ``implicit_gemm_conv3d`` (``_nax_conv.pack_weight``);
    ``dtype`` one of ``PRECISIONS`` (default: the active precision)."""
    code = _DTYPE_CODES[dtype or _precision.get()]
    w = weight.to(torch.float32).contiguous()
    o, c, k = int(w.shape[0]), int(w.shape[1]), int(w.shape[2])
    return ops.pack_weight(w, c, o, k, _lib.MODE_PLAIN, code)


def pack_upsample_weight(weight: Tensor, *, dtype: Optional[str] = None) -> Tensor:
    """Eight 2x2x2 nearest-2x parity filters folded in fp32 (``_nax_conv.pack_upsample_weight``)."""
    code = _DTYPE_CODES[dtype or _precision.get()]
    w = weight.to(torch.float32).contiguous()
    if tuple(w.shape[2:]) != (3, 3, 3):
        raise ValueError("upsample packing needs a 3x3x3 weight")
    return ops.pack_weight(w, int(w.shape[1]), int(w.shape[0]), 3, _lib.MODE_NEAREST2X, code)


def _keeps_fp32(weight: Tensor) -> bool:
    """Convs that stay fp32 under ``precision("bf16")``, where the bf16 form costs more than it saves:
    every bf16 GEMM reads a bf16 copy of its input made by a conversion pass.

    * 1x1x1 convs: the pass costs more than the fp32 GEMM it would speed up (the UNet's skip
      projections read their input once, at 2 MFLOP per byte moved);
    * at most 4 output channels (the UNet and VAE output convs): the fp32 direct kernel (GN affine +
      SiLU staged, VALU FMAs) takes 77 us at the UNet's 2x64x64x32 and 0.63 ms at the decoder's
      80x256x256, where the bf16 tap-expanded GEMM, its tap sum and the pass take ~0.1 and ~0.9 ms;
    * at most 8 input channels (the 4-channel input convs, the condition encoder's 8-channel convs):
      the fp32 LDS-staged im2col GEMM takes 53 us for the UNet's conv_in, the bf16 im2col rows and
      GEMM 130 us."""
    if weight.dim() != 5:
        return False
    o, c, k = (int(v) for v in weight.shape[:3])
    return k == 1 or o <= 4 or c <= 8


_split_routes: dict[tuple, bool] = {}


def _f16x2_route(x_shape: tuple[int, ...], cout: int, mode: int, stride: int, cin2: int) -> bool:
    """Whether a conv of this shape runs on the split-fp16 GEMM (``ctmr_conv3d_kernel`` accepts the
    descriptor with ``CTMR_F16X2``); a function of the shape only, cached."""
    key = (x_shape, cout, mode, stride, cin2)
    hit = _split_routes.get(key)
    if hit is None:
        desc = ops.make_desc(x_shape, cout, 3, stride, mode, 0, _lib.DT_F16X2, 0, cin2)
        hit = _lib.lib().ctmr_conv3d_kernel(ctypes.byref(desc)) == _lib.K_LDS_F16X2
        _split_routes[key] = hit
    return hit


def _pack(weight: Tensor, mode: int, x=None, stride: int = 1) -> Tensor:
    """Packed weight for the active precision (``_keeps_fp32`` convs stay fp32 under bf16; under
    f16x2 only convs of ``x``'s shape that the split-fp16 GEMM takes are packed for it)."""
    if not isinstance(weight, Tensor) or weight.device.type != "cuda":
        raise ValueError("conv weight must be a torch.Tensor on the GPU (there is no CPU path)")
    code = _lib.DT_F32 if _keeps_fp32(weight) else _dtype_code()
    if code == _lib.DT_F16X2:
        first, second = (x.first, x.second) if isinstance(x, ChannelCat) else (x, None)
        ok = (first is not None and weight.dim() == 5 and int(weight.shape[2]) == 3 and
              _f16x2_route(tuple(int(v) for v in first.shape), int(weight.shape[0]), mode, stride,
                           0 if second is None else int(second.shape[-1])))
        if not ok:
            code = _lib.DT_F32
    dtype = {v: k for k, v in _DTYPE_CODES.items()}[code]
    packer = pack_upsample_weight if mode == _lib.MODE_NEAREST2X else pack_weight
    return cached_derived(_packed, _packed_lock, ("conv", mode, code, id(weight)), (weight,),
                          lambda: packer(weight, dtype=dtype))


def drop_packed_weights(weights: Iterable[Tensor]) -> None:
    """Forget every cached tensor derived from ``weights`` (packed conv weights, fused Q/K/V
    projections); a later use derives them again.  A recorded graph that used them keeps its
    own references (``retain_cached``), so its replays stay valid."""
    ids = {id(w) for w in weights}
    for cache, lock in _caches:
        with lock:
            for key in [k for k, entry in cache.items() if any(id(r()) in ids for r in entry[0] if r() is not None)]:
                del cache[key]


def register_cache(cache: dict, lock) -> None:
    """Add a ``cached_derived`` cache to those ``drop_packed_weights`` and ``cache_size`` cover."""
    _caches.append((cache, lock))


def cache_size() -> int:
    """Number of live derived-weight cache entries (every registered cache)."""
    total = 0
    for cache, lock in _caches:
        with lock:
            total += len(cache)
    return total


# ---------------------------------------------------------------------------
# NDHWC-native operators
# ---------------------------------------------------------------------------
# Largest conv workspace (padded input copy + split partial planes) built at once,
# or None: no limit (the default; one MI355X holds 288 GB).  Above it a stride-1
# conv runs in depth slabs with the whole volume's kernel and split, so it returns
# the whole volume's bits (the reference's _SLAB_PACK_BYTES, _nax_conv.py:348-349,
# 667-684, fixed at 512 MiB there for unified-memory Macs).
SLAB_WORKSPACE_BYTES: Optional[int] = None


def _slabs(x: Tensor, x2: Optional[Tensor], *, cout: int, ksize: int, mode: int, flags: int, code: int, split: int,
           budget: int):
    """Plan of a depth-slabbed conv: ``(split, [(input planes a:b, kept input planes s0:s1)], extra flags)``, or None
    when no slab depth keeps the whole volume's kernel and split for every slab (each output's summation
    order is fixed by those two: the slabs then give the whole volume's bits)."""
    n, d, h, w, c1 = (int(v) for v in x.shape)
    cin2 = 0 if x2 is None else int(x2.shape[-1])
    whole = ops.make_desc(tuple(x.shape), cout, ksize, 1, mode, flags, code, split, cin2)
    route, whole_split = _lib.conv_kernel(whole), _lib.conv_split(whole)
    if route == "split_waves":  # a form the library picks by its own policy only: request it explicitly
        flags |= _lib.F_SPLIT_WAVES
    halo = 1 if ksize == 3 else 0
    per_plane = max(1, _lib.workspace_bytes(whole) // d)
    depth = max(1, budget // per_plane - 2 * halo)
    for depth in range(min(depth, d - 1), 0, -1):
        plan = []
        for s0 in range(0, d, depth):
            s1 = min(d, s0 + depth)
            a, b = max(s0 - halo, 0), min(s1 + halo, d)
            desc = ops.make_desc((n, b - a, h, w, c1), cout, ksize, 1, mode, flags, code, whole_split, cin2)
            try:
                same = _lib.conv_kernel(desc) == route and _lib.conv_split(desc) == whole_split
            except _lib.CtmrError:
                same = False
            if not same:
                break
            plan.append((a, b, s0, s1))
        else:
            return whole_split, plan, flags & _lib.F_SPLIT_WAVES
    return None


def _conv_in_slabs(x, x2, packed, bias, affine, residual, out_shape, *, cout, ksize, mode, silu, code, split,
                   stream_gemm, scale: int, plan, flags: int) -> Tensor:
    """Run ``plan`` (``_slabs``): each slab convolves its input planes with a one-plane halo and keeps the
    planes whose halo is real data (``scale`` output planes per input plane for trilinear-2x)."""
    y = torch.empty(out_shape, device=x.device, dtype=torch.float32)
    for a, b, s0, s1 in plan:
        xs = x[:, a:b].contiguous()
        xs2 = None if x2 is None else x2[:, a:b].contiguous()
        res = None if residual is None else residual[:, scale * a:scale * b].contiguous()
        ys = ops.conv3d(xs, packed, bias, affine, res, cout, ksize, 1, mode, silu, code, split, stream_gemm, xs2,
                        flags)
        y[:, scale * s0:scale * s1] = ys[:, scale * (s0 - a):scale * (s1 - a)]
        del xs, xs2, res, ys
    return y


def implicit_gemm_conv3d(
    x: Tensor,
    packed: Tensor,
    bias: Optional[Tensor],
    *,
    cout: int,
    ksize: int = 3,
    affine: Optional[Tensor] = None,
    silu: bool = False,
    stride: int = 1,
    upsample: bool = False,
    trilinear: bool = False,
    residual: Optional[Tensor] = None,
    split: int = 0,
    stream_gemm: bool = False,
    gn_groups: int = 0,
) -> Tensor:
    """Padding-1 3x3x3 (or 1x1x1) convolution of NDHWC ``x`` (``_nax_conv.nax_conv3d``).

    Args mirror the reference (``_nax_conv.py:488-525``): ``bias`` is ``(O,)``
    or per batch item ``(N, O)``; ``affine`` is ``(N, C, 2)`` (scale, offset)
    pairs applied before SiLU; ``upsample`` convolves the nearest-2x upsampling
    with weights from ``pack_upsample_weight``; ``trilinear`` convolves the
    half-pixel trilinear-2x upsampling (plain stride-1 only); ``residual`` has
    the output's shape.  ``split`` forces a K split (0: library policy).
    ``stream_gemm`` keeps the register-streaming GEMM where the library would
    pick the LDS-staged one (large stride-1 fp32 volumes); both are exact to
    fp32 rounding with different fixed summation orders.  ``gn_groups`` asks
    the epilogue for the group-norm statistics of the output over that many
    groups (``ctmr_conv3d_gn``; same output bits); a later ``group_norm_affine``
    of the unmodified output, alone or in a ``ChannelCat``, uses them instead of
    reading the output again when its groups are unions of these (``gn_groups =
    cout`` gives per-channel statistics, usable by any grouping).  Shapes that
    cannot produce them are computed without.

    With ``SLAB_WORKSPACE_BYTES`` set and a stride-1 conv (plain, trilinear-2x or
    1x1x1) whose workspace exceeds it, the conv runs in depth slabs, each with
    the whole volume's kernel and K split, and returns the whole volume's bits
    (as the reference's slabbed packs, ``_nax_conv.py:571-573,667-684``); such a
    conv writes no group-norm statistics.  If no slab depth keeps the kernel and
    split, the volume runs whole.

    Raises:
        ValueError: on a packed weight that does not fit, unsupported option
            combinations, or a residual of the wrong shape.
    """
    x, x2 = _split_input(x)
    cin2 = 0 if x2 is None else int(x2.shape[-1])
    n, d, h, w, cin = (int(v) for v in x.shape)
    cin += cin2
    if x2 is not None and (upsample or trilinear):
        raise ValueError("a concatenated input supports only a plain convolution")
    if trilinear and (upsample or stride != 1 or affine is not None or silu):
        raise ValueError("trilinear packing supports only a plain stride-1 convolution")
    if upsample and stride != 1:
        raise ValueError("nearest upsampling supports only stride 1")
    if ksize == 1 and (upsample or trilinear or stride != 1):
        raise ValueError("1x1x1 convolution supports only stride 1 without resampling")
    mode = _lib.MODE_NEAREST2X if upsample else (_lib.MODE_TRILINEAR2X if trilinear else _lib.MODE_PLAIN)
    code = _PACKED_DTYPES.get(packed.dtype)
    if code is None:
        raise ValueError(f"packed weight dtype {packed.dtype} is not one this library writes")
    desc = ops.make_desc(tuple(x.shape), cout, ksize, stride, mode, _lib.F_STREAM if stream_gemm else 0, code,
                         split, cin2)
    if packed.numel() != _lib.packed_weight_elems(desc):
        raise ValueError(
            f"packed weight of {packed.numel()} elements does not fit {cin} input / {cout} output "
            f"channels ({'nearest-2x' if upsample else 'plain'}, {('fp32', 'bf16', 'f16x2')[code]})"
        )
    bias = _vec(bias, cout, "bias", x.device)
    if bias is not None and bias.dim() == 2 and bias.shape[0] != n:
        raise ValueError(f"per-batch bias has {bias.shape[0]} rows for batch {n}")
    if affine is not None:
        affine = affine.to(torch.float32).contiguous()
        if tuple(affine.shape) != (n, cin, 2):
            raise ValueError(f"affine shape {tuple(affine.shape)} != {(n, cin, 2)}")
    out_shape = (n, *_lib.output_dims(desc), cout)
    if residual is not None:
        residual = _require(residual, "residual")
        if tuple(residual.shape) != out_shape:
            raise ValueError(f"residual shape {tuple(residual.shape)} != output {out_shape}")
    budget = SLAB_WORKSPACE_BYTES
    if budget is not None and stride == 1 and not upsample and int(x.shape[1]) > 1:
        flags = ops._flags(affine is not None, silu, bias is not None and bias.dim() == 2, residual is not None)
        flags |= _lib.F_STREAM if stream_gemm else 0
        whole = ops.make_desc(tuple(x.shape), cout, ksize, 1, mode, flags, code, split, cin2)
        if _lib.workspace_bytes(whole) > int(budget):
            plan = _slabs(x, x2, cout=cout, ksize=ksize, mode=mode, flags=flags, code=code, split=split,
                          budget=int(budget))
            if plan is not None:
                return _conv_in_slabs(x, x2, packed, bias, affine, residual, out_shape, cout=cout, ksize=ksize,
                                      mode=mode, silu=silu, code=code, split=plan[0], stream_gemm=stream_gemm,
                                      scale=2 if trilinear else 1, plan=plan[1], flags=plan[2])
    # Statistics ride on the output tensor, valid while its version counter is unchanged; under
    # torch.inference_mode the output is an inference tensor without one, so nothing is attached and
    # the group norm reading it makes its own pass.
    if (gn_groups > 0 and not torch.is_inference_mode_enabled()
            and ops.conv_stats_tiles(tuple(x.shape), cout, ksize, stride, mode, code, split, stream_gemm,
                                     int(gn_groups), cin2) > 0):
        y, stats = ops.conv3d_gn(x, packed, bias, affine, residual, cout, ksize, stride, mode, silu, code, split,
                                 stream_gemm, int(gn_groups), x2)
        y._ctmr_gn_stats = (int(gn_groups), stats, y._version)
        return y
    return ops.conv3d(x, packed, bias, affine, residual, cout, ksize, stride, mode, silu, code, split,
                      stream_gemm, x2)


def _attached_stats(x: Tensor) -> Optional[tuple[int, Tensor]]:
    """``(stat groups, (N, tiles, stat groups, 2) partials)`` written for ``x`` by the op that produced
    it, or None if there are none or ``x`` was modified in place since."""
    info = getattr(x, "_ctmr_gn_stats", None)
    if info is None or x.is_inference() or info[2] != x._version:
        return None
    return info[0], info[1]


def conv_output_stats(x: Tensor, groups: int) -> Optional[Tensor]:
    """The ``(N, tiles, groups, 2)`` group-norm partials a conv epilogue wrote for ``x``, or None if
    ``x`` carries none for ``groups`` or was modified in place since."""
    info = _attached_stats(x)
    return info[1] if info is not None and info[0] == groups else None


@functools.lru_cache(maxsize=1024)
def _stats_tile_groups(c0: int, c: int, sgroups: int, total: int, groups: int) -> bool:
    """Whether ``sgroups`` equal stat groups over channels ``[c0, c0 + c)`` of a ``total``-channel
    tensor tile every share of its ``groups`` norm groups (``ctmr_gn_affine_from_stats2``'s rule)."""
    if sgroups <= 0 or c % sgroups:
        return False
    scpg, cpg = c // sgroups, total // groups
    for g in range(groups):
        a, e = max(g * cpg, c0) - c0, min((g + 1) * cpg, c0 + c) - c0
        if a < e and (a % scpg or e % scpg):
            return False
    return True


def add_with_stats(a: Tensor, b: Tensor) -> Tensor:
    """``a + b`` (NDHWC fp32, same shape) with per-channel group-norm partials attached, so a group
    norm of the sum, or of a ``ChannelCat`` holding it, reads no statistics pass (the ControlNet
    residuals added to the UNet skips, ``controlnet.py:160-163``).  Same bits as ``a + b``."""
    if (a.shape != b.shape or a.dim() != 5 or int(a.shape[-1]) % 4 or int(a.shape[-1]) > 1024
            or torch.is_inference_mode_enabled()):
        return a + b  # broadcasting or unsupported shapes: the plain sum, without statistics
    a, b = _require(a, "a"), _require(b, "b")
    y, stats = ops.add_gn(a, b)
    y._ctmr_gn_stats = (int(a.shape[-1]), stats, y._version)
    return y


nax_conv3d = implicit_gemm_conv3d  # the reference orchestrator's name (_nax_conv.py:475)


def conv3d(x: Tensor, weight: Tensor, bias: Optional[Tensor], *, padding: int, stride: int = 1,
           gn_groups: int = 0) -> Tensor:
    """NDHWC convolution with a Torch ``(O, C, k, k, k)`` weight (``fast_fp32.conv3d_ncdhw``, :133-154);
    ``gn_groups`` as in ``implicit_gemm_conv3d``."""
    k = int(weight.shape[2])
    if tuple(weight.shape[2:]) != (k, k, k) or (k, padding) not in ((3, 1), (1, 0)):
        raise ValueError(f"supported kernels: 3x3x3 padding 1 and 1x1x1 padding 0; got k={k}, padding={padding}")
    if k == 1 and stride != 1:
        raise ValueError("1x1x1 convolution supports only stride 1")
    if int(weight.shape[1]) != int(x.shape[-1]):
        raise ValueError(f"weight expects {int(weight.shape[1])} input channels; x has {int(x.shape[-1])}")
    return implicit_gemm_conv3d(x, _pack(weight, _lib.MODE_PLAIN, x, stride), bias, cout=int(weight.shape[0]),
                                ksize=k, stride=stride, gn_groups=gn_groups)


def pointwise_conv(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """1x1x1 convolution on FP32 MFMA (``fast_fp32.pointwise_conv_ncdhw``, :121-130)."""
    o = int(weight.shape[0])
    w = weight.reshape(o, -1, 1, 1, 1) if weight.dim() != 5 else weight
    return conv3d(x, w, bias, padding=0)


def group_norm_affine(x: Tensor, weight: Tensor, bias: Tensor, *, groups: int, eps: float) -> Tensor:
    """``(N, C, 2)`` scale/offset pairs of a group norm of NDHWC ``x`` (``medmlx_core.group_norm_affine``).
    Uses the statistics a convolution epilogue (or ``add_with_stats``) wrote for ``x`` when there are
    any at this grouping or a finer one; ``x`` may be a ``ChannelCat``, whose halves' statistics are
    used when both have them."""
    x, x2 = _split_input(x)
    c = int(x.shape[-1]) + (0 if x2 is None else int(x2.shape[-1]))
    if c % groups != 0:
        raise ValueError(f"{c} channels are not divisible by {groups} groups")
    gamma = _vec(weight, c, "norm weight", x.device)
    beta = _vec(bias, c, "norm bias", x.device)
    groups, c1 = int(groups), int(x.shape[-1])
    count = (x.numel() // (int(x.shape[0]) * c1)) * (c // groups)
    first = _attached_stats(x)
    if x2 is None:
        if first is None:
            return ops.gn_affine(x, gamma, beta, groups, float(eps))
        if first[0] == groups:
            return ops.gn_affine_from_stats(first[1], gamma, beta, count, float(eps))
        if _stats_tile_groups(0, c, first[0], c, groups):
            return ops.gn_affine_from_stats2(first[1], c, gamma, beta, groups, count, float(eps))
        return ops.gn_affine(x, gamma, beta, groups, float(eps))
    second = _attached_stats(x2)
    if (first is not None and second is not None and _stats_tile_groups(0, c1, first[0], c, groups)
            and _stats_tile_groups(c1, c - c1, second[0], c, groups)):
        return ops.gn_affine_from_stats2(first[1], c1, gamma, beta, groups, count, float(eps), second[1])
    return ops.gn_affine(x, gamma, beta, groups, float(eps), x2)


def group_norm(x: Tensor, weight: Tensor, bias: Tensor, *, num_groups: int, eps: float,
               apply_silu: bool = False) -> Tensor:
    """Group norm with fp64-accumulated statistics and optional fused SiLU (:102-118); a ``ChannelCat``
    input is normalised into one tensor."""
    affine = group_norm_affine(x, weight, bias, groups=num_groups, eps=eps)
    if isinstance(x, ChannelCat):
        x = x.materialize()
    return ops.gn_apply(x.contiguous(), affine, bool(apply_silu))


def silu_ndhwc(x: Tensor) -> Tensor:
    return ops.silu(x.contiguous())


def avg_pool3d(x: Tensor) -> Tensor:
    """2x2x2 average pooling, stride 2."""
    return ops.resample(_require(x, "x"), _lib.AVGPOOL2)


def upsample_nearest(x: Tensor) -> Tensor:
    """Nearest-neighbour 2x upsampling."""
    return ops.resample(_require(x, "x"), _lib.NEAREST2X)


def upsample_trilinear(x: Tensor) -> Tensor:
    """Half-pixel (align_corners=False) trilinear 2x upsampling, clamped at the edges."""
    return ops.resample(_require(x, "x"), _lib.TRILINEAR2X)


def norm_conv3d(
    x: Tensor,
    weight: Tensor,
    bias: Tensor,
    *,
    norm: Optional[tuple[Tensor, Tensor]],
    num_groups: int,
    eps: float,
    apply_silu: bool,
    upsample: bool = False,
    residual: Optional[Tensor] = None,
    out_gn_groups: int = 0,
) -> Tensor:
    """``conv(upsample?(silu?(norm?(x)))) + bias (+ residual)`` for 3x3x3 kernels (:162-211);
    ``out_gn_groups`` asks for the output's group-norm statistics (``implicit_gemm_conv3d``).  ``x``
    may be a ``ChannelCat`` (no upsampling then)."""
    if not isinstance(x, ChannelCat):
        x = _require(x, "x")
    affine = None if norm is None else group_norm_affine(x, norm[0], norm[1], groups=num_groups, eps=eps)
    mode = _lib.MODE_NEAREST2X if upsample else _lib.MODE_PLAIN
    return implicit_gemm_conv3d(x, _pack(weight, mode, x), bias, cout=int(weight.shape[0]), affine=affine,
                                silu=apply_silu, upsample=upsample, residual=residual, gn_groups=out_gn_groups)


def trilinear_conv3d(x: Tensor, weight: Tensor, bias: Tensor, *, gn_groups: int = 0) -> Tensor:
    """Padding-1 3x3x3 conv of the trilinear 2x upsampling, sampled while packing (:339-349)."""
    return implicit_gemm_conv3d(x, _pack(weight, _lib.MODE_TRILINEAR2X, x), bias, cout=int(weight.shape[0]),
                                trilinear=True, gn_groups=gn_groups)


def linear(x: Tensor, weight: Tensor, bias: Optional[Tensor], mx=None) -> Tensor:
    """FP32 ``x @ weight.T + bias`` (``medmlx_core.ops.linear``, re-exported by the reference's
    fast_fp32.py:48-53; embedding MLPs and attention projections, not on the conv hot path)."""
    return F.linear(x, weight, bias)


def sinusoidal_timestep_embedding(timesteps: Tensor, embedding_dim: int, *, mx=None,
                                  max_period: int = 10000) -> Tensor:
    """``[cos, sin]`` sinusoidal embedding of ``(N,)`` timesteps (embed.py:15-40), padded with one
    zero column for odd ``embedding_dim``."""
    if timesteps.dim() != 1:
        raise ValueError("Timesteps should be a 1d-array")
    half = embedding_dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32, device=timesteps.device)
    freqs = torch.exp(exponent / half)
    args = timesteps.to(torch.float32).reshape(-1, 1) * freqs.reshape(1, -1)
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    if embedding_dim % 2 == 1:
        emb = F.pad(emb, (0, 1))
    return emb


def kernels_available(mx=None) -> bool:
    """Whether the HIP kernels can run here (the reference's ``nax_available`` gate,
    _nax_conv.py:352-363): the library loads and the current device is a gfx950 GPU.  Nothing
    falls back when this is False -- the operators raise."""
    try:
        _lib.lib()
    except _lib.CtmrError:
        return False
    if not torch.cuda.is_available():
        return False
    return torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName.startswith("gfx950")


nax_available = kernels_available


# ---------------------------------------------------------------------------
# attention (fast_fp32.py:352-392, _flash_attention.py:276-360)
# ---------------------------------------------------------------------------
FLASH_HEAD_DIM = 32


def flash_eligible(q: Tensor, k: Tensor, heads: int, mx=None) -> bool:
    """Whether ``(B, L, heads * 32)`` FP32 projections fit the HIP kernel
    (``_flash_attention.flash_eligible``, :276-289; any L here, ragged key blocks are masked)."""
    return (q.dtype == torch.float32 and k.dtype == torch.float32
            and int(q.shape[-1]) == heads * FLASH_HEAD_DIM and int(k.shape[-1]) == heads * FLASH_HEAD_DIM)


def _rows(t: Tensor, name: str) -> Tensor:
    if t.dim() != 3 or t.dtype != torch.float32:
        raise ValueError(f"{name} must be a 3-D float32 (B, L, C) tensor; got {tuple(t.shape)} {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (there is no CPU path); got {t.device}")
    if t.stride(2) != 1 or t.stride(1) % 4 or t.stride(0) != t.shape[1] * t.stride(1) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def flash_attention(q: Tensor, k: Tensor, v: Tensor, *, heads: int, scale: float, mx=None,
                    query_tiles: int = 0) -> Tensor:
    """``softmax(q k^T * scale) v`` on head-interleaved ``(B, L, heads * 32)`` projections
    (``_flash_attention.flash_attention``, :320-360); FP32 MFMA, or under ``precision("f16x2")``
    the reference's split-fp16 kernel; output in the same layout."""
    q, k, v = _rows(q, "q"), _rows(k, "k"), _rows(v, "v")
    if not flash_eligible(q, k, heads) or v.shape != k.shape or q.shape[0] != k.shape[0]:
        raise ValueError(f"flash attention needs (B, L, heads*32) q/k/v with heads={heads}; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    return _flash(q, k, v, int(heads), float(scale), int(query_tiles))


def _flash(q: Tensor, k: Tensor, v: Tensor, heads: int, scale: float, query_tiles: int) -> Tensor:
    """The HIP flash kernel for the active precision: under ``precision("f16x2")`` the
    reference's split-fp16 attention (its matrix-unit path, ``_flash_attention.py:336-350``),
    else FP32 MFMA (``bf16`` keeps attention in FP32, as its norms and projections)."""
    if _precision.get() == "f16x2":
        return ops.flash_attention_f16x2(q, k, v, heads, scale, query_tiles)
    return ops.flash_attention(q, k, v, heads, scale, query_tiles)


# Fused (3C, C) Q/K/V projection weights and biases, keyed by all six source
# tensors and validated like the packed conv weights.
_qkv: dict[tuple, tuple] = {}
_caches: list[tuple[dict, object]] = [(_packed, _packed_lock), (_qkv, _packed_lock)]


def _fused_qkv(wq: Tensor, wk: Tensor, wv: Tensor, biases) -> tuple[Tensor, Optional[Tensor]]:
    sources = (wq, wk, wv) + (() if biases is None else tuple(biases))

    def build():
        weight = torch.cat([wq, wk, wv], dim=0).to(torch.float32).contiguous()
        if biases is None:
            return (weight,)
        return weight, torch.cat(list(biases), dim=0).to(torch.float32).contiguous()

    fused = cached_derived(_qkv, _packed_lock, tuple(id(t) for t in sources), sources, build)
    return fused[0], (fused[1] if len(fused) > 1 else None)


def attention(query: Tensor, key: Tensor, value: Tensor, *, scale: float, mx=None) -> Tensor:
    """Scaled dot-product attention on ``(B, H, L, D)`` heads (the ``AttentionArithmetic``
    surface, reference fast_fp32.py:399-401).  32-wide heads run the HIP flash kernel, each
    (batch, head) pair as one single-head item; other widths use PyTorch's attention on the GPU."""
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("attention expects (B, H, L, D) query, key and value")
    b, h, lq, d = (int(v) for v in query.shape)
    if d == FLASH_HEAD_DIM and query.dtype == key.dtype == value.dtype == torch.float32:
        q = query.contiguous().reshape(b * h, lq, d)
        k = key.contiguous().reshape(b * h, -1, d)
        v = value.contiguous().reshape(b * h, -1, d)
        return _flash(_rows(q, "query"), _rows(k, "key"), _rows(v, "value"), 1, float(scale),
                      0).reshape(b, h, lq, d)
    return F.scaled_dot_product_attention(query, key, value, scale=scale)


def attention_projection(array: Tensor, weight: Tensor, bias: Tensor, mx=None) -> Tensor:
    """Attention output projection, the same FP32 GEMM as ``linear`` (reference fast_fp32.py:404-406)."""
    return F.linear(array, weight, bias)


def self_attention_tokens(tokens: Tensor, weights: Mapping[str, Tensor], *, heads: int, scale: float,
                          include_fc: bool, mx=None, prefix: str = "attn", qkv_bias: bool = True) -> Tensor:
    """Q/K/V projections, multi-head self-attention and optional ``out_proj`` on ``(B, L, C)``
    tokens (``fast_fp32.self_attention_tokens``, :352-392).  32-wide heads run the HIP flash
    kernel on one fused Q/K/V projection; other head widths use PyTorch's attention on the
    GPU, as the reference falls back to ``mx.fast.scaled_dot_product_attention``."""
    tokens = _rows(tokens, "tokens")
    n, length, c = (int(s) for s in tokens.shape)
    names = ("q", "k", "v")
    biases = tuple(weights[f"{prefix}.to_{m}.bias"] for m in names) if qkv_bias else None
    w, b = _fused_qkv(*(weights[f"{prefix}.to_{m}.weight"] for m in names), biases)
    qkv = F.linear(tokens, w, b)
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    if c == heads * FLASH_HEAD_DIM:
        merged = _flash(q, k, v, int(heads), float(scale), 0)
    else:
        def split(t: Tensor) -> Tensor:
            return t.reshape(n, length, heads, c // heads).transpose(1, 2).contiguous()

        att = F.scaled_dot_product_attention(split(q), split(k), split(v), scale=scale)
        merged = att.transpose(1, 2).reshape(n, length, c)
    if include_fc:
        merged = F.linear(merged, weights[f"{prefix}.out_proj.weight"], weights[f"{prefix}.out_proj.bias"])
    return merged


def residual_block(
    x: Tensor,
    emb: Tensor,
    weights: Mapping[str, Tensor],
    *,
    num_groups: int,
    eps: float,
    up: bool = False,
    down: bool = False,
    conv1_bias: Optional[Tensor] = None,
    out_gn_groups: int = 0,
) -> Tensor:
    """Fused ``DiffusionUNetResnetBlock`` on NDHWC ``x`` (``fast_fp32.residual_block_ncdhw``, :214-291);
    ``x`` may be a ``ChannelCat`` (the up path's hidden state and skip).

    The time-embedding projection joins conv1's bias per batch item, the skip
    path (after its optional 1x1x1 projection) joins conv2's accumulator.
    ``down`` normalizes separately before pooling (pooling does not commute
    with SiLU); ``up`` folds the nearest-2x upsampling into conv1's weights and
    projects the skip before upsampling it.  ``conv1_bias`` (``(N, O)``) is
    ``conv1.bias + time_emb_proj(silu(emb))`` when the caller has computed it
    already (the UNet batches every block's projection into one GEMM); ``emb``
    is then unused.  conv1's epilogue writes norm2's statistics; conv2's writes
    them for the block's output when ``out_gn_groups`` is set (the next
    consumer is a group norm with that many groups).
    """
    if isinstance(x, ChannelCat) and (up or down or
                                      int(x.shape[-1]) == int(weights["conv1.conv.weight"].shape[0])):
        x = x.materialize()  # resampled or unprojected inputs need the concatenated tensor itself
    if conv1_bias is None:
        temb = linear(F.silu(emb), weights["time_emb_proj.weight"], weights["time_emb_proj.bias"])
        bias1 = weights["conv1.conv.bias"].reshape(1, -1) + temb
    else:
        bias1 = conv1_bias
    norm1 = (weights["norm1.weight"], weights["norm1.bias"])
    project = int(x.shape[-1]) != int(weights["conv1.conv.weight"].shape[0])

    def project_skip(skip: Tensor) -> Tensor:
        if not project:
            return skip
        return pointwise_conv(skip, weights["skip_connection.conv.weight"], weights["skip_connection.conv.bias"])

    if down:
        # both pools (of norm1 + SiLU, and of x for the skip) from one read of x (ctmr_gn_avgpool)
        affine = group_norm_affine(x, *norm1, groups=num_groups, eps=eps)
        hidden, pooled = ops.gn_avgpool(_require(x, "x").contiguous(), affine, True)
        skip = project_skip(pooled)
        hidden = norm_conv3d(hidden, weights["conv1.conv.weight"], bias1, norm=None, num_groups=num_groups,
                             eps=eps, apply_silu=False, out_gn_groups=num_groups)
    else:
        skip = project_skip(x)
        if up:
            skip = upsample_nearest(skip)
        hidden = norm_conv3d(x, weights["conv1.conv.weight"], bias1, norm=norm1, num_groups=num_groups,
                             eps=eps, apply_silu=True, upsample=up, out_gn_groups=num_groups)
    return norm_conv3d(hidden, weights["conv2.conv.weight"], weights["conv2.conv.bias"],
                       norm=(weights["norm2.weight"], weights["norm2.bias"]), num_groups=num_groups,
                       eps=eps, apply_silu=True, residual=skip, out_gn_groups=out_gn_groups)


def vae_resblock(
    state: list[Tensor],
    conv1: tuple[Tensor, Tensor],
    conv2: tuple[Tensor, Tensor],
    norm1: tuple[Tensor, Tensor],
    norm2: tuple[Tensor, Tensor],
    shortcut: Optional[tuple[Tensor, Tensor]],
    *,
    num_groups: int,
    eps: float,
    out_gn_groups: int = 0,
) -> Tensor:
    """Fused ``MaisiResBlock``: GN-SiLU-conv twice, skip in conv2's accumulator (:294-336).
    Group-norm statistics as in ``residual_block``.

    ``state`` holds the block input and is emptied so the caller's reference
    does not keep a multi-gigabyte input alive past its last use.
    """
    x = state.pop()
    hidden = norm_conv3d(x, *conv1, norm=norm1, num_groups=num_groups, eps=eps, apply_silu=True,
                         out_gn_groups=num_groups)
    skip = x if shortcut is None else pointwise_conv(x, *shortcut)
    del x
    return norm_conv3d(hidden, *conv2, norm=norm2, num_groups=num_groups, eps=eps, apply_silu=True,
                       residual=skip, out_gn_groups=out_gn_groups)


# ---------------------------------------------------------------------------
# NCDHW adapters with the reference's names and keywords
# ---------------------------------------------------------------------------
def to_ndhwc(x: Tensor) -> Tensor:
    return x.permute(0, 2, 3, 4, 1).contiguous()


def to_ncdhw(x: Tensor) -> Tensor:
    return x.permute(0, 4, 1, 2, 3).contiguous()


def conv3d_ncdhw(array: Tensor, weight: Tensor, bias: Optional[Tensor], *, padding: int, mx=None,
                 stride: int = 1) -> Tensor:
    return to_ncdhw(conv3d(to_ndhwc(array), weight, bias, padding=padding, stride=stride))


def pointwise_conv_ncdhw(array: Tensor, weight: Tensor, bias: Optional[Tensor], *, mx=None) -> Tensor:
    return to_ncdhw(pointwise_conv(to_ndhwc(array), weight, bias))


def group_norm_ncdhw(array: Tensor, weight: Tensor, bias: Tensor, *, num_groups: int, eps: float, mx=None,
                     apply_silu: bool = False) -> Tensor:
    return to_ncdhw(group_norm(to_ndhwc(array), weight, bias, num_groups=num_groups, eps=eps,
                               apply_silu=apply_silu))


def norm_conv3d_ncdhw(array: Tensor, weight: Tensor, bias: Tensor, *, norm, num_groups: int, eps: float,
                      apply_silu: bool, mx=None, upsample: bool = False,
                      residual: Optional[Tensor] = None) -> Tensor:
    res = None if residual is None else to_ndhwc(residual)
    return to_ncdhw(norm_conv3d(to_ndhwc(array), weight, bias, norm=norm, num_groups=num_groups, eps=eps,
                                apply_silu=apply_silu, upsample=upsample, residual=res))


def residual_block_ncdhw(x: Tensor, emb: Tensor, weights: Mapping[str, Tensor], *, num_groups: int, eps: float,
                         mx=None, up: bool = False, down: bool = False) -> Tensor:
    return to_ncdhw(residual_block(to_ndhwc(x), emb, weights, num_groups=num_groups, eps=eps, up=up, down=down))


def vae_resblock_ncdhw(state: list[Tensor], conv1, conv2, norm1, norm2, shortcut, *, num_groups: int,
                       eps: float, mx=None) -> Tensor:
    inner = [to_ndhwc(state.pop())]
    return to_ncdhw(vae_resblock(inner, conv1, conv2, norm1, norm2, shortcut, num_groups=num_groups, eps=eps))


def trilinear_conv3d_ncdhw(array: Tensor, weight: Tensor, bias: Tensor, *, mx=None) -> Tensor:
    return to_ncdhw(trilinear_conv3d(to_ndhwc(array), weight, bias))


def avg_pool3d_ncdhw(array: Tensor, *, mx=None) -> Tensor:
    return to_ncdhw(avg_pool3d(to_ndhwc(array)))


def upsample_nearest_ncdhw(array: Tensor, *, mx=None) -> Tensor:
    return to_ncdhw(upsample_nearest(to_ndhwc(array)))


def upsample_trilinear_ncdhw(array: Tensor, *, mx=None, scale: int = 2) -> Tensor:
    if scale != 2:
        raise ValueError("only 2x trilinear upsampling is supported")
    return to_ncdhw(upsample_trilinear(to_ndhwc(array)))


def silu(array: Tensor, mx=None) -> Tensor:
    """SiLU of any-layout fp32 tensor on the GPU (HIP kernel)."""
    return ops.silu(array.contiguous())
