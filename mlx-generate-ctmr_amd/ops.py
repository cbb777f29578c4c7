"""PyTorch-ROCm custom operators (``ctmr::*``) over the C ABI of ``libctmr_hip.so``.

Each operator allocates its outputs and scratch through PyTorch's caching
allocator, passes raw device pointers and the current HIP stream to the
library, and raises on a non-zero status.  Shapes are validated by the
callers in ``fast_fp32``; these functions assume contiguous fp32 NDHWC CUDA
tensors.  Every operator has a fake (meta) implementation so it traces.

An eager call on plain CUDA tensors (no tracing, compilation, dispatch mode or
autograd input) runs the operator's implementation directly: the dispatcher
round trip of a Python custom operator costs about 25 us of host time per call,
more than many of the kernels these operators launch, and an eager network pass
issues a few hundred of them.  Every other call goes through the registered
operator.
"""

from __future__ import annotations

import ctypes
import functools
from typing import Callable, Optional

import torch
from torch import Tensor

from . import _lib


class _CustomOp:
    """A registered ``ctmr::*`` operator (``.op``) whose eager calls on plain tensors skip the
    dispatcher."""

    def __init__(self, name: str, fn: Callable):
        self.op = torch.library.custom_op(name, mutates_args=())(fn)
        self.fn = fn
        functools.update_wrapper(self, fn)

    def register_fake(self, fake: Callable) -> Callable:
        return self.op.register_fake(fake)

    def __call__(self, *args, **kwargs):
        if _direct(args) and _direct(kwargs.values()):
            return self.fn(*args, **kwargs)
        return self.op(*args, **kwargs)


def _direct(values) -> bool:
    """Whether a call with these arguments may bypass the dispatcher: nothing traces or compiles, and
    every tensor is a plain tensor that autograd does not track."""
    if torch._C._len_torch_dispatch_stack() or torch.compiler.is_compiling():
        return False
    grad = torch.is_grad_enabled()
    for v in values:
        if isinstance(v, Tensor) and (type(v) is not Tensor or (grad and v.requires_grad)):
            return False
    return True


def _custom_op(name: str) -> Callable[[Callable], _CustomOp]:
    return lambda fn: _CustomOp(name, fn)


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(*tensors: Optional[Tensor]) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("ctmr operators run only on the GPU (HIP); got a CPU tensor")


def _aligned16(t: Optional[Tensor]) -> Optional[Tensor]:
    """``t`` itself when its data starts on a 16-byte boundary (the kernels read and store 16 bytes
    at a time), else a fresh contiguous copy (a view with an odd storage offset)."""
    if t is None or t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _flags(affine: bool, silu: bool, batch_bias: bool, residual: bool) -> int:
    return (
        (_lib.F_AFFINE if affine else 0)
        | (_lib.F_SILU if silu else 0)
        | (_lib.F_BATCH_BIAS if batch_bias else 0)
        | (_lib.F_RESIDUAL if residual else 0)
    )


def make_desc(
    x_shape: tuple[int, ...],
    cout: int,
    ksize: int,
    stride: int,
    mode: int,
    flags: int,
    dtype: int,
    split: int,
    cin2: int = 0,
) -> _lib.ConvDesc:
    """Descriptor of a conv of ``x_shape`` (NDHWC); ``cin2`` > 0: the input is the channel concatenation
    of that tensor and a second one of ``cin2`` channels (``ctmr_conv3d_cat``)."""
    n, d, h, w, cin = (int(v) for v in x_shape)
    return _lib.conv_desc(n, d, h, w, cin + cin2, cout, ksize=ksize, stride=stride, mode=mode,
                          flags=flags, dtype=dtype, split=split, cin1=cin if cin2 else 0)


def _cin2(x2: Optional[Tensor]) -> int:
    return 0 if x2 is None else int(x2.shape[-1])


# ---------------------------------------------------------------------------
# weight packing
# ---------------------------------------------------------------------------
# element type of a packed weight per ctmr_dtype (split fp16: 16-bit halves and the fp32 column
# scales, as raw 16-bit elements)
_PACKED_TORCH_DTYPES = {_lib.DT_F32: torch.float32, _lib.DT_BF16: torch.bfloat16, _lib.DT_F16X2: torch.float16}


@_custom_op("ctmr::pack_weight")
def pack_weight(weight: Tensor, cin: int, cout: int, ksize: int, mode: int, dtype: int) -> Tensor:
    """Packed conv weight (``ctmr_pack_weight`` / ``ctmr_pack_upsample_weight``)."""
    _require_device(weight)
    desc = _lib.conv_desc(1, 2, 2, 2, cin, cout, ksize=ksize, mode=mode, dtype=dtype)
    elems = _lib.packed_weight_elems(desc)
    out = torch.empty(elems, device=weight.device, dtype=_PACKED_TORCH_DTYPES[dtype])
    fn = _lib.lib().ctmr_pack_upsample_weight if mode == _lib.MODE_NEAREST2X else _lib.lib().ctmr_pack_weight
    _lib.check(fn(ctypes.byref(desc), weight.data_ptr(), out.data_ptr(), _stream(weight.device)),
               "ctmr_pack_weight")
    return out


@pack_weight.register_fake
def _(weight, cin, cout, ksize, mode, dtype):
    desc = _lib.conv_desc(1, 2, 2, 2, cin, cout, ksize=ksize, mode=mode, dtype=dtype)
    return weight.new_empty(_lib.packed_weight_elems(desc), dtype=_PACKED_TORCH_DTYPES[dtype])


# ---------------------------------------------------------------------------
# convolution
# ---------------------------------------------------------------------------
@_custom_op("ctmr::conv3d")
def conv3d(
    x: Tensor,
    packed: Tensor,
    bias: Optional[Tensor],
    affine: Optional[Tensor],
    residual: Optional[Tensor],
    cout: int,
    ksize: int,
    stride: int,
    mode: int,
    silu: bool,
    dtype: int,
    split: int,
    stream_gemm: bool = False,
    x2: Optional[Tensor] = None,
    extra_flags: int = 0,
) -> Tensor:
    """``ctmr_conv3d`` on an NDHWC fp32 tensor; returns the NDHWC output.  ``stream_gemm``
    forces the register-streaming GEMM where the LDS-staged one would be chosen.  With ``x2`` the
    input is the channel concatenation of ``x`` and ``x2`` (``ctmr_conv3d_cat``).  ``extra_flags``:
    route flags OR-ed into the descriptor (``CTMR_F_SPLIT_WAVES``)."""
    _require_device(x, packed, bias, affine, residual, x2)
    x, residual, x2 = _aligned16(x), _aligned16(residual), _aligned16(x2)
    batch_bias = bias is not None and bias.dim() == 2
    flags = _flags(affine is not None, silu, batch_bias, residual is not None) | int(extra_flags)
    if stream_gemm:
        flags |= _lib.F_STREAM
    desc = make_desc(tuple(x.shape), cout, ksize, stride, mode, flags, dtype, split, _cin2(x2))
    od, oh, ow = _lib.output_dims(desc)
    y = torch.empty((x.shape[0], od, oh, ow, cout), device=x.device, dtype=torch.float32)
    ws_bytes = _lib.workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 1), device=x.device, dtype=torch.uint8)
    if x2 is None:
        _lib.check(
            _lib.lib().ctmr_conv3d(
                ctypes.byref(desc), x.data_ptr(), packed.data_ptr(), _ptr(bias), _ptr(affine),
                _ptr(residual), y.data_ptr(), ws.data_ptr(), ws_bytes, _stream(x.device),
            ),
            "ctmr_conv3d",
        )
    else:
        _lib.check(
            _lib.lib().ctmr_conv3d_cat(
                ctypes.byref(desc), x.data_ptr(), x2.data_ptr(), packed.data_ptr(), _ptr(bias), _ptr(affine),
                _ptr(residual), y.data_ptr(), ws.data_ptr(), ws_bytes, _stream(x.device),
            ),
            "ctmr_conv3d_cat",
        )
    return y


@conv3d.register_fake
def _(x, packed, bias, affine, residual, cout, ksize, stride, mode, silu, dtype, split, stream_gemm=False,
      x2=None, extra_flags=0):
    desc = make_desc(tuple(x.shape), cout, ksize, stride, mode, int(extra_flags), dtype, split, _cin2(x2))
    od, oh, ow = _lib.output_dims(desc)
    return x.new_empty((x.shape[0], od, oh, ow, cout))


def conv_stats_tiles(x_shape: tuple[int, ...], cout: int, ksize: int, stride: int, mode: int, dtype: int,
                     split: int, stream_gemm: bool, groups: int, cin2: int = 0) -> int:
    """Group-norm partials per batch item that ``conv3d_gn`` writes for this shape, 0 if it cannot."""
    flags = _lib.F_STREAM if stream_gemm else 0
    desc = make_desc(tuple(x_shape), cout, ksize, stride, mode, flags, dtype, split, cin2)
    return max(int(_lib.lib().ctmr_conv3d_stats_tiles(ctypes.byref(desc), groups)), 0)


@_custom_op("ctmr::conv3d_gn")
def conv3d_gn(
    x: Tensor,
    packed: Tensor,
    bias: Optional[Tensor],
    affine: Optional[Tensor],
    residual: Optional[Tensor],
    cout: int,
    ksize: int,
    stride: int,
    mode: int,
    silu: bool,
    dtype: int,
    split: int,
    stream_gemm: bool,
    groups: int,
    x2: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor]:
    """``ctmr_conv3d_gn``: the ``conv3d`` output plus float64 group-norm partials of it, shape
    ``(N, tiles, groups, 2)`` holding (sum, sum of squares) per output tile and group.  ``x2`` as in
    ``conv3d`` (``ctmr_conv3d_cat_gn``)."""
    _require_device(x, packed, bias, affine, residual, x2)
    x, residual, x2 = _aligned16(x), _aligned16(residual), _aligned16(x2)
    batch_bias = bias is not None and bias.dim() == 2
    flags = _flags(affine is not None, silu, batch_bias, residual is not None)
    if stream_gemm:
        flags |= _lib.F_STREAM
    desc = make_desc(tuple(x.shape), cout, ksize, stride, mode, flags, dtype, split, _cin2(x2))
    tiles = _lib.check(_lib.lib().ctmr_conv3d_stats_tiles(ctypes.byref(desc), groups), "ctmr_conv3d_stats_tiles")
    if tiles == 0:
        raise ValueError("this convolution cannot produce group-norm partials")
    od, oh, ow = _lib.output_dims(desc)
    y = torch.empty((x.shape[0], od, oh, ow, cout), device=x.device, dtype=torch.float32)
    stats = torch.empty((x.shape[0], tiles, groups, 2), device=x.device, dtype=torch.float64)
    ws_bytes = _lib.workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 1), device=x.device, dtype=torch.uint8)
    if x2 is None:
        _lib.check(
            _lib.lib().ctmr_conv3d_gn(
                ctypes.byref(desc), x.data_ptr(), packed.data_ptr(), _ptr(bias), _ptr(affine),
                _ptr(residual), y.data_ptr(), ws.data_ptr(), ws_bytes, groups, stats.data_ptr(),
                _stream(x.device),
            ),
            "ctmr_conv3d_gn",
        )
    else:
        _lib.check(
            _lib.lib().ctmr_conv3d_cat_gn(
                ctypes.byref(desc), x.data_ptr(), x2.data_ptr(), packed.data_ptr(), _ptr(bias), _ptr(affine),
                _ptr(residual), y.data_ptr(), ws.data_ptr(), ws_bytes, groups, stats.data_ptr(),
                _stream(x.device),
            ),
            "ctmr_conv3d_cat_gn",
        )
    return y, stats


@conv3d_gn.register_fake
def _(x, packed, bias, affine, residual, cout, ksize, stride, mode, silu, dtype, split, stream_gemm, groups,
      x2=None):
    desc = make_desc(tuple(x.shape), cout, ksize, stride, mode, _lib.F_STREAM if stream_gemm else 0, dtype, split,
                     _cin2(x2))
    od, oh, ow = _lib.output_dims(desc)
    tiles = max(int(_lib.lib().ctmr_conv3d_stats_tiles(ctypes.byref(desc), groups)), 1)
    return (x.new_empty((x.shape[0], od, oh, ow, cout)),
            x.new_empty((x.shape[0], tiles, groups, 2), dtype=torch.float64))


# ---------------------------------------------------------------------------
# group norm
# ---------------------------------------------------------------------------
@_custom_op("ctmr::gn_affine_from_stats")
def gn_affine_from_stats(stats: Tensor, gamma: Tensor, beta: Tensor, count: int, eps: float) -> Tensor:
    """``ctmr_gn_affine_from_stats``: (N, C, 2) (scale, offset) pairs from ``conv3d_gn`` partials
    ``(N, tiles, groups, 2)``; ``count`` is the number of values in one (batch item, group)."""
    _require_device(stats, gamma, beta)
    n, tiles, groups = (int(v) for v in stats.shape[:3])
    c = int(gamma.numel())
    out = torch.empty((n, c, 2), device=stats.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().ctmr_gn_affine_from_stats(n, tiles, c, groups, count, float(eps), stats.data_ptr(),
                                             gamma.data_ptr(), beta.data_ptr(), out.data_ptr(),
                                             _stream(stats.device)),
        "ctmr_gn_affine_from_stats",
    )
    return out


@gn_affine_from_stats.register_fake
def _(stats, gamma, beta, count, eps):
    return stats.new_empty((stats.shape[0], gamma.numel(), 2), dtype=torch.float32)


@_custom_op("ctmr::gn_affine_from_stats2")
def gn_affine_from_stats2(stats1: Tensor, c1: int, gamma: Tensor, beta: Tensor, groups: int, count: int,
                          eps: float, stats2: Optional[Tensor] = None) -> Tensor:
    """``ctmr_gn_affine_from_stats2``: (N, C, 2) (scale, offset) pairs over ``groups`` groups from
    partials ``(N, tiles, sgroups, 2)`` at a finer grouping: ``stats1`` over the first ``c1``
    channels and, if given, ``stats2`` over the remaining ``C - c1`` (a channel concatenation)."""
    _require_device(stats1, gamma, beta, stats2)
    n, tiles1, sg1 = (int(v) for v in stats1.shape[:3])
    c = int(gamma.numel())
    tiles2, sg2 = (0, 1) if stats2 is None else (int(stats2.shape[1]), int(stats2.shape[2]))
    out = torch.empty((n, c, 2), device=stats1.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().ctmr_gn_affine_from_stats2(n, groups, count, float(eps), stats1.data_ptr(), tiles1, c1, sg1,
                                              _ptr(stats2), tiles2, c - c1, sg2, gamma.data_ptr(),
                                              beta.data_ptr(), out.data_ptr(), _stream(stats1.device)),
        "ctmr_gn_affine_from_stats2",
    )
    return out


@gn_affine_from_stats2.register_fake
def _(stats1, c1, gamma, beta, groups, count, eps, stats2=None):
    return stats1.new_empty((stats1.shape[0], gamma.numel(), 2), dtype=torch.float32)


@_custom_op("ctmr::add_gn")
def add_gn(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor]:
    """``ctmr_add_gn_partials``: ``a + b`` (same NDHWC shape) and its per-channel float64 partials
    ``(N, tiles, C, 2)``."""
    _require_device(a, b)
    if a.shape != b.shape:
        raise ValueError(f"add_gn operands differ in shape: {tuple(a.shape)} vs {tuple(b.shape)}")
    a, b = _aligned16(a), _aligned16(b)
    n, c = int(a.shape[0]), int(a.shape[-1])
    s = a.numel() // (n * c)
    ws_bytes = _lib.gn_workspace_bytes(n, s, c)
    y = torch.empty(a.shape, device=a.device, dtype=torch.float32)
    stats = torch.empty((n, ws_bytes // (n * c * 16), c, 2), device=a.device, dtype=torch.float64)
    _lib.check(
        _lib.lib().ctmr_add_gn_partials(n, s, c, a.data_ptr(), b.data_ptr(), y.data_ptr(), stats.data_ptr(),
                                        ws_bytes, _stream(a.device)),
        "ctmr_add_gn_partials",
    )
    return y, stats


@add_gn.register_fake
def _(a, b):
    n, c = int(a.shape[0]), int(a.shape[-1])
    s = a.numel() // (n * c)
    tiles = _lib.gn_workspace_bytes(n, s, c) // (n * c * 16)
    return a.new_empty(a.shape), a.new_empty((n, tiles, c, 2), dtype=torch.float64)


@_custom_op("ctmr::gn_affine")
def gn_affine(x: Tensor, gamma: Tensor, beta: Tensor, groups: int, eps: float,
              x2: Optional[Tensor] = None) -> Tensor:
    """Per-(batch, channel) (scale, offset) pairs, shape ``(N, C, 2)``; with ``x2`` of the channel
    concatenation of ``x`` and ``x2`` (``ctmr_gn_affine_cat``)."""
    _require_device(x, gamma, beta, x2)
    x, x2 = _aligned16(x), _aligned16(x2)
    n, c1 = int(x.shape[0]), int(x.shape[-1])
    c2 = _cin2(x2)
    c = c1 + c2
    s = x.numel() // (n * c1)
    out = torch.empty((n, c, 2), device=x.device, dtype=torch.float32)
    ws_bytes = _lib.gn_workspace_bytes(n, s, c)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    if x2 is None:
        _lib.check(
            _lib.lib().ctmr_gn_affine(n, s, c, groups, float(eps), x.data_ptr(), gamma.data_ptr(),
                                      beta.data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes,
                                      _stream(x.device)),
            "ctmr_gn_affine",
        )
    else:
        _lib.check(
            _lib.lib().ctmr_gn_affine_cat(n, s, c1, c2, groups, float(eps), x.data_ptr(), x2.data_ptr(),
                                          gamma.data_ptr(), beta.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                          ws_bytes, _stream(x.device)),
            "ctmr_gn_affine_cat",
        )
    return out


@gn_affine.register_fake
def _(x, gamma, beta, groups, eps, x2=None):
    return x.new_empty((x.shape[0], x.shape[-1] + _cin2(x2), 2))


@_custom_op("ctmr::gn_apply")
def gn_apply(x: Tensor, affine: Tensor, silu: bool) -> Tensor:
    """``silu?(x * scale + offset)`` with pairs from ``gn_affine``."""
    _require_device(x, affine)
    n, c = int(x.shape[0]), int(x.shape[-1])
    s = x.numel() // (n * c)
    y = torch.empty_like(x)
    _lib.check(
        _lib.lib().ctmr_gn_apply(n, s, c, x.data_ptr(), affine.data_ptr(), int(silu), y.data_ptr(),
                                 _stream(x.device)),
        "ctmr_gn_apply",
    )
    return y


@gn_apply.register_fake
def _(x, affine, silu):
    return torch.empty_like(x)


@_custom_op("ctmr::silu")
def silu(x: Tensor) -> Tensor:
    """Elementwise ``x / (1 + exp(-x))``."""
    _require_device(x)
    y = torch.empty_like(x)
    _lib.check(_lib.lib().ctmr_silu(x.numel(), x.data_ptr(), y.data_ptr(), _stream(x.device)),
               "ctmr_silu")
    return y


@silu.register_fake
def _(x):
    return torch.empty_like(x)


# ---------------------------------------------------------------------------
# resampling
# ---------------------------------------------------------------------------
@_custom_op("ctmr::resample")
def resample(x: Tensor, op: int) -> Tensor:
    """2x average pool, nearest or trilinear upsampling of an NDHWC tensor."""
    _require_device(x)
    n, d, h, w, c = (int(v) for v in x.shape)
    if op == _lib.AVGPOOL2:
        shape = (n, d // 2, h // 2, w // 2, c)
    else:
        shape = (n, 2 * d, 2 * h, 2 * w, c)
    y = torch.empty(shape, device=x.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().ctmr_resample(op, n, d, h, w, c, x.data_ptr(), y.data_ptr(), _stream(x.device)),
        "ctmr_resample",
    )
    return y


@resample.register_fake
def _(x, op):
    n, d, h, w, c = x.shape
    if op == _lib.AVGPOOL2:
        return x.new_empty((n, d // 2, h // 2, w // 2, c))
    return x.new_empty((n, 2 * d, 2 * h, 2 * w, c))


@_custom_op("ctmr::gn_avgpool")
def gn_avgpool(x: Tensor, affine: Tensor, silu: bool) -> tuple[Tensor, Tensor]:
    """``(avg_pool(silu?(x * scale + offset)), avg_pool(x))`` of an NDHWC tensor from one read of ``x``
    (the down-sampling residual block's two inputs); bit-identical to ``gn_apply`` then ``resample``."""
    _require_device(x, affine)
    n, d, h, w, c = (int(v) for v in x.shape)
    shape = (n, d // 2, h // 2, w // 2, c)
    y = torch.empty(shape, device=x.device, dtype=torch.float32)
    y_skip = torch.empty(shape, device=x.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().ctmr_gn_avgpool(n, d, h, w, c, x.data_ptr(), affine.data_ptr(), int(silu), y.data_ptr(),
                                   y_skip.data_ptr(), _stream(x.device)),
        "ctmr_gn_avgpool",
    )
    return y, y_skip


@gn_avgpool.register_fake
def _(x, affine, silu):
    n, d, h, w, c = x.shape
    return x.new_empty((n, d // 2, h // 2, w // 2, c)), x.new_empty((n, d // 2, h // 2, w // 2, c))


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
@_custom_op("ctmr::flash_attention")
def flash_attention(q: Tensor, k: Tensor, v: Tensor, heads: int, scale: float, query_tiles: int = 0) -> Tensor:
    """``softmax(q k^T * scale) v`` per head on ``(B, L, heads * 32)`` projections.

    ``q``/``k``/``v`` may be column slices of one fused projection: the last
    dimension must be unit-stride and the batch stride ``L * row stride``.
    """
    _require_device(q, k, v)
    n, lq, c = (int(s) for s in q.shape)
    lk = int(k.shape[1])
    out = torch.empty((n, lq, c), device=q.device, dtype=torch.float32)
    desc = _lib.AttnDesc(n, lq, lk, int(heads), c // int(heads), int(query_tiles),
                         q.stride(1), k.stride(1), v.stride(1), c, float(scale))
    _lib.check(
        _lib.lib().ctmr_flash_attention(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        out.data_ptr(), _stream(q.device)),
        "ctmr_flash_attention",
    )
    return out


@flash_attention.register_fake
def _(q, k, v, heads, scale, query_tiles=0):
    return q.new_empty(q.shape)


@_custom_op("ctmr::flash_attention_f16x2")
def flash_attention_f16x2(q: Tensor, k: Tensor, v: Tensor, heads: int, scale: float,
                          query_tiles: int = 0) -> Tensor:
    """``flash_attention`` in the reference's split-fp16 arithmetic (its matrix-unit kernel,
    ``_flash_attention.py:140-290``): q (scaled by ``scale * log2(e)``), k and v split into fp16
    halves in a workspace, products hi*hi + (hi*lo + lo*hi) * 2^-11 on fp16 MFMA with fp32
    accumulation.  ``|q * scale * log2(e)|``, ``|k|`` and ``|v|`` must stay below 65504."""
    _require_device(q, k, v)
    n, lq, c = (int(s) for s in q.shape)
    lk = int(k.shape[1])
    out = torch.empty((n, lq, c), device=q.device, dtype=torch.float32)
    desc = _lib.AttnDesc(n, lq, lk, int(heads), c // int(heads), int(query_tiles),
                         q.stride(1), k.stride(1), v.stride(1), c, float(scale))
    lib = _lib.lib()
    nbytes = int(lib.ctmr_flash_attention_f16x2_workspace_bytes(ctypes.byref(desc)))
    if nbytes < 0:
        raise ValueError(f"flash_attention_f16x2: invalid shape {(n, lq, lk, heads)}")
    ws = torch.empty((nbytes,), device=q.device, dtype=torch.uint8)
    _lib.check(
        lib.ctmr_flash_attention_f16x2(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       out.data_ptr(), ws.data_ptr(), nbytes, _stream(q.device)),
        "ctmr_flash_attention_f16x2",
    )
    return out


@flash_attention_f16x2.register_fake
def _(q, k, v, heads, scale, query_tiles=0):
    return q.new_empty(q.shape)
