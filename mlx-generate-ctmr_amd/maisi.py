"""MAISI networks and samplers composed over the HIP hot path (NDHWC, fp32, GPU).

The callers of the conv3d / group-norm path, restated from the reference so the
configs' UNet step and windowed VAE decode run end to end on MI355X:

* ``denoise_unet``      DiffusionModelUNetMaisi forward (reference unet.py:42-487)
* ``spatial_attention`` residual GN -> QKV -> SDPA -> out_proj (attention.py:92-160;
                        the token layout of NDHWC is free, SDPA is PyTorch's)
* ``decode_vae``        post_quant 1x1 + MaisiDecoder (vae.py:29-62, 273-379)
* ``sliding_window_decode`` Gaussian-blended windows (decode.py:30-245)
* ``set_timesteps_rflow`` / ``step_rflow`` / ``sample_rflow`` (rflow.py:19-177)
* ``guided_velocity``   classifier-free guidance (image.py:118-175)
* ``UNetGraph``         a UNet pass recorded once as a HIP graph and replayed per step
* ``output_intensities`` int16 conversion (image.py:68-87)

Every convolution and group norm goes through ``fast_fp32`` (the HIP kernels).
Weights are flat state dicts with Torch layouts (MONAI names), as torch tensors
on the GPU.  Each public ``*_ncdhw`` function takes and returns NCDHW.
"""

from __future__ import annotations

import contextlib
import gc
import math
import threading
from collections.abc import Callable, Mapping, Sequence
from itertools import product
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from . import fast_fp32 as ff

Z_SCALE = 4
_GAUSSIAN_FLOOR = 1e-3
_TRAIN_STEPS = 1000
_BASE_NUMEL = 32 * 32 * 32


def _prefixed(weights: Mapping[str, Tensor], prefix: str) -> dict[str, Tensor]:
    start = prefix + "."
    return {k[len(start):]: v for k, v in weights.items() if k.startswith(start)}


def _need(weights: Mapping[str, Tensor], key: str) -> Tensor:
    if key not in weights:
        raise ValueError(f"weights missing: {key}")
    return weights[key]


def _per_level(value, n: int) -> tuple[int, ...]:
    if isinstance(value, int) and not isinstance(value, bool):
        return (int(value),) * n
    out = tuple(int(v) for v in value)
    if len(out) != n:
        raise ValueError(f"per-level setting has {len(out)} entries for {n} levels")
    return out


# ---------------------------------------------------------------------------
# embeddings (embed.py:15-87)
# ---------------------------------------------------------------------------
def sinusoidal_timestep_embedding(timesteps: Tensor, dim: int, max_period: int = 10000) -> Tensor:
    """``[cos, sin]`` sinusoidal embedding of ``(N,)`` timesteps (embed.py:15-40)."""
    return ff.sinusoidal_timestep_embedding(timesteps, dim, max_period=max_period)


def _silu_mlp(x: Tensor, weights: Mapping[str, Tensor], prefix: str) -> Tensor:
    h = F.linear(x, _need(weights, f"{prefix}.0.weight"), _need(weights, f"{prefix}.0.bias"))
    return F.linear(F.silu(h), _need(weights, f"{prefix}.2.weight"), _need(weights, f"{prefix}.2.bias"))


def condition_embedding(timesteps: Tensor, class_labels: Optional[Tensor], spacing: Optional[Tensor],
                        weights: Mapping[str, Tensor], constructor: Mapping) -> tuple[Tensor, Tensor]:
    """``(t_emb, emb)``: time MLP + class embedding, spacing MLP concatenated (unet.py:190-271)."""
    t_emb = sinusoidal_timestep_embedding(timesteps, int(constructor["num_channels"][0]))
    emb = _silu_mlp(t_emb, weights, "time_embed")
    if constructor.get("num_class_embeds") is not None:
        if class_labels is None:
            raise ValueError("class_labels should be provided when num_class_embeds > 0")
        emb = emb + _need(weights, "class_embedding.weight")[class_labels.to(torch.long)]
    for flag in ("include_top_region_index_input", "include_bottom_region_index_input"):
        if constructor.get(flag):
            raise ValueError(f"{flag} (ddpm-ct region inputs) is not part of this path")
    if constructor.get("include_spacing_input"):
        if spacing is None:
            raise ValueError("spacing should be provided when include_spacing_input is true")
        if spacing.dim() != 2 or spacing.shape[-1] != 3:
            raise ValueError(f"spacing must be [N, 3]; got shape={tuple(spacing.shape)}")
        emb = torch.cat([emb, _silu_mlp(spacing.to(torch.float32), weights, "spacing_layer")], dim=-1)
    return t_emb, emb


# ---------------------------------------------------------------------------
# attention (attention.py:92-160), NDHWC: tokens are the voxel rows
# ---------------------------------------------------------------------------
def spatial_attention(x: Tensor, weights: Mapping[str, Tensor], *, num_groups: int, eps: float,
                      num_head_channels: int, include_fc: bool) -> Tensor:
    """Residual self-attention over all voxels of NDHWC ``x`` (attention.py:92-160): group
    norm (HIP), tokens are the NDHWC rows as they lie, Q/K/V + flash attention + out_proj.  The
    residual sum carries per-channel statistics for the group norm that reads it next."""
    n, d, h, w, c = x.shape
    if c % num_head_channels != 0:
        raise ValueError("num_channels must be divisible by num_head_channels")
    heads = c // num_head_channels
    scale = float(num_head_channels) ** -0.5
    hidden = ff.group_norm(x, weights["norm.weight"], weights["norm.bias"], num_groups=num_groups, eps=eps)
    merged = ff.self_attention_tokens(hidden.reshape(n, d * h * w, c), weights, heads=heads, scale=scale,
                                      include_fc=include_fc)
    return ff.add_with_stats(x, merged.reshape(n, d, h, w, c))


# ---------------------------------------------------------------------------
# UNet (unet.py:42-487)
# ---------------------------------------------------------------------------
# Every residual block's time-embedding projection stacked into one GEMM, with
# conv1's bias folded into the GEMM bias: keyed by every source tensor (the
# projection weights and biases and the conv1 biases), rebuilt when one is
# collected or modified in place (fast_fp32.cached_derived).
_TIME_SUFFIX = ".time_emb_proj.weight"
_time_proj: dict[tuple[int, ...], tuple] = {}
_time_proj_lock = threading.RLock()
ff.register_cache(_time_proj, _time_proj_lock)


def _time_projections(weights: Mapping[str, Tensor]) -> tuple[Tensor, Tensor, dict[str, tuple[int, int]]]:
    prefixes = sorted(k[: -len(_TIME_SUFFIX)] for k in weights if k.endswith(_TIME_SUFFIX))
    mats = [weights[p + _TIME_SUFFIX] for p in prefixes]
    biases = [(_need(weights, f"{p}.time_emb_proj.bias"), _need(weights, f"{p}.conv1.conv.bias")) for p in prefixes]
    sources = tuple(mats) + tuple(t for pair in biases for t in pair)

    def build():
        weight = torch.cat(mats, dim=0).to(torch.float32).contiguous()
        bias = torch.cat([tb + cb for tb, cb in biases]).to(torch.float32).contiguous()
        return weight, bias

    weight, bias = ff.cached_derived(_time_proj, _time_proj_lock, tuple(id(t) for t in sources), sources, build)
    spans, start = {}, 0
    for p, m in zip(prefixes, mats):
        spans[p] = (start, start + int(m.shape[0]))
        start += int(m.shape[0])
    return weight, bias, spans


_block_index: dict[tuple, tuple[Tensor, dict[str, tuple[int, int]]]] = {}
_block_index_lock = threading.Lock()


def _block_major_index(spans: Mapping[str, tuple[int, int]], n: int, total: int, device) -> tuple:
    """Gather index that reorders an (n, total) row-major matrix of per-block columns
    [lo, hi) into block-major order (block, batch item, column), and each block's
    (offset, width) in it; cached per (spans, n, total, device)."""
    key = (tuple(sorted(spans.items())), n, total, str(device))
    with _block_index_lock:
        hit = _block_index.get(key)
    if hit is not None:
        return hit
    parts, offsets, off = [], {}, 0
    for prefix, (lo, hi) in sorted(spans.items(), key=lambda kv: kv[1][0]):
        rows = torch.arange(n, dtype=torch.int64).unsqueeze(1) * total
        parts.append((rows + torch.arange(lo, hi, dtype=torch.int64)).reshape(-1))
        offsets[prefix] = (off, hi - lo)
        off += n * (hi - lo)
    hit = (torch.cat(parts).to(device), offsets)
    with _block_index_lock:
        _block_index[key] = hit
    return hit


def _blocks(weights: Mapping[str, Tensor], emb: Tensor, groups: int, eps: float, include_fc: bool):
    """Residual-block and attention callables bound to one embedding and weight dict.  The
    per-block conv1 biases (``conv1.bias + time_emb_proj(silu(emb))``) come from one GEMM."""
    proj_w, proj_b, spans = _time_projections(weights)
    conv1_bias = F.linear(F.silu(emb), proj_w, proj_b)  # (n, all blocks' channels)
    # One gather into block-major order, so each block's (n, cout) bias is a
    # contiguous view (instead of a copy kernel per block).
    n = int(conv1_bias.shape[0])
    index, offsets = _block_major_index(spans, n, int(conv1_bias.shape[1]), conv1_bias.device)
    blocked = conv1_bias.reshape(-1).index_select(0, index)

    def resnet(h, prefix: str, *, stats: Optional[str] = "groups", **kw) -> Tensor:
        """``stats``: the group-norm statistics conv2's epilogue writes for the output -- ``"groups"``
        when a group norm over the output alone reads it next, ``"channels"`` (per channel) when it is
        also read as half of an up-path concatenation, whose norm groups may straddle the halves,
        None when no group norm reads it."""
        off, width = offsets[prefix]
        cout = int(_need(weights, f"{prefix}.conv2.conv.weight").shape[0])
        return ff.residual_block(h, emb, _prefixed(weights, prefix), num_groups=groups, eps=eps,
                                 conv1_bias=blocked[off:off + n * width].view(n, width),
                                 out_gn_groups={"groups": groups, "channels": cout, None: 0}[stats], **kw)

    def attention(h: Tensor, prefix: str, n_heads: int) -> Tensor:
        return spatial_attention(h, _prefixed(weights, prefix), num_groups=groups, eps=eps,
                                 num_head_channels=n_heads, include_fc=include_fc)

    return resnet, attention


def _down_path(hidden: Tensor, resnet, attention, res_blocks, attn_levels, heads) -> tuple[Tensor, list[Tensor]]:
    """Encoder levels; returns the hidden state and every skip (unet.py:274-356).  Outputs that
    become skips carry per-channel statistics (the up path's norm1 reads them in a concatenation)."""
    skips = [hidden]
    n_levels = len(res_blocks)
    for index in range(n_levels):
        for r in range(res_blocks[index]):
            hidden = resnet(hidden, f"down_blocks.{index}.resnets.{r}",
                            stats="groups" if attn_levels[index] else "channels")
            if attn_levels[index]:
                hidden = attention(hidden, f"down_blocks.{index}.attentions.{r}", heads[index])
            skips.append(hidden)
        if index != n_levels - 1:
            hidden = resnet(hidden, f"down_blocks.{index}.downsampler", down=True, stats="channels")
            skips.append(hidden)
    return hidden, skips


def _mid_block(hidden: Tensor, resnet, attention, n_heads: int, out_stats: Optional[str] = "channels") -> Tensor:
    """resnet -> attention -> resnet (unet.py:359-399); the output is concatenated with a skip next."""
    hidden = resnet(hidden, "middle_block.resnet_1")
    hidden = attention(hidden, "middle_block.attention", n_heads)
    return resnet(hidden, "middle_block.resnet_2", stats=out_stats)


def denoise_unet(
    x: Tensor,
    timesteps: Tensor,
    class_labels: Optional[Tensor],
    spacing: Optional[Tensor],
    weights: Mapping[str, Tensor],
    *,
    constructor: Mapping,
    down_block_additional_residuals: Optional[Sequence[Tensor]] = None,
    mid_block_additional_residual: Optional[Tensor] = None,
    residuals_ready: Optional["torch.cuda.Event"] = None,
) -> tuple[Tensor, Tensor]:
    """One DiffusionModelUNetMaisi pass on NDHWC ``x``; returns ``(t_emb, y)`` (NDHWC).

    ``residuals_ready``: an event the current stream waits for after the encoder and before the ControlNet
    residuals are read (they may still be in flight on another stream until then; see
    ``controlnet_unet_step``)."""
    if int(constructor.get("spatial_dims", 3)) != 3 or constructor.get("use_flash_attention"):
        raise ValueError("MAISI UNet destination is 3D without CUDA flash attention")
    if constructor.get("with_conditioning"):
        raise ValueError("cross-attention conditioning is not part of this path")
    if x.shape[-1] != int(constructor["in_channels"]):
        raise ValueError(f"unet input channels {x.shape[-1]} != in_channels {constructor['in_channels']}")
    channels = tuple(int(c) for c in constructor["num_channels"])
    n_levels = len(channels)
    res_blocks = _per_level(constructor["num_res_blocks"], n_levels)
    attn_levels = tuple(bool(a) for a in constructor["attention_levels"])
    heads = _per_level(constructor["num_head_channels"], n_levels)
    groups, eps = int(constructor["norm_num_groups"]), float(constructor["norm_eps"])
    include_fc = bool(constructor.get("include_fc", True))
    if not constructor.get("resblock_updown", True):
        raise ValueError("resblock_updown=False (ddpm-ct) is not part of this path")

    t_emb, emb = condition_embedding(timesteps, class_labels, spacing, weights, constructor)
    resnet, attention = _blocks(weights, emb, groups, eps, include_fc)

    conv_in_w = _need(weights, "conv_in.conv.weight")
    hidden = ff.conv3d(x, conv_in_w, _need(weights, "conv_in.conv.bias"), padding=1,
                       gn_groups=int(conv_in_w.shape[0]))  # per channel: the first skip
    hidden, skips = _down_path(hidden, resnet, attention, res_blocks, attn_levels, heads)
    if residuals_ready is not None:
        torch.cuda.current_stream(x.device).wait_event(residuals_ready)
    if down_block_additional_residuals is not None:
        extras = list(down_block_additional_residuals)
        if len(extras) != len(skips):
            raise ValueError(f"ControlNet residuals length {len(extras)} != UNet skip count {len(skips)}")
        skips = [ff.add_with_stats(s, e) for s, e in zip(skips, extras)]
        hidden = skips[-1]
    mid_extra = mid_block_additional_residual
    hidden = _mid_block(hidden, resnet, attention, heads[-1], out_stats=None if mid_extra is not None else "channels")
    if mid_extra is not None:
        hidden = ff.add_with_stats(hidden, mid_extra)
    rev_res, rev_attn, rev_heads = res_blocks[::-1], attn_levels[::-1], heads[::-1]
    for index in range(n_levels):
        n_res = rev_res[index] + 1
        samples, skips = skips[-n_res:], skips[:-n_res]
        for r in range(n_res):
            skip = samples.pop()
            # cat([hidden, skip]) (unet.py:444) read in place by the block's norm and convolutions; an
            # output concatenated next carries per-channel statistics, one normalised alone next
            # (by attention, the up-sampler or the output norm) the groups'
            hidden = resnet(ff.concat_channels(hidden, skip), f"up_blocks.{index}.resnets.{r}",
                            stats="groups" if rev_attn[index] or r == n_res - 1 else "channels")
            if rev_attn[index]:
                hidden = attention(hidden, f"up_blocks.{index}.attentions.{r}", rev_heads[index])
        if index != n_levels - 1:
            hidden = resnet(hidden, f"up_blocks.{index}.upsampler", up=True, stats="channels")
    if skips:
        raise ValueError(f"UNet skip list leftover after up blocks: {len(skips)}")
    y = ff.norm_conv3d(hidden, _need(weights, "out.2.conv.weight"), _need(weights, "out.2.conv.bias"),
                       norm=(_need(weights, "out.0.weight"), _need(weights, "out.0.bias")), num_groups=groups,
                       eps=eps, apply_silu=True)
    return t_emb, y


class UNetGraph:
    """One ``denoise_unet`` pass recorded as a HIP graph (``torch.cuda.CUDAGraph``) for fixed input shapes
    and replayed per call.

    A production step issues several hundred kernel launches from Python; with the convolutions in bf16
    the eager step is bound by that issue rate (measured on MI355X: 7.5 ms of host issue for a 7.7 ms
    step), a replay issues them as one graph.  Every launch of the step (the HIP conv / norm / attention
    kernels, the PyTorch projections and element-wise ops) is recorded with the buffers it used; a replay
    therefore computes exactly what the eager pass computes (bit-identical, tested).

    Each call copies its inputs into the graph's static input buffers and returns the static outputs
    ``(t_emb, y)``, which the next call overwrites (clone them to keep them).  The weights, their packed
    copies and the precision mode (``fast_fp32.precision``) are those at construction; build a new graph
    after changing any of them.  Construction runs the step twice eagerly (filling the packed-weight and
    projection caches) before recording.  The graph holds its own references to every cached derived
    tensor the recording read (``fast_fp32.retain_cached``), so ``drop_packed_weights`` or a cache
    refresh cannot free memory its kernels still address.
    """

    def __init__(self, x: Tensor, timesteps: Tensor, class_labels: Optional[Tensor], spacing: Optional[Tensor],
                 weights: Mapping[str, Tensor], *, constructor: Mapping,
                 down_block_additional_residuals: Optional[Sequence[Tensor]] = None,
                 mid_block_additional_residual: Optional[Tensor] = None):
        if x.device.type != "cuda":
            raise ValueError("UNetGraph records GPU work; x must be a CUDA tensor")
        clone = lambda t: None if t is None else t.detach().clone()
        self._inputs = [clone(x), clone(timesteps), clone(class_labels), clone(spacing)]
        self._down = None if down_block_additional_residuals is None else [
            clone(r) for r in down_block_additional_residuals]
        self._mid = clone(mid_block_additional_residual)
        self._weights, self._constructor = weights, constructor
        self.precision = ff.active_precision()

        def run():
            return denoise_unet(*self._inputs, self._weights, constructor=self._constructor,
                                down_block_additional_residuals=self._down,
                                mid_block_additional_residual=self._mid)

        dev = x.device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                run()
        torch.cuda.current_stream(dev).wait_stream(side)
        self._graph = torch.cuda.CUDAGraph()
        self._retained: list[Tensor] = []
        with ff.retain_cached(self._retained), torch.cuda.graph(self._graph):
            self._out = run()

    @staticmethod
    def _fill(static: Optional[Tensor], value: Optional[Tensor], name: str) -> None:
        if static is None or value is None:
            if static is not value:
                raise ValueError(f"{name} must be given exactly when it was given at construction")
            return
        if tuple(value.shape) != tuple(static.shape) or value.dtype != static.dtype:
            raise ValueError(f"{name} {tuple(value.shape)}/{value.dtype} does not match the recorded "
                             f"{tuple(static.shape)}/{static.dtype}")
        static.copy_(value)

    def __call__(self, x: Tensor, timesteps: Tensor, class_labels: Optional[Tensor] = None,
                 spacing: Optional[Tensor] = None, *,
                 down_block_additional_residuals: Optional[Sequence[Tensor]] = None,
                 mid_block_additional_residual: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
        for static, value, name in zip(self._inputs, (x, timesteps, class_labels, spacing),
                                       ("x", "timesteps", "class_labels", "spacing")):
            self._fill(static, value, name)
        if (self._down is None) != (down_block_additional_residuals is None):
            raise ValueError("down_block_additional_residuals must be given exactly when recorded")
        if self._down is not None:
            if len(down_block_additional_residuals) != len(self._down):
                raise ValueError("ControlNet residual count differs from the recorded one")
            for i, (static, value) in enumerate(zip(self._down, down_block_additional_residuals)):
                self._fill(static, value, f"down residual {i}")
        self._fill(self._mid, mid_block_additional_residual, "mid_block_additional_residual")
        self._graph.replay()
        return self._out


def denoise_unet_ncdhw(x: Tensor, timesteps: Tensor, class_labels, spacing, weights, *, constructor, mx=None,
                       down_block_additional_residuals=None, mid_block_additional_residual=None):
    """NCDHW adapter with the reference's name and keywords (unet.py:42)."""
    down = None if down_block_additional_residuals is None else [ff.to_ndhwc(r) for r in down_block_additional_residuals]
    mid = None if mid_block_additional_residual is None else ff.to_ndhwc(mid_block_additional_residual)
    t_emb, y = denoise_unet(ff.to_ndhwc(x), timesteps, class_labels, spacing, weights, constructor=constructor,
                            down_block_additional_residuals=down, mid_block_additional_residual=mid)
    return t_emb, ff.to_ncdhw(y)


# ---------------------------------------------------------------------------
# ControlNet (controlnet.py:31-274)
# ---------------------------------------------------------------------------
def _check_controlnet(constructor: Mapping) -> tuple[int, ...]:
    if int(constructor.get("spatial_dims", 3)) != 3 or constructor.get("use_flash_attention"):
        raise ValueError("MAISI ControlNet destination is 3D without CUDA flash attention")
    if not constructor.get("resblock_updown", True) or constructor.get("with_conditioning"):
        raise ValueError("ddpm-ct / cross-attention ControlNet variants are not part of this path")
    return tuple(int(c) for c in constructor["conditioning_embedding_num_channels"])


def encode_controlnet_condition(cond: Tensor, weights: Mapping[str, Tensor], *, constructor: Mapping) -> Tensor:
    """Conditioning encoder on an NDHWC label condition (controlnet.py:167-249):
    conv_in -> SiLU, then per level a stride-1 conv -> SiLU and a stride-2 conv -> SiLU,
    then conv_out; output ``(N, D/s, H/s, W/s, num_channels[0])``."""
    channels = _check_controlnet(constructor)
    cond_in = int(constructor["conditioning_embedding_in_channels"])
    if cond.shape[-1] != cond_in:
        raise ValueError(f"controlnet cond channels {cond.shape[-1]} != {cond_in}")
    scale = 2 ** (len(channels) - 1)
    if any(int(s) % scale for s in cond.shape[1:4]):
        raise ValueError(f"controlnet cond spatial sizes must be multiples of {scale}")
    p = "controlnet_cond_embedding"
    hidden = ff.silu(ff.conv3d(cond, weights[f"{p}.conv_in.conv.weight"], weights[f"{p}.conv_in.conv.bias"], padding=1))
    block = 0
    for _ in range(len(channels) - 1):
        for stride in (1, 2):
            hidden = ff.silu(ff.conv3d(hidden, _need(weights, f"{p}.blocks.{block}.conv.weight"),
                                       _need(weights, f"{p}.blocks.{block}.conv.bias"), padding=1, stride=stride))
            block += 1
    return ff.conv3d(hidden, _need(weights, f"{p}.conv_out.conv.weight"), _need(weights, f"{p}.conv_out.conv.bias"),
                     padding=1)


def _zero_conv(x: Tensor, weights: Mapping[str, Tensor], prefix: str) -> Tensor:
    """1x1 zero convolution, wrapped (``.conv.weight``) or raw naming (controlnet.py:252-266)."""
    for key in (f"{prefix}.conv", prefix):
        if f"{key}.weight" in weights:
            return ff.pointwise_conv(x, weights[f"{key}.weight"], _need(weights, f"{key}.bias"))
    raise ValueError(f"ControlNet weights missing: {prefix}.conv.weight or {prefix}.weight")


def controlnet_residuals(
    x: Tensor,
    timesteps: Tensor,
    class_labels: Optional[Tensor],
    cond: Tensor,
    weights: Mapping[str, Tensor],
    *,
    constructor: Mapping,
    conditioning_scale: float = 1.0,
    conditioning_embedding: Optional[Tensor] = None,
) -> tuple[list[Tensor], Tensor]:
    """ControlNetMaisi on NDHWC ``x``/``cond``: ``(down, mid)`` residuals for the UNet (controlnet.py:31-164)."""
    cond_channels = _check_controlnet(constructor)
    if x.shape[-1] != int(constructor["in_channels"]):
        raise ValueError(f"controlnet latent channels {x.shape[-1]} != in_channels {constructor['in_channels']}")
    scale = 2 ** (len(cond_channels) - 1)
    if conditioning_embedding is None:
        expected = tuple(int(s) * scale for s in x.shape[1:4])
        if tuple(int(s) for s in cond.shape[1:4]) != expected:
            raise ValueError(f"controlnet cond spatial {tuple(cond.shape[1:4])} must be {scale}x latent")
    channels = tuple(int(c) for c in constructor["num_channels"])
    if conditioning_embedding is not None:  # controlnet.py:96-104
        expected = (int(x.shape[0]), *(int(s) for s in x.shape[1:4]), channels[0])
        if tuple(int(s) for s in conditioning_embedding.shape) != expected:
            raise ValueError(f"controlnet conditioning embedding shape {tuple(conditioning_embedding.shape)} "
                             f"must be {expected}")
        if conditioning_embedding.dtype != torch.float32:
            raise ValueError("controlnet conditioning embedding must be float32")
    n_levels = len(channels)
    res_blocks = _per_level(constructor["num_res_blocks"], n_levels)
    attn_levels = tuple(bool(a) for a in constructor["attention_levels"])
    heads = _per_level(constructor["num_head_channels"], n_levels)
    groups, eps = int(constructor["norm_num_groups"]), float(constructor["norm_eps"])
    include_fc = bool(constructor.get("include_fc", True))
    t_emb = sinusoidal_timestep_embedding(timesteps, channels[0])
    emb = _silu_mlp(t_emb, weights, "time_embed")
    if constructor.get("num_class_embeds") is not None:
        if class_labels is None:
            raise ValueError("class_labels should be provided when num_class_embeds > 0")
        emb = emb + _need(weights, "class_embedding.weight")[class_labels.to(torch.long)]
    resnet, attention = _blocks(weights, emb, groups, eps, include_fc)
    hidden = ff.conv3d(x, _need(weights, "conv_in.conv.weight"), _need(weights, "conv_in.conv.bias"), padding=1)
    embedding = (encode_controlnet_condition(cond, weights, constructor=constructor)
                 if conditioning_embedding is None else conditioning_embedding)
    hidden = ff.add_with_stats(hidden, embedding)  # with the statistics of the first block's norm1
    hidden, skips = _down_path(hidden, resnet, attention, res_blocks, attn_levels, heads)
    hidden = _mid_block(hidden, resnet, attention, heads[-1])
    down = [_zero_conv(s, weights, f"controlnet_down_blocks.{i}") for i, s in enumerate(skips)]
    mid = _zero_conv(hidden, weights, "controlnet_mid_block")
    if conditioning_scale != 1.0:
        down = [d * conditioning_scale for d in down]
        mid = mid * conditioning_scale
    return down, mid


_side_streams: dict[int, "torch.cuda.Stream"] = {}


def controlnet_unet_step(
    x: Tensor,
    timesteps: Tensor,
    class_labels: Optional[Tensor],
    spacing: Optional[Tensor],
    unet_weights: Mapping[str, Tensor],
    controlnet_weights: Mapping[str, Tensor],
    *,
    unet_constructor: Mapping,
    controlnet_constructor: Mapping,
    cond: Optional[Tensor] = None,
    conditioning_embedding: Optional[Tensor] = None,
    conditioning_scale: float = 1.0,
) -> tuple[Tensor, Tensor]:
    """One CT-from-mask denoiser evaluation: the ControlNet's residuals fed to the UNet
    (``controlnet_residuals`` then ``denoise_unet``), with the ControlNet issued on a second stream of
    default priority so it runs while the UNet's encoder (which does not read the residuals) runs on the
    current one; the current stream waits for the residuals after the encoder.  Same kernels, same inputs
    per kernel: the result equals the serial composition bit for bit.  Returns ``(t_emb, y)``."""
    if x.device.type != "cuda":
        raise ValueError("controlnet_unet_step runs on the GPU; x must be a CUDA tensor")
    main = torch.cuda.current_stream(x.device)
    side = _side_streams.get(x.device.index)
    if side is None:
        side = _side_streams.setdefault(x.device.index, torch.cuda.Stream(device=x.device))
    side.wait_stream(main)  # inputs written on the current stream
    with torch.cuda.stream(side):
        down, mid = controlnet_residuals(x, timesteps, class_labels, cond, controlnet_weights,
                                         constructor=controlnet_constructor, conditioning_scale=conditioning_scale,
                                         conditioning_embedding=conditioning_embedding)
        ready = torch.cuda.Event()
        ready.record(side)
    for r in (*down, mid):  # read on the current stream: keep their memory until that use is done
        r.record_stream(main)
    return denoise_unet(x, timesteps, class_labels, spacing, unet_weights, constructor=unet_constructor,
                        down_block_additional_residuals=down, mid_block_additional_residual=mid,
                        residuals_ready=ready)


def controlnet_residuals_ncdhw(x, timesteps, class_labels, cond, weights, *, constructor, mx=None,
                               conditioning_scale=1.0, conditioning_embedding=None):
    emb = None if conditioning_embedding is None else ff.to_ndhwc(conditioning_embedding)
    down, mid = controlnet_residuals(ff.to_ndhwc(x), timesteps, class_labels, ff.to_ndhwc(cond), weights,
                                     constructor=constructor, conditioning_scale=conditioning_scale,
                                     conditioning_embedding=emb)
    return [ff.to_ncdhw(d) for d in down], ff.to_ncdhw(mid)


# ---------------------------------------------------------------------------
# VAE decoder (vae.py:29-62, 273-379, 465-487)
# ---------------------------------------------------------------------------
def _conv_weights(weights: Mapping[str, Tensor], prefix: str) -> tuple[Tensor, Tensor]:
    """MAISI-wrapped (``conv.conv``) or plain (``conv``) convolution weights (vae.py:527-537)."""
    for key in (f"{prefix}.conv.conv", f"{prefix}.conv"):
        if f"{key}.weight" in weights:
            return weights[f"{key}.weight"], _need(weights, f"{key}.bias")
    raise ValueError(f"VAE weights missing: {prefix}.conv.conv.weight or {prefix}.conv.weight")


def run_vae_decoder(x: Tensor, weights: Mapping[str, Tensor], *, constructor: Mapping) -> Tensor:
    """MaisiDecoder on an NDHWC post-quant latent (vae.py:273-379)."""
    channels = tuple(int(c) for c in constructor["num_channels"])
    res_blocks = tuple(int(r) for r in constructor["num_res_blocks"])
    if any(bool(a) for a in constructor["attention_levels"]):
        raise ValueError("image VAE dest has no attention blocks")
    if constructor.get("use_convtranspose"):
        raise ValueError("transposed-convolution upsampling is not part of this path")
    groups, eps = int(constructor["norm_num_groups"]), float(constructor["norm_eps"])
    hidden = ff.conv3d(x, *_conv_weights(weights, "decoder.blocks.0"), padding=1, gn_groups=groups)
    index = 1
    rev = channels[::-1]
    for level, n_res in enumerate(res_blocks[::-1]):
        for r in range(n_res):
            p = f"decoder.blocks.{index}"
            shortcut = _conv_weights(weights, f"{p}.nin_shortcut") if any(
                k.startswith(f"{p}.nin_shortcut.") for k in weights) else None
            state = [hidden]
            del hidden
            hidden = ff.vae_resblock(state, _conv_weights(weights, f"{p}.conv1"), _conv_weights(weights, f"{p}.conv2"),
                                     (_need(weights, f"{p}.norm1.weight"), _need(weights, f"{p}.norm1.bias")),
                                     (_need(weights, f"{p}.norm2.weight"), _need(weights, f"{p}.norm2.bias")),
                                     shortcut, num_groups=groups, eps=eps,
                                     out_gn_groups=groups if r < n_res - 1 or level == len(rev) - 1 else 0)
            index += 1
        if level != len(rev) - 1:
            w, b = _conv_weights(weights, f"decoder.blocks.{index}.conv")
            hidden = ff.trilinear_conv3d(hidden, w, b, gn_groups=groups)
            index += 1
    norm = (_need(weights, f"decoder.blocks.{index}.weight"), _need(weights, f"decoder.blocks.{index}.bias"))
    return ff.norm_conv3d(hidden, *_conv_weights(weights, f"decoder.blocks.{index + 1}"), norm=norm,
                          num_groups=groups, eps=eps, apply_silu=False)


def decode_vae(latent: Tensor, weights: Mapping[str, Tensor], *, constructor: Mapping) -> tuple[Tensor, Tensor]:
    """``(post_quant, decoded)`` of an NDHWC latent (vae.py:29-62)."""
    if constructor.get("with_encoder_nonlocal_attn") or constructor.get("with_decoder_nonlocal_attn"):
        raise ValueError("image VAE dest has no nonlocal attention")
    post_quant = ff.pointwise_conv(latent, *_conv_weights(weights, "post_quant_conv"))
    return post_quant, run_vae_decoder(post_quant, weights, constructor=constructor)


def decode_vae_ncdhw(latent: Tensor, weights, *, constructor, mx=None):
    post_quant, decoded = decode_vae(ff.to_ndhwc(latent), weights, constructor=constructor)
    return ff.to_ncdhw(post_quant), ff.to_ncdhw(decoded)


# ---------------------------------------------------------------------------
# sliding-window decode (decode.py:30-245)
# ---------------------------------------------------------------------------
DEFAULT_ROI_SIZE = (48, 48, 64)
DEFAULT_OVERLAP = 0.6666
DEFAULT_SIGMA_SCALE = 0.125
DEFAULT_MODE = "gaussian"


def _check_roi(roi: Sequence[int]) -> tuple[int, int, int]:
    """Three positive window sizes (decode.py _check_roi)."""
    if len(roi) != 3:
        raise ValueError(f"roi must be three positive ints; got {tuple(roi)}")
    windows = (int(roi[0]), int(roi[1]), int(roi[2]))
    if any(v < 1 for v in windows):
        raise ValueError(f"roi must be three positive ints; got {windows}")
    return windows


def _check_overlap(overlap: float) -> None:
    """``0 <= overlap < 1`` (decode.py _check_overlap)."""
    if not 0.0 <= float(overlap) < 1.0:
        raise ValueError(f"overlap must be >= 0 and < 1; got {overlap}")


def _spatial3(values: Sequence[int], name: str) -> tuple[int, int, int]:
    if len(values) != 3:
        raise ValueError(f"{name} must have 3 spatial axes; got {tuple(values)}")
    out = (int(values[0]), int(values[1]), int(values[2]))
    if any(v < 1 for v in out):
        raise ValueError(f"{name} must be positive; got {out}")
    return out


def scan_interval(image_size: Sequence[int], roi: Sequence[int], overlap: float) -> tuple[int, int, int]:
    """``int(roi * (1 - overlap))`` (at least 1), or ``roi`` where it equals the axis (decode.py:30-45).

    Raises:
        ValueError: on a roi that is not three positive sizes, an overlap outside [0, 1) or a
            non-positive image size."""
    roi = _check_roi(roi)
    _check_overlap(overlap)
    out = []
    for size, window in zip(_spatial3(image_size, "image_size"), roi):
        if window == size:
            out.append(int(window))
            continue
        step = int(window * (1.0 - float(overlap)))
        out.append(step if step > 0 else 1)
    return out[0], out[1], out[2]


def dense_patch_slices(image_size: Sequence[int], patch: Sequence[int], interval: Sequence[int]):
    """Window slices; the last start of each axis is pulled back inside (decode.py:48-78)."""
    image_size, patch, interval = _spatial3(image_size, "image_size"), _check_roi(patch), _spatial3(interval,
                                                                                                   "interval")
    starts = []
    for size, window, step in zip(image_size, patch, interval):
        count = int(math.ceil(float(size) / float(step)))
        last = next((i for i in range(count) if i * step + window >= size), None)
        n_starts = 1 if last is None else last + 1
        axis = []
        for i in range(n_starts):
            start = i * step
            start -= max(start + window - size, 0)
            axis.append(start)
        starts.append(axis)
    return tuple((slice(a, a + patch[0]), slice(b, b + patch[1]), slice(c, c + patch[2]))
                 for a, b, c in product(*starts))


def gaussian_importance(roi: Sequence[int], sigma_scale: float = 0.125, device=None) -> Tensor:
    """Outer product of 1-D Gaussians, floored at 1e-3, ``(D, H, W)`` fp32 (decode.py:81-101)."""
    roi = _check_roi(roi)
    if float(sigma_scale) <= 0.0:
        raise ValueError(f"sigma_scale must be > 0; got {sigma_scale}")
    axes = []
    for length in roi:
        half = (length - 1) / 2.0
        x = torch.arange(-half, half + 1.0, dtype=torch.float32, device=device)
        sigma = float(sigma_scale) * float(length)
        axes.append(torch.exp((x * x) / (-2.0 * sigma * sigma)))
    imp = axes[0].reshape(-1, 1, 1) * axes[1].reshape(1, -1, 1) * axes[2].reshape(1, 1, -1)
    return torch.clamp(imp, min=_GAUSSIAN_FLOOR)


def sliding_window(latent: Tensor, predict: Callable[[Tensor], Tensor], *, roi: Sequence[int] = DEFAULT_ROI_SIZE,
                   overlap: float = DEFAULT_OVERLAP, sigma_scale: float = DEFAULT_SIGMA_SCALE,
                   mode: str = DEFAULT_MODE, z_scale: int = Z_SCALE) -> Tensor:
    """Blend ``predict`` over overlapping NDHWC latent windows (decode.py:104-184).

    Each window's prediction is weighted by the nearest-x4-resized Gaussian and
    accumulated with the weights in window order; the result is the ratio.

    Raises:
        ValueError: if ``mode`` is not ``"gaussian"``, ``z_scale`` is not 4, the window or
            overlap is invalid, or ``predict`` returns the wrong size (decode.py:132-146).
    """
    if mode != DEFAULT_MODE:
        raise ValueError(f"from-mask dest mode is {DEFAULT_MODE!r}; got {mode!r}")
    if int(z_scale) != Z_SCALE:
        raise ValueError(f"image VAE dest z_scale is {Z_SCALE}; got {z_scale}")
    roi = _check_roi(roi)
    _check_overlap(overlap)
    n, d, h, w, c = latent.shape
    pads = []
    for size, window in zip((d, h, w), roi):
        extra = max(int(window) - int(size), 0)
        pads.append((extra // 2, extra - extra // 2))
    if any(a or b for a, b in pads):
        latent = F.pad(latent, (0, 0, pads[2][0], pads[2][1], pads[1][0], pads[1][1], pads[0][0], pads[0][1]))
    spatial = tuple(int(s) for s in latent.shape[1:4])
    interval = scan_interval(spatial, roi, overlap)
    windows = dense_patch_slices(spatial, roi, interval)
    weight = gaussian_importance(roi, sigma_scale, device=latent.device)
    for axis in range(3):
        weight = weight.repeat_interleave(z_scale, dim=axis)
    weight = weight.unsqueeze(-1)
    with gc_paused():
        output, weight_sum = _blend_windows(latent, predict, windows, weight, roi, spatial, z_scale)
    stitched = output / weight_sum
    sl = [slice(a * z_scale, stitched.shape[i + 1] - b * z_scale) for i, (a, b) in enumerate(pads)]
    return stitched[:, sl[0], sl[1], sl[2], :].contiguous()


def _blend_windows(latent: Tensor, predict: Callable[[Tensor], Tensor], windows, weight: Tensor, roi, spatial,
                   z_scale: int) -> tuple[Tensor, Tensor]:
    """Sum of the Gaussian-weighted window predictions and of the weights, in window order."""
    output = weight_sum = None
    for sd, sh, sw in windows:
        pred = predict(latent[:, sd, sh, sw, :].contiguous())
        expected = tuple(int(r) * z_scale for r in roi)
        if tuple(pred.shape[1:4]) != expected:
            raise ValueError(f"prediction spatial shape {tuple(pred.shape[1:4])} != {expected}")
        od = slice(sd.start * z_scale, sd.stop * z_scale)
        oh = slice(sh.start * z_scale, sh.stop * z_scale)
        ow = slice(sw.start * z_scale, sw.stop * z_scale)
        if output is None:
            out_spatial = tuple(s * z_scale for s in spatial)
            output = torch.zeros((pred.shape[0], *out_spatial, pred.shape[-1]), device=pred.device)
            weight_sum = torch.zeros((1, *out_spatial, 1), device=pred.device)
        output[:, od, oh, ow, :] += pred * weight
        weight_sum[:, od, oh, ow, :] += weight
        del pred
    return output, weight_sum


def sliding_window_decode(latent: Tensor, weights: Mapping[str, Tensor], *, constructor: Mapping,
                          roi: Sequence[int] = DEFAULT_ROI_SIZE, overlap: float = DEFAULT_OVERLAP,
                          sigma_scale: float = DEFAULT_SIGMA_SCALE, mode: str = DEFAULT_MODE,
                          scale_factor: Optional[float] = None) -> Tensor:
    """Decode an NDHWC latent, tiling with Gaussian-blended windows when larger than ``roi``
    (decode.py:187-245).  As in the reference, the one-pass branch validates ``roi`` only;
    ``overlap``, ``sigma_scale`` and ``mode`` are validated when tiling."""
    roi = _check_roi(roi)
    if scale_factor is not None:
        value = float(scale_factor)
        if not math.isfinite(value) or value == 0.0:
            raise ValueError("scale_factor must be a finite non-zero caller value")
        latent = latent / value
    spatial = tuple(int(s) for s in latent.shape[1:4])

    def decode_window(window: Tensor) -> Tensor:
        return decode_vae(window, weights, constructor=constructor)[1]

    if math.prod(spatial) <= math.prod(roi):
        return decode_window(latent)
    adjusted = tuple(min(r, s) for r, s in zip(roi, spatial))
    return sliding_window(latent, decode_window, roi=adjusted, overlap=overlap, sigma_scale=sigma_scale, mode=mode)


def sliding_window_decode_ncdhw(latent: Tensor, weights, *, constructor, mx=None, roi=DEFAULT_ROI_SIZE,
                                overlap=DEFAULT_OVERLAP, sigma_scale=DEFAULT_SIGMA_SCALE, mode=DEFAULT_MODE,
                                scale_factor=None) -> Tensor:
    return ff.to_ncdhw(sliding_window_decode(ff.to_ndhwc(latent), weights, constructor=constructor, roi=roi,
                                             overlap=overlap, sigma_scale=sigma_scale, mode=mode,
                                             scale_factor=scale_factor))


# ---------------------------------------------------------------------------
# rectified-flow sampler (rflow.py:19-177) and guidance (image.py:118-175)
# ---------------------------------------------------------------------------
def timestep_transform_rflow(t: float, input_img_size_numel: int, *, base_img_size_numel: int = _BASE_NUMEL,
                             scale: float = 1.0, num_train_timesteps: int = _TRAIN_STEPS,
                             spatial_dim: int = 3) -> float:
    unit = float(t) / float(num_train_timesteps)
    ratio = (float(input_img_size_numel) / float(base_img_size_numel)) ** (1.0 / float(spatial_dim)) * float(scale)
    return float(num_train_timesteps) * ratio * unit / (1.0 + (ratio - 1.0) * unit)


def set_timesteps_rflow(*, num_inference_steps: int = 30, num_train_timesteps: int = _TRAIN_STEPS,
                        input_img_size_numel: int, base_img_size_numel: int = _BASE_NUMEL):
    """``(timesteps, next_timesteps)`` float32, rounded through float16 (rflow.py:47-97)."""
    if num_inference_steps < 1 or num_inference_steps > num_train_timesteps:
        raise ValueError(f"num_inference_steps {num_inference_steps} must be in 1..{num_train_timesteps}")
    steps = [timestep_transform_rflow((1.0 - i / num_inference_steps) * num_train_timesteps, input_img_size_numel,
                                      base_img_size_numel=base_img_size_numel,
                                      num_train_timesteps=num_train_timesteps)
             for i in range(num_inference_steps)]
    timesteps = np.asarray(steps, dtype=np.float16).astype(np.float32)
    return timesteps, np.concatenate([timesteps[1:], np.zeros((1,), dtype=np.float32)])


def step_rflow(z: Tensor, v: Tensor, timestep: float, next_timestep: float,
               num_train_timesteps: int = _TRAIN_STEPS) -> tuple[Tensor, Tensor, float]:
    """Euler step with ``dt = (t - int(next_t)) / T`` (rflow.py:100-119)."""
    dt = (float(timestep) - int(float(next_timestep))) / float(num_train_timesteps)
    return z + v * dt, z + v * (float(timestep) / float(num_train_timesteps)), dt


@contextlib.contextmanager
def gc_paused():
    """Pause Python's cyclic garbage collector for a multi-step GPU loop, restoring its state after.

    Every tensor of a step is freed by reference counting; what the pause avoids is a full
    collection landing inside the loop: it walks every tracked object of the process (about 270k
    with torch imported, 60-105 ms measured on the MI355X host, four UNet steps) while the GPU
    idles behind the stalled launch thread.  ``timeit`` pauses it the same way.
    """
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()


def sample_rflow(z: Tensor, velocity_fn: Callable[[Tensor, float], Tensor], timesteps: np.ndarray) -> Tensor:
    """Integrate ``z`` over the schedule (rflow.py:144-177); the cyclic collector is paused meanwhile
    (``gc_paused``)."""
    nxt = np.concatenate([timesteps[1:], np.zeros((1,), dtype=np.float32)])
    hidden = z
    with gc_paused():
        for t, tn in zip(timesteps.tolist(), nxt.tolist()):
            hidden, _, _ = step_rflow(hidden, velocity_fn(hidden, float(t)), float(t), float(tn))
    return hidden


def guided_velocity(state: Tensor, timestep: float, *, class_labels: Tensor, spacing: Tensor,
                    weights: Mapping[str, Tensor], constructor: Mapping, guidance_scale: float,
                    guidance_execution: str = "batched", unet: Optional[Callable] = None) -> Tensor:
    """Velocity with modality CFG: ``uncond + g * (cond - uncond)``, class 0 unconditional
    (image.py:118-175).  ``state`` is NDHWC.  ``unet`` replaces ``denoise_unet`` for the UNet passes
    (called as ``unet(x, timesteps, class_labels, spacing)``), e.g. a ``UNetGraph`` recorded for the
    batched-guidance shapes."""
    t = torch.full((state.shape[0],), float(timestep), dtype=torch.float32, device=state.device)
    if unet is None:
        unet = lambda xx, tt, cc, ss: denoise_unet(xx, tt, cc, ss, weights, constructor=constructor)
    if guidance_scale == 0.0:
        return unet(state, t, class_labels, spacing)[1]
    if guidance_execution == "sequential":
        cond = unet(state, t, class_labels, spacing)[1].clone()
        uncond = unet(state, t, torch.zeros_like(class_labels), spacing)[1]
        return uncond + guidance_scale * (cond - uncond)
    if guidance_execution != "batched":
        raise ValueError("guidance_execution must be 'batched' or 'sequential'")
    batch = state.shape[0]
    _, velocity = unet(torch.cat([state, state]), torch.cat([t, t]),
                       torch.cat([class_labels, torch.zeros_like(class_labels)]), torch.cat([spacing, spacing]))
    cond, uncond = velocity[:batch], velocity[batch:]
    return uncond + guidance_scale * (cond - uncond)


# ---------------------------------------------------------------------------
# production constructors and weight catalogs (random-init configs)
# ---------------------------------------------------------------------------
PRODUCTION_UNET_CONSTRUCTOR = {
    # maisi_mlx_from_mask.py:43-62 of the reference
    "spatial_dims": 3, "in_channels": 4, "out_channels": 4, "num_channels": [64, 128, 256, 512],
    "attention_levels": [False, False, True, True], "num_head_channels": [0, 0, 32, 32], "num_res_blocks": 2,
    "norm_num_groups": 32, "norm_eps": 1e-6, "use_flash_attention": False, "include_top_region_index_input": False,
    "include_bottom_region_index_input": False, "include_spacing_input": True, "num_class_embeds": 128,
    "resblock_updown": True, "include_fc": True, "with_conditioning": False, "use_combined_linear": False,
}
PRODUCTION_VAE_CONSTRUCTOR = {
    # maisi_mlx_from_mask.py:20-42 of the reference
    "spatial_dims": 3, "in_channels": 1, "out_channels": 1, "latent_channels": 4, "num_channels": [64, 128, 256],
    "num_res_blocks": [2, 2, 2], "norm_num_groups": 32, "norm_eps": 1e-6, "attention_levels": [False, False, False],
    "with_encoder_nonlocal_attn": False, "with_decoder_nonlocal_attn": False, "include_fc": False,
    "use_combined_linear": False, "use_flash_attention": False, "use_checkpointing": False,
    "use_convtranspose": False, "num_splits": 4, "dim_split": 1, "norm_float16": False, "print_info": False,
    "save_mem": False,
}


def _resnet_shapes(prefix: str, cin: int, cout: int, temb: int) -> list[tuple[str, tuple[int, ...]]]:
    out = [(f"{prefix}.norm1.weight", (cin,)), (f"{prefix}.norm1.bias", (cin,)),
           (f"{prefix}.conv1.conv.weight", (cout, cin, 3, 3, 3)), (f"{prefix}.conv1.conv.bias", (cout,)),
           (f"{prefix}.time_emb_proj.weight", (cout, temb)), (f"{prefix}.time_emb_proj.bias", (cout,)),
           (f"{prefix}.norm2.weight", (cout,)), (f"{prefix}.norm2.bias", (cout,)),
           (f"{prefix}.conv2.conv.weight", (cout, cout, 3, 3, 3)), (f"{prefix}.conv2.conv.bias", (cout,))]
    if cin != cout:
        out += [(f"{prefix}.skip_connection.conv.weight", (cout, cin, 1, 1, 1)),
                (f"{prefix}.skip_connection.conv.bias", (cout,))]
    return out


def _attention_shapes(prefix: str, c: int) -> list[tuple[str, tuple[int, ...]]]:
    out = [(f"{prefix}.norm.weight", (c,)), (f"{prefix}.norm.bias", (c,))]
    for name in ("to_q", "to_k", "to_v", "out_proj"):
        out += [(f"{prefix}.attn.{name}.weight", (c, c)), (f"{prefix}.attn.{name}.bias", (c,))]
    return out


def unet_weight_shapes(constructor: Mapping) -> list[tuple[str, tuple[int, ...]]]:
    """MONAI state-dict names and shapes of DiffusionModelUNetMaisi for ``constructor``."""
    ch = [int(c) for c in constructor["num_channels"]]
    nl = len(ch)
    nres = _per_level(constructor["num_res_blocks"], nl)
    attn = [bool(a) for a in constructor["attention_levels"]]
    t = 4 * ch[0]
    temb = t + (t if constructor.get("include_spacing_input") else 0)
    s = [("time_embed.0.weight", (t, ch[0])), ("time_embed.0.bias", (t,)), ("time_embed.2.weight", (t, t)),
         ("time_embed.2.bias", (t,))]
    if constructor.get("num_class_embeds") is not None:
        s.append(("class_embedding.weight", (int(constructor["num_class_embeds"]), t)))
    if constructor.get("include_spacing_input"):
        s += [("spacing_layer.0.weight", (t, 3)), ("spacing_layer.0.bias", (t,)), ("spacing_layer.2.weight", (t, t)),
              ("spacing_layer.2.bias", (t,))]
    s += [("conv_in.conv.weight", (ch[0], int(constructor["in_channels"]), 3, 3, 3)), ("conv_in.conv.bias", (ch[0],))]
    out_ch = ch[0]
    for i in range(nl):
        in_ch, out_ch = out_ch, ch[i]
        for r in range(nres[i]):
            s += _resnet_shapes(f"down_blocks.{i}.resnets.{r}", in_ch if r == 0 else out_ch, out_ch, temb)
            if attn[i]:
                s += _attention_shapes(f"down_blocks.{i}.attentions.{r}", out_ch)
        if i != nl - 1:
            s += _resnet_shapes(f"down_blocks.{i}.downsampler", out_ch, out_ch, temb)
    s += _resnet_shapes("middle_block.resnet_1", ch[-1], ch[-1], temb)
    s += _attention_shapes("middle_block.attention", ch[-1])
    s += _resnet_shapes("middle_block.resnet_2", ch[-1], ch[-1], temb)
    rc, rres, rattn = ch[::-1], nres[::-1], attn[::-1]
    out_ch = rc[0]
    for i in range(nl):
        prev, out_ch = out_ch, rc[i]
        in_ch = rc[min(i + 1, nl - 1)]
        n = rres[i] + 1
        for r in range(n):
            skip_ch = in_ch if r == n - 1 else out_ch
            s += _resnet_shapes(f"up_blocks.{i}.resnets.{r}", (prev if r == 0 else out_ch) + skip_ch, out_ch, temb)
            if rattn[i]:
                s += _attention_shapes(f"up_blocks.{i}.attentions.{r}", out_ch)
        if i != nl - 1:
            s += _resnet_shapes(f"up_blocks.{i}.upsampler", out_ch, out_ch, temb)
    s += [("out.0.weight", (ch[0],)), ("out.0.bias", (ch[0],)),
          ("out.2.conv.weight", (int(constructor["out_channels"]), ch[0], 3, 3, 3)),
          ("out.2.conv.bias", (int(constructor["out_channels"]),))]
    return s


PRODUCTION_CONTROLNET_CONSTRUCTOR = {
    # maisi_mlx_from_mask.py:63-80 of the reference
    "spatial_dims": 3, "in_channels": 4, "num_channels": [64, 128, 256, 512],
    "attention_levels": [False, False, True, True], "num_head_channels": [0, 0, 32, 32], "num_res_blocks": 2,
    "norm_num_groups": 32, "norm_eps": 1e-6, "use_flash_attention": False, "conditioning_embedding_in_channels": 8,
    "conditioning_embedding_num_channels": [8, 32, 64], "num_class_embeds": 128, "resblock_updown": True,
    "include_fc": True, "with_conditioning": False, "use_combined_linear": False,
}


def controlnet_weight_shapes(constructor: Mapping) -> list[tuple[str, tuple[int, ...]]]:
    """State-dict names and shapes of ControlNetMaisi for ``constructor`` (the first zero
    conv is a bare Conv3d, the others are wrapped, as in the released checkpoints)."""
    ch = [int(c) for c in constructor["num_channels"]]
    nl = len(ch)
    nres = _per_level(constructor["num_res_blocks"], nl)
    attn = [bool(a) for a in constructor["attention_levels"]]
    t = 4 * ch[0]
    s = [("time_embed.0.weight", (t, ch[0])), ("time_embed.0.bias", (t,)), ("time_embed.2.weight", (t, t)),
         ("time_embed.2.bias", (t,))]
    if constructor.get("num_class_embeds") is not None:
        s.append(("class_embedding.weight", (int(constructor["num_class_embeds"]), t)))
    s += [("conv_in.conv.weight", (ch[0], int(constructor["in_channels"]), 3, 3, 3)), ("conv_in.conv.bias", (ch[0],))]
    cc = [int(c) for c in constructor["conditioning_embedding_num_channels"]]
    p = "controlnet_cond_embedding"
    s += [(f"{p}.conv_in.conv.weight", (cc[0], int(constructor["conditioning_embedding_in_channels"]), 3, 3, 3)),
          (f"{p}.conv_in.conv.bias", (cc[0],))]
    block = 0
    for i in range(len(cc) - 1):
        for cout in (cc[i], cc[i + 1]):
            s += [(f"{p}.blocks.{block}.conv.weight", (cout, cc[i], 3, 3, 3)), (f"{p}.blocks.{block}.conv.bias", (cout,))]
            block += 1
    s += [(f"{p}.conv_out.conv.weight", (ch[0], cc[-1], 3, 3, 3)), (f"{p}.conv_out.conv.bias", (ch[0],))]
    temb = t
    out_ch = ch[0]
    skip_ch = [ch[0]]
    for i in range(nl):
        in_ch, out_ch = out_ch, ch[i]
        for r in range(nres[i]):
            s += _resnet_shapes(f"down_blocks.{i}.resnets.{r}", in_ch if r == 0 else out_ch, out_ch, temb)
            if attn[i]:
                s += _attention_shapes(f"down_blocks.{i}.attentions.{r}", out_ch)
            skip_ch.append(out_ch)
        if i != nl - 1:
            s += _resnet_shapes(f"down_blocks.{i}.downsampler", out_ch, out_ch, temb)
            skip_ch.append(out_ch)
    s += _resnet_shapes("middle_block.resnet_1", ch[-1], ch[-1], temb)
    s += _attention_shapes("middle_block.attention", ch[-1])
    s += _resnet_shapes("middle_block.resnet_2", ch[-1], ch[-1], temb)
    for i, c in enumerate(skip_ch):
        key = f"controlnet_down_blocks.{i}" + ("" if i == 0 else ".conv")
        s += [(f"{key}.weight", (c, c, 1, 1, 1)), (f"{key}.bias", (c,))]
    s += [("controlnet_mid_block.conv.weight", (ch[-1], ch[-1], 1, 1, 1)), ("controlnet_mid_block.conv.bias", (ch[-1],))]
    return s


def vae_decoder_weight_shapes(constructor: Mapping) -> list[tuple[str, tuple[int, ...]]]:
    """State-dict names and shapes of the AutoencoderKlMaisi decode path for ``constructor``."""
    ch = [int(c) for c in constructor["num_channels"]]
    lat = int(constructor["latent_channels"])
    rc = ch[::-1]
    nres = [int(r) for r in constructor["num_res_blocks"]][::-1]
    s = [("post_quant_conv.conv.weight", (lat, lat, 1, 1, 1)), ("post_quant_conv.conv.bias", (lat,)),
         ("decoder.blocks.0.conv.conv.weight", (rc[0], lat, 3, 3, 3)), ("decoder.blocks.0.conv.conv.bias", (rc[0],))]
    idx, block_in = 1, rc[0]
    for level, n in enumerate(nres):
        block_out = rc[level]
        for _ in range(n):
            p = f"decoder.blocks.{idx}"
            s += [(f"{p}.norm1.weight", (block_in,)), (f"{p}.norm1.bias", (block_in,)),
                  (f"{p}.conv1.conv.conv.weight", (block_out, block_in, 3, 3, 3)), (f"{p}.conv1.conv.conv.bias", (block_out,)),
                  (f"{p}.norm2.weight", (block_out,)), (f"{p}.norm2.bias", (block_out,)),
                  (f"{p}.conv2.conv.conv.weight", (block_out, block_out, 3, 3, 3)),
                  (f"{p}.conv2.conv.conv.bias", (block_out,))]
            if block_in != block_out:
                s += [(f"{p}.nin_shortcut.conv.conv.weight", (block_out, block_in, 1, 1, 1)),
                      (f"{p}.nin_shortcut.conv.conv.bias", (block_out,))]
            block_in = block_out
            idx += 1
        if level != len(nres) - 1:
            s += [(f"decoder.blocks.{idx}.conv.conv.conv.weight", (block_in, block_in, 3, 3, 3)),
                  (f"decoder.blocks.{idx}.conv.conv.conv.bias", (block_in,))]
            idx += 1
    s += [(f"decoder.blocks.{idx}.weight", (block_in,)), (f"decoder.blocks.{idx}.bias", (block_in,)),
          (f"decoder.blocks.{idx + 1}.conv.conv.weight", (int(constructor["out_channels"]), block_in, 3, 3, 3)),
          (f"decoder.blocks.{idx + 1}.conv.conv.bias", (int(constructor["out_channels"]),))]
    return s


def random_weights(shapes: Sequence[tuple[str, tuple[int, ...]]], *, seed: int) -> dict[str, np.ndarray]:
    """Random-init fp32 weights (host): conv/linear ~ N(0, 1/fan_in), biases ~ N(0, 0.01^2),
    norm scales ~ 1 + N(0, 0.1^2), norm shifts ~ N(0, 0.1^2), embeddings ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in shapes:
        if len(shape) == 1:
            is_norm = ".norm" in name or name.startswith("out.0") or name.split(".")[-2].isdigit() and "conv" not in name
            if name.endswith("weight") and is_norm:
                v = 1.0 + 0.1 * rng.standard_normal(shape)
            else:
                v = (0.1 if is_norm else 0.01) * rng.standard_normal(shape)
        elif name == "class_embedding.weight":
            v = rng.standard_normal(shape)
        else:
            fan_in = int(np.prod(shape[1:]))
            v = rng.standard_normal(shape) / np.sqrt(fan_in)
        out[name] = v.astype(np.float32)
    return out


CONFIGURATIONS = ("ct", "mr", "mr-brain")


def output_intensities(decoded: np.ndarray, *, configuration: str = "ct") -> np.ndarray:
    """int16 image: CT ``clip(x*2000-1000, -1000, 1000)``, MR and MR-Brain ``max(x*1000, 0)`` (no
    upper clip), truncated (image.py:68-87).

    Raises:
        ValueError: for a configuration other than ``"ct"``, ``"mr"`` or ``"mr-brain"`` (the
            reference's InvalidInputError, configurations.py:188-200), or a non-finite image.
    """
    if not isinstance(configuration, str) or configuration not in CONFIGURATIONS:
        raise ValueError("configuration must be 'ct', 'mr', or 'mr-brain'")
    data = np.asarray(decoded, dtype=np.float32)
    if not np.isfinite(data).all():
        raise ValueError("decoded image must be finite")
    if configuration == "ct":
        scaled = np.clip(data * 2000.0 - 1000.0, -1000.0, 1000.0)
    else:
        scaled = np.clip(data * 1000.0, 0.0, None)
    return scaled.astype(np.int16)


def spacing_tensor(spacing_mm: Sequence[float], device=None) -> Tensor:
    """``spacing_mm * 100`` rounded through float16, ``(1, 3)`` fp32 (image.py:90-115)."""
    scaled = np.asarray([spacing_mm], dtype=np.float64) * 100.0
    return torch.from_numpy(scaled.astype(np.float16).astype(np.float32)).to(device)


# ---------------------------------------------------------------------------
# CT from a label mask: ControlNet-conditioned rflow sampling + windowed decode
# + label-masked Hounsfield units (from_mask.py:121-338, condition.py:20-62,
# decode.py:248-259)
# ---------------------------------------------------------------------------
CT_MODALITY = 1  # modality index "ct" of the reference's configurations table (default for CT)
LABEL_BITS = 8
BODY_LABEL = 200
VALID_LABELS = frozenset(range(133)) | {BODY_LABEL}  # MAISI ids 0..132 plus the body envelope
SUPPORTED_PRODUCTION_SHAPES = ((256, 256, 128), (256, 256, 256))
SEAM_NOT_APPLICABLE = "not_applicable_below_roi"
DEFAULT_STEPS = 30


def require_ct_label(label: np.ndarray) -> np.ndarray:
    """Host ``(N, 1, D, H, W)`` integer MAISI label map, validated (from_mask.py:355-378): ids in
    0..132 plus body 200, body present, spatial sizes multiples of 4."""
    host = np.asarray(label)
    if host.ndim != 5 or int(host.shape[1]) != 1:
        raise ValueError(f"label must be NCDHW with 1 channel; got {host.shape}")
    if not np.issubdtype(host.dtype, np.integer):
        raise ValueError(f"label must be integer; got {host.dtype}")
    unique = {int(v) for v in np.unique(host)}
    unknown = sorted(v for v in unique if v not in VALID_LABELS)
    if unknown:
        raise ValueError("MAISI mask contains labels outside 0..132 plus body label 200: "
                         + ", ".join(str(v) for v in unknown[:10]))
    if BODY_LABEL not in unique:
        raise ValueError("MAISI mask is missing body-envelope label 200; add it before generation")
    spatial = tuple(int(s) for s in host.shape[2:])
    if any(s % Z_SCALE for s in spatial):
        raise ValueError(f"label spatial {spatial} must be multiples of {Z_SCALE}")
    return host


def require_supported_production_shape(shape: Sequence[int]) -> tuple[int, int, int]:
    """The label grids the reference's from-mask sampler accepts (from_mask.py:101-118)."""
    spatial = tuple(int(v) for v in shape)
    if len(spatial) != 3:
        raise ValueError(f"MLX NV-Generate-CT mask shape must be 3D; got {spatial}")
    if spatial not in SUPPORTED_PRODUCTION_SHAPES:
        raise ValueError(f"from_mask shape {spatial} is not production-proven; supported shapes: "
                         "(256, 256, 128) and (256, 256, 256)")
    return spatial[0], spatial[1], spatial[2]


def require_scale_factor(scale_factor: float) -> float:
    """A finite non-zero latent scale from the UNet checkpoint; no default (from_mask.py:341-352)."""
    value = float(scale_factor)
    if not math.isfinite(value) or value == 0.0:
        raise ValueError(f"scale_factor must be a finite non-zero caller value; got {scale_factor!r}")
    return value


def binarize_labels(label: Tensor) -> Tensor:
    """The 8-channel ControlNet condition of an integer label map, NDHWC: channel ``k`` of the
    ``(N, D, H, W, 8)`` float32 result is bit ``k`` of the id, least significant first
    (condition.py:20-43).  ``label`` is ``(N, D, H, W)`` or ``(N, D, H, W, 1)`` integers."""
    if label.dim() == 5:
        if int(label.shape[-1]) != 1:
            raise ValueError(f"maisi label must have 1 channel; got {int(label.shape[-1])}")
        label = label[..., 0]
    if label.dim() != 4:
        raise ValueError(f"maisi label must be (N, D, H, W[, 1]); got {tuple(label.shape)}")
    ids = label.to(torch.int32).unsqueeze(-1)
    powers = torch.bitwise_left_shift(torch.ones(LABEL_BITS, dtype=torch.int32, device=label.device),
                                      torch.arange(LABEL_BITS, dtype=torch.int32, device=label.device))
    return (torch.bitwise_and(ids, powers) != 0).to(torch.float32).contiguous()


def ct_spacing_tensor(spacing_mm: Sequence[float], device=None) -> Tensor:
    """``spacing_mm * 100`` as a ``(1, 3)`` float32 tensor, no float16 rounding (the from-mask
    path, condition.py:46-62; the image-only path rounds, ``spacing_tensor``)."""
    if len(spacing_mm) != 3:
        raise ValueError(f"spacing_mm must have 3 values; got {tuple(spacing_mm)}")
    values = [float(v) * 100.0 for v in spacing_mm]
    if any(not math.isfinite(v) or v <= 0.0 for v in values):
        raise ValueError(f"spacing_mm * 100.0 must be finite and > 0; got {values}")
    return torch.tensor([values], dtype=torch.float32, device=device)


def to_hu(image: Tensor, label: Tensor) -> Tensor:
    """Decoded intensities to float32 Hounsfield units: ``clip(x, 0, 1) * 2000 - 1000``, and -1000
    where the label is background (0) (decode.py:248-259).  NDHWC ``image`` ``(N, D, H, W, 1)``;
    ``label`` of the same spatial shape, with or without the channel axis."""
    if label.dim() == image.dim() - 1:
        label = label.unsqueeze(-1)
    if tuple(label.shape) != tuple(image.shape):
        raise ValueError(f"label shape {tuple(label.shape)} does not match the image {tuple(image.shape)}")
    hu = torch.clamp(image, 0.0, 1.0) * 2000.0 - 1000.0
    return torch.where(label == 0, torch.full_like(hu, -1000.0), hu)


class FromMaskResult:
    """Outputs of ``sample_ct_from_mask`` (the reference's FromMaskArrays, from_mask.py:67-86), NDHWC on
    the GPU: ``latent`` the sampled latent before the scale division, ``decoded`` the VAE output,
    ``hu`` float32 Hounsfield units (label 0 forced to -1000), ``seam_audit`` ``"tiled"`` when the decode
    used more than one window, ``stage_timings_s`` synchronized wall-clock seconds per stage."""

    def __init__(self, latent, decoded, hu, scale_factor, num_inference_steps, seam_audit, stage_timings_s):
        self.latent, self.decoded, self.hu = latent, decoded, hu
        self.scale_factor, self.num_inference_steps = scale_factor, num_inference_steps
        self.seam_audit, self.stage_timings_s = seam_audit, dict(stage_timings_s)


def ct_velocity(cond_embedding: Tensor, class_labels: Tensor, spacing: Tensor, *, unet_weights, controlnet_weights,
                unet_constructor, controlnet_constructor, overlap_streams: bool = True) -> Callable[[Tensor, float], Tensor]:
    """The ControlNet-conditioned UNet velocity of one generation (from_mask.py:298-338): per step the
    ControlNet's residuals (from the conditioning embedding computed once) feed the UNet.  With
    ``overlap_streams`` the ControlNet runs on a second stream beside the UNet encoder
    (``controlnet_unet_step``; the same bits as the serial composition)."""

    def velocity(state: Tensor, timestep: float) -> Tensor:
        t = torch.full((state.shape[0],), float(timestep), dtype=torch.float32, device=state.device)
        if overlap_streams:
            return controlnet_unet_step(state, t, class_labels, spacing, unet_weights, controlnet_weights,
                                        unet_constructor=unet_constructor, controlnet_constructor=controlnet_constructor,
                                        conditioning_embedding=cond_embedding)[1]
        down, mid = controlnet_residuals(state, t, class_labels, None, controlnet_weights,
                                         constructor=controlnet_constructor, conditioning_embedding=cond_embedding)
        return denoise_unet(state, t, class_labels, spacing, unet_weights, constructor=unet_constructor,
                            down_block_additional_residuals=down, mid_block_additional_residual=mid)[1]

    return velocity


def _synced_time(device) -> float:
    import time

    torch.cuda.synchronize(device)
    return time.perf_counter()


def sample_ct_latent(label: np.ndarray, spacing_mm: Sequence[float], *, unet_weights: Mapping[str, Tensor],
                     controlnet_weights: Mapping[str, Tensor], unet_constructor: Mapping,
                     controlnet_constructor: Mapping, scale_factor: float, latent: Optional[Tensor] = None,
                     seed: Optional[int] = None, num_inference_steps: int = DEFAULT_STEPS,
                     guidance_scale: float = 0.0, device=None, overlap_streams: bool = True,
                     drop_weights: bool = True) -> tuple[Tensor, float]:
    """ControlNet-conditioned rflow sampling of a CT latent (from_mask.py:177-248); returns the NDHWC
    latent ``(N, D/4, H/4, W/4, 4)`` and the sampling seconds.

    The condition is encoded once; each of the ``num_inference_steps`` steps runs the ControlNet and
    the UNet at the label's batch (no guidance: ``guidance_scale`` must be 0).  ``latent`` (NDHWC) or
    ``seed`` gives the start: the reference draws it from MLX's generator, here ``seed`` seeds a torch
    generator on the device, so seeded latents differ from the reference's (pass ``latent`` for the
    same start).  With ``drop_weights`` the packed copies of both networks' weights are released after
    sampling, as the reference does before decoding (from_mask.py:240).
    """
    if float(guidance_scale) != 0.0:
        raise ValueError("CFG>0 majority vote is not an MLX destination")
    require_scale_factor(scale_factor)
    host = require_ct_label(label)
    device = torch.device(device) if device is not None else next(iter(unet_weights.values())).device
    n = int(host.shape[0])
    latent_shape = (n, *(int(s) // Z_SCALE for s in host.shape[2:]), 4)
    if latent is None:
        if seed is None:
            raise ValueError("seed is required when latent is omitted")
        gen = torch.Generator(device=device).manual_seed(int(seed))
        latent = torch.randn(latent_shape, generator=gen, device=device, dtype=torch.float32)
    elif tuple(int(s) for s in latent.shape) != latent_shape:
        raise ValueError(f"latent shape {tuple(int(s) for s in latent.shape)} != {latent_shape}")
    label_dev = torch.from_numpy(np.ascontiguousarray(host[:, 0])).to(device)
    cond = binarize_labels(label_dev)
    spacing = ct_spacing_tensor(spacing_mm, device=device).repeat(n, 1)
    class_labels = torch.full((n,), CT_MODALITY, dtype=torch.int64, device=device)
    timesteps, _ = set_timesteps_rflow(num_inference_steps=int(num_inference_steps),
                                       input_img_size_numel=int(np.prod(latent_shape[1:4])))
    start = _synced_time(device)
    embedding = encode_controlnet_condition(cond, controlnet_weights, constructor=controlnet_constructor)
    del cond
    velocity = ct_velocity(embedding, class_labels, spacing, unet_weights=unet_weights,
                           controlnet_weights=controlnet_weights, unet_constructor=unet_constructor,
                           controlnet_constructor=controlnet_constructor, overlap_streams=overlap_streams)
    final = sample_rflow(latent, velocity, timesteps)
    seconds = _synced_time(device) - start
    del embedding, velocity
    if drop_weights:
        ff.drop_packed_weights([*unet_weights.values(), *controlnet_weights.values()])
    return final, seconds


def decode_ct_latent(latent: Tensor, label: np.ndarray, *, vae_weights: Mapping[str, Tensor], vae_constructor: Mapping,
                     scale_factor: float, roi: Sequence[int] = DEFAULT_ROI_SIZE,
                     overlap: float = DEFAULT_OVERLAP) -> tuple[Tensor, Tensor, str, dict[str, float]]:
    """Windowed decode of a sampled CT latent and its label-masked HU image (from_mask.py:251-295):
    returns ``(decoded, hu, seam_audit, timings)``, NDHWC."""
    host = require_ct_label(label)
    factor = require_scale_factor(scale_factor)
    device = latent.device
    start = _synced_time(device)
    decoded = sliding_window_decode(latent, vae_weights, constructor=vae_constructor, roi=roi, overlap=overlap,
                                    scale_factor=factor)
    mid = _synced_time(device)
    hu = to_hu(decoded, torch.from_numpy(np.ascontiguousarray(host[:, 0])).to(device))
    end = _synced_time(device)
    spatial = tuple(int(s) for s in decoded.shape[1:4])
    seam = SEAM_NOT_APPLICABLE if math.prod(spatial) <= math.prod(int(r) * Z_SCALE for r in roi) else "tiled"
    return decoded, hu, seam, {"vae_decode": mid - start, "hu_postprocess": end - mid}


def sample_ct_from_mask(label: np.ndarray, spacing_mm: Sequence[float], *, unet_weights: Mapping[str, Tensor],
                        controlnet_weights: Mapping[str, Tensor], vae_weights: Mapping[str, Tensor],
                        unet_constructor: Mapping, controlnet_constructor: Mapping, vae_constructor: Mapping,
                        scale_factor: float, seed: Optional[int] = None, latent: Optional[Tensor] = None,
                        num_inference_steps: int = DEFAULT_STEPS, guidance_scale: float = 0.0,
                        roi: Sequence[int] = DEFAULT_ROI_SIZE, overlap: float = DEFAULT_OVERLAP,
                        overlap_streams: bool = True, drop_weights: bool = True) -> FromMaskResult:
    """A CT volume from a MAISI label map (from_mask.py:121-174): ControlNet-conditioned rflow sampling,
    then the windowed VAE decode of ``latent / scale_factor`` and the HU conversion.  ``label`` is a host
    ``(N, 1, D, H, W)`` integer array; results are NDHWC GPU tensors."""
    final, rflow_s = sample_ct_latent(label, spacing_mm, unet_weights=unet_weights,
                                      controlnet_weights=controlnet_weights, unet_constructor=unet_constructor,
                                      controlnet_constructor=controlnet_constructor, scale_factor=scale_factor,
                                      latent=latent, seed=seed, num_inference_steps=num_inference_steps,
                                      guidance_scale=guidance_scale, overlap_streams=overlap_streams,
                                      drop_weights=drop_weights)
    decoded, hu, seam, timings = decode_ct_latent(final, label, vae_weights=vae_weights,
                                                  vae_constructor=vae_constructor, scale_factor=scale_factor,
                                                  roi=roi, overlap=overlap)
    stages = {"rflow_controlnet_unet": rflow_s, **timings}
    stages["total_synchronized_inference"] = rflow_s + timings["vae_decode"] + timings["hu_postprocess"]
    return FromMaskResult(final, decoded, hu, float(scale_factor), int(num_inference_steps), seam, stages)
