"""PyTorch-CPU restatement of the MAISI networks — TEST INFRASTRUCTURE ONLY.

Unfused NCDHW math in float64 (or float32 for the full-size config checks),
written from the reference's *unfused* paths so it is independent of the fused
HIP composition it checks:
  residual block   residual.py:80-134 (GN, SiLU, up/down, conv1, +temb, GN, SiLU, conv2, +skip)
  attention        attention.py:92-160, 349-414 (GN, QKV, softmax(QK^T s)V, out_proj, +x)
  UNet             unet.py:42-487, embed.py:15-87
  VAE decoder      vae.py:29-62, 103-200, 273-379 (materialized trilinear upsampling)
  sliding window   decode.py:30-245
  ControlNet       controlnet.py:31-274
  CT from mask     from_mask.py:177-338 (sampling loop), condition.py:20-43 (label bits),
                   decode.py:248-259 (HU)
Pinned by the reference goldens in tests/golden (tests/test_oracle_networks.py).  The ControlNet
has no recorded outputs in the reference fixtures (its boundary arrays live outside the repository),
so it is pinned without a recording: its shared down path through the UNet goldens and an identity
invariant (identity zero convs and a zero condition give the UNet's skips), its conditioning encoder
against a brute-force loop, its first residual against conv_in plus the embedding, and the
conditioning scale against a closed form, each with planted mistakes that must fail
(tests/test_oracle_networks.py).
"""

from __future__ import annotations

import math
from collections.abc import Mapping, Sequence

import numpy as np
import torch
import torch.nn.functional as F

from . import reference_math as rm


def _pre(w: Mapping[str, torch.Tensor], prefix: str) -> dict[str, torch.Tensor]:
    s = prefix + "."
    return {k[len(s):]: v for k, v in w.items() if k.startswith(s)}


def _gn(x, weight, bias, groups, eps):
    return F.group_norm(x, groups, weight, bias, eps)


def residual_block(x, emb, w, groups, eps, up=False, down=False):
    """DiffusionUNetResnetBlock, unfused (residual.py:80-134)."""
    h = F.silu(_gn(x, w["norm1.weight"], w["norm1.bias"], groups, eps))
    skip = x
    if up:
        skip = F.interpolate(skip, scale_factor=2, mode="nearest")
        h = F.interpolate(h, scale_factor=2, mode="nearest")
    elif down:
        skip = F.avg_pool3d(skip, 2)
        h = F.avg_pool3d(h, 2)
    h = F.conv3d(h, w["conv1.conv.weight"], w["conv1.conv.bias"], padding=1)
    temb = F.linear(F.silu(emb), w["time_emb_proj.weight"], w["time_emb_proj.bias"])
    h = h + temb[:, :, None, None, None]
    h = F.silu(_gn(h, w["norm2.weight"], w["norm2.bias"], groups, eps))
    h = F.conv3d(h, w["conv2.conv.weight"], w["conv2.conv.bias"], padding=1)
    if "skip_connection.conv.weight" in w:
        skip = F.conv3d(skip, w["skip_connection.conv.weight"], w["skip_connection.conv.bias"])
    return skip + h


def attention(x, w, groups, eps, head_channels, include_fc):
    """Residual spatial self-attention (attention.py:92-160)."""
    n, c = x.shape[:2]
    heads = c // head_channels
    h = _gn(x, w["norm.weight"], w["norm.bias"], groups, eps)
    tokens = h.reshape(n, c, -1).transpose(1, 2)

    def split(t):
        return t.reshape(n, -1, heads, head_channels).transpose(1, 2)

    q = split(F.linear(tokens, w["attn.to_q.weight"], w["attn.to_q.bias"]))
    k = split(F.linear(tokens, w["attn.to_k.weight"], w["attn.to_k.bias"]))
    v = split(F.linear(tokens, w["attn.to_v.weight"], w["attn.to_v.bias"]))
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * (float(head_channels) ** -0.5)
    out = torch.matmul(torch.softmax(scores, dim=-1), v).transpose(1, 2).reshape(n, -1, c)
    if include_fc:
        out = F.linear(out, w["attn.out_proj.weight"], w["attn.out_proj.bias"])
    return x + out.transpose(1, 2).reshape(x.shape)


def timestep_embedding(t, dim, max_period=10000):
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32)
    freqs = torch.exp(exponent / half).to(t.dtype)
    args = t[:, None] * freqs[None, :]
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    return F.pad(emb, (0, 1)) if dim % 2 else emb


def _mlp(x, w, prefix):
    h = F.silu(F.linear(x, w[f"{prefix}.0.weight"], w[f"{prefix}.0.bias"]))
    return F.linear(h, w[f"{prefix}.2.weight"], w[f"{prefix}.2.bias"])


def _levels(ctor):
    ch = list(ctor["num_channels"])
    nl = len(ch)
    nres = ctor["num_res_blocks"]
    nres = [nres] * nl if isinstance(nres, int) else list(nres)
    heads = ctor["num_head_channels"]
    heads = [heads] * nl if isinstance(heads, int) else list(heads)
    return ch, nl, nres, list(ctor["attention_levels"]), heads


def down_path(h, emb, w, ctor):
    """Encoder levels and mid block shared by UNet and ControlNet (unet.py:274-399);
    returns (hidden after the mid block, skips)."""
    ch, nl, nres, attn, heads = _levels(ctor)
    g, eps, fc = ctor["norm_num_groups"], ctor["norm_eps"], ctor.get("include_fc", True)
    skips = [h]
    for i in range(nl):
        for r in range(nres[i]):
            h = residual_block(h, emb, _pre(w, f"down_blocks.{i}.resnets.{r}"), g, eps)
            if attn[i]:
                h = attention(h, _pre(w, f"down_blocks.{i}.attentions.{r}"), g, eps, heads[i], fc)
            skips.append(h)
        if i != nl - 1:
            h = residual_block(h, emb, _pre(w, f"down_blocks.{i}.downsampler"), g, eps, down=True)
            skips.append(h)
    return h, skips


def mid_block(h, emb, w, ctor):
    _, _, _, _, heads = _levels(ctor)
    g, eps, fc = ctor["norm_num_groups"], ctor["norm_eps"], ctor.get("include_fc", True)
    h = residual_block(h, emb, _pre(w, "middle_block.resnet_1"), g, eps)
    h = attention(h, _pre(w, "middle_block.attention"), g, eps, heads[-1], fc)
    return residual_block(h, emb, _pre(w, "middle_block.resnet_2"), g, eps)


def unet(x, t, class_labels, spacing, w, ctor, down_residuals=None, mid_residual=None):
    """DiffusionModelUNetMaisi forward (unet.py:42-487); returns (t_emb, y), NCDHW."""
    ch, nl, nres, attn, heads = _levels(ctor)
    g, eps, fc = ctor["norm_num_groups"], ctor["norm_eps"], ctor.get("include_fc", True)
    t_emb = timestep_embedding(t, ch[0])
    emb = _mlp(t_emb, w, "time_embed")
    if ctor.get("num_class_embeds") is not None:
        emb = emb + w["class_embedding.weight"][class_labels.long()]
    if ctor.get("include_spacing_input"):
        emb = torch.cat([emb, _mlp(spacing, w, "spacing_layer")], dim=-1)
    h = F.conv3d(x, w["conv_in.conv.weight"], w["conv_in.conv.bias"], padding=1)
    h, skips = down_path(h, emb, w, ctor)
    if down_residuals is not None:
        skips = [s + e for s, e in zip(skips, down_residuals)]
        h = skips[-1]
    h = mid_block(h, emb, w, ctor)
    if mid_residual is not None:
        h = h + mid_residual
    for i in range(nl):
        li = nl - 1 - i
        n = nres[li] + 1
        samples, skips = skips[-n:], skips[:-n]
        for r in range(n):
            h = torch.cat([h, samples.pop()], dim=1)
            h = residual_block(h, emb, _pre(w, f"up_blocks.{i}.resnets.{r}"), g, eps)
            if attn[li]:
                h = attention(h, _pre(w, f"up_blocks.{i}.attentions.{r}"), g, eps, heads[li], fc)
        if i != nl - 1:
            h = residual_block(h, emb, _pre(w, f"up_blocks.{i}.upsampler"), g, eps, up=True)
    h = F.silu(_gn(h, w["out.0.weight"], w["out.0.bias"], g, eps))
    return t_emb, F.conv3d(h, w["out.2.conv.weight"], w["out.2.conv.bias"], padding=1)


def controlnet_condition(cond, w, ctor):
    """Conditioning encoder (controlnet.py:167-249): conv_in, SiLU; per level conv s1 SiLU,
    conv s2 SiLU; conv_out."""
    p = "controlnet_cond_embedding"
    h = F.silu(F.conv3d(cond, w[f"{p}.conv_in.conv.weight"], w[f"{p}.conv_in.conv.bias"], padding=1))
    block = 0
    for _ in range(len(ctor["conditioning_embedding_num_channels"]) - 1):
        for stride in (1, 2):
            h = F.silu(F.conv3d(h, w[f"{p}.blocks.{block}.conv.weight"], w[f"{p}.blocks.{block}.conv.bias"],
                                padding=1, stride=stride))
            block += 1
    return F.conv3d(h, w[f"{p}.conv_out.conv.weight"], w[f"{p}.conv_out.conv.bias"], padding=1)


def _zero_conv(x, w, prefix):
    key = f"{prefix}.conv" if f"{prefix}.conv.weight" in w else prefix
    return F.conv3d(x, w[f"{key}.weight"], w[f"{key}.bias"])


def controlnet(x, t, class_labels, cond, w, ctor, scale=1.0):
    """ControlNetMaisi (controlnet.py:31-164); returns (down residuals, mid residual), NCDHW."""
    ch = list(ctor["num_channels"])
    emb = _mlp(timestep_embedding(t, ch[0]), w, "time_embed")
    if ctor.get("num_class_embeds") is not None:
        emb = emb + w["class_embedding.weight"][class_labels.long()]
    h = F.conv3d(x, w["conv_in.conv.weight"], w["conv_in.conv.bias"], padding=1) + controlnet_condition(cond, w, ctor)
    h, skips = down_path(h, emb, w, ctor)
    h = mid_block(h, emb, w, ctor)
    down = [_zero_conv(s, w, f"controlnet_down_blocks.{i}") * scale for i, s in enumerate(skips)]
    return down, _zero_conv(h, w, "controlnet_mid_block") * scale


def _cw(w, prefix):
    for key in (f"{prefix}.conv.conv", f"{prefix}.conv"):
        if f"{key}.weight" in w:
            return w[f"{key}.weight"], w[f"{key}.bias"]
    raise KeyError(prefix)


def vae_decode(z, w, ctor):
    """post_quant_conv + MaisiDecoder, unfused (vae.py:29-62, 103-200, 273-379)."""
    g, eps = ctor["norm_num_groups"], ctor["norm_eps"]
    post = F.conv3d(z, *_cw(w, "post_quant_conv"))
    h = F.conv3d(post, *_cw(w, "decoder.blocks.0"), padding=1)
    idx = 1
    nres = list(ctor["num_res_blocks"])[::-1]
    for level, n in enumerate(nres):
        for _ in range(n):
            p = f"decoder.blocks.{idx}"
            x = h
            h = F.silu(_gn(x, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], g, eps))
            h = F.conv3d(h, *_cw(w, f"{p}.conv1"), padding=1)
            h = F.silu(_gn(h, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], g, eps))
            h = F.conv3d(h, *_cw(w, f"{p}.conv2"), padding=1)
            if any(k.startswith(f"{p}.nin_shortcut.") for k in w):
                x = F.conv3d(x, *_cw(w, f"{p}.nin_shortcut"))
            h = x + h
            idx += 1
        if level != len(nres) - 1:
            h = F.interpolate(h, scale_factor=2, mode="trilinear", align_corners=False)
            h = F.conv3d(h, *_cw(w, f"decoder.blocks.{idx}.conv"), padding=1)
            idx += 1
    h = _gn(h, w[f"decoder.blocks.{idx}.weight"], w[f"decoder.blocks.{idx}.bias"], g, eps)
    return post, F.conv3d(h, *_cw(w, f"decoder.blocks.{idx + 1}"), padding=1)


def sliding_window_decode(z, w, ctor, roi, overlap, scale_factor=None, sigma_scale=0.125):
    """Gaussian-blended windowed decode (decode.py:104-245), NCDHW, CPU."""
    if scale_factor is not None:
        z = z / scale_factor
    spatial = tuple(z.shape[2:])
    if math.prod(spatial) <= math.prod(roi):
        return vae_decode(z, w, ctor)[1]
    roi = tuple(min(r, s) for r, s in zip(roi, spatial))
    interval = []
    for size, win in zip(spatial, roi):
        interval.append(win if win == size else max(int(win * (1.0 - overlap)), 1))
    starts = []
    for size, win, step in zip(spatial, roi, interval):
        count = int(math.ceil(size / step))
        last = next((i for i in range(count) if i * step + win >= size), None)
        starts.append([i * step - max(i * step + win - size, 0) for i in range(1 if last is None else last + 1)])
    axes = []
    for length in roi:
        half = (length - 1) / 2.0
        x = torch.arange(-half, half + 1.0, dtype=torch.float32)
        sig = sigma_scale * length
        axes.append(torch.exp((x * x) / (-2.0 * sig * sig)))
    imp = torch.clamp(axes[0][:, None, None] * axes[1][None, :, None] * axes[2][None, None, :], min=1e-3)
    imp = imp.repeat_interleave(4, 0).repeat_interleave(4, 1).repeat_interleave(4, 2).to(z.dtype)
    out = None
    for a in starts[0]:
        for b in starts[1]:
            for c in starts[2]:
                pred = vae_decode(z[:, :, a:a + roi[0], b:b + roi[1], c:c + roi[2]], w, ctor)[1]
                if out is None:
                    out = torch.zeros((pred.shape[0], pred.shape[1], *(4 * s for s in spatial)), dtype=z.dtype)
                    wsum = torch.zeros((1, 1, *(4 * s for s in spatial)), dtype=z.dtype)
                sl = (slice(None), slice(None), slice(4 * a, 4 * (a + roi[0])), slice(4 * b, 4 * (b + roi[1])),
                      slice(4 * c, 4 * (c + roi[2])))
                out[sl] += pred * imp
                wsum[sl] += imp
    return out / wsum


def binarize_labels(label):
    """``(N, 1, D, H, W)`` integer ids -> ``(N, 8, D, H, W)`` float condition, channel k = bit k
    (condition.py:20-43), written as repeated halving instead of masks."""
    ids = label[:, 0].long()
    bits = []
    for _ in range(8):
        bits.append((ids % 2).to(torch.float32))
        ids = torch.div(ids, 2, rounding_mode="floor")
    return torch.stack(bits, dim=1)


def to_hu(image, label):
    """Label-masked Hounsfield units (decode.py:248-259), NCDHW."""
    hu = image.clamp(0.0, 1.0) * 2000.0 - 1000.0
    return torch.where(label == 0, torch.full_like(hu, -1000.0), hu)


def ct_sample(latent, cond, spacing, class_labels, unet_w, ctrl_w, unet_ctor, ctrl_ctor, timesteps):
    """ControlNet-conditioned rflow Euler sampling (from_mask.py:177-248, 298-338; rflow.py:100-177),
    NCDHW, with the ControlNet's residuals recomputed from ``cond`` every step."""
    nxt = list(timesteps[1:]) + [0.0]
    z = latent
    for t, tn in zip(timesteps, nxt):
        tt = torch.full((z.shape[0],), float(t), dtype=z.dtype)
        down, mid = controlnet(z, tt, class_labels, cond, ctrl_w, ctrl_ctor)
        _, v = unet(z, tt, class_labels, spacing, unet_w, unet_ctor, down_residuals=down, mid_residual=mid)
        z = z + v * ((float(t) - int(float(tn))) / 1000.0)
    return z


def rflow_timesteps(steps: int, numel: int) -> np.ndarray:
    """The float16-rounded rflow schedule (rflow.py:19-97)."""
    out = []
    for i in range(steps):
        u = (1.0 - i / steps)
        r = (numel / 32768.0) ** (1.0 / 3.0)
        out.append(1000.0 * r * u / (1.0 + (r - 1.0) * u))
    return np.asarray(out, dtype=np.float16).astype(np.float32)


def to_torch(weights: Mapping[str, np.ndarray], dtype=torch.float64, strip: str = "weight.") -> dict[str, torch.Tensor]:
    return {k[len(strip):] if k.startswith(strip) else k: torch.from_numpy(np.asarray(v)).to(dtype)
            for k, v in weights.items() if k.startswith(strip)}


__all__ = ["residual_block", "attention", "unet", "down_path", "mid_block", "controlnet", "controlnet_condition",
           "vae_decode", "sliding_window_decode", "rflow_timesteps", "to_torch", "binarize_labels", "to_hu",
           "ct_sample", "rm"]
