"""Benchmark of the MI355X conv3d hot path (one JSON line on stdout).

Headline workload (the north-star conv target):
conv3d 3x3x3, stride 1, padding 1, +bias, NDHWC fp32, N=1, 64^3 voxels,
Cin = Cout = 64; 57.98 GFLOP per step.  One step = the full operator on
inputs already resident in HBM: one implicit-GEMM kernel (the LDS-staged GEMM,
which stages halo bricks of x itself; no pack pass).

``roofline`` is the GEMM kernel, timed live with HIP events on the stream it
is launched on around each GEMM of (pack, GEMM) rounds through the two-stage
C ABI (the pack stage has nothing to do for this conv), against the FP32 MFMA
peak (157.3 TFLOP/s).
``cpu_baseline`` is the same conv via PyTorch CPU (the op the reference's
parity tests compare against), timed on this host's cores.
``secondary`` reports the other configs' GPU numbers (config 1 residual
block, config 2 resolution-change convs, bf16 variant of config 0).

Warm-up before the headline timed region: W untimed steps, continued until 1 s
has passed so the GPU clock settles (a cold device runs ~10 % slower for its
first several hundred milliseconds of work).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]
"""

from __future__ import annotations

import argparse
import contextlib
import ctypes
import gc
import importlib
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

FP32_PEAK = 157.3e12
BF16_PEAK = 2516.6e12
HBM_PEAK = 8.0e12
# split fp16 (CTMR_F16X2): per fp32 multiply-add two K=32 fp16 MFMAs over 16 channels (hi and lo of the
# input against the weight's hi, then against its lo): 4 fp16 MFMA FLOPs per algorithmic FLOP
F16X2_PEAK = BF16_PEAK / 4
# split-fp16 attention: three fp16 MFMA products (hi*hi, hi*lo, lo*hi) per algorithmic multiply-add
ATTN_F16X2_PEAK = BF16_PEAK / 3


def progress(msg):
    """One line per finished stage on stderr (stdout carries only the JSON result)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def conv_flops(n, d, h, w, cin, cout, taps=27):
    return 2.0 * n * d * h * w * cin * cout * taps


SETTLE_S = 1.0


def warm_up(fn, steps, settle_s=SETTLE_S):
    """Untimed warm-up: `steps` calls, continued until `settle_s` seconds have passed so the
    GPU clock reaches its steady state (measured on MI355X: config 0 runs ~10 % slower until
    several hundred milliseconds of work have passed).  Returns the number of calls made."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < steps or time.perf_counter() - t0 < settle_s:
        fn()
        done += 1
        if done % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return done


@contextlib.contextmanager
def gc_quiet():
    """A timed region without Python's cyclic garbage collector (as ``timeit`` runs).  A full
    collection walks every tracked object of this process (~270k with torch imported; 60-105 ms
    measured on the MI355X host), which would otherwise land in whichever step happens to trigger
    it.  No collection is forced on entry: the GPU would idle for its duration right before the
    timed steps and its clock drop (measured: the config-2c 1x1 conv 0.166 -> 0.199 ms)."""
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()


def _wall_ms(fn, steps):
    import torch

    with gc_quiet():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps


def staged_op(pkg, x, w, b, dtype_code, stream_gemm=False):
    """The operator as its two C-ABI stages (ctmr_conv3d_pack, ctmr_conv3d_gemm) for timing
    the GEMM kernel in context: every GEMM reads a freshly packed input, as in the full op.
    ``stream_gemm`` forces the register-streaming GEMM (CTMR_F_STREAM)."""
    import torch

    L, ops = pkg._lib, pkg.ops
    cin, cout = int(x.shape[-1]), int(w.shape[0])
    desc = ops.make_desc(tuple(x.shape), cout, 3, 1, L.MODE_PLAIN, L.F_STREAM if stream_gemm else 0, dtype_code, 0)
    ws_bytes = L.workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 1), device=x.device, dtype=torch.uint8)
    packed_w = ops.pack_weight(w, cin, cout, 3, L.MODE_PLAIN, dtype_code)
    y = torch.empty((*x.shape[:-1], cout), device=x.device, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    lib = L.lib()
    args = (ctypes.byref(desc), x.data_ptr(), packed_w.data_ptr(), b.data_ptr(), None, y.data_ptr(),
            ws.data_ptr(), ws_bytes, stream)

    def pack():
        L.check(lib.ctmr_conv3d_pack(ctypes.byref(desc), x.data_ptr(), None, ws.data_ptr(), ws_bytes, stream),
                "ctmr_conv3d_pack")

    def gemm():
        L.check(lib.ctmr_conv3d_gemm(*args), "ctmr_conv3d_gemm")

    return pack, gemm, (ws, packed_w, y)


def gemm_ms_in_context(pack, gemm, iters):
    """Mean GEMM kernel time over `iters` pack+GEMM rounds, HIP events on the launch stream
    bracketing each GEMM (the pack of the same round runs just before it)."""
    import torch

    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in pairs:
        pack()
        e0.record()
        gemm()
        e1.record()
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in pairs) / iters


def cpu_baseline(budget_s=20.0):
    """Config 0 conv via PyTorch CPU fp32 (oracle.cpu_baseline), best of layouts."""
    from oracle import cpu_baseline as cb

    return cb.time_config0_conv(budget_s=budget_s)


def secondary(pkg, dev, steps, cpu=False):
    """Config 1 (VAE residual block at 128^3 x 128) and config 2 GPU numbers; with ``cpu`` the same
    operations via PyTorch fp32 on the host cores beside each (the reference's CPU path)."""
    import numpy as np
    import torch

    f = pkg.fast_fp32
    out = {}
    rng = np.random.default_rng(1)
    c, s = 128, 128
    x = torch.from_numpy(rng.standard_normal((1, s, s, s, c), dtype=np.float32)).to(dev)
    mk = lambda cout, cin, k=3: torch.from_numpy(
        (rng.standard_normal((cout, cin, k, k, k)) / np.sqrt(k**3 * cin)).astype(np.float32)).to(dev)
    w1, w2 = mk(c, c), mk(c, c)
    b1 = torch.from_numpy((0.01 * rng.standard_normal(c)).astype(np.float32)).to(dev)
    b2 = torch.from_numpy((0.01 * rng.standard_normal(c)).astype(np.float32)).to(dev)
    g = torch.ones(c, device=dev)
    z = torch.zeros(c, device=dev)

    def block():
        return f.vae_resblock([x], (w1, b1), (w2, b2), (g, z), (g, z), None, num_groups=32, eps=1e-6)

    for _ in range(2):
        block()
    ms = _wall_ms(block, max(2, steps // 4))
    flops = 2 * conv_flops(1, s, s, s, c, c)
    progress(f"config 1 {ms:.3f} ms")
    out["config1_vae_resblock_128c_128^3"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 2),
                                              "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    with f.precision("f16x2"):
        for _ in range(2):
            block()
        msx = _wall_ms(block, max(2, steps // 4))
    out["config1_vae_resblock_128c_128^3"].update({"f16x2_ms": round(msx, 3),
                                                   "f16x2_tflops": round(flops / msx / 1e9, 2),
                                                   "f16x2_frac_peak": round(flops / msx / 1e-3 / F16X2_PEAK, 4)})
    del x
    # config 2a: stride-2 conv 64->128, 128^3 -> 64^3
    xa = torch.from_numpy(rng.standard_normal((1, 128, 128, 128, 64), dtype=np.float32)).to(dev)
    wa, ba = mk(128, 64), torch.zeros(128, device=dev)
    run = lambda: f.conv3d(xa, wa, ba, padding=1, stride=2)
    warm_up(run, 2, settle_s=0.5)  # the device idled while the input was drawn on the CPU
    ms = _wall_ms(run, steps)
    flops = conv_flops(1, 64, 64, 64, 64, 128)
    out["config2a_down_s2_64to128"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 2),
                                       "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    del xa
    # config 2b: nearest-2x + conv 256->128, 64^3 -> 128^3 (8-tap parity fold)
    xb = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 256), dtype=np.float32)).to(dev)
    wb, bb = mk(128, 256), torch.zeros(128, device=dev)
    run = lambda: f.norm_conv3d(xb, wb, bb, norm=None, num_groups=1, eps=1e-6, apply_silu=False, upsample=True)
    warm_up(run, 2, settle_s=0.5)  # the device idled while the input was drawn on the CPU
    ms = _wall_ms(run, max(2, steps // 2))
    flops = conv_flops(8, 64, 64, 64, 256, 128, taps=8)
    out["config2b_nearest_up_256to128"] = {"ms": round(ms, 3), "tflops_folded": round(flops / ms / 1e9, 2),
                                           "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4)}
    del xb
    # config 2c: 1x1x1 128 -> 256 at 64^3
    xc = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 128), dtype=np.float32)).to(dev)
    wc, bc = mk(256, 128, 1), torch.zeros(256, device=dev)
    run = lambda: f.pointwise_conv(xc, wc, bc)
    warm_up(run, 2, settle_s=0.5)  # the device idled while the input was drawn on the CPU
    ms = _wall_ms(run, steps)
    flops = 2.0 * 64**3 * 128 * 256
    nbytes = 4.0 * 64**3 * (128 + 256)
    out["config2c_pointwise_128to256"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                                          "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4),
                                          "hbm_GBps": round(nbytes / ms / 1e6, 1),
                                          "frac_hbm": round(nbytes / ms / 1e-3 / HBM_PEAK, 4)}
    del xc
    # flash attention at the production UNet's 2048-token level (16x16x8 latent, 8 heads of 32, batch 2):
    # FP32 MFMA, and the reference's split-fp16 kernel (whole operator: the split pass and the kernel)
    g = torch.Generator(device=dev).manual_seed(0)
    qkv = torch.randn(2, 2048, 768, device=dev, generator=g)
    q, k, v = qkv[..., :256], qkv[..., 256:512], qkv[..., 512:]
    run = lambda: f.flash_attention(q, k, v, heads=8, scale=32 ** -0.5)
    flops = 4.0 * 2048 * 2048 * 32 * 8 * 2
    warm_up(run, 5, settle_s=0.3)
    ms = _wall_ms(run, 4 * steps)
    with f.precision("f16x2"):
        warm_up(run, 5, settle_s=0.3)
        msx = _wall_ms(run, 4 * steps)
    out["attention_level2_2048tok_8h"] = {"ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 2),
                                          "frac_fp32_peak": round(flops / ms / 1e-3 / FP32_PEAK, 4),
                                          "f16x2_ms": round(msx, 4), "f16x2_tflops": round(flops / msx / 1e9, 2),
                                          "f16x2_frac_peak": round(flops / msx / 1e-3 / ATTN_F16X2_PEAK, 4)}
    del qkv
    if cpu:
        from oracle import cpu_baseline as cb

        legs = cb.config_legs()
        progress("CPU legs of configs 1-2c done")
        for key, leg in (("config1_vae_resblock_128c_128^3", "config1"), ("config2a_down_s2_64to128", "config2a"),
                         ("config2b_nearest_up_256to128", "config2b"), ("config2c_pointwise_128to256", "config2c")):
            out[key].update({"cpu_ms": round(legs[leg], 2), "cpu_cores": cb.cores(),
                             "gpu_speedup": round(legs[leg] / out[key]["ms"], 1)})
    return out


def controlnet_flops(constructor, batch, d, h, w):
    """Conv and attention FLOPs of one ControlNetMaisi pass with a precomputed conditioning embedding:
    the UNet's encoder (conv_in, down path, mid block) plus a 1x1 zero conv per residual."""
    conv, attn_f = unet_flops(constructor, batch, d, h, w, encoder_only=True)
    ch = list(constructor["num_channels"])
    nl, nres = len(ch), constructor["num_res_blocks"]
    vox = [batch * d * h * w // 8**i for i in range(nl)]
    conv += 2.0 * vox[0] * ch[0] * ch[0]  # conv_in's residual
    for i in range(nl):
        conv += nres * 2.0 * vox[i] * ch[i] * ch[i]  # res-block outputs
        if i != nl - 1:
            conv += 2.0 * vox[i + 1] * ch[i] * ch[i]  # down-sampler outputs
    conv += 2.0 * vox[-1] * ch[-1] * ch[-1]  # mid block
    return conv, attn_f


def unet_flops(constructor, batch, d, h, w, encoder_only=False):
    """Conv FLOPs of one UNet pass (8-tap folded upsample convs) and attention FLOPs; with
    ``encoder_only`` the conv_in + down path + mid block part."""
    ch = list(constructor["num_channels"])
    nl = len(ch)
    nres = [constructor["num_res_blocks"]] * nl
    attn = list(constructor["attention_levels"])
    head = list(constructor["num_head_channels"])
    conv = attn_f = 0.0
    vox = [batch * d * h * w // 8**i for i in range(nl)]

    def res(v, cin, cout, taps1=27):
        f = 2.0 * v * cin * cout * taps1 + 2.0 * v * cout * cout * 27
        return f + (2.0 * v * cin * cout if cin != cout else 0.0)

    def att(v, c):
        tokens = v // batch
        return batch * (4 * 2.0 * tokens * c * c + 2 * 2.0 * tokens * tokens * c)

    conv += 2.0 * vox[0] * constructor["in_channels"] * ch[0] * 27
    prev = ch[0]
    for i in range(nl):
        for r in range(nres[i]):
            conv += res(vox[i], prev if r == 0 else ch[i], ch[i])
            attn_f += att(vox[i], ch[i]) if attn[i] else 0.0
        prev = ch[i]
        if i != nl - 1:
            conv += res(vox[i + 1], ch[i], ch[i])  # down: convs at the pooled grid
    conv += 2 * res(vox[-1], ch[-1], ch[-1])
    attn_f += att(vox[-1], ch[-1])
    if encoder_only:
        return conv, attn_f
    rc = ch[::-1]
    out = rc[0]
    for i in range(nl):
        li = nl - 1 - i
        prev, out = out, rc[i]
        cin_skip = rc[min(i + 1, nl - 1)]
        n = nres[li] + 1
        for r in range(n):
            skip = cin_skip if r == n - 1 else out
            conv += res(vox[li], (prev if r == 0 else out) + skip, out)
            attn_f += att(vox[li], out) if attn[li] else 0.0
        if i != nl - 1:
            # up: conv1 on the source grid with 8 folded taps per parity (x8 outputs)
            conv += 2.0 * vox[li] * out * out * 8 * 8 + 2.0 * vox[li - 1] * out * out * 27
    conv += 2.0 * vox[0] * ch[0] * constructor["out_channels"] * 27
    return conv, attn_f


def controlnet_cond_flops(constructor, n, d, h, w):
    """Conv FLOPs of the ControlNet conditioning encoder on an (n, d, h, w) label grid (once per
    generation): conv_in, per level a stride-1 and a stride-2 conv, conv_out at the latent grid."""
    cc = list(constructor["conditioning_embedding_num_channels"])
    vox = n * d * h * w
    f = 2.0 * vox * constructor["conditioning_embedding_in_channels"] * cc[0] * 27
    for i in range(len(cc) - 1):
        f += 2.0 * vox * cc[i] * cc[i] * 27
        vox //= 8
        f += 2.0 * vox * cc[i] * cc[i + 1] * 27
    return f + 2.0 * vox * cc[-1] * constructor["num_channels"][0] * 27


def vae_decoder_flops(constructor, d, h, w):
    """Conv FLOPs of one decoder pass on a (d, h, w) latent (trilinear convs on the 2x grid)."""
    ch = list(constructor["num_channels"])[::-1]
    nres = list(constructor["num_res_blocks"])[::-1]
    lat = constructor["latent_channels"]
    v = d * h * w
    f = 2.0 * v * lat * lat + 2.0 * v * lat * ch[0] * 27
    block_in = ch[0]
    for level, n in enumerate(nres):
        for _ in range(n):
            out = ch[level]
            f += 2.0 * v * 27 * (block_in * out + out * out) + (2.0 * v * block_in * out if block_in != out else 0)
            block_in = out
        if level != len(nres) - 1:
            v *= 8
            f += 2.0 * v * 27 * block_in * block_in
    return f + 2.0 * v * 27 * block_in * constructor["out_channels"]


def networks(pkg, dev, steps, generation=True, cpu=False):
    """Config 3 (UNet step), config 4 (256^3 windowed decode + int16) and the full
    256^3 generation (30 CFG UNet steps at a 64^3 latent + decode)."""
    import numpy as np
    import torch

    m = pkg.maisi
    out = {}
    uc, vc = m.PRODUCTION_UNET_CONSTRUCTOR, m.PRODUCTION_VAE_CONSTRUCTOR
    uw = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.unet_weight_shapes(uc), seed=7).items()}
    vw = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.vae_decoder_weight_shapes(vc), seed=11).items()}
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((2, 64, 64, 32, 4), dtype=np.float32)).to(dev)
    t = torch.full((2,), float(rng.uniform(0, 1000)), device=dev)
    classes = torch.tensor([9, 0], device=dev)
    spacing = m.spacing_tensor([0.94, 0.94, 1.36], device=dev).repeat(2, 1)
    step = lambda: m.denoise_unet(x, t, classes, spacing, uw, constructor=uc)
    for _ in range(2):
        step()
    ms = _wall_ms(step, max(3, steps // 2))
    progress(f"config 3 UNet step {ms:.3f} ms")
    conv_f, attn_f = unet_flops(uc, 2, 64, 64, 32)
    floor_ms = (conv_f + attn_f) / FP32_PEAK * 1e3
    out["config3_unet_step_batch2_64x64x32"] = {
        "ms": round(ms, 3), "conv_tflop": round(conv_f / 1e12, 4), "attention_tflop": round(attn_f / 1e12, 4),
        "tflops": round((conv_f + attn_f) / ms / 1e9, 2), "roofline_ms": round(floor_ms, 3),
        "frac_roofline": round(floor_ms / ms, 4)}
    # the same step replayed from a HIP graph (one launch instead of the eager per-kernel issue)
    graph = m.UNetGraph(x, t, classes, spacing, uw, constructor=uc)
    gstep = lambda: graph(x, t, classes, spacing)
    gms = _wall_ms(gstep, max(3, steps // 2))
    del graph
    # the bf16-in / fp32-accumulate variant of the same step (convolutions on bf16 MFMA; attention,
    # norms and projections stay fp32): floor = convs at the bf16 peak + attention at the fp32 peak
    with pkg.fast_fp32.precision("bf16"):
        for _ in range(2):
            step()
        ms16 = _wall_ms(step, max(3, steps // 2))
        graph = m.UNetGraph(x, t, classes, spacing, uw, constructor=uc)
        gms16 = _wall_ms(gstep, max(3, steps // 2))
        del graph
    floor16 = (conv_f / BF16_PEAK + attn_f / FP32_PEAK) * 1e3
    # split fp16 (the reference's exact mode): same floor rule with every conv at the split peak
    with pkg.fast_fp32.precision("f16x2"):
        for _ in range(2):
            step()
        msx = _wall_ms(step, max(3, steps // 2))
        graph = m.UNetGraph(x, t, classes, spacing, uw, constructor=uc)
        gmsx = _wall_ms(gstep, max(3, steps // 2))
        del graph
    progress(f"config 3 UNet step f16x2 {msx:.3f} ms, graph {gmsx:.3f} ms")
    floorx = (conv_f / F16X2_PEAK + attn_f / ATTN_F16X2_PEAK) * 1e3
    out["config3_unet_step_batch2_64x64x32"].update(
        {"graph_ms": round(gms, 3), "graph_frac_roofline": round(floor_ms / gms, 4),
         "bf16_ms": round(ms16, 3), "bf16_graph_ms": round(gms16, 3), "bf16_roofline_ms": round(floor16, 3),
         "bf16_frac_roofline": round(floor16 / min(ms16, gms16), 4),
         "f16x2_ms": round(msx, 3), "f16x2_graph_ms": round(gmsx, 3), "f16x2_roofline_ms": round(floorx, 3),
         "f16x2_frac_roofline": round(floorx / min(msx, gmsx), 4)})
    # CT from mask: ControlNetMaisi (production constructor, conditioning embedding computed once per
    # generation) + the UNet with its residuals, per denoising step
    cc = m.PRODUCTION_CONTROLNET_CONSTRUCTOR
    cw = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.controlnet_weight_shapes(cc), seed=13).items()}
    cond_emb = torch.from_numpy(rng.standard_normal((2, 64, 64, 32, 64), dtype=np.float32)).to(dev)

    def ct_step():  # the ControlNet on a second stream, overlapping the UNet encoder
        return m.controlnet_unet_step(x, t, classes, spacing, uw, cw, unet_constructor=uc, controlnet_constructor=cc,
                                      conditioning_embedding=cond_emb)

    ctrl = lambda: m.controlnet_residuals(x, t, classes, None, cw, constructor=cc, conditioning_embedding=cond_emb)
    for _ in range(2):
        ct_step()
    ct_ms = _wall_ms(ct_step, max(3, steps // 2))
    ctrl_ms = _wall_ms(ctrl, max(3, steps // 2))
    with pkg.fast_fp32.precision("f16x2"):
        for _ in range(2):
            ct_step()
        ct_msx = _wall_ms(ct_step, max(3, steps // 2))
    cconv, cattn = controlnet_flops(cc, 2, 64, 64, 32)
    ct_flop = conv_f + attn_f + cconv + cattn
    ct_floorx = ((conv_f + cconv) / F16X2_PEAK + (attn_f + cattn) / ATTN_F16X2_PEAK) * 1e3
    out["ct_controlnet_unet_step_batch2_64x64x32"] = {
        "ms": round(ct_ms, 3), "controlnet_ms": round(ctrl_ms, 3),
        "controlnet_tflop": round((cconv + cattn) / 1e12, 4), "tflops": round(ct_flop / ct_ms / 1e9, 2),
        "roofline_ms": round(ct_flop / FP32_PEAK * 1e3, 3), "frac_roofline": round(ct_flop / FP32_PEAK * 1e3 / ct_ms, 4),
        "f16x2_ms": round(ct_msx, 3), "f16x2_roofline_ms": round(ct_floorx, 3),
        "f16x2_frac_roofline": round(ct_floorx / ct_msx, 4)}
    del cw, cond_emb
    if cpu:
        from oracle import cpu_baseline as cb
        from oracle import maisi_torch as mt

        host_w = {k: v.cpu() for k, v in uw.items()}
        xc = x.cpu().permute(0, 4, 1, 2, 3).contiguous()
        torch.set_num_threads(cb.cores())
        with torch.no_grad():
            cpu_s = cb.median_seconds(lambda: mt.unet(xc, t.cpu(), classes.cpu(), spacing.cpu(), host_w, uc), reps=3)
        progress(f"config 3 CPU {cpu_s:.2f} s")
        out["config3_unet_step_batch2_64x64x32"].update({"cpu_ms": round(cpu_s * 1e3, 1), "cpu_cores": cb.cores(),
                                                         "cpu_timing": "median of 3 after 1 warm-up"})
        del host_w, xc
    del x
    # config 4: 64^3 latent -> 256^3, 4 windows along D (roi 20x64x64, overlap 0.25), int16
    z = torch.from_numpy(np.random.default_rng(4).standard_normal((1, 64, 64, 64, 4), dtype=np.float32)).to(dev)

    def decode():
        y = m.sliding_window_decode(z, vw, constructor=vc, roi=(20, 64, 64), overlap=0.25, scale_factor=1.0)
        img = torch.clamp(y * 1000.0, min=0.0).to(torch.int16)
        return img

    def timed(fn, reps=3):
        """Median synchronized seconds of ``reps`` runs after one warm-up, and the peak device memory
        allocated during them."""
        fn()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        times = []
        for _ in range(reps):
            with gc_quiet():
                t0 = time.perf_counter()
                r = fn()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
            del r
        return float(np.median(times)), torch.cuda.max_memory_allocated(dev)

    sec, peak = timed(decode)
    progress(f"config 4 decode {sec:.3f} s")
    dec_f = 4 * vae_decoder_flops(vc, 20, 64, 64)
    out["config4_vae_decode_256^3_4windows"] = {
        "s": round(sec, 4), "tflop": round(dec_f / 1e12, 3), "tflops": round(dec_f / sec / 1e12, 2),
        "roofline_s": round(dec_f / FP32_PEAK, 4), "frac_roofline": round(dec_f / FP32_PEAK / sec, 4),
        "timing": "median of 3 after 1 warm-up", "peak_device_GiB": round(peak / 2**30, 2),
        "output": [1, 256, 256, 256, 1]}
    with pkg.fast_fp32.precision("bf16"):
        sec16, _ = timed(decode)
    with pkg.fast_fp32.precision("f16x2"):
        secx, _ = timed(decode)
    progress(f"config 4 decode f16x2 {secx:.3f} s")
    out["config4_vae_decode_256^3_4windows"].update(
        {"bf16_s": round(sec16, 4), "bf16_roofline_s": round(dec_f / BF16_PEAK, 4),
         "bf16_frac_roofline": round(dec_f / BF16_PEAK / sec16, 4),
         "f16x2_s": round(secx, 4), "f16x2_roofline_s": round(dec_f / F16X2_PEAK, 4),
         "f16x2_frac_roofline": round(dec_f / F16X2_PEAK / secx, 4)})
    if cpu:
        from oracle import cpu_baseline as cb

        host_v = {k: v.cpu().numpy() for k, v in vw.items()}
        full = cb.vae_decode_seconds(host_v, vc, np.ascontiguousarray(z.cpu().numpy()), (20, 64, 64), 0.25)
        out["config4_vae_decode_256^3_4windows"].update(
            {"cpu_decode_s": round(full, 2), "cpu_cores": cb.cores(), "cpu_repetitions": 1,
             "cpu_sample": "the full 256^3 decode (4 windows of 20x64x64 latent, Gaussian blend, int16) with "
                           "the PyTorch fp32 decoder, one timed run after a small warm-up window"})
    del z
    if generation:
        # full 256^3 generation: 30 rflow steps with batched CFG at a 64^3 latent, then decode
        lat = torch.from_numpy(np.random.default_rng(5).standard_normal((1, 64, 64, 64, 4), dtype=np.float32)).to(dev)
        sp = m.spacing_tensor([1.0, 1.0, 1.0], device=dev)
        cls = torch.tensor([9], device=dev)
        times, _ = m.set_timesteps_rflow(num_inference_steps=30, input_img_size_numel=64**3)
        vel = lambda s, tt: m.guided_velocity(s, tt, class_labels=cls, spacing=sp, weights=uw, constructor=uc,
                                              guidance_scale=5.0)
        phases = []

        def generate():
            t0 = time.perf_counter()
            final = m.sample_rflow(lat, vel, times)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            y = m.sliding_window_decode(final, vw, constructor=vc, roi=(20, 64, 64), overlap=0.25, scale_factor=1.0)
            img = torch.clamp(y * 1000.0, min=0.0).to(torch.int16).cpu()
            phases.append(t1 - t0)
            return img

        total, peak = timed(generate)
        progress(f"256^3 MR generation {total:.3f} s")
        phases32 = list(phases)
        phases.clear()
        with pkg.fast_fp32.precision("f16x2"):
            totalx, _ = timed(generate)
        progress(f"256^3 MR generation f16x2 {totalx:.3f} s")
        gen_f = 30 * sum(unet_flops(uc, 2, 64, 64, 64)) + dec_f
        gen_attn = 30 * unet_flops(uc, 2, 64, 64, 64)[1]
        gen_floorx = (gen_f - gen_attn) / F16X2_PEAK + gen_attn / ATTN_F16X2_PEAK
        out["generation_256^3_30steps_cfg"] = {
            "s": round(total, 3), "sampling_s": round(float(np.median(phases32[1:])), 3), "tflop": round(gen_f / 1e12, 2),
            "roofline_s": round(gen_f / FP32_PEAK, 3), "frac_roofline": round(gen_f / FP32_PEAK / total, 4),
            "f16x2_s": round(totalx, 3), "f16x2_sampling_s": round(float(np.median(phases[1:])), 3),
            "f16x2_roofline_s": round(gen_floorx, 3), "f16x2_frac_roofline": round(gen_floorx / totalx, 4),
            "target_s": 60, "timing": "median of 3 after 1 warm-up", "peak_device_GiB": round(peak / 2**30, 2),
            "image_dtype": "torch.int16"}
        del lat
        out["ct_from_mask_256^3_30steps"] = ct_generation(pkg, dev, uw, vw, timed)
        out.update(production_grids(pkg, dev, uw, vw, timed))
    return out


def ct_generation(pkg, dev, uw, vw, timed):
    """CT from a 256^3 label map (from_mask.py:121-295): condition encoded once, 30 ControlNet + UNet
    steps at batch 1 (64^3 latent), windowed decode (roi 48x48x64, overlap 0.6666: 4 windows), HU."""
    import numpy as np
    import torch

    m = pkg.maisi
    uc, cc, vc = m.PRODUCTION_UNET_CONSTRUCTOR, m.PRODUCTION_CONTROLNET_CONSTRUCTOR, m.PRODUCTION_VAE_CONSTRUCTOR
    cw = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.controlnet_weight_shapes(cc), seed=13).items()}
    rng = np.random.default_rng(8)
    label = rng.choice(np.array(sorted(m.VALID_LABELS)), size=(1, 1, 256, 256, 256)).astype(np.int16)
    lat = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 4), dtype=np.float32)).to(dev)
    results = []

    def run():
        r = m.sample_ct_from_mask(label, (0.75, 0.75, 0.75), unet_weights=uw, controlnet_weights=cw,
                                  vae_weights=vw, unet_constructor=uc, controlnet_constructor=cc, vae_constructor=vc,
                                  scale_factor=1.0, latent=lat, drop_weights=False)
        hu = r.hu.cpu()
        results.append(r.stage_timings_s)
        return hu

    sec, peak = timed(run)
    progress(f"CT from mask generation {sec:.3f} s")
    stages32 = list(results)
    results.clear()
    with pkg.fast_fp32.precision("f16x2"):
        secx, _ = timed(run)
    progress(f"CT from mask generation f16x2 {secx:.3f} s")
    windows = len(m.dense_patch_slices((64, 64, 64), (48, 48, 64), m.scan_interval((64, 64, 64), (48, 48, 64), 0.6666)))
    unet_f = sum(unet_flops(uc, 1, 64, 64, 64))
    ctrl_f = sum(controlnet_flops(cc, 1, 64, 64, 64))
    flop = controlnet_cond_flops(cc, 1, 256, 256, 256) + 30 * (unet_f + ctrl_f) + windows * vae_decoder_flops(
        vc, 48, 48, 64)
    stages = {k: round(float(np.median([r[k] for r in stages32[1:]])), 3) for k in stages32[0]}
    stagesx = {k: round(float(np.median([r[k] for r in results[1:]])), 3) for k in results[0]}
    attn = 30 * (unet_flops(uc, 1, 64, 64, 64)[1] + controlnet_flops(cc, 1, 64, 64, 64)[1])
    floorx = (flop - attn) / F16X2_PEAK + attn / ATTN_F16X2_PEAK
    return {"s": round(sec, 3), "stages_s": stages, "tflop": round(flop / 1e12, 2), "decode_windows": windows,
            "roofline_s": round(flop / FP32_PEAK, 3), "frac_roofline": round(flop / FP32_PEAK / sec, 4),
            "f16x2_s": round(secx, 3), "f16x2_stages_s": stagesx, "f16x2_roofline_s": round(floorx, 3),
            "f16x2_frac_roofline": round(floorx / secx, 4),
            "timing": "median of 3 after 1 warm-up, label upload to HU download", "peak_device_GiB":
            round(peak / 2**30, 2)}


def production_grids(pkg, dev, uw, vw, timed):
    """The reference's other production grids (its configurations table): MR-Brain 256x256x128 with
    guidance 2 and general MR 128x256x256 with guidance 15 (batched CFG, batch 2 per step), and CT from
    a 256x256x128 mask (ControlNet + UNet at batch 1); 30 rflow steps each, then the windowed decode
    with the default window (both latents are below it: one pass).  One timed run after a warm-up,
    fp32 and split fp16."""
    import numpy as np
    import torch

    m = pkg.maisi
    uc, cc, vc = m.PRODUCTION_UNET_CONSTRUCTOR, m.PRODUCTION_CONTROLNET_CONSTRUCTOR, m.PRODUCTION_VAE_CONSTRUCTOR
    rng = np.random.default_rng(9)
    out = {}

    def mr(name, latent, spacing_mm, guidance):
        lat = torch.from_numpy(rng.standard_normal((1, *latent, 4), dtype=np.float32)).to(dev)
        sp = m.spacing_tensor(spacing_mm, device=dev)
        cls = torch.tensor([9], device=dev)
        times, _ = m.set_timesteps_rflow(num_inference_steps=30, input_img_size_numel=int(np.prod(latent)))
        vel = lambda s, tt: m.guided_velocity(s, tt, class_labels=cls, spacing=sp, weights=uw, constructor=uc,
                                              guidance_scale=guidance)

        def generate():
            final = m.sample_rflow(lat, vel, times)
            return torch.clamp(m.sliding_window_decode(final, vw, constructor=vc) * 1000.0, min=0.0).to(
                torch.int16).cpu()

        sec, peak = timed(generate, reps=1)
        with pkg.fast_fp32.precision("f16x2"):
            secx, _ = timed(generate, reps=1)
        progress(f"{name} generation {sec:.3f} s, f16x2 {secx:.3f} s")
        flop = 30 * sum(unet_flops(uc, 2, *latent)) + vae_decoder_flops(vc, *latent)
        attn = 30 * unet_flops(uc, 2, *latent)[1]
        floorx = (flop - attn) / F16X2_PEAK + attn / ATTN_F16X2_PEAK
        out[name] = {"s": round(sec, 3), "tflop": round(flop / 1e12, 2), "roofline_s": round(flop / FP32_PEAK, 3),
                     "frac_roofline": round(flop / FP32_PEAK / sec, 4), "f16x2_s": round(secx, 3),
                     "f16x2_roofline_s": round(floorx, 3), "f16x2_frac_roofline": round(floorx / secx, 4),
                     "guidance_scale": guidance, "output": [4 * v for v in latent],
                     "timing": "one run after a warm-up", "peak_device_GiB": round(peak / 2**30, 2)}

    mr("mr_brain_256x256x128_30steps_cfg", (64, 64, 32), [0.94, 0.94, 1.36], 2.0)
    mr("mr_128x256x256_30steps_cfg", (32, 64, 64), [1.25, 1.0, 1.0], 15.0)

    cw = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.controlnet_weight_shapes(cc), seed=13).items()}
    label = rng.choice(np.array(sorted(m.VALID_LABELS)), size=(1, 1, 256, 256, 128)).astype(np.int16)
    lat = torch.from_numpy(rng.standard_normal((1, 64, 64, 32, 4), dtype=np.float32)).to(dev)

    def ct():
        r = m.sample_ct_from_mask(label, (1.7, 1.7, 2.0), unet_weights=uw, controlnet_weights=cw, vae_weights=vw,
                                  unet_constructor=uc, controlnet_constructor=cc, vae_constructor=vc,
                                  scale_factor=1.0, latent=lat, drop_weights=False)
        return r.hu.cpu()

    sec, peak = timed(ct, reps=1)
    with pkg.fast_fp32.precision("f16x2"):
        secx, _ = timed(ct, reps=1)
    progress(f"CT 256x256x128 from mask {sec:.3f} s, f16x2 {secx:.3f} s")
    step_f = sum(unet_flops(uc, 1, 64, 64, 32)) + sum(controlnet_flops(cc, 1, 64, 64, 32))
    flop = controlnet_cond_flops(cc, 1, 256, 256, 128) + 30 * step_f + vae_decoder_flops(vc, 64, 64, 32)
    attn = 30 * (unet_flops(uc, 1, 64, 64, 32)[1] + controlnet_flops(cc, 1, 64, 64, 32)[1])
    floorx = (flop - attn) / F16X2_PEAK + attn / ATTN_F16X2_PEAK
    out["ct_from_mask_256x256x128_30steps"] = {
        "s": round(sec, 3), "tflop": round(flop / 1e12, 2), "roofline_s": round(flop / FP32_PEAK, 3),
        "frac_roofline": round(flop / FP32_PEAK / sec, 4), "f16x2_s": round(secx, 3),
        "f16x2_roofline_s": round(floorx, 3), "f16x2_frac_roofline": round(floorx / secx, 4),
        "timing": "one run after a warm-up, label upload to HU download", "peak_device_GiB": round(peak / 2**30, 2)}
    return out


def _sclk_under(fn, seconds=4.0):
    """Shader clock read by ``rocm-smi --showclocks`` (a child process) while ``fn`` runs back to back."""
    import subprocess

    import torch

    fn()
    torch.cuda.synchronize()
    probe = subprocess.Popen(["rocm-smi", "--showclocks"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                             text=True)
    t0 = time.perf_counter()
    while probe.poll() is None and time.perf_counter() - t0 < 30:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    while time.perf_counter() - t0 < seconds:  # keep the load on for the whole sample window
        fn()
    torch.cuda.synchronize()
    text = probe.communicate()[0]
    for line in text.splitlines():
        if "sclk" in line.lower():
            return line.split(":")[-1].strip()
    return None


def reference_gemms(pkg, dev):
    """hipBLASLt GEMM rates (torch.matmul) at square and conv-shaped sizes, and the shader clock under each
    sustained MFMA load, beside this library's config-0 fp32 and bf16 implicit GEMMs."""
    import numpy as np
    import torch

    def med_us(fn, n=10):
        warm_up(fn, 3)
        times = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3)
        return float(np.median(times))

    out = {"gemms": {}, "sclk_under_load": {}}
    cases = [("bf16", 16384, 16384, 16384), ("bf16", 8192, 8192, 8192), ("bf16", 262144, 1728, 64),
             ("fp32", 8192, 8192, 8192), ("fp32", 262144, 1728, 64)]
    for dt, m, k, n in cases:
        dtype = torch.bfloat16 if dt == "bf16" else torch.float32
        a = torch.randn(m, k, device=dev, dtype=dtype)
        bt = torch.randn(n, k, device=dev, dtype=dtype)
        fn = lambda: a @ bt.t()
        us = med_us(fn)
        key = f"{dt}_{m}x{k}x{n}"
        peak = BF16_PEAK if dt == "bf16" else FP32_PEAK
        tf = 2.0 * m * k * n / us / 1e6
        out["gemms"][key] = {"us": round(us, 1), "tflops": round(tf, 1), "frac_nominal_peak": round(tf * 1e12 / peak, 4)}
        if (m, k, n) in ((16384, 16384, 16384), (8192, 8192, 8192)) and not (dt == "bf16" and m == 8192):
            out["sclk_under_load"][f"hipblaslt_{key}"] = _sclk_under(fn)
        del a, bt
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 64), dtype=np.float32)).to(dev)
    w = torch.from_numpy((rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)).to(dev)
    b = torch.zeros(64, device=dev)
    for code, name in ((pkg._lib.DT_F32, "fp32"), (pkg._lib.DT_BF16, "bf16")):
        pack, gemm, _keep = staged_op(pkg, x, w, b, code)
        pack()
        us = med_us(gemm, 20)
        tf = conv_flops(1, 64, 64, 64, 64, 64) / us / 1e6
        out["gemms"][f"ctmr_config0_{name}_gemm"] = {"us": round(us, 1), "tflops": round(tf, 1)}
        out["sclk_under_load"][f"ctmr_config0_{name}_gemm"] = _sclk_under(gemm)
    print(json.dumps(out), flush=True)
    return 0


def profile_only(pkg, dev, what, steps, warmup):
    """Run one workload alone (for rocprofv3 traces) and print its mean time."""
    import numpy as np
    import torch

    m, f = pkg.maisi, pkg.fast_fp32
    if what in ("unet", "unet_bf16", "unet_f16x2"):
        uc = m.PRODUCTION_UNET_CONSTRUCTOR
        w = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.unet_weight_shapes(uc), seed=7).items()}
        x = torch.from_numpy(np.random.default_rng(3).standard_normal((2, 64, 64, 32, 4), dtype=np.float32)).to(dev)
        t = torch.full((2,), 500.0, device=dev)
        cls = torch.tensor([9, 0], device=dev)
        sp = m.spacing_tensor([0.94, 0.94, 1.36], device=dev).repeat(2, 1)
        fn = lambda: m.denoise_unet(x, t, cls, sp, w, constructor=uc)
    elif what in ("controlnet", "controlnet_f16x2"):
        # the CT step's ControlNet (production constructor, batch 2, conditioning embedding precomputed)
        cc = m.PRODUCTION_CONTROLNET_CONSTRUCTOR
        w = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.controlnet_weight_shapes(cc), seed=13).items()}
        rng = np.random.default_rng(3)
        x = torch.from_numpy(rng.standard_normal((2, 64, 64, 32, 4), dtype=np.float32)).to(dev)
        emb = torch.from_numpy(rng.standard_normal((2, 64, 64, 32, 64), dtype=np.float32)).to(dev)
        t = torch.full((2,), 500.0, device=dev)
        cls = torch.tensor([9, 0], device=dev)
        fn = lambda: m.controlnet_residuals(x, t, cls, None, w, constructor=cc, conditioning_embedding=emb)
    elif what in ("decode", "decode_bf16", "decode_f16x2"):
        vc = m.PRODUCTION_VAE_CONSTRUCTOR
        w = {k: torch.from_numpy(v).to(dev) for k, v in m.random_weights(m.vae_decoder_weight_shapes(vc), seed=11).items()}
        z = torch.from_numpy(np.random.default_rng(4).standard_normal((1, 20, 64, 64, 4), dtype=np.float32)).to(dev)
        fn = lambda: m.decode_vae(z, w, constructor=vc)
    elif what in ("gemms", "gemms_stream"):
        # config-0 fp32, bf16 and split-fp16 GEMM kernels alone (one pack each), for counter passes;
        # gemms_stream forces the register-streaming GEMM for the bf16 stage (no split-fp16 stage)
        rng = np.random.default_rng(0)
        x = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 64), dtype=np.float32)).to(dev)
        w = torch.from_numpy((rng.standard_normal((64, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)).to(dev)
        b = torch.zeros(64, device=dev)
        codes = (pkg._lib.DT_F32, pkg._lib.DT_BF16) if what == "gemms_stream" else (
            pkg._lib.DT_F32, pkg._lib.DT_BF16, pkg._lib.DT_F16X2)
        stages = [staged_op(pkg, x, w, b, code, stream_gemm=what == "gemms_stream") for code in codes]
        for pack, _, _ in stages:
            pack()

        def fn():
            for _, gemm, _ in stages:
                gemm()
    elif what == "pointwise":
        # config 2c: 1x1x1 128 -> 256 at 64^3 (persistent pointwise GEMM)
        rng = np.random.default_rng(1)
        x = torch.from_numpy(rng.standard_normal((1, 64, 64, 64, 128), dtype=np.float32)).to(dev)
        w = torch.from_numpy((rng.standard_normal((256, 128, 1, 1, 1)) / np.sqrt(128)).astype(np.float32)).to(dev)
        b = torch.zeros(256, device=dev)
        fn = lambda: f.pointwise_conv(x, w, b)
    elif what == "output_convs":
        # the cout <= 4 direct convs with GN + SiLU staged: the VAE decoder's 64 -> 1 at a full 80x256x256
        # window and the UNet's 64 -> 4 at 2x64x64x32
        rng = np.random.default_rng(1)
        calls = []
        for shape, cout in (((1, 80, 256, 256, 64), 1), ((2, 64, 64, 32, 64), 4)):
            x = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dev)
            w = torch.from_numpy((rng.standard_normal((cout, 64, 3, 3, 3)) / np.sqrt(27 * 64)).astype(np.float32)).to(dev)
            g, z0 = torch.ones(64, device=dev), torch.zeros(64, device=dev)
            calls.append((x, w, torch.zeros(cout, device=dev), (g, z0)))

        def fn():
            for x, w, b, norm in calls:
                f.norm_conv3d(x, w, b, norm=norm, num_groups=32, eps=1e-6, apply_silu=True)
    elif what in ("config2a", "config2b"):
        # config 2a: stride-2 conv 64->128, 128^3 -> 64^3; config 2b: nearest-2x + conv 256->128, 64^3 -> 128^3
        rng = np.random.default_rng(1)
        cin, cout, s = (64, 128, 128) if what == "config2a" else (256, 128, 64)
        x = torch.from_numpy(rng.standard_normal((1, s, s, s, cin), dtype=np.float32)).to(dev)
        w = torch.from_numpy((rng.standard_normal((cout, cin, 3, 3, 3)) / np.sqrt(27 * cin)).astype(np.float32)).to(dev)
        b = torch.zeros(cout, device=dev)
        if what == "config2a":
            fn = lambda: f.conv3d(x, w, b, padding=1, stride=2)
        else:
            fn = lambda: f.norm_conv3d(x, w, b, norm=None, num_groups=1, eps=1e-6, apply_silu=False, upsample=True)
    elif what in ("attention", "attention_f16x2"):
        # production UNet level-2 attention: 16x16x8 latent = 2048 tokens, 256 channels = 8 heads, batch 2
        g = torch.Generator(device=dev).manual_seed(0)
        qkv = torch.randn(2, 2048, 3 * 256, device=dev, generator=g)
        q, k, v = qkv[..., :256], qkv[..., 256:512], qkv[..., 512:]
        fn = lambda: f.flash_attention(q, k, v, heads=8, scale=32 ** -0.5)
    else:
        rng = np.random.default_rng(1)
        x = torch.from_numpy(rng.standard_normal((1, 128, 128, 128, 128), dtype=np.float32)).to(dev)
        w1 = torch.from_numpy((rng.standard_normal((128, 128, 3, 3, 3)) / np.sqrt(27 * 128)).astype(np.float32)).to(dev)
        b = torch.zeros(128, device=dev)
        g, z0 = torch.ones(128, device=dev), torch.zeros(128, device=dev)
        fn = lambda: f.vae_resblock([x], (w1, b), (w1, b), (g, z0), (g, z0), None, num_groups=32, eps=1e-6)
    with f.precision(what.rsplit("_", 1)[1] if what.endswith(("_bf16", "_f16x2")) else "fp32"):
        warm_up(fn, warmup)
        ms = _wall_ms(fn, steps)
    print(json.dumps({"only": what, "ms": round(ms, 3), "steps": steps}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip the config 1/2 measurements")
    ap.add_argument("--no-networks", action="store_true", help="skip configs 3/4 and the full generation")
    ap.add_argument("--no-generation", action="store_true", help="skip the full 256^3 generation")
    ap.add_argument("--only", choices=["unet", "unet_bf16", "unet_f16x2", "controlnet", "controlnet_f16x2", "decode",
                                       "decode_bf16", "decode_f16x2", "resblock", "resblock_f16x2",
                                       "attention", "attention_f16x2", "pointwise", "gemms", "gemms_stream", "config2a", "config2b",
                                       "output_convs"],
                    help="profiling mode: run only this workload --steps times and print its timing")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM-counter scale reference for rocprofv3 --pmc)")
    ap.add_argument("--reference-gemms", action="store_true",
                    help="only time the platform's own GEMMs (torch.matmul -> hipBLASLt) and sample the shader "
                         "clock under sustained fp32 / bf16 MFMA load, this library's config-0 GEMMs included")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (N=1); multi-GPU runs are not part of it",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy:
        src = torch.ones(1 << 28, device="cuda:0")  # 1 GiB fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                          "launches": 3}), flush=True)
        return 0

    pkg = importlib.import_module("mlx-generate-ctmr_amd")
    f = pkg.fast_fp32
    dev = torch.device("cuda:0")
    if args.reference_gemms:
        return reference_gemms(pkg, dev)
    if args.only:
        return profile_only(pkg, dev, args.only, args.steps, args.warmup)
    rng = np.random.default_rng(0)
    n, s, cin, cout = 1, 64, 64, 64
    x = torch.from_numpy(rng.standard_normal((n, s, s, s, cin), dtype=np.float32)).to(dev)
    w = torch.from_numpy((rng.standard_normal((cout, cin, 3, 3, 3)) / np.sqrt(27 * cin)).astype(np.float32)).to(dev)
    b = torch.from_numpy((0.01 * rng.standard_normal(cout)).astype(np.float32)).to(dev)
    flops = conv_flops(n, s, s, s, cin, cout)

    step = lambda: f.conv3d(x, w, b, padding=1)
    warm_up(step, args.warmup)
    with gc_quiet():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
    value = flops / (ms * 1e-3) / 1e12

    # dominant kernel (implicit GEMM), HIP events on its stream around each GEMM
    # launch of pack+GEMM rounds
    pack, gemm, _keep = staged_op(pkg, x, w, b, pkg._lib.DT_F32)
    for _ in range(3):
        pack()
        gemm()
    gemm_ms = gemm_ms_in_context(pack, gemm, max(args.steps, 10))
    achieved = flops / (gemm_ms * 1e-3)
    # bf16 variant of the same layer (secondary)
    pack16, gemm16, _keep16 = staged_op(pkg, x, w, b, pkg._lib.DT_BF16)
    for _ in range(3):
        pack16()
        gemm16()
    bf16_ms = gemm_ms_in_context(pack16, gemm16, max(args.steps, 10))
    # split-fp16 variant (the reference's exact mode on fp16 MFMA): the whole operator (pack + GEMM)
    # and its GEMM kernel alone
    with f.precision("f16x2"):
        warm_up(step, args.warmup, settle_s=0.3)
        x16_ms = _wall_ms(step, args.steps)
    packx, gemmx, _keepx = staged_op(pkg, x, w, b, pkg._lib.DT_F16X2)
    for _ in range(3):
        packx()
        gemmx()
    x16_gemm_ms = gemm_ms_in_context(packx, gemmx, max(args.steps, 10))

    result = {
        "metric": "conv3d fp32 TFLOP/s (implicit GEMM, FP32 MFMA)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy default_rng(0) Gaussian input/weights, bias N(0,0.01))",
        "config": {"workload": "config0: conv3d 3x3x3 s1 p1 +bias, NDHWC fp32, N=1, 64^3, Cin=Cout=64",
                   "flop_per_step": flops, "step": "implicit-GEMM conv reading x directly"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 3), "peak": FP32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK, 4), "traffic": None,
                     "kernel": "conv_lds_kernel<false, 0, 1> (fp32 LDS-staged implicit GEMM, one input tensor, no staging transform, one wave set, reads x directly)",
                     "kernel_ms": round(gemm_ms, 4), "kernel_timing": "HIP events around each GEMM launch "
                     "of pack+GEMM rounds on the launch stream"},
    }
    # HBM bytes per GEMM launch from the committed rocprofv3 --pmc passes
    # (FETCH_SIZE x read scale + WRITE_SIZE x write scale, copy-calibrated).
    traffic_file = REPO / "profiles" / "conv3d_config0_traffic.json"
    if traffic_file.exists():
        result["roofline"]["traffic"] = json.loads(traffic_file.read_text())["traffic_bytes"]
        result["roofline"]["traffic_source"] = "profiles/conv3d_config0_traffic.json"
    sec = {"config0_bf16_gemm": {"ms": round(bf16_ms, 4), "tflops": round(flops / bf16_ms / 1e9, 2),
                                 "frac_bf16_peak": round(flops / (bf16_ms * 1e-3) / BF16_PEAK, 4)},
           "config0_f16x2": {"ms": round(x16_ms, 4), "tflops": round(flops / x16_ms / 1e9, 2),
                             "gemm_ms": round(x16_gemm_ms, 4), "gemm_tflops": round(flops / x16_gemm_ms / 1e9, 2),
                             "gemm_frac_f16x2_peak": round(flops / (x16_gemm_ms * 1e-3) / F16X2_PEAK, 4),
                             "f16x2_peak_tflops": round(F16X2_PEAK / 1e12, 1),
                             "kernel": "conv_lds_bf16_kernel<CTMR_F16X2> (split fp16: 4 fp16 MFMA FLOPs per fp32 "
                                       "FLOP; whole op = split pack + GEMM)"}}
    if not args.no_secondary:
        sec.update(secondary(pkg, dev, args.steps, cpu=not args.no_cpu))
    if not args.no_networks:
        sec.update(networks(pkg, dev, args.steps, generation=not args.no_generation, cpu=not args.no_cpu))
    result["secondary"] = sec
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
        progress("config 0 CPU baseline done")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
