"""CPU tests of the C ABI: the library loads, exports every declared symbol, and
its host-side geometry, policy and error paths behave (no kernel is launched)."""

from __future__ import annotations

import ctypes
import subprocess

import pytest


def test_library_exports_every_header_symbol(ctmr, native_loaded):
    declared = ctmr._lib.header_symbols()
    assert "ctmr_conv3d" in declared and len(declared) >= 14
    out = subprocess.run(["nm", "-D", "--defined-only", str(ctmr._lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for name in declared:
        getattr(native_loaded, name)
    assert native_loaded.ctmr_abi_version() == ctmr._lib.ABI_VERSION


def test_prototypes_cover_header(ctmr):
    assert sorted(ctmr._lib._PROTOTYPES) == ctmr._lib.header_symbols()


@pytest.mark.parametrize(
    ("dims", "kw", "expected"),
    [
        ((1, 64, 64, 64, 64, 64), {}, (64, 64, 64)),
        ((1, 7, 6, 5, 32, 64), {"stride": 2}, (4, 3, 3)),
        ((2, 4, 8, 8, 256, 128), {"mode": 1}, (8, 16, 16)),
        ((2, 3, 5, 6, 24, 32), {"mode": 2}, (6, 10, 12)),
        ((1, 9, 6, 8, 128, 256), {"ksize": 1}, (9, 6, 8)),
    ],
)
def test_output_dims(ctmr, dims, kw, expected):
    L = ctmr._lib
    assert L.output_dims(L.conv_desc(*dims, **kw)) == expected


def test_workspace_and_packed_sizes(ctmr):
    L = ctmr._lib
    d = L.conv_desc(1, 64, 64, 64, 64, 64)
    # the LDS-staged GEMM (cin >= 64) reads x directly: no workspace, the (n, cin, 2) affine table with a
    # GN affine; the streaming GEMM (CTMR_F_STREAM, or cin < 64) reads a plain conv with whole 16-channel
    # blocks directly too and packs a padded copy (66^3 rows x 64 fp32 channels, 256-byte aligned) for
    # a GN-affine one
    assert L.workspace_bytes(d) == 0
    assert L.workspace_bytes(L.conv_desc(1, 64, 64, 64, 64, 64, flags=L.F_AFFINE)) == 512
    assert L.workspace_bytes(L.conv_desc(1, 64, 64, 64, 64, 64, flags=L.F_AFFINE | L.F_STREAM)) == \
        ((66**3 * 64 * 4 + 255) // 256) * 256
    assert L.workspace_bytes(L.conv_desc(1, 64, 64, 64, 32, 64, flags=L.F_AFFINE)) == \
        ((66**3 * 32 * 4 + 255) // 256) * 256
    assert L.packed_weight_elems(d) == 27 * 64 * 64
    assert L.conv_split(d) == 1
    # the LDS-staged GEMM (cin >= 64) reads x directly: no workspace without affine or
    # split, just the (n, cin, 2) affine table with one; same packed weight
    d128 = L.conv_desc(1, 64, 64, 64, 128, 128)
    assert L.workspace_bytes(d128) == 0
    assert L.workspace_bytes(L.conv_desc(1, 64, 64, 64, 128, 128, flags=L.F_AFFINE)) == 1024
    assert L.packed_weight_elems(d128) == 27 * 128 * 128
    ds = L.conv_desc(1, 64, 64, 64, 128, 128, flags=L.F_STREAM)
    assert L.workspace_bytes(ds) == 0
    ds = L.conv_desc(1, 64, 64, 64, 128, 128, flags=L.F_STREAM | L.F_SILU)
    assert L.workspace_bytes(ds) == ((66**3 * 128 * 4 + 255) // 256) * 256
    # cin below one K block packs im2col rows: K = 27 * cin rounded to the block; the stride-1
    # fp32 cin 4 / 8 convs read those rows from an LDS halo (no workspace, the affine table with one)
    d4 = L.conv_desc(1, 8, 8, 8, 4, 64)
    assert L.packed_weight_elems(d4) == 112 * 64
    assert L.workspace_bytes(d4) == 0
    assert L.workspace_bytes(L.conv_desc(1, 8, 8, 8, 4, 64, flags=L.F_AFFINE)) == 256
    assert L.workspace_bytes(L.conv_desc(1, 8, 8, 8, 4, 64, flags=L.F_STREAM)) == 8**3 * 112 * 4
    assert L.workspace_bytes(L.conv_desc(1, 8, 8, 8, 4, 64, stride=2)) == 4**3 * 112 * 4
    d16 = L.conv_desc(1, 8, 8, 8, 4, 4, dtype=L.DT_BF16)
    assert L.packed_weight_elems(d16) == 128 * 16
    # cout <= 4: weights packed for one GEMM with 27 * cout columns (padded to
    # 16); fp32 stride-1 convs with whole 16-channel chunks and no residual run
    # the direct conv over an LDS halo (no workspace, the affine table with
    # one), the others the GEMM over every padded row plus the planar tap
    # columns it writes
    d1 = L.conv_desc(1, 8, 8, 8, 64, 1)
    assert L.packed_weight_elems(d1) == 4 * 32 * 16
    assert L.workspace_bytes(d1) == 0
    assert L.workspace_bytes(L.conv_desc(1, 8, 8, 8, 64, 1, flags=L.F_AFFINE)) == 512
    assert L.workspace_bytes(L.conv_desc(1, 8, 8, 8, 64, 1, flags=L.F_STREAM)) == \
        ((10**3 * 64 * 4 + 255) // 256) * 256 + 27 * 10**3 * 4
    assert L.conv_split(d1) == 1
    assert L.packed_weight_elems(L.conv_desc(1, 8, 8, 8, 64, 4, stride=2)) == 4 * 112 * 16
    # nearest-2x parity weights: 8 phases x 8 taps
    du = L.conv_desc(1, 4, 4, 4, 32, 48, mode=L.MODE_NEAREST2X)
    assert L.packed_weight_elems(du) == 8 * 8 * 32 * 48
    # 1x1 with 16-aligned channels reads x directly: no workspace
    assert L.workspace_bytes(L.conv_desc(1, 4, 4, 4, 128, 256, ksize=1)) == 0
    assert L.workspace_bytes(L.conv_desc(1, 4, 4, 4, 4, 4, ksize=1)) > 0


def test_split_policy_is_shape_only(ctmr):
    L = ctmr._lib
    # UNet levels at a 64x64x32 latent, batch 2: the split fills 512 resident workgroups; the deep levels
    # take 64 x 64 tiles whose four waves each sum a quarter of a split range, so a quarter of the planes
    assert L.conv_split(L.conv_desc(2, 4, 8, 8, 512, 512)) == 8  # 64 tiles x 8 (x 4 wave ranges)
    assert L.conv_split(L.conv_desc(2, 4, 8, 8, 512, 512, split=32)) == 32  # an explicit split stays
    assert L.conv_split(L.conv_desc(2, 8, 16, 16, 256, 256)) == 2  # 256 tiles x 2 (x 4 wave ranges)
    assert L.conv_split(L.conv_desc(2, 16, 32, 32, 128, 128)) == 2  # 256 tiles x 2
    assert L.conv_split(L.conv_desc(2, 16, 32, 32, 64, 64)) == 4  # streaming: 128 tiles x 4
    # bf16 stride-1 convs with 64-wide column tiles use the LDS-staged bf16 GEMM: its split divides the
    # 32-channel chunks (2 here) over 4x8x8 bricks; the streaming bf16 GEMM splits the 54 K steps
    assert L.conv_split(L.conv_desc(2, 8, 16, 16, 64, 64, dtype=L.DT_BF16)) == 2  # 16 bricks x 2 chunks
    assert L.conv_split(L.conv_desc(2, 8, 16, 16, 64, 64, dtype=L.DT_BF16, flags=L.F_STREAM)) == 6
    # the persistent one-tap GEMM (1x1x1) splits only launches of under 256 tiles, up to 256 work items
    assert L.conv_split(L.conv_desc(2, 16, 32, 32, 384, 128, ksize=1)) == 1  # 256 tiles of 128 x 128
    assert L.conv_split(L.conv_desc(2, 8, 16, 16, 768, 256, ksize=1)) == 4  # 64 tiles x 4
    assert L.conv_split(L.conv_desc(2, 4, 8, 8, 1024, 512, ksize=1)) == 8  # 32 tiles x 8
    assert L.conv_split(L.conv_desc(2, 4, 8, 8, 128, 512, ksize=1)) == 1  # 8 K steps: below 16, no split
    # large grids never split
    assert L.conv_split(L.conv_desc(1, 128, 128, 128, 128, 128)) == 1
    assert L.conv_split(L.conv_desc(1, 64, 64, 64, 64, 64)) == 1
    # an LDS grid of under 4 rounds whose last round is far from full takes two K ranges: the decoder's
    # 256-channel level, 320 bricks x 4 column tiles = 1280 workgroups (2.5 rounds -> 5 whole rounds);
    # whole rounds (1024) and grids of 4 rounds or more do not
    assert L.conv_split(L.conv_desc(1, 20, 64, 64, 256, 256)) == 2
    # two K ranges over an even chunk count run as two wave sets of one workgroup: no partial planes
    assert L.workspace_bytes(L.conv_desc(1, 20, 64, 64, 256, 256)) == 0
    # three ranges keep the partial planes
    assert L.workspace_bytes(L.conv_desc(1, 20, 64, 64, 256, 256, split=3)) == 3 * 20 * 64 * 64 * 256 * 4
    assert L.conv_split(L.conv_desc(2, 64, 64, 32, 64, 64)) == 1  # 1024
    assert L.conv_split(L.conv_desc(1, 40, 128, 128, 128, 128)) == 1  # 5120
    # an explicit split may be any count up to the K step count (27 taps x 32
    # blocks here); the LDS-staged GEMM takes a split only while each range keeps
    # at least 4 of its 16-channel chunks (5 here: no packed copy in the
    # workspace), larger splits go to the streaming GEMM, which reads a plain
    # conv straight from x (only the partial planes) and packs a GN-affine one
    d5 = L.conv_desc(2, 4, 8, 8, 512, 512, split=5)
    assert L.conv_split(d5) == 5
    assert L.workspace_bytes(d5) == 5 * 2 * 256 * 512 * 4
    d33 = L.conv_desc(2, 4, 8, 8, 512, 512, split=33)
    assert L.conv_split(d33) == 33
    assert L.workspace_bytes(d33) == 33 * 2 * 256 * 512 * 4
    d33a = L.conv_desc(2, 4, 8, 8, 512, 512, split=33, flags=L.F_AFFINE)
    assert L.workspace_bytes(d33a) > 33 * 2 * 256 * 512 * 4
    assert L.conv_split(L.conv_desc(2, 4, 8, 8, 512, 512, split=27 * 32, flags=L.F_STREAM)) == 27 * 32
    with pytest.raises(L.CtmrError, match="step count"):
        L.conv_split(L.conv_desc(2, 4, 8, 8, 512, 512, split=27 * 32 + 1, flags=L.F_STREAM))


@pytest.mark.parametrize(
    ("kw", "status", "message"),
    [
        ({"ksize": 5}, -2, "ksize"),
        ({"stride": 3}, -2, "stride"),
        ({"mode": 2, "flags": 1}, -2, "trilinear"),
        ({"mode": 1, "stride": 2}, -2, "stride 1"),
        ({"ksize": 1, "stride": 2}, -2, "1x1x1"),
        ({"dtype": 7}, -1, "dtype"),
    ],
)
def test_invalid_descriptors(ctmr, native_loaded, kw, status, message):
    L = ctmr._lib
    d = L.conv_desc(1, 4, 4, 4, 16, 16, **kw)
    assert native_loaded.ctmr_conv3d_workspace_bytes(ctypes.byref(d)) == status
    assert message in L.last_error()


def test_conv_rejects_null_and_small_workspace_before_launch(ctmr, native_loaded):
    L = ctmr._lib
    d = L.conv_desc(1, 4, 4, 4, 16, 16)
    rc = native_loaded.ctmr_conv3d(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == L.E_INVALID
    fake = 0x1000  # never dereferenced: the size check fails first
    rc = native_loaded.ctmr_conv3d(ctypes.byref(d), fake, fake, None, None, None, fake, fake, 16, None)
    assert rc == L.E_WORKSPACE and "workspace" in L.last_error()
    d.flags = L.F_RESIDUAL
    rc = native_loaded.ctmr_conv3d_gemm(ctypes.byref(d), fake, fake, None, None, fake, fake, 1 << 40, None)
    assert rc == L.E_INVALID and "residual" in L.last_error()


def test_group_norm_host_checks(ctmr, native_loaded):
    L = ctmr._lib
    assert L.gn_workspace_bytes(1, 128**3, 128) == 1 * 2048 * 128 * 2 * 8  # capped at 2048 chunks
    assert L.gn_workspace_bytes(2, 64 * 64 * 32, 64) == 2 * 512 * 64 * 2 * 8  # 256-voxel chunks
    rc = native_loaded.ctmr_gn_affine(1, 64, 12, 5, 1e-6, 0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 1 << 30, None)
    assert rc == L.E_INVALID and "divisible" in L.last_error()
    rc = native_loaded.ctmr_gn_affine(1, 64, 258, 2, 1e-6, 0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 1 << 30, None)
    assert rc == L.E_UNSUPPORTED
    rc = native_loaded.ctmr_resample(0, 1, 1, 4, 4, 4, 0x1000, 0x1000, None)
    assert rc == L.E_INVALID and "pooling" in L.last_error()


def test_attention_desc_layout_matches_header(ctmr):
    """ctmr_attn_desc: six int32, four int64 strides, one float (natural alignment)."""
    D = ctmr._lib.AttnDesc
    assert D.ldq.offset == 24 and D.ldo.offset == 48 and D.scale.offset == 56
    assert ctypes.sizeof(D) == 64


@pytest.mark.parametrize(
    ("kw", "status", "message"),
    [
        ({"head_dim": 16}, -2, "head_dim 16 unsupported"),
        ({"query_tiles": 3}, -1, "query_tiles"),
        ({"lk": 0}, -1, ">= 1"),
        ({"n": 300, "heads": 256}, -1, "65535"),
        ({"ldk": 60}, -1, "below heads"),
        ({"ldv": 66}, -1, "multiples of 4"),
        ({"scale": float("inf")}, -1, "finite"),
    ],
)
def test_attention_host_checks(ctmr, native_loaded, kw, status, message):
    """Every rejection happens on the host, before any launch (fake pointers are never touched)."""
    base = dict(n=2, lq=64, lk=64, heads=2, head_dim=32, query_tiles=0, ldq=64, ldk=64, ldv=64, ldo=64, scale=0.17)
    base.update(kw)
    d = ctmr._lib.AttnDesc(**base)
    fake = ctypes.c_void_p(1 << 20)
    rc = native_loaded.ctmr_flash_attention(ctypes.byref(d), fake, fake, fake, fake, None)
    assert rc == status
    assert message in ctmr._lib.last_error()
    assert native_loaded.ctmr_flash_attention(ctypes.byref(d), None, fake, fake, fake, None) == -1
    good = ctmr._lib.AttnDesc(**{**base, **dict(head_dim=32, query_tiles=0, lk=64, n=2, heads=2, ldk=64,
                                                 ldv=64, scale=0.17)})
    misaligned = ctypes.c_void_p((1 << 20) + 4)
    assert native_loaded.ctmr_flash_attention(ctypes.byref(good), misaligned, fake, fake, fake, None) == -1
    assert "16-byte aligned" in ctmr._lib.last_error()


@pytest.mark.parametrize(
    ("kw", "status", "message"),
    [
        ({"head_dim": 16}, -2, "head_dim 16 unsupported"),
        ({"query_tiles": 3}, -1, "query_tiles"),
        ({"lq": 0}, -1, ">= 1"),
        ({"n": 300, "heads": 256}, -1, "65535"),
        ({"ldo": 60}, -1, "below heads"),
        ({"ldq": 66}, -1, "multiples of 4"),
        ({"scale": float("nan")}, -1, "finite"),
    ],
)
def test_split_attention_host_checks(ctmr, native_loaded, kw, status, message):
    """ctmr_flash_attention_f16x2 applies the same checks, then its workspace's size and alignment,
    all on the host before any launch (fake pointers are never touched)."""
    base = dict(n=2, lq=64, lk=50, heads=2, head_dim=32, query_tiles=0, ldq=64, ldk=64, ldv=64, ldo=64, scale=0.17)
    fake, ws = ctypes.c_void_p(1 << 20), ctypes.c_void_p(1 << 24)
    d = ctmr._lib.AttnDesc(**{**base, **kw})
    assert native_loaded.ctmr_flash_attention_f16x2(ctypes.byref(d), fake, fake, fake, fake, ws, 1 << 30, None) == status
    assert message in ctmr._lib.last_error() and "ctmr_flash_attention_f16x2" in ctmr._lib.last_error()
    good = ctmr._lib.AttnDesc(**base)
    # six fp16 planes of n * heads * 32 values per row: Q over lq rows, K and V over lk rounded up to 32
    need = native_loaded.ctmr_flash_attention_f16x2_workspace_bytes(ctypes.byref(good))
    assert need == 2 * 2 * 2 * 2 * 32 * (64 + 2 * 64)
    if kw.get("lq") == 0:
        assert native_loaded.ctmr_flash_attention_f16x2_workspace_bytes(ctypes.byref(d)) == -1
    args = (ctypes.byref(good), fake, fake, fake, fake)
    assert native_loaded.ctmr_flash_attention_f16x2(*args, ws, need - 1, None) == -1
    assert "workspace of" in ctmr._lib.last_error()
    assert native_loaded.ctmr_flash_attention_f16x2(*args, None, need, None) == -1
    assert native_loaded.ctmr_flash_attention_f16x2(*args, ctypes.c_void_p((1 << 24) + 128), need, None) == -1
    assert "256-byte aligned" in ctmr._lib.last_error()


def test_conv_group_norm_partial_tiles(ctmr, native_loaded):
    """``ctmr_conv3d_stats_tiles``: partials per batch item, or 0 where the epilogue cannot write them."""
    L = ctmr._lib

    def tiles(groups, *dims, **kw):
        return native_loaded.ctmr_conv3d_stats_tiles(ctypes.byref(L.conv_desc(*dims, **kw)), groups)

    assert tiles(32, 1, 64, 64, 64, 128, 128) == 16 * 8 * 8  # LDS-staged: one per 4x8x8 brick
    assert tiles(32, 1, 64, 64, 64, 64, 64) == 64**3 // 256  # streaming: one per 256-voxel M tile
    # K split: the reduction writes them, one per chunk of 16 * rows output voxels (rows keeps ~1024 blocks)
    assert tiles(32, 2, 4, 8, 8, 512, 512) == 256 // 16
    assert tiles(32, 2, 16, 32, 32, 128, 128, split=4) == 16 * 32 * 32 // (16 * 4)
    # a split of two over an even chunk count runs as two wave sets of one LDS-GEMM workgroup, whose
    # epilogue writes them: one per 4x8x8 brick
    assert L.conv_split(L.conv_desc(2, 16, 32, 32, 128, 128)) == 2
    assert tiles(32, 2, 16, 32, 32, 128, 128) == 4 * 4 * 4
    assert tiles(3, 1, 8, 8, 8, 256, 96, split=4) == 0  # split reduce works on 64-column tiles
    assert tiles(2, 1, 8, 8, 8, 256, 256, split=4) == 0  # 128-wide groups
    assert tiles(1, 1, 8, 8, 8, 64, 1) == 0  # cout <= 4: outputs come from the tap sum
    assert tiles(3, 1, 8, 8, 8, 64, 128) == 0  # groups must divide cout
    # 256 columns in two 128-wide workgroup tiles: a group may not straddle them
    assert tiles(1, 1, 16, 16, 16, 256, 256, flags=L.F_STREAM, split=1) == 0
    assert tiles(2, 1, 16, 16, 16, 256, 256, flags=L.F_STREAM, split=1) == 16**3 // 128
    # nearest-2x upsample: one tile per (parity phase, source M tile)
    assert tiles(3, 1, 4, 4, 4, 32, 48, mode=L.MODE_NEAREST2X, split=1) == 8
    # bf16 nearest-2x on the LDS GEMM: one per (4x8x8 source brick, parity)
    assert tiles(32, 2, 32, 32, 16, 128, 128, mode=L.MODE_NEAREST2X, dtype=L.DT_BF16, split=1) == (32 // 4) * (32 // 8) * (16 // 8) * 8
    assert tiles(2, 1, 4, 4, 4, 32, 48, mode=L.MODE_NEAREST2X, split=1) == 0  # 24-wide groups vs 64 columns
    d = L.conv_desc(1, 8, 8, 8, 64, 1)
    fake = 0x1000  # never dereferenced: the checks fail first
    rc = native_loaded.ctmr_conv3d_gn(ctypes.byref(d), fake, fake, None, None, None, fake, fake, 1 << 40, 1, fake,
                                      None)
    assert rc == L.E_UNSUPPORTED and "partials" in L.last_error()
    d = L.conv_desc(1, 8, 8, 8, 64, 64)
    rc = native_loaded.ctmr_conv3d_gn(ctypes.byref(d), fake, fake, None, None, None, fake, fake, 1 << 40, 32, None,
                                      None)
    assert rc == L.E_INVALID
    rc = native_loaded.ctmr_gn_affine_from_stats(1, 4, 12, 5, 64, 1e-6, fake, fake, fake, fake, None)
    assert rc == L.E_INVALID and "divisible" in L.last_error()
    rc = native_loaded.ctmr_gn_affine_from_stats(1, 0, 12, 4, 64, 1e-6, fake, fake, fake, fake, None)
    assert rc == L.E_INVALID


@pytest.mark.parametrize(("shape", "cout", "kw", "expected"), [
    ((1, 64, 64, 64, 64), 64, {}, "lds"),                                 # config 0
    ((1, 128, 128, 128, 128), 128, {"flags": 3}, "lds"),                  # config 1 (GN affine + SiLU)
    ((1, 128, 128, 128, 64), 128, {"stride": 2}, "stream_direct"),       # config 2a
    ((1, 64, 64, 64, 256), 128, {"mode": 1}, "stream"),                   # config 2b
    ((1, 64, 64, 64, 128), 256, {"ksize": 1}, "pointwise"),               # config 2c
    ((1, 64, 64, 64, 64), 64, {"flags": 16}, "stream_direct"),            # CTMR_F_STREAM
    ((1, 64, 64, 64, 64), 64, {"dtype": 1}, "lds_bf16"),
    ((2, 32, 32, 16, 128), 128, {"dtype": 1, "mode": 1}, "lds_bf16"),     # bf16 nearest-2x: 8 parity GEMMs
    ((2, 8, 8, 4, 512), 512, {"dtype": 1}, "lds_bf16"),                   # bf16, bricks half full (w = 4)
    ((2, 8, 8, 3, 512), 512, {"dtype": 1}, "split_waves"),                # bf16, bricks under half full
    ((2, 32, 32, 16, 128), 128, {"mode": 1}, "stream"),                   # fp32 nearest-2x
    ((2, 32, 32, 16, 128), 128, {"dtype": 1, "mode": 1, "flags": 16}, "stream"),  # CTMR_F_STREAM
    ((2, 4, 8, 8, 512), 512, {}, "split_waves"),                          # deep UNet level
    ((1, 20, 64, 64, 64), 1, {"flags": 3}, "small_cout"),                 # decoder output conv (GN + SiLU)
    ((2, 64, 64, 32, 64), 4, {"flags": 3}, "small_cout"),                 # UNet output conv
    ((2, 64, 64, 32, 64), 4, {"flags": 3 | 8}, "tap_expand"),             # with a residual
    ((1, 20, 64, 64, 64), 1, {"flags": 16}, "tap_expand"),                # CTMR_F_STREAM
    ((2, 64, 64, 32, 4), 64, {}, "lds_small"),                            # conv_in: im2col rows from LDS
    ((1, 256, 256, 256, 8), 8, {}, "lds_small"),                          # condition encoder 8 -> 8
    ((1, 256, 256, 256, 8), 32, {"stride": 2}, "stream"),                 # stride 2: im2col rows in HBM
    ((2, 64, 64, 32, 4), 64, {"flags": 16}, "stream"),                    # CTMR_F_STREAM: the im2col GEMM
    # brick epilogues store at 32-bit offsets from the brick's first output plane: the brick's output
    # planes (4, or 8 for nearest-2x) must span under 2 GiB; at 2 GiB the route moves off the brick GEMMs
    ((1, 8, 256, 256, 64), 1024, {}, "lds"),                              # 4 x 256 x 256 x 1024 x 4 B = 1 GiB
    ((1, 8, 256, 256, 64), 2048, {}, "stream_direct"),                    # 2 GiB
    ((1, 8, 256, 256, 64), 1024, {"dtype": 1}, "lds_bf16"),
    ((1, 8, 256, 256, 64), 2048, {"dtype": 1}, "stream"),
    ((1, 8, 128, 128, 64), 512, {"dtype": 1, "mode": 1}, "lds_bf16"),     # 8 x 256 x 256 x 512 x 4 B = 1 GiB
    ((1, 8, 128, 128, 64), 1024, {"dtype": 1, "mode": 1}, "stream"),      # 2 GiB
    ((1, 8, 256, 256, 4), 1024, {}, "lds_small"),
    ((1, 8, 256, 256, 4), 2048, {}, "pointwise"),                         # the im2col GEMM
])
def test_conv_kernel_route(ctmr, shape, cout, kw, expected):
    """``ctmr_conv3d_kernel`` names the formulation the library picks (a function of the desc only)."""
    L = ctmr._lib
    n, d, h, w, cin = shape
    desc = L.conv_desc(n, d, h, w, cin, cout, **kw)
    assert L.conv_kernel(desc) == expected


@pytest.mark.parametrize(("shape", "cin1", "cout", "kw", "expected"), [
    ((2, 64, 64, 32, 192), 128, 64, {}, "lds"),                      # up-block conv1: hidden 128 + skip 64
    ((2, 64, 64, 32, 192), 128, 64, {"flags": 3}, "lds"),            # with the GN affine + SiLU staging
    ((2, 64, 64, 32, 192), 128, 64, {"ksize": 1}, "pointwise"),      # skip projection: read in place
    ((2, 64, 64, 32, 192), 128, 64, {"ksize": 1, "flags": 4}, "stream"),  # per-batch bias: packed first
    ((2, 4, 8, 8, 1024), 512, 512, {}, "split_waves"),               # deep level: packed first
    ((2, 64, 64, 32, 192), 128, 64, {"flags": 16}, "stream"),        # CTMR_F_STREAM: packed, never direct
    ((2, 32, 32, 16, 384), 256, 128, {"dtype": 1}, "lds_bf16"),      # bf16: the packed copy
    ((2, 64, 64, 32, 96), 64, 4, {"flags": 3}, "small_cout"),        # cout <= 4 direct conv: read in place
])
def test_two_source_routes(ctmr, shape, cin1, cout, kw, expected):
    """A two-source input (cin1 > 0) is read in place by the LDS-staged GEMM, the persistent 1x1 GEMM
    and the cout <= 4 direct conv, and packed (both tensors into the usual padded copy) for every other
    route."""
    L = ctmr._lib
    n, d, h, w, cin = shape
    desc = L.conv_desc(n, d, h, w, cin, cout, cin1=cin1, **kw)
    assert L.conv_kernel(desc) == expected
    one = L.conv_desc(n, d, h, w, cin, cout, **kw)
    assert L.packed_weight_elems(desc) == L.packed_weight_elems(one)  # the weight does not change
    if expected in ("lds", "pointwise", "small_cout"):
        assert L.workspace_bytes(desc) == L.workspace_bytes(one)
    else:
        assert L.workspace_bytes(desc) > 0  # the packed copy of both tensors


def test_two_source_validation(ctmr, native_loaded):
    L = ctmr._lib
    fake = 0x1000  # never dereferenced: the checks fail first
    for cin1 in (-16, 8, 192, 200):  # negative, not a multiple of 16, not below cin
        d = L.conv_desc(1, 8, 8, 8, 192, 64, cin1=cin1)
        with pytest.raises(RuntimeError):
            L.conv_kernel(d)
    d = L.conv_desc(1, 8, 8, 8, 192, 64, cin1=128, mode=L.MODE_NEAREST2X)
    with pytest.raises(RuntimeError, match="PLAIN"):
        L.conv_kernel(d)
    d = L.conv_desc(1, 8, 8, 8, 192, 64, cin1=128)
    rc = native_loaded.ctmr_conv3d(ctypes.byref(d), fake, fake, None, None, None, fake, fake, 1 << 20, None)
    assert rc == L.E_INVALID and "ctmr_conv3d_cat" in L.last_error()
    one = L.conv_desc(1, 8, 8, 8, 192, 64)
    rc = native_loaded.ctmr_conv3d_cat(ctypes.byref(one), fake, fake, fake, None, None, None, fake, fake, 1 << 20,
                                       None)
    assert rc == L.E_INVALID and "cin1" in L.last_error()
    rc = native_loaded.ctmr_conv3d_cat(ctypes.byref(d), fake, None, fake, None, None, None, fake, fake, 1 << 20,
                                       None)
    assert rc == L.E_INVALID
    rc = native_loaded.ctmr_gn_affine_cat(1, 512, 128, 0, 32, 1e-6, fake, fake, fake, fake, fake, fake, 1 << 20,
                                          None)
    assert rc == L.E_INVALID
    rc = native_loaded.ctmr_gn_affine_cat(1, 512, 126, 66, 32, 1e-6, fake, fake, fake, fake, fake, fake, 1 << 20,
                                          None)
    assert rc == L.E_INVALID and "multiples of 4" in L.last_error()


def test_group_norm_from_finer_statistics_host_checks(ctmr, native_loaded):
    """``ctmr_gn_affine_from_stats2`` accepts exactly the stat groupings ``fast_fp32`` routes to it (the
    tiling rule is checked before the pointers, so a null gamma marks an accepted grouping), and
    ``ctmr_add_gn_partials`` rejects what its kernel cannot read."""
    from importlib import import_module

    L = ctmr._lib
    ff = import_module(ctmr.__name__ + ".fast_fp32")
    fake = 0x1000
    fn = native_loaded.ctmr_gn_affine_from_stats2
    cases = 0
    for c1, c2, groups in ((64, 64, 32), (256, 128, 32), (128, 64, 32), (64, 0, 32), (96, 0, 32), (256, 256, 32),
                           (512, 256, 32), (48, 16, 8)):
        c = c1 + c2
        for sg1 in sorted({1, 2, 4, 8, 16, 32, 64, c1 // 4, c1 // 2, c1} - {0}):
            for sg2 in (sorted({1, 4, 16, 32, c2 // 2, c2} - {0}) if c2 else [1]):
                ok = ff._stats_tile_groups(0, c1, sg1, c, groups) and (
                    c2 == 0 or ff._stats_tile_groups(c1, c2, sg2, c, groups))
                rc = fn(1, groups, 64, 1e-6, fake, 4, c1, sg1, fake if c2 else None, 4 if c2 else 0, c2, sg2, None,
                        fake, fake, None)
                assert rc == L.E_INVALID
                assert ("null pointer" if ok else "do not tile") in L.last_error(), (c1, c2, groups, sg1, sg2)
                cases += 1
    assert cases > 100
    # per-channel statistics tile every grouping; the norm's own groups tile it; a 12-wide group straddling
    # 256 + 128 channels does not split into 8-channel stat groups
    assert ff._stats_tile_groups(0, 256, 256, 384, 32) and ff._stats_tile_groups(256, 128, 32, 384, 32)
    assert not ff._stats_tile_groups(0, 256, 32, 384, 32)
    assert not ff._stats_tile_groups(0, 64, 16, 64, 32)  # stat groups coarser than the norm's
    rc = fn(1, 5, 64, 1e-6, fake, 4, 64, 64, None, 0, 0, 1, fake, fake, fake, None)
    assert rc == L.E_INVALID and "divisible" in L.last_error()
    rc = fn(1, 32, 64, 1e-6, fake, 0, 64, 64, None, 0, 0, 1, fake, fake, fake, None)
    assert rc == L.E_INVALID
    add = native_loaded.ctmr_add_gn_partials
    rc = add(1, 64, 6, fake, fake, fake, fake, 1 << 20, None)
    assert rc == L.E_UNSUPPORTED
    rc = add(1, 64, 64, fake + 4, fake, fake, fake, 1 << 20, None)
    assert rc == L.E_INVALID and "aligned" in L.last_error()
    rc = add(1, 64, 64, fake, fake, fake, fake, 16, None)
    assert rc == L.E_WORKSPACE
    assert add(1, 64, 64, None, fake, fake, fake, 1 << 20, None) == L.E_INVALID
