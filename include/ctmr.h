/*
 * ctmr.h — C ABI of libctmr_hip.so, the MI355X (gfx950) implementation of
 * mlx-generate-ctmr's fast FP32 convolution / group-norm hot path.
 *
 * Every activation is NDHWC (channels innermost), fp32 unless a descriptor
 * says bf16.  All pointers are device pointers owned by the caller; the
 * library never allocates or frees device memory.  Every call is enqueued on
 * the caller's HIP stream (`stream`, a hipStream_t passed as void*; NULL is
 * the default stream) and returns immediately.  Return value: CTMR_OK (0) or
 * one of the negative CTMR_E* codes; ctmr_last_error() gives a message for
 * the calling thread.  Nothing in the library calls exit/abort.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   ctmr_conv3d               <- _nax_conv.nax_conv3d (src/mlx_generate_ctmr/_nax_conv.py:475-684),
 *                                i.e. its pack (:144-198), conv (:200-318) and
 *                                reduce (:320-332) metal_kernel launches (:586-665)
 *   ctmr_conv3d_workspace_bytes <- the packed-copy / split-plane sizing in
 *                                nax_conv3d (:571-581, :667-672)
 *   ctmr_pack_weight          <- _nax_conv.pack_weight (:391-404)
 *   ctmr_pack_upsample_weight <- _nax_conv.pack_upsample_weight (:407-445)
 *   ctmr_gn_affine            <- medmlx_core.group_norm.group_norm_affine, called at
 *                                fast_fp32.py:185-189 (per-(b,c) scale/offset pairs,
 *                                layout described at _nax_conv.py:502-504)
 *   ctmr_gn_apply             <- fast_fp32.group_norm_ncdhw (fast_fp32.py:102-118)
 *   ctmr_conv3d (ksize 1)     <- fast_fp32.pointwise_conv_ncdhw (fast_fp32.py:121-130)
 *   ctmr_resample             <- medmlx_core.ops.avg_pool3d_ncdhw / upsample_nearest_ncdhw
 *                                (fast_fp32.py:48-59) and source_vae.upsample_trilinear_ncdhw
 *                                (fast_fp32.py:66-68; formula at _nax_conv.py:115-142)
 *   ctmr_gn_avgpool           <- the down branch of fast_fp32.residual_block_ncdhw
 *                                (fast_fp32.py:250-255: group norm + SiLU, then pooling)
 *   ctmr_flash_attention      <- _flash_attention.flash_attention (_flash_attention.py:320-360),
 *                                selected by flash_eligible (_flash_attention.py:276-289) from
 *                                fast_fp32.self_attention_tokens (fast_fp32.py:352-392)
 *   ctmr_flash_attention_f16x2 <- the split-fp16 branch of _flash_attention.flash_attention
 *                                (_flash_attention.py:336-350: _split, _nax_kernel / _NAX_SOURCE)
 */
#ifndef CTMR_H
#define CTMR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CTMR_ABI_VERSION 5

enum ctmr_status {
  CTMR_OK = 0,
  CTMR_E_INVALID = -1,     /* bad descriptor / shape / null pointer */
  CTMR_E_UNSUPPORTED = -2, /* valid request this build does not implement */
  CTMR_E_WORKSPACE = -3,   /* workspace smaller than ctmr_conv3d_workspace_bytes */
  CTMR_E_LAUNCH = -4       /* HIP reported an error at launch */
};

/* Input resampling applied while staging the convolution input. */
enum ctmr_conv_mode {
  CTMR_MODE_PLAIN = 0,       /* conv of x itself (stride 1 or 2) */
  CTMR_MODE_NEAREST2X = 1,   /* conv of nearest-2x upsampled x; weights from
                                ctmr_pack_upsample_weight (parity fold) */
  CTMR_MODE_TRILINEAR2X = 2  /* conv of half-pixel trilinear-2x upsampled x */
};

enum ctmr_conv_flags {
  CTMR_F_AFFINE = 1,     /* y = x*affine[b,c,0] + affine[b,c,1] before the conv */
  CTMR_F_SILU = 2,       /* SiLU after the affine (or on x) before the conv */
  CTMR_F_BATCH_BIAS = 4, /* bias is (N, Cout) instead of (Cout) */
  CTMR_F_RESIDUAL = 8,   /* residual (output-shaped, NDHWC) added before the store */
  CTMR_F_STREAM = 16,    /* use the one-tile-per-workgroup register-streaming GEMM even
                            where the LDS-staged or the persistent pointwise one
                            applies (comparisons and tests) */
  CTMR_F_SPLIT_WAVES = 32 /* the CTMR_K_SPLIT_WAVES form (each split range over the four
                            waves) with desc->split (2 .. taps * K blocks / 32) ranges,
                            which the library otherwise picks only by its own policy
                            (split 0): a depth slab of such a conv keeps its summation
                            order (CTMR_E_INVALID where the form does not apply) */
};

enum ctmr_dtype {
  CTMR_F32 = 0,   /* fp32 operands, FP32 MFMA (v_mfma_f32_16x16x4_f32) */
  CTMR_BF16 = 1,  /* bf16 operands, fp32 accumulate (v_mfma_f32_16x16x32_bf16);
                     activations and outputs stay fp32 in memory */
  CTMR_F16X2 = 2  /* split fp16, the reference's "exact" mode for fp32 tensors
                     (_nax_conv.py:27-35): each fp32 input value is held as
                     hi = fp16(v) and lo = fp16((v - hi) * 2^11), each weight
                     (scaled per output column by a power of two) as hi and
                     lo = fp16(w - hi), and every product is summed as
                     hi*hi + (lo*hi)*2^-11 + hi*lo on fp16 MFMA
                     (v_mfma_f32_16x16x32_f16) with fp32 accumulation: about
                     2^-22 relative per product, against 2^-24 for fp32.  Values
                     must stay below 65504 in magnitude (fp16 range of hi).
                     Stride-1 3x3x3 convs with cout % 64 == 0 and bricks at
                     least half full only (the LDS-staged 16-bit GEMM);
                     CTMR_E_UNSUPPORTED otherwise. */
};

typedef struct ctmr_conv_desc {
  int32_t n, d, h, w;   /* input (source-grid) batch and spatial size */
  int32_t cin, cout;    /* channels */
  int32_t ksize;        /* 3 (padding 1) or 1 (padding 0) */
  int32_t stride;       /* 1 or 2 (2 only for ksize 3, CTMR_MODE_PLAIN) */
  int32_t mode;         /* enum ctmr_conv_mode */
  int32_t flags;        /* enum ctmr_conv_flags, OR-ed */
  int32_t dtype;        /* enum ctmr_dtype */
  int32_t split;        /* K split: 0 = library policy (from the shape only: grids of under
                           512 workgroups, and fp32 LDS-GEMM grids of under 4 rounds whose
                           last round would be far from full), else the number of
                           contiguous ranges of the (tap, channel block) step sequence,
                           1 .. taps * ceil(cin / K block) */
  int32_t cin1;         /* 0: the input is one tensor of cin channels.  Else the input is the
                           channel concatenation of two tensors (ctmr_conv3d_cat), x1 with
                           channels [0, cin1) and x2 with [cin1, cin); cin1 and cin multiples
                           of 16, CTMR_MODE_PLAIN */
} ctmr_conv_desc;

/* Library identity; returns CTMR_ABI_VERSION. */
int ctmr_abi_version(void);
/* Message for the last non-zero status returned on this thread. */
const char* ctmr_last_error(void);

/* Output spatial extent of a conv described by `desc` (out[0..2] = D', H', W'). */
int ctmr_conv3d_output_dims(const ctmr_conv_desc* desc, int32_t out[3]);

/* Packed-weight element count (fp32 for CTMR_F32, bf16 for CTMR_BF16, 16-bit
 * elements for CTMR_F16X2: per (phase, tap, 16-channel block, column) 48
 * halves -- hi, hi * 2^-11 and lo of the scaled weight -- then one fp32
 * power-of-two column scale per packed column). */
int64_t ctmr_packed_weight_elems(const ctmr_conv_desc* desc);

/* Scratch bytes ctmr_conv3d needs for `desc` (padded input copy + split planes). */
int64_t ctmr_conv3d_workspace_bytes(const ctmr_conv_desc* desc);

/* The split ctmr_conv3d will use for `desc` (resolves desc->split == 0). */
int ctmr_conv3d_split(const ctmr_conv_desc* desc);

/* GEMM formulation ctmr_conv3d runs for `desc`.  No entry point of its own in
 * the reference, whose route is the _use_nax gate plus the split choice
 * (fast_fp32.py:93-99, _nax_conv.py:578-581); tests and tools use it to
 * assert which kernel a shape takes (the choice depends on the desc only). */
enum ctmr_conv_kernel {
  CTMR_K_STREAM = 0,        /* register-streaming GEMM over the packed copy */
  CTMR_K_STREAM_DIRECT = 1, /* register-streaming GEMM reading x itself */
  CTMR_K_LDS = 2,           /* fp32 LDS-staged GEMM (halo bricks of x) */
  CTMR_K_LDS_BF16 = 3,      /* bf16 LDS-staged GEMM over the packed copy */
  CTMR_K_POINTWISE = 4,     /* persistent one-tap GEMM (1x1x1, im2col rows) */
  CTMR_K_SPLIT_WAVES = 5,   /* 64 x 64 tiles, each split range over the four waves */
  CTMR_K_TAP_EXPAND = 6,    /* cout <= 4: 27*cout-column GEMM + tap sum */
  CTMR_K_LDS_SMALL = 7,     /* cin 4 / 8: im2col rows read from an LDS halo brick */
  CTMR_K_SMALL_COUT = 8,    /* cout <= 4: direct FMA conv from an LDS halo brick */
  CTMR_K_LDS_F16X2 = 9      /* split-fp16 LDS-staged GEMM over the packed hi/lo copy */
};
int ctmr_conv3d_kernel(const ctmr_conv_desc* desc);

/*
 * Reorder a Torch-layout weight (Cout, Cin, k, k, k) fp32 into the layout the
 * conv kernel reads.  desc->mode NEAREST2X is rejected here (use
 * ctmr_pack_upsample_weight); desc->dtype selects fp32 or bf16 output.
 */
int ctmr_pack_weight(const ctmr_conv_desc* desc, const float* weight, void* packed,
                     void* stream);

/* Fold a 3x3x3 weight into the eight 2x2x2 nearest-2x parity filters, summed
 * in fp32 (mirrors pack_upsample_weight's fold, _nax_conv.py:407-445). */
int ctmr_pack_upsample_weight(const ctmr_conv_desc* desc, const float* weight, void* packed,
                              void* stream);

/*
 * y = conv(resample(silu?(affine?(x)))) + bias (+ residual), NDHWC fp32.
 *   x        (n, d, h, w, cin)
 *   packed   from ctmr_pack_weight / ctmr_pack_upsample_weight with the same desc
 *   bias     (cout) or (n, cout) with CTMR_F_BATCH_BIAS; may be NULL (zero bias)
 *   affine   (n, cin, 2) fp32 (scale, offset) pairs with CTMR_F_AFFINE, else NULL
 *   residual output-shaped NDHWC with CTMR_F_RESIDUAL, else NULL
 *   y        (n, D', H', W', cout); must not alias x or residual
 * y, residual and workspace must start on 16-byte boundaries where the
 * persistent pointwise GEMM or the bf16 LDS GEMM is chosen (16-byte stores);
 * CTMR_E_INVALID otherwise.
 * Accumulation order is fixed for a given desc.  The register-streaming GEMM
 * visits taps kd*9+kh*3+kw ascending (outer) and input channels in ascending
 * 16-wide (fp32) / 32-wide (bf16) blocks (inner).  The LDS-staged GEMM, chosen
 * by shape for large stride-1 fp32 volumes (cin >= 64 and a multiple of 16,
 * cout % 64 == 0, no resampling, CTMR_F_STREAM not set), stages 16-channel chunks of the input
 * with their halo (affine + SiLU and zero padding applied while staging) and
 * visits chunks ascending (outer), taps ascending (inner).  The LDS-staged
 * bf16 GEMM, chosen for stride-1 bf16 convs (plain, trilinear-2x, or
 * nearest-2x as the eight parity GEMMs of the fold) with cout % 64 == 0 and
 * 4x8x8 bricks at least half full (CTMR_F_STREAM not set), reads the bf16
 * packed copy and visits 32-channel chunks ascending (outer), taps ascending
 * (inner).  Deep small grids split by the library's policy (split of
 * at least 4 for the 128-wide tiles) run 64 x 64 tiles whose four waves sum
 * four contiguous quarters of each split range, added in ascending order
 * before the partial plane is stored; ctmr_conv3d_split reports the ranges.
 * A split of two of those (and of the fp32 LDS-staged GEMM, over an even
 * count of 16-channel chunks) runs inside one 512-thread workgroup as two
 * wave sets: the second range's sum is added after the bias, the order of
 * the split reduction, with no partial planes in the workspace.
 * One-tap GEMMs (1x1x1, im2col rows) with cout % 4 == 0 and
 * no per-batch bias or residual run on a persistent grid with the streaming
 * GEMM's per-output order, so their outputs equal the CTMR_F_STREAM ones bit
 * for bit.  With a split, each
 * contiguous range of the sequence is summed separately and the partial planes
 * are added in ascending order after the bias.  Kernel, split and tiling depend
 * on the desc only, so results are bit-identical run to run.
 */
int ctmr_conv3d(const ctmr_conv_desc* desc, const float* x, const void* packed,
                const float* bias, const float* affine, const float* residual, float* y,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * ctmr_conv3d of the channel concatenation of two NDHWC tensors without
 * materialising it: x1 holds channels [0, desc->cin1), x2 channels
 * [desc->cin1, desc->cin) (cin1 and cin multiples of 16, CTMR_MODE_PLAIN),
 * both on the same voxel grid.  Replaces the concatenation ahead of the
 * UNet's up-path residual blocks (unet.py:444, mx.concatenate of the hidden
 * state and the skip, then fast_fp32.residual_block_ncdhw); no separate
 * entry point exists in the reference.  The LDS-staged GEMM stages each
 * 16-channel chunk from its tensor and the persistent 1x1x1 GEMM reads each
 * K block from its tensor; other routes pack both into the usual padded copy.
 * Same products in the same order as ctmr_conv3d on the concatenated tensor,
 * so bit-identical outputs.  Workspace: ctmr_conv3d_workspace_bytes(desc).
 * ctmr_conv3d_cat_gn is the ctmr_conv3d_gn counterpart.
 */
int ctmr_conv3d_cat(const ctmr_conv_desc* desc, const float* x1, const float* x2, const void* packed,
                    const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * ctmr_conv3d without a caller workspace and without any allocation: the
 * workspace is a library-owned device array of CTMR_NOALLOC_SCRATCH_BYTES per
 * GPU (allocated when the library's code is loaded on that GPU, held until
 * the process ends).  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same kernels and bits as
 * ctmr_conv3d.  A convolution whose ctmr_conv3d_workspace_bytes exceeds the
 * limit returns CTMR_E_WORKSPACE (256 MiB covers every conv of the MAISI UNet
 * and ControlNet steps at a 64x64x32 latent, batch 2; not the decoder's
 * full-resolution levels).  Every call on one GPU shares that GPU's array, so
 * the library orders them: each call's stream first waits for a per-device
 * event (created once, with the array's address lookup, on the first call on
 * that device) that the previous call recorded after its kernels, so calls
 * from any streams and host threads run on the GPU one after another, in the
 * order the host issued them.  Calls enqueued under stream capture are not
 * chained (the graph orders its own nodes): replays of such graphs that
 * overlap with each other or with other calls on the same GPU race on the
 * array, and ordering them is the caller's job.  The stream's device must be
 * current (CTMR_E_INVALID otherwise).
 */
#define CTMR_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int ctmr_conv3d_noalloc(const ctmr_conv_desc* desc, const float* x, const void* packed, const float* bias,
                        const float* affine, const float* residual, float* y, void* stream);

/*
 * The two stages of ctmr_conv3d, callable separately with the same arguments
 * (ctmr_conv3d == ctmr_conv3d_pack then ctmr_conv3d_gemm on one stream).
 * _pack writes the zero-padded, transformed input copy (the reference's pack
 * kernel, _nax_conv.py:144-198) at the start of `workspace`; _gemm runs the
 * implicit GEMM (and split reduce) reading it (_nax_conv.py:200-332).  A
 * packed input may be reused by several _gemm calls with the same desc.
 * For a 1x1x1 fp32 conv with cin % 16 == 0 and no affine/SiLU nothing is
 * packed and _gemm reads x directly; for the LDS-staged GEMM _pack only keeps
 * the affine table in `workspace` and _gemm reads x directly.
 */
int ctmr_conv3d_pack(const ctmr_conv_desc* desc, const float* x, const float* affine,
                     void* workspace, size_t workspace_bytes, void* stream);
int ctmr_conv3d_gemm(const ctmr_conv_desc* desc, const float* x, const void* packed,
                     const float* bias, const float* residual, float* y, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * Group-norm statistics of a convolution's output, produced by its epilogue so a
 * following group norm needs no read pass (the reference computes them in a
 * separate medmlx-core pass, fast_fp32.py:185-189).  No counterpart entry point
 * exists in the reference; these replace group_norm_affine on a conv output.
 *   ctmr_conv3d_stats_tiles: the per-batch-item partial count ("tiles") that
 *     ctmr_conv3d_gn writes for `groups`, or 0 when this descriptor cannot
 *     produce them (cout <= 4, groups not dividing cout, a group that does not
 *     divide the GEMM's column tile; on a K split, cout not a multiple of 64 or
 *     a group wider than 64 channels); use ctmr_gn_affine on the output then.
 *     A tile is a GEMM output tile, or on a K split with partial planes a
 *     chunk of output voxels of the reduction.
 *   ctmr_conv3d_gn: ctmr_conv3d that also writes fp64 (sum, sum of squares) of
 *     the stored output per (batch item, tile, group), each summed in a fixed
 *     order, into stats[((b * tiles + tile) * groups + g) * 2 + {0, 1}].  The
 *     output is bit-identical to ctmr_conv3d's.
 *   ctmr_gn_affine_from_stats: the (n, c, 2) affine from those partials with the
 *     semantics of ctmr_gn_affine (count = output voxels * c / groups).
 */
int32_t ctmr_conv3d_stats_tiles(const ctmr_conv_desc* desc, int32_t groups);
int ctmr_conv3d_gn(const ctmr_conv_desc* desc, const float* x, const void* packed, const float* bias,
                   const float* affine, const float* residual, float* y, void* workspace,
                   size_t workspace_bytes, int32_t groups, double* stats, void* stream);
int ctmr_gn_affine_from_stats(int32_t n, int32_t tiles, int32_t c, int32_t groups, int64_t count, float eps,
                              const double* stats, const float* gamma, const float* beta, float* affine,
                              void* stream);
int ctmr_conv3d_cat_gn(const ctmr_conv_desc* desc, const float* x1, const float* x2, const void* packed,
                       const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                       size_t workspace_bytes, int32_t groups, double* stats, void* stream);

/* Group-norm statistics: affine (n, c, 2) = (gamma*rstd, beta - mean*gamma*rstd)
 * over (c/groups channels) x s voxels, biased variance, fp64 accumulation combined
 * in a fixed order.  Needs ctmr_gn_workspace_bytes(n, s, c) of scratch. */
int64_t ctmr_gn_workspace_bytes(int32_t n, int64_t s, int32_t c);
int ctmr_gn_affine(int32_t n, int64_t s, int32_t c, int32_t groups, float eps, const float* x,
                   const float* gamma, const float* beta, float* affine, void* workspace,
                   size_t workspace_bytes, void* stream);
/* ctmr_gn_affine of the channel concatenation of x1 (c1 channels) and x2 (c2
 * channels) on the same voxels, without materialising it (the norm1 of an
 * up-path residual block, whose input is that concatenation, unet.py:444);
 * c1 and c2 multiples of 4; workspace ctmr_gn_workspace_bytes(n, s, c1 + c2).
 * Bit-identical to ctmr_gn_affine on the concatenated tensor. */
int ctmr_gn_affine_cat(int32_t n, int64_t s, int32_t c1, int32_t c2, int32_t groups, float eps, const float* x1,
                       const float* x2, const float* gamma, const float* beta, float* affine, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * Group norm from statistics at a finer grouping than the norm's, over one tensor
 * or the channel concatenation of two (the up-path norm1 over cat([hidden, skip]),
 * unet.py:444, when both halves' producers wrote statistics; the reference reads
 * the concatenated tensor in a medmlx-core pass, fast_fp32.py:185-189).  No
 * counterpart entry point exists in the reference.
 *   ctmr_gn_affine_from_stats2: source k (k = 1, 2) holds partials
 *     stats_k[((b * tiles_k + tile) * sgroups_k + sg) * 2 + {0, 1}] over its c_k
 *     channels in sgroups_k equal stat groups (ctmr_conv3d_gn's layout; per channel
 *     when sgroups_k = c_k); source 2 is channels [c1, c1 + c2) of the normalised
 *     tensor (c2 = 0: one source, stats2 unused).  Every norm group's share of a
 *     source must be a union of its stat groups, else CTMR_E_INVALID.  count =
 *     voxels * (c1 + c2) / groups.  The items are summed in a fixed order (source
 *     1's tiles, then source 2's; stat groups ascending in each tile).
 *   ctmr_add_gn_partials: y = a + b (NDHWC fp32, c % 4 == 0, c <= 1024, 16-byte
 *     aligned; bit-identical to the fp32 sum) and per-channel partials of y into
 *     workspace, (n, tiles, c, 2) with tiles = workspace size of
 *     ctmr_gn_workspace_bytes(n, s, c) / (n * c * 16): a source for
 *     ctmr_gn_affine_from_stats2 with sgroups = c.  For the UNet skips to which
 *     ControlNet residuals are added (controlnet.py:160-163, unet.py:426-431).
 */
int ctmr_gn_affine_from_stats2(int32_t n, int32_t groups, int64_t count, float eps, const double* stats1,
                               int32_t tiles1, int32_t c1, int32_t sgroups1, const double* stats2, int32_t tiles2,
                               int32_t c2, int32_t sgroups2, const float* gamma, const float* beta, float* affine,
                               void* stream);
int ctmr_add_gn_partials(int32_t n, int64_t s, int32_t c, const float* a, const float* b, float* y,
                         void* workspace, size_t workspace_bytes, void* stream);

/* y = silu?(x*scale + offset) with affine from ctmr_gn_affine; y may equal x. */
int ctmr_gn_apply(int32_t n, int64_t s, int32_t c, const float* x, const float* affine,
                  int32_t silu, float* y, void* stream);

/* Down-sampling residual-block input (fast_fp32.residual_block_ncdhw's down
 * branch, fast_fp32.py:250-255: avg_pool3d of group_norm_ncdhw(x, silu) and
 * avg_pool3d of x) from one read of x: y = 2x2x2 average pool of
 * silu?(x*scale + offset) (affine from ctmr_gn_affine), y_skip (optional) =
 * the pool of x.  NDHWC, output (n, d/2, h/2, w/2, c); bit-identical to
 * ctmr_gn_apply followed by ctmr_resample(CTMR_AVGPOOL2), and to the pool of x. */
int ctmr_gn_avgpool(int32_t n, int32_t d, int32_t h, int32_t w, int32_t c, const float* x, const float* affine,
                    int32_t silu, float* y, float* y_skip, void* stream);

/* Elementwise SiLU, y may equal x. */
int ctmr_silu(int64_t count, const float* x, float* y, void* stream);

enum ctmr_resample_op {
  CTMR_AVGPOOL2 = 0,     /* (d,h,w) -> (d/2,h/2,w/2), mean of 2x2x2 */
  CTMR_NEAREST2X = 1,    /* (d,h,w) -> (2d,2h,2w) */
  CTMR_TRILINEAR2X = 2   /* (d,h,w) -> (2d,2h,2w), half-pixel, clamped */
};
int ctmr_resample(int32_t op, int32_t n, int32_t d, int32_t h, int32_t w, int32_t c,
                  const float* x, float* y, void* stream);

/* Multi-head softmax(Q K^T * scale) V in FP32 on head-interleaved projections,
 * without materialising the scores.  q is (n, lq, heads * head_dim) with row
 * stride ldq floats (batch stride lq * ldq); head h is columns
 * [h * head_dim, (h + 1) * head_dim).  k and v are (n, lk, ...) with row strides
 * ldk / ldv; out is (n, lq, heads * head_dim) with row stride ldo.  q, k and v
 * may be column slices of one fused (n, l, 3C) projection.  head_dim must be
 * 32 (the MAISI UNet's num_head_channels).  Any lq, lk >= 1.  query_tiles
 * picks 16 (1) or 32 (2) queries per wave, 0 = the library's policy; results
 * are bit-identical either way (keys are visited in the same fixed order:
 * ascending 32-key blocks, or -- for grids of under two waves per SIMD, decided
 * from n, lq, lk and heads only -- two such runs over the key halves, combined
 * first half first). */
typedef struct ctmr_attn_desc {
  int32_t n, lq, lk, heads, head_dim, query_tiles;
  int64_t ldq, ldk, ldv, ldo;
  float scale;
} ctmr_attn_desc;

int ctmr_flash_attention(const ctmr_attn_desc* desc, const float* q, const float* k, const float* v,
                         float* out, void* stream);

/* The same attention in the reference's split-fp16 arithmetic, its matrix-unit
 * kernel (_flash_attention.py:140-290, chosen at :336-350 when the device has
 * one): q * scale * log2(e), k and v are split into fp16 halves hi = fp16(x),
 * lo = fp16((x - hi) * 2^11) (_flash_attention.py:314-317) in the caller's
 * workspace, and each product runs as hi*hi + (hi*lo + lo*hi) * 2^-11 on fp16
 * MFMA with fp32 accumulation; P = 2^(S - m) is split the same way and the
 * cross terms of P V are summed apart and added at the end.  About 2^-22
 * relative per product; |q * scale * log2(e)|, |k| and |v| must stay below
 * 65504.  Same descriptor, checks, tilings and bit-identity across
 * query_tiles as ctmr_flash_attention.  workspace: at least
 * ctmr_flash_attention_f16x2_workspace_bytes(desc) bytes, 256-byte aligned
 * (-1 from that call for an invalid shape); calls sharing a workspace must not
 * overlap. */
int64_t ctmr_flash_attention_f16x2_workspace_bytes(const ctmr_attn_desc* desc);
int ctmr_flash_attention_f16x2(const ctmr_attn_desc* desc, const float* q, const float* k, const float* v,
                               float* out, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* CTMR_H */
