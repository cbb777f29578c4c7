// Group-norm statistics, group-norm apply (+SiLU), SiLU and the 2x resampling
// kernels for NDHWC fp32 activations on MI355X.
//
// Group norm (semantics of medmlx_core.group_norm_affine as used at
// src/mlx_generate_ctmr/fast_fp32.py:102-118,185-189 and restated in
// tests/test_fast_fp32.py:41-48): per (batch item, group) the mean and the
// biased variance over (C/G channels) x (all voxels); the output is per
// (batch item, channel) scale = gamma*rstd and offset = beta - mean*scale so a
// consumer computes x*scale + offset (fused into the conv input pack).
//
// Statistics are HBM-bound (4 bytes read per element).  Pass 1 splits the
// voxels of each batch item into chunks (the chunking depends on the shape
// only: about 64 KiB of input per chunk, at most ~2048 workgroups per launch);
// each 256-thread workgroup streams one chunk with coalesced 16-byte loads,
// every thread owning 4 channels, and accumulates
// sum and sum of squares in fp64.  The per-thread partials are combined in a
// fixed order (butterflies across each wave, then across the waves), so the
// result is bit-identical run to run and independent of the device.  Pass 2
// combines the chunk partials of one group, again in fixed order.
#include "ctmr_common.hpp"

#include <algorithm>

namespace ctmr {

// Statistics chunking, a function of (n, s, c) only: chunks of about 64 KiB
// of fp32 input, capped so one launch has at most ~2048 workgroups.
struct GnChunks {
  int64_t vox, count;
};
static inline GnChunks gn_chunks(int32_t n, int64_t s, int32_t c) {
  const int64_t target_vox = std::max<int64_t>(1, 16384 / c);
  const int64_t cap = std::max<int64_t>(1, 2048 / std::max<int32_t>(n, 1));
  const int64_t count = std::min<int64_t>(ceil_div(s, target_vox), cap);
  const int64_t vox = ceil_div(s, count);
  return {vox, ceil_div(s, vox)};
}

// Butterfly sum over the lanes l ^ m, m = 32, 16, .., LOW of a wave: every
// lane ends with the same sum, combined in the same fixed order.
template <int LOW>
__device__ __forceinline__ double wave_butterfly_sum(double v) {
#pragma unroll
  for (int m = 32; m >= LOW; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// VEC channels per thread: 4 (16-byte loads) when c % 4 == 0, else 1.
// Thread t owns channels [VEC (t % cgn), +VEC) of voxels vl, vl + V, vl + 2V,
// .. of the chunk (vl = t / cgn, V = 256 / cgn voxel lanes): each voxel row is
// read by consecutive threads, 16 bytes each (measured on MI355X: keeping four
// row loads in flight per thread is no faster, 5.1 against 5.4 TB/s over the
// 1 GiB config-1 input).  Each thread adds its rows in ascending order in fp64.
// The voxel lanes of one channel group are then combined in a fixed order:
// when cgn is a power of two below 64 the lanes of a wave holding that group
// are summed by a butterfly across the wave (lanes l ^ 32, l ^ 16, ..), then
// the four waves' sums in wave order; otherwise (one voxel lane per wave or
// cgn not a power of two) the voxel lanes in ascending order through LDS.
// A two-source input (x2 non-null) is the channel concatenation of x
// (channels [0, c1)) and x2 (channels [c1, c)); a thread's channels lie in one
// of them (c1 % VEC == 0) and it reads the same values in the same order as
// from the concatenated tensor.  With `addend` (single source, VEC 4) the
// statistics are those of x + addend, which the kernel also stores to y.
template <int VEC>
__global__ __launch_bounds__(256) void gn_partial_kernel(const float* __restrict__ x, const float* __restrict__ x2,
                                                         int c1, int64_t s, int c, int64_t chunk_vox, int chunks,
                                                         double* __restrict__ part,
                                                         const float* __restrict__ addend = nullptr,
                                                         float* __restrict__ y = nullptr) {
  const int chunk = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int cgn = c / VEC;
  const int vl_count = 256 / cgn;
  const int cg = t % cgn, vl = t / cgn;
  double acc[2 * VEC];  // sums, then sums of squares
#pragma unroll
  for (int k = 0; k < 2 * VEC; ++k) acc[k] = 0.0;
  const int64_t v0 = (int64_t)chunk * chunk_vox;
  const int64_t v1 = min(s, v0 + chunk_vox);
  auto add = [&](const float (&q)[VEC]) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const double d = (double)q[k];
      acc[k] += d;
      acc[VEC + k] = fma(d, d, acc[VEC + k]);
    }
  };
  auto load = [&](const float* row, float (&q)[VEC]) {
    if constexpr (VEC == 4) {
      const f4 w = *reinterpret_cast<const f4*>(row);
      q[0] = w[0]; q[1] = w[1]; q[2] = w[2]; q[3] = w[3];
    } else {
      q[0] = row[0];
    }
  };
  if (vl < vl_count) {
    const bool second = x2 != nullptr && cg * VEC >= c1;
    const int stride = x2 == nullptr ? c : (second ? c - c1 : c1);
    const float* xb = second ? x2 + (int64_t)b * s * stride + (cg * VEC - c1) : x + (int64_t)b * s * stride + cg * VEC;
    const int64_t step = vl_count;
    if (addend != nullptr) {
      const int64_t off = (int64_t)b * s * stride + cg * VEC;
      for (int64_t v = v0 + vl; v < v1; v += step) {
        float q[VEC], r[VEC];
        load(xb + v * stride, q);
        load(addend + off + v * stride, r);
#pragma unroll
        for (int k = 0; k < VEC; ++k) q[k] += r[k];
        if constexpr (VEC == 4) *reinterpret_cast<f4*>(y + off + v * stride) = f4{q[0], q[1], q[2], q[3]};
        add(q);
      }
    } else {
      for (int64_t v = v0 + vl; v < v1; v += step) {
        float q[VEC];
        load(xb + v * stride, q);
        add(q);
      }
    }
  }
  double* out = part + (((int64_t)b * chunks + chunk) * c) * 2;
  const bool butterfly = cgn < 64 && (cgn & (cgn - 1)) == 0;  // uniform: a kernel argument
  if (butterfly) {
    // Lane l holds channel group l % cgn; lanes l ^ m (m >= cgn) hold the
    // same group.
    __shared__ double wsum[4][32 * 2 * VEC];
    const int lane = t & 63, wave = t >> 6;
#pragma unroll
    for (int k = 0; k < 2 * VEC; ++k) {
      double v = acc[k];
      if (cgn <= 1) v = wave_butterfly_sum<1>(v);
      else if (cgn == 2) v = wave_butterfly_sum<2>(v);
      else if (cgn == 4) v = wave_butterfly_sum<4>(v);
      else if (cgn == 8) v = wave_butterfly_sum<8>(v);
      else if (cgn == 16) v = wave_butterfly_sum<16>(v);
      else v = wave_butterfly_sum<32>(v);
      acc[k] = v;
    }
    if (lane < cgn) {
#pragma unroll
      for (int k = 0; k < 2 * VEC; ++k) wsum[wave][lane * 2 * VEC + k] = acc[k];
    }
    __syncthreads();
    if (t < cgn) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const double sm = ((wsum[0][t * 2 * VEC + k] + wsum[1][t * 2 * VEC + k]) + wsum[2][t * 2 * VEC + k]) +
                          wsum[3][t * 2 * VEC + k];
        const double sq = ((wsum[0][t * 2 * VEC + VEC + k] + wsum[1][t * 2 * VEC + VEC + k]) +
                           wsum[2][t * 2 * VEC + VEC + k]) +
                          wsum[3][t * 2 * VEC + VEC + k];
        out[(t * VEC + k) * 2] = sm;
        out[(t * VEC + k) * 2 + 1] = sq;
      }
    }
    return;
  }
  __shared__ double red[256 * 2 * VEC];
#pragma unroll
  for (int k = 0; k < 2 * VEC; ++k) red[t * 2 * VEC + k] = acc[k];
  __syncthreads();
  if (t < cgn) {
    double a[2 * VEC];
#pragma unroll
    for (int k = 0; k < 2 * VEC; ++k) a[k] = 0.0;
    for (int j = 0; j < vl_count; ++j) {
      const double* r = red + (j * cgn + t) * 2 * VEC;
#pragma unroll
      for (int k = 0; k < 2 * VEC; ++k) a[k] += r[k];
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      out[(t * VEC + k) * 2] = a[k];
      out[(t * VEC + k) * 2 + 1] = a[VEC + k];
    }
  }
}

// Norm group of finalize workgroup `idx` of `groups` (grid x = groups, so the
// hardware deals workgroups idx, idx + 8, .. to one XCD): each XCD takes a
// contiguous run of groups, whose partials share 128-byte lines of the
// (tile, group) layout -- the lines are fetched by one or two XCDs' L2s
// instead of all eight.  The order inside a group is unchanged.
__device__ __forceinline__ int finalize_group(int idx, int groups) {
  if (groups % 8 != 0) return idx;
  return (idx % 8) * (groups / 8) + idx / 8;
}

// Thread t's sums of items t, t + 256, t + 512, .. (ascending, one running
// (sum, sum of squares) pair): pair(i) is item i's partial pair.  Sixteen
// items' loads are issued before their adds, so the loop waits for memory once
// per sixteen items instead of once per item; the order of the adds is
// unchanged.
template <typename Pair>
__device__ __forceinline__ void strided_pair_sums(int64_t items, Pair pair, double& sm, double& sq) {
  constexpr int kDepth = 16;
  int64_t i = threadIdx.x;
  for (; i + (kDepth - 1) * 256 < items; i += kDepth * 256) {
    double a[kDepth], q[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const double* p = pair(i + u * 256);
      a[u] = p[0];
      q[u] = p[1];
    }
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      sm += a[u];
      sq += q[u];
    }
  }
  for (; i < items; i += 256) {
    const double* p = pair(i);
    sm += p[0];
    sq += p[1];
  }
}

// Fixed-order combine of the 256 per-thread (sum, sum of squares) of group g of
// batch item b (a butterfly across each wave, then the four waves in order),
// then that group's (scale, offset) pairs.
__device__ void gn_group_affine(double sm, double sq, int g, int b, int c, int groups, int64_t count,
                                const float* __restrict__ gamma, const float* __restrict__ beta,
                                float eps, float* __restrict__ affine);

__global__ __launch_bounds__(256) void gn_finalize_kernel(const double* __restrict__ part,
                                                          int chunks, int c, int groups,
                                                          int64_t count,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta,
                                                          float eps, float* __restrict__ affine) {
  const int g = finalize_group(blockIdx.x, groups), b = blockIdx.y;
  const int cpg = c / groups;
  const int64_t items = (int64_t)chunks * cpg;
  double sm = 0, sq = 0;
  strided_pair_sums(items, [&](int64_t i) {
    const int chunk = (int)(i / cpg), cc = (int)(i % cpg);
    return part + (((int64_t)b * chunks + chunk) * c + g * cpg + cc) * 2;
  }, sm, sq);
  gn_group_affine(sm, sq, g, b, c, groups, count, gamma, beta, eps, affine);
}

// Affine from per-(batch item, tile, group) partials written by a conv
// epilogue (ctmr_conv3d_gn): tiles strided over the threads, then the same
// fixed-order combine.
__global__ __launch_bounds__(256) void gn_tiles_finalize_kernel(const double* __restrict__ part, int tiles,
                                                                int c, int groups, int64_t count,
                                                                const float* __restrict__ gamma,
                                                                const float* __restrict__ beta, float eps,
                                                                float* __restrict__ affine) {
  const int g = finalize_group(blockIdx.x, groups), b = blockIdx.y;
  double sm = 0, sq = 0;
  strided_pair_sums(tiles, [&](int64_t i) { return part + (((int64_t)b * tiles + i) * groups + g) * 2; }, sm, sq);
  gn_group_affine(sm, sq, g, b, c, groups, count, gamma, beta, eps, affine);
}

// Partials of one source of ctmr_gn_affine_from_stats2: (n, tiles, sgroups, 2)
// fp64 (sum, sum of squares) over its c channels, channels [c0, c0 + c) of the
// normalised (possibly concatenated) tensor.
struct StatSource {
  const double* stats;
  int tiles, c, sgroups, c0;
};

// Affine of norm group g of batch item b from the stat groups of one or two
// sources that tile its channels (checked on the host): the items (source,
// tile, stat group) strided over the threads in a fixed order -- source 1's
// tiles then source 2's, each tile's stat groups ascending -- then the fixed
// combine of gn_group_affine.
__global__ __launch_bounds__(256) void gn_stats_finalize_kernel(StatSource s1, StatSource s2, int c, int groups,
                                                                int64_t count, const float* __restrict__ gamma,
                                                                const float* __restrict__ beta, float eps,
                                                                float* __restrict__ affine) {
  const int g = finalize_group(blockIdx.x, groups), b = blockIdx.y;
  const int cpg = c / groups, lo = g * cpg, hi = lo + cpg;
  double sm = 0, sq = 0;
  const StatSource* src[2] = {&s1, &s2};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const StatSource& s = *src[k];
    if (s.c == 0) continue;
    const int a = max(lo, s.c0) - s.c0, e = min(hi, s.c0 + s.c) - s.c0;  // source-local channel range
    if (a >= e) continue;
    const int scpg = s.c / s.sgroups, g0 = a / scpg, ng = (e - a) / scpg;
    const int64_t items = (int64_t)s.tiles * ng;
    strided_pair_sums(items, [&](int64_t i) {
      const int tile = (int)(i / ng), sg = g0 + (int)(i % ng);
      return s.stats + (((int64_t)b * s.tiles + tile) * s.sgroups + sg) * 2;
    }, sm, sq);
  }
  gn_group_affine(sm, sq, g, b, c, groups, count, gamma, beta, eps, affine);
}

__device__ void gn_group_affine(double sm, double sq, int g, int b, int c, int groups, int64_t count,
                                const float* __restrict__ gamma, const float* __restrict__ beta,
                                float eps, float* __restrict__ affine) {
  const int t = threadIdx.x;
  const int cpg = c / groups;
  __shared__ double ws[4][2];
  __shared__ double stat[2];
  // Butterfly across each wave, then the four wave sums in wave order.
  sm = wave_butterfly_sum<1>(sm);
  sq = wave_butterfly_sum<1>(sq);
  if ((t & 63) == 0) {
    ws[t >> 6][0] = sm;
    ws[t >> 6][1] = sq;
  }
  __syncthreads();
  if (t == 0) {
    const double n = (double)count;
    const double mean = (((ws[0][0] + ws[1][0]) + ws[2][0]) + ws[3][0]) / n;
    double var = (((ws[0][1] + ws[1][1]) + ws[2][1]) + ws[3][1]) / n - mean * mean;
    if (var < 0) var = 0;
    stat[0] = mean;
    stat[1] = 1.0 / sqrt(var + (double)eps);
  }
  __syncthreads();
  for (int cc = t; cc < cpg; cc += 256) {
    const int ch = g * cpg + cc;
    const double scale = (double)gamma[ch] * stat[1];
    const double offset = (double)beta[ch] - stat[0] * scale;
    affine[((int64_t)b * c + ch) * 2] = (float)scale;
    affine[((int64_t)b * c + ch) * 2 + 1] = (float)offset;
  }
}

template <int VEC>
__global__ __launch_bounds__(256) void gn_apply_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ affine,
                                                       int64_t total, int64_t s, int c, int silu,
                                                       float* __restrict__ y) {
  const int cgn = c / VEC;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int ch = (int)(i % cgn) * VEC;
    const int64_t b = i / ((int64_t)cgn * s);
    const float* a = affine + (b * c + ch) * 2;
    if constexpr (VEC == 4) {
      f4 q = reinterpret_cast<const f4*>(x)[i];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float t = fmaf(q[k], a[2 * k], a[2 * k + 1]);
        q[k] = silu ? silu_f(t) : t;
      }
      reinterpret_cast<f4*>(y)[i] = q;
    } else {
      const float t = fmaf(x[i], a[0], a[1]);
      y[i] = silu ? silu_f(t) : t;
    }
  }
}

// Down-sampling residual block input (fast_fp32.py:250-255): the 2x2x2 average
// pool of silu?(x * scale + offset) and, optionally, of x itself, from one
// read of x.  Per output the same operations in the same order as gn_apply
// followed by the average pool (and the pool of x alone): bit-identical to
// them.
template <int VEC>
__global__ __launch_bounds__(256) void gn_avgpool_kernel(int n, int d, int h, int w, int c,
                                                         const float* __restrict__ x,
                                                         const float* __restrict__ affine, int silu,
                                                         float* __restrict__ y, float* __restrict__ y_skip) {
#pragma clang fp contract(off)
  const int od = d / 2, oh = h / 2, ow = w / 2;
  const int cg = c / VEC;
  const int64_t total = (int64_t)n * od * oh * ow * cg;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = i;
    const int cc = (int)(t % cg);
    t /= cg;
    const int xo = (int)(t % ow);
    t /= ow;
    const int yo = (int)(t % oh);
    t /= oh;
    const int zo = (int)(t % od);
    const int b = (int)(t / od);
    const float* src = x + (int64_t)b * d * h * w * c + cc * VEC;
    const float* a = affine + ((int64_t)b * c + cc * VEC) * 2;
    float sc[VEC], of[VEC], sg[VEC], sx[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      sc[k] = a[2 * k];
      of[k] = a[2 * k + 1];
      sg[k] = 0.f;
      sx[k] = 0.f;
    }
    for (int p = 0; p < 2; ++p)
      for (int q = 0; q < 2; ++q)
        for (int e = 0; e < 2; ++e) {
          const float* v = src + (((int64_t)(2 * zo + p) * h + (2 * yo + q)) * w + (2 * xo + e)) * c;
          float u[VEC];
          if constexpr (VEC == 4) {
            const f4 w4 = *reinterpret_cast<const f4*>(v);
            u[0] = w4[0]; u[1] = w4[1]; u[2] = w4[2]; u[3] = w4[3];
          } else {
            u[0] = v[0];
          }
#pragma unroll
          for (int k = 0; k < VEC; ++k) {
            const float g = fmaf(u[k], sc[k], of[k]);
            sg[k] += silu ? silu_f(g) : g;
            sx[k] += u[k];
          }
        }
    const int64_t obase = ((((int64_t)b * od + zo) * oh + yo) * ow + xo) * c + cc * VEC;
    if constexpr (VEC == 4) {
      *reinterpret_cast<f4*>(y + obase) = f4{sg[0], sg[1], sg[2], sg[3]} * 0.125f;
      if (y_skip) *reinterpret_cast<f4*>(y_skip + obase) = f4{sx[0], sx[1], sx[2], sx[3]} * 0.125f;
    } else {
      y[obase] = sg[0] * 0.125f;
      if (y_skip) y_skip[obase] = sx[0] * 0.125f;
    }
  }
}

__global__ __launch_bounds__(256) void silu_kernel(const float* __restrict__ x, int64_t count,
                                                   float* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = silu_f(x[i]);
}

// One thread per output (voxel, 4 channels) when c % 4 == 0, else per channel.
__global__ __launch_bounds__(256) void resample_kernel(int op, int n, int d, int h, int w, int c,
                                                       int vec, const float* __restrict__ x,
                                                       float* __restrict__ y) {
#pragma clang fp contract(off)
  const int od = op == CTMR_AVGPOOL2 ? d / 2 : 2 * d;
  const int oh = op == CTMR_AVGPOOL2 ? h / 2 : 2 * h;
  const int ow = op == CTMR_AVGPOOL2 ? w / 2 : 2 * w;
  const int cg = vec ? c / 4 : c;
  const int64_t total = (int64_t)n * od * oh * ow * cg;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
  int64_t t = i;
  const int cc = (int)(t % cg);
  t /= cg;
  const int xo = (int)(t % ow);
  t /= ow;
  const int yo = (int)(t % oh);
  t /= oh;
  const int zo = (int)(t % od);
  const int b = (int)(t / od);
  const float* src = x + (int64_t)b * d * h * w * c;
  auto at4 = [&](int zz, int yy, int xx) -> f4 {
    return *reinterpret_cast<const f4*>(src + (((int64_t)zz * h + yy) * w + xx) * c + cc * 4);
  };
  auto at1 = [&](int zz, int yy, int xx) -> float {
    return src[(((int64_t)zz * h + yy) * w + xx) * c + cc];
  };
  const int64_t obase = ((((int64_t)b * od + zo) * oh + yo) * ow + xo) * c;
  if (op == CTMR_AVGPOOL2) {
    if (vec) {
      f4 s = {0.f, 0.f, 0.f, 0.f};
      for (int a = 0; a < 2; ++a)
        for (int bb = 0; bb < 2; ++bb)
          for (int e = 0; e < 2; ++e) s += at4(2 * zo + a, 2 * yo + bb, 2 * xo + e);
      *reinterpret_cast<f4*>(y + obase + cc * 4) = s * 0.125f;
    } else {
      float s = 0.f;
      for (int a = 0; a < 2; ++a)
        for (int bb = 0; bb < 2; ++bb)
          for (int e = 0; e < 2; ++e) s += at1(2 * zo + a, 2 * yo + bb, 2 * xo + e);
      y[obase + cc] = s * 0.125f;
    }
  } else if (op == CTMR_NEAREST2X) {
    if (vec)
      *reinterpret_cast<f4*>(y + obase + cc * 4) = at4(zo >> 1, yo >> 1, xo >> 1);
    else
      y[obase + cc] = at1(zo >> 1, yo >> 1, xo >> 1);
  } else {
    if (vec)
      *reinterpret_cast<f4*>(y + obase + cc * 4) = trilinear_sample4(src, d, h, w, c, cc * 4, zo, yo, xo);
    else
      y[obase + cc] = trilinear_sample1(src, d, h, w, c, cc, zo, yo, xo);
  }
  }
}

}  // namespace ctmr

using namespace ctmr;

extern "C" {

int64_t ctmr_gn_workspace_bytes(int32_t n, int64_t s, int32_t c) {
  if (n <= 0 || s <= 0 || c <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  return (int64_t)n * gn_chunks(n, s, c).count * c * 2 * (int64_t)sizeof(double);
}

// ctmr_gn_affine and ctmr_gn_affine_cat: x2 null for one source.
static int gn_affine_run(int32_t n, int64_t s, int32_t c, int32_t c1, int32_t groups, float eps, const float* x,
                         const float* x2, const float* gamma, const float* beta, float* affine, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (n <= 0 || s <= 0 || c <= 0 || groups <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (c % groups != 0) return fail(CTMR_E_INVALID, "channels must be divisible by groups");
  const bool vec = (c % 4 == 0);
  if ((vec && c > 1024) || (!vec && c > 256))
    return fail(CTMR_E_UNSUPPORTED, "group norm needs c <= 1024 (c % 4 == 0) or c <= 256");
  if (!x || !gamma || !beta || !affine || (c1 != c && !x2)) return fail(CTMR_E_INVALID, "null pointer");
  if (c1 != c && (!vec || c1 <= 0 || c1 >= c || c1 % 4 != 0))
    return fail(CTMR_E_INVALID, "two-source group norm needs 0 < c1 < c, both multiples of 4");
  if (vec && (((uintptr_t)x | (c1 != c ? (uintptr_t)x2 : 0)) & 15) != 0)
    return fail(CTMR_E_INVALID, "x must be 16-byte aligned");
  const GnChunks ch = gn_chunks(n, s, c);
  const int64_t chunk_vox = ch.vox, chunks = ch.count;
  const int64_t need = (int64_t)n * chunks * c * 2 * (int64_t)sizeof(double);
  if ((int64_t)workspace_bytes < need || !workspace) {
    set_error("group-norm workspace %zu bytes < required %lld", workspace_bytes, (long long)need);
    return CTMR_E_WORKSPACE;
  }
  if (chunks >= (1 << 30) || n > 65535) return fail(CTMR_E_UNSUPPORTED, "volume too large");
  hipStream_t st = (hipStream_t)stream;
  double* part = (double*)workspace;
  const float* second = c1 != c ? x2 : nullptr;
  if (vec)
    hipLaunchKernelGGL(gn_partial_kernel<4>, dim3((unsigned)chunks, n), dim3(256), 0, st, x, second, c1, s, c,
                       chunk_vox, (int)chunks, part);
  else
    hipLaunchKernelGGL(gn_partial_kernel<1>, dim3((unsigned)chunks, n), dim3(256), 0, st, x, second, c1, s, c,
                       chunk_vox, (int)chunks, part);
  int rc = check_launch("gn_partial");
  if (rc) return rc;
  hipLaunchKernelGGL(gn_finalize_kernel, dim3(groups, n), dim3(256), 0, st, part, (int)chunks, c,
                     groups, s * (c / groups), gamma, beta, eps, affine);
  return check_launch("gn_finalize");
}

int ctmr_gn_affine(int32_t n, int64_t s, int32_t c, int32_t groups, float eps, const float* x,
                   const float* gamma, const float* beta, float* affine, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return gn_affine_run(n, s, c, c, groups, eps, x, nullptr, gamma, beta, affine, workspace, workspace_bytes,
                       stream);
}

int ctmr_gn_affine_cat(int32_t n, int64_t s, int32_t c1, int32_t c2, int32_t groups, float eps, const float* x1,
                       const float* x2, const float* gamma, const float* beta, float* affine, void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (c1 <= 0 || c2 <= 0) return fail(CTMR_E_INVALID, "two-source group norm needs c1 > 0 and c2 > 0");
  return gn_affine_run(n, s, c1 + c2, c1, groups, eps, x1, x2, gamma, beta, affine, workspace, workspace_bytes,
                       stream);
}

int ctmr_gn_affine_from_stats(int32_t n, int32_t tiles, int32_t c, int32_t groups, int64_t count, float eps,
                              const double* stats, const float* gamma, const float* beta, float* affine,
                              void* stream) {
  if (n <= 0 || tiles <= 0 || c <= 0 || groups <= 0 || count <= 0)
    return fail(CTMR_E_INVALID, "non-positive dimension");
  if (c % groups != 0) return fail(CTMR_E_INVALID, "channels must be divisible by groups");
  if (n > 65535 || groups > 65535) return fail(CTMR_E_UNSUPPORTED, "too many batch items or groups");
  if (!stats || !gamma || !beta || !affine) return fail(CTMR_E_INVALID, "null pointer");
  hipLaunchKernelGGL(gn_tiles_finalize_kernel, dim3(groups, n), dim3(256), 0, (hipStream_t)stream, stats, tiles,
                     c, groups, count, gamma, beta, eps, affine);
  return check_launch("gn_tiles_finalize");
}

int ctmr_add_gn_partials(int32_t n, int64_t s, int32_t c, const float* a, const float* b, float* y,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (n <= 0 || s <= 0 || c <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (c % 4 != 0 || c > 1024) return fail(CTMR_E_UNSUPPORTED, "add with statistics needs c % 4 == 0 and c <= 1024");
  if (!a || !b || !y) return fail(CTMR_E_INVALID, "null pointer");
  if ((((uintptr_t)a | (uintptr_t)b | (uintptr_t)y) & 15) != 0)
    return fail(CTMR_E_INVALID, "a, b and y must be 16-byte aligned");
  const GnChunks ch = gn_chunks(n, s, c);
  const int64_t need = (int64_t)n * ch.count * c * 2 * (int64_t)sizeof(double);
  if ((int64_t)workspace_bytes < need || !workspace) {
    set_error("statistics workspace %zu bytes < required %lld", workspace_bytes, (long long)need);
    return CTMR_E_WORKSPACE;
  }
  if (ch.count >= (1 << 30) || n > 65535) return fail(CTMR_E_UNSUPPORTED, "volume too large");
  hipLaunchKernelGGL(gn_partial_kernel<4>, dim3((unsigned)ch.count, n), dim3(256), 0, (hipStream_t)stream, a,
                     nullptr, c, s, c, ch.vox, (int)ch.count, (double*)workspace, b, y);
  return check_launch("add_gn_partials");
}

// Whether the stat groups of a source tile every norm group's share of it.
static bool stats_tile_groups(int c0, int c, int sgroups, int ctot, int groups) {
  if (c == 0) return true;
  if (sgroups <= 0 || c % sgroups != 0) return false;
  const int scpg = c / sgroups, cpg = ctot / groups;
  for (int g = 0; g < groups; ++g) {
    const int a = std::max(g * cpg, c0) - c0, e = std::min((g + 1) * cpg, c0 + c) - c0;
    if (a < e && (a % scpg != 0 || e % scpg != 0)) return false;
  }
  return true;
}

int ctmr_gn_affine_from_stats2(int32_t n, int32_t groups, int64_t count, float eps, const double* stats1,
                               int32_t tiles1, int32_t c1, int32_t sgroups1, const double* stats2, int32_t tiles2,
                               int32_t c2, int32_t sgroups2, const float* gamma, const float* beta, float* affine,
                               void* stream) {
  if (n <= 0 || groups <= 0 || count <= 0 || c1 <= 0 || tiles1 <= 0 || c2 < 0 || (c2 > 0 && tiles2 <= 0))
    return fail(CTMR_E_INVALID, "non-positive dimension");
  const int c = c1 + c2;
  if (c % groups != 0) return fail(CTMR_E_INVALID, "channels must be divisible by groups");
  if (n > 65535 || groups > 65535) return fail(CTMR_E_UNSUPPORTED, "too many batch items or groups");
  if (!stats_tile_groups(0, c1, sgroups1, c, groups) || !stats_tile_groups(c1, c2, sgroups2, c, groups))
    return fail(CTMR_E_INVALID, "the sources' statistic groups do not tile the norm's groups");
  if (!stats1 || (c2 > 0 && !stats2) || !gamma || !beta || !affine) return fail(CTMR_E_INVALID, "null pointer");
  const StatSource s1{stats1, tiles1, c1, sgroups1, 0};
  const StatSource s2{c2 > 0 ? stats2 : nullptr, c2 > 0 ? tiles2 : 0, c2, c2 > 0 ? sgroups2 : 1, c1};
  hipLaunchKernelGGL(gn_stats_finalize_kernel, dim3(groups, n), dim3(256), 0, (hipStream_t)stream, s1, s2, c, groups,
                     count, gamma, beta, eps, affine);
  return check_launch("gn_stats_finalize");
}

int ctmr_gn_apply(int32_t n, int64_t s, int32_t c, const float* x, const float* affine,
                  int32_t silu, float* y, void* stream) {
  if (n <= 0 || s <= 0 || c <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (!x || !affine || !y) return fail(CTMR_E_INVALID, "null pointer");
  const bool vec = (c % 4 == 0) && ((((uintptr_t)x | (uintptr_t)y) & 15) == 0);
  const int64_t total = (int64_t)n * s * (vec ? c / 4 : c);
  if (vec)
    hipLaunchKernelGGL(gn_apply_kernel<4>, dim3(elementwise_blocks(total)), dim3(256), 0,
                       (hipStream_t)stream, x, affine, total, s, c, silu, y);
  else
    hipLaunchKernelGGL(gn_apply_kernel<1>, dim3(elementwise_blocks(total)), dim3(256), 0,
                       (hipStream_t)stream, x, affine, total, s, c, silu, y);
  return check_launch("gn_apply");
}

int ctmr_silu(int64_t count, const float* x, float* y, void* stream) {
  if (count < 0 || (count > 0 && (!x || !y))) return fail(CTMR_E_INVALID, "bad arguments");
  if (count == 0) return CTMR_OK;
  hipLaunchKernelGGL(silu_kernel, dim3(elementwise_blocks(count)), dim3(256), 0,
                     (hipStream_t)stream, x, count, y);
  return check_launch("silu");
}

int ctmr_gn_avgpool(int32_t n, int32_t d, int32_t h, int32_t w, int32_t c, const float* x, const float* affine,
                    int32_t silu, float* y, float* y_skip, void* stream) {
  if (n <= 0 || d <= 0 || h <= 0 || w <= 0 || c <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (d < 2 || h < 2 || w < 2) return fail(CTMR_E_INVALID, "average pooling needs every axis >= 2");
  if (!x || !affine || !y) return fail(CTMR_E_INVALID, "null pointer");
  const uintptr_t ptrs = (uintptr_t)x | (uintptr_t)y | (y_skip ? (uintptr_t)y_skip : 0);
  const int vec = (c % 4 == 0) && ((ptrs & 15) == 0);
  const int64_t total = (int64_t)n * (d / 2) * (h / 2) * (w / 2) * (vec ? c / 4 : c);
  if (vec)
    hipLaunchKernelGGL(gn_avgpool_kernel<4>, dim3(elementwise_blocks(total)), dim3(256), 0, (hipStream_t)stream,
                       n, d, h, w, c, x, affine, silu, y, y_skip);
  else
    hipLaunchKernelGGL(gn_avgpool_kernel<1>, dim3(elementwise_blocks(total)), dim3(256), 0, (hipStream_t)stream,
                       n, d, h, w, c, x, affine, silu, y, y_skip);
  return check_launch("gn_avgpool");
}

int ctmr_resample(int32_t op, int32_t n, int32_t d, int32_t h, int32_t w, int32_t c,
                  const float* x, float* y, void* stream) {
  if (op < CTMR_AVGPOOL2 || op > CTMR_TRILINEAR2X) return fail(CTMR_E_INVALID, "bad resample op");
  if (n <= 0 || d <= 0 || h <= 0 || w <= 0 || c <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (op == CTMR_AVGPOOL2 && (d < 2 || h < 2 || w < 2))
    return fail(CTMR_E_INVALID, "average pooling needs every axis >= 2");
  if (!x || !y) return fail(CTMR_E_INVALID, "null pointer");
  const int vec = (c % 4 == 0) && ((((uintptr_t)x | (uintptr_t)y) & 15) == 0);
  const int64_t od = op == CTMR_AVGPOOL2 ? d / 2 : 2 * (int64_t)d;
  const int64_t oh = op == CTMR_AVGPOOL2 ? h / 2 : 2 * (int64_t)h;
  const int64_t ow = op == CTMR_AVGPOOL2 ? w / 2 : 2 * (int64_t)w;
  const int64_t total = (int64_t)n * od * oh * ow * (vec ? c / 4 : c);
  hipLaunchKernelGGL(resample_kernel, dim3(elementwise_blocks(total)), dim3(256), 0,
                     (hipStream_t)stream, op, n, d, h, w, c, vec, x, y);
  return check_launch("resample");
}

}  // extern "C"
