// Implicit-GEMM 3x3x3 / 1x1x1 convolution for MI355X (gfx950) on NDHWC fp32
// activations, with FP32 MFMA (v_mfma_f32_16x16x4_f32) or bf16-in /
// fp32-accumulate MFMA (v_mfma_f32_16x16x32_bf16).
//
// Dataflow (reference: src/mlx_generate_ctmr/_nax_conv.py:1-35, 475-684):
//   1. pack_input: x (NDHWC) -> zero-padded NDHWC copy with channels rounded up
//      to the MFMA K block, applying group-norm affine + SiLU (fast_fp32.py:
//      162-211) or the trilinear-2x sample (_nax_conv.py:115-142) on the way,
//      in fp32 or rounded once to bf16.  Padding voxels are zero after the
//      transform, as in the reference pack (_nax_conv.py:185-197).
//   2. conv_kernel: GEMM rows are output voxels, columns output channels, K is
//      taps x input channels.  Tap (kd,kh,kw) of the window starting at padded
//      row r reads row r + kd*P + kh*Q + kw (P, Q = padded plane / row pitch),
//      so no im2col buffer exists.  K order per output is fixed: taps
//      kd*9+kh*3+kw ascending, then 64-byte channel blocks ascending.  Bias,
//      per-batch bias and residual join the fp32 sum before the single store
//      (_nax_conv.py:282-317).
//   3. split_reduce: when the grid is small the K steps are split into
//      contiguous ranges whose fp32 partial planes are added in ascending
//      order with bias and residual (_nax_conv.py:320-332).
//
// Wave tile: 64 output voxels (4 MFMA row blocks of 16) x NSUB*16 channels;
// a 256-thread workgroup holds WM x WN waves.  Each lane loads 16 bytes per
// fragment: for fp32, channels 4g..4g+3 of a 16-channel block (g = lane/16),
// consumed by four 16x16x4 MFMAs; for bf16, channels 8g..8g+7 of a 32-channel
// block, consumed by one 16x16x32 MFMA.  The packed weight stores each
// (block, output channel) pair as 64 contiguous bytes in the same order, so A
// and B lanes always pair the same input channel.
#include "ctmr_common.hpp"

#include <algorithm>
#include <cstdarg>
#include <type_traits>

namespace ctmr {

static thread_local char g_error[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// 1. Input packing
// ---------------------------------------------------------------------------
struct PackArgs {
  const float* x;       // source (channels [0, c1) of a two-source input)
  const float* x2;      // channels [c1, c) of a two-source input, or null
  int c1;               // channels of x (c for one source; a multiple of 4)
  void* out;
  const float* affine;
  int64_t total4;       // 4-channel groups to write
  int gd, gh, gw;       // interior grid of the packed copy
  int halo;             // 1 for 3x3x3, 0 for 1x1x1
  int c, cp;            // source / packed channels
  int id, ih, iw;       // source grid (trilinear)
  int affine_on, silu_on, trilinear, bf16;
  int split16;          // split-fp16 copy (CTMR_F16X2): per 16-channel block [hi 0..15 | lo 0..15]
  int n;                // batch items
};

// Packed-copy formats: fp32, bf16, or split fp16 (CTMR_F16X2), whose 16-channel
// blocks hold the hi halves of channels 0..15 and then their lo halves (64
// bytes, the size of the fp32 copy's block).
enum { PF_F32 = 0, PF_BF16 = 1, PF_SPLIT = 2 };

// Byte offset of channel ch (a multiple of 4) of packed voxel `vox` in the
// split-fp16 copy of cp channels: its hi half; the lo half lies 32 bytes on.
__device__ __forceinline__ int64_t split_offset(int64_t vox, int cp, int ch) {
  return vox * cp * 4 + (ch >> 4) * 64 + (ch & 15) * 2;
}

// Split-fp16 store of 4 channels (8-byte halves) and of 8 (16-byte halves,
// ch % 8 == 0) at a split_offset.
__device__ __forceinline__ void store_split4(void* out, int64_t off, f4 v) {
  h4 hi, lo;
  split_f16x4(v, hi, lo);
  char* p = reinterpret_cast<char*>(out) + off;
  *reinterpret_cast<h4*>(p) = hi;
  *reinterpret_cast<h4*>(p + 32) = lo;
}
__device__ __forceinline__ void store_split8(void* out, int64_t off, f4 v0, f4 v1) {
  h4 hi0, lo0, hi1, lo1;
  split_f16x4(v0, hi0, lo0);
  split_f16x4(v1, hi1, lo1);
  char* p = reinterpret_cast<char*>(out) + off;
  *reinterpret_cast<h8*>(p) = h8{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
  *reinterpret_cast<h8*>(p + 32) = h8{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
}

// The packed value of channels ch..ch+3 at padded voxel (pz, py, px) of batch
// item b: zero in the halo and past the source channels, else the source (or
// its trilinear-2x sample) with the optional GN affine and SiLU.
__device__ __forceinline__ f4 pack_value4(const PackArgs& a, int b, int pz, int py, int px, int ch) {
  const int z = pz - a.halo, y = py - a.halo, x = px - a.halo;
  f4 v = {0.f, 0.f, 0.f, 0.f};
  if (z >= 0 && z < a.gd && y >= 0 && y < a.gh && x >= 0 && x < a.gw && ch < a.c) {
    if ((a.c & 3) == 0) {
      if (a.trilinear) {
        const float* src = a.x + (int64_t)b * a.id * a.ih * a.iw * a.c;
        v = trilinear_sample4(src, a.id, a.ih, a.iw, a.c, ch, z, y, x);
      } else {
        const int64_t vox = (((int64_t)b * a.gd + z) * a.gh + y) * a.gw + x;
        v = ch < a.c1 ? *reinterpret_cast<const f4*>(a.x + vox * a.c1 + ch)
                      : *reinterpret_cast<const f4*>(a.x2 + vox * (a.c - a.c1) + (ch - a.c1));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (ch + k < a.c) {
          if (a.trilinear) {
            const float* src = a.x + (int64_t)b * a.id * a.ih * a.iw * a.c;
            v[k] = trilinear_sample1(src, a.id, a.ih, a.iw, a.c, ch + k, z, y, x);
          } else {
            v[k] = a.x[((((int64_t)b * a.gd + z) * a.gh + y) * a.gw + x) * a.c + ch + k];
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (ch + k < a.c) {
        float t = v[k];
        if (a.affine_on) {
          const float* p = a.affine + ((int64_t)b * a.c + ch + k) * 2;
          t = fmaf(t, p[0], p[1]);
        }
        if (a.silu_on) t = silu_f(t);
        v[k] = t;
      }
    }
  }
  return v;
}

// Grid: blockIdx.y walks the (batch item, padded plane) pairs, blockIdx.x
// and the thread the plane's (row, column, channel group) items, so the index
// arithmetic is 32-bit (the host checks a plane holds < 2^31 items).  A
// thread packs 4 channels (fp32: one 16-byte store) or 8 (bf16: one 16-byte
// store of 8 rounded values; the bf16 copy's cp is a multiple of 32), or 8
// (split fp16: 16-byte hi and lo stores; cp a multiple of 16).
__global__ __launch_bounds__(256) void pack_input_kernel(PackArgs a) {
  const int G = (a.bf16 || a.split16) ? 2 : 1;
  const int cgn = (a.cp >> 2) / G;
  const int PW = a.gw + 2 * a.halo, PH = a.gh + 2 * a.halo, PD = a.gd + 2 * a.halo;
  const unsigned plane = (unsigned)PH * (unsigned)PW * (unsigned)cgn;
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= plane) return;
  const int cg = (int)(i % (unsigned)cgn);
  const unsigned r = i / (unsigned)cgn;
  const int px = (int)(r % (unsigned)PW), py = (int)(r / (unsigned)PW);
  for (int bz = blockIdx.y; bz < a.n * PD; bz += gridDim.y) {
    const int b = bz / PD, pz = bz - b * PD;
    const int64_t idx = (int64_t)bz * plane + i;
    if (a.split16) {
      const f4 v0 = pack_value4(a, b, pz, py, px, cg * 8), v1 = pack_value4(a, b, pz, py, px, cg * 8 + 4);
      store_split8(a.out, split_offset((idx - cg) / cgn, a.cp, cg * 8), v0, v1);
    } else if (a.bf16) {
      const f4 v0 = pack_value4(a, b, pz, py, px, cg * 8), v1 = pack_value4(a, b, pz, py, px, cg * 8 + 4);
      u4 packed;
      packed.x = (unsigned)f32_to_bf16_bits(v0[0]) | ((unsigned)f32_to_bf16_bits(v0[1]) << 16);
      packed.y = (unsigned)f32_to_bf16_bits(v0[2]) | ((unsigned)f32_to_bf16_bits(v0[3]) << 16);
      packed.z = (unsigned)f32_to_bf16_bits(v1[0]) | ((unsigned)f32_to_bf16_bits(v1[1]) << 16);
      packed.w = (unsigned)f32_to_bf16_bits(v1[2]) | ((unsigned)f32_to_bf16_bits(v1[3]) << 16);
      reinterpret_cast<u4*>(a.out)[idx] = packed;
    } else {
      reinterpret_cast<f4*>(a.out)[idx] = pack_value4(a, b, pz, py, px, cg * 4);
    }
  }
}

// GN affine (scale, offset) pairs of channels ch..ch+3 of batch item b: two
// 16-byte loads (the host checks the table's 16-byte alignment).
__device__ __forceinline__ void load_affine4(const PackArgs& a, int b, int ch, f4& s, f4& o) {
  const f4* p = reinterpret_cast<const f4*>(a.affine + ((int64_t)b * a.c + ch) * 2);
  const f4 p0 = p[0], p1 = p[1];
  s = f4{p0[0], p0[2], p1[0], p1[2]};
  o = f4{p0[1], p0[3], p1[1], p1[3]};
}

// The pack transform of one interior vector: affine, then SiLU (the order and
// operations of pack_value4).
__device__ __forceinline__ f4 pack_transform4(const PackArgs& a, f4 v, f4 s, f4 o) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float t = v[k];
    if (a.affine_on) t = fmaf(t, s[k], o[k]);
    if (a.silu_on) t = silu_f(t);
    v[k] = t;
  }
  return v;
}

__device__ __forceinline__ unsigned bf16_pair(float lo, float hi) {
  return (unsigned)f32_to_bf16_bits(lo) | ((unsigned)f32_to_bf16_bits(hi) << 16);
}

// Store one packed item: V vectors of 4 channels, as V f4 (fp32), one
// 16-byte store of 8 rounded values (bf16, V = 2), or 16-byte hi and lo
// stores of channel group cg's 8 values (split fp16, V = 2: a voxel's cp / 8
// groups occupy cp * 4 = 32 * (cp / 8) bytes).
template <int V, bool SPLIT = false>
__device__ __forceinline__ void store_packed(const PackArgs& a, int64_t idx, int cg, const f4* v) {
  if constexpr (SPLIT) {
    static_assert(V == 2, "split-fp16 packing stores 8 channels per item");
    store_split8(a.out, (idx - cg) * 32 + (cg >> 1) * 64 + (cg & 1) * 16, v[0], v[1]);
  } else if constexpr (V == 2) {
    u4 packed;
    packed.x = bf16_pair(v[0][0], v[0][1]);
    packed.y = bf16_pair(v[0][2], v[0][3]);
    packed.z = bf16_pair(v[1][0], v[1][1]);
    packed.w = bf16_pair(v[1][2], v[1][3]);
    reinterpret_cast<u4*>(a.out)[idx] = packed;
  } else {
    reinterpret_cast<f4*>(a.out)[idx] = v[0];
  }
}

// Non-resampled pack for c % 4 == 0 (the common case): same values as
// pack_input_kernel.  A thread takes one (row, column, channel group) item of
// the padded plane over PZ consecutive padded planes and issues all their
// source loads before its first store (PZ times the bytes in flight per wave
// of a one-item thread); the group's affine pairs are read once per batch item
// as 16-byte vectors.
template <int V, int PZ, bool SPLIT = false>
__global__ __launch_bounds__(256) void pack_planes_kernel(PackArgs a) {
  const int cgn = a.cp / (4 * V);
  const int PW = a.gw + 2 * a.halo, PH = a.gh + 2 * a.halo, PD = a.gd + 2 * a.halo;
  const unsigned plane = (unsigned)PH * (unsigned)PW * (unsigned)cgn;
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= plane) return;
  const int cg = (int)(i % (unsigned)cgn);
  const unsigned r = i / (unsigned)cgn;
  const int x = (int)(r % (unsigned)PW) - a.halo, y = (int)(r / (unsigned)PW) - a.halo;
  const bool row_in = x >= 0 && x < a.gw && y >= 0 && y < a.gh;
  const int total = a.n * PD;
  for (int bz0 = blockIdx.y * PZ; bz0 < total; bz0 += gridDim.y * PZ) {
    f4 v[PZ][V];
    bool in[PZ];
#pragma unroll
    for (int s = 0; s < PZ; ++s) {
      const int bz = bz0 + s;
      const int b = bz / PD, z = bz - b * PD - a.halo;
      in[s] = bz < total && row_in && z >= 0 && z < a.gd;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const int ch = cg * 4 * V + 4 * k;
        v[s][k] = f4{0.f, 0.f, 0.f, 0.f};
        if (in[s] && ch < a.c) {
          const int64_t vox = (((int64_t)b * a.gd + z) * a.gh + y) * a.gw + x;
          v[s][k] = ch < a.c1 ? *reinterpret_cast<const f4*>(a.x + vox * a.c1 + ch)
                              : *reinterpret_cast<const f4*>(a.x2 + vox * (a.c - a.c1) + (ch - a.c1));
        }
      }
    }
    int cur_b = -1;
    f4 sc[V], of[V];
#pragma unroll
    for (int k = 0; k < V; ++k) sc[k] = of[k] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < PZ; ++s) {
      const int bz = bz0 + s;
      if (bz >= total) break;
      const int b = bz / PD;
      if (a.affine_on && b != cur_b) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
          const int ch = cg * 4 * V + 4 * k;
          if (ch < a.c) load_affine4(a, b, ch, sc[k], of[k]);
        }
        cur_b = b;
      }
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (in[s] && cg * 4 * V + 4 * k < a.c) v[s][k] = pack_transform4(a, v[s][k], sc[k], of[k]);
      store_packed<V, SPLIT>(a, (int64_t)bz * plane + i, cg, v[s]);
    }
  }
}

// Trilinear-2x pack for c % 4 == 0 (one source tensor): same values as
// pack_input_kernel.  A thread takes one 4-channel group of one source cell
// column (cy, cx) and marches ZC cells cz along z; cells run over [-1, n] on
// each axis, and cell (cz, cy, cx) owns the padded copy's 2x2x2 block of
// 2x-grid voxels (2cz + dz, 2cy + dy, 2cx + dx): voxels at -1 and 2n are the
// zero halo, -2 and 2n + 1 lie past the copy.  A column's voxels have fixed
// x and y source pairs (tri_axis), so the thread keeps three x-then-y-
// interpolated source planes (clamped planes cz - 1, cz, cz + 1) and computes
// one new plane per cell: 9 loads where cy and cx lie in [1, n - 2] (the four
// voxel columns share the 3x3 source rows), 16 at the faces, against 8 per
// voxel.  Each voxel is then the z blend of two of those planes with
// tri_axis's weights: the expression trilinear_sample4 evaluates, with the
// same operands (a plane repeated by the clamp holds the same bits in either
// slot), so the two agree bitwise.
struct TriPlane {
  f4 p[2][2];  // [dy][dx]
};

// Column geometry of pack_trilinear_kernel's thread: its cell (cy, cx), its
// channel offset, and its voxels' y/x source pairs and weights.
struct TriColumn {
  int cy, cx, ch;
  int ya[2], yb[2], xa[2], xb[2];
  float ly[2], lx[2];
};

// The 3x3 source vectors of an inner column's plane (clamped into the
// volume): rows cy - 1 .. cy + 1, columns cx - 1 .. cx + 1.
struct TriRows {
  f4 v[3][3];
};

__device__ __forceinline__ TriRows tri_rows(const PackArgs& a, const TriColumn& t, const float* src, int zs) {
  TriRows o;
  zs = min(max(zs, 0), a.id - 1);
  const float* pl = src + (int64_t)zs * a.ih * a.iw * a.c;
#pragma unroll
  for (int ys = 0; ys < 3; ++ys) {
    const float* row = pl + ((int64_t)(t.cy - 1 + ys) * a.iw + (t.cx - 1)) * a.c;
#pragma unroll
    for (int xs = 0; xs < 3; ++xs) o.v[ys][xs] = *reinterpret_cast<const f4*>(row + xs * a.c);
  }
  return o;
}

// x-then-y interpolation of an inner column's plane: the four voxel columns
// share the 3x3 source rows (x pairs (cx - 1, cx), (cx, cx + 1); y likewise).
__device__ __forceinline__ TriPlane tri_inner_plane(const TriColumn& t, const TriRows& s) {
#pragma clang fp contract(off)
  TriPlane o;
  f4 rr[3][2];  // [source row][dx]
#pragma unroll
  for (int ys = 0; ys < 3; ++ys)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      rr[ys][0][q] = fmaf(1.0f - t.lx[0], s.v[ys][0][q], t.lx[0] * s.v[ys][1][q]);
      rr[ys][1][q] = fmaf(1.0f - t.lx[1], s.v[ys][1][q], t.lx[1] * s.v[ys][2][q]);
    }
#pragma unroll
  for (int dx = 0; dx < 2; ++dx)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o.p[0][dx][q] = fmaf(1.0f - t.ly[0], rr[0][dx][q], t.ly[0] * rr[1][dx][q]);
      o.p[1][dx][q] = fmaf(1.0f - t.ly[1], rr[1][dx][q], t.ly[1] * rr[2][dx][q]);
    }
  return o;
}

// x-then-y-interpolated source plane zs (clamped into the volume) of a face
// column: its four voxel columns' y/x pairs loaded apart (16 loads).
__device__ __forceinline__ TriPlane tri_face_plane(const PackArgs& a, const TriColumn& t, const float* src, int zs) {
#pragma clang fp contract(off)
  TriPlane o;
  zs = min(max(zs, 0), a.id - 1);
  const float* pl = src + (int64_t)zs * a.ih * a.iw * a.c;
#pragma unroll
  for (int dy = 0; dy < 2; ++dy) {
    const float* r0 = pl + (int64_t)t.ya[dy] * a.iw * a.c;
    const float* r1 = pl + (int64_t)t.yb[dy] * a.iw * a.c;
#pragma unroll
    for (int dx = 0; dx < 2; ++dx) {
      const f4 a0 = *reinterpret_cast<const f4*>(r0 + (int64_t)t.xa[dx] * a.c);
      const f4 a1 = *reinterpret_cast<const f4*>(r0 + (int64_t)t.xb[dx] * a.c);
      const f4 b0 = *reinterpret_cast<const f4*>(r1 + (int64_t)t.xa[dx] * a.c);
      const f4 b1 = *reinterpret_cast<const f4*>(r1 + (int64_t)t.xb[dx] * a.c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float ra = fmaf(1.0f - t.lx[dx], a0[q], t.lx[dx] * a1[q]);
        const float rb = fmaf(1.0f - t.lx[dx], b0[q], t.lx[dx] * b1[q]);
        o.p[dy][dx][q] = fmaf(1.0f - t.ly[dy], ra, t.ly[dy] * rb);
      }
    }
  }
  return o;
}

// One column's march over cells [cz0, cz1) of batch item b (see
// pack_trilinear_kernel): blend, transform and store each cell's 2x2x2 voxels.
template <int FMT, bool INNER>
__device__ __forceinline__ void tri_march(const PackArgs& a, const TriColumn& t, int b, int cz0, int cz1) {
#pragma clang fp contract(off)
  const int PW = a.gw + 2, PH = a.gh + 2, PD = a.gd + 2;
  const float* src = a.x + (int64_t)b * a.id * a.ih * a.iw * a.c + t.ch;
  f4 sc = {0.f, 0.f, 0.f, 0.f}, of = {0.f, 0.f, 0.f, 0.f};
  if (a.affine_on) load_affine4(a, b, t.ch, sc, of);
  // inner columns load the next plane's rows one cell ahead of its blend
  TriPlane pm, p0;
  TriRows next;
  if constexpr (INNER) {
    pm = tri_inner_plane(t, tri_rows(a, t, src, cz0 - 1));
    next = tri_rows(a, t, src, cz0 + 1);
    p0 = tri_inner_plane(t, tri_rows(a, t, src, cz0));
  } else {
    pm = tri_face_plane(a, t, src, cz0 - 1);
    p0 = tri_face_plane(a, t, src, cz0);
  }
  for (int cz = cz0; cz < cz1; ++cz) {
    TriPlane p1;
    if constexpr (INNER) {
      p1 = tri_inner_plane(t, next);
      if (cz + 1 < cz1) next = tri_rows(a, t, src, cz + 2);
    } else {
      p1 = tri_face_plane(a, t, src, cz + 1);
    }
    f4 out[8];
    if (cz >= 1 && cz <= a.id - 2) {
      // both voxels' z pairs are unclamped: (cz - 1, cz) and (cz, cz + 1)
      float lz[2];
      int z0, z1;
      tri_axis(2 * cz, a.id, z0, z1, lz[0]);
      tri_axis(2 * cz + 1, a.id, z0, z1, lz[1]);
#pragma unroll
      for (int dy = 0; dy < 2; ++dy)
#pragma unroll
        for (int dx = 0; dx < 2; ++dx)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            out[dy * 2 + dx][q] = fmaf(1.0f - lz[0], pm.p[dy][dx][q], lz[0] * p0.p[dy][dx][q]);
            out[4 + dy * 2 + dx][q] = fmaf(1.0f - lz[1], p0.p[dy][dx][q], lz[1] * p1.p[dy][dx][q]);
          }
    } else {
      // near the z faces: pick each voxel's two planes among the clamped
      // planes cz - 1, cz, cz + 1 (equal clamped planes hold equal bits; the
      // halo cells' voxels are not stored from these)
      const int zlo = max(cz - 1, 0), zmid = min(max(cz, 0), a.id - 1);
#pragma unroll
      for (int dz = 0; dz < 2; ++dz) {
        int z0, z1;
        float lz;
        tri_axis(2 * cz + dz, a.id, z0, z1, lz);
        const int sa = z0 == zlo ? 0 : z0 == zmid ? 1 : 2, sb = z1 == zlo ? 0 : z1 == zmid ? 1 : 2;
#pragma unroll
        for (int dy = 0; dy < 2; ++dy)
#pragma unroll
          for (int dx = 0; dx < 2; ++dx)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float va = sa == 0 ? pm.p[dy][dx][q] : sa == 1 ? p0.p[dy][dx][q] : p1.p[dy][dx][q];
              const float vb = sb == 0 ? pm.p[dy][dx][q] : sb == 1 ? p0.p[dy][dx][q] : p1.p[dy][dx][q];
              out[dz * 4 + dy * 2 + dx][q] = fmaf(1.0f - lz, va, lz * vb);
            }
      }
    }
    pm = p0;
    p0 = p1;
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      const int oz = 2 * cz + (o >> 2), oy = 2 * t.cy + ((o >> 1) & 1), ox = 2 * t.cx + (o & 1);
      if (oz < -1 || oz > a.gd || oy < -1 || oy > a.gh || ox < -1 || ox > a.gw) continue;
      const bool inside = oz >= 0 && oz < a.gd && oy >= 0 && oy < a.gh && ox >= 0 && ox < a.gw;
      const f4 v = inside ? pack_transform4(a, out[o], sc, of) : f4{0.f, 0.f, 0.f, 0.f};
      const int64_t vox = (((int64_t)b * PD + oz + 1) * PH + oy + 1) * PW + ox + 1;
      if constexpr (FMT == PF_SPLIT) {
        store_split4(a.out, split_offset(vox, a.cp, t.ch), v);
      } else if constexpr (FMT == PF_BF16) {
        uint2 packed;
        packed.x = bf16_pair(v[0], v[1]);
        packed.y = bf16_pair(v[2], v[3]);
        *reinterpret_cast<uint2*>(reinterpret_cast<unsigned*>(a.out) + (vox * a.cp + t.ch) / 2) = packed;
      } else {
        *reinterpret_cast<f4*>(reinterpret_cast<float*>(a.out) + vox * a.cp + t.ch) = v;
      }
    }
  }
}

// Zeros of the padded copy for a column's channel group past the source
// channels, over cells [cz0, cz1) of batch item b.
template <int FMT>
__device__ __forceinline__ void tri_zero(const PackArgs& a, const TriColumn& t, int b, int cz0, int cz1) {
  const int PW = a.gw + 2, PH = a.gh + 2, PD = a.gd + 2;
  for (int cz = cz0; cz < cz1; ++cz)
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      const int oz = 2 * cz + (o >> 2), oy = 2 * t.cy + ((o >> 1) & 1), ox = 2 * t.cx + (o & 1);
      if (oz < -1 || oz > a.gd || oy < -1 || oy > a.gh || ox < -1 || ox > a.gw) continue;
      const int64_t vox = (((int64_t)b * PD + oz + 1) * PH + oy + 1) * PW + ox + 1;
      if constexpr (FMT == PF_SPLIT)
        store_split4(a.out, split_offset(vox, a.cp, t.ch), f4{0.f, 0.f, 0.f, 0.f});
      else if constexpr (FMT == PF_BF16)
        *reinterpret_cast<uint2*>(reinterpret_cast<unsigned*>(a.out) + (vox * a.cp + t.ch) / 2) = uint2{0u, 0u};
      else
        *reinterpret_cast<f4*>(reinterpret_cast<float*>(a.out) + vox * a.cp + t.ch) = f4{0.f, 0.f, 0.f, 0.f};
    }
}

template <int FMT, int ZC>
__global__ __launch_bounds__(256) void pack_trilinear_kernel(PackArgs a) {
  const int cgn = a.cp >> 2;
  const int CW = a.iw + 2, CH = a.ih + 2, CD = a.id + 2;
  const unsigned cells = (unsigned)CH * (unsigned)CW * (unsigned)cgn;
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= cells) return;
  TriColumn t;
  t.ch = (int)(i % (unsigned)cgn) * 4;
  const unsigned r = i / (unsigned)cgn;
  t.cx = (int)(r % (unsigned)CW) - 1;
  t.cy = (int)(r / (unsigned)CW) - 1;
  // the halo cells' pairs are clamped into the volume: their voxels are
  // zeros or lie past the copy, only the loads need to stay in bounds
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    tri_axis(2 * t.cy + d, a.ih, t.ya[d], t.yb[d], t.ly[d]);
    tri_axis(2 * t.cx + d, a.iw, t.xa[d], t.xb[d], t.lx[d]);
    t.ya[d] = min(t.ya[d], a.ih - 1);
    t.xa[d] = min(t.xa[d], a.iw - 1);
  }
  const bool inner = t.cy >= 1 && t.cy <= a.ih - 2 && t.cx >= 1 && t.cx <= a.iw - 2;
  const int chunks = (CD + ZC - 1) / ZC;
  for (int bc = blockIdx.y; bc < a.n * chunks; bc += gridDim.y) {
    const int b = bc / chunks, cz0 = (bc - b * chunks) * ZC - 1;
    const int cz1 = min(cz0 + ZC, a.id + 1);
    if (t.ch >= a.c)
      tri_zero<FMT>(a, t, b, cz0, cz1);
    else if (inner)
      tri_march<FMT, true>(a, t, b, cz0, cz1);
    else
      tri_march<FMT, false>(a, t, b, cz0, cz1);
  }
}

// Small-cin packing (cin below one K block): one row per output voxel holding
// every tap's channels, K index tap*cin + c (tap = kd*9 + kh*3 + kw), so the
// GEMM runs ceil(27*cin / K block) steps instead of 27 padded ones.  Values
// outside the volume are zero; inside ones get pack_input's affine + SiLU, or
// its trilinear-2x sample (same helper, so both packings agree bitwise).
struct Im2colArgs {
  const float* x;
  void* out;
  const float* affine;
  int64_t total4;        // n * output voxels * cp / 4
  int d, h, w, c, cp;    // convolved grid (2x the source for trilinear), channels, packed channels
  int od, oh, ow, stride;
  int sd, sh, sw;        // source grid
  int affine_on, silu_on, trilinear, bf16;
};

__global__ __launch_bounds__(256) void im2col_kernel(Im2colArgs a) {
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total4;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c4n = a.cp >> 2;
    const int k0 = (int)(idx % c4n) * 4;
    int64_t v = idx / c4n;
    const int ox = (int)(v % a.ow);
    v /= a.ow;
    const int oy = (int)(v % a.oh);
    v /= a.oh;
    const int oz = (int)(v % a.od);
    const int b = (int)(v / a.od);
    f4 val = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + j;
      if (k >= 27 * a.c) continue;
      const int tap = k / a.c, ch = k - tap * a.c;
      const int z = oz * a.stride + tap / 9 - 1, y = oy * a.stride + (tap / 3) % 3 - 1,
                x = ox * a.stride + tap % 3 - 1;
      if (z < 0 || z >= a.d || y < 0 || y >= a.h || x < 0 || x >= a.w) continue;
      float t;
      if (a.trilinear)
        t = trilinear_sample1(a.x + (int64_t)b * a.sd * a.sh * a.sw * a.c, a.sd, a.sh, a.sw, a.c, ch, z, y, x);
      else
        t = a.x[((((int64_t)b * a.d + z) * a.h + y) * a.w + x) * a.c + ch];
      if (a.affine_on) {
        const float* q = a.affine + ((int64_t)b * a.c + ch) * 2;
        t = fmaf(t, q[0], q[1]);
      }
      if (a.silu_on) t = silu_f(t);
      val[j] = t;
    }
    if (a.bf16) {
      uint2 packed;
      packed.x = (unsigned)f32_to_bf16_bits(val[0]) | ((unsigned)f32_to_bf16_bits(val[1]) << 16);
      packed.y = (unsigned)f32_to_bf16_bits(val[2]) | ((unsigned)f32_to_bf16_bits(val[3]) << 16);
      reinterpret_cast<uint2*>(a.out)[idx] = packed;
    } else {
      reinterpret_cast<f4*>(a.out)[idx] = val;
    }
  }
}

// Small-cout convolution, second stage: the tap-expanded GEMM left, for every
// padded input row r and column tap*cout + o, z[(tap*cout + o) * zstride + r]
// = sum_c xpad[r, c] * W[o, c, tap].  Output voxel v sums the 27 taps of its
// window (top-left padded row stride * v) in ascending tap order after the
// bias, then adds the residual.  At stride 1 the window rows of consecutive
// voxels are consecutive for a fixed tap, so each z element is read once and
// every load is coalesced.
__global__ __launch_bounds__(256) void tap_sum_kernel(const float* __restrict__ z, int64_t zstride,
                                                      int64_t rows_per_batch, int P, int Q, int stride, int n,
                                                      int d, int h, int w, int cout, const float* __restrict__ bias,
                                                      int batch_bias, const float* __restrict__ res,
                                                      float* __restrict__ y) {
  const int64_t S = (int64_t)d * h * w;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < (int64_t)n * S;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int b = (int)(idx / S);
    const int v = (int)(idx - (int64_t)b * S);
    const int dd = v / (h * w), r = v - dd * (h * w);
    const int hh = r / w, ww = r - hh * w;
    const int64_t row = (int64_t)b * rows_per_batch + (int64_t)stride * dd * P + (int64_t)stride * hh * Q +
                        stride * ww;
    for (int o = 0; o < cout; ++o) {
      float sum = bias ? bias[(batch_bias ? (int64_t)b * cout : 0) + o] : 0.f;
      const float* zc = z + (int64_t)o * zstride + row;
#pragma unroll
      for (int tap = 0; tap < 27; ++tap)
        sum += zc[(int64_t)tap * cout * zstride + (tap / 9) * P + ((tap / 3) % 3) * Q + tap % 3];
      if (res) sum += res[idx * cout + o];
      y[idx * cout + o] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. Weight packing (reference: _nax_conv.py:372-445)
// ---------------------------------------------------------------------------
// Packed layout: [phase][tap][kblock][np][KSTEP] where KSTEP is 16 fp32 or 32
// bf16 values (64 bytes), tap = kd*KT*KT + kh*KT + kw, channel = kblock*KSTEP + e,
// zero for channels >= cin or columns >= cout.
struct WPackArgs {
  const float* w;  // Torch (cout, cin, ks, ks, ks)
  void* out;
  int64_t total;
  int cout, cin, ks, np, kblocks, kstep, taps, up, bf16;
  int layout;      // WL_TAPS, or WL_EXPAND / WL_IM2COL with taps = 1
  int phases;
  float* colscale; // split fp16: (np) power-of-two column scales after the packed blocks, else null
};

// Packed-weight layouts.  WL_TAPS: K = (tap, channel).  WL_EXPAND (cout <= 4):
// one 1x1 GEMM whose column tap*cout + o holds W[o, :, tap].  WL_IM2COL
// (cin below one K block): K index tap*cin + c holds W[:, c, tap].
enum { WL_TAPS = 0, WL_EXPAND = 1, WL_IM2COL = 2 };

// Nearest-2x parity fold: tap t of parity p on one axis merges the 3x3x3
// taps k in [lo, hi]: p=0 -> t0:{0}, t1:{1,2}; p=1 -> t0:{0,1}, t1:{2}
// (derivation at _nax_conv.py:407-414).
__device__ __forceinline__ void fold_range(int p, int t, int& lo, int& hi) {
  lo = (p == 0) ? (t == 0 ? 0 : 1) : (t == 0 ? 0 : 2);
  hi = (p == 0) ? (t == 0 ? 0 : 2) : (t == 0 ? 1 : 2);
}

// Packed value of channel c (K index for WL_IM2COL) of column col at tap `tap`
// of parity `phase`: zero past the weight's channels / columns.
__device__ __forceinline__ float packed_weight_value(const WPackArgs& a, int phase, int tap, int c, int col) {
  float val = 0.f;
  if (a.layout == WL_EXPAND) {
    if (col < 27 * a.cout && c < a.cin) val = a.w[((int64_t)(col % a.cout) * a.cin + c) * 27 + col / a.cout];
  } else if (a.layout == WL_IM2COL) {
    if (col < a.cout && c < 27 * a.cin) val = a.w[((int64_t)col * a.cin + c % a.cin) * 27 + c / a.cin];
  } else if (col < a.cout && c < a.cin) {
    const float* wc = a.w + ((int64_t)col * a.cin + c) * a.ks * a.ks * a.ks;
    if (!a.up) {
      const int kd = tap / (a.ks * a.ks), kh = (tap / a.ks) % a.ks, kw = tap % a.ks;
      val = wc[(kd * a.ks + kh) * a.ks + kw];
    } else {
      const int td = tap >> 2, th = (tap >> 1) & 1, tw = tap & 1;
      const int pd = phase >> 2, ph = (phase >> 1) & 1, pw = phase & 1;
      int d0, d1, h0, h1, w0, w1;
      fold_range(pd, td, d0, d1);
      fold_range(ph, th, h0, h1);
      fold_range(pw, tw, w0, w1);
      float s = 0.f;
      for (int kd = d0; kd <= d1; ++kd)
        for (int kh = h0; kh <= h1; ++kh)
          for (int kw = w0; kw <= w1; ++kw) s += wc[(kd * 3 + kh) * 3 + kw];
      val = s;
    }
  }
  return val;
}

__global__ __launch_bounds__(256) void pack_weight_kernel(WPackArgs a) {
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = idx;
    const int e = (int)(t % a.kstep);
    t /= a.kstep;
    const int col = (int)(t % a.np);
    t /= a.np;
    const int kb = (int)(t % a.kblocks);
    t /= a.kblocks;
    const int tap = (int)(t % a.taps);
    const int phase = (int)(t / a.taps);
    const float val = packed_weight_value(a, phase, tap, kb * a.kstep + e, col);
    if (a.bf16)
      reinterpret_cast<unsigned short*>(a.out)[idx] = f32_to_bf16_bits(val);
    else
      reinterpret_cast<float*>(a.out)[idx] = val;
  }
}

// Split-fp16 weights (CTMR_F16X2), step 1: the power-of-two scale 2^-k of
// each packed column, k chosen so that the column's largest magnitude m
// (over every phase, tap and channel of the packed values, nearest-2x folds
// included) times 2^k lies in [2^14, 2^15): fp16 holds the scaled weights'
// hi and lo halves as normal numbers.  k = 0 for an all-zero column; k is
// kept within [-100, 100].  One workgroup per column (a max is exact in any
// order).
__global__ __launch_bounds__(256) void weight_colscale_kernel(WPackArgs a) {
  const int col = blockIdx.x;
  const int count = a.phases * a.taps * a.cin;
  float m = 0.f;
  for (int i = threadIdx.x; i < count; i += 256) {
    const int c = i % a.cin, t = i / a.cin;
    m = fmaxf(m, fabsf(packed_weight_value(a, t / a.taps, t % a.taps, c, col)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  __shared__ float wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int k = 0;
    if (m > 0.f) {
      const int e = (int)((__float_as_uint(m) >> 23) & 0xff) - 127;  // floor(log2 m) for normal m
      k = min(max(14 - e, -100), 100);
    }
    a.colscale[col] = ldexpf(1.0f, -k);
  }
}

// Split-fp16 weights, step 2: per (phase, tap, 16-channel block, column) 96
// bytes -- hi (channels 0..15), hi * 2^-11 (the same, for the input's lo
// halves, which carry 2^11), lo -- of the column-scaled weight ws = w * 2^k:
// hi = fp16(ws), lo = fp16(ws - hi); ws - hi is exact in fp32.
__global__ __launch_bounds__(256) void pack_weight_split_kernel(WPackArgs a) {
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = idx;
    const int e = (int)(t % 16);
    t /= 16;
    const int col = (int)(t % a.np);
    t /= a.np;
    const int kb = (int)(t % a.kblocks);
    t /= a.kblocks;
    const int tap = (int)(t % a.taps);
    const int phase = (int)(t / a.taps);
    const float ws = packed_weight_value(a, phase, tap, kb * 16 + e, col) / a.colscale[col];  // exact: 2^k
    const _Float16 hi = (_Float16)ws;
    _Float16* block = reinterpret_cast<_Float16*>(a.out) + (idx - e) * 3;  // 48 halves per 16 channels
    block[e] = hi;
    block[16 + e] = (_Float16)((float)hi * (1.0f / 2048.0f));
    block[32 + e] = (_Float16)(ws - (float)hi);
  }
}

// ---------------------------------------------------------------------------
// 3. Implicit-GEMM convolution
// ---------------------------------------------------------------------------
struct ConvArgs {
  const char* xp;          // packed input (or x itself for unpacked 1x1)
  const char* wp;          // packed weight
  const float* bias;       // (cout) or (n, cout) or null
  const float* res;        // output-shaped residual or null
  float* y;                // output, or split partial planes
  int64_t x_bytes;         // bytes of the packed input (buffer-descriptor range)
  int64_t w_bytes;         // bytes of the packed weight
  int64_t rows_per_batch;  // rows of the packed input per batch item
  int64_t row_bytes;       // bytes per packed row (cp * element size)
  int64_t plane;           // elements per split plane (n * s_out * cout)
  int kb, np, cout;        // 64-byte K blocks per tap, packed / real columns
  int gd, gh, gw;          // iteration grid (output grid; source grid for UP)
  int P, Q;                // padded plane / row pitch in rows
  int oh, ow, s_out;       // output H, W and voxel count (UP remap)
  int taps, split, m_tiles, n_tiles;
  int batch_bias, has_res, has_bias;
  int planar;              // store column c of voxel v at y[c * zstride + v] (tap-expanded GEMM)
  int64_t zstride;
  double* stats;           // group-norm partials of the output (ctmr_conv3d_gn) or null
  int gn_groups, gn_cpg, stats_tiles;
  int items;               // pointwise_kernel: row tiles x batch items x split ranges
  int in_d, in_h, in_w;    // input extent (conv_kernel<.., DIRECT>: A read from x itself)
  // Two-source input (pointwise_kernel reading x directly): K blocks from kb1
  // on come from xp2, rows of row_bytes2 bytes; kb1 = kb for one source.
  const char* xp2;
  int64_t row_bytes2;
  int kb1;
};

// Final step of the group-norm partials of a stored tile: red[wave][c] holds
// the fp64 (sum, sum of squares) of column c of each wave's 64 x (NSUB*16)
// block over its rows (published by a barrier); each group's columns and
// waves are added in ascending order -- a fixed order for a given shape.
template <int NSUB, int WM, int WN>
__device__ __forceinline__ void combine_gn_partials(const double (*red)[64][2], int col0, int cout, int cpg,
                                                    int groups, double* __restrict__ stats_tile) {
  constexpr int kWaveCols = NSUB * 16;
  const int groups_here = (WN * kWaveCols) / cpg;
  for (int gl = threadIdx.x; gl < groups_here; gl += 256) {
    const int g = col0 / cpg + gl;
    if (g >= groups || g * cpg >= cout) continue;
    double a = 0.0, q = 0.0;
    for (int wm = 0; wm < WM; ++wm)
      for (int cc = 0; cc < cpg; ++cc) {
        const int col = gl * cpg + cc;
        const int wv = (col / kWaveCols) * WM + wm;
        a += red[wv][col % kWaveCols][0];
        q += red[wv][col % kWaveCols][1];
      }
    stats_tile[(int64_t)g * 2] = a;
    stats_tile[(int64_t)g * 2 + 1] = q;
  }
}

template <int DT>
__device__ __forceinline__ void mfma_step(f4& acc, const u4& a, const u4& b);

template <>
__device__ __forceinline__ void mfma_step<CTMR_F32>(f4& acc, const u4& a, const u4& b) {
  const f4 fa = __builtin_bit_cast(f4, a), fb = __builtin_bit_cast(f4, b);
  // Four K=4 products; component j of lane group g is input channel 4g + j.
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[0], fb[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[1], fb[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[2], fb[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[3], fb[3], acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ void mfma_step<CTMR_BF16>(f4& acc, const u4& a, const u4& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a),
                                                 __builtin_bit_cast(bf8, b), acc, 0, 0, 0);
}

// One K block of a wave's 64 x (NSUB*16) tile: A[ms] holds rows ms*16 + lane%16,
// B[ns] columns ns*16 + lane%16, each 16 bytes of K per lane group.  fp32: the
// K sub-step is outermost, so consecutive MFMAs always write different
// accumulators and none waits for the previous one's result.
// TRANSPOSED multiplies B^T A^T instead: the same products summed in the same
// K order (each output is the same dot product), but the result block holds
// row lane%16 and columns 4*(lane/16) .. +3 in a lane's four registers.
template <int DT, int NSUB, bool TRANSPOSED = false>
__device__ __forceinline__ void mma_block(f4 (&acc)[4][NSUB], const u4 (&A)[4], const u4 (&B)[NSUB]) {
  if constexpr (DT == CTMR_F32) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns) {
          const float a = __builtin_bit_cast(f4, A[ms])[j], b = __builtin_bit_cast(f4, B[ns])[j];
          acc[ms][ns] = TRANSPOSED ? __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, acc[ms][ns], 0, 0, 0)
                                   : __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[ms][ns], 0, 0, 0);
        }
  } else {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) {
        if constexpr (TRANSPOSED)
          mfma_step<DT>(acc[ms][ns], B[ns], A[ms]);
        else
          mfma_step<DT>(acc[ms][ns], A[ms], B[ns]);
      }
  }
}

// One DPP lane move of an fp64 value (two 32-bit halves; every source lane
// lies inside the lane's row of 16).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_mov_dpp((int)(unsigned)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Sum over the 16 lanes of a row, in the tree of an xor butterfly (partners
// 1, 2, 4, 8): quad_perm [1,0,3,2] and [2,3,0,1] are xor 1 and xor 2; after
// them lane 7 - i of a half row holds the value lane i ^ 4 holds (fp32/fp64
// addition commutes), so the half-row mirror is the xor-4 step and the row
// mirror the xor-8 step.  VALU moves instead of LDS permutes.
__device__ __forceinline__ double row16_sum(double v) {
  v += dpp_f64<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f64<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f64<0x141>(v);  // row_half_mirror
  v += dpp_f64<0x140>(v);  // row_mirror
  return v;
}

// Column sums over a wave's 64 rows of a transposed accumulator block set
// (lane l of block (ms, ns): row ms*16 + l%16, columns ns*16 + 4*(l/16) .. +3),
// masked by row_ok[ms] and col_ok[ns]: per block ns the 4 row blocks in the
// lane, then the butterfly tree over l%16 (row16_sum); lanes l%16 == 0
// publish the fp64 (sum, sum of squares) of their 4 columns in
// red[wave][column].  A fixed order.
template <int NSUB>
__device__ __forceinline__ void column_sums(const f4 (&acc)[4][NSUB], const bool (&row_ok)[4],
                                            const bool (&col_ok)[NSUB], double (*red)[64][2], int wave, int lane) {
  const int lrow = lane & 15, lgrp = lane >> 4;
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) {
    double q1[4] = {0.0, 0.0, 0.0, 0.0}, q2[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) {
      const bool ok = row_ok[ms] && col_ok[ns];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const double d = ok ? (double)acc[ms][ns][r] : 0.0;
        q1[r] += d;
        q2[r] = fma(d, d, q2[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      q1[r] = row16_sum(q1[r]);
      q2[r] = row16_sum(q2[r]);
    }
    if (lrow == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        red[wave][ns * 16 + 4 * lgrp + r][0] = q1[r];
        red[wave][ns * 16 + 4 * lgrp + r][1] = q2[r];
      }
    }
  }
}

// Bias of the lane's output columns n0 + ns*16 + 4*(lane/16) + r (transposed
// accumulator layout) for batch item b; zero for a split's partial planes or
// without bias.
template <int NSUB>
__device__ __forceinline__ void load_bias(const ConvArgs& p, int b, int n0, int lane, f4 (&bq)[NSUB]) {
  const float* bias_b = p.bias + (p.batch_bias ? (int64_t)b * p.cout : 0);
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bq[ns][r] = (p.split == 1 && p.has_bias) ? bias_b[min(n0 + ns * 16 + 4 * (lane >> 4) + r, p.cout - 1)] : 0.f;
}

// Epilogue of one wave's 64 x (NSUB*16) tile from transposed accumulators
// (mma_block<.., true>): lane l of block (ms, ns) holds row m0 + ms*16 + l%16
// and columns n0 + ns*16 + 4*(l/16) .. +3; output voxel v of batch item b is
// stored at out_voxel(v) (the nearest-2x remap, or b * s_out + v).  With
// cout % 4 == 0 (not the planar tap-expanded output) each block is one
// 16-byte store (and residual load); otherwise four masked scalar ones.
// Residual values are all loaded before the first store: interleaved, each
// load would wait for the stores before it (the compiler cannot prove the
// output and its inputs apart).  Rows past the grid are clamped for the loads
// and masked for the stores.
// Cache-policy operands of the GEMMs' output stores (gfx950 encoding: bit 1 =
// NT, non-temporal; bit 4 = SC1, device scope).  Same values under every
// policy; measured on MI355X, default / NT / SC1, A/B twice in one run: the
// brick GEMMs (fp32 and bf16 LDS-staged) and the streaming GEMM take SC1
// (config-0 fp32 + bf16 GEMMs 0.462 / 0.505 / 0.451 ms, UNet step 17.72 /
// 17.80 / 17.69 ms, config-1 block 26.18 / 26.17 / 26.14 ms, config 2a and
// the decoder window within 0.5 % either way); the persistent 1x1 GEMM takes
// NT (config 2c 0.165 / 0.160 / 0.171 ms).
constexpr int kStoreSC1 = 16;
constexpr int kStoreNT = 2;

// IDENT: GEMM row v of batch item b is output voxel b * s_out + v (every route
// but the nearest-2x parity phases), so a wave's 64 rows are contiguous and
// its stores go through one buffer descriptor with the SC1 cache policy.
// No term after the bias (the epilogues' default `after_bias`).
struct NoTerm {
  template <typename Acc>
  __device__ void operator()(Acc&) const {}
};

template <int NSUB, int WM, int WN, bool IDENT, typename OutVoxel, typename AfterBias = NoTerm>
__device__ __forceinline__ void store_tile(const ConvArgs& p, f4 (&acc)[4][NSUB], const f4 (&bq)[NSUB], int b,
                                           int m0, int n0, int S, int split_id, int wave, int lane, int col0,
                                           int tile_id, OutVoxel out_voxel, AfterBias after_bias = {}) {
  const int lrow = lane & 15, lgrp = lane >> 4;
  const bool partial = p.split > 1;
  float* out = p.y + (partial ? (int64_t)split_id * p.plane : 0);
  const bool add_res = !partial && p.has_res;
  const bool wide = !p.planar && (p.cout & 3) == 0;
  bool row_ok[4], col_ok[NSUB];
  int64_t vox[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    const int v = m0 + ms * 16 + lrow;
    row_ok[ms] = v < S;
    vox[ms] = out_voxel(min(v, S - 1));
  }
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) col_ok[ns] = n0 + ns * 16 + 4 * lgrp < p.cout;  // whole quad when wide
  if (!partial && p.has_bias) {  // bias first, then the residual (the reference's epilogue order)
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] += bq[ns];
  }
  after_bias(acc);  // a second K range, between the bias and the residual
  if (add_res) {
    f4 rq[4][NSUB];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) {
        const int c0 = n0 + ns * 16 + 4 * lgrp;
        if (wide) {
          rq[ms][ns] = *reinterpret_cast<const f4*>(p.res + vox[ms] * p.cout + min(c0, p.cout - 4));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) rq[ms][ns][r] = p.res[vox[ms] * p.cout + min(c0 + r, p.cout - 1)];
        }
      }
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] += rq[ms][ns];
  }
  int64_t vbase = 0;
  __amdgpu_buffer_rsrc_t ors;
  if constexpr (IDENT) {
    vbase = out_voxel(min(m0, S - 1));  // the wave's first row; the others follow it
    ors = __builtin_amdgcn_make_buffer_rsrc(out + vbase * p.cout, (short)0,
                                            (int)min(max((int64_t)p.plane - vbase * p.cout, (int64_t)0) * 4,
                                                     (int64_t)0x7fffffff), 0x00020000);
  }
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) {
      const int c0 = n0 + ns * 16 + 4 * lgrp;
      const f4 val = acc[ms][ns];
      if (wide) {
        if constexpr (IDENT) {
          if (row_ok[ms] && col_ok[ns])
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, val), ors,
                                                   (int)(((vox[ms] - vbase) * p.cout + c0) * 4), 0, kStoreSC1);
        } else {
          if (row_ok[ms] && col_ok[ns]) *reinterpret_cast<f4*>(out + vox[ms] * p.cout + c0) = val;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (row_ok[ms] && c0 + r < p.cout)
            out[p.planar ? (int64_t)(c0 + r) * p.zstride + vox[ms] : vox[ms] * p.cout + c0 + r] = val[r];
      }
    }
  if (p.stats) {  // wave-uniform (a kernel argument): every thread reaches the barrier
    __shared__ double red[WM * WN][64][2];
    if (!wide) {
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) col_ok[ns] = true;  // per-column masks below
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n0 + ns * 16 + 4 * lgrp + r >= p.cout) acc[ms][ns][r] = 0.f;
    }
    column_sums<NSUB>(acc, row_ok, col_ok, red, wave, lane);
    __syncthreads();
    combine_gn_partials<NSUB, WM, WN>(red, col0, p.cout, p.gn_cpg, p.gn_groups,
                                      p.stats + ((int64_t)b * p.stats_tiles + tile_id) * p.gn_groups * 2);
  }
}

// DIRECT: a plain fp32 3x3x3 conv with cin % 16 == 0 reads its A rows from the
// unpadded input x itself instead of a zero-padded packed copy (no pack pass).
// A lane's window may cross the volume border, so for each tap the lane's
// offset is either the real row or one past the buffer's range, which the
// hardware reads as zeros -- the padded copy's zeros, so the products and their
// order, and the output bits, are those of the packed form.
// KWS = 4 (small K-split grids, a 64 x 64 tile per workgroup): the four waves
// sum four contiguous quarters of the workgroup's K range for the same tile and
// combine them through LDS in ascending order, so a launch needs a quarter of
// the split partial planes (and their reduction traffic).  SETS = 2 with it:
// a split of two inside the workgroup -- wave set s (waves 4s .. 4s + 3) sums
// K range s as above, and set 0 adds set 1's sum after the bias (the split
// reduction's order: bias, range 0, range 1, residual), so the launch writes
// the outputs and their group-norm partials with no partial planes.
template <int DT, int NSUB, int WM, int WN, int KT, int STRIDE, bool UP, bool DIRECT = false, int KWS = 1,
          int SETS = 1>
__global__ __launch_bounds__(256 * SETS, SETS == 1 ? 2 : 1) void conv_kernel(ConvArgs p) {
  static_assert(WM * WN * KWS == 4, "four waves per wave set");
  static_assert(SETS == 1 || (SETS == 2 && KWS == 4), "two wave sets only with the four-wave K split");
  static_assert(!DIRECT || (KT == 3 && !UP && DT == CTMR_F32), "direct reads: plain fp32 3x3x3 convs");
  const int lane = threadIdx.x & 63;
  // Wave index made provably uniform so every address base below lives in SGPRs.
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int set = wave_all >> 2, wave = wave_all & 3;
  const int wave_mn = wave % (WM * WN), wave_k = wave / (WM * WN);
  const int wave_m = wave_mn % WM, wave_n = wave_mn / WM;

  // XCD-aware tile order: hardware deals consecutive workgroups round-robin
  // to the 8 XCDs; give each XCD a contiguous range of tiles so neighbouring
  // windows (shared halo rows) and column tiles of one voxel tile share an L2.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot = bid >> 3, per = nb >> 3, rem = nb & 7;
  const int tile = (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = tile % p.n_tiles;
  const int rest = tile / p.n_tiles;
  const int m_tile = rest % p.m_tiles;
  const int z = rest / p.m_tiles;
  const int split_id = z % p.split, zb = z / p.split;
  const int b = UP ? (zb >> 3) : zb;
  const int phase = UP ? (zb & 7) : 0;
  const int pd = phase >> 2, ph = (phase >> 1) & 1, pw = phase & 1;

  const int ghw = p.gh * p.gw;
  const int S = p.gd * ghw;
  const int m0 = m_tile * (WM * 64) + wave_m * 64;
  const int lrow = lane & 15, lgrp = lane >> 4;

  // Loads go through buffer descriptors: a wave-uniform base (SGPRs), a
  // per-lane 32-bit offset fixed for the whole kernel, and one scalar offset
  // per K step, so a step costs no vector address arithmetic.
  auto window_row = [&](int v) -> int64_t {
    const int d = v / ghw, r = v - d * ghw;
    const int h = r / p.gw, w = r - h * p.gw;
    return (int64_t)(STRIDE * d + pd) * p.P + (int64_t)(STRIDE * h + ph) * p.Q + STRIDE * w + pw;
  };
  // A: one window-start row per 16-voxel block; rows past the grid reuse the
  // last voxel and are not stored.  Rows grow with the voxel index, so the
  // wave's first voxel has the smallest row and every lane offset is >= 0.
  const int64_t row0 = DIRECT ? 0 : window_row(min(m0, S - 1));
  const int64_t abase_off = ((int64_t)b * p.rows_per_batch + row0) * p.row_bytes;
  const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.xp + abase_off), (short)0, (int)min(p.x_bytes - abase_off, (int64_t)0x7fffffff), 0x00020000);
  int aoff[4];
  // DIRECT: per lane and row block, the byte offset of the window origin (the
  // voxel at -1, -1, -1 from the window centre; negative at the low borders)
  // and 9 validity bits: bit t / 3 + t / 6 + t set when origin + t lies inside
  // the volume along d / h / w.
  int lane_off[4];
  unsigned vmask[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    if constexpr (DIRECT) {
      const int v = min(m0 + ms * 16 + lrow, S - 1);
      const int d = v / ghw, r = v - d * ghw;
      const int h = r / p.gw, w = r - h * p.gw;
      const int zi = STRIDE * d - 1, yi = STRIDE * h - 1, xi = STRIDE * w - 1;
      lane_off[ms] = ((zi * p.in_h + yi) * p.in_w + xi) * (int)p.row_bytes + lgrp * 16;
      unsigned m = 0;
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        m |= (unsigned)(zi + t >= 0 && zi + t < p.in_d) << t;
        m |= (unsigned)(yi + t >= 0 && yi + t < p.in_h) << (3 + t);
        m |= (unsigned)(xi + t >= 0 && xi + t < p.in_w) << (6 + t);
      }
      vmask[ms] = m;
      aoff[ms] = 0;
    } else {
      aoff[ms] = (int)((window_row(min(m0 + ms * 16 + lrow, S - 1)) - row0) * p.row_bytes) + lgrp * 16;
    }
  }
  // B: one output column per lane per 16-column block.
  const int n0 = n_tile * (WN * NSUB * 16) + wave_n * (NSUB * 16);
  const int64_t bbase_off = (int64_t)phase * p.taps * p.kb * p.np * 64;
  const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wp + bbase_off), (short)0, (int)min(p.w_bytes - bbase_off, (int64_t)0x7fffffff), 0x00020000);
  int boff[NSUB];
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) boff[ns] = min(n0 + ns * 16 + lrow, p.np - 1) * 64 + lgrp * 16;

  f4 acc[4][NSUB];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] = f4{0.f, 0.f, 0.f, 0.f};

  const int steps = p.taps * p.kb;
  // Wave-uniform (readfirstlane) so the loop counter and the load cursor
  // derived from them stay in SGPRs.
  const int kpart = split_id * SETS + set, kparts = p.split * SETS;
  const int g_begin = (int)((int64_t)kpart * steps / kparts);
  const int g_end = (int)((int64_t)(kpart + 1) * steps / kparts);
  const int s_begin = __builtin_amdgcn_readfirstlane(g_begin + (g_end - g_begin) * wave_k / KWS);
  const int s_end = __builtin_amdgcn_readfirstlane(g_begin + (g_end - g_begin) * (wave_k + 1) / KWS);
  const int bstep = p.np * 64;

  // Load cursor over the step sequence (tap-major, 64-byte channel block
  // minor), advanced incrementally so a step costs a few scalar adds.
  const int rb = (int)p.row_bytes;
  int c_kb, c_tw, c_th, c_td, c_tapoff, c_bo;
  {
    const int tap = s_begin / p.kb;
    c_kb = s_begin - tap * p.kb;
    c_tw = tap % KT;
    c_th = (tap / KT) % KT;
    c_td = tap / (KT * KT);
    c_tapoff = (c_td * p.P + c_th * p.Q + c_tw) * rb;
    c_bo = s_begin * bstep;
  }
  // DIRECT: the lane offsets of the cursor's tap (recomputed when the tap
  // changes): the real row, or 0x80000000 -- past any buffer range -- where the
  // tap leaves the volume.  A prefetch past the last step may test bits of a
  // tap that does not exist; its offset is then a row inside the input or out
  // of range, and the data is never used.
  auto direct_offsets = [&]() {
    if constexpr (DIRECT) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        const unsigned m = vmask[ms];
        const bool in = ((m >> c_td) & (m >> (3 + c_th)) & (m >> (6 + c_tw)) & 1u) != 0;
        aoff[ms] = in ? lane_off[ms] + c_tapoff : (int)0x80000000;
      }
    }
  };
  direct_offsets();
  auto load = [&](u4 (&A)[4], u4 (&B)[NSUB]) {
    // readfirstlane: the step offsets are wave-uniform; saying so keeps them in
    // SGPRs (buffer soffset) instead of a per-lane waterfall.
    const int ao = __builtin_amdgcn_readfirstlane(DIRECT ? c_kb * 64 : c_tapoff + c_kb * 64);
    const int bo = __builtin_amdgcn_readfirstlane(c_bo);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) A[ms] = __builtin_amdgcn_raw_buffer_load_b128(arsrc, aoff[ms], ao, 0);
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) B[ns] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, boff[ns], bo, 0);
    c_bo += bstep;
    if (++c_kb == p.kb) {
      c_kb = 0;
      c_tapoff += rb;
      if (++c_tw == KT) {
        c_tw = 0;
        c_tapoff += (p.Q - KT) * rb;
        if (++c_th == KT) {
          c_th = 0;
          ++c_td;
          c_tapoff += (p.P - KT * p.Q) * rb;
        }
      }
      direct_offsets();
    }
  };
  auto compute = [&](const u4 (&A)[4], const u4 (&B)[NSUB]) { mma_block<DT, NSUB, true>(acc, A, B); };

  // Register double buffer: the next K block is in flight while this one
  // multiplies.  The scheduling barriers keep the prefetch loads ahead of the
  // MFMAs that would otherwise be hoisted above them (the compiler's default
  // order issues the loads after the MFMA burst and exposes their latency).
  //
  // The prefetch loads are unconditional: under a branch the compiler cannot
  // count the loads in flight and waits for all of them (vmcnt(0)) before the
  // current block's MFMAs, i.e. for the prefetch too.  A prefetch past the
  // last step reads through the buffer descriptors -- in range it is data
  // that is never used, out of range the hardware returns zeros -- so it is
  // harmless.
  u4 A0[4], B0[NSUB], A1[4], B1[NSUB];
  load(A0, B0);  // step s_begin; each load() fetches the cursor's step, then advances it
  for (int s = s_begin; s < s_end; s += 2) {
    load(A1, B1);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);  // MFMA bursts win issue slots over address/load code
    compute(A0, B0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 >= s_end) break;
    load(A0, B0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    compute(A1, B1);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int tile_id = UP ? phase * p.m_tiles + m_tile : m_tile;
  auto out_voxel = [&](int v) -> int64_t {
    int o = v;
    if (UP) {
      const int d = v / ghw, rr = v - d * ghw;
      const int h = rr / p.gw, w = rr - h * p.gw;
      o = ((2 * d + pd) * p.oh + 2 * h + ph) * p.ow + 2 * w + pw;
    }
    return (int64_t)b * p.s_out + o;
  };
  auto finish = [&](auto after_bias) {
    f4 bq[NSUB];
    load_bias<NSUB>(p, b, n0, lane, bq);
    store_tile<NSUB, WM, WN, !UP>(p, acc, bq, b, m0, n0, S, split_id, wave, lane, n_tile * (WN * NSUB * 16),
                                  tile_id, out_voxel, after_bias);
  };
  if constexpr (KWS > 1) {
    // Quarters 1..3 of a set hand their sums to the set's wave 0, which adds
    // them in ascending order (with one set and a split: a split partial
    // plane, whose bias, residual and statistics come from the reduction).
    // With two sets, set 1's wave 0 then hands its sum to set 0's (the
    // barriers wait only for the waves still running).
    __shared__ f4 xk[SETS][KWS - 1][4][NSUB][64];
    if (wave_k > 0) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns) xk[set][wave_k - 1][ms][ns][lane] = acc[ms][ns];
    }
    __syncthreads();
    if (wave_k > 0) return;
#pragma unroll
    for (int w = 0; w < KWS - 1; ++w)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] += xk[set][w][ms][ns][lane];
    if constexpr (SETS == 2) {
      if (set == 1) {
#pragma unroll
        for (int ms = 0; ms < 4; ++ms)
#pragma unroll
          for (int ns = 0; ns < NSUB; ++ns) xk[1][0][ms][ns][lane] = acc[ms][ns];
      }
      __syncthreads();
      if (set == 1) return;
      finish([&](f4 (&a)[4][NSUB]) {
#pragma unroll
        for (int ms = 0; ms < 4; ++ms)
#pragma unroll
          for (int ns = 0; ns < NSUB; ++ns) a[ms][ns] += xk[1][0][ms][ns][lane];
      });
    } else {
      finish(NoTerm{});
    }
  } else {
    finish(NoTerm{});
  }
}

// ---------------------------------------------------------------------------
// 3b. LDS-staged implicit GEMM (large stride-1 fp32 volumes)
// ---------------------------------------------------------------------------
// A workgroup owns a 4x8x8 brick of output voxels (256 GEMM rows: wave m holds
// depth m, MFMA row block ms holds brick rows ms and ms+4, lane%16 -> (row
// half, column)) and 64 output channels.  For each 16-channel chunk it
// stages the brick's 6x10x10 halo from the unpadded NDHWC input into LDS --
// zero outside the volume, group-norm affine + SiLU applied on the way, so the
// streaming path's separate pack pass disappears -- then runs all 27 taps with
// A read from LDS at compile-time offsets and B (packed weight) fetched one tap
// ahead through buffer loads.  The next chunk's halo is in flight in registers
// while the current chunk multiplies.  A staged voxel row is 80 bytes (16
// channels + 16 bytes of padding): the 16 rows a 16-lane group reads (8
// columns of brick lines y and y+4, 40 voxels apart) then fall on 16 distinct
// 16-byte bank groups of the 256-byte LDS line -- 5*x + 2*y (mod 16) takes
// every value once over x < 8, y in {y0, y0+4}.
constexpr int kBD = 4, kBH = 8, kBW = 8;
constexpr int kHD = kBD + 2, kHH = kBH + 2, kHW = kBW + 2;
constexpr int kHaloVox = kHD * kHH * kHW;                 // 600
constexpr int kLdsRow = 80;
constexpr int kStageIters = (kHaloVox * 4 + 255) / 256;  // 16-byte pieces per thread


// Epilogue of the brick GEMMs (conv_lds_kernel, conv_lds_bf16_kernel) from
// transposed accumulators: lane l of block (ms, ns) holds voxel (z0 + wave,
// y0 + ms + 4*((l/8)%2), x0 + l%8) of the 4x8x8 brick and output columns
// n0 + ns*16 + 4*(l/16) .. +3 (cout % 64 == 0), stored -- bias first, then the
// residual -- as 16 bytes (`after_bias` adds any term that follows the bias:
// a second K range).  UP: the brick is of the source grid (p.d, p.h,
// p.w) and voxel (z, y, x) of parity `phase` = 4a + 2b + c is output voxel
// (2z + a, 2y + b, 2x + c) of the doubled grid; statistics tiles are
// (brick, parity) pairs.  Group-norm column sums go through `red` (4 KiB of
// LDS, which may alias the kernel's staging buffers: a barrier precedes it).
template <bool UP = false, typename Args, typename AfterBias = NoTerm>
__device__ __forceinline__ void store_brick(const Args& p, f4 (&acc)[4][4], int b, int split_id, int z0, int y0,
                                            int x0, int n0, int wave, int lane, int tile_id,
                                            double (*red)[64][2], int phase = 0, AfterBias after_bias = {}) {
  const int lrow = lane & 15, lgrp = lane >> 4;
  const bool partial = p.split > 1;
  float* out = p.y + (partial ? (int64_t)split_id * p.plane : 0);
  const int z = z0 + wave, x = x0 + (lrow & 7);
  constexpr int S = UP ? 2 : 1;
  const int pa = UP ? phase >> 2 : 0, pb = UP ? (phase >> 1) & 1 : 0, pc = UP ? phase & 1 : 0;
  bool row_ok[4];
  int64_t base[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    const int y = y0 + ms + 4 * (lrow >> 3);
    row_ok[ms] = z < p.d && y < p.h && x < p.w;
    const int oz = S * min(z, p.d - 1) + pa, oy = S * min(y, p.h - 1) + pb, ox = S * min(x, p.w - 1) + pc;
    base[ms] = ((((int64_t)b * (S * p.d) + oz) * (S * p.h) + oy) * (S * p.w) + ox) * p.cout + n0 + 4 * lgrp;
  }
  if (!partial && p.has_bias) {
    const float* bias_b = p.bias + (p.batch_bias ? (int64_t)b * p.cout : 0) + n0 + 4 * lgrp;
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const f4 bq = f4{bias_b[ns * 16], bias_b[ns * 16 + 1], bias_b[ns * 16 + 2], bias_b[ns * 16 + 3]};
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) acc[ms][ns] += bq;
    }
  }
  after_bias(acc);
  if (!partial && p.has_res) {  // every residual load before the first store
    f4 rq[4][4];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) rq[ms][ns] = *reinterpret_cast<const f4*>(p.res + base[ms] + ns * 16);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) acc[ms][ns] += rq[ms][ns];
  }
  {
    // Buffer stores relative to the brick's first output plane (its rows lie
    // within S * 4 planes of it, so the offsets stay 32-bit), with the device-
    // scope cache policy (kStoreSC1).
    const int64_t origin = ((int64_t)b * (S * p.d) + S * min(z0, p.d - 1)) * (S * p.h) * (int64_t)(S * p.w) * p.cout;
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
        out + origin, (short)0, (int)min(max((int64_t)p.plane - origin, (int64_t)0) * 4, (int64_t)0x7fffffff),
        0x00020000);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns)
        if (row_ok[ms])
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[ms][ns]), ors,
                                                 (int)((base[ms] - origin + ns * 16) * 4), 0, kStoreSC1);
  }
  if (p.stats) {  // a kernel argument: every thread reaches the barriers
    __syncthreads();
    const bool col_ok[4] = {true, true, true, true};
    column_sums<4>(acc, row_ok, col_ok, red, wave, lane);
    __syncthreads();
    combine_gn_partials<4, 4, 1>(red, n0, p.cout, p.gn_cpg, p.gn_groups,
                                 p.stats + ((int64_t)b * p.tz * p.ty * p.tx * S * S * S + tile_id) * p.gn_groups * 2);
  }
}

struct LdsArgs {
  const float* x;       // unpadded NDHWC input (channels [0, c1) of a two-source input)
  const float* x2;      // channels [c1, cin) of a two-source input, or null
  int c1;               // channels of x (cin for one source; a multiple of 16)
  const float* affine;  // (n, cin, 2) or null
  const char* wp;       // packed weight [tap][kblock][np][64 bytes]
  const float* bias;
  const float* res;
  float* y;             // output, or split partial planes
  int64_t x_bytes, w_bytes, plane;
  int n, d, h, w, cin, cout, np, kb;
  int tz, ty, tx;       // bricks per axis
  int n_tiles, split;
  int affine_on, silu_on, batch_bias, has_res, has_bias;
  double* stats;        // group-norm partials of the output (ctmr_conv3d_gn) or null
  int gn_groups, gn_cpg;
};

// TWO: the input is two tensors (ctmr_conv3d_cat); the one-tensor kernel keeps
// precomputed byte offsets and a single descriptor.  XF: the staging
// transform, bit 0 the GN affine and bit 1 SiLU (p.affine_on, p.silu_on), as
// template flags so the transform is branch-free code.  WS = 2: a K split of
// two ranges inside the workgroup -- wave set s (waves 4s .. 4s + 3, each set
// with its own halo buffer) runs the chunks of range s of one brick, and set
// 0 adds set 1's sums after the bias, the order of the split reduction
// (bias, range 0, range 1, residual), with no partial planes in memory.
template <bool TWO, int XF, int WS>
__global__ __launch_bounds__(256 * WS, WS == 1 ? 2 : 1) void conv_lds_kernel(LdsArgs p) {
  static_assert(WS == 1 || WS == 2, "one or two wave sets");
  __shared__ __attribute__((aligned(16))) char lds_sets[WS * kHaloVox * kLdsRow];
  const int set = WS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
  char* const lds = lds_sets + set * (kHaloVox * kLdsRow);
  const int tid = threadIdx.x & 255, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware order (as conv_kernel): neighbouring bricks share halo planes.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot = bid >> 3, per = nb >> 3, rem = nb & 7;
  const int tile = (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = tile % p.n_tiles;
  int rest = tile / p.n_tiles;
  const int bx = rest % p.tx;
  rest /= p.tx;
  const int by = rest % p.ty;
  rest /= p.ty;
  const int bz = rest % p.tz;
  rest /= p.tz;
  const int b = rest % p.n;
  const int split_id = rest / p.n;
  const int z0 = bz * kBD, y0 = by * kBH, x0 = bx * kBW;
  const int lrow = lane & 15, lgrp = lane >> 4;

  // Staging: piece i of thread t is channels 4*(t&3)..+3 of the chunk at halo
  // voxel (t>>2) + 64i.  Offsets are relative to the first staged plane, so
  // they stay within 32 bits (the host checks 6 planes fit).  goff[i] is the
  // piece's byte offset; with TWO it is the piece's voxel index instead: a
  // chunk comes from x (chunks below c1 / 16) or from x2, whose rows hold the
  // remaining channels, and the byte offset follows from the chunk's source.
  const int part = tid & 3;
  const int zb = max(z0 - 1, 0);
  const int c2 = p.cin - p.c1;
  const int kb1 = p.c1 >> 4;
  const int64_t vbase = ((int64_t)b * p.d + zb) * p.h * p.w;     // first staged voxel
  const int64_t vtotal = (int64_t)p.n * p.d * p.h * p.w;
  const __amdgpu_buffer_rsrc_t xrsrc1 = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + vbase * p.c1), (short)0, (int)min((vtotal - vbase) * p.c1 * 4, (int64_t)0x7fffffff),
      0x00020000);
  const __amdgpu_buffer_rsrc_t xrsrc2 = TWO ? __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x2 + vbase * c2), (short)0, (int)min((vtotal - vbase) * c2 * 4, (int64_t)0x7fffffff),
      0x00020000) : xrsrc1;
  int goff[kStageIters];
  unsigned valid = 0;
#pragma unroll
  for (int i = 0; i < kStageIters; ++i) {
    const int hv = (tid >> 2) + 64 * i;
    goff[i] = 0;
    if (hv < kHaloVox) {
      const int hz = hv / (kHH * kHW), hr = hv - hz * (kHH * kHW);
      const int hy = hr / kHW, hx = hr - hy * kHW;
      const int gz = z0 - 1 + hz, gy = y0 - 1 + hy, gx = x0 - 1 + hx;
      if (gz >= 0 && gz < p.d && gy >= 0 && gy < p.h && gx >= 0 && gx < p.w) {
        valid |= 1u << i;
        const int vox = ((gz - zb) * p.h + gy) * p.w + gx;
        goff[i] = TWO ? vox : vox * p.cin * 4 + part * 16;
      }
    }
  }
  // Source of a chunk: descriptor, row bytes (TWO) and the chunk's byte offset in a row.
  struct ChunkSrc {
    __amdgpu_buffer_rsrc_t rs;
    int row, so;
  };
  auto chunk_src = [&](int chunk) {
    ChunkSrc c;
    const bool second = TWO && chunk >= kb1;
    c.rs = second ? xrsrc2 : xrsrc1;
    c.row = (second ? c2 : p.c1) * 4;
    c.so = __builtin_amdgcn_readfirstlane((second ? chunk - kb1 : chunk) * 64);
    return c;
  };
  auto piece_off = [&](int i, const ChunkSrc& c) { return TWO ? goff[i] * c.row + part * 16 : goff[i]; };

  // A: LDS byte address of this lane's voxel at tap (0,0,0) per row block.
  int abase[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
    abase[ms] = ((wave * kHH + ms + 4 * (lrow >> 3)) * kHW + (lrow & 7)) * kLdsRow + lgrp * 16;
  // B: one output column per lane per 16-column block.
  const int n0 = n_tile * 64;
  const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wp, (short)0, (int)min(p.w_bytes, (int64_t)0x7fffffff), 0x00020000);
  int boff[4];
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) boff[ns] = min(n0 + ns * 16 + lrow, p.np - 1) * 64 + lgrp * 16;
  const int bchunk = p.np * 64;

  f4 acc[4][4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = f4{0.f, 0.f, 0.f, 0.f};

  const int kpart = split_id * WS + set, kparts = p.split * WS;
  const int c_begin = __builtin_amdgcn_readfirstlane((int)((int64_t)kpart * p.kb / kparts));
  const int c_end = __builtin_amdgcn_readfirstlane((int)((int64_t)(kpart + 1) * p.kb / kparts));

  u4 stage[kStageIters];
  auto fetch = [&](int chunk) {
    const ChunkSrc c = chunk_src(chunk);
#pragma unroll
    for (int i = 0; i < kStageIters; ++i)
      stage[i] = __builtin_amdgcn_raw_buffer_load_b128(c.rs, piece_off(i, c), c.so, 0);
  };
  // GN affine of this thread's four channels of a chunk: (scale, offset) pairs.
  auto load_affine = [&](int chunk, f4& sc, f4& of) {
    sc = f4{1.f, 1.f, 1.f, 1.f};
    of = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr ((XF & 1) != 0) {
      const f4* q = reinterpret_cast<const f4*>(p.affine + ((int64_t)b * p.cin + chunk * 16 + part * 4) * 2);
      const f4 a0 = q[0], a1 = q[1];
      sc = f4{a0[0], a0[2], a1[0], a1[2]};
      of = f4{a0[1], a0[3], a1[1], a1[3]};
    }
  };
  // Piece i as staged: GN affine, SiLU, zero outside the volume.
  auto transform = [&](int i, const f4& sc, const f4& of) {
    f4 v = __builtin_bit_cast(f4, stage[i]);
    const bool in = (valid >> i) & 1u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t = v[j];
      if constexpr ((XF & 1) != 0) t = fmaf(t, sc[j], of[j]);
      if constexpr ((XF & 2) != 0) t = silu_f(t);
      v[j] = in ? t : 0.f;
    }
    stage[i] = __builtin_bit_cast(u4, v);
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < kStageIters; ++i) {
      const int hv = (tid >> 2) + 64 * i;
      if (hv >= kHaloVox) continue;
      *reinterpret_cast<u4*>(lds + hv * kLdsRow + part * 16) = stage[i];
    }
  };
  auto load_a = [&](f4 (&A)[4], int tap) {
    const int off = (((tap / 9) * kHH + (tap / 3) % 3) * kHW + tap % 3) * kLdsRow;
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) A[ms] = *reinterpret_cast<const f4*>(lds + abase[ms] + off);
  };
  auto load_b = [&](u4 (&B)[4], int tap, int chunk) {
    const int so = __builtin_amdgcn_readfirstlane((tap * p.kb + chunk) * bchunk);
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) B[ns] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, boff[ns], so, 0);
  };
  auto mma = [&](const f4 (&A)[4], const u4 (&B)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns)
          acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(f4, B[ns])[j], A[ms][j],
                                                             acc[ms][ns], 0, 0, 0);  // B^T A^T: see store_brick
  };

  // Without affine or SiLU the staging transform is the zero mask alone: it
  // runs inside the previous chunk's tap loop, among the MFMAs, and the
  // commit between the barriers only writes LDS (config 0: 409-412 -> 405-406
  // us).  With affine + SiLU the same placement measured ~1 % slower than
  // transforming at the commit, which those variants keep.
  constexpr bool kInLoop = XF == 0;
  fetch(c_begin);
  if constexpr (kInLoop) {
    f4 sc, of;
    load_affine(c_begin, sc, of);
#pragma unroll
    for (int i = 0; i < kStageIters; ++i) transform(i, sc, of);
  }
  for (int chunk = c_begin; chunk < c_end; ++chunk) {
    __syncthreads();  // every wave has finished reading the previous chunk
    if constexpr (!kInLoop) {
      f4 sc, of;
      load_affine(chunk, sc, of);
#pragma unroll
      for (int i = 0; i < kStageIters; ++i) transform(i, sc, of);
    }
    commit();
    __syncthreads();
    f4 A[2][4];
    u4 B[2][4];
    load_b(B[0], 0, chunk);
    load_a(A[0], 0);
    // Unconditional (see conv_kernel): the last chunk re-reads itself.
    const int next = min(chunk + 1, c_end - 1);
    const ChunkSrc nx = chunk_src(next);
    f4 nsc, nof;
    load_affine(next, nsc, nof);
#pragma unroll
    for (int t = 0; t < 27; ++t) {
      if (t + 1 < 27) {
        load_b(B[(t + 1) & 1], t + 1, chunk);
        load_a(A[(t + 1) & 1], t + 1);
      }
      // The next chunk's halo, one 16-byte piece every other tap: loads
      // retire in order, so each piece has two taps of products to arrive
      // before a later weight load has to wait for it.
      if ((t & 1) && (t >> 1) < kStageIters)
        stage[t >> 1] = __builtin_amdgcn_raw_buffer_load_b128(nx.rs, piece_off(t >> 1, nx), nx.so, 0);
      __builtin_amdgcn_sched_barrier(0);
      // Raised priority while this wave's MFMAs issue, so a wave whose
      // operands are ready wins issue slots over waves in their staging code.
      __builtin_amdgcn_s_setprio(1);
      mma(A[t & 1], B[t & 1]);
      // Piece i, loaded at tap 2i + 1, is masked at tap 2i + 6.
      if (kInLoop && t >= 6 && !(t & 1) && ((t - 6) >> 1) < kStageIters) {
        transform((t - 6) >> 1, nsc, nof);
      }
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  __shared__ double red[4][64][2];
  const int tile_id = (bz * p.ty + by) * p.tx + bx;
  if constexpr (WS == 2) {
    // Set 1 hands its sums to set 0 through the halo buffers (64 KiB of the
    // 2 x 47 KiB) once every wave has finished reading them, then ends; the
    // barriers after that wait only for set 0's waves.
    f4* const xs = reinterpret_cast<f4*>(lds_sets);
    __syncthreads();
    if (set == 1) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) xs[(wave * 16 + ms * 4 + ns) * 64 + lane] = acc[ms][ns];
    }
    __syncthreads();
    if (set == 1) return;
    store_brick(p, acc, b, split_id, z0, y0, x0, n0, wave, lane, tile_id, red, 0, [&](f4 (&a)[4][4]) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) a[ms][ns] += xs[(wave * 16 + ms * 4 + ns) * 64 + lane];
    });
  } else {
    store_brick(p, acc, b, split_id, z0, y0, x0, n0, wave, lane, tile_id, red);
  }
}

// ---------------------------------------------------------------------------
// 3b''. Direct conv for cout <= 4 (fp32, stride 1, cin a multiple of 16: the
// 64 -> 4 UNet and 64 -> 1 VAE output convs)
// ---------------------------------------------------------------------------
// A 16-column MFMA tile would idle 12-15 of its columns here, and the
// tap-expanded GEMM pays a padded copy, 27 * cout columns of scratch and a tap
// sum.  Instead each thread owns one output voxel of a 4x8x8 brick and
// accumulates its cout outputs with FMAs: per 16-channel chunk the brick's
// 6x10x10 halo is staged in LDS with the group-norm affine and SiLU applied
// (as conv_lds_kernel; the next chunk's halo is loaded during this chunk's
// products), and the thread reads its 27 neighbours' 16 channels as four
// 16-byte pieces.  Weights come from the tap-expanded packing (column
// tap * cout + o, 16 channels per K block) with workgroup-uniform addresses.
// Summation order per output: chunks ascending, taps ascending, channels
// ascending, then the bias -- fixed for a given shape.
// Halo voxel v stores piece g at slot g ^ small_halo_swizzle(v): the reads of
// a wave (8 x 8 voxels of one plane, one piece) then fall on twice fewer
// conflicted bank groups than unswizzled (exhaustive check over taps under
// the gfx950 ds_read_b128 service order), and the staging writes stay
// conflict-free.
struct SmallOutArgs {
  const float* x;       // unpadded NDHWC input (channels [0, c1) of a two-source input)
  const float* x2;      // channels [c1, cin) of a two-source input, or null
  int c1;               // channels of x (cin for one source; a multiple of 16)
  const float* affine;  // (n, cin, 2) or null
  const float* wp;      // tap-expanded packed weight [kblock][np][16 floats]
  const float* bias;    // (cout) or null
  float* y;
  int n, d, h, w, cin, np, kb;
  int tz, ty, tx;
};

__host__ __device__ constexpr int small_halo_swizzle(int v) { return (v ^ (v >> 3)) & 3; }

template <int COUT, bool AFF, bool SILU>
__global__ __launch_bounds__(256, 2) void conv_small_cout_kernel(SmallOutArgs p) {
  __shared__ __attribute__((aligned(16))) char lds[kHaloVox * 64];
  const int tid = threadIdx.x;
  // XCD-aware brick order (as conv_lds_kernel).  On wide planes (at least 256
  // bricks per brick plane, the decoder's 256x256 output conv) depth
  // neighbours are adjacent instead of x neighbours: in x order a brick's
  // depth neighbour runs a whole brick plane later, long after its halo planes
  // left the XCD's L2 (measured on 80x256x256, 64 -> 1: 3.54 GB fetched for a
  // 1.34 GB input in x order, 2.35 GB depth-first; on the UNet's 64x64x32 the
  // x order's compact blocks fetch less, 95 against 145 MB).
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot = bid >> 3, per = nb >> 3, rem = nb & 7;
  int rest = (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  int bx, by, bz;
  if (p.tx * p.ty >= 256) {  // uniform: kernel arguments
    bz = rest % p.tz;
    rest /= p.tz;
    bx = rest % p.tx;
    rest /= p.tx;
    by = rest % p.ty;
    rest /= p.ty;
  } else {
    bx = rest % p.tx;
    rest /= p.tx;
    by = rest % p.ty;
    rest /= p.ty;
    bz = rest % p.tz;
    rest /= p.tz;
  }
  const int b = rest;
  const int z0 = bz * kBD, y0 = by * kBH, x0 = bx * kBW;

  // Staging: piece i of thread t is channels 4*(t&3)..+3 of the chunk at halo
  // voxel (t>>2) + 64i; goff[i] is that voxel's index relative to the first
  // staged plane.  A chunk comes from x (chunks below c1 / 16) or from x2,
  // whose rows hold the remaining channels.
  const int part = tid & 3;
  const int zb = max(z0 - 1, 0);
  const int c2 = p.cin - p.c1, kb1 = p.c1 >> 4;
  const int64_t vbase = ((int64_t)b * p.d + zb) * p.h * p.w;
  const int64_t vtotal = (int64_t)p.n * p.d * p.h * p.w;
  const __amdgpu_buffer_rsrc_t xrsrc1 = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + vbase * p.c1), (short)0, (int)min((vtotal - vbase) * p.c1 * 4, (int64_t)0x7fffffff),
      0x00020000);
  const __amdgpu_buffer_rsrc_t xrsrc2 = p.x2 ? __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x2 + vbase * c2), (short)0, (int)min((vtotal - vbase) * c2 * 4, (int64_t)0x7fffffff),
      0x00020000) : xrsrc1;
  int goff[kStageIters];
  unsigned valid = 0;
#pragma unroll
  for (int i = 0; i < kStageIters; ++i) {
    const int hv = (tid >> 2) + 64 * i;
    goff[i] = 0;
    if (hv < kHaloVox) {
      const int hz = hv / (kHH * kHW), hr = hv - hz * (kHH * kHW);
      const int hy = hr / kHW, hx = hr - hy * kHW;
      const int gz = z0 - 1 + hz, gy = y0 - 1 + hy, gx = x0 - 1 + hx;
      if (gz >= 0 && gz < p.d && gy >= 0 && gy < p.h && gx >= 0 && gx < p.w) {
        valid |= 1u << i;
        goff[i] = ((gz - zb) * p.h + gy) * p.w + gx;
      }
    }
  }
  u4 stage[kStageIters];
  auto fetch = [&](int chunk) {
    const bool second = p.x2 != nullptr && chunk >= kb1;  // uniform
    const __amdgpu_buffer_rsrc_t rs = second ? xrsrc2 : xrsrc1;
    const int row = (second ? c2 : p.c1) * 4;
    const int so = __builtin_amdgcn_readfirstlane((second ? chunk - kb1 : chunk) * 64);
#pragma unroll
    for (int i = 0; i < kStageIters; ++i)
      stage[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, goff[i] * row + part * 16, so, 0);
  };
  auto commit = [&](int chunk) {
    f4 sc = {1.f, 1.f, 1.f, 1.f}, of = {0.f, 0.f, 0.f, 0.f};
    if constexpr (AFF) {
      const f4* q = reinterpret_cast<const f4*>(p.affine + ((int64_t)b * p.cin + chunk * 16 + part * 4) * 2);
      const f4 a0 = q[0], a1 = q[1];
      sc = f4{a0[0], a0[2], a1[0], a1[2]};
      of = f4{a0[1], a0[3], a1[1], a1[3]};
    }
#pragma unroll
    for (int i = 0; i < kStageIters; ++i) {
      const int hv = (tid >> 2) + 64 * i;
      if (hv >= kHaloVox) continue;
      f4 v = __builtin_bit_cast(f4, stage[i]);
      const bool in = (valid >> i) & 1u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float t = v[j];
        if constexpr (AFF) t = fmaf(t, sc[j], of[j]);
        if constexpr (SILU) t = silu_f(t);
        v[j] = in ? t : 0.f;
      }
      *reinterpret_cast<f4*>(lds + hv * 64 + ((part ^ small_halo_swizzle(hv)) << 4)) = v;
    }
  };

  // This thread's output voxel and its halo voxel at tap (0,0,0); the swizzle
  // depends on a voxel's bits 0, 1, 3 and 4 only, so the slot base of the
  // voxel at tap offset `off` is entry off % 32 of a two-word table.
  const int oz = tid >> 6, oy = (tid >> 3) & 7, ox = tid & 7;
  const int hv0 = (oz * kHH + oy) * kHW + ox;
  unsigned tab[2] = {0u, 0u};
#pragma unroll
  for (int k = 0; k < 32; ++k) tab[k >> 4] |= (unsigned)small_halo_swizzle(hv0 + k) << (2 * (k & 15));

  float acc[COUT];
#pragma unroll
  for (int o = 0; o < COUT; ++o) acc[o] = 0.f;
  fetch(0);
  for (int chunk = 0; chunk < p.kb; ++chunk) {
    __syncthreads();  // every thread has finished reading the previous chunk
    commit(chunk);
    __syncthreads();
    if (chunk + 1 < p.kb) fetch(chunk + 1);  // uniform; lands during this chunk's products
    int base = hv0 * 64;
    unsigned t0 = tab[0], t1 = tab[1];
    // Keeps the per-tap address arithmetic inside the chunk loop.
    asm volatile("" : "+v"(base), "+v"(t0), "+v"(t1));
    // The constant address space: uniform weight reads become scalar loads.
    const __attribute__((address_space(4))) float* wc =
        (const __attribute__((address_space(4))) float*)(p.wp + (int64_t)chunk * p.np * 16);
#pragma unroll
    for (int tap = 0; tap < 27; ++tap) {
      const int off = ((tap / 9) * kHH + (tap / 3) % 3) * kHW + tap % 3;
      const int k = off & 31;
      const unsigned sw = ((k < 16 ? t0 : t1) >> (2 * (k & 15))) & 3u;
#pragma unroll
      for (int pc = 0; pc < 4; ++pc) {
        const f4 a = *reinterpret_cast<const f4*>(lds + base + off * 64 + (int)((pc ^ sw) << 4));
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int o = 0; o < COUT; ++o) acc[o] = fmaf(a[j], wc[(tap * COUT + o) * 16 + pc * 4 + j], acc[o]);
      }
    }
  }
  const int z = z0 + oz, y = y0 + oy, x = x0 + ox;
  if (z < p.d && y < p.h && x < p.w) {
    float* out = p.y + ((((int64_t)b * p.d + z) * p.h + y) * p.w + x) * COUT;
#pragma unroll
    for (int o = 0; o < COUT; ++o) out[o] = acc[o] + (p.bias ? p.bias[o] : 0.f);
  }
}

// ---------------------------------------------------------------------------
// 3b'. LDS-staged im2col GEMM for small channel counts (fp32, stride 1, cin 4
// or 8: the 4-channel latent input convs, the 8-channel label-condition convs)
// ---------------------------------------------------------------------------
// The im2col formulation (K = tap * cin + c, blocks of 16, the packed weight of
// WL_IM2COL) without its HBM rows: a workgroup stages the brick's 6x10x10 halo
// with all cin channels (plus a zero slot) in LDS once, then each K block's A
// fragment is read straight from the halo -- lane group g of block b takes
// K 16b + 4g .. +3, four consecutive channels of one tap of one voxel, or the
// zero slot past tap 26.  Same operands, same K blocks in the same order and
// the same MFMA sequence as the im2col GEMMs (B^T A^T, fixed order), so the
// outputs are bit-identical to them.  Bricks and the wave / row mapping are
// those of conv_lds_kernel; B (the weight) comes from L2 one block ahead.
struct LdsSmallArgs {
  const float* x;       // unpadded NDHWC input, cin channels
  const float* affine;  // (n, cin, 2) or null
  const char* wp;       // packed im2col weight [kblock][np][64 bytes]
  const float* bias;
  const float* res;
  float* y;
  int64_t x_bytes, w_bytes, plane;
  int n, d, h, w, cin, cout, np, kb;
  int tz, ty, tx, n_tiles, split;
  int affine_on, silu_on, batch_bias, has_res, has_bias;
  double* stats;
  int gn_groups, gn_cpg;
};

template <int CIN, int NSUB>
__global__ __launch_bounds__(256, 2) void conv_lds_small_kernel(LdsSmallArgs p) {
  static_assert(CIN == 4 || CIN == 8, "4 or 8 input channels");
  constexpr int kVox = CIN * 4;                      // bytes per halo voxel
  constexpr int kQuads = kHaloVox * (CIN / 4);       // 16-byte halo pieces
  constexpr int kIters = (kQuads + 255) / 256;
  constexpr int kZero = kHaloVox * kVox;             // a 16-byte zero slot after the halo
  constexpr int KB = (27 * CIN + 15) / 16;           // K blocks
  __shared__ __attribute__((aligned(16))) char halo[kZero + 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot = bid >> 3, per = nb >> 3, rem = nb & 7;
  const int tile = (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = tile % p.n_tiles;
  int rest = tile / p.n_tiles;
  const int bx = rest % p.tx;
  rest /= p.tx;
  const int by = rest % p.ty;
  rest /= p.ty;
  const int bz = rest % p.tz;
  const int b = rest / p.tz;
  const int z0 = bz * kBD, y0 = by * kBH, x0 = bx * kBW;
  const int lrow = lane & 15, lgrp = lane >> 4;

  // B: one output column per lane per 16-column block, from the block's rows
  // of the packed weight; the first block's loads go out before the staging.
  const int n0 = n_tile * NSUB * 16;
  const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wp, (short)0, (int)min(p.w_bytes, (int64_t)0x7fffffff), 0x00020000);
  int boff[NSUB];
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) boff[ns] = min(n0 + ns * 16 + lrow, p.np - 1) * 64 + lgrp * 16;
  const int bblock = p.np * 64;
  auto load_b = [&](u4 (&B)[NSUB], int kblock) {
    const int so = __builtin_amdgcn_readfirstlane(kblock * bblock);
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) B[ns] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, boff[ns], so, 0);
  };
  u4 B[2][NSUB];
  load_b(B[0], 0);

  // Halo: piece q is channels 4 (q % (CIN/4)) .. +3 of halo voxel q / (CIN/4);
  // outside the volume it is zero (after the affine and SiLU, as the padding of
  // the reference's pack kernel).  Offsets are relative to the first staged
  // plane (the host checks 6 planes fit 31 bits).
  const int zb = max(z0 - 1, 0);
  const int64_t xbase = ((int64_t)b * p.d + zb) * p.h * p.w * CIN * 4;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)p.x + xbase), (short)0, (int)min(p.x_bytes - xbase, (int64_t)0x7fffffff),
      0x00020000);
  u4 stage[kIters];
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int q = tid + 256 * i;
    stage[i] = u4{0u, 0u, 0u, 0u};
    if (q < kQuads) {
      const int hv = q / (CIN / 4), part = q % (CIN / 4);
      const int hz = hv / (kHH * kHW), hr = hv - hz * (kHH * kHW);
      const int hy = hr / kHW, hx = hr - hy * kHW;
      const int gz = z0 - 1 + hz, gy = y0 - 1 + hy, gx = x0 - 1 + hx;
      if (gz >= 0 && gz < p.d && gy >= 0 && gy < p.h && gx >= 0 && gx < p.w) {
        const int off = (int)((((int64_t)(gz - zb) * p.h + gy) * p.w + gx) * CIN * 4) + part * 16;
        f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
        if (p.affine_on) {
          const f4* a = reinterpret_cast<const f4*>(p.affine + ((int64_t)b * CIN + part * 4) * 2);
          const f4 a0 = a[0], a1 = a[1];
          v = f4{fmaf(v[0], a0[0], a0[1]), fmaf(v[1], a0[2], a0[3]), fmaf(v[2], a1[0], a1[1]),
                 fmaf(v[3], a1[2], a1[3])};
        }
        if (p.silu_on) {
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = silu_f(v[j]);
        }
        stage[i] = __builtin_bit_cast(u4, v);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int q = tid + 256 * i;
    if (q < kQuads) *reinterpret_cast<u4*>(halo + (q / (CIN / 4)) * kVox + (q % (CIN / 4)) * 16) = stage[i];
  }
  if (tid == 0) *reinterpret_cast<u4*>(halo + kZero) = u4{0u, 0u, 0u, 0u};
  __syncthreads();

  // A: this lane's voxel at tap (0,0,0) per row block (rows as conv_lds_kernel).
  int abase[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) abase[ms] = ((wave * kHH + ms + 4 * (lrow >> 3)) * kHW + (lrow & 7)) * kVox;
  auto load_a = [&](f4 (&A)[4], int kblock) {
    const int k0 = kblock * 16 + lgrp * 4;
    const int tap = k0 / CIN, c0 = k0 - tap * CIN;
    const int off = (((tap / 9) * kHH + (tap / 3) % 3) * kHW + tap % 3) * kVox + c0 * 4;
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
      A[ms] = *reinterpret_cast<const f4*>(halo + (tap < 27 ? abase[ms] + off : kZero));
  };

  f4 acc[4][NSUB];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] = f4{0.f, 0.f, 0.f, 0.f};
  f4 A[2][4];
  load_a(A[0], 0);
#pragma unroll
  for (int kbk = 0; kbk < KB; ++kbk) {
    if (kbk + 1 < KB) {
      load_b(B[(kbk + 1) & 1], kbk + 1);
      load_a(A[(kbk + 1) & 1], kbk + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns)
          acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(f4, B[kbk & 1][ns])[j],
                                                             A[kbk & 1][ms][j], acc[ms][ns], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (NSUB == 4) {
    __shared__ double red[4][64][2];
    store_brick(p, acc, b, 0, z0, y0, x0, n0, wave, lane, (bz * p.ty + by) * p.tx + bx, red);
  } else {
    // Narrow outputs (cout <= 32): lane holds columns n0 + 16 ns + 4 lgrp .. +3
    // (all valid or all past cout: cout is a multiple of 4); no statistics.
    const int z = z0 + wave, x = x0 + (lrow & 7);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) {
      const int y = y0 + ms + 4 * (lrow >> 3);
      if (!(z < p.d && y < p.h && x < p.w)) continue;
      const int64_t base = ((((int64_t)b * p.d + z) * p.h + y) * p.w + x) * p.cout;
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) {
        const int col = n0 + ns * 16 + 4 * lgrp;
        if (col >= p.cout) continue;
        f4 v = acc[ms][ns];
        if (p.has_bias) {
          const float* bq = p.bias + (p.batch_bias ? (int64_t)b * p.cout : 0) + col;
          v += f4{bq[0], bq[1], bq[2], bq[3]};
        }
        if (p.has_res) v += *reinterpret_cast<const f4*>(p.res + base + col);
        *reinterpret_cast<f4*>(p.y + base + col) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3c. LDS-staged bf16 implicit GEMM (stride-1 bf16 volumes)
// ---------------------------------------------------------------------------
// The bf16 MFMA (16x16x32, 16 cycles) consumes operands 8x faster per cycle
// than the fp32 one, more than the texture path can feed from L2 (the
// register-streaming bf16 GEMM saturates it at ~15 % of the bf16 peak).  Here
// both operands come from LDS, filled by direct-to-LDS buffer loads (no
// register staging): per 32-channel chunk the 6x10x10 halo of a 4x8x8 output
// brick from the bf16 packed copy (already zero-padded, affine + SiLU or the
// trilinear sample applied by the pack), and per tap row (kd, kh) the three
// taps' 64-column weight tiles, double buffered two rows ahead.  A lane's
// 16-byte slot s of a fill lands at LDS byte 16 s, so a voxel's (a column's)
// 64 bytes -- its four 16-byte K pieces, channels 8g..8g+7 of the chunk --
// arrive from four consecutive lanes reading one 64-byte line.
// Bank layout.  A ds_read_b128 is served in four cycles of 16 lanes, the
// lanes with equal bit 5 and equal parity of bits 2-4 of the lane id (fitted,
// as the only such lane partition consistent with all of them, to 15 address
// patterns timed on MI355X with the LDS bank-conflict counter), at the full
// 256 bytes/clock only if those 16 lanes hit distinct 16-byte bank groups
// (address bits 4-7).  With 64-byte rows the group of row v, slot s is
// (4 v + s) mod 16: lanes 0-1 of a row index give four different 4 v, and the
// four lanes of a cycle that share them differ in (row bit 2, row bit 3) for
// B (K piece bit 0 is fixed by the parity) and in (brick column bit 2, brick
// line bit 2) for A (MFMA rows 8-15 are brick line y + 4, 40 voxels on: the
// same 4 v).  The fills therefore store piece g at slot g ^ f with f = 3 *
// bit 3 of the column (B: slot bit 0 = g0 ^ bit 3 follows bit 2 through the
// parity, slot bit 1 = g1 ^ bit 3) or f = (bit 2 of the halo line) << 1 (A:
// slot bit 0 = g0 follows the column bit, slot bit 1 the line bit), which
// gives those four lanes the four slots of their group at every tap.
// Tiles, wave layout and epilogue are those of conv_lds_kernel.
constexpr int kB16HaloBytes = kHaloVox * 64;                 // 38400
constexpr int kB16HaloSlots = kHaloVox * 4;                  // 2400
constexpr int kB16HaloIters = (kB16HaloSlots + 255) / 256;   // 10
constexpr int kB16TapBytes = 64 * 64;                        // one tap's 64 columns

// Split fp16 (CTMR_F16X2) on the same GEMM.  A K block is 16 input channels
// whose packed voxel holds [hi 0..15 | lo 0..15] (64 bytes, as a bf16 chunk),
// so the halo fill and the A reads are the bf16 ones; lane group g (K 8g ..
// 8g + 7 of the MFMA) reads hi 0..7, hi 8..15, lo 0..7, lo 8..15.  A packed
// weight column holds 96 bytes per K block: Bh = [hi | hi * 2^-11] (64 bytes,
// laid out and swizzled like a bf16 column) and Bl = [lo] (32 bytes; lane
// groups 2 and 3 read a zeroed 16-byte slot instead).  Per (tap, row block,
// column block) two MFMAs: Bh^T A^T adds hi*hi + (lo * 2^11)(hi * 2^-11), Bl^T
// A^T adds lo*hi -- every product of the split but the 2^-22-relative lo*lo.
// In LDS a tap is 384 16-byte slots (Bh 256, Bl 128) followed by a zeroed
// 16-byte slot, which lane groups 2 and 3 read for Bl at the same tap offset
// as groups 0 and 1 (so a Bl address is one register per column block, as for
// Bh).  A fill wave writes 64 consecutive slots, and 384 = 6 * 64, so no
// wave's slots straddle a tap: wave block q of a row lands at slot 64 q +
// q / 6.  4.5 fill iterations per three-tap row, exactly 3 per two-tap
// nearest-2x row.  Bl rows of 32 bytes need no swizzle: under the
// ds_read_b128 service order (four cycles of 16 lanes, equal bit 5 and equal
// parity of bits 2-4) a cycle's lanes of groups 0 and 1 hit 16 distinct bank
// groups 2 * column + piece (mod 16), and groups 2 and 3 read one zero slot.
constexpr int kF2TapBytes = 385 * 16;                        // 6160: Bh, Bl, zero slot
constexpr int kF2BlOff = 256 * 16;                           // Bl after the tap's Bh
constexpr int kF2ZeroOff = 384 * 16;                         // the tap's zero slot

template <int DT>
struct Lds16Cfg {
  static constexpr int tap_bytes = DT == CTMR_F16X2 ? kF2TapBytes : kB16TapBytes;  // LDS bytes per tap
  static constexpr int row_bytes = 3 * tap_bytes;
  static constexpr int col_bytes = DT == CTMR_F16X2 ? 96 : 64;                     // packed bytes per column
  static constexpr int row_iters = DT == CTMR_F16X2 ? 5 : 3;                       // fill iterations per row
};

__host__ __device__ constexpr int lds16_halo_swizzle(int hy) { return ((hy >> 2) & 1) << 1; }
__host__ __device__ constexpr int row64_swizzle(int c) { return ((c >> 3) & 1) * 3; }

struct Lds16Args {
  const char* xp;       // bf16 / split-fp16 packed copy (n, d+2, h+2, w+2, cp)
  const char* wp;       // packed weight [tap][kblock][np][64 or 96 bytes]
  const float* bias;
  const float* res;
  float* y;             // output, or split partial planes
  int64_t x_bytes, w_bytes, plane, rows_per_batch;
  int d, h, w;          // output grid = packed interior
  int P, Q;             // padded plane / row pitch in voxels
  int vbytes;           // bytes per packed voxel (cp * 2 bf16, cp * 4 split fp16)
  int cout, np, kb, n;
  int tz, ty, tx, n_tiles, split;
  int batch_bias, has_res, has_bias;
  double* stats;
  int gn_groups, gn_cpg;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Direct-to-LDS 16-byte load of lane i into LDS byte `lds_addr + 16 i` (a
// wave-uniform address).  Written as inline assembly because the compiler
// cannot tell this LDS target apart from the buffers being read meanwhile and
// would wait for the load before every following ds_read; callers wait for
// it themselves (s_waitcnt vmcnt(0) before the barrier that publishes it).
__device__ __forceinline__ void lds_dma16(const void* gptr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(gptr)
               : "memory", "m0");
}

// Operand fragments of one tap: A (4 row blocks), B (4 column blocks) and,
// for split fp16, the Bl column blocks.
struct Lds16Frag {
  u4 a[4], b[4], c[4];
};

// Reads tap (kd, kh, kw) of the halo and slot BS of weight row `brow` (the
// row's tap kw for the 3x3x3 GEMM) into `f`.  A row (lane % 16) is brick
// column x = lane % 8 of line ms + 4 * ((lane / 8) % 2), K piece lane / 16; at
// tap (kd, kh, kw) it reads halo column x + kw of halo line
// ms + 4 * ((lane / 8) % 2) + kh.  Split fp16: cbase[ns] is the lane's Bl
// offset within a tap (lane groups 0, 1) or the tap's zero slot (2, 3).
template <int DT, int KD, int KH, int KW, int BS = KW>
__device__ __forceinline__ void lds16_load(Lds16Frag& f, const char* brow, const char* halo_p,
                                           const int (&abase)[4], const int (&bbase)[4], const int (&cbase)[4],
                                           int lane) {
  const int h = (lane >> 3) & 1, g = (lane >> 4) & 3;
  constexpr int off = ((KD * kHH + KH) * kHW + KW) * 64;
  constexpr int tb = Lds16Cfg<DT>::tap_bytes;
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    const int piece = g ^ lds16_halo_swizzle(ms + 4 * h + KH);
    f.a[ms] = *reinterpret_cast<const u4*>(halo_p + (abase[ms] | (piece << 4)) + off);
  }
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) f.b[ns] = *reinterpret_cast<const u4*>(brow + BS * tb + bbase[ns]);
  if constexpr (DT == CTMR_F16X2) {
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) f.c[ns] = *reinterpret_cast<const u4*>(brow + BS * tb + cbase[ns]);
  }
}

__device__ __forceinline__ void mfma_f16(f4& acc, const u4& a, const u4& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), acc, 0, 0, 0);
}

// B^T A^T (operands exchanged: the same dot products) so that a lane's result
// registers are four adjacent output columns of one voxel.  Split fp16: the
// sixteen Bh products, then the sixteen Bl ones (no MFMA waits on the one
// before it).
template <int DT>
__device__ __forceinline__ void lds16_mma(f4 (&acc)[4][4], const Lds16Frag& f) {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
  if constexpr (DT == CTMR_F16X2) {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) mfma_f16(acc[ms][ns], f.b[ns], f.a[ms]);
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) mfma_f16(acc[ms][ns], f.c[ns], f.a[ms]);
  } else {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) mfma_step<CTMR_BF16>(acc[ms][ns], f.b[ns], f.a[ms]);
  }
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_sched_barrier(0);
}

// Tap row R (kd, kh) = (R / 3, R % 3) of conv_lds_bf16_kernel, B from this
// row's weight buffer `brow`; its first tap is already in fr[R % 2].  The
// row's single barrier sits after the last ds_read of the row and before the
// last tap's products: once every wave is past it (and has waited for its own
// fills), the fill issued two rows ago is visible to all and `brow` is free,
// so `after_barrier` can refill it with the row two ahead -- a fill has three
// taps of products to arrive.  The next row's first tap (NEXT) is read into
// fr[(R + 1) % 2] while this row's last products run.
template <int DT, int R, bool NEXT, typename AfterBarrier>
__device__ __forceinline__ void lds16_row(f4 (&acc)[4][4], Lds16Frag (&fr)[2], const char* brow,
                                          const char* brow_next, const char* halo_p, const int (&abase)[4],
                                          const int (&bbase)[4], const int (&cbase)[4], int lane,
                                          AfterBarrier&& after_barrier) {
  constexpr int KD = R / 3, KH = R % 3, P = R & 1;
  lds16_load<DT, KD, KH, 1>(fr[P ^ 1], brow, halo_p, abase, bbase, cbase, lane);
  lds16_mma<DT>(acc, fr[P]);
  lds16_load<DT, KD, KH, 2>(fr[P], brow, halo_p, abase, bbase, cbase, lane);
  lds16_mma<DT>(acc, fr[P ^ 1]);
  // Every read of this row has returned and this wave's fills have landed.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  after_barrier();
  if (NEXT)
    lds16_load<DT, (R + 1) / 3, (R + 1) % 3, 0>(fr[P ^ 1], brow_next, halo_p, abase, bbase, cbase, lane);
  lds16_mma<DT>(acc, fr[P]);
}

// Tap row (KD, KH) of the nearest-2x parity GEMM in conv_lds_bf16_kernel<.., true>:
// halo taps (KD, KH, KW0) and (KD, KH, KW0 + 1), B from slots 0 and 1 of this
// row's weight buffer `brow`; its first tap is already in fr[0].  Barrier and
// refill as in lds16_row: the barrier follows the row's last ds_read; after
// it `after_barrier` refills `brow`, and the next row's first tap (NEXT: halo
// tap (NKD, NKH, KW0), buffer `brow_next`) is read into fr[0] while this
// row's second products run.
template <int DT, int KD, int KH, int KW0, bool NEXT, int NKD, int NKH, typename AfterBarrier>
__device__ __forceinline__ void lds16_row2(f4 (&acc)[4][4], Lds16Frag (&fr)[2], const char* brow,
                                           const char* brow_next, const char* halo_p, const int (&abase)[4],
                                           const int (&bbase)[4], const int (&cbase)[4], int lane,
                                           AfterBarrier&& after_barrier) {
  lds16_load<DT, KD, KH, KW0 + 1, 1>(fr[1], brow, halo_p, abase, bbase, cbase, lane);
  lds16_mma<DT>(acc, fr[0]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  after_barrier();
  if constexpr (NEXT) lds16_load<DT, NKD, NKH, KW0, 0>(fr[0], brow_next, halo_p, abase, bbase, cbase, lane);
  lds16_mma<DT>(acc, fr[1]);
}

// Halo-fill geometry of a thread of conv_lds_bf16_kernel.
struct Lds16Geo {
  int tid, y0, x0, pd_max, ph_max, pw_max, P, Q, vbytes;
};

// Packed-copy byte offset (from the brick's first padded plane) of halo slot
// tid + 256 i: slot s % 4 of halo voxel s / 4, coordinates past the padded
// volume clamped (they feed only masked output rows).
__device__ __forceinline__ int lds16_halo_offset(const Lds16Geo& g, int i) {
  const int sl = g.tid + 256 * i;
  const int v = sl >> 2, q = sl & 3;
  const int hz = v / (kHH * kHW), hr = v - hz * (kHH * kHW);
  const int hy = hr / kHW, hx = hr - hy * kHW;
  const int pz = min(hz, g.pd_max), py = min(g.y0 + hy, g.ph_max), px = min(g.x0 + hx, g.pw_max);
  return ((pz * g.P + py * g.Q + px) * g.vbytes) + 16 * (q ^ lds16_halo_swizzle(hy));
}

// Packed-weight byte offset (from a row's first tap) of weight-row fill slot
// tid + 256 j.  bf16: slot s % 4 of column (s / 4) % 64 of tap j.  Split
// fp16: slot s is in tap s / 384; its first 256 slots are the Bh pieces (slot
// r: piece r % 4 of column r / 4, swizzled as bf16), the next 128 the Bl
// pieces (piece r % 2 of column r / 2).
template <int DT>
__device__ __forceinline__ int lds16_weight_offset(int tid, int j, int n0, int tap_bytes) {
  const int s = tid + 256 * j;
  if constexpr (DT == CTMR_F16X2) {
    const int t = s / 384, r = s - 384 * t;
    if (r < 256) {
      const int col = r >> 2;
      return t * tap_bytes + (n0 + col) * 96 + 16 * ((r & 3) ^ row64_swizzle(col & 15));
    }
    const int col = (r - 256) >> 1;
    return t * tap_bytes + (n0 + col) * 96 + 64 + 16 * (r & 1);
  } else {
    return j * tap_bytes + (n0 + (tid >> 2)) * 64 + 16 * ((tid & 3) ^ row64_swizzle((tid >> 2) & 15));
  }
}

// UP: nearest-2x upsampling folded into 8 parity filters of 2x2x2 taps
// (pack_weight_kernel's [phase][tap] layout).  Parity (a, b, c) of source
// brick (z0, y0, x0) computes output voxels (2(z0 + z) + a, 2(y0 + y) + b,
// 2(x0 + x) + c) from the same halo of the packed source copy as the 3x3x3
// GEMM, reading its taps (a + td, b + th, c + tw), td, th, tw in {0, 1}: four
// two-tap rows per chunk.  The parity is part of the workgroup index, so one
// launch covers all eight.  DT: CTMR_BF16 (32-channel chunks) or CTMR_F16X2
// (16-channel chunks of hi/lo pairs, outputs scaled back by the packed
// weight's power-of-two column scales before the epilogue).  WS = 2: a K
// split of two inside the workgroup, as conv_lds_kernel's wave sets (each set
// its own halo and weight rows; every barrier is the workgroup's, and both
// sets run the same chunk count).
template <int DT, bool UP, int WS>
__global__ __launch_bounds__(256 * WS, WS == 1 ? 2 : 1) void conv_lds_bf16_kernel(Lds16Args p) {
  using Cfg = Lds16Cfg<DT>;
  static_assert(WS == 1 || WS == 2, "one or two wave sets");
  // A set's region: the halo, then the two weight rows; regions start on
  // 256-byte boundaries, as the single set's arrays did.
  constexpr int kSetBytes = (kB16HaloBytes + 2 * Cfg::row_bytes + 255) / 256 * 256;
  static_assert(kB16HaloBytes % 256 == 0 && Cfg::row_bytes % 16 == 0, "aligned halo and weight rows");
  __shared__ __attribute__((aligned(256))) char lds_sets[WS * kSetBytes];
  const int set = WS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
  char* const halo = lds_sets + set * kSetBytes;
  char (*const bbuf)[Cfg::row_bytes] = reinterpret_cast<char (*)[Cfg::row_bytes]>(halo + kB16HaloBytes);
  const int tid = threadIdx.x & 255, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot = bid >> 3, per = nb >> 3, rem = nb & 7;
  const int tile = (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int n_tile = tile % p.n_tiles;
  int rest = tile / p.n_tiles;
  const int bx = rest % p.tx;
  rest /= p.tx;
  const int by = rest % p.ty;
  rest /= p.ty;
  const int bz = rest % p.tz;
  rest /= p.tz;
  int phase = 0;
  if constexpr (UP) {
    phase = rest & 7;
    rest >>= 3;
  }
  const int b = rest % p.n;
  const int split_id = rest / p.n;
  const int z0 = bz * kBD, y0 = by * kBH, x0 = bx * kBW;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int n0 = n_tile * 64;
  if constexpr (DT == CTMR_F16X2) {
    // the taps' zero slots read by lane groups 2 and 3 for Bl (published by
    // the first chunk's barrier; fills never write them)
    if (tid < 6) *reinterpret_cast<u4*>(&bbuf[tid / 3][(tid % 3) * kF2TapBytes + kF2ZeroOff]) = u4{0u, 0u, 0u, 0u};
  }

  // Halo fill: slot s = tid + 256 i is slot s % 4 of halo voxel s / 4.  The
  // brick's halo origin in padded coordinates is (z0, y0, x0); coordinates
  // past the padded volume (ragged bricks) are clamped -- they feed only
  // masked output rows.
  const int64_t xbase = ((int64_t)b * p.rows_per_batch + (int64_t)z0 * p.P) * p.vbytes;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.xp + xbase), (short)0, (int)min(p.x_bytes - xbase, (int64_t)0x7fffffff), 0x00020000);
  const int pd_max = p.d + 1 - z0, ph_max = p.h + 1, pw_max = p.w + 1;
  const Lds16Geo geo{tid, y0, x0, pd_max, ph_max, pw_max, p.P, p.Q, p.vbytes};
  // Split fp16 holds more operand registers (the Bl fragments): its fill
  // offsets are recomputed per fill (a few VALU operations per chunk or row)
  // instead of being kept in 15 registers.
  constexpr bool kKeepOffsets = DT != CTMR_F16X2;
  int hoff[kB16HaloIters];
  unsigned hload = 0;
#pragma unroll
  for (int i = 0; i < kB16HaloIters; ++i) {
    hoff[i] = 0;
    if (tid + 256 * i < kB16HaloSlots) {
      hload |= 1u << i;
      if constexpr (kKeepOffsets) hoff[i] = lds16_halo_offset(geo, i);
    }
  }
  // Weight-row fill (lds16_weight_offset).
  const int tap_bytes = p.kb * p.np * Cfg::col_bytes;  // packed bytes between consecutive taps
  constexpr int row_slots = (UP ? 2 : 3) * (DT == CTMR_F16X2 ? 384 : Cfg::tap_bytes / 16);
  int woff[Cfg::row_iters];
#pragma unroll
  for (int j = 0; j < Cfg::row_iters; ++j) woff[j] = kKeepOffsets ? lds16_weight_offset<DT>(tid, j, n0, tap_bytes) : 0;
  auto fill_halo = [&](int chunk) {
    const int so = __builtin_amdgcn_readfirstlane(chunk * 64);
#pragma unroll
    for (int i = 0; i < kB16HaloIters; ++i)
      if ((hload >> i) & 1u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xrsrc, (lds_ptr_t)(halo + (i * 256 + wave * 64) * 16), 16,
                                                 kKeepOffsets ? hoff[i] : lds16_halo_offset(geo, i), so, 0, 0);
  };
  // First tap of weight row `row`: 3 * row of the 27 (or 8 * phase + 2 * row
  // with UP), K block `chunk`.
  auto row_so = [&](int chunk, int row) {
    const int tap = UP ? 8 * phase + 2 * row : 3 * row;
    return __builtin_amdgcn_readfirstlane((tap * p.kb + chunk) * p.np * Cfg::col_bytes);
  };

  int abase[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
    abase[ms] = ((wave * kHH + ms + 4 * (lrow >> 3)) * kHW + (lrow & 7)) * 64;
  int bbase[4], cbase[4];
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) {
    bbase[ns] = (ns * 16 + lrow) * 64 + 16 * (lgrp ^ row64_swizzle(lrow));
    cbase[ns] = lgrp < 2 ? kF2BlOff + (ns * 16 + lrow) * 32 + 16 * lgrp : kF2ZeroOff;
  }

  f4 acc[4][4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = f4{0.f, 0.f, 0.f, 0.f};

  const int kpart = split_id * WS + set, kparts = p.split * WS;
  const int c_begin = __builtin_amdgcn_readfirstlane((int)((int64_t)kpart * p.kb / kparts));
  const int c_end = __builtin_amdgcn_readfirstlane((int)((int64_t)(kpart + 1) * p.kb / kparts));

  // Weight rows are numbered k = 9 * (chunk - c_begin) + row and live in
  // buffer k & 1; row k refills its own buffer with row k + 2.
  auto fill_row = [&](int chunk, int row, int buf) {
    const char* src = p.wp + row_so(chunk, row);
#pragma unroll
    for (int j = 0; j < Cfg::row_iters; ++j)
      if (j * 256 + wave * 64 < row_slots) {  // wave-uniform
        const int q = 4 * j + wave;  // wave block of 64 slots; split fp16 skips each tap's zero slot
        const int slot0 = 64 * q + (DT == CTMR_F16X2 ? q / 6 : 0);
        lds_dma16(src + (kKeepOffsets ? woff[j] : lds16_weight_offset<DT>(tid, j, n0, tap_bytes)),
                  (unsigned)(uintptr_t)(lds_ptr_t)(&bbuf[buf][0] + slot0 * 16));
      }
  };
  fill_halo(c_begin);
  fill_row(c_begin, 0, 0);
  if (c_end - c_begin > 0) fill_row(c_begin, 1, 1);
  int k = 0;
  if constexpr (UP) {
    // Rows R = 2 td + th of a chunk; row k refills its buffer with row k + 2.
    auto chunks = [&](auto pa, auto pb, auto pc) {
      constexpr int A = decltype(pa)::value, B = decltype(pb)::value, C = decltype(pc)::value;
      for (int chunk = c_begin; chunk < c_end; ++chunk) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        const bool more = chunk + 1 < c_end;
        Lds16Frag fr[2];
        lds16_load<DT, A, B, C, 0>(fr[0], &bbuf[k & 1][0], halo, abase, bbase, cbase, lane);
#define CTMR_LDS16_UP_ROW(R, NEXT)                                                                        \
        lds16_row2<DT, A + (R) / 2, B + (R) % 2, C, NEXT, A + ((R) + 1) / 2, B + ((R) + 1) % 2>(            \
            acc, fr, &bbuf[k & 1][0], &bbuf[(k + 1) & 1][0], halo, abase, bbase, cbase, lane, [&]() {        \
              if ((R) < 2) fill_row(chunk, (R) + 2, k & 1);                                                 \
              else if (more) fill_row(chunk + 1, (R) - 2, k & 1);                                           \
              if ((R) == 3 && more) fill_halo(chunk + 1);                                                   \
            });                                                                                             \
        ++k;
        CTMR_LDS16_UP_ROW(0, true) CTMR_LDS16_UP_ROW(1, true) CTMR_LDS16_UP_ROW(2, true)
        CTMR_LDS16_UP_ROW(3, false)
#undef CTMR_LDS16_UP_ROW
      }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    switch (phase) {
      case 0: chunks(I0{}, I0{}, I0{}); break;
      case 1: chunks(I0{}, I0{}, I1{}); break;
      case 2: chunks(I0{}, I1{}, I0{}); break;
      case 3: chunks(I0{}, I1{}, I1{}); break;
      case 4: chunks(I1{}, I0{}, I0{}); break;
      case 5: chunks(I1{}, I0{}, I1{}); break;
      case 6: chunks(I1{}, I1{}, I0{}); break;
      default: chunks(I1{}, I1{}, I1{}); break;
    }
  } else
  for (int chunk = c_begin; chunk < c_end; ++chunk) {
    // The chunk's halo (and the first weight rows) must have landed.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const bool more = chunk + 1 < c_end;
    Lds16Frag fr[2];
    lds16_load<DT, 0, 0, 0>(fr[0], &bbuf[k & 1][0], halo, abase, bbase, cbase, lane);
#define CTMR_LDS16_ROW(R)                                                                                   \
    lds16_row<DT, (R), (R) < 8>(acc, fr, &bbuf[k & 1][0], &bbuf[(k + 1) & 1][0], halo, abase, bbase, cbase,  \
                                lane, [&]() {                                                               \
      if ((R) < 7) fill_row(chunk, (R) + 2, k & 1);                                                        \
      else if (more) fill_row(chunk + 1, (R) - 7, k & 1);                                                  \
      if ((R) == 8 && more) fill_halo(chunk + 1);                                                          \
    });                                                                                                    \
    ++k;
    CTMR_LDS16_ROW(0) CTMR_LDS16_ROW(1) CTMR_LDS16_ROW(2)
    CTMR_LDS16_ROW(3) CTMR_LDS16_ROW(4) CTMR_LDS16_ROW(5)
    CTMR_LDS16_ROW(6) CTMR_LDS16_ROW(7) CTMR_LDS16_ROW(8)
#undef CTMR_LDS16_ROW
  }

  if constexpr (DT == CTMR_F16X2) {
    // undo the weights' power-of-two column scales (exact), per partial plane alike
    const float* colscale = reinterpret_cast<const float*>(p.wp + p.w_bytes);
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const f4 sc = *reinterpret_cast<const f4*>(colscale + n0 + ns * 16 + 4 * lgrp);
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) acc[ms][ns] *= sc;
    }
  }
  const int tile_id = ((bz * p.ty + by) * p.tx + bx) * (UP ? 8 : 1) + phase;
  // The statistics' reduction buffer reuses set 0's halo (its first 4 KiB).
  double (*const red)[64][2] = reinterpret_cast<double (*)[64][2]>(lds_sets);
  if constexpr (WS == 2) {
    // Set 1 hands its sums to set 0 through LDS past that buffer (64 KiB of
    // the two sets' regions) once every wave has finished its last chunk.
    f4* const xs = reinterpret_cast<f4*>(lds_sets + 4096);
    static_assert(4096 + 4 * 16 * 64 * 16 <= WS * kSetBytes, "hand-over buffer");
    __syncthreads();
    if (set == 1) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) xs[(wave * 16 + ms * 4 + ns) * 64 + lane] = acc[ms][ns];
    }
    __syncthreads();
    if (set == 1) return;
    store_brick<UP>(p, acc, b, split_id, z0, y0, x0, n0, wave, lane, tile_id, red, phase, [&](f4 (&a)[4][4]) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) a[ms][ns] += xs[(wave * 16 + ms * 4 + ns) * 64 + lane];
    });
  } else {
    store_brick<UP>(p, acc, b, split_id, z0, y0, x0, n0, wave, lane, tile_id, red, phase);
  }
}

// ---------------------------------------------------------------------------
// 3d. Persistent pointwise GEMM over an LDS ring (one K tap: 1x1x1 convs and
// the im2col and tap-expanded formulations)
// ---------------------------------------------------------------------------
// These GEMMs read their A rows from HBM once, with only 4-32 K blocks per
// tile; a one-step register prefetch does not cover HBM latency, and a launch
// of one tile per workgroup also exposes every tile's first loads.  Here:
//  * operands go straight from memory into a ring of kStages LDS stages
//    (buffer_load_dwordx4 ... lds), kStages - 1 K blocks ahead of the MFMAs,
//    one barrier per K block;
//  * a grid of as many workgroups as the device holds walks the tiles: a
//    workgroup keeps one column tile and visits row items l, l + L, l + 2L, ...
//    (an item is a WM*64-row tile of one batch item and one K range), and the
//    ring runs straight across items, so the next item's first blocks land
//    while this item's epilogue stores.
// A stage holds the tile's A rows (WM*64 voxels) then its B columns (WN*64),
// 64 bytes (one K block) each, the four 16-byte pieces of row r in slots
// piece ^ row64_swizzle(r) -- the layout conflict-free for ds_read_b128 that
// the bf16 LDS GEMM uses.  Each wave multiplies exactly the fragments
// conv_kernel<DT, 4, WM, WN, 1, 1, false> loads, in the same order, with the
// two MFMA operands exchanged (B^T A^T: every output is the same dot product,
// and a lane ends with four adjacent columns of one row, stored as 16 bytes),
// so the outputs are bit-identical to it.  Rows past the volume are outside
// the A descriptor's range and stage as zeros (their outputs are not stored).
template <int WM, int WN>
struct PwRing {
  static constexpr int kRows = (WM + WN) * 64;           // A rows + B columns of a stage
  static constexpr int kStageBytes = kRows * 64;
  static constexpr int kStages = kStageBytes <= 16384 ? 4 : 3;  // <= 64 KiB: two workgroups per CU
  static constexpr int kDma = kRows / 64;                 // 1 KiB loads per wave per stage
};

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor (raw, 32-bit range) with wave-uniform fields.
__device__ __forceinline__ u32x4 raw_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = (uint64_t)base;
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((unsigned)a);
  r.y = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  r.z = __builtin_amdgcn_readfirstlane((unsigned)min(max(bytes, (int64_t)0), (int64_t)0x7fffffff));
  r.w = 0x00020000u;
  return r;
}

// A descriptor chosen by a wave-uniform condition, kept in scalar registers.
__device__ __forceinline__ u32x4 uniform4(u32x4 v) {
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(v.x);
  r.y = __builtin_amdgcn_readfirstlane(v.y);
  r.z = __builtin_amdgcn_readfirstlane(v.z);
  r.w = __builtin_amdgcn_readfirstlane(v.w);
  return r;
}

// Direct-to-LDS 16-byte buffer load of lane i (offset voff + soff, zero out
// of range) into LDS byte lds_addr + 16 i.  Inline assembly for the reason
// given at lds_dma16; callers wait with wait_vmcnt.
__device__ __forceinline__ void lds_dma_buf16(u32x4 rsrc, int voff, int soff, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) (other counters unconstrained).  Vector-memory loads,
// direct-to-LDS ones included, complete in issue order, so with N loads
// issued after a given one this returns once that one has landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// TWO: A rows of a two-source input read in place (ctmr_conv3d_cat, fp32).
template <int DT, int WM, int WN, bool TWO>
__global__ __launch_bounds__(256, 2) void pointwise_kernel(ConvArgs p) {
  static_assert(WM * WN == 4, "four waves per workgroup");
  using R = PwRing<WM, WN>;
  constexpr int NSUB = 4, TM = WM * 64, TN = WN * 64;
  __shared__ __attribute__((aligned(16))) char ring[R::kStages * R::kStageBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave_m = wave % WM, wave_n = wave / WM;
  // XCD-aware order (as conv_kernel): consecutive ids share an XCD, so the
  // column tiles of one row lane, which read the same input rows, share an L2.
  const int nb = gridDim.x, bid = blockIdx.x;
  const int xcd = bid & 7, slot8 = bid >> 3, per = nb >> 3, rem = nb & 7;
  const int vid = (xcd < rem) ? xcd * (per + 1) + slot8 : rem * (per + 1) + (xcd - rem) * per + slot8;
  const int n_tile = vid % p.n_tiles;
  const int lanes = nb / p.n_tiles;  // the host launches lanes * n_tiles workgroups
  const int first = vid / p.n_tiles;
  const int lrow = lane & 15, lgrp = lane >> 4;
  const int S = p.gd * p.gh * p.gw;
  const int rb = (int)p.row_bytes;
  const int steps = p.kb;
  const int bstep = p.np * 64;
  const int n0 = n_tile * TN + wave_n * 64;

  // Item r: split range r % split of row tile (r / split) % m_tiles of batch
  // item r / (split * m_tiles), K blocks [s_begin, s_end).
  struct Item {
    int b, m_tile, split_id, s_begin, s_end;
  };
  auto item = [&](int r) {
    Item it;
    it.split_id = r % p.split;
    const int rest = r / p.split;
    it.m_tile = rest % p.m_tiles;
    it.b = rest / p.m_tiles;
    it.s_begin = __builtin_amdgcn_readfirstlane((int)((int64_t)it.split_id * steps / p.split));
    it.s_end = __builtin_amdgcn_readfirstlane((int)((int64_t)(it.split_id + 1) * steps / p.split));
    return it;
  };

  // Load t of this wave fills stage rows 16 * (wave * kDma + t) + lane / 4,
  // slot lane % 4 -- piece (lane % 4) ^ swizzle of that row: an A row (voxel)
  // or a B column.  The lane offsets are fixed; items move the A base only.
  // A rows of a two-source input (TWO): K blocks below kb1 from xp (rows of
  // rb bytes), the rest from xp2 (rows of rb2 bytes).
  const int rb2 = TWO ? (int)p.row_bytes2 : 0;
  int voff[R::kDma], voff2[TWO ? R::kDma : 1];
#pragma unroll
  for (int t = 0; t < R::kDma; ++t) {
    const int row = 16 * (wave * R::kDma + t) + (lane >> 2);
    const int piece = (lane & 3) ^ row64_swizzle(row);
    voff[t] = row < TM ? row * rb + piece * 16 : (n_tile * TN + row - TM) * 64 + piece * 16;
    if constexpr (TWO) voff2[t] = row < TM ? row * rb2 + piece * 16 : voff[t];
  }
  const u32x4 brsrc = raw_rsrc(p.wp, p.w_bytes);
  const unsigned ring_lds = (unsigned)(uintptr_t)(lds_ptr_t)ring;

  // Load cursor: item d_r, K block d_s of [.., d_end), the item's A rows.
  int d_r = first, d_s, d_end;
  u32x4 arsrc, arsrc2;
  auto start_item = [&](int r) {
    const Item it = item(r);
    d_s = it.s_begin;
    d_end = it.s_end;
    const int64_t row = (int64_t)it.b * p.rows_per_batch + (int64_t)it.m_tile * TM;
    arsrc = raw_rsrc(p.xp + row * rb, (int64_t)(S - it.m_tile * TM) * rb);
    if constexpr (TWO) arsrc2 = raw_rsrc(p.xp2 + row * rb2, (int64_t)(S - it.m_tile * TM) * rb2);
  };
  start_item(d_r);
  auto fill = [&](int st) {
    const unsigned lds = ring_lds + st * R::kStageBytes + wave * R::kDma * 1024;
    if constexpr (TWO) {
      const bool second = __builtin_amdgcn_readfirstlane(d_s) >= p.kb1;  // wave-uniform
      const int sa = __builtin_amdgcn_readfirstlane((second ? d_s - p.kb1 : d_s) * 64);
      const int sb = __builtin_amdgcn_readfirstlane(d_s * bstep);
      const u32x4 asrc = uniform4(second ? arsrc2 : arsrc);
#pragma unroll
      for (int t = 0; t < R::kDma; ++t) {
        const bool a_rows = 16 * (wave * R::kDma + t) < TM;  // wave-uniform: a scalar select, no branch
        lds_dma_buf16(a_rows ? asrc : brsrc, second ? voff2[t] : voff[t], a_rows ? sa : sb, lds + t * 1024);
      }
    } else {
      const int sa = __builtin_amdgcn_readfirstlane(d_s * 64);
      const int sb = __builtin_amdgcn_readfirstlane(d_s * bstep);
#pragma unroll
      for (int t = 0; t < R::kDma; ++t) {
        const bool a_rows = 16 * (wave * R::kDma + t) < TM;  // wave-uniform: a scalar select, no branch
        lds_dma_buf16(a_rows ? arsrc : brsrc, voff[t], a_rows ? sa : sb, lds + t * 1024);
      }
    }
    if (++d_s == d_end) {
      if (d_r + lanes < p.items) {
        d_r += lanes;
        start_item(d_r);
      } else {
        d_s = d_end - 1;  // past the last item: re-read its last block into a stage never read
      }
    }
  };

  f4 acc[4][NSUB];
  auto clear = [&]() {
#pragma unroll
    for (int ms = 0; ms < 4; ++ms)
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] = f4{0.f, 0.f, 0.f, 0.f};
  };
  clear();
  // The accumulators hold B^T A^T blocks (mma_block<.., true>): lane l of
  // block (ms, ns) has row ms*16 + l%16, columns ns*16 + 4*(l/16) .. +3.  The
  // column tile is fixed, so those columns' bias is loaded once, before any
  // ring load is in flight.
  f4 bq[NSUB];
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) {
    const float* bias = p.bias;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bq[ns][r] = (p.split == 1 && p.has_bias) ? bias[min(n0 + ns * 16 + 4 * lgrp + r, p.cout - 1)] : 0.f;
  }
  int c_r = first, left;
  {
    const Item it = item(c_r);
    left = it.s_end - it.s_begin;
  }
  // Epilogue: one 16-byte store per block and lane, through a buffer
  // descriptor over the wave's output rows.  Rows past the volume fall
  // outside its range and column quads past cout (a multiple of 4 here) get
  // an offset outside it, so the hardware drops both without branches.  No
  // global load happens here (per-batch bias and residual stay on
  // conv_kernel): a load would make the compiler wait for every ring load in
  // flight.
  int q_off[NSUB];
#pragma unroll
  for (int ns = 0; ns < NSUB; ++ns) {
    const int col = n0 + ns * 16 + 4 * lgrp;
    q_off[ns] = col < p.cout ? (lrow * p.cout + col) * 4 : 0x40000000;
  }
  __shared__ double red[4][64][2];
  auto finish = [&]() -> bool {
    const Item it = item(c_r);
    const int m0 = it.m_tile * TM + wave_m * 64;
    const int valid_rows = min(max(S - m0, 0), 64);
    float* out = p.y + (p.split > 1 ? (int64_t)it.split_id * p.plane : 0) + ((int64_t)it.b * p.s_out + m0) * p.cout;
    // Both descriptor fields are wave-uniform; the compiler cannot prove it (the row count goes
    // through a VALU clamp) and would wrap every store in a loop over distinct descriptors.
    const uint64_t oaddr = (uint64_t)out;
    out = (float*)(((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(oaddr >> 32)) << 32) |
                   (unsigned)__builtin_amdgcn_readfirstlane((unsigned)oaddr));
    const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
        out, (short)0, __builtin_amdgcn_readfirstlane(valid_rows * p.cout * 4), 0x00020000);
    if (p.split == 1 && p.has_bias) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns) acc[ms][ns] += bq[ns];
    }
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns)
#pragma unroll
      for (int ms = 0; ms < 4; ++ms)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[ms][ns]), orsrc,
                                               q_off[ns] + ms * 16 * p.cout * 4, 0, kStoreNT);
    if (p.stats) {  // a kernel argument: every thread reaches the barriers
      bool row_ok[4], col_ok[NSUB];
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) row_ok[ms] = ms * 16 + lrow < valid_rows;
#pragma unroll
      for (int ns = 0; ns < NSUB; ++ns) col_ok[ns] = q_off[ns] < 0x40000000;
      column_sums<NSUB>(acc, row_ok, col_ok, red, wave, lane);
      __syncthreads();
      combine_gn_partials<NSUB, WM, WN>(red, n_tile * TN, p.cout, p.gn_cpg, p.gn_groups,
                                        p.stats + ((int64_t)it.b * p.stats_tiles + it.m_tile) * p.gn_groups * 2);
      __syncthreads();  // the next item's partials reuse `red`
    }
    c_r += lanes;
    if (c_r >= p.items) return false;
    const Item nx = item(c_r);
    left = nx.s_end - nx.s_begin;
    clear();
    return true;
  };

  // Fragment addresses in a stage: A row wave_m*64 + ms*16 + lane%16, B column
  // wave_n*64 + ns*16 + lane%16, K piece lane/16 (swizzle bits 2-3 of the row
  // are those of lane%16).
  const int sw = lgrp ^ row64_swizzle(lrow);
  const int a_lds = (wave_m * 64 + lrow) * 64 + sw * 16;
  const int b_lds = (TM + wave_n * 64 + lrow) * 64 + sw * 16;

#pragma unroll
  for (int st = 0; st < R::kStages - 1; ++st) fill(st);
  int cur = 0;
  for (;;) {
    wait_vmcnt<R::kDma * (R::kStages - 2)>();  // this wave's loads of stage `cur`
    __syncthreads();  // everyone's loads of `cur` landed; everyone is done reading the stage before it
    fill(cur == 0 ? R::kStages - 1 : cur - 1);
    const char* stage = ring + cur * R::kStageBytes;
    u4 A[4], B[NSUB];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) A[ms] = *reinterpret_cast<const u4*>(stage + a_lds + ms * 1024);
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) B[ns] = *reinterpret_cast<const u4*>(stage + b_lds + ns * 1024);
    __builtin_amdgcn_s_setprio(1);
    mma_block<DT, NSUB, true>(acc, A, B);
    __builtin_amdgcn_s_setprio(0);
    cur = cur + 1 == R::kStages ? 0 : cur + 1;
    if (--left == 0 && !finish()) break;
  }
  __builtin_amdgcn_s_waitcnt(0);  // no ring load may land after the workgroup ends
}

// Sum of split partial planes in ascending order, then residual; bias first
// as in the reference reduce (_nax_conv.py:320-332).
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part,
                                                           int64_t plane, int split,
                                                           const float* __restrict__ bias,
                                                           int has_bias, int batch_bias,
                                                           const float* __restrict__ res,
                                                           float* __restrict__ y, int cout,
                                                           int64_t s_out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < plane;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cout);
    const int64_t b = i / (s_out * cout);
    float v = has_bias ? bias[(batch_bias ? b * cout : 0) + c] : 0.f;
    for (int k = 0; k < split; ++k) v += part[(int64_t)k * plane + i];
    if (res) v += res[i];
    y[i] = v;
  }
}

// The same reduction (same order per element, so the same output bits) that
// also writes group-norm partials (ctmr_conv3d_gn on a K split).  Block
// (chunk, 64-column tile) of batch item blockIdx.y: thread t sums columns
// 4*(t%16)..+3 of voxels chunk*16*rows + 16*j + t/16, keeping fp64 sums; the
// 16 voxel lanes and each group's columns are then added in ascending order.
// Partials: stats[((b * chunks + chunk) * groups + g) * 2 + {0, 1}].
__global__ __launch_bounds__(256) void split_reduce_gn_kernel(const float* __restrict__ part,
                                                              int64_t plane, int split,
                                                              const float* __restrict__ bias,
                                                              int has_bias, int batch_bias,
                                                              const float* __restrict__ res,
                                                              float* __restrict__ y, int cout,
                                                              int64_t s_out, int rows, int chunks,
                                                              int cpg, int groups,
                                                              double* __restrict__ stats) {
  const int ctiles = cout / 64;
  const int chunk = blockIdx.x / ctiles, ct = blockIdx.x % ctiles, b = blockIdx.y;
  const int t = threadIdx.x, cv = t & 15, vl = t >> 4;
  const int c0 = ct * 64 + cv * 4;
  float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (has_bias) bv = *(const float4*)(bias + (batch_bias ? (int64_t)b * cout : 0) + c0);
  double s1[4] = {0.0, 0.0, 0.0, 0.0}, s2[4] = {0.0, 0.0, 0.0, 0.0};
  for (int j = 0; j < rows; ++j) {
    const int64_t v = ((int64_t)chunk * rows + j) * 16 + vl;
    if (v >= s_out) break;
    const int64_t i = ((int64_t)b * s_out + v) * cout + c0;
    float4 a = bv;
    // Four partial planes' loads in flight at a time, added in ascending order.
    int k = 0;
    for (; k + 4 <= split; k += 4) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = *(const float4*)(part + (int64_t)(k + u) * plane + i);
#pragma unroll
      for (int u = 0; u < 4; ++u) { a.x += q[u].x; a.y += q[u].y; a.z += q[u].z; a.w += q[u].w; }
    }
    for (; k < split; ++k) {
      const float4 q = *(const float4*)(part + (int64_t)k * plane + i);
      a.x += q.x; a.y += q.y; a.z += q.z; a.w += q.w;
    }
    if (res) {
      const float4 r = *(const float4*)(res + i);
      a.x += r.x; a.y += r.y; a.z += r.z; a.w += r.w;
    }
    *(float4*)(y + i) = a;
    const float e[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      s1[k] += (double)e[k];
      s2[k] = fma((double)e[k], (double)e[k], s2[k]);
    }
  }
  __shared__ double red[16][64][2];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    red[vl][cv * 4 + k][0] = s1[k];
    red[vl][cv * 4 + k][1] = s2[k];
  }
  __syncthreads();
  if (t < 64 / cpg) {
    double a = 0.0, q = 0.0;
    for (int l = 0; l < 16; ++l)
      for (int cc = 0; cc < cpg; ++cc) {
        a += red[l][t * cpg + cc][0];
        q += red[l][t * cpg + cc][1];
      }
    double* out = stats + (((int64_t)b * chunks + chunk) * groups + ct * (64 / cpg) + t) * 2;
    out[0] = a;
    out[1] = q;
  }
}

// ---------------------------------------------------------------------------
// Host side: geometry, policy and dispatch
// ---------------------------------------------------------------------------
struct Geometry {
  int ks, halo, KT, taps, phases;
  int gd, gh, gw;        // iteration grid
  int td, th, tw;        // packed interior grid
  int od, oh, ow;        // output grid
  bool pack;             // build a packed copy of the input
  int kstep, esize, cp, np, kblocks;
  int P, Q;
  int64_t rows_per_batch;
  int split;
  int nsub, wm, wn, m_tiles, n_tiles;
  bool lds;              // LDS-staged GEMM (conv_lds_kernel)
  int wsets;             // its K ranges as wave sets of one workgroup (2: a split of 2 without partial planes)
  bool lds16;            // LDS-staged bf16 GEMM over the packed copy (conv_lds_bf16_kernel)
  bool small_out;        // direct cout <= 4 conv from an LDS halo (conv_small_cout_kernel)
  bool lds_small;        // LDS-staged im2col GEMM for cin 4 / 8 (conv_lds_small_kernel)
  bool cat;              // input given as two tensors, channels [0, c1) and [c1, cin)
  int c1;
  bool pointwise;        // one-tap GEMM on the persistent pointwise_kernel
  bool direct;           // streaming GEMM reading the unpadded input (no pack)
  bool kws;              // 64 x 64 tiles, the K range of each split over the four waves
  int tz, ty, tx;        // its bricks per axis
  int layout;            // WL_TAPS, WL_EXPAND (cout <= 4) or WL_IM2COL (small cin)
  int ncols;             // GEMM columns: cout, or 27 * cout for WL_EXPAND
  int64_t pack_bytes, part_bytes, z_bytes;
};

// K-range (chunk) split of the fp32 LDS-staged GEMM, from the shape only:
// small grids are split until they fill a round of 512 resident workgroups
// (two per CU on 256 CUs); grids of under 4 rounds whose last round would run
// at most 90 % as full as with two ranges take two (e.g. 1280 workgroups: 2.5
// rounds -> 5 whole rounds).  `chunks` caps it.  (The bf16 LDS GEMM keeps
// only the first rule: its products are 8x faster, so the partial planes and
// their reduction cost more than the fuller rounds save -- measured on the
// decoder's 256-channel level, 257 -> 314 us.)
static int64_t lds_policy_split(int64_t base, int64_t chunks) {
  if (base < 512) return std::min<int64_t>(ceil_div(512, base), chunks);
  if (base < 2048 && chunks >= 8) {
    const double e1 = (double)base / (512.0 * ceil_div(base, 512));
    const double e2 = (double)(2 * base) / (512.0 * ceil_div(2 * base, 512));
    if (e2 >= e1 + 0.1) return 2;
  }
  return 1;
}

static int geometry(const ctmr_conv_desc* d, Geometry& g) {
  if (!d) return fail(CTMR_E_INVALID, "null descriptor");
  if (d->n <= 0 || d->d <= 0 || d->h <= 0 || d->w <= 0 || d->cin <= 0 || d->cout <= 0)
    return fail(CTMR_E_INVALID, "non-positive dimension");
  if (d->dtype != CTMR_F32 && d->dtype != CTMR_BF16 && d->dtype != CTMR_F16X2)
    return fail(CTMR_E_INVALID, "bad dtype");
  if (d->ksize != 1 && d->ksize != 3) return fail(CTMR_E_UNSUPPORTED, "ksize must be 1 or 3");
  if (d->stride != 1 && d->stride != 2) return fail(CTMR_E_UNSUPPORTED, "stride must be 1 or 2");
  if (d->mode < CTMR_MODE_PLAIN || d->mode > CTMR_MODE_TRILINEAR2X)
    return fail(CTMR_E_INVALID, "bad mode");
  if (d->mode != CTMR_MODE_PLAIN && d->stride != 1)
    return fail(CTMR_E_UNSUPPORTED, "upsampling modes need stride 1");
  if (d->mode == CTMR_MODE_TRILINEAR2X && (d->flags & (CTMR_F_AFFINE | CTMR_F_SILU)))
    return fail(CTMR_E_UNSUPPORTED, "trilinear packing supports only a plain convolution");
  if (d->ksize == 1 && (d->mode != CTMR_MODE_PLAIN || d->stride != 1))
    return fail(CTMR_E_UNSUPPORTED, "1x1x1 conv supports only stride 1, no resampling");
  g.cat = d->cin1 != 0;
  g.c1 = g.cat ? d->cin1 : d->cin;
  if (g.cat && (d->cin1 < 0 || d->cin1 >= d->cin || d->cin1 % 16 != 0 || d->cin % 16 != 0))
    return fail(CTMR_E_INVALID, "two-source input needs 0 < cin1 < cin, both multiples of 16");
  if (g.cat && d->mode != CTMR_MODE_PLAIN)
    return fail(CTMR_E_UNSUPPORTED, "a two-source input supports only CTMR_MODE_PLAIN");
  g.ks = d->ksize;
  g.kstep = d->dtype == CTMR_BF16 ? 32 : 16;
  g.esize = d->dtype == CTMR_BF16 ? 2 : 4;  // packed-copy bytes per channel (split fp16: hi + lo)
  g.np = (int)round_up(d->cout, 16);
  g.phases = 1;
  if (d->ksize == 3) {
    g.halo = 1;
    g.KT = 3;
    g.taps = 27;
    g.td = d->d; g.th = d->h; g.tw = d->w;
    if (d->mode == CTMR_MODE_TRILINEAR2X) { g.td *= 2; g.th *= 2; g.tw *= 2; }
    if (d->stride == 2) {
      g.gd = (d->d - 1) / 2 + 1; g.gh = (d->h - 1) / 2 + 1; g.gw = (d->w - 1) / 2 + 1;
    } else {
      g.gd = g.td; g.gh = g.th; g.gw = g.tw;
    }
    g.od = g.gd; g.oh = g.gh; g.ow = g.gw;
    if (d->mode == CTMR_MODE_NEAREST2X) {
      g.KT = 2;
      g.taps = 8;
      g.phases = 8;
      g.od = 2 * g.gd; g.oh = 2 * g.gh; g.ow = 2 * g.gw;
    }
    g.pack = true;
  } else {
    g.halo = 0;
    g.KT = 1;
    g.taps = 1;
    g.td = g.gd = g.od = d->d;
    g.th = g.gh = g.oh = d->h;
    g.tw = g.gw = g.ow = d->w;
    g.pack = (d->flags & (CTMR_F_AFFINE | CTMR_F_SILU)) || d->dtype != CTMR_F32 ||
             (d->cin % g.kstep) != 0;
    // A two-source input is read directly only by the persistent pointwise
    // GEMM (its conditions below); every other one-tap route packs it.
    if (g.cat && !(d->cout > 32 && d->cout % 4 == 0 &&
                   !(d->flags & (CTMR_F_STREAM | CTMR_F_BATCH_BIAS | CTMR_F_RESIDUAL))))
      g.pack = true;
  }
  g.cp = g.pack ? (int)round_up(d->cin, g.kstep) : d->cin;
  g.kblocks = g.cp / g.kstep;
  if (g.pack) {
    g.Q = g.tw + 2 * g.halo;
    g.P = (g.th + 2 * g.halo) * g.Q;
    g.rows_per_batch = (int64_t)(g.td + 2 * g.halo) * g.P;
  } else {
    g.Q = g.tw;
    g.P = g.th * g.tw;
    g.rows_per_batch = (int64_t)g.td * g.P;
  }
  // Shape-selected GEMM formulations of a plain 3x3x3 conv (same results to
  // fp32 rounding; each keeps a fixed summation order):
  //  * WL_IM2COL, cin below one K block: K = 27 * cin packed per output voxel
  //    instead of 27 zero-padded channel blocks (the 4-channel input convs);
  //  * WL_EXPAND, cout <= 4: a 1x1 GEMM over every padded input
  //    row with 27 * cout columns, then a 27-tap gather sum (the 1- and
  //    4-channel output convs, where 16-column MFMA tiles would idle).
  g.layout = WL_TAPS;
  g.ncols = d->cout;
  g.z_bytes = 0;
  const bool plain_weights = d->mode == CTMR_MODE_PLAIN || d->mode == CTMR_MODE_TRILINEAR2X;
  if (d->ksize == 3 && plain_weights && d->cin < g.kstep) {
    g.layout = WL_IM2COL;
    g.KT = 1;
    g.taps = 1;
    g.halo = 0;  // td/th/tw stay the convolved grid: the window bounds of the im2col pack
    g.cp = (int)round_up(27 * d->cin, g.kstep);
    g.kblocks = g.cp / g.kstep;
    g.Q = g.gw;
    g.P = g.gh * g.gw;
    g.rows_per_batch = (int64_t)g.gd * g.P;
  } else if (d->ksize == 3 && plain_weights && d->cout <= 4) {
    g.layout = WL_EXPAND;
    g.KT = 1;
    g.taps = 1;
    g.ncols = 27 * d->cout;
    g.np = (int)round_up(g.ncols, 16);
    g.gd = g.td + 2; g.gh = g.th + 2; g.gw = g.tw + 2;  // GEMM rows: every padded row
  }
  const int64_t S = (int64_t)g.gd * g.gh * g.gw;
  const int64_t s_out = (int64_t)g.od * g.oh * g.ow;
  if (S > (1ll << 30) || s_out * d->cout > (1ll << 40))
    return fail(CTMR_E_UNSUPPORTED, "volume too large for 32-bit voxel indexing");
  // The brick GEMMs' epilogues (store_brick) store at 32-bit byte offsets from
  // the brick's first output plane: the kBD output planes of a brick (2 kBD
  // for the nearest-2x phases) must span under 2 GiB, or the route is not
  // taken (outputs past that span would be dropped by the buffer range).
  const bool brick_out_fits =
      (int64_t)kBD * (g.phases == 8 ? 2 : 1) * g.oh * g.ow * d->cout * 4 < (1ll << 31);
  // LDS-staged im2col GEMM: the im2col formulation of stride-1 fp32 convs with
  // 4 or 8 input channels, its rows read from a halo brick in LDS instead of
  // HBM (same K blocks and products: bit-identical outputs); 64-column tiles
  // for cout a multiple of 64, one 16- or 32-column tile for cout <= 32;
  // bricks at least 3/4 full; 6 staged planes within 32-bit buffer offsets.
  g.lds_small = false;
  g.lds = false;
  g.lds16 = false;
  g.small_out = false;
  if (g.layout == WL_IM2COL && !g.cat && d->dtype == CTMR_F32 && d->stride == 1 && d->mode == CTMR_MODE_PLAIN &&
      (d->cin == 4 || d->cin == 8) && d->cout % 4 == 0 && (d->cout % 64 == 0 || d->cout <= 32) &&
      !(d->flags & CTMR_F_STREAM)) {
    const int tz = (int)ceil_div(d->d, kBD), ty = (int)ceil_div(d->h, kBH), tx = (int)ceil_div(d->w, kBW);
    const int64_t slots = (int64_t)tz * ty * tx * kBD * kBH * kBW;
    const int64_t planes = (int64_t)kHD * d->h * d->w * d->cin * 4;
    if (4 * S >= 3 * slots && planes < (1ll << 31) && brick_out_fits) {
      g.lds_small = true;
      g.pack = false;
      g.tz = tz; g.ty = ty; g.tx = tx;
      g.nsub = d->cout % 64 == 0 ? 4 : (d->cout <= 16 ? 1 : 2);
      g.wm = 4; g.wn = 1;
      g.m_tiles = tz * ty * tx;
      g.n_tiles = (int)ceil_div(d->cout, g.nsub * 16);
      g.split = 1;
      if (d->split > 1) return fail(CTMR_E_INVALID, "split must be 1 for the small-channel LDS GEMM");
      g.direct = false;
      g.kws = false;
      g.pointwise = false;
      g.pack_bytes = (d->flags & CTMR_F_AFFINE) ? round_up((int64_t)d->n * d->cin * 2 * 4, 256) : 0;
      g.part_bytes = 0;
      const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * d->n;
      if (blocks * 256 >= (1ll << 32)) return fail(CTMR_E_UNSUPPORTED, "grid too large");
      return CTMR_OK;
    }
  }
  // Direct conv for cout <= 4 (the tap-expanded layout's shapes, fp32, stride
  // 1, channels in whole 16-channel chunks, no residual or per-batch bias, no
  // K split): reads x through an LDS halo, no padded copy, no tap-expanded
  // scratch, no tap sum.
  g.small_out = false;
  if (g.layout == WL_EXPAND && d->dtype == CTMR_F32 && d->stride == 1 && d->mode == CTMR_MODE_PLAIN &&
      d->cin % 16 == 0 && !(d->flags & (CTMR_F_STREAM | CTMR_F_RESIDUAL | CTMR_F_BATCH_BIAS))) {
    const int tz = (int)ceil_div(d->d, kBD), ty = (int)ceil_div(d->h, kBH), tx = (int)ceil_div(d->w, kBW);
    const int64_t planes = (int64_t)kHD * d->h * d->w * d->cin * 4;
    if (planes < (1ll << 31)) {
      if (d->split > 1) return fail(CTMR_E_INVALID, "split must be 1 for the cout <= 4 direct conv");
      g.small_out = true;
      g.pack = false;
      g.tz = tz; g.ty = ty; g.tx = tx;
      g.m_tiles = tz * ty * tx;
      g.n_tiles = 1;
      g.split = 1;
      g.direct = false;
      g.kws = false;
      g.pointwise = false;
      g.pack_bytes = (d->flags & CTMR_F_AFFINE) ? round_up((int64_t)d->n * d->cin * 2 * 4, 256) : 0;
      g.part_bytes = 0;
      g.z_bytes = 0;
      if ((int64_t)g.m_tiles * d->n * 256 >= (1ll << 32)) return fail(CTMR_E_UNSUPPORTED, "grid too large");
      return CTMR_OK;
    }
  }
  // LDS-staged GEMM: stride-1 fp32 volumes whose 4x8x8 bricks are at least
  // 3/4 full, with at least 64 input channels (4 staged chunks; measured on
  // MI355X: 64-channel UNet-level convs 3-6 % faster than the streaming GEMM
  // with or without its pack pass; below that the per-chunk staging and
  // barriers dominate), 64-wide column tiles, at least 4 chunks per split, and
  // 6 staged planes within 32-bit buffer offsets.
  g.lds = false;
  g.wsets = 1;
  g.lds16 = false;
  g.small_out = false;
  if (g.layout == WL_TAPS && d->dtype == CTMR_F32 && d->ksize == 3 && d->stride == 1 &&
      d->mode == CTMR_MODE_PLAIN && d->cin % 16 == 0 && d->cin >= 64 && d->cout % 64 == 0 &&
      !(d->flags & (CTMR_F_STREAM | CTMR_F_SPLIT_WAVES))) {
    g.tz = (int)ceil_div(d->d, kBD);
    g.ty = (int)ceil_div(d->h, kBH);
    g.tx = (int)ceil_div(d->w, kBW);
    const int64_t slots = (int64_t)g.tz * g.ty * g.tx * kBD * kBH * kBW;
    const int64_t planes = (int64_t)kHD * d->h * d->w * d->cin * 4;
    // The policy split (below) must leave each workgroup at least 4 chunks:
    // with fewer, the exposed first-chunk staging outweighs the saved pack
    // (measured on the UNet's 16x16x8 level: streaming 68 % vs LDS 63 %).
    const int64_t base = (int64_t)g.tz * g.ty * g.tx * (d->cout / 64) * d->n;
    const int64_t policy_split = lds_policy_split(base, d->cin / 16);
    const int64_t split = d->split > 0 ? d->split : policy_split;
    if (4 * S >= 3 * slots && planes < (1ll << 31) && brick_out_fits && (d->cin / 16) / split >= 4) g.lds = true;
  }
  if (g.lds) {
    g.pack = false;
    g.cp = d->cin;
    g.kblocks = d->cin / 16;
    g.nsub = 4; g.wm = 4; g.wn = 1;
    g.m_tiles = g.tz * g.ty * g.tx;
    g.n_tiles = d->cout / 64;
    const int chunks = g.kblocks;
    if (d->split > 0) {
      if (d->split > chunks) return fail(CTMR_E_INVALID, "split must not exceed the 16-channel chunk count");
      g.split = d->split;
    } else {
      const int64_t base = (int64_t)g.m_tiles * g.n_tiles * d->n;
      g.split = (int)lds_policy_split(base, chunks);
    }
    // A split of two over an even chunk count runs as two wave sets of one
    // workgroup (the same K ranges and output bits, no partial planes and no
    // reduction launch; group-norm partials per brick as without a split).
    g.wsets = (g.split == 2 && chunks % 2 == 0) ? 2 : 1;
    g.pack_bytes = (d->flags & CTMR_F_AFFINE) ? round_up((int64_t)d->n * d->cin * 2 * 4, 256) : 0;
    g.part_bytes = (g.split > 1 && g.wsets == 1) ? (int64_t)g.split * d->n * s_out * d->cout * 4 : 0;
    const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * d->n * (g.wsets == 2 ? 1 : g.split) * g.wsets;
    if (blocks * 256 >= (1ll << 32)) return fail(CTMR_E_UNSUPPORTED, "grid too large");
    return CTMR_OK;
  }
  // LDS-staged bf16 GEMM: stride-1 bf16 convs (plain or trilinear-2x, both
  // sampled by the pack, or nearest-2x as 8 parity GEMMs over the packed
  // source) with 64-wide column tiles whose 4x8x8 bricks (of the source grid
  // for nearest-2x) are at least half full: even with half its rows masked
  // (the UNet's 8x8x4 level) it outruns the register-streaming bf16 GEMM
  // (bf16 UNet step from a HIP graph 5.91 -> 5.71 ms against a 3/4 bound);
  // the halo fill's 32-bit offsets span 6 packed planes.
  g.lds16 = false;
  g.small_out = false;
  if (g.layout == WL_TAPS && (d->dtype == CTMR_BF16 || d->dtype == CTMR_F16X2) && d->ksize == 3 &&
      d->stride == 1 && d->cout % 64 == 0 && !(d->flags & (CTMR_F_STREAM | CTMR_F_SPLIT_WAVES))) {
    const int tz = (int)ceil_div(g.gd, kBD), ty = (int)ceil_div(g.gh, kBH), tx = (int)ceil_div(g.gw, kBW);
    const int64_t slots = (int64_t)tz * ty * tx * kBD * kBH * kBW;
    const int64_t planes = (int64_t)kHD * g.P * g.cp * g.esize;
    const int64_t w_bytes = (int64_t)g.taps * g.phases * g.kblocks * g.np * (d->dtype == CTMR_F16X2 ? 96 : 64);
    if (2 * S >= slots && planes < (1ll << 31) && w_bytes < (1ll << 31) && brick_out_fits) {
      g.lds16 = true;
      g.tz = tz; g.ty = ty; g.tx = tx;
    }
  }
  // Split fp16 runs only on the LDS-staged 16-bit GEMM.
  if (d->dtype == CTMR_F16X2 && !g.lds16)
    return fail(CTMR_E_UNSUPPORTED,
                "split fp16 (CTMR_F16X2) needs a stride-1 3x3x3 conv with cin >= 16, cout % 64 == 0, 4x8x8 bricks "
                "at least half full and no CTMR_F_STREAM");
  // Plain fp32 3x3x3 convs whose channels fill whole 16-channel K blocks
  // need no packed copy: the streaming GEMM reads x itself, with out-of-range
  // offsets for taps outside the volume (the padded copy's zeros).  Its lane
  // offsets are 32-bit: one batch item must stay below 2 GiB.
  g.direct = !g.lds16 && !g.cat && g.layout == WL_TAPS && d->dtype == CTMR_F32 && d->ksize == 3 &&
             d->mode == CTMR_MODE_PLAIN && !(d->flags & (CTMR_F_AFFINE | CTMR_F_SILU)) && d->cin % 16 == 0 &&
             (int64_t)d->d * d->h * d->w * d->cin * 4 < (1ll << 31) - (1ll << 20);
  if (g.direct) {
    g.pack = false;
    g.cp = d->cin;
    g.kblocks = d->cin / 16;
    g.Q = d->w;
    g.P = d->h * d->w;
    g.rows_per_batch = (int64_t)d->d * g.P;
  }
  // Tile shape by GEMM width.
  if (g.lds16) { g.nsub = 4; g.wm = 4; g.wn = 1; }
  else if (g.ncols <= 16) { g.nsub = 1; g.wm = 4; g.wn = 1; }
  else if (g.ncols <= 32) { g.nsub = 2; g.wm = 4; g.wn = 1; }
  else if (g.ncols <= 64) { g.nsub = 4; g.wm = 4; g.wn = 1; }
  else { g.nsub = 4; g.wm = 2; g.wn = 2; }
  g.m_tiles = g.lds16 ? g.tz * g.ty * g.tx : (int)ceil_div(S, g.wm * 64);
  g.n_tiles = (int)ceil_div(g.np, g.wn * g.nsub * 16);
  // K split: the (tap, channel-block) step sequence of every output is cut
  // into `split` contiguous ranges whose fp32 partial planes are summed in
  // ascending order.  Chosen from the shape only (never from the device), so
  // each output's summation order is fixed for a given problem.  Small grids
  // are split so the launch fills whole rounds of 512 resident workgroups
  // (two per CU on 256 CUs), keeping at least 8 steps per range.
  const int steps = g.taps * g.kblocks;
  if (g.layout == WL_EXPAND) {
    if (d->split > 1) return fail(CTMR_E_INVALID, "split must be 1 for the cout <= 4 tap-expanded GEMM");
    g.split = 1;
  } else if (g.lds16) {  // chunk-range split, as the fp32 LDS GEMM
    if (d->split > g.kblocks) return fail(CTMR_E_INVALID, "split must not exceed the chunk count");
    const int64_t base = (int64_t)g.m_tiles * g.n_tiles * d->n * g.phases;
    g.split = d->split > 0 ? d->split
                           : (base < 512 ? (int)std::min<int64_t>(ceil_div(512, base), g.kblocks) : 1);
    // A split of two over an even chunk count runs as two wave sets of one
    // workgroup (same output bits, no partial planes, no reduction launch).
    g.wsets = (g.split == 2 && g.kblocks % 2 == 0) ? 2 : 1;
  } else if (d->split > 0) {
    if (d->split > steps) return fail(CTMR_E_INVALID, "split must not exceed the K step count");
    g.split = d->split;
  } else {
    // The persistent one-tap GEMM (below) keeps every resident workgroup busy
    // once a launch has 256 tiles: splitting it further only adds the partial
    // planes and their reduction (measured on MI355X: the 32x32x16-level
    // 384 -> 128 skip projection 49.5 us with a split of 2, 35.5 us without;
    // the 16x16x8- and 8x8x4-level ones fastest at 256 / base ranges).
    const bool one_tap = g.KT == 1 && g.nsub == 4 && g.layout != WL_EXPAND && d->cout % 4 == 0 &&
                         !(d->flags & (CTMR_F_STREAM | CTMR_F_BATCH_BIAS | CTMR_F_RESIDUAL));
    const int64_t base = (int64_t)g.m_tiles * g.n_tiles * d->n * g.phases;
    const int64_t slots = one_tap ? 256 : 512;
    g.split = 1;
    if (base < slots && steps >= 16) {
      g.split = (int)std::min<int64_t>(ceil_div(slots, base), std::max(1, steps / 8));
    }
  }
  // Deep small grids (library policy, 3x3x3 or nearest-2x, a split of at least
  // 4): 64 x 64 tiles with the four waves summing quarters of each split range
  // need a quarter of the partial planes.  Chosen only while that leaves at
  // least 2 planes (the waves' quarter sums go to a partial plane; the bias,
  // residual and statistics come from the reduction) and 8 steps per wave.
  g.kws = false;
  if (d->flags & CTMR_F_SPLIT_WAVES) {  // this form with the caller's split (a depth slab of such a conv)
    if (g.layout != WL_TAPS || g.lds16 || g.KT == 1 || d->split < 2 || d->split > steps / 32)
      return fail(CTMR_E_INVALID, "CTMR_F_SPLIT_WAVES needs a 3x3x3 or nearest-2x streaming GEMM and a split of "
                                  "2 .. (taps * K blocks) / 32");
    g.kws = true;
    g.nsub = 4; g.wm = 1; g.wn = 1;
    g.m_tiles = (int)ceil_div(S, 64);
    g.n_tiles = (int)ceil_div(g.np, 64);
    g.split = d->split;
    g.wsets = g.split == 2 ? 2 : 1;
  } else if (d->split == 0 && g.layout == WL_TAPS && !g.lds16 && g.KT != 1 && g.split >= 4) {
    const int64_t mt = ceil_div(S, 64), nt = ceil_div(g.np, 64);
    const int64_t base1 = mt * nt * d->n * g.phases;
    const int64_t split1 = std::min<int64_t>(ceil_div(512, base1), steps / 32);
    if (split1 >= 2) {
      g.kws = true;
      g.nsub = 4; g.wm = 1; g.wn = 1;
      g.m_tiles = (int)mt;
      g.n_tiles = (int)nt;
      g.split = (int)split1;
      // A split of two runs as two wave sets of one workgroup: the same K
      // ranges and output bits, no partial planes and no reduction launch.
      g.wsets = g.split == 2 ? 2 : 1;
    }
  }
  const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * d->n * g.phases * g.split;
  if (blocks * 256 >= (1ll << 32)) return fail(CTMR_E_UNSUPPORTED, "grid too large");
  // One-tap GEMMs (1x1x1, im2col) with 64-column wave tiles walk their tiles
  // persistently over an LDS ring; per-batch bias, residual and the planar
  // tap-expanded output stay on conv_kernel.
  g.pointwise = g.KT == 1 && g.nsub == 4 && g.layout != WL_EXPAND && d->cout % 4 == 0 &&
                !(d->flags & (CTMR_F_STREAM | CTMR_F_BATCH_BIAS | CTMR_F_RESIDUAL));
  g.pack_bytes = g.pack ? round_up((int64_t)d->n * g.rows_per_batch * g.cp * g.esize, 256) : 0;
  g.part_bytes = (g.split > 1 && g.wsets == 1) ? (int64_t)g.split * d->n * s_out * d->cout * 4 : 0;
  if (g.layout == WL_EXPAND) g.z_bytes = (int64_t)g.ncols * d->n * g.rows_per_batch * 4;
  return CTMR_OK;
}

// Per-batch-item partial count of ctmr_conv3d_gn for `groups`, or 0 when the
// epilogue cannot produce them: a K split (partial planes, not outputs), the
// tap-expanded cout <= 4 GEMM (outputs come from the tap sum), or a group that
// does not divide the workgroup's column tile.
// On a K split the partials come from split_reduce_gn_kernel, one per chunk of
// 16 * split_gn_rows() output voxels; the row count keeps about 1024 blocks.
static int split_gn_rows(const ctmr_conv_desc* d, const Geometry& g) {
  const int64_t s_out = (int64_t)g.od * g.oh * g.ow;
  const int64_t rows = s_out * (d->cout / 64) * d->n / (16 * 1024);
  return (int)std::min<int64_t>(std::max<int64_t>(rows, 1), 16);
}

static int gn_stats_tiles(const ctmr_conv_desc* d, const Geometry& g, int groups) {
  if (groups <= 0 || d->cout % groups != 0) return 0;
  if (g.layout == WL_EXPAND) return 0;
  if (g.lds_small) {  // 64-column bricks only (the narrow epilogue writes no statistics)
    const int cpg = d->cout / groups;
    return (g.nsub == 4 && cpg <= 64 && 64 % cpg == 0) ? g.tz * g.ty * g.tx : 0;
  }
  const int cpg = d->cout / groups;
  if (g.split > 1 && g.wsets == 1) {
    if (d->cout % 64 != 0 || 64 % cpg != 0) return 0;
    const int64_t s_out = (int64_t)g.od * g.oh * g.ow, per = 16 * (int64_t)split_gn_rows(d, g);
    const int64_t chunks = (s_out + per - 1) / per;
    return chunks > 65535 ? 0 : (int)chunks;
  }
  const int width = g.lds ? 64 : g.wn * g.nsub * 16;
  if (cpg > width || width % cpg != 0) return 0;
  return (g.lds || g.lds16) ? g.tz * g.ty * g.tx * g.phases : g.m_tiles * g.phases;
}

// The K-split reduction, with group-norm partials when `stats` is set.
static void launch_split_reduce(const ctmr_conv_desc* d, const Geometry& g, const float* part, int64_t plane,
                                const float* bias, int batch_bias, const float* residual, float* y,
                                int64_t s_out, int groups, double* stats, hipStream_t st) {
  const float* res = (d->flags & CTMR_F_RESIDUAL) ? residual : nullptr;
  if (!stats) {
    hipLaunchKernelGGL(split_reduce_kernel, dim3(elementwise_blocks(plane)), dim3(256), 0, st, part, plane,
                       g.split, bias, bias != nullptr ? 1 : 0, batch_bias, res, y, d->cout, s_out);
    return;
  }
  const int rows = split_gn_rows(d, g), chunks = gn_stats_tiles(d, g, groups);
  hipLaunchKernelGGL(split_reduce_gn_kernel, dim3((unsigned)chunks * (d->cout / 64), d->n), dim3(256), 0, st,
                     part, plane, g.split, bias, bias != nullptr ? 1 : 0, batch_bias, res, y, d->cout, s_out,
                     rows, chunks, d->cout / groups, groups, stats);
}

typedef void (*ConvFn)(dim3, dim3, hipStream_t, const ConvArgs&);

// conv_lds_bf16_kernel, nearest-2x parity form or not.
template <int DT, int WS>
static void launch_lds16(bool up, dim3 grid, hipStream_t st, const Lds16Args& a) {
  if (up) hipLaunchKernelGGL((conv_lds_bf16_kernel<DT, true, WS>), grid, dim3(256 * WS), 0, st, a);
  else hipLaunchKernelGGL((conv_lds_bf16_kernel<DT, false, WS>), grid, dim3(256 * WS), 0, st, a);
}

// conv_lds_kernel for a staging transform xf (bit 0 affine, bit 1 SiLU).
template <bool TWO, int WS>
static void launch_lds(int xf, dim3 grid, hipStream_t st, const LdsArgs& a) {
  const dim3 block(256 * WS);
  switch (xf) {
    case 0: hipLaunchKernelGGL((conv_lds_kernel<TWO, 0, WS>), grid, block, 0, st, a); break;
    case 1: hipLaunchKernelGGL((conv_lds_kernel<TWO, 1, WS>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((conv_lds_kernel<TWO, 2, WS>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((conv_lds_kernel<TWO, 3, WS>), grid, block, 0, st, a); break;
  }
}

// The 64-column register-streaming GEMM is tuned for two resident workgroups
// per CU (two waves per SIMD; its split policy and round sizes assume 512 per
// launch).  Its ~160 VGPRs would let a third in, which measured slower
// (config 0: 0.533 ms against 0.443 ms), so the launch reserves LDS it does
// not use: 60 KiB + 4 KiB of partial buffers per workgroup, two per 160 KiB CU.
constexpr size_t kConvTwoPerCuLds = 60 * 1024;

template <int DT, int NSUB, int WM, int WN, int KT, int STRIDE, bool UP, bool DIRECT = false, int KWS = 1,
          int SETS = 1>
static void launch_conv(dim3 grid, dim3, hipStream_t st, const ConvArgs& a) {
  // KWS = 4 holds 48 KiB of quarter sums in LDS: 8 KiB more keeps it at two per CU.  Two wave sets (512
  // threads, 96 KiB of quarter sums) run one per CU.
  hipLaunchKernelGGL((conv_kernel<DT, NSUB, WM, WN, KT, STRIDE, UP, DIRECT, KWS, SETS>), grid, dim3(256 * SETS),
                     SETS == 2 ? 0 : KWS > 1 ? 8 * 1024 : NSUB == 4 ? kConvTwoPerCuLds : 0, st, a);
}

// Compute units of the current device (cached per device).
static int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  static int cache[64];
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// The persistent pointwise GEMM runs as many row lanes of n_tiles workgroups
// as the device holds at once (capped by the item count).  Each tile is summed
// by one wave in a fixed order whatever the grid, so the grid may follow the
// device without changing a bit of the output.
template <int DT, int WM, int WN, bool TWO>
static void launch_pointwise(dim3, dim3 block, hipStream_t st, const ConvArgs& a) {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pointwise_kernel<DT, WM, WN, TWO>, 256, 0) !=
            hipSuccess ||
        n <= 0)
      n = 2;
    return n;
  }();
  const int64_t lanes = std::min<int64_t>(a.items, std::max(1, per_cu * device_cus() / a.n_tiles));
  hipLaunchKernelGGL((pointwise_kernel<DT, WM, WN, TWO>), dim3((unsigned)(lanes * a.n_tiles)), block, 0, st, a);
}

template <int DT, int NSUB, int WM, int WN>
static ConvFn pick_kind(int KT, int stride, bool up) {
  if (up) return launch_conv<DT, NSUB, WM, WN, 2, 1, true>;
  if (KT == 1) return launch_conv<DT, NSUB, WM, WN, 1, 1, false>;
  if (stride == 2) return launch_conv<DT, NSUB, WM, WN, 3, 2, false>;
  return launch_conv<DT, NSUB, WM, WN, 3, 1, false>;
}

template <int DT, int NSUB, int WM, int WN>
static ConvFn pick_kind(const Geometry& g, int stride, bool up) {
  if constexpr (WM * WN == 1) {  // the K split over the four waves (g.kws), in one or two wave sets
    if (g.wsets == 2) {
      if constexpr (DT == CTMR_F32) {
        if (g.direct) return stride == 2 ? launch_conv<DT, NSUB, 1, 1, 3, 2, false, true, 4, 2>
                                         : launch_conv<DT, NSUB, 1, 1, 3, 1, false, true, 4, 2>;
      }
      if (up) return launch_conv<DT, NSUB, 1, 1, 2, 1, true, false, 4, 2>;
      if (stride == 2) return launch_conv<DT, NSUB, 1, 1, 3, 2, false, false, 4, 2>;
      return launch_conv<DT, NSUB, 1, 1, 3, 1, false, false, 4, 2>;
    }
    if constexpr (DT == CTMR_F32) {
      if (g.direct) return stride == 2 ? launch_conv<DT, NSUB, 1, 1, 3, 2, false, true, 4>
                                       : launch_conv<DT, NSUB, 1, 1, 3, 1, false, true, 4>;
    }
    if (up) return launch_conv<DT, NSUB, 1, 1, 2, 1, true, false, 4>;
    if (stride == 2) return launch_conv<DT, NSUB, 1, 1, 3, 2, false, false, 4>;
    return launch_conv<DT, NSUB, 1, 1, 3, 1, false, false, 4>;
  } else {
    if constexpr (NSUB == 4) {
      if constexpr (DT == CTMR_F32) {
        if (g.pointwise && g.cat && !g.pack) return launch_pointwise<DT, WM, WN, true>;
      }
      if (g.pointwise) return launch_pointwise<DT, WM, WN, false>;
    }
    if constexpr (DT == CTMR_F32) {
      if (g.direct) return stride == 2 ? launch_conv<DT, NSUB, WM, WN, 3, 2, false, true>
                                       : launch_conv<DT, NSUB, WM, WN, 3, 1, false, true>;
    }
    return pick_kind<DT, NSUB, WM, WN>(g.KT, stride, up);
  }
}

static ConvFn pick(const ctmr_conv_desc* d, const Geometry& g) {
  const bool up = d->mode == CTMR_MODE_NEAREST2X;
  const int st = d->stride;
#define CTMR_PICK(DT)                                                            \
  if (g.kws) return pick_kind<DT, 4, 1, 1>(g, st, up);                           \
  if (g.nsub == 1) return pick_kind<DT, 1, 4, 1>(g, st, up);                     \
  if (g.nsub == 2) return pick_kind<DT, 2, 4, 1>(g, st, up);                     \
  if (g.wn == 1) return pick_kind<DT, 4, 4, 1>(g, st, up);                       \
  return pick_kind<DT, 4, 2, 2>(g, st, up);
  if (d->dtype == CTMR_F32) {
    CTMR_PICK(CTMR_F32)
  } else {
    CTMR_PICK(CTMR_BF16)
  }
#undef CTMR_PICK
}

}  // namespace ctmr

using namespace ctmr;

extern "C" {

int ctmr_abi_version(void) { return CTMR_ABI_VERSION; }

const char* ctmr_last_error(void) { return g_error; }

int ctmr_conv3d_output_dims(const ctmr_conv_desc* desc, int32_t out[3]) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (!out) return fail(CTMR_E_INVALID, "null output");
  out[0] = g.od; out[1] = g.oh; out[2] = g.ow;
  return CTMR_OK;
}

// Packed-weight geometry of a split-fp16 (CTMR_F16X2) weight, which does not
// depend on the input grid: [phase][tap][16-channel block][np][96 bytes], then
// np fp32 column scales.
static int split_weight_layout(const ctmr_conv_desc* d, int& phases, int& taps, int& kblocks, int& np,
                               int64_t& block_bytes) {
  if (!d) return fail(CTMR_E_INVALID, "null descriptor");
  if (d->cin <= 0 || d->cout <= 0) return fail(CTMR_E_INVALID, "non-positive dimension");
  if (d->ksize != 3) return fail(CTMR_E_UNSUPPORTED, "split fp16 (CTMR_F16X2) supports only 3x3x3 weights");
  if (d->mode < CTMR_MODE_PLAIN || d->mode > CTMR_MODE_TRILINEAR2X) return fail(CTMR_E_INVALID, "bad mode");
  phases = d->mode == CTMR_MODE_NEAREST2X ? 8 : 1;
  taps = d->mode == CTMR_MODE_NEAREST2X ? 8 : 27;
  kblocks = (int)ceil_div(d->cin, 16);
  np = (int)round_up(d->cout, 16);
  block_bytes = (int64_t)phases * taps * kblocks * np * 96;
  return CTMR_OK;
}

int64_t ctmr_packed_weight_elems(const ctmr_conv_desc* desc) {
  if (desc && desc->dtype == CTMR_F16X2) {
    int phases, taps, kblocks, np;
    int64_t bytes;
    const int rc = split_weight_layout(desc, phases, taps, kblocks, np, bytes);
    if (rc) return rc;
    return (bytes + (int64_t)np * 4) / 2;
  }
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  const int kblocks = g.layout == WL_IM2COL ? g.kblocks : (int)ceil_div(desc->cin, g.kstep);
  return (int64_t)g.phases * g.taps * kblocks * g.np * g.kstep;
}

int64_t ctmr_conv3d_workspace_bytes(const ctmr_conv_desc* desc) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  return g.pack_bytes + g.part_bytes + g.z_bytes;
}

int ctmr_conv3d_split(const ctmr_conv_desc* desc) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  return g.split;
}

int ctmr_conv3d_kernel(const ctmr_conv_desc* desc) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (g.lds) return CTMR_K_LDS;
  if (g.lds_small) return CTMR_K_LDS_SMALL;
  if (g.lds16) return desc->dtype == CTMR_F16X2 ? CTMR_K_LDS_F16X2 : CTMR_K_LDS_BF16;
  if (g.small_out) return CTMR_K_SMALL_COUT;
  if (g.layout == WL_EXPAND) return CTMR_K_TAP_EXPAND;
  if (g.kws) return CTMR_K_SPLIT_WAVES;
  if (g.pointwise) return CTMR_K_POINTWISE;
  return g.direct ? CTMR_K_STREAM_DIRECT : CTMR_K_STREAM;
}

static int pack_weight_impl(const ctmr_conv_desc* desc, const float* weight, void* packed,
                            void* stream, bool up) {
  if (desc && desc->dtype == CTMR_F16X2) {
    WPackArgs a;
    int64_t bytes;
    int rc = split_weight_layout(desc, a.phases, a.taps, a.kblocks, a.np, bytes);
    if (rc) return rc;
    if (!weight || !packed) return fail(CTMR_E_INVALID, "null pointer");
    if (up != (desc->mode == CTMR_MODE_NEAREST2X))
      return fail(CTMR_E_INVALID, up ? "ctmr_pack_upsample_weight needs CTMR_MODE_NEAREST2X"
                                     : "use ctmr_pack_upsample_weight for CTMR_MODE_NEAREST2X");
    if (((uintptr_t)packed & 15) != 0) return fail(CTMR_E_INVALID, "packed weight must be 16-byte aligned");
    a.w = weight;
    a.out = packed;
    a.cout = desc->cout;
    a.cin = desc->cin;
    a.ks = 3;
    a.kstep = 16;
    a.up = up ? 1 : 0;
    a.bf16 = 0;
    a.layout = WL_TAPS;
    a.colscale = reinterpret_cast<float*>(reinterpret_cast<char*>(packed) + bytes);
    a.total = (int64_t)a.phases * a.taps * a.kblocks * a.np * 16;
    hipLaunchKernelGGL(weight_colscale_kernel, dim3((unsigned)a.np), dim3(256), 0, (hipStream_t)stream, a);
    if ((rc = check_launch("weight_colscale"))) return rc;
    hipLaunchKernelGGL(pack_weight_split_kernel, dim3(elementwise_blocks(a.total)), dim3(256), 0,
                       (hipStream_t)stream, a);
    return check_launch("pack_weight_split");
  }
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (!weight || !packed) return fail(CTMR_E_INVALID, "null pointer");
  if (up != (desc->mode == CTMR_MODE_NEAREST2X))
    return fail(CTMR_E_INVALID, up ? "ctmr_pack_upsample_weight needs CTMR_MODE_NEAREST2X"
                                   : "use ctmr_pack_upsample_weight for CTMR_MODE_NEAREST2X");
  WPackArgs a;
  a.phases = g.phases;
  a.colscale = nullptr;
  a.w = weight;
  a.out = packed;
  a.cout = desc->cout;
  a.cin = desc->cin;
  a.ks = desc->ksize;
  a.np = g.np;
  a.kstep = g.kstep;
  a.kblocks = g.layout == WL_IM2COL ? g.kblocks : (int)ceil_div(desc->cin, g.kstep);
  a.taps = g.taps;
  a.up = up ? 1 : 0;
  a.bf16 = desc->dtype == CTMR_BF16;
  a.layout = g.layout;
  a.total = (int64_t)g.phases * g.taps * a.kblocks * g.np * g.kstep;
  hipLaunchKernelGGL(pack_weight_kernel, dim3(elementwise_blocks(a.total)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("pack_weight");
}

int ctmr_pack_weight(const ctmr_conv_desc* desc, const float* weight, void* packed, void* stream) {
  return pack_weight_impl(desc, weight, packed, stream, false);
}

int ctmr_pack_upsample_weight(const ctmr_conv_desc* desc, const float* weight, void* packed,
                              void* stream) {
  return pack_weight_impl(desc, weight, packed, stream, true);
}

static int check_workspace(const Geometry& g, const void* workspace, size_t workspace_bytes) {
  const int64_t need = g.pack_bytes + g.part_bytes + g.z_bytes;
  if ((int64_t)workspace_bytes < need || (need > 0 && !workspace)) {
    set_error("workspace %zu bytes < required %lld", workspace_bytes, (long long)need);
    return CTMR_E_WORKSPACE;
  }
  return CTMR_OK;
}

static int pack_impl(const ctmr_conv_desc* desc, const float* x, const float* x2, const float* affine,
                     void* workspace, size_t workspace_bytes, void* stream);

int ctmr_conv3d_pack(const ctmr_conv_desc* desc, const float* x, const float* affine,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (desc && desc->cin1 != 0) return fail(CTMR_E_INVALID, "two-source input: use ctmr_conv3d_cat");
  return pack_impl(desc, x, nullptr, affine, workspace, workspace_bytes, stream);
}

// x2: channels [cin1, cin) of a two-source input (desc->cin1 != 0), else null.
static int pack_impl(const ctmr_conv_desc* desc, const float* x, const float* x2, const float* affine,
                     void* workspace, size_t workspace_bytes, void* stream) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (!x || (g.cat && !x2)) return fail(CTMR_E_INVALID, "null input");
  if ((desc->flags & CTMR_F_AFFINE) && !affine) return fail(CTMR_E_INVALID, "affine flag without affine");
  if ((rc = check_workspace(g, workspace, workspace_bytes))) return rc;
  if (g.lds || g.lds_small || g.small_out) {
    if (!(desc->flags & CTMR_F_AFFINE)) return CTMR_OK;
    if (hipMemcpyAsync(workspace, affine, (size_t)desc->n * desc->cin * 2 * 4, hipMemcpyDeviceToDevice,
                       (hipStream_t)stream) != hipSuccess)
      return fail(CTMR_E_LAUNCH, "affine copy failed");
    return CTMR_OK;
  }
  if (!g.pack) return CTMR_OK;
  if (g.layout == WL_IM2COL) {
    Im2colArgs ia;
    ia.x = x;
    ia.out = workspace;
    ia.affine = affine;
    ia.d = g.td; ia.h = g.th; ia.w = g.tw;
    ia.sd = desc->d; ia.sh = desc->h; ia.sw = desc->w;
    ia.trilinear = desc->mode == CTMR_MODE_TRILINEAR2X;
    ia.c = desc->cin;
    ia.cp = g.cp;
    ia.od = g.od; ia.oh = g.oh; ia.ow = g.ow;
    ia.stride = desc->stride;
    ia.affine_on = (desc->flags & CTMR_F_AFFINE) != 0;
    ia.silu_on = (desc->flags & CTMR_F_SILU) != 0;
    ia.bf16 = desc->dtype == CTMR_BF16;
    ia.total4 = (int64_t)desc->n * g.rows_per_batch * (g.cp / 4);
    hipLaunchKernelGGL(im2col_kernel, dim3(elementwise_blocks(ia.total4)), dim3(256), 0,
                       (hipStream_t)stream, ia);
    return check_launch("im2col");
  }
  if ((desc->cin & 3) == 0 && (((uintptr_t)x | (g.cat ? (uintptr_t)x2 : 0)) & 15) != 0)
    return fail(CTMR_E_INVALID, "x must be 16-byte aligned");
  PackArgs pa;
  pa.x = x;
  pa.x2 = g.cat ? x2 : nullptr;
  pa.c1 = g.c1;
  pa.out = workspace;
  pa.affine = affine;
  pa.gd = g.td; pa.gh = g.th; pa.gw = g.tw;
  pa.halo = g.halo;
  pa.c = desc->cin;
  pa.cp = g.cp;
  pa.id = desc->d; pa.ih = desc->h; pa.iw = desc->w;
  pa.affine_on = (desc->flags & CTMR_F_AFFINE) != 0;
  pa.silu_on = (desc->flags & CTMR_F_SILU) != 0;
  pa.trilinear = desc->mode == CTMR_MODE_TRILINEAR2X;
  pa.bf16 = desc->dtype == CTMR_BF16;
  pa.split16 = desc->dtype == CTMR_F16X2;
  pa.total4 = (int64_t)desc->n * g.rows_per_batch * (g.cp / 4);
  pa.n = desc->n;
  const int64_t plane_items =
      (int64_t)(g.th + 2 * g.halo) * (g.tw + 2 * g.halo) * (g.cp / (pa.bf16 || pa.split16 ? 8 : 4));
  const int64_t planes = (int64_t)desc->n * (g.td + 2 * g.halo);
  if (plane_items >= (1ll << 31)) return fail(CTMR_E_UNSUPPORTED, "padded plane too large for the pack");
  const bool vec = (desc->cin & 3) == 0 && (!pa.affine_on || ((uintptr_t)affine & 15) == 0);
  if (vec && pa.trilinear && !g.cat && g.halo == 1) {
    // one thread per (source cell, channel group), cells over [-1, n] per axis
    // runs of 8 cells along z; one cell per thread where runs of 8 would
    // leave under ~4 waves per SIMD (no serial chain of loads)
    const int64_t cells = (int64_t)(desc->h + 2) * (desc->w + 2) * (g.cp / 4);
    if (cells >= (1ll << 31)) return fail(CTMR_E_UNSUPPORTED, "source plane too large for the pack");
    const bool long_runs = cells * desc->n * ceil_div(desc->d + 2, 8) >= (1ll << 18);
    const int zc = long_runs ? 8 : 1;
    const int64_t runs = (int64_t)desc->n * ceil_div(desc->d + 2, zc);
    const dim3 grid((unsigned)ceil_div(cells, 256), (unsigned)std::min<int64_t>(runs, 65535));
    const hipStream_t ts = (hipStream_t)stream;
    if (long_runs) {
      if (pa.split16) hipLaunchKernelGGL((pack_trilinear_kernel<PF_SPLIT, 8>), grid, dim3(256), 0, ts, pa);
      else if (pa.bf16) hipLaunchKernelGGL((pack_trilinear_kernel<PF_BF16, 8>), grid, dim3(256), 0, ts, pa);
      else hipLaunchKernelGGL((pack_trilinear_kernel<PF_F32, 8>), grid, dim3(256), 0, ts, pa);
    } else {
      if (pa.split16) hipLaunchKernelGGL((pack_trilinear_kernel<PF_SPLIT, 1>), grid, dim3(256), 0, ts, pa);
      else if (pa.bf16) hipLaunchKernelGGL((pack_trilinear_kernel<PF_BF16, 1>), grid, dim3(256), 0, ts, pa);
      else hipLaunchKernelGGL((pack_trilinear_kernel<PF_F32, 1>), grid, dim3(256), 0, ts, pa);
    }
    return check_launch("pack_trilinear");
  }
  if (vec && !pa.trilinear) {
    // Four planes per thread; copies that would then fill under four
    // workgroups per CU (the deep levels' 1-4 MB copies) take one plane per
    // thread, four times the workgroups and a quarter of each thread's chain.
    const int64_t gx = ceil_div(plane_items, 256);
    const bool one = gx * ceil_div(planes, 4) < 4 * (int64_t)device_cus();
    const dim3 grid((unsigned)gx, (unsigned)std::min<int64_t>(ceil_div(planes, one ? 1 : 4), 65535));
    const hipStream_t ps = (hipStream_t)stream;
    if (pa.split16) {
      if (one) hipLaunchKernelGGL((pack_planes_kernel<2, 1, true>), grid, dim3(256), 0, ps, pa);
      else hipLaunchKernelGGL((pack_planes_kernel<2, 4, true>), grid, dim3(256), 0, ps, pa);
    } else if (pa.bf16) {
      if (one) hipLaunchKernelGGL((pack_planes_kernel<2, 1>), grid, dim3(256), 0, ps, pa);
      else hipLaunchKernelGGL((pack_planes_kernel<2, 4>), grid, dim3(256), 0, ps, pa);
    } else {
      if (one) hipLaunchKernelGGL((pack_planes_kernel<1, 1>), grid, dim3(256), 0, ps, pa);
      else hipLaunchKernelGGL((pack_planes_kernel<1, 4>), grid, dim3(256), 0, ps, pa);
    }
    return check_launch("pack_planes");
  }
  hipLaunchKernelGGL(pack_input_kernel,
                     dim3((unsigned)ceil_div(plane_items, 256), (unsigned)std::min<int64_t>(planes, 65535)),
                     dim3(256), 0, (hipStream_t)stream, pa);
  return check_launch("pack_input");
}

static int conv3d_gemm_impl(const ctmr_conv_desc* desc, const float* x, const float* x2, const void* packed,
                            const float* bias, const float* affine_direct, const float* residual, float* y,
                            void* workspace, size_t workspace_bytes, int groups, double* stats, void* stream);

int ctmr_conv3d_gemm(const ctmr_conv_desc* desc, const float* x, const void* packed,
                     const float* bias, const float* residual, float* y, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (desc && desc->cin1 != 0) return fail(CTMR_E_INVALID, "two-source input: use ctmr_conv3d_cat");
  return conv3d_gemm_impl(desc, x, nullptr, packed, bias, nullptr, residual, y, workspace, workspace_bytes, 0,
                          nullptr, stream);
}

// affine_direct: the caller's (n, cin, 2) table when the pack stage was skipped
// (ctmr_conv3d on the LDS path); null means "read it from the workspace".
// stats: group-norm partials for `groups` (validated by the caller) or null.
static int conv3d_gemm_impl(const ctmr_conv_desc* desc, const float* x, const float* x2, const void* packed,
                            const float* bias, const float* affine_direct, const float* residual, float* y,
                            void* workspace, size_t workspace_bytes, int groups, double* stats, void* stream) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (g.cat && !g.pack && !g.lds && !g.pointwise && !g.small_out)
    return fail(CTMR_E_UNSUPPORTED, "internal: unpacked two-source input on a route that reads one tensor");
  if (g.cat && !g.pack && (!x2 || ((uintptr_t)x2 & 15) != 0))
    return fail(CTMR_E_INVALID, "x2 must be non-null and 16-byte aligned");
  const int tiles = stats ? gn_stats_tiles(desc, g, groups) : 0;
  if (stats && tiles == 0) return fail(CTMR_E_UNSUPPORTED, "this convolution cannot produce group-norm partials");
  if (!packed || !y || (!g.pack && !x)) return fail(CTMR_E_INVALID, "null input, weight or output");
  if ((desc->flags & CTMR_F_RESIDUAL) && !residual)
    return fail(CTMR_E_INVALID, "residual flag without residual");
  if ((desc->flags & CTMR_F_BATCH_BIAS) && !bias) return fail(CTMR_E_INVALID, "batch bias flag without bias");
  if ((rc = check_workspace(g, workspace, workspace_bytes))) return rc;
  const char* xp = g.pack ? (const char*)workspace : (const char*)x;
  if (!g.pack && ((uintptr_t)x & 15) != 0) return fail(CTMR_E_INVALID, "x must be 16-byte aligned");
  // The bf16 LDS GEMM and the pointwise GEMM store (and read the residual) 16 bytes at a time.
  const uintptr_t wide = (uintptr_t)y | ((desc->flags & CTMR_F_RESIDUAL) ? (uintptr_t)residual : 0) |
                         (g.split > 1 ? (uintptr_t)workspace : 0);
  if ((g.lds16 || g.pointwise) && (wide & 15) != 0)
    return fail(CTMR_E_INVALID, "y, residual and workspace must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const int64_t s_out = (int64_t)g.od * g.oh * g.ow;
  if (g.lds) {
    LdsArgs a;
    a.x = x;
    a.x2 = g.cat ? x2 : nullptr;
    a.c1 = g.c1;
    a.affine = (desc->flags & CTMR_F_AFFINE) ? (affine_direct ? affine_direct : (const float*)workspace) : nullptr;
    a.wp = (const char*)packed;
    a.bias = bias;
    a.res = residual;
    a.x_bytes = (int64_t)desc->n * desc->d * desc->h * desc->w * desc->cin * 4;
    a.w_bytes = (int64_t)27 * g.kblocks * g.np * 64;
    a.plane = (int64_t)desc->n * s_out * desc->cout;
    a.n = desc->n; a.d = desc->d; a.h = desc->h; a.w = desc->w;
    a.cin = desc->cin; a.cout = desc->cout; a.np = g.np; a.kb = g.kblocks;
    a.tz = g.tz; a.ty = g.ty; a.tx = g.tx;
    a.n_tiles = g.n_tiles;
    a.split = g.split;
    a.affine_on = (desc->flags & CTMR_F_AFFINE) != 0;
    a.silu_on = (desc->flags & CTMR_F_SILU) != 0;
    a.batch_bias = (desc->flags & CTMR_F_BATCH_BIAS) != 0;
    a.has_bias = bias != nullptr;
    a.has_res = (desc->flags & CTMR_F_RESIDUAL) != 0;
    // A split's partial planes: the reduce writes outputs and statistics (one
    // in two wave sets: the kernel does).
    const bool partial = g.split > 1 && g.wsets == 1;
    a.stats = partial ? nullptr : stats;
    a.gn_groups = stats ? groups : 0;
    a.gn_cpg = stats ? desc->cout / groups : 1;
    float* part = (float*)((char*)workspace + g.pack_bytes);
    a.y = partial ? part : y;
    if (partial) { a.res = nullptr; a.has_res = 0; }
    if (g.wsets == 2) a.split = 1;  // the kernel's two K ranges are its wave sets
    const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * desc->n * a.split;
    const dim3 grid((unsigned)blocks);
    const int xf = (a.affine_on ? 1 : 0) | (a.silu_on ? 2 : 0);
    if (a.x2) {
      if (g.wsets == 2) launch_lds<true, 2>(xf, grid, st, a);
      else launch_lds<true, 1>(xf, grid, st, a);
    } else {
      if (g.wsets == 2) launch_lds<false, 2>(xf, grid, st, a);
      else launch_lds<false, 1>(xf, grid, st, a);
    }
    if ((rc = check_launch("conv_lds"))) return rc;
    if (partial) {
      launch_split_reduce(desc, g, part, a.plane, bias, a.batch_bias, residual, y, s_out, groups, stats, st);
      if ((rc = check_launch("split_reduce"))) return rc;
    }
    return CTMR_OK;
  }
  if (g.lds_small) {
    LdsSmallArgs a;
    a.x = x;
    a.affine = (desc->flags & CTMR_F_AFFINE) ? (affine_direct ? affine_direct : (const float*)workspace) : nullptr;
    a.wp = (const char*)packed;
    a.bias = bias;
    a.res = residual;
    a.y = y;
    a.x_bytes = (int64_t)desc->n * desc->d * desc->h * desc->w * desc->cin * 4;
    a.w_bytes = (int64_t)g.kblocks * g.np * 64;
    a.plane = (int64_t)desc->n * s_out * desc->cout;  // the output (store_brick's store range)
    a.n = desc->n; a.d = desc->d; a.h = desc->h; a.w = desc->w;
    a.cin = desc->cin; a.cout = desc->cout; a.np = g.np; a.kb = g.kblocks;
    a.tz = g.tz; a.ty = g.ty; a.tx = g.tx;
    a.n_tiles = g.n_tiles;
    a.split = 1;
    a.affine_on = (desc->flags & CTMR_F_AFFINE) != 0;
    a.silu_on = (desc->flags & CTMR_F_SILU) != 0;
    a.batch_bias = (desc->flags & CTMR_F_BATCH_BIAS) != 0;
    a.has_bias = bias != nullptr;
    a.has_res = (desc->flags & CTMR_F_RESIDUAL) != 0;
    a.stats = stats;
    a.gn_groups = stats ? groups : 0;
    a.gn_cpg = stats ? desc->cout / groups : 1;
    if (a.affine_on && !a.affine) return fail(CTMR_E_INVALID, "affine flag without affine");
    const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * desc->n;
    const dim3 grid((unsigned)blocks), block(256);
    if (desc->cin == 4) {
      if (g.nsub == 4) hipLaunchKernelGGL((conv_lds_small_kernel<4, 4>), grid, block, 0, st, a);
      else if (g.nsub == 2) hipLaunchKernelGGL((conv_lds_small_kernel<4, 2>), grid, block, 0, st, a);
      else hipLaunchKernelGGL((conv_lds_small_kernel<4, 1>), grid, block, 0, st, a);
    } else {
      if (g.nsub == 4) hipLaunchKernelGGL((conv_lds_small_kernel<8, 4>), grid, block, 0, st, a);
      else if (g.nsub == 2) hipLaunchKernelGGL((conv_lds_small_kernel<8, 2>), grid, block, 0, st, a);
      else hipLaunchKernelGGL((conv_lds_small_kernel<8, 1>), grid, block, 0, st, a);
    }
    return check_launch("conv_lds_small");
  }
  if (g.small_out) {
    SmallOutArgs a;
    a.x = x;
    a.x2 = g.cat ? x2 : nullptr;
    a.c1 = g.c1;
    a.affine = (desc->flags & CTMR_F_AFFINE) ? (affine_direct ? affine_direct : (const float*)workspace) : nullptr;
    a.wp = (const float*)packed;
    a.bias = bias;
    a.y = y;
    a.n = desc->n; a.d = desc->d; a.h = desc->h; a.w = desc->w;
    a.cin = desc->cin; a.np = g.np; a.kb = desc->cin / 16;
    a.tz = g.tz; a.ty = g.ty; a.tx = g.tx;
    const int form = (desc->cout - 1) * 4 + ((desc->flags & CTMR_F_AFFINE) ? 2 : 0) + ((desc->flags & CTMR_F_SILU) ? 1 : 0);
    static void (*const kernels[16])(SmallOutArgs) = {
        conv_small_cout_kernel<1, false, false>, conv_small_cout_kernel<1, false, true>,
        conv_small_cout_kernel<1, true, false>,  conv_small_cout_kernel<1, true, true>,
        conv_small_cout_kernel<2, false, false>, conv_small_cout_kernel<2, false, true>,
        conv_small_cout_kernel<2, true, false>,  conv_small_cout_kernel<2, true, true>,
        conv_small_cout_kernel<3, false, false>, conv_small_cout_kernel<3, false, true>,
        conv_small_cout_kernel<3, true, false>,  conv_small_cout_kernel<3, true, true>,
        conv_small_cout_kernel<4, false, false>, conv_small_cout_kernel<4, false, true>,
        conv_small_cout_kernel<4, true, false>,  conv_small_cout_kernel<4, true, true>};
    const int64_t blocks = (int64_t)g.m_tiles * desc->n;
    hipLaunchKernelGGL(kernels[form], dim3((unsigned)blocks), dim3(256), 0, st, a);
    return check_launch("conv_small_cout");
  }
  if (g.lds16) {
    Lds16Args a;
    a.xp = xp;
    a.wp = (const char*)packed;
    a.bias = bias;
    a.res = residual;
    a.rows_per_batch = g.rows_per_batch;
    const bool f16x2 = desc->dtype == CTMR_F16X2;
    a.x_bytes = (int64_t)desc->n * g.rows_per_batch * g.cp * g.esize;
    a.w_bytes = (int64_t)g.taps * g.phases * g.kblocks * g.np * (f16x2 ? 96 : 64);
    a.plane = (int64_t)desc->n * s_out * desc->cout;
    a.d = g.gd; a.h = g.gh; a.w = g.gw;
    a.P = g.P; a.Q = g.Q;
    a.vbytes = g.cp * g.esize;
    a.cout = desc->cout; a.np = g.np; a.kb = g.kblocks; a.n = desc->n;
    a.tz = g.tz; a.ty = g.ty; a.tx = g.tx;
    a.n_tiles = g.n_tiles;
    a.split = g.split;
    a.batch_bias = (desc->flags & CTMR_F_BATCH_BIAS) != 0;
    a.has_bias = bias != nullptr;
    a.has_res = (desc->flags & CTMR_F_RESIDUAL) != 0;
    const bool partial = g.split > 1 && g.wsets == 1;  // partial planes and a reduction launch
    a.stats = partial ? nullptr : stats;
    a.gn_groups = stats ? groups : 0;
    a.gn_cpg = stats ? desc->cout / groups : 1;
    float* part = (float*)((char*)workspace + g.pack_bytes);
    a.y = partial ? part : y;
    if (partial) { a.res = nullptr; a.has_res = 0; }
    if (g.wsets == 2) a.split = 1;  // the kernel's two K ranges are its wave sets
    const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * desc->n * g.phases * a.split;
    if (f16x2 && ((uintptr_t)packed & 15) != 0) return fail(CTMR_E_INVALID, "packed weight must be 16-byte aligned");
    const dim3 grid((unsigned)blocks);
    if (f16x2) {
      if (g.wsets == 2) launch_lds16<CTMR_F16X2, 2>(g.phases == 8, grid, st, a);
      else launch_lds16<CTMR_F16X2, 1>(g.phases == 8, grid, st, a);
    } else {
      if (g.wsets == 2) launch_lds16<CTMR_BF16, 2>(g.phases == 8, grid, st, a);
      else launch_lds16<CTMR_BF16, 1>(g.phases == 8, grid, st, a);
    }
    if ((rc = check_launch("conv_lds_bf16"))) return rc;
    if (partial) {
      launch_split_reduce(desc, g, part, a.plane, bias, a.batch_bias, residual, y, s_out, groups, stats, st);
      if ((rc = check_launch("split_reduce"))) return rc;
    }
    return CTMR_OK;
  }
  ConvArgs a;
  a.xp = xp;
  // A two-source input reaches the GEMM unpacked only on the pointwise route.
  const bool two = g.cat && !g.pack;
  a.xp2 = two ? (const char*)x2 : nullptr;
  a.kb1 = two ? g.c1 / 16 : g.kblocks;
  a.row_bytes2 = two ? (int64_t)(desc->cin - g.c1) * 4 : 0;
  a.wp = (const char*)packed;
  a.bias = bias;
  a.res = residual;
  a.has_bias = bias != nullptr;
  a.batch_bias = (desc->flags & CTMR_F_BATCH_BIAS) != 0;
  a.has_res = (desc->flags & CTMR_F_RESIDUAL) != 0;
  a.rows_per_batch = g.rows_per_batch;
  a.row_bytes = two ? (int64_t)g.c1 * 4 : (int64_t)g.cp * g.esize;
  a.x_bytes = (int64_t)desc->n * g.rows_per_batch * a.row_bytes;
  a.w_bytes = (int64_t)g.phases * g.taps * g.kblocks * g.np * 64;
  a.plane = (int64_t)desc->n * s_out * desc->cout;
  a.kb = g.kblocks;
  a.np = g.np;
  a.cout = desc->cout;
  a.gd = g.gd; a.gh = g.gh; a.gw = g.gw;
  a.P = g.P; a.Q = g.Q;
  a.oh = g.oh; a.ow = g.ow; a.s_out = (int)s_out;
  a.taps = g.taps;
  a.split = g.split;
  a.m_tiles = g.m_tiles;
  a.n_tiles = g.n_tiles;
  a.planar = 0;
  a.zstride = 0;
  const bool partial = g.split > 1 && g.wsets == 1;  // partial planes and a reduction launch
  a.stats = partial ? nullptr : stats;
  a.gn_groups = stats ? groups : 0;
  a.gn_cpg = stats ? desc->cout / groups : 1;
  a.stats_tiles = tiles;
  float* part = (float*)((char*)workspace + g.pack_bytes);
  a.y = partial ? part : y;
  if (partial) { a.res = nullptr; a.has_res = 0; }
  if (g.wsets == 2) a.split = 1;  // the kernel's two K ranges are its wave sets
  float* z = (float*)((char*)workspace + g.pack_bytes + g.part_bytes);
  if (g.layout == WL_EXPAND) {
    // GEMM over every padded row into planar tap columns; bias and residual
    // join in the tap sum.
    a.cout = g.ncols;
    a.s_out = (int)g.rows_per_batch;
    a.plane = 0;
    a.planar = 1;
    a.zstride = (int64_t)desc->n * g.rows_per_batch;
    a.y = z;
    a.bias = nullptr;
    a.has_bias = 0;
    a.batch_bias = 0;
    a.res = nullptr;
    a.has_res = 0;
  }
  const int64_t blocks = (int64_t)g.m_tiles * g.n_tiles * desc->n * g.phases * a.split;
  a.items = g.pointwise ? (int)((int64_t)g.m_tiles * desc->n * g.split) : 0;  // launch_pointwise sizes its grid
  a.in_d = desc->d;
  a.in_h = desc->h;
  a.in_w = desc->w;
  ConvFn fn = pick(desc, g);
  fn(dim3((unsigned)blocks), dim3(256), st, a);
  if ((rc = check_launch("conv"))) return rc;
  if (g.layout == WL_EXPAND) {
    hipLaunchKernelGGL(tap_sum_kernel, dim3(elementwise_blocks((int64_t)desc->n * s_out)), dim3(256), 0, st,
                       z, (int64_t)desc->n * g.rows_per_batch, g.rows_per_batch, g.P, g.Q, desc->stride,
                       desc->n, g.od,
                       g.oh, g.ow, desc->cout, bias, (desc->flags & CTMR_F_BATCH_BIAS) ? 1 : 0,
                       (desc->flags & CTMR_F_RESIDUAL) ? residual : nullptr, y);
    return check_launch("tap_sum");
  }
  if (partial) {
    launch_split_reduce(desc, g, part, a.plane, bias, a.batch_bias, residual, y, s_out, groups, stats, st);
    if ((rc = check_launch("split_reduce"))) return rc;
  }
  return CTMR_OK;
}

// ctmr_conv3d and ctmr_conv3d_cat: x2 null for one source.
static int conv3d_run(const ctmr_conv_desc* desc, const float* x, const float* x2, const void* packed,
                      const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                      size_t workspace_bytes, void* stream) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (!x || !packed || !y || (g.cat && !x2)) return fail(CTMR_E_INVALID, "null input, weight or output");
  if (g.lds || g.lds_small || g.small_out) {  // no pack stage: these read x and the caller's affine table directly
    if ((desc->flags & CTMR_F_AFFINE) && !affine) return fail(CTMR_E_INVALID, "affine flag without affine");
    return conv3d_gemm_impl(desc, x, x2, packed, bias, affine, residual, y, workspace, workspace_bytes, 0,
                            nullptr, stream);
  }
  if ((rc = pack_impl(desc, x, x2, affine, workspace, workspace_bytes, stream))) return rc;
  return conv3d_gemm_impl(desc, x, x2, packed, bias, nullptr, residual, y, workspace, workspace_bytes, 0,
                          nullptr, stream);
}

int ctmr_conv3d(const ctmr_conv_desc* desc, const float* x, const void* packed, const float* bias,
                const float* affine, const float* residual, float* y, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (desc && desc->cin1 != 0) return fail(CTMR_E_INVALID, "two-source input: use ctmr_conv3d_cat");
  return conv3d_run(desc, x, nullptr, packed, bias, affine, residual, y, workspace, workspace_bytes, stream);
}

int ctmr_conv3d_cat(const ctmr_conv_desc* desc, const float* x1, const float* x2, const void* packed,
                    const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (!desc || desc->cin1 == 0) return fail(CTMR_E_INVALID, "ctmr_conv3d_cat needs desc->cin1 > 0");
  return conv3d_run(desc, x1, x2, packed, bias, affine, residual, y, workspace, workspace_bytes, stream);
}

int32_t ctmr_conv3d_stats_tiles(const ctmr_conv_desc* desc, int32_t groups) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  return gn_stats_tiles(desc, g, groups);
}

static int conv3d_gn_run(const ctmr_conv_desc* desc, const float* x, const float* x2, const void* packed,
                         const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                         size_t workspace_bytes, int32_t groups, double* stats, void* stream) {
  Geometry g;
  int rc = geometry(desc, g);
  if (rc) return rc;
  if (!x || !packed || !y || !stats || (g.cat && !x2))
    return fail(CTMR_E_INVALID, "null input, weight, output or stats");
  if (gn_stats_tiles(desc, g, groups) == 0)
    return fail(CTMR_E_UNSUPPORTED, "this convolution cannot produce group-norm partials");
  const bool direct_affine = g.lds || g.lds_small || g.small_out;
  if (direct_affine) {
    if ((desc->flags & CTMR_F_AFFINE) && !affine) return fail(CTMR_E_INVALID, "affine flag without affine");
  } else if ((rc = pack_impl(desc, x, x2, affine, workspace, workspace_bytes, stream))) {
    return rc;
  }
  return conv3d_gemm_impl(desc, x, x2, packed, bias, direct_affine ? affine : nullptr, residual, y, workspace,
                          workspace_bytes, groups, stats, stream);
}

int ctmr_conv3d_gn(const ctmr_conv_desc* desc, const float* x, const void* packed, const float* bias,
                   const float* affine, const float* residual, float* y, void* workspace,
                   size_t workspace_bytes, int32_t groups, double* stats, void* stream) {
  if (desc && desc->cin1 != 0) return fail(CTMR_E_INVALID, "two-source input: use ctmr_conv3d_cat_gn");
  return conv3d_gn_run(desc, x, nullptr, packed, bias, affine, residual, y, workspace, workspace_bytes, groups,
                       stats, stream);
}

int ctmr_conv3d_cat_gn(const ctmr_conv_desc* desc, const float* x1, const float* x2, const void* packed,
                       const float* bias, const float* affine, const float* residual, float* y, void* workspace,
                       size_t workspace_bytes, int32_t groups, double* stats, void* stream) {
  if (!desc || desc->cin1 == 0) return fail(CTMR_E_INVALID, "ctmr_conv3d_cat_gn needs desc->cin1 > 0");
  return conv3d_gn_run(desc, x1, x2, packed, bias, affine, residual, y, workspace, workspace_bytes, groups, stats,
                       stream);
}

}  // extern "C"
