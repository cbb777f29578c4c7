// Shared helpers for the ctmr HIP sources: vector types, error reporting and
// launch checking.  Host-visible entry points live in conv.hip and norm.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "ctmr.h"

namespace ctmr {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// Message for the last failing call on this thread (ctmr_last_error).
void set_error(const char* fmt, ...);

inline int fail(int code, const char* what) {
  set_error("%s", what);
  return code;
}

// Map a launch status to CTMR_OK / CTMR_E_LAUNCH with a message.
inline int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", kernel, hipGetErrorString(e));
    return CTMR_E_LAUNCH;
  }
  return CTMR_OK;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Workgroups for a grid-stride elementwise kernel of 256 threads: one item per
// thread up to 2^20 workgroups (the dispatch packet counts work-items in 32
// bits), looping beyond that.
inline unsigned elementwise_blocks(int64_t items) {
  const int64_t b = ceil_div(items, 256);
  return (unsigned)(b < (1 << 20) ? (b > 0 ? b : 1) : (1 << 20));
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN stays NaN).
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float v) {
  unsigned int u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

// Split-fp16 operand of an fp32 value v (CTMR_F16X2): hi = fp16(v) and
// lo = fp16((v - hi) * 2^11), both rounded to nearest even.  v - hi is exact
// in fp32 (at most 13 significant bits) and the 2^11 scale keeps lo a normal
// fp16 for |v| down to about 2^-14, so hi + lo * 2^-11 holds v to about 2^-22
// relative.  |v| must stay below 65504 (the fp16 range of hi).
__device__ __forceinline__ void split_f16x4(f4 v, h4& hi, h4& lo) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    hi[k] = (_Float16)v[k];
    lo[k] = (_Float16)((v[k] - (float)hi[k]) * 2048.0f);
  }
}

// SiLU y * sigmoid(y) = y / (1 + e^-y), with e^-y = 2^(-y log2 e) on the
// hardware exponential (v_exp_f32) and the quotient as y times the hardware
// reciprocal (v_rcp_f32): within 1e-6 relative of the exact value over the
// fp32 range, against ~25 instructions for the correctly rounded expf and
// division.  It sits in every pack and LDS staging pass that applies a group
// norm's SiLU.  The exponent -y log2 e is carried as t + c (c = the rounding
// error of the fp32 product, from an fma, plus y times the part of log2 e
// below fp32), and 2^(t + c) = 2^t (1 + c ln 2), so its relative error does
// not grow with |y|.  Limits: e^-y overflows to +inf below y = -88.7, giving -0;
// large positive y gives y.
__device__ __forceinline__ float silu_f(float y) {
  constexpr float kLog2e = 1.44269502162933349609375f;  // log2(e) rounded to fp32
  constexpr float kLog2eLow = 1.925962989e-8f;            // log2(e) - kLog2e
  constexpr float kLn2 = 0.693147180559945f;
  const float t = -kLog2e * y;
  const float c = fmaf(-kLog2e, y, -t) - kLog2eLow * y;
  const float e = __builtin_amdgcn_exp2f(t) * fmaf(c, kLn2, 1.0f);
  return y * __builtin_amdgcn_rcpf(1.0f + e);
}

// Half-pixel (align_corners=False) source coordinate of output index o for a
// 2x upsampling of an axis of n inputs: max(0, o/2 - 1/4), lower index i0,
// upper index i1 (clamped), weight of the upper sample l1.
__device__ __forceinline__ void tri_axis(int o, int n, int& i0, int& i1, float& l1) {
  float src = fmaxf(0.0f, 0.5f * (float)o - 0.25f);
  i0 = (int)src;
  i1 = min(i0 + 1, n - 1);
  l1 = src - (float)i0;
}

// Trilinear 2x sample of one channel group at output voxel (z, y, x) of the
// doubled grid, NDHWC source base `src` (batch item already applied) with
// channel pitch c; `cofs` is the channel offset.  Fixed evaluation order with
// explicit fma and no contraction so the fused and materialized paths of this
// library agree bitwise.
__device__ __forceinline__ f4 trilinear_sample4(const float* __restrict__ src, int id, int ih,
                                                 int iw, int c, int cofs, int z, int y, int x) {
#pragma clang fp contract(off)
  int z0, z1, y0, y1, x0, x1;
  float lz, ly, lx;
  tri_axis(z, id, z0, z1, lz);
  tri_axis(y, ih, y0, y1, ly);
  tri_axis(x, iw, x0, x1, lx);
  const float hz = 1.0f - lz, hy = 1.0f - ly, hx = 1.0f - lx;
  auto at = [&](int zz, int yy, int xx) -> f4 {
    return *reinterpret_cast<const f4*>(src + (((int64_t)zz * ih + yy) * iw + xx) * c + cofs);
  };
  f4 r[4];
  const int zs[2] = {z0, z1}, ys[2] = {y0, y1};
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      f4 p = at(zs[a], ys[b], x0), q = at(zs[a], ys[b], x1);
      f4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = fmaf(hx, p[k], lx * q[k]);
      r[a * 2 + b] = o;
    }
  f4 out;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float p0 = fmaf(hy, r[0][k], ly * r[1][k]);
    float p1 = fmaf(hy, r[2][k], ly * r[3][k]);
    out[k] = fmaf(hz, p0, lz * p1);
  }
  return out;
}

// Scalar variant for channel counts that are not a multiple of 4.
__device__ __forceinline__ float trilinear_sample1(const float* __restrict__ src, int id, int ih,
                                                   int iw, int c, int ch, int z, int y, int x) {
#pragma clang fp contract(off)
  int z0, z1, y0, y1, x0, x1;
  float lz, ly, lx;
  tri_axis(z, id, z0, z1, lz);
  tri_axis(y, ih, y0, y1, ly);
  tri_axis(x, iw, x0, x1, lx);
  const float hz = 1.0f - lz, hy = 1.0f - ly, hx = 1.0f - lx;
  auto at = [&](int zz, int yy, int xx) -> float {
    return src[(((int64_t)zz * ih + yy) * iw + xx) * c + ch];
  };
  const int zs[2] = {z0, z1}, ys[2] = {y0, y1};
  float r[4];
  for (int a = 0; a < 2; ++a)
    for (int b = 0; b < 2; ++b) r[a * 2 + b] = fmaf(hx, at(zs[a], ys[b], x0), lx * at(zs[a], ys[b], x1));
  float p0 = fmaf(hy, r[0], ly * r[1]);
  float p1 = fmaf(hy, r[2], ly * r[3]);
  return fmaf(hz, p0, lz * p1);
}

}  // namespace ctmr
