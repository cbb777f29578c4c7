// FP32 flash attention for 32-wide heads on gfx950 matrix cores.
//
// Computes softmax(Q K^T * scale) V per (batch item, head) without writing the
// scores, as _flash_attention.flash_attention does (_flash_attention.py:1-27,
// 320-360): an online softmax over key blocks with a running row maximum and
// sum, exp2 of log2(e)-scaled scores (the scale is folded into Q once).
//
// MI355X layout.  One wave owns QT x 16 queries and walks all keys in blocks of
// 32.  Both products run on v_mfma_f32_16x16x4_f32 in the transposed form:
//   S^T = K Q^T   (rows = keys, columns = queries; k runs over the 32 head dims)
//   O^T += V^T P^T (rows = head dims, columns = queries; k runs over keys)
// With the MFMA result layout (lane l, register r -> row 4*(l/16)+r, column
// l%16) a lane's S^T registers are 4 keys of ONE query, so
//   * the per-query max/sum need only 2 cross-lane steps (lanes l^16, l^32),
//   * the S^T registers are already P^T's B operand for the next product
//     (step r of a 16-key tile pairs lane group g with key 4g+r), and
//   * the running-output rescale is one scalar per lane.
// The head-dim order inside Q K^T is permuted the same way in both operands
// (step s, lane group g -> dim 8g+s) so each lane loads 8 contiguous floats.
// Everything accumulates in FP32; keys are visited in ascending blocks, so the
// result does not depend on the launch shape or on other work on the device.
// Within a wave the loop is software-pipelined: the next block's K Q^T
// products are issued between this block's softmax instructions, so the
// exp2 / max / rescale work runs while the matrix core is busy.
#include "ctmr_common.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace ctmr {
namespace {

constexpr int kHeadDim = 32;
constexpr int kWaves = 4;     // waves per workgroup (independent; no LDS, no barriers)
constexpr int kKeyTiles = 2;  // 16-key tiles per key block
constexpr int kBlock = 16 * kKeyTiles;
constexpr float kLazyMax = 8.0f;  // log2 headroom before the softmax reference max moves

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t ldq, ldk, ldv, ldo;
  int lq, lk, heads;
  float qscale;  // scale * log2(e)
};

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Maximum over lanes l, l^16, l^32, l^48 (the four lane groups holding one
// query's scores): v_permlane16_swap / v_permlane32_swap of a value with
// itself yield the pair {x[l], x[l^16]} / {x[l], x[l^32]} (VALU, no LDS round
// trip as with ds_bpermute).
__device__ __forceinline__ float lane_group_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// First key of the second part of a two-part key split: half the keys,
// rounded up to a multiple of 64 keys (whole key blocks, so only the second
// part is ragged).
__device__ __forceinline__ int attention_key_split_point(int lk) {
  return min(lk, (((lk + 1) / 2 + 63) / 64) * 64);
}

// Keys and values of one key block in MFMA operand order.
struct KeyTiles {
  f4 k[kKeyTiles][2];  // K row (tile*16 + l%16), dims 8g .. 8g+7
};
struct ValueTiles {
  float v[kKeyTiles][4][2];  // V row (tile*16 + 4g + r), dims (l%16) and (16 + l%16)
};

// KS = 2 splits the keys of each query group between two waves of the
// workgroup (keys [0, split) and [split, lk), split a multiple of 64 keys):
// small grids then keep two waves per SIMD.  The second wave hands its
// running max, sum and output to the first through LDS, which combines them
// in that fixed order.
template <int QT, int KS>
__global__ __launch_bounds__(256) void flash_attention_kernel(AttnArgs a) {
  static_assert(KS == 1 || KS == 2, "one or two key parts");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int b = blockIdx.y / a.heads, h = blockIdx.y % a.heads;
  const int q0 = (blockIdx.x * (kWaves / KS) + wave / KS) * (QT * 16);
  const int part = wave % KS;
  // Wave-uniform.  With KS = 2 every wave reaches the combine barrier: a query
  // group past the end runs on clamped rows and stores nothing.
  if (KS == 1 && q0 >= a.lq) return;
  const int split = KS == 1 ? a.lk : attention_key_split_point(a.lk);
  const int k_begin = part == 0 ? 0 : split, k_end = part == 0 ? split : a.lk;

  const float* Q = a.q + (int64_t)b * a.lq * a.ldq + h * kHeadDim;
  const float* K = a.k + (int64_t)b * a.lk * a.ldk + h * kHeadDim;
  const float* V = a.v + (int64_t)b * a.lk * a.ldv + h * kHeadDim;
  // K and V rows of a key block through a buffer descriptor built per block
  // from wave-uniform values (scalar instructions): base = row k0, range =
  // the rows left before lk.  Per-lane offsets inside a block are fixed for the
  // whole loop and rows at or past lk read as zero (masked below) -- no
  // per-lane address arithmetic or clamping inside the loop.  The host keeps
  // lk * ld * 4 within 31 bits.
  auto rows_rsrc = [&](const float* base, int64_t ld, int k0) {
    const int64_t left = (int64_t)max(a.lk - k0, 0) * ld * 4;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)k0 * ld), (short)0, (int)left, 0x00020000);
  };
  int koff[kKeyTiles], voff[kKeyTiles][4];
#pragma unroll
  for (int u = 0; u < kKeyTiles; ++u) {
    koff[u] = (int)(((int64_t)(u * 16 + col) * a.ldk + 8 * g) * 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) voff[u][r] = (int)(((int64_t)(u * 16 + 4 * g + r) * a.ldv + col) * 4);
  }

  f4 qa[QT][2];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int row = min(q0 + t * 16 + col, a.lq - 1);
    const f4* p = reinterpret_cast<const f4*>(Q + (int64_t)row * a.ldq + 8 * g);
    qa[t][0] = p[0] * a.qscale;
    qa[t][1] = p[1] * a.qscale;
  }

  f4 o[QT][2];
  float m[QT], l[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    o[t][0] = f4{0.f, 0.f, 0.f, 0.f};
    o[t][1] = f4{0.f, 0.f, 0.f, 0.f};
    m[t] = -INFINITY;
    l[t] = 0.f;
  }

  // Rows past the end read as zero (outside the descriptors' range) and are masked below.
  auto load_k = [&](KeyTiles& kt, int k0) {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(K, a.ldk, k0);
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u) {
      kt.k[u][0] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, koff[u], 0, 0));
      kt.k[u][1] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, koff[u] + 16, 0, 0));
    }
  };
  auto load_v = [&](ValueTiles& vt, int k0) {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(V, a.ldv, k0);
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vt.v[u][r][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff[u][r], 0, 0));
        vt.v[u][r][1] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff[u][r] + 64, 0, 0));
      }
  };
  // S^T tiles of one key block.
  auto qk = [&](const KeyTiles& kt, f4 (&s)[kKeyTiles][QT]) {
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = mfma4(kt.k[u][j][e], qa[t][j][e], acc);
        s[u][t] = acc;
      }
  };
  // Online softmax of one block: scores -> P^T in place, running reference
  // max and sum, and the factor alpha[t] the output must be scaled by before
  // this block's P V products.  The reference m[t] of a query moves only when
  // the block's max exceeds it by more than kLazyMax (in log2 units; always on
  // the first block, where m = -inf): P = 2^(s - m) then stays below 2^8, and
  // in most blocks alpha is exactly 1, so the output rescale is skipped
  // (output / sum is the same quotient for any reference).  The decision is
  // per query, so every tiling computes the same bits.  RAGGED masks keys at or
  // past k_end (the last block only).
  float alpha[QT];
  auto softmax = [&](f4 (&s)[kKeyTiles][QT], int k0, auto ragged) {
    if constexpr (decltype(ragged)::value) {
#pragma unroll
      for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (k0 + u * 16 + 4 * g + r >= k_end)
#pragma unroll
            for (int t = 0; t < QT; ++t) s[u][t][r] = -INFINITY;
    }
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      float bm = s[0][t][0];
#pragma unroll
      for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) bm = fmaxf(bm, s[u][t][r]);
      bm = lane_group_max(bm);
      // Every block holds at least one real key, so bm is finite and the first
      // block moves the reference (alpha = 2^-inf = 0).  Arguments are <= 8:
      // the hardware exp2 (v_exp_f32) differs from exp2f only below 2^-126,
      // far under the resolution of the running sum (>= 1).
      const bool move = bm > m[t] + kLazyMax;
      const float mn = move ? bm : m[t];
      alpha[t] = move ? __builtin_amdgcn_exp2f(m[t] - mn) : 1.0f;
      m[t] = mn;
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[u][t][r] - mn);
          s[u][t][r] = p;
          ps += p;
        }
      l[t] = l[t] * alpha[t] + ps;
    }
  };
  // o *= alpha, skipped (same bits: every factor is exactly 1) unless a lane of
  // the wave moved its reference.
  auto rescale = [&]() {
#pragma unroll
    for (int t = 0; t < QT; ++t)
      if (__builtin_amdgcn_ballot_w64(alpha[t] != 1.0f)) {
        o[t][0] *= alpha[t];
        o[t][1] *= alpha[t];
      }
  };
  auto pv = [&](const ValueTiles& vt, const f4 (&s)[kKeyTiles][QT]) {
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < QT; ++t) {
          o[t][0] = mfma4(vt.v[u][r][0], s[u][t][r], o[t][0]);
          o[t][1] = mfma4(vt.v[u][r][1], s[u][t][r], o[t][1]);
        }
  };
  // One pipeline step for a full block k0 that has a successor, scores in
  // `sc`: the loads of the next block's V and of the K after next (rows past
  // the end are clamped: in bounds, unused) go out first; then the next
  // block's K Q^T products (into `sn`, from `kn`) are interleaved with this
  // block's softmax -- one MFMA, then VALU work while the matrix core runs --
  // and this block's P V products follow.  Branch-free, so the scheduler can
  // interleave.
  auto step = [&](f4 (&sc)[kKeyTiles][QT], f4 (&sn)[kKeyTiles][QT], const ValueTiles& vc, ValueTiles& vn,
                  const KeyTiles& kn, KeyTiles& kf, int k0) {
    load_v(vn, k0 + kBlock);
    load_k(kf, k0 + 2 * kBlock);
    __builtin_amdgcn_sched_barrier(0);
    qk(kn, sn);
    softmax(sc, k0, std::false_type{});
#pragma unroll
    for (int i = 0; i < kKeyTiles * QT * 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    rescale();
    pv(vc, sc);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The last block (possibly ragged): softmax, then its products.
  auto last = [&](f4 (&sc)[kKeyTiles][QT], const ValueTiles& vc, int k0) {
    softmax(sc, k0, std::true_type{});
    rescale();
    pv(vc, sc);
  };

  // Registers: K of the next two blocks, V of this and the next block, the
  // scores of this and the next block (names alternate between steps).
  KeyTiles ka, kb;
  ValueTiles va, vb;
  f4 sa[kKeyTiles][QT], sb[kKeyTiles][QT];
  const int nb = k_begin < k_end ? (k_end - k_begin + kBlock - 1) / kBlock : 0;
  if (nb > 0) {
    load_k(ka, k_begin);
    load_v(va, k_begin);
    load_k(kb, k_begin + kBlock);
    qk(ka, sa);
    int i = 0;
    for (; i + 2 < nb; i += 2) {
      step(sa, sb, va, vb, kb, ka, k_begin + i * kBlock);
      step(sb, sa, vb, va, ka, kb, k_begin + (i + 1) * kBlock);
    }
    if (nb - i == 2) {
      step(sa, sb, va, vb, kb, ka, k_begin + i * kBlock);
      last(sb, vb, k_begin + (i + 1) * kBlock);
    } else {
      last(sa, va, k_begin + i * kBlock);
    }
  }

  if constexpr (KS == 2) {
    // Lane-for-lane state of the second key part: max, partial sum, output.
    __shared__ float xch[kWaves / 2][QT][10][64];
    float(*mine)[10][64] = xch[wave / 2];
    if (part == 1) {
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        mine[t][0][lane] = m[t];
        mine[t][1][lane] = l[t];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          mine[t][2 + e][lane] = o[t][0][e];
          mine[t][6 + e][lane] = o[t][1][e];
        }
      }
    }
    __syncthreads();
    if (part == 1) return;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const float m1 = mine[t][0][lane];
      const float mm = fmaxf(m[t], m1);  // the first part always holds keys: finite
      const float a0 = exp2f(m[t] - mm), a1 = exp2f(m1 - mm);  // a1 = 0 for an empty second part
      l[t] = l[t] * a0 + mine[t][1][lane] * a1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[t][0][e] = o[t][0][e] * a0 + mine[t][2 + e][lane] * a1;
        o[t][1][e] = o[t][1][e] * a0 + mine[t][6 + e][lane] * a1;
      }
    }
  }

  float* O = a.out + (int64_t)b * a.lq * a.ldo + h * kHeadDim;
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    // The four lane groups hold partial sums of the same query; xor pairs add
    // commutatively, so every lane ends with the same bits.
    float lt = l[t];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = 1.0f / lt;
    const int query = q0 + t * 16 + col;
    if (query < a.lq) {
      f4* dst = reinterpret_cast<f4*>(O + (int64_t)query * a.ldo + 4 * g);
      dst[0] = o[t][0] * inv;  // dims 4g .. 4g+3
      dst[4] = o[t][1] * inv;  // dims 16 + 4g .. 16 + 4g+3
    }
  }
}

template <int QT, int KS>
int launch_attention(const AttnArgs& a, int n, hipStream_t stream) {
  const int64_t per_block = (int64_t)(kWaves / KS) * QT * 16;
  dim3 grid((unsigned)ceil_div(a.lq, per_block), (unsigned)(n * a.heads));
  hipLaunchKernelGGL((flash_attention_kernel<QT, KS>), grid, dim3(256), 0, stream, a);
  return check_launch("flash_attention_kernel");
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// Query tiles per wave: two (more reuse of each key block) when that still
// gives at least one wave per SIMD of the 256-CU device, else one.
int attention_query_tiles(int n, int lq, int heads) {
  const int64_t waves2 = ceil_div(lq, 32) * (int64_t)n * heads;
  return waves2 >= 1024 ? 2 : 1;
}

// Key parts per query group, from the shape only (never from query_tiles, so
// both tilings give the same bits): two when there are at least 128 keys and
// fewer than two waves per SIMD would run otherwise.
int attention_key_parts(int n, int lq, int lk, int heads) {
  const int64_t waves2 = ceil_div(lq, 32) * (int64_t)n * heads;
  return (lk >= 128 && waves2 < 2048) ? 2 : 1;
}

}  // namespace ctmr

extern "C" int ctmr_flash_attention(const ctmr_attn_desc* d, const float* q, const float* k, const float* v,
                                    float* out, void* stream) {
  using namespace ctmr;
  if (!d || !q || !k || !v || !out) return fail(CTMR_E_INVALID, "ctmr_flash_attention: null argument");
  if (d->head_dim != kHeadDim) {
    set_error("ctmr_flash_attention: head_dim %d unsupported (32 only)", d->head_dim);
    return CTMR_E_UNSUPPORTED;
  }
  if (d->query_tiles < 0 || d->query_tiles > 2)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: query_tiles must be 0, 1 or 2");
  if (d->n < 1 || d->lq < 1 || d->lk < 1 || d->heads < 1)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: n, lq, lk and heads must be >= 1");
  if ((int64_t)d->n * d->heads > 65535)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: n * heads exceeds 65535");
  const int64_t width = (int64_t)d->heads * kHeadDim;
  if (d->ldq < width || d->ldk < width || d->ldv < width || d->ldo < width)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: row stride below heads * head_dim");
  if ((d->ldq | d->ldk | d->ldv | d->ldo) & 3)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: row strides must be multiples of 4 floats");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(CTMR_E_INVALID, "ctmr_flash_attention: q, k, v and out must be 16-byte aligned");
  if ((int64_t)d->lk * std::max(d->ldk, d->ldv) * 4 > 0x7fffffffll)
    return fail(CTMR_E_UNSUPPORTED, "ctmr_flash_attention: lk * row stride exceeds 2^31 bytes");
  if (!std::isfinite(d->scale)) return fail(CTMR_E_INVALID, "ctmr_flash_attention: scale must be finite");
  AttnArgs a{q, k, v, out, d->ldq, d->ldk, d->ldv, d->ldo, d->lq, d->lk, d->heads,
             (float)((double)d->scale * 1.4426950408889634)};
  hipStream_t st = (hipStream_t)stream;
  const int qt = d->query_tiles ? d->query_tiles : attention_query_tiles(d->n, d->lq, d->heads);
  if (attention_key_parts(d->n, d->lq, d->lk, d->heads) == 2)
    return qt == 2 ? launch_attention<2, 2>(a, d->n, st) : launch_attention<1, 2>(a, d->n, st);
  return qt == 2 ? launch_attention<2, 1>(a, d->n, st) : launch_attention<1, 1>(a, d->n, st);
}
