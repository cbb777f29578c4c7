// Flash attention for 32-wide heads on gfx950 matrix cores: FP32 MFMA, and
// the reference's split-fp16 form (further below).
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

// Online softmax of one 32-key block, shared by both kernels: scores -> P^T in
// place, running reference max m and sum l, and the factor alpha the outputs
// must be scaled by before this block's P V products.  A lane holds keys
// 16u + 4g + r (u < 2, r < 4) of its query.  The reference m[t] of a query
// moves only when the block's max exceeds it by more than kLazyMax (in log2
// units; always on the first block, where m = -inf): P = 2^(s - m) then stays
// below 2^8, and in most blocks alpha is exactly 1, so the output rescale is
// skipped (output / sum is the same quotient for any reference).  The decision
// is per query, so every tiling computes the same bits.  RAGGED masks keys at
// or past k_end (the last block only).
template <int QT, bool RAGGED>
__device__ __forceinline__ void block_softmax(f4 (&s)[kKeyTiles][QT], float (&m)[QT], float (&l)[QT],
                                              float (&alpha)[QT], int k0, int k_end, int g) {
  if constexpr (RAGGED) {
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
}

// Combine of a two-part key split (KS = 2): the second wave of each pair hands
// its running max, partial sum and N output accumulators to the first through
// LDS, which rescales both and adds them in that fixed order.  Every wave of
// the workgroup must call it (one barrier); returns true for the waves that go
// on to store.
template <int QT, int N>
__device__ __forceinline__ bool combine_key_parts(f4 (&acc)[QT][N], float (&m)[QT], float (&l)[QT], int lane,
                                                  int wave, int part) {
  __shared__ float xch[kWaves / 2][QT][2 + 4 * N][64];
  float(*mine)[2 + 4 * N][64] = xch[wave / 2];
  if (part == 1) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      mine[t][0][lane] = m[t];
      mine[t][1][lane] = l[t];
#pragma unroll
      for (int j = 0; j < N; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) mine[t][2 + 4 * j + e][lane] = acc[t][j][e];
    }
  }
  __syncthreads();
  if (part == 1) return false;
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const float m1 = mine[t][0][lane];
    const float mm = fmaxf(m[t], m1);  // the first part always holds keys: finite
    const float a0 = exp2f(m[t] - mm), a1 = exp2f(m1 - mm);  // a1 = 0 for an empty second part
    l[t] = l[t] * a0 + mine[t][1][lane] * a1;
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[t][j][e] = acc[t][j][e] * a0 + mine[t][2 + 4 * j + e][lane] * a1;
  }
  return true;
}

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
  float alpha[QT];
  auto softmax = [&](f4 (&sc)[kKeyTiles][QT], int k0, auto ragged) {
    block_softmax<QT, decltype(ragged)::value>(sc, m, l, alpha, k0, k_end, g);
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
    if (!combine_key_parts<QT, 2>(o, m, l, lane, wave, part)) return;
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

// ---------------------------------------------------------------------------
// Split-fp16 flash attention: the reference's matrix-unit kernel
// (_flash_attention.py:140-290, selected at :336-350).  Q (scaled by
// scale * log2(e)), K and V are split once into fp16 halves, hi = fp16(x) and
// lo = fp16((x - hi) * 2^11) (split_f16x4; _flash_attention.py:314-317), and
// every product runs on v_mfma_f32_16x16x32_f16 with fp32 accumulation as
//   S = Kh Qh + (Kh Ql + Kl Qh) * 2^-11          (per 32-key block)
//   O = Vh Ph + (Vh Pl + Vl Ph) * 2^-11          (P split the same way)
// with the cross terms of O kept in their own accumulator over all key blocks
// and added at the end, as the reference does.  One MFMA covers all 32 head
// dims of S (k = dims) and a whole 32-key block of O (k = keys), so a block
// takes 24 MFMAs per 32 queries instead of 64 FP32 ones.
//
// Workspace (fp16, per (batch item, head)): Q and K row-major, 32 dims per
// row, K's rows padded with zeros to lkp = lk rounded up to 32; V transposed,
// 32 rows of lkp keys, so a lane's eight keys of the P V product's A operand
// are two 8-byte runs.  The S^T result layout is the FP32 kernel's (a lane
// holds keys 16u + 4g + r of one query), so the softmax is shared; P^T's k
// slot 8g + 4u + r of the P V product is key 16u + 4g + r, and V^T's loads
// follow the same map.
struct SplitArgs {
  const float* x[3];   // q, k, v
  int64_t ld[3];       // row strides (floats)
  int rows[3];         // lq, lk, lk
  int rowsp[3];        // lq, lkp, lkp
  _Float16* hi[3];
  _Float16* lo[3];
  int heads;
  float qscale;        // scale * log2(e), applied to q before the split
};

// One thread per (tensor, batch item, head, row, 8-dim group), the four dim
// groups of a row in adjacent lanes: a row's 128 bytes are read by one
// quarter-wave, Q's and K's split rows written as 64 contiguous bytes, and V's
// transposed stores as 32-byte runs.  Rows at or past the tensor's length (K
// and V padding) are written as zeros.
__global__ __launch_bounds__(256) void attention_split_kernel(SplitArgs a, int n) {
  const int which = blockIdx.y;
  const int rp = a.rowsp[which];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n * a.heads * 4 * rp) return;
  const int grp = (int)(i & 3);
  const int row = (int)((i >> 2) % rp);
  const int64_t bh = (i >> 2) / rp;
  const int b = (int)(bh / a.heads), h = (int)(bh % a.heads);
  f4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = {0.f, 0.f, 0.f, 0.f};
  if (row < a.rows[which]) {
    const float* src = a.x[which] + ((int64_t)b * a.rows[which] + row) * a.ld[which] + h * kHeadDim + grp * 8;
    v0 = *reinterpret_cast<const f4*>(src);
    v1 = *reinterpret_cast<const f4*>(src + 4);
    if (which == 0) {
      v0 *= a.qscale;
      v1 *= a.qscale;
    }
  }
  h4 hi0, lo0, hi1, lo1;
  split_f16x4(v0, hi0, lo0);
  split_f16x4(v1, hi1, lo1);
  if (which < 2) {
    const int64_t off = (bh * rp + row) * kHeadDim + grp * 8;
    *reinterpret_cast<h8*>(a.hi[which] + off) = h8{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
    *reinterpret_cast<h8*>(a.lo[which] + off) = h8{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
  } else {
    const int64_t off = (bh * kHeadDim + grp * 8) * rp + row;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a.hi[2][off + e * rp] = hi0[e];
      a.lo[2][off + e * rp] = lo0[e];
      a.hi[2][off + (e + 4) * rp] = hi1[e];
      a.lo[2][off + (e + 4) * rp] = lo1[e];
    }
  }
}

struct SplitAttnArgs {
  const _Float16 *qh, *ql, *kh, *kl, *vh, *vl;
  float* out;
  int64_t ldo;
  int lq, lk, lkp, heads;
};


__device__ __forceinline__ f4 mfma_h(const h8& a, const h8& b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Grid, waves and key parts as flash_attention_kernel<QT, KS>.  Every load is
// in bounds by construction: K rows k0 + 31 < lkp and V^T keys k0 + 31 < lkp
// for any block start k0 < lk (a multiple of 32), and the next block's loads
// are clamped to the last block.
template <int QT, int KS>
__global__ __launch_bounds__(256) void flash_attention_split_kernel(SplitAttnArgs a) {
  static_assert(KS == 1 || KS == 2, "one or two key parts");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int bh = blockIdx.y, b = bh / a.heads, h = bh % a.heads;
  const int q0 = (blockIdx.x * (kWaves / KS) + wave / KS) * (QT * 16);
  const int part = wave % KS;
  if (KS == 1 && q0 >= a.lq) return;
  const int split = KS == 1 ? a.lk : attention_key_split_point(a.lk);
  const int k_begin = part == 0 ? 0 : split, k_end = part == 0 ? split : a.lk;

  const _Float16* Qh = a.qh + (int64_t)bh * a.lq * kHeadDim;
  const _Float16* Ql = a.ql + (int64_t)bh * a.lq * kHeadDim;
  const _Float16* Kh = a.kh + (int64_t)bh * a.lkp * kHeadDim;
  const _Float16* Kl = a.kl + (int64_t)bh * a.lkp * kHeadDim;
  const _Float16* Vh = a.vh + (int64_t)bh * kHeadDim * a.lkp;
  const _Float16* Vl = a.vl + (int64_t)bh * kHeadDim * a.lkp;

  // Q^T as the B operand of S^T = K Q^T: query q0 + 16t + col, dims 8g .. 8g+7.
  h8 qh[QT], ql[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int row = min(q0 + t * 16 + col, a.lq - 1);
    qh[t] = *reinterpret_cast<const h8*>(Qh + (int64_t)row * kHeadDim + 8 * g);
    ql[t] = *reinterpret_cast<const h8*>(Ql + (int64_t)row * kHeadDim + 8 * g);
  }

  // acc[t][0..1]: hi products for dims 16j + 4g + r; acc[t][2..3]: their
  // 2^11-scaled cross terms.
  f4 acc[QT][4];
  float m[QT], l[QT], alpha[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = f4{0.f, 0.f, 0.f, 0.f};
    m[t] = -INFINITY;
    l[t] = 0.f;
  }

  // Operands of one key block: K rows k0 + 16u + col (dims 8g .. 8g+7); V^T
  // rows 16j + col at keys k0 + 4g .. +3 and k0 + 16 + 4g .. +3.  Loads go
  // through buffer descriptors whose base moves with k0 (scalar work), so the
  // per-lane offsets are fixed for the whole loop.
  struct Block {
    h8 kh[kKeyTiles], kl[kKeyTiles], vh[2], vl[2];
  };
  int koff[kKeyTiles], voff[2];
#pragma unroll
  for (int u = 0; u < kKeyTiles; ++u) koff[u] = ((16 * u + col) * kHeadDim + 8 * g) * 2;
#pragma unroll
  for (int j = 0; j < 2; ++j) voff[j] = (int)(((int64_t)(16 * j + col) * a.lkp + 4 * g) * 2);
  const int k_bytes = (int)((int64_t)a.lkp * kHeadDim * 2);  // one (batch item, head) plane; < 2^31 (host check)
  auto rsrc = [&](const _Float16* base, int64_t shift) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + shift), (short)0, k_bytes, 0x00020000);
  };
  auto load = [&](Block& x, int k0) {
    const __amdgpu_buffer_rsrc_t rkh = rsrc(Kh, (int64_t)k0 * kHeadDim), rkl = rsrc(Kl, (int64_t)k0 * kHeadDim);
    const __amdgpu_buffer_rsrc_t rvh = rsrc(Vh, k0), rvl = rsrc(Vl, k0);
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u) {
      x.kh[u] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rkh, koff[u], 0, 0));
      x.kl[u] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rkl, koff[u], 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const h4 h0 = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvh, voff[j], 0, 0));
      const h4 h1 = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvh, voff[j] + 32, 0, 0));
      const h4 l0 = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvl, voff[j], 0, 0));
      const h4 l1 = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvl, voff[j] + 32, 0, 0));
      x.vh[j] = h8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
      x.vl[j] = h8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
    }
  };
  // One key block: S^T (hi * hi, then the cross terms in their own
  // accumulator), the softmax, the split of P, and the P V products.
  auto block = [&](const Block& x, int k0, auto ragged) {
    f4 s[kKeyTiles][QT];
#pragma unroll
    for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        const f4 hh = mfma_h(x.kh[u], qh[t], z);
        f4 cr = mfma_h(x.kh[u], ql[t], z);
        cr = mfma_h(x.kl[u], qh[t], cr);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[u][t][r] = fmaf(cr[r], 1.0f / 2048.0f, hh[r]);
      }
    block_softmax<QT, decltype(ragged)::value>(s, m, l, alpha, k0, k_end, g);
#pragma unroll
    for (int t = 0; t < QT; ++t)
      if (__builtin_amdgcn_ballot_w64(alpha[t] != 1.0f)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j] *= alpha[t];
      }
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      h8 ph, pl;
#pragma unroll
      for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) ph[4 * u + r] = (_Float16)s[u][t][r];
      // The low halves below read hi from these packed registers (an opaque
      // copy: otherwise the compiler converts each p to fp16 a second time).
      asm volatile("" : "+v"(ph));
      // lo = fp16((p - hi) * 2^11) = fp16(2^11 p - 2^11 hi): both products and
      // their difference are exact in fp32, so one rounding of the fused form
      // (v_fma_mix) gives the same half.
#pragma unroll
      for (int u = 0; u < kKeyTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          pl[4 * u + r] = (_Float16)__builtin_fmaf((float)ph[4 * u + r], -2048.0f, s[u][t][r] * 2048.0f);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[t][j] = mfma_h(x.vh[j], ph, acc[t][j]);
        acc[t][2 + j] = mfma_h(x.vh[j], pl, acc[t][2 + j]);
        acc[t][2 + j] = mfma_h(x.vl[j], ph, acc[t][2 + j]);
      }
    }
  };

  // Three operand buffers in rotation (the loop unrolled by three, so no
  // register copies): each block's loads go out two blocks ahead, into the
  // buffer the block just processed has freed.  Loads past the last block are
  // clamped to it (in bounds, unused).
  const int nb = k_begin < k_end ? (k_end - k_begin + kBlock - 1) / kBlock : 0;
  if (nb > 0) {
    const int k_last = k_begin + (nb - 1) * kBlock;
    auto kat = [&](int i) { return min(k_begin + i * kBlock, k_last); };
    Block x0, x1, x2;
    load(x0, kat(0));
    load(x1, kat(1));
    int i = 0;
    for (; i + 3 < nb; i += 3) {
      load(x2, kat(i + 2));
      block(x0, kat(i), std::false_type{});
      load(x0, kat(i + 3));
      block(x1, kat(i + 1), std::false_type{});
      load(x1, kat(i + 4));
      block(x2, kat(i + 2), std::false_type{});
    }
    // one to three blocks left: x0 holds block i, x1 block i + 1
    if (nb - i == 1) {
      block(x0, kat(i), std::true_type{});
    } else if (nb - i == 2) {
      block(x0, kat(i), std::false_type{});
      block(x1, kat(i + 1), std::true_type{});
    } else {
      load(x2, kat(i + 2));
      block(x0, kat(i), std::false_type{});
      block(x1, kat(i + 1), std::false_type{});
      block(x2, kat(i + 2), std::true_type{});
    }
  }

  if constexpr (KS == 2) {
    if (!combine_key_parts<QT, 4>(acc, m, l, lane, wave, part)) return;
  }

  float* O = a.out + (int64_t)b * a.lq * a.ldo + h * kHeadDim;
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    float lt = l[t];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = 1.0f / lt;
    const int query = q0 + t * 16 + col;
    if (query < a.lq) {
      f4* dst = reinterpret_cast<f4*>(O + (int64_t)query * a.ldo + 4 * g);
      f4 o0, o1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o0[r] = (acc[t][0][r] + acc[t][2][r] * (1.0f / 2048.0f)) * inv;
        o1[r] = (acc[t][1][r] + acc[t][3][r] * (1.0f / 2048.0f)) * inv;
      }
      dst[0] = o0;  // dims 4g .. 4g+3
      dst[4] = o1;  // dims 16 + 4g .. 16 + 4g+3
    }
  }
}

template <int QT, int KS>
int launch_attention_split(const SplitAttnArgs& a, int n, hipStream_t stream) {
  const int64_t per_block = (int64_t)(kWaves / KS) * QT * 16;
  dim3 grid((unsigned)ceil_div(a.lq, per_block), (unsigned)(n * a.heads));
  hipLaunchKernelGGL((flash_attention_split_kernel<QT, KS>), grid, dim3(256), 0, stream, a);
  return check_launch("flash_attention_split_kernel");
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

namespace ctmr {
namespace {

// Argument checks shared by both entry points (messages name the caller).
int check_attn(const ctmr_attn_desc* d, const float* q, const float* k, const float* v, const float* out,
               const char* fn) {
  if (!d || !q || !k || !v || !out) {
    set_error("%s: null argument", fn);
    return CTMR_E_INVALID;
  }
  if (d->head_dim != kHeadDim) {
    set_error("%s: head_dim %d unsupported (32 only)", fn, d->head_dim);
    return CTMR_E_UNSUPPORTED;
  }
  const char* bad = nullptr;
  int code = CTMR_E_INVALID;
  const int64_t width = (int64_t)d->heads * kHeadDim;
  if (d->query_tiles < 0 || d->query_tiles > 2)
    bad = "query_tiles must be 0, 1 or 2";
  else if (d->n < 1 || d->lq < 1 || d->lk < 1 || d->heads < 1)
    bad = "n, lq, lk and heads must be >= 1";
  else if ((int64_t)d->n * d->heads > 65535)
    bad = "n * heads exceeds 65535";
  else if (d->ldq < width || d->ldk < width || d->ldv < width || d->ldo < width)
    bad = "row stride below heads * head_dim";
  else if ((d->ldq | d->ldk | d->ldv | d->ldo) & 3)
    bad = "row strides must be multiples of 4 floats";
  else if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    bad = "q, k, v and out must be 16-byte aligned";
  else if ((int64_t)d->lk * std::max(d->ldk, d->ldv) * 4 > 0x7fffffffll)
    bad = "lk * row stride exceeds 2^31 bytes", code = CTMR_E_UNSUPPORTED;
  else if (!std::isfinite(d->scale))
    bad = "scale must be finite";
  if (bad) {
    set_error("%s: %s", fn, bad);
    return code;
  }
  return CTMR_OK;
}

// Split-fp16 workspace: six fp16 planes (Q hi/lo, K hi/lo, V^T hi/lo), each
// starting on a 256-byte boundary.
struct SplitPlan {
  int64_t lkp, plane_bytes[3], offset[6], bytes;
};

SplitPlan split_plan(const ctmr_attn_desc* d) {
  SplitPlan s{};
  s.lkp = round_up(d->lk, kBlock);
  const int64_t items = (int64_t)d->n * d->heads * kHeadDim * 2;
  s.plane_bytes[0] = round_up(items * d->lq, 256);
  s.plane_bytes[1] = s.plane_bytes[2] = round_up(items * s.lkp, 256);
  int64_t at = 0;
  for (int i = 0; i < 6; ++i) {
    s.offset[i] = at;
    at += s.plane_bytes[i / 2];
  }
  s.bytes = at;
  return s;
}

}  // namespace
}  // namespace ctmr

extern "C" int ctmr_flash_attention(const ctmr_attn_desc* d, const float* q, const float* k, const float* v,
                                    float* out, void* stream) {
  using namespace ctmr;
  if (const int rc = check_attn(d, q, k, v, out, "ctmr_flash_attention")) return rc;
  AttnArgs a{q, k, v, out, d->ldq, d->ldk, d->ldv, d->ldo, d->lq, d->lk, d->heads,
             (float)((double)d->scale * 1.4426950408889634)};
  hipStream_t st = (hipStream_t)stream;
  const int qt = d->query_tiles ? d->query_tiles : attention_query_tiles(d->n, d->lq, d->heads);
  if (attention_key_parts(d->n, d->lq, d->lk, d->heads) == 2)
    return qt == 2 ? launch_attention<2, 2>(a, d->n, st) : launch_attention<1, 2>(a, d->n, st);
  return qt == 2 ? launch_attention<2, 1>(a, d->n, st) : launch_attention<1, 1>(a, d->n, st);
}

extern "C" int64_t ctmr_flash_attention_f16x2_workspace_bytes(const ctmr_attn_desc* d) {
  using namespace ctmr;
  if (!d || d->n < 1 || d->lq < 1 || d->lk < 1 || d->heads < 1) return -1;
  return split_plan(d).bytes;
}

extern "C" int ctmr_flash_attention_f16x2(const ctmr_attn_desc* d, const float* q, const float* k, const float* v,
                                          float* out, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace ctmr;
  if (const int rc = check_attn(d, q, k, v, out, "ctmr_flash_attention_f16x2")) return rc;
  const SplitPlan plan = split_plan(d);
  if (!workspace || workspace_bytes < plan.bytes) {
    set_error("ctmr_flash_attention_f16x2: workspace of %lld bytes needed, %lld given", (long long)plan.bytes,
              (long long)(workspace ? workspace_bytes : 0));
    return CTMR_E_INVALID;
  }
  if (((uintptr_t)workspace & 255u) != 0)
    return fail(CTMR_E_INVALID, "ctmr_flash_attention_f16x2: workspace must be 256-byte aligned");
  // One split thread per (tensor, batch item, head, row, 8-dim group): the
  // dispatch packet counts work-items in 32 bits.
  if ((int64_t)d->n * d->heads * 4 * std::max<int64_t>(d->lq, plan.lkp) > 0x7fffff00ll)
    return fail(CTMR_E_UNSUPPORTED, "ctmr_flash_attention_f16x2: n * heads * length exceeds the split pass's grid");
  char* ws = static_cast<char*>(workspace);
  _Float16* planes[6];
  for (int i = 0; i < 6; ++i) planes[i] = reinterpret_cast<_Float16*>(ws + plan.offset[i]);
  hipStream_t st = (hipStream_t)stream;
  SplitArgs sa{{q, k, v},
               {d->ldq, d->ldk, d->ldv},
               {d->lq, d->lk, d->lk},
               {d->lq, (int)plan.lkp, (int)plan.lkp},
               {planes[0], planes[2], planes[4]},
               {planes[1], planes[3], planes[5]},
               d->heads,
               (float)((double)d->scale * 1.4426950408889634)};
  const int64_t rows = std::max<int64_t>(d->lq, plan.lkp);
  dim3 grid((unsigned)ceil_div((int64_t)d->n * d->heads * 4 * rows, 256), 3);
  hipLaunchKernelGGL(attention_split_kernel, grid, dim3(256), 0, st, sa, d->n);
  if (const int rc = check_launch("attention_split_kernel")) return rc;
  SplitAttnArgs a{planes[0], planes[1], planes[2], planes[3], planes[4], planes[5], out, d->ldo,
                  d->lq, d->lk, (int)plan.lkp, d->heads};
  const int qt = d->query_tiles ? d->query_tiles : attention_query_tiles(d->n, d->lq, d->heads);
  if (attention_key_parts(d->n, d->lq, d->lk, d->heads) == 2)
    return qt == 2 ? launch_attention_split<2, 2>(a, d->n, st) : launch_attention_split<1, 2>(a, d->n, st);
  return qt == 2 ? launch_attention_split<2, 1>(a, d->n, st) : launch_attention_split<1, 1>(a, d->n, st);
}
