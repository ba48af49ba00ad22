// ss_device.h - device helpers shared by the gfx950 kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ss_kernels.h"

namespace ssk {

constexpr int kWave = 64;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over 8 consecutive lanes (all 8 must be active), result in every lane.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  return v;
}

// Sum over the whole wave, result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = sum8(v);
  v += dpp<0x140>(v);  // row_mirror: 16-lane rows
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xb1>(v));
  v = fmaxf(v, dpp<0x4e>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// The FFN activations of layer_scheduler.c:529-547: SiLU (g / (1 + e^-g))
// and the tanh form of GELU for Gemma's GeGLU (tensor.c:181-190).
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_tanh(float g) {
  const float inner = 0.7978845608028654f * (g + 0.044715f * (g * g * g));
  return 0.5f * g * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);   // round to nearest even
}

// "b beats a" for the first-maximum argmax of tensor.c:318-328: larger
// value, or equal value at a smaller index. NaN never beats anything.
__device__ __forceinline__ bool beats(float bv, int bi, float av, int ai) {
  return bv > av || (bv == av && bi < ai);
}

// Best (value, index) over the wave, in every lane.
__device__ __forceinline__ void wave_best(float& bv, int& bi) {
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (beats(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

// Attention split of positions 0..ctx-1 over ns workgroups per KV head:
// chunk positions each, `active` of them non-empty. chunk is ctx / ns
// rounded up, at least 32, and with fill > 0 at least fill (one round of
// attention loads). So while ns * fill covers the context every split is
// one round starting at split * fill, which the attention can compute
// before it reads the position, and while kMergeSplits * fill covers it at
// most kMergeSplits splits are active (a consumer merges that many while
// staging). Shared by the attention kernel and the consumers that merge
// its splits, which must pass the same fill.
__device__ __forceinline__ void attn_chunks(int ctx, int ns, int fill, int& chunk, int& active) {
  chunk = (ctx + ns - 1) / ns;
  if (fill > 0) chunk = max(chunk, fill);
  if (chunk < 32) chunk = 32;
  active = (ctx + chunk - 1) / chunk;
}

// The strided split of the grouped-head attention (groups of 4 or 8 query
// heads): split s holds positions s, s + ns, s + 2 ns, ..., so the first
// min(ctx, ns) splits are non-empty. Shared by that attention and the
// consumers that merge its splits.
__device__ __forceinline__ int attn_strided_active(int ctx, int ns) { return min(ctx, ns); }

// Packed weight tiles: 16 rows x 4 blocks of 32 columns, one block chunk per
// lane (layout documented in ss_gemv.hip).
constexpr int kRowsPerTile = 16;
constexpr int kBlocksPerTile = 4;
constexpr int kTilesPerScaleGroup = 8;

__device__ __forceinline__ size_t tile_idx(int g, int ntk, int t, int lane) {
  return ((size_t)g * ntk + t) * kWave + lane;
}

// lane of a tile that holds block b of row r
__device__ __forceinline__ int tile_lane(int r, int b) {
  return (b % kBlocksPerTile) * kRowsPerTile + r % kRowsPerTile;
}

// binary16 index of the scale of (tile t, lane) of row group g: each lane's
// scales of a unit of 8 tiles are 16 contiguous bytes
__device__ __forceinline__ size_t scale_idx(int g, int ntk, int t, int lane) {
  const int nu = (ntk + kTilesPerScaleGroup - 1) / kTilesPerScaleGroup;
  return (((size_t)g * nu + t / kTilesPerScaleGroup) * kWave + lane) * kTilesPerScaleGroup +
         t % kTilesPerScaleGroup;
}

__device__ __forceinline__ int sdot4(uint32_t a, int b, int c) {
  return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int q8c(float f) {   // round to nearest even, then clamp to int8
  return (int)fminf(fmaxf(rintf(f), -127.f), 127.f);
}

// Coherent exchange between workgroups of one launch: relaxed agent-scope
// atomic loads and stores (global_load/global_store sc1 on gfx950) reach
// the device-coherent level without flushing or invalidating the L2; a
// writer drains its stores (vm_drain) before it signals.
__device__ __forceinline__ uint32_t cld(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t cld64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cst(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cst64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float cldf(const float* p) {
  return __uint_as_float(cld(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void cstf(float* p, float v) {
  cst(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
// every vector memory operation of this wave has completed
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)d << 24);
}

template <int QT>
struct QTraits;
template <>
struct QTraits<2> {            // Q4_0
  static constexpr int kQB = 16;         // code bytes per block
  static constexpr int kGgufBytes = 18;  // GGUF block bytes
};
template <>
struct QTraits<8> {            // Q8_0
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 34;
};
template <>
struct QTraits<3> {             // Q4_1: nibbles as Q4_0's, (d, m) scale entry
  static constexpr int kQB = 16;
  static constexpr int kGgufBytes = 20;
};
template <>
struct QTraits<6> {             // Q5_0 (packed into the Q8_0 format)
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 22;
};
template <>
struct QTraits<7> {             // Q5_1: 5-bit codes as int8, (d, m) scale entry
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 24;
};
template <>
struct QTraits<9> {             // Q8_1: int8 codes, fp32 d
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 40;
};
template <>
struct QTraits<1> {             // F16: 32 binary16 weights per block chunk
  static constexpr int kQB = 64;
  static constexpr int kGgufBytes = 64;
};
template <>
struct QTraits<0> {             // F32: 32 fp32 weights per block chunk
  static constexpr int kQB = 128;
  static constexpr int kGgufBytes = 128;
};
template <>
struct QTraits<12> {           // Q4_K: a 32-weight sub-block packs like a Q4_0 block
  static constexpr int kQB = 16;
  static constexpr int kGgufBytes = 144;   // per 256-weight super-block
};
template <>
struct QTraits<10> {           // Q2_K: 2-bit codes in nibbles
  static constexpr int kQB = 16;
  static constexpr int kGgufBytes = 84;
};
template <>
struct QTraits<11> {           // Q3_K: 3-bit codes + 4 in nibbles
  static constexpr int kQB = 16;
  static constexpr int kGgufBytes = 110;
};
template <>
struct QTraits<13> {           // Q5_K: 5-bit codes as int8
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 176;
};
template <>
struct QTraits<14> {           // Q6_K: 6-bit codes - 32 as int8
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 210;
};


// ------------------------------------------------------------ x records
// Matvec inputs as x records: 16 consecutive values v (times the consumer's
// RMSNorm weight when it has one) as three int8 levels,
// v ~= s3 * (16384*q1 + 128*q2 + q3) with s1 = max|v|/127, s3 = s1/16384,
// exact to max|v| * 2.4e-7 (fp32 rounding size). Record words: [0,4) q1,
// [4,8) q2, [8,12) q3 (4 codes per word, value order), [12] 8*sum X (the
// Q4_0 offset term), [13] s3, [14] sum of squares of the unnormalised values
// (the consumer's RMSNorm statistic), [15] 0. A block dot product of 32
// weights is two exact integer sums of v_dot4 over the levels (one per
// 16-value half) and one fp32 rounding per half.
constexpr int kRW = 16;    // words per x record

// Raw buffer view flags (dword 3 of the descriptor). Loads past the view's
// range return zero.
constexpr int kBufferFlags = 0x00020000;

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// reductions over the 16 lanes of a DPP row (all 16 active)
__device__ __forceinline__ float row16_max(float m) {
  m = fmaxf(m, dppf<0xb1>(m));
  m = fmaxf(m, dppf<0x4e>(m));
  m = fmaxf(m, dppf<0x141>(m));
  m = fmaxf(m, dppf<0x140>(m));
  return m;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dppf<0xb1>(v);
  v += dppf<0x4e>(v);
  v += dppf<0x141>(v);
  v += dppf<0x140>(v);
  return v;
}
__device__ __forceinline__ int row16_sum_i(int v) {
  v += dpp_i<0xb1>(v);
  v += dpp_i<0x4e>(v);
  v += dpp_i<0x141>(v);
  v += dpp_i<0x140>(v);
  return v;
}
// the low bytes of the 4 lanes of a quad as one word, in every lane of it
__device__ __forceinline__ uint32_t quad_pack(int q) {
  return ((uint32_t)dpp_i<0x00>(q) & 0xffu) | (((uint32_t)dpp_i<0x55>(q) & 0xffu) << 8) |
         (((uint32_t)dpp_i<0xaa>(q) & 0xffu) << 16) | ((uint32_t)dpp_i<0xff>(q) << 24);
}

struct Enc {
  uint32_t w[3];
  uint32_t x8, s3, ssq;
};

// Encode the values v of the 16 lanes of a row (lane r holds value r);
// raw is the unnormalised value for the sum of squares. Lane r with r%4 == 0
// gets words 4l + r/4 (l = 0, 1, 2); every lane gets words 12..14.
__device__ __forceinline__ Enc enc16(float v, float raw) {
  const float m = row16_max(fabsf(v));
  const float s3 = m * (1.0f / (127.0f * 16384.0f));
  const float s1 = s3 * 16384.0f, s2 = s3 * 128.0f;
  const float i1 = m > 0.f ? 127.0f / m : 0.f;   // 1 / s1
  const int q1 = q8c(v * i1);
  const float r1 = fmaf((float)-q1, s1, v);
  const int q2 = q8c(r1 * (i1 * 128.0f));
  const float r2 = fmaf((float)-q2, s2, r1);
  const int q3 = q8c(r2 * (i1 * 16384.0f));
  const int X = row16_sum_i(q1 * 16384 + q2 * 128 + q3);
  Enc e;
  e.w[0] = quad_pack(q1);
  e.w[1] = quad_pack(q2);
  e.w[2] = quad_pack(q3);
  e.x8 = (uint32_t)(8 * X);
  e.s3 = __float_as_uint(m == m && m < INFINITY ? s3 : m);   // non-finite input stays non-finite
  e.ssq = __float_as_uint(row16_sum(raw * raw));
  return e;
}

// Write a record (16 lanes, lane r) to LDS or, coherently, to global memory.
__device__ __forceinline__ void put_rec_lds(uint32_t* dst, const Enc& e, int r) {
  if ((r & 3) == 0) {
#pragma unroll
    for (int l = 0; l < 3; ++l) dst[4 * l + r / 4] = e.w[l];
  }
  if (r == 0) {
    dst[12] = e.x8;
    dst[13] = e.s3;
    dst[14] = e.ssq;
    dst[15] = 0;
  }
}
__device__ __forceinline__ void put_rec_global(uint32_t* dst, const Enc& e, int r) {
  if ((r & 3) == 0) {
#pragma unroll
    for (int l = 0; l < 3; ++l) cst(dst + 4 * l + r / 4, e.w[l]);
  }
  if (r == 0) {
    cst(dst + 12, e.x8);
    cst(dst + 13, e.s3);
    cst(dst + 14, e.ssq);
    cst(dst + 15, 0u);
  }
}

// ------------------------------------------------------------ block dot products
// Q4_0 block (quantize.c:60-72: byte j holds weight j in its low nibble and
// weight j+16 in its high nibble, value d * (nibble - 8)) against the x
// records of its two 16-column halves; the caller multiplies by d. The -8
// offset comes from the records' 8 * sum X. |sum nibble * X| <= 16 * 15 *
// 2097151 < 2^31.
__device__ __forceinline__ float q4_dot(const uint4 q, const uint32_t* ra, const uint32_t* rb) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  int a = 0, b = 0;
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    const uint4 xa = *reinterpret_cast<const uint4*>(ra + 4 * l);
    const uint4 xb = *reinterpret_cast<const uint4*>(rb + 4 * l);
    if (l) {
      a <<= 7;
      b <<= 7;
    }
    a = sdot4(w[0] & 0x0F0F0F0Fu, (int)xa.x, a);
    a = sdot4(w[1] & 0x0F0F0F0Fu, (int)xa.y, a);
    a = sdot4(w[2] & 0x0F0F0F0Fu, (int)xa.z, a);
    a = sdot4(w[3] & 0x0F0F0F0Fu, (int)xa.w, a);
    b = sdot4((w[0] >> 4) & 0x0F0F0F0Fu, (int)xb.x, b);
    b = sdot4((w[1] >> 4) & 0x0F0F0F0Fu, (int)xb.y, b);
    b = sdot4((w[2] >> 4) & 0x0F0F0F0Fu, (int)xb.z, b);
    b = sdot4((w[3] >> 4) & 0x0F0F0F0Fu, (int)xb.w, b);
  }
  const uint2 ta = *reinterpret_cast<const uint2*>(ra + 12);
  const uint2 tb = *reinterpret_cast<const uint2*>(rb + 12);
  return fmaf((float)(a - (int)ta.x), __uint_as_float(ta.y), (float)(b - (int)tb.x) * __uint_as_float(tb.y));
}

// Q4_K sub-block (quantize.c:265-310: weight = dsc * q - dmn with q the
// nibble, dsc = d * scale and dmn = dmin * min of the sub-block, both exact
// in fp32), packed like a Q4_0 block (nibble j of weight j, j + 16 in the
// high nibble) but without the -8 offset: sum w x = dsc * sum q X s3 -
// dmn * sum X s3 per 16-value record, sum X being the records' [12] / 8.
__device__ __forceinline__ float q4k_dot(const uint4 q, const uint32_t* ra, const uint32_t* rb, float dsc,
                                         float dmn) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  int a = 0, b = 0;
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    const uint4 xa = *reinterpret_cast<const uint4*>(ra + 4 * l);
    const uint4 xb = *reinterpret_cast<const uint4*>(rb + 4 * l);
    if (l) {
      a <<= 7;
      b <<= 7;
    }
    a = sdot4(w[0] & 0x0F0F0F0Fu, (int)xa.x, a);
    a = sdot4(w[1] & 0x0F0F0F0Fu, (int)xa.y, a);
    a = sdot4(w[2] & 0x0F0F0F0Fu, (int)xa.z, a);
    a = sdot4(w[3] & 0x0F0F0F0Fu, (int)xa.w, a);
    b = sdot4((w[0] >> 4) & 0x0F0F0F0Fu, (int)xb.x, b);
    b = sdot4((w[1] >> 4) & 0x0F0F0F0Fu, (int)xb.y, b);
    b = sdot4((w[2] >> 4) & 0x0F0F0F0Fu, (int)xb.z, b);
    b = sdot4((w[3] >> 4) & 0x0F0F0F0Fu, (int)xb.w, b);
  }
  const uint2 ta = *reinterpret_cast<const uint2*>(ra + 12);
  const uint2 tb = *reinterpret_cast<const uint2*>(rb + 12);
  const float sa = __uint_as_float(ta.y), sb = __uint_as_float(tb.y);
  const float qx = fmaf((float)a, sa, (float)b * sb);
  const float sx = fmaf((float)((int)ta.x >> 3), sa, (float)((int)tb.x >> 3) * sb);
  return fmaf(dsc, qx, -dmn * sx);
}

// The K-quants other than Q4_K: a 32-weight block is two 16-weight groups,
// each with weight = A * c - B (A = d * scale, B = dmin * min, or B = 4 A for
// Q3_K's codes stored + 4, B = 0 for Q6_K; all exact in fp32). The block's
// scale entry e and super-block word sup = d | dmin << 16 give A and B:
//   Q2_K (quantize.c:180-215)  e = scale byte of each group (scale | min << 4)
//   Q3_K (:219-263)            e = the groups' 6-bit scales; A = d (s - 32)
//   Q5_K (:312-346)            e = scale | min << 8, one pair for the block
//   Q4_K (:265-310)            as Q5_K (the prompt products; the matvec uses q4k_dot)
//   Q6_K (:350-383)            e = the groups' int8 scales
template <int QT>
__device__ __forceinline__ void kq_affine(uint32_t e, uint32_t sup, float (&A)[2], float (&B)[2]) {
  const float d = h2f((uint16_t)(sup & 0xffffu)), dm = h2f((uint16_t)(sup >> 16));
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint32_t b = (e >> (8 * g)) & 0xffu;
    if constexpr (QT == 10) {
      A[g] = d * (float)(b & 15u);
      B[g] = dm * (float)(b >> 4);
    } else if constexpr (QT == 11) {
      A[g] = d * (float)((int)b - 32);
      B[g] = 4.0f * A[g];
    } else if constexpr (QT == 13 || QT == 12) {   // Q5_K, Q4_K: one pair for the block
      A[g] = d * (float)(e & 0xffu);
      B[g] = dm * (float)(e >> 8);
    } else {
      A[g] = d * (float)(int8_t)b;
      B[g] = 0.f;
    }
  }
}

// sum over one 16-value record of code * X, exact: X = 16384 q1 + 128 q2 + q3
// from the record's three int8 levels; nibble codes (w[i] & 0x0F0F0F0F or
// >> 4) or int8 codes (|code| <= 32 keeps the sum inside int32)
template <bool NIB, bool HIGH>
__device__ __forceinline__ int rec_sum(const uint32_t (&w)[4], const uint32_t* r) {
  int a = 0;
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    const uint4 x = *reinterpret_cast<const uint4*>(r + 4 * l);
    if (l) a <<= 7;
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = NIB ? (HIGH ? (w[i] >> 4) & 0x0F0F0F0Fu : w[i] & 0x0F0F0F0Fu) : w[i];
      a = sdot4(c, (int)xs[i], a);
    }
  }
  return a;
}

// One 32-weight block of a K-quant other than Q4_K: sum over both groups of
// A * (sum c X) s3 - B * (sum X) s3, sum X being the record's word 12 / 8.
template <int QT>
__device__ __forceinline__ float kq_dot(const uint4 qa, const uint4 qb, const uint32_t* ra, const uint32_t* rb,
                                        uint32_t e, uint32_t sup) {
  float A[2], B[2];
  kq_affine<QT>(e, sup, A, B);
  int a, b;
  if constexpr (QT == 10 || QT == 11) {   // nibbles: weight j low, j + 16 high
    const uint32_t w[4] = {qa.x, qa.y, qa.z, qa.w};
    a = rec_sum<true, false>(w, ra);
    b = rec_sum<true, true>(w, rb);
  } else {                                // int8 codes: 16 per record
    const uint32_t wa[4] = {qa.x, qa.y, qa.z, qa.w}, wb[4] = {qb.x, qb.y, qb.z, qb.w};
    a = rec_sum<false, false>(wa, ra);
    b = rec_sum<false, false>(wb, rb);
  }
  const uint2 ta = *reinterpret_cast<const uint2*>(ra + 12);
  const uint2 tb = *reinterpret_cast<const uint2*>(rb + 12);
  const float sa = __uint_as_float(ta.y), sb = __uint_as_float(tb.y);
  const float qx = fmaf(A[0], (float)a * sa, A[1] * ((float)b * sb));
  const float sx = fmaf(B[0], (float)((int)ta.x >> 3) * sa, B[1] * ((float)((int)tb.x >> 3) * sb));
  return qx - sx;
}

// Q8_0 block (quantize.c:139-149: 32 int8 codes, value d * code); levels 1-2
// and level 3 are summed apart to stay in int32 and joined in fp32.
__device__ __forceinline__ float q8_dot(const uint4 qa, const uint4 qb, const uint32_t* ra, const uint32_t* rb) {
  const uint32_t wa[4] = {qa.x, qa.y, qa.z, qa.w}, wb[4] = {qb.x, qb.y, qb.z, qb.w};
  int a12 = 0, b12 = 0, a3 = 0, b3 = 0;
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    const uint4 xa = *reinterpret_cast<const uint4*>(ra + 4 * l);
    const uint4 xb = *reinterpret_cast<const uint4*>(rb + 4 * l);
    int sa = l == 1 ? a12 << 7 : 0, sb = l == 1 ? b12 << 7 : 0;
    sa = sdot4(wa[0], (int)xa.x, sa);
    sa = sdot4(wa[1], (int)xa.y, sa);
    sa = sdot4(wa[2], (int)xa.z, sa);
    sa = sdot4(wa[3], (int)xa.w, sa);
    sb = sdot4(wb[0], (int)xb.x, sb);
    sb = sdot4(wb[1], (int)xb.y, sb);
    sb = sdot4(wb[2], (int)xb.z, sb);
    sb = sdot4(wb[3], (int)xb.w, sb);
    if (l < 2) {
      a12 = sa;
      b12 = sb;
    } else {
      a3 = sa;
      b3 = sb;
    }
  }
  const float sa3 = __uint_as_float(ra[13]), sb3 = __uint_as_float(rb[13]);
  return fmaf(fmaf((float)a12, 128.0f, (float)a3), sa3, fmaf((float)b12, 128.0f, (float)b3) * sb3);
}

// Q5_1 block (quantize.c:114-137: weight = q * d + m, q = 0..31, stored as
// int8 codes): d * sum q X s3 + m * sum X s3 per 16-value record, sum X
// being the records' [12] / 8.
__device__ __forceinline__ float q51_dot(const uint4 qa, const uint4 qb, const uint32_t* ra, const uint32_t* rb,
                                         float d, float m) {
  const float qx = q8_dot(qa, qb, ra, rb);
  const uint2 ta = *reinterpret_cast<const uint2*>(ra + 12);
  const uint2 tb = *reinterpret_cast<const uint2*>(rb + 12);
  const float sx = fmaf((float)((int)ta.x >> 3), __uint_as_float(ta.y),
                        (float)((int)tb.x >> 3) * __uint_as_float(tb.y));
  return fmaf(d, qx, m * sx);
}


// A 32-column block staged in LDS by a matvec: the records of its two
// 16-value halves, back to back.
constexpr int kXW = 2 * kRW;   // words per block

// Encode one group of 4 values into the block's records in LDS: 8 lanes per
// block (all active), lane sub holding values 4*sub .. 4*sub+3, so each
// record is one DPP quad. Word [14] (the sum of squares) is not written: a
// matvec that encodes its own x sums the squares itself.
__device__ __forceinline__ void encode4(int* xb, int sub, float4 v) {
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  m = fmaxf(m, dpp<0xb1>(m));
  m = fmaxf(m, dpp<0x4e>(m));
  const float s3 = m * (1.0f / (127.0f * 16384.0f));
  const float s1 = s3 * 16384.0f, s2 = s3 * 128.0f;
  const float i1 = m > 0.f ? 127.0f / m : 0.f;   // 1 / s1
  const float f[4] = {v.x, v.y, v.z, v.w};
  int q1[4], q2[4], q3[4], X = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    q1[k] = q8c(f[k] * i1);
    const float r1 = fmaf((float)-q1[k], s1, f[k]);
    q2[k] = q8c(r1 * (i1 * 128.0f));
    const float r2 = fmaf((float)-q2[k], s2, r1);
    q3[k] = q8c(r2 * (i1 * 16384.0f));
    X += q1[k] * 16384 + q2[k] * 128 + q3[k];
  }
  X += dpp_i<0xb1>(X);
  X += dpp_i<0x4e>(X);
  int* r = xb + (sub >> 2) * kRW;
  const int w = sub & 3;
  r[w] = (int)pack4(q1[0], q1[1], q1[2], q1[3]);
  r[4 + w] = (int)pack4(q2[0], q2[1], q2[2], q2[3]);
  r[8 + w] = (int)pack4(q3[0], q3[1], q3[2], q3[3]);
  if (w == 0) {
    r[12] = 8 * X;
    r[13] = __float_as_int(m == m && m < INFINITY ? s3 : m);   // non-finite x stays non-finite
  }
}

}  // namespace ssk
