// ss_device.h - device helpers shared by the gfx950 kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
// chunk positions each (at least 32), `active` of them non-empty. Shared by
// the attention kernel and the consumers that merge its splits.
__device__ __forceinline__ void attn_chunks(int ctx, int ns, int& chunk, int& active) {
  chunk = (ctx + ns - 1) / ns;
  if (chunk < 32) chunk = 32;
  active = (ctx + chunk - 1) / chunk;
}

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

// An x record: 32 values v_j of one block as three int8 levels,
// v_j ~= s3 * X_j with X_j = 16384*q1_j + 128*q2_j + q3_j (q1 = v/s1 rounded,
// q2 and q3 the rounded remainders at 1/128 and 1/16384 of s1 = max|v|/127).
// Words: [0,8) q1, [8,16) q2, [16,24) q3 (4 codes per word, column order),
// [24] 8 * sum_j X_j (the Q4_0 offset term), [25] s3 (fp32 bits).
constexpr int kXW = 28;   // words per block (7 x 16 B)

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)d << 24);
}

// Encode one group of 4 staged values (8 lanes per block, all active).
__device__ __forceinline__ void encode4(int* xb, int sub, float4 v) {
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  m = fmaxf(m, dpp<0xb1>(m));
  m = fmaxf(m, dpp<0x4e>(m));
  m = fmaxf(m, dpp<0x141>(m));
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
  X += dpp_i<0x141>(X);
  xb[sub] = (int)pack4(q1[0], q1[1], q1[2], q1[3]);
  xb[8 + sub] = (int)pack4(q2[0], q2[1], q2[2], q2[3]);
  xb[16 + sub] = (int)pack4(q3[0], q3[1], q3[2], q3[3]);
  if (sub == 0) {
    xb[24] = 8 * X;
    xb[25] = __float_as_int(m == m && m < INFINITY ? s3 : m);   // non-finite x stays non-finite
  }
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

}  // namespace ssk
