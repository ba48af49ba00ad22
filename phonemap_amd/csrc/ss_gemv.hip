// ss_gemv.hip - block-quantized matrix-vector kernels for gfx950.
//
// Device weight layout (made by k_pack from GGUF blocks): a tile is 16 rows
// x 4 consecutive 32-column blocks = 64 block chunks, one per lane; chunk
// (row, block) sits at lane (block % 4) * 16 + row % 16 of tile
// (row / 16, block / 4), tiles of a row group being consecutive:
// code[(g * ntk + t) * 64 + lane] of 16 (Q4_0) or 32 (Q8_0) bytes. The
// binary16 scales follow in a second plane, each lane's scales of 8
// consecutive tiles in 16 contiguous bytes. Rows are padded to a multiple of
// 16 and blocks to a multiple of 4 with zero codes and scales. A wave loads a
// tile as one contiguous 1 KiB (Q4_0) read.
//
// Q4_K matrices (256-weight super-blocks of eight 32-weight sub-blocks, each
// with a 6-bit scale and min, quantize.c:265-310) use the same tiles: a
// sub-block's 32 nibbles are stored as a Q4_0 block's (without the -8
// offset), its entry in the scale plane is scale | min << 8, and a third
// plane holds each row's super-block (d, dmin) pair of binary16s:
// su[(g * nsb + sb) * 16 + row % 16], nsb = cols / 256. 18.5 bytes per 32
// weights against the GGUF format's 18.
//
// The other 32-weight block types use the same tiles. Q4_1 (d * q + m)
// stores its nibbles as Q4_0 does, Q5_1 its 5-bit codes as int8 and Q8_1
// its int8 codes, each with a 32-bit scale-plane entry per block (d | m << 16
// as binary16, or Q8_1's fp32 d; a lane's 8 tiles in 32 contiguous bytes).
// Q5_0 ((q - 16) * d) is packed into the Q8_0 format. F16 and F32 matrices
// store each block's 32 weights (64 or 128 bytes per lane chunk) and have no
// scale plane; their dot products take x as fp32 values decoded from the
// staged records.
//
// k_gemv: workgroup = one 16-row group; wave s takes units (UT consecutive
// tiles) s, s+S, ... of it. A wave requests its x slice, then every chunk and
// scale of its unit, before using any; it encodes its own slice of x into its
// own LDS region (no workgroup barrier before the dot products) and
// accumulates exact integer block dot products scaled in fp32. Per row, the
// 4 lanes holding it are added with two shuffles and the S waves in LDS in
// wave order, so results do not depend on timing; no data passes between
// workgroups. 16-row groups give >= 256 workgroups for every 7B-shape matrix.

#include <math.h>

#include <type_traits>
#include <utility>

#include <hip/hip_ext.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

// x in LDS, per 32-column block: the staged values v_j (x_j times the RMSNorm
// weight) as three int8 levels, v_j ~= s3 * X_j with
// X_j = 16384*q1_j + 128*q2_j + q3_j (q1 = v/s1 rounded, q2 and q3 the
// rounded remainders at 1/128 and 1/16384 of s1 = max|v|/127). The error is
// at most s3/2 = max|v| * 2.4e-7 per value, the size of fp32 rounding, so
// dot products become exact integer sums (v_dot4) plus one fp32 rounding per
// block. Words: [0,8) q1, [8,16) q2, [16,24) q3 (4 codes per word, column
// order), [24] 8 * sum_j X_j (the Q4_0 offset term), [25] s3 (fp32 bits).

// A wave stages only the x slice of its own unit (UT*4 blocks of 32 values),
// times the RMSNorm weight nw when set (the x*w of cpu_neon.c:114; the 1/rms
// factor is applied to the row sums), into its own LDS region: the waves of a
// workgroup cover disjoint columns, so no barrier precedes the dot products.
// Blocks at or past nb (tile padding) are zero. Lane l handles groups of 4
// values j*64 + l (eight lanes per block). xfetch issues the loads and xput
// encodes them, so the weight loads can be issued in between: vector loads
// complete in issue order, and x must not queue behind the weights.
template <int UT>
struct XSlice {
  float4 v[UT / 2], w[UT / 2];
};

template <int UT>
__device__ __forceinline__ void xfetch(XSlice<UT>& p, const float* __restrict__ x, const float* __restrict__ nw,
                                       int u, int nb, int lane) {
  const float* wp = nw ? nw : x;   // branch-free: the loads are counted exactly
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    const int gi = j * kWave + lane;
    const int col = min(u * UT * kTB + (gi >> 3), nb - 1) * 32 + (gi & 7) * 4;
    p.v[j] = *reinterpret_cast<const float4*>(x + col);
    p.w[j] = *reinterpret_cast<const float4*>(wp + col);
  }
}

// Ties the x registers to this point of the program, so the compiler cannot
// sink their loads below the weight loads (xput only uses them under a mask).
__device__ __forceinline__ void pin(float4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// Returns this lane's share of sum(x^2) over the slice.
template <int UT>
__device__ __forceinline__ float xput(XSlice<UT>& p, int* xw, const float* nw, int u, int nb, int lane) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    pin(p.v[j]);
    pin(p.w[j]);
  }
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    const int gi = j * kWave + lane;
    const bool in = u * UT * kTB + (gi >> 3) < nb;
    float4 t = in ? p.v[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    ss = fmaf(t.x, t.x, ss);
    ss = fmaf(t.y, t.y, ss);
    ss = fmaf(t.z, t.z, ss);
    ss = fmaf(t.w, t.w, ss);
    if (nw) {
      t.x *= p.w[j].x;
      t.y *= p.w[j].y;
      t.z *= p.w[j].z;
      t.w *= p.w[j].w;
    }
    encode4(xw + (gi >> 3) * kXW, gi & 7, t);
  }
  return ss;
}

// Merge staging (the attention split merge inside the Wo matvec): x[col] for
// col in head h = G*kvh + g is sum_s o_s * e^(m_s - M) / sum_s l_s e^(m_s - M)
// over the active attention splits s of KV head kvh. A lane fetches the 4 o
// values of all kMergeSplits split slots for its group of 4 columns (slots
// past the active ones reload the last active split and get weight 0), and
// the (m, l) of one slot, lane % 8, of its head, before the weight loads, in
// one batch. The split weights e^(m_s - M) / sum are then formed once per
// aligned group of 8 lanes (the lanes of a group share a head: a head spans
// head_dim / 4 >= 16 lanes) with one exponential per lane and DPP
// reductions, and read back by every lane of the group with lane shuffles.
// head_dim and the group size are powers of two.
template <int UT>
struct MSlice {
  float2 ml[UT / 2];
  float4 o[UT / 2][kMergeSplits];
};

// the attention's active splits: the strided rule for groups of 4 or 8
// query heads, the range rule of attn_chunks for 1 or 2
__device__ __forceinline__ int merge_active(const GemvArgs& a) {
  if (a.att_group >= 4) return attn_strided_active(*a.dpos + 1, a.att_ns);
  int chunk, active;
  attn_chunks(*a.dpos + 1, a.att_ns, a.att_split_fill, chunk, active);
  return active;
}

// lim: slots at or past lim reload slot lim - 1 (the active count, or, before
// the position is read, the launch's split count: mput then excludes the
// slots past the active ones by selection)
template <int UT>
__device__ __forceinline__ void mfetch(MSlice<UT>& p, const GemvArgs& a, int u, int lim, int lane) {
  const int hd = a.head_dim, G = a.att_group;
  const int hs = __builtin_ctz(hd), gs = __builtin_ctz(G);
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    const int gi = j * kWave + lane;
    const int col = min(u * UT * kTB * 32 + (gi >> 3) * 32 + (gi & 7) * 4, a.cols - 4);
    const int h = col >> hs, d = col & (hd - 1);
    const int kvh = h >> gs, g = h & (G - 1);
    const size_t im = ((size_t)kvh * a.att_ns + min(lane & 7, lim - 1)) * G + g;
    p.ml[j] = *reinterpret_cast<const float2*>(a.att_ml + im * 2);
#pragma unroll
    for (int s = 0; s < kMergeSplits; ++s) {
      const size_t i = ((size_t)kvh * a.att_ns + min(s, lim - 1)) * G + g;
      p.o[j][s] = *reinterpret_cast<const float4*>(a.att_o + i * hd + d);
    }
  }
}

// max and sum over the aligned group of 8 lanes (all 8 active), in every lane
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp<0xb1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4e>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0x141>(v));   // row_half_mirror
  return v;
}

template <int UT>
__device__ __forceinline__ void mput(MSlice<UT>& p, int* xw, int u, int nb, int active, int lane) {
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    asm volatile("" : "+v"(p.ml[j].x), "+v"(p.ml[j].y));
#pragma unroll
    for (int s = 0; s < kMergeSplits; ++s) pin(p.o[j][s]);
  }
#pragma unroll
  for (int j = 0; j < UT / 2; ++j) {
    const int gi = j * kWave + lane;
    // this lane's slot: lane % 8 (slot 0 is always active, so M is finite)
    const bool live = (lane & 7) < active;
    const float M = max8(live ? p.ml[j].x : -INFINITY);
    const float e = live ? expf(p.ml[j].x - M) : 0.f;
    const float L = sum8(live ? p.ml[j].y * e : 0.f);
    const float w = e * (1.0f / L);
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < kMergeSplits; ++s) {
      const float ws = __shfl(w, (lane & ~7) | s, kWave);   // 0 past the active slots
      // a slot past the active ones may hold an earlier token's partials:
      // selected out, never multiplied in
      const float4 o = s < active ? p.o[j][s] : make_float4(0.f, 0.f, 0.f, 0.f);
      t.x = fmaf(o.x, ws, t.x);
      t.y = fmaf(o.y, ws, t.y);
      t.z = fmaf(o.z, ws, t.z);
      t.w = fmaf(o.w, ws, t.w);
    }
    if (u * UT * kTB + (gi >> 3) >= nb) t = make_float4(0.f, 0.f, 0.f, 0.f);
    encode4(xw + (gi >> 3) * kXW, gi & 7, t);
  }
}

// F16 / F32 matrices take x as fp32 values: the unit's records in this wave's
// LDS slice become v = s3 * (16384 q1 + 128 q2 + q3) in place, value j of a
// block at word j of its kXW (every lane reads all its record words before
// any lane writes; one wave owns the slice). Lanes read words other lanes
// wrote (a record's s3), so wavefront fences order the accesses: without
// them the compiler may hoist a lane's read of s3 above the write another
// lane makes on the other side of a branch.
template <int UT>
__device__ __forceinline__ void rec_to_float(int* xw, int lane) {
  constexpr int kN = UT * kTB * 8 / kWave;   // groups of 4 values per lane
  uint32_t q1[kN], q2[kN], q3[kN];
  float s3[kN];
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // the staged records are written
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    const int gi = i * kWave + lane, grp = gi & 7;
    const int* rp = xw + (gi >> 3) * kXW + (grp >> 2) * kRW;
    q1[i] = (uint32_t)rp[grp & 3];
    q2[i] = (uint32_t)rp[4 + (grp & 3)];
    q3[i] = (uint32_t)rp[8 + (grp & 3)];
    s3[i] = __int_as_float(rp[13]);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // all reads before the first write
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    const int gi = i * kWave + lane;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int X = 16384 * (int)(int8_t)(q1[i] >> (8 * k)) + 128 * (int)(int8_t)(q2[i] >> (8 * k)) +
                    (int)(int8_t)(q3[i] >> (8 * k));
      v[k] = s3[i] * (float)X;
    }
    *reinterpret_cast<float4*>(xw + (gi >> 3) * kXW + 4 * (gi & 7)) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// One F16 / F32 block chunk (32 weights in column order) against its 32 fp32
// x values, in four interleaved partial sums.
template <int QT>
__device__ __forceinline__ float float_dot(const uint4 (&q)[QTraits<QT>::kQB / 16], const float* xv) {
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < 8; ++v) {   // values 4v .. 4v+3
    const float4 x = *reinterpret_cast<const float4*>(xv + 4 * v);
    float w[4];
    if constexpr (QT == kF16) {
      const uint4 c = q[v / 2];
      const uint32_t lo = v & 1 ? c.z : c.x, hi = v & 1 ? c.w : c.y;
      w[0] = h2f((uint16_t)(lo & 0xffffu));
      w[1] = h2f((uint16_t)(lo >> 16));
      w[2] = h2f((uint16_t)(hi & 0xffffu));
      w[3] = h2f((uint16_t)(hi >> 16));
    } else {
      const uint4 c = q[v];
      w[0] = __uint_as_float(c.x);
      w[1] = __uint_as_float(c.y);
      w[2] = __uint_as_float(c.z);
      w[3] = __uint_as_float(c.w);
    }
    s[0] = fmaf(w[0], x.x, s[0]);
    s[1] = fmaf(w[1], x.y, s[1]);
    s[2] = fmaf(w[2], x.z, s[2]);
    s[3] = fmaf(w[3], x.w, s[3]);
  }
  return (s[0] + s[1]) + (s[2] + s[3]);
}

// One wave's share per round: a unit of UT (2, 4 or 8) consecutive tiles
// (those < ntk), every chunk of it requested before any is used. A unit lies
// inside one 8-tile scale group, whose 16 bytes per lane it reads UT/2 words of.
template <int QT, int NMAT, int UT>
struct Round {
  static constexpr int kNV = QTraits<QT>::kQB / 16;
  uint4 q[NMAT][UT][kNV];
  // the unit's scale entries, tile order: binary16 pairs (Q4_K: scale | min
  // << 8), or one 32-bit entry per tile (Q4_1, Q5_1: d | m << 16; Q8_1: fp32 d)
  uint32_t sc[NMAT][is_wide(QT) ? UT : UT / 2];
  uint32_t su[NMAT][is_kq(QT) ? UT / 2 : 1];   // K-quants: (d, dmin) of the unit's super-blocks
};

template <int QT, int NMAT, int UT>
__device__ __forceinline__ void load_round(Round<QT, NMAT, UT>& f, const GemvArgs& a, int g, int ntk,
                                           int u, int lane) {
  constexpr int kQB = QTraits<QT>::kQB;
  constexpr int kNV = kQB / 16;
  const int t0 = u * UT;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    const PackedMat& w = m == 0 ? a.w : a.w2;
    if constexpr (is_wide(QT)) {   // 32-bit entries: 4 bytes per tile
      const uint32_t* sp = reinterpret_cast<const uint32_t*>(w.ds) + scale_idx(g, ntk, t0, lane);
#pragma unroll
      for (int k = 0; k < UT; k += 4) {
        if constexpr (UT >= 4) {
          const uint4 v = *reinterpret_cast<const uint4*>(sp + k);
          f.sc[m][k] = v.x; f.sc[m][k + 1] = v.y; f.sc[m][k + 2] = v.z; f.sc[m][k + 3] = v.w;
        } else {
          const uint2 v = *reinterpret_cast<const uint2*>(sp);
          f.sc[m][0] = v.x; f.sc[m][1] = v.y;
        }
      }
    } else if constexpr (!is_float(QT)) {   // F16 / F32 have no scales
      const uint32_t* sp = reinterpret_cast<const uint32_t*>(w.ds + scale_idx(g, ntk, t0, lane));
      if constexpr (UT == 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(sp);
        f.sc[m][0] = v.x; f.sc[m][1] = v.y; f.sc[m][2] = v.z; f.sc[m][3] = v.w;
      } else if constexpr (UT == 4) {
        const uint2 v = *reinterpret_cast<const uint2*>(sp);
        f.sc[m][0] = v.x; f.sc[m][1] = v.y;
      } else {
        f.sc[m][0] = *sp;
      }
    }
    if constexpr (is_kq(QT)) {   // a unit (an even number of tiles) covers UT / 2 super-blocks
      const int nsb = ntk / 2;
#pragma unroll
      for (int j = 0; j < UT / 2; ++j)
        f.su[m][j] = w.su[((size_t)g * nsb + min(t0 / 2 + j, nsb - 1)) * kRG + lane % kRG];
    }
#pragma unroll
    for (int k = 0; k < UT; ++k) {
      // tiles past the row (last unit) reload the last tile and are skipped in fma_round
      const int t = min(t0 + k, ntk - 1);
      const uint4* src = reinterpret_cast<const uint4*>(w.qs + tile_idx(g, ntk, t, lane) * kQB);
#pragma unroll
      for (int v = 0; v < kNV; ++v) f.q[m][k][v] = src[v];
    }
  }
}

typedef int v4i __attribute__((ext_vector_type(4)));

// Q4_0 and Q8_0 tiles on the matrix cores. Lane l holds block l/16 of row
// l%16 (Q4_0: weight j in the low nibble of byte j and weight j+16 in its
// high nibble; Q8_0: weights 0-15, then 16-31, as int8). Each 16-value half
// of the tile is one v_mfma_i32_16x16x64_i8: lane l gives its half's 16
// weights as column l%16 of B at k = 16(l/16) .. +15, and A is block
// diagonal, row 4b + i holding level i of block b's x record at the same k
// (lanes l%16 = 4(l/16) + i, i < 3; every other lane gives zeros), so
// D[4b + i][n], register i of lane l, is the lane's own level-i sum over its
// half: the integers the sdot4 form (q4_dot, q8_dot) adds, combined the same
// way, so the results are bit for bit the same. zero: kZeroPad<UT> zero
// words in LDS (the A rows of the other lanes: every tile's offset from it
// stays inside it, so the addresses differ by constants alone).
template <int UT>
constexpr int kZeroPad = ((UT - 1) * kTB * kXW + kRW + 4 + 3) / 4 * 4;

template <int QT, int NMAT, int UT>
__device__ __forceinline__ void mfma_round(float (&acc)[NMAT], const Round<QT, NMAT, UT>& f, const int* xs,
                                           const int* zero, int lane) {
  const int kb = lane >> 4;
  const bool mine = ((lane & 15) >> 2) == kb && (lane & 3) < 3;
  // A rows of this lane: its level in the tile's records, or zeros
  const int* a0 = mine ? xs + kb * kXW + 4 * (lane & 3) : zero;
  const v4i z = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < UT; ++k) {
    const uint32_t* ra = reinterpret_cast<const uint32_t*>(xs + (k * kTB + kb) * kXW);
    const int* pa = a0 + k * kTB * kXW;
    const v4i alo = *reinterpret_cast<const v4i*>(pa);
    const v4i ahi = *reinterpret_cast<const v4i*>(pa + kRW);
    const uint2 ta = *reinterpret_cast<const uint2*>(ra + 12);         // (8 sum X, s3) of each half
    const uint2 tb = *reinterpret_cast<const uint2*>(ra + kRW + 12);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      const uint32_t sw = f.sc[m][k / 2];
      const uint32_t e = k & 1 ? sw >> 16 : sw & 0xffffu;
      v4i blo, bhi;
      if constexpr (QT == 2) {
        const uint4 q = f.q[m][k][0];
        blo = v4i{(int)(q.x & 0x0F0F0F0Fu), (int)(q.y & 0x0F0F0F0Fu), (int)(q.z & 0x0F0F0F0Fu),
                  (int)(q.w & 0x0F0F0F0Fu)};
        bhi = v4i{(int)((q.x >> 4) & 0x0F0F0F0Fu), (int)((q.y >> 4) & 0x0F0F0F0Fu),
                  (int)((q.z >> 4) & 0x0F0F0F0Fu), (int)((q.w >> 4) & 0x0F0F0F0Fu)};
      } else {
        blo = __builtin_bit_cast(v4i, f.q[m][k][0]);
        bhi = __builtin_bit_cast(v4i, f.q[m][k][1]);
      }
      const v4i dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, blo, z, 0, 0, 0);
      const v4i dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bhi, z, 0, 0, 0);
      float s;
      if constexpr (QT == 2) {   // q4_dot: sum X * nibble - 8 sum X, |.| < 2^31 per half
        const int a = (dl[0] << 14) + (dl[1] << 7) + dl[2];
        const int b = (dh[0] << 14) + (dh[1] << 7) + dh[2];
        s = fmaf((float)(a - (int)ta.x), __uint_as_float(ta.y), (float)(b - (int)tb.x) * __uint_as_float(tb.y));
      } else {                   // q8_dot: levels 1-2 in one integer, level 3 added in fp32
        const int a12 = (dl[0] << 7) + dl[1], b12 = (dh[0] << 7) + dh[1];
        s = fmaf(fmaf((float)a12, 128.0f, (float)dl[2]), __uint_as_float(ta.y),
                 fmaf((float)b12, 128.0f, (float)dh[2]) * __uint_as_float(tb.y));
      }
      acc[m] = fmaf(h2f((uint16_t)e), s, acc[m]);
    }
  }
}

// xs holds the unit's staged x records; kb is this lane's block within a
// tile. Tiles past the row (last unit) meet all-zero records (s3 = 0) and
// add exactly 0, so every tile is processed and the loads have no
// conditional use.
template <int QT, int NMAT, int UT>
__device__ __forceinline__ void fma_round(float (&acc)[NMAT], const Round<QT, NMAT, UT>& f, const int* xs,
                                          int kb, const int* zero, int lane) {
  if constexpr (QT == 2 || QT == 8) {
    mfma_round<QT, NMAT, UT>(acc, f, xs, zero, lane);
    return;
  }
#pragma unroll
  for (int k = 0; k < UT; ++k) {
    const uint32_t* ra = reinterpret_cast<const uint32_t*>(xs + (k * kTB + kb) * kXW);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      const uint32_t sw = f.sc[m][is_wide(QT) ? k : k / 2];
      const uint32_t e = is_wide(QT) ? sw : k & 1 ? sw >> 16 : sw & 0xffffu;
      if constexpr (is_float(QT)) {
        acc[m] += float_dot<QT>(f.q[m][k], reinterpret_cast<const float*>(ra));
      } else if constexpr (QT == kQ4_1) {   // d * q + m: Q4_K's dot with dsc = d, dmn = -m
        acc[m] += q4k_dot(f.q[m][k][0], ra, ra + kRW, h2f((uint16_t)(e & 0xffffu)), -h2f((uint16_t)(e >> 16)));
      } else if constexpr (QT == kQ5_1) {
        acc[m] += q51_dot(f.q[m][k][0], f.q[m][k][1], ra, ra + kRW, h2f((uint16_t)(e & 0xffffu)),
                          h2f((uint16_t)(e >> 16)));
      } else if constexpr (QT == kQ8_1) {
        acc[m] = fmaf(__uint_as_float(e), q8_dot(f.q[m][k][0], f.q[m][k][1], ra, ra + kRW), acc[m]);
      } else if constexpr (QT == kQ4K) {
        const uint32_t sup = f.su[m][k / 2];
        const float dsc = h2f((uint16_t)(sup & 0xffffu)) * (float)(e & 0xffu);   // exact
        const float dmn = h2f((uint16_t)(sup >> 16)) * (float)(e >> 8);
        acc[m] += q4k_dot(f.q[m][k][0], ra, ra + kRW, dsc, dmn);
      } else if constexpr (is_kq(QT)) {
        acc[m] += kq_dot<QT>(f.q[m][k][0], f.q[m][k][Round<QT, NMAT, UT>::kNV - 1], ra, ra + kRW, e, f.su[m][k / 2]);
      } else {
        float s;
        if constexpr (QT == 2)
          s = q4_dot(f.q[m][k][0], ra, ra + kRW);
        else
          s = q8_dot(f.q[m][k][0], f.q[m][k][1], ra, ra + kRW);
        acc[m] = fmaf(h2f((uint16_t)e), s, acc[m]);
      }
    }
  }
}

// Pre-encoded x: the unit's records (UT tiles x 4 blocks x 2 records of
// 64 B, written by the producer of x), 16 bytes per lane per piece, loaded
// into registers before the unit's weights and written to this wave's LDS
// slice once they land. The record buffer is padded with zero records to a
// multiple of 8 tiles, so the last unit of a row reads zeros past the
// vector. The pieces are separate named registers (an array or a struct
// here is kept in scratch memory), and going through registers lets the
// compiler wait for each tile's loads alone: a direct global-to-LDS copy of
// the records makes it wait for every load of the unit before the first LDS
// read.
template <int UT>
constexpr int kRecPieces = UT * kTB * kXW / 4 / kWave;   // 16-byte record pieces per lane
static_assert(kRecPieces<2> >= 1 && kRecPieces<8> <= 4, "one to four record pieces per lane");

// Epilogue in wave 0: every lane holds row `row`'s final value(s) v[]; lanes
// with `own` set (one per row) write.
// Values every lane of wave 0 loads before the weights, for its epilogue:
// the residual y[row] (EPI_ADD) and the next consumer's RMSNorm weight
// nw_out[row], so no load waits at the end of the kernel.
struct EpiPre {
  float y = 0.f, nw = 1.f;
};

template <int EPI>
__device__ __forceinline__ EpiPre epi_prefetch(const GemvArgs& a, int row) {
  EpiPre p;
  const int rr = min(row, a.rows - 1);
  if constexpr (EPI == EPI_ADD) p.y = a.y[rr];
  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_SWIGLU)
    if (a.xr_out && a.nw_out) p.nw = a.nw_out[rr];
  return p;
}

// Epilogue in wave 0: every lane holds row `row`'s final value(s) v[]; lanes
// with `own` set (one per row) write. With xr_out set, the 16 rows of the
// group are also written as one x record of (value * nw_out) for the next
// matvec (each DPP row of the wave holds the group's 16 rows in order).
template <int EPI, int NMAT>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int row, bool own, const float (&v)[NMAT],
                                         const EpiPre& pre) {
  const bool valid = own && row < a.rows;
  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_SWIGLU) {
    float out;
    if constexpr (EPI == EPI_SWIGLU) {
      const float g = v[0], u = v[NMAT - 1];
      // GeGLU for Gemma (layer_scheduler.c:529-531), else SwiGLU (:540-547)
      out = u * (a.act == 1 ? gelu_tanh(g) : silu(g));
    } else {
      out = EPI == EPI_ADD ? v[0] + pre.y : v[0];                       // layer_scheduler.c:484,566
    }
    if (row >= a.rows) out = 0.f;
    if (valid) a.y[row] = out;
    if (a.xr_out) {
      const Enc e = enc16(out * pre.nw, out);
      if (own) put_rec_lds(a.xr_out + (size_t)(row / kRG) * kRW, e, row % kRG);
    }
  } else if constexpr (EPI == EPI_QKV) {
    // rows of [Wq; Wk; Wv]; q and k rows (i, i+1) are lanes (2j, 2j+1): rotate
    // the pair with the position's (cos, sin), tensor.c:250-273
    // the bias (layer_scheduler.c:367-402) is added before RoPE
    const float x = a.bias && row < a.rows ? v[0] + a.bias[row] : v[0];
    const float partner = __shfl_xor(x, 1, kWave);
    if (!valid) return;
    const int pos = *a.dpos;
    const int hd = a.head_dim;
    float out = x;
    if (row < a.qdim + a.kvdim) {
      const int i = (row < a.qdim ? row : row - a.qdim) % hd;
      const int i0 = i & ~1;
      if (i0 < a.rope_dim) {
        const float* cs = a.rope_cs + (size_t)pos * a.rope_dim;
        const float c = cs[i0], s = cs[i0 + 1];
        out = (i & 1) ? partner * s + x * c : x * c - partner * s;
      }
    }
    if (row < a.qdim) {
      a.y[row] = out;
    } else {
      const bool is_v = row >= a.qdim + a.kvdim;
      const int kr = row - a.qdim - (is_v ? a.kvdim : 0);
      if (a.kv_type == 0) {   // fp16 cache [kvh][max_seq][hd]
        uint16_t* c = reinterpret_cast<uint16_t*>(is_v ? a.vcache : a.kcache);
        c[((size_t)(kr / hd) * a.max_seq + pos) * hd + kr % hd] = f2h(out);
      } else {                 // int8 cache: encoded by k_kv_append from this staging
        a.kv_f32[(is_v ? a.kvdim : 0) + kr] = out;
      }
    }
  } else if constexpr (EPI == EPI_LOGITS) {
    // Gemma's 1/sqrt(d) (layer_scheduler.c:667-672), then the final softcap
    // (:674-676, tensor.c:194-200), before the argmax sees the logit
    float y = v[0] * a.out_scale;
    if (a.softcap > 0.f) y = a.softcap * tanhf(y * a.softcap_inv);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (valid) {
      a.y[row] = y;
      bv = y;
      bi = row;
    }
    wave_best(bv, bi);
    if ((threadIdx.x & 63) == 0) a.part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

// Q8_0 and two-matrix rounds hold 64 VGPRs of codes: at most 8 waves, so
// 256 VGPRs are available to them.
template <int QT, int NMAT>
constexpr int gemv_max_waves() { return QT == 2 && NMAT == 1 ? 16 : 8; }

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
template <class F, int... I>
__device__ __forceinline__ void for_each_index_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void for_each_index(F&& f) {
  for_each_index_impl(f, std::make_integer_sequence<int, N>{});
}
template <int I, class T>
__device__ __forceinline__ T& pick(T& a0, T& a1, T& a2, T& a3) {
  static_assert(I >= 0 && I < 4, "at most four rounds");
  if constexpr (I == 0) return a0;
  else if constexpr (I == 1) return a1;
  else if constexpr (I == 2) return a2;
  else return a3;
}

// A unit's x records through registers (NR > 0): lane l holds 16-byte pieces
// l, l + 64, ... of the unit's UT*kTB*kXW words, written to the wave's LDS
// slice just before the unit is used. Register dependencies let the compiler
// wait for exactly the unit in use while the next one is in flight.
template <int UT>
struct XRec {
  uint4 v[UT * kTB * kXW / 4 / kWave];
};
template <int UT>
__device__ __forceinline__ void rload(XRec<UT>& r, const uint32_t* __restrict__ xr, int u, int lane) {
  const uint4* src = reinterpret_cast<const uint4*>(xr + (size_t)u * UT * kTB * kXW);
#pragma unroll
  for (int i = 0; i < UT * kTB * kXW / 4 / kWave; ++i) r.v[i] = src[i * kWave + lane];
}
template <int UT>
__device__ __forceinline__ void rput(int* xw, const XRec<UT>& r, int lane) {
#pragma unroll
  for (int i = 0; i < UT * kTB * kXW / 4 / kWave; ++i) reinterpret_cast<uint4*>(xw)[i * kWave + lane] = r.v[i];
}

// MERGE: how the matvec stages x. kMergeNone: from x or its records.
// Otherwise it merges the attention's split partials while staging (or, as
// the attention left them, takes its records): kMergeEarly with at most
// kMergeSplits splits launched requests the first unit's partials and
// weights before it reads the position; kMergeLate reads the position first.
constexpr int kMergeNone = 0, kMergeEarly = 1, kMergeLate = 2;

// NR > 0 (records path, every wave with at most NR units): all of a wave's
// units are requested at once, their records and weights in registers, and
// used in order.
template <int QT, int NMAT, int EPI, int UT, int MERGE, bool PX, int NR>
__global__ void __launch_bounds__((gemv_max_waves<QT, NMAT>() * 64)) k_gemv(const GemvArgs a) {
  extern __shared__ float4 smem4[];
  // zeros per wave for the matrix-core A rows (Q4_0, Q8_0)
  __shared__ v4i zpad[gemv_max_waves<QT, NMAT>()][(QT == 2 || QT == 8) ? kZeroPad<UT> / 4 : 1];
  int* xs = reinterpret_cast<int*>(smem4);
  static_assert(NR == 0 || PX, "rounds issued up front take x from the records");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (scalar)
  // written by its own wave before any use (fences below order the accesses)
  if constexpr (QT == 2 || QT == 8) {
    for (int i = lane; i < kZeroPad<UT> / 4; i += kWave) zpad[wave][i] = v4i{0, 0, 0, 0};
  }
  const int S = blockDim.x >> 6;
  const int kb = lane / kRG;
  const int g = blockIdx.x;
  const int nb = a.cols >> 5;
  const int ntk = (nb + kTB - 1) / kTB;
  const int nu = (ntk + UT - 1) / UT;
  constexpr int kSlice = UT * kTB * kXW;                              // words of one x slice
  int* xw = xs + wave * kSlice;                                       // this wave's x slice
  // [NMAT][16 rows][kMaxS waves], then [kMaxS]: a row's wave partials are
  // contiguous (16-byte aligned: kSlice is a multiple of 4 words)
  constexpr int kMaxS = gemv_max_waves<QT, NMAT>();
  float* red = reinterpret_cast<float*>(xs + S * kSlice);

  float acc[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) acc[m] = 0.f;
  float ssq = 0.f;
  Round<QT, NMAT, UT> rd;
  EpiPre pre;
  if (wave == 0) pre = epi_prefetch<EPI>(a, g * kRG + lane % kRG);

  // units go to waves round robin (one round for rows of up to S units)
  // REC: x from the records xr. A merging kernel takes them when the
  // attention wrote its output there itself: one active split directly,
  // more than kMergeSplits through its last split's merge. The choice is
  // made once, outside the loop, so each loop keeps its own load schedule.
  // LOAD: the unit's weights are requested here (otherwise before the loop).
  auto unit = [&](int u, auto rec, auto load, int active) {
    if constexpr (decltype(rec)::value) {
      // records first: vector memory operations complete in order
      constexpr int kXP = kRecPieces<UT>;
      const uint4* xsrc = reinterpret_cast<const uint4*>(a.xr + (size_t)u * UT * kTB * kXW) + lane;
      const uint4 x0 = xsrc[0];
      const uint4 x1 = kXP > 1 ? xsrc[kWave] : x0;
      const uint4 x2 = kXP > 2 ? xsrc[2 * kWave] : x0;
      const uint4 x3 = kXP > 3 ? xsrc[3 * kWave] : x0;
      if constexpr (decltype(load)::value) load_round<QT, NMAT, UT>(rd, a, g, ntk, u, lane);
      uint4* xd = reinterpret_cast<uint4*>(xw) + lane;
      xd[0] = x0;
      if constexpr (kXP > 1) xd[kWave] = x1;
      if constexpr (kXP > 2) xd[2 * kWave] = x2;
      if constexpr (kXP > 3) xd[3 * kWave] = x3;
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // other lanes' pieces are written
      if (a.nw && lane < UT * kTB * 2) ssq += __int_as_float(xw[lane * kRW + 14]);
    } else if constexpr (MERGE != kMergeNone) {
      MSlice<UT> mp;
      mfetch<UT>(mp, a, u, active, lane);
      if constexpr (decltype(load)::value) load_round<QT, NMAT, UT>(rd, a, g, ntk, u, lane);
      mput<UT>(mp, xw, u, nb, active, lane);
    } else {
      XSlice<UT> xp;
      xfetch<UT>(xp, a.x, a.nw, u, nb, lane);
      if constexpr (decltype(load)::value) load_round<QT, NMAT, UT>(rd, a, g, ntk, u, lane);
      ssq += xput<UT>(xp, xw, a.nw, u, nb, lane);
    }
    if constexpr (is_float(QT)) rec_to_float<UT>(xw, lane);
    // the slice is written and read by this wave only: LDS operations of a
    // wave complete in order, the fence keeps the compiler from reordering
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    fma_round<QT, NMAT, UT>(acc, rd, xw, kb, reinterpret_cast<const int*>(zpad[wave]), lane);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  // PRE: the first unit's weights were requested before the loop (the first
  // unit is peeled, so no branch sits around a load)
  auto rounds = [&](auto rec, auto pre, int active) {
    int u0 = wave;
    if constexpr (decltype(pre)::value) {
      unit(wave, rec, std::false_type{}, active);
      u0 += S;
    }
    for (int u = u0; u < nu; u += S) unit(u, rec, std::true_type{}, active);
  };
  // Every unit of the wave in flight at once: unit wave + i*S in round i
  // (rounds past the row reload the last unit, branch-free, and are not
  // used); each is used once its own loads have landed (the compiler waits
  // for them by register while the later units' are still in flight).
  auto rounds_all = [&]() {
    // one named variable per round (no array the compiler could keep in
    // scratch memory); rounds past NR are never touched
    Round<QT, NMAT, UT> r0, r1, r2, r3;
    XRec<UT> x0, x1, x2, x3;
    for_each_index<NR>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      auto& r = pick<i>(r0, r1, r2, r3);
      auto& x = pick<i>(x0, x1, x2, x3);
      const int u = min(wave + i * S, nu - 1);
      rload<UT>(x, a.xr, u, lane);
      load_round<QT, NMAT, UT>(r, a, g, ntk, u, lane);
    });
    __builtin_amdgcn_sched_barrier(0);
    for_each_index<NR>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if (wave + i * S < nu) {   // wave-uniform
        // a marker per round keeps the compiler from merging the rounds' uses
        // into one block that picks its registers at run time (through memory)
        asm volatile("; round %0" ::"n"(i));
        rput<UT>(xw, pick<i>(x0, x1, x2, x3), lane);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (a.nw && lane < UT * kTB * 2) ssq += __int_as_float(xw[lane * kRW + 14]);
        fma_round<QT, NMAT, UT>(acc, pick<i>(r0, r1, r2, r3), xw, kb, reinterpret_cast<const int*>(zpad[wave]), lane);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      }
    });
  };
  if constexpr (NR > 0) {
    rounds_all();
  } else if constexpr (PX) {
    rounds(std::true_type{}, std::false_type{}, 0);
  } else if constexpr (MERGE == kMergeEarly) {
    // At most kMergeSplits splits launched: past one active split, Wo
    // merges them. The first unit's split partials (every launched split:
    // the position is not read yet) and weights are requested before the
    // position, which picks the x path and the active splits; the partials
    // come first, so the merge does not wait for the weights. wave < S <= nu:
    // every wave has a first unit.
    MSlice<UT> mp0;
    mfetch<UT>(mp0, a, wave, min(a.att_ns, kMergeSplits), lane);
    load_round<QT, NMAT, UT>(rd, a, g, ntk, wave, lane);
    const int active = merge_active(a);
    if (a.xr && (active == 1 || active > kMergeSplits)) {
      // the partials are not needed here; this use keeps the compiler from
      // moving their loads into the other branch, behind the position
#pragma unroll
      for (int j = 0; j < UT / 2; ++j) {
        asm volatile("" ::"v"(mp0.ml[j].x), "v"(mp0.ml[j].y));
#pragma unroll
        for (int s = 0; s < kMergeSplits; ++s) {
          const float4 o = mp0.o[j][s];
          asm volatile("" ::"v"(o.x), "v"(o.y), "v"(o.z), "v"(o.w));
        }
      }
      rounds(std::true_type{}, std::true_type{}, active);
    } else {
      mput<UT>(mp0, xw, wave, nb, active, lane);
      if constexpr (is_float(QT)) rec_to_float<UT>(xw, lane);
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      fma_round<QT, NMAT, UT>(acc, rd, xw, kb, reinterpret_cast<const int*>(zpad[wave]), lane);
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      for (int u = wave + S; u < nu; u += S) unit(u, std::false_type{}, std::true_type{}, active);
    }
  } else if constexpr (MERGE == kMergeLate) {
    // More splits launched (long contexts): past kMergeSplits active ones
    // the attention's last split merges them into records, so the position
    // is read first (requesting the partials before it would read them for
    // nothing there).
    const int active = merge_active(a);
    if (a.xr && (active == 1 || active > kMergeSplits))
      rounds(std::true_type{}, std::false_type{}, active);
    else
      rounds(std::false_type{}, std::false_type{}, active);
  } else {
    rounds(std::false_type{}, std::false_type{}, 0);
  }

  // lanes r, r+16, r+32, r+48 hold row r's four block columns
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    acc[m] += __shfl_xor(acc[m], 16, kWave);
    acc[m] += __shfl_xor(acc[m], 32, kWave);
    if (lane < kRG) red[(m * kRG + lane) * kMaxS + wave] = acc[m];
  }
  if (a.nw) {
    const float w = wave_sum(ssq);
    if (lane == 0) red[NMAT * kRG * kMaxS + wave] = w;
  }
  __syncthreads();
  if (wave != 0) return;
  const int r = lane % kRG;
  // every wave's partials requested at once, 16 bytes per read (slots past
  // S hold no partial and are not added), then added in wave order
  float v[NMAT];
  float4 pw[NMAT][kMaxS / 4], pn[kMaxS / 4];
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int i = 0; i < kMaxS / 4; ++i) pw[m][i] = reinterpret_cast<const float4*>(red + (m * kRG + r) * kMaxS)[i];
#pragma unroll
  for (int i = 0; i < kMaxS / 4; ++i) pn[i] = reinterpret_cast<const float4*>(red + NMAT * kRG * kMaxS)[i];
  auto part = [](const float4& q, int k) { return k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w; };
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kMaxS; ++w)
      if (w < S) s += part(pw[m][w / 4], w % 4);
    v[m] = s;
  }
  // RMSNorm scale of tensor.c:114-131: 1 / sqrt(mean(x^2) + eps), or exactly
  // 1 without a norm weight (its slots then hold no sums); branch-free, so
  // the norm partials are requested with the row partials
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kMaxS; ++w)
    if (w < S) t += part(pn[w / 4], w % 4);
  const float scale = a.nw ? 1.0f / sqrtf(t / (float)a.cols + a.eps) : 1.0f;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) v[m] *= scale;
  epilogue<EPI, NMAT>(a, g * kRG + r, lane < kRG, v, pre);
}

// GGUF blocks -> tiled planes. Source block i of a [rows x nb] tensor whose
// rows start at row_off of the packed matrix.
template <int QT>
__global__ void k_pack(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs,
                       uint16_t* __restrict__ ds, int64_t nblocks, int nb, int64_t row_off) {
  constexpr int kQB = QTraits<QT>::kQB, kBytes = QTraits<QT>::kGgufBytes;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  const int64_t row = row_off + i / nb;
  const int b = (int)(i % nb);
  const int ntk = (nb + kTB - 1) / kTB, g = (int)(row / kRG), l = tile_lane((int)(row % kRG), b);
  const size_t o = tile_idx(g, ntk, b / kTB, l);
  const uint8_t* s = src + i * kBytes;
  ds[scale_idx(g, ntk, b / kTB, l)] = (uint16_t)(s[0] | (s[1] << 8));
  uint4* dst = reinterpret_cast<uint4*>(qs + o * kQB);
#pragma unroll
  for (int v = 0; v < kQB / 16; ++v) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint8_t* p = s + 2 + v * 16 + k * 4;
      w[k] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    dst[v] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// GGUF Q4_K super-blocks -> tiled planes: thread i takes sub-block i % nb of
// row row_off + i / nb (nb = cols / 32 sub-blocks per row): its 6-bit scale
// and min (get_scale_min_k4, quantize.c:267-275) into the scale plane, its
// 32 nibbles (low or high nibbles of 32 bytes, quantize.c:296-305) in Q4_0
// order into the code plane, and with sub-block 0 of a super-block the
// super-block's (d, dmin) into the third plane.
__global__ void k_pack_q4k(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs, uint16_t* __restrict__ ds,
                           uint32_t* __restrict__ su, int64_t nsub, int nb, int64_t row_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nsub) return;
  const int64_t r = i / nb;
  const int b = (int)(i % nb), k = b % 8, nsb = nb / 8;
  const int64_t row = row_off + r;
  const uint8_t* sb = src + (r * nsb + b / 8) * 144;
  const uint8_t* sc = sb + 4;
  uint32_t s6, m6;
  if (k < 4) {
    s6 = sc[k] & 63u;
    m6 = sc[k + 4] & 63u;
  } else {
    s6 = (sc[k + 4] & 0xFu) | ((uint32_t)(sc[k - 4] >> 6) << 4);
    m6 = (sc[k + 4] >> 4) | ((uint32_t)(sc[k] >> 6) << 4);
  }
  const uint8_t* q = sb + 16 + 32 * (k / 2);
  const int sh = 4 * (k % 2);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t lo = (q[j] >> sh) & 0xFu, hi = (q[j + 16] >> sh) & 0xFu;
    w[j / 4] |= (lo | (hi << 4)) << (8 * (j % 4));
  }
  const int ntk = (nb + kTB - 1) / kTB, g = (int)(row / kRG), l = tile_lane((int)(row % kRG), b);
  *reinterpret_cast<uint4*>(qs + tile_idx(g, ntk, b / kTB, l) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  ds[scale_idx(g, ntk, b / kTB, l)] = (uint16_t)(s6 | (m6 << 8));
  if (k == 0)
    su[((size_t)g * nsb + b / 8) * kRG + row % kRG] =
        (uint32_t)(sb[0] | (sb[1] << 8)) | ((uint32_t)(sb[2] | (sb[3] << 8)) << 16);
}

// GGUF Q2_K / Q3_K / Q5_K / Q6_K super-blocks -> tiled planes: thread i
// takes 32-weight block b = i % nb (k = b % 8 within its super-block, weights
// 128h + 32j + l with h = k / 4, j = k % 4) of row row_off + i / nb. Its 32
// codes go to the code plane (nibbles in Q4_0 order for Q2_K and Q3_K, the
// latter + 4; int8 for Q5_K and Q6_K, the latter - 32), its scale entry (see
// kq_affine) to the scale plane and, with block 0, the super-block's d and
// dmin to the third plane. Field offsets: quantize.h:61-99.
template <int QT>
__global__ void k_pack_kq(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs, uint16_t* __restrict__ ds,
                          uint32_t* __restrict__ su, int64_t nblk, int nb, int64_t row_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblk) return;
  constexpr int kBytes = QTraits<QT>::kGgufBytes;
  const int64_t r = i / nb;
  const int b = (int)(i % nb), k = b % 8, nsb = nb / 8, h = k / 4, j = k % 4;
  const int64_t row = row_off + r;
  const uint8_t* sb = src + (r * nsb + b / 8) * kBytes;
  int c[32];
  uint32_t e, d, dm = 0;
  if constexpr (QT == kQ2K) {   // quantize.c:180-215
#pragma unroll
    for (int l = 0; l < 32; ++l) c[l] = (sb[16 + 32 * h + l] >> (2 * j)) & 3;
    e = sb[8 * h + 2 * j] | ((uint32_t)sb[8 * h + 2 * j + 1] << 8);
    d = sb[80] | ((uint32_t)sb[81] << 8);
    dm = sb[82] | ((uint32_t)sb[83] << 8);
  } else if constexpr (QT == kQ3K) {   // :219-263, the code + 4 (0..7)
#pragma unroll
    for (int l = 0; l < 32; ++l)
      c[l] = ((sb[32 + 32 * h + l] >> (2 * j)) & 3) | (((sb[l] >> (4 * h + j)) & 1) << 2);
    uint32_t sv[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int si = 8 * h + 2 * j + g;
      const uint32_t low = si < 8 ? sb[96 + si] & 15u : sb[96 + si - 8] >> 4;
      sv[g] = low | (((uint32_t)(sb[104 + si % 4] >> (2 * (si / 4))) & 3u) << 4);
    }
    e = sv[0] | (sv[1] << 8);
    d = sb[108] | ((uint32_t)sb[109] << 8);
  } else if constexpr (QT == kQ5K) {   // :312-346
    const uint8_t* sc = sb + 4;
    uint32_t s6, m6;
    if (k < 4) {
      s6 = sc[k] & 63u;
      m6 = sc[k + 4] & 63u;
    } else {
      s6 = (sc[k + 4] & 0xFu) | ((uint32_t)(sc[k - 4] >> 6) << 4);
      m6 = (sc[k + 4] >> 4) | ((uint32_t)(sc[k] >> 6) << 4);
    }
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const uint32_t byte = sb[48 + 32 * (k / 2) + l];
      c[l] = (int)(k % 2 ? byte >> 4 : byte & 15u) + 16 * ((sb[16 + l] >> k) & 1);
    }
    e = s6 | (m6 << 8);
    d = sb[0] | ((uint32_t)sb[1] << 8);
    dm = sb[2] | ((uint32_t)sb[3] << 8);
  } else {   // Q6_K, :350-383
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const uint32_t lb = sb[64 * h + 32 * (j & 1) + l];
      const uint32_t lo = j < 2 ? lb & 15u : lb >> 4;
      c[l] = (int)(lo | (((sb[128 + 32 * h + l] >> (2 * j)) & 3u) << 4)) - 32;
    }
    e = sb[192 + 8 * h + 2 * j] | ((uint32_t)sb[192 + 8 * h + 2 * j + 1] << 8);
    d = sb[208] | ((uint32_t)sb[209] << 8);
  }
  const int ntk = (nb + kTB - 1) / kTB, g = (int)(row / kRG), tl = tile_lane((int)(row % kRG), b);
  uint8_t* dst = qs + tile_idx(g, ntk, b / kTB, tl) * QTraits<QT>::kQB;
  if constexpr (QTraits<QT>::kQB == 16) {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int m = 0; m < 16; ++m) w[m / 4] |= ((uint32_t)(c[m] & 15) | ((uint32_t)(c[m + 16] & 15) << 4)) << (8 * (m % 4));
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int m = 0; m < 32; ++m) w[m / 4] |= ((uint32_t)c[m] & 0xffu) << (8 * (m % 4));
    reinterpret_cast<uint4*>(dst)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint4*>(dst)[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
  ds[scale_idx(g, ntk, b / kTB, tl)] = (uint16_t)e;
  if (k == 0) su[((size_t)g * nsb + b / 8) * kRG + row % kRG] = d | (dm << 16);
}

// GGUF Q4_1 / Q5_0 / Q5_1 / Q8_1 blocks (quantize.h:20-53) and F16 / F32
// rows -> tiled planes; thread i takes 32-weight block b = i % nb of row
// row_off + i / nb. Q4_1: its 16 nibble bytes as they are (Q4_0 order) and
// d | m << 16. Q5_0 (into the Q8_0 format): int8 codes q - 16 in weight order
// (q = nibble | bit j of qh << 4; weight j < 16 the low nibble of byte j,
// weight j + 16 the high one, quantize.c:93-112) and d. Q5_1: int8 codes q
// (0..31) and d | m << 16. Q8_1: its 32 int8 codes and the fp32 bits of d.
// F16 / F32: the block's 32 weights.
template <int QT>
__global__ void k_pack_more(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs, uint16_t* __restrict__ ds,
                            int64_t nblocks, int nb, int64_t row_off) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  constexpr int kBytes = QTraits<QT>::kGgufBytes;
  constexpr int DT = dev_type(QT);
  constexpr int kQB = code_bytes_of(DT);
  const int64_t row = row_off + i / nb;
  const int b = (int)(i % nb);
  const int ntk = (nb + kTB - 1) / kTB, g = (int)(row / kRG), l = tile_lane((int)(row % kRG), b);
  const uint8_t* sb = src + i * kBytes;
  uint8_t* dst = qs + tile_idx(g, ntk, b / kTB, l) * kQB;
  auto u16 = [&](int o) { return (uint32_t)sb[o] | ((uint32_t)sb[o + 1] << 8); };
  auto u32 = [&](int o) { return u16(o) | (u16(o + 2) << 16); };
  if constexpr (is_float(QT)) {
#pragma unroll
    for (int v = 0; v < kQB / 16; ++v)
      reinterpret_cast<uint4*>(dst)[v] = make_uint4(u32(16 * v), u32(16 * v + 4), u32(16 * v + 8), u32(16 * v + 12));
    return;
  } else {
    uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if constexpr (QT == kQ4_1) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = u32(4 + 4 * k);
      reinterpret_cast<uint32_t*>(ds)[scale_idx(g, ntk, b / kTB, l)] = u16(0) | (u16(2) << 16);
    } else if constexpr (QT == kQ8_1) {
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = u32(8 + 4 * k);
      reinterpret_cast<uint32_t*>(ds)[scale_idx(g, ntk, b / kTB, l)] = u32(0);
    } else {   // Q5_0, Q5_1
      constexpr bool one = QT == kQ5_1;
      const uint32_t qh = u32(one ? 4 : 2);
      const uint8_t* q = sb + (one ? 8 : 6);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const uint32_t nib = j < 16 ? q[j] & 15u : q[j - 16] >> 4;
        const int c = (int)(nib | (((qh >> j) & 1u) << 4)) - (one ? 0 : 16);
        w[j / 4] |= ((uint32_t)c & 0xffu) << (8 * (j % 4));
      }
      if constexpr (one)
        reinterpret_cast<uint32_t*>(ds)[scale_idx(g, ntk, b / kTB, l)] = u16(0) | (u16(2) << 16);
      else
        ds[scale_idx(g, ntk, b / kTB, l)] = (uint16_t)u16(0);
    }
    reinterpret_cast<uint4*>(dst)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    if constexpr (kQB == 32) reinterpret_cast<uint4*>(dst)[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

// Row `token` of a packed table, dequantised exactly as quantize.c:60-72 /
// 139-149 (one fp32 multiply per weight). With tokens set, workgroup row z
// writes row tokens[*dpos + z] to out + z * cols (a prompt's rows at once).
// With xr set (one row), the row is also written as x records of
// row * nw (the first layer's attn_norm) for the first matvec.
template <int QT>
__device__ __forceinline__ float embed_value(const PackedMat& t, int tok, int ntk, int j) {
  constexpr int kQB = QTraits<QT>::kQB;
  const int b = j >> 5, p = j & 31;
  const int l = tile_lane(tok % kRG, b);
  const uint8_t* q = t.qs + tile_idx(tok / kRG, ntk, b / kTB, l) * kQB;
  if constexpr (QT == kF16) {   // quantize.c:167-172
    return h2f(reinterpret_cast<const uint16_t*>(q)[p]);
  } else if constexpr (QT == kF32) {
    return reinterpret_cast<const float*>(q)[p];
  } else if constexpr (is_wide(QT)) {
    const uint32_t e = reinterpret_cast<const uint32_t*>(t.ds)[scale_idx(tok / kRG, ntk, b / kTB, l)];
    const float d = h2f((uint16_t)(e & 0xffffu)), m = h2f((uint16_t)(e >> 16));
    if constexpr (QT == kQ4_1) {   // quantize.c:76-91: d * q + m
      const uint8_t v = q[p & 15];
      return __fadd_rn(__fmul_rn(d, (float)(p < 16 ? v & 0xF : v >> 4)), m);
    } else if constexpr (QT == kQ5_1) {   // :114-137: q * d + m
      return __fadd_rn(__fmul_rn((float)q[p], d), m);
    } else {   // Q8_1, :153-163: fp32 d * q
      return __fmul_rn(__uint_as_float(e), (float)(int8_t)q[p]);
    }
  } else if constexpr (QT == 2) {
    const float d = h2f(t.ds[scale_idx(tok / kRG, ntk, b / kTB, l)]);
    const uint8_t v = q[p & 15];
    return d * (float)((int)(p < 16 ? v & 0xF : v >> 4) - 8);
  } else if constexpr (QT == kQ4K) {
    // quantize.c:287-305: d1 = d * scale, m1 = dmin * min, weight d1 * q - m1
    // with both fp32 roundings kept apart (no fused multiply-add)
    const uint8_t v = q[p & 15];
    const uint32_t e = t.ds[scale_idx(tok / kRG, ntk, b / kTB, l)];
    const uint32_t sup = t.su[((size_t)(tok / kRG) * (ntk / 2) + b / 8) * kRG + tok % kRG];
    const float d1 = h2f((uint16_t)(sup & 0xffffu)) * (float)(e & 0xffu);
    const float m1 = h2f((uint16_t)(sup >> 16)) * (float)(e >> 8);
    return __fsub_rn(__fmul_rn(d1, (float)(p < 16 ? v & 0xF : v >> 4)), m1);
  } else if constexpr (is_kq(QT)) {
    // the reference's per-weight expressions (quantize.c:180-383), each
    // product and difference rounded once
    const uint32_t e = t.ds[scale_idx(tok / kRG, ntk, b / kTB, l)];
    const uint32_t sup = t.su[((size_t)(tok / kRG) * (ntk / 2) + b / 8) * kRG + tok % kRG];
    const float dd = h2f((uint16_t)(sup & 0xffffu)), dm = h2f((uint16_t)(sup >> 16));
    const uint32_t sg = (e >> (8 * (p / 16))) & 0xffu;   // the group's scale byte
    if constexpr (QT == kQ2K || QT == kQ3K) {
      const uint8_t v = q[p & 15];
      const int nib = p < 16 ? v & 0xF : v >> 4;
      if constexpr (QT == kQ2K)
        return __fsub_rn(__fmul_rn(__fmul_rn(dd, (float)(sg & 15u)), (float)nib), __fmul_rn(dm, (float)(sg >> 4)));
      else
        return __fmul_rn(__fmul_rn(dd, (float)((int)sg - 32)), (float)(nib - 4));
    } else if constexpr (QT == kQ5K) {
      return __fsub_rn(__fmul_rn(__fmul_rn(dd, (float)(e & 0xffu)), (float)(int8_t)q[p]),
                       __fmul_rn(dm, (float)(e >> 8)));
    } else {
      return __fmul_rn(__fmul_rn(dd, (float)(int8_t)sg), (float)(int8_t)q[p]);
    }
  } else {   // Q8_0, and Q5_0 in the Q8_0 format: (q - 16) * d, quantize.c:93-112
    return h2f(t.ds[scale_idx(tok / kRG, ntk, b / kTB, l)]) * (float)(int8_t)q[p];
  }
}

// Grid (ceil(cols / 256), rows): thread j of a row writes value j; with xr,
// lane r of each 16-lane row holds value 16 * record + r, so the records are
// encoded in the same pass (every lane of a wave takes part in enc16).
template <int QT>
__global__ void __launch_bounds__(256) k_embed(PackedMat t, int cols, const int* tokens, const int* dpos,
                                               int token, float* out, const float* nw, uint32_t* xr,
                                               float scale) {
  const int tok = tokens ? tokens[*dpos + blockIdx.y] : token;
  out += (size_t)blockIdx.y * cols;
  const int ntk = (cols / 32 + kTB - 1) / kTB;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in = j < cols;
  // the dequantised value, then (Gemma) times sqrt(d): two roundings, as
  // layer_scheduler.c:584-602 (scale 1 is exact)
  const float v = in ? __fmul_rn(embed_value<QT>(t, tok, ntk, j), scale) : 0.f;
  if (in) out[j] = v;
  if (!xr) return;
  const Enc e = enc16(in ? v * nw[j] : 0.f, v);
  if (in) put_rec_lds(xr + (size_t)(j >> 4) * kRW, e, j & 15);
}

// Picks the first maximum among per-workgroup candidates, writes it, and for
// device-side greedy decoding appends it at tokens[pos+1] and advances pos.
// One workgroup of kArgmaxThreads; each thread requests up to kArgmaxBatch
// candidates at once (clamped addresses, the ones past n not compared) before
// comparing any, so a 128256-row head's 8016 candidates cost one round trip
// instead of a chain of dependent loads. `beats` is a total order on the
// non-NaN (value, index) pairs and NaN never wins, so the result does not
// depend on the order of the comparisons.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxBatch = 8;

__global__ void __launch_bounds__(kArgmaxThreads) k_argmax_merge(const float2* part, int n, const float* y,
                                                                 int* out_idx, int* tokens, int* dpos) {
  __shared__ float2 wb[kArgmaxThreads / kWave];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i0 = threadIdx.x; i0 < n; i0 += kArgmaxThreads * kArgmaxBatch) {
    float2 p[kArgmaxBatch];
#pragma unroll
    for (int k = 0; k < kArgmaxBatch; ++k) p[k] = part[min(i0 + k * kArgmaxThreads, n - 1)];
#pragma unroll
    for (int k = 0; k < kArgmaxBatch; ++k) {
      const int pi = __float_as_int(p[k].y);
      if (i0 + k * kArgmaxThreads < n && beats(p[k].x, pi, bv, bi)) {
        bv = p[k].x;
        bi = pi;
      }
    }
  }
  wave_best(bv, bi);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < kArgmaxThreads / kWave; ++w)
    if (beats(wb[w].x, __float_as_int(wb[w].y), bv, bi)) {
      bv = wb[w].x;
      bi = __float_as_int(wb[w].y);
    }
  if (bi == 0x7fffffff || isnan(y[0])) bi = 0;   // all NaN, or x[0] NaN (tensor.c:319-320)
  *out_idx = bi;
  if (tokens) {
    const int pos = *dpos;
    tokens[pos + 1] = bi;
    *dpos = pos + 1;
  }
}

template <int QT, int NMAT, int EPI, int MERGE, bool PX, int UT, int NR>
hipError_t launch_k(const GemvArgs& a, const GemvPlan& p, hipStream_t s) {
  KernelEvents& ev = kernel_events();
  if (ev.start) {
    hipExtLaunchKernelGGL((k_gemv<QT, NMAT, EPI, UT, MERGE, PX, NR>), dim3(p.grid), dim3(p.threads),
                          p.lds_bytes, s, ev.start, ev.stop, 0, a);
    ev.used = true;
  } else {
    hipLaunchKernelGGL((k_gemv<QT, NMAT, EPI, UT, MERGE, PX, NR>), dim3(p.grid), dim3(p.threads),
                       p.lds_bytes, s, a);
  }
  return hipGetLastError();
}

// Records path of Q4_0 / Q8_0 matrices with two-tile units whose rows take
// 2 to 4 units per wave: every unit of a wave requested at once (NR rounds;
// four-tile units would keep their records in scratch memory).
template <int QT, int NMAT, int EPI, int MERGE = kMergeNone, bool PX = false, int UT = kGemvUnit>
hipError_t launch_t(const GemvArgs& a, hipStream_t s) {
  const GemvPlan p = gemv_plan(a.rows, a.cols, QT, NMAT, UT);
  if constexpr (PX && MERGE == kMergeNone && (QT == 2 || QT == 8) && UT == 2) {   // four-tile units keep their records in scratch
    const int ntk = (a.cols / 32 + kTB - 1) / kTB;
    const int S = p.threads / kWave, nr = ((ntk + UT - 1) / UT + S - 1) / S;
    // more rounds per wave (up to 7 for the 8B down projection, fewer and
    // fatter waves) measured slower than the loop over units
    const int cap = 4;
    if (nr <= cap) {
      switch (nr) {
        case 2: return launch_k<QT, NMAT, EPI, MERGE, PX, UT, 2>(a, p, s);
        case 3: return launch_k<QT, NMAT, EPI, MERGE, PX, UT, 3>(a, p, s);
        case 4: return launch_k<QT, NMAT, EPI, MERGE, PX, UT, 4>(a, p, s);
        default: break;
      }
    }
  }
  return launch_k<QT, NMAT, EPI, MERGE, PX, UT, 0>(a, p, s);
}

// x read from the producer's records (a.xr) or staged from a.x by the matvec
template <int QT, int NMAT, int EPI>
hipError_t launch_x(const GemvArgs& a, hipStream_t s) {
  return a.xr ? launch_t<QT, NMAT, EPI, false, true>(a, s) : launch_t<QT, NMAT, EPI>(a, s);
}

// [Wq;Wk;Wv] from records: four-tile units (8-wave workgroups) when there are
// at least kQkvWideGroups row groups (7B shape: 7.8 against 8.6 us per launch
// with two-tile units; the other matrices measured fastest with two)
constexpr int kQkvWideGroups = 512;
template <int QT>
hipError_t launch_qkv(const GemvArgs& a, hipStream_t s) {
  if (QT == 2 && a.xr && (a.rows + kRG - 1) / kRG >= kQkvWideGroups)
    return launch_t<QT, 1, EPI_QKV, false, true, 4>(a, s);
  return launch_x<QT, 1, EPI_QKV>(a, s);
}

template <int QT>
hipError_t launch_q(int epi, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE:
      if (!a.att_o) return launch_x<QT, 1, EPI_STORE>(a, s);
      return a.att_ns <= kMergeSplits ? launch_t<QT, 1, EPI_STORE, kMergeEarly>(a, s)
                                      : launch_t<QT, 1, EPI_STORE, kMergeLate>(a, s);
    case EPI_ADD:
      if (!a.att_o) return launch_x<QT, 1, EPI_ADD>(a, s);
      return a.att_ns <= kMergeSplits ? launch_t<QT, 1, EPI_ADD, kMergeEarly>(a, s)
                                      : launch_t<QT, 1, EPI_ADD, kMergeLate>(a, s);
    case EPI_SWIGLU: return launch_x<QT, 2, EPI_SWIGLU>(a, s);
    case EPI_QKV: return launch_qkv<QT>(a, s);
    case EPI_LOGITS: return launch_x<QT, 1, EPI_LOGITS>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

KernelEvents& kernel_events() {
  static thread_local KernelEvents ev;
  return ev;
}

// One workgroup per 16-row group; one wave per unit of kGemvUnit tiles of the
// row, up to 16 (Q4_0, one matrix) or 8 waves; rows wider than that take
// several rounds per wave. Two-tile units measured fastest for every 7B shape
// (fewest registers, most waves resident, shortest work after the last load).
GemvPlan gemv_plan(int rows, int cols, int type, int nmat, int unit) {
  GemvPlan p;
  const int groups = (rows + kRG - 1) / kRG;
  const int ntk = (cols / 32 + kTB - 1) / kTB;
  const int smax = dev_type(type) == 2 && nmat == 1 ? gemv_max_waves<2, 1>() : gemv_max_waves<8, 1>();
  const int ut = unit;
  const int nu = (ntk + ut - 1) / ut;
  const int S = nu < smax ? nu : smax;
  p.unit = ut;
  p.grid = groups;
  p.threads = S * kWave;
  // the x slices, then the wave partials padded to smax waves per row
  p.lds_bytes = (size_t)S * ut * kTB * kXW * sizeof(int) + (size_t)(nmat * kRG * smax + smax) * sizeof(float);
  return p;
}

// code and scale bytes of a packed [rows x cols] matrix
// code, scale and (Q4_K) super-block plane bytes of a packed [rows x cols]
// matrix; the scale plane starts at a 256-byte boundary, and so does the
// super-block plane
static void packed_sizes(int type, int64_t rows, int cols, size_t* code, size_t* scales, size_t* sup) {
  type = dev_type(type);
  const size_t groups = (size_t)((rows + kRG - 1) / kRG);
  const int ntk = (cols / 32 + kTB - 1) / kTB;
  const int nu = (ntk + kUT - 1) / kUT;
  const int kqb = code_bytes_of(type);
  *code = ((groups * ntk * kWave * kqb) + 255) & ~(size_t)255;
  // 16-bit entries, 32-bit for Q4_1 / Q5_1 / Q8_1, none for F16 / F32
  *scales = is_float(type) ? 0 : groups * nu * kWave * kUT * (is_wide(type) ? 4 : 2);
  *sup = 0;
  if (is_kq(type)) {
    *scales = (*scales + 255) & ~(size_t)255;
    *sup = groups * (size_t)(cols / 256) * kRG * 4;
  }
}

size_t packed_bytes(int type, int64_t rows, int cols) {
  size_t c, sc, su;
  packed_sizes(type, rows, cols, &c, &sc, &su);
  return c + sc + su;
}

PackedMat packed_view(const void* base, int type, int64_t rows, int cols) {
  size_t c, sc, su;
  packed_sizes(type, rows, cols, &c, &sc, &su);
  PackedMat m;
  m.qs = static_cast<const uint8_t*>(base);
  m.ds = reinterpret_cast<const uint16_t*>(m.qs + c);
  m.su = su ? reinterpret_cast<const uint32_t*>(m.qs + c + sc) : nullptr;
  return m;
}

hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t s) {
  if (a.xr_out && epi != EPI_STORE && epi != EPI_ADD && epi != EPI_SWIGLU) return hipErrorInvalidValue;
  // merge staging: more than kMergeSplits splits only with the records of
  // the attention's own merge (xr) to fall back on; power-of-two head_dim
  // and group
  if (a.att_o && ((epi != EPI_ADD && epi != EPI_STORE) || !a.att_ml || !a.dpos || a.att_ns < 1 ||
                  (a.att_ns > kMergeSplits && !a.xr) || a.att_group < 1 || (a.att_group & (a.att_group - 1)) ||
                  a.head_dim < 32 || (a.head_dim & (a.head_dim - 1)) || a.cols % a.head_dim))
    return hipErrorInvalidValue;
  switch (dev_type(a.type)) {
    case 2: return launch_q<2>(epi, a, s);
    case 8: return launch_q<8>(epi, a, s);
    case kQ4K: return launch_q<kQ4K>(epi, a, s);
    case kQ2K: return launch_q<kQ2K>(epi, a, s);
    case kQ3K: return launch_q<kQ3K>(epi, a, s);
    case kQ5K: return launch_q<kQ5K>(epi, a, s);
    case kQ6K: return launch_q<kQ6K>(epi, a, s);
    case kQ4_1: return launch_q<kQ4_1>(epi, a, s);
    case kQ5_1: return launch_q<kQ5_1>(epi, a, s);
    case kQ8_1: return launch_q<kQ8_1>(epi, a, s);
    case kF16: return launch_q<kF16>(epi, a, s);
    case kF32: return launch_q<kF32>(epi, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_argmax_merge(const float2* part, int n, const float* y, int* out_idx, int* tokens,
                               int* dpos, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_merge, dim3(1), dim3(kArgmaxThreads), 0, s, part, n, y, out_idx, tokens, dpos);
  return hipGetLastError();
}

hipError_t launch_pack(int type, const uint8_t* src, PackedMat dst, int64_t nblocks, int nb, int64_t row_off,
                       hipStream_t s) {
  const int64_t grid = (nblocks + 255) / 256;
  uint8_t* qs = const_cast<uint8_t*>(dst.qs);
  uint16_t* ds = const_cast<uint16_t*>(dst.ds);
  if (type == 2)
    hipLaunchKernelGGL(k_pack<2>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == 8)
    hipLaunchKernelGGL(k_pack<8>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kQ4K && dst.su && nb % 8 == 0)
    hipLaunchKernelGGL(k_pack_q4k, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, const_cast<uint32_t*>(dst.su),
                       nblocks, nb, row_off);
  else if (type == kQ2K && dst.su && nb % 8 == 0)
    hipLaunchKernelGGL(k_pack_kq<kQ2K>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds,
                       const_cast<uint32_t*>(dst.su), nblocks, nb, row_off);
  else if (type == kQ3K && dst.su && nb % 8 == 0)
    hipLaunchKernelGGL(k_pack_kq<kQ3K>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds,
                       const_cast<uint32_t*>(dst.su), nblocks, nb, row_off);
  else if (type == kQ5K && dst.su && nb % 8 == 0)
    hipLaunchKernelGGL(k_pack_kq<kQ5K>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds,
                       const_cast<uint32_t*>(dst.su), nblocks, nb, row_off);
  else if (type == kQ6K && dst.su && nb % 8 == 0)
    hipLaunchKernelGGL(k_pack_kq<kQ6K>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds,
                       const_cast<uint32_t*>(dst.su), nblocks, nb, row_off);
  else if (type == kQ4_1)
    hipLaunchKernelGGL(k_pack_more<kQ4_1>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kQ5_0)
    hipLaunchKernelGGL(k_pack_more<kQ5_0>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kQ5_1)
    hipLaunchKernelGGL(k_pack_more<kQ5_1>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kQ8_1)
    hipLaunchKernelGGL(k_pack_more<kQ8_1>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kF16)
    hipLaunchKernelGGL(k_pack_more<kF16>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == kF32)
    hipLaunchKernelGGL(k_pack_more<kF32>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int QT>
static hipError_t embed_t(const PackedMat& t, int cols, const int* tokens, const int* dpos, int token, float* out,
                          const float* nw, uint32_t* xr, float scale, int n, hipStream_t s) {
  hipLaunchKernelGGL(k_embed<QT>, dim3((cols + 255) / 256, n), dim3(256), 0, s, t, cols, tokens, dpos, token, out, nw,
                     xr, scale);
  return hipGetLastError();
}

static hipError_t embed_any(int type, const PackedMat& t, int cols, const int* tokens, const int* dpos, int token,
                            float* out, const float* nw, uint32_t* xr, float scale, int n, hipStream_t s) {
  switch (dev_type(type)) {
    case 2: return embed_t<2>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case 8: return embed_t<8>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ4K: return embed_t<kQ4K>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ2K: return embed_t<kQ2K>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ3K: return embed_t<kQ3K>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ5K: return embed_t<kQ5K>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ6K: return embed_t<kQ6K>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ4_1: return embed_t<kQ4_1>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ5_1: return embed_t<kQ5_1>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kQ8_1: return embed_t<kQ8_1>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kF16: return embed_t<kF16>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    case kF32: return embed_t<kF32>(t, cols, tokens, dpos, token, out, nw, xr, scale, n, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_embed(int type, PackedMat t, int cols, const int* tokens, const int* dpos,
                        int token, float* out, const float* nw, uint32_t* xr, float scale, hipStream_t s) {
  if (xr && !nw) return hipErrorInvalidValue;
  return embed_any(type, t, cols, tokens, dpos, token, out, nw, xr, scale, 1, s);
}

hipError_t launch_embed_rows(int type, PackedMat t, int cols, const int* tokens, const int* dpos, int n,
                             float* out, float scale, hipStream_t s) {
  if (n <= 0 || !tokens || !dpos) return hipErrorInvalidValue;
  return embed_any(type, t, cols, tokens, dpos, 0, out, nullptr, nullptr, scale, n, s);
}

}  // namespace ssk
