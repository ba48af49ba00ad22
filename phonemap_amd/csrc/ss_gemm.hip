// ss_gemm.hip - block-quantized matrix x token-block products on MFMA (gfx950),
// for prompts: Y[t] = W X[t] over T tokens at once (layer_scheduler.c:681-803
// evaluates a prompt layer by layer; every token of a layer multiplies the
// same matrices).
//
// v_mfma_f32_16x16x4f32: A is a 16-row x 4-column slice of the weights,
// dequantised exactly in fp32 (d * (nibble - 8), quantize.c:60-72, or d *
// code, quantize.c:139-149: an fp16 d times a small integer is exact in
// fp32), B the 4 x 16 matching slice of 16 tokens' x (times the RMSNorm weight
// when set), and the accumulator runs in fp32 over all blocks, as the
// reference's fp32 dot product does. The RMSNorm scale 1/rms of each token
// multiplies its outputs (tensor.c:114-131 applies it to x).
//
// MFMA operand layout (checked on the device): lane l supplies A[l%16][l/16]
// and B[l/16][l%16] and receives D[4*(l/16) + i][l%16], i = 0..3.
//
// The fast path (k_gemm_h, with a split-x scratch) runs the same products on
// v_mfma_f32_16x16x32_f16 for every block format (Q4_0, Q8_0, Q4_1, Q5_1,
// Q8_1, the K-quants; Q5_0 as Q8_0): the codes are exact fp16 integers, x is
// split into two fp16 parts, and each block's (or 16-weight group's) fp32
// result is scaled by its A, with B times the sum of x subtracted (see
// below): eight times the fp32 MFMA rate per product, with x kept to 2^-22.

#include <hip/hip_runtime.h>
#include <math.h>

#include <atomic>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;     // row groups of 16 per workgroup
constexpr int kGemmTiles = 4;     // 16-token tiles per wave
constexpr int kGemmTok = kGemmTiles * 16;
constexpr int kXsPad = kGemmTok + 4;   // LDS row (one column of x for 64 tokens), padded

// Sum of squares of each token's x (one workgroup per token), for the RMSNorm scale.
__global__ void __launch_bounds__(256) k_sumsq(const float* __restrict__ x, int ldx, int cols,
                                               float* __restrict__ ssq) {
  __shared__ float red[4];
  const float* xt = x + (size_t)blockIdx.x * ldx;
  float ss = 0.f;
  for (int c = threadIdx.x * 4; c < cols; c += 1024) {
    const float4 v = *reinterpret_cast<const float4*>(xt + c);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) ssq[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// This lane's eight weights of block b, row m = l%16: columns kq + 4s,
// s = 0..7, kq = l/16 (the A operands of the block's eight K=4 steps).
template <int QT>
struct WBlock {
  uint32_t w[QT == 2 ? 4 : 8];
  float d;
};
template <int QT>
__device__ __forceinline__ void load_w(WBlock<QT>& f, const PackedMat& w, int g, int ntk, int b, int lane) {
  const int tl = tile_lane(lane & 15, b);
  const uint4* p = reinterpret_cast<const uint4*>(w.qs + tile_idx(g, ntk, b / kTB, tl) * QTraits<QT>::kQB);
  const uint4 v0 = p[0];
  f.w[0] = v0.x; f.w[1] = v0.y; f.w[2] = v0.z; f.w[3] = v0.w;
  if constexpr (QT == 8) {
    const uint4 v1 = p[1];
    f.w[4] = v1.x; f.w[5] = v1.y; f.w[6] = v1.z; f.w[7] = v1.w;
  }
  f.d = h2f(w.ds[scale_idx(g, ntk, b / kTB, tl)]);
}
template <int QT>
__device__ __forceinline__ float weight(const WBlock<QT>& f, int s, int kq) {
  if constexpr (QT == 2) {   // column kq + 4s: byte kq of word s % 4, low nibble (s < 4) or high
    const int nib = (int)((f.w[s & 3] >> (8 * kq + (s >= 4 ? 4 : 0))) & 0xFu);
    return f.d * (float)(nib - 8);
  } else {                   // byte kq of word s
    return f.d * (float)(int8_t)((f.w[s] >> (8 * kq)) & 0xFFu);
  }
}

// Rows r0 .. r0+3 of token t from the products g (and u, the up projection,
// for EPI_SWIGLU): the RMSNorm scale of the token, the epilogue, the store.
template <int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, int t, int r0, const float (&g)[4],
                                              const float (&u)[4]) {
  const float scale = a.nw ? 1.0f / sqrtf(a.ssq[t] / (float)a.cols + a.eps) : 1.0f;
  float* yp = a.y + (size_t)t * a.ldy + r0;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = g[i] * scale;
    if constexpr (EPI == EPI_SWIGLU) {
      const float up = u[i] * scale;
      v[i] = up * (a.act == 1 ? gelu_tanh(x0) : silu(x0));   // layer_scheduler.c:529-547
    } else {
      v[i] = x0;
    }
  }
  if (r0 + 3 < a.rows) {
    float4 o = make_float4(v[0], v[1], v[2], v[3]);
    if constexpr (EPI == EPI_ADD) {
      const float4 p = *reinterpret_cast<const float4*>(yp);
      o.x += p.x;
      o.y += p.y;
      o.z += p.z;
      o.w += p.w;
    }
    *reinterpret_cast<float4*>(yp) = o;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (r0 + i < a.rows) yp[i] = EPI == EPI_ADD ? yp[i] + v[i] : v[i];
  }
}

template <int QT, int NMAT, int EPI>
__global__ void __launch_bounds__(kGemmWaves * 64) k_gemm(const GemmArgs a) {
  __shared__ float xs[2][32][kXsPad];   // x of the block: [column][token]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x * kGemmWaves + wave;   // row group (past the last: computes, stores nothing)
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const int gl = min(g, ngroups - 1);
  const int nb = a.cols >> 5;
  const int ntk = (nb + kTB - 1) / kTB;
  const int t0 = blockIdx.y * kGemmTok;
  const int n = lane & 15, kq = lane >> 4;

  // staging: thread -> token t0 + tid/4, columns (tid%4)*8 .. +7 of the block
  const int st = tid >> 2, sc = (tid & 3) * 8;
  const float* xrow = a.x + (size_t)min(t0 + st, a.T - 1) * a.ldx;
  float xv[8];
  auto fetch_x = [&](int b) {
    const float4 u = *reinterpret_cast<const float4*>(xrow + b * 32 + sc);
    const float4 v = *reinterpret_cast<const float4*>(xrow + b * 32 + sc + 4);
    xv[0] = u.x; xv[1] = u.y; xv[2] = u.z; xv[3] = u.w;
    xv[4] = v.x; xv[5] = v.y; xv[6] = v.z; xv[7] = v.w;
    if (a.nw) {
      const float4 p = *reinterpret_cast<const float4*>(a.nw + b * 32 + sc);
      const float4 q = *reinterpret_cast<const float4*>(a.nw + b * 32 + sc + 4);
      xv[0] *= p.x; xv[1] *= p.y; xv[2] *= p.z; xv[3] *= p.w;
      xv[4] *= q.x; xv[5] *= q.y; xv[6] *= q.z; xv[7] *= q.w;
    }
  };
  auto put_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) xs[buf][sc + j][st] = xv[j];
  };

  v4f acc[NMAT][kGemmTiles];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int tt = 0; tt < kGemmTiles; ++tt) acc[mt][tt] = v4f{0.f, 0.f, 0.f, 0.f};

  WBlock<QT> wb[NMAT];
  fetch_x(0);
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt) load_w<QT>(wb[mt], mt == 0 ? a.w : a.w2, gl, ntk, 0, lane);
  put_x(0);
  __syncthreads();
  for (int b = 0; b < nb; ++b) {
    const int buf = b & 1;
    const bool more = b + 1 < nb;
    WBlock<QT> wn[NMAT];
    if (more) {   // the next block's x and weights in flight during this block's products
      fetch_x(b + 1);
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) load_w<QT>(wn[mt], mt == 0 ? a.w : a.w2, gl, ntk, b + 1, lane);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      float bx[kGemmTiles];
#pragma unroll
      for (int tt = 0; tt < kGemmTiles; ++tt) bx[tt] = xs[buf][4 * s + kq][tt * 16 + n];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        const float av = weight<QT>(wb[mt], s, kq);
#pragma unroll
        for (int tt = 0; tt < kGemmTiles; ++tt)
          acc[mt][tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bx[tt], acc[mt][tt], 0, 0, 0);
      }
    }
    if (more) {
      put_x(buf ^ 1);
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) wb[mt] = wn[mt];
    }
    __syncthreads();
  }
  if (g >= ngroups) return;

  // epilogue: lane holds rows g*16 + 4kq + i of token t0 + 16tt + n
  const int r0 = g * kRG + 4 * kq;
#pragma unroll
  for (int tt = 0; tt < kGemmTiles; ++tt) {
    const int t = t0 + tt * 16 + n;
    if (t >= a.T) continue;
    float gv[4], uv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      gv[i] = acc[0][tt][i];
      uv[i] = acc[NMAT - 1][tt][i];
    }
    gemm_epilogue<EPI>(a, t, r0, gv, uv);
  }
}

// ---- fp16 products -----------------------------------------------------------
// Each 16x16x32 step is one 32-column block: B holds the block's codes as
// exact fp16 integers (nibble - 8, or the Q8_0 code), A the 16 tokens' x as
// two fp16 parts, and the step's fp32 result is scaled by the block's d (one
// per output row) into the accumulator. Codes come from a magic number: the
// fp16 with bits 0x6400 | u is 1024 + u for u < 1024, and subtracting 1032
// (Q4_0) or 1152 (Q8_0, u = code + 128) is exact.
//
// x of each token is scaled by a power of two s_t (its largest |x| then lies
// in [2^13, 2^14)) and split into xh = fp16(x s_t) and xl = fp16(x s_t - xh):
// xh + xl is within 2^-22 |x| of x (or 2^-25 / s_t absolute for the small
// elements), against 2^-24 for fp32 itself; 1/s_t is applied in the epilogue.
//
// Slot order: lane group kq (= lane/16) supplies slots 8kq .. 8kq+7 of the
// step. Q4_0: the 8 nibbles of 32-bit word kq of the block, two per fp16 pair
// (bits 4k and 4k+16: slot 2k and 2k+1), i.e. slot s is column
// 4kq + 2(s&1) + (s>>2) + 16((s>>1)&1). Q8_0: bytes 8kq .. 8kq+7, slot s is
// column 8kq + 4(s>>2) + 2(s&1) + ((s>>1)&1). The split x holds each block in
// slot order, so lane group kq reads 16 contiguous bytes.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kHWaves = 4;
constexpr int kHTiles = 4;                // 16-token tiles per workgroup
constexpr int kHTok = kHTiles * 16;
constexpr int kHChunks = 16;              // 16-byte chunks of one token's 128 columns

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

constexpr v8h kOnes = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};

template <int QT>
__host__ __device__ constexpr int slot_col(int s) {   // column within the block of slot s (s < 32)
  return QT == 2 ? 4 * (s >> 3) + 2 * (s & 1) + ((s >> 2) & 1) + 16 * ((s >> 1) & 1)
                 : 8 * (s >> 3) + 4 * ((s >> 2) & 1) + 2 * (s & 1) + ((s >> 1) & 1);
}

// Token blockIdx.x of x (times nw): the scale 1/s_t into xinv[t], then the
// fp16 parts in slot order (ldxs: row length, a multiple of 128; columns past
// cols are zero); with ssq set, first its sum of squares (of x alone).
// Thread i takes the 32-column blocks i, i + 256, ...: a block is 8 float4 of
// x (and of nw), all requested before any is used, so each pass over the row
// is one round trip per block a thread holds; a block's four 16-byte chunks
// of each part are then formed in registers, in slot order.
template <int QT>
__global__ void __launch_bounds__(256) k_split_x(const float* __restrict__ x, int ldx, const float* __restrict__ nw,
                                                 int cols, float* __restrict__ ssq, uint16_t* __restrict__ xh,
                                                 uint16_t* __restrict__ xl, float* __restrict__ xinv, int ldxs) {
  __shared__ float red[2][4];
  const int t = blockIdx.x;
  const float* xt = x + (size_t)t * ldx;
  const int nb = cols >> 5;   // cols is a multiple of 32: whole blocks
  // block blk: v = x, u = x * nw (x when nw is null)
  auto load_block = [&](int blk, float (&v)[32], float (&u)[32]) {
    const float4* xp = reinterpret_cast<const float4*>(xt + 32 * blk);
    float4 xv[8], wv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = xp[i];
    if (nw) {
      const float4* wp = reinterpret_cast<const float4*>(nw + 32 * blk);
#pragma unroll
      for (int i = 0; i < 8; ++i) wv[i] = wp[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[4 * i] = xv[i].x;
      v[4 * i + 1] = xv[i].y;
      v[4 * i + 2] = xv[i].z;
      v[4 * i + 3] = xv[i].w;
      if (nw) {
        u[4 * i] = xv[i].x * wv[i].x;
        u[4 * i + 1] = xv[i].y * wv[i].y;
        u[4 * i + 2] = xv[i].z * wv[i].z;
        u[4 * i + 3] = xv[i].w * wv[i].w;
      } else {
        u[4 * i] = xv[i].x;
        u[4 * i + 1] = xv[i].y;
        u[4 * i + 2] = xv[i].z;
        u[4 * i + 3] = xv[i].w;
      }
    }
  };
  float ss = 0.f, mx = 0.f;
  for (int blk = threadIdx.x; blk < nb; blk += 256) {
    float v[32], u[32];
    load_block(blk, v, u);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      ss = fmaf(v[j], v[j], ss);
      mx = fmaxf(mx, fabsf(u[j]));
    }
  }
  ss = wave_sum(ss);
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = ss;
    red[1][threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  int e = 0;
  if (mx > 0.f && mx <= 3.0e38f) frexpf(mx, &e);        // mx < 2^e
  const float sc = ldexpf(1.0f, 14 - e);                // largest |x s| in [2^13, 2^14)
  if (threadIdx.x == 0) {
    if (ssq) ssq[t] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    xinv[t] = ldexpf(1.0f, e - 14);
  }
  uint4* oh = reinterpret_cast<uint4*>(xh + (size_t)t * ldxs);
  uint4* ol = reinterpret_cast<uint4*>(xl + (size_t)t * ldxs);
  for (int blk = threadIdx.x; blk < ldxs / 32; blk += 256) {
    float u[32];
    if (blk < nb) {
      float v[32];
      load_block(blk, v, u);
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) u[j] = 0.f;   // padding columns past cols
    }
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {   // chunk 4 blk + kq: slots 8 kq .. 8 kq + 7
      uint32_t h[4], l[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v0 = u[slot_col<QT>(8 * kq + 2 * k)] * sc;
        const float v1 = u[slot_col<QT>(8 * kq + 2 * k + 1)] * sc;
        const _Float16 a = (_Float16)v0, b = (_Float16)v1;
        const _Float16 la = (_Float16)(v0 - (float)a), lb = (_Float16)(v1 - (float)b);
        h[k] = __builtin_bit_cast(uint32_t, h2{a, b});
        l[k] = __builtin_bit_cast(uint32_t, h2{la, lb});
      }
      oh[4 * blk + kq] = make_uint4(h[0], h[1], h[2], h[3]);
      ol[4 * blk + kq] = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
}

// The weight formats of the products. Every 32-weight block is
// sum_g (A_g * sum c x - B_g * sum x) over its two 16-weight groups g, c
// being the stored code (an exact fp16 integer) and A, B exact fp32:
//   Q4_0, Q8_0: A = d, B = 0 (Q4_0 codes are nibble - 8)
//   Q4_1, Q5_1: A = d, B = -m (nibbles; 5-bit codes as int8)
//   Q8_1:       A = fp32 d, B = 0
//   K-quants:   kq_affine (Q4_K and Q5_K one (A, B) pair per block; Q2_K,
//               Q3_K and Q6_K one per 16-weight group)
// kLay: the code layout, and so the slot order of the split x (2: nibbles
// as Q4_0's, 8: int8 codes as Q8_0's).
template <int QT>
struct PQ {
  static constexpr int kLay = code_bytes_of(QT) == 16 ? 2 : 8;
  static constexpr bool kGroups = QT == kQ2K || QT == kQ3K || QT == kQ6K;
  static constexpr bool kMin =
      QT == kQ4_1 || QT == kQ5_1 || QT == kQ2K || QT == kQ3K || QT == kQ4K || QT == kQ5K;
  static constexpr float kNibOff = QT == 2 ? -1032.0f : -1024.0f;   // 0x6400 | u is 1024 + u
};

// A lane's 8 codes of one block as exact fp16 values in slot order (nibble
// layout: w0 = 32-bit word kq of the block; int8 layout: w0, w1 = words 2kq,
// 2kq+1).
template <int QT>
__device__ __forceinline__ v8h codes_f16(uint32_t w0, uint32_t w1) {
  v4u r;
  if constexpr (PQ<QT>::kLay == 2) {
    const h2 off = {(_Float16)PQ<QT>::kNibOff, (_Float16)PQ<QT>::kNibOff};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      r[k] = __builtin_bit_cast(uint32_t,
                                __builtin_bit_cast(h2, ((w0 >> (4 * k)) & 0x000F000Fu) | 0x64006400u) + off);
  } else {
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (u0 & 0x00FF00FFu) | 0x64006400u) + off);
    r[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, ((u0 >> 8) & 0x00FF00FFu) | 0x64006400u) + off);
    r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (u1 & 0x00FF00FFu) | 0x64006400u) + off);
    r[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, ((u1 >> 8) & 0x00FF00FFu) | 0x64006400u) + off);
  }
  return __builtin_bit_cast(v8h, r);
}

// (A_g, B_g) of a block from its scale entry e (16 bits, or 32 for Q4_1 /
// Q5_1 / Q8_1) and, for the K-quants, its super-block word sup.
template <int QT>
__device__ __forceinline__ void block_affine(uint32_t e, uint32_t sup, float (&A)[2], float (&B)[2]) {
  if constexpr (QT == 2 || QT == 8) {
    A[0] = A[1] = h2f((uint16_t)e);
    B[0] = B[1] = 0.f;
  } else if constexpr (QT == kQ4_1 || QT == kQ5_1) {
    A[0] = A[1] = h2f((uint16_t)(e & 0xffffu));
    B[0] = B[1] = -h2f((uint16_t)(e >> 16));
  } else if constexpr (QT == kQ8_1) {
    A[0] = A[1] = __uint_as_float(e);
    B[0] = B[1] = 0.f;
  } else {
    kq_affine<QT>(e, sup, A, B);
  }
}

// The slots of 16-weight group g among a lane's 8 (slot order above): nibble
// layout, slots 2, 3, 6, 7 are the block's weights 16..31 (pairs 1 and 3 of
// the four fp16 pairs); int8 layout, lane groups kq 2 and 3 hold them.
template <int QT>
__device__ __forceinline__ v8h group_part(v8h v, int g, int kq) {
  if constexpr (PQ<QT>::kLay == 2) {
    v4u r = __builtin_bit_cast(v4u, v);
    if (g == 0) {
      r[1] = 0u;
      r[3] = 0u;
    } else {
      r[0] = 0u;
      r[2] = 0u;
    }
    return __builtin_bit_cast(v8h, r);
  } else {
    return (kq >= 2) == (g == 1) ? v : v8h{};
  }
}

// Workgroup: 4 waves x kHRG row groups of 16 rows x 64 tokens. Per packed tile
// (4 blocks, 128 columns) the split x of the 64 tokens is copied into LDS by
// direct global-to-LDS loads (double buffered; the next tile's x, codes and
// scales in flight during this tile's products). Chunk q of token r sits at
// slot q ^ (r % 16) of its LDS row, so the 16 tokens of a tile read one
// chunk each from distinct banks. Lane (n, kq): weight row n of each row
// group, token rows 4kq .. 4kq+3 of each 16-token tile in the results.
template <int QT, int NMAT, int EPI, int kHRG>
__global__ void __launch_bounds__(kHWaves * 64, 2) k_gemm_h(const GemmArgs a, int ldxs) {
  __shared__ v4u xs[2][2][kHTok][kHChunks];   // [buffer][high, low][token][slot]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const int g0 = (blockIdx.x * kHWaves + wave) * kHRG;
  const int nb = a.cols >> 5;
  const int ntk = (nb + kTB - 1) / kTB;
  const int t0 = blockIdx.y * kHTok;
  const int n = lane & 15, kq = lane >> 4;
  constexpr int kQW = PQ<QT>::kLay == 2 ? 1 : 2;   // code words per lane per block
  const uint16_t* xlo = a.xs + (size_t)a.T * ldxs;
  const float* xinv = reinterpret_cast<const float*>(a.xs + 2 * (size_t)a.T * ldxs);

  // staging: 2 parts x 64 tokens x 16 chunks per tile = 32 rows of 1 KB; wave
  // w copies rows 8w .. 8w+7 (part R / 16, tokens 4(R % 16) .. +3), lane i
  // token 4(R % 16) + i/16, slot i % 16
  auto stage_x = [&](int tk, int buf) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int R = 8 * wave + k, part = R >> 4, r = 4 * (R & 15) + (lane >> 4), slot = lane & 15;
      const int t = min(t0 + r, a.T - 1);
      const uint16_t* src = (part ? xlo : a.xs) + (size_t)t * ldxs + tk * 128 + 8 * (slot ^ (r & 15));
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)&xs[buf][part][4 * (R & 15)][0], 16, 0, 0);
    }
  };
  // per block: codes, the raw scale entry; per tile: the K-quants' super-block word
  uint32_t wq[NMAT][kHRG][kTB][kQW];
  uint32_t we[NMAT][kHRG][kTB];
  uint32_t wsu[NMAT][kHRG];
  // Blocks past the row (the last tile's padding of a 32-weight type) are
  // read and weighted 0 (entry 0: A = B = 0). Where that selection sits
  // decides where the compiler waits for the next tile: made at load, it
  // waits for the whole next tile (its loads complete in order) inside the
  // current tile's first block; made at use, those loads overlap all four
  // blocks. Measured per variant at the 7B and 70B shapes (512-token chunks):
  // at use, the stores and the one-row-group accumulation ran 9-13% faster
  // (7B QKV 179 -> 160 us, Wo + down 118 -> 105 us, 70B QKV 319 -> 279 us);
  // gate+up (1191 -> 1228 us at 70B) and the two-row-group accumulation
  // (377 -> 426 us) ran slower, so those keep the selection at load.
  constexpr bool kMaskAtLoad = EPI == EPI_SWIGLU || (EPI == EPI_ADD && kHRG == 2);
  auto load_w = [&](int tk, uint32_t (&q)[NMAT][kHRG][kTB][kQW], uint32_t (&e)[NMAT][kHRG][kTB],
                    uint32_t (&su)[NMAT][kHRG]) {
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int r = 0; r < kHRG; ++r) {
        const PackedMat& w = mt == 0 ? a.w : a.w2;
        const int g = min(g0 + r, ngroups - 1);
#pragma unroll
        for (int b = 0; b < kTB; ++b) {
          const int tl = tile_lane(n, b);
          const uint32_t* p =
              reinterpret_cast<const uint32_t*>(w.qs + tile_idx(g, ntk, tk, tl) * QTraits<QT>::kQB) + kQW * kq;
#pragma unroll
          for (int k = 0; k < kQW; ++k) q[mt][r][b][k] = p[k];
          const uint32_t ev = is_wide(QT) ? reinterpret_cast<const uint32_t*>(w.ds)[scale_idx(g, ntk, tk, tl)]
                                          : (uint32_t)w.ds[scale_idx(g, ntk, tk, tl)];
          e[mt][r][b] = !kMaskAtLoad || tk * kTB + b < nb ? ev : 0u;
        }
        // K-quants: the 4 blocks of a tile lie in super-block tk / 2 (nb is a multiple of 8)
        su[mt][r] = is_kq(QT) ? w.su[((size_t)g * (ntk / 2) + tk / 2) * kRG + n] : 0u;
      }
  };

  v4f acc[NMAT][kHRG][kHTiles];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int r = 0; r < kHRG; ++r)
#pragma unroll
      for (int tt = 0; tt < kHTiles; ++tt) acc[mt][r][tt] = v4f{0.f, 0.f, 0.f, 0.f};

  stage_x(0, 0);
  load_w(0, wq, we, wsu);
  vm_drain();
  __syncthreads();
#pragma unroll 1
  for (int tk = 0; tk < ntk; ++tk) {
    const int buf = tk & 1;
    // the next tile in flight (the last iteration reloads its own tile into
    // the idle buffer: branch-free, read by no one)
    const int tn = min(tk + 1, ntk - 1);
    uint32_t nq[NMAT][kHRG][kTB][kQW];
    uint32_t ne[NMAT][kHRG][kTB];
    uint32_t nsu[NMAT][kHRG];
    stage_x(tn, buf ^ 1);
    load_w(tn, nq, ne, nsu);
#pragma unroll
    for (int b = 0; b < kTB; ++b) {
      constexpr int NG = PQ<QT>::kGroups ? 2 : 1;   // codes split by 16-weight group
      v8h wc[NMAT][kHRG][NG];
      float A[NMAT][kHRG][2], B[NMAT][kHRG][2];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int r = 0; r < kHRG; ++r) {
          const v8h c = codes_f16<QT>(wq[mt][r][b][0], wq[mt][r][b][kQW - 1]);
#pragma unroll
          for (int gg = 0; gg < NG; ++gg) wc[mt][r][gg] = NG == 1 ? c : group_part<QT>(c, gg, kq);
          block_affine<QT>(kMaskAtLoad || tk * kTB + b < nb ? we[mt][r][b] : 0u, wsu[mt][r], A[mt][r], B[mt][r]);
        }
#pragma unroll
      for (int tt = 0; tt < kHTiles; ++tt) {
        const v8h xh = __builtin_bit_cast(v8h, xs[buf][0][tt * 16 + n][(4 * b + kq) ^ n]);
        const v8h xl = __builtin_bit_cast(v8h, xs[buf][1][tt * 16 + n][(4 * b + kq) ^ n]);
        v4f sx[NG];   // sum of x over the block (or group), for the B terms
        if constexpr (PQ<QT>::kMin) {
#pragma unroll
          for (int gg = 0; gg < NG; ++gg) {
            const v8h one = NG == 1 ? kOnes : group_part<QT>(kOnes, gg, kq);
            sx[gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, one, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            sx[gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, one, sx[gg], 0, 0, 0);
          }
        }
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int r = 0; r < kHRG; ++r)
#pragma unroll
            for (int gg = 0; gg < NG; ++gg) {
              v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wc[mt][r][gg], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
              c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wc[mt][r][gg], c, 0, 0, 0);
              const float ag = A[mt][r][gg];
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[mt][r][tt][i] = fmaf(ag, c[i], acc[mt][r][tt][i]);
              if constexpr (PQ<QT>::kMin) {
                const float bg = -B[mt][r][gg];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][r][tt][i] = fmaf(bg, sx[gg][i], acc[mt][r][tt][i]);
              }
            }
      }
      __builtin_amdgcn_sched_barrier(0);   // one block's operands live at a time
    }
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
      for (int r = 0; r < kHRG; ++r) {
#pragma unroll
        for (int b = 0; b < kTB; ++b) {
#pragma unroll
          for (int k = 0; k < kQW; ++k) wq[mt][r][b][k] = nq[mt][r][b][k];
          we[mt][r][b] = ne[mt][r][b];
        }
        wsu[mt][r] = nsu[mt][r];
      }
    vm_drain();   // this wave's direct LDS loads of the next tile have landed
    __syncthreads();
  }

  // epilogue: lane holds row g*16 + n of tokens t0 + 16tt + 4kq + i
  // per token: 1/s_t, times the RMSNorm scale. The sums of squares come
  // through a buffer view (empty without a norm weight: reads return 0 and
  // the scale is 1), so no branch separates the loads and all are in flight
  // together.
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.ssq), (short)0, a.nw ? a.T * 4 : 0, kBufferFlags);
  float tsc[kHTiles][4];
#pragma unroll
  for (int tt = 0; tt < kHTiles; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = min(t0 + tt * 16 + 4 * kq + i, a.T - 1);
      const float ss = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, t * 4, 0, 0));
      const float rn = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
      tsc[tt][i] = xinv[t] * (a.nw ? rn : 1.0f);
    }
  // the accumulating form reads every old value before it writes any (a
  // load after a store to y would wait for it: the compiler cannot tell the
  // addresses apart); clamped addresses, used only where the output exists
  float yo[kHRG][kHTiles][4];
  if constexpr (EPI == EPI_ADD) {
#pragma unroll
    for (int r = 0; r < kHRG; ++r) {
      const int row = min((g0 + r) * kRG + n, a.rows - 1);
#pragma unroll
      for (int tt = 0; tt < kHTiles; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          yo[r][tt][i] = a.y[(size_t)min(t0 + tt * 16 + 4 * kq + i, a.T - 1) * a.ldy + row];
    }
  }
#pragma unroll
  for (int r = 0; r < kHRG; ++r) {
    const int g = g0 + r;
    const int row = g * kRG + n;
    if (g >= ngroups || row >= a.rows) continue;
#pragma unroll
    for (int tt = 0; tt < kHTiles; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + tt * 16 + 4 * kq + i;
        if (t >= a.T) continue;
        const float scale = tsc[tt][i];
        const float x0 = acc[0][r][tt][i] * scale;
        float v;
        if constexpr (EPI == EPI_SWIGLU) {
          const float up = acc[NMAT - 1][r][tt][i] * scale;
          v = up * (a.act == 1 ? gelu_tanh(x0) : silu(x0));   // layer_scheduler.c:529-547
        } else {
          v = x0;
        }
        float* yp = a.y + (size_t)t * a.ldy + row;
        if constexpr (EPI == EPI_ADD)
          *yp = yo[r][tt][i] + v;
        else
          *yp = v;
      }
  }
}

template <int QT, int NMAT, int EPI>
hipError_t launch_gemm_t(const GemmArgs& a, hipStream_t s) {
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const dim3 grid((ngroups + kGemmWaves - 1) / kGemmWaves, (a.T + kGemmTok - 1) / kGemmTok);
  hipLaunchKernelGGL((k_gemm<QT, NMAT, EPI>), grid, dim3(kGemmWaves * 64), 0, s, a);
  return hipGetLastError();
}

std::atomic<int64_t> g_gemm_h_launches[kGemmVariants];

template <int QT, int NMAT, int EPI, int RG>
hipError_t launch_gemm_h_t(const GemmArgs& a, int ldxs, hipStream_t s) {
  constexpr int slot = EPI == EPI_STORE ? 0 : EPI == EPI_ADD ? 1 : 2;
  g_gemm_h_launches[2 * slot + RG - 1].fetch_add(1, std::memory_order_relaxed);
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const dim3 grid((ngroups + kHWaves * RG - 1) / (kHWaves * RG), (a.T + kHTok - 1) / kHTok);
  hipLaunchKernelGGL((k_gemm_h<QT, NMAT, EPI, RG>), grid, dim3(kHWaves * 64), 0, s, a, ldxs);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_gemm_q(int epi, const GemmArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return launch_gemm_t<QT, 1, EPI_STORE>(a, s);
    case EPI_ADD: return launch_gemm_t<QT, 1, EPI_ADD>(a, s);
    case EPI_SWIGLU: return launch_gemm_t<QT, 2, EPI_SWIGLU>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// Two matrices (gate/up) take one row group of each per wave; one matrix two
// row groups per wave, or one when that leaves fewer than two workgroups per
// compute unit.
template <int QT>
hipError_t launch_gemm_h(int epi, const GemmArgs& a, int ldxs, int n_cu, hipStream_t s) {
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const long wg2 = (long)((ngroups + 2 * kHWaves - 1) / (2 * kHWaves)) * ((a.T + kHTok - 1) / kHTok);
  const bool one = wg2 < 2L * n_cu;
  switch (epi) {
    case EPI_STORE:
      return one ? launch_gemm_h_t<QT, 1, EPI_STORE, 1>(a, ldxs, s) : launch_gemm_h_t<QT, 1, EPI_STORE, 2>(a, ldxs, s);
    case EPI_ADD:
      return one ? launch_gemm_h_t<QT, 1, EPI_ADD, 1>(a, ldxs, s) : launch_gemm_h_t<QT, 1, EPI_ADD, 2>(a, ldxs, s);
    case EPI_SWIGLU: return launch_gemm_h_t<QT, 2, EPI_SWIGLU, 1>(a, ldxs, s);
    default: return hipErrorInvalidValue;
  }
}

int device_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) n = p.multiProcessorCount;
    if (n <= 0) n = 256;
  }
  return n;
}

}  // namespace

const int64_t* gemm_h_launch_counts() {
  static int64_t snap[kGemmVariants];
  for (int i = 0; i < kGemmVariants; ++i) snap[i] = g_gemm_h_launches[i].load(std::memory_order_relaxed);
  return snap;
}

hipError_t launch_sumsq(const float* x, int cols, int T, float* ssq, hipStream_t s) {
  if (T <= 0 || cols <= 0 || cols % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sumsq, dim3(T), dim3(256), 0, s, x, cols, cols, ssq);
  return hipGetLastError();
}

hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.rows <= 0 || a.cols <= 0 || a.cols % 32 || a.ldy < a.rows || a.ldx < a.cols || a.ldx % 4 ||
      (a.nw && !a.ssq))
    return hipErrorInvalidValue;
  if (epi != EPI_STORE && epi != EPI_ADD && epi != EPI_SWIGLU) return hipErrorInvalidValue;
  const int t = dev_type(a.type);
  if (a.xs && product_format(t)) {
    if (is_kq(t) && a.cols % 256) return hipErrorInvalidValue;   // whole super-blocks
    const int ldxs = (a.cols + 127) / 128 * 128;
    uint16_t* xl = a.xs + (size_t)a.T * ldxs;
    float* xinv = reinterpret_cast<float*>(a.xs + 2 * (size_t)a.T * ldxs);
    float* ssq = a.nw ? a.ssq : nullptr;
    if (code_bytes_of(t) == 16)   // nibble layouts: Q4_0's slot order
      hipLaunchKernelGGL(k_split_x<2>, dim3(a.T), dim3(256), 0, s, a.x, a.ldx, a.nw, a.cols, ssq, a.xs, xl, xinv, ldxs);
    else
      hipLaunchKernelGGL(k_split_x<8>, dim3(a.T), dim3(256), 0, s, a.x, a.ldx, a.nw, a.cols, ssq, a.xs, xl, xinv, ldxs);
    if (hipError_t e = hipGetLastError()) return e;
    const int n_cu = device_cus();
    switch (t) {
      case 2: return launch_gemm_h<2>(epi, a, ldxs, n_cu, s);
      case 8: return launch_gemm_h<8>(epi, a, ldxs, n_cu, s);
      case kQ4_1: return launch_gemm_h<kQ4_1>(epi, a, ldxs, n_cu, s);
      case kQ5_1: return launch_gemm_h<kQ5_1>(epi, a, ldxs, n_cu, s);
      case kQ8_1: return launch_gemm_h<kQ8_1>(epi, a, ldxs, n_cu, s);
      case kQ2K: return launch_gemm_h<kQ2K>(epi, a, ldxs, n_cu, s);
      case kQ3K: return launch_gemm_h<kQ3K>(epi, a, ldxs, n_cu, s);
      case kQ4K: return launch_gemm_h<kQ4K>(epi, a, ldxs, n_cu, s);
      case kQ5K: return launch_gemm_h<kQ5K>(epi, a, ldxs, n_cu, s);
      default: return launch_gemm_h<kQ6K>(epi, a, ldxs, n_cu, s);
    }
  }
  if (a.nw) {
    hipLaunchKernelGGL(k_sumsq, dim3(a.T), dim3(256), 0, s, a.x, a.ldx, a.cols, a.ssq);
    if (hipError_t e = hipGetLastError()) return e;
  }
  if (t == 2) return launch_gemm_q<2>(epi, a, s);
  if (t == 8) return launch_gemm_q<8>(epi, a, s);
  return hipErrorInvalidValue;
}

}  // namespace ssk
