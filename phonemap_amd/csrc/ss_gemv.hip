// ss_gemv.hip - block-quantized matrix-vector kernels for gfx950.
//
// Device weight layout (made by k_pack from GGUF blocks): rows are taken in
// groups of 64 (padded with zero rows); for row group g and 32-column block
// b, the 64 rows' code chunks are contiguous - code[(g*nb + b)*64 + lane]
// of 16 (Q4_0) or 32 (Q8_0) bytes - and the binary16 scales follow in a
// second plane with the same index. A wave therefore loads one block of 64
// different rows as one contiguous 1 KiB (Q4_0) read, one row per lane.
//
// k_gemv3: workgroup = S waves x one row group. Lane l owns row 64g + l;
// wave s walks blocks [s*nb/S, (s+1)*nb/S) of it, dequantising in registers
// with fp32 accumulation, double-buffering batches of blocks. x (times the
// RMSNorm weight when there is one) is staged once per workgroup in LDS and
// read with broadcast loads. The S partial sums of each row are added in LDS
// in wave order, so results do not depend on timing. There is no cross-lane
// reduction per row and no data handed between workgroups.

#include <math.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

// floats of LDS per 32-column block of x: 32 values, their sum, 3 pad
constexpr int kXBlk = 36;

// Q4_0 block (quantize.c:60-72): byte j holds weight j (low nibble) and
// weight j+16 (high nibble), value = d * (nibble - 8). Returns
// sum_j (nibble_j - 8) * x_j; the caller multiplies by d. The -8 offset is
// folded through the block sum of x staged at xb[32]; high nibbles are used
// in place (x16) and rescaled by 1/16 exactly.
__device__ __forceinline__ float q4_block(const uint4 q, const float* __restrict__ xb) {
  const float4* x4 = reinterpret_cast<const float4*>(xb);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float slo = 0.f, shi = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = w[k] & 0x0F0F0F0Fu;
    const uint32_t hi = w[k] & 0xF0F0F0F0u;
    const float4 xl = x4[k];
    const float4 xh = x4[4 + k];
    slo = fmaf((float)(lo & 0xffu), xl.x, slo);
    slo = fmaf((float)((lo >> 8) & 0xffu), xl.y, slo);
    slo = fmaf((float)((lo >> 16) & 0xffu), xl.z, slo);
    slo = fmaf((float)(lo >> 24), xl.w, slo);
    shi = fmaf((float)(hi & 0xffu), xh.x, shi);
    shi = fmaf((float)((hi >> 8) & 0xffu), xh.y, shi);
    shi = fmaf((float)((hi >> 16) & 0xffu), xh.z, shi);
    shi = fmaf((float)(hi >> 24), xh.w, shi);
  }
  return fmaf(shi, 0.0625f, slo) - 8.0f * xb[32];
}

// Q8_0 block (quantize.c:139-149): 32 int8 codes, value = d * code.
__device__ __forceinline__ float q8_block(const uint4 a, const uint4 b, const float* __restrict__ xb) {
  const float4* x4 = reinterpret_cast<const float4*>(xb);
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k += 2) {
    const float4 xa = x4[k];
    const float4 xc = x4[k + 1];
    s0 = fmaf((float)(int8_t)(w[k] & 0xffu), xa.x, s0);
    s0 = fmaf((float)(int8_t)((w[k] >> 8) & 0xffu), xa.y, s0);
    s0 = fmaf((float)(int8_t)((w[k] >> 16) & 0xffu), xa.z, s0);
    s0 = fmaf((float)(int8_t)(w[k] >> 24), xa.w, s0);
    s1 = fmaf((float)(int8_t)(w[k + 1] & 0xffu), xc.x, s1);
    s1 = fmaf((float)(int8_t)((w[k + 1] >> 8) & 0xffu), xc.y, s1);
    s1 = fmaf((float)(int8_t)((w[k + 1] >> 16) & 0xffu), xc.z, s1);
    s1 = fmaf((float)(int8_t)(w[k + 1] >> 24), xc.w, s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ size_t tile_idx(int g, int nb, int b, int lane) {
  return ((size_t)g * nb + b) * kWave + lane;
}

// Stage blocks [cb, cb+nblk) of x into LDS, times the RMSNorm weight nw when
// set (the x*w of cpu_neon.c:114; the 1/rms factor is applied to the row sums),
// with each block's sum at slot 32. Returns this thread's share of sum(x^2).
__device__ float stage_x(float* xs, const float* __restrict__ x, const float* __restrict__ nw,
                         int cb, int nblk) {
  float ss = 0.f;
  const int ngroups = nblk * 8;
  for (int g = threadIdx.x; g < ngroups; g += blockDim.x) {
    const int blk = g >> 3, sub = g & 7;
    const int col = (cb + blk) * 32 + sub * 4;
    float4 v = *reinterpret_cast<const float4*>(x + col);
    if (nw) {
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
      const float4 w = *reinterpret_cast<const float4*>(nw + col);
      v.x *= w.x;
      v.y *= w.y;
      v.z *= w.z;
      v.w *= w.w;
    }
    *reinterpret_cast<float4*>(xs + blk * kXBlk + sub * 4) = v;
    const float s = sum8((v.x + v.y) + (v.z + v.w));
    if (sub == 0) xs[blk * kXBlk + 32] = s;
  }
  return ss;
}

template <int QT, int NB, int NMAT>
struct Batch {
  static constexpr int kNV = QTraits<QT>::kQB / 16;
  uint4 q[NMAT][NB][kNV];
  float d[NMAT][NB];
};

template <int QT, int NB, int NMAT>
__device__ __forceinline__ void load_batch(Batch<QT, NB, NMAT>& f, const GemvArgs& a, int g, int nb,
                                           int b, int lim, int lane) {
  constexpr int kQB = QTraits<QT>::kQB;
  constexpr int kNV = kQB / 16;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    const PackedMat& w = m == 0 ? a.w : a.w2;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (b + k < lim) {
        const size_t i = tile_idx(g, nb, b + k, lane);
        const uint4* src = reinterpret_cast<const uint4*>(w.qs + i * kQB);
#pragma unroll
        for (int v = 0; v < kNV; ++v) f.q[m][k][v] = src[v];
        f.d[m][k] = h2f(w.ds[i]);
      }
    }
  }
}

template <int QT, int NB, int NMAT>
__device__ __forceinline__ void fma_batch(float (&acc)[NMAT], const Batch<QT, NB, NMAT>& f,
                                          const float* xs, int b, int lim, int cb) {
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    if (b + k < lim) {
      const float* xb = xs + (b + k - cb) * kXBlk;
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        float s;
        if constexpr (QT == 2)
          s = q4_block(f.q[m][k][0], xb);
        else
          s = q8_block(f.q[m][k][0], f.q[m][k][1], xb);
        acc[m] = fmaf(f.d[m][k], s, acc[m]);
      }
    }
  }
}

// Per-lane epilogue of wave 0: v[] holds row `row`'s final value(s).
template <int EPI, int NMAT>
__device__ __forceinline__ void epilogue(const GemvArgs& a, int row, const float (&v)[NMAT]) {
  const bool valid = row < a.rows;
  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
    if (valid) a.y[row] = EPI == EPI_ADD ? v[0] + a.y[row] : v[0];   // layer_scheduler.c:484,566
  } else if constexpr (EPI == EPI_SWIGLU) {
    const float g = v[0], u = v[NMAT - 1];
    if (valid) a.y[row] = u * (g / (1.0f + expf(-g)));                // layer_scheduler.c:540-547
  } else if constexpr (EPI == EPI_QKV) {
    // rows of [Wq; Wk; Wv]; q and k rows (i, i+1) are lanes (2j, 2j+1): rotate
    // the pair with the position's (cos, sin), tensor.c:250-273
    const float partner = __shfl_xor(v[0], 1, kWave);
    if (!valid) return;
    const int pos = *a.dpos;
    const int hd = a.head_dim;
    float out = v[0];
    if (row < a.qdim + a.kvdim) {
      const int i = (row < a.qdim ? row : row - a.qdim) % hd;
      const int i0 = i & ~1;
      if (i0 < a.rope_dim) {
        const float* cs = a.rope_cs + (size_t)pos * a.rope_dim;
        const float c = cs[i0], s = cs[i0 + 1];
        out = (i & 1) ? partner * s + v[0] * c : v[0] * c - partner * s;
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
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (valid) {
      a.y[row] = v[0];
      bv = v[0];
      bi = row;
    }
    wave_best(bv, bi);
    if ((threadIdx.x & 63) == 0) a.part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

template <int QT, int NMAT, int EPI>
__global__ void __launch_bounds__(1024) k_gemv3(const GemvArgs a) {
  constexpr int NB = (QT == 2 ? 4 : 2) / NMAT;   // blocks per batch and buffer (4 KiB per wave)
  extern __shared__ float4 smem4[];
  float* xs = reinterpret_cast<float*>(smem4);
  float* red = xs + a.chunk_blocks * kXBlk;      // [NMAT][S][64] partial sums, then [S] sum(x^2)

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int S = blockDim.x >> 6;
  const int g = blockIdx.x;
  const int nb = a.cols >> 5;
  const int b0 = wave * nb / S, b1 = (wave + 1) * nb / S;

  float acc[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) acc[m] = 0.f;
  float ssq = 0.f;
  Batch<QT, NB, NMAT> cur, nxt;

  for (int cb = 0; cb < nb; cb += a.chunk_blocks) {
    const int ce = min(nb, cb + a.chunk_blocks);
    const int lo = max(b0, cb), hi = min(b1, ce);
    if (lo < hi) load_batch<QT, NB, NMAT>(cur, a, g, nb, lo, hi, lane);   // in flight during staging
    if (cb) __syncthreads();   // everyone is done with the previous chunk of x
    ssq += stage_x(xs, a.x, a.nw, cb, ce - cb);
    __syncthreads();
    for (int b = lo; b < hi; b += NB) {
      if (b + NB < hi) load_batch<QT, NB, NMAT>(nxt, a, g, nb, b + NB, hi, lane);
      fma_batch<QT, NB, NMAT>(acc, cur, xs, b, hi, cb);
      cur = nxt;
    }
  }

#pragma unroll
  for (int m = 0; m < NMAT; ++m) red[(m * S + wave) * kWave + lane] = acc[m];
  if (a.nw) {
    const float w = wave_sum(ssq);
    if (lane == 0) red[NMAT * S * kWave + wave] = w;
  }
  __syncthreads();
  if (wave != 0) return;
  float v[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    float s = 0.f;
    for (int w = 0; w < S; ++w) s += red[(m * S + w) * kWave + lane];
    v[m] = s;
  }
  if (a.nw) {   // RMSNorm scale of tensor.c:114-131: 1 / sqrt(mean(x^2) + eps)
    float t = 0.f;
    for (int w = 0; w < S; ++w) t += red[NMAT * S * kWave + w];
    const float scale = 1.0f / sqrtf(t / (float)a.cols + a.eps);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) v[m] *= scale;
  }
  epilogue<EPI, NMAT>(a, g * kWave + lane, v);
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
  const size_t o = tile_idx((int)(row >> 6), nb, b, (int)(row & 63));
  const uint8_t* s = src + i * kBytes;
  ds[o] = (uint16_t)(s[0] | (s[1] << 8));
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

// Row `token` of a packed table, dequantised exactly as quantize.c:60-72 /
// 139-149 (one fp32 multiply per weight).
template <int QT>
__global__ void k_embed(PackedMat t, int cols, const int* tokens, const int* dpos, int token,
                        float* out) {
  constexpr int kQB = QTraits<QT>::kQB;
  const int tok = tokens ? tokens[*dpos] : token;
  const int nb = cols >> 5;
  for (int b = threadIdx.x; b < nb; b += blockDim.x) {
    const size_t i = tile_idx(tok >> 6, nb, b, tok & 63);
    const float d = h2f(t.ds[i]);
    const uint8_t* q = t.qs + i * kQB;
    float* o = out + b * 32;
    if constexpr (QT == 2) {
      for (int j = 0; j < 16; ++j) {
        const uint8_t v = q[j];
        o[j] = d * (float)((int)(v & 0xF) - 8);
        o[j + 16] = d * (float)((int)(v >> 4) - 8);
      }
    } else {
      for (int j = 0; j < 32; ++j) o[j] = d * (float)(int8_t)q[j];
    }
  }
}

// Picks the first maximum among per-workgroup candidates, writes it, and for
// device-side greedy decoding appends it at tokens[pos+1] and advances pos.
__global__ void k_argmax_merge(const float2* part, int n, const float* y, int* out_idx, int* tokens,
                               int* dpos) {
  __shared__ float2 wb[4];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float2 p = part[i];
    const int pi = __float_as_int(p.y);
    if (beats(p.x, pi, bv, bi)) {
      bv = p.x;
      bi = pi;
    }
  }
  wave_best(bv, bi);
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < 4; ++w)
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

template <int QT, int NMAT, int EPI>
hipError_t launch_t(const GemvArgs& a, hipStream_t s) {
  GemvPlan p = gemv_plan(a.rows, a.cols, a.n_cu, NMAT);
  GemvArgs b = a;
  b.chunk_blocks = p.chunk_blocks;
  hipLaunchKernelGGL((k_gemv3<QT, NMAT, EPI>), dim3(p.grid), dim3(p.threads), p.lds_bytes, s, b);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_q(int epi, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return launch_t<QT, 1, EPI_STORE>(a, s);
    case EPI_ADD: return launch_t<QT, 1, EPI_ADD>(a, s);
    case EPI_SWIGLU: return launch_t<QT, 2, EPI_SWIGLU>(a, s);
    case EPI_QKV: return launch_t<QT, 1, EPI_QKV>(a, s);
    case EPI_LOGITS: return launch_t<QT, 1, EPI_LOGITS>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// One workgroup per 64-row group with S waves splitting the columns; S is the
// power of two (<= 16) that brings the launch closest to 8 waves per CU.
GemvPlan gemv_plan(int rows, int cols, int n_cu, int nmat) {
  GemvPlan p;
  const int groups = (rows + 63) / 64;
  const int nb = cols / 32;
  const int want = (n_cu > 0 ? n_cu : 256) * 8;
  int S = 1;
  while (S < kGemvMaxSplit && groups * S * 2 <= want && S * 2 <= (nb + 3) / 4) S *= 2;
  p.grid = groups;
  p.threads = S * kWave;
  p.chunk_blocks = nb < kGemvMaxChunkBlocks ? nb : kGemvMaxChunkBlocks;
  p.lds_bytes = (size_t)p.chunk_blocks * kXBlk * sizeof(float) +
                (size_t)(nmat * S * kWave + S) * sizeof(float);
  return p;
}

size_t packed_bytes(int type, int64_t rows, int cols) {
  const int kqb = type == 2 ? 16 : type == 8 ? 32 : 0;
  const size_t tiles = (size_t)((rows + 63) / 64) * 64 * (cols / 32);
  const size_t code = (tiles * kqb + 255) & ~(size_t)255;
  return code + tiles * 2;
}

PackedMat packed_view(const void* base, int type, int64_t rows, int cols) {
  const int kqb = type == 2 ? 16 : 32;
  const size_t tiles = (size_t)((rows + 63) / 64) * 64 * (cols / 32);
  PackedMat m;
  m.qs = static_cast<const uint8_t*>(base);
  m.ds = reinterpret_cast<const uint16_t*>(m.qs + ((tiles * kqb + 255) & ~(size_t)255));
  return m;
}

hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t s) {
  if (a.type == 2) return launch_q<2>(epi, a, s);
  if (a.type == 8) return launch_q<8>(epi, a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_argmax_merge(const float2* part, int n, const float* y, int* out_idx, int* tokens,
                               int* dpos, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_merge, dim3(1), dim3(256), 0, s, part, n, y, out_idx, tokens, dpos);
  return hipGetLastError();
}

hipError_t launch_pack(int type, const uint8_t* src, uint8_t* qs, uint16_t* ds, int64_t nblocks,
                       int nb, int64_t row_off, hipStream_t s) {
  const int64_t grid = (nblocks + 255) / 256;
  if (type == 2)
    hipLaunchKernelGGL(k_pack<2>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else if (type == 8)
    hipLaunchKernelGGL(k_pack<8>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks, nb, row_off);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_embed(int type, PackedMat t, int cols, const int* tokens, const int* dpos,
                        int token, float* out, hipStream_t s) {
  if (type == 2)
    hipLaunchKernelGGL(k_embed<2>, dim3(1), dim3(256), 0, s, t, cols, tokens, dpos, token, out);
  else if (type == 8)
    hipLaunchKernelGGL(k_embed<8>, dim3(1), dim3(256), 0, s, t, cols, tokens, dpos, token, out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace ssk
