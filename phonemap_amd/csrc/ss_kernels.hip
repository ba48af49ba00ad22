// ss_kernels.hip - gfx950 (MI355X) kernels of the SlipStream token loop.
//
// Batch-1 decode is a sweep of matrix-vector products over block-quantized
// weights, so every kernel here is HBM-bound integer/fp32 work on 64-wide
// wavefronts: 128-bit coalesced loads, dequantisation in registers, fp32
// accumulation, DPP/shuffle reductions. No MFMA.
//
// Weight layout (made by k_pack from GGUF blocks): for a matrix of R rows and
// nb = C/32 blocks per row, the code plane holds R*nb blocks of 16 (Q4_0) or
// 32 (Q8_0) bytes, 16-byte aligned, row-major; the scale plane holds R*nb
// binary16 scales. A wave reads 64 consecutive blocks of a row per load
// instruction (1 KiB of codes, 128 B of scales).

#include "ss_kernels.h"

#include <hip/hip_fp16.h>
#include <math.h>

namespace ssk {
namespace {

constexpr int kWave = 64;
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kWave * kGemvWaves;
// floats of LDS per 32-column block of x: 32 values, their sum, 3 pad
// (the pad makes the per-lane 144-byte stride bank-conflict free for b128 reads)
constexpr int kXBlk = 36;

// ---------------------------------------------------------------- reductions
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

// Cross-workgroup hand-off: the L2s of the 8 XCDs are not coherent with one
// another, so partial results another workgroup will merge are written and
// read with agent-scope atomics (they bypass the non-coherent cache level).
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// "b beats a" for the first-maximum argmax of tensor.c:318-328: larger
// value, or equal value at a smaller index. NaN never beats anything.
__device__ __forceinline__ bool beats(float bv, int bi, float av, int ai) {
  return bv > av || (bv == av && bi < ai);
}

// ------------------------------------------------------------ block dots
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

template <int QT>
struct QTraits;
template <>
struct QTraits<2> {
  static constexpr int kQB = 16;   // code bytes per block
  static constexpr int kGgufBytes = 18;
};
template <>
struct QTraits<8> {
  static constexpr int kQB = 32;
  static constexpr int kGgufBytes = 34;
};

// ------------------------------------------------------------ GEMV staging
// RMSNorm scale of tensor.c:114-131 (1 / sqrt(mean(x^2) + eps)), computed by
// the whole workgroup; every thread returns it.
__device__ float block_rms_scale(const float* __restrict__ x, int n, float eps, float* red) {
  float ss = 0.f;
  for (int i = threadIdx.x * 4; i < n; i += kGemvThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  return 1.0f / sqrtf(tot / (float)n + eps);
}

// Stage blocks [b0, b0+nblk) of x into LDS (x * scale * nw when nw is set,
// the element order of cpu_neon.c:114), with each block's sum at slot 32.
__device__ void stage_x(float* xs, const float* __restrict__ x, const float* __restrict__ nw,
                        float scale, int b0, int nblk) {
  const int ngroups = nblk * 8;
  for (int g = threadIdx.x; g < ngroups; g += kGemvThreads) {
    const int blk = g >> 3, sub = g & 7;
    const int col = (b0 + blk) * 32 + sub * 4;
    float4 v = *reinterpret_cast<const float4*>(x + col);
    if (nw) {
      const float4 w = *reinterpret_cast<const float4*>(nw + col);
      v.x = v.x * scale * w.x;
      v.y = v.y * scale * w.y;
      v.z = v.z * scale * w.z;
      v.w = v.w * scale * w.w;
    }
    *reinterpret_cast<float4*>(xs + blk * kXBlk + sub * 4) = v;
    const float s = sum8((v.x + v.y) + (v.z + v.w));
    if (sub == 0) xs[blk * kXBlk + 32] = s;
  }
}

template <int QT, int R, int NMAT>
struct Frag {
  static constexpr int kNV = QTraits<QT>::kQB / 16;
  uint4 q[NMAT][R][kNV];
  float d[NMAT][R];
};

template <int QT, int R, int NMAT>
__device__ __forceinline__ void load_frag(Frag<QT, R, NMAT>& f, const GemvArgs& a, const int* rowc,
                                          int nb, int b) {
  constexpr int kQB = QTraits<QT>::kQB;
  constexpr int kNV = kQB / 16;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    const PackedMat& w = m == 0 ? a.w : a.w2;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t bi = (size_t)rowc[r] * nb + b;
      const uint4* src = reinterpret_cast<const uint4*>(w.qs + bi * kQB);
#pragma unroll
      for (int v = 0; v < kNV; ++v) f.q[m][r][v] = src[v];
      f.d[m][r] = h2f(w.ds[bi]);
    }
  }
}

template <int QT, int R, int NMAT>
__device__ __forceinline__ void fma_frag(float (&acc)[NMAT][R], const Frag<QT, R, NMAT>& f,
                                         const float* xb) {
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s;
      if constexpr (QT == 2)
        s = q4_block(f.q[m][r][0], xb);
      else
        s = q8_block(f.q[m][r][0], f.q[m][r][1], xb);
      acc[m][r] = fmaf(f.d[m][r], s, acc[m][r]);
    }
}

// ------------------------------------------------------------ GEMV kernel
// Workgroup = 4 waves; wave w owns rows (blockIdx.x*4 + w)*R .. +R-1 (times
// NMAT matrices); lane l walks blocks l, l+64, ... of those rows, one block
// of codes per row per step, with the next step's codes in flight. x (with
// the optional RMSNorm folded in) sits in LDS, read once per block and
// shared by the R*NMAT rows.
template <int QT, int R, int NMAT, int EPI>
__global__ void __launch_bounds__(kGemvThreads) k_gemv(const GemvArgs a) {
  extern __shared__ float4 smem4[];
  float* xs = reinterpret_cast<float*>(smem4);
  __shared__ float red[kGemvWaves];
  __shared__ float2 wbest[kGemvWaves];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = a.cols >> 5;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
  int rowc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rowc[r] = min(row0 + r, a.rows - 1);

  float acc[NMAT][R];
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  Frag<QT, R, NMAT> cur;
  int nblk = min(a.chunk_blocks, nb);
  int b = lane;
  bool have = b < nblk;
  if (have) load_frag<QT, R, NMAT>(cur, a, rowc, nb, b);   // in flight while x is staged

  const float scale = a.nw ? block_rms_scale(a.x, a.cols, a.eps, red) : 1.0f;

  for (int cb = 0; cb < nb; cb += a.chunk_blocks) {
    if (cb) {
      nblk = min(a.chunk_blocks, nb - cb);
      __syncthreads();   // everyone is done with the previous chunk of x
      b = lane;
      have = b < nblk;
      if (have) load_frag<QT, R, NMAT>(cur, a, rowc, nb, cb + b);
    }
    stage_x(xs, a.x, a.nw, scale, cb, nblk);
    __syncthreads();
    while (have) {
      const int bn = b + kWave;
      const bool hn = bn < nblk;
      Frag<QT, R, NMAT> nxt;
      if (hn) load_frag<QT, R, NMAT>(nxt, a, rowc, nb, cb + bn);
      fma_frag<QT, R, NMAT>(acc, cur, xs + b * kXBlk);
      cur = nxt;
      b = bn;
      have = hn;
    }
  }

#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);

  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < a.rows) a.y[row] = EPI == EPI_ADD ? acc[0][r] + a.y[row] : acc[0][r];
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        const float g = acc[0][r], u = acc[1][r];
        if (row < a.rows) a.y[row] = u * (g / (1.0f + expf(-g)));
      }
    }
  } else if constexpr (EPI == EPI_QKV) {
    static_assert(R % 2 == 0, "QKV epilogue works on row pairs");
    if (lane == 0) {
      const int pos = *a.dpos;
      const int hd = a.head_dim;
      const float* cs = a.rope_cs + (size_t)pos * a.rope_dim;   // (rope_dim/2) pairs
#pragma unroll
      for (int r = 0; r < R; r += 2) {
        const int gr = row0 + r;
        if (gr >= a.rows) break;
        float v0 = acc[0][r], v1 = acc[0][r + 1];
        if (gr < a.qdim + a.kvdim) {   // q or k: rotate the (i, i+1) pair, tensor.c:250-273
          const int i = (gr < a.qdim ? gr : gr - a.qdim) % hd;
          if (i < a.rope_dim) {
            const float c = cs[i], s = cs[i + 1];
            const float r0 = v0 * c - v1 * s;
            const float r1 = v0 * s + v1 * c;
            v0 = r0;
            v1 = r1;
          }
        }
        if (gr < a.qdim) {
          a.y[gr] = v0;
          a.y[gr + 1] = v1;
        } else {
          const bool is_v = gr >= a.qdim + a.kvdim;
          const int kr = gr - a.qdim - (is_v ? a.kvdim : 0);
          if (a.kv_type == 0) {
            const int g = kr / hd, i = kr % hd;
            uint16_t* c = reinterpret_cast<uint16_t*>(is_v ? a.vcache : a.kcache);
            const size_t o = ((size_t)g * a.max_seq + pos) * hd + i;
            c[o] = f2h(v0);
            c[o + 1] = f2h(v1);
          } else {
            a.kv_f32[(is_v ? a.kvdim : 0) + kr] = v0;
            a.kv_f32[(is_v ? a.kvdim : 0) + kr + 1] = v1;
          }
        }
      }
    }
  } else if constexpr (EPI == EPI_LOGITS) {
    __shared__ bool s_last;
    if (lane == 0) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < a.rows) {
          a.y[row] = acc[0][r];
          if (beats(acc[0][r], row, bv, bi)) {
            bv = acc[0][r];
            bi = row;
          }
        }
      }
      wbest[wave] = make_float2(bv, __int_as_float(bi));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = wbest[0].x;
      int bi = __float_as_int(wbest[0].y);
      for (int w = 1; w < kGemvWaves; ++w) {
        const float v = wbest[w].x;
        const int i = __float_as_int(wbest[w].y);
        if (beats(v, i, bv, bi)) {
          bv = v;
          bi = i;
        }
      }
      st_agent(&a.part[blockIdx.x].x, bv);
      st_agent(&a.part[blockIdx.x].y, __int_as_float(bi));
      __threadfence();
      const unsigned prev = atomicAdd(a.counter, 1u);
      s_last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (s_last) {
      __threadfence();
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = threadIdx.x; i < (int)gridDim.x; i += kGemvThreads) {
        const float pv = ld_agent(&a.part[i].x);
        const int pi = __float_as_int(ld_agent(&a.part[i].y));
        if (beats(pv, pi, bv, bi)) {
          bv = pv;
          bi = pi;
        }
      }
      // workgroup reduction in index order is not needed: beats() is a
      // total order on (value desc, index asc), so any tree gives the same result
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (beats(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) wbest[wave] = make_float2(bv, __int_as_float(bi));
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int w = 1; w < kGemvWaves; ++w) {
          const float v = wbest[w].x;
          const int i = __float_as_int(wbest[w].y);
          if (beats(v, i, bv, bi)) {
            bv = v;
            bi = i;
          }
        }
        if (bi == 0x7fffffff) bi = 0;                 // every logit NaN
        if (isnan(ld_agent(a.y))) bi = 0;   // tensor.c:319-320 starts from x[0]
        *a.out_idx = bi;
        if (a.tokens) {
          const int pos = *a.dpos_mut;
          a.tokens[pos + 1] = bi;
          *a.dpos_mut = pos + 1;
        }
        st_agent_u(a.counter, 0u);
      }
    }
  }
}

// ------------------------------------------------------------ attention
// Single-query GQA attention (layer_scheduler.c:415-468) with the sequence
// split over gridDim.x workgroups (flash-decoding): workgroup (s, g) runs an
// online softmax over its slice of positions for the G query heads that
// share KV head g, staging 64-position K and V tiles in LDS, and the last
// workgroup of each KV head merges the partial (max, sum, output) triples.
template <int KVT>
struct KvElem;
template <>
struct KvElem<0> {
  using T = uint16_t;
  static __device__ __forceinline__ float get(T v, float) { return h2f(v); }
};
template <>
struct KvElem<1> {
  using T = int8_t;
  static __device__ __forceinline__ float get(T v, float s) { return (float)v * s; }
};

template <int HD, int G, int KVT>
__global__ void __launch_bounds__(256) k_attn(const AttnArgs a) {
  using E = typename KvElem<KVT>::T;
  constexpr int kT = 64;                         // positions per tile
  constexpr int kChunkBytes = 16;
  constexpr int kRowBytes = HD * (int)sizeof(E);
  constexpr int kCpr = kRowBytes / kChunkBytes;  // 16-byte chunks per row
  constexpr int kEpc = kChunkBytes / (int)sizeof(E);
  constexpr int kStride = HD + kEpc;             // padded LDS row, elements
  // score phase: NG head groups x SPLIT threads per (position, head)
  constexpr int kNG = G >= 4 ? 4 : G;
  constexpr int kHPT = G >= 4 ? G / 4 : 1;
  constexpr int kSplit = 4 / kNG;
  constexpr int kCps = kCpr / kSplit;            // chunks per split
  // value phase: OPT outputs per thread, TPO threads (position phases) per output
  constexpr int kNPV = G * HD;
  constexpr int kOPT = kNPV >= 256 ? kNPV / 256 : 1;
  constexpr int kTPO = kNPV >= 256 ? 1 : 256 / kNPV;
  constexpr int kOThreads = 256 / kTPO;

  __shared__ __attribute__((aligned(16))) E kt[kT * kStride];
  __shared__ __attribute__((aligned(16))) E vt[kT * kStride];
  __shared__ __attribute__((aligned(16))) float qsh[G][HD + 4];
  __shared__ float st[G][kT];
  __shared__ float ksc[kT], vsc[kT];
  __shared__ float m_run[G], l_run[G], corr[G];
  __shared__ float red[kTPO > 1 ? kTPO * 256 : 1];
  __shared__ bool s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kvh = blockIdx.y;
  const int ctx = a.dpos ? *a.dpos + 1 : a.seq_len;
  int chunk = (ctx + a.ns - 1) / a.ns;
  if (chunk < kT) chunk = kT;
  const int active = (ctx + chunk - 1) / chunk;
  if ((int)blockIdx.x >= active) return;
  const int t0 = blockIdx.x * chunk;
  const int t1 = min(ctx, t0 + chunk);

  const size_t head_base = (size_t)kvh * a.max_seq;
  const E* kbase = reinterpret_cast<const E*>(a.kc) + head_base * HD;
  const E* vbase = reinterpret_cast<const E*>(a.vc) + head_base * HD;

  for (int i = tid; i < G * HD; i += 256) qsh[i / HD][i % HD] = a.q[(size_t)kvh * G * HD + i];
  if (tid < G) {
    m_run[tid] = -INFINITY;
    l_run[tid] = 0.f;
  }

  // value-phase ownership
  const int vphase = tid / kOThreads;
  const int o0 = (tid % kOThreads) * kOPT;
  const int vg = o0 / HD, vd = o0 % HD;
  float acc[kOPT];
#pragma unroll
  for (int j = 0; j < kOPT; ++j) acc[j] = 0.f;

  // score-phase ownership
  const int sp = (tid / kSplit) % kT;        // position in tile
  const int sg = tid / (kT * kSplit);        // head group
  const int ss = tid % kSplit;               // split index

  for (int tile = t0; tile < t1; tile += kT) {
    const int nv = min(kT, t1 - tile);
    __syncthreads();   // previous tile fully consumed (and q/m/l initialised)
    for (int c = tid; c < nv * kCpr; c += 256) {
      const int row = c / kCpr, part = c % kCpr;
      const size_t go = (size_t)(tile + row) * HD + part * kEpc;
      *reinterpret_cast<uint4*>(kt + row * kStride + part * kEpc) =
          *reinterpret_cast<const uint4*>(kbase + go);
      *reinterpret_cast<uint4*>(vt + row * kStride + part * kEpc) =
          *reinterpret_cast<const uint4*>(vbase + go);
    }
    if constexpr (KVT == 1) {
      if (tid < nv) {
        ksc[tid] = a.ks[tile + tid];
        vsc[tid] = a.vs[tile + tid];
      }
    }
    __syncthreads();

    // scores s[g][p] = (q_g . k_p) * scale
#pragma unroll
    for (int hh = 0; hh < kHPT; ++hh) {
      const int g = sg * kHPT + hh;
      float dot = 0.f;
      if (sp < nv) {
        const float kscale = KVT == 1 ? ksc[sp] : 1.f;
        const E* krow = kt + sp * kStride;
#pragma unroll
        for (int cc = 0; cc < kCps; ++cc) {
          const int chunk_i = cc * kSplit + ss;
          const E* kp = krow + chunk_i * kEpc;
          const float* qp = &qsh[g][chunk_i * kEpc];
#pragma unroll
          for (int e = 0; e < kEpc; ++e) dot = fmaf(qp[e], KvElem<KVT>::get(kp[e], kscale), dot);
        }
      }
      if constexpr (kSplit >= 2) dot += __shfl_xor(dot, 1, kWave);
      if constexpr (kSplit >= 4) dot += __shfl_xor(dot, 2, kWave);
      if (ss == 0) st[g][sp] = sp < nv ? dot * a.scale : -INFINITY;
    }
    __syncthreads();

    // online softmax update, one wave per head
    for (int g = wave; g < G; g += 4) {
      const float sv = st[g][lane];
      const float mt = wave_max(sv);
      const float mo = m_run[g];
      const float mn = fmaxf(mo, mt);
      const float p = expf(sv - mn);
      st[g][lane] = p;
      const float lt = wave_sum(p);
      if (lane == 0) {
        const float c = expf(mo - mn);
        corr[g] = c;
        l_run[g] = l_run[g] * c + lt;
        m_run[g] = mn;
      }
    }
    __syncthreads();

    // acc = acc * corr + sum_p p[g][p] * v[p]
    const float c = corr[vg];
#pragma unroll
    for (int j = 0; j < kOPT; ++j) acc[j] *= c;
    for (int p = vphase; p < nv; p += kTPO) {
      const float w = st[vg][p];
      const float vscale = KVT == 1 ? vsc[p] : 1.f;
      const E* vrow = vt + p * kStride + vd;
#pragma unroll
      for (int j = 0; j < kOPT; ++j) acc[j] = fmaf(w, KvElem<KVT>::get(vrow[j], vscale), acc[j]);
    }
  }

  // merge the position phases
  if constexpr (kTPO > 1) {
    __syncthreads();
    red[vphase * kOThreads + (tid % kOThreads)] = acc[0];
    __syncthreads();
    if (vphase == 0) {
      float s = acc[0];
      for (int ph = 1; ph < kTPO; ++ph) s += red[ph * kOThreads + tid];
      acc[0] = s;
    }
  }
  // partial results of this split
  float* po = a.part_o + (((size_t)kvh * a.ns + blockIdx.x) * G) * HD;
  float* pml = a.part_ml + (((size_t)kvh * a.ns + blockIdx.x) * G) * 2;
  if (vphase == 0) {
#pragma unroll
    for (int j = 0; j < kOPT; ++j) st_agent(&po[vg * HD + vd + j], acc[j]);
  }
  if (tid < G) {
    st_agent(&pml[tid * 2], m_run[tid]);
    st_agent(&pml[tid * 2 + 1], l_run[tid]);
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(a.counter + kvh, 1u) == (unsigned)active - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // merge splits: out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M)
  float* wts = &st[0][0];   // reuse: active*G <= 64*G weights needed; st holds G*64
  for (int i = tid; i < G; i += 256) {
    const float* ml = a.part_ml + ((size_t)kvh * a.ns * G) * 2;
    float M = -INFINITY;
    for (int s = 0; s < active; ++s) M = fmaxf(M, ld_agent(ml + (s * G + i) * 2));
    float L = 0.f;
    for (int s = 0; s < active; ++s)
      L += ld_agent(ml + (s * G + i) * 2 + 1) * expf(ld_agent(ml + (s * G + i) * 2) - M);
    m_run[i] = M;
    l_run[i] = 1.0f / L;
  }
  __syncthreads();
  for (int o = tid; o < G * HD; o += 256) {
    const int g = o / HD, d = o % HD;
    const float* ml = a.part_ml + ((size_t)kvh * a.ns * G) * 2;
    const float* pob = a.part_o + ((size_t)kvh * a.ns * G) * HD;
    float s = 0.f;
    for (int sI = 0; sI < active; ++sI)
      s = fmaf(ld_agent(pob + ((size_t)sI * G + g) * HD + d),
               expf(ld_agent(ml + (sI * G + g) * 2) - m_run[g]), s);
    a.out[((size_t)kvh * G + g) * HD + d] = s * l_run[g];
  }
  (void)wts;
  if (tid == 0) st_agent_u(a.counter + kvh, 0u);
}

// ------------------------------------------------------------ small kernels
template <int QT>
__global__ void k_pack(const uint8_t* __restrict__ src, uint8_t* __restrict__ qs,
                       uint16_t* __restrict__ ds, int64_t nblocks, int64_t blk_offset) {
  constexpr int kQB = QTraits<QT>::kQB, kBytes = QTraits<QT>::kGgufBytes;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nblocks) return;
  const uint8_t* s = src + i * kBytes;
  ds[blk_offset + i] = (uint16_t)(s[0] | (s[1] << 8));
  uint4* dst = reinterpret_cast<uint4*>(qs + (blk_offset + i) * kQB);
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
    const size_t bi = (size_t)tok * nb + b;
    const float d = h2f(t.ds[bi]);
    const uint8_t* q = t.qs + bi * kQB;
    float* o = out + b * 32;
    if constexpr (QT == 2) {
      for (int i = 0; i < 16; ++i) {
        const uint8_t v = q[i];
        o[i] = d * (float)((int)(v & 0xF) - 8);
        o[i + 16] = d * (float)((int)(v >> 4) - 8);
      }
    } else {
      for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)q[i];
    }
  }
}

__global__ void k_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
  __shared__ float red[4];
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(x[i], x[i], ss);
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += 256) out[i] = x[i] * scale * w[i];
}

// tensor.c:220-275 with the per-pair (cos, sin) precomputed on the host
__global__ void k_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int rope_dim,
                       const float* cs, int is_neox) {
  const int half = rope_dim / 2;
  const int total = (n_heads + n_kv_heads) * half;
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    const int h = t / half, p = t % half;
    float* v = h < n_heads ? q + h * head_dim : k + (h - n_heads) * head_dim;
    const int i0 = is_neox ? p : 2 * p;
    const int i1 = is_neox ? p + half : 2 * p + 1;
    const float c = cs[2 * p], s = cs[2 * p + 1];
    const float a = v[i0], b = v[i1];
    v[i0] = a * c - b * s;
    v[i1] = a * s + b * c;
  }
}

// KV append: fp16 (one thread per element) or the int8 absmax encoding of
// layer_scheduler.c:101-118 (one workgroup each for K and V).
__global__ void k_kv_append(void* kc, void* vc, float* ksc, float* vsc, const float* k,
                            const float* v, int n_kv_heads, int head_dim, int max_seq,
                            const int* dpos, int pos_arg, int kv_type) {
  const int pos = dpos ? *dpos : pos_arg;
  const int kvdim = n_kv_heads * head_dim;
  if (kv_type == 0) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < 2 * kvdim; i += gridDim.x * blockDim.x) {
      const bool is_v = i >= kvdim;
      const int e = is_v ? i - kvdim : i;
      const int g = e / head_dim, d = e % head_dim;
      uint16_t* c = reinterpret_cast<uint16_t*>(is_v ? vc : kc);
      c[((size_t)g * max_seq + pos) * head_dim + d] = f2h(is_v ? v[e] : k[e]);
    }
    return;
  }
  __shared__ float red[4];
  const bool is_v = blockIdx.x == 1;
  const float* src = is_v ? v : k;
  float m = 0.f;
  for (int i = threadIdx.x; i < kvdim; i += 256) m = fmaxf(m, fabsf(src[i]));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax / 127.0f;
  const float inv = s > 0.0f ? 1.0f / s : 0.0f;
  int8_t* c = reinterpret_cast<int8_t*>(is_v ? vc : kc);
  for (int i = threadIdx.x; i < kvdim; i += 256) {
    const int g = i / head_dim, d = i % head_dim;
    c[((size_t)g * max_seq + pos) * head_dim + d] = (int8_t)roundf(src[i] * inv);
  }
  if (threadIdx.x == 0) (is_v ? vsc : ksc)[pos] = s;
}

__global__ void k_swiglu(float* out, const float* g, const float* u, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float gv = g[i];
    out[i] = u[i] * (gv / (1.0f + expf(-gv)));
  }
}

__global__ void k_argmax(int* out, const float* x, int n, float2* part, unsigned* counter) {
  __shared__ float2 wb[4];
  __shared__ bool s_last;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    if (beats(x[i], i, bv, bi)) {
      bv = x[i];
      bi = i;
    }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (beats(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (beats(wb[w].x, __float_as_int(wb[w].y), bv, bi)) {
        bv = wb[w].x;
        bi = __float_as_int(wb[w].y);
      }
    st_agent(&part[blockIdx.x].x, bv);
    st_agent(&part[blockIdx.x].y, __int_as_float(bi));
    __threadfence();
    s_last = atomicAdd(counter, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last || threadIdx.x != 0) return;
  __threadfence();
  bv = -INFINITY;
  bi = 0x7fffffff;
  for (unsigned i = 0; i < gridDim.x; ++i) {
    const float pv = ld_agent(&part[i].x);
    const int pi = __float_as_int(ld_agent(&part[i].y));
    if (beats(pv, pi, bv, bi)) {
      bv = pv;
      bi = pi;
    }
  }
  if (bi == 0x7fffffff || isnan(x[0])) bi = 0;
  *out = bi;
  st_agent_u(counter, 0u);
}

__global__ void k_set_state(int* dpos, int* tokens, int pos, int token) {
  *dpos = pos;
  tokens[pos] = token;
}

__global__ void k_advance(int* dpos) { *dpos += 1; }

template <int QT, int R, int NMAT, int EPI>
hipError_t launch_gemv_t(const GemvArgs& a, hipStream_t s) {
  const int rows_per_wg = kGemvWaves * R;
  const int grid = (a.rows + rows_per_wg - 1) / rows_per_wg;
  const size_t lds = (size_t)a.chunk_blocks * kXBlk * sizeof(float);
  hipLaunchKernelGGL((k_gemv<QT, R, NMAT, EPI>), dim3(grid), dim3(kGemvThreads), lds, s, a);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_gemv_q(int epi, const GemvArgs& a, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: return launch_gemv_t<QT, 4, 1, EPI_STORE>(a, s);
    case EPI_ADD: return launch_gemv_t<QT, 4, 1, EPI_ADD>(a, s);
    case EPI_SWIGLU: return launch_gemv_t<QT, 2, 2, EPI_SWIGLU>(a, s);
    case EPI_QKV: return launch_gemv_t<QT, 4, 1, EPI_QKV>(a, s);
    case EPI_LOGITS: return launch_gemv_t<QT, 4, 1, EPI_LOGITS>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <int HD, int G>
hipError_t launch_attn_t(int kv_type, const AttnArgs& a, hipStream_t s) {
  const dim3 grid(a.ns, a.n_kv_heads);
  if (kv_type == 0)
    hipLaunchKernelGGL((k_attn<HD, G, 0>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn<HD, G, 1>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(int group, int kv_type, const AttnArgs& a, hipStream_t s) {
  switch (group) {
    case 1: return launch_attn_t<HD, 1>(kv_type, a, s);
    case 2: return launch_attn_t<HD, 2>(kv_type, a, s);
    case 4: return launch_attn_t<HD, 4>(kv_type, a, s);
    case 8: return launch_attn_t<HD, 8>(kv_type, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int gemv_rows_per_wave(int epi) { return epi == EPI_SWIGLU ? 2 : 4; }

int gemv_grid(int epi, int rows) {
  const int per = kGemvWaves * gemv_rows_per_wave(epi);
  return (rows + per - 1) / per;
}

hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t s) {
  if (a.type == 2) return launch_gemv_q<2>(epi, a, s);
  if (a.type == 8) return launch_gemv_q<8>(epi, a, s);
  return hipErrorInvalidValue;
}

bool attention_supported(int head_dim, int group) {
  return (head_dim == 64 || head_dim == 128) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

hipError_t launch_attention(int head_dim, int group, int kv_type, const AttnArgs& a,
                            hipStream_t s) {
  if (head_dim == 64) return launch_attn_hd<64>(group, kv_type, a, s);
  if (head_dim == 128) return launch_attn_hd<128>(group, kv_type, a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_pack(int type, const uint8_t* src, uint8_t* qs, uint16_t* ds, int64_t nblocks,
                       int64_t blk_offset, hipStream_t s) {
  const int64_t grid = (nblocks + 255) / 256;
  if (type == 2)
    hipLaunchKernelGGL(k_pack<2>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks,
                       blk_offset);
  else if (type == 8)
    hipLaunchKernelGGL(k_pack<8>, dim3((unsigned)grid), dim3(256), 0, s, src, qs, ds, nblocks,
                       blk_offset);
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

hipError_t launch_rmsnorm(float* out, const float* x, const float* w, int n, float eps,
                          hipStream_t s) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(256), 0, s, out, x, w, n, eps);
  return hipGetLastError();
}

hipError_t launch_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim,
                       int rope_dim, const float* cs_row, int is_neox, hipStream_t s) {
  const int total = (n_heads + n_kv_heads) * (rope_dim / 2);
  const int grid = (total + 255) / 256;
  hipLaunchKernelGGL(k_rope, dim3(grid > 0 ? grid : 1), dim3(256), 0, s, q, k, n_heads, n_kv_heads,
                     head_dim, rope_dim, cs_row, is_neox);
  return hipGetLastError();
}

hipError_t launch_kv_append(void* kc, void* vc, float* ksc, float* vsc, const float* k,
                            const float* v, int n_kv_heads, int head_dim, int max_seq,
                            const int* dpos, int pos, int kv_type, hipStream_t s) {
  const int grid = kv_type == 0 ? (2 * n_kv_heads * head_dim + 255) / 256 : 2;
  hipLaunchKernelGGL(k_kv_append, dim3(grid), dim3(256), 0, s, kc, vc, ksc, vsc, k, v, n_kv_heads,
                     head_dim, max_seq, dpos, pos, kv_type);
  return hipGetLastError();
}

hipError_t launch_swiglu(float* out, const float* g, const float* u, int n, hipStream_t s) {
  const int grid = (n + 255) / 256;
  hipLaunchKernelGGL(k_swiglu, dim3(grid > 0 ? grid : 1), dim3(256), 0, s, out, g, u, n);
  return hipGetLastError();
}

hipError_t launch_argmax(int* out, const float* x, int n, float2* part, unsigned* counter,
                         hipStream_t s) {
  int grid = (n + 255) / 256;
  if (grid > kArgmaxMaxBlocks) grid = kArgmaxMaxBlocks;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, s, out, x, n, part, counter);
  return hipGetLastError();
}

hipError_t launch_set_state(int* dpos, int* tokens, int pos, int token, hipStream_t s) {
  hipLaunchKernelGGL(k_set_state, dim3(1), dim3(1), 0, s, dpos, tokens, pos, token);
  return hipGetLastError();
}

hipError_t launch_advance(int* dpos, hipStream_t s) {
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, s, dpos);
  return hipGetLastError();
}

}  // namespace ssk
