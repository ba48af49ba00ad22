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

#include <hip/hip_runtime.h>
#include <math.h>

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
__global__ void __launch_bounds__(256) k_sumsq(const float* __restrict__ x, int cols, float* __restrict__ ssq) {
  __shared__ float red[4];
  const float* xt = x + (size_t)blockIdx.x * cols;
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
    const float scale = a.ssq ? 1.0f / sqrtf(a.ssq[t] / (float)a.cols + a.eps) : 1.0f;
    float* yp = a.y + (size_t)t * a.ldy + r0;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = acc[0][tt][i] * scale;
      if constexpr (EPI == EPI_SWIGLU) {
        const float u = acc[NMAT - 1][tt][i] * scale;
        v[i] = u * (x0 / (1.0f + expf(-x0)));   // layer_scheduler.c:540-547
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
}

template <int QT, int NMAT, int EPI>
hipError_t launch_gemm_t(const GemmArgs& a, hipStream_t s) {
  const int ngroups = (a.rows + kRG - 1) / kRG;
  const dim3 grid((ngroups + kGemmWaves - 1) / kGemmWaves, (a.T + kGemmTok - 1) / kGemmTok);
  hipLaunchKernelGGL((k_gemm<QT, NMAT, EPI>), grid, dim3(kGemmWaves * 64), 0, s, a);
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

}  // namespace

hipError_t launch_sumsq(const float* x, int cols, int T, float* ssq, hipStream_t s) {
  if (T <= 0 || cols <= 0 || cols % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sumsq, dim3(T), dim3(256), 0, s, x, cols, ssq);
  return hipGetLastError();
}

hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.rows <= 0 || a.cols <= 0 || a.cols % 32 || a.ldy < a.rows || a.ldx < a.cols)
    return hipErrorInvalidValue;
  if (a.type == 2) return launch_gemm_q<2>(epi, a, s);
  if (a.type == 8) return launch_gemm_q<8>(epi, a, s);
  return hipErrorInvalidValue;
}

}  // namespace ssk
