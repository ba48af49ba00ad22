// ss_kernels.hip - attention and the small per-token kernels for gfx950.
//
// Split results (attention splits, per-workgroup argmax candidates) are
// merged by a following small kernel, so no workgroup hands data to another
// workgroup of the same launch and none needs a device-scope fence.

#include <math.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

// ------------------------------------------------------------ attention
// Single-query GQA attention (layer_scheduler.c:415-468) with the sequence
// split over gridDim.x workgroups (flash-decoding): workgroup (s, g) runs an
// online softmax over its slice of positions for the G query heads that
// share KV head g, staging 64-position K and V tiles in LDS, and writes a
// partial (max, sum, unnormalised output); k_attn_merge combines them.
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

__device__ __forceinline__ void attn_split(const AttnArgs& a, int& ctx, int& chunk, int& active) {
  ctx = a.dpos ? *a.dpos + 1 : a.seq_len;
  chunk = (ctx + a.ns - 1) / a.ns;
  if (chunk < 64) chunk = 64;
  active = (ctx + chunk - 1) / chunk;
}

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

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kvh = blockIdx.y;
  int ctx, chunk, active;
  attn_split(a, ctx, chunk, active);
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
  float* po = a.part_o + (((size_t)kvh * a.ns + blockIdx.x) * G) * HD;
  float* pml = a.part_ml + (((size_t)kvh * a.ns + blockIdx.x) * G) * 2;
  if (vphase == 0) {
#pragma unroll
    for (int j = 0; j < kOPT; ++j) po[vg * HD + vd + j] = acc[j];
  }
  if (tid < G) {
    pml[tid * 2] = m_run[tid];
    pml[tid * 2 + 1] = l_run[tid];
  }
}

// out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M) over the active splits
template <int HD, int G>
__global__ void __launch_bounds__(256) k_attn_merge(const AttnArgs a) {
  __shared__ float mg[G], lg[G];
  __shared__ float wts[64 * G];
  const int tid = threadIdx.x;
  const int kvh = blockIdx.x;
  int ctx, chunk, active;
  attn_split(a, ctx, chunk, active);
  const float* ml = a.part_ml + ((size_t)kvh * a.ns * G) * 2;
  const float* pob = a.part_o + ((size_t)kvh * a.ns * G) * HD;
  for (int i = tid; i < G; i += 256) {
    float M = -INFINITY;
    for (int s = 0; s < active; ++s) M = fmaxf(M, ml[(s * G + i) * 2]);
    float L = 0.f;
    for (int s = 0; s < active; ++s) L += ml[(s * G + i) * 2 + 1] * expf(ml[(s * G + i) * 2] - M);
    mg[i] = M;
    lg[i] = 1.0f / L;
  }
  __syncthreads();
  for (int i = tid; i < active * G; i += 256) {
    const int g = i % G;
    wts[i] = expf(ml[i * 2] - mg[g]) * lg[g];
  }
  __syncthreads();
  for (int o = tid; o < G * HD; o += 256) {
    const int g = o / HD, d = o % HD;
    float s = 0.f;
    for (int si = 0; si < active; ++si) s = fmaf(pob[((size_t)si * G + g) * HD + d], wts[si * G + g], s);
    a.out[((size_t)kvh * G + g) * HD + d] = s;
  }
}

// ------------------------------------------------------------ small kernels
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

// per-workgroup first-maximum candidates; k_argmax_merge finishes
__global__ void k_argmax_part(const float* x, int n, float2* part) {
  __shared__ float2 wb[4];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    if (beats(x[i], i, bv, bi)) {
      bv = x[i];
      bi = i;
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
  part[blockIdx.x] = make_float2(bv, __int_as_float(bi));
}

__global__ void k_set_state(int* dpos, int* tokens, int pos, int token) {
  *dpos = pos;
  tokens[pos] = token;
}

__global__ void k_advance(int* dpos) { *dpos += 1; }

// ------------------------------------------------------------ launchers
template <int HD, int G>
hipError_t launch_attn_t(int kv_type, const AttnArgs& a, hipStream_t s) {
  const dim3 grid(a.ns, a.n_kv_heads);
  if (kv_type == 0)
    hipLaunchKernelGGL((k_attn<HD, G, 0>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((k_attn<HD, G, 1>), grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_attn_merge<HD, G>), dim3(a.n_kv_heads), dim3(256), 0, s, a);
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

bool attention_supported(int head_dim, int group) {
  return (head_dim == 64 || head_dim == 128) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

hipError_t launch_attention(int head_dim, int group, int kv_type, const AttnArgs& a,
                            hipStream_t s) {
  if (a.ns > 64) return hipErrorInvalidValue;   // k_attn_merge holds 64 split weights per head
  if (head_dim == 64) return launch_attn_hd<64>(group, kv_type, a, s);
  if (head_dim == 128) return launch_attn_hd<128>(group, kv_type, a, s);
  return hipErrorInvalidValue;
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

hipError_t launch_argmax(int* out, const float* x, int n, float2* part, hipStream_t s) {
  int grid = (n + 255) / 256;
  if (grid > kArgmaxMaxBlocks) grid = kArgmaxMaxBlocks;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(k_argmax_part, dim3(grid), dim3(256), 0, s, x, n, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_argmax_merge(part, grid, x, out, nullptr, nullptr, s);
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
