// ss_sample.hip - non-greedy sampling of the next token on the device.
//
// k_sample follows ss_sample (tensor.c:363-451) step by step over the logits
// the LM head left in HBM, in one workgroup:
//   1. x_i = logit_i / T (NaN logits become -FLT_MAX), softmax (tensor.c:154-173);
//   2. top-k: probabilities below the k-th largest (NaN counted as 0 for the
//      ranking, as the reference's sort key) become 0;
//   3. top-p: going down the probabilities in descending order, the cutoff is
//      the probability at which the running sum of the positive ones first
//      reaches top_p; probabilities below it become 0;
//   4. renormalise, draw r from xorshift64 (state passed in, advanced state
//      written back), return the first index whose cumulative probability
//      exceeds r (vocab - 1 when none does).
// The reference sorts all probabilities (qsort) and sums sequentially in
// fp32. Here the k-th largest value and the top-p cutoff come from radix
// selections over the float bit patterns (non-negative floats order like
// their bits), 8 bits per pass with LDS histograms; sums are exact fixed
// point (each probability truncated to a multiple of 2^-52) in uint64, so
// they do not depend on the order the atomics land in. The cumulative
// search is a two-level scan: per-thread chunk sums, a workgroup scan, then
// one sequential walk inside the chunk that holds r. The index differs from
// the reference's only when r lies within the reference's fp32 rounding of a
// cumulative boundary.

#include <float.h>
#include <math.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr double kFix = 4503599627370496.0;   // 2^52: probabilities (each <= 1, sums <= ~1)
constexpr double kFixE = 1099511627776.0;     // 2^40: softmax terms (each <= 1, up to 2^18 of them)

// a probability as fixed point; NaN and non-positive values count 0, values
// are clamped to 2 (a probability never exceeds 1 + rounding)
__device__ __forceinline__ uint64_t fix(float p) {
  return p > 0.f ? (uint64_t)((double)fminf(p, 2.0f) * kFix) : 0ull;
}
// sort key of tensor.c:384-385 (NaN ranks as 0)
__device__ __forceinline__ uint32_t key(float p) { return __float_as_uint(p == p ? p : 0.f); }

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

struct Shared {
  float f[kWaves];
  uint64_t u[kWaves];
  uint32_t hist[256];
  uint64_t hsum[256];
  uint32_t sel, kk;
  int first;
  uint64_t above;
  int done;
};

__device__ float block_max(float v, Shared& sh) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = sh.f[0];
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, sh.f[w]);
  return m;
}

__device__ uint64_t block_sum(uint64_t v, Shared& sh) {
  v = wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.u[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t t = 0;
  for (int w = 0; w < kWaves; ++w) t += sh.u[w];
  return t;
}

__device__ int block_min_i(int v, Shared& sh) {
  __syncthreads();
  if (threadIdx.x == 0) sh.first = 0x7fffffff;
  __syncthreads();
  atomicMin(&sh.first, v);
  __syncthreads();
  return sh.first;
}

// The k-th largest key (1 <= k <= V), MSB first.
__device__ uint32_t kth_largest(const float* p, int V, int k, Shared& sh) {
  uint32_t prefix = 0, mask = 0;
  uint32_t kk = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += kThreads) sh.hist[b] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += kThreads) {
      const uint32_t u = key(p[i]);
      if ((u & mask) == prefix) atomicAdd(&sh.hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t acc = 0, b = 255;
      for (;; --b) {
        if (acc + sh.hist[b] >= kk || b == 0) break;
        acc += sh.hist[b];
      }
      sh.sel = b;
      sh.kk = kk - acc;
    }
    __syncthreads();
    prefix |= sh.sel << shift;
    mask |= 255u << shift;
    kk = sh.kk;
    __syncthreads();
  }
  return prefix;
}

// The top-p cutoff: the largest positive value v with sum(p >= v, p > 0)
// reaching target (fixed point), or 0 when the positive values never do.
__device__ float top_p_cutoff(const float* p, int V, uint64_t target, Shared& sh) {
  uint32_t prefix = 0, mask = 0;
  uint64_t above = 0;   // sum of the values whose key is above the current prefix range
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += kThreads) sh.hsum[b] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += kThreads) {
      const float v = p[i];
      if (!(v > 0.f)) continue;
      const uint32_t u = __float_as_uint(v);
      if ((u & mask) == prefix) atomicAdd(reinterpret_cast<unsigned long long*>(&sh.hsum[(u >> shift) & 255u]),
                                          (unsigned long long)fix(v));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int b = 255;
      uint64_t acc = above;
      for (; b >= 0; --b) {
        if (acc + sh.hsum[b] >= target) break;
        acc += sh.hsum[b];
      }
      sh.done = b < 0;
      sh.sel = b < 0 ? 0u : (uint32_t)b;
      sh.above = acc;
    }
    __syncthreads();
    if (sh.done) return 0.f;   // uniform: the positive values sum to less than top_p
    prefix |= sh.sel << shift;
    mask |= 255u << shift;
    above = sh.above;
    __syncthreads();
  }
  return __uint_as_float(prefix);
}

__global__ void __launch_bounds__(kThreads) k_sample(const SampleArgs a) {
  __shared__ Shared sh;
  const int V = a.V, tid = threadIdx.x;
  float* p = a.probs;

  // 1. temperature and softmax (tensor.c:374-381, 154-173)
  float mx = -FLT_MAX;
  for (int i = tid; i < V; i += kThreads) {
    const float l = a.logits[i];
    const float x = l != l ? -FLT_MAX : l / a.temperature;
    p[i] = x;
    mx = fmaxf(mx, x);
  }
  mx = block_max(mx, sh);
  uint64_t s = 0;
  int nan_at = 0x7fffffff;
  for (int i = tid; i < V; i += kThreads) {
    const float e = expf(p[i] - mx);
    p[i] = e;
    s += e > 0.f ? (uint64_t)((double)e * kFixE) : 0ull;   // e <= 1
    if (e != e) nan_at = min(nan_at, i);
  }
  const bool nan_sum = block_min_i(nan_at, sh) != 0x7fffffff;
  const uint64_t esum = block_sum(s, sh);
  const float inv = nan_sum ? NAN : 1.0f / (float)((double)esum / kFixE);
  for (int i = tid; i < V; i += kThreads) p[i] *= inv;
  __syncthreads();

  // 2. top-k (tensor.c:390-396)
  if (a.top_k > 0 && a.top_k < V) {
    const float th = __uint_as_float(kth_largest(p, V, a.top_k, sh));
    for (int i = tid; i < V; i += kThreads)
      if (p[i] < th) p[i] = 0.f;
    __syncthreads();
  }

  // 3. top-p (tensor.c:398-417)
  if (a.top_p > 0.f && a.top_p < 1.0f) {
    const uint64_t target = (uint64_t)((double)a.top_p * kFix);
    const float cutoff = top_p_cutoff(p, V, target, sh);
    for (int i = tid; i < V; i += kThreads)
      if (p[i] < cutoff) p[i] = 0.f;
    __syncthreads();
  }

  // 4. renormalise (tensor.c:423-429); a NaN probability makes the sum NaN
  nan_at = 0x7fffffff;
  s = 0;
  for (int i = tid; i < V; i += kThreads) {
    const float v = p[i];
    s += fix(v);
    if (v != v) nan_at = min(nan_at, i);
  }
  const int first_nan = block_min_i(nan_at, sh);
  const uint64_t psum = block_sum(s, sh);
  if (first_nan == 0x7fffffff && psum > 0) {
    const float pinv = 1.0f / (float)((double)psum / kFix);
    for (int i = tid; i < V; i += kThreads) p[i] *= pinv;
  }
  __syncthreads();

  // 5. draw (tensor.c:341-343, 431-442): first i with r < cdf_i, i before any
  // NaN (a NaN term makes every later comparison false)
  uint64_t st = a.rng;
  st ^= st << 13;
  st ^= st >> 7;
  st ^= st << 17;
  const float r = (float)(st >> 11) / (float)(1ull << 53);
  const uint64_t rf = (uint64_t)((double)r * kFix);
  const int C = (V + kThreads - 1) / kThreads;   // contiguous chunk per thread
  const int i0 = min(tid * C, V), i1 = min(i0 + C, V);
  uint64_t cs = 0;
  for (int i = i0; i < i1; ++i) cs += fix(p[i]);
  // exclusive scan of the chunk sums over the workgroup
  uint64_t incl = cs;
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t o = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += o;
  }
  __syncthreads();
  if (lane == kWave - 1) sh.u[wave] = incl;
  __syncthreads();
  uint64_t base = incl - cs;
  for (int w = 0; w < wave; ++w) base += sh.u[w];
  int found = 0x7fffffff;
  if (i0 < i1 && rf < base + cs) {
    uint64_t c = base;
    for (int i = i0; i < i1; ++i) {
      c += fix(p[i]);
      if (rf < c) {
        found = i;
        break;
      }
    }
  }
  found = block_min_i(found, sh);
  if (tid != 0) return;
  const int idx = found < first_nan && found < V ? found : V - 1;
  *a.out = idx;
  *a.rng_out = st;
  if (a.tokens) {
    const int pos = *a.dpos;
    a.tokens[pos + 1] = idx;
    *a.dpos = pos + 1;
  }
}

}  // namespace

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
  if (a.V <= 0 || !a.logits || !a.probs || !a.out || !a.rng_out || !(a.temperature > 0.f) ||
      (a.tokens && !a.dpos))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace ssk
