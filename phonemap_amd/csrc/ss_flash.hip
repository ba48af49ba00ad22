// ss_flash.hip - causal attention of a prompt's rows on MFMA (gfx950).
//
// The reference evaluates a prompt token by token, each token attending to
// positions 0..its own over the fp16 cache (layer_scheduler.c:415-468, called
// per token from ss_scheduler_prefill, :681-803). Here the tokens of a prompt
// chunk attend together, one workgroup per 64 query rows of one KV head
// (row r: token z0 + r / G, head r % G), on v_mfma_f32_16x16x32_f16.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (checked on the device by the
// prompt products): lane l supplies A[l%16][8(l/16) + i] and B[8(l/16) + i][l%16],
// i = 0..7, and receives D[4(l/16) + i][l%16], i = 0..3.
//
// Each wave owns 16 query rows and computes transposed tiles: S^T = K Q^T
// (A = 16 keys of K, B = Q^T), so lane (n, kq) receives the scores of query
// row n, and O^T = V^T P^T (A = V^T, B = P^T), whose B operand is exactly
// the scores' D registers once the keys of S^T tile t are ordered
// key(t, r) = 8(r / 4) + 4t + r % 4: lane (n, kq) then holds keys 8kq + j,
// j = 0..7, of query row n, the B layout. Softmax statistics of a row live in
// the 4 lanes n, n+16, n+32, n+48 (two shuffles per reduction).
//
// Precision: K and V are fp16 in the cache (exact MFMA operands). q is
// scaled per row by a power of two (its largest magnitude to [2^13, 2^14))
// and split into two fp16 parts, hi + lo = q to 2^-22; P (in [0, 1], times
// 2^12) is split the same way; each product is two MFMAs accumulating in
// fp32. The softmax is the online form (running max and sum per row) in fp32.
//
// Staging, per 64-key block, double buffered: K rows go to LDS by direct
// global-to-LDS loads (16-byte chunk c of key k at slot c ^ kswz(k) of its
// row); V is loaded into registers and written to LDS transposed (V^T rows
// of 64 keys, 8-key chunk c of row d at slot c ^ (d % 8)). Both swizzles
// spread one MFMA operand read over all banks.

#include <hip/hip_runtime.h>
#include <math.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

constexpr int kFWaves = 4;               // waves per workgroup, 16 query rows each
constexpr int kFRows = 16 * kFWaves;     // query rows per workgroup
// keys per block: 64, or 32 at head_dim 256 (the K and V^T tiles stay 64 KB)
__host__ __device__ constexpr int flash_keys(int hd) { return hd == 256 ? 32 : 64; }
constexpr float kPScale = 4096.0f;       // P is split as P * 2^12

// K row slot swizzle: the 16 keys of one S^T operand read (8(r/4) + 4t + r%4)
// take 8 distinct values, two keys each.
__device__ __forceinline__ int kswz(int key) { return (key & 3) | ((key >> 1) & 4); }

__device__ __forceinline__ float max4(float v) {   // over lanes n, n+16, n+32, n+48
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float sum4(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}
__device__ __forceinline__ int wave_max_int(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
  return v;
}

// hi + lo = v (to 2^-22 of |v| for normal values) as two fp16 vectors
__device__ __forceinline__ void split8(const float (&v)[8], v8h& hi, v8h& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 h = (_Float16)v[i];
    hi[i] = h;
    lo[i] = (_Float16)(v[i] - (float)h);
  }
}

template <int HD, int G>
__global__ void __launch_bounds__(kFWaves * 64) k_flash_rows(const AttnArgs a) {
  constexpr int CH = HD / 8;             // 16-byte chunks per K row
  constexpr int NC = HD / 32;            // 32-wide slices of the head dimension
  constexpr int NDT = HD / 16;           // 16-dim tiles of O^T
  constexpr int kTQ = kFRows / G;        // tokens per workgroup
  constexpr int kFKeys = flash_keys(HD);  // keys per block
  constexpr int NS = kFKeys / 32;         // 32-key halves per block
  constexpr int kVC = kFKeys / 8;         // 8-key chunks per V^T row
  constexpr int kKG = kFKeys / 4;         // 4-key groups per block
  constexpr int kVItems = kKG * CH;       // (4-key group, chunk) staging items of V
  static_assert(HD == 64 || HD == 128 || HD == 256, "head_dim 64, 128 or 256");
  static_assert(kFKeys * CH % (kFWaves * 64) == 0, "K staging rounds");
  static_assert(kVItems <= kFWaves * 64, "V staging items");

  // two buffers of each, as separate arrays: the loop names them at compile
  // time, so the compiler can tell the buffer being read from the one the
  // direct global-to-LDS loads of the next block fill, and does not wait for
  // those loads before the current block's reads
  __shared__ v4u ks0[kFKeys * CH], ks1[kFKeys * CH];   // K rows, swizzled slots
  __shared__ v4u vt0[HD * kVC], vt1[HD * kVC];         // V^T rows of the block's keys, swizzled slots

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, kq = lane >> 4;
  const int kvh = blockIdx.y;
  const int z0 = (gridDim.x - 1 - blockIdx.x) * kTQ;   // the longest prefixes first
  auto pos_of = [&](int z) { return a.dpos ? a.dpos[z] : a.pos0 + z; };

  // this lane's query row: token z, head h of the KV head's group
  const int r = 16 * wave + n;
  const int z = z0 + r / G, h = r % G;
  const int zc = min(z, a.n_tok - 1);
  const int lim = z < a.n_tok ? pos_of(zc) : -1;   // last position the row sees
  // positions 0..ctx-1 serve every token of the workgroup; wlim bounds this wave's rows
  const int ctx = wave_max_int(pos_of(min(z0 + lane % kTQ, a.n_tok - 1))) + 1;
  const int wlim = __builtin_amdgcn_readfirstlane(wave_max_int(lim));
  const int nblk = (ctx + kFKeys - 1) / kFKeys;

  // q as the B operand of S^T: lane (n, kq) holds q[32c + 8kq + i] of row n
  v8h qh[NC], ql[NC];
  float qscale;
  {
    const float* qp = a.q + (size_t)zc * a.tok_q + ((size_t)kvh * G + h) * HD + 8 * kq;
    float qv[NC][8];
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * c + 4);
      const float t[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qv[c][i] = t[i];
        amax = fmaxf(amax, fabsf(t[i]));
      }
    }
    amax = max4(amax);
    int e = 0;
    frexpf(amax, &e);   // amax = f * 2^e, f in [0.5, 1); 0 gives e = 0
    const int shift = min(max(14 - e, -100), 100);
    const float sc = ldexpf(1.0f, shift);
    qscale = a.scale * ldexpf(1.0f, -shift);   // S^T holds (q . k) * 2^shift
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[c][i] *= sc;
      split8(qv[c], qh[c], ql[c]);
    }
  }

  const size_t head_base = (size_t)kvh * a.max_seq * HD;
  const uint16_t* kc = static_cast<const uint16_t*>(a.kc) + head_base;
  const uint16_t* vc = static_cast<const uint16_t*>(a.vc) + head_base;

  // K block -> LDS (positions past ctx - 1 reload ctx - 1: finite, masked)
  auto stage_k = [&](int blk, v4u* dst) {
#pragma unroll
    for (int k = 0; k < kFKeys * CH / (kFWaves * 64); ++k) {
      const int P = k * kFWaves * 64 + wave * 64 + lane;   // LDS chunk this lane fills
      const int key = P / CH, slot = P % CH;
      const int p = min(blk * kFKeys + key, ctx - 1);
      const uint16_t* src = kc + (size_t)p * HD + 8 * (slot ^ kswz(key));
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)&dst[k * kFWaves * 64 + wave * 64], 16, 0, 0);
    }
  };
  // V block: thread (kg, c) loads dims 8c..8c+7 of keys 4kg..4kg+3
  const int vkg = tid % kKG, vch = tid / kKG;
  uint4 vr[4];
  auto load_v = [&](int blk) {
    if (tid < kVItems) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = min(blk * kFKeys + 4 * vkg + u, ctx - 1);
        vr[u] = *reinterpret_cast<const uint4*>(vc + (size_t)p * HD + 8 * vch);
      }
    }
  };
  auto store_v = [&](v4u* vdst) {   // dim 8c + j of the 4 keys -> V^T row 8c + j
    if (tid < kVItems) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t word = j < 2 ? vr[u].x : j < 4 ? vr[u].y : j < 6 ? vr[u].z : vr[u].w;
          w[u] = (j & 1) ? word >> 16 : word & 0xffffu;
        }
        uint8_t* row = reinterpret_cast<uint8_t*>(&vdst[(8 * vch + j) * kVC]);
        *reinterpret_cast<uint2*>(row + 16 * ((vkg >> 1) ^ (j & (kVC - 1))) + 8 * (vkg & 1)) =
            make_uint2(w[0] | (w[1] << 16), w[2] | (w[3] << 16));
      }
    }
  };

  v4f o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = v4f{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;   // l: this lane's share of the row's sum

  stage_k(0, ks0);
  load_v(0);
  store_v(vt0);
  vm_drain();
  __syncthreads();
  // one block: the next block's K and V requested into the other buffers,
  // this block's keys used from kcur / vcur
  auto step = [&](int blk, const v4u* kcur, const v4u* vcur, v4u* knxt, v4u* vnxt) {
    const bool next = blk + 1 < nblk;
    if (next) {
      load_v(blk + 1);
      stage_k(blk + 1, knxt);
    }
    const int kb = blk * kFKeys;
    if (kb <= wlim) {
      // S^T tiles (s, t): keys kb + 32s + 8(n/4) + 4t + n%4 against the wave's 16 rows
      v4f st[NS][2];
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int key = 32 * s + 8 * (n >> 2) + 4 * t + (n & 3);
          v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const v8h kv = __builtin_bit_cast(v8h, kcur[key * CH + ((4 * c + kq) ^ kswz(key))]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qh[c], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, ql[c], acc, 0, 0, 0);
          }
          st[s][t] = acc;
        }
      // lane (n, kq): element i of tile (s, t) is key kb + 32s + 8kq + 4t + i of row n
      float sc[NS][2][4];
      float bmax = -INFINITY;
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 32 * s + 8 * kq + 4 * t + i;
            // (q . k) / sqrt(hd), softcapped when set (layer_scheduler.c:442-448); causal limit
            const float v = key <= lim ? softcap(st[s][t][i] * qscale, a) : -INFINITY;
            sc[s][t][i] = v;
            bmax = fmaxf(bmax, v);
          }
      bmax = max4(bmax);
      const float mn = fmaxf(m, bmax);
      const float ms = mn == -INFINITY ? 0.f : mn;   // nothing seen yet: weights stay 0
      const float corr = expf(m - ms);
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
      v8h ph[NS], pl[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        float pv[8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = expf(sc[s][t][i] - ms);   // layer_scheduler.c:450-458
            l += p;
            pv[4 * t + i] = p * kPScale;
          }
        split8(pv, ph[s], pl[s]);
      }
      m = mn;
      // O^T += V^T P^T over the block's 32-key halves
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int d = 16 * dt + n;
          const v8h vv = __builtin_bit_cast(v8h, vcur[d * kVC + ((4 * s + kq) ^ (d & (kVC - 1)))]);
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, ph[s], o[dt], 0, 0, 0);
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, pl[s], o[dt], 0, 0, 0);
        }
    }
    if (next) store_v(vnxt);
    vm_drain();   // this wave's direct LDS loads of the next block have landed
    __syncthreads();
  };
#pragma unroll 1
  for (int blk = 0; blk < nblk; blk += 2) {
    step(blk, ks0, vt0, ks1, vt1);
    if (blk + 1 < nblk) step(blk + 1, ks1, vt1, ks0, vt0);
  }

  // lane (n, kq) holds dims 16dt + 4kq .. +3 of row n   (layer_scheduler.c:460-466)
  l = sum4(l);
  if (z < a.n_tok) {
    const float inv = 1.0f / (l * kPScale);
    float* op = a.out + (size_t)z * a.tok_o + ((size_t)kvh * G + h) * HD + 4 * kq;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      *reinterpret_cast<float4*>(op + 16 * dt) =
          make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
  }
}

template <int HD>
hipError_t launch_flash_hd(int group, const AttnArgs& a, hipStream_t s) {
  const dim3 block(kFWaves * 64);
  auto grid = [&](int g) { return dim3((a.n_tok * g + kFRows - 1) / kFRows, a.n_kv_heads); };
  switch (group) {
    case 1: hipLaunchKernelGGL((k_flash_rows<HD, 1>), grid(1), block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_flash_rows<HD, 2>), grid(2), block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_flash_rows<HD, 4>), grid(4), block, 0, s, a); break;
    case 8: hipLaunchKernelGGL((k_flash_rows<HD, 8>), grid(8), block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_rows(int head_dim, int group, const AttnArgs& a, hipStream_t s) {
  if (a.n_tok < 1 || a.n_kv_heads < 1 || a.max_seq < 1 || !a.q || !a.out || !a.kc || !a.vc || a.tok_q % 4 ||
      a.tok_o % 4)
    return hipErrorInvalidValue;
  if (head_dim == 64) return launch_flash_hd<64>(group, a, s);
  if (head_dim == 128) return launch_flash_hd<128>(group, a, s);
  if (head_dim == 256) return launch_flash_hd<256>(group, a, s);   // Gemma
  return hipErrorInvalidValue;
}

}  // namespace ssk
