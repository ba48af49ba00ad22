// ss_kernels.hip - attention and the small per-token kernels for gfx950.
//
// Per-workgroup argmax candidates are merged by a following small kernel.
// Attention splits of one KV head are merged by the last of its workgroups
// to finish (a device-scope release/acquire around one atomic counter per KV
// head), or left for the Wo matvec, which merges a few splits while staging.

#include <math.h>

#include <type_traits>

#include <hip/hip_ext.h>

#include "ss_device.h"
#include "ss_kernels.h"

namespace ssk {
namespace {

// ------------------------------------------------------------ attention
// Single-query GQA attention (layer_scheduler.c:415-468) with the sequence
// split over gridDim.x workgroups (flash-decoding). In workgroup (s, g), serving the G query heads that share KV head
// g, lane l of wave w holds 8 consecutive elements (column chunk l % LPR) of
// the K and V rows (l / LPR) + RPI*w + ... of its positions; a round of
// positions is requested at once, straight into registers. Scores are summed
// over the LPR lanes of a row with DPP, each wave keeps its own online
// softmax, and the 8 waves are combined once at the end.
template <int KVT>
struct KvElem;
template <>
struct KvElem<0> {   // binary16, 8 elements = 16 bytes
  using Chunk = uint4;
  static __device__ __forceinline__ void get(const Chunk& c, float s, float (&v)[8]) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
    (void)s;
  }
  // the chunk, or zeros for a row that is not live
  static __device__ __forceinline__ Chunk live_or_zero(const Chunk& c, float& s, bool live) {
    (void)s;
    return make_uint4(live ? c.x : 0u, live ? c.y : 0u, live ? c.z : 0u, live ? c.w : 0u);
  }
};
template <>
struct KvElem<1> {   // int8 codes times the position's scale (layer_scheduler.c:120-125)
  using Chunk = uint2;
  static __device__ __forceinline__ void get(const Chunk& c, float s, float (&v)[8]) {
    const uint32_t w[2] = {c.x, c.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)((w[i / 4] >> (8 * (i % 4))) & 0xffu) * s;
  }
  // a row that is not live: scale 0 (the codes are finite)
  static __device__ __forceinline__ Chunk live_or_zero(const Chunk& c, float& s, bool live) {
    s = live ? s : 0.f;
    return c;
  }
};

// The sc1 cache policy bit: loads through a raw buffer view with it read
// the device-coherent level.
constexpr int kSc1 = 16;

// positions of the context: the device position + 1, or the launch's
__device__ __forceinline__ int attn_ctx(const AttnArgs& a) { return a.dpos ? *a.dpos + 1 : a.seq_len; }

__device__ __forceinline__ void attn_split(const AttnArgs& a, int& ctx, int& chunk, int& active) {
  ctx = attn_ctx(a);
  attn_chunks(ctx, a.ns, a.split_fill, chunk, active);
}

// Sum over aligned groups of N (4, 8 or 16) lanes, result in every lane.
template <int N>
__device__ __forceinline__ float sum_lanes(float v) {
  v += dpp<0xb1>(v);                           // quad_perm [1,0,3,2]
  v += dpp<0x4e>(v);                           // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp<0x141>(v);    // row_half_mirror
  if constexpr (N >= 16) v += dpp<0x140>(v);   // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16, kWave);   // the neighbouring 16-lane row
  return v;
}

constexpr int kAttnWaves = 8;
// rows of K and V per lane per round: 128 positions per round at hd 128, G <= 2
__host__ __device__ constexpr int attn_rows_per_lane(int group) {
  return group >= 8 ? 1 : group >= 4 ? 2 : 4;
}

// Four consecutive outputs (quad q of the output vector) into out and, with
// xr_out set, into the x records of the Wo matvec's input: the 4 lanes of an
// aligned quad (all active) hold one record's 16 values.
__device__ __forceinline__ void attn_store4(const AttnArgs& a, int q, float4 v) {
  reinterpret_cast<float4*>(a.out)[q] = v;
  if (a.xr_out) encode4(reinterpret_cast<int*>(a.xr_out) + (q / 8) * kXW, q % 8, v);
}

// The workgroup's W waves hold per-wave (m, l, o) for the G heads in LDS:
// combine them, then either write the output (one active split, with a.cnt
// or a.xr_out set), leave the split's partials for a merging consumer (a.cnt
// null, or a.wo_merge with at most kMergeSplits active splits), or write
// them and let the last split of this KV head to finish merge all of them.
template <int HD, int G, int W>
__device__ __forceinline__ void attn_finish(const AttnArgs& a, int kvh, int active, const float (&wm)[W][G],
                                            const float (&wl)[W][G], const float (&wo)[W][G][HD], int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  constexpr int kThreads = W * 64;
  const bool merge_here = a.cnt && !(a.wo_merge && active <= kMergeSplits);
  if ((a.cnt || a.xr_out) && active == 1) {
    // the only split: the output directly (the merge below with one split),
    // four consecutive outputs per thread; quads of lanes hold the 16 values
    // of one x record (G * HD / 4 is a multiple of 8)
    for (int i4 = tid; i4 < G * HD / 4; i4 += kThreads) {
      float r[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = i4 * 4 + c, g = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, wm[w][g]);
        float so = 0.f, sl = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float f = expf(wm[w][g] - M);
          so = fmaf(f, wo[w][g][d], so);
          sl = fmaf(f, wl[w][g], sl);
        }
        r[c] = so * (1.0f / sl);
      }
      attn_store4(a, kvh * G * HD / 4 + i4, make_float4(r[0], r[1], r[2], r[3]));
    }
    return;
  }
  float* po = a.part_o + (((size_t)kvh * a.ns + blockIdx.x) * G) * HD;
  float* pml = a.part_ml + (((size_t)kvh * a.ns + blockIdx.x) * G) * 2;
  for (int i = tid; i < G * HD; i += kThreads) {
    const int g = i / HD, d = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, wm[w][g]);   // finite: wave 0 holds the split's first position
    float so = 0.f, sl = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = expf(wm[w][g] - M);
      so = fmaf(f, wo[w][g][d], so);
      sl = fmaf(f, wl[w][g], sl);
    }
    if (merge_here) {   // merged below by another workgroup: coherent stores
      cstf(po + g * HD + d, so);
      if (d == 0) {
        cstf(pml + g * 2, M);
        cstf(pml + g * 2 + 1, sl);
      }
    } else {       // merged by the next kernel
      po[g * HD + d] = so;
      if (d == 0) {
        pml[g * 2] = M;
        pml[g * 2 + 1] = sl;
      }
    }
  }
  if (!merge_here) return;   // the consumer (the Wo matvec) merges the splits

  // The last split of this KV head to finish merges all of them:
  // out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
  __shared__ uint32_t last;
  __shared__ float wts[kMaxSplits * G];
  vm_drain();        // this wave's partials have reached the coherent level
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(a.cnt + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (uint32_t)(active - 1);
  __syncthreads();
  if (!last) return;
  const float* ml = a.part_ml + (size_t)kvh * a.ns * G * 2;
  const float* pob = a.part_o + (size_t)kvh * a.ns * G * HD;
  // Thread (sub, quad) sums four consecutive outputs over the splits
  // sub, sub + kSub, ..., kBatch 16-byte coherent loads in flight at a time
  // (out-of-range loads of the buffer view read zero); the kSub partial sums
  // are then added in subset order. The batch is smaller for small groups,
  // whose registers the main loop does not fill (occupancy). The first batch
  // is requested before the split weights are formed.
  constexpr int kBatch = G >= 4 ? 16 : 8;
  constexpr int kQuads = G * HD / 4;
  constexpr int kSub = kThreads / kQuads;
  static_assert(kThreads % kQuads == 0, "outputs in quads must divide the workgroup");
  __shared__ float4 red[kThreads];
  const int qd = tid % kQuads, sub = tid / kQuads;
  const int gq = qd * 4 / HD;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(pob), (short)0, active * G * HD * 4, kBufferFlags);
  float4 v[kBatch];
  auto fetch = [&](int sp0) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k)   // the builtin returns the 16 bytes as four 32-bit integers
      v[k] = __builtin_bit_cast(
          float4, __builtin_amdgcn_raw_buffer_load_b128(ro, ((sp0 + k * kSub) * kQuads + qd) * 16, 0, kSc1));
  };
  fetch(sub);
  for (int g = wave; g < G; g += W) {
    float mx = -INFINITY;
    float mv[kMaxSplits / kWave], lv[kMaxSplits / kWave];
#pragma unroll
    for (int k = 0; k < kMaxSplits / kWave; ++k) {
      const int sp = lane + k * kWave;
      mv[k] = sp < active ? cldf(ml + (sp * G + g) * 2) : -INFINITY;
      lv[k] = sp < active ? cldf(ml + (sp * G + g) * 2 + 1) : 0.f;
    }
    for (int k = 0; k < kMaxSplits / kWave; ++k) mx = fmaxf(mx, mv[k]);
    mx = wave_max(mx);
    float ls = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxSplits / kWave; ++k) ls += lv[k] * expf(mv[k] - mx);
    const float inv = 1.0f / wave_sum(ls);
#pragma unroll
    for (int k = 0; k < kMaxSplits / kWave; ++k) {
      const int sp = lane + k * kWave;
      if (sp < active) wts[sp * G + g] = expf(mv[k] - mx) * inv;
    }
  }
  __syncthreads();
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp0 = sub; sp0 < active; sp0 += kBatch * kSub) {
    if (sp0 != sub) fetch(sp0);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int sp = sp0 + k * kSub;
      const float w = sp < active ? wts[sp * G + gq] : 0.f;
      acc.x = fmaf(v[k].x, w, acc.x);
      acc.y = fmaf(v[k].y, w, acc.y);
      acc.z = fmaf(v[k].z, w, acc.z);
      acc.w = fmaf(v[k].w, w, acc.w);
    }
  }
  red[tid] = acc;
  __syncthreads();
  if (sub == 0) {
    for (int k = 1; k < kSub; ++k) {
      const float4 r = red[k * kQuads + qd];
      acc.x += r.x;
      acc.y += r.y;
      acc.z += r.z;
      acc.w += r.w;
    }
    attn_store4(a, kvh * G * HD / 4 + qd, acc);
  }
  if (tid == 0) cst(a.cnt + kvh, 0u);   // every split of this launch has arrived: ready for the next
}

// FIX: every split is one round of kRound positions starting at split *
// kRound (fill = kRound and ns * kRound covers the cache): the query and the
// round are requested before the position is read, rows past the context
// are masked in use, and a split past the active ones leaves after its loads.
template <int HD, int G, int KVT, bool FIX>
__global__ void __launch_bounds__(kAttnWaves * 64) k_attn(const AttnArgs a) {
  using KE = KvElem<KVT>;
  using Chunk = typename KE::Chunk;
  constexpr int kLpr = HD / 8;                  // lanes per row
  constexpr int kRpi = kWave / kLpr;            // rows per wave and load
  constexpr int kK = attn_rows_per_lane(G);     // rows per lane per round
  constexpr int kRound = kK * kAttnWaves * kRpi;    // positions per round
  constexpr int kEb = KVT == 0 ? 2 : 1;          // bytes per element

  __shared__ float wm[kAttnWaves][G], wl[kAttnWaves][G];
  __shared__ float wo[kAttnWaves][G][HD];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar)
  const int kvh = blockIdx.y;
  int ctx = 0, chunk = kRound, active = 0;
  if constexpr (!FIX) {
    attn_split(a, ctx, chunk, active);
    if ((int)blockIdx.x >= active) return;   // whole workgroup
  }
  const int t0 = blockIdx.x * chunk;
  // the end of the split's rows: with FIX, until the position is read, the
  // end of its round inside the cache (the loads' range)
  int t1 = FIX ? min(t0 + kRound, a.max_seq) : min(ctx, t0 + chunk);
  const int c = lane % kLpr, rsub = lane / kLpr;

  // K and V rows [r0, t1) of this KV head as a buffer view per round (base
  // and range in scalar registers): a lane's row chunk is one load at a
  // loop-invariant offset, rows past t1 read zero (and are masked)
  const size_t head_base = (size_t)kvh * a.max_seq * HD * kEb;
  const uint8_t* kbase = static_cast<const uint8_t*>(a.kc) + head_base;
  const uint8_t* vbase = static_cast<const uint8_t*>(a.vc) + head_base;
  auto row_in = [&](int k) { return (k * kAttnWaves + wave) * kRpi + rsub; };   // row within a round

  float q[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float4* qp = reinterpret_cast<const float4*>(a.q + ((size_t)kvh * G + g) * HD + c * 8);
    const float4 x0 = qp[0], x1 = qp[1];
    q[g][0] = x0.x; q[g][1] = x0.y; q[g][2] = x0.z; q[g][3] = x0.w;
    q[g][4] = x1.x; q[g][5] = x1.y; q[g][6] = x1.z; q[g][7] = x1.w;
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }

  // One round: kK rows of K and V per lane; two rounds in flight (the next
  // one is requested before the current one is used).
  struct Round {
    Chunk k[kK], v[kK];
    float ks[kK], vs[kK];
  };
  auto load = [&](Round& rd, int r0) {
    const int n = max(t1 - r0, 0);   // rows of the round inside the split
    const __amdgpu_buffer_rsrc_t kx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(kbase + (size_t)r0 * HD * kEb), (short)0, n * HD * kEb, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(vbase + (size_t)r0 * HD * kEb), (short)0, n * HD * kEb, kBufferFlags);
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      const int off = row_in(k) * (HD * kEb) + c * 8 * kEb;
      if constexpr (KVT == 0) {
        rd.k[k] = __builtin_bit_cast(Chunk, __builtin_amdgcn_raw_buffer_load_b128(kx, off, 0, 0));
        rd.v[k] = __builtin_bit_cast(Chunk, __builtin_amdgcn_raw_buffer_load_b128(vx, off, 0, 0));
        rd.ks[k] = rd.vs[k] = 1.f;
      } else {
        rd.k[k] = __builtin_bit_cast(Chunk, __builtin_amdgcn_raw_buffer_load_b64(kx, off, 0, 0));
        rd.v[k] = __builtin_bit_cast(Chunk, __builtin_amdgcn_raw_buffer_load_b64(vx, off, 0, 0));
        // the rows' scales (one fp32 per position) through views of the same rows
        const __amdgpu_buffer_rsrc_t ksx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.ks + r0), (short)0, n * 4, kBufferFlags);
        const __amdgpu_buffer_rsrc_t vsx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.vs + r0), (short)0, n * 4, kBufferFlags);
        rd.ks[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksx, row_in(k) * 4, 0, 0));
        rd.vs[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vsx, row_in(k) * 4, 0, 0));
      }
    }
  };
  // cap: the attention softcap is set (decided once, outside the loop, so the
  // loop has no branch between a round's loads and their use)
  auto use = [&](const Round& rd, int r0, auto cap) {
    float sc[G][kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      float kv[8];
      KE::get(rd.k[k], rd.ks[k], kv);
      const bool live = r0 + row_in(k) < t1;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(q[g][e], kv[e], d);
        d = sum_lanes<kLpr>(d) * a.scale;   // (q . k) / sqrt(hd), layer_scheduler.c:442-448
        if constexpr (decltype(cap)::value) d = softcap(d, a);
        sc[g][k] = live ? d : -INFINITY;
      }
    }
    // V rows, zeroed where not live: a row past the end reads zero, or, in a
    // round requested before the position was read, whatever an earlier
    // sequence left there, and its weight 0 must not meet a non-finite value
    typename KE::Chunk vm[kK];
    float vsm[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) {
      vsm[k] = rd.vs[k];
      vm[k] = KE::live_or_zero(rd.v[k], vsm[k], r0 + row_in(k) < t1);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = sc[g][0];
#pragma unroll
      for (int k = 1; k < kK; ++k) mt = fmaxf(mt, sc[g][k]);
      mt = wave_max(mt);
      const float mn = fmaxf(m[g], mt);
      const float mref = mn == -INFINITY ? 0.f : mn;   // nothing live yet: all weights 0
      const float corr = expf(m[g] - mref);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= corr;
#pragma unroll
      for (int k = 0; k < kK; ++k) {
        const float p = expf(sc[g][k] - mref);
        ps += p;
        float vv[8];
        KE::get(vm[k], vsm[k], vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(p, vv[e], o[g][e]);
      }
      l[g] = l[g] * corr + wave_sum(c == 0 ? ps : 0.f);
      m[g] = mn;
    }
  };
  // the scheduling barriers keep each round's loads ahead of the other
  // round's arithmetic (the scheduler would otherwise sink them to their
  // uses, leaving one round in flight)
  // The marker starts each loop's version with a different instruction: the
  // two would otherwise share their first round's loads, hoisted above the
  // branch, and each copy them into its own registers, waiting for them
  // before the second round is requested.
  auto rounds = [&](auto cap) {
    asm volatile("; softcap %0" ::"n"(decltype(cap)::value ? 1 : 0));
    Round A, B;
    load(A, t0);
    for (int r0 = t0;; r0 += 2 * kRound) {
      load(B, r0 + kRound);
      __builtin_amdgcn_sched_barrier(0);
      use(A, r0, cap);
      if (r0 + kRound >= t1) break;
      load(A, r0 + 2 * kRound);
      __builtin_amdgcn_sched_barrier(0);
      use(B, r0 + kRound, cap);
      if (r0 + 2 * kRound >= t1) break;
    }
  };
  if constexpr (FIX) {
    Round A;
    load(A, t0);
    attn_split(a, ctx, chunk, active);       // chunk == kRound
    if ((int)blockIdx.x >= active) return;   // whole workgroup
    t1 = min(ctx, t0 + kRound);
    if (a.softcap > 0.f)
      use(A, t0, std::true_type{});
    else
      use(A, t0, std::false_type{});
  } else if (a.softcap > 0.f) {
    rounds(std::true_type{});
  } else {
    rounds(std::false_type{});
  }

  // rows of a wave: lanes with the same column chunk are kLpr apart
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      for (int off = kLpr; off < kWave; off <<= 1) o[g][e] += __shfl_xor(o[g][e], off, kWave);
  if (rsub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) wo[wave][g][c * 8 + e] = o[g][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wm[wave][g] = m[g];
      wl[wave][g] = l[g];
    }
  }
  __syncthreads();
  attn_finish<HD, G, kAttnWaves>(a, kvh, active, wm, wl, wo, tid);
}

// ------------------------------------------------------------ attention, heads on lanes
// For groups of 4 or 8 query heads per KV head: lane l of a wave serves query
// head l / (64/G) of the group and dims [c*DPL, c*DPL + DPL), c = l % (64/G),
// DPL = HD*G/64, so a wave covers all G heads of one K/V row at once (64
// lanes x DPL = G x HD multiply-adds per position). Scores are summed over
// the 64/G lanes of a head with DPP. The positions are split by stride,
// not by range: workgroup s of a KV head holds positions s, s + ns,
// s + 2 ns, ..., and wave w of it the positions s + ns (w + 8 r), r = 0, 1,
// ..., so the rows of every batch are known at launch and the first two
// batches are requested together with the query, before the position is
// read (a range split needs the context to place its rows). The first
// min(ctx, ns) workgroups are active (attn_strided_active, which the
// consumers merging the splits use too). Each wave takes its rows in
// batches of B (all of a batch's K and V loaded before any is used, the
// next batch's loads issued before the current one is used), keeps an
// online softmax per head (every lane of a head holds the same m, l), and
// the waves are combined at the end by attn_finish. Per lane: DPL query
// values, DPL outputs and two batches.
constexpr int kHgWaves = 8;

// B: rows of K and V per lane per batch; two batches (the one in use and
// the next, in flight) hold at most 64 VGPRs: 2 * B * DPL words of fp16
__host__ __device__ constexpr int hg_batch(int hd, int group) {
  return 32 / (hd * group / kWave);
}

// N elements of one K or V row (fp16, or int8 times the row's scale)
template <int KVT, int N>
struct KvRow {
  static constexpr int kWords = N * (KVT == 0 ? 2 : 1) / 4;
  uint32_t w[kWords];
  __device__ __forceinline__ void load(const uint8_t* p) {
    if constexpr (kWords == 1) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (kWords == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < kWords / 4; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(p)[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    }
  }
  // the same words through a buffer view (offset in bytes; past the view's
  // range the words read zero)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (kWords == 1) {
      w[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else if constexpr (kWords == 2) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
      w[0] = v[0];
      w[1] = v[1];
    } else {
#pragma unroll
      for (int i = 0; i < kWords / 4; ++i) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
        w[4 * i] = v[0];
        w[4 * i + 1] = v[1];
        w[4 * i + 2] = v[2];
        w[4 * i + 3] = v[3];
      }
    }
  }
  __device__ __forceinline__ float get(int i, float s) const {
    if constexpr (KVT == 0)
      return h2f((uint16_t)(w[i / 2] >> (16 * (i % 2))));
    else
      return (float)(int8_t)((w[i / 4] >> (8 * (i % 4))) & 0xffu) * s;
  }
};

template <int HD, int G, int KVT>
__global__ void __launch_bounds__(kHgWaves * 64) k_attn_hg(const AttnArgs a) {
  constexpr int kLph = kWave / G;          // lanes per head
  constexpr int kDpl = HD / kLph;          // dims per lane
  constexpr int kB = hg_batch(HD, G);
  constexpr int kEb = KVT == 0 ? 2 : 1;
  constexpr int kRowB = HD * kEb;          // bytes of a K or V row
  using Row = KvRow<KVT, kDpl>;
  static_assert(kLph == 8 || kLph == 16, "heads of 8 or 16 lanes");

  __shared__ float wm[kHgWaves][G], wl[kHgWaves][G];
  __shared__ float wo[kHgWaves][G][HD];

  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index as a wave-uniform (scalar) value: the per-batch buffer
  // views derived from it stay in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kvh = blockIdx.y;
  const int h = lane / kLph, c = lane % kLph;
  // this wave's rows: positions pw + rstride * r, r = 0, 1, ...; batch b
  // holds rows b * kB .. b * kB + kB - 1
  const int ns = a.ns;
  const int pw = (int)blockIdx.x + ns * wave;
  const int rstride = ns * kHgWaves;
  const int rstep = rstride * kRowB;       // bytes between the wave's rows

  // K and V rows of one batch of this KV head as a buffer view per batch
  // (base and range in scalar registers): row j of the batch is one load at
  // j * rstep past the lane's column offset, and rows at or past the view's
  // limit read zero
  const size_t head_base = (size_t)kvh * a.max_seq * kRowB;
  const uint8_t* kbase = static_cast<const uint8_t*>(a.kc) + head_base;
  const uint8_t* vbase = static_cast<const uint8_t*>(a.vc) + head_base;
  const int lane_off = c * kDpl * kEb;

  float q[kDpl], o[kDpl];
  {
    const float4* qp = reinterpret_cast<const float4*>(a.q + ((size_t)kvh * G + h) * HD + c * kDpl);
#pragma unroll
    for (int i = 0; i < kDpl / 4; ++i) {
      const float4 x = qp[i];
      q[4 * i] = x.x;
      q[4 * i + 1] = x.y;
      q[4 * i + 2] = x.z;
      q[4 * i + 3] = x.w;
    }
  }
#pragma unroll
  for (int i = 0; i < kDpl; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;
  int ctx = 0;

  struct Batch {
    Row k[kB], v[kB];
    float ks[kB], vs[kB];
  };
  // batch b's rows below lim (the cache's end before the position is read,
  // the context after); branch-free: every row is loaded and rows past lim
  // read zero
  auto load = [&](Batch& bt, int b, int lim) {
    const int pb = pw + rstride * kB * b;
    const int n = max(lim - pb, 0);
    const __amdgpu_buffer_rsrc_t kx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(kbase + (size_t)pb * kRowB), (short)0, n * kRowB, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(vbase + (size_t)pb * kRowB), (short)0, n * kRowB, kBufferFlags);
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      bt.k[j].load(kx, lane_off + j * rstep);
      bt.v[j].load(vx, lane_off + j * rstep);
    }
    if constexpr (KVT == 1) {   // the rows' scales, one fp32 per position
      const __amdgpu_buffer_rsrc_t ksx =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.ks + pb), (short)0, n * 4, kBufferFlags);
      const __amdgpu_buffer_rsrc_t vsx =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.vs + pb), (short)0, n * 4, kBufferFlags);
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        bt.ks[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksx, 4 * j * rstride, 0, 0));
        bt.vs[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vsx, 4 * j * rstride, 0, 0));
      }
    } else {
#pragma unroll
      for (int j = 0; j < kB; ++j) bt.ks[j] = bt.vs[j] = 1.f;
    }
  };
  // Rows at or past the context are masked: score -inf, and a V row of
  // zeros (the first two batches are read up to the cache's end, and a row
  // there holds whatever an earlier sequence left, so its weight 0 must not
  // meet a non-finite value). A wave with no row below the context (its
  // first batch all masked) keeps m = -inf, l = 0, o = 0.
  // cap: the attention softcap is set (decided once, outside the loop, so the
  // loop has no branch between a batch's loads and their use)
  auto use = [&](const Batch& bt, int b, auto cap) {
    const int pb = pw + rstride * kB * b;
    float sc[kB];
    bool live[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      live[j] = pb + j * rstride < ctx;
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < kDpl; ++i) d = fmaf(q[i], bt.k[j].get(i, bt.ks[j]), d);
      d = sum_lanes<kLph>(d) * a.scale;   // (q . k) / sqrt(hd), layer_scheduler.c:442-448
      if constexpr (decltype(cap)::value) d = softcap(d, a);
      sc[j] = live[j] ? d : -INFINITY;
    }
    float bm = sc[0];
#pragma unroll
    for (int j = 1; j < kB; ++j) bm = fmaxf(bm, sc[j]);
    const float mn = fmaxf(m, bm);
    const float mref = mn == -INFINITY ? 0.f : mn;   // nothing live yet: every weight 0
    const float corr = expf(m - mref);               // 0 while m = -inf
    l *= corr;
#pragma unroll
    for (int i = 0; i < kDpl; ++i) o[i] *= corr;
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const float pj = expf(sc[j] - mref);
      l += pj;
      Row v = bt.v[j];
      float vs = bt.vs[j];
      if constexpr (KVT == 0) {
#pragma unroll
        for (int w = 0; w < Row::kWords; ++w) v.w[w] = live[j] ? v.w[w] : 0u;
      } else {
        vs = live[j] ? vs : 0.f;   // int8 codes are finite: a zero scale zeroes the row
      }
#pragma unroll
      for (int i = 0; i < kDpl; ++i) o[i] = fmaf(pj, v.get(i, vs), o[i]);
    }
    m = mn;
  };
  // a use of a batch's registers, on a path that does not read them: keeps
  // their loads where they are written (ahead of the position's read) rather
  // than sunk to the path that does
  auto pin = [&](const Batch& bt) {
#pragma unroll
    for (int j = 0; j < kB; ++j) {
#pragma unroll
      for (int w = 0; w < Row::kWords; ++w) asm volatile("" ::"v"(bt.k[j].w[w]), "v"(bt.v[j].w[w]));
      if constexpr (KVT == 1) asm volatile("" ::"v"(bt.ks[j]), "v"(bt.vs[j]));
    }
  };
  // The query, the position and batches 0 and 1 are requested together (the
  // position first: loads complete in order, so the wait for it does not
  // include the batches); then each use is followed by the request of the
  // batch two further on. The scheduling barriers keep each batch's loads
  // ahead of the other batch's arithmetic (the scheduler would otherwise
  // sink them to their uses, leaving one batch in flight). The marker
  // starts each version with a different instruction (shared first loads
  // would be hoisted above the branch and copied into each version's
  // registers, a wait for them before the second batch is requested).
  // Returns the active split count.
  auto run = [&](auto cap) -> int {
    asm volatile("; softcap %0" ::"n"(decltype(cap)::value ? 1 : 0));
    // the device position through a view (of range 0, reading zero, when
    // the launch gives the context): no branch, so nothing waits for it
    // before the batches are requested
    const __amdgpu_buffer_rsrc_t px = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int*>(a.dpos), (short)0, a.dpos ? 4 : 0, kBufferFlags);
    const int dp = __builtin_amdgcn_raw_buffer_load_b32(px, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    Batch A, B;
    load(A, 0, a.max_seq);
    load(B, 1, a.max_seq);
    __builtin_amdgcn_sched_barrier(0);
    ctx = a.dpos ? dp + 1 : a.seq_len;
    const int active = attn_strided_active(ctx, ns);
    if ((int)blockIdx.x >= active) {   // whole workgroup
      pin(A);
      pin(B);
#pragma unroll
      for (int i = 0; i < kDpl; ++i) asm volatile("" ::"v"(q[i]));
      return active;
    }
    const int nr = pw < ctx ? (ctx - 1 - pw) / rstride + 1 : 0;   // the wave's rows below ctx
    const int nb = (nr + kB - 1) / kB;
    // No batch past the wave's last is requested: a load returns in order
    // behind the others, out of range or not, and the barrier before the
    // waves combine waits for it, a whole round trip at the tail. So pairs
    // of batches run while both reloads are needed, and the last one to
    // three batches are taken apart. The barriers before the reloads keep
    // each use ahead of its batch's reload (a reload overlapping the use
    // would take fresh registers, copied back at the loop's end, which
    // waits for every load).
    int b = 0;
    for (; b + 3 < nb; b += 2) {
      use(A, b, cap);
      __builtin_amdgcn_sched_barrier(0);
      load(A, b + 2, ctx);
      __builtin_amdgcn_sched_barrier(0);
      use(B, b + 1, cap);
      __builtin_amdgcn_sched_barrier(0);
      load(B, b + 3, ctx);
      __builtin_amdgcn_sched_barrier(0);
    }
    use(A, b, cap);   // a wave without rows: all masked
    if (b + 2 < nb) {
      __builtin_amdgcn_sched_barrier(0);
      load(A, b + 2, ctx);
      __builtin_amdgcn_sched_barrier(0);
      use(B, b + 1, cap);
      use(A, b + 2, cap);
    } else if (b + 1 < nb) {
      use(B, b + 1, cap);
    }
    return active;
  };
  const int active = a.softcap > 0.f ? run(std::true_type{}) : run(std::false_type{});
  if ((int)blockIdx.x >= active) return;

  if (c == 0) {
    wm[wave][h] = m;   // a wave without positions: -inf and 0, weight 0 below
    wl[wave][h] = l;
  }
#pragma unroll
  for (int i = 0; i < kDpl; ++i) wo[wave][h][c * kDpl + i] = o[i];
  __syncthreads();
  attn_finish<HD, G, kHgWaves>(a, kvh, active, wm, wl, wo, tid);
}

// ------------------------------------------------------------ split merge
// The splits of a layer's attention merged after the attention kernel, for
// groups of 4 or 8 query heads, whose splits are too many for the Wo matvec
// to merge while staging: out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M)
// (the softmax of layer_scheduler.c:450-468 over all positions). The
// attention leaves its partials with plain stores (a.cnt null) and, with a
// single active split, writes the output itself, in which case this kernel
// does nothing. Workgroup: one wave, 16 quads (64 consecutive outputs of one
// query head) x 4 subsets of the splits; grid: n_kv_heads * G * HD / 64, so
// the partials are read by many compute units at once rather than by one
// workgroup per KV head.
template <int HD, int G>
__global__ void __launch_bounds__(kWave) k_attn_merge(const AttnArgs a) {
  constexpr int kQuads = G * HD / 4;   // quads of one KV head's G heads
  constexpr int kWgPerKvh = kQuads / 16;
  constexpr int kBatch = 8;            // 16-byte loads in flight per lane (32 splits per batch)
  constexpr int kMlPerLane = kMaxSplits / kWave;
  __shared__ float wts[kMaxSplits];
  __shared__ float4 red[kWave];
  const int lane = threadIdx.x;
  const int kvh = blockIdx.x / kWgPerKvh;
  const int q0 = (blockIdx.x % kWgPerKvh) * 16;   // first quad of the workgroup
  const int g = q0 * 4 / HD;                      // its query head within the group
  const int ns = a.ns;
  const int quad = lane & 15, sub = lane >> 4;
  const float* ml = a.part_ml + (size_t)kvh * ns * G * 2;
  const float4* po = reinterpret_cast<const float4*>(a.part_o + (size_t)kvh * ns * G * HD) + q0 + quad;
  // Every split's (m, l) and this lane's first batch of partial outputs are
  // requested together with the position, before the active count is known:
  // slots past the active splits hold values of earlier calls and are
  // excluded by selection (never multiplied in), so no load waits for
  // another.
  float2 mlv[kMlPerLane];
#pragma unroll
  for (int k = 0; k < kMlPerLane; ++k) {
    const int sp = lane + k * kWave;
    mlv[k] = sp < ns ? *reinterpret_cast<const float2*>(ml + (sp * G + g) * 2) : make_float2(-INFINITY, 0.f);
  }
  float4 v[kBatch];
#pragma unroll
  for (int k = 0; k < kBatch; ++k) v[k] = po[(size_t)min(sub + 4 * k, ns - 1) * kQuads];
  const int active = attn_strided_active(attn_ctx(a), ns);
  if (active <= 1) return;   // whole workgroup: the attention wrote the output
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMlPerLane; ++k)
    if (lane + k * kWave < active) mx = fmaxf(mx, mlv[k].x);
  mx = wave_max(mx);
  float ls = 0.f;
#pragma unroll
  for (int k = 0; k < kMlPerLane; ++k)
    if (lane + k * kWave < active) ls += mlv[k].y * expf(mlv[k].x - mx);
  const float inv = 1.0f / wave_sum(ls);
#pragma unroll
  for (int k = 0; k < kMlPerLane; ++k)
    if (lane + k * kWave < active) wts[lane + k * kWave] = expf(mlv[k].x - mx) * inv;
  __syncthreads();
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp0 = sub;;) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int sp = sp0 + 4 * k;
      if (sp < active) {
        const float w = wts[sp];
        acc.x = fmaf(v[k].x, w, acc.x);
        acc.y = fmaf(v[k].y, w, acc.y);
        acc.z = fmaf(v[k].z, w, acc.z);
        acc.w = fmaf(v[k].w, w, acc.w);
      }
    }
    sp0 += 4 * kBatch;
    if (sp0 >= active) break;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) v[k] = po[(size_t)min(sp0 + 4 * k, active - 1) * kQuads];
  }
  red[lane] = acc;
  __syncthreads();
  if (sub == 0) {   // lanes 0..15: 16 aligned quads, four per x record
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      const float4 r = red[k * 16 + quad];
      acc.x += r.x;
      acc.y += r.y;
      acc.z += r.z;
      acc.w += r.w;
    }
    attn_store4(a, kvh * kQuads + q0 + quad, acc);
  }
}

template <int HD, int G>
hipError_t launch_merge_t(const AttnArgs& a, hipStream_t s) {
  const dim3 grid(a.n_kv_heads * G * HD / 64);
  KernelEvents& ev = kernel_events();
  if (ev.start) {
    hipExtLaunchKernelGGL((k_attn_merge<HD, G>), grid, dim3(kWave), 0, s, ev.start, ev.stop, 0, a);
    ev.used = true;
  } else {
    hipLaunchKernelGGL((k_attn_merge<HD, G>), grid, dim3(kWave), 0, s, a);
  }
  return hipGetLastError();
}

template <int HD>
hipError_t launch_merge_hd(int group, const AttnArgs& a, hipStream_t s) {
  switch (group) {
    case 4: return launch_merge_t<HD, 4>(a, s);
    case 8: return launch_merge_t<HD, 8>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------------------ embedding of a prompt
// ss_scheduler_embed (layer_scheduler.c:864-911): every token's final hidden
// state through the output norm (x * k_t * w, k_t = 1/sqrt(ssq_t/d + eps)),
// summed over the tokens in order into acc (one thread per column), then the
// mean and the L2 normalisation.
__global__ void k_pool_rows(const float* __restrict__ x, int T, int d, const float* __restrict__ w,
                            const float* __restrict__ ssq, float eps, float* __restrict__ acc) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= d) return;
  float s = acc[j];
  for (int t = 0; t < T; ++t) {
    const float v = x[(size_t)t * d + j];
    s += w ? v * (1.0f / sqrtf(ssq[t] / (float)d + eps)) * w[j] : v;
  }
  acc[j] = s;
}

__global__ void __launch_bounds__(256) k_embed_finish(const float* __restrict__ acc, int d, int n,
                                                      float* __restrict__ out) {
  __shared__ float red[4];
  const float inv = 1.0f / (float)n;
  float l2 = 0.f;
  for (int j = threadIdx.x; j < d; j += 256) {
    const float e = acc[j] * inv;
    l2 = fmaf(e, e, l2);
  }
  l2 = wave_sum(l2);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = l2;
  __syncthreads();
  const float sc = 1.0f / (sqrtf((red[0] + red[1]) + (red[2] + red[3])) + 1e-12f);
  for (int j = threadIdx.x; j < d; j += 256) out[j] = acc[j] * inv * sc;
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

// A prompt's rows after the [Wq;Wk;Wv] products: row z of qkv (stride ld)
// is [q | k | v] of the token at position dpos[z]. Pairs (2j, 2j+1) of each
// q and k head below rope_dim rotate by the position's (cos, sin)
// (tensor.c:250-273; q in place for the attention that follows), then k and
// v go to the fp16 cache [kvh][max_seq][hd] (layer_scheduler.c:392-413).
// One thread per pair; grid y = tokens.
__global__ void k_rope_kv_rows(float* qkv, const float* bias, int ld, int qdim, int kvdim, int head_dim,
                               int rope_dim, const float* cs, const int* dpos, uint16_t* kc, uint16_t* vc,
                               int max_seq) {
  const int pos = dpos[blockIdx.y];
  float* row = qkv + (size_t)blockIdx.y * ld;
  const int npairs = (qdim + 2 * kvdim) >> 1;
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < npairs; p += gridDim.x * blockDim.x) {
    const int r = 2 * p;
    const float2 v = reinterpret_cast<const float2*>(row)[p];
    float a = v.x, b = v.y;
    if (bias) {   // layer_scheduler.c:367-402, before RoPE
      const float2 bb = reinterpret_cast<const float2*>(bias)[p];
      a = a + bb.x;
      b = b + bb.y;
    }
    if (r < qdim + kvdim) {
      const int i0 = (r < qdim ? r : r - qdim) % head_dim;
      if (i0 < rope_dim) {
        const float c = cs[(size_t)pos * rope_dim + i0], s = cs[(size_t)pos * rope_dim + i0 + 1];
        const float ra = a * c - b * s;
        const float rb = a * s + b * c;
        a = ra;
        b = rb;
      }
    }
    if (r < qdim) {
      reinterpret_cast<float2*>(row)[p] = make_float2(a, b);
    } else {
      const bool is_v = r >= qdim + kvdim;
      const int kr = r - qdim - (is_v ? kvdim : 0);
      uint16_t* c = (is_v ? vc : kc) + ((size_t)(kr / head_dim) * max_seq + pos) * head_dim + kr % head_dim;
      c[0] = f2h(a);
      c[1] = f2h(b);
    }
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

// Post norm (layer_scheduler.c:474-481, 553-560: ss_gemma_rmsnorm of the
// projection's output y, then the residual add): hidden[i] += y[i] * s * w[i]
// with s = 1 / sqrt(mean(y^2) + eps) and w already 1 + weight. With xr set,
// also the x records of the new hidden * nw_out (nw_out null: weight 1) for
// the next matvec. One workgroup; every iteration of the element loop runs
// in all threads, so the 16 lanes of a record encode together (n % 16 == 0).
__global__ void __launch_bounds__(1024) k_post_norm(float* hidden, const float* y, const float* w, int n,
                                                   float eps, uint32_t* xr, const float* nw_out) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  float ss = 0.f;
  for (int i = tid; i < n; i += 1024) {
    const float v = y[i];
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int k = 0; k < 16; ++k) t += red[k];
  const float sc = 1.0f / sqrtf(t / (float)n + eps);
  for (int i0 = 0; i0 < n; i0 += 1024) {
    const int i = i0 + tid;
    const bool in = i < n;
    float out = 0.f;
    if (in) {
      out = hidden[i] + y[i] * sc * w[i];
      hidden[i] = out;
    }
    if (xr) {
      const Enc e = enc16(in ? out * (nw_out ? nw_out[i] : 1.f) : 0.f, out);
      if (in) put_rec_lds(xr + (size_t)(i >> 4) * kRW, e, i & 15);
    }
  }
}

// The same for the rows of a prompt: workgroup t adds the normalised row t
// of y (n values, row stride n) to row t of hidden.
__global__ void __launch_bounds__(1024) k_post_norm_rows(float* hidden, const float* y, const float* w, int n,
                                                         float eps) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  hidden += (size_t)blockIdx.x * n;
  y += (size_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = tid; i < n; i += 1024) {
    const float v = y[i];
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int k = 0; k < 16; ++k) t += red[k];
  const float sc = 1.0f / sqrtf(t / (float)n + eps);
  for (int i = tid; i < n; i += 1024) hidden[i] = hidden[i] + y[i] * sc * w[i];
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
  KernelEvents& ev = kernel_events();
  if constexpr (G >= 4) {   // heads on lanes
    const dim3 block(kHgWaves * 64);
    if (ev.start) {
      if (kv_type == 0)
        hipExtLaunchKernelGGL((k_attn_hg<HD, G, 0>), grid, block, 0, s, ev.start, ev.stop, 0, a);
      else
        hipExtLaunchKernelGGL((k_attn_hg<HD, G, 1>), grid, block, 0, s, ev.start, ev.stop, 0, a);
      ev.used = true;
    } else if (kv_type == 0) {
      hipLaunchKernelGGL((k_attn_hg<HD, G, 0>), grid, block, 0, s, a);
    } else {
      hipLaunchKernelGGL((k_attn_hg<HD, G, 1>), grid, block, 0, s, a);
    }
    return hipGetLastError();
  } else {
    // one-round splits whose starts do not depend on the context (the split
    // rule of attn_chunks with fill = one round and ns rounds covering the
    // cache)
    const int round = attn_round_positions(HD, G);
    const bool fix = a.split_fill == round && (long)a.ns * round >= a.max_seq;
    auto go = [&](auto kernel) {
      if (ev.start) {
        hipExtLaunchKernelGGL(kernel, grid, dim3(kAttnWaves * 64), 0, s, ev.start, ev.stop, 0, a);
        ev.used = true;
      } else {
        hipLaunchKernelGGL(kernel, grid, dim3(kAttnWaves * 64), 0, s, a);
      }
    };
    if (kv_type == 0)
      fix ? go(k_attn<HD, G, 0, true>) : go(k_attn<HD, G, 0, false>);
    else
      fix ? go(k_attn<HD, G, 1, true>) : go(k_attn<HD, G, 1, false>);
    return hipGetLastError();
  }
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

namespace {
template <int HD, int G>
const void* attn_kernel_t(int kv_type) {
  if constexpr (G >= 4)
    return kv_type == 0 ? reinterpret_cast<const void*>(&k_attn_hg<HD, G, 0>)
                        : reinterpret_cast<const void*>(&k_attn_hg<HD, G, 1>);
  else
    return kv_type == 0 ? reinterpret_cast<const void*>(&k_attn<HD, G, 0, false>)
                        : reinterpret_cast<const void*>(&k_attn<HD, G, 1, false>);
}
template <int HD>
const void* attn_kernel_hd(int group, int kv_type) {
  switch (group) {
    case 1: return attn_kernel_t<HD, 1>(kv_type);
    case 2: return attn_kernel_t<HD, 2>(kv_type);
    case 4: return attn_kernel_t<HD, 4>(kv_type);
    case 8: return attn_kernel_t<HD, 8>(kv_type);
    default: return nullptr;
  }
}
}  // namespace

int attn_resident_groups(int head_dim, int group, int kv_type) {
  const void* f = head_dim == 64 ? attn_kernel_hd<64>(group, kv_type)
                : head_dim == 128 ? attn_kernel_hd<128>(group, kv_type)
                : head_dim == 256 ? attn_kernel_hd<256>(group, kv_type) : nullptr;
  if (!f) return 0;
  const int threads = (group >= 4 ? kHgWaves : kAttnWaves) * kWave;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, 0) != hipSuccess) return 0;
  return n;
}

int attn_round_positions(int head_dim, int group) {
  if (group >= 4) return kHgWaves * hg_batch(head_dim, group);   // k_attn_hg: one batch per wave
  const int rows_per_load = kWave / (head_dim / 8);
  return attn_rows_per_lane(group) * kAttnWaves * rows_per_load;
}

bool attention_supported(int head_dim, int group) {
  return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

hipError_t launch_attention(int head_dim, int group, int kv_type, const AttnArgs& a, hipStream_t s) {
  if (a.ns < 1 || a.ns > kMaxSplits) return hipErrorInvalidValue;   // merge weights: kMaxSplits per head
  if (head_dim == 64) return launch_attn_hd<64>(group, kv_type, a, s);
  if (head_dim == 128) return launch_attn_hd<128>(group, kv_type, a, s);
  if (head_dim == 256) return launch_attn_hd<256>(group, kv_type, a, s);   // Gemma
  return hipErrorInvalidValue;
}

hipError_t launch_attention_merge(int head_dim, int group, const AttnArgs& a, hipStream_t s) {
  if (a.ns < 1 || a.ns > kMaxSplits || a.cnt || !a.out) return hipErrorInvalidValue;
  if (head_dim == 64) return launch_merge_hd<64>(group, a, s);
  if (head_dim == 128) return launch_merge_hd<128>(group, a, s);
  if (head_dim == 256) return launch_merge_hd<256>(group, a, s);
  return hipErrorInvalidValue;
}

hipError_t launch_pool_rows(const float* x, int T, int d, const float* w, const float* ssq, float eps, float* acc,
                            hipStream_t s) {
  if (T < 1 || d < 1 || (w && !ssq)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pool_rows, dim3((d + 255) / 256), dim3(256), 0, s, x, T, d, w, ssq, eps, acc);
  return hipGetLastError();
}

hipError_t launch_embed_finish(const float* acc, int d, int n, float* out, hipStream_t s) {
  if (d < 1 || n < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_embed_finish, dim3(1), dim3(256), 0, s, acc, d, n, out);
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

hipError_t launch_rope_kv_rows(float* qkv, const float* bias, int ld, int qdim, int kvdim, int head_dim, int rope_dim,
                               const float* cs, const int* dpos, uint16_t* kc, uint16_t* vc, int max_seq,
                               int n, hipStream_t s) {
  if (n <= 0 || ld % 2 || qdim % 2 || kvdim % 2 || head_dim % 2 || ld < qdim + 2 * kvdim) return hipErrorInvalidValue;
  const int npairs = (qdim + 2 * kvdim) / 2;
  const int gx = (npairs + 255) / 256;
  hipLaunchKernelGGL(k_rope_kv_rows, dim3(gx, n), dim3(256), 0, s, qkv, bias, ld, qdim, kvdim, head_dim, rope_dim,
                     cs, dpos, kc, vc, max_seq);
  return hipGetLastError();
}

hipError_t launch_post_norm(float* hidden, const float* y, const float* w, int n, float eps, uint32_t* xr,
                            const float* nw_out, hipStream_t s) {
  if (n <= 0 || n % 16 || !hidden || !y || !w) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_post_norm, dim3(1), dim3(1024), 0, s, hidden, y, w, n, eps, xr, nw_out);
  return hipGetLastError();
}

hipError_t launch_post_norm_rows(float* hidden, const float* y, const float* w, int n, int T, float eps,
                                 hipStream_t s) {
  if (n <= 0 || T <= 0 || !hidden || !y || !w) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_post_norm_rows, dim3(T), dim3(1024), 0, s, hidden, y, w, n, eps);
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
