// ss_sweep.hip - the whole decode token in one persistent launch (gfx950).
//
// Grid: one workgroup per compute unit, all co-resident (cooperative
// launch). Each workgroup has kSweepComputeWaves compute waves and one
// control wave.
//
// * Compute waves only read weights and the KV cache (plain loads, constant
//   during the launch) and LDS, and do the arithmetic. At the end of every
//   phase they already issue the weight (or K/V) loads of their first two
//   work items of the next phase, so the weight stream keeps running while
//   the control wave waits for the other workgroups.
// * The control wave does everything that crosses workgroups: the phase
//   epilogue (row sums from LDS, RoPE, KV append, residual, SwiGLU), the
//   stores of the results, its workgroup's progress flag, the wait for the
//   other workgroups' flags, and the staging of the next phase's input into
//   LDS. Its loads never queue behind the compute waves' weight loads
//   (vector memory completes in issue order per wave).
//
// Data handed between workgroups inside the launch is written with the sc1
// cache policy (what agent-scope atomic stores compile to on gfx950: the
// store goes through to memory), and a workgroup publishes its progress flag
// (also sc1) only after those stores have completed (s_waitcnt vmcnt(0)).
// Every exchange buffer has its own address per layer and phase, so within a
// launch each address is written once, before anyone reads it: consumers can
// read it with ordinary loads - the first read on an XCD misses its L2 and
// fetches the new data, later reads on that XCD hit - instead of all 256
// workgroups fetching the same lines from memory. Flags are polled with sc1
// loads. No agent-scope fence (L2 writeback/invalidate) is used. Every wait has a wall-clock bound: a workgroup that gives up raises
// the abort word, every other workgroup stops at its next wait, and the
// launch ends with the error recorded for the host.
//
// Matvec inputs travel as x records: 16 consecutive values v (the producer
// multiplies in the consumer's RMSNorm weight) as three int8 levels,
// v ~= s3 * (16384*q1 + 128*q2 + q3) with s1 = max|v|/127, s3 = s1/16384,
// which is exact to max|v| * 2.4e-7 (fp32 rounding size). Record words:
// [0,4) q1, [4,8) q2, [8,12) q3 (4 codes per word, value order), [12] 8*sum X
// (the Q4_0 offset term), [13] s3, [14] sum of squares of the unnormalised
// values (the consumer's RMSNorm statistic), [15] 0. The producer encodes
// each record once; consumers copy records straight into LDS. A block dot
// product of 32 weights is then two exact integer sums of v_dot4 over the
// levels and one fp32 rounding per 16 values.

#include <math.h>

#include "ss_device.h"
#include "ss_sweep.h"

namespace ssk {
namespace {

constexpr int kCW = kSweepComputeWaves;
// ------------------------------------------------------------ shapes
__host__ __device__ inline int tiles_of(int cols) { return (cols / 32 + 3) / 4; }
__host__ __device__ inline int rgs_of(int rows) { return (rows + 15) / 16; }
// row groups g = wg, wg + nwg, ... of nrg that workgroup wg owns
__host__ __device__ inline int rg_count(int nrg, int wg, int nwg) {
  return wg < nrg ? (nrg - 1 - wg) / nwg + 1 : 0;
}
__host__ __device__ inline int rg_max(int nrg, int nwg) { return (nrg + nwg - 1) / nwg; }
// tiles per work item: 8 uint4 of codes per lane per item buffer
__host__ __device__ constexpr int item_tiles(int qt, int nmat) { return qt == 8 && nmat == 2 ? 2 : 4; }
__host__ __device__ inline int units_of(int cols, int st) { return (tiles_of(cols) + st - 1) / st; }
// x record words for cols columns including the tile padding of the last item
__host__ __device__ inline int rec_words(int cols, int st) { return units_of(cols, st) * st * 8 * kRW; }
__host__ __device__ constexpr int attn_rows_per_lane_s(int group) {
  return group >= 8 ? 1 : group >= 4 ? 2 : 4;
}

// Shared memory, in words: the launch parameters (the argument block, every
// layer's descriptor, the RoPE row of the position, this workgroup's norm
// weight rows), the x records (aliased by the attention scratch), the row
// partials of the work items, the residual rows owned, and 16 words misc.
// Parameters are read from here rather than from device memory, where every
// read would be a round trip through a memory system the weight stream keeps
// saturated.
constexpr int kArgWords = ((int)sizeof(SweepArgs) + 15) / 16 * 4;
constexpr int kLayerWords = ((int)sizeof(SweepLayer) + 15) / 16 * 4;
static_assert(kLayerWords * 4 == (int)sizeof(SweepLayer), "descriptor copy stride != SweepLayer array stride");
static_assert(kArgWords * 4 >= (int)sizeof(SweepArgs), "argument block larger than its shared-memory slot");

struct LdsPlan {
  int params, x, red, hrow;   // words
  int total() const { return params + x + red + hrow + 16; }
};

__host__ __device__ inline LdsPlan lds_plan(const SweepArgs& a, int hd, int group, int ql, int qh) {
  const int s1 = item_tiles(ql, 1), s2 = item_tiles(ql, 2), sh = item_tiles(qh, 1);
  int x = rec_words(a.d, s1) + a.d;                // layer-0 records + raw embedding row
  int t = rec_words(a.d, s2);
  x = x > t ? x : t;
  t = rec_words(a.d, sh);
  x = x > t ? x : t;
  t = rec_words(a.qdim, s1);
  x = x > t ? x : t;
  t = rec_words(a.ffn, s1);
  x = x > t ? x : t;
  t = group * hd + 2 * hd + kCW * group * (hd + 2);   // attention scratch
  x = x > t ? x : t;
  const int qkv_rows = a.qdim + 2 * a.kvdim;
  int red = rg_max(rgs_of(qkv_rows), a.nwg) * units_of(a.d, s1);
  t = rg_max(rgs_of(a.d), a.nwg) * units_of(a.qdim, s1);
  red = red > t ? red : t;
  t = rg_max(rgs_of(a.ffn), a.nwg) * units_of(a.d, s2) * 2;
  red = red > t ? red : t;
  t = rg_max(rgs_of(a.d), a.nwg) * units_of(a.ffn, s1);
  red = red > t ? red : t;
  t = rg_max(rgs_of(a.vocab), a.nwg) * units_of(a.d, sh);
  red = red > t ? red : t;
  LdsPlan p;
  p.hrow = rg_max(rgs_of(a.d), a.nwg) * 16;
  p.params = kArgWords + a.n_layers * kLayerWords + (a.rope_dim + 3) / 4 * 4 + 2 * p.hrow;
  p.x = x;
  p.red = red * 16;
  return p;
}


// Progress flags: one word per workgroup, the epoch it last published.
// Workgroups 16g .. 16g+15 share one 64-byte line, and the lines of
// successive groups are a page apart (kSweepFlagStride words), so both the
// stores (16 per line) and the polls (a waiter reads one line per group)
// spread over the memory channels instead of meeting on one.
__device__ __forceinline__ bool reached(uint32_t f, uint32_t target) { return (int)(f - target) >= 0; }
__device__ __forceinline__ uint32_t* flag_of(const SweepArgs& a, int w) {
  return a.flags + (size_t)(w / 16) * kSweepFlagStride + w % 16;
}

__device__ __forceinline__ void give_up(const SweepArgs& a, int phase) {
  cst(a.flags + kSweepErr, ((uint32_t)phase << 16) | blockIdx.x);
  cst(a.flags + kSweepAbort, 1u);
}

// Control wave: until every workgroup has published `target`. False when
// the launch is being abandoned.
__device__ bool wait_all(const SweepArgs& a, uint32_t target, int lane, int phase) {
  const uint64_t start = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    // lane l reads flags 4l .. 4l+3 (of each block of 256 workgroups)
    bool ok = true;
    for (int w0 = 0; w0 < a.nwg; w0 += 4 * kWave) {
      const int w = min(w0 + 4 * lane, (a.nwg - 1) & ~3);
      const uint64_t* p = reinterpret_cast<const uint64_t*>(flag_of(a, w));
      const uint64_t f01 = cld64(p), f23 = cld64(p + 1);
      const uint32_t f[4] = {(uint32_t)f01, (uint32_t)(f01 >> 32), (uint32_t)f23, (uint32_t)(f23 >> 32)};
#pragma unroll
      for (int b = 0; b < 4; ++b) ok &= w + b >= a.nwg || reached(f[b], target);
    }
    if (__all(ok)) return true;
    if (cld(a.flags + kSweepAbort) != 0) return false;
    if (__builtin_amdgcn_s_memrealtime() - start > a.timeout_ticks) {
      if (lane == 0) give_up(a, phase);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Control wave: until the workgroups owning row groups [g0, g0+n0),
// [g1, g1+n1), [g2, g2+n2) have published `target`.
__device__ bool wait_groups(const SweepArgs& a, uint32_t target, int lane, int phase, int g0, int n0,
                            int g1, int n1, int g2, int n2) {
  const uint64_t start = __builtin_amdgcn_s_memrealtime();
  const int n = n0 + n1 + n2;
  for (;;) {
    bool ok = true;
    for (int i = lane; i < n; i += kWave) {
      const int g = i < n0 ? g0 + i : i < n0 + n1 ? g1 + i - n0 : g2 + i - n0 - n1;
      ok &= reached(cld(flag_of(a, g % a.nwg)), target);
    }
    if (__all(ok)) return true;
    if (cld(a.flags + kSweepAbort) != 0) return false;
    if (__builtin_amdgcn_s_memrealtime() - start > a.timeout_ticks) {
      if (lane == 0) give_up(a, phase);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Control wave: publish that this workgroup finished `epoch` (after all of
// its stores have completed).
__device__ __forceinline__ void signal(const SweepArgs& a, uint32_t epoch, int lane) {
  vm_drain();
  if (lane == 0) cst(flag_of(a, blockIdx.x), epoch);
}

// Control wave: copy n records (each address written once per launch, see
// the top of the file) into LDS and zero the padding records [n, npad).
__device__ __forceinline__ void stage_recs(uint32_t* xs, const uint32_t* src, int n, int npad, int lane) {
  const int nv = n * 4;   // 16-byte pieces
  for (int i = 0; i < nv; i += kWave) {
    if (i + lane < nv)
      __builtin_amdgcn_global_load_lds((gbl_ptr_t)(src + (size_t)(i + lane) * 4), (lds_ptr_t)(xs + i * 4),
                                       16, 0, 0);
  }
  for (int w = n * kRW + lane; w < npad * kRW; w += kWave) xs[w] = 0u;
  vm_drain();
}

// RMSNorm scale 1/sqrt(mean(x^2) + eps) (tensor.c:114-131) from the records'
// sums of squares; every lane of the wave gets it.
__device__ __forceinline__ float norm_scale(const uint32_t* xs, int nrec, int cols, float eps, int lane) {
  float s = 0.f;
  for (int i = lane; i < nrec; i += kWave) s += __uint_as_float(xs[i * kRW + 14]);
  s = wave_sum(s);
  return 1.0f / sqrtf(s / (float)cols + eps);
}

// ------------------------------------------------------------ matvec work items
// A work item: ST consecutive tiles of one row group of NMAT matrices (gate
// and up share rows and x). Item i of this workgroup's list: row group
// wg + (i / U) * nwg, tiles (i % U) * ST ...
struct MvGeo {
  int ntk, U, n;
};
__device__ __forceinline__ MvGeo mv_geo(int rows, int cols, int st, int wg, int nwg) {
  MvGeo g;
  g.ntk = tiles_of(cols);
  g.U = (g.ntk + st - 1) / st;
  g.n = rg_count(rgs_of(rows), wg, nwg) * g.U;
  return g;
}

template <int QT, int NMAT>
__device__ __forceinline__ void load_item(uint4 (&R)[8], uint32_t (&RS)[4], const PackedMat* w, int ntk, int rg,
                                          int u, int lane) {
  constexpr int kQB = QTraits<QT>::kQB, kNV = kQB / 16, ST = item_tiles(QT, NMAT);
  const int t0 = u * ST;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    const uint16_t* sp = w[m].ds + scale_idx(rg, ntk, t0, lane);
    if constexpr (ST == 4) {
      const uint2 v = *reinterpret_cast<const uint2*>(sp);
      RS[m * 2] = v.x;
      RS[m * 2 + 1] = v.y;
    } else {
      RS[m] = *reinterpret_cast<const uint32_t*>(sp);
    }
#pragma unroll
    for (int k = 0; k < ST; ++k) {
      const int t = min(t0 + k, ntk - 1);   // padding tiles reload the last one; their x is zero
      const uint4* src = reinterpret_cast<const uint4*>(w[m].qs + tile_idx(rg, ntk, t, lane) * kQB);
#pragma unroll
      for (int v = 0; v < kNV; ++v) R[(m * ST + k) * kNV + v] = src[v];
    }
  }
}

template <int QT, int NMAT>
__device__ __forceinline__ void item_fma(float (&acc)[NMAT], const uint4 (&R)[8], const uint32_t (&RS)[4],
                                         const uint32_t* xs, int u, int kb) {
  constexpr int kNV = QTraits<QT>::kQB / 16, ST = item_tiles(QT, NMAT);
#pragma unroll
  for (int k = 0; k < ST; ++k) {
    const uint32_t* ra = xs + (((u * ST + k) * 4 + kb) * 2) * kRW;
    const uint32_t* rb = ra + kRW;
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      float s;
      if constexpr (QT == 2)
        s = q4_dot(R[(m * ST + k) * kNV], ra, rb);
      else
        s = q8_dot(R[(m * ST + k) * kNV], R[(m * ST + k) * kNV + 1], ra, rb);
      const uint32_t sw = RS[m * (ST / 2) + k / 2];
      const float d = h2f((uint16_t)(k & 1 ? sw >> 16 : sw & 0xffffu));
      acc[m] = fmaf(d, s, acc[m]);
    }
  }
}

// Row partials of item i: the 4 lanes of a row (one per block column) are
// added, lanes 0..15 store red[(i * NMAT + m) * 16 + row].
template <int NMAT>
__device__ __forceinline__ void put_red(float* red, int i, float (&acc)[NMAT], int lane) {
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    float v = acc[m];
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    if (lane < 16) red[(i * NMAT + m) * 16 + lane] = v;
  }
}

// Item i = j * U + u of a workgroup's list, tracked as (j, u) and advanced
// without dividing: the row group is wg + j * nwg.
struct ItemPos {
  int i, j, u;
};
__device__ __forceinline__ ItemPos item_pos(int i, int U) {
  ItemPos p;
  p.i = i;
  p.j = 0;
  p.u = i;
  while (p.u >= U) {
    p.u -= U;
    ++p.j;
  }
  return p;
}
__device__ __forceinline__ void item_advance(ItemPos& p, int step, int U) {
  p.i += step;
  p.u += step;
  while (p.u >= U) {
    p.u -= U;
    ++p.j;
  }
}

template <int QT, int NMAT>
__device__ __forceinline__ void load_at(uint4 (&R)[8], uint32_t (&RS)[4], const PackedMat* w, const MvGeo& g,
                                        const ItemPos& p, int lane) {
  load_item<QT, NMAT>(R, RS, w, g.ntk, (int)blockIdx.x + p.j * (int)gridDim.x, p.u, lane);
}

__device__ __forceinline__ void clear(uint4 (&R)[8], uint32_t (&RS)[4]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) R[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) RS[i] = 0;
}

// Issue this wave's first two items of a phase (A: item wave, B: item wave +
// kCW). A buffer without an item is cleared, so that no value of an earlier
// phase stays live in it (it would hold registers through the phases).
template <int QT, int NMAT>
__device__ __forceinline__ void prefetch_items(uint4 (&A)[8], uint32_t (&As)[4], uint4 (&B)[8], uint32_t (&Bs)[4],
                                               const PackedMat* w, const MvGeo& g, int wave, int lane) {
  ItemPos p = item_pos(wave, g.U);
  if (p.i < g.n)
    load_at<QT, NMAT>(A, As, w, g, p, lane);
  else
    clear(A, As);
  item_advance(p, kCW, g.U);
  if (p.i < g.n)
    load_at<QT, NMAT>(B, Bs, w, g, p, lane);
  else
    clear(B, Bs);
}

// A wave's items of a phase, double-buffered: A and B hold items wave and
// wave + kCW on entry; each buffer is reloaded with the item 2*kCW further
// on as soon as it has been used.
__device__ __forceinline__ void stamp(const SweepArgs& a, int p, int e, int lane);

template <int QT, int NMAT>
__device__ __forceinline__ void run_items(uint4 (&A)[8], uint32_t (&As)[4], uint4 (&B)[8], uint32_t (&Bs)[4],
                                          const PackedMat* w, const MvGeo& g, const uint32_t* xs, float* red,
                                          int wave, int lane, const SweepArgs& a, int ph) {
  const int kb = lane / 16;
  ItemPos pa = item_pos(wave, g.U);       // item in A
  ItemPos pb = pa;                         // item in B
  item_advance(pb, kCW, g.U);
  while (pa.i < g.n) {
    {
      float acc[NMAT];
#pragma unroll
      for (int m = 0; m < NMAT; ++m) acc[m] = 0.f;
      item_fma<QT, NMAT>(acc, A, As, xs, pa.u, kb);
      put_red<NMAT>(red, pa.i, acc, lane);
      if (pa.i == 0) stamp(a, ph, 5, lane);
      item_advance(pa, 2 * kCW, g.U);
      if (pa.i < g.n) load_at<QT, NMAT>(A, As, w, g, pa, lane);
    }
    if (pb.i < g.n) {
      float acc[NMAT];
#pragma unroll
      for (int m = 0; m < NMAT; ++m) acc[m] = 0.f;
      item_fma<QT, NMAT>(acc, B, Bs, xs, pb.u, kb);
      put_red<NMAT>(red, pb.i, acc, lane);
      item_advance(pb, 2 * kCW, g.U);
      if (pb.i < g.n) load_at<QT, NMAT>(B, Bs, w, g, pb, lane);
    }
  }
}

// Control wave: the rows of local row groups j0..j0+3 (lane = 16*(j-j0) + r)
// summed over their items in item order (results independent of timing).
template <int NMAT>
__device__ __forceinline__ void rg_sums(float (&v)[NMAT], const float* red, int j, int U, int r, bool valid) {
#pragma unroll
  for (int m = 0; m < NMAT; ++m) v[m] = 0.f;
  if (!valid) return;
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int m = 0; m < NMAT; ++m) v[m] += red[((j * U + u) * NMAT + m) * 16 + r];
}

// ------------------------------------------------------------ attention
// Item: KV head kvh, split sp of positions [t0, t1), t1 <= pos + 1; the
// positions below pos come from the cache (written by earlier launches),
// position pos (this token's K/V, written by this launch) from LDS.
struct AttnItem {
  bool has;
  int kvh, sp, t0, t1, active;
};
__device__ __forceinline__ AttnItem attn_item(const SweepArgs& a, int pos) {
  AttnItem it;
  it.has = false;
  it.kvh = it.sp = it.t0 = it.t1 = it.active = 0;
  const int i = blockIdx.x;
  if (i >= a.n_kv_heads * a.ns) return it;
  int chunk, active;
  attn_chunks(pos + 1, a.ns, 0, chunk, active);
  it.kvh = i / a.ns;
  it.sp = i % a.ns;
  it.active = active;
  if (it.sp >= active) return it;
  it.has = true;
  it.t0 = it.sp * chunk;
  it.t1 = min(pos + 1, it.t0 + chunk);
  return it;
}

template <int HD, int G>
struct AttnShape {
  static constexpr int kLpr = HD / 8;               // lanes per K/V row
  static constexpr int kRpi = kWave / kLpr;         // rows per wave load
  static constexpr int kK = attn_rows_per_lane_s(G);
  static constexpr int kRound = kK * kCW * kRpi;    // positions per round
};

// K and V chunks (8 fp16 values) of a round's cached rows (below `end`,
// which is at most the current position) into R[k], R[4 + k]; rows at or
// past `end` load row end - 1 instead, or are zero when the round has no
// cached row (the caller masks them). Every register of R is defined here,
// and the current position, which this launch writes, is never read.
template <int HD, int G>
__device__ __forceinline__ void attn_load(uint4 (&R)[8], const uint16_t* kc, const uint16_t* vc, int r0, int end,
                                          int wave, int lane) {
  using S = AttnShape<HD, G>;
  const int c = lane % S::kLpr, rsub = lane / S::kLpr;
  if (r0 < end) {
#pragma unroll
    for (int k = 0; k < S::kK; ++k) {
      const int p = min(r0 + (k * kCW + wave) * S::kRpi + rsub, end - 1);
      R[k] = *reinterpret_cast<const uint4*>(kc + (size_t)p * HD + c * 8);
      R[4 + k] = *reinterpret_cast<const uint4*>(vc + (size_t)p * HD + c * 8);
    }
  } else {
#pragma unroll
    for (int k = 0; k < S::kK; ++k) R[k] = R[4 + k] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int k = S::kK; k < 4; ++k) R[k] = R[4 + k] = make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ void unpack8(const uint4 c, float (&v)[8]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
    v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
  }
}

template <int N>
__device__ __forceinline__ float sum_lanes_s(float v) {
  v += dppf<0xb1>(v);
  v += dppf<0x4e>(v);
  if constexpr (N >= 8) v += dppf<0x141>(v);
  if constexpr (N >= 16) v += dppf<0x140>(v);
  return v;
}

// Compute waves: online-softmax attention of the G query heads of KV head
// kvh over [t0, t1) (layer_scheduler.c:415-468): scores (q.k) * scale, max,
// exp, sum, sum of p*v, per wave; the wave's (o, m, l) go to LDS.
template <int HD, int G>
__device__ void attn_compute(uint4 (&R)[8], const SweepArgs& a, const AttnItem& it, int pos, const uint16_t* kc,
                             const uint16_t* vc, const float* qs, const float* kcur, const float* vcur,
                             float* wpart, int wave, int lane) {
  using S = AttnShape<HD, G>;
  const int c = lane % S::kLpr, rsub = lane / S::kLpr;
  const int cend = min(it.t1, pos);   // cached positions end
  float q[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) q[g][e] = qs[g * HD + c * 8 + e];
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
  }
  for (int r0 = it.t0; r0 < it.t1; r0 += S::kRound) {
    if (r0 != it.t0) attn_load<HD, G>(R, kc, vc, r0, cend, wave, lane);
    float sc[G][S::kK];
#pragma unroll
    for (int k = 0; k < S::kK; ++k) {
      const int p = r0 + (k * kCW + wave) * S::kRpi + rsub;
      const bool live = p < it.t1;
      float kv[8];
      unpack8(R[k], kv);
      if (p == pos) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kv[e] = kcur[c * 8 + e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) kv[e] = live ? kv[e] : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(q[g][e], kv[e], d);
        d = sum_lanes_s<S::kLpr>(d) * a.attn_scale;   // (q . k) / sqrt(hd), layer_scheduler.c:442-446
        sc[g][k] = live ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mt = sc[g][0];
#pragma unroll
      for (int k = 1; k < S::kK; ++k) mt = fmaxf(mt, sc[g][k]);
      mt = wave_max(mt);
      const float mn = fmaxf(m[g], mt);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float corr = expf(m[g] - mref);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= corr;
#pragma unroll
      for (int k = 0; k < S::kK; ++k) {
        const int p = r0 + (k * kCW + wave) * S::kRpi + rsub;
        const float pw = expf(sc[g][k] - mref);
        ps += pw;
        float vv[8];
        unpack8(R[4 + k], vv);
        if (p == pos) {
#pragma unroll
          for (int e = 0; e < 8; ++e) vv[e] = vcur[c * 8 + e];
        }
        const bool live = p < it.t1;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pw, live ? vv[e] : 0.f, o[g][e]);
      }
      l[g] = l[g] * corr + wave_sum(c == 0 ? ps : 0.f);
      m[g] = mn;
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      for (int off = S::kLpr; off < kWave; off <<= 1) o[g][e] += __shfl_xor(o[g][e], off, kWave);
  float* wp = wpart + wave * G * (HD + 2);
  if (rsub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) wp[g * (HD + 2) + c * 8 + e] = o[g][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wp[g * (HD + 2) + HD] = m[g];
      wp[g * (HD + 2) + HD + 1] = l[g];
    }
  }
}

// ------------------------------------------------------------ tracing
// Control wave, lane 0: stamp event e of phase p (when tracing is on).
__device__ __forceinline__ void stamp(const SweepArgs& a, int p, int e, int lane) {
  uint64_t* t = a.trace;
  if (t && lane == 0) {
    const size_t per_wg = kSweepTraceHead + kSweepTracePerPhase * (5 * (size_t)a.n_layers + 1);
    t[blockIdx.x * per_wg + kSweepTraceHead + kSweepTracePerPhase * p + e] = __builtin_amdgcn_s_memrealtime();
  }
}

// ------------------------------------------------------------ the kernel
struct Lds {
  const SweepLayer* layers;   // every layer's descriptor
  float* rope;                // (cos, sin) pairs of the token's position, rope_dim
  float* nrm;                 // norm weights of the residual rows owned: [0, nh) ffn_norm of
                              // this layer, [nh, 2 nh) attn_norm of the next (or output_norm)
  uint32_t* x;
  float* red;
  float* hrow;
  uint32_t* misc;             // [0] norm scale, [1] abort
};

// Residual row groups of d that this workgroup owns: wg, wg + nwg, ...
__device__ __forceinline__ int own_rgs(const SweepArgs& a) { return rg_count(rgs_of(a.d), blockIdx.x, a.nwg); }

// Every wave: the x records of embedding * attn_norm[0] and the residual
// rows this workgroup owns, from the raw row the control wave staged.
template <int S1>
__device__ __forceinline__ void encode_embedding(const SweepArgs& a, const Lds& s, int wave, int lane) {
  const int d = a.d, nwg = a.nwg, wg = blockIdx.x;
  const float* raw = reinterpret_cast<const float*>(s.x + rec_words(d, S1));
  const float* nw = s.layers[0].attn_norm;
  const int npad = rec_words(d, S1) / kRW;
  const int r = lane & 15;
  for (int j = wave * 4 + lane / 16; j < npad; j += (kCW + 1) * 4) {
    if (j < d / 16) {
      const float hv = raw[j * 16 + r];
      const Enc e = enc16(hv * nw[j * 16 + r], hv);
      put_rec_lds(s.x + j * kRW, e, r);
      if (j % nwg == wg) s.hrow[(j / nwg) * 16 + r] = hv;
    } else {
      s.x[j * kRW + r] = 0u;
    }
  }
}

// The compute waves' side of the token. Every __syncthreads here pairs with
// one in ctrl_main.
template <int QL, int QH, int HD, int G>
__device__ __forceinline__ void compute_main(const SweepArgs& a, const Lds& s, int pos, int with_head, int wave,
                                             int lane) {
  constexpr int S1 = item_tiles(QL, 1), S2 = item_tiles(QL, 2), SH = item_tiles(QH, 1);
  const int wg = blockIdx.x, nwg = a.nwg, d = a.d;
  const AttnItem it = attn_item(a, pos);
  const float* qs = reinterpret_cast<const float*>(s.x);   // attention scratch (aliases x)
  const float* kcur = qs + G * HD;
  const float* vcur = kcur + HD;
  float* wpart = const_cast<float*>(vcur) + HD;

  uint4 A[8], B[8];
  uint32_t As[4], Bs[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) A[i] = B[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) As[i] = Bs[i] = 0;

  const int tl = wave == 0 ? lane : 1;   // compute wave 0, lane 0 stamps the trace
  prefetch_items<QL, 1>(A, As, B, Bs, &s.layers[0].qkv, mv_geo(a.qdim + 2 * a.kvdim, d, S1, wg, nwg), wave,
                        lane);
  __syncthreads();
  encode_embedding<S1>(a, s, wave, lane);
  __syncthreads();

  for (int l = 0; l < a.n_layers; ++l) {
    const SweepLayer* ly = s.layers + l;
    // Each phase: this wave's work items, the first barrier (the control wave
    // takes the row partials), then the loads of the next phase's first items
    // (issuing them can stall while the memory system is saturated, so they
    // come after the barrier the control wave waits for), then the second
    // barrier (the next phase's input is staged).
    // 1. [Wq;Wk;Wv]; then the K/V loads of this workgroup's attention split
    stamp(a, 5 * l, 4, tl);
    run_items<QL, 1>(A, As, B, Bs, &ly->qkv, mv_geo(a.qdim + 2 * a.kvdim, d, S1, wg, nwg), s.x, s.red, wave,
                     lane, a, 5 * l);
    stamp(a, 5 * l, 6, tl);
    __syncthreads();
    const uint16_t* kcl = ly->kc + (size_t)it.kvh * a.max_seq * HD;
    const uint16_t* vcl = ly->vc + (size_t)it.kvh * a.max_seq * HD;
    if (it.has)
      attn_load<HD, G>(A, kcl, vcl, it.t0, min(it.t1, pos), wave, lane);
    else
      clear(A, As);
    stamp(a, 5 * l, 7, tl);
    __syncthreads();
    if (s.misc[1]) return;
    // 2. attention
    stamp(a, 5 * l + 1, 4, tl);
    if (it.has) attn_compute<HD, G>(A, a, it, pos, kcl, vcl, qs, kcur, vcur, wpart, wave, lane);
    stamp(a, 5 * l + 1, 6, tl);
    __syncthreads();
    const MvGeo g_o = mv_geo(d, a.qdim, S1, wg, nwg);
    prefetch_items<QL, 1>(A, As, B, Bs, &ly->o, g_o, wave, lane);
    stamp(a, 5 * l + 1, 7, tl);
    __syncthreads();
    if (s.misc[1]) return;
    // 3. Wo
    stamp(a, 5 * l + 2, 4, tl);
    run_items<QL, 1>(A, As, B, Bs, &ly->o, g_o, s.x, s.red, wave, lane, a, 5 * l + 2);
    stamp(a, 5 * l + 2, 6, tl);
    __syncthreads();
    const MvGeo g_gu = mv_geo(a.ffn, d, S2, wg, nwg);
    prefetch_items<QL, 2>(A, As, B, Bs, &ly->gate, g_gu, wave, lane);
    stamp(a, 5 * l + 2, 7, tl);
    __syncthreads();
    if (s.misc[1]) return;
    // 4. gate, up
    stamp(a, 5 * l + 3, 4, tl);
    run_items<QL, 2>(A, As, B, Bs, &ly->gate, g_gu, s.x, s.red, wave, lane, a, 5 * l + 3);
    stamp(a, 5 * l + 3, 6, tl);
    __syncthreads();
    const MvGeo g_dn = mv_geo(d, a.ffn, S1, wg, nwg);
    prefetch_items<QL, 1>(A, As, B, Bs, &ly->down, g_dn, wave, lane);
    stamp(a, 5 * l + 3, 7, tl);
    __syncthreads();
    if (s.misc[1]) return;
    // 5. down; then the first items of the next layer or of the LM head
    stamp(a, 5 * l + 4, 4, tl);
    run_items<QL, 1>(A, As, B, Bs, &ly->down, g_dn, s.x, s.red, wave, lane, a, 5 * l + 4);
    stamp(a, 5 * l + 4, 6, tl);
    __syncthreads();
    if (l + 1 < a.n_layers)
      prefetch_items<QL, 1>(A, As, B, Bs, &s.layers[l + 1].qkv, mv_geo(a.qdim + 2 * a.kvdim, d, S1, wg, nwg),
                            wave, lane);
    else if (with_head)
      prefetch_items<QH, 1>(A, As, B, Bs, &a.out, mv_geo(a.vocab, d, SH, wg, nwg), wave, lane);
    stamp(a, 5 * l + 4, 7, tl);
    __syncthreads();
    if (s.misc[1]) return;
  }
  if (with_head) {
    stamp(a, 5 * a.n_layers, 4, tl);
    run_items<QH, 1>(A, As, B, Bs, &a.out, mv_geo(a.vocab, d, SH, wg, nwg), s.x, s.red, wave, lane, a,
                     5 * a.n_layers);
    stamp(a, 5 * a.n_layers, 6, tl);
    __syncthreads();
  }
}

// The control wave's side of the token.
template <int QL, int QH, int HD, int G>
__device__ __forceinline__ void ctrl_main(const SweepArgs& a, const Lds& s, int pos, uint32_t epoch0, int with_head,
                                          int lane) {
  constexpr int S1 = item_tiles(QL, 1), S2 = item_tiles(QL, 2), SH = item_tiles(QH, 1);
  const int wg = blockIdx.x, nwg = a.nwg, d = a.d, L = a.n_layers;
  const int r = lane & 15;
  const int rec_d = d / 16;
  const AttnItem it = attn_item(a, pos);
  float* const qs = reinterpret_cast<float*>(s.x);
  float* const kcur = qs + G * HD;
  float* const vcur = kcur + HD;
  const float* const wpart = vcur + HD;
  const int n_hrg = own_rgs(a);

  // ---- token embedding (layer_scheduler.c:578-595), staged by every workgroup
  if (lane == 0) s.misc[1] = 0;
  for (int i = lane; i < a.rope_dim; i += kWave) s.rope[i] = a.rope_cs[(size_t)pos * a.rope_dim + i];
  if (a.trace && lane == 0)
    a.trace[blockIdx.x * (kSweepTraceHead + kSweepTracePerPhase * (5 * (size_t)L + 1))] =
        __builtin_amdgcn_s_memrealtime();
  {
    const int tok = a.tokens[pos];
    float* raw = reinterpret_cast<float*>(s.x + rec_words(d, S1));
    const int ntk = tiles_of(d);
    const int kqb = a.embd_type == 2 ? 16 : 32;
    for (int b = lane; b < d / 32; b += kWave) {
      const int tl = tile_lane(tok % 16, b);
      const float sc = h2f(a.embd.ds[scale_idx(tok / 16, ntk, b / 4, tl)]);
      const uint8_t* q = a.embd.qs + tile_idx(tok / 16, ntk, b / 4, tl) * kqb;
      if (a.embd_type == 2) {
        for (int j = 0; j < 16; ++j) {
          const uint8_t v = q[j];
          raw[b * 32 + j] = sc * (float)((int)(v & 0xF) - 8);
          raw[b * 32 + j + 16] = sc * (float)((int)(v >> 4) - 8);
        }
      } else {
        for (int j = 0; j < 32; ++j) raw[b * 32 + j] = sc * (float)(int8_t)q[j];
      }
    }
  }
  __syncthreads();
  encode_embedding<S1>(a, s, kCW, lane);
  __syncthreads();

  uint32_t ep = epoch0;   // this workgroup's last published epoch
  for (int l = 0; l < L; ++l) {
    const SweepLayer* ly = s.layers + l;
    // ---- 1. rmsnorm(attn_norm) -> [Wq;Wk;Wv] -> RoPE -> KV append (:320-413)
    if (l == 0) s.misc[0] = __float_as_uint(norm_scale(s.x, rec_d, d, a.eps, lane));
    {
      // the norm weights this layer's epilogues apply to the residual rows owned
      const int nh = rg_max(rgs_of(d), nwg) * 16;
      const float* fw = ly->ffn_norm;
      const float* nw = l + 1 < L ? s.layers[l + 1].attn_norm : a.out_norm;
      for (int i = lane; i < n_hrg * 16; i += kWave) {
        const int row = (wg + (i >> 4) * nwg) * 16 + (i & 15);
        s.nrm[i] = fw[row];
        s.nrm[nh + i] = nw ? nw[row] : 1.0f;
      }
    }
    __syncthreads();
    stamp(a, 5 * l, 0, lane);
    {
      const float scale = __uint_as_float(s.misc[0]);
      const int qkv_rows = a.qdim + 2 * a.kvdim;
      const int nrg = rg_count(rgs_of(qkv_rows), wg, nwg);
      const int U = units_of(d, S1);
      for (int j0 = 0; j0 < nrg; j0 += 4) {
        const int j = j0 + lane / 16;
        float v[1];
        rg_sums<1>(v, s.red, j, U, r, j < nrg);
        const int row = (wg + j * nwg) * 16 + r;
        const bool valid = j < nrg && row < qkv_rows;
        const float x = v[0] * scale;
        const float partner = __shfl_xor(x, 1, kWave);
        float out = x;
        if (row < a.qdim + a.kvdim) {   // RoPE, GPT-J pairs (tensor.c:249-274)
          const int i = (row < a.qdim ? row : row - a.qdim) % HD;
          const int i0 = i & ~1;
          if (i0 < a.rope_dim) {
            const float cv = s.rope[i0], sv = s.rope[i0 + 1];
            out = (i & 1) ? partner * sv + x * cv : x * cv - partner * sv;
          }
        }
        const float pout = __shfl_xor(out, 1, kWave);
        if (valid) {
          if (row < a.qdim) {
            cstf(a.q + (size_t)l * a.qdim + row, out);
          } else if ((r & 1) == 0) {   // fp16 pair into the cache at pos
            const bool is_v = row >= a.qdim + a.kvdim;
            const int kr = row - a.qdim - (is_v ? a.kvdim : 0);
            uint16_t* c = is_v ? ly->vc : ly->kc;
            const size_t e = ((size_t)(kr / HD) * a.max_seq + pos) * HD + kr % HD;
            cst(reinterpret_cast<uint32_t*>(c + e), (uint32_t)f2h(out) | ((uint32_t)f2h(pout) << 16));
          }
        }
      }
      signal(a, ++ep, lane);
      stamp(a, 5 * l, 1, lane);
      if (it.has) {
        const int kvh = it.kvh;
        if (!wait_groups(a, ep, lane, 5 * l + 1, kvh * G * HD / 16, G * HD / 16, (a.qdim + kvh * HD) / 16,
                         HD / 16, (a.qdim + a.kvdim + kvh * HD) / 16, HD / 16)) {
          s.misc[1] = 1;
        } else {
          const float* ql = a.q + (size_t)l * a.qdim + kvh * G * HD;
          for (int i = lane; i < G * HD; i += kWave) qs[i] = ql[i];
          for (int i = lane; i < HD / 2; i += kWave) {
            const size_t e = ((size_t)kvh * a.max_seq + pos) * HD + 2 * i;
            const uint32_t kw = cld(reinterpret_cast<const uint32_t*>(ly->kc + e));
            const uint32_t vw = cld(reinterpret_cast<const uint32_t*>(ly->vc + e));
            kcur[2 * i] = h2f((uint16_t)(kw & 0xffffu));
            kcur[2 * i + 1] = h2f((uint16_t)(kw >> 16));
            vcur[2 * i] = h2f((uint16_t)(vw & 0xffffu));
            vcur[2 * i + 1] = h2f((uint16_t)(vw >> 16));
          }
        }
      }
      stamp(a, 5 * l, 2, lane);
      stamp(a, 5 * l, 3, lane);
    }
    __syncthreads();
    if (s.misc[1]) return;

    // ---- 2. attention over positions 0..pos (:415-468): combine the waves,
    // then the last split of a KV head to finish merges all of its splits
    __syncthreads();
    stamp(a, 5 * l + 1, 0, lane);
    if (it.has) {
      float* const part_l = a.part + (size_t)l * a.n_kv_heads * a.ns * G * (HD + 2);
      uint32_t* const arec_l = a.arec + (size_t)l * a.qdim;
      float* pp = part_l + ((size_t)it.kvh * a.ns + it.sp) * G * (HD + 2);
      for (int i = lane; i < G * HD; i += kWave) {
        const int g = i / HD, dd = i % HD;
        float M = -INFINITY;
        for (int w = 0; w < kCW; ++w) M = fmaxf(M, wpart[(w * G + g) * (HD + 2) + HD]);
        float so = 0.f, sl = 0.f;
        for (int w = 0; w < kCW; ++w) {
          const float* wpw = wpart + (w * G + g) * (HD + 2);
          const float f = expf(wpw[HD] - M);
          so = fmaf(f, wpw[dd], so);
          sl = fmaf(f, wpw[HD + 1], sl);
        }
        if (it.active == 1) {
          const float ov = so / sl;
          const Enc e = enc16(ov, ov);
          put_rec_global(arec_l + (size_t)(((it.kvh * G + g) * HD + dd - r) / 16) * kRW, e, r);
        } else {
          cstf(pp + g * (HD + 2) + dd, so);
          if (dd == 0) {
            cstf(pp + g * (HD + 2) + HD, M);
            cstf(pp + g * (HD + 2) + HD + 1, sl);
          }
        }
      }
      if (it.active > 1) {
        vm_drain();
        uint32_t old = 0;
        if (lane == 0)
          old = __hip_atomic_fetch_add(a.att_cnt + l * a.n_kv_heads + it.kvh, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, kWave);
        if ((int)old == it.active - 1) {
          const float* hp = part_l + (size_t)it.kvh * a.ns * G * (HD + 2);
          for (int g = 0; g < G; ++g) {
            float ms = -INFINITY;
            for (int sp = lane; sp < it.active; sp += kWave) ms = fmaxf(ms, cldf(hp + (sp * G + g) * (HD + 2) + HD));
            const float M = wave_max(ms);
            float ls = 0.f;
            for (int sp = lane; sp < it.active; sp += kWave) {
              const float* q = hp + (sp * G + g) * (HD + 2);
              ls += cldf(q + HD + 1) * expf(cldf(q + HD) - M);
            }
            const float inv = 1.0f / wave_sum(ls);
            for (int dd = lane; dd < HD; dd += kWave) {
              float acc = 0.f;
              for (int sp0 = 0; sp0 < it.active; sp0 += 8) {
                float ov[8], mv[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                  const float* q = hp + (min(sp0 + k, it.active - 1) * G + g) * (HD + 2);
                  ov[k] = cldf(q + dd);
                  mv[k] = cldf(q + HD);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k)
                  if (sp0 + k < it.active) acc = fmaf(ov[k], expf(mv[k] - M) * inv, acc);
              }
              const Enc e = enc16(acc, acc);
              put_rec_global(arec_l + (size_t)(((it.kvh * G + g) * HD + dd - r) / 16) * kRW, e, r);
            }
          }
        }
      }
    }
    signal(a, ++ep, lane);
    stamp(a, 5 * l + 1, 1, lane);
    if (!wait_all(a, ep, lane, 5 * l + 2)) s.misc[1] = 1;
    stamp(a, 5 * l + 1, 2, lane);
    if (!s.misc[1]) stage_recs(s.x, a.arec + (size_t)l * a.qdim, a.qdim / 16, rec_words(a.qdim, S1) / kRW, lane);
    stamp(a, 5 * l + 1, 3, lane);
    __syncthreads();
    if (s.misc[1]) return;

    // ---- 3. hidden += Wo attn (:470-484); x of the FFN = hidden * ffn_norm
    __syncthreads();
    stamp(a, 5 * l + 2, 0, lane);
    {
      const int U = units_of(a.qdim, S1);
      for (int j0 = 0; j0 < n_hrg; j0 += 4) {
        const int j = j0 + lane / 16;
        float v[1];
        rg_sums<1>(v, s.red, j, U, r, j < n_hrg);
        if (j >= n_hrg) continue;   // whole 16-lane rows
        const int row = (wg + j * nwg) * 16 + r;
        const float hn = s.hrow[j * 16 + r] + v[0];   // layer_scheduler.c:484
        s.hrow[j * 16 + r] = hn;
        const Enc e = enc16(hn * s.nrm[j * 16 + r], hn);
        put_rec_global(a.hrec + (size_t)(2 * l) * d + (size_t)(wg + j * nwg) * kRW, e, r);
      }
    }
    signal(a, ++ep, lane);
    stamp(a, 5 * l + 2, 1, lane);
    if (!wait_all(a, ep, lane, 5 * l + 3)) {
      s.misc[1] = 1;
    } else {
      stamp(a, 5 * l + 2, 2, lane);
      stage_recs(s.x, a.hrec + (size_t)(2 * l) * d, rec_d, rec_words(d, S2) / kRW, lane);
      s.misc[0] = __float_as_uint(norm_scale(s.x, rec_d, d, a.eps, lane));
      stamp(a, 5 * l + 2, 3, lane);
    }
    __syncthreads();
    if (s.misc[1]) return;

    // ---- 4. rmsnorm(ffn_norm) -> gate, up -> silu(gate) * up (:486-550)
    __syncthreads();
    stamp(a, 5 * l + 3, 0, lane);
    {
      const float scale = __uint_as_float(s.misc[0]);
      const int nrg = rg_count(rgs_of(a.ffn), wg, nwg);
      const int U = units_of(d, S2);
      for (int j0 = 0; j0 < nrg; j0 += 4) {
        const int j = j0 + lane / 16;
        float v[2];
        rg_sums<2>(v, s.red, j, U, r, j < nrg);
        if (j >= nrg) continue;
        const float gv = v[0] * scale, uv = v[1] * scale;
        const float f = uv * (gv / (1.0f + expf(-gv)));   // layer_scheduler.c:540-547
        const Enc e = enc16(f, f);
        put_rec_global(a.frec + (size_t)l * a.ffn + (size_t)(wg + j * nwg) * kRW, e, r);
      }
    }
    signal(a, ++ep, lane);
    stamp(a, 5 * l + 3, 1, lane);
    if (!wait_all(a, ep, lane, 5 * l + 4)) s.misc[1] = 1;
    stamp(a, 5 * l + 3, 2, lane);
    if (!s.misc[1]) stage_recs(s.x, a.frec + (size_t)l * a.ffn, a.ffn / 16, rec_words(a.ffn, S1) / kRW, lane);
    stamp(a, 5 * l + 3, 3, lane);
    __syncthreads();
    if (s.misc[1]) return;

    // ---- 5. hidden += Wdown act (:552-566); x of the next layer (or head)
    const bool last = l == L - 1;
    __syncthreads();
    stamp(a, 5 * l + 4, 0, lane);
    {
      const int nh = rg_max(rgs_of(d), nwg) * 16;
      const int U = units_of(a.ffn, S1);
      for (int j0 = 0; j0 < n_hrg; j0 += 4) {
        const int j = j0 + lane / 16;
        float v[1];
        rg_sums<1>(v, s.red, j, U, r, j < n_hrg);
        if (j >= n_hrg) continue;
        const int row = (wg + j * nwg) * 16 + r;
        const float hn = s.hrow[j * 16 + r] + v[0];   // layer_scheduler.c:566
        s.hrow[j * 16 + r] = hn;
        if (last) a.hidden[row] = hn;
        const Enc e = enc16(hn * s.nrm[nh + j * 16 + r], hn);
        put_rec_global(a.hrec + (size_t)(2 * l + 1) * d + (size_t)(wg + j * nwg) * kRW, e, r);
      }
    }
    signal(a, ++ep, lane);
    stamp(a, 5 * l + 4, 1, lane);
    if (!last || with_head) {
      if (!wait_all(a, ep, lane, 5 * l + 5)) {
        s.misc[1] = 1;
      } else {
        stamp(a, 5 * l + 4, 2, lane);
        stage_recs(s.x, a.hrec + (size_t)(2 * l + 1) * d, rec_d, rec_words(d, last ? SH : S1) / kRW, lane);
        s.misc[0] = __float_as_uint(norm_scale(s.x, rec_d, d, a.eps, lane));
        stamp(a, 5 * l + 4, 3, lane);
      }
    }
    __syncthreads();
    if (s.misc[1]) return;
  }

  if (with_head) {
    // ---- output_norm + LM head + first-max argmax (:634-662, tensor.c:318-328)
    __syncthreads();
    stamp(a, 5 * L, 0, lane);
    const float scale = a.out_norm ? __uint_as_float(s.misc[0]) : 1.0f;
    const int nrg = rg_count(rgs_of(a.vocab), wg, nwg);
    const int U = units_of(d, SH);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j0 = 0; j0 < nrg; j0 += 4) {
      const int j = j0 + lane / 16;
      float v[1];
      rg_sums<1>(v, s.red, j, U, r, j < nrg);
      const int row = (wg + j * nwg) * 16 + r;
      if (j < nrg && row < a.vocab) {
        const float y = v[0] * scale;
        a.logits[row] = y;
        if (beats(y, row, bv, bi)) {
          bv = y;
          bi = row;
        }
      }
    }
    wave_best(bv, bi);
    if (lane == 0)
      cst64(reinterpret_cast<uint64_t*>(a.cand + wg), (uint64_t)__float_as_uint(bv) | ((uint64_t)(uint32_t)bi << 32));
    signal(a, ++ep, lane);
    stamp(a, 5 * L, 1, lane);
    if (wg != 0) return;
    if (!wait_all(a, ep, lane, 5 * L + 1)) return;
    stamp(a, 5 * L, 2, lane);
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int i = lane; i < nwg; i += kWave) {
      const uint64_t c = cld64(reinterpret_cast<const uint64_t*>(a.cand + i));
      const float cv = __uint_as_float((uint32_t)c);
      const int ci = (int)(uint32_t)(c >> 32);
      if (beats(cv, ci, bv, bi)) {
        bv = cv;
        bi = ci;
      }
    }
    wave_best(bv, bi);
    if (lane == 0) {
      if (bi == 0x7fffffff || isnan(a.logits[0])) bi = 0;   // all NaN, or x[0] NaN (tensor.c:319-320)
      a.argmax[0] = bi;
      a.tokens[pos + 1] = bi;
      *a.dpos = pos + 1;
    }
    stamp(a, 5 * L, 3, lane);
  } else {
    if (wg != 0) return;
    if (lane == 0) *a.dpos = pos + 1;
  }
  // every workgroup is past the last attention phase: reset the split counters
  for (int i = lane; i < L * a.n_kv_heads; i += kWave) cst(a.att_cnt + i, 0u);
}

template <int QL, int QH, int HD, int G>
__global__ void __launch_bounds__(kSweepThreads, 1) k_sweep(const SweepLaunch launch) {
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SweepArgs& ga = *launch.args;
  const LdsPlan lp = lds_plan(ga, HD, G, QL, QH);
  {
    // the argument block and the layer descriptors into shared memory
    const uint32_t* src = reinterpret_cast<const uint32_t*>(launch.args);
    for (int i = tid; i < (int)(sizeof(SweepArgs) / 4); i += kSweepThreads) smem[i] = src[i];
    const uint32_t* ls = reinterpret_cast<const uint32_t*>(ga.layers);
    constexpr int kLw = (int)(sizeof(SweepLayer) / 4);
    for (int i = tid; i < ga.n_layers * kLw; i += kSweepThreads)
      smem[kArgWords + (i / kLw) * kLayerWords + i % kLw] = ls[i];
  }
  Lds s;
  s.layers = reinterpret_cast<const SweepLayer*>(smem + kArgWords);
  s.rope = reinterpret_cast<float*>(smem + kArgWords + ga.n_layers * kLayerWords);
  s.nrm = s.rope + (ga.rope_dim + 3) / 4 * 4;
  s.x = smem + lp.params;
  s.red = reinterpret_cast<float*>(s.x + lp.x);
  s.hrow = s.red + lp.red;
  s.misc = reinterpret_cast<uint32_t*>(s.hrow + lp.hrow);
  const int pos = *ga.dpos;
  __syncthreads();
  const SweepArgs& a = *reinterpret_cast<const SweepArgs*>(smem);
  if (wave == kCW)
    ctrl_main<QL, QH, HD, G>(a, s, pos, launch.epoch0, launch.with_head, lane);
  else
    compute_main<QL, QH, HD, G>(a, s, pos, launch.with_head, wave, lane);
}

template <int QL, int QH, int HD, int G>
hipError_t launch_t(const SweepArgs& a, const SweepLaunch& l, size_t lds, hipStream_t s) {
  void* args[] = {const_cast<SweepLaunch*>(&l)};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&k_sweep<QL, QH, HD, G>), dim3(a.nwg),
                                    dim3(kSweepThreads), args, (unsigned)lds, s);
}

template <int QL, int QH, int HD, int G>
const void* kernel_ptr() {
  return reinterpret_cast<const void*>(&k_sweep<QL, QH, HD, G>);
}

template <int QL, int QH, int HD>
const void* pick_g(int group) {
  switch (group) {
    case 1: return kernel_ptr<QL, QH, HD, 1>();
    case 2: return kernel_ptr<QL, QH, HD, 2>();
    case 4: return kernel_ptr<QL, QH, HD, 4>();
    case 8: return kernel_ptr<QL, QH, HD, 8>();
    default: return nullptr;
  }
}

template <int QL, int QH>
const void* pick_hd(int hd, int group) {
  if (hd == 64) return pick_g<QL, QH, 64>(group);
  if (hd == 128) return pick_g<QL, QH, 128>(group);
  return nullptr;
}

const void* pick(int hd, int group, int ql, int qh) {
  if (ql == 2 && qh == 2) return pick_hd<2, 2>(hd, group);
  if (ql == 2 && qh == 8) return pick_hd<2, 8>(hd, group);
  if (ql == 8 && qh == 8) return pick_hd<8, 8>(hd, group);
  if (ql == 8 && qh == 2) return pick_hd<8, 2>(hd, group);
  return nullptr;
}

}  // namespace

int sweep_phases(int n_layers, int with_head) { return 5 * n_layers + (with_head ? 1 : 0); }

bool sweep_supported(int head_dim, int group, int layer_type, int out_type) {
  return pick(head_dim, group, layer_type, out_type) != nullptr;
}

size_t sweep_lds_bytes(const SweepArgs& a, int head_dim, int group) {
  // the plan depends on the item sizes of the layer and head types; take the
  // largest over the supported combinations so one size serves all
  size_t best = 0;
  const int qts[2] = {2, 8};
  for (int ql : qts)
    for (int qh : qts) {
      const LdsPlan p = lds_plan(a, head_dim, group, ql, qh);
      const size_t b = (size_t)p.total() * 4;
      if (b > best) best = b;
    }
  return best;
}

hipError_t sweep_max_workgroups(int head_dim, int group, int layer_type, int out_type, size_t lds, int* max_wg) {
  const void* k = pick(head_dim, group, layer_type, out_type);
  if (!k) return hipErrorInvalidValue;
  hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kSweepThreads, lds);
  if (e != hipSuccess) return e;
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, dev);
  if (e != hipSuccess) return e;
  *max_wg = per_cu * p.multiProcessorCount;
  return hipSuccess;
}

hipError_t launch_sweep(const SweepArgs& a, const SweepLaunch& l, int head_dim, int group, int layer_type,
                        int out_type, hipStream_t s) {
  if (a.nwg < 1 || a.nwg > kSweepMaxWg) return hipErrorInvalidValue;
  const size_t lds = sweep_lds_bytes(a, head_dim, group);
#define SS_SWEEP_CASE(QL, QH, HD, G)                                                         \
  if (layer_type == QL && out_type == QH && head_dim == HD && group == G) return launch_t<QL, QH, HD, G>(a, l, lds, s);
#define SS_SWEEP_G(QL, QH, HD) \
  SS_SWEEP_CASE(QL, QH, HD, 1) SS_SWEEP_CASE(QL, QH, HD, 2) SS_SWEEP_CASE(QL, QH, HD, 4) SS_SWEEP_CASE(QL, QH, HD, 8)
#define SS_SWEEP_HD(QL, QH) SS_SWEEP_G(QL, QH, 64) SS_SWEEP_G(QL, QH, 128)
  SS_SWEEP_HD(2, 2)
  SS_SWEEP_HD(2, 8)
  SS_SWEEP_HD(8, 8)
  SS_SWEEP_HD(8, 2)
#undef SS_SWEEP_HD
#undef SS_SWEEP_G
#undef SS_SWEEP_CASE
  return hipErrorInvalidValue;
}

}  // namespace ssk
