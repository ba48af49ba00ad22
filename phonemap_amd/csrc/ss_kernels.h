// ss_kernels.h - launch interface of the gfx950 kernels (internal, C++).
// The C-ABI in ss_hip.hip is the only user.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssk {

// Matvec epilogues.
enum Epi : int {
  EPI_STORE = 0,   // y[r] = W x
  EPI_ADD = 1,     // y[r] = W x + y[r]          (residual, layer_scheduler.c:484,566)
  EPI_SWIGLU = 2,  // y[r] = u * silu(g)          (layer_scheduler.c:533-549), W = gate, W2 = up
  EPI_QKV = 3,     // rows of [Wq;Wk;Wv]: RoPE on q/k pairs, K/V appended to the cache
  EPI_LOGITS = 4,  // y[r] = W x, plus one first-max argmax candidate per workgroup in part[]
};

// ggml types: the K-quants (256-weight super-blocks), the other 32-weight
// block types and the float matrices
constexpr int kQ2K = 10, kQ3K = 11, kQ4K = 12, kQ5K = 13, kQ6K = 14;
constexpr int kF32 = 0, kF16 = 1, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_1 = 9;
__host__ __device__ constexpr bool is_kq(int t) { return t >= kQ2K && t <= kQ6K; }
__host__ __device__ constexpr bool is_float(int t) { return t == kF32 || t == kF16; }
// a 32-bit scale entry per block: the (d, m) binary16 pair of Q4_1 / Q5_1,
// or Q8_1's fp32 d
__host__ __device__ constexpr bool is_wide(int t) { return t == kQ4_1 || t == kQ5_1 || t == kQ8_1; }
// The device format a GGUF type is packed into: Q5_0 blocks ((q - 16) * d,
// quantize.c:93-112) become Q8_0 blocks with code q - 16 and the same d, an
// exact restatement; every other type keeps its own format.
__host__ __device__ constexpr int dev_type(int t) { return t == kQ5_0 ? 8 : t; }
// device formats the fp16-MFMA prompt products take (all but F16 / F32)
__host__ __device__ constexpr bool product_format(int t) {
  return t == 2 || t == 8 || t == kQ4_1 || t == kQ5_1 || t == kQ8_1 || is_kq(t);
}
// device code bytes of a 32-weight block: nibbles (Q4_0, Q4_1 and the 2-, 3-
// and 4-bit K-quants), int8 codes (Q8_0, Q5_1, Q8_1, Q5_K, Q6_K), or the
// weights themselves (F16, F32)
__host__ __device__ constexpr int code_bytes_of(int t) {
  return t == 2 || t == kQ4_1 || t == kQ2K || t == kQ3K || t == kQ4K         ? 16
         : t == 8 || t == kQ5_1 || t == kQ8_1 || t == kQ5K || t == kQ6K ? 32
         : t == kF16                                                      ? 64
         : t == kF32                                                      ? 128
                                                                          : 0;
}

// A packed matrix on the device: code plane, scale plane (none for F16 and
// F32) and, for the K-quants, a super-block plane (see ss_gemv.hip).
struct PackedMat {
  const uint8_t* qs;
  const uint16_t* ds;
  const uint32_t* su = nullptr;
};

struct GemvArgs {
  PackedMat w, w2;           // w2: up projection for EPI_SWIGLU
  const float* x;            // input vector [cols]
  const float* nw;           // RMSNorm weight [cols] or nullptr
  float eps;
  float* y;                  // output [rows]
  int rows, cols, type;
  int n_cu;                  // compute units (sizes the grid)
  // EPI_QKV
  int qdim, kvdim, head_dim, rope_dim, max_seq, kv_type;
  const float* rope_cs;      // [max_seq][rope_dim/2][2]
  const float* bias;         // EPI_QKV: q/k/v bias [qdim + 2*kvdim] added before RoPE, or nullptr
  const int* dpos;           // device position
  void* kcache;              // this layer: [kvh][max_seq][head_dim] fp16 (kv_type 0)
  void* vcache;
  float* kv_f32;             // kv_type 1: fp32 K,V staging [2*kvdim]
  // EPI_LOGITS
  float2* part;              // one (value, index bits) candidate per workgroup
  float out_scale;           // EPI_LOGITS: y = (W x) * out_scale (1: none; Gemma 1/sqrt(d))
  float softcap, softcap_inv;  // EPI_LOGITS: then y = softcap * tanh(y * softcap_inv) when softcap > 0
  int act;                   // EPI_SWIGLU: 0 up * SiLU(gate), 1 up * GELU(gate) (tanh form, GeGLU)
  // x = the attention output merged from its splits while staging (x unused):
  // the attention split merge folded into the Wo matvec; needs att_ns <= kMergeSplits
  const float* att_o;        // [kvh][ns][G][head_dim] partial outputs, or nullptr
  const float* att_ml;       // [kvh][ns][G][2] partial (max, sum)
  int att_ns, att_group;     // splits per KV head, query heads per KV head
  int att_split_fill;        // the attention's split_fill
  // With att_o and xr both set, the split count decides per token: at most
  // kMergeSplits active splits are merged while staging, more were merged
  // by the attention's last split into the records xr.
  // x records (ss_device.h): when xr is set, x is read from these records
  // (written by the producer of x, with the RMSNorm weight nw already
  // applied and the sums of squares in word 14) instead of from x; the
  // buffer holds xrec_words(cols) words, zero past the vector
  const uint32_t* xr;
  // producer side (EPI_STORE, EPI_ADD, EPI_SWIGLU): also write the output as
  // records of y * nw_out (nw_out may be nullptr) for the next matvec
  uint32_t* xr_out;
  const float* nw_out;
};
// 32-bit words of an x record buffer for a vector of n values: 16-value
// records, padded with zero records to a multiple of 1024 values
inline size_t xrec_words(int n) { return (size_t)((n + 1023) / 1024) * 64 * 16; }

// Prompt products: Y[t] = W X[t] (+ epilogue) for T tokens on MFMA.
struct GemmArgs {
  PackedMat w, w2;           // w2: up projection for EPI_SWIGLU
  const float* x;            // [T][ldx] token-major
  const float* nw;           // RMSNorm weight [cols]: x is normalised (tensor.c:114-131), or nullptr
  float* ssq;                // [T] scratch for the sums of squares of x (required with nw)
  float eps;
  float* y;                  // [T][ldy] (EPI_ADD: accumulated into)
  uint16_t* xs;              // scratch of gemm_split_elems(T, cols) 16-bit words: x split into
                             // two fp16 parts and a scale per token (fp16 products), or
                             // nullptr (fp32 products)
  int ldx, ldy, rows, cols, T, type;
  int act;                   // EPI_SWIGLU: 0 SiLU, 1 GELU (Gemma's GeGLU)
};
// 16-bit words of GemmArgs::xs for T tokens of cols columns
inline size_t gemm_split_elems(int T, int cols) {
  return 2 * (size_t)T * (size_t)((cols + 127) / 128 * 128) + 2 * (size_t)T;
}

struct AttnArgs {
  const float* q;            // [n_heads][hd]
  const void* kc;            // this layer: [kvh][max_seq][hd] fp16 or int8
  const void* vc;
  const float* ks;           // int8: this layer's per-position scales [max_seq]
  const float* vs;
  const int* dpos;           // ctx = *dpos + 1 when set, else seq_len
  int seq_len, max_seq, ns, n_kv_heads;
  float scale;
  float softcap, softcap_inv;  // > 0: scores = softcap * tanh(scores * softcap_inv) before the softmax
  float* out;                // [n_heads][hd]
  float* part_o;             // [kvh][ns][G][hd]
  float* part_ml;            // [kvh][ns][G][2]
  uint32_t* cnt;             // [n_kv_heads] split arrivals, zero between launches: the last
                             // split merges into out; nullptr: the splits stay in part_o/part_ml
                             // for a merging consumer (ns <= kMergeSplits)
  uint32_t* xr_out;          // with cnt set: also the output as x records (xrec_words(n_heads * hd))
  int split_fill;            // attn_chunks' fill (0: none)
  int wo_merge;              // with cnt set: when at most kMergeSplits splits are active, leave
                             // them in part_o/part_ml for the Wo matvec (which then merges them)
  int n_tok;                 // prompt rows (launch_attention_rows): token z at position dpos[z]
  int pos0;                  // (or pos0 + z when dpos is null),
  int tok_q, tok_o;          // its query at q + z*tok_q, its output at out + z*tok_o
};

// The attention softcap (layer_scheduler.c:446-448, tensor.c:194-200) of a
// scaled score: cap * tanh(score / cap), or the score when no cap is set.
__device__ __forceinline__ float softcap(float d, const AttnArgs& a) {
  return a.softcap > 0.f ? a.softcap * tanhf(d * a.softcap_inv) : d;
}

// Profiling: when start is set, the next matvec or attention launch on this
// thread passes start/stop to hipExtLaunchKernel, so the dispatch records them
// when the kernel begins and ends (kernel execution time), and sets used.
struct KernelEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};
KernelEvents& kernel_events();   // this thread's

struct GemvPlan {
  int grid, threads, unit;
  size_t lds_bytes;
};
// unit: tiles per wave per round (2, 4 or 8); two unless the launcher chooses
GemvPlan gemv_plan(int rows, int cols, int type, int nmat, int unit = 2);
// bytes and plane views of a packed matrix (16-row x 4-block tiles, see ss_gemv.hip)
size_t packed_bytes(int type, int64_t rows, int cols);
PackedMat packed_view(const void* base, int type, int64_t rows, int cols);
hipError_t launch_gemv(int epi, const GemvArgs& a, hipStream_t s);
hipError_t launch_argmax_merge(const float2* part, int n, const float* y, int* out_idx, int* tokens,
                               int* dpos, hipStream_t s);
hipError_t launch_attention(int head_dim, int group, int kv_type, const AttnArgs& a, hipStream_t s);
// Groups of 4 or 8: merge the splits a launch_attention with a.cnt null left
// in part_o / part_ml into out (and xr_out), after it on the same stream;
// nothing when one split is active (the attention wrote the output).
hipError_t launch_attention_merge(int head_dim, int group, const AttnArgs& a, hipStream_t s);
// Causal attention of a.n_tok prompt rows (token z: query a.q + z*a.tok_q,
// positions 0..a.dpos[z] (or a.pos0 + z), output a.out + z*a.tok_o), fp16
// cache, head_dim 64, 128 or 256, on MFMA (ss_flash.hip).
hipError_t launch_attention_rows(int head_dim, int group, const AttnArgs& a, hipStream_t s);
// ssq[t] = sum of x[t][c]^2 (x [T][cols])
hipError_t launch_sumsq(const float* x, int cols, int T, float* ssq, hipStream_t s);
// Y = W X over T tokens with EPI_STORE, EPI_ADD or EPI_SWIGLU; with nw set,
// first the sums of squares of X into a.ssq. With a.xs: X is split into fp16
// parts first and the products run in fp16 (exact codes, fp32 accumulation
// and scales); otherwise in fp32.
hipError_t launch_gemm(int epi, const GemmArgs& a, hipStream_t s);
// Launches of the fp16-MFMA products since the library was loaded, per
// epilogue (EPI_STORE, EPI_ADD, EPI_SWIGLU) and row groups per wave (1, 2):
// index 2 * epilogue_slot + RG - 1.
constexpr int kGemmVariants = 6;
const int64_t* gemm_h_launch_counts();
bool attention_supported(int head_dim, int group);
// positions one attention workgroup covers in one round of loads
int attn_round_positions(int head_dim, int group);
// attention workgroups of this shape resident on one compute unit (0: unknown)
int attn_resident_groups(int head_dim, int group, int kv_type);

hipError_t launch_pack(int type, const uint8_t* src, PackedMat dst, int64_t nblocks, int nb, int64_t row_off,
                       hipStream_t s);
// The row times scale (1: none; Gemma sqrt(d)). With xr set, also the x
// records of row * nw (xrec_words(cols) words).
hipError_t launch_embed(int type, PackedMat t, int cols, const int* tokens, const int* dpos,
                        int token, float* out, const float* nw, uint32_t* xr, float scale, hipStream_t s);
// Rows tokens[*dpos + z], z < n, of the table (times scale) into out[z][cols].
hipError_t launch_embed_rows(int type, PackedMat t, int cols, const int* tokens, const int* dpos, int n,
                             float* out, float scale, hipStream_t s);
// Post norm (layer_scheduler.c:474-481, 553-560): hidden += y * w / rms(y),
// w the (1 + weight) vector; with xr set, also the x records of the new
// hidden * nw_out (nw_out may be nullptr). One workgroup; n a multiple of 16.
hipError_t launch_post_norm(float* hidden, const float* y, const float* w, int n, float eps, uint32_t* xr,
                            const float* nw_out, hipStream_t s);
// hidden[t] += rmsnorm(y[t]) * w for the T rows of a prompt (row stride n)
hipError_t launch_post_norm_rows(float* hidden, const float* y, const float* w, int n, int T, float eps,
                                 hipStream_t s);
hipError_t launch_rmsnorm(float* out, const float* x, const float* w, int n, float eps,
                          hipStream_t s);
hipError_t launch_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim,
                       int rope_dim, const float* cs_row, int is_neox, hipStream_t s);
hipError_t launch_kv_append(void* kc, void* vc, float* ksc, float* vsc, const float* k,
                            const float* v, int n_kv_heads, int head_dim, int max_seq,
                            const int* dpos, int pos, int kv_type, hipStream_t s);
// RoPE of the q and k parts of n prompt rows [q | k | v] (stride ld; token z
// at position dpos[z]) and the fp16 cache append of k and v.
hipError_t launch_rope_kv_rows(float* qkv, const float* bias, int ld, int qdim, int kvdim, int head_dim, int rope_dim,
                               const float* cs, const int* dpos, uint16_t* kc, uint16_t* vc, int max_seq,
                               int n, hipStream_t s);
// acc[j] += sum over the T rows x[t] (stride d) of x[t][j] * k_t * w[j] (the
// output RMSNorm, k_t from ssq[t]), or of x[t][j] when w is null
hipError_t launch_pool_rows(const float* x, int T, int d, const float* w, const float* ssq, float eps, float* acc,
                            hipStream_t s);
// out = (acc / n) / (|acc / n| + 1e-12)
hipError_t launch_embed_finish(const float* acc, int d, int n, float* out, hipStream_t s);
hipError_t launch_swiglu(float* out, const float* g, const float* u, int n, hipStream_t s);
hipError_t launch_argmax(int* out, const float* x, int n, float2* part, hipStream_t s);
// Non-greedy sampling of ss_sample (tensor.c:363-451) over logits[V] on the
// device (ss_sample.hip); one workgroup.
struct SampleArgs {
  const float* logits;
  int V;
  float temperature, top_p;  // temperature > 0
  int top_k;
  uint64_t rng;              // xorshift64 state before the draw
  float* probs;              // scratch [V]
  int* out;                  // sampled index
  uint64_t* rng_out;         // state after the draw
  int* tokens;               // optional: tokens[*dpos + 1] = index, then *dpos += 1
  int* dpos;
};
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);
hipError_t launch_set_state(int* dpos, int* tokens, int pos, int token, hipStream_t s);
hipError_t launch_advance(int* dpos, hipStream_t s);

constexpr int kArgmaxMaxBlocks = 1024;
constexpr int kRG = 16;                    // rows per packed row group
constexpr int kTB = 4;                     // 32-column blocks per tile (kRG * kTB = 64 lanes)
constexpr int kUT = 8;                     // tiles per scale group (16 B of scales per lane)
constexpr int kGemvUnit = 2;               // default tiles per wave per round (2, 4 or 8)
constexpr int kGemvMaxSplit = 16;          // waves per matvec workgroup
constexpr int kMaxSplits = 256;            // attention splits per KV head
constexpr int kMergeSplits = 8;            // splits the Wo matvec merges itself

}  // namespace ssk
