// ss_sweep.h - the persistent whole-token decode kernel (internal, C++).
//
// One cooperative launch evaluates one token: embedding, every layer
// (RMSNorm + [Wq;Wk;Wv] + RoPE + fp16 KV append, attention, Wo + residual,
// RMSNorm + gate/up + SwiGLU, down + residual), output norm, LM head and the
// first-max argmax, i.e. layer_scheduler.c:571-679 with process_layer
// (:291-567). One workgroup runs on each compute unit for the whole token;
// phases hand their outputs to the next through device memory and per
// workgroup progress flags instead of kernel boundaries. The C-ABI in
// ss_hip.hip is the only user.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ss_kernels.h"

namespace ssk {

// Weights and cache of one decoder layer on the device. 16-byte aligned:
// the kernel copies the descriptors into shared memory in 16-byte units and
// reads them back as an array, so the array stride must be such a multiple.
struct alignas(16) SweepLayer {
  PackedMat qkv, o, gate, up, down;   // [Wq;Wk;Wv] packed as one matrix
  const float* attn_norm;
  const float* ffn_norm;
  uint16_t* kc;                       // fp16 [n_kv_heads][max_seq][head_dim]
  uint16_t* vc;
};

struct SweepArgs {
  const SweepLayer* layers;           // device array [n_layers]
  PackedMat embd, out;                // token embedding table, LM head (may alias embd)
  int embd_type;                      // 2 (Q4_0) or 8 (Q8_0)
  const float* out_norm;              // may be null: no output norm
  const float* rope_cs;               // [max_seq][rope_dim] (cos, sin) pairs
  int n_layers, d, qdim, kvdim, ffn, vocab, max_seq, rope_dim, n_kv_heads;
  int ns;                             // attention splits per KV head
  int nwg;                            // workgroups (one per compute unit)
  float eps, attn_scale;
  int* tokens;                        // [max_seq + 1]; the token is tokens[*dpos]
  int* dpos;                          // device position
  int* argmax;                        // [1] last argmax
  // exchange buffers, one slot per layer (and phase) so that each address is
  // written at most once per launch
  float* q;                           // [n_layers][qdim] roped queries
  float* hidden;                      // [d] residual stream after the last layer (for ss_embed)
  uint32_t* hrec;                     // [n_layers][2][d / 16] x records of the residual stream
                                      // (after Wo, after down)
  uint32_t* frec;                     // [n_layers][ffn / 16] x records of the SwiGLU output
  uint32_t* arec;                     // [n_layers][qdim / 16] x records of the attention output
  float* part;                        // [n_layers][kvh][ns][G][hd + 2] attention split partials
  uint32_t* att_cnt;                  // split arrivals [n_layers][n_kv_heads], zero between launches
  float* logits;                      // [vocab]
  float2* cand;                       // per-workgroup first-max candidates [nwg]
  uint32_t* flags;                    // per workgroup its last epoch (see flag_of); words
                                      // kSweepAbort, kSweepErr
  uint64_t timeout_ticks;             // bound on any wait, in s_memrealtime ticks (100 MHz)
  uint64_t* trace;                    // null, or per workgroup kSweepTraceHead + 4 per phase
                                      // s_memrealtime stamps (see sweep_trace_words)
};

// Per launch: the argument block lives in device memory (written once per
// model), so the kernel reads its fields where it uses them instead of
// holding all of them in registers for the whole token.
struct SweepLaunch {
  const SweepArgs* args;              // device copy of the model's SweepArgs
  uint32_t epoch0;                    // flag value every workgroup holds at launch
  int with_head;                      // 0: prompt token without LM head (position advance only)
};

constexpr int kSweepComputeWaves = 7;
constexpr int kSweepThreads = (kSweepComputeWaves + 1) * 64;
constexpr int kSweepTiles = 4;        // tiles per work item
constexpr int kSweepFlagStride = 1024;                  // words between 16-workgroup flag lines
constexpr int kSweepAbort = 64 * kSweepFlagStride;       // nonzero: some workgroup gave up waiting
constexpr int kSweepErr = kSweepAbort + 1;               // (phase << 16 | workgroup) of a timeout
constexpr int kSweepFlagWords = kSweepAbort + 64;        // flags array (words)
constexpr int kSweepMaxWg = 1024;

// Flag increments of one launch (phases signalled per token).
int sweep_phases(int n_layers, int with_head);
// Trace of one launch: per workgroup, word 0 = launch start, then per phase
// p = 0 .. 5L (layer l phase k = 5l + k, k = 0 QKV, 1 attention, 2 Wo,
// 3 gate/up, 4 down; 5L the LM head) eight stamps: [0, 4) by the control
// wave - compute waves done, own results published, wait for the others
// done, next input staged - and [4, 8) by compute wave 0 - phase start,
// first work item done, all items done, next phase's loads issued.
constexpr int kSweepTraceHead = 4;
constexpr int kSweepTracePerPhase = 8;
inline size_t sweep_trace_words(int n_layers, int nwg) {
  return (size_t)nwg * (kSweepTraceHead + kSweepTracePerPhase * (5 * n_layers + 1));
}
// Shared memory a launch needs, or 0 when the shape is not supported.
size_t sweep_lds_bytes(const SweepArgs& a, int head_dim, int group);
bool sweep_supported(int head_dim, int group, int layer_type, int out_type);
// Largest workgroup count that is co-resident on the device for this shape.
hipError_t sweep_max_workgroups(int head_dim, int group, int layer_type, int out_type, size_t lds,
                                int* max_wg);
// a: the host copy of the block that l.args points to (sizes the launch)
hipError_t launch_sweep(const SweepArgs& a, const SweepLaunch& l, int head_dim, int group, int layer_type,
                        int out_type, hipStream_t s);

}  // namespace ssk
