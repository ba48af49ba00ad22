/*
 * ss_hip.h - C-ABI of the MI355X (gfx950) backend.
 *
 * The C host code (engine, GGUF loader) reaches the GPU only through these
 * functions: plain pointers and sizes, no HIP or C++ types. They replace the
 * reference's Metal backend plug (SlipStream/src/backends/metal_backend.h:21-75)
 * and the CPU kernels it falls back to (src/core/quantize.h:106-117,
 * src/core/tensor.h:38-123), and take over the whole per-token sweep that
 * src/core/layer_scheduler.c:291-679 runs on the CPU.
 *
 * Conventions: functions return 0 or a negative ss_error_t value
 * (SS_ERROR_INVALID_PARAMS -5, SS_ERROR_OUT_OF_MEMORY -3, SS_ERROR_BACKEND -7)
 * and never throw; ss_hip_last_error() holds a message for the calling
 * thread. "dev" pointers are device memory; a NULL stream means the
 * context's own stream. One context is used by one thread at a time.
 *
 * Device weight layout: a GGUF Q4_0/Q8_0 matrix of R rows and C columns
 * (R*C/32 blocks of fp16 d + 16/32 code bytes) is stored on the device in
 * tiles of 16 rows x 4 blocks. Tile (g, t) holds rows 16g..16g+15, blocks
 * 4t..4t+3; the block chunk of (row r, block b) is entry
 * (g*T + t)*64 + (b%4)*16 + r%16, T = ceil(C/128). Two planes, codes first
 * (16 or 32 bytes per entry), then at the next 256-byte boundary the
 * binary16 scales with the same index. R is padded to a multiple of 16 and
 * C/32 to a multiple of 4 with zero entries. ss_hip_pack_matrix makes it;
 * ss_hip_packed_bytes gives its size. A Q4_K matrix (quantize.c:265-310)
 * uses the same tiles for its 32-weight sub-blocks (nibbles without offset,
 * scale-plane entry = 6-bit scale | 6-bit min << 8), then at the next
 * 256-byte boundary a third plane with each row's super-block (d, dmin)
 * binary16 pairs, [row group][super-block][16 rows]. The other 32-weight
 * block types use the same tiles: Q4_1 nibbles and Q5_1 / Q8_1 int8 codes
 * with a 32-bit scale entry per block (d | m << 16 as binary16, or Q8_1's
 * fp32 d), Q5_0 as Q8_0 (codes q - 16); F16 and F32 matrices store each
 * block's 32 weights (64 or 128 bytes) and have no scale plane.
 */
#ifndef SS_HIP_H
#define SS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ss_hip_ctx ss_hip_ctx_t;
typedef struct ss_hip_model ss_hip_model_t;

/* ggml tensor types accepted (src/core/gguf_loader.h:41-55) */
#define SS_HIP_F32 0     /* float matrices: 32-weight chunks, no scales */
#define SS_HIP_F16 1
#define SS_HIP_Q4_0 2
#define SS_HIP_Q4_1 3    /* 32-bit (d, m) scale entries */
#define SS_HIP_Q5_0 6    /* stored as Q8_0: code q - 16, the same d */
#define SS_HIP_Q5_1 7    /* int8 codes, 32-bit (d, m) scale entries */
#define SS_HIP_Q8_0 8
#define SS_HIP_Q8_1 9    /* int8 codes, 32-bit (fp32 d) scale entries */
#define SS_HIP_Q4_K 12   /* 256-weight super-blocks (cols a multiple of 256) */
#define SS_HIP_Q2_K 10   /* the other K-quants, also 256-weight super-blocks */
#define SS_HIP_Q3_K 11
#define SS_HIP_Q5_K 13
#define SS_HIP_Q6_K 14

/* token launch modes (match SS_LAUNCH_* in slipstream.h): per-kernel eager,
 * per-kernel replayed from a HIP graph, or one persistent launch per token
 * (fp16 KV cache; falls back to GRAPH for shapes it does not cover) */
#define SS_HIP_LAUNCH_EAGER 0
#define SS_HIP_LAUNCH_GRAPH 1
#define SS_HIP_LAUNCH_SWEEP 2

/* KV cache types (match ss_kv_type_t in slipstream.h) */
#define SS_HIP_KV_F16 0
#define SS_HIP_KV_INT8 1

/* ---- context (metal_backend.h:21 ss_metal_init, :75 ss_metal_free) ---- */
ss_hip_ctx_t *ss_hip_init(int32_t device);
void ss_hip_free(ss_hip_ctx_t *ctx);
const char *ss_hip_last_error(void);
int32_t ss_hip_device_count(void);
int32_t ss_hip_device_name(int32_t device, char *buf, int32_t len);
/* compute units and HBM bytes of a device (for ss_get_device_info) */
int32_t ss_hip_device_info(int32_t device, int32_t *n_cu, uint64_t *hbm_bytes);
void *ss_hip_stream(ss_hip_ctx_t *ctx);          /* the context's hipStream_t */
int32_t ss_hip_sync(ss_hip_ctx_t *ctx);

/* ---- device memory, so C callers need no HIP headers ---- */
void *ss_hip_malloc(ss_hip_ctx_t *ctx, size_t bytes);
int32_t ss_hip_mfree(ss_hip_ctx_t *ctx, void *dev);
int32_t ss_hip_memcpy_h2d(ss_hip_ctx_t *ctx, void *dev, const void *host, size_t bytes);
int32_t ss_hip_memcpy_d2h(ss_hip_ctx_t *ctx, void *host, const void *dev, size_t bytes);

/* ---- weight packing: GGUF block layout (host) -> device planes ---- */
size_t ss_hip_packed_bytes(int32_t ggml_type, int32_t rows, int32_t cols);
int32_t ss_hip_pack_matrix(ss_hip_ctx_t *ctx, void *dst_dev, const void *src_host,
                           int32_t ggml_type, int32_t rows, int32_t cols);

/* ---- single ops on device buffers ---- */

/* y = W x, W packed Q4_0/Q8_0 [rows x cols], fp32 x/y, fp32 accumulation.
 * Replaces ss_dequant_matvec (quantize.h:111-112, quantize.c:446-494) and
 * ss_metal_matvec_q4_0 (metal_backend.h:37-42). */
int32_t ss_hip_matvec(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev, const float *x_dev,
                      int32_t rows, int32_t cols, int32_t ggml_type, void *stream);
/* The same for one block type: ss_metal_matvec_q4_0 (metal_backend.h:37-42)
 * on device buffers, and its Q8_0 counterpart (the reference has Q8_0 on the
 * CPU only, quantize.c:139-149, 446-494). */
/* Prompt products on MFMA: y[t] = W x[t] for n_tokens tokens (x [n][cols],
 * y [n][rows], token-major), the matrix read once per 64 tokens. With nw,
 * each token's x is RMSNorm'ed first (tensor.c:114-131, weight nw, eps);
 * accumulate != 0 adds to y (the residual of layer_scheduler.c:484,566).
 * Serves the layer-major prompt of ss_scheduler_prefill
 * (layer_scheduler.c:681-803), which multiplies every token of a layer by
 * the same matrices. */
int32_t ss_hip_gemm(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev, const float *x_dev,
                    const float *nw_dev, float eps, int32_t accumulate, int32_t rows, int32_t cols,
                    int32_t n_tokens, int32_t ggml_type, void *stream);
int32_t ss_hip_matvec_q4_0(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev, const float *x_dev,
                           int32_t rows, int32_t cols, void *stream);
int32_t ss_hip_matvec_q8_0(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev, const float *x_dev,
                           int32_t rows, int32_t cols, void *stream);
/* The Q4_K matvec: ss_metal_matvec_q4_K (metal_backend.h:44-52) on device
 * buffers (the reference runs it on Metal, or dequant_q4_K + the CPU GEMV,
 * quantize.c:265-310, 446-494). */
int32_t ss_hip_matvec_q4_k(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev, const float *x_dev,
                           int32_t rows, int32_t cols, void *stream);

/* y = W rmsnorm(x, nw, eps) (+ y when accumulate != 0): the matvec with the
 * RMSNorm of tensor.c:114-131 folded in front and the residual add of
 * layer_scheduler.c:484 folded behind. nw may be NULL (no norm). */
int32_t ss_hip_matvec_fused(ss_hip_ctx_t *ctx, float *y_dev, const void *w_dev,
                            const float *x_dev, const float *nw_dev, float eps, int32_t accumulate,
                            int32_t rows, int32_t cols, int32_t ggml_type, void *stream);

/* out = u * silu(g) with g = Wg rmsnorm(x), u = Wu rmsnorm(x):
 * layer_scheduler.c:489-549 in one kernel. */
int32_t ss_hip_ffn_gate_up(ss_hip_ctx_t *ctx, float *out_dev, const void *wg_dev,
                           const void *wu_dev, const float *x_dev, const float *nw_dev, float eps,
                           int32_t rows, int32_t cols, int32_t ggml_type, void *stream);

/* tensor.c:114-131 */
int32_t ss_hip_rmsnorm(ss_hip_ctx_t *ctx, float *out_dev, const float *x_dev, const float *w_dev,
                       int32_t n, float eps, void *stream);

/* tensor.c:220-275 (GPT-J pairs when is_neox == 0, halves otherwise) */
int32_t ss_hip_rope(ss_hip_ctx_t *ctx, float *q_dev, float *k_dev, int32_t n_heads,
                    int32_t n_kv_heads, int32_t head_dim, int32_t rope_dim, int32_t pos,
                    float theta, int32_t is_neox, void *stream);

/* KV append at pos (layer_scheduler.c:409-413). Cache layout
 * [n_kv_heads][max_seq][head_dim] of binary16 (SS_HIP_KV_F16) or int8
 * codes (SS_HIP_KV_INT8, with k_scale/v_scale [max_seq] fp32, one absmax
 * scale per position over all heads, layer_scheduler.c:101-118). */
int32_t ss_hip_kv_append(ss_hip_ctx_t *ctx, void *k_cache, void *v_cache, float *k_scale,
                         float *v_scale, const float *k_dev, const float *v_dev,
                         int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, int32_t pos,
                         int32_t kv_type, void *stream);

/* Single-query GQA attention over positions 0..seq_len-1 of one layer's
 * cache (layer_scheduler.c:415-468): out[n_heads*head_dim]. */
int32_t ss_hip_attention(ss_hip_ctx_t *ctx, float *out_dev, const float *q_dev,
                         const void *k_cache, const void *v_cache, const float *k_scale,
                         const float *v_scale, int32_t n_heads, int32_t n_kv_heads,
                         int32_t head_dim, int32_t max_seq, int32_t seq_len, int32_t kv_type,
                         void *stream);

/* Causal attention of n_tokens prompt rows on MFMA: token t (query
 * q[t][n_heads*head_dim], output out[t][n_heads*head_dim]) attends to
 * positions 0..pos0+t of one layer's fp16 cache, whose rows pos0 ..
 * pos0+n_tokens-1 already hold the tokens' own K and V. The per-token
 * attention of layer_scheduler.c:415-468 for every token of a layer-major
 * prompt (ss_scheduler_prefill, layer_scheduler.c:681-803) in one launch;
 * head_dim 64, 128 or 256. */
int32_t ss_hip_attention_rows(ss_hip_ctx_t *ctx, float *out_dev, const float *q_dev,
                              const void *k_cache, const void *v_cache, int32_t n_heads,
                              int32_t n_kv_heads, int32_t head_dim, int32_t max_seq, int32_t pos0,
                              int32_t n_tokens, void *stream);

/* ss_hip_attention with no device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split partials and arrival counters live in one fixed
 * 12 MiB device array per GPU (held until the process ends); a shape that
 * needs more fails with SS_ERROR_INVALID_PARAMS. Every call on a GPU shares
 * that array, so calls that overlap on one GPU (other streams or threads)
 * race; calls in one stream are safe. Same arguments and results as
 * ss_hip_attention. */
int32_t ss_hip_attention_noalloc(ss_hip_ctx_t *ctx, float *out_dev, const float *q_dev,
                                 const void *k_cache, const void *v_cache, const float *k_scale,
                                 const float *v_scale, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t max_seq, int32_t seq_len, int32_t kv_type,
                                 void *stream);

/* out[i] = up[i] * (g / (1 + exp(-g))), g = gate[i] (layer_scheduler.c:533-549) */
int32_t ss_hip_swiglu(ss_hip_ctx_t *ctx, float *out_dev, const float *gate_dev,
                      const float *up_dev, int32_t n, void *stream);

/* index of the first maximum (tensor.c:318-328) into *out_dev (int32) */
int32_t ss_hip_argmax(ss_hip_ctx_t *ctx, int32_t *out_dev, const float *x_dev, int32_t n,
                      void *stream);

/* ss_sample (tensor.c:363-451) over n device logits: with temperature > 0,
 * softmax of logits / temperature, top-k and top-p filtering, renormalising
 * and one xorshift64 draw from *rng_state (advanced in place); the sampled
 * index goes to *out_host. temperature <= 0 is the first-max argmax and
 * leaves the state alone. Sums are exact fixed point rather than the
 * reference's sequential fp32, so the index can differ from the reference's
 * only where the draw lies within fp32 rounding of a cumulative boundary. */
int32_t ss_hip_sample_logits(ss_hip_ctx_t *ctx, const float *logits_dev, int32_t n, float temperature,
                             float top_p, int32_t top_k, uint64_t *rng_state, int32_t *out_host);

/* dequantise row `token` of a packed [rows x cols] table (layer_scheduler.c:584-595) */
int32_t ss_hip_embed_row(ss_hip_ctx_t *ctx, float *out_dev, const void *table_dev,
                         int32_t ggml_type, int32_t rows, int32_t cols, int32_t token,
                         void *stream);

/* ---- Metal-shaped plug on host pointers (metal_backend.h:27-70) ----
 * W is a host pointer in GGUF block layout (e.g. into the GGUF mmap); it is
 * packed and uploaded the first time it is seen and kept, keyed by pointer
 * (the zero-copy registry of metal_backend.m:190-235).
 * ss_hip_matvec_host returns the Metal calls' bool, NOT the 0-on-success
 * convention of the rest of this header: nonzero (true) when out holds
 * W vec, 0 (false) on any failure, after which the caller computes on the
 * CPU (gpu_success in layer_scheduler.c:251-263). ss_hip_should_use_gpu is
 * metal_backend.m:336-340's size test (true when rows * cols > 1024). */
int32_t ss_hip_matvec_host(ss_hip_ctx_t *ctx, float *out, const void *mat, const float *vec,
                           int32_t rows, int32_t cols, int32_t ggml_type);
int32_t ss_hip_should_use_gpu(int32_t rows, int32_t cols);

/* Metal's command-buffer batch (ss_metal_begin_batch / ss_metal_end_batch,
 * metal_backend.h:59-70, metal_backend.m:307-330), which the scheduler opens
 * around Q/K/V and around gate/up (layer_scheduler.c:353-361,509-516).
 * Between the two calls ss_hip_matvec_host only enqueues: its true means
 * that out will hold the product after ss_hip_end_batch, which waits for
 * the batch once and copies every output to its host array (0, or a
 * negative ss_error_t if a copy failed). Each call of a batch stages its
 * own vector, so the calls may read different vectors (Metal's share one
 * buffer). At most 16 calls of a batch are deferred, as Metal's; a further
 * call returns false and the caller computes it on the CPU (Metal's returns
 * true and never fills out). Beginning an open batch or ending none does
 * nothing. */
void ss_hip_begin_batch(ss_hip_ctx_t *ctx);
int32_t ss_hip_end_batch(ss_hip_ctx_t *ctx);

/* ---- whole-model decode ---- */

typedef struct {
    const void *data;   /* host pointer, GGUF layout (borrowed during create) */
    int32_t type;       /* SS_HIP_* */
    int32_t rows;       /* GGUF dims[1]; 1 for vectors */
    int32_t cols;       /* GGUF dims[0] */
} ss_hip_tensor_t;

/* per-layer tensor order in ss_hip_model_desc_t.layers */
enum {
    SS_HIP_ATTN_NORM = 0, SS_HIP_WQ, SS_HIP_WK, SS_HIP_WV, SS_HIP_WO,
    SS_HIP_FFN_NORM, SS_HIP_W_GATE, SS_HIP_W_UP, SS_HIP_W_DOWN, SS_HIP_LAYER_TENSORS
};

typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, rope_dim, ffn, vocab, max_seq;
    float rms_eps, rope_theta;
    int32_t kv_type;     /* SS_HIP_KV_* */
    int32_t launch;      /* SS_HIP_LAUNCH_* */
    int32_t streaming;   /* nonzero: the layer matrices stay in pinned host
                          * memory and each layer is uploaded (hipMemcpyAsync,
                          * side stream) into a ring of device slots while the
                          * previous layers compute; prompts run layer-major.
                          * Launches are then per kernel (EAGER). */
    ss_hip_tensor_t token_embd, output_norm, output;
    const ss_hip_tensor_t *layers;   /* n_layers * SS_HIP_LAYER_TENSORS */
    /* NULL, or n_layers * 3 bias vectors (q, k, v; F32 or F16; data NULL where
     * a layer has none), added to the projections before RoPE
     * (layer_scheduler.c:367-402). */
    const ss_hip_tensor_t *qkv_bias;
    /* Gemma ("gemma" in the architecture name, layer_scheduler.c:152-155):
     * nonzero applies attn_norm, ffn_norm and output_norm in the (1 + w) form
     * (tensor.c:133-152), scales the embedding by sqrt(hidden) (:597-602)
     * and the logits by 1/sqrt(hidden) (:667-672), and uses GeGLU (the
     * tanh-form GELU of the gate, :529-531, tensor.c:181-190) for SwiGLU. */
    int32_t gemma;
    /* > 0: cap * tanh(x / cap) on the attention scores before the softmax
     * (:446-448) and on the logits (:674-676), for any architecture */
    float attn_softcap, final_softcap;
    /* NULL, or n_layers * 2 norm vectors (post_attention_norm, post_ffw_norm;
     * F32 or F16; data NULL where a layer has none), applied in the (1 + w)
     * form to the Wo and down outputs before the residual (:474-481,
     * 553-560) */
    const ss_hip_tensor_t *post_norms;
} ss_hip_model_desc_t;

/* ss_scheduler_init (layer_scheduler.h:95-96): upload + pack all weights,
 * allocate the KV cache and working buffers. */
ss_hip_model_t *ss_hip_model_create(ss_hip_ctx_t *ctx, const ss_hip_model_desc_t *desc);
void ss_hip_model_free(ss_hip_model_t *m);

/* ss_scheduler_forward (layer_scheduler.h:107) */
int32_t ss_hip_eval_token(ss_hip_model_t *m, int32_t token, int32_t pos, float *logits_host,
                          int32_t *argmax_out);
/* ss_scheduler_prefill (layer_scheduler.h:119). With an fp16 cache a prompt
 * of at least the batch threshold (default 8 tokens) runs as matrix products
 * over chunks of up to 512 tokens; shorter prompts and int8 caches run token
 * by token. */
int32_t ss_hip_eval_prompt(ss_hip_model_t *m, const int32_t *tokens, int32_t n,
                           int32_t start_pos, float *logits_host, int32_t *argmax_out);
/* Batch threshold of ss_hip_eval_prompt: 0 restores the default, a negative
 * value makes every prompt run token by token (no counterpart in the
 * reference; for measurement and comparison). */
int32_t ss_hip_set_prompt_batch(ss_hip_model_t *m, int32_t min_tokens);
/* ss_scheduler_embed (layer_scheduler.c:805-911): tokens at positions
 * 0..n-1 (the cache is overwritten there), every token's final hidden state
 * through the output norm, mean-pooled and L2-normalised into out_host[hidden].
 * With the fp16 cache the prompt runs as matrix products. */
int32_t ss_hip_embed(ss_hip_model_t *m, const int32_t *tokens, int32_t n, float *out_host);
/* ss_hip_sample_logits over the logits of the model's last evaluated token
 * (left in HBM by ss_hip_eval_token / ss_hip_eval_prompt, which need not
 * copy them to the host) */
int32_t ss_hip_sample(ss_hip_model_t *m, float temperature, float top_p, int32_t top_k,
                      uint64_t *rng_state, int32_t *token_out);
/* device-side greedy continuation (see ss_decode_greedy) */
int32_t ss_hip_decode_greedy(ss_hip_model_t *m, int32_t n_steps, int32_t *tokens_out);
/* ss_scheduler_reset (layer_scheduler.h:132) */
int32_t ss_hip_kv_reset(ss_hip_model_t *m);
int32_t ss_hip_kv_write(ss_hip_model_t *m, int32_t layer, int32_t pos0, int32_t n_pos,
                        const uint16_t *k_f16, const uint16_t *v_f16);
/* final hidden state (after the output norm) of the last evaluated token */
int32_t ss_hip_hidden(ss_hip_model_t *m, float *host_out);
/* cancellation flag polled between layers when the sweep is not a graph */
void ss_hip_set_cancel_flag(ss_hip_model_t *m, const volatile int32_t *flag);
/* bytes of device memory held by the model (weights, KV, buffers) */
uint64_t ss_hip_model_bytes(const ss_hip_model_t *m);
/* bytes of pinned host memory held by the model (streaming mode weights) */
uint64_t ss_hip_model_host_bytes(const ss_hip_model_t *m);
/* the launch mode in effect (SS_HIP_LAUNCH_*; SWEEP may have been
 * replaced by GRAPH for a shape the persistent launch does not cover) */
int32_t ss_hip_model_launch(const ss_hip_model_t *m);
/* Test support: launches of the fp16-MFMA prompt products since the library
 * was loaded, per epilogue (store, add, SwiGLU) and row groups per wave (1,
 * 2); out[2 * epilogue + rg - 1], at most n (6) entries. */
int32_t ss_hip_gemm_launch_counts(int64_t *out, int32_t n);

/* Phase timing of the persistent launch: with tracing on, every launch
 * records per workgroup its start and, for each phase p = 0 .. 5L (layer l:
 * 5l + 0 QKV, +1 attention, +2 Wo, +3 gate/up, +4 down; 5L the LM head),
 * four 100 MHz wall-clock stamps: compute done, own results published, wait
 * for the other workgroups done, next input staged. Layout per workgroup:
 * 4 header words (word 0 = start), then 4 per phase. trace_read copies the
 * last launch's stamps and returns the word count (workgroups = count /
 * (4 + 4 * (5L + 1))). */
int32_t ss_hip_trace_enable(ss_hip_model_t *m, int32_t on);
int64_t ss_hip_trace_read(ss_hip_model_t *m, uint64_t *host, size_t n_words);

/* ---- timing support for the benchmark ----
 * Records device time per launch class (HIP events on the launching stream)
 * for the next eval calls: 0 = Q4_0 matvecs, 1 = Q8_0 matvecs, 2 =
 * attention, 3 = other kernels, 4 = persistent token launches; per class
 * three doubles (total ms, launches, algorithmic bytes), 15 in all. */
int32_t ss_hip_profile_begin(ss_hip_model_t *m);
int32_t ss_hip_profile_end(ss_hip_model_t *m, double *ms_out, int32_t n);

#ifdef __cplusplus
}
#endif
#endif /* SS_HIP_H */
