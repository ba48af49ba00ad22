/*
 * ss_oracle.h - CPU restatement of SlipStream's per-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP product is
 * compared against and the CPU baseline timed beside it. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product (phonemap_amd/, include/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates. Paths are
 * relative to the reference repository's SlipStream/ directory.
 */
#ifndef SS_ORACLE_H
#define SS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types used on the path (src/core/gguf_loader.h:41-55) */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_Q8_0 = 8,
       ORC_Q8_1 = 9, ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

/* KV cache storage modes */
enum { ORC_KV_INT8 = 0,   /* reference: per-(layer,pos) absmax int8, layer_scheduler.c:101-125 */
       ORC_KV_F16  = 1 }; /* binary16 cache (the GPU path's default), laid out as the fp32 KV of layer_scheduler.c.orig:289-342 */

/* ---- element ops ---- */
float    orc_f16_to_f32(uint16_t h);                 /* quantize.c:20-56 */
uint16_t orc_f32_to_f16(float f);                    /* IEEE binary16, round-to-nearest-even */
void     orc_dequantize(const void *src, float *dst, int32_t n, int32_t type); /* quantize.c:389-442 */
float    orc_dot(const float *a, const float *b, int32_t n);   /* vDSP_dotpr stand-in */
void     orc_dequant_matvec(float *out, const void *w, const float *x,
                            int32_t rows, int32_t cols, int32_t type);  /* quantize.c:446-494 */
void     orc_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps); /* cpu_neon.c:109-115 */
void     orc_softmax(float *x, int32_t n);           /* tensor.c:154-173 */
float    orc_silu_mul(float g, float u);             /* layer_scheduler.c:533-549 */
void     orc_gemma_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps); /* cpu_neon.c:153-158 */
float    orc_gelu(float v);                          /* tensor.c:181-190 (one element) */
void     orc_softcap(float *x, int32_t n, float cap);  /* tensor.c:194-200 */
void     orc_rope(float *q, float *k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                  int32_t rope_dim, int32_t pos, float theta, int32_t is_neox); /* tensor.c:220-275 */
void     orc_rope_table(float *cs, int32_t rope_dim, int32_t n_pos, float theta); /* cos/sin of tensor.c:250-254 */
int32_t  orc_argmax(const float *x, int32_t n);      /* tensor.c:318-328 */
int32_t  orc_sample(const float *logits, int32_t n, float temperature, float top_p, int32_t top_k,
                    uint64_t *rng, float *probs_out, float *r_out);      /* tensor.c:363-451 */
void     orc_kv_int8_encode(const float *src, int8_t *q, float *scale, int32_t n); /* layer_scheduler.c:101-118 */
void     orc_attention_head(float *out, const float *q, const float *keys, const float *values,
                            int32_t head_dim, int32_t seq_len, int32_t kv_stride); /* layer_scheduler.c:421-467 */

/* ---- thread pool used by the matvec and the per-head attention ---- */
void     orc_set_threads(int32_t n);  /* 0 = hardware concurrency; 1 = serial */
int32_t  orc_get_threads(void);

/* ---- model (GGUF parse + scheduler) ---- */
typedef struct orc_model orc_model_t;
orc_model_t *orc_model_open(const char *path, int32_t max_seq, int32_t kv_mode); /* gguf_loader.c:210-485 + layer_scheduler.c:129-244 */
void         orc_model_close(orc_model_t *m);
void         orc_model_dims(const orc_model_t *m, int32_t *out8); /* L, d, H, KVH, hd, ffn, vocab, max_seq */
float        orc_model_eps(const orc_model_t *m);
float        orc_model_theta(const orc_model_t *m);
const float *orc_forward(orc_model_t *m, int32_t token, int32_t pos);    /* layer_scheduler.c:571-679 */
const float *orc_prefill(orc_model_t *m, const int32_t *tokens, int32_t n, int32_t start_pos); /* :681-803 */
/* the same, token by token as the reference loops (bit-identical to orc_prefill) */
const float *orc_prefill_serial(orc_model_t *m, const int32_t *tokens, int32_t n, int32_t start_pos);
int32_t      orc_embed(orc_model_t *m, const int32_t *tokens, int32_t n, float *out); /* :805-915 */
void         orc_reset(orc_model_t *m);                                  /* :917-936 */
int32_t      orc_kv_write(orc_model_t *m, int32_t layer, int32_t pos,
                          const uint16_t *k_f16, const uint16_t *v_f16); /* KV injection */
const float *orc_hidden(const orc_model_t *m);                           /* hidden state after forward */

#ifdef __cplusplus
}
#endif
#endif
