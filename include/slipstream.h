/*
 * slipstream.h - public C API of the MI355X-native SlipStream token loop.
 *
 * Drop-in for the reference's include/slipstream.h: every type, enum value
 * and function declared there is declared here with the same name, layout and
 * meaning (SlipStream/include/slipstream.h:1-300), so existing callers
 * (examples/cli/main.c, the Swift binding) compile and link unchanged.
 *
 * Additions, all below the reference set:
 *   - SS_BACKEND_HIP in ss_backend_t;
 *   - ss_model_load_ex with an extension struct (KV cache type, device,
 *     context override) so ss_model_config_t keeps its reference layout;
 *   - the engine-internal "eval-token" API the reference keeps private
 *     (layer_scheduler.h:95-137, tensor.h:115-123, tokenizer.h:28-53):
 *     tokenize, eval one token, eval a prompt, greedy argmax, KV injection.
 */
#ifndef SLIPSTREAM_H
#define SLIPSTREAM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_VERSION_MAJOR 0
#define SS_VERSION_MINOR 1
#define SS_VERSION_PATCH 0
#define SS_VERSION_STRING "0.1.0"

/* slipstream.h:32-43 */
typedef enum {
    SS_OK = 0,
    SS_ERROR_FILE_NOT_FOUND = -1,
    SS_ERROR_INVALID_MODEL = -2,
    SS_ERROR_OUT_OF_MEMORY = -3,
    SS_ERROR_MMAP_FAILED = -4,
    SS_ERROR_INVALID_PARAMS = -5,
    SS_ERROR_CANCELLED = -6,
    SS_ERROR_BACKEND = -7,
    SS_ERROR_TOKENIZER = -8,
    SS_ERROR_UNKNOWN = -99,
} ss_error_t;

/* slipstream.h:47-51, plus the HIP backend */
typedef enum {
    SS_BACKEND_AUTO = 0,
    SS_BACKEND_CPU = 1,
    SS_BACKEND_METAL = 2,
    SS_BACKEND_HIP = 3,
} ss_backend_t;

/* slipstream.h:55-61 */
typedef enum {
    SS_QUANT_F32 = 0,
    SS_QUANT_F16 = 1,
    SS_QUANT_Q8_0 = 2,
    SS_QUANT_Q4_0 = 3,
    SS_QUANT_Q4_1 = 4,
} ss_quant_type_t;

/* slipstream.h:65-79 */
typedef struct {
    char model_name[256];
    char architecture[64];
    char chat_format[64];
    uint32_t num_layers;
    uint32_t hidden_size;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t vocab_size;
    uint32_t context_length;
    uint32_t intermediate_size;
    ss_quant_type_t quant_type;
    uint64_t file_size;
    uint64_t per_layer_size;
} ss_model_info_t;

typedef struct ss_model ss_model_t;

/* slipstream.h:87-94 */
typedef struct {
    ss_backend_t backend;
    uint32_t n_threads;
    uint64_t max_memory;
    bool use_mmap;
    bool prefetch;
    uint32_t context_size;
} ss_model_config_t;

/* slipstream.h:98-106 */
typedef struct {
    uint32_t max_tokens;
    float temperature;
    float top_p;
    uint32_t top_k;
    float repeat_penalty;
    uint32_t seed;
    const char *stop_sequence;
} ss_generate_params_t;

/* slipstream.h:118-122 */
typedef bool (*ss_token_callback_t)(const char *token_text, uint32_t token_id, void *user_data);

/* slipstream.h:132-137 */
typedef void (*ss_progress_callback_t)(uint32_t current, uint32_t total, const char *phase,
                                       void *user_data);

ss_model_config_t ss_default_config(void);                                          /* :144 */
ss_generate_params_t ss_default_params(void);                                       /* :150 */
ss_model_t *ss_model_load(const char *path, const ss_model_config_t *config);       /* :163 */
ss_error_t ss_model_get_info(const ss_model_t *model, ss_model_info_t *info);       /* :168 */
void ss_model_free(ss_model_t *model);                                              /* :173 */
void ss_set_throttle(ss_model_t *model, uint32_t delay_us);                         /* :176 */
uint64_t ss_get_memory_usage(void);                                                 /* :179 */
const char *ss_get_last_profile_path(void);                                         /* :182 */
void ss_set_profile_output_dir(const char *dir);                                    /* :183 */
ss_error_t ss_generate(ss_model_t *model, const char *prompt,
                       const ss_generate_params_t *params, ss_token_callback_t token_cb,
                       void *user_data);                                            /* :206-212 */
ss_error_t ss_embed(ss_model_t *model, const char *prompt, float **out_embedding,
                    uint32_t *out_dim);                                             /* :215-220 */
void ss_cancel(ss_model_t *model);                                                  /* :225 */
void ss_set_progress_callback(ss_model_t *model, ss_progress_callback_t callback,
                              void *user_data);                                     /* :232-236 */
ss_error_t ss_last_error(void);                                                     /* :243 */
const char *ss_error_string(ss_error_t error);                                      /* :248 */
const char *ss_version(void);                                                       /* :255 */
ss_error_t ss_estimate_memory(const char *path, uint32_t context_size,
                              uint64_t *peak_memory);                               /* :266-270 */

/* slipstream.h:274-284 */
typedef struct {
    char device_model[64];
    char chip_name[64];
    uint32_t cpu_core_count;
    uint32_t perf_core_count;
    uint32_t efficiency_core_count;
    uint32_t gpu_core_count;
    uint64_t total_memory;
    uint64_t available_memory;
    int32_t thermal_state;
} ss_device_info_t;

ss_error_t ss_get_device_info(ss_device_info_t *info);                              /* :289 */
double ss_get_cpu_usage(void);                                                      /* :294 */

/* ---------------------------------------------------------------------------
 * Additions
 * ------------------------------------------------------------------------- */

/* KV cache storage. SS_KV_INT8 is the reference's absmax int8 cache
 * (layer_scheduler.c:101-125); SS_KV_F16 stores binary16 K/V. */
typedef enum { SS_KV_F16 = 0, SS_KV_INT8 = 1 } ss_kv_type_t;

typedef struct {
    ss_kv_type_t kv_type;   /* default SS_KV_F16 */
    int32_t device;         /* HIP device ordinal, default 0 */
    uint32_t max_context;   /* 0 = config->context_size, else model default; no 512 cap */
    uint32_t streaming;     /* 0 = weights resident in HBM */
    uint32_t launch;        /* SS_LAUNCH_* below, default SS_LAUNCH_GRAPH */
} ss_model_ext_t;

/* How a token is launched on the GPU. SWEEP: one persistent launch per
 * token (fp16 KV; other cases use GRAPH). GRAPH: one kernel per step, the
 * token's kernels replayed from a HIP graph. EAGER: one kernel per step,
 * launched one by one. */
enum { SS_LAUNCH_EAGER = 0, SS_LAUNCH_GRAPH = 1, SS_LAUNCH_SWEEP = 2 };

ss_model_ext_t ss_default_ext(void);
ss_model_t *ss_model_load_ex(const char *path, const ss_model_config_t *config,
                             const ss_model_ext_t *ext);

/* tokenizer.h:28-31,37,43-49 */
int32_t ss_tokenize(const ss_model_t *model, const char *text, int32_t *out, int32_t max_tokens);
const char *ss_token_text(const ss_model_t *model, int32_t token_id);
int32_t ss_bos_id(const ss_model_t *model);
int32_t ss_eos_id(const ss_model_t *model);

/* Logits length (the vocab clamp of layer_scheduler.c:185-197) and the
 * context capacity of the loaded model. */
int32_t ss_n_vocab(const ss_model_t *model);
int32_t ss_n_ctx(const ss_model_t *model);
int32_t ss_n_embd(const ss_model_t *model);

/* ss_scheduler_reset (layer_scheduler.h:132): zero the KV cache. */
ss_error_t ss_reset(ss_model_t *model);

/* ss_scheduler_forward (layer_scheduler.h:107): evaluate token_id at pos.
 * logits (nullable) receives ss_n_vocab floats; argmax (nullable) the index
 * of the first maximum of those logits. */
ss_error_t ss_eval_token(ss_model_t *model, int32_t token_id, int32_t pos, float *logits,
                         int32_t *argmax);

/* ss_scheduler_prefill (layer_scheduler.h:119): evaluate n tokens at
 * start_pos.. and return the last token's logits / argmax. */
ss_error_t ss_eval_prompt(ss_model_t *model, const int32_t *tokens, int32_t n,
                          int32_t start_pos, float *logits, int32_t *argmax);

/* Greedy continuation: after ss_eval_token/ss_eval_prompt has produced an
 * argmax at position p, feed it back n_steps times entirely on the device
 * and return the n_steps tokens it produced (positions p+1 .. p+n_steps are
 * evaluated). Equivalent to n_steps calls of ss_eval_token with the previous
 * argmax, without a host round trip per token. */
ss_error_t ss_decode_greedy(ss_model_t *model, int32_t n_steps, int32_t *tokens_out);

/* Write K/V for (layer, pos0 .. pos0+n_pos-1): binary16 arrays of
 * n_pos * n_kv_heads * head_dim, position-major (the reference's
 * [pos][kv_dim] row order). Used to pre-fill long contexts. */
ss_error_t ss_kv_write(ss_model_t *model, int32_t layer, int32_t pos0, int32_t n_pos,
                       const uint16_t *k_f16, const uint16_t *v_f16);

/* The backend handle of a loaded model (an ss_hip_model_t*, include/ss_hip.h),
 * for callers that use the backend C-ABI directly (profiling, tests). */
void *ss_model_hip(ss_model_t *model);

/* tensor.h:115 and :121-123 (host-side, no device involved) */
int32_t ss_argmax(const float *x, int32_t size);
int32_t ss_sample(const float *logits, int32_t vocab_size, float temperature, float top_p,
                  int32_t top_k, uint64_t *rng_state);

#ifdef __cplusplus
}
#endif
#endif /* SLIPSTREAM_H */
