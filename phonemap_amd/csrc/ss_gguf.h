/*
 * ss_gguf.h - GGUF v2/v3 model file reader (host C).
 *
 * Same parsing rules as the reference loader
 * (SlipStream/src/core/gguf_loader.c:210-485): metadata keys matched by
 * suffix and by value type, vocabulary size from the tokenizer.ggml.tokens
 * array, tensor data at the first 32-byte boundary after the tensor infos,
 * tensors indexed per "blk.N." layer. The file is mmapped read-only; tensor
 * data pointers point into the mapping.
 */
#ifndef SS_GGUF_H
#define SS_GGUF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor types (gguf_loader.h:41-55) */
enum {
    SS_GGML_F32 = 0, SS_GGML_F16 = 1, SS_GGML_Q4_0 = 2, SS_GGML_Q4_1 = 3, SS_GGML_Q5_0 = 6,
    SS_GGML_Q5_1 = 7, SS_GGML_Q8_0 = 8, SS_GGML_Q8_1 = 9, SS_GGML_Q2_K = 10, SS_GGML_Q3_K = 11,
    SS_GGML_Q4_K = 12, SS_GGML_Q5_K = 13, SS_GGML_Q6_K = 14
};

typedef struct {
    char name[256];
    uint32_t n_dims;
    uint64_t dims[4];      /* dims[0] = columns, dims[1] = rows */
    int32_t type;
    uint64_t offset;       /* absolute file offset */
    uint64_t size_bytes;
    int32_t layer_index;   /* -1 for non-layer tensors */
} ss_gguf_tensor_t;

typedef struct {
    uint32_t num_tensors;
    ss_gguf_tensor_t **tensors;   /* pointers into the catalog */
    uint64_t total_size;
} ss_gguf_layer_t;

typedef struct {
    int fd;
    uint64_t file_size;
    uint8_t *base;
    uint64_t data_offset;
    uint32_t version;
    uint64_t n_tensors, n_kv;
    ss_gguf_tensor_t *tensors;
    ss_gguf_layer_t *layers;
    uint32_t num_layers;
    char arch[64];
    uint32_t hidden_size, num_heads, num_kv_heads, vocab_size, context_length;
    uint32_t intermediate_size, head_dim, rope_dim;
    float rope_theta, rms_norm_eps, attn_logit_softcapping, final_logit_softcapping;
    char **vocab;
    float *vocab_scores;
    char **merges;
    uint32_t n_merges;
} ss_gguf_file_t;

/* error detail of the last failed ss_gguf_open on this thread */
const char *ss_gguf_error(void);

ss_gguf_file_t *ss_gguf_open(const char *path);
void ss_gguf_close(ss_gguf_file_t *f);
const void *ss_gguf_tensor_data(const ss_gguf_file_t *f, const ss_gguf_tensor_t *t);
const ss_gguf_tensor_t *ss_gguf_find(const ss_gguf_file_t *f, const char *name);
const ss_gguf_tensor_t *ss_gguf_find_in_layer(const ss_gguf_file_t *f, uint32_t layer,
                                              const char *suffix);
uint64_t ss_ggml_type_size(int32_t type);
uint32_t ss_ggml_block_size(int32_t type);

#ifdef __cplusplus
}
#endif
#endif
