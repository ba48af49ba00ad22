/*
 * ss_synth.h - seeded synthetic Llama-architecture GGUF writer.
 *
 * Produces benchmark and test models with random-initialised weights in the
 * layout the reference loader reads (SlipStream/src/core/gguf_loader.c:282-361:
 * UINT32/FLOAT32 metadata, a 32-byte-aligned data section, dims[0] = columns,
 * dims[1] = rows). No counterpart in the reference; it stands in for the
 * checkpoints that cannot be downloaded.
 *
 * Distributions: Q4_0 blocks have uniform random nibbles, Q8_0 blocks int8
 * codes uniform in [-127, 127]. The block scale d is, with scale_mode 0,
 * fp16(|N(0, scale_sigma)|) for Q4_0 and fp16(|N(0, scale_sigma / 16)|) for
 * Q8_0 (the codes' spread is 16 times the nibbles', so both types give
 * weights of the same spread); with scale_mode 1 it is signed,
 * fp16(N(0, 1 / (c * sqrt(cols)))) with c the RMS of the codes (sqrt(21.5)
 * for Q4_0 nibbles - 8, sqrt(127 * 128 / 3) for Q8_0), so every weight has
 * standard deviation 1/sqrt(cols) and zero mean. Q4_K super-blocks have
 * random 6-bit scales and mins and uniform nibbles, with d and dmin drawn as
 * the Q4_0 d (mode 1: weight spread 1/sqrt(cols) again; mode 0:
 * |N(0, scale_sigma / 64)|). Q2_K, Q3_K, Q5_K and Q6_K super-blocks have
 * every code and scale byte uniformly random and d (and dmin) drawn so that
 * the weights spread 1/sqrt(cols) in mode 1. Mode 0 with positive d
 * gives every Q4_0 block the mean -d/2 (nibbles average 7.5 - 8): a shared
 * direction that, compounded over the layers, makes deep models emit nearly
 * the same logits for any input; mode 1 models respond to their input.
 * Norm weights are fp32 1 + N(0, norm_sigma) (Gemma: N(0, norm_sigma), the
 * file format's weight minus one); q/k/v biases (when asked for) are
 * N(0, 0.1).
 * The bytes depend only on the spec (seed included), not on n_threads.
 */
#ifndef SS_SYNTH_H
#define SS_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, context_length;
    float rope_theta, rms_eps;
    int32_t layer_type;   /* ggml type of the layer matrices: 0 (F32), 1 (F16), 2 (Q4_0),
                           * 3 (Q4_1), 6 (Q5_0), 7 (Q5_1), 8 (Q8_0), 9 (Q8_1) or a K-quant,
                           * 10 (Q2_K), 11 (Q3_K), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) (hidden, ffn
                           * and n_heads * head_dim multiples of 256) */
    int32_t embd_type;    /* token_embd.weight */
    int32_t out_type;     /* output.weight; -1 = tied to token_embd (no output.weight) */
    uint64_t seed;
    float scale_sigma;    /* 0 = 0.02 */
    float norm_sigma;     /* 0 = 0.01 */
    int32_t with_vocab;   /* write tokenizer.ggml.tokens/scores (SentencePiece-style) */
    int32_t n_threads;    /* 0 = hardware concurrency */
    /* Architecture variants. A variant changes no weight: a fused or biased
     * file holds the same matrices as the plain one with the same seed. */
    int32_t arch;         /* 0: "llama"; 1: "qwen2" (NeoX RoPE, layer_scheduler.c:145-149);
                           * 2: "gemma" (norm weights N(0, norm_sigma), applied as 1 + w);
                           * 3: "gemma2" (as 2, plus blk.N.post_attention_norm and
                           * blk.N.post_ffw_norm, layer_scheduler.c:309-310) */
    int32_t fused_qkv;    /* blk.N.attn_qkv.weight = [Wq; Wk; Wv] in place of three tensors */
    int32_t fused_up;     /* blk.N.ffn_up.weight = [Wgate; Wup] (2 * ffn rows), no ffn_gate */
    int32_t qkv_bias;     /* blk.N.attn_q/k/v.bias: 0 none, 1 F32, 2 F16; values N(0, 0.1) */
    int32_t alignment;    /* general.alignment and the data/tensor alignment in bytes (a power
                           * of two); 0 = 32, the only alignment the reference reads */
    int32_t scale_mode;   /* block scale distribution, see above: 0 |N(0, scale_sigma)|,
                           * 1 signed fan-in scaled */
    int32_t vocab_tokens; /* with with_vocab: tokenizer strings written, when in [1, vocab)
                           * (0 = vocab). Fewer than vocab leaves token_embd/output rows past
                           * the vocabulary, as padded tables do; the loaders clamp the
                           * vocabulary to the tokenizer (layer_scheduler.c:186-197). */
    float attn_softcap;   /* > 0: <arch>.attn_logit_softcapping (layer_scheduler.c:446-448) */
    float final_softcap;  /* > 0: <arch>.final_logit_softcapping (:674-676) */
} ss_synth_spec_t;

/* Returns 0, or a negative ss_error_t value (-5 bad spec, -1 cannot write). */
int32_t ss_synth_gguf_write(const char *path, const ss_synth_spec_t *spec);

/* Vocabulary string i of the synthetic tokenizer (for tests); NULL if i is out of range. */
const char *ss_synth_vocab_string(int32_t vocab, int32_t i, char *buf, int32_t len);

#ifdef __cplusplus
}
#endif
#endif
