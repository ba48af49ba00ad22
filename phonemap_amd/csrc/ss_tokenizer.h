/*
 * ss_tokenizer.h - GGUF-vocabulary tokenizer (host C).
 *
 * Same observable behaviour as the reference's minimal tokenizer
 * (SlipStream/src/core/tokenizer.c:98-524): SentencePiece score merges or
 * GPT-2 rank merges, "<...>"/"[...]" special-token matching, byte fallback
 * to id byte+3, BOS 1 / EOS 2. Vocabulary lookups use a hash table that
 * resolves a string to the lowest id holding it, which is what the
 * reference's first-match linear scans return.
 */
#ifndef SS_TOKENIZER_H
#define SS_TOKENIZER_H

#include <stdint.h>

typedef struct ss_tok ss_tok_t;

ss_tok_t *ss_tok_create(char **vocab, const float *scores, uint32_t vocab_size, char **merges,
                        uint32_t n_merges, const char *arch);
void ss_tok_free(ss_tok_t *t);
int32_t ss_tok_encode(const ss_tok_t *t, const char *text, int32_t *out, int32_t max_tokens);
const char *ss_tok_decode(const ss_tok_t *t, int32_t id);
int32_t ss_tok_bos(const ss_tok_t *t);
int32_t ss_tok_eos(const ss_tok_t *t);

#endif
