/*
 * ss_tokenizer.c - GGUF-vocabulary tokenizer; behaviour of the reference's
 * src/core/tokenizer.c:98-524, with hash lookups in place of linear scans.
 *
 * Where the reference reads out of bounds (pair strings past 255 bytes are
 * truncated by its snprintf; a merge rule of 512+ bytes overflows its buffer;
 * byte-fallback ids beyond a tiny vocabulary index past its arrays) this
 * implementation truncates the same way, skips the rule, or treats the
 * string as empty, respectively.
 */
#define _GNU_SOURCE
#include "ss_tokenizer.h"

#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct ss_tok {
    char **vocab;
    float *scores;
    int32_t vocab_size;
    int32_t bos_id, eos_id;
    char arch[64];
    char **merges;
    int32_t n_merges;
    bool is_bpe;
    uint32_t hmask;
    int32_t *slots;       /* open addressing: vocab id or -1 */
    int32_t *special;     /* ids of "<...>" / "[...]" entries longer than 2 bytes */
    int32_t n_special;
    uint32_t byte_map[256];
};

static uint32_t fnv1a(const char *s) {
    uint32_t h = 2166136261u;
    for (; *s; s++) h = (h ^ (uint8_t)*s) * 16777619u;
    return h;
}

/* lowest id whose string equals s, or -1 (= the reference's first-match scan) */
static int32_t lookup(const ss_tok_t *t, const char *s) {
    if (!t->slots) return -1;
    for (uint32_t i = fnv1a(s) & t->hmask;; i = (i + 1) & t->hmask) {
        int32_t id = t->slots[i];
        if (id < 0) return -1;
        if (strcmp(t->vocab[id], s) == 0) return id;
    }
}

static int utf8_len(unsigned char c) {   /* tokenizer.c:16-22 */
    if ((c & 0x80) == 0) return 1;
    if ((c & 0xE0) == 0xC0) return 2;
    if ((c & 0xF0) == 0xE0) return 3;
    if ((c & 0xF8) == 0xF0) return 4;
    return 1;
}

/* GPT-2 byte -> code point map (tokenizer.c:45-71) */
static void build_byte_map(uint32_t map[256]) {
    int n = 0;
    for (int b = 0; b < 256; b++) {
        bool raw = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        map[b] = raw ? (uint32_t)b : 0xFFFFFFFFu;
    }
    for (int b = 0; b < 256; b++)
        if (map[b] == 0xFFFFFFFFu) map[b] = 256 + (uint32_t)n++;
}

static int put_utf8(uint32_t c, char *o) {
    if (c <= 0x7F) { o[0] = (char)c; return 1; }
    if (c <= 0x7FF) { o[0] = (char)(0xC0 | (c >> 6)); o[1] = (char)(0x80 | (c & 0x3F)); return 2; }
    if (c <= 0xFFFF) {
        o[0] = (char)(0xE0 | (c >> 12)); o[1] = (char)(0x80 | ((c >> 6) & 0x3F));
        o[2] = (char)(0x80 | (c & 0x3F));
        return 3;
    }
    o[0] = (char)(0xF0 | ((c >> 18) & 0x07)); o[1] = (char)(0x80 | ((c >> 12) & 0x3F));
    o[2] = (char)(0x80 | ((c >> 6) & 0x3F)); o[3] = (char)(0x80 | (c & 0x3F));
    return 4;
}

ss_tok_t *ss_tok_create(char **vocab, const float *scores, uint32_t vocab_size, char **merges,
                        uint32_t n_merges, const char *arch) {
    ss_tok_t *t = (ss_tok_t *)calloc(1, sizeof(ss_tok_t));
    if (!t) return NULL;
    if (arch) strncpy(t->arch, arch, sizeof(t->arch) - 1);
    t->is_bpe = strncmp(t->arch, "qwen2", 5) == 0 || strncmp(t->arch, "qwen35", 6) == 0 ||
                strncmp(t->arch, "llama3", 6) == 0;
    t->bos_id = 1;
    t->eos_id = 2;
    t->vocab_size = (int32_t)vocab_size;
    build_byte_map(t->byte_map);
    if (vocab_size > 0 && vocab) {
        t->vocab = (char **)calloc(vocab_size, sizeof(char *));
        t->scores = (float *)calloc(vocab_size, sizeof(float));
        uint32_t cap = 16;
        while (cap < vocab_size * 2u) cap <<= 1;
        t->slots = (int32_t *)malloc(cap * sizeof(int32_t));
        t->special = (int32_t *)malloc(vocab_size * sizeof(int32_t));
        if (!t->vocab || !t->scores || !t->slots || !t->special) { ss_tok_free(t); return NULL; }
        memset(t->slots, 0xFF, cap * sizeof(int32_t));
        t->hmask = cap - 1;
        for (uint32_t i = 0; i < vocab_size; i++) {
            if (vocab[i]) t->vocab[i] = strdup(vocab[i]);
            t->scores[i] = scores ? scores[i] : (float)strlen(vocab[i] ? vocab[i] : "");
            const char *s = t->vocab[i];
            if (!s) continue;
            size_t n = strlen(s);
            if (n > 2 && ((s[0] == '<' && s[n - 1] == '>') || (s[0] == '[' && s[n - 1] == ']')))
                t->special[t->n_special++] = (int32_t)i;
            if (lookup(t, s) >= 0) continue;   /* keep the lowest id */
            uint32_t h = fnv1a(s) & t->hmask;
            while (t->slots[h] >= 0) h = (h + 1) & t->hmask;
            t->slots[h] = (int32_t)i;
        }
    }
    if (n_merges > 0 && merges) {
        t->n_merges = (int32_t)n_merges;
        t->merges = (char **)calloc(n_merges, sizeof(char *));
        if (!t->merges) { ss_tok_free(t); return NULL; }
        for (uint32_t i = 0; i < n_merges; i++)
            if (merges[i]) t->merges[i] = strdup(merges[i]);
        t->is_bpe = true;
    }
    return t;
}

void ss_tok_free(ss_tok_t *t) {
    if (!t) return;
    if (t->vocab) {
        for (int32_t i = 0; i < t->vocab_size; i++) free(t->vocab[i]);
        free(t->vocab);
    }
    if (t->merges) {
        for (int32_t i = 0; i < t->n_merges; i++) free(t->merges[i]);
        free(t->merges);
    }
    free(t->scores);
    free(t->slots);
    free(t->special);
    free(t);
}

int32_t ss_tok_bos(const ss_tok_t *t) { return t ? t->bos_id : 1; }
int32_t ss_tok_eos(const ss_tok_t *t) { return t ? t->eos_id : 2; }

static const char *tok_str(const ss_tok_t *t, int32_t id) {
    return (id >= 0 && id < t->vocab_size && t->vocab[id]) ? t->vocab[id] : NULL;
}

/* tokenizer.c:153-411 */
int32_t ss_tok_encode(const ss_tok_t *t, const char *text, int32_t *out, int32_t max_tokens) {
    if (!t || !text || !out || max_tokens <= 0) return 0;
    int32_t count = 0;
    if (!t->vocab || t->vocab_size == 0) {
        for (const char *p = text; *p && count < max_tokens; p++) out[count++] = (unsigned char)*p + 3;
        return count;
    }
    static __thread char sp[8192];
    memset(sp, 0, sizeof(sp));
    int si = 0;
    if (t->is_bpe) {
        for (int i = 0; text[i] && si < 8000; i++) si += put_utf8(t->byte_map[(uint8_t)text[i]], sp + si);
    } else {
        sp[si++] = (char)0xE2; sp[si++] = (char)0x96; sp[si++] = (char)0x81;
        for (int i = 0; text[i] && si < 8000; i++) {
            if (text[i] == ' ') { sp[si++] = (char)0xE2; sp[si++] = (char)0x96; sp[si++] = (char)0x81; }
            else sp[si++] = text[i];
        }
    }
    int32_t tokens[4096];
    int n = 0;
    if (!t->is_bpe) tokens[n++] = t->bos_id;
    const char *p = sp;
    while (*p && n < 4000) {
        int off;
        if (p[0] == (char)0xE2 && p[1] == (char)0x96 && p[2] == (char)0x81 && (p[3] == '<' || p[3] == '['))
            off = 3;
        else if (p[0] == '<' || p[0] == '[')
            off = 0;
        else
            off = -1;
        if (off >= 0) {
            const char *ts = p + off;
            int best = -1, best_len = -1;
            for (int32_t k = 0; k < t->n_special; k++) {
                const char *v = t->vocab[t->special[k]];
                int vl = (int)strlen(v);
                if (v[0] == ts[0] && strncmp(ts, v, (size_t)vl) == 0 && vl > best_len) {
                    best_len = vl;
                    best = t->special[k];
                }
            }
            if (best >= 0) {
                tokens[n++] = best;
                p += off + best_len;
                continue;
            }
        }
        int cl = utf8_len((unsigned char)*p);
        char cb[8] = {0};
        for (int i = 0; i < cl && p[i]; i++) cb[i] = p[i];
        int32_t id = lookup(t, cb);
        if (id >= 0) {
            tokens[n++] = id;
        } else {
            for (int i = 0; i < cl && p[i]; i++) tokens[n++] = (int32_t)(unsigned char)p[i] + 3;
        }
        p += cl;
    }

    if (t->is_bpe && t->merges && t->n_merges > 0) {              /* rank merges, :283-341 */
        for (int32_t rank = 0; rank < t->n_merges; rank++) {
            if (n <= 1) break;
            const char *rule = t->merges[rank];
            if (!rule) continue;
            const char *sp2 = strchr(rule, ' ');
            if (!sp2) continue;
            int l1 = (int)(sp2 - rule);
            const char *part2 = sp2 + 1;
            int l2 = (int)strlen(part2);
            if (l1 + l2 >= 512) continue;
            char merged[512];
            memcpy(merged, rule, (size_t)l1);
            memcpy(merged + l1, part2, (size_t)l2);
            merged[l1 + l2] = 0;
            int32_t mid = lookup(t, merged);
            if (mid < 0) continue;
            bool found = true;
            while (found) {
                found = false;
                for (int i = 0; i < n - 1; i++) {
                    const char *s1 = tok_str(t, tokens[i]), *s2 = tok_str(t, tokens[i + 1]);
                    if (!s1 || !s2) continue;
                    if ((int)strlen(s1) == l1 && (int)strlen(s2) == l2 &&
                        strncmp(s1, rule, (size_t)l1) == 0 && strcmp(s2, part2) == 0) {
                        tokens[i] = mid;
                        memmove(tokens + i + 1, tokens + i + 2, sizeof(int32_t) * (size_t)(n - i - 2));
                        n--;
                        found = true;
                        break;
                    }
                }
            }
        }
    } else {                                                       /* score merges, :342-392 */
        for (;;) {
            float best_score = -1e10f;
            int32_t best_id = -1;
            int best_idx = -1;
            for (int i = 0; i < n - 1; i++) {
                const char *s1 = tok_str(t, tokens[i]);
                const char *s2 = tok_str(t, tokens[i + 1]);
                if (!s1) s1 = "";
                if (!s2) s2 = "";
                char f1[2] = {0}, f2[2] = {0};
                if (tokens[i] >= 3 && tokens[i] < 259) { f1[0] = (char)(tokens[i] - 3); s1 = f1; }
                if (tokens[i + 1] >= 3 && tokens[i + 1] < 259) { f2[0] = (char)(tokens[i + 1] - 3); s2 = f2; }
                char pair[256];
                snprintf(pair, sizeof(pair), "%s%s", s1, s2);
                int32_t id = lookup(t, pair);
                if (id != -1 && t->scores[id] > best_score) {
                    best_score = t->scores[id];
                    best_id = id;
                    best_idx = i;
                }
            }
            if (best_idx == -1) break;
            tokens[best_idx] = best_id;
            memmove(tokens + best_idx + 1, tokens + best_idx + 2, sizeof(int32_t) * (size_t)(n - best_idx - 2));
            n--;
        }
    }
    for (int i = 0; i < n && count < max_tokens; i++) out[count++] = tokens[i];
    return count;
}

static int hexv(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'A' && c <= 'F') return 10 + c - 'A';
    if (c >= 'a' && c <= 'f') return 10 + c - 'a';
    return -1;
}

/* tokenizer.c:422-524 */
const char *ss_tok_decode(const ss_tok_t *t, int32_t id) {
    if (!t) return "";
    if (id == t->bos_id || id == t->eos_id || id == 0) return "";
    static __thread char buf[512];
    if (t->vocab && id >= 0 && id < t->vocab_size) {
        const char *raw = t->vocab[id];
        if (!raw) return "";
        if (strlen(raw) == 6 && raw[0] == '<' && raw[1] == '0' && raw[2] == 'x' && raw[5] == '>') {
            int hi = hexv(raw[3]), lo = hexv(raw[4]);
            if (hi >= 0 && lo >= 0) {
                buf[0] = (char)((hi << 4) | lo);
                buf[1] = 0;
                return buf;
            }
        }
        int o = 0, i = 0;
        if (t->is_bpe) {
            while (raw[i] && o < 500) {
                unsigned char c = (unsigned char)raw[i];
                uint32_t cp;
                int cl;
                if ((c & 0x80) == 0) { cp = c; cl = 1; }
                else if ((c & 0xE0) == 0xC0 && raw[i + 1]) { cp = ((c & 0x1Fu) << 6) | (raw[i + 1] & 0x3F); cl = 2; }
                else if ((c & 0xF0) == 0xE0 && raw[i + 1] && raw[i + 2]) {
                    cp = ((c & 0x0Fu) << 12) | ((raw[i + 1] & 0x3Fu) << 6) | (raw[i + 2] & 0x3F);
                    cl = 3;
                } else if (raw[i + 1] && raw[i + 2] && raw[i + 3]) {
                    cp = ((c & 0x07u) << 18) | ((raw[i + 1] & 0x3Fu) << 12) | ((raw[i + 2] & 0x3Fu) << 6) |
                         (raw[i + 3] & 0x3F);
                    cl = 4;
                } else { cp = c; cl = 1; }
                int mapped = -1;
                for (int b = 0; b < 256; b++)
                    if (t->byte_map[b] == cp) { mapped = b; break; }
                if (mapped >= 0) buf[o++] = (char)mapped;
                else
                    for (int j = 0; j < cl && o < 500; j++) buf[o++] = raw[i + j];
                i += cl;
            }
        } else {
            while (raw[i] && o < 500) {
                if ((unsigned char)raw[i] == 0xE2 && (unsigned char)raw[i + 1] == 0x96 &&
                    (unsigned char)raw[i + 2] == 0x81) {
                    buf[o++] = ' ';
                    i += 3;
                } else {
                    buf[o++] = raw[i++];
                }
            }
        }
        buf[o] = 0;
        return buf;
    }
    if (id >= 3 && id < 259) {
        buf[0] = (char)(id - 3);
        buf[1] = 0;
        return buf;
    }
    return "";
}
