/*
 * ss_gguf.c - GGUF v2/v3 reader with the reference loader's rules
 * (SlipStream/src/core/gguf_loader.c:210-485).
 */
#define _GNU_SOURCE
#include "ss_gguf.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static __thread char g_gguf_err[256];

static void gerr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_gguf_err, sizeof(g_gguf_err), fmt, ap);
    va_end(ap);
}

const char *ss_gguf_error(void) { return g_gguf_err; }

/* gguf_loader.c:22-62 */
uint64_t ss_ggml_type_size(int32_t t) {
    switch (t) {
    case SS_GGML_F32: return 4;
    case SS_GGML_F16: return 2;
    case SS_GGML_Q4_0: return 18;
    case SS_GGML_Q4_1: return 20;
    case SS_GGML_Q5_0: return 22;
    case SS_GGML_Q5_1: return 24;
    case SS_GGML_Q8_0: return 34;
    case SS_GGML_Q8_1: return 40;
    case SS_GGML_Q2_K: return 84;
    case SS_GGML_Q3_K: return 110;
    case SS_GGML_Q4_K: return 144;
    case SS_GGML_Q5_K: return 176;
    case SS_GGML_Q6_K: return 210;
    default: return 0;
    }
}

uint32_t ss_ggml_block_size(int32_t t) {
    switch (t) {
    case SS_GGML_Q4_0: case SS_GGML_Q4_1: case SS_GGML_Q5_0: case SS_GGML_Q5_1:
    case SS_GGML_Q8_0: case SS_GGML_Q8_1: return 32;
    case SS_GGML_Q2_K: case SS_GGML_Q3_K: case SS_GGML_Q4_K: case SS_GGML_Q5_K:
    case SS_GGML_Q6_K: return 256;
    default: return 1;
    }
}

typedef struct {
    const uint8_t *p;
    uint64_t pos, size;
    int bad;
} reader_t;

static int need(reader_t *r, uint64_t n) {
    if (r->bad || n > r->size - r->pos) { r->bad = 1; return 0; }
    return 1;
}
static uint32_t u32(reader_t *r) {
    uint32_t v = 0;
    if (need(r, 4)) { memcpy(&v, r->p + r->pos, 4); r->pos += 4; }
    return v;
}
static uint64_t u64(reader_t *r) {
    uint64_t v = 0;
    if (need(r, 8)) { memcpy(&v, r->p + r->pos, 8); r->pos += 8; }
    return v;
}
static float f32(reader_t *r) {
    uint32_t u = u32(r);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* length-prefixed string view into the file */
static const char *str(reader_t *r, uint64_t *len) {
    *len = u64(r);
    if (!need(r, *len)) return NULL;
    const char *s = (const char *)r->p + r->pos;
    r->pos += *len;
    return s;
}
static char *dupstr(reader_t *r) {
    uint64_t n;
    const char *s = str(r, &n);
    if (!s) return NULL;
    char *o = (char *)malloc(n + 1);
    if (!o) { r->bad = 1; return NULL; }
    memcpy(o, s, n);
    o[n] = 0;
    return o;
}

static void skip_value(reader_t *r, uint32_t type, int depth) {   /* gguf_loader.c:130-165 */
    uint64_t n;
    if (depth > 4) { r->bad = 1; return; }
    switch (type) {
    case 0: case 1: case 7: if (need(r, 1)) r->pos += 1; break;
    case 2: case 3: if (need(r, 2)) r->pos += 2; break;
    case 4: case 5: case 6: if (need(r, 4)) r->pos += 4; break;
    case 10: case 11: case 12: if (need(r, 8)) r->pos += 8; break;
    case 8: str(r, &n); break;
    case 9: {
        uint32_t at = u32(r);
        uint64_t cnt = u64(r);
        for (uint64_t i = 0; i < cnt && !r->bad; i++) skip_value(r, at, depth + 1);
        break;
    }
    default: r->bad = 1; break;
    }
}

static int ends_with(const char *k, uint64_t kl, const char *s) {
    size_t sl = strlen(s);
    return kl >= sl && memcmp(k + kl - sl, s, sl) == 0;
}
static int equals(const char *k, uint64_t kl, const char *s) {
    return kl == strlen(s) && memcmp(k, s, kl) == 0;
}

static int32_t layer_of(const char *name) {   /* gguf_loader.c:174-189 */
    const char *b = strstr(name, "blk.");
    if (!b) return -1;
    int32_t idx = 0;
    const char *p = b + 4;
    while (*p >= '0' && *p <= '9') { idx = idx * 10 + (*p - '0'); p++; }
    return *p == '.' ? idx : -1;
}

void ss_gguf_close(ss_gguf_file_t *f) {
    if (!f) return;
    if (f->vocab) {
        for (uint32_t i = 0; i < f->vocab_size; i++) free(f->vocab[i]);
        free(f->vocab);
    }
    free(f->vocab_scores);
    if (f->merges) {
        for (uint32_t i = 0; i < f->n_merges; i++) free(f->merges[i]);
        free(f->merges);
    }
    if (f->layers) {
        for (uint32_t i = 0; i < f->num_layers; i++) free(f->layers[i].tensors);
        free(f->layers);
    }
    free(f->tensors);
    if (f->base) munmap(f->base, f->file_size);
    if (f->fd >= 0) close(f->fd);
    free(f);
}

static int read_string_array(reader_t *r, char ***out, uint32_t *count) {
    uint32_t at = u32(r);
    uint64_t n = u64(r);
    if (r->bad) return -1;
    if (at != 8 || n == 0) {
        for (uint64_t i = 0; i < n && !r->bad; i++) skip_value(r, at, 1);
        return r->bad ? -1 : 0;
    }
    if (n > r->size / 8) { r->bad = 1; return -1; }
    char **a = (char **)calloc(n, sizeof(char *));
    if (!a) return -1;
    for (uint64_t i = 0; i < n; i++) {
        a[i] = dupstr(r);
        if (!a[i]) {
            for (uint64_t j = 0; j < i; j++) free(a[j]);
            free(a);
            return -1;
        }
    }
    if (*out) {   /* a repeated key: keep the last one */
        for (uint32_t i = 0; i < *count; i++) free((*out)[i]);
        free(*out);
    }
    *out = a;
    *count = (uint32_t)n;
    return 0;
}

ss_gguf_file_t *ss_gguf_open(const char *path) {
    g_gguf_err[0] = 0;
    if (!path) { gerr("null path"); return NULL; }
    ss_gguf_file_t *f = (ss_gguf_file_t *)calloc(1, sizeof(ss_gguf_file_t));
    if (!f) { gerr("out of memory"); return NULL; }
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) { gerr("cannot open %s", path); free(f); return NULL; }
    struct stat st;
    if (fstat(f->fd, &st) < 0 || st.st_size < 24) {
        gerr("cannot stat %s or file too small", path);
        ss_gguf_close(f);
        return NULL;
    }
    f->file_size = (uint64_t)st.st_size;
    void *base = mmap(NULL, f->file_size, PROT_READ, MAP_SHARED, f->fd, 0);
    if (base == MAP_FAILED) { gerr("mmap failed"); ss_gguf_close(f); return NULL; }
    f->base = (uint8_t *)base;

    reader_t r = {f->base, 0, f->file_size, 0};
    if (u32(&r) != 0x46554747u) { gerr("bad magic"); ss_gguf_close(f); return NULL; }
    f->version = u32(&r);
    if (f->version < 2 || f->version > 3) {
        gerr("unsupported GGUF version %u", f->version);
        ss_gguf_close(f);
        return NULL;
    }
    f->n_tensors = u64(&r);
    f->n_kv = u64(&r);
    uint32_t n_tok_strings = 0;
    uint64_t n_scores = 0;
    /* Data alignment: general.alignment when present (the GGUF format's rule;
     * a power of two), else 32. The reference always uses 32
     * (gguf_loader.c:426), which misplaces the data of any other alignment. */
    uint64_t align = 32;
    for (uint64_t i = 0; i < f->n_kv && !r.bad; i++) {   /* gguf_loader.c:270-364 */
        uint64_t kl;
        const char *k = str(&r, &kl);
        if (!k) break;
        uint32_t vt = u32(&r);
        if (equals(k, kl, "general.architecture") && vt == 8) {
            uint64_t sl;
            const char *s = str(&r, &sl);
            if (s) {
                size_t c = sl < sizeof(f->arch) - 1 ? sl : sizeof(f->arch) - 1;
                memcpy(f->arch, s, c);
                f->arch[c] = 0;
            }
        } else if (equals(k, kl, "general.alignment") && vt == 4) {
            align = u32(&r);
            if (align == 0 || (align & (align - 1))) {
                gerr("general.alignment %llu is not a power of two", (unsigned long long)align);
                ss_gguf_close(f);
                return NULL;
            }
        } else if (ends_with(k, kl, ".embedding_length") && vt == 4) {
            f->hidden_size = u32(&r);
        } else if (ends_with(k, kl, ".attention.head_count_kv") && vt == 4) {
            f->num_kv_heads = u32(&r);
        } else if (ends_with(k, kl, ".attention.head_count") && vt == 4) {
            f->num_heads = u32(&r);
        } else if (ends_with(k, kl, ".context_length") && vt == 4) {
            f->context_length = u32(&r);
        } else if (ends_with(k, kl, ".feed_forward_length") && vt == 4) {
            f->intermediate_size = u32(&r);
        } else if (ends_with(k, kl, ".block_count") && vt == 4) {
            f->num_layers = u32(&r);
        } else if (ends_with(k, kl, ".vocab_size") && vt == 4) {
            f->vocab_size = u32(&r);
        } else if (ends_with(k, kl, ".rope.freq_base") && vt == 6) {
            f->rope_theta = f32(&r);
        } else if (ends_with(k, kl, ".attention.layer_norm_rms_epsilon") && vt == 6) {
            f->rms_norm_eps = f32(&r);
        } else if (ends_with(k, kl, ".attention.key_length") && vt == 4) {
            f->head_dim = u32(&r);
        } else if (ends_with(k, kl, ".rope.dimension_count") && vt == 4) {
            f->rope_dim = u32(&r);
        } else if (ends_with(k, kl, ".attn_logit_softcapping") && vt == 6) {
            f->attn_logit_softcapping = f32(&r);
        } else if (ends_with(k, kl, ".final_logit_softcapping") && vt == 6) {
            f->final_logit_softcapping = f32(&r);
        } else if (equals(k, kl, "tokenizer.ggml.tokens") && vt == 9) {
            if (read_string_array(&r, &f->vocab, &n_tok_strings) != 0) break;
            if (n_tok_strings) f->vocab_size = n_tok_strings;
        } else if (equals(k, kl, "tokenizer.ggml.scores") && vt == 9) {
            uint32_t at = u32(&r);
            uint64_t n = u64(&r);
            if (at == 6 && n > 0 && n <= r.size / 4) {
                free(f->vocab_scores);
                f->vocab_scores = (float *)malloc(n * sizeof(float));
                if (!f->vocab_scores) { r.bad = 1; break; }
                for (uint64_t v = 0; v < n; v++) f->vocab_scores[v] = f32(&r);
                n_scores = n;
            } else {
                for (uint64_t v = 0; v < n && !r.bad; v++) skip_value(&r, at, 1);
            }
        } else if (equals(k, kl, "tokenizer.ggml.merges") && vt == 9) {
            if (read_string_array(&r, &f->merges, &f->n_merges) != 0) break;
        } else {
            skip_value(&r, vt, 0);
        }
    }
    if (r.bad) { gerr("metadata truncated or malformed"); ss_gguf_close(f); return NULL; }
    /* scores are used only with a vocab of exactly as many tokens; otherwise
     * the tokenizer ranks merges by string length (the reference reads
     * scores[i] for every token regardless, past the end of a short array) */
    if (f->vocab_scores && (!f->vocab || n_scores != n_tok_strings)) {
        free(f->vocab_scores);
        f->vocab_scores = NULL;
    }
    if (f->vocab && f->vocab_size != n_tok_strings) f->vocab_size = n_tok_strings;

    if (f->rms_norm_eps == 0.0f) f->rms_norm_eps = 1e-5f;            /* gguf_loader.c:370-379 */
    if (f->rope_theta == 0.0f) f->rope_theta = strstr(f->arch, "qwen") ? 1000000.0f : 10000.0f;
    if (f->context_length == 0) f->context_length = 2048;

    if (f->n_tensors > r.size / 24) { gerr("tensor count %llu implausible", (unsigned long long)f->n_tensors); ss_gguf_close(f); return NULL; }
    f->tensors = (ss_gguf_tensor_t *)calloc(f->n_tensors ? f->n_tensors : 1, sizeof(ss_gguf_tensor_t));
    if (!f->tensors) { gerr("out of memory"); ss_gguf_close(f); return NULL; }
    for (uint64_t i = 0; i < f->n_tensors && !r.bad; i++) {          /* :389-417 */
        ss_gguf_tensor_t *t = &f->tensors[i];
        uint64_t nl;
        const char *nm = str(&r, &nl);
        if (!nm) break;
        size_t c = nl < sizeof(t->name) - 1 ? nl : sizeof(t->name) - 1;
        memcpy(t->name, nm, c);
        t->name[c] = 0;
        t->n_dims = u32(&r);
        if (t->n_dims > 4) { r.bad = 1; break; }
        for (uint32_t d = 0; d < t->n_dims; d++) t->dims[d] = u64(&r);
        t->type = (int32_t)u32(&r);
        t->offset = u64(&r);
        if (f->vocab_size == 0 && strcmp(t->name, "token_embd.weight") == 0 && t->n_dims == 2)
            f->vocab_size = (uint32_t)t->dims[1];
        uint64_t ne = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) ne *= t->dims[d];
        uint32_t bs = ss_ggml_block_size(t->type);
        t->size_bytes = (bs == 1 ? ne : ne / bs) * ss_ggml_type_size(t->type);
        t->layer_index = layer_of(t->name);
    }
    if (r.bad) { gerr("tensor table truncated or malformed"); ss_gguf_close(f); return NULL; }
    f->data_offset = (r.pos + align - 1) & ~(align - 1);             /* :426 */
    for (uint64_t i = 0; i < f->n_tensors; i++) f->tensors[i].offset += f->data_offset;

    if (f->num_layers > 0) {                                           /* :434-475 */
        if (f->num_layers > 100000) { gerr("block_count implausible"); ss_gguf_close(f); return NULL; }
        f->layers = (ss_gguf_layer_t *)calloc(f->num_layers, sizeof(ss_gguf_layer_t));
        if (!f->layers) { gerr("out of memory"); ss_gguf_close(f); return NULL; }
        for (uint64_t i = 0; i < f->n_tensors; i++) {
            int32_t li = f->tensors[i].layer_index;
            if (li >= 0 && (uint32_t)li < f->num_layers) f->layers[li].num_tensors++;
        }
        for (uint32_t l = 0; l < f->num_layers; l++) {
            f->layers[l].tensors = (ss_gguf_tensor_t **)calloc(
                f->layers[l].num_tensors ? f->layers[l].num_tensors : 1, sizeof(ss_gguf_tensor_t *));
            if (!f->layers[l].tensors) { gerr("out of memory"); ss_gguf_close(f); return NULL; }
            f->layers[l].num_tensors = 0;
        }
        for (uint64_t i = 0; i < f->n_tensors; i++) {
            int32_t li = f->tensors[i].layer_index;
            if (li >= 0 && (uint32_t)li < f->num_layers) {
                ss_gguf_layer_t *L = &f->layers[li];
                L->tensors[L->num_tensors++] = &f->tensors[i];
                L->total_size += f->tensors[i].size_bytes;
            }
        }
    }
    madvise(f->base, (size_t)f->file_size, MADV_SEQUENTIAL);          /* :480-482 */
    return f;
}

const void *ss_gguf_tensor_data(const ss_gguf_file_t *f, const ss_gguf_tensor_t *t) {
    if (!f || !t || !f->base) return NULL;                             /* :487-492 */
    if (t->offset > f->file_size || t->size_bytes > f->file_size - t->offset) return NULL;
    return f->base + t->offset;
}

const ss_gguf_tensor_t *ss_gguf_find(const ss_gguf_file_t *f, const char *name) {
    for (uint64_t i = 0; f && i < f->n_tensors; i++)
        if (strcmp(f->tensors[i].name, name) == 0) return &f->tensors[i];
    return NULL;
}

/* layer_scheduler.c:27-39: first tensor of the layer whose name ends in suffix */
const ss_gguf_tensor_t *ss_gguf_find_in_layer(const ss_gguf_file_t *f, uint32_t layer,
                                              const char *suffix) {
    if (!f || !f->layers || layer >= f->num_layers) return NULL;
    size_t sl = strlen(suffix);
    const ss_gguf_layer_t *L = &f->layers[layer];
    for (uint32_t i = 0; i < L->num_tensors; i++) {
        const char *n = L->tensors[i]->name;
        size_t nl = strlen(n);
        if (nl >= sl && strcmp(n + nl - sl, suffix) == 0) return L->tensors[i];
    }
    return NULL;
}
