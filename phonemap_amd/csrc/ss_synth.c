/*
 * ss_synth.c - seeded synthetic Llama GGUF writer (see include/ss_synth.h).
 *
 * Tensor bytes are generated in independent chunks, each from its own
 * xoshiro256** stream seeded from (seed, tensor, chunk), and written with
 * pwrite by a small thread pool, so a 40 GB file is produced at disk speed
 * and the bytes do not depend on the thread count.
 */
#define _GNU_SOURCE
#include "ss_synth.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define T_F32 0
#define T_F16 1
#define T_Q4_0 2
#define T_Q4_1 3
#define T_Q5_0 6
#define T_Q5_1 7
#define T_Q8_0 8
#define T_Q8_1 9
#define T_Q4_K 12
#define T_Q2_K 10
#define T_Q3_K 11
#define T_Q5_K 13
#define T_Q6_K 14
/* the K-quants: super-blocks of 256 weights */
static int is_k(int32_t type) { return type >= T_Q2_K && type <= T_Q6_K; }
static size_t k_bytes(int32_t type) {
    return type == T_Q2_K ? 84 : type == T_Q3_K ? 110 : type == T_Q4_K ? 144 : type == T_Q5_K ? 176 : 210;
}
/* the matrix types the writer makes: float, 32-weight blocks, K-quants */
static int matrix_type_ok(int32_t type) {
    return type == T_F32 || type == T_F16 || type == T_Q4_0 || type == T_Q4_1 || type == T_Q5_0 || type == T_Q5_1 ||
           type == T_Q8_0 || type == T_Q8_1 || is_k(type);
}
#define CHUNK_BLOCKS (1u << 18)   /* 256 Ki blocks per work item */
#define MAX_BLOCK_BYTES 128       /* F32: 32 weights */

typedef struct {
    char name[64];
    uint32_t n_dims;
    uint64_t dims[2];
    int32_t type;
    uint64_t offset;   /* relative to the data section */
    uint64_t bytes;
    int norm;          /* 1: norm weight 1 + N(0, norm_sigma); 2: bias N(0, kBiasSigma);
                        * 3: Gemma norm weight N(0, norm_sigma) (applied as 1 + w) */
    uint64_t sid;      /* seed id of the random stream: the tensor's index in the unfused,
                        * bias-free layout, so fused and biased files keep every weight */
    int join_next;     /* the next tensor continues this one's rows (one fused GGUF tensor) */
} syn_tensor_t;

static const double kBiasSigma = 0.1;

/* ---- random numbers ---- */
static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
typedef struct { uint64_t s[4]; } xo_t;
static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
static uint64_t xo_next(xo_t *x) {
    uint64_t r = rotl(x->s[1] * 5, 7) * 9, t = x->s[1] << 17;
    x->s[2] ^= x->s[0]; x->s[3] ^= x->s[1]; x->s[1] ^= x->s[2]; x->s[0] ^= x->s[3];
    x->s[2] ^= t; x->s[3] = rotl(x->s[3], 45);
    return r;
}
static void xo_seed(xo_t *x, uint64_t seed, uint64_t a, uint64_t b) {
    uint64_t s = seed ^ (a * 0xD1B54A32D192ED03ull) ^ (b * 0x8CB92BA72F3D8DD7ull);
    for (int i = 0; i < 4; i++) x->s[i] = splitmix64(&s);
}
static double xo_unit(xo_t *x) { return ((xo_next(x) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
static double xo_normal(xo_t *x) {   /* Box-Muller */
    double u1 = xo_unit(x), u2 = xo_unit(x);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static uint16_t to_f16(float f) {    /* IEEE binary16, round to nearest even */
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x477FF000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    uint32_t e = ax >> 23;
    if (e >= 113) {
        uint32_t m = ax & 0x7FFFFFu, h = ((e - 112) << 10) | (m >> 13), rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (e < 102) return (uint16_t)sign;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u, sh = 126 - e, h = m >> sh;
    uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* tokenizer strings written: vocab_tokens when set (a table with rows past the vocabulary) */
static int32_t n_tokens(const ss_synth_spec_t *s) {
    return s->vocab_tokens > 0 && s->vocab_tokens < s->vocab ? s->vocab_tokens : s->vocab;
}

/* ---- synthetic SentencePiece-style vocabulary ---- */
static void word_of(uint64_t n, char *out) {   /* bijective base-26: a..z, aa, ab, ... */
    char tmp[16];
    int k = 0;
    n += 1;
    while (n > 0 && k < 15) { n -= 1; tmp[k++] = (char)('a' + n % 26); n /= 26; }
    for (int i = 0; i < k; i++) out[i] = tmp[k - 1 - i];
    out[k] = 0;
}

const char *ss_synth_vocab_string(int32_t vocab, int32_t i, char *buf, int32_t len) {
    if (i < 0 || i >= vocab || !buf || len < 32) return NULL;
    if (i == 0) { snprintf(buf, len, "<unk>"); return buf; }
    if (i == 1) { snprintf(buf, len, "<s>"); return buf; }
    if (i == 2) { snprintf(buf, len, "</s>"); return buf; }
    if (i < 259) { snprintf(buf, len, "<0x%02X>", i - 3); return buf; }
    if (i == 259) { snprintf(buf, len, "\xE2\x96\x81"); return buf; }   /* U+2581 */
    if (i < 259 + 1 + 94) { buf[0] = (char)(0x21 + (i - 260)); buf[1] = 0; return buf; }
    uint64_t k = (uint64_t)(i - 354);
    char w[16];
    word_of(k / 2, w);
    if (k % 2 == 0) snprintf(buf, len, "\xE2\x96\x81%s", w);
    else snprintf(buf, len, "%s", w);
    return buf;
}

/* ---- GGUF serialisation ---- */
typedef struct { uint8_t *p; size_t n, cap; int bad; } wbuf_t;
static void wb_put(wbuf_t *b, const void *d, size_t n) {
    if (b->bad) return;
    if (b->n + n > b->cap) {
        size_t c = b->cap ? b->cap * 2 : 1 << 16;
        while (c < b->n + n) c *= 2;
        uint8_t *q = (uint8_t *)realloc(b->p, c);
        if (!q) { b->bad = 1; return; }
        b->p = q;
        b->cap = c;
    }
    memcpy(b->p + b->n, d, n);
    b->n += n;
}
static void wb_u32(wbuf_t *b, uint32_t v) { wb_put(b, &v, 4); }
static void wb_u64(wbuf_t *b, uint64_t v) { wb_put(b, &v, 8); }
static void wb_f32(wbuf_t *b, float v) { wb_put(b, &v, 4); }
static void wb_str(wbuf_t *b, const char *s) { uint64_t n = strlen(s); wb_u64(b, n); wb_put(b, s, n); }
static void kv_u32(wbuf_t *b, const char *k, uint32_t v) { wb_str(b, k); wb_u32(b, 4); wb_u32(b, v); }
static void kv_f32(wbuf_t *b, const char *k, float v) { wb_str(b, k); wb_u32(b, 6); wb_f32(b, v); }
static void kv_str(wbuf_t *b, const char *k, const char *v) { wb_str(b, k); wb_u32(b, 8); wb_str(b, v); }

typedef struct {
    int fd;
    uint64_t data_off, seed;
    float scale_sigma, norm_sigma;
    int scale_mode;
    syn_tensor_t *t;
    int nt;
    /* work items: (tensor, chunk) flattened */
    uint64_t *item_tensor, *item_chunk;
    uint64_t n_items, next;
    int failed;
} job_t;

/* quantisation blocks of a matrix: 32 weights (Q4_0, Q8_0) or 256 (Q4_K) */
static uint64_t tensor_blocks(const syn_tensor_t *t) {
    return t->dims[0] * t->dims[1] / (is_k(t->type) ? 256 : 32);
}
static size_t block_bytes(int32_t type) {
    switch (type) {
    case T_F32: return 128;   /* matrices are generated in 32-weight pieces */
    case T_F16: return 64;
    case T_Q4_0: return 18;
    case T_Q4_1: return 20;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q8_0: return 34;
    case T_Q8_1: return 40;
    default: return k_bytes(type);
    }
}
/* blocks per work item: Q4_K super-blocks are 8 blocks of 32 weights */
static uint64_t chunk_blocks(int32_t type) { return is_k(type) ? CHUNK_BLOCKS / 8 : CHUNK_BLOCKS; }

static void gen_item(job_t *j, uint64_t it, uint8_t *buf) {
    const syn_tensor_t *t = &j->t[j->item_tensor[it]];
    uint64_t chunk = j->item_chunk[it];
    xo_t x;
    xo_seed(&x, j->seed, t->sid + 1, chunk);
    size_t n = 0;
    uint64_t off = 0;
    if (t->norm == 2) {
        uint64_t ne = t->dims[0];
        for (uint64_t i = 0; i < ne; i++) {
            float v = (float)(kBiasSigma * xo_normal(&x));
            if (t->type == T_F16) {
                uint16_t h = to_f16(v);
                memcpy(buf + 2 * i, &h, 2);
            } else {
                memcpy(buf + 4 * i, &v, 4);
            }
        }
        n = ne * (t->type == T_F16 ? 2 : 4);
    } else if (t->norm) {   /* norm weight vectors (F32) */
        uint64_t ne = t->dims[0] * (t->n_dims > 1 ? t->dims[1] : 1);
        float *f = (float *)buf;
        const double one = t->norm == 3 ? 0.0 : 1.0;
        for (uint64_t i = 0; i < ne; i++) f[i] = (float)(one + j->norm_sigma * xo_normal(&x));
        n = ne * 4;
    } else {
        const uint64_t cb = chunk_blocks(t->type);
        uint64_t nb = tensor_blocks(t), b0 = chunk * cb;
        uint64_t b1 = b0 + cb < nb ? b0 + cb : nb;
        size_t bb = block_bytes(t->type);
        /* mode 0: int8 codes spread 16 times as wide as nibbles, so both
         * types give weights of the same spread. mode 1: signed d with the
         * weights' standard deviation 1/sqrt(cols), the RMS of the codes
         * being sqrt(21.5) for Q4_0 (nibble - 8) and sqrt(127*128/3) for
         * uniform int8 in [-127, 127]. */
        double sigma;
        if (t->type == T_Q4_K) {
            /* weight d*sc*q - dmin*m with sc, m uniform 0..63 and q 0..15:
             * RMS sigma * sqrt(E[sc^2] (E[q^2] + 1)) = sigma * 323.5 */
            sigma = j->scale_mode == 1 ? 1.0 / (323.5 * sqrt((double)t->dims[0])) : j->scale_sigma / 64.0;
        } else if (is_k(t->type)) {
            /* the RMS of a weight per unit d (every field uniform): Q2_K
             * d*sc*q - dmin*m, sc, m < 16, q < 4: sqrt(77.5 * (3.5 + 1));
             * Q3_K d*(s - 32)*q, q in [-4, 3]: sqrt(341.5 * 5.5); Q5_K
             * d*sc*q - dmin*m, sc, m < 64, q < 32: sqrt(1333.5 * (325.5 + 1));
             * Q6_K d*sc*q, sc int8, q in [-32, 31]: sqrt(5461.5 * 341.5) */
            const double rms = t->type == T_Q2_K ? 18.675 : t->type == T_Q3_K ? 43.34
                             : t->type == T_Q5_K ? 659.8 : 1365.7;
            sigma = j->scale_mode == 1 ? 1.0 / (rms * sqrt((double)t->dims[0])) : j->scale_sigma * 4.6 / rms;
        } else if (t->type != T_Q4_0 && t->type != T_Q8_0) {
            /* the RMS of a weight per unit d: F16 / F32 weights are sigma *
             * N(0, 1); Q4_1 d*q + m with m = 8 d' (d' another N(0, 1) draw),
             * q < 16: sqrt(77.5 + 64); Q5_0 (q - 16) d: sqrt(85.5); Q5_1
             * d*q + m with m = 16 d', q < 32: sqrt(325.5 + 256); Q8_1 as
             * Q8_0. Mode 0 spreads the weights like Q4_0's. */
            const double rms = t->type == T_F32 || t->type == T_F16 ? 1.0
                             : t->type == T_Q4_1 ? sqrt(141.5) : t->type == T_Q5_0 ? sqrt(85.5)
                             : t->type == T_Q5_1 ? sqrt(581.5) : sqrt(127.0 * 128.0 / 3.0);
            sigma = j->scale_mode == 1 ? 1.0 / (rms * sqrt((double)t->dims[0])) : j->scale_sigma * 4.6 / rms;
        } else if (j->scale_mode == 1) {
            sigma = 1.0 / ((t->type == T_Q4_0 ? sqrt(21.5) : sqrt(127.0 * 128.0 / 3.0)) *
                           sqrt((double)t->dims[0]));
        } else {
            sigma = t->type == T_Q4_0 ? j->scale_sigma : j->scale_sigma / 16.0;
        }
        for (uint64_t b = b0; b < b1 && t->type == T_Q4_K; b++) {
            /* Q4_K super-block: d, dmin, 8 random 6-bit scales and mins in
             * the 12-byte K-quant packing, 128 bytes of random nibbles */
            uint8_t *p = buf + (b - b0) * bb;
            const double dv = sigma * xo_normal(&x), mv = sigma * xo_normal(&x);
            const uint16_t d = to_f16((float)(j->scale_mode == 1 ? dv : fabs(dv)));
            const uint16_t dm = to_f16((float)(j->scale_mode == 1 ? mv : fabs(mv)));
            memcpy(p, &d, 2);
            memcpy(p + 2, &dm, 2);
            uint8_t sc[8], mn[8];
            const uint64_t rs = xo_next(&x), rm = xo_next(&x);
            for (int i = 0; i < 8; i++) {
                sc[i] = (uint8_t)((rs >> (6 * i)) & 63);
                mn[i] = (uint8_t)((rm >> (6 * i)) & 63);
            }
            for (int i = 0; i < 4; i++) {
                p[4 + i] = (uint8_t)((sc[i] & 63) | ((sc[4 + i] >> 4) << 6));
                p[8 + i] = (uint8_t)((mn[i] & 63) | ((mn[4 + i] >> 4) << 6));
                p[12 + i] = (uint8_t)((sc[4 + i] & 15) | ((mn[4 + i] & 15) << 4));
            }
            for (int i = 0; i < 16; i++) {
                const uint64_t q = xo_next(&x);
                memcpy(p + 16 + 8 * i, &q, 8);
            }
        }
        for (uint64_t b = b0; b < b1 && is_k(t->type) && t->type != T_Q4_K; b++) {
            /* Q2_K, Q3_K, Q5_K, Q6_K: every code and scale byte random, then
             * d (and dmin) */
            uint8_t *p = buf + (b - b0) * bb;
            for (size_t i = 0; i + 8 <= bb; i += 8) {
                const uint64_t r = xo_next(&x);
                memcpy(p + i, &r, 8);
            }
            for (size_t i = bb / 8 * 8; i < bb; i++) p[i] = (uint8_t)xo_next(&x);
            const double dv = sigma * xo_normal(&x), mv = sigma * xo_normal(&x);
            const uint16_t d = to_f16((float)(j->scale_mode == 1 ? dv : fabs(dv)));
            const uint16_t dm = to_f16((float)(j->scale_mode == 1 ? mv : fabs(mv)));
            const size_t od = t->type == T_Q2_K ? 80 : t->type == T_Q3_K ? 108 : t->type == T_Q5_K ? 0 : 208;
            memcpy(p + od, &d, 2);
            if (t->type == T_Q2_K || t->type == T_Q5_K) memcpy(p + od + 2, &dm, 2);
        }
        for (uint64_t b = b0; b < b1 && (t->type == T_F32 || t->type == T_F16); b++) {
            uint8_t *p = buf + (b - b0) * bb;
            for (int i = 0; i < 32; i++) {
                const float v = (float)(sigma * xo_normal(&x));
                if (t->type == T_F32) {
                    memcpy(p + 4 * i, &v, 4);
                } else {
                    const uint16_t h = to_f16(v);
                    memcpy(p + 2 * i, &h, 2);
                }
            }
        }
        for (uint64_t b = b0; b < b1 && (t->type == T_Q4_1 || t->type == T_Q5_0 || t->type == T_Q5_1); b++) {
            /* d (and m) binary16, then random high bits (Q5) and nibbles */
            uint8_t *p = buf + (b - b0) * bb;
            const double dv = sigma * xo_normal(&x), mv = sigma * xo_normal(&x);
            const uint16_t d = to_f16((float)(j->scale_mode == 1 ? dv : fabs(dv)));
            const uint16_t m = to_f16((float)((t->type == T_Q5_1 ? -16.0 : -8.0) * mv));
            memcpy(p, &d, 2);
            size_t o = 2;
            if (t->type != T_Q5_0) {
                memcpy(p + 2, &m, 2);
                o = 4;
            }
            if (t->type != T_Q4_1) {
                const uint32_t qh = (uint32_t)(xo_next(&x) >> 32);
                memcpy(p + o, &qh, 4);
                o += 4;
            }
            uint64_t r0 = xo_next(&x), r1 = xo_next(&x);
            memcpy(p + o, &r0, 8);
            memcpy(p + o + 8, &r1, 8);
        }
        for (uint64_t b = b0; b < b1 && t->type == T_Q8_1; b++) {
            /* fp32 d, fp32 s = d * sum q (the field the reference ignores), 32 int8 */
            uint8_t *p = buf + (b - b0) * bb;
            const float d = (float)(sigma * xo_normal(&x));
            int sum = 0;
            for (int i = 0; i < 32; i++) {
                uint32_t r = (uint32_t)(xo_next(&x) >> 32);
                const int q = (int)(((uint64_t)r * 255u) >> 32) - 127;
                p[8 + i] = (uint8_t)(int8_t)q;
                sum += q;
            }
            const float sv = d * (float)sum;
            memcpy(p, &d, 4);
            memcpy(p + 4, &sv, 4);
        }
        for (uint64_t b = b0; b < b1 && (t->type == T_Q4_0 || t->type == T_Q8_0); b++) {
            uint8_t *p = buf + (b - b0) * bb;
            const double dv = sigma * xo_normal(&x);
            uint16_t d = to_f16((float)(j->scale_mode == 1 ? dv : fabs(dv)));
            memcpy(p, &d, 2);
            if (t->type == T_Q4_0) {
                uint64_t r0 = xo_next(&x), r1 = xo_next(&x);
                memcpy(p + 2, &r0, 8);
                memcpy(p + 10, &r1, 8);
            } else {
                for (int i = 0; i < 32; i++) {
                    uint32_t r = (uint32_t)(xo_next(&x) >> 32);
                    p[2 + i] = (uint8_t)(int8_t)((int)(((uint64_t)r * 255u) >> 32) - 127);
                }
            }
        }
        n = (b1 - b0) * bb;
        off = b0 * bb;
    }
    if (pwrite(j->fd, buf, n, (off_t)(j->data_off + t->offset + off)) != (ssize_t)n)
        __atomic_store_n(&j->failed, 1, __ATOMIC_RELAXED);
}

static void *worker(void *arg) {
    job_t *j = (job_t *)arg;
    uint8_t *buf = (uint8_t *)malloc((size_t)CHUNK_BLOCKS * MAX_BLOCK_BYTES + (1u << 20));
    uint64_t max_vec = 0;
    for (int i = 0; i < j->nt; i++)
        if (j->t[i].norm && j->t[i].bytes > max_vec) max_vec = j->t[i].bytes;
    uint8_t *vbuf = max_vec > (size_t)CHUNK_BLOCKS * MAX_BLOCK_BYTES ? (uint8_t *)malloc(max_vec) : NULL;
    if (!buf) { __atomic_store_n(&j->failed, 1, __ATOMIC_RELAXED); return NULL; }
    for (;;) {
        uint64_t it = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (it >= j->n_items || __atomic_load_n(&j->failed, __ATOMIC_RELAXED)) break;
        gen_item(j, it, (vbuf && j->t[j->item_tensor[it]].norm) ? vbuf : buf);
    }
    free(vbuf);
    free(buf);
    return NULL;
}

int32_t ss_synth_gguf_write(const char *path, const ss_synth_spec_t *s) {
    if (!path || !s) return -5;
    if (s->n_layers <= 0 || s->hidden <= 0 || s->n_heads <= 0 || s->n_kv_heads <= 0 ||
        s->head_dim <= 0 || s->ffn <= 0 || s->vocab <= 3 || s->hidden % 32 || s->ffn % 32 ||
        (s->n_heads * s->head_dim) % 32 || (s->n_kv_heads * s->head_dim) % 32 ||
        !matrix_type_ok(s->layer_type) || !matrix_type_ok(s->embd_type) ||
        (s->out_type != -1 && !matrix_type_ok(s->out_type)) ||
        /* K-quant rows are whole super-blocks of 256 */
        (is_k(s->layer_type) && (s->hidden % 256 || s->ffn % 256 || (s->n_heads * s->head_dim) % 256)) ||
        ((is_k(s->embd_type) || is_k(s->out_type)) && s->hidden % 256) ||
        s->arch < 0 || s->arch > 3 || s->attn_softcap < 0 || s->final_softcap < 0 || s->qkv_bias < 0 || s->qkv_bias > 2 || s->scale_mode < 0 ||
        s->scale_mode > 1)
        return -5;
    static const char *const kArch[4] = {"llama", "qwen2", "gemma", "gemma2"};
    const char *arch = kArch[s->arch];
    const int gemma = s->arch >= 2, post_norms = s->arch == 3;
    const int nk = gemma ? 3 : 1;   /* norm kind */
    const uint64_t align = s->alignment > 0 ? (uint64_t)s->alignment : 32;
    if (align & (align - 1)) return -5;
    const int L = s->n_layers;
    const uint64_t d = (uint64_t)s->hidden, q = (uint64_t)s->n_heads * s->head_dim,
                   kv = (uint64_t)s->n_kv_heads * s->head_dim, f = (uint64_t)s->ffn;
    int nt = 1 + 9 * L + 1 + (s->out_type >= 0 ? 1 : 0) + (s->qkv_bias ? 3 * L : 0) + (post_norms ? 2 * L : 0);
    syn_tensor_t *t = (syn_tensor_t *)calloc((size_t)nt, sizeof(syn_tensor_t));
    if (!t) return -3;
    int k = 0;
    uint64_t sid = 0;
#define ADD(nm, type_, cols, rows, isnorm)                                           \
    do {                                                                             \
        snprintf(t[k].name, sizeof(t[k].name), "%s", nm);                           \
        t[k].type = (type_);                                                         \
        t[k].dims[0] = (cols);                                                       \
        t[k].dims[1] = (rows);                                                       \
        t[k].n_dims = (isnorm) ? 1 : 2;                                              \
        t[k].norm = (isnorm);                                                        \
        t[k].sid = (isnorm) == 2 ? 0x100000u + (uint64_t)k : sid++;                 \
        t[k].bytes = (isnorm) == 2 ? (uint64_t)(cols) * ((type_) == T_F16 ? 2 : 4)   \
                     : (isnorm) ? (uint64_t)(cols) * 4                               \
                     : is_k(type_) ? (uint64_t)(cols) * (rows) / 256 * k_bytes(type_) \
                                : (uint64_t)(cols) * (rows) / 32 * block_bytes(type_);           \
        k++;                                                                         \
    } while (0)
    ADD("token_embd.weight", s->embd_type, d, (uint64_t)s->vocab, 0);
    char nm[64];
    for (int l = 0; l < L; l++) {
        snprintf(nm, sizeof(nm), "blk.%d.attn_norm.weight", l); ADD(nm, T_F32, d, 1, nk);
        /* fused: one tensor [Wq; Wk; Wv] (layer_scheduler.c:337-347) of the same parts */
        snprintf(nm, sizeof(nm), "blk.%d.%s.weight", l, s->fused_qkv ? "attn_qkv" : "attn_q");
        ADD(nm, s->layer_type, d, q, 0);
        t[k - 1].join_next = s->fused_qkv;
        snprintf(nm, sizeof(nm), "blk.%d.attn_k.weight", l); ADD(nm, s->layer_type, d, kv, 0);
        t[k - 1].join_next = s->fused_qkv;
        snprintf(nm, sizeof(nm), "blk.%d.attn_v.weight", l); ADD(nm, s->layer_type, d, kv, 0);
        if (s->qkv_bias) {   /* Qwen2 biases (layer_scheduler.c:367-402) */
            const int bt = s->qkv_bias == 2 ? T_F16 : T_F32;
            snprintf(nm, sizeof(nm), "blk.%d.attn_q.bias", l); ADD(nm, bt, q, 1, 2);
            snprintf(nm, sizeof(nm), "blk.%d.attn_k.bias", l); ADD(nm, bt, kv, 1, 2);
            snprintf(nm, sizeof(nm), "blk.%d.attn_v.bias", l); ADD(nm, bt, kv, 1, 2);
        }
        snprintf(nm, sizeof(nm), "blk.%d.attn_output.weight", l); ADD(nm, s->layer_type, q, d, 0);
        if (post_norms) {   /* Gemma 2 (layer_scheduler.c:309-310); own seed range, like biases */
            snprintf(nm, sizeof(nm), "blk.%d.post_attention_norm.weight", l); ADD(nm, T_F32, d, 1, 3);
            t[k - 1].sid = 0x200000u + (uint64_t)(k - 1);
            sid--;   /* the matrices keep the seed ids of the file without post norms */
        }
        snprintf(nm, sizeof(nm), "blk.%d.ffn_norm.weight", l); ADD(nm, T_F32, d, 1, nk);
        /* fused: ffn_up = [Wgate; Wup], 2 * ffn rows (layer_scheduler.c:518-524) */
        snprintf(nm, sizeof(nm), "blk.%d.%s.weight", l, s->fused_up ? "ffn_up" : "ffn_gate");
        ADD(nm, s->layer_type, d, f, 0);
        t[k - 1].join_next = s->fused_up;
        snprintf(nm, sizeof(nm), "blk.%d.ffn_up.weight", l); ADD(nm, s->layer_type, d, f, 0);
        snprintf(nm, sizeof(nm), "blk.%d.ffn_down.weight", l); ADD(nm, s->layer_type, f, d, 0);
        if (post_norms) {
            snprintf(nm, sizeof(nm), "blk.%d.post_ffw_norm.weight", l); ADD(nm, T_F32, d, 1, 3);
            t[k - 1].sid = 0x200000u + (uint64_t)(k - 1);
            sid--;   /* the matrices keep the seed ids of the file without post norms */
        }
    }
    ADD("output_norm.weight", T_F32, d, 1, nk);
    if (s->out_type >= 0) ADD("output.weight", s->out_type, d, (uint64_t)s->vocab, 0);
#undef ADD
    /* the parts of a fused tensor are contiguous; tensors start aligned */
    uint64_t off = 0;
    int n_phys = 0;
    for (int i = 0; i < nt; i++) {
        t[i].offset = off;
        off += t[i].bytes;
        if (!t[i].join_next) {
            off = (off + align - 1) & ~(align - 1);
            n_phys++;
        }
    }
    const uint64_t data_bytes = off;

    wbuf_t b = {0};
    const uint32_t n_kv = 12 + (s->with_vocab ? 3 : 0) + (s->attn_softcap > 0) + (s->final_softcap > 0);
    wb_u32(&b, 0x46554747u);
    wb_u32(&b, 3);
    wb_u64(&b, (uint64_t)n_phys);
    wb_u64(&b, n_kv);
    char key[96], gname[48];
#define AK(sfx) (snprintf(key, sizeof(key), "%s.%s", arch, sfx), key)
    snprintf(gname, sizeof(gname), "synthetic-%s", arch);
    kv_str(&b, "general.architecture", arch);
    kv_str(&b, "general.name", gname);
    kv_u32(&b, "general.alignment", (uint32_t)align);
    kv_u32(&b, AK("block_count"), (uint32_t)L);
    kv_u32(&b, AK("context_length"), (uint32_t)(s->context_length > 0 ? s->context_length : 2048));
    kv_u32(&b, AK("embedding_length"), (uint32_t)d);
    kv_u32(&b, AK("feed_forward_length"), (uint32_t)f);
    kv_u32(&b, AK("attention.head_count"), (uint32_t)s->n_heads);
    kv_u32(&b, AK("attention.head_count_kv"), (uint32_t)s->n_kv_heads);
    kv_u32(&b, AK("rope.dimension_count"), (uint32_t)s->head_dim);
    kv_f32(&b, AK("rope.freq_base"), s->rope_theta > 0 ? s->rope_theta : 10000.0f);
    kv_f32(&b, AK("attention.layer_norm_rms_epsilon"), s->rms_eps > 0 ? s->rms_eps : 1e-5f);
    if (s->attn_softcap > 0) kv_f32(&b, AK("attn_logit_softcapping"), s->attn_softcap);   /* gguf_loader.c:314-317 */
    if (s->final_softcap > 0) kv_f32(&b, AK("final_logit_softcapping"), s->final_softcap);
    if (s->with_vocab) {
        char vb[64];
        const int32_t nv = n_tokens(s);
        kv_str(&b, "tokenizer.ggml.model", "llama");
        wb_str(&b, "tokenizer.ggml.tokens");
        wb_u32(&b, 9);
        wb_u32(&b, 8);
        wb_u64(&b, (uint64_t)nv);
        for (int i = 0; i < nv; i++) wb_str(&b, ss_synth_vocab_string(nv, i, vb, sizeof(vb)));
        wb_str(&b, "tokenizer.ggml.scores");
        wb_u32(&b, 9);
        wb_u32(&b, 6);
        wb_u64(&b, (uint64_t)nv);
        for (int i = 0; i < nv; i++) wb_f32(&b, i < 259 ? 0.0f : -(float)(i - 259) * 0.01f);
    }
#undef AK
    for (int i = 0; i < nt;) {
        int e = i;   /* parts i..e form one GGUF tensor */
        uint64_t rows = t[i].dims[1];
        while (t[e].join_next) rows += t[++e].dims[1];
        wb_str(&b, t[i].name);
        wb_u32(&b, t[i].n_dims);
        wb_u64(&b, t[i].dims[0]);
        if (t[i].n_dims > 1) wb_u64(&b, rows);
        wb_u32(&b, (uint32_t)t[i].type);
        wb_u64(&b, t[i].offset);
        i = e + 1;
    }
    if (b.bad) { free(b.p); free(t); return -3; }
    const uint64_t data_off = (b.n + align - 1) & ~(align - 1);
    while (b.n < data_off) { uint8_t z = 0; wb_put(&b, &z, 1); }

    int fd = open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) { free(b.p); free(t); return -1; }
    int32_t rc = 0;
    if (ftruncate(fd, (off_t)(data_off + data_bytes)) != 0 ||
        pwrite(fd, b.p, b.n, 0) != (ssize_t)b.n)
        rc = -1;
    free(b.p);

    job_t j = {0};
    j.fd = fd;
    j.data_off = data_off;
    j.seed = s->seed;
    j.scale_sigma = s->scale_sigma > 0 ? s->scale_sigma : 0.02f;
    j.norm_sigma = s->norm_sigma > 0 ? s->norm_sigma : 0.01f;
    j.scale_mode = s->scale_mode;
    j.t = t;
    j.nt = nt;
    uint64_t items = 0;
    for (int i = 0; i < nt; i++)
        items += t[i].norm ? 1 : (tensor_blocks(&t[i]) + chunk_blocks(t[i].type) - 1) / chunk_blocks(t[i].type);
    j.item_tensor = (uint64_t *)malloc(items * 8);
    j.item_chunk = (uint64_t *)malloc(items * 8);
    if (!j.item_tensor || !j.item_chunk) rc = -3;
    uint64_t it = 0;
    for (int i = 0; rc == 0 && i < nt; i++) {
        uint64_t nc = t[i].norm ? 1 : (tensor_blocks(&t[i]) + chunk_blocks(t[i].type) - 1) / chunk_blocks(t[i].type);
        for (uint64_t c = 0; c < nc; c++) { j.item_tensor[it] = (uint64_t)i; j.item_chunk[it] = c; it++; }
    }
    j.n_items = items;
    if (rc == 0) {
        int nth = s->n_threads > 0 ? s->n_threads : (int)sysconf(_SC_NPROCESSORS_ONLN);
        if (nth < 1) nth = 1;
        if (nth > 64) nth = 64;
        pthread_t th[64];
        int started = 0;
        for (int i = 0; i < nth; i++)
            if (pthread_create(&th[started], NULL, worker, &j) == 0) started++;
        if (started == 0) worker(&j);
        for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
        if (j.failed) rc = -1;
    }
    free(j.item_tensor);
    free(j.item_chunk);
    free(t);
    if (close(fd) != 0) rc = -1;
    return rc;
}
