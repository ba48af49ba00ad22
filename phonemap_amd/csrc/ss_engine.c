/*
 * ss_engine.c - include/slipstream.h on the MI355X backend (host C).
 *
 * Follows the reference engine (SlipStream/src/core/engine.c) for load,
 * generate, embed, cancel and errors, and the reference scheduler's
 * initialisation rules (src/core/layer_scheduler.c:129-244) for the model
 * shape. The per-token work is one call into the HIP C-ABI
 * (include/ss_hip.h); no CPU compute backend is provided: SS_BACKEND_CPU and
 * SS_BACKEND_METAL fail with SS_ERROR_BACKEND, SS_BACKEND_AUTO means HIP.
 */
#define _GNU_SOURCE
#include "slipstream.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/sysinfo.h>
#include <sys/time.h>
#include <time.h>
#include <unistd.h>

#include "ss_gguf.h"
#include "ss_hip.h"
#include "ss_tokenizer.h"

struct ss_model {
    ss_gguf_file_t *gguf;
    ss_tok_t *tok;
    ss_hip_ctx_t *ctx;
    ss_hip_model_t *hm;
    ss_model_config_t config;
    ss_model_ext_t ext;
    int32_t cancelled;      /* written by ss_cancel from any thread */
    ss_progress_callback_t progress_cb;
    void *progress_user_data;
    int32_t vocab, n_ctx, n_embd;
    float *logits;
    int32_t neox_hd, neox_rope, kvdim;   /* NeoX models: the K order of neox_order (else 0) */
};

static __thread ss_error_t g_last_error = SS_OK;   /* engine.c:27 */

static double now_sec(void) {
    struct timeval tv;
    gettimeofday(&tv, NULL);
    return (double)tv.tv_sec + (double)tv.tv_usec / 1e6;
}

static ss_error_t set_err(ss_error_t e) {
    g_last_error = e;
    return e;
}

/* engine.c:31-52 */
ss_model_config_t ss_default_config(void) {
    ss_model_config_t c;
    memset(&c, 0, sizeof(c));
    c.backend = SS_BACKEND_AUTO;
    c.use_mmap = true;
    c.prefetch = true;
    return c;
}

ss_generate_params_t ss_default_params(void) {
    ss_generate_params_t p;
    memset(&p, 0, sizeof(p));
    p.max_tokens = 512;
    p.temperature = 0.7f;
    p.top_p = 0.9f;
    p.top_k = 40;
    p.repeat_penalty = 1.1f;
    return p;
}

ss_model_ext_t ss_default_ext(void) {
    ss_model_ext_t e;
    memset(&e, 0, sizeof(e));
    e.kv_type = SS_KV_F16;
    e.launch = SS_LAUNCH_GRAPH;
    return e;
}

static void fill_tensor(ss_hip_tensor_t *d, const ss_gguf_file_t *f, const ss_gguf_tensor_t *t) {
    memset(d, 0, sizeof(*d));
    if (!t) return;
    d->data = ss_gguf_tensor_data(f, t);
    d->type = t->type;
    d->cols = (int32_t)t->dims[0];
    d->rows = t->n_dims >= 2 ? (int32_t)t->dims[1] : 1;
}

/* bytes of one row of a GGUF tensor (gguf_loader.c:22-62) */
static size_t row_bytes(int32_t type, int32_t cols) {
    switch (type) {
    case SS_HIP_F32: return (size_t)cols * 4;
    case SS_HIP_F16: return (size_t)cols * 2;
    case SS_HIP_Q4_0: return (size_t)cols / 32 * 18;
    case SS_HIP_Q4_1: return (size_t)cols / 32 * 20;
    case SS_HIP_Q5_0: return (size_t)cols / 32 * 22;
    case SS_HIP_Q5_1: return (size_t)cols / 32 * 24;
    case SS_HIP_Q8_0: return (size_t)cols / 32 * 34;
    case SS_HIP_Q8_1: return (size_t)cols / 32 * 40;
    case SS_HIP_Q2_K: return (size_t)cols / 256 * 84;
    case SS_HIP_Q3_K: return (size_t)cols / 256 * 110;
    case SS_HIP_Q4_K: return (size_t)cols / 256 * 144;
    case SS_HIP_Q5_K: return (size_t)cols / 256 * 176;
    case SS_HIP_Q6_K: return (size_t)cols / 256 * 210;
    default: return 0;
    }
}

/* rows [r0, r0 + n) of a fused matrix as a tensor of their own */
static ss_hip_tensor_t row_view(const ss_hip_tensor_t *t, int32_t r0, int32_t n) {
    ss_hip_tensor_t v = *t;
    v.data = (const uint8_t *)t->data + (size_t)r0 * row_bytes(t->type, t->cols);
    v.rows = n;
    return v;
}

/* NeoX RoPE (tensor.c:223-248) rotates the pairs (i, i + rope_dim/2) of each
 * head. In the order where unit 2i of a head holds source unit i and unit
 * 2i+1 holds i + rope_dim/2 (units at or past rope_dim stay), those pairs are
 * adjacent, and the GPT-J branch (:249-274) rotates them with the same angle,
 * cos and sin, term for term. Attention uses q and K of a head only through
 * q.k, which is the same when both are in that order. So a NeoX model runs
 * as a GPT-J one whose Wq and Wk rows (and q/k biases, and injected K rows)
 * are put in this order once. Returns a malloc'd copy of n_units units of
 * `unit` bytes. */
static void *neox_order(const void *src, size_t unit, int32_t n_units, int32_t hd, int32_t rope_dim) {
    uint8_t *dst = (uint8_t *)malloc((size_t)n_units * unit);
    if (!dst) return NULL;
    const int32_t half = rope_dim / 2;
    for (int32_t u = 0; u < n_units; u++) {
        const int32_t h = u / hd, p = u % hd;
        const int32_t from = p < 2 * half ? (p & 1 ? p / 2 + half : p / 2) : p;
        memcpy(dst + (size_t)u * unit, (const uint8_t *)src + ((size_t)h * hd + from) * unit, unit);
    }
    return dst;
}

ss_model_t *ss_model_load(const char *path, const ss_model_config_t *config) {
    return ss_model_load_ex(path, config, NULL);
}

ss_model_t *ss_model_load_ex(const char *path, const ss_model_config_t *config,
                             const ss_model_ext_t *ext) {
    if (!path) { set_err(SS_ERROR_INVALID_PARAMS); return NULL; }
    ss_model_t *m = (ss_model_t *)calloc(1, sizeof(ss_model_t));
    if (!m) { set_err(SS_ERROR_OUT_OF_MEMORY); return NULL; }
    m->config = config ? *config : ss_default_config();
    m->ext = ext ? *ext : ss_default_ext();

    if (m->config.backend == SS_BACKEND_CPU || m->config.backend == SS_BACKEND_METAL) {
        fprintf(stderr, "SlipStream: backend %d is not provided by this build (use SS_BACKEND_HIP)\n",
                (int)m->config.backend);
        free(m);
        set_err(SS_ERROR_BACKEND);
        return NULL;
    }
    m->gguf = ss_gguf_open(path);
    if (!m->gguf) {
        fprintf(stderr, "SlipStream: cannot load %s: %s\n", path, ss_gguf_error());
        free(m);
        set_err(SS_ERROR_INVALID_MODEL);
        return NULL;
    }
    ss_gguf_file_t *g = m->gguf;
    m->tok = ss_tok_create(g->vocab, g->vocab_scores, g->vocab ? g->vocab_size : 0, g->merges,
                           g->n_merges, g->arch);

    const int gemma = strstr(g->arch, "gemma") != NULL;   /* layer_scheduler.c:152-155 */
    /* layer_scheduler.c:144-149 */
    const int neox = strstr(g->arch, "qwen") || strstr(g->arch, "falcon") || strstr(g->arch, "phi") ||
                     strstr(g->arch, "deepseek");

    /* shape, layer_scheduler.c:157-197 */
    int32_t d = (int32_t)g->hidden_size, H = (int32_t)g->num_heads;
    int32_t KVH = g->num_kv_heads ? (int32_t)g->num_kv_heads : H;
    if (d <= 0 || H <= 0 || g->num_layers == 0) {
        ss_model_free(m);
        set_err(SS_ERROR_INVALID_MODEL);
        return NULL;
    }
    int32_t hd = 0;
    if (g->head_dim > 0) {
        hd = (int32_t)g->head_dim;
    } else {
        const ss_gguf_tensor_t *wq0 = ss_gguf_find(g, "blk.0.attn_q.weight");
        if (wq0 && wq0->n_dims >= 2) hd = (int32_t)(wq0->dims[1] / (uint64_t)H);
    }
    if (hd == 0) hd = d / H;
    int32_t rope_dim = g->rope_dim > 0 ? (int32_t)g->rope_dim : hd;
    int32_t vocab = (int32_t)g->vocab_size;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const ss_gguf_tensor_t *t = &g->tensors[i];
        if ((strcmp(t->name, "output.weight") == 0 || strcmp(t->name, "token_embd.weight") == 0) &&
            t->n_dims == 2 && (int32_t)t->dims[1] < vocab)
            vocab = (int32_t)t->dims[1];
    }
    /* context: engine.c:99-106 caps at 8192; the scheduler's 512 cap
     * (layer_scheduler.c:202) is not applied. ext.max_context overrides both. */
    uint32_t ctx_size = m->config.context_size > 0 ? m->config.context_size : g->context_length;
    if (ctx_size == 0 || ctx_size > 8192) ctx_size = 8192;
    if (m->ext.max_context > 0) ctx_size = m->ext.max_context;

    const uint32_t L = g->num_layers;
    const int32_t qdim = H * hd, kvdim = KVH * hd, ffn = (int32_t)g->intermediate_size;
    if (neox && (rope_dim % 2 || rope_dim > hd)) {
        fprintf(stderr, "SlipStream: NeoX RoPE needs an even rope dimension <= head_dim\n");
        ss_model_free(m);
        set_err(SS_ERROR_INVALID_MODEL);
        return NULL;
    }
    ss_hip_tensor_t *lt = (ss_hip_tensor_t *)calloc((size_t)L * SS_HIP_LAYER_TENSORS, sizeof(ss_hip_tensor_t));
    ss_hip_tensor_t *bias = (ss_hip_tensor_t *)calloc((size_t)L * 3, sizeof(ss_hip_tensor_t));
    ss_hip_tensor_t *post = (ss_hip_tensor_t *)calloc((size_t)L * 2, sizeof(ss_hip_tensor_t));
    void **owned = (void **)calloc((size_t)L * 4 + 1, sizeof(void *));   /* NeoX-ordered copies */
    int n_owned = 0, any_bias = 0, any_post = 0;
    ss_error_t err = SS_OK;
    if (!lt || !bias || !post || !owned) err = SS_ERROR_OUT_OF_MEMORY;
    static const char *sfx[SS_HIP_LAYER_TENSORS] = {
        "attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
        "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    static const char *bsfx[3] = {"attn_q.bias", "attn_k.bias", "attn_v.bias"};
    for (uint32_t l = 0; l < L && err == SS_OK; l++) {
        ss_hip_tensor_t *t = lt + (size_t)l * SS_HIP_LAYER_TENSORS;
        /* Gemma 2 post norms, wherever they exist (layer_scheduler.c:309-310) */
        fill_tensor(&post[l * 2], g, ss_gguf_find_in_layer(g, l, "post_attention_norm.weight"));
        fill_tensor(&post[l * 2 + 1], g, ss_gguf_find_in_layer(g, l, "post_ffw_norm.weight"));
        if (post[l * 2].data || post[l * 2 + 1].data) any_post = 1;
        const ss_gguf_tensor_t *wqkv = ss_gguf_find_in_layer(g, l, "attn_qkv.weight");
        const ss_gguf_tensor_t *wgate = ss_gguf_find_in_layer(g, l, "ffn_gate.weight");
        for (int k = 0; k < SS_HIP_LAYER_TENSORS && err == SS_OK; k++) {
            if ((wqkv && (k == SS_HIP_WQ || k == SS_HIP_WK || k == SS_HIP_WV)) || (!wgate && k == SS_HIP_W_GATE))
                continue;
            const ss_gguf_tensor_t *tt = ss_gguf_find_in_layer(g, l, sfx[k]);
            if (!tt) {
                fprintf(stderr, "SlipStream: blk.%u.%s missing\n", l, sfx[k]);
                err = SS_ERROR_INVALID_MODEL;
                break;
            }
            fill_tensor(&t[k], g, tt);
        }
        if (err != SS_OK) break;
        if (wqkv) {   /* layer_scheduler.c:337-347: [Wq; Wk; Wv] in one tensor */
            ss_hip_tensor_t f;
            fill_tensor(&f, g, wqkv);
            if (f.rows != qdim + 2 * kvdim || !row_bytes(f.type, f.cols)) {
                fprintf(stderr, "SlipStream: blk.%u.attn_qkv.weight has %d rows, %d expected\n", l, f.rows,
                        qdim + 2 * kvdim);
                err = SS_ERROR_INVALID_MODEL;
                break;
            }
            t[SS_HIP_WQ] = row_view(&f, 0, qdim);
            t[SS_HIP_WK] = row_view(&f, qdim, kvdim);
            t[SS_HIP_WV] = row_view(&f, qdim + kvdim, kvdim);
        }
        if (!wgate) {  /* :518-524: ffn_up = [gate; up], 2 * ffn rows */
            const ss_hip_tensor_t f = t[SS_HIP_W_UP];
            if (f.rows != 2 * ffn || !row_bytes(f.type, f.cols)) {
                fprintf(stderr, "SlipStream: blk.%u has no ffn_gate and ffn_up is not [gate; up]\n", l);
                err = SS_ERROR_INVALID_MODEL;
                break;
            }
            t[SS_HIP_W_GATE] = row_view(&f, 0, ffn);
            t[SS_HIP_W_UP] = row_view(&f, ffn, ffn);
        }
        /* :367-402 (attn_qkv.bias is looked up there but never applied) */
        for (int k = 0; k < 3; k++) {
            fill_tensor(&bias[l * 3 + k], g, ss_gguf_find_in_layer(g, l, bsfx[k]));
            if (bias[l * 3 + k].data) any_bias = 1;
        }
        if (neox) {
            for (int k = 0; k < 2 && err == SS_OK; k++) {   /* Wq, Wk and their biases */
                ss_hip_tensor_t *w = &t[SS_HIP_WQ + k], *b = &bias[l * 3 + k];
                const size_t rb = row_bytes(w->type, w->cols);
                void *c = rb && w->rows % hd == 0 ? neox_order(w->data, rb, w->rows, hd, rope_dim) : NULL;
                if (!c) { err = rb && w->rows % hd == 0 ? SS_ERROR_OUT_OF_MEMORY : SS_ERROR_INVALID_MODEL; break; }
                owned[n_owned++] = c;
                w->data = c;
                if (b->data) {
                    const int32_t n = b->rows * b->cols;
                    const size_t eb = row_bytes(b->type, 1);
                    void *cb = eb && n % hd == 0 ? neox_order(b->data, eb, n, hd, rope_dim) : NULL;
                    if (!cb) { err = eb && n % hd == 0 ? SS_ERROR_OUT_OF_MEMORY : SS_ERROR_INVALID_MODEL; break; }
                    owned[n_owned++] = cb;
                    b->data = cb;
                }
            }
        }
    }
    if (err != SS_OK) {
        for (int i = 0; i < n_owned; i++) free(owned[i]);
        free(owned);
        free(post);
        free(bias);
        free(lt);
        ss_model_free(m);
        set_err(err);
        return NULL;
    }
    ss_hip_model_desc_t desc;
    memset(&desc, 0, sizeof(desc));
    desc.n_layers = (int32_t)L;
    desc.hidden = d;
    desc.n_heads = H;
    desc.n_kv_heads = KVH;
    desc.head_dim = hd;
    desc.rope_dim = rope_dim;
    desc.ffn = (int32_t)g->intermediate_size;
    desc.vocab = vocab;
    desc.max_seq = (int32_t)ctx_size;
    desc.rms_eps = g->rms_norm_eps;
    desc.rope_theta = g->rope_theta;
    desc.kv_type = m->ext.kv_type == SS_KV_INT8 ? SS_HIP_KV_INT8 : SS_HIP_KV_F16;
    desc.launch = (int32_t)m->ext.launch;
    desc.streaming = m->ext.streaming ? 1 : 0;
    fill_tensor(&desc.token_embd, g, ss_gguf_find(g, "token_embd.weight"));
    fill_tensor(&desc.output_norm, g, ss_gguf_find(g, "output_norm.weight"));
    fill_tensor(&desc.output, g, ss_gguf_find(g, "output.weight"));
    desc.layers = lt;
    desc.qkv_bias = any_bias ? bias : NULL;
    desc.gemma = gemma;
    desc.attn_softcap = g->attn_logit_softcapping;   /* gguf_loader.c:314-317 */
    desc.final_softcap = g->final_logit_softcapping;
    desc.post_norms = any_post ? post : NULL;

    m->ctx = ss_hip_init(m->ext.device);
    if (!m->ctx) {
        fprintf(stderr, "SlipStream: HIP backend unavailable: %s\n", ss_hip_last_error());
        for (int i = 0; i < n_owned; i++) free(owned[i]);
        free(owned);
        free(post);
        free(bias);
        free(lt);
        ss_model_free(m);
        set_err(SS_ERROR_BACKEND);
        return NULL;
    }
    m->hm = ss_hip_model_create(m->ctx, &desc);
    for (int i = 0; i < n_owned; i++) free(owned[i]);
    free(owned);
    free(post);
    free(bias);
    free(lt);
    if (!m->hm) {
        fprintf(stderr, "SlipStream: model upload failed: %s\n", ss_hip_last_error());
        ss_model_free(m);
        set_err(SS_ERROR_BACKEND);
        return NULL;
    }
    ss_hip_set_cancel_flag(m->hm, &m->cancelled);
    if (neox) {
        m->neox_hd = hd;
        m->neox_rope = rope_dim;
    }
    m->kvdim = kvdim;
    m->vocab = vocab;
    m->n_ctx = (int32_t)ctx_size;
    m->n_embd = d;
    m->logits = (float *)malloc(sizeof(float) * (size_t)vocab);
    if (!m->logits) { ss_model_free(m); set_err(SS_ERROR_OUT_OF_MEMORY); return NULL; }

    char dev[160] = "";
    ss_hip_device_name(m->ext.device, dev, sizeof(dev));
    fprintf(stderr, "SlipStream: Model loaded - %s\n", path);                 /* engine.c:126-133 */
    fprintf(stderr, "  Architecture: %s\n  Layers: %u\n  Hidden size: %d\n  Heads: %d (KV: %d)\n"
                    "  Vocab: %d\n  Context: %u\n  Backend: HIP on %s, %.2f GB on device\n",
            g->arch, L, d, H, KVH, vocab, ctx_size, dev, (double)ss_hip_model_bytes(m->hm) / 1e9);
    set_err(SS_OK);
    return m;
}

ss_error_t ss_model_get_info(const ss_model_t *m, ss_model_info_t *info) {   /* engine.c:141-170 */
    if (!m || !info) return SS_ERROR_INVALID_PARAMS;
    memset(info, 0, sizeof(*info));
    const ss_gguf_file_t *g = m->gguf;
    strncpy(info->architecture, g->arch, sizeof(info->architecture) - 1);
    const char *chat = "unknown";
    if (strstr(g->arch, "gemma")) chat = "gemma";
    else if (strstr(g->arch, "phi")) chat = "phi3";
    else if (strstr(g->arch, "qwen")) chat = "chatml";
    else if (strstr(g->arch, "llama")) chat = "llama3";
    strncpy(info->chat_format, chat, sizeof(info->chat_format) - 1);
    info->num_layers = g->num_layers;
    info->hidden_size = g->hidden_size;
    info->num_heads = g->num_heads;
    info->num_kv_heads = g->num_kv_heads;
    info->vocab_size = g->vocab_size;
    info->context_length = g->context_length;
    info->intermediate_size = g->intermediate_size;
    info->file_size = g->file_size;
    if (g->layers && g->num_layers > 0) info->per_layer_size = g->layers[0].total_size;
    return SS_OK;
}

void ss_model_free(ss_model_t *m) {
    if (!m) return;
    if (m->hm) ss_hip_model_free(m->hm);
    if (m->ctx) ss_hip_free(m->ctx);
    ss_tok_free(m->tok);
    ss_gguf_close(m->gguf);
    free(m->logits);
    free(m);
}

void ss_set_throttle(ss_model_t *m, uint32_t delay_us) { (void)m; (void)delay_us; }  /* engine.c:364-368 */

uint64_t ss_get_memory_usage(void) {
    FILE *f = fopen("/proc/self/statm", "r");
    unsigned long pages = 0, rss = 0;
    if (f) {
        if (fscanf(f, "%lu %lu", &pages, &rss) != 2) rss = 0;
        fclose(f);
    }
    return (uint64_t)rss * (uint64_t)sysconf(_SC_PAGESIZE);
}

const char *ss_get_last_profile_path(void) { return NULL; }   /* engine.c:355-357 */
void ss_set_profile_output_dir(const char *dir) { (void)dir; }

/* ---- host sampling, tensor.c:318-451 ---- */
int32_t ss_argmax(const float *x, int32_t size) {
    int32_t idx = 0;
    float mv = x[0];
    for (int32_t i = 1; i < size; i++)
        if (x[i] > mv) { mv = x[i]; idx = i; }
    return idx;
}

static uint64_t xorshift64(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

typedef struct { int32_t id; float prob; } tokprob_t;

static int cmp_prob(const void *a, const void *b) {
    float pa = ((const tokprob_t *)a)->prob, pb = ((const tokprob_t *)b)->prob;
    if (isnan(pa)) pa = 0.0f;
    if (isnan(pb)) pb = 0.0f;
    return pa > pb ? -1 : pa < pb ? 1 : 0;
}

static void softmax_inplace(float *x, int32_t n) {   /* tensor.c:154-173 */
    float mv = -FLT_MAX;
    for (int32_t i = 0; i < n; i++) if (x[i] > mv) mv = x[i];
    float sum = 0.0f;
    for (int32_t i = 0; i < n; i++) { x[i] = expf(x[i] - mv); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int32_t i = 0; i < n; i++) x[i] *= inv;
}

int32_t ss_sample(const float *logits, int32_t V, float temperature, float top_p, int32_t top_k,
                  uint64_t *rng) {
    if (temperature <= 0.0f) return ss_argmax(logits, V);
    float *probs = (float *)malloc(sizeof(float) * (size_t)V);
    if (!probs) return ss_argmax(logits, V);
    for (int32_t i = 0; i < V; i++) probs[i] = isnan(logits[i]) ? -FLT_MAX : logits[i] / temperature;
    softmax_inplace(probs, V);
    tokprob_t *sorted = (tokprob_t *)malloc(sizeof(tokprob_t) * (size_t)V);
    if (sorted) {
        for (int32_t i = 0; i < V; i++) { sorted[i].id = i; sorted[i].prob = isnan(probs[i]) ? 0.0f : probs[i]; }
        qsort(sorted, (size_t)V, sizeof(tokprob_t), cmp_prob);
    }
    if (top_k > 0 && top_k < V && sorted) {
        float th = sorted[top_k - 1].prob;
        for (int32_t i = 0; i < V; i++) if (probs[i] < th) probs[i] = 0.0f;
    }
    if (top_p > 0.0f && top_p < 1.0f && sorted) {
        float cum = 0.0f, cutoff = 0.0f;
        for (int32_t i = 0; i < V; i++) {
            float p = probs[sorted[i].id];
            if (p > 0.0f) cum += p;
            if (cum >= top_p) { cutoff = p; break; }
        }
        for (int32_t i = 0; i < V; i++) if (probs[i] < cutoff) probs[i] = 0.0f;
    }
    free(sorted);
    float sum = 0.0f;
    for (int32_t i = 0; i < V; i++) sum += probs[i];
    if (sum > 0.0f) { float inv = 1.0f / sum; for (int32_t i = 0; i < V; i++) probs[i] *= inv; }
    float r = (float)(xorshift64(rng) >> 11) / (float)(1ULL << 53);
    float cdf = 0.0f;
    int32_t out = V - 1;
    for (int32_t i = 0; i < V; i++) {
        cdf += probs[i];
        if (r < cdf) { out = i; break; }
    }
    free(probs);
    return out;
}

/* ---- eval-token API ---- */
int32_t ss_tokenize(const ss_model_t *m, const char *text, int32_t *out, int32_t max_tokens) {
    if (!m || !m->tok) return 0;
    return ss_tok_encode(m->tok, text, out, max_tokens);
}
const char *ss_token_text(const ss_model_t *m, int32_t id) { return m ? ss_tok_decode(m->tok, id) : ""; }
int32_t ss_bos_id(const ss_model_t *m) { return ss_tok_bos(m ? m->tok : NULL); }
int32_t ss_eos_id(const ss_model_t *m) { return ss_tok_eos(m ? m->tok : NULL); }
int32_t ss_n_vocab(const ss_model_t *m) { return m ? m->vocab : 0; }
int32_t ss_n_ctx(const ss_model_t *m) { return m ? m->n_ctx : 0; }
int32_t ss_n_embd(const ss_model_t *m) { return m ? m->n_embd : 0; }
void *ss_model_hip(ss_model_t *m) { return m ? (void *)m->hm : NULL; }

static ss_error_t map_rc(int32_t rc) {
    if (rc == 0) return set_err(SS_OK);
    if (rc == SS_ERROR_INVALID_PARAMS || rc == SS_ERROR_CANCELLED || rc == SS_ERROR_OUT_OF_MEMORY)
        return set_err((ss_error_t)rc);
    return set_err(SS_ERROR_BACKEND);
}

ss_error_t ss_reset(ss_model_t *m) {
    if (!m) return set_err(SS_ERROR_INVALID_PARAMS);
    __atomic_store_n(&m->cancelled, 0, __ATOMIC_SEQ_CST);
    return map_rc(ss_hip_kv_reset(m->hm));
}

ss_error_t ss_eval_token(ss_model_t *m, int32_t token, int32_t pos, float *logits, int32_t *argmax) {
    if (!m) return set_err(SS_ERROR_INVALID_PARAMS);
    return map_rc(ss_hip_eval_token(m->hm, token, pos, logits, argmax));
}

ss_error_t ss_eval_prompt(ss_model_t *m, const int32_t *tokens, int32_t n, int32_t start,
                          float *logits, int32_t *argmax) {
    if (!m) return set_err(SS_ERROR_INVALID_PARAMS);
    return map_rc(ss_hip_eval_prompt(m->hm, tokens, n, start, logits, argmax));
}

ss_error_t ss_decode_greedy(ss_model_t *m, int32_t n_steps, int32_t *out) {
    if (!m) return set_err(SS_ERROR_INVALID_PARAMS);
    return map_rc(ss_hip_decode_greedy(m->hm, n_steps, out));
}

ss_error_t ss_kv_write(ss_model_t *m, int32_t layer, int32_t pos0, int32_t n_pos, const uint16_t *k,
                       const uint16_t *v) {
    if (!m) return set_err(SS_ERROR_INVALID_PARAMS);
    if (!m->neox_hd || !k || n_pos <= 0) return map_rc(ss_hip_kv_write(m->hm, layer, pos0, n_pos, k, v));
    /* K rows in the NeoX model's head order (see neox_order) */
    uint16_t *kk = (uint16_t *)neox_order(k, 2, n_pos * m->kvdim, m->neox_hd, m->neox_rope);
    if (!kk) return set_err(SS_ERROR_OUT_OF_MEMORY);
    ss_error_t rc = map_rc(ss_hip_kv_write(m->hm, layer, pos0, n_pos, kk, v));
    free(kk);
    return rc;
}

/* ---- generate, engine.c:174-306 ---- */
ss_error_t ss_generate(ss_model_t *m, const char *prompt, const ss_generate_params_t *params,
                       ss_token_callback_t cb, void *ud) {
    if (!m || !prompt) return set_err(SS_ERROR_INVALID_PARAMS);
    ss_generate_params_t p = params ? *params : ss_default_params();
    __atomic_store_n(&m->cancelled, 0, __ATOMIC_SEQ_CST);
    if (ss_hip_kv_reset(m->hm) != 0) return set_err(SS_ERROR_BACKEND);
    int32_t toks[4096];
    int32_t n = ss_tok_encode(m->tok, prompt, toks, 4096);
    if (n <= 0) return set_err(SS_ERROR_TOKENIZER);
    if (n >= m->n_ctx) return set_err(SS_ERROR_INVALID_PARAMS);
    uint64_t rng = p.seed > 0 ? (uint64_t)p.seed : (uint64_t)time(NULL);
    const int greedy = p.temperature <= 0.0f;
    if (m->progress_cb) m->progress_cb(0, (uint32_t)n, "prefill", m->progress_user_data);
    double t0 = now_sec();
    int32_t next = 0;
    /* the logits stay in HBM: greedy tokens come from the device argmax,
     * sampled ones from ss_hip_sample over the same logits */
    int32_t rc = ss_hip_eval_prompt(m->hm, toks, n, 0, NULL, &next);
    double t1 = now_sec();
    if (m->progress_cb) m->progress_cb((uint32_t)n, (uint32_t)n, "prefill", m->progress_user_data);
    if (rc != 0) return map_rc(rc) == SS_ERROR_CANCELLED ? SS_ERROR_CANCELLED : set_err(SS_ERROR_BACKEND);

    const int32_t eos = ss_tok_eos(m->tok);
    int32_t generated = 0, pos = n;
    char outbuf[8192];
    int32_t outlen = 0;
    outbuf[0] = 0;
    double t2 = now_sec();
    for (uint32_t t = 0; t < p.max_tokens; t++) {
        if (__atomic_load_n(&m->cancelled, __ATOMIC_SEQ_CST)) return set_err(SS_ERROR_CANCELLED);
        /* sample over the logits the model produces (the clamped vocab) */
        int32_t id = next;
        if (!greedy && (rc = ss_hip_sample(m->hm, p.temperature, p.top_p, (int32_t)p.top_k, &rng, &id)) != 0) break;
        if (id == eos) break;
        const char *text = ss_tok_decode(m->tok, id);
        if (text && (!strcmp(text, "<|im_end|>") || !strcmp(text, "<|eot_id|>") || !strcmp(text, "<|end|>") ||
                     !strcmp(text, "<|endoftext|>") || !strcmp(text, "<|user|>") || !strcmp(text, "</s>") ||
                     !strcmp(text, "<end_of_turn>") || !strcmp(text, "<eos>")))
            break;
        if (p.stop_sequence && text) {
            size_t tl = strlen(text);
            if (outlen + (int32_t)tl < (int32_t)sizeof(outbuf)) {
                memcpy(outbuf + outlen, text, tl);
                outlen += (int32_t)tl;
                outbuf[outlen] = 0;
                if (strstr(outbuf, p.stop_sequence)) break;
            }
        }
        if (cb && !cb(text, (uint32_t)id, ud)) break;
        if (pos >= m->n_ctx) break;
        rc = ss_hip_eval_token(m->hm, id, pos, NULL, &next);
        if (rc != 0) break;
        pos++;
        generated++;
    }
    double t3 = now_sec();
    fprintf(stderr, "\n=== SlipStream Diagnostic Recap ===\n");                 /* engine.c:295-302 */
    if (t1 - t0 > 0.0) fprintf(stderr, "Prefill: %d tokens in %.2f seconds (%.2f tok/s)\n", n, t1 - t0, n / (t1 - t0));
    if (generated > 0 && t3 - t2 > 0.0)
        fprintf(stderr, "Decode : %d tokens in %.2f seconds (%.2f tok/s)\n", generated, t3 - t2, generated / (t3 - t2));
    fprintf(stderr, "===================================\n\n");
    if (rc == SS_ERROR_CANCELLED) return set_err(SS_ERROR_CANCELLED);
    /* A failed step (e.g. a persistent launch abandoned at its wait bound)
     * ends the loop with the text so far delivered; the reference's loop
     * (engine.c:283-290) stops the same way but reports success, which here
     * would hide a truncated output. */
    if (rc != 0) return set_err(SS_ERROR_BACKEND);
    return set_err(SS_OK);
}

/* ---- embed, engine.c:310-352 + layer_scheduler.c:805-915 ---- */
ss_error_t ss_embed(ss_model_t *m, const char *prompt, float **out, uint32_t *out_dim) {
    if (!m || !prompt || !out || !out_dim) return set_err(SS_ERROR_INVALID_PARAMS);
    __atomic_store_n(&m->cancelled, 0, __ATOMIC_SEQ_CST);
    if (ss_hip_kv_reset(m->hm) != 0) return set_err(SS_ERROR_BACKEND);
    int32_t toks[4096];
    int32_t n = ss_tok_encode(m->tok, prompt, toks, 4096);
    if (n <= 0) return set_err(SS_ERROR_TOKENIZER);
    if (n > m->n_ctx) return set_err(SS_ERROR_INVALID_PARAMS);
    if (m->progress_cb) m->progress_cb(0, (uint32_t)n, "embedding", m->progress_user_data);
    const int32_t d = m->n_embd;
    float *e = (float *)malloc(sizeof(float) * (size_t)d);
    if (!e) return set_err(SS_ERROR_OUT_OF_MEMORY);
    int32_t rc = ss_hip_embed(m->hm, toks, n, e);   /* layer_scheduler.c:805-911 */
    if (rc != 0) {
        free(e);
        return map_rc(rc) == SS_ERROR_CANCELLED ? SS_ERROR_CANCELLED : set_err(SS_ERROR_BACKEND);
    }
    *out = e;
    *out_dim = (uint32_t)d;
    return set_err(SS_OK);
}

void ss_cancel(ss_model_t *m) {   /* engine.c:372-379, with an atomic flag */
    if (m) __atomic_store_n(&m->cancelled, 1, __ATOMIC_SEQ_CST);
}

void ss_set_progress_callback(ss_model_t *m, ss_progress_callback_t cb, void *ud) {
    if (!m) return;
    m->progress_cb = cb;
    m->progress_user_data = ud;
}

ss_error_t ss_last_error(void) { return g_last_error; }

const char *ss_error_string(ss_error_t e) {   /* engine.c:401-417 */
    switch (e) {
    case SS_OK: return "OK";
    case SS_ERROR_FILE_NOT_FOUND: return "File not found";
    case SS_ERROR_INVALID_MODEL: return "Invalid GGUF model file";
    case SS_ERROR_OUT_OF_MEMORY: return "Out of memory";
    case SS_ERROR_MMAP_FAILED: return "Memory mapping failed";
    case SS_ERROR_INVALID_PARAMS: return "Invalid parameters";
    case SS_ERROR_CANCELLED: return "Operation cancelled";
    case SS_ERROR_BACKEND: return "Compute backend error";
    case SS_ERROR_TOKENIZER: return "Tokenizer error";
    default: return "Unknown error";
    }
}

const char *ss_version(void) { return SS_VERSION_STRING; }

/* Device bytes the HIP backend needs: every tensor resident (the packed
 * layout has the same size as the GGUF blocks) plus the fp16 KV cache and
 * working buffers. */
ss_error_t ss_estimate_memory(const char *path, uint32_t context_size, uint64_t *peak) {
    if (!path || !peak) return SS_ERROR_INVALID_PARAMS;
    ss_gguf_file_t *g = ss_gguf_open(path);
    if (!g) return SS_ERROR_INVALID_MODEL;
    uint64_t w = 0;
    for (uint64_t i = 0; i < g->n_tensors; i++) w += g->tensors[i].size_bytes;
    uint32_t ctx = context_size > 0 ? context_size : g->context_length;
    uint32_t kvh = g->num_kv_heads ? g->num_kv_heads : g->num_heads;
    uint32_t hd = g->head_dim ? g->head_dim : (g->num_heads ? g->hidden_size / g->num_heads : 0);
    uint64_t kv = 2ull * g->num_layers * ctx * kvh * hd * 2;
    uint64_t bufs = (uint64_t)g->hidden_size * 4 * 4 + (uint64_t)g->intermediate_size * 4 +
                    (uint64_t)g->vocab_size * 4 + (uint64_t)ctx * hd * 4;
    *peak = w + kv + bufs;
    ss_gguf_close(g);
    return SS_OK;
}

ss_error_t ss_get_device_info(ss_device_info_t *info) {
    if (!info) return SS_ERROR_INVALID_PARAMS;
    memset(info, 0, sizeof(*info));
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    info->cpu_core_count = n > 0 ? (uint32_t)n : 0;
    info->perf_core_count = info->cpu_core_count;
    struct sysinfo si;
    if (sysinfo(&si) == 0) {
        info->total_memory = (uint64_t)si.totalram * si.mem_unit;
        info->available_memory = (uint64_t)si.freeram * si.mem_unit;
    }
    if (ss_hip_device_count() > 0) {
        int32_t cus = 0;
        uint64_t hbm = 0;
        if (ss_hip_device_info(0, &cus, &hbm) == 0) info->gpu_core_count = (uint32_t)cus;
        char name[160];
        if (ss_hip_device_name(0, name, sizeof(name)) == 0) strncpy(info->chip_name, name, sizeof(info->chip_name) - 1);
    }
    snprintf(info->device_model, sizeof(info->device_model), "linux");
    return SS_OK;
}

/* process CPU time over wall time since the previous call, in percent */
double ss_get_cpu_usage(void) {
    static double last_wall = 0.0, last_cpu = 0.0;
    struct timespec ts;
    clock_gettime(CLOCK_PROCESS_CPUTIME_ID, &ts);
    double cpu = (double)ts.tv_sec + ts.tv_nsec / 1e9, wall = now_sec();
    double r = 0.0;
    if (last_wall > 0.0 && wall > last_wall) r = 100.0 * (cpu - last_cpu) / (wall - last_wall);
    last_wall = wall;
    last_cpu = cpu;
    return r;
}
