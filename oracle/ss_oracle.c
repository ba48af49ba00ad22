/*
 * ss_oracle.c - CPU restatement of SlipStream's per-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP product and the CPU
 * baseline timed beside it. The product never links, loads or calls this.
 *
 * Citations are file:line in the reference repository, relative to its
 * SlipStream/ directory. Deliberate differences from the reference:
 *  - The context cap of 512 positions (src/core/layer_scheduler.c:202) and the
 *    stack arrays scores[512]/tmp_kv[256] (:430-431) are lifted; max_seq is
 *    the caller's.
 *  - Apple vDSP_dotpr (quantize.c:488, layer_scheduler.c:442), whose
 *    summation order is unspecified, is restated as orc_dot: eight strided
 *    fp32 partial sums folded pairwise. cblas_saxpy (:466) is y = w*x + y
 *    element by element. No FMA contraction (built with -ffp-contract=off).
 *  - GCD dispatch_apply (quantize.c:475, layer_scheduler.c:424) is restated
 *    as a pthread pool with the same chunking: rows in ceil(rows/ncpu)
 *    chunks, attention one task per query head.
 *  - Besides the reference's int8 KV cache there is an fp16 KV mode: K and V
 *    are rounded to binary16 when appended and widened when read, inside the
 *    fp32 KV structure of layer_scheduler.c.orig:289-342.
 *  - The llama block and the branches the reference takes by tensor name or
 *    by architecture are restated: fused attn_qkv and fused ffn_up
 *    (layer_scheduler.c:337-347,518-524), q/k/v biases (:367-402), NeoX RoPE
 *    pairs for qwen/falcon/phi/deepseek (:144-149), and for "gemma" files the
 *    (1 + w) RMSNorm (tensor.c:133-152), the sqrt(d) embedding scale
 *    (:597-602), GeGLU (:529-531, tensor.c:181-190) and the 1/sqrt(d) logit
 *    scale (:667-672); post-attention / post-FFN norms wherever those
 *    tensors exist (:474-481,553-560) and the attention / final logit
 *    softcaps wherever the GGUF keys are set (:446-448,674-676,
 *    tensor.c:194-200), as the reference applies them, for any architecture.
 *
 * Parity unpinned: the summation order of Apple vDSP_dotpr / cblas_saxpy
 * (system frameworks, no version pin; orc_dot's order is checked against the
 * reference's own portable ss_neon_dot instead). End-to-end logits have no
 * reference fixture: the model functions (forward, prefill, embed) are
 * pinned instead by an independent fp64 restatement of layer_scheduler.c
 * (tests/ref_model.py, tests/test_cpu_model_pin.py), which three mis-wired
 * variants of it miss by more than twenty times the bar.
 */
#define _GNU_SOURCE
#include "ss_oracle.h"

#include <fcntl.h>
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* Element ops                                                              */
/* ------------------------------------------------------------------------ */

/* quantize.c:20-56 - exact half to float, with subnormals, inf and NaN. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 1;
            while (!(m & 0x400)) { m <<= 1; e--; }
            m &= 0x3FF;
            bits = sign | ((e + 127 - 15) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE binary16 with round-to-nearest-even (what a hardware f32->f16
 * conversion does); used by the fp16 KV mode. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 -> inf */
    uint32_t ef = ax >> 23;
    if (ef >= 113) {                               /* normal half */
        uint32_t mant = ax & 0x7FFFFFu;
        uint32_t h = ((ef - 112) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ef < 102) return (uint16_t)sign;           /* below half of the smallest subnormal */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126 - ef;                     /* 14..24 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* quantize.c:60-72 (Q4_0), :139-149 (Q8_0), :389-442 (dispatch; F32 copy,
 * F16 widen). Blocks: Q4_0 = fp16 d + 16 bytes of nibbles (18 B),
 * Q8_0 = fp16 d + 32 int8 (34 B) (quantize.h:14-17,43-46). */
void orc_dequantize(const void *src, float *dst, int32_t n, int32_t type) {
    const uint8_t *p = (const uint8_t *)src;
    switch (type) {
    case ORC_F32:
        memcpy(dst, src, (size_t)n * sizeof(float));
        break;
    case ORC_F16:
        for (int32_t i = 0; i < n; i++) {
            uint16_t h;
            memcpy(&h, p + 2 * (size_t)i, 2);
            dst[i] = orc_f16_to_f32(h);
        }
        break;
    case ORC_Q4_0:
        for (int32_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = p + (size_t)b * 18;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            float scale = orc_f16_to_f32(dh);
            for (int32_t i = 0; i < 16; i++) {
                uint8_t byte = blk[2 + i];
                dst[b * 32 + i] = scale * ((int32_t)(byte & 0xF) - 8);
                dst[b * 32 + i + 16] = scale * ((int32_t)(byte >> 4) - 8);
            }
        }
        break;
    case ORC_Q8_0:
        for (int32_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = p + (size_t)b * 34;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            float scale = orc_f16_to_f32(dh);
            for (int32_t i = 0; i < 32; i++)
                dst[b * 32 + i] = scale * (float)(int8_t)blk[2 + i];
        }
        break;
    case ORC_Q4_1:
        /* quantize.c:76-91: fp16 d, fp16 m, 16 bytes of nibbles (20 B,
         * quantize.h:20-24); weight j = d * nibble + m, low nibbles first. */
        for (int32_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = p + (size_t)b * 20;
            uint16_t dh, mh;
            memcpy(&dh, blk, 2);
            memcpy(&mh, blk + 2, 2);
            float d = orc_f16_to_f32(dh), m = orc_f16_to_f32(mh);
            for (int32_t i = 0; i < 16; i++) {
                uint8_t byte = blk[4 + i];
                dst[b * 32 + i] = d * (float)(byte & 0xF) + m;
                dst[b * 32 + i + 16] = d * (float)(byte >> 4) + m;
            }
        }
        break;
    case ORC_Q5_0:
    case ORC_Q5_1: {
        /* quantize.c:93-137: 5-bit codes, the low 4 bits in nibbles (weight
         * i low, i + 16 high) and bit 4 of weight i in bit i of the 32-bit
         * little-endian qh. Q5_0 (22 B: d, qh, qs): (q - 16) * d. Q5_1
         * (24 B: d, m, qh, qs): q * d + m (quantize.h:26-41). */
        const int one = type == ORC_Q5_1;
        const size_t bytes = one ? 24 : 22;
        for (int32_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = p + (size_t)b * bytes;
            uint16_t dh, mh = 0;
            uint32_t qh;
            memcpy(&dh, blk, 2);
            if (one) memcpy(&mh, blk + 2, 2);
            memcpy(&qh, blk + (one ? 4 : 2), 4);
            const uint8_t *qs = blk + (one ? 8 : 6);
            float d = orc_f16_to_f32(dh), m = orc_f16_to_f32(mh);
            for (int32_t i = 0; i < 16; i++) {
                int32_t q0 = (qs[i] & 0xF) | (int32_t)(((qh >> i) & 1u) << 4);
                int32_t q1 = (qs[i] >> 4) | (int32_t)(((qh >> (i + 16)) & 1u) << 4);
                if (one) {
                    dst[b * 32 + i] = (float)q0 * d + m;
                    dst[b * 32 + i + 16] = (float)q1 * d + m;
                } else {
                    dst[b * 32 + i] = (float)(q0 - 16) * d;
                    dst[b * 32 + i + 16] = (float)(q1 - 16) * d;
                }
            }
        }
        break;
    }
    case ORC_Q8_1:
        /* quantize.c:153-163: fp32 d, fp32 s (unused), 32 int8 (40 B,
         * quantize.h:49-53); weight = d * q. */
        for (int32_t b = 0; b < n / 32; b++) {
            const uint8_t *blk = p + (size_t)b * 40;
            float d;
            memcpy(&d, blk, 4);
            for (int32_t i = 0; i < 32; i++) dst[b * 32 + i] = d * (float)(int8_t)blk[8 + i];
        }
        break;
    case ORC_Q4_K:
        /* quantize.c:265-310: super-blocks of 256 weights, 144 bytes: d and
         * dmin (binary16), 12 bytes of packed 6-bit sub-block scales and
         * mins, 128 bytes of nibbles. Sub-blocks 2j and 2j + 1 take the low
         * and the high nibbles of bytes 32j .. 32j + 31; weight = d*sc * q -
         * dmin*m. The scale and min of sub-block k (get_scale_min_k4,
         * :267-275): k < 4 from the low 6 bits of bytes k and k + 4;
         * otherwise the low and high nibbles of byte k + 4 with the top two
         * bits of bytes k - 4 and k on top. */
        for (int32_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = p + (size_t)b * 144;
            uint16_t dh, mh;
            memcpy(&dh, blk, 2);
            memcpy(&mh, blk + 2, 2);
            const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
            const uint8_t *sc = blk + 4, *q = blk + 16;
            for (int32_t k = 0; k < 8; k++) {
                uint8_t s6, m6;
                if (k < 4) {
                    s6 = sc[k] & 63;
                    m6 = sc[k + 4] & 63;
                } else {
                    s6 = (uint8_t)((sc[k + 4] & 0xF) | ((sc[k - 4] >> 6) << 4));
                    m6 = (uint8_t)((sc[k + 4] >> 4) | ((sc[k] >> 6) << 4));
                }
                const float d1 = d * (float)s6, m1 = dmin * (float)m6;
                const uint8_t *qk = q + 32 * (k / 2);
                for (int32_t l = 0; l < 32; l++) {
                    const int32_t nib = k % 2 ? qk[l] >> 4 : qk[l] & 0xF;
                    dst[b * 256 + k * 32 + l] = d1 * (float)nib - m1;
                }
            }
        }
        break;
    case ORC_Q2_K:
        /* quantize.c:180-215: 84 bytes: 16 scale bytes (low nibble scale,
         * high nibble min, one per 16 weights), 64 bytes of 2-bit codes, d,
         * dmin. Weights 128h + 32j + l (l < 32, h < 2, j < 4) take bits
         * 2j..2j+1 of byte 32h + l; weight = d*sc * q - dmin*m with the
         * scale byte 8h + 2j + l/16. */
        for (int32_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = p + (size_t)b * 84;
            uint16_t dh, mh;
            memcpy(&dh, blk + 80, 2);
            memcpy(&mh, blk + 82, 2);
            const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
            for (int32_t h = 0; h < 2; h++)
                for (int32_t j = 0; j < 4; j++)
                    for (int32_t l = 0; l < 32; l++) {
                        const uint8_t sc = blk[8 * h + 2 * j + l / 16];
                        const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                        const int32_t q = (blk[16 + 32 * h + l] >> (2 * j)) & 3;
                        dst[b * 256 + 128 * h + 32 * j + l] = dl * (float)q - ml;
                    }
        }
        break;
    case ORC_Q3_K: {
        /* quantize.c:219-263: 110 bytes: 32 bytes of high bits, 64 bytes of
         * 2-bit codes, 12 bytes of 6-bit scales, d. Weights 128h + 32j + l
         * take bits 2j..2j+1 of byte 32h + l, minus 4 unless bit 4h + j of
         * hmask byte l is set; weight = d * (scale - 32) * q with scale
         * 8h + 2j + l/16. The 16 scales: low nibbles of bytes 0..7 (scales
         * 0..7) and high nibbles of bytes 0..7 (8..15), each with two more
         * bits from byte 8 + i%4, at bit 2*(i/4). */
        for (int32_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = p + (size_t)b * 110;
            uint16_t dh;
            memcpy(&dh, blk + 108, 2);
            const float d = orc_f16_to_f32(dh);
            const uint8_t *hm = blk, *qs = blk + 32, *sb = blk + 96;
            int32_t scl[16];
            for (int32_t i = 0; i < 16; i++) {
                const int32_t low = i < 8 ? sb[i] & 0xF : sb[i - 8] >> 4;
                const int32_t high = (sb[8 + i % 4] >> (2 * (i / 4))) & 3;
                scl[i] = low | (high << 4);
            }
            for (int32_t h = 0; h < 2; h++)
                for (int32_t j = 0; j < 4; j++)
                    for (int32_t l = 0; l < 32; l++) {
                        const float dl = d * (float)(scl[8 * h + 2 * j + l / 16] - 32);
                        const int32_t q = ((qs[32 * h + l] >> (2 * j)) & 3) - ((hm[l] >> (4 * h + j)) & 1 ? 0 : 4);
                        dst[b * 256 + 128 * h + 32 * j + l] = dl * (float)q;
                    }
        }
        break;
    }
    case ORC_Q5_K:
        /* quantize.c:312-346: 176 bytes: d, dmin, 12 bytes of 6-bit scales
         * and mins (as Q4_K), 32 bytes of fifth bits, 128 bytes of nibbles.
         * Sub-block k (32 weights) takes the low (k even) or high nibbles of
         * bytes 32(k/2)..+31 plus 16 times bit k of qh byte l; weight =
         * d*sc * q - dmin*m. */
        for (int32_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = p + (size_t)b * 176;
            uint16_t dh, mh;
            memcpy(&dh, blk, 2);
            memcpy(&mh, blk + 2, 2);
            const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
            const uint8_t *sc = blk + 4, *qh = blk + 16, *qs = blk + 48;
            for (int32_t k = 0; k < 8; k++) {
                uint8_t s6, m6;
                if (k < 4) {
                    s6 = sc[k] & 63;
                    m6 = sc[k + 4] & 63;
                } else {
                    s6 = (uint8_t)((sc[k + 4] & 0xF) | ((sc[k - 4] >> 6) << 4));
                    m6 = (uint8_t)((sc[k + 4] >> 4) | ((sc[k] >> 6) << 4));
                }
                const float d1 = d * (float)s6, m1 = dmin * (float)m6;
                for (int32_t l = 0; l < 32; l++) {
                    const uint8_t byte = qs[32 * (k / 2) + l];
                    const int32_t q = (k % 2 ? byte >> 4 : byte & 0xF) + ((qh[l] >> k) & 1 ? 16 : 0);
                    dst[b * 256 + k * 32 + l] = d1 * (float)q - m1;
                }
            }
        }
        break;
    case ORC_Q6_K:
        /* quantize.c:350-383: 210 bytes: 128 bytes of low nibbles, 64 bytes
         * of high 2-bit pairs, 16 int8 scales (one per 16 weights), d.
         * Weight 128h + 32c + l (c < 4, l < 32): low nibble of byte
         * 64h + l (c = 0), 64h + 32 + l (1), high nibbles of the same (2,
         * 3); high bits 2c..2c+1 of qh byte 32h + l; minus 32; weight =
         * d * scale[8h + 2c + l/16] * q. */
        for (int32_t b = 0; b < n / 256; b++) {
            const uint8_t *blk = p + (size_t)b * 210;
            uint16_t dh;
            memcpy(&dh, blk + 208, 2);
            const float d = orc_f16_to_f32(dh);
            const uint8_t *ql = blk, *qh = blk + 128;
            const int8_t *sc = (const int8_t *)(blk + 192);
            for (int32_t h = 0; h < 2; h++)
                for (int32_t c = 0; c < 4; c++)
                    for (int32_t l = 0; l < 32; l++) {
                        const uint8_t lb = ql[64 * h + 32 * (c & 1) + l];
                        const int32_t lo = c < 2 ? lb & 0xF : lb >> 4;
                        const int32_t q = (lo | (((qh[32 * h + l] >> (2 * c)) & 3) << 4)) - 32;
                        dst[b * 256 + 128 * h + 32 * c + l] = d * (float)sc[8 * h + 2 * c + l / 16] * (float)q;
                    }
        }
        break;
    default:
        memset(dst, 0, (size_t)n * sizeof(float));
        break;
    }
}

static size_t orc_row_bytes(int32_t cols, int32_t type) {
    switch (type) {
    case ORC_F32: return (size_t)cols * 4;
    case ORC_F16: return (size_t)cols * 2;
    case ORC_Q4_0: return (size_t)(cols / 32) * 18;
    case ORC_Q8_0: return (size_t)(cols / 32) * 34;
    case ORC_Q4_1: return (size_t)(cols / 32) * 20;
    case ORC_Q5_0: return (size_t)(cols / 32) * 22;
    case ORC_Q5_1: return (size_t)(cols / 32) * 24;
    case ORC_Q8_1: return (size_t)(cols / 32) * 40;
    case ORC_Q2_K: return (size_t)(cols / 256) * 84;
    case ORC_Q3_K: return (size_t)(cols / 256) * 110;
    case ORC_Q4_K: return (size_t)(cols / 256) * 144;
    case ORC_Q5_K: return (size_t)(cols / 256) * 176;
    case ORC_Q6_K: return (size_t)(cols / 256) * 210;
    default: return 0;
    }
}

/* Stand-in for vDSP_dotpr: eight strided partial sums, folded pairwise. */
float orc_dot(const float *a, const float *b, int32_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int32_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) acc[j] += a[i + j] * b[i + j];
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* cpu_neon.c:109-115 (scalar branch of ss_neon_rmsnorm, reached through
 * tensor.c:114-118 for F32 weights). */
void orc_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int32_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* tensor.c:154-173 */
void orc_softmax(float *x, int32_t n) {
    float max_val = -FLT_MAX;
    for (int32_t i = 0; i < n; i++)
        if (x[i] > max_val) max_val = x[i];
    float sum = 0.0f;
    for (int32_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int32_t i = 0; i < n; i++) x[i] *= inv;
}

/* layer_scheduler.c:540-547: up * (g / (1 + exp(-g))) */
float orc_silu_mul(float g, float u) { return u * (g / (1.0f + expf(-g))); }

/* cpu_neon.c:153-158 (scalar branch of ss_neon_gemma_rmsnorm, reached through
 * tensor.c:133-137 for F32 weights): the weight is applied as (w + 1). */
void orc_gemma_rmsnorm(float *out, const float *x, const float *w, int32_t n, float eps) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int32_t i = 0; i < n; i++) out[i] = x[i] * scale * (w[i] + 1.0f);
}

/* tensor.c:181-190: tanh-form GELU, in place */
float orc_gelu(float v) {
    const float sqrt_2_over_pi = 0.7978845608028654f;
    float cube = v * v * v;
    float inner = sqrt_2_over_pi * (v + 0.044715f * cube);
    return 0.5f * v * (1.0f + tanhf(inner));
}

/* tensor.c:194-200 */
void orc_softcap(float *x, int32_t n, float cap) {
    if (cap <= 0.0f) return;
    float inv_cap = 1.0f / cap;
    for (int32_t i = 0; i < n; i++) x[i] = cap * tanhf(x[i] * inv_cap);
}

/* tensor.c:220-275 */
void orc_rope(float *q, float *k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
              int32_t rope_dim, int32_t pos, float theta, int32_t is_neox) {
    if (is_neox) {
        int32_t half_d = rope_dim / 2;
        for (int32_t i = 0; i < half_d; i++) {
            float freq = 1.0f / powf(theta, (float)(i * 2) / (float)rope_dim);
            float angle = (float)pos * freq;
            float c = cosf(angle), s = sinf(angle);
            for (int32_t h = 0; h < n_heads; h++) {
                float *qh = q + h * head_dim;
                float a = qh[i], b = qh[i + half_d];
                qh[i] = a * c - b * s;
                qh[i + half_d] = a * s + b * c;
            }
            for (int32_t h = 0; h < n_kv_heads; h++) {
                float *kh = k + h * head_dim;
                float a = kh[i], b = kh[i + half_d];
                kh[i] = a * c - b * s;
                kh[i + half_d] = a * s + b * c;
            }
        }
        return;
    }
    for (int32_t i = 0; i < rope_dim; i += 2) {
        float freq = 1.0f / powf(theta, (float)i / (float)rope_dim);
        float angle = (float)pos * freq;
        float c = cosf(angle), s = sinf(angle);
        for (int32_t h = 0; h < n_heads; h++) {
            float *qh = q + h * head_dim;
            float a = qh[i], b = qh[i + 1];
            qh[i] = a * c - b * s;
            qh[i + 1] = a * s + b * c;
        }
        for (int32_t h = 0; h < n_kv_heads; h++) {
            float *kh = k + h * head_dim;
            float a = kh[i], b = kh[i + 1];
            kh[i] = a * c - b * s;
            kh[i + 1] = a * s + b * c;
        }
    }
}

/* The (cos, sin) pairs tensor.c:250-254 computes, tabulated per position:
 * cs[(pos * rope_dim/2 + i/2) * 2 + {0,1}]. */
void orc_rope_table(float *cs, int32_t rope_dim, int32_t n_pos, float theta) {
    for (int32_t p = 0; p < n_pos; p++)
        for (int32_t i = 0; i < rope_dim; i += 2) {
            float freq = 1.0f / powf(theta, (float)i / (float)rope_dim);
            float angle = (float)p * freq;
            size_t o = ((size_t)p * (rope_dim / 2) + i / 2) * 2;
            cs[o] = cosf(angle);
            cs[o + 1] = sinf(angle);
        }
}

/* tensor.c:318-328: index of the first strict maximum. */
int32_t orc_argmax(const float *x, int32_t n) {
    int32_t idx = 0;
    float mv = x[0];
    for (int32_t i = 1; i < n; i++)
        if (x[i] > mv) { mv = x[i]; idx = i; }
    return idx;
}

/* tensor.c:330-343: xorshift64 and the 53-bit uniform draw. */
static uint64_t orc_xorshift64(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

typedef struct { int32_t id; float prob; } orc_tp_t;

/* tensor.c:352-361: descending, NaN ranked as 0. */
static int orc_tp_cmp(const void *a, const void *b) {
    float pa = ((const orc_tp_t *)a)->prob, pb = ((const orc_tp_t *)b)->prob;
    if (isnan(pa)) pa = 0.0f;
    if (isnan(pb)) pb = 0.0f;
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    return 0;
}

/* tensor.c:363-451 (ss_sample). probs_out (optional, n floats) receives the
 * final distribution the draw walks, r_out (optional) the uniform draw. */
int32_t orc_sample(const float *logits, int32_t n, float temperature, float top_p, int32_t top_k,
                   uint64_t *rng, float *probs_out, float *r_out) {
    if (temperature <= 0.0f) return orc_argmax(logits, n);
    float *p = (float *)malloc(sizeof(float) * (size_t)n);
    orc_tp_t *srt = (orc_tp_t *)malloc(sizeof(orc_tp_t) * (size_t)n);
    if (!p || !srt) { free(p); free(srt); return orc_argmax(logits, n); }
    for (int32_t i = 0; i < n; i++) p[i] = isnan(logits[i]) ? -FLT_MAX : logits[i] / temperature;
    orc_softmax(p, n);
    for (int32_t i = 0; i < n; i++) { srt[i].id = i; srt[i].prob = isnan(p[i]) ? 0.0f : p[i]; }
    qsort(srt, (size_t)n, sizeof(orc_tp_t), orc_tp_cmp);
    if (top_k > 0 && top_k < n) {                         /* :391-396 */
        const float th = srt[top_k - 1].prob;
        for (int32_t i = 0; i < n; i++) if (p[i] < th) p[i] = 0.0f;
    }
    if (top_p > 0.0f && top_p < 1.0f) {                   /* :399-417 */
        float cum = 0.0f, cutoff = 0.0f;
        for (int32_t i = 0; i < n; i++) {
            const float v = p[srt[i].id];
            if (v > 0.0f) cum += v;
            if (cum >= top_p) { cutoff = v; break; }
        }
        for (int32_t i = 0; i < n; i++) if (p[i] < cutoff) p[i] = 0.0f;
    }
    free(srt);
    float sum = 0.0f;                                     /* :423-429 */
    for (int32_t i = 0; i < n; i++) sum += p[i];
    if (sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (int32_t i = 0; i < n; i++) p[i] *= inv;
    }
    const float r = (float)(orc_xorshift64(rng) >> 11) / (float)(1ULL << 53);   /* :431-442 */
    float cdf = 0.0f;
    int32_t out = n - 1;
    for (int32_t i = 0; i < n; i++) {
        cdf += p[i];
        if (r < cdf) { out = i; break; }
    }
    if (probs_out) memcpy(probs_out, p, sizeof(float) * (size_t)n);
    if (r_out) *r_out = r;
    free(p);
    return out;
}

/* layer_scheduler.c:101-118 */
void orc_kv_int8_encode(const float *src, int8_t *q, float *scale, int32_t n) {
    float max_val = 0.0f;
    for (int32_t i = 0; i < n; i++) {
        float v = fabsf(src[i]);
        if (v > max_val) max_val = v;
    }
    float s = max_val / 127.0f;
    *scale = s;
    float inv = s > 0.0f ? 1.0f / s : 0.0f;
    for (int32_t i = 0; i < n; i++) q[i] = (int8_t)roundf(src[i] * inv);
}

/* One head of layer_scheduler.c:421-467 over fp32 keys/values whose
 * consecutive positions are kv_stride floats apart. */
void orc_attention_head(float *out, const float *q, const float *keys, const float *values,
                        int32_t head_dim, int32_t seq_len, int32_t kv_stride) {
    float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc((size_t)seq_len * sizeof(float));
    for (int32_t t = 0; t < seq_len; t++)
        scores[t] = orc_dot(q, keys + (size_t)t * kv_stride, head_dim) * scale;
    orc_softmax(scores, seq_len);
    memset(out, 0, (size_t)head_dim * sizeof(float));
    for (int32_t t = 0; t < seq_len; t++) {
        const float *vt = values + (size_t)t * kv_stride;
        for (int32_t d = 0; d < head_dim; d++) out[d] = scores[t] * vt[d] + out[d];
    }
    free(scores);
}

/* ------------------------------------------------------------------------ */
/* Thread pool (stand-in for GCD dispatch_apply)                             */
/* ------------------------------------------------------------------------ */

#define ORC_MAX_THREADS 128

typedef void (*orc_task_fn)(void *arg, int32_t idx);

static struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_go, cv_idle;
    pthread_t th[ORC_MAX_THREADS];
    int nworkers;    /* threads besides the caller */
    int nthreads;    /* total, caller included */
    unsigned gen;
    int active;
    int stop;
    orc_task_fn fn;
    void *arg;
    int32_t count;
    int32_t next;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};

static void pool_drain(orc_task_fn fn, void *arg, int32_t count) {
    for (;;) {
        int32_t i = __atomic_fetch_add(&g_pool.next, 1, __ATOMIC_RELAXED);
        if (i >= count) break;
        fn(arg, i);
    }
}

/* arg: the job generation current when the worker was created, so a job
 * posted before the worker first takes the mutex is still seen as new. */
static void *pool_worker(void *arg) {
    unsigned seen = (unsigned)(uintptr_t)arg;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.gen == seen && !g_pool.stop) pthread_cond_wait(&g_pool.cv_go, &g_pool.mu);
        if (g_pool.stop) break;
        seen = g_pool.gen;
        orc_task_fn fn = g_pool.fn;
        void *arg = g_pool.arg;
        int32_t count = g_pool.count;
        pthread_mutex_unlock(&g_pool.mu);
        pool_drain(fn, arg, count);
        pthread_mutex_lock(&g_pool.mu);
        if (--g_pool.active == 0) pthread_cond_signal(&g_pool.cv_idle);
    }
    pthread_mutex_unlock(&g_pool.mu);
    return NULL;
}

static void pool_stop(void) {
    pthread_mutex_lock(&g_pool.mu);
    g_pool.stop = 1;
    pthread_cond_broadcast(&g_pool.cv_go);
    pthread_mutex_unlock(&g_pool.mu);
    for (int i = 0; i < g_pool.nworkers; i++) pthread_join(g_pool.th[i], NULL);
    g_pool.nworkers = 0;
    g_pool.stop = 0;
}

void orc_set_threads(int32_t n) {
    if (n <= 0) {
        const char *env = getenv("OMP_NUM_THREADS");
        n = env ? atoi(env) : 0;
        if (n <= 0) {   /* the CPUs this process may run on */
            cpu_set_t set;
            n = sched_getaffinity(0, sizeof set, &set) == 0 ? CPU_COUNT(&set)
                                                           : (int32_t)sysconf(_SC_NPROCESSORS_ONLN);
        }
    }
    if (n < 1) n = 1;
    if (n > ORC_MAX_THREADS) n = ORC_MAX_THREADS;
    if (g_pool.nthreads == n) return;
    if (g_pool.nworkers) pool_stop();
    pthread_mutex_lock(&g_pool.mu);
    g_pool.nthreads = n;
    int started = 0;
    for (int i = 0; i < n - 1; i++)
        if (pthread_create(&g_pool.th[started], NULL, pool_worker,
                           (void *)(uintptr_t)g_pool.gen) == 0)
            started++;
    g_pool.nworkers = started;
    g_pool.nthreads = started + 1;
    pthread_mutex_unlock(&g_pool.mu);
}

int32_t orc_get_threads(void) {
    if (g_pool.nthreads == 0) orc_set_threads(0);
    return g_pool.nthreads;
}

static void pool_run(orc_task_fn fn, void *arg, int32_t count) {
    if (g_pool.nthreads == 0) orc_set_threads(0);
    if (count <= 0) return;
    if (g_pool.nworkers == 0 || count == 1) {
        for (int32_t i = 0; i < count; i++) fn(arg, i);
        return;
    }
    pthread_mutex_lock(&g_pool.mu);
    g_pool.fn = fn;
    g_pool.arg = arg;
    g_pool.count = count;
    g_pool.next = 0;
    g_pool.active = g_pool.nworkers;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.cv_go);
    pthread_mutex_unlock(&g_pool.mu);
    pool_drain(fn, arg, count);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.active > 0) pthread_cond_wait(&g_pool.cv_idle, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

/* ------------------------------------------------------------------------ */
/* Matvec: quantize.c:446-494                                               */
/* ------------------------------------------------------------------------ */

typedef struct {
    float *out;
    const uint8_t *w;
    const float *x;
    float *tmp;
    int32_t rows, cols, type, rows_per_chunk;
    size_t row_bytes;
} mv_job_t;

static void mv_chunk(void *arg, int32_t chunk) {
    mv_job_t *j = (mv_job_t *)arg;
    int32_t r0 = chunk * j->rows_per_chunk;
    int32_t r1 = r0 + j->rows_per_chunk;
    if (r1 > j->rows) r1 = j->rows;
    float *tmp = j->tmp + (size_t)chunk * j->cols;
    for (int32_t r = r0; r < r1; r++) {
        orc_dequantize(j->w + (size_t)r * j->row_bytes, tmp, j->cols, j->type);
        j->out[r] = orc_dot(tmp, j->x, j->cols);
    }
}

void orc_dequant_matvec(float *out, const void *w, const float *x, int32_t rows, int32_t cols,
                        int32_t type) {
    size_t rb = orc_row_bytes(cols, type);
    if (rb == 0 || rows <= 0) return;
    int32_t ncpu = orc_get_threads();
    if (ncpu > rows) ncpu = rows;
    mv_job_t j = {out, (const uint8_t *)w, x, NULL, rows, cols, type, (rows + ncpu - 1) / ncpu, rb};
    j.tmp = (float *)malloc((size_t)ncpu * cols * sizeof(float));
    if (!j.tmp) return;
    pool_run(mv_chunk, &j, ncpu);
    free(j.tmp);
}

/* Four dot products sharing a: each in exactly orc_dot's order (eight
 * strided partial sums folded pairwise, then the tail), so every result is
 * bit-identical to orc_dot(a, bk, n). */
/* eight fp32 lanes: lane j is orc_dot's partial sum j */
typedef float orc_v8 __attribute__((vector_size(32)));

static inline orc_v8 ld8(const float *p) {
    orc_v8 v;
    memcpy(&v, p, sizeof v);
    return v;
}

static inline float fold8(orc_v8 c) {
    return ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
}

static void dot4(const float *a, const float *b0, const float *b1, const float *b2, const float *b3,
                 int32_t n, float *out) {
    orc_v8 c0 = {0}, c1 = {0}, c2 = {0}, c3 = {0};
    int32_t i = 0;
    for (; i + 8 <= n; i += 8) {
        const orc_v8 av = ld8(a + i);
        c0 += av * ld8(b0 + i);
        c1 += av * ld8(b1 + i);
        c2 += av * ld8(b2 + i);
        c3 += av * ld8(b3 + i);
    }
    float s0 = fold8(c0), s1 = fold8(c1), s2 = fold8(c2), s3 = fold8(c3);
    for (; i < n; i++) {
        s0 += a[i] * b0[i];
        s1 += a[i] * b1[i];
        s2 += a[i] * b2[i];
        s3 += a[i] * b3[i];
    }
    out[0] = s0;
    out[1] = s1;
    out[2] = s2;
    out[3] = s3;
}

/* out[t*ldo + r] = W x_t for n vectors x_t = x + t*ldx: the per-token matvec
 * of orc_dequant_matvec (same row chunks, same dequantisation, same dot
 * order), with each row dequantised once for all n vectors. Serves the
 * layer-major prompt (layer_scheduler.c:721-755), where every token of a
 * layer meets the same matrices. */
typedef struct {
    float *out;
    const uint8_t *w;
    const float *x;
    float *tmp;
    int32_t rows, cols, type, n, ldx, ldo, rows_per_chunk;
    size_t row_bytes;
} mm_job_t;

static void mm_chunk(void *arg, int32_t chunk) {
    mm_job_t *j = (mm_job_t *)arg;
    int32_t r0 = chunk * j->rows_per_chunk;
    int32_t r1 = r0 + j->rows_per_chunk;
    if (r1 > j->rows) r1 = j->rows;
    const size_t cols = (size_t)j->cols;
    float *tmp = j->tmp + (size_t)chunk * j->rows_per_chunk * cols;
    /* rows in blocks of 4: the block's dequantised rows stay in cache while
     * every token's x meets them (a*b and b*a round alike, so dot4 over
     * (x, four rows) gives each row's orc_dot(row, x) exactly) */
    for (int32_t r = r0; r < r1; r++) orc_dequantize(j->w + (size_t)r * j->row_bytes, tmp + (r - r0) * cols, j->cols, j->type);
    int32_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        const float *w0 = tmp + (r - r0) * cols;
        for (int32_t t = 0; t < j->n; t++) {
            float o[4];
            dot4(j->x + (size_t)t * j->ldx, w0, w0 + cols, w0 + 2 * cols, w0 + 3 * cols, j->cols, o);
            for (int k = 0; k < 4; k++) j->out[(size_t)t * j->ldo + r + k] = o[k];
        }
    }
    for (; r < r1; r++)
        for (int32_t t = 0; t < j->n; t++)
            j->out[(size_t)t * j->ldo + r] = orc_dot(tmp + (r - r0) * cols, j->x + (size_t)t * j->ldx, j->cols);
}

static void dequant_matmul(float *out, int32_t ldo, const void *w, const float *x, int32_t ldx, int32_t n,
                           int32_t rows, int32_t cols, int32_t type) {
    size_t rb = orc_row_bytes(cols, type);
    if (rb == 0 || rows <= 0 || n <= 0) return;
    /* chunks of a few rows (a multiple of 4, about 256 KB of dequantised
     * weights) handed to the threads dynamically */
    int32_t per = (int32_t)((256u << 10) / ((size_t)cols * 4)) & ~3;
    if (per < 4) per = 4;
    mm_job_t j = {out, (const uint8_t *)w, x, NULL, rows, cols, type, n, ldx, ldo, per, rb};
    int32_t nchunk = (rows + per - 1) / per;
    j.tmp = (float *)malloc((size_t)nchunk * per * cols * sizeof(float));
    if (!j.tmp) abort();
    pool_run(mm_chunk, &j, nchunk);
    free(j.tmp);
}

/* ------------------------------------------------------------------------ */
/* GGUF parse: gguf_loader.c:22-62, 174-206, 210-485                         */
/* ------------------------------------------------------------------------ */

typedef struct {
    char name[256];
    uint32_t n_dims;
    uint64_t dims[4];
    int32_t type;
    uint64_t offset; /* absolute */
    uint64_t size;
    int32_t layer;
} orc_tensor_t;

typedef struct {
    const orc_tensor_t *attn_norm, *wq, *wk, *wv, *wo, *ffn_norm, *wg, *wu, *wd;
    const orc_tensor_t *wqkv, *bq, *bk, *bv;   /* fused [Wq;Wk;Wv]; Qwen biases (optional) */
    const orc_tensor_t *post_attn_norm, *post_ffn_norm;   /* Gemma 2 (optional, :309-310) */
} orc_layer_t;

struct orc_model {
    int fd;
    uint8_t *base;
    uint64_t fsize;
    orc_tensor_t *tensors;
    uint64_t n_tensors;
    orc_layer_t *layers;
    const orc_tensor_t *embd, *out_norm, *out;
    char arch[64];
    uint32_t n_layers, d, n_heads, n_kv_heads, vocab_meta, ctx_len, ffn, key_len, rope_dim_meta;
    float theta, eps, attn_softcap, final_softcap;
    int32_t hd, rope_dim, vocab, max_seq, kv_mode, kv_dim, neox, gemma;
    /* KV cache, [L][max_seq][kv_dim] (+ per-(L,pos) scales in int8 mode) */
    int8_t *kq, *vq;
    float *ks, *vs;
    uint16_t *kh, *vh;
    /* working state */
    float *hidden, *residual, *attn_out, *ffn_buf, *ffn_gate, *q, *k, *v, *logits;
};

typedef struct {
    const uint8_t *p;
    uint64_t pos, size;
    int bad;
} rd_t;

static uint32_t rd_u32(rd_t *r) {
    if (r->pos + 4 > r->size) { r->bad = 1; return 0; }
    uint32_t v;
    memcpy(&v, r->p + r->pos, 4);
    r->pos += 4;
    return v;
}
static uint64_t rd_u64(rd_t *r) {
    if (r->pos + 8 > r->size) { r->bad = 1; return 0; }
    uint64_t v;
    memcpy(&v, r->p + r->pos, 8);
    r->pos += 8;
    return v;
}
static float rd_f32(rd_t *r) {
    uint32_t u = rd_u32(r);
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* returns pointer into the file and its length; NULL on overrun */
static const char *rd_str(rd_t *r, uint64_t *len) {
    *len = rd_u64(r);
    if (r->bad || r->pos + *len > r->size) { r->bad = 1; return NULL; }
    const char *s = (const char *)r->p + r->pos;
    r->pos += *len;
    return s;
}

static void rd_skip(rd_t *r, uint32_t type) {  /* gguf_loader.c:130-165 */
    uint64_t len;
    switch (type) {
    case 0: case 1: case 7: r->pos += 1; break;
    case 2: case 3: r->pos += 2; break;
    case 4: case 5: case 6: r->pos += 4; break;
    case 10: case 11: case 12: r->pos += 8; break;
    case 8: rd_str(r, &len); break;
    case 9: {
        uint32_t at = rd_u32(r);
        uint64_t n = rd_u64(r);
        for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip(r, at);
        break;
    }
    default: break;
    }
}

static int key_is(const char *k, uint64_t kl, const char *s) {
    return kl == strlen(s) && memcmp(k, s, kl) == 0;
}
static int key_ends(const char *k, uint64_t kl, const char *s) {
    size_t sl = strlen(s);
    return kl >= sl && memcmp(k + kl - sl, s, sl) == 0;
}

/* gguf_loader.c:22-62: weights per block and bytes per block */
static int is_kquant(int32_t t) { return t >= ORC_Q2_K && t <= ORC_Q6_K; }
static int is_legacy(int32_t t) {
    return t == ORC_Q4_0 || t == ORC_Q4_1 || t == ORC_Q5_0 || t == ORC_Q5_1 || t == ORC_Q8_0 || t == ORC_Q8_1;
}
static uint32_t type_block(int32_t t) {
    return is_legacy(t) ? 32 : is_kquant(t) ? 256 : 1;
}
static uint32_t type_size(int32_t t) {
    switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q8_0: return 34;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_1: return 40;
    case ORC_Q2_K: return 84;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    default: return 0;
    }
}

/* gguf_loader.c:174-189 */
static int32_t parse_layer(const char *name) {
    const char *blk = strstr(name, "blk.");
    if (!blk) return -1;
    int32_t idx = 0;
    const char *p = blk + 4;
    while (*p >= '0' && *p <= '9') { idx = idx * 10 + (*p - '0'); p++; }
    return *p == '.' ? idx : -1;
}

/* layer_scheduler.c:27-39: first tensor of the layer whose name ends in suffix */
static const orc_tensor_t *find_suffix(const orc_model_t *m, int32_t layer, const char *suffix) {
    size_t sl = strlen(suffix);
    for (uint64_t i = 0; i < m->n_tensors; i++) {
        const orc_tensor_t *t = &m->tensors[i];
        if (t->layer != layer) continue;
        size_t nl = strlen(t->name);
        if (nl >= sl && strcmp(t->name + nl - sl, suffix) == 0) return t;
    }
    return NULL;
}
static const orc_tensor_t *find_global(const orc_model_t *m, const char *name) {
    for (uint64_t i = 0; i < m->n_tensors; i++)
        if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
    return NULL;
}

static const void *tdata(const orc_model_t *m, const orc_tensor_t *t) {
    if (!t || t->offset + t->size > m->fsize) return NULL;
    return m->base + t->offset;
}

static int parse_gguf(orc_model_t *m) {
    rd_t r = {m->base, 0, m->fsize, 0};
    if (rd_u32(&r) != 0x46554747u) return -1;
    uint32_t ver = rd_u32(&r);
    if (ver < 2 || ver > 3) return -1;
    uint64_t n_tensors = rd_u64(&r);
    uint64_t n_kv = rd_u64(&r);
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t kl;
        const char *k = rd_str(&r, &kl);
        if (!k) return -1;
        uint32_t vt = rd_u32(&r);
        if (key_is(k, kl, "general.architecture") && vt == 8) {
            uint64_t sl;
            const char *s = rd_str(&r, &sl);
            if (!s) return -1;
            size_t c = sl < sizeof(m->arch) - 1 ? sl : sizeof(m->arch) - 1;
            memcpy(m->arch, s, c);
            m->arch[c] = 0;
        } else if (key_ends(k, kl, ".embedding_length") && vt == 4) {
            m->d = rd_u32(&r);
        } else if (key_ends(k, kl, ".attention.head_count_kv") && vt == 4) {
            m->n_kv_heads = rd_u32(&r);
        } else if (key_ends(k, kl, ".attention.head_count") && vt == 4) {
            m->n_heads = rd_u32(&r);
        } else if (key_ends(k, kl, ".context_length") && vt == 4) {
            m->ctx_len = rd_u32(&r);
        } else if (key_ends(k, kl, ".feed_forward_length") && vt == 4) {
            m->ffn = rd_u32(&r);
        } else if (key_ends(k, kl, ".block_count") && vt == 4) {
            m->n_layers = rd_u32(&r);
        } else if (key_ends(k, kl, ".vocab_size") && vt == 4) {
            m->vocab_meta = rd_u32(&r);
        } else if (key_ends(k, kl, ".rope.freq_base") && vt == 6) {
            m->theta = rd_f32(&r);
        } else if (key_ends(k, kl, ".attention.layer_norm_rms_epsilon") && vt == 6) {
            m->eps = rd_f32(&r);
        } else if (key_ends(k, kl, ".attention.key_length") && vt == 4) {
            m->key_len = rd_u32(&r);
        } else if (key_ends(k, kl, ".rope.dimension_count") && vt == 4) {
            m->rope_dim_meta = rd_u32(&r);
        } else if (key_ends(k, kl, ".attn_logit_softcapping") && vt == 6) {   /* gguf_loader.c:314-317 */
            m->attn_softcap = rd_f32(&r);
        } else if (key_ends(k, kl, ".final_logit_softcapping") && vt == 6) {
            m->final_softcap = rd_f32(&r);
        } else if (key_is(k, kl, "tokenizer.ggml.tokens") && vt == 9) {
            uint32_t at = rd_u32(&r);
            uint64_t n = rd_u64(&r);
            if (at == 8 && n > 0) m->vocab_meta = (uint32_t)n;
            for (uint64_t v = 0; v < n && !r.bad; v++) rd_skip(&r, at);
        } else {
            rd_skip(&r, vt);
        }
        if (r.bad) return -1;
    }
    if (m->eps == 0.0f) m->eps = 1e-5f;                       /* gguf_loader.c:370 */
    if (m->theta == 0.0f) m->theta = strstr(m->arch, "qwen") ? 1000000.0f : 10000.0f;
    if (m->ctx_len == 0) m->ctx_len = 2048;

    m->n_tensors = n_tensors;
    m->tensors = (orc_tensor_t *)calloc(n_tensors ? n_tensors : 1, sizeof(orc_tensor_t));
    if (!m->tensors) return -1;
    for (uint64_t i = 0; i < n_tensors; i++) {
        orc_tensor_t *t = &m->tensors[i];
        uint64_t nl;
        const char *nm = rd_str(&r, &nl);
        if (!nm) return -1;
        size_t c = nl < 255 ? nl : 255;
        memcpy(t->name, nm, c);
        t->name[c] = 0;
        t->n_dims = rd_u32(&r);
        if (t->n_dims > 4) return -1;
        for (uint32_t dd = 0; dd < t->n_dims; dd++) t->dims[dd] = rd_u64(&r);
        t->type = (int32_t)rd_u32(&r);
        t->offset = rd_u64(&r);
        if (r.bad) return -1;
        if (m->vocab_meta == 0 && strcmp(t->name, "token_embd.weight") == 0 && t->n_dims == 2)
            m->vocab_meta = (uint32_t)t->dims[1];
        uint64_t ne = 1;
        for (uint32_t dd = 0; dd < t->n_dims; dd++) ne *= t->dims[dd];
        uint32_t bs = type_block(t->type);
        t->size = bs == 1 ? ne * type_size(t->type) : (ne / bs) * type_size(t->type);
        t->layer = parse_layer(t->name);
    }
    uint64_t data_off = (r.pos + 31) & ~(uint64_t)31;      /* gguf_loader.c:426 */
    for (uint64_t i = 0; i < n_tensors; i++) m->tensors[i].offset += data_off;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Scheduler: layer_scheduler.c:129-244, 291-567, 571-936                    */
/* ------------------------------------------------------------------------ */

void orc_model_close(orc_model_t *m) {
    if (!m) return;
    free(m->tensors);
    free(m->layers);
    free(m->kq); free(m->vq); free(m->ks); free(m->vs); free(m->kh); free(m->vh);
    free(m->hidden); free(m->residual); free(m->attn_out); free(m->ffn_buf);
    free(m->ffn_gate); free(m->q); free(m->k); free(m->v); free(m->logits);
    if (m->base && m->base != MAP_FAILED) munmap(m->base, m->fsize);
    if (m->fd >= 0) close(m->fd);
    free(m);
}

static int matrix_ok(const orc_tensor_t *t, uint64_t rows, uint64_t cols) {
    return t && t->n_dims == 2 && t->dims[0] == cols && t->dims[1] == rows &&
           ((is_legacy(t->type) && cols % 32 == 0) || t->type == ORC_F32 || t->type == ORC_F16 ||
            (is_kquant(t->type) && cols % 256 == 0));
}
static int vector_ok(const orc_tensor_t *t, uint64_t n) {
    return t && t->type == ORC_F32 && t->dims[0] == n;
}
static int bias_ok(const orc_tensor_t *t, uint64_t n) {
    return (t->type == ORC_F32 || t->type == ORC_F16) && t->dims[0] == n;
}

/* layer_scheduler.c:367-402 with safe_load_f32 (:284-289): x[i] += b[i] */
static void add_bias(const orc_model_t *m, float *x, const orc_tensor_t *b, int32_t n) {
    if (!b) return;
    const void *p = m->base + b->offset;
    for (int32_t i = 0; i < n; i++)
        x[i] = x[i] + (b->type == ORC_F16 ? orc_f16_to_f32(((const uint16_t *)p)[i]) : ((const float *)p)[i]);
}

orc_model_t *orc_model_open(const char *path, int32_t max_seq, int32_t kv_mode) {
    if (!path) return NULL;
    orc_model_t *m = (orc_model_t *)calloc(1, sizeof(orc_model_t));
    if (!m) return NULL;
    m->fd = open(path, O_RDONLY);
    if (m->fd < 0) { free(m); return NULL; }
    struct stat st;
    if (fstat(m->fd, &st) < 0) { close(m->fd); free(m); return NULL; }
    m->fsize = (uint64_t)st.st_size;
    m->base = (uint8_t *)mmap(NULL, m->fsize, PROT_READ, MAP_SHARED, m->fd, 0);
    if (m->base == MAP_FAILED) { m->base = NULL; orc_model_close(m); return NULL; }
    if (parse_gguf(m) != 0) { orc_model_close(m); return NULL; }

    m->gemma = strstr(m->arch, "gemma") != NULL;                   /* :152-155 */
    /* layer_scheduler.c:144-149 */
    m->neox = strstr(m->arch, "qwen") || strstr(m->arch, "falcon") || strstr(m->arch, "phi") ||
              strstr(m->arch, "deepseek");
    if (m->n_kv_heads == 0) m->n_kv_heads = m->n_heads;
    if (m->n_layers == 0 || m->d == 0 || m->n_heads == 0) { orc_model_close(m); return NULL; }

    /* head_dim derivation, layer_scheduler.c:161-181 */
    int32_t hd = 0;
    if (m->key_len > 0) {
        hd = (int32_t)m->key_len;
    } else {
        const orc_tensor_t *wq0 = find_global(m, "blk.0.attn_q.weight");
        if (wq0) hd = (int32_t)(wq0->dims[1] / m->n_heads);
    }
    if (hd == 0) hd = (int32_t)(m->d / m->n_heads);
    m->hd = hd;
    m->rope_dim = m->rope_dim_meta > 0 ? (int32_t)m->rope_dim_meta : hd;

    /* vocab clamp, layer_scheduler.c:185-197 */
    int32_t vocab = (int32_t)m->vocab_meta;
    for (uint64_t i = 0; i < m->n_tensors; i++) {
        const orc_tensor_t *t = &m->tensors[i];
        if ((strcmp(t->name, "output.weight") == 0 || strcmp(t->name, "token_embd.weight") == 0) &&
            t->n_dims == 2 && (int32_t)t->dims[1] < vocab)
            vocab = (int32_t)t->dims[1];
    }
    m->vocab = vocab;
    m->max_seq = max_seq > 0 ? max_seq : (int32_t)m->ctx_len;
    m->kv_mode = kv_mode;
    m->kv_dim = (int32_t)m->n_kv_heads * hd;

    int32_t L = (int32_t)m->n_layers, d = (int32_t)m->d, ffn = (int32_t)m->ffn;
    int32_t qdim = (int32_t)m->n_heads * hd;
    m->embd = find_global(m, "token_embd.weight");
    m->out_norm = find_global(m, "output_norm.weight");
    m->out = find_global(m, "output.weight");
    if (!m->out) m->out = m->embd;                            /* tied, :652-655 */
    if (!m->embd || !matrix_ok(m->embd, m->embd->dims[1], (uint64_t)d) || !m->out ||
        !matrix_ok(m->out, m->out->dims[1], (uint64_t)d) || (m->out_norm && !vector_ok(m->out_norm, d))) {
        orc_model_close(m);
        return NULL;
    }
    m->layers = (orc_layer_t *)calloc((size_t)L, sizeof(orc_layer_t));
    if (!m->layers) { orc_model_close(m); return NULL; }
    for (int32_t l = 0; l < L; l++) {
        orc_layer_t *ly = &m->layers[l];
        ly->attn_norm = find_suffix(m, l, "attn_norm.weight");
        ly->wq = find_suffix(m, l, "attn_q.weight");
        ly->wk = find_suffix(m, l, "attn_k.weight");
        ly->wv = find_suffix(m, l, "attn_v.weight");
        ly->wo = find_suffix(m, l, "attn_output.weight");
        ly->ffn_norm = find_suffix(m, l, "ffn_norm.weight");
        ly->wg = find_suffix(m, l, "ffn_gate.weight");
        ly->wu = find_suffix(m, l, "ffn_up.weight");
        ly->wd = find_suffix(m, l, "ffn_down.weight");
        ly->wqkv = find_suffix(m, l, "attn_qkv.weight");
        ly->bq = find_suffix(m, l, "attn_q.bias");
        ly->bk = find_suffix(m, l, "attn_k.bias");
        ly->bv = find_suffix(m, l, "attn_v.bias");
        ly->post_attn_norm = find_suffix(m, l, "post_attention_norm.weight");
        ly->post_ffn_norm = find_suffix(m, l, "post_ffw_norm.weight");
        int qkv_ok = ly->wqkv ? matrix_ok(ly->wqkv, qdim + 2 * (uint64_t)m->kv_dim, d)
                              : matrix_ok(ly->wq, qdim, d) && matrix_ok(ly->wk, m->kv_dim, d) &&
                                    matrix_ok(ly->wv, m->kv_dim, d);
        int ffn_ok = ly->wg ? matrix_ok(ly->wg, ffn, d) && matrix_ok(ly->wu, ffn, d)
                            : matrix_ok(ly->wu, 2 * (uint64_t)ffn, d);   /* fused, :518-524 */
        if (!vector_ok(ly->attn_norm, d) || !qkv_ok || !matrix_ok(ly->wo, d, qdim) ||
            !vector_ok(ly->ffn_norm, d) || !ffn_ok || !matrix_ok(ly->wd, d, ffn) ||
            (ly->bq && !bias_ok(ly->bq, qdim)) || (ly->bk && !bias_ok(ly->bk, m->kv_dim)) ||
            (ly->bv && !bias_ok(ly->bv, m->kv_dim)) ||
            (ly->post_attn_norm && !vector_ok(ly->post_attn_norm, d)) ||
            (ly->post_ffn_norm && !vector_ok(ly->post_ffn_norm, d))) {
            orc_model_close(m);
            return NULL;
        }
    }

    size_t vecs = (size_t)L * m->max_seq;
    size_t elems = vecs * m->kv_dim;
    if (kv_mode == ORC_KV_INT8) {
        m->kq = (int8_t *)calloc(elems, 1);
        m->vq = (int8_t *)calloc(elems, 1);
        m->ks = (float *)calloc(vecs, sizeof(float));
        m->vs = (float *)calloc(vecs, sizeof(float));
        if (!m->kq || !m->vq || !m->ks || !m->vs) { orc_model_close(m); return NULL; }
    } else {
        m->kh = (uint16_t *)calloc(elems, 2);
        m->vh = (uint16_t *)calloc(elems, 2);
        if (!m->kh || !m->vh) { orc_model_close(m); return NULL; }
    }
    m->hidden = (float *)calloc((size_t)d, 4);
    m->residual = (float *)calloc((size_t)d, 4);
    m->attn_out = (float *)calloc((size_t)(qdim > d ? qdim : d), 4);
    m->ffn_buf = (float *)calloc((size_t)ffn, 4);
    m->ffn_gate = (float *)calloc((size_t)ffn, 4);
    m->q = (float *)calloc((size_t)qdim, 4);
    m->k = (float *)calloc((size_t)m->kv_dim, 4);
    m->v = (float *)calloc((size_t)m->kv_dim, 4);
    m->logits = (float *)calloc((size_t)vocab, 4);
    if (!m->hidden || !m->residual || !m->attn_out || !m->ffn_buf || !m->ffn_gate || !m->q ||
        !m->k || !m->v || !m->logits) {
        orc_model_close(m);
        return NULL;
    }
    return m;
}

void orc_model_dims(const orc_model_t *m, int32_t *o) {
    o[0] = (int32_t)m->n_layers; o[1] = (int32_t)m->d; o[2] = (int32_t)m->n_heads;
    o[3] = (int32_t)m->n_kv_heads; o[4] = m->hd; o[5] = (int32_t)m->ffn; o[6] = m->vocab;
    o[7] = m->max_seq;
}
float orc_model_eps(const orc_model_t *m) { return m->eps; }
float orc_model_theta(const orc_model_t *m) { return m->theta; }
const float *orc_hidden(const orc_model_t *m) { return m->hidden; }

static void matvec_t(orc_model_t *m, float *out, const orc_tensor_t *t, const float *x) {
    orc_dequant_matvec(out, tdata(m, t), x, (int32_t)t->dims[1], (int32_t)t->dims[0], t->type);
}

/* KV row (layer, pos) -> fp32, head slice [head*hd, head*hd+hd) */
static void kv_read(const orc_model_t *m, int is_v, int32_t layer, int32_t t, int32_t head, float *dst) {
    size_t vi = (size_t)layer * m->max_seq + t;
    size_t off = vi * m->kv_dim + (size_t)head * m->hd;
    if (m->kv_mode == ORC_KV_INT8) {
        const int8_t *q = (is_v ? m->vq : m->kq) + off;
        float s = (is_v ? m->vs : m->ks)[vi];
        for (int32_t i = 0; i < m->hd; i++) dst[i] = (float)q[i] * s;   /* :120-125 */
    } else {
        const uint16_t *h = (is_v ? m->vh : m->kh) + off;
        for (int32_t i = 0; i < m->hd; i++) dst[i] = orc_f16_to_f32(h[i]);
    }
}

static void kv_store(orc_model_t *m, int32_t layer, int32_t pos, const float *k, const float *v) {
    size_t vi = (size_t)layer * m->max_seq + pos;
    size_t off = vi * m->kv_dim;
    if (m->kv_mode == ORC_KV_INT8) {                                 /* :409-413 */
        orc_kv_int8_encode(k, m->kq + off, &m->ks[vi], m->kv_dim);
        orc_kv_int8_encode(v, m->vq + off, &m->vs[vi], m->kv_dim);
    } else {
        for (int32_t i = 0; i < m->kv_dim; i++) {
            m->kh[off + i] = orc_f32_to_f16(k[i]);
            m->vh[off + i] = orc_f32_to_f16(v[i]);
        }
    }
}

typedef struct {
    orc_model_t *m;
    int32_t layer, seq_len, heads_per_kv;
    float scale;
} attn_job_t;

/* layer_scheduler.c:424-468 for one query head: scores over positions
 * 0..seq_len-1 of KV head kvh, softmax, weighted sum of values into dst. */
static void attend(const orc_model_t *m, int32_t layer, int32_t seq_len, int32_t kvh, float scale,
                   const float *q, float *dst) {
    int32_t hd = m->hd;
    float *scores = (float *)malloc((size_t)seq_len * sizeof(float));
    float *tmp = (float *)malloc((size_t)hd * sizeof(float));
    if (!scores || !tmp) abort();
    for (int32_t t = 0; t < seq_len; t++) {
        kv_read(m, 0, layer, t, kvh, tmp);
        scores[t] = orc_dot(q, tmp, hd) * scale;
    }
    orc_softcap(scores, seq_len, m->attn_softcap);                  /* :446-448 */
    orc_softmax(scores, seq_len);
    memset(dst, 0, (size_t)hd * sizeof(float));
    for (int32_t t = 0; t < seq_len; t++) {
        kv_read(m, 1, layer, t, kvh, tmp);
        float w = scores[t];
        for (int32_t i = 0; i < hd; i++) dst[i] = w * tmp[i] + dst[i];
    }
    free(tmp);
    free(scores);
}

/* one query head per task */
static void attn_head(void *arg, int32_t h) {
    attn_job_t *j = (attn_job_t *)arg;
    orc_model_t *m = j->m;
    attend(m, j->layer, j->seq_len, h / j->heads_per_kv, j->scale, m->q + (size_t)h * m->hd,
           m->attn_out + (size_t)h * m->hd);
}

/* the pre-norms: (1 + w) for Gemma (:328-334, 492-498), w otherwise */
static void norm_in(const orc_model_t *m, float *out, const float *x, const orc_tensor_t *w) {
    if (m->gemma)
        orc_gemma_rmsnorm(out, x, (const float *)tdata(m, w), (int32_t)m->d, m->eps);
    else
        orc_rmsnorm(out, x, (const float *)tdata(m, w), (int32_t)m->d, m->eps);
}

/* :474-481, 553-560: a post norm (always the (1 + w) form) on the
 * projection's output, before the residual, when the tensor exists */
static void post_norm(const orc_model_t *m, float *x, const orc_tensor_t *w) {
    if (w) orc_gemma_rmsnorm(x, x, (const float *)tdata(m, w), (int32_t)m->d, m->eps);
}

/* :529-549: up * GELU(gate) for Gemma (ss_geglu then ss_elementwise_mul),
 * up * SiLU(gate) otherwise; u is overwritten */
static void ffn_act(const orc_model_t *m, const float *g, float *u, int32_t n) {
    if (m->gemma)
        for (int32_t i = 0; i < n; i++) u[i] = u[i] * orc_gelu(g[i]);
    else
        for (int32_t i = 0; i < n; i++) u[i] = orc_silu_mul(g[i], u[i]);
}

/* layer_scheduler.c:291-567 */
static void process_layer(orc_model_t *m, int32_t l, int32_t pos) {
    const orc_layer_t *ly = &m->layers[l];
    int32_t d = (int32_t)m->d, ffn = (int32_t)m->ffn;
    memcpy(m->residual, m->hidden, (size_t)d * 4);
    norm_in(m, m->hidden, m->residual, ly->attn_norm);
    int32_t qdim = (int32_t)m->n_heads * m->hd, kvd = m->kv_dim;
    if (ly->wqkv) {   /* :337-347: one product, then split (attn_qkv.bias is never applied) */
        float *qkv = (float *)malloc((size_t)(qdim + 2 * kvd) * 4);
        if (!qkv) abort();
        matvec_t(m, qkv, ly->wqkv, m->hidden);
        memcpy(m->q, qkv, (size_t)qdim * 4);
        memcpy(m->k, qkv + qdim, (size_t)kvd * 4);
        memcpy(m->v, qkv + qdim + kvd, (size_t)kvd * 4);
        free(qkv);
    } else {
        matvec_t(m, m->q, ly->wq, m->hidden);
        matvec_t(m, m->k, ly->wk, m->hidden);
        matvec_t(m, m->v, ly->wv, m->hidden);
    }
    add_bias(m, m->q, ly->bq, qdim);
    add_bias(m, m->k, ly->bk, kvd);
    add_bias(m, m->v, ly->bv, kvd);
    orc_rope(m->q, m->k, (int32_t)m->n_heads, (int32_t)m->n_kv_heads, m->hd, m->rope_dim, pos,
             m->theta, m->neox);
    kv_store(m, l, pos, m->k, m->v);

    attn_job_t j = {m, l, pos + 1, (int32_t)(m->n_heads / m->n_kv_heads),
                    1.0f / sqrtf((float)m->hd)};
    memset(m->attn_out, 0, (size_t)d * 4);
    pool_run(attn_head, &j, (int32_t)m->n_heads);

    matvec_t(m, m->hidden, ly->wo, m->attn_out);
    post_norm(m, m->hidden, ly->post_attn_norm);
    for (int32_t i = 0; i < d; i++) m->hidden[i] = m->hidden[i] + m->residual[i];   /* :484 */

    memcpy(m->residual, m->hidden, (size_t)d * 4);
    norm_in(m, m->hidden, m->residual, ly->ffn_norm);
    if (ly->wg) {
        matvec_t(m, m->ffn_gate, ly->wg, m->hidden);
        matvec_t(m, m->ffn_buf, ly->wu, m->hidden);
    } else {          /* :518-524: fused [gate; up] */
        float *gu = (float *)malloc((size_t)2 * ffn * 4);
        if (!gu) abort();
        matvec_t(m, gu, ly->wu, m->hidden);
        memcpy(m->ffn_gate, gu, (size_t)ffn * 4);
        memcpy(m->ffn_buf, gu + ffn, (size_t)ffn * 4);
        free(gu);
    }
    ffn_act(m, m->ffn_gate, m->ffn_buf, ffn);
    matvec_t(m, m->hidden, ly->wd, m->ffn_buf);
    post_norm(m, m->hidden, ly->post_ffn_norm);
    for (int32_t i = 0; i < d; i++) m->hidden[i] = m->hidden[i] + m->residual[i];   /* :566 */
}

/* process_layer for tokens start..start+n-1 of one layer at once (the
 * layer-major order of layer_scheduler.c:721-755). Every token goes through
 * exactly process_layer's arithmetic; the matrices are applied to all n
 * tokens by dequant_matmul (each row dequantised once, the same dot order),
 * and all n tokens' K/V are stored before any attends, which reads only
 * positions up to its own: every output is bit-identical to n calls of
 * process_layer. X is [n][d], in place. */
/* attend() over fp32 rows: K row t at K + t * ld (the cache widened once
 * per layer; kv_read's widening is exact or one fp32 product, so the rows
 * hold the values attend() reads) */
static void attend_rows(const float *K, const float *V, size_t ld, int32_t seq_len, int32_t hd, float scale,
                        float softcap, const float *q, float *dst) {
    float *scores = (float *)malloc((size_t)seq_len * sizeof(float));
    if (!scores) abort();
    for (int32_t t = 0; t < seq_len; t++) scores[t] = orc_dot(q, K + t * ld, hd) * scale;
    orc_softcap(scores, seq_len, softcap);
    orc_softmax(scores, seq_len);
    memset(dst, 0, (size_t)hd * sizeof(float));
    for (int32_t t = 0; t < seq_len; t++) {
        const float w = scores[t], *v = V + t * ld;
        for (int32_t i = 0; i < hd; i++) dst[i] = w * v[i] + dst[i];
    }
    free(scores);
}

typedef struct {
    const orc_model_t *m;
    int32_t start, heads_per_kv;
    float scale;
    const float *K, *V;   /* the layer's cache rows 0..start+n-1, widened, [pos][kv_dim] */
    const float *q;       /* [n][qdim] */
    float *out;           /* [n][qdim] */
} attn_batch_job_t;

static void attn_batch_task(void *arg, int32_t task) {
    attn_batch_job_t *j = (attn_batch_job_t *)arg;
    const orc_model_t *m = j->m;
    int32_t H = (int32_t)m->n_heads, i = task / H, h = task % H, hd = m->hd;
    size_t qdim = (size_t)H * hd, koff = (size_t)(h / j->heads_per_kv) * hd;
    attend_rows(j->K + koff, j->V + koff, (size_t)m->kv_dim, j->start + i + 1, hd, j->scale, m->attn_softcap,
                j->q + i * qdim + (size_t)h * hd, j->out + i * qdim + (size_t)h * hd);
}

static void layer_batch(orc_model_t *m, int32_t l, int32_t start, int32_t n, float *X) {
    const orc_layer_t *ly = &m->layers[l];
    const int32_t d = (int32_t)m->d, ffn = (int32_t)m->ffn, qdim = (int32_t)m->n_heads * m->hd;
    const int32_t kvd = m->kv_dim, nqkv = qdim + 2 * kvd;
    float *res = (float *)malloc((size_t)n * d * 4), *xn = (float *)malloc((size_t)n * d * 4);
    float *qkv = (float *)malloc((size_t)n * nqkv * 4), *att = (float *)malloc((size_t)n * qdim * 4);
    float *gu = (float *)malloc((size_t)n * 2 * ffn * 4);
    if (!res || !xn || !qkv || !att || !gu) abort();
    for (int32_t i = 0; i < n; i++) {
        memcpy(res + (size_t)i * d, X + (size_t)i * d, (size_t)d * 4);
        norm_in(m, xn + (size_t)i * d, res + (size_t)i * d, ly->attn_norm);
    }
    /* [q | k | v] per token, from one fused product or three */
    if (ly->wqkv) {
        dequant_matmul(qkv, nqkv, tdata(m, ly->wqkv), xn, d, n, nqkv, d, ly->wqkv->type);
    } else {
        dequant_matmul(qkv, nqkv, tdata(m, ly->wq), xn, d, n, qdim, d, ly->wq->type);
        dequant_matmul(qkv + qdim, nqkv, tdata(m, ly->wk), xn, d, n, kvd, d, ly->wk->type);
        dequant_matmul(qkv + qdim + kvd, nqkv, tdata(m, ly->wv), xn, d, n, kvd, d, ly->wv->type);
    }
    float *q = (float *)malloc((size_t)n * qdim * 4);
    if (!q) abort();
    for (int32_t i = 0; i < n; i++) {
        float *qi = qkv + (size_t)i * nqkv, *ki = qi + qdim, *vi = ki + kvd;
        add_bias(m, qi, ly->bq, qdim);
        add_bias(m, ki, ly->bk, kvd);
        add_bias(m, vi, ly->bv, kvd);
        orc_rope(qi, ki, (int32_t)m->n_heads, (int32_t)m->n_kv_heads, m->hd, m->rope_dim, start + i, m->theta,
                 m->neox);
        kv_store(m, l, start + i, ki, vi);
        memcpy(q + (size_t)i * qdim, qi, (size_t)qdim * 4);
    }
    const int32_t npos = start + n;
    float *K = (float *)malloc((size_t)npos * kvd * 4), *V = (float *)malloc((size_t)npos * kvd * 4);
    if (!K || !V) abort();
    for (int32_t t = 0; t < npos; t++)
        for (int32_t g = 0; g < (int32_t)m->n_kv_heads; g++) {
            kv_read(m, 0, l, t, g, K + (size_t)t * kvd + (size_t)g * m->hd);
            kv_read(m, 1, l, t, g, V + (size_t)t * kvd + (size_t)g * m->hd);
        }
    attn_batch_job_t aj = {m, start, (int32_t)(m->n_heads / m->n_kv_heads), 1.0f / sqrtf((float)m->hd), K, V, q, att};
    pool_run(attn_batch_task, &aj, n * (int32_t)m->n_heads);
    free(V);
    free(K);
    dequant_matmul(X, d, tdata(m, ly->wo), att, qdim, n, (int32_t)ly->wo->dims[1], (int32_t)ly->wo->dims[0],
                   ly->wo->type);
    for (int32_t i = 0; i < n; i++) post_norm(m, X + (size_t)i * d, ly->post_attn_norm);
    for (size_t e = 0; e < (size_t)n * d; e++) X[e] = X[e] + res[e];                 /* :484 */
    for (int32_t i = 0; i < n; i++) {
        memcpy(res + (size_t)i * d, X + (size_t)i * d, (size_t)d * 4);
        norm_in(m, xn + (size_t)i * d, res + (size_t)i * d, ly->ffn_norm);
    }
    /* gate | up per token: two products, or the fused [gate; up] (:518-524) */
    if (ly->wg) {
        dequant_matmul(gu, 2 * ffn, tdata(m, ly->wg), xn, d, n, ffn, d, ly->wg->type);
        dequant_matmul(gu + ffn, 2 * ffn, tdata(m, ly->wu), xn, d, n, ffn, d, ly->wu->type);
    } else {
        dequant_matmul(gu, 2 * ffn, tdata(m, ly->wu), xn, d, n, 2 * ffn, d, ly->wu->type);
    }
    for (int32_t i = 0; i < n; i++) {
        float *g = gu + (size_t)i * 2 * ffn, *u = g + ffn;
        ffn_act(m, g, u, ffn);
    }
    dequant_matmul(X, d, tdata(m, ly->wd), gu + ffn, 2 * ffn, n, (int32_t)ly->wd->dims[1], (int32_t)ly->wd->dims[0],
                   ly->wd->type);
    for (int32_t i = 0; i < n; i++) post_norm(m, X + (size_t)i * d, ly->post_ffn_norm);
    for (size_t e = 0; e < (size_t)n * d; e++) X[e] = X[e] + res[e];                 /* :566 */
    free(q);
    free(gu);
    free(att);
    free(qkv);
    free(xn);
    free(res);
}

static void embed_row(orc_model_t *m, int32_t token, float *dst) {   /* :584-602 */
    size_t rb = orc_row_bytes((int32_t)m->d, m->embd->type);
    const uint8_t *row = (const uint8_t *)tdata(m, m->embd) + (size_t)token * rb;
    orc_dequantize(row, dst, (int32_t)m->d, m->embd->type);
    if (m->gemma) {
        float sq = sqrtf((float)m->d);
        for (int32_t i = 0; i < (int32_t)m->d; i++) dst[i] *= sq;
    }
}

static void head(orc_model_t *m) {                                   /* :634-676 */
    if (m->out_norm) norm_in(m, m->hidden, m->hidden, m->out_norm);
    orc_dequant_matvec(m->logits, tdata(m, m->out), m->hidden, m->vocab, (int32_t)m->d, m->out->type);
    if (m->gemma) {
        float inv_sq = 1.0f / sqrtf((float)m->d);
        for (int32_t i = 0; i < m->vocab; i++) m->logits[i] *= inv_sq;
    }
    orc_softcap(m->logits, m->vocab, m->final_softcap);
}

const float *orc_forward(orc_model_t *m, int32_t token, int32_t pos) {
    if (!m || pos < 0 || pos >= m->max_seq || token < 0 || (uint64_t)token >= m->embd->dims[1])
        return NULL;
    embed_row(m, token, m->hidden);
    for (int32_t l = 0; l < (int32_t)m->n_layers; l++) process_layer(m, l, pos);
    head(m);
    return m->logits;
}

/* The prompt's embeddings, layer-major through the layers (:681-803). The
 * tokens of a layer go through layer_batch; orc_prefill_serial is the
 * literal token-by-token loop, kept to show the two agree bit for bit. */
static float *prefill_embed(orc_model_t *m, const int32_t *tokens, int32_t n) {
    int32_t d = (int32_t)m->d;
    float *batch = (float *)malloc((size_t)n * d * 4);
    if (!batch) return NULL;
    for (int32_t i = 0; i < n; i++) {
        if (tokens[i] < 0 || (uint64_t)tokens[i] >= m->embd->dims[1]) { free(batch); return NULL; }
        embed_row(m, tokens[i], batch + (size_t)i * d);
    }
    return batch;
}

/* at most this many tokens per layer_batch call (bounds its buffers) */
#define ORC_BATCH_TOKENS 256

static void layers_batched(orc_model_t *m, int32_t start_pos, int32_t n, float *batch) {
    for (int32_t l = 0; l < (int32_t)m->n_layers; l++)
        for (int32_t i0 = 0; i0 < n; i0 += ORC_BATCH_TOKENS) {
            int32_t nb = n - i0 < ORC_BATCH_TOKENS ? n - i0 : ORC_BATCH_TOKENS;
            layer_batch(m, l, start_pos + i0, nb, batch + (size_t)i0 * m->d);
        }
}

const float *orc_prefill(orc_model_t *m, const int32_t *tokens, int32_t n, int32_t start_pos) {
    if (!m || n <= 0 || start_pos < 0 || start_pos + n > m->max_seq) return NULL;
    float *batch = prefill_embed(m, tokens, n);
    if (!batch) return NULL;
    layers_batched(m, start_pos, n, batch);
    memcpy(m->hidden, batch + (size_t)(n - 1) * m->d, (size_t)m->d * 4);
    free(batch);
    head(m);
    return m->logits;
}

const float *orc_prefill_serial(orc_model_t *m, const int32_t *tokens, int32_t n, int32_t start_pos) {
    if (!m || n <= 0 || start_pos < 0 || start_pos + n > m->max_seq) return NULL;
    int32_t d = (int32_t)m->d;
    float *batch = prefill_embed(m, tokens, n);
    if (!batch) return NULL;
    for (int32_t l = 0; l < (int32_t)m->n_layers; l++)               /* layer-major, :721-755 */
        for (int32_t i = 0; i < n; i++) {
            memcpy(m->hidden, batch + (size_t)i * d, (size_t)d * 4);
            process_layer(m, l, start_pos + i);
            memcpy(batch + (size_t)i * d, m->hidden, (size_t)d * 4);
        }
    memcpy(m->hidden, batch + (size_t)(n - 1) * d, (size_t)d * 4);
    free(batch);
    head(m);
    return m->logits;
}

/* layer_scheduler.c:805-915: positions 0..n-1, final norm on every token,
 * mean pool, L2 normalise. */
int32_t orc_embed(orc_model_t *m, const int32_t *tokens, int32_t n, float *out) {
    if (!m || n <= 0 || n > m->max_seq) return -1;
    int32_t d = (int32_t)m->d;
    float *batch = prefill_embed(m, tokens, n);
    if (!batch) return -1;
    layers_batched(m, 0, n, batch);
    if (m->out_norm)
        for (int32_t i = 0; i < n; i++) norm_in(m, batch + (size_t)i * d, batch + (size_t)i * d, m->out_norm);
    memset(out, 0, (size_t)d * 4);
    for (int32_t i = 0; i < n; i++)
        for (int32_t j = 0; j < d; j++) out[j] += batch[(size_t)i * d + j];
    float inv = 1.0f / (float)n, l2 = 0.0f;
    for (int32_t j = 0; j < d; j++) {
        out[j] *= inv;
        l2 += out[j] * out[j];
    }
    float s = 1.0f / (sqrtf(l2) + 1e-12f);
    for (int32_t j = 0; j < d; j++) out[j] *= s;
    free(batch);
    return 0;
}

void orc_reset(orc_model_t *m) {                                     /* :917-936 */
    if (!m) return;
    size_t vecs = (size_t)m->n_layers * m->max_seq, elems = vecs * m->kv_dim;
    if (m->kv_mode == ORC_KV_INT8) {
        memset(m->kq, 0, elems); memset(m->vq, 0, elems);
        memset(m->ks, 0, vecs * 4); memset(m->vs, 0, vecs * 4);
    } else {
        memset(m->kh, 0, elems * 2); memset(m->vh, 0, elems * 2);
    }
    memset(m->hidden, 0, (size_t)m->d * 4);
}

int32_t orc_kv_write(orc_model_t *m, int32_t layer, int32_t pos, const uint16_t *k_f16,
                     const uint16_t *v_f16) {
    if (!m || layer < 0 || layer >= (int32_t)m->n_layers || pos < 0 || pos >= m->max_seq) return -1;
    if (m->kv_mode == ORC_KV_F16) {
        size_t off = ((size_t)layer * m->max_seq + pos) * m->kv_dim;
        memcpy(m->kh + off, k_f16, (size_t)m->kv_dim * 2);
        memcpy(m->vh + off, v_f16, (size_t)m->kv_dim * 2);
        return 0;
    }
    float *kf = (float *)malloc((size_t)m->kv_dim * 4), *vf = (float *)malloc((size_t)m->kv_dim * 4);
    for (int32_t i = 0; i < m->kv_dim; i++) {
        kf[i] = orc_f16_to_f32(k_f16[i]);
        vf[i] = orc_f16_to_f32(v_f16[i]);
    }
    kv_store(m, layer, pos, kf, vf);
    free(kf);
    free(vf);
    return 0;
}
