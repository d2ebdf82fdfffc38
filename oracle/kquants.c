/*
 * Oracle: decoder weight formats and the matrix-vector products that read them
 * (TEST INFRASTRUCTURE ONLY).
 *
 * The decoder's projections are ggml_mul_mat(W, x) on GGUF weights
 * (src/voxtral.cpp:2656-2659 Q/K/V, :2857 O, :2878-2882 SwiGLU FFN); in the
 * Q4_K_M files the quantizer writes, attn_v / ffn_w2 / tok_embeddings / output
 * are Q6_K and the other decoder matrices Q4_K (src/voxtral-quantize.cpp:
 * 148-159).  The block formats and the CPU arithmetic belong to ggml, which the
 * reference fetches at 5cecdad6 (CMakeLists.txt:81-95) and which is not in the
 * tree; what follows restates ggml's published formats and its portable
 * ("generic") CPU routines:
 *
 *   block_q4_K (144 B): fp16 d, fp16 dmin, u8 scales[12], u8 qs[128].
 *       Eight sub-blocks of 32.  Sub-block j has a 6-bit scale sc_j and a
 *       6-bit min m_j packed in scales[]: for j < 4, sc = s[j] & 63 and
 *       m = s[j+4] & 63; for j >= 4, sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4
 *       and m = (s[j+4] >> 4) | (s[j] >> 6) << 4.  qs[32c + l] holds element
 *       l of sub-block 2c in its low nibble and of sub-block 2c+1 in its high
 *       nibble.  Value = (d*sc_j) * q - (dmin*m_j).
 *   block_q6_K (210 B): u8 ql[128], u8 qh[64], i8 scales[16], fp16 d.
 *       Element 128n + 32g + l (n < 2, g < 4, l < 32) has 6-bit code
 *       (low nibble of ql[64n + l] for g = 0, of ql[64n + 32 + l] for g = 1,
 *       high nibble of ql[64n + l] for g = 2, of ql[64n + 32 + l] for g = 3)
 *       | ((qh[32n + l] >> 2g) & 3) << 4, and scale scales[8n + 2g + l/16].
 *       Value = (d*scale) * (code - 32).
 *   block_q8_K (292 B): f32 d, i8 qs[256], i16 bsums[16]: the activation
 *       format the CPU path quantizes x into before the dot products
 *       (quantize_row_q8_K_ref: iscale = -127/max where max is the first
 *       element of largest magnitude, q = min(127, nearest_int(iscale*x)),
 *       d = 1/iscale, bsums = sums of 16 consecutive q; all-zero block: d = 0).
 *   ggml_vec_dot_q4_K_q8_K / _q6_K_q8_K (generic): per block, integer sums
 *       of scale * q_w * q_x into eight lanes aux32[l] (element index mod 8),
 *       then sums[l] += (fp16(d) * d_x) * aux32[l]; Q4_K also subtracts
 *       (fp16(dmin) * d_x) * sum_j m_j * (bsums[2j] + bsums[2j+1]) from sumf;
 *       finally sumf += sums[0..7].
 *   ggml rms_norm (f32): the sum of x*x (f32 products) accumulated in double,
 *       mean = (float)(sum / n), scale = 1/sqrtf(mean + eps), y = x * scale.
 *
 *   block_q8_0 (34 B): fp16 d, i8 qs[32].  Value = d * q.  A Q8_0 file
 *       (src/voxtral-quantize.cpp:95-96) stores every matrix so; its
 *       products take a q8_0 activation (Q8_0's vec_dot_type), quantized by
 *       quantize_row_q8_0 as the x86 CPU backend compiles it (the AVX/AVX2
 *       branch: amax = max |x| of the 32 elements, d = amax / 127 stored as
 *       fp16 with F16C's round to nearest even, id = amax ? 127 / amax : 0,
 *       q = round half to even (x * id)); the portable
 *       quantize_row_q8_0_ref, which the q8_0 KV rows follow, takes
 *       id = 1 / d and rounds half away from zero instead.
 *   ggml_vec_dot_q8_0_q8_0 (x86 AVX2 branch): per block, d = fp16(d_w) *
 *       fp16(d_x) in f32; eight f32 lanes, lane k holding the exact integer
 *       sum of the products of elements 4k .. 4k+3, accumulate
 *       acc[k] = fma(d, sum_k, acc[k]) over the row's blocks; the row's value
 *       is ((acc0 + acc4) + (acc2 + acc6)) + ((acc1 + acc5) + (acc3 + acc7)).
 *
 * Pinned by tests/test_kquants.py: pack/unpack round trips of constructed
 * blocks against the formulas above, the integer dot products against fp64
 * dots of the dequantized operands, and closed forms of the Q8_K and q8_0
 * activation quantizers (extreme element to -127 / +-127, tie to the first
 * occurrence, half-way codes to even, error <= d/2).  No ggml output is
 * available offline, so bitwise agreement with ggml's own binaries (the f32
 * order of the per-block sums) is parity unpinned.
 */
#include "vkv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 256

static float h2f(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | p[1] << 8)); }

/* 6-bit scale and min of sub-block j (0..7) of a Q4_K block's scales[12] */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* 4-bit code of element e (0..255) of a Q4_K block */
static int q4k_code(const uint8_t *blk, int e) {
    const uint8_t *qs = blk + 16;
    const int j = e / 32, l = e % 32;
    const uint8_t b = qs[32 * (j / 2) + l];
    return (j & 1) ? (b >> 4) : (b & 15);
}

/* 6-bit code (0..63) and scale of element e of a Q6_K block */
static int q6k_code(const uint8_t *blk, int e, int *scale) {
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    const int n = e / 128, g = (e % 128) / 32, l = e % 32;
    const uint8_t lo = ql[64 * n + 32 * (g & 1) + l];
    const int nib = (g < 2) ? (lo & 15) : (lo >> 4);
    *scale = sc[8 * n + 2 * g + l / 16];
    return nib | (((qh[32 * n + l] >> (2 * g)) & 3) << 4);
}

void orc_q4_k_dequantize(const uint8_t *blocks, float *y, int64_t n) {
    for (int64_t b = 0; b < n / QK; ++b) {
        const uint8_t *blk = blocks + b * 144;
        const float d = h2f(blk), dmin = h2f(blk + 2);
        for (int e = 0; e < QK; ++e) {
            int sc, m;
            q4k_scale_min(blk + 4, e / 32, &sc, &m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            y[b * QK + e] = d1 * (float)q4k_code(blk, e) - m1;
        }
    }
}

void orc_q6_k_dequantize(const uint8_t *blocks, float *y, int64_t n) {
    for (int64_t b = 0; b < n / QK; ++b) {
        const uint8_t *blk = blocks + b * 210;
        const float d = h2f(blk + 208);
        for (int e = 0; e < QK; ++e) {
            int sc;
            const int q = q6k_code(blk, e, &sc) - 32;
            y[b * QK + e] = d * (float)sc * (float)q;
        }
    }
}

/* ggml nearest_int: add 1.5*2^23 and read the mantissa, i.e. round half to
 * even for |v| < 2^22 */
static int nearest_int(float v) {
    const float t = v + 12582912.0f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

void orc_q8_k_quantize(const float *x, uint8_t *blocks, int64_t n) {
    for (int64_t b = 0; b < n / QK; ++b) {
        const float *xb = x + b * QK;
        uint8_t *blk = blocks + b * 292;
        int8_t *qs = (int8_t *)(blk + 4);
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(qs, 0, QK);
        } else {
            const float iscale = -127.0f / max;
            for (int j = 0; j < QK; ++j) {
                const int v = nearest_int(iscale * xb[j]);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            d = 1.0f / iscale;
        }
        memcpy(blk, &d, 4);
        for (int j = 0; j < QK / 16; ++j) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += qs[16 * j + i];
            const int16_t s16 = (int16_t)s;
            memcpy(blk + 260 + 2 * j, &s16, 2);
        }
    }
}

void orc_q8_k_dequantize(const uint8_t *blocks, float *y, int64_t n) {
    for (int64_t b = 0; b < n / QK; ++b) {
        const uint8_t *blk = blocks + b * 292;
        float d;
        memcpy(&d, blk, 4);
        for (int e = 0; e < QK; ++e) y[b * QK + e] = d * (float)((const int8_t *)(blk + 4))[e];
    }
}

static float q8k_d(const uint8_t *blk) { float d; memcpy(&d, blk, 4); return d; }
static int q8k_bsum(const uint8_t *blk, int j) {
    int16_t s;
    memcpy(&s, blk + 260 + 2 * j, 2);
    return s;
}

float orc_vec_dot_q4_k_q8_k(int64_t n, const uint8_t *w, const uint8_t *x) {
    float sums[8] = {0}, sumf = 0.0f;
    for (int64_t b = 0; b < n / QK; ++b) {
        const uint8_t *wb = w + b * 144, *xb = x + b * 292;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        int32_t aux32[8] = {0};
        int summ = 0;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(wb + 4, j, &sc, &m);
            summ += m * (q8k_bsum(xb, 2 * j) + q8k_bsum(xb, 2 * j + 1));
            for (int l = 0; l < 32; ++l) {
                const int e = 32 * j + l;
                aux32[e % 8] += sc * (int16_t)(q8[e] * q4k_code(wb, e));
            }
        }
        const float dx = q8k_d(xb);
        const float d = h2f(wb) * dx;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        const float dmin = h2f(wb + 2) * dx;
        sumf -= dmin * (float)summ;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

float orc_vec_dot_q6_k_q8_k(int64_t n, const uint8_t *w, const uint8_t *x) {
    float sums[8] = {0}, sumf = 0.0f;
    for (int64_t b = 0; b < n / QK; ++b) {
        const uint8_t *wb = w + b * 210, *xb = x + b * 292;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        int32_t aux32[8] = {0};
        for (int e = 0; e < QK; ++e) {
            int sc;
            const int q = q6k_code(wb, e, &sc) - 32;
            aux32[e % 8] += sc * (int16_t)(q8[e] * q);
        }
        const float d = h2f(wb + 208) * q8k_d(xb);
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

void orc_q8_0_quantize_x86(const float *x, uint8_t *blocks, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *xb = x + b * 32;
        uint8_t *blk = blocks + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        memcpy(blk, &dh, 2);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < 32; ++j) {
            const int8_t q = (int8_t)nearest_int(xb[j] * id);
            memcpy(blk + 2 + j, &q, 1);
        }
    }
}

float orc_vec_dot_q8_0_q8_0(int64_t n, const uint8_t *w, const uint8_t *x) {
    float acc[8] = {0};
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *wb = w + b * 34, *xb = x + b * 34;
        const float d = h2f(wb) * h2f(xb);
        const int8_t *qw = (const int8_t *)(wb + 2), *qx = (const int8_t *)(xb + 2);
        for (int k = 0; k < 8; ++k) {
            int s = 0;
            for (int e = 4 * k; e < 4 * k + 4; ++e) s += qw[e] * qx[e];
            acc[k] = fmaf(d, (float)s, acc[k]);
        }
    }
    return ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
}

void orc_rms_norm(const float *x, float *y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * scale;
}

void orc_norm_act_b(const float *x, int64_t n, const float *norm_w, const float *norm_b,
                    const float *ada, float eps, float *y) {
    if (!norm_w) {
        memcpy(y, x, (size_t)n * sizeof(float));
        return;
    }
    orc_rms_norm(x, y, n, eps);
    for (int64_t i = 0; i < n; ++i) y[i] = y[i] * norm_w[i];
    if (norm_b) /* enc_apply_norm's bias (src/voxtral.cpp:1855-1861) */
        for (int64_t i = 0; i < n; ++i) y[i] = y[i] + norm_b[i];
    if (ada)
        for (int64_t i = 0; i < n; ++i) {
            const float t = y[i] * ada[i];
            y[i] = y[i] + t;
        }
}

void orc_norm_act(const float *x, int64_t n, const float *norm_w, const float *ada, float eps,
                  float *y) {
    orc_norm_act_b(x, n, norm_w, NULL, ada, eps, y);
}

float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* ggml_vec_argmax_f32: max = MAX(max, x[i]) with MAX(a, b) = a > b ? a : b,
 * and idx = i whenever max == x[i] (ggml_argmax, src/voxtral.cpp:2970) */
int32_t orc_argmax(const float *x, int64_t n) {
    float max = -INFINITY;
    int32_t idx = 0;
    for (int64_t i = 0; i < n; ++i) {
        max = max > x[i] ? max : x[i];
        if (max == x[i]) idx = (int32_t)i;
    }
    return idx;
}

int64_t orc_wrow_bytes(int dtype, int64_t n_in) {
    if (dtype == ORC_Q8_0) return (n_in / 32) * 34;
    return (n_in / QK) * (dtype == ORC_Q4_K ? 144 : dtype == ORC_Q6_K ? 210 : 292);
}

typedef struct {
    int dtype;
    const uint8_t *w;
    int64_t r0, r1, n_in;
    const uint8_t *xq;
    float *y;
} mv_job;

static void *mv_worker(void *p) {
    const mv_job *j = (const mv_job *)p;
    const int64_t rb = orc_wrow_bytes(j->dtype, j->n_in);
    for (int64_t r = j->r0; r < j->r1; ++r)
        j->y[r] = j->dtype == ORC_Q4_K   ? orc_vec_dot_q4_k_q8_k(j->n_in, j->w + r * rb, j->xq)
                  : j->dtype == ORC_Q8_0 ? orc_vec_dot_q8_0_q8_0(j->n_in, j->w + r * rb, j->xq)
                                         : orc_vec_dot_q6_k_q8_k(j->n_in, j->w + r * rb, j->xq);
    return NULL;
}

/* ggml_mul_mat(W, x) on the CPU path: x quantized once to the weight type's
 * vec_dot_type (Q8_K for Q4_K / Q6_K, q8_0 for Q8_0), then one vec_dot per
 * row of W; rows are split over n_threads */
void orc_matvec(int dtype, const uint8_t *w, int64_t n_rows, int64_t n_in, const float *x,
                float *y, int n_threads) {
    uint8_t *xq = (uint8_t *)malloc(dtype == ORC_Q8_0 ? (size_t)(n_in / 32) * 34
                                                      : (size_t)(n_in / QK) * 292);
    if (dtype == ORC_Q8_0) orc_q8_0_quantize_x86(x, xq, n_in);
    else orc_q8_k_quantize(x, xq, n_in);
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    mv_job jobs[64];
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (mv_job){dtype, w, n_rows * t / n_threads, n_rows * (t + 1) / n_threads, n_in,
                           xq, y};
        if (n_threads == 1) mv_worker(&jobs[t]);
        else pthread_create(&th[t], NULL, mv_worker, &jobs[t]);
    }
    if (n_threads > 1)
        for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
    free(xq);
}
