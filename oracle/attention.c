/*
 * Oracle: attention over the KV cache (TEST INFRASTRUCTURE ONLY).
 *
 * orc_decode_attn_f64   -- exact single-query GQA attention,
 *                          out[h] = sum_j softmax_j(scale*q_h.k_{j,h/g}) v_{j,h/g},
 *                          over the listed slots (src/voxtral.cpp:2716-2854:
 *                          reusable-graph, one-segment, physical-full, logical
 *                          gather and manual split-score variants all compute
 *                          this function; they differ only in slot order).
 *                          K/V are read exactly from the stored dtype.
 * orc_decode_attn_mimic -- the same function in the reduction order of ggml's
 *                          CPU flash attention, which the reference reaches via
 *                          ggml_flash_attn_ext (src/voxtral.cpp:2759): Q is
 *                          converted to K's dot type (f16 for F16 K, q8_0 blocks
 *                          for Q8_0 K), keys are visited in order with a per-key
 *                          online softmax, and an F16 V is accumulated in f16.
 *                          ggml is not vendored (CMakeLists.txt:81-95), so this
 *                          reduction order is restated, not imported.
 * orc_decode_attn_mimic_acc32 -- orc_decode_attn_mimic with an f32 V
 *                          accumulator: ggml's reduction with every rounding
 *                          but the f16 accumulator (the one ggml applies to an
 *                          F32 V, ggml_vec_mad_f32 into VKQ32).
 * orc_window_attn_f64   -- multi-query attention with the causal sliding-window
 *                          predicate of voxtral_enc_kv_mask_allows
 *                          (src/voxtral.cpp:3636-3638, mask build :4259-4279)
 *                          or the causal prefill mask (src/voxtral.cpp:3316-3323).
 * orc_window_attn_mimic -- the same function in the arithmetic of the
 *                          reference's encoder graph on ggml's CPU backend:
 *                          below 32 query rows the segmented manual path
 *                          (src/voxtral.cpp:2201-2284: ggml_mul_mat of each
 *                          K segment with the query, which ggml converts to
 *                          f16 for an F16 K; ggml_soft_max_ext in f32 at the
 *                          scale with the -inf mask; ggml_mul_mat of each V^T
 *                          segment with its slice of the weights, converted
 *                          to f16 for an F16 V; the segments' f32 sums added
 *                          in order), from 32 rows the flash path with the
 *                          window gathered (:2285-2350), i.e. the decode
 *                          mimic over each query's allowed keys.
 * orc_decode_step_mimic_mt -- the CPU baseline: one decode step of every layer
 *                          (append of the new K/V row, then attention over
 *                          slots [0, n_valid)) threaded over query heads within
 *                          a layer, as ggml's CPU backend splits rows.
 * orc_decode_step_simd_mt  -- the same step with orc_simd_head (attention_simd.c:
 *                          AVX2/FMA/F16C lanes, the mimic's roundings).
 */
#include "vkv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static void orc_load_row(int dtype, const uint8_t *layer, int64_t row_bytes, int32_t slot,
                         int32_t elem0, int32_t n, float *dst) {
    const uint8_t *row = layer + (int64_t)slot * row_bytes;
    if (dtype == ORC_F32) {
        memcpy(dst, row + (int64_t)elem0 * 4, (size_t)n * 4);
    } else if (dtype == ORC_F16) {
        orc_f16_to_f32_n((const uint16_t *)(row + (int64_t)elem0 * 2), dst, n);
    } else {
        orc_q8_0_dequantize(row + (int64_t)(elem0 / 32) * 34, dst, n);
    }
}

void orc_decode_attn_f64(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                         int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                         const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                         int32_t head_dim, double scale, double *out) {
    int32_t group = n_q_heads / n_kv_heads;
    double *s = (double *)malloc(sizeof(double) * (size_t)(n_slots > 0 ? n_slots : 1));
    float *kr = (float *)malloc(sizeof(float) * (size_t)head_dim);
    for (int32_t h = 0; h < n_q_heads; ++h) {
        int32_t g = h / group;
        const float *qh = q + (int64_t)h * head_dim;
        double m = -INFINITY;
        for (int32_t j = 0; j < n_slots; ++j) {
            orc_load_row(dtype, k_layer, row_bytes, slots[j], g * head_dim, head_dim, kr);
            double acc = 0.0;
            for (int32_t d = 0; d < head_dim; ++d) acc += (double)qh[d] * (double)kr[d];
            s[j] = acc * scale;
            if (s[j] > m) m = s[j];
        }
        double l = 0.0;
        double *oh = out + (int64_t)h * head_dim;
        for (int32_t d = 0; d < head_dim; ++d) oh[d] = 0.0;
        for (int32_t j = 0; j < n_slots; ++j) {
            double p = exp(s[j] - m);
            l += p;
            orc_load_row(dtype, v_layer, row_bytes, slots[j], g * head_dim, head_dim, kr);
            for (int32_t d = 0; d < head_dim; ++d) oh[d] += p * (double)kr[d];
        }
        for (int32_t d = 0; d < head_dim; ++d) oh[d] = l > 0.0 ? oh[d] / l : 0.0;
    }
    free(kr);
    free(s);
}

/* ggml vec_dot of an F16 K row with the f16-rounded query: products of two
 * binary16 values are exact in f32 and are summed in double. */
static float orc_dot_f16(const uint16_t *k, const uint16_t *qh, int32_t n) {
    double sum = 0.0;
    for (int32_t i = 0; i < n; ++i)
        sum += (double)(orc_f16_to_f32(k[i]) * orc_f16_to_f32(qh[i]));
    return (float)sum;
}

/* ggml q8_0 x q8_0 dot: integer block sums scaled by d_k*d_q. */
static float orc_dot_q8_0(const uint8_t *kb, const uint8_t *qb, int32_t n) {
    float sum = 0.0f;
    for (int32_t b = 0; b < n / 32; ++b) {
        const uint8_t *x = kb + b * 34;
        const uint8_t *y = qb + b * 34;
        uint16_t dx, dy;
        memcpy(&dx, x, 2);
        memcpy(&dy, y, 2);
        int32_t sumi = 0;
        for (int j = 0; j < 32; ++j) sumi += (int32_t)(int8_t)x[2 + j] * (int32_t)(int8_t)y[2 + j];
        sum += (float)sumi * (orc_f16_to_f32(dx) * orc_f16_to_f32(dy));
    }
    return sum;
}

static void orc_mimic_head(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                           int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                           int32_t first_slot, const float *qh, int32_t g, int32_t head_dim,
                           float scale, int acc16, float *oh) {
    uint16_t qf16[512];
    uint8_t qq8[16 * 34];
    uint16_t vkq16[512];
    float vkq32[512];
    float vrow[512];
    if (dtype == ORC_F16) orc_f32_to_f16_n(qh, qf16, head_dim);
    if (dtype == ORC_Q8_0) orc_q8_0_quantize(qh, qq8, head_dim);
    for (int32_t d = 0; d < head_dim; ++d) { vkq16[d] = 0; vkq32[d] = 0.0f; }
    float S = 0.0f, M = -INFINITY;
    for (int32_t j = 0; j < n_slots; ++j) {
        int32_t slot = slots ? slots[j] : first_slot + j;
        const uint8_t *krow = k_layer + (int64_t)slot * row_bytes;
        const uint8_t *vrow_p = v_layer + (int64_t)slot * row_bytes;
        float s;
        if (dtype == ORC_F16) {
            s = orc_dot_f16((const uint16_t *)krow + (int64_t)g * head_dim, qf16, head_dim);
        } else if (dtype == ORC_Q8_0) {
            s = orc_dot_q8_0(krow + (int64_t)(g * head_dim / 32) * 34, qq8, head_dim);
        } else {
            const float *kf = (const float *)krow + (int64_t)g * head_dim;
            double acc = 0.0;
            for (int32_t d = 0; d < head_dim; ++d) acc += (double)(kf[d] * qh[d]);
            s = (float)acc;
        }
        s = s * scale;
        float Mold = M, ms = 1.0f, vs = 1.0f;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            if (acc16) {
                for (int32_t d = 0; d < head_dim; ++d)
                    vkq16[d] = orc_f32_to_f16(orc_f16_to_f32(vkq16[d]) * ms);
            } else {
                for (int32_t d = 0; d < head_dim; ++d) vkq32[d] *= ms;
            }
        } else {
            vs = expf(s - M);
        }
        if (acc16) {
            const uint16_t *vh = (const uint16_t *)vrow_p + (int64_t)g * head_dim;
            for (int32_t d = 0; d < head_dim; ++d)
                vkq16[d] = orc_f32_to_f16(fmaf(orc_f16_to_f32(vh[d]), vs, orc_f16_to_f32(vkq16[d])));
        } else {
            orc_load_row(dtype, v_layer, row_bytes, slot, g * head_dim, head_dim, vrow);
            for (int32_t d = 0; d < head_dim; ++d) vkq32[d] = fmaf(vrow[d], vs, vkq32[d]);
        }
        S = S * ms + vs;
    }
    if (acc16)
        for (int32_t d = 0; d < head_dim; ++d) vkq32[d] = orc_f16_to_f32(vkq16[d]);
    float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int32_t d = 0; d < head_dim; ++d) oh[d] = vkq32[d] * S_inv;
}

void orc_decode_attn_mimic(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                           int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                           const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                           int32_t head_dim, float scale, float *out) {
    int32_t group = n_q_heads / n_kv_heads;
    for (int32_t h = 0; h < n_q_heads; ++h)
        orc_mimic_head(dtype, k_layer, v_layer, row_bytes, slots, n_slots, 0,
                       q + (int64_t)h * head_dim, h / group, head_dim, scale,
                       dtype == ORC_F16, out + (int64_t)h * head_dim);
}

void orc_decode_attn_mimic_acc32(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                                 int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                                 const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, float scale, float *out) {
    int32_t group = n_q_heads / n_kv_heads;
    for (int32_t h = 0; h < n_q_heads; ++h)
        orc_mimic_head(dtype, k_layer, v_layer, row_bytes, slots, n_slots, 0,
                       q + (int64_t)h * head_dim, h / group, head_dim, scale, 0,
                       out + (int64_t)h * head_dim);
}

void orc_window_attn_f64(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                         int64_t row_bytes, const int32_t *k_slot, const int64_t *k_pos,
                         int32_t n_keys, const float *q, const int64_t *q_pos, int32_t n_q,
                         int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t window, double scale, double *out) {
    int32_t group = n_q_heads / n_kv_heads;
    double *s = (double *)malloc(sizeof(double) * (size_t)(n_keys > 0 ? n_keys : 1));
    float *kr = (float *)malloc(sizeof(float) * (size_t)head_dim);
    for (int32_t i = 0; i < n_q; ++i) {
        for (int32_t h = 0; h < n_q_heads; ++h) {
            int32_t g = h / group;
            const float *qh = q + ((int64_t)i * n_q_heads + h) * head_dim;
            double *oh = out + ((int64_t)i * n_q_heads + h) * head_dim;
            double m = -INFINITY;
            for (int32_t j = 0; j < n_keys; ++j) {
                int allowed = k_pos[j] <= q_pos[i] &&
                              (window <= 0 || k_pos[j] >= q_pos[i] - (int64_t)(window - 1));
                if (!allowed) { s[j] = -INFINITY; continue; }
                orc_load_row(dtype, k_layer, row_bytes, k_slot[j], g * head_dim, head_dim, kr);
                double acc = 0.0;
                for (int32_t d = 0; d < head_dim; ++d) acc += (double)qh[d] * (double)kr[d];
                s[j] = acc * scale;
                if (s[j] > m) m = s[j];
            }
            for (int32_t d = 0; d < head_dim; ++d) oh[d] = 0.0;
            double l = 0.0;
            for (int32_t j = 0; j < n_keys; ++j) {
                if (s[j] == -INFINITY) continue;
                double p = exp(s[j] - m);
                l += p;
                orc_load_row(dtype, v_layer, row_bytes, k_slot[j], g * head_dim, head_dim, kr);
                for (int32_t d = 0; d < head_dim; ++d) oh[d] += p * (double)kr[d];
            }
            for (int32_t d = 0; d < head_dim; ++d) oh[d] = l > 0.0 ? oh[d] / l : 0.0;
        }
    }
    free(kr);
    free(s);
}

static int orc_key_allowed(int64_t kp, int64_t qp, int32_t window) {
    return kp <= qp && (window <= 0 || kp >= qp - (int64_t)(window - 1));
}

int orc_window_attn_mimic(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                          int64_t row_bytes, const int32_t *k_slot, const int64_t *k_pos,
                          int32_t n_keys, int32_t new_start, const float *q,
                          const int64_t *q_pos, int32_t n_q, int32_t n_q_heads,
                          int32_t n_kv_heads, int32_t head_dim, int32_t window, float scale,
                          int flash, float *out) {
    /* The reference's encoder ring is F16 or F32 (src/voxtral.cpp:82-92). */
    if ((dtype != ORC_F16 && dtype != ORC_F32) || head_dim > 512 || n_keys < 0) return -1;
    int32_t group = n_q_heads / n_kv_heads;
    size_t nk = (size_t)(n_keys > 0 ? n_keys : 1);
    float *w = (float *)malloc(sizeof(float) * nk);
    int32_t *allowed = (int32_t *)malloc(sizeof(int32_t) * nk);
    for (int32_t i = 0; i < n_q; ++i) {
        for (int32_t h = 0; h < n_q_heads; ++h) {
            int32_t g = h / group;
            const float *qh = q + ((int64_t)i * n_q_heads + h) * head_dim;
            float *oh = out + ((int64_t)i * n_q_heads + h) * head_dim;
            if (flash) {
                /* :2347-2349: ggml_flash_attn_ext over the gathered window;
                 * masked keys (-inf) are skipped (ggml's CPU loop continues
                 * past them), so it is the decode mimic over the allowed keys
                 * in logical order. */
                int32_t na = 0;
                for (int32_t j = 0; j < n_keys; ++j)
                    if (orc_key_allowed(k_pos[j], q_pos[i], window)) allowed[na++] = k_slot[j];
                orc_mimic_head(dtype, k_layer, v_layer, row_bytes, allowed, na, 0, qh, g,
                               head_dim, scale, dtype == ORC_F16, oh);
                continue;
            }
            /* :2259-2266: scores = concat_s mul_mat(K_s, q).  ggml's CPU
             * mul_mat converts the f32 query to the weights' dot type (f16
             * for an F16 ring); products of two f16 values are exact in f32. */
            uint16_t q16[512];
            if (dtype == ORC_F16) orc_f32_to_f16_n(qh, q16, head_dim);
            /* :2268 soft_max_ext: w = s*scale + mask (0 or -inf), max, expf,
             * the sum in double, then every weight times the f32 of its
             * reciprocal. */
            float mx = -INFINITY;
            for (int32_t j = 0; j < n_keys; ++j) {
                if (!orc_key_allowed(k_pos[j], q_pos[i], window)) { w[j] = -INFINITY; continue; }
                const uint8_t *krow = k_layer + (int64_t)k_slot[j] * row_bytes;
                double acc = 0.0;
                if (dtype == ORC_F16) {
                    const uint16_t *kh = (const uint16_t *)krow + (int64_t)g * head_dim;
                    for (int32_t d = 0; d < head_dim; ++d)
                        acc += (double)(orc_f16_to_f32(kh[d]) * orc_f16_to_f32(q16[d]));
                } else {
                    const float *kf = (const float *)krow + (int64_t)g * head_dim;
                    for (int32_t d = 0; d < head_dim; ++d) acc += (double)(kf[d] * qh[d]);
                }
                w[j] = (float)acc * scale;
                if (w[j] > mx) mx = w[j];
            }
            double sum = 0.0;
            for (int32_t j = 0; j < n_keys; ++j) {
                float e = w[j] == -INFINITY ? 0.0f : expf(w[j] - mx);
                w[j] = e;
                sum += (double)e;
            }
            float inv = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
            for (int32_t j = 0; j < n_keys; ++j) w[j] *= inv;
            /* :2270-2281: per segment (maximal runs of consecutive ring
             * slots, and the new rows), mul_mat(V_s^T, weights_s): the
             * weights converted to f16 for an F16 V; the segments' f32
             * results added in order. */
            for (int32_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
            int32_t j0 = 0;
            while (j0 < n_keys) {
                int32_t j1 = j0 + 1;
                while (j1 < n_keys && j1 != new_start && k_slot[j1] == k_slot[j1 - 1] + 1) ++j1;
                for (int32_t d = 0; d < head_dim; ++d) {
                    double acc = 0.0;
                    for (int32_t j = j0; j < j1; ++j) {
                        const uint8_t *vrow = v_layer + (int64_t)k_slot[j] * row_bytes;
                        if (dtype == ORC_F16) {
                            float pw = orc_f16_to_f32(orc_f32_to_f16(w[j]));
                            float vv = orc_f16_to_f32(((const uint16_t *)vrow)[(int64_t)g * head_dim + d]);
                            acc += (double)(pw * vv);
                        } else {
                            acc += (double)(w[j] * ((const float *)vrow)[(int64_t)g * head_dim + d]);
                        }
                    }
                    oh[d] += (float)acc;
                }
                j0 = j1;
            }
        }
    }
    free(allowed);
    free(w);
    return 0;
}

/* ---- threaded CPU baseline ---- */

typedef struct orc_step_job {
    int dtype;
    const uint8_t *k_cache, *v_cache;
    int64_t layer_bytes, row_bytes;
    int32_t n_layers, n_valid, n_q_heads, n_kv_heads, head_dim, n_threads;
    const float *q;
    float scale;
    float *out;
    const float *k_new, *v_new;
    int32_t new_slot;
    pthread_barrier_t *barrier;
    int32_t ith;
    int simd;
} orc_step_job;

static void *orc_step_worker(void *arg) {
    orc_step_job *j = (orc_step_job *)arg;
    int32_t group = j->n_q_heads / j->n_kv_heads;
    int32_t dr = (j->n_q_heads + j->n_threads - 1) / j->n_threads;
    int32_t h0 = dr * j->ith;
    int32_t h1 = h0 + dr < j->n_q_heads ? h0 + dr : j->n_q_heads;
    for (int32_t l = 0; l < j->n_layers; ++l) {
        const uint8_t *kl = j->k_cache + (int64_t)l * j->layer_bytes;
        const uint8_t *vl = j->v_cache + (int64_t)l * j->layer_bytes;
        const float *ql = j->q + (int64_t)l * j->n_q_heads * j->head_dim;
        float *ol = j->out + (int64_t)l * j->n_q_heads * j->head_dim;
        if (j->k_new) {
            /* append (src/voxtral.cpp:2682-2694) precedes the layer's attention */
            int32_t kv_dim = j->n_kv_heads * j->head_dim;
            if (j->ith == 0) {
                orc_seg seg = {j->new_slot, 1};
                orc_append(j->dtype, (uint8_t *)kl, j->row_bytes, kv_dim, &seg, 1,
                           j->k_new + (int64_t)l * kv_dim);
                orc_append(j->dtype, (uint8_t *)vl, j->row_bytes, kv_dim, &seg, 1,
                           j->v_new + (int64_t)l * kv_dim);
            }
            pthread_barrier_wait(j->barrier);
        }
        for (int32_t h = h0; h < h1; ++h) {
            if (j->simd)
                orc_simd_head(j->dtype, kl, vl, j->row_bytes, j->n_valid,
                              ql + (int64_t)h * j->head_dim, h / group, j->head_dim, j->scale,
                              ol + (int64_t)h * j->head_dim);
            else
                orc_mimic_head(j->dtype, kl, vl, j->row_bytes, NULL, j->n_valid, 0,
                               ql + (int64_t)h * j->head_dim, h / group, j->head_dim, j->scale,
                               j->dtype == ORC_F16, ol + (int64_t)h * j->head_dim);
        }
        pthread_barrier_wait(j->barrier);   /* one graph node per layer */
    }
    return NULL;
}

static double orc_decode_step_mt(int simd, int dtype, const uint8_t *k_cache,
                                 const uint8_t *v_cache, int64_t layer_bytes, int64_t row_bytes,
                                 int32_t n_layers, int32_t n_valid, const float *q,
                                 int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                 float scale, float *out, const float *k_new, const float *v_new,
                                 int32_t new_slot, int32_t n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t tid[64];
    orc_step_job jobs[64];
    pthread_barrier_t barrier;
    pthread_barrier_init(&barrier, NULL, (unsigned)n_threads);
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int32_t t = 0; t < n_threads; ++t) {
        orc_step_job jb = {dtype, k_cache, v_cache, layer_bytes, row_bytes, n_layers, n_valid,
                           n_q_heads, n_kv_heads, head_dim, n_threads, q, scale, out, k_new, v_new,
                           new_slot, &barrier, t, simd};
        jobs[t] = jb;
        if (t > 0) pthread_create(&tid[t], NULL, orc_step_worker, &jobs[t]);
    }
    orc_step_worker(&jobs[0]);
    for (int32_t t = 1; t < n_threads; ++t) pthread_join(tid[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    pthread_barrier_destroy(&barrier);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

double orc_decode_step_mimic_mt(int dtype, const uint8_t *k_cache, const uint8_t *v_cache,
                                int64_t layer_bytes, int64_t row_bytes, int32_t n_layers,
                                int32_t n_valid, const float *q, int32_t n_q_heads,
                                int32_t n_kv_heads, int32_t head_dim, float scale,
                                float *out, const float *k_new, const float *v_new,
                                int32_t new_slot, int32_t n_threads) {
    return orc_decode_step_mt(0, dtype, k_cache, v_cache, layer_bytes, row_bytes, n_layers,
                              n_valid, q, n_q_heads, n_kv_heads, head_dim, scale, out, k_new,
                              v_new, new_slot, n_threads);
}

double orc_decode_step_simd_mt(int dtype, const uint8_t *k_cache, const uint8_t *v_cache,
                               int64_t layer_bytes, int64_t row_bytes, int32_t n_layers,
                               int32_t n_valid, const float *q, int32_t n_q_heads,
                               int32_t n_kv_heads, int32_t head_dim, float scale,
                               float *out, const float *k_new, const float *v_new,
                               int32_t new_slot, int32_t n_threads) {
    if (!orc_simd_available() || head_dim % 32 || head_dim > 512) return -1.0;
    return orc_decode_step_mt(1, dtype, k_cache, v_cache, layer_bytes, row_bytes, n_layers,
                              n_valid, q, n_q_heads, n_kv_heads, head_dim, scale, out, k_new,
                              v_new, new_slot, n_threads);
}
