/*
 * Oracle: the CPU baseline's vector leg (TEST INFRASTRUCTURE ONLY).
 *
 * orc_simd_head -- one query head of ggml's CPU flash-attention decode step
 *                  (the path the reference reaches via ggml_flash_attn_ext,
 *                  src/voxtral.cpp:2759) written the way ggml's x86 build runs
 *                  it with AVX2 + FMA + F16C: the K-row dot as four 8-wide f32
 *                  FMA accumulators over f16-converted lanes (ggml_vec_dot_f16's
 *                  32-element step), q8_0 x q8_0 block dots as exact 16-bit
 *                  pair sums widened to 8 i32 lanes and scaled into an 8-wide
 *                  f32 accumulator, and the V accumulator kept in f16 and
 *                  re-rounded after every key for an F16 cache
 *                  (ggml_vec_mad_f16 / ggml_vec_scale_f16 through F16C).
 *                  The roundings the scalar mimic pins (f16-rounded Q for F16
 *                  K, q8_0 Q for q8_0 K, the per-key f16 V accumulator, the
 *                  per-key online softmax) are the same; only the order of the
 *                  K-row sums differs (8 lanes x 4 accumulators against one
 *                  double sum).  ggml itself is not vendored (CMakeLists.txt:
 *                  81-95), so this is a restatement of its published
 *                  algorithm, used to time a vectorised CPU step.
 */
#include "vkv_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>

static inline float orc_hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
    return _mm_cvtss_f32(lo);
}

/* four accumulators of 8 lanes, folded pairwise, then across lanes */
static inline float orc_reduce4(__m256 s0, __m256 s1, __m256 s2, __m256 s3) {
    return orc_hsum8(_mm256_add_ps(_mm256_add_ps(s0, s2), _mm256_add_ps(s1, s3)));
}

static float orc_dot_f16_simd(const uint16_t *k, const float *q, int32_t n) {
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    for (int32_t i = 0; i < n; i += 32) {
        s0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + i))),
                             _mm256_loadu_ps(q + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + i + 8))),
                             _mm256_loadu_ps(q + i + 8), s1);
        s2 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + i + 16))),
                             _mm256_loadu_ps(q + i + 16), s2);
        s3 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + i + 24))),
                             _mm256_loadu_ps(q + i + 24), s3);
    }
    return orc_reduce4(s0, s1, s2, s3);
}

static float orc_dot_f32_simd(const float *k, const float *q, int32_t n) {
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    for (int32_t i = 0; i < n; i += 32) {
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(k + i), _mm256_loadu_ps(q + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(k + i + 8), _mm256_loadu_ps(q + i + 8), s1);
        s2 = _mm256_fmadd_ps(_mm256_loadu_ps(k + i + 16), _mm256_loadu_ps(q + i + 16), s2);
        s3 = _mm256_fmadd_ps(_mm256_loadu_ps(k + i + 24), _mm256_loadu_ps(q + i + 24), s3);
    }
    return orc_reduce4(s0, s1, s2, s3);
}

/* q8_0 x q8_0: per block the 32 int8 products summed exactly (|x| * sign(y, x)
 * as u8 x i8 pairs into i16, pairs of i16 into 8 i32 lanes), converted to f32
 * and scaled by d_k d_q into an 8-lane accumulator */
static float orc_dot_q8_0_simd(const uint8_t *kb, const uint8_t *qb, int32_t n) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int32_t b = 0; b < n / 32; ++b) {
        const uint8_t *x = kb + b * 34, *y = qb + b * 34;
        uint16_t dx, dy;
        memcpy(&dx, x, 2);
        memcpy(&dy, y, 2);
        const __m256i qx = _mm256_loadu_si256((const __m256i *)(x + 2));
        const __m256i qy = _mm256_loadu_si256((const __m256i *)(y + 2));
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i p16 = _mm256_maddubs_epi16(ax, sy);
        const __m256 p = _mm256_cvtepi32_ps(_mm256_madd_epi16(p16, ones));
        const __m256 d = _mm256_set1_ps(orc_f16_to_f32(dx) * orc_f16_to_f32(dy));
        acc = _mm256_fmadd_ps(d, p, acc);
    }
    return orc_hsum8(acc);
}

/* y (f16) = y * s, through f32 */
static void orc_scale_f16_simd(uint16_t *y, float s, int32_t n) {
    const __m256 vs = _mm256_set1_ps(s);
    for (int32_t i = 0; i < n; i += 8) {
        const __m256 a = _mm256_mul_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i))), vs);
        _mm_storeu_si128((__m128i *)(y + i), _mm256_cvtps_ph(a, _MM_FROUND_TO_NEAREST_INT));
    }
}

/* y (f16) = y + x (f16) * s, through f32, rounded to f16 */
static void orc_mad_f16_simd(uint16_t *y, const uint16_t *x, float s, int32_t n) {
    const __m256 vs = _mm256_set1_ps(s);
    for (int32_t i = 0; i < n; i += 8) {
        const __m256 a = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i))),
                                         vs, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i))));
        _mm_storeu_si128((__m128i *)(y + i), _mm256_cvtps_ph(a, _MM_FROUND_TO_NEAREST_INT));
    }
}

static void orc_mad_f32_simd(float *y, const float *x, float s, int32_t n) {
    const __m256 vs = _mm256_set1_ps(s);
    for (int32_t i = 0; i < n; i += 8)
        _mm256_storeu_ps(y + i, _mm256_fmadd_ps(_mm256_loadu_ps(x + i), vs, _mm256_loadu_ps(y + i)));
}

static void orc_scale_f32_simd(float *y, float s, int32_t n) {
    const __m256 vs = _mm256_set1_ps(s);
    for (int32_t i = 0; i < n; i += 8) _mm256_storeu_ps(y + i, _mm256_mul_ps(_mm256_loadu_ps(y + i), vs));
}

/* a q8_0 row segment of n elements to f32 (d * code, 8 lanes at a time) */
static void orc_q8_0_to_f32_simd(const uint8_t *blocks, float *dst, int32_t n) {
    for (int32_t b = 0; b < n / 32; ++b) {
        const uint8_t *x = blocks + b * 34;
        uint16_t dh;
        memcpy(&dh, x, 2);
        const __m256 d = _mm256_set1_ps(orc_f16_to_f32(dh));
        for (int j = 0; j < 32; j += 8) {
            const __m256i c = _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(x + 2 + j)));
            _mm256_storeu_ps(dst + b * 32 + j, _mm256_mul_ps(d, _mm256_cvtepi32_ps(c)));
        }
    }
}

int orc_simd_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
           __builtin_cpu_supports("f16c");
}

void orc_simd_head(int dtype, const uint8_t *k_layer, const uint8_t *v_layer, int64_t row_bytes,
                   int32_t n_slots, const float *qh, int32_t g, int32_t head_dim, float scale,
                   float *oh) {
    uint16_t qf16[512];
    float q32[512];
    uint8_t qq8[16 * 34];
    uint16_t vkq16[512];
    float vkq32[512];
    float vrow[512];
    if (dtype == ORC_F16) {
        orc_f32_to_f16_n(qh, qf16, head_dim);
        orc_f16_to_f32_n(qf16, q32, head_dim);
    } else if (dtype == ORC_Q8_0) {
        orc_q8_0_quantize(qh, qq8, head_dim);
    } else {
        memcpy(q32, qh, sizeof(float) * (size_t)head_dim);
    }
    memset(vkq16, 0, sizeof(uint16_t) * (size_t)head_dim);
    memset(vkq32, 0, sizeof(float) * (size_t)head_dim);
    float S = 0.0f, M = -INFINITY;
    for (int32_t j = 0; j < n_slots; ++j) {
        const uint8_t *krow = k_layer + (int64_t)j * row_bytes;
        const uint8_t *vrow_p = v_layer + (int64_t)j * row_bytes;
        float s;
        if (dtype == ORC_F16)
            s = orc_dot_f16_simd((const uint16_t *)krow + (int64_t)g * head_dim, q32, head_dim);
        else if (dtype == ORC_Q8_0)
            s = orc_dot_q8_0_simd(krow + (int64_t)(g * head_dim / 32) * 34, qq8, head_dim);
        else
            s = orc_dot_f32_simd((const float *)krow + (int64_t)g * head_dim, q32, head_dim);
        s = s * scale;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            const float Mold = M;
            M = s;
            ms = expf(Mold - M);
            if (dtype == ORC_F16) orc_scale_f16_simd(vkq16, ms, head_dim);
            else orc_scale_f32_simd(vkq32, ms, head_dim);
        } else {
            vs = expf(s - M);
        }
        if (dtype == ORC_F16) {
            orc_mad_f16_simd(vkq16, (const uint16_t *)vrow_p + (int64_t)g * head_dim, vs, head_dim);
        } else if (dtype == ORC_Q8_0) {
            orc_q8_0_to_f32_simd(vrow_p + (int64_t)(g * head_dim / 32) * 34, vrow, head_dim);
            orc_mad_f32_simd(vkq32, vrow, vs, head_dim);
        } else {
            orc_mad_f32_simd(vkq32, (const float *)vrow_p + (int64_t)g * head_dim, vs, head_dim);
        }
        S = S * ms + vs;
    }
    if (dtype == ORC_F16) orc_f16_to_f32_n(vkq16, vkq32, head_dim);
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int32_t d = 0; d < head_dim; ++d) oh[d] = vkq32[d] * S_inv;
}
