/*
 * Oracle: element formats, synthetic inputs and the cache image
 * (TEST INFRASTRUCTURE ONLY).
 *
 * F16: IEEE-754 binary16, round-to-nearest-even, overflow to +-Inf, gradual
 *      underflow.  This is what ggml's F32->F16 row conversion computes when
 *      ggml_set_rows / ggml_cpy write a projected F32 K/V row into the F16
 *      cache (src/voxtral.cpp:2682-2713 decoder, :2166-2185 encoder).  ggml is
 *      not vendored (fetched at 5cecdad6, CMakeLists.txt:81-95), so the rule is
 *      pinned here against numpy's astype(float16) and exhaustive/edge tests.
 * Q8_0: ggml block_q8_0 = { fp16 d; int8 qs[32] } (34 bytes).  q8_0 KV does
 *      not exist in the reference (src/voxtral.cpp:82-92 accepts only F16/F32);
 *      this build adopts ggml's reference-quantizer rule: amax = max|x|,
 *      d = amax/127, id = d ? 1/d : 0, qs = round-half-away(x*id), d stored as
 *      fp16(RNE).  Dequant: x = f32(d) * qs.
 * Synthetic N(0,1): integer Irwin-Hall (sum of twelve 16-bit uniforms from
 *      splitmix64), exactly representable in f32, so CPU and GPU agree bit for
 *      bit without any transcendental function.
 */
#include "vkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e == 0xffu) {
        if (m == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (m >> 13));   /* quiet NaN, top payload bits */
    }
    int32_t E = (int32_t)e - 127 + 15;                    /* binary16 biased exponent */
    if (E >= 31) return (uint16_t)(sign | 0x7c00u);       /* |f| >= 65536 */
    if (E <= 0) {
        /* result is subnormal (or rounds to the smallest normal / zero):
         * value = (m|2^23) * 2^(e-150); binary16 subnormal unit = 2^-24. */
        if (E < -10) return (uint16_t)sign;               /* |f| < 2^-25 */
        uint32_t mant = m | 0x800000u;
        uint32_t shift = (uint32_t)(14 - E);              /* 14..24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)E << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;   /* carry may reach Inf: correct */
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_f32_to_f16_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_n(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

/* round half away from zero, exact for |v| < 2^23 */
static float orc_round_half_away(float v) {
    float t = truncf(v);
    float r = v - t;   /* exact */
    if (r >= 0.5f) t += 1.0f;
    else if (r <= -0.5f) t -= 1.0f;
    return t;
}

void orc_q8_0_quantize(const float *x, uint8_t *blocks, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float *xb = x + b * 32;
        uint8_t *blk = blocks + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = orc_f32_to_f16(d);
        memcpy(blk, &dh, 2);
        for (int j = 0; j < 32; ++j) {
            float r = orc_round_half_away(xb[j] * id);
            int8_t q = (int8_t)(int)r;
            memcpy(blk + 2 + j, &q, 1);
        }
    }
}

void orc_q8_0_dequantize(const uint8_t *blocks, float *y, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = blocks + b * 34;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        float d = orc_f16_to_f32(dh);
        for (int j = 0; j < 32; ++j) {
            int8_t q;
            memcpy(&q, blk + 2 + j, 1);
            y[b * 32 + j] = (float)q * d;
        }
    }
}

int64_t orc_row_bytes(int dtype, int64_t n_elems) {
    switch (dtype) {
    case ORC_F32: return n_elems * 4;
    case ORC_F16: return n_elems * 2;
    case ORC_Q8_0: return (n_elems / 32) * 34;
    default: return -1;
    }
}

void orc_row_to_f32(int dtype, const void *row, float *y, int64_t n) {
    if (dtype == ORC_F32) memcpy(y, row, (size_t)n * 4);
    else if (dtype == ORC_F16) orc_f16_to_f32_n((const uint16_t *)row, y, n);
    else orc_q8_0_dequantize((const uint8_t *)row, y, n);
}

void orc_row_from_f32(int dtype, const float *x, void *row, int64_t n) {
    if (dtype == ORC_F32) memcpy(row, x, (size_t)n * 4);
    else if (dtype == ORC_F16) orc_f32_to_f16_n(x, (uint16_t *)row, n);
    else orc_q8_0_quantize(x, (uint8_t *)row, n);
}

/* splitmix64 output function (Steele, Lea & Flood, OOPSLA 2014) */
uint64_t orc_mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t orc_row_key(uint64_t seed, uint32_t tag, int64_t stream, int64_t layer, int64_t pos) {
    uint64_t k = orc_mix64(seed ^ ((uint64_t)tag << 32));
    k = orc_mix64(k ^ (uint64_t)stream);
    k = orc_mix64(k ^ (uint64_t)layer);
    return orc_mix64(k ^ (uint64_t)pos);
}

float orc_synth_value(uint64_t key, int64_t index) {
    uint64_t b = key ^ ((uint64_t)index * 0xD1B54A32D192ED03ull);
    int32_t s = 0;
    for (int k = 0; k < 3; ++k) {
        uint64_t h = orc_mix64(b + (uint64_t)k * 0x9E3779B97F4A7C15ull);
        s += (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
             (int32_t)((h >> 32) & 0xffffu) + (int32_t)(h >> 48);
    }
    return (float)(s - 393210) * (1.0f / 65536.0f);
}

void orc_synth_row(uint64_t key, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_synth_value(key, i);
}

/* src/voxtral.cpp:2696-2713: rows are laid down in logical order across the
 * write segments, each converted to the cache dtype once. */
void orc_append(int dtype, uint8_t *cache_layer, int64_t row_bytes, int32_t kv_dim,
                const orc_seg *write_seg, int32_t write_nseg, const float *src) {
    int64_t col = 0;
    for (int32_t s = 0; s < write_nseg; ++s) {
        for (int32_t i = 0; i < write_seg[s].len; ++i) {
            orc_row_from_f32(dtype, src + col * kv_dim,
                             cache_layer + (int64_t)(write_seg[s].slot + i) * row_bytes, kv_dim);
            ++col;
        }
    }
}

/* src/voxtral.cpp:2774-2799: logical window = concat(read_seg[0], read_seg[1]). */
void orc_gather(const uint8_t *cache_layer, int64_t row_bytes, const orc_seg *read_seg,
                int32_t read_nseg, uint8_t *dst) {
    int64_t off = 0;
    for (int32_t s = 0; s < read_nseg; ++s) {
        int64_t bytes = (int64_t)read_seg[s].len * row_bytes;
        memcpy(dst + off, cache_layer + (int64_t)read_seg[s].slot * row_bytes, (size_t)bytes);
        off += bytes;
    }
}

void orc_expected_layer(int dtype, uint8_t *dst, int64_t backing, int64_t capacity,
                        int32_t kv_dim, int64_t next, uint64_t seed, uint32_t tag,
                        int64_t stream, int64_t layer) {
    int64_t row_bytes = orc_row_bytes(dtype, kv_dim);
    float tmp[8192];
    memset(dst, 0, (size_t)(backing * row_bytes));
    if (next <= 0) return;
    int64_t last = next - 1;
    int64_t r = last % capacity;
    for (int64_t s = 0; s < capacity; ++s) {
        int64_t pos = last - ((r - s + capacity) % capacity);
        if (pos < 0) continue;
        orc_synth_row(orc_row_key(seed, tag, stream, layer, pos), tmp, kv_dim);
        orc_row_from_f32(dtype, tmp, dst + s * row_bytes, kv_dim);
    }
}

/* ggml's CPU rope, mode 0 (src/voxtral.cpp:2667-2671 -> ggml_rope_ext):
 * rope cache theta = p; theta *= theta_scale per pair; rotation
 * x0*cos - x1*sin, x0*sin + x1*cos.  The Makefile builds without contraction. */
void orc_rope_f32(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                  int64_t pos0, float theta) {
    const float theta_scale = powf(theta, -2.0f / (float)head_dim);
    const int32_t n_pairs = head_dim / 2;
    float *cs = (float *)malloc(sizeof(float) * 2 * (size_t)n_pairs);
    for (int64_t o = 0; o < n_outer; ++o) {
        for (int64_t r = 0; r < n_rows; ++r) {
            float th = (float)(pos0 + r);
            for (int32_t i = 0; i < n_pairs; ++i) {
                cs[2 * i] = (float)cos((double)th);
                cs[2 * i + 1] = (float)sin((double)th);
                th *= theta_scale;
            }
            float *row = x + (o * n_rows + r) * (int64_t)row_len;
            for (int32_t h0 = 0; h0 < row_len; h0 += head_dim) {
                for (int32_t i = 0; i < n_pairs; ++i) {
                    const float x0 = row[h0 + 2 * i], x1 = row[h0 + 2 * i + 1];
                    row[h0 + 2 * i] = x0 * cs[2 * i] - x1 * cs[2 * i + 1];
                    row[h0 + 2 * i + 1] = x0 * cs[2 * i + 1] + x1 * cs[2 * i];
                }
            }
        }
    }
    free(cs);
}
