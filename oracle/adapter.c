/*
 * Oracle: the realtime rows rings and the adapter (TEST INFRASTRUCTURE ONLY).
 *
 * The encoder-output ring ([capacity][1280] f32) and the audio-embedding ring
 * ([capacity][3072] f32) keep logical row r at row r % capacity
 * (src/voxtral.cpp:42-55, 1467-1485).  Writes follow
 * copy_chunk_to_enc_out_ring (:4018-4043): rows split at the wrap into
 * contiguous segments; reads follow read_realtime_ring_rows (:5530-5554).
 *
 * The adapter follows voxtral_ctx_adapter_commit (:5424-5485) and
 * build_adapter_ring_graph_reusable (:2589-2620): for group g, the encoder
 * rows (g * down + j) % enc_cap, j < down, are gathered (ggml_get_rows) and
 * read as one row of enc_dim * down floats; x = W0 row, gelu_erf, y = W2 h,
 * stored at audio row g % aemb_cap (ggml_set_rows).  Each product is
 * orc_matvec (the CPU mul_mat: input quantized to Q8_K, integer block dots).
 *
 * The decoder's ada time conditioning (build_decoder_layer :2864-2874):
 * scale = W2 gelu(W0 e(t)) with the time embedding of compute_time_embedding
 * (:729-740) evaluated as the reference does on the host; W0 through
 * orc_matvec, W2 (f16 [dim][ada_dim]) through ggml's f16 vec-dot: the input
 * rounded to f16, products summed in double (the generic path).  In a Q8_0
 * file W2 is Q8_0 too (its 32-wide rows are row-compatible with Q8_0,
 * src/voxtral-quantize.cpp:161-164, :410): then it is an orc_matvec as well.
 *
 * Pinned by tests/test_adapter.py: the gather against an independent index
 * rule (the 4-frame reshape of a contiguous run of encoder frames), the
 * products against fp64 products of the dequantized weights and the Q8_K
 * images, GELU against math.erf, the rings against a dictionary model of the
 * logical rows; the time embedding against fp64 cos/sin of the stated
 * frequencies, the ada scale against an fp64 composition of the dequantized
 * weights.
 */
#include "vkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int32_t orc_row_ring_write(float *ring, int32_t capacity, int32_t width, int64_t row_start,
                           const float *src, int32_t n_rows) {
    if (!ring || capacity < 1 || width < 1 || row_start < 0 || n_rows < 0 || n_rows > capacity)
        return -1;
    int32_t done = 0;
    while (done < n_rows) {
        const int32_t slot = (int32_t)((row_start + done) % capacity);
        int32_t seg = capacity - slot;
        if (seg > n_rows - done) seg = n_rows - done;
        memcpy(ring + (int64_t)slot * width, src + (int64_t)done * width,
               (size_t)seg * width * sizeof(float));
        done += seg;
    }
    return 0;
}

int32_t orc_row_ring_read(const float *ring, int32_t capacity, int32_t width, int64_t row_start,
                          int32_t n_rows, float *dst) {
    if (!ring || !dst || capacity < 1 || width < 1 || row_start < 0 || n_rows < 1 ||
        n_rows > capacity)
        return -1;
    int32_t done = 0;
    while (done < n_rows) {
        const int32_t slot = (int32_t)((row_start + done) % capacity);
        int32_t seg = capacity - slot;
        if (seg > n_rows - done) seg = n_rows - done;
        memcpy(dst + (int64_t)done * width, ring + (int64_t)slot * width,
               (size_t)seg * width * sizeof(float));
        done += seg;
    }
    return 0;
}

int32_t orc_adapter_commit(const float *enc_ring, int32_t enc_cap, int32_t enc_dim, int32_t down,
                           float *aemb_ring, int32_t aemb_cap, int32_t dec_dim,
                           int64_t group_start, int32_t n_groups, int w0_type, const uint8_t *w0,
                           int w2_type, const uint8_t *w2, int n_threads) {
    if (enc_cap < 1 || down < 1 || enc_cap % down || aemb_cap < 1 || group_start < 0 ||
        n_groups < 1)
        return -1;
    const int64_t n_in = (int64_t)enc_dim * down;
    float *x = malloc((size_t)n_in * sizeof(float));
    float *h = malloc((size_t)dec_dim * sizeof(float));
    if (!x || !h) {
        free(x);
        free(h);
        return -1;
    }
    for (int32_t i = 0; i < n_groups; ++i) {
        const int64_t g = group_start + i;
        for (int32_t j = 0; j < down; ++j) {
            const int64_t row = (g * down + j) % enc_cap;
            memcpy(x + (int64_t)j * enc_dim, enc_ring + row * enc_dim, (size_t)enc_dim * sizeof(float));
        }
        orc_matvec(w0_type, w0, dec_dim, n_in, x, h, n_threads);
        for (int32_t r = 0; r < dec_dim; ++r) h[r] = orc_gelu_erf(h[r]);
        orc_matvec(w2_type, w2, dec_dim, dec_dim, h, aemb_ring + (g % aemb_cap) * dec_dim, n_threads);
    }
    free(x);
    free(h);
    return n_groups;
}

void orc_time_embedding(float t, int32_t dim, float *out) {
    const int32_t half = dim / 2;
    for (int32_t i = 0; i < half; i++) {
        const float inv_freq = expf(-logf(10000.0f) * (float)i / (float)half);
        const float angle = t * inv_freq;
        out[i] = cosf(angle);
        out[i + half] = sinf(angle);
    }
}

int32_t orc_ada_scale(int w0_type, const uint8_t *w0, int w2_type, const void *w2, int32_t dim,
                      int32_t ada_dim, float t, float *out) {
    if (dim < 2 || ada_dim < 1) return -1;
    if (w2_type == ORC_Q8_0 && ada_dim % 32) return -1;
    const int w2_f16 = w2_type == ORC_F16;
    float *e = malloc((size_t)dim * sizeof(float));
    float *h = malloc((size_t)ada_dim * sizeof(float));
    if (!e || !h) {
        free(e);
        free(h);
        return -1;
    }
    orc_time_embedding(t, dim, e);
    orc_matvec(w0_type, w0, ada_dim, dim, e, h, 1);
    for (int32_t k = 0; k < ada_dim; k++) h[k] = orc_gelu_erf(h[k]);
    if (w2_type == ORC_Q8_0) orc_matvec(ORC_Q8_0, (const uint8_t *)w2, dim, ada_dim, h, out, 1);
    for (int32_t r = 0; r < dim && w2_type != ORC_Q8_0; r++) {
        double acc = 0.0;
        for (int32_t k = 0; k < ada_dim; k++) {
            if (w2_f16) {
                const float a = orc_f16_to_f32(((const uint16_t *)w2)[(int64_t)r * ada_dim + k]);
                const float b = orc_f16_to_f32(orc_f32_to_f16(h[k]));
                acc += (double)(a * b);
            } else {
                acc += (double)(((const float *)w2)[(int64_t)r * ada_dim + k] * h[k]);
            }
        }
        out[r] = (float)acc;
    }
    free(e);
    free(h);
    return 0;
}
