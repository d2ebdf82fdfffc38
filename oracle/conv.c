/*
 * Oracle: the encoder's conv stem (TEST INFRASTRUCTURE ONLY).
 *
 * build_encoder_kv_graph (src/voxtral.cpp:2094-2126) runs two causal 1-D
 * convolutions over the plan's Mel window: conv0 (kernel 3, stride 1) and
 * conv1 (kernel 3, stride 2), each followed by the bias and ggml_gelu_erf,
 * and keeps n_new conv1 frames from conv_slice_start.  causal_conv1d_graph
 * (:1767-1816) pads with compute_causal_conv1d_dims (:1670-1687) and calls
 * ggml_conv_1d, i.e. im2col into f16 (column ic*3 + k) and a mul_mat against
 * the f16 weights [out][in][3]: inputs rounded to f16, products exact in f32,
 * summed in f32 (here in column order; ggml's SIMD order differs, parity
 * unpinned bit for bit).  GELU: 0.5 x (1 + erff(x / sqrt 2)).
 *
 * Pinned by tests/test_conv.py: an independent fp64 numpy im2col of the same
 * f16-rounded operands, the dependence window the reference states (encoder
 * frame e reads Mel[2e-3 .. 2e+1], :3678-3680), and bit-exact agreement of
 * frames computed from different plans' windows past the stream start.
 */
#include "vkv_oracle.h"

#include <math.h>
#include <stdlib.h>

void orc_conv_dims(int32_t in_len, int32_t kernel, int32_t stride, int32_t *pad_left,
                   int32_t *out_len) {
    *pad_left = 0;
    *out_len = 0;
    if (in_len <= 0 || kernel <= 0 || stride <= 0) return;
    const int32_t padding_total = kernel - stride;
    const float n_frames = ((float)(in_len - kernel + padding_total) / (float)stride) + 1.0f;
    const int32_t target = ((int32_t)ceilf(n_frames) - 1) * stride + (kernel - padding_total);
    const int32_t extra = target - in_len > 0 ? target - in_len : 0;
    *pad_left = padding_total;
    *out_len = (in_len + padding_total + extra - kernel) / stride + 1;
}

/* ggml_gelu_erf on f32 (ggml_vec_gelu_erf_f32): 0.5 x (1 + erff(x / sqrt 2)) */
float orc_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f)); }

void orc_conv1d(const float *in, int64_t stride_c, int64_t stride_t, int32_t in_len, int32_t n_ch,
                const uint16_t *w, const float *b, int32_t n_out_ch, int32_t stride, int32_t pad,
                int32_t t0, int32_t n_out, int32_t gelu, float *y) {
    const int32_t kk = n_ch * 3;
    float *col = (float *)malloc((size_t)kk * sizeof(float));
    for (int32_t t = 0; t < n_out; ++t) {
        for (int32_t j = 0; j < kk; ++j) {
            const int32_t ic = j / 3, k = j % 3, src = (t0 + t) * stride + k - pad;
            const float v = (src >= 0 && src < in_len) ? in[(int64_t)ic * stride_c + (int64_t)src * stride_t] : 0.0f;
            col[j] = orc_f16_to_f32(orc_f32_to_f16(v));
        }
        for (int32_t oc = 0; oc < n_out_ch; ++oc) {
            const uint16_t *wr = w + (int64_t)oc * kk;
            float acc = 0.0f;
            for (int32_t j = 0; j < kk; ++j) acc += orc_f16_to_f32(wr[j]) * col[j];
            acc = acc + b[oc];
            y[(int64_t)t * n_out_ch + oc] = gelu ? orc_gelu_erf(acc) : acc;
        }
    }
    free(col);
}

/* mel [n_mel][conv_len]; out x [n_new][dim] */
void orc_conv_stem(const float *mel, int32_t n_mel, int32_t conv_len, int32_t slice_start,
                   int32_t n_new, const uint16_t *w0, const float *b0, const uint16_t *w1,
                   const float *b1, int32_t dim, float *x) {
    int32_t pad0, len0, pad1, len1;
    orc_conv_dims(conv_len, 3, 1, &pad0, &len0);
    orc_conv_dims(len0, 3, 2, &pad1, &len1);
    float *y0 = (float *)malloc((size_t)len0 * dim * sizeof(float));
    orc_conv1d(mel, conv_len, 1, conv_len, n_mel, w0, b0, dim, 1, pad0, 0, len0, 1, y0);
    orc_conv1d(y0, 1, dim, len0, dim, w1, b1, dim, 2, pad1, slice_start, n_new, 1, x);
    free(y0);
}
