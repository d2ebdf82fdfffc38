// gfx950 kernels of the encoder's conv stem (build_encoder_kv_graph,
// src/voxtral.cpp:2094-2126; causal_conv1d_graph :1767-1816 and
// compute_causal_conv1d_dims :1670-1687): two causal 1-D convolutions
// (kernel 3; stride 1 then 2) with bias and GELU, over the plan's Mel window.
// ggml computes each as im2col into f16 followed by a mul_mat against the f16
// weights; the same steps run here, so the inputs are rounded to f16 exactly
// as there and the products are exact in f32.
//
//   k_im2col_f16  -- cols[t][ic * 3 + k] = f16(in[ic][t * stride + k - pad]),
//                    zero outside [0, in_len) (the causal left pad)
//   k_gemm_f16    -- Y[t][m] = gelu(sum_j W[m][j] cols[t][j] + b[m]) on
//                    v_mfma_f32_16x16x32_f16: a work group owns 16 output
//                    channels x 16 positions, its 8 waves split K and meet in
//                    LDS
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "vkv_internal.h"

namespace vkv {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kConvWaves = 8;

__global__ void __launch_bounds__(256) k_im2col_f16(const float *__restrict__ in,
                                                    int64_t stride_c, int64_t stride_t,
                                                    int in_len, int n_ch, int stride, int pad,
                                                    int t0, int n_out, _Float16 *__restrict__ cols) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int kk = n_ch * 3;
    if (idx >= (int64_t)n_out * kk) return;
    const int t = (int)(idx / kk), j = (int)(idx % kk);
    const int ic = j / 3, k = j % 3;
    const int src = (t0 + t) * stride + k - pad;
    const float v = (src >= 0 && src < in_len) ? in[(int64_t)ic * stride_c + (int64_t)src * stride_t] : 0.0f;
    cols[idx] = (_Float16)v;
}

__global__ void __launch_bounds__(64 * kConvWaves) k_gemm_f16(const _Float16 *__restrict__ w,
                                                              const _Float16 *__restrict__ cols,
                                                              const float *__restrict__ bias,
                                                              float *__restrict__ y, int M, int N,
                                                              int K, int gelu) {
    __shared__ float red[kConvWaves][16][17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kg = lane >> 4, rr = lane & 15;
    const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16;
    const int m = min(m0 + rr, M - 1), n = min(n0 + rr, N - 1);
    const _Float16 *wa = w + (int64_t)m * K + 8 * kg;
    const _Float16 *cb = cols + (int64_t)n * K + 8 * kg;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // lane (kg, r): A = W[m0 + r][32s + 8kg, +8), B = cols[n0 + r][32s + 8kg, +8);
    // C lane (kg, n) element i = Y[m0 + 4kg + i][n0 + n]
    for (int s = wave; s < K / 32; s += kConvWaves) {
        const half8_t a = *reinterpret_cast<const half8_t *>(wa + 32 * s);
        const half8_t b = *reinterpret_cast<const half8_t *>(cb + 32 * s);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * kg + i][rr] = acc[i];
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 256) {
        const int c = t >> 4, r = t & 15;
        const int om = m0 + r, on = n0 + c;
        if (om < M && on < N) {
            float v = 0.0f;
#pragma unroll
            for (int q = 0; q < kConvWaves; ++q) v += red[q][r][c];
            v = v + bias[om];
            y[(int64_t)on * M + om] = gelu ? gelu_erf(v) : v;
        }
    }
}

}  // namespace

hipError_t launch_im2col_f16(const float *in, int64_t stride_c, int64_t stride_t, int in_len,
                             int n_ch, int stride, int pad, int t0, int n_out, void *cols,
                             hipStream_t st) {
    const int64_t total = (int64_t)n_out * n_ch * 3;
    k_im2col_f16<<<(unsigned)((total + 255) / 256), 256, 0, st>>>(
        in, stride_c, stride_t, in_len, n_ch, stride, pad, t0, n_out, (_Float16 *)cols);
    return hipGetLastError();
}

hipError_t launch_gemm_f16(const void *w, const void *cols, const float *bias, float *y, int M,
                           int N, int K, bool gelu, hipStream_t st) {
    const dim3 grid((unsigned)((M + 15) / 16), (unsigned)((N + 15) / 16));
    k_gemm_f16<<<grid, 64 * kConvWaves, 0, st>>>((const _Float16 *)w, (const _Float16 *)cols, bias,
                                                 y, M, N, K, gelu ? 1 : 0);
    return hipGetLastError();
}

}  // namespace vkv
