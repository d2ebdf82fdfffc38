// Internal interface between the C++ host layer (vkv_host.cpp) and the gfx950
// kernels (vkv_kernels.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "vkv.h"

namespace vkv {

// The library's per-thread error state (vkv_last_error), for host sources
// other than vkv_host.cpp.
vkv_status host_fail(vkv_status st, const char *msg);
vkv_status host_hip_fail(hipError_t e, const char *what);
vkv_status host_ok();
// HIP device ordinal of a cache (non-null)
int cache_device(const vkv_cache *c);

// ggml_gelu_erf as the CPU path computes it: 0.5 x (1 + erf(x / sqrt(2)))
__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

constexpr int kMaxStreams = VKV_MAX_BATCH_STREAMS;

// Logical window of one stream: logical index i maps to physical slot
// s0 + i for i < n0, else s1 + (i - n0)  (the <=2 read segments of a plan).
struct SegPair {
    int32_t s0, n0, s1, n1;
};

struct CacheGeom {
    uint8_t *k;            // cache base (stream 0, layer 0, slot 0)
    uint8_t *v;
    int64_t stream_bytes;
    int64_t layer_bytes;
    int64_t row_bytes;
    int32_t kv_dim;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t dtype;
};

// Decode attention (split over slot chunks, merged by the combine kernel).
struct DecodeArgs {
    const uint8_t *k;      // base of stream0, layer0
    const uint8_t *v;
    int64_t stream_bytes, layer_bytes, row_bytes;
    const float *q;        // [stream][layer][n_q_heads][head_dim]
    int64_t q_sstride, q_lstride;
    float *part_o;         // [stream][layer][n_q_heads][n_chunks][head_dim]
    float *part_ml;        // [stream][layer][n_q_heads][n_chunks][2]
    float *out;            // [stream][layer][n_q_heads][head_dim]
    int32_t n_chunks, chunk;
    int32_t xcd_swizzle;   // 1: XCD-grouped work-group order (8 kv heads, grid % 64 == 0)
    int32_t n_layers, n_kv_heads, n_q_heads;
    float scale_log2;      // scale * log2(e)
    // fused append (decoder step): new rows [stream][layer][kv_dim] f32
    uint8_t *k_w;          // writable aliases of k/v for the fused append
    uint8_t *v_w;
    const float *k_new;
    const float *v_new;
    int64_t new_sstride, new_lstride;
    // RoPE of the step's Q and new K row (rope != 0): ggml mode 0 with
    // theta_i = pos * theta_scale^i; the query/key of stream s sit at
    // position rope_pos[s]
    int32_t rope;
    float rope_theta_scale;
    float rope_pos[kMaxStreams];
    SegPair seg[kMaxStreams];
    // rope_host != 0 (one stream): the position's 64 (cos, sin) pairs of
    // ggml's angles, evaluated on the host, so no work group evaluates them
    int32_t rope_host;
    alignas(16) float2 rope_tab[64];
};

struct CombineArgs {
    const float *part_o;
    const float *part_ml;
    float *out;            // [stream][layer][n_q_heads][head_dim]
    int32_t n_chunks, n_q_heads, n_layers, head_dim;
};

struct AppendArgs {
    uint8_t *k;            // base of the stream, layer0
    uint8_t *v;
    int64_t layer_bytes, row_bytes;
    const float *k_src;
    const float *v_src;
    int64_t src_lstride;   // floats between layers of the source
    int32_t kv_dim, n_rows;
    SegPair seg;           // write segments in logical order
};

// Work groups per (head, tile) of the split per-layer encoder window tile.
constexpr int kWinSplit = 8;

struct WindowArgs {
    const uint8_t *k;      // base of stream, layer0
    const uint8_t *v;
    int64_t layer_bytes, row_bytes;
    const float *q;        // [layer][n_q][n_q_heads][head_dim]
    float *out;
    int64_t q_lstride;     // floats between layers of q/out
    int32_t n_q, n_q_heads, n_kv_heads, head_dim, n_layers;
    int64_t q_pos0, key_pos0;
    int32_t window;        // <= 0: unbounded (causal only)
    float scale_log2;
    SegPair seg;           // logical key window
    // Optional append of n_new rows ([layer][n_new][kv_dim] f32) through the
    // write segments wseg before the attention (k_new == nullptr: none).
    const float *k_new;
    const float *v_new;
    uint8_t *k_w;          // writable aliases of k/v
    uint8_t *v_w;
    int32_t n_new;
    SegPair wseg;
    // Split-key partials of the per-layer encoder tile (k_window_mfma with
    // SPL > 1): room for split_vecs (query row, head, split) partials; the
    // launch covers query tiles [tile0, ...).
    float *part_o;
    float *part_ml;
    int64_t split_vecs;
    int32_t tile0;
};

// Matrix-vector products on ggml Q4_K / Q6_K rows (vkv_matvec.hip).
constexpr int kMvMaxIn = VKV_MV_MAX_IN;
constexpr int kMvMaxOuts = VKV_MV_MAX_OUTS;

struct MvOut {
    const uint8_t *w;      // [n_rows][n_in / 256 blocks]
    float *y;
    const float *add;      // nullable: y = add + W x
    int32_t dtype, n_rows;
    int32_t wg0;           // first work group of this matrix
};

struct MvArgs {
    const float *x;
    const float *norm_w;   // nullable: x := rms_norm(x) * norm_w
    const float *ada;      // nullable: then x := x + x * ada
    float eps;
    int32_t n_in, n_outs;
    int32_t rows_per_wg;   // multiple of 4 (one contiguous quarter per wave)
    int32_t swiglu;        // out[0].y = silu(W0 x) * (W1 x), rows paired
    int32_t gelu;          // every y = gelu_erf(W x) (no residual)
    MvOut out[kMvMaxOuts];
    // Fused argmax of out[0].y (one matrix, no SwiGLU): each work group
    // atomically maxes its best (order key of the value, row) into *amax;
    // the last one (by *amax_count) writes the row to *amax_out and resets
    // both words to 0 for the next use.  nullptr: none.
    unsigned long long *amax;
    unsigned int *amax_count;
    int32_t *amax_out;
};

hipError_t launch_matvec(const MvArgs &a, int n_wg, hipStream_t st);

// Several input rows (vkv_matvec.hip, k_gemm_kq): Y[p][r] for 16 x 16 tiles.
struct MmOut {
    const uint8_t *w;      // [n_rows][n_in / 256 blocks]
    float *y;              // [n_cols][n_rows]
    const float *add;      // nullable: y = add + (W h + bias), same layout as y
    const float *bias;     // nullable: [n_rows]
    int32_t dtype, n_rows;
    int32_t tile0;         // first work group of this matrix (set by launch_gemm_kq)
    int32_t rope;          // rows rotated by RoPE (ggml mode 0) after the bias
};

struct MmArgs {
    const int8_t *xq;      // Q8_K image: codes [n_cols][n_in]
    const float *xd;       // block scales [n_cols][n_in / 256]
    const int16_t *xbs;    // 32-element sums [n_cols][n_in / 32] (q8_0 image: fp16 d)
    // Fused input (x != nullptr): each work group quantizes its own input
    // rows into LDS (k_q8k_rows' arithmetic) instead of reading the image:
    // input row p at x + ((x_row0 + p) % x_ring) * x_stride (x_ring > 0) or
    // x + p * x_stride; rms_norm(x) * norm_w (+ norm_b) (* (1 + ada)) when
    // norm_w is given.
    const float *x;
    int64_t x_stride;
    int32_t x_ring, x_row0;
    const float *norm_w, *norm_b, *ada;
    float eps;
    int32_t n_in, n_cols, n_outs, swiglu;
    int32_t gelu;          // y = gelu_erf(W h + bias) (no residual)
    // Input row p's output (and residual) row: (y_row0 + p) % y_ring when
    // y_ring > 0 (rows of a ring buffer), else p.
    int32_t y_ring, y_row0;
    // RoPE of the outputs with MmOut::rope: pairs (2i, 2i+1) of each
    // rope_hd-wide head at position rope_pos0 + input row, angle
    // pos * rope_ts^i (vkv_rope's arithmetic)
    float rope_ts;
    int32_t rope_hd;
    int64_t rope_pos0;
    MmOut out[kMvMaxOuts];
};

// Input row p is read at x + ((x_row0 + p) % x_ring) * x_stride when
// x_ring > 0 (rows of a ring buffer), else at x + p * x_stride.
// q80: the q8_0 image (Q8_0 weights): codes, and the fp16 d of every
// 32-element block in bs16 (xd unused)
hipError_t launch_q8k_rows(const float *x, int64_t x_stride, int x_ring, int x_row0, int n_rows,
                           int n, const float *norm_w, const float *norm_b, const float *ada,
                           float eps, int8_t *codes, float *xd, int16_t *bs16, bool q80,
                           hipStream_t st);
hipError_t launch_gemm_kq(MmArgs a, int n_col_tiles, hipStream_t st);
// input rows one work group of launch_gemm_kq covers for this call
int gemm_cols_per_wg(const MmArgs &a, int n_col_tiles);
// whether launch_gemm_kq may quantize this call's input inside its work
// groups (MmArgs::x): few (row, block) tasks per work group, LDS to spare
bool gemm_fused_ok(const MmArgs &a, int n_col_tiles);
hipError_t launch_q8k_quant(const float *x, int n, const float *norm_w, const float *ada, float eps,
                            uint8_t *out, hipStream_t st);
hipError_t launch_kq_dequant(int dtype, const uint8_t *src, int64_t n, const float *add, float *y,
                             hipStream_t st, unsigned long long *zero_words = nullptr);
// token ids of one embedding launch, passed by value in the kernel arguments
constexpr int kEmbedChunk = 256;
struct EmbedTokens {
    int32_t id[kEmbedChunk];
};
hipError_t launch_embed_rows(int dtype, const uint8_t *table, int64_t row_bytes,
                             const EmbedTokens &tok, int n_rows, int64_t n, const float *add,
                             int add_ring, int add_row0, float *y, hipStream_t st,
                             unsigned long long *zero_words = nullptr);
hipError_t launch_argmax(const float *x, int n, int32_t *out, hipStream_t st);
// w_type: VKV_DTYPE_F32, _F16 or _Q8_0 (n_in % 32 == 0)
hipError_t launch_rows_small(const void *w, int w_type, const float *x, int n_in, int n_rows,
                             float *y, hipStream_t st);
// The encoder conv stem (vkv_conv.hip)
hipError_t launch_im2col_f16(const float *in, int64_t stride_c, int64_t stride_t, int in_len,
                             int n_ch, int stride, int pad, int t0, int n_out, void *cols,
                             hipStream_t st);
hipError_t launch_gemm_f16(const void *w, const void *cols, const float *bias, float *y, int M,
                           int N, int K, bool gelu, hipStream_t st);
// Row p's output goes to y + ((y_row0 + p) % y_ring) * n when y_ring > 0,
// else y + p * n.
hipError_t launch_rms_norm_rows(const float *x, int n_rows, int n, const float *w, const float *b,
                                float eps, float *y, int y_ring, int y_row0, hipStream_t st);

hipError_t launch_append(int dtype, const AppendArgs &a, int n_layers, hipStream_t st);
hipError_t launch_gather(const uint8_t *src, int64_t row_bytes, SegPair seg, uint8_t *dst,
                         hipStream_t st);
// mfma: the q8_0 decode on the matrix cores (4 waves)
hipError_t launch_decode(int dtype, int gqa, int waves, int stages, bool mfma, bool fuse_append,
                         int n_streams, const DecodeArgs &a, hipStream_t st);
hipError_t launch_decode_rows(bool fuse_append, int n_streams, const DecodeArgs &a, hipStream_t st);
// q8_0 by whole rows (8 kv heads x 128, 4 query heads each, chunk % 16 == 0)
hipError_t launch_decode_q8rows(bool fuse_append, int n_streams, const DecodeArgs &a,
                               hipStream_t st);
hipError_t launch_combine(const CombineArgs &a, int n_streams, hipStream_t st);
hipError_t launch_window(int dtype, bool valu, const WindowArgs &a, hipStream_t st);
hipError_t launch_q8_0_pack(const float *x, uint8_t *blocks, int64_t n, hipStream_t st);
hipError_t launch_q8_0_unpack(const uint8_t *blocks, float *y, int64_t n, hipStream_t st);
hipError_t launch_fill_zero(void *dst, int64_t bytes, hipStream_t st);
// RoPE in place of x [n_outer][n_rows][row_len] f32; row r at position pos0 + r
hipError_t launch_rope(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                       int64_t pos0, float theta_scale, hipStream_t st);
hipError_t launch_synth(float *dst, int32_t row_len, uint64_t seed, uint32_t tag, int64_t s0,
                        int32_t ns, int64_t s_stride, int64_t l0, int32_t nl, int64_t l_stride,
                        int64_t p0, int32_t np, int64_t p_stride, hipStream_t st);

}  // namespace vkv
