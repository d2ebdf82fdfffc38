/*
 * vkv_oracle.h -- CPU oracle for the voxtral.cpp decoder/encoder KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product (libvkv.so) never links, loads or calls it.
 *
 * It restates, in plain C, what the reference computes on this path:
 *   - the decoder KV ring planner and commit (src/voxtral.cpp:1590-1656),
 *   - the encoder KV ring planner and causal-window mask predicate
 *     (src/voxtral.cpp:3636-3692),
 *   - the F32->F16 conversion performed by ggml_set_rows / ggml_cpy into an
 *     F16 cache (src/voxtral.cpp:2682-2713, 2166-2185),
 *   - the ring append and logical-window gather (src/voxtral.cpp:2677-2713,
 *     2774-2799),
 *   - single-query GQA decode attention (src/voxtral.cpp:2716-2854), both
 *     exactly (fp64) and as a restatement of ggml's CPU flash-attention
 *     reduction order ("mimic": f16 Q, per-key online softmax, f16 V
 *     accumulator),
 *   - the encoder causal sliding-window attention (src/voxtral.cpp:2201-2284,
 *     mask built at :4259-4279) and the causal decoder prefill
 *     (src/voxtral.cpp:2893-2961, mask :3316-3323),
 *   - q8_0 KV block pack/unpack (absent from the reference; ggml's
 *     block_q8_0 format with the reference-quantizer rounding rule),
 *   - the decoder's weight formats (ggml Q4_K / Q6_K), the Q8_K activation
 *     quantizer, RMSNorm and the CPU matrix-vector product of ggml_mul_mat on
 *     them (src/voxtral.cpp:2653-2659, 2856-2886).
 *
 * Struct layouts are field-for-field identical to src/voxtral-internal.h.
 */
#ifndef VKV_ORACLE_H
#define VKV_ORACLE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/voxtral-internal.h:195-204 */
typedef struct orc_ring {
    int64_t capacity;
    int64_t used;
    int64_t oldest_absolute_position;
    int64_t next_absolute_position;
    int64_t wraps;
    int64_t evictions;
    int64_t bytes_moved;
    int64_t full_buffer_moves;
} orc_ring;

/* src/voxtral-internal.h:206-209 */
typedef struct orc_seg {
    int32_t slot;
    int32_t len;
} orc_seg;

/* src/voxtral-internal.h:211-223 */
typedef struct orc_plan_t {
    int64_t absolute_start;
    int32_t n_new;
    orc_seg write_seg[2];
    int32_t write_nseg;
    orc_seg read_seg[2];
    int32_t read_nseg;
    int64_t used_after;
    int64_t oldest_after;
    int64_t next_after;
    int64_t evicted;
    bool wrapped;
} orc_plan_t;

/* src/voxtral-internal.h:392-427 */
typedef struct orc_enc_plan_t {
    int64_t q_start;
    int32_t n_new;
    int64_t win_start;
    int64_t win_end;
    int32_t win_len;
    orc_seg read_seg[2];
    int32_t read_nseg;
    bool read_wraps;
    orc_seg write_seg[2];
    int32_t write_nseg;
    bool write_wraps;
    int64_t conv_mel_start;
    int64_t conv_mel_end;
    int32_t conv_slice_start;
    int64_t evicted;
} orc_enc_plan_t;

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14, ORC_Q8_K = 15 };

/* ---- planners ---- */
bool orc_decoder_plan(const orc_ring *ring, int64_t absolute_start, int32_t n_new, orc_plan_t *out);
void orc_decoder_commit(orc_ring *ring, const orc_plan_t *plan);
void orc_decoder_clear(orc_ring *ring, int64_t capacity);
bool orc_enc_plan(int64_t q_start, int32_t n_new, int32_t capacity, int32_t window, orc_enc_plan_t *out);
bool orc_enc_mask_allows(int64_t kv_abs, int64_t q_abs, int32_t window);

/* ggml_rope_ext mode 0 as the reference's decoder applies it
 * (src/voxtral.cpp:2667-2671), in place on x[n_outer][n_rows][row_len]; row r
 * at position pos0 + r; pairs (2i, 2i+1) of each head_dim-wide head turn by
 * theta_i, with theta_0 = position and theta_{i+1} = theta_i * powf(theta,
 * -2/head_dim) in f32 (ggml's CPU rope cache); cos/sin in double rounded to
 * f32. */
void orc_rope_f32(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                  int64_t pos0, float theta);

/* Encoder run scheduling (src/voxtral.cpp:104-111 normalize_physical_rows,
 * :125-154 encoder_kv_schedule_from_env with the variables passed in (<= 0 =
 * unset), :3700-3702 enc_frames_realizable, :4379-4426 one iteration of
 * encoder_kv_drive). */
typedef struct orc_enc_run {
    int64_t q0;
    int32_t n;          /* 0: stop */
    int32_t physical;
    int32_t warmup;
} orc_enc_run;
int32_t orc_enc_normalize_physical(int32_t rows);
void orc_enc_schedule(int32_t throughput, int32_t grid, int32_t logical, int32_t physical,
                      int32_t *out_logical, int32_t *out_physical);
int64_t orc_enc_frames_realizable(int64_t mel_frames);
/* false where the reference's drive fails */
bool orc_enc_drive_next(int64_t emitted, int64_t target, bool final, int32_t logical,
                        int32_t physical, int32_t finish_physical, bool batch_terminal,
                        orc_enc_run *out);

/* ---- numerics ---- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float *x, uint16_t *y, int64_t n);
void orc_f16_to_f32_n(const uint16_t *x, float *y, int64_t n);
/* one ggml block_q8_0 = {fp16 d; int8 qs[32]} = 34 bytes */
void orc_q8_0_quantize(const float *x, uint8_t *blocks, int64_t n);
void orc_q8_0_dequantize(const uint8_t *blocks, float *y, int64_t n);
int64_t orc_row_bytes(int dtype, int64_t n_elems);
/* element value of a stored row, any dtype, as float (exact) */
void orc_row_to_f32(int dtype, const void *row, float *y, int64_t n);
void orc_row_from_f32(int dtype, const float *x, void *row, int64_t n);

/* ---- seeded synthetic N(0,1) generator (integer Irwin-Hall) ---- */
uint64_t orc_mix64(uint64_t x);
uint64_t orc_row_key(uint64_t seed, uint32_t tag, int64_t stream, int64_t layer, int64_t pos);
float orc_synth_value(uint64_t key, int64_t index);
void orc_synth_row(uint64_t key, float *dst, int64_t n);

/* ---- cache model: host image of [layer][slot][row] for one stream ---- */
/* Write n_new rows (f32 src [n_new][kv_dim]) through the plan's write segments. */
void orc_append(int dtype, uint8_t *cache_layer, int64_t row_bytes, int32_t kv_dim,
                const orc_seg *write_seg, int32_t write_nseg, const float *src);
/* Copy the logical window (<=2 read segments, oldest->newest) into dst rows. */
void orc_gather(const uint8_t *cache_layer, int64_t row_bytes, const orc_seg *read_seg,
                int32_t read_nseg, uint8_t *dst);
/* Expected state of one layer after appending absolute positions [0, next) with
 * rows generated by orc_row_key(seed, tag, stream, layer, pos); slots never
 * written stay zero. capacity = ring capacity, backing = allocated slots. */
void orc_expected_layer(int dtype, uint8_t *dst, int64_t backing, int64_t capacity,
                        int32_t kv_dim, int64_t next, uint64_t seed, uint32_t tag,
                        int64_t stream, int64_t layer);

/* ---- attention ---- */
/* Single-query GQA attention over the listed physical slots of one layer.
 * q: [n_q_heads][head_dim] f32; out: [n_q_heads][head_dim]. */
void orc_decode_attn_f64(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                         int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                         const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                         int32_t head_dim, double scale, double *out);
void orc_decode_attn_mimic(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                           int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                           const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                           int32_t head_dim, float scale, float *out);
/* orc_decode_attn_mimic with an f32 V accumulator (every other rounding of
 * ggml's CPU flash attention kept). */
void orc_decode_attn_mimic_acc32(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                                 int64_t row_bytes, const int32_t *slots, int32_t n_slots,
                                 const float *q, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, float scale, float *out);
/* Multi-query window attention (encoder sliding window / decoder prefill).
 * Query i has absolute position q_pos[i]; key j has absolute position
 * k_pos[j] at physical slot k_slot[j]; key allowed iff k_pos<=q_pos and
 * k_pos >= q_pos-(window-1) (window<=0 means unbounded).
 * q: [n_q][n_q_heads][head_dim] f32; out same shape. */
void orc_window_attn_f64(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                         int64_t row_bytes, const int32_t *k_slot, const int64_t *k_pos,
                         int32_t n_keys, const float *q, const int64_t *q_pos, int32_t n_q,
                         int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t window, double scale, double *out);

/* orc_window_attn_f64's function in the reference encoder's ggml CPU
 * arithmetic: flash == 0 is the segmented path of fewer than 32 query rows
 * (f16 query against an F16 K, f32 softmax, f16 weights against an F16 V,
 * f32 sums per segment added in order), flash == 1 the flash path of 32 and
 * more (the decode mimic over each query's allowed keys).  Keys are listed in
 * logical order; segments break where slots stop being consecutive and at key
 * index new_start (the block's new rows).  F16 and F32 only (returns -1
 * otherwise).  out: [n_q][n_q_heads][head_dim] f32. */
int orc_window_attn_mimic(int dtype, const uint8_t *k_layer, const uint8_t *v_layer,
                          int64_t row_bytes, const int32_t *k_slot, const int64_t *k_pos,
                          int32_t n_keys, int32_t new_start, const float *q,
                          const int64_t *q_pos, int32_t n_q, int32_t n_q_heads,
                          int32_t n_kv_heads, int32_t head_dim, int32_t window, float scale,
                          int flash, float *out);

/* ---- CPU baseline: threaded ggml-mimic decode step ---- */
/* For each of n_layers layers: if k_new != NULL append k_new[layer]/v_new[layer]
 * (f32 [kv_dim]) at new_slot, then attention of q[layer] over slots
 * [0, n_valid) of cache layer `layer` (layer stride = layer_bytes).
 * n_threads workers split the q heads of each layer.  Returns wall seconds. */
double orc_decode_step_mimic_mt(int dtype, const uint8_t *k_cache, const uint8_t *v_cache,
                                int64_t layer_bytes, int64_t row_bytes, int32_t n_layers,
                                int32_t n_valid, const float *q, int32_t n_q_heads,
                                int32_t n_kv_heads, int32_t head_dim, float scale,
                                float *out, const float *k_new, const float *v_new,
                                int32_t new_slot, int32_t n_threads);
/* orc_decode_step_mimic_mt with each head on AVX2 + FMA + F16C lanes
 * (attention_simd.c): -1.0 where the host lacks them or head_dim is not a
 * multiple of 32 up to 512. */
double orc_decode_step_simd_mt(int dtype, const uint8_t *k_cache, const uint8_t *v_cache,
                               int64_t layer_bytes, int64_t row_bytes, int32_t n_layers,
                               int32_t n_valid, const float *q, int32_t n_q_heads,
                               int32_t n_kv_heads, int32_t head_dim, float scale,
                               float *out, const float *k_new, const float *v_new,
                               int32_t new_slot, int32_t n_threads);
/* internal to the oracle: one head of the vector leg, and whether the host
 * has AVX2, FMA and F16C */
void orc_simd_head(int dtype, const uint8_t *k_layer, const uint8_t *v_layer, int64_t row_bytes,
                   int32_t n_slots, const float *qh, int32_t g, int32_t head_dim, float scale,
                   float *oh);
int orc_simd_available(void);

/* ---- decoder weights (kquants.c): ggml Q4_K (144 B / 256), Q6_K (210 B),
 * Q8_K activations (292 B: f32 d, i8 qs[256], i16 bsums[16]) ---- */
void orc_q4_k_dequantize(const uint8_t *blocks, float *y, int64_t n);
void orc_q6_k_dequantize(const uint8_t *blocks, float *y, int64_t n);
void orc_q8_k_quantize(const float *x, uint8_t *blocks, int64_t n);
void orc_q8_k_dequantize(const uint8_t *blocks, float *y, int64_t n);
float orc_vec_dot_q4_k_q8_k(int64_t n, const uint8_t *w, const uint8_t *x);
float orc_vec_dot_q6_k_q8_k(int64_t n, const uint8_t *w, const uint8_t *x);
/* q8_0 activation blocks as ggml's x86 quantize_row_q8_0 writes them
 * (id = 127/amax, round half to even), and the Q8_0 x q8_0 row dot */
void orc_q8_0_quantize_x86(const float *x, uint8_t *blocks, int64_t n);
float orc_vec_dot_q8_0_q8_0(int64_t n, const uint8_t *w, const uint8_t *x);
void orc_rms_norm(const float *x, float *y, int64_t n, float eps);
/* rms_norm(x) * norm_w, then h + h * ada when ada is given; a copy of x when
 * norm_w is NULL */
void orc_norm_act(const float *x, int64_t n, const float *norm_w, const float *ada, float eps,
                  float *y);
/* rms_norm(x) * norm_w + norm_b (enc_apply_norm), then + h * ada */
void orc_norm_act_b(const float *x, int64_t n, const float *norm_w, const float *norm_b,
                    const float *ada, float eps, float *y);
float orc_silu(float x);
int32_t orc_argmax(const float *x, int64_t n);
int64_t orc_wrow_bytes(int dtype, int64_t n_in);
void orc_matvec(int dtype, const uint8_t *w, int64_t n_rows, int64_t n_in, const float *x,
                float *y, int n_threads);

/* ---- the encoder conv stem (conv.c) ---- */
void orc_conv_dims(int32_t in_len, int32_t kernel, int32_t stride, int32_t *pad_left,
                   int32_t *out_len);
void orc_conv1d(const float *in, int64_t stride_c, int64_t stride_t, int32_t in_len, int32_t n_ch,
                const uint16_t *w, const float *b, int32_t n_out_ch, int32_t stride, int32_t pad,
                int32_t t0, int32_t n_out, int32_t gelu, float *y);
void orc_conv_stem(const float *mel, int32_t n_mel, int32_t conv_len, int32_t slice_start,
                   int32_t n_new, const uint16_t *w0, const float *b0, const uint16_t *w1,
                   const float *b1, int32_t dim, float *x);

/* ggml_gelu_erf of one f32 (conv.c) */
float orc_gelu_erf(float x);

/* ---- the realtime rows rings and the adapter (adapter.c) ---- */
int32_t orc_row_ring_write(float *ring, int32_t capacity, int32_t width, int64_t row_start,
                           const float *src, int32_t n_rows);
int32_t orc_row_ring_read(const float *ring, int32_t capacity, int32_t width, int64_t row_start,
                          int32_t n_rows, float *dst);
int32_t orc_adapter_commit(const float *enc_ring, int32_t enc_cap, int32_t enc_dim, int32_t down,
                           float *aemb_ring, int32_t aemb_cap, int32_t dec_dim,
                           int64_t group_start, int32_t n_groups, int w0_type, const uint8_t *w0,
                           int w2_type, const uint8_t *w2, int n_threads);
void orc_time_embedding(float t, int32_t dim, float *out);
/* w2_type: ORC_F32, ORC_F16 or ORC_Q8_0 (ada_dim % 32 == 0) */
int32_t orc_ada_scale(int w0_type, const uint8_t *w0, int w2_type, const void *w2, int32_t dim,
                      int32_t ada_dim, float t, float *out);

#ifdef __cplusplus
}
#endif
#endif
