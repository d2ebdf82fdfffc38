/*
 * vkv.h -- C ABI of the MI355X (gfx950) KV-cache hot path for voxtral.cpp.
 *
 * Replaces, for the decoder and encoder KV-cache step only, the ggml nodes the
 * reference builds inside build_decoder_layer (src/voxtral.cpp:2677-2854),
 * build_encoder_kv_graph (:2166-2350) and build_encoder_steady_graph
 * (:2459-2487), and the host driver contract of run_decoder_step
 * (:5219-5360) / run_decoder_prefill (:5161-5213).  The public voxtral.h /
 * voxtral-stream.h surface is unchanged; its callers reach this path through
 * voxtral_ctx_decoder_step_incremental (src/voxtral-internal.h:249).
 *
 * Conventions (mirroring include/voxtral.h:97-110 and
 * src/voxtral-c-api.cpp:612-747):
 *   - every entry point returns vkv_status; nothing throws across the ABI;
 *   - out-parameters are cleared before validation;
 *   - device pointers are plain pointers into HIP device memory owned by the
 *     caller; the cache handle owns the KV storage it allocates;
 *   - hot-path calls are asynchronous and ordered on the caller's hipStream_t
 *     (passed as void*, NULL = the null stream); synchronisation is the
 *     caller's (one sync per token, as at src/voxtral.cpp:5273);
 *   - one handle is not thread-safe; distinct handles are independent.
 */
#ifndef VKV_H
#define VKV_H

#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define VKV_API_VERSION 1u
#define VKV_MAX_BATCH_STREAMS 32
/* Encoder streaming constants: VOXTRAL_ENC_WINDOW (include/voxtral.h:44),
 * VOXTRAL_ENC_KV_MAX_NEW and VOXTRAL_ENC_KV_CAP (src/voxtral.cpp:39-40). */
#define VKV_ENC_WINDOW 750
#define VKV_ENC_MAX_NEW 128
#define VKV_ENC_KV_CAP (VKV_ENC_WINDOW + VKV_ENC_MAX_NEW)

/* Status values keep the numbering of voxtral_status (include/voxtral.h:97-110). */
typedef enum vkv_status {
    VKV_STATUS_OK = 0,
    VKV_STATUS_INVALID_ARGUMENT = 1,
    VKV_STATUS_INVALID_STATE = 2,
    VKV_STATUS_OUT_OF_MEMORY = 3,
    VKV_STATUS_MODEL_ERROR = 8,
    VKV_STATUS_BACKEND_ERROR = 9,
    VKV_STATUS_INTERNAL_ERROR = 10,
    VKV_STATUS_BUFFER_TOO_SMALL = 11
} vkv_status;

/* Storage types; values follow ggml_type (GGML_TYPE_F32=0, F16=1, Q8_0=8),
 * the type the reference selects in kv_type_from_env (src/voxtral.cpp:82-105). */
typedef enum vkv_dtype {
    VKV_DTYPE_F32 = 0,
    VKV_DTYPE_F16 = 1,
    VKV_DTYPE_Q8_0 = 8,    /* 34 B per 32: fp16 d, int8 codes (KV rows; also weights) */
    /* model weights (ggml block formats, 256 elements per block) */
    VKV_DTYPE_Q4_K = 12,   /* 144 B: fp16 d, fp16 dmin, 6-bit scales/mins, 4-bit codes */
    VKV_DTYPE_Q6_K = 14,   /* 210 B: 4+2-bit codes, int8 scales per 16, fp16 d */
    VKV_DTYPE_Q8_K = 15    /* 292 B: f32 d, int8 codes, int16 sums per 16 (activations) */
} vkv_dtype;

/* Decoder ring metadata: voxtral_decoder_kv_ring (src/voxtral-internal.h:195-204).
 * Storage addressing is modulo capacity; positions are absolute. */
typedef struct vkv_ring {
    int64_t capacity;
    int64_t used;
    int64_t oldest_absolute_position;
    int64_t next_absolute_position;
    int64_t wraps;
    int64_t evictions;
    int64_t bytes_moved;
    int64_t full_buffer_moves;
} vkv_ring;

/* voxtral_decoder_kv_seg / voxtral_enc_kv_seg (src/voxtral-internal.h:206-209, 390) */
typedef struct vkv_seg {
    int32_t slot;
    int32_t len;
} vkv_seg;

/* voxtral_decoder_kv_plan_t (src/voxtral-internal.h:211-223) */
typedef struct vkv_plan {
    int64_t absolute_start;
    int32_t n_new;
    vkv_seg write_seg[2];
    int32_t write_nseg;
    vkv_seg read_seg[2]; /* oldest -> newest logical order */
    int32_t read_nseg;
    int64_t used_after;
    int64_t oldest_after;
    int64_t next_after;
    int64_t evicted;
    bool wrapped;
} vkv_plan;

/* voxtral_enc_kv_plan_t (src/voxtral-internal.h:392-427) */
typedef struct vkv_enc_plan {
    int64_t q_start;
    int32_t n_new;
    int64_t win_start;
    int64_t win_end;
    int32_t win_len;
    vkv_seg read_seg[2];
    int32_t read_nseg;
    bool read_wraps;
    vkv_seg write_seg[2];
    int32_t write_nseg;
    bool write_wraps;
    int64_t conv_mel_start;
    int64_t conv_mel_end;
    int32_t conv_slice_start;
    int64_t evicted;
} vkv_enc_plan;

/* ---------------------------------------------------------------------------
 * Ring planners (host only; no device work).
 * ------------------------------------------------------------------------- */

/* voxtral_decoder_kv_plan (src/voxtral.cpp:1615-1644).  INVALID_ARGUMENT
 * where the reference returns false (discontinuity, n_new out of (0, capacity],
 * inconsistent ring). */
vkv_status vkv_decoder_plan(const vkv_ring *ring, int64_t absolute_start, int32_t n_new,
                            vkv_plan *out);
/* decoder_kv_commit_plan (src/voxtral.cpp:1646-1656); bytes_moved stays 0. */
vkv_status vkv_decoder_commit(vkv_ring *ring, const vkv_plan *plan);
/* clear_kv_cache (src/voxtral.cpp:1590-1602): metadata-only invalidation. */
vkv_status vkv_decoder_clear(vkv_ring *ring, int64_t capacity);
/* voxtral_enc_kv_plan (src/voxtral.cpp:3653-3692). */
vkv_status vkv_enc_plan_build(int64_t q_start, int32_t n_new, int32_t capacity, int32_t window,
                              vkv_enc_plan *out);
/* voxtral_enc_kv_mask_allows (src/voxtral.cpp:3636-3638): 1 if allowed. */
int32_t vkv_enc_mask_allows(int64_t kv_abs, int64_t q_abs, int32_t window);

/* ---------------------------------------------------------------------------
 * Encoder run scheduling (host only): which blocks of new encoder frames a
 * streaming caller submits to vkv_enc_step, as encoder_kv_drive does
 * (src/voxtral.cpp:4379-4426).  `logical` frames form one submission during
 * feed; `physical` is the query block a submission never crosses (the
 * reference's graph row count; this library needs no padding rows, so it only
 * shapes the schedule).
 * ------------------------------------------------------------------------- */
typedef struct vkv_enc_schedule {
    int32_t logical;
    int32_t physical;
} vkv_enc_schedule;

typedef struct vkv_enc_run {
    int64_t q0;            /* first new frame of the run */
    int32_t n;             /* frames in the run; 0 = nothing to submit now */
    int32_t physical;      /* query block containing [q0, q0+n) */
    int32_t warmup;        /* 1 for the 128-frame startup block */
} vkv_enc_run;

/* normalize_physical_rows (src/voxtral.cpp:104-111): the smallest of
 * 4/8/16/32/64/128 not below rows (128 above). */
int32_t vkv_enc_normalize_physical(int32_t rows);
/* encoder_kv_schedule_from_env (src/voxtral.cpp:125-154) with the environment
 * passed in: throughput != 0 is VOXTRAL_ENC_KV_MODE=throughput|offline; grid,
 * logical, physical are VOXTRAL_ENC_KV_GRID, _LOGICAL_BATCH, _PHYSICAL_ROWS
 * (<= 0 = unset).  Defaults 4/4. */
vkv_status vkv_enc_schedule_make(int32_t throughput, int32_t grid, int32_t logical,
                                 int32_t physical, vkv_enc_schedule *out);
/* enc_frames_realizable (src/voxtral.cpp:3700-3702): encoder frames a Mel
 * prefix of mel_frames yields. */
int64_t vkv_enc_frames_realizable(int64_t mel_frames);
/* One iteration of encoder_kv_drive (src/voxtral.cpp:4379-4426): the next run
 * after `emitted` frames when `target` are realizable.  final != 0 is the
 * finish flush; batch_terminal != 0 flushes in blocks of finish_physical
 * (4/8/16/32/128; the reference's default is 8).  out->n == 0: stop (wait for
 * more input, or done).  INVALID_ARGUMENT where the reference fails. */
vkv_status vkv_enc_drive_next(int64_t emitted, int64_t target, int32_t final,
                              const vkv_enc_schedule *schedule, int32_t finish_physical,
                              int32_t batch_terminal, vkv_enc_run *out);

/* ---------------------------------------------------------------------------
 * KV cache storage.
 * Layout in HBM (one allocation each for K and V):
 *   [stream][layer][slot][kv_head][head_dim] in `dtype`,
 * i.e. the reference's ggml tensor [kv_dim, capacity, layers] (ne0 fastest,
 * src/voxtral.cpp:1443-1454) repeated per stream.  Q8_0 rows are ggml
 * block_q8_0 arrays (kv_dim/32 blocks of 34 bytes).  Zero-filled once at
 * creation (src/voxtral.cpp:1456-1464); never cleared per stream.
 * ------------------------------------------------------------------------- */
typedef struct vkv_cache vkv_cache;

typedef struct vkv_cache_params {
    uint32_t struct_size;  /* sizeof(vkv_cache_params), or offsetof(.., kernel_flags) */
    int32_t n_streams;     /* independent rings sharing the allocation (>=1) */
    int32_t n_layers;      /* decoder 26, encoder 32 */
    int32_t capacity;      /* backing slots per (stream, layer): 8192 / 878 */
    int32_t n_kv_heads;    /* decoder 8, encoder 32 */
    int32_t head_dim;      /* decoder 128, encoder 64 */
    int32_t n_q_heads;     /* attention heads (multiple of n_kv_heads): 32 */
    int32_t dtype;         /* vkv_dtype */
    int32_t device;        /* HIP device ordinal */
    /* Kernel selection, for cross-checks and A/B measurement only; all zero
     * (or a struct_size that ends at `device`) = the automatic choice, which
     * is what production callers use.  Fixed for the cache's lifetime: no
     * process environment is consulted. */
    int32_t kernel_flags;  /* VKV_KERNEL_* bits */
    int32_t decode_chunk;  /* slots per split decode work group (multiple of 16); 0 = automatic */
    int32_t decode_waves;  /* waves per per-head decode work group (4 or 8); 0 = automatic */
    int32_t decode_stages; /* K/V batches in flight per decode wave (2..4); 0 = automatic */
} vkv_cache_params;

/* vkv_cache_params.kernel_flags */
#define VKV_KERNEL_DECODE_HEADS 0x1    /* F16 / q8_0 decode: per-kv-head kernel where whole rows would run */
#define VKV_KERNEL_DECODE_ROWS 0x2     /* F16 / q8_0 decode: whole-row kernel whenever the shape allows */
#define VKV_KERNEL_DECODE_VALU 0x4     /* q8_0 decode: vector-ALU kernel for every call (default: short-chunk calls only) */
#define VKV_KERNEL_WINDOW_VALU 0x8     /* window attention: vector-ALU kernel, not the matrix cores */
#define VKV_KERNEL_XCD_SWIZZLE 0x10    /* XCD-grouped decode work-group order for every dtype */
#define VKV_KERNEL_NO_XCD_SWIZZLE 0x20 /* no XCD-grouped order (q8_0's default is on) */
#define VKV_KERNEL_FLAGS_ALL 0x3f

typedef struct vkv_cache_layout {
    uint64_t row_bytes;    /* bytes per (slot) row = kv_dim elements */
    uint64_t layer_bytes;  /* capacity * row_bytes */
    uint64_t stream_bytes; /* n_layers * layer_bytes */
    uint64_t total_bytes;  /* n_streams * stream_bytes (per K or V) */
    void *k_base;          /* device pointers */
    void *v_base;
} vkv_cache_layout;

vkv_status vkv_cache_create(const vkv_cache_params *params, vkv_cache **out);
vkv_status vkv_cache_destroy(vkv_cache *cache);
vkv_status vkv_cache_get_layout(const vkv_cache *cache, vkv_cache_layout *out);
/* Synchronous device->host copy of rows [slot0, slot0+n_slots) of one
 * (K or V, stream, layer); which: 0 = K, 1 = V.  For state checks only. */
vkv_status vkv_cache_read_rows(const vkv_cache *cache, int32_t which, int32_t stream,
                               int32_t layer, int32_t slot0, int32_t n_slots, void *host_dst,
                               size_t dst_bytes);
/* Zero the whole cache (stream-ordered fill kernel, capture-safe). */
vkv_status vkv_cache_zero(vkv_cache *cache, void *hip_stream);

/* ---------------------------------------------------------------------------
 * Hot path.  All pointers are device pointers.  Rows are f32 [.. ][kv_dim].
 * ------------------------------------------------------------------------- */

/* Append: ggml_set_rows / ggml_cpy of projected K/V into the cache
 * (src/voxtral.cpp:2682-2713 decoder, :2166-2185 encoder).  Rows
 * src[layer][i] for i in [0, sum(write_seg.len)) are laid down in logical
 * order across the <=2 write segments, converted once to the cache dtype
 * (F16: IEEE round-to-nearest-even; Q8_0: block quantizer).  layer_stride is
 * the distance in floats between consecutive layers of k_src/v_src (0 =
 * packed).  Layers [layer0, layer0+n_layers) are written in one launch. */
vkv_status vkv_append(vkv_cache *cache, int32_t stream, int32_t layer0, int32_t n_layers,
                      const vkv_seg *write_seg, int32_t write_nseg, const float *k_src,
                      const float *v_src, int64_t layer_stride, void *hip_stream);

/* Ring gather: the logical window concat(read_seg[0], read_seg[1]) of one
 * layer copied, bit-exact and in the cache dtype, into contiguous rows
 * (src/voxtral.cpp:2774-2799 decoder oracle, :2285-2331 encoder P>=32). */
vkv_status vkv_gather(const vkv_cache *cache, int32_t stream, int32_t layer,
                      const vkv_seg *read_seg, int32_t read_nseg, void *k_dst, void *v_dst,
                      void *hip_stream);

/* Single-query GQA decode attention over the ring (ggml_flash_attn_ext at
 * src/voxtral.cpp:2749-2819).  For each stream s in [stream0, stream0+n_streams)
 * and layer l in [layer0, layer0+n_layers):
 *   out[s][l][h] = sum_j softmax_j(scale * q[s][l][h] . K[j][h/G]) V[j][h/G]
 * over the slots of plans[s - stream0].read_seg (the logical window; slot
 * order is irrelevant, which is the permutation argument of :2801-2807).
 * q/out: f32 [stream][layer][n_q_heads][head_dim], packed. */
vkv_status vkv_decode_attn(vkv_cache *cache, int32_t stream0, int32_t n_streams,
                           int32_t layer0, int32_t n_layers, const vkv_plan *plans,
                           const float *q, float *out, int32_t n_q_heads, float scale,
                           void *hip_stream);

/* One decoder KV step for a batch of streams, the KV part of run_decoder_step
 * (src/voxtral.cpp:5219-5360): plan every ring at positions[s] with n_new=1
 * (INVALID_ARGUMENT and nothing launched or committed if any plan is
 * invalid), append k/v (f32 [stream][layer][kv_dim]) at slot pos % capacity,
 * run decode attention over the post-append window, then commit each ring
 * (decoder_kv_commit_plan, :1646-1656).  Append and attention are fused in
 * one launch.  plans_out (optional, host) receives the plans used. */
vkv_status vkv_decoder_step(vkv_cache *cache, int32_t stream0, int32_t n_streams,
                            vkv_ring *rings, const int64_t *positions, int32_t layer0,
                            int32_t n_layers, const float *q, const float *k, const float *v,
                            float *out, int32_t n_q_heads, float scale, vkv_plan *plans_out,
                            void *hip_stream);

/* vkv_decoder_step with the decoder's RoPE fused in: q and k are the
 * projections before RoPE, as build_decoder_layer rotates them
 * (ggml_rope_ext mode 0, src/voxtral.cpp:2667-2671): pairs (2i, 2i+1) of
 * each head turn by theta_i = position * rope_theta^(-2i/head_dim), with
 * ggml's f32 running product for theta_i; cos/sin are evaluated in double and
 * rounded to f32.  The new K row is rotated before it is stored, Q before the
 * attention; V is stored as given.  Positions < 2^24. */
vkv_status vkv_decoder_step_rope(vkv_cache *cache, int32_t stream0, int32_t n_streams,
                                 vkv_ring *rings, const int64_t *positions, int32_t layer0,
                                 int32_t n_layers, const float *q, const float *k, const float *v,
                                 float *out, int32_t n_q_heads, float scale, float rope_theta,
                                 vkv_plan *plans_out, void *hip_stream);

/* One layer range of a decoder step whose one-row plan the caller made for
 * the token with vkv_decoder_plan(ring, position, 1, plan): append k/v
 * ([layer][kv_dim]) at the plan's slot, rotate q and k by RoPE at `position`
 * when rope_theta > 0, and attend over the plan's read window; the caller
 * calls vkv_decoder_commit once after the last layer (run_decoder_step,
 * src/voxtral.cpp:5227-5232 and :5358).  This is the per-layer form that
 * build_decoder_layer needs (:2629-2887): layer l+1's projections read layer
 * l's attention output. */
vkv_status vkv_decoder_layer_step(vkv_cache *cache, int32_t stream, const vkv_plan *plan,
                                  int64_t position, int32_t layer0, int32_t n_layers,
                                  const float *q, const float *k, const float *v, float *out,
                                  int32_t n_q_heads, float scale, float rope_theta,
                                  void *hip_stream);

/* The same RoPE in place on f32 rows x[n_outer][n_rows][row_len] (row_len a
 * multiple of head_dim, head_dim % 8 == 0); row r is at position pos0 + r.
 * For the prefill's q and k before vkv_decoder_prefill. */
vkv_status vkv_rope(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                    int64_t pos0, float theta, void *hip_stream);

/* Multi-token causal prefill of one stream (run_decoder_prefill,
 * src/voxtral.cpp:5161-5213; causal mask :3316-3323): plan n_tokens from
 * ring->next_absolute_position, append k/v ([layer][n_tokens][kv_dim]), then
 * attention of q ([layer][n_tokens][n_q_heads][head_dim]) where token t at
 * absolute position a attends every retained key with position <= a; commit.
 * Requires the post-append window to be one read segment (as the reference's
 * one-segment path, :2763-2773). */
vkv_status vkv_decoder_prefill(vkv_cache *cache, int32_t stream, vkv_ring *ring, int32_t layer0,
                               int32_t n_layers, int32_t n_tokens, const float *q,
                               const float *k, const float *v, float *out, int32_t n_q_heads,
                               float scale, void *hip_stream);

/* Encoder KV step for one stream (build_encoder_kv_graph ring write +
 * window attention, src/voxtral.cpp:2166-2284; mask :4259-4279): write the
 * plan's n_new K/V rows ([layer][n_new][kv_dim] f32) through write_seg, then
 * for query i (absolute position q_start+i) attend the keys of the window
 * [win_start, win_end) allowed by voxtral_enc_kv_mask_allows(kv, q, window).
 * q/out: [layer][n_new][n_q_heads][head_dim]. */
vkv_status vkv_enc_step(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                        int32_t window, int32_t layer0, int32_t n_layers, const float *q,
                        const float *k, const float *v, float *out, int32_t n_q_heads,
                        float scale, void *hip_stream);

/* Window attention without append: n_q queries with absolute positions
 * q_pos[0] + i, over keys whose absolute positions are key_pos0 + j for the
 * logical window described by read_seg (j counts across the segments);
 * allowed iff kv <= q and (window <= 0 or kv >= q - (window-1)). */
vkv_status vkv_window_attn(vkv_cache *cache, int32_t stream, int32_t layer0, int32_t n_layers,
                           const vkv_seg *read_seg, int32_t read_nseg, int64_t key_pos0,
                           int64_t q_pos0, int32_t n_q, int32_t window, const float *q,
                           float *out, int32_t n_q_heads, float scale, void *hip_stream);

/* ---------------------------------------------------------------------------
 * q8_0 KV pack/unpack (ggml block_q8_0 {fp16 d; int8 qs[32]}); n % 32 == 0.
 * Quantizer: amax = max|x|, d = amax/127, id = d ? 1/d : 0,
 * qs = round-half-away(x*id), d stored as fp16 (RNE).
 * ------------------------------------------------------------------------- */
vkv_status vkv_q8_0_pack(const float *x, void *blocks, int64_t n, void *hip_stream);
vkv_status vkv_q8_0_unpack(const void *blocks, float *y, int64_t n, void *hip_stream);

/* ---------------------------------------------------------------------------
 * Decoder projections on ggml Q4_K / Q6_K / Q8_0 weights: ggml_mul_mat(W, x) for one
 * token (src/voxtral.cpp:2656-2659 Q/K/V, :2857 O, :2878-2882 SwiGLU FFN),
 * with the RMSNorm that precedes them (:2653-2654, :2861-2862) and the ada
 * time conditioning (:2864-2874) fused into the input side.
 *
 * The input is formed as the CPU path forms it: h = rms_norm(x, eps) * norm_w
 * (sum of squares in double, mean rounded to f32, scale = 1/sqrtf(mean+eps)),
 * then h + h * ada; or h = x when norm_w is NULL.  h is quantized to Q8_K
 * (ggml quantize_row_q8_K_ref) and every row is an integer dot product per
 * 256-block, scaled by fp16(d) * d_x (Q4_K: minus fp16(dmin) * d_x * the
 * mins against 32-element sums).  For Q8_0 rows (a Q8_0 file,
 * src/voxtral-quantize.cpp:95-96) h is quantized to q8_0 instead, as ggml's
 * x86 quantize_row_q8_0 does (d = fp16(amax/127), codes rint(h * 127/amax),
 * half to even), and each 32-block's integer dot is scaled by fp16(d_w) * d_x.
 * Rows are W's rows in ggml's row-major block layout, i.e. a GGUF tensor's
 * bytes unchanged; matrices of one call may mix the three formats.
 * ------------------------------------------------------------------------- */
#define VKV_MV_MAX_IN 12288      /* n_in limit (multiple of 256) */
#define VKV_MV_MAX_OUTS 4        /* matrices per call */

typedef struct vkv_mv_out {
    const void *w;        /* [n_rows] rows of Q4_K / Q6_K / Q8_0 blocks, device memory, 4-byte aligned */
    int32_t dtype;        /* VKV_DTYPE_Q4_K, VKV_DTYPE_Q6_K or VKV_DTYPE_Q8_0 */
    int32_t n_rows;
    float *y;             /* [n_rows] */
    const float *add;     /* NULL, or the residual: y = add + W h (may alias y) */
} vkv_mv_out;

#define VKV_MV_STORE 0
#define VKV_MV_SWIGLU 1   /* n_outs = 2, equal rows and dtype: outs[0].y = silu(W0 h) * (W1 h) */
#define VKV_MV_GELU 2     /* every y = gelu_erf(W h) (+ bias first in vkv_matmul); no residual */

/* y_k = W_k h for up to VKV_MV_MAX_OUTS matrices reading the same input (the
 * Q/K/V projections in one call).  x, norm_w, ada: 16-byte aligned device
 * arrays of n_in floats; ada requires norm_w. */
vkv_status vkv_matvec(const float *x, int64_t n_in, const float *norm_w, const float *ada,
                      float eps, const vkv_mv_out *outs, int32_t n_outs, int32_t epilogue,
                      void *hip_stream);

/* The input side alone: h quantized to n/256 ggml block_q8_K (292 B each,
 * 4-byte aligned device memory); n <= VKV_MV_MAX_IN. */
vkv_status vkv_quantize_q8_k(const float *x, int64_t n, const float *norm_w, const float *ada,
                             float eps, void *blocks, void *hip_stream);

/* ggml dequantize_row_q4_K / _q6_K / _q8_0 of n elements (n % 256 == 0) to f32: the
 * token-embedding lookup (ggml_get_rows on tok_embeddings, src/voxtral.cpp:
 * 3008) for one row of the table. */
vkv_status vkv_dequantize(int32_t dtype, const void *blocks, int64_t n, float *y,
                          void *hip_stream);

/* ---------------------------------------------------------------------------
 * The same products for several input rows at once: the encoder's P new
 * frames per chunk (build_encoder_kv_graph, src/voxtral.cpp:2147-2370) and the
 * decoder prefill.  x: [n_cols][n_in] f32 (one input row per frame/token);
 * every row is formed and quantized to Q8_K as in vkv_matvec, with the
 * norm's optional bias added after the weight (enc_apply_norm, :1855-1861).
 * y: [n_cols][n_rows] per matrix, plus bias[r], plus add (same layout) when
 * given.  SwiGLU pairs the rows of two matrices as vkv_matvec does.  The Q8_K
 * image of x lives in the caller's workspace (vkv_matmul_workspace bytes,
 * 256-byte aligned); matrices of one call may mix Q4_K and Q6_K.  Q8_0
 * matrices take the q8_0 image of x (as vkv_matvec forms it) and share a
 * call only with other Q8_0 matrices.
 * ------------------------------------------------------------------------- */
typedef struct vkv_mm_out {
    const void *w;        /* [n_rows] rows of Q4_K / Q6_K / Q8_0 blocks, 4-byte aligned */
    int32_t dtype;
    int32_t n_rows;
    float *y;             /* [n_cols][n_rows] */
    const float *add;     /* NULL, or the residual [n_cols][n_rows] (may alias y) */
    const float *bias;    /* NULL, or [n_rows] added before the residual */
} vkv_mm_out;

size_t vkv_matmul_workspace(int32_t n_cols, int64_t n_in);
vkv_status vkv_matmul(const float *x, int32_t n_cols, int64_t n_in, const float *norm_w,
                      const float *norm_b, const float *ada, float eps, const vkv_mm_out *outs,
                      int32_t n_outs, int32_t epilogue, void *workspace, size_t workspace_bytes,
                      void *hip_stream);

/* ---------------------------------------------------------------------------
 * One encoder chunk through every layer (build_encoder_kv_graph's transformer,
 * src/voxtral.cpp:2144-2370): for the plan's n_new frames x ([n_new][dim], the
 * conv stem's output, replaced in place by the output), per layer
 * h = rms_norm(x) * attn_norm + attn_norm_b; q = Wq h + bq ([n_heads *
 * head_dim] rows), k = Wk h, v = Wv h + bv (the cache's kv width);
 * RoPE of q and k at positions q_start..; K/V append to the
 * ring and causal sliding-window attention (vkv_enc_step); x += Wo a + bo;
 * h = rms_norm(x) * ffn_norm + ffn_norm_b; x += W2 (silu(W1 h) * (W3 h)) + b2;
 * finally x = rms_norm(x) * out_norm + out_norm_b.  Bias pointers may be NULL.
 * ------------------------------------------------------------------------- */
typedef struct vkv_enc_layer {
    const float *attn_norm, *attn_norm_b;
    const void *attn_q, *attn_k, *attn_v, *attn_o;
    int32_t attn_q_type, attn_k_type, attn_v_type, attn_o_type;
    const float *attn_q_b, *attn_v_b, *attn_o_b;
    const float *ffn_norm, *ffn_norm_b;
    const void *ffn_w1, *ffn_w2, *ffn_w3;
    int32_t ffn_w1_type, ffn_w2_type, ffn_w3_type;
    const float *ffn_w2_b;
} vkv_enc_layer;

typedef struct vkv_enc_model {
    int32_t n_layers, dim, hidden, n_heads, head_dim;
    float norm_eps, rope_theta;
    const float *out_norm, *out_norm_b;
    const vkv_enc_layer *layers;   /* host array of n_layers */
} vkv_enc_model;

/* The conv stem for an encoder plan (build_encoder_kv_graph, src/voxtral.cpp:
 * 2094-2126): mel is the plan's Mel window [n_mel][conv_len] (bins major,
 * frames contiguous, conv_len = conv_mel_end - conv_mel_start); conv0
 * (kernel 3, stride 1, n_mel -> dim, causal pad 2) + bias + GELU(erf), conv1
 * (kernel 3, stride 2, dim -> dim, causal pad 1) + bias + GELU(erf), both as
 * ggml computes them (im2col in f16, f16 weights [out][in][3], f32 sums); the
 * plan's n_new frames from conv_slice_start go to x [n_new][dim]. */
size_t vkv_enc_conv_stem_workspace(int32_t conv_len, int32_t n_mel, int32_t dim, int32_t n_new);
vkv_status vkv_enc_conv_stem(const float *mel, int32_t n_mel, const vkv_enc_plan *plan,
                             const void *conv0_w, const float *conv0_b, const void *conv1_w,
                             const float *conv1_b, int32_t dim, float *x, void *workspace,
                             size_t workspace_bytes, void *hip_stream);

size_t vkv_encoder_chunk_workspace(const vkv_enc_model *model, int32_t n_new);
vkv_status vkv_encoder_chunk(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                             int32_t window, const vkv_enc_model *model, float *x,
                             void *workspace, size_t workspace_bytes, void *hip_stream);

/* ---------------------------------------------------------------------------
 * The realtime rings between encoder, adapter and decoder (src/voxtral.cpp:
 * 42-55, 388-404, 1467-1485): the encoder-output ring holds encoder frames
 * ([256][1280] f32) until the adapter consumes them DOWNSAMPLE (4) at a time;
 * the audio-embedding ring holds one adapter output per group ([256][3072]
 * f32) until the decoder step reads it (audio position p at row p % 256).
 * Logical row r lives at row r % capacity.  The caller owns the memory
 * (capacity * width floats of 16-byte aligned device memory).
 * ------------------------------------------------------------------------- */
typedef struct vkv_row_ring {
    float *rows;          /* [capacity][width] */
    int32_t capacity;     /* rows */
    int32_t width;        /* floats per row */
} vkv_row_ring;

/* src rows i -> logical rows row_start + i, n_rows <= capacity
 * (copy_chunk_to_enc_out_ring, src/voxtral.cpp:4018-4043: one device copy
 * per contiguous segment, at most two). */
vkv_status vkv_row_ring_write(vkv_row_ring *ring, int64_t row_start, const float *src,
                              int32_t n_rows, void *hip_stream);

/* Logical rows row_start.. -> dst (host or device memory), 1 <= n_rows <=
 * capacity (read_realtime_ring_rows, src/voxtral.cpp:5530-5554); returns
 * after the copy has completed. */
vkv_status vkv_row_ring_read(const vkv_row_ring *ring, int64_t row_start, int32_t n_rows,
                             float *dst, void *hip_stream);

/* vkv_encoder_chunk with the final norm's rows stored at the encoder-output
 * ring's logical rows plan->q_start .. + n_new (build_encoder_steady_graph's
 * ggml_set_rows, src/voxtral.cpp:2505-2508); x ends holding the last layer's
 * residual stream.  ring width = model dim, n_new <= capacity. */
vkv_status vkv_encoder_chunk_ring(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                                  int32_t window, const vkv_enc_model *model, float *x,
                                  vkv_row_ring *enc_out, void *workspace, size_t workspace_bytes,
                                  void *hip_stream);

/* The adapter over ring groups (build_adapter_ring_graph_reusable,
 * src/voxtral.cpp:2589-2620, as voxtral_ctx_adapter_commit :5424-5485 runs
 * it): for each group g in [group_start, group_start + n_groups), its
 * frames downsample*g .. downsample*g + downsample-1 of the encoder-output ring (one
 * contiguous row of enc_dim * downsample floats: the ring capacity must be a
 * multiple of downsample), h = gelu_erf(W0 x), audio-embedding logical row
 * g = W2 h.  Both products as vkv_matmul computes them (Q8_K input,
 * integer block sums); Q4_K, Q6_K or Q8_0 weights (q8_0 input for Q8_0). */
typedef struct vkv_adapter {
    const void *w0;       /* adapter.0.weight [dec_dim][enc_dim * downsample] */
    const void *w2;       /* adapter.2.weight [dec_dim][dec_dim] */
    int32_t w0_type, w2_type;
    int32_t enc_dim, dec_dim, downsample;
} vkv_adapter;

size_t vkv_adapter_workspace(const vkv_adapter *adapter, int32_t n_groups);
vkv_status vkv_adapter_commit(const vkv_adapter *adapter, const vkv_row_ring *enc_out,
                              vkv_row_ring *audio_emb, int64_t group_start, int32_t n_groups,
                              void *workspace, size_t workspace_bytes, void *hip_stream);

/* The decoder step's input row: ggml_get_rows(tok_embeddings, token) +
 * audio embedding (src/voxtral.cpp:3008-3019): row `token` of a Q4_K/Q6_K/Q8_0
 * table [n_rows][n_cols], dequantized, plus add[] when add is not NULL. */
vkv_status vkv_embed(int32_t dtype, const void *table, int32_t n_rows, int64_t n_cols,
                     int32_t token, const float *add, float *y, void *hip_stream);

/* The decoder's ada time conditioning, constant for a session
 * (build_decoder_layer src/voxtral.cpp:2864-2874 on the time embedding of
 * compute_time_embedding :729-740, evaluated at t = VOXTRAL_N_DELAY_TOKENS,
 * :1535): scale = W2 gelu_erf(W0 e(t)) with e(t)[i] = cos(t f_i),
 * e(t)[i + dim/2] = sin(t f_i), f_i = expf(-logf(10000) i / (dim/2)), as the
 * reference computes it on the host.  W0: Q4_K/Q6_K/Q8_0 [ada_dim][dim] (the
 * product as vkv_matvec computes it); W2: F16 or F32 (dtype 1 / 0)
 * [dim][ada_dim], its input rounded to f16 for F16 as ggml's vec-dot type
 * does, or Q8_0 (dtype 8, a Q8_0 file: ada_dim % 32 == 0, the input
 * quantized to q8_0 as for any Q8_0 product).  out: [dim] f32 device memory,
 * the vkv_dec_layer.ada_scale of the layer.  workspace:
 * vkv_ada_scale_workspace bytes of device memory. */
size_t vkv_ada_scale_workspace(int32_t dim, int32_t ada_dim);
vkv_status vkv_ada_scale(const void *w0, int32_t w0_type, const void *w2, int32_t w2_type,
                         int32_t dim, int32_t ada_dim, float t, float *out, void *workspace,
                         size_t workspace_bytes, void *hip_stream);

/* ggml_argmax of f32 logits (emit_logits_argmax, src/voxtral.cpp:2966-2972):
 * the last index of the maximum (ggml_vec_argmax_f32 keeps updating the index
 * while x[i] equals the running max); NaN input gives an unspecified index.
 * x: 16-byte aligned device array; out: one int32 in device memory. */
vkv_status vkv_argmax(const float *x, int64_t n, int32_t *out, void *hip_stream);

/* ---------------------------------------------------------------------------
 * One decoder token (run_decoder_step's graph, src/voxtral.cpp:2981-3040 and
 * build_decoder_layer :2629-2887): x = get_rows(tok_embeddings, token) +
 * audio_emb; per layer h = rms_norm(x) * attn_norm, q/k/v = W h, RoPE of q
 * and k at the token's position, K/V append at the ring slot, attention over
 * the window, x += W_o attn, h = rms_norm(x) * ffn_norm (* (1 + ada)),
 * x += W2 (silu(W1 h) * (W3 h)); logits = output (rms_norm(x) * out_norm);
 * argmax.  Weights are GGUF tensors' bytes in device memory (Q4_K / Q6_K /
 * Q8_0);
 * norms and ada scales f32.  The ring is planned once and committed after
 * the last layer.
 * ------------------------------------------------------------------------- */
typedef struct vkv_dec_layer {
    const float *attn_norm;        /* [dim] */
    const void *attn_q, *attn_k, *attn_v, *attn_o;
    int32_t attn_q_type, attn_k_type, attn_v_type, attn_o_type;
    const float *ffn_norm;         /* [dim] */
    const float *ada_scale;        /* [dim] ada_mlp(time_emb) of this layer, or NULL */
    const void *ffn_w1, *ffn_w2, *ffn_w3;
    int32_t ffn_w1_type, ffn_w2_type, ffn_w3_type;
} vkv_dec_layer;

typedef struct vkv_dec_model {
    int32_t n_layers, dim, hidden, n_q_heads, n_kv_heads, head_dim, vocab;
    float norm_eps, rope_theta;
    const void *tok_embeddings;    /* [vocab][dim] */
    int32_t tok_embeddings_type;
    const float *out_norm;         /* [dim] */
    const void *output;            /* [vocab][dim]; the tied model passes tok_embeddings */
    int32_t output_type;
    const vkv_dec_layer *layers;   /* host array of n_layers */
} vkv_dec_model;

/* Device workspace the token needs (bytes); 256-byte aligned by the caller. */
size_t vkv_decoder_token_workspace(const vkv_dec_model *model);

/* Runs the token at position ring->next_absolute_position of `stream` in the
 * cache (whose n_layers / heads must match the model).  audio_emb: [dim] f32
 * device row or NULL; logits: [vocab] f32 device; token_out: one int32 in
 * device memory (the greedy token).  plan_out (host, may be NULL) receives
 * the committed plan.  The workspace keeps, after the call, x (the final
 * residual stream) at offset 0 as dim floats. */
vkv_status vkv_decoder_token(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                             const vkv_dec_model *model, int32_t token, const float *audio_emb,
                             float *logits, int32_t *token_out, void *workspace,
                             size_t workspace_bytes, vkv_plan *plan_out, void *hip_stream);

/* vkv_decoder_token without the workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference (its
 * step graph allocates its work buffers once per context).  The workspace is
 * a fixed device array of VKV_TOKEN_SCRATCH_BYTES inside the library, one
 * copy per GPU held until the process ends; the call allocates nothing.
 * BUFFER_TOO_SMALL when vkv_decoder_token_workspace(model) exceeds it (the
 * realtime decoder needs ~90 KB).  Every call on one GPU shares that GPU's
 * copy: calls that overlap on a GPU (other HIP streams, other threads) race,
 * so serialize them.  Otherwise identical to vkv_decoder_token (the final
 * residual stream stays in the library's array, not visible to the caller). */
#define VKV_TOKEN_SCRATCH_BYTES (1u << 20)
vkv_status vkv_decoder_token_noalloc(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                                     const vkv_dec_model *model, int32_t token,
                                     const float *audio_emb, float *logits, int32_t *token_out,
                                     vkv_plan *plan_out, void *hip_stream);

/* Device workspace of a prompt of n_tokens (bytes); 0 for a bad model or count. */
size_t vkv_decoder_prompt_workspace(const vkv_dec_model *model, int32_t n_tokens);

/* The decoder prefill of a prompt (run_decoder_prefill, src/voxtral.cpp:
 * 5161-5213, graph build_decoder_prefill_graph :2893-2961): n_tokens prompt
 * tokens at positions ring->next_absolute_position + i, each embedded
 * (get_rows) plus its audio row, through every layer (the multi-row products
 * with the RoPE in their epilogue, the causal window attention appending the
 * K/V rows, SwiGLU, residuals), the final norm of the last token and its
 * logits with the greedy token; then commits the ring.  tokens: host array,
 * each in [0, vocab); audio_emb: device ring whose logical row
 * next_absolute_position + i is token i's audio row (width dim), or NULL.
 * The post-append window must be one read segment, as for
 * vkv_decoder_prefill.  The workspace keeps, after the call, the residual
 * stream of all n_tokens rows ([n_tokens][dim] f32) at offset 0. */
vkv_status vkv_decoder_prompt(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                              const vkv_dec_model *model, const int32_t *tokens, int32_t n_tokens,
                              const vkv_row_ring *audio_emb, float *logits, int32_t *token_out,
                              void *workspace, size_t workspace_bytes, vkv_plan *plan_out,
                              void *hip_stream);

/* ---------------------------------------------------------------------------
 * GGUF model files (voxtral_model_load_from_file, src/voxtral.cpp:1035-1316,
 * over ggml's gguf reader; the files tools/convert_voxtral_to_gguf.py and
 * src/voxtral-quantize.cpp write).  GGUF v2/v3: magic "GGUF", version,
 * tensor and key counts, typed key/value metadata, tensor infos (name, dims
 * ne[] fastest first, ggml type, offset), then the data section at the
 * file's alignment (general.alignment, default 32) with every tensor at its
 * packed, aligned offset.  Files are mapped read-only; strings returned stay
 * valid until vkv_gguf_close.  Reading metadata needs no GPU.
 * ------------------------------------------------------------------------- */
typedef struct vkv_gguf vkv_gguf;

/* GGUF value types (the file's type codes) */
#define VKV_GGUF_UINT8 0
#define VKV_GGUF_INT8 1
#define VKV_GGUF_UINT16 2
#define VKV_GGUF_INT16 3
#define VKV_GGUF_UINT32 4
#define VKV_GGUF_INT32 5
#define VKV_GGUF_FLOAT32 6
#define VKV_GGUF_BOOL 7
#define VKV_GGUF_STRING 8
#define VKV_GGUF_ARRAY 9
#define VKV_GGUF_UINT64 10
#define VKV_GGUF_INT64 11
#define VKV_GGUF_FLOAT64 12

typedef struct vkv_gguf_tensor {
    const char *name;
    int32_t type;          /* ggml_type */
    int32_t n_dims;
    int64_t ne[4];         /* elements per dimension, ne[0] fastest; 1 past n_dims */
    uint64_t offset;       /* from the start of the data section */
    uint64_t nbytes;
} vkv_gguf_tensor;

/* MODEL_ERROR for a missing, truncated or malformed file (the message says
 * what was wrong); *out is NULL then. */
vkv_status vkv_gguf_open(const char *path, vkv_gguf **out);
vkv_status vkv_gguf_close(vkv_gguf *gguf);
uint32_t vkv_gguf_version(const vkv_gguf *gguf);
uint64_t vkv_gguf_alignment(const vkv_gguf *gguf);
uint64_t vkv_gguf_data_offset(const vkv_gguf *gguf);   /* file offset of the data section */
int64_t vkv_gguf_n_kv(const vkv_gguf *gguf);
int64_t vkv_gguf_find_key(const vkv_gguf *gguf, const char *key);   /* -1 when absent */
const char *vkv_gguf_key(const vkv_gguf *gguf, int64_t i);         /* NULL out of range */
int32_t vkv_gguf_kv_type(const vkv_gguf *gguf, int64_t i);         /* -1 out of range */
/* Scalar values; INVALID_ARGUMENT when the key's type differs (ggml's
 * gguf_get_val_* assert it).  bool reads as 0/1. */
vkv_status vkv_gguf_get_i32(const vkv_gguf *gguf, int64_t i, int32_t *out);
vkv_status vkv_gguf_get_u32(const vkv_gguf *gguf, int64_t i, uint32_t *out);
vkv_status vkv_gguf_get_i64(const vkv_gguf *gguf, int64_t i, int64_t *out);
vkv_status vkv_gguf_get_f32(const vkv_gguf *gguf, int64_t i, float *out);
vkv_status vkv_gguf_get_f64(const vkv_gguf *gguf, int64_t i, double *out);
vkv_status vkv_gguf_get_bool(const vkv_gguf *gguf, int64_t i, int32_t *out);
/* any scalar value's bytes (1, 2, 4 or 8 by its type), little-endian */
vkv_status vkv_gguf_get_scalar(const vkv_gguf *gguf, int64_t i, void *out, uint64_t out_bytes);
/* NUL-terminated copy of a string value (len excludes the NUL) */
vkv_status vkv_gguf_get_str(const vkv_gguf *gguf, int64_t i, const char **out, uint64_t *len);
/* Arrays: element type and count; data points at the elements in the file
 * (NULL for string arrays, read with vkv_gguf_get_arr_str). */
vkv_status vkv_gguf_get_arr(const vkv_gguf *gguf, int64_t i, int32_t *elem_type, uint64_t *n,
                            const void **data);
vkv_status vkv_gguf_get_arr_str(const vkv_gguf *gguf, int64_t i, uint64_t j, const char **out,
                                uint64_t *len);
int64_t vkv_gguf_n_tensors(const vkv_gguf *gguf);
int64_t vkv_gguf_find_tensor(const vkv_gguf *gguf, const char *name);   /* -1 when absent */
vkv_status vkv_gguf_tensor_info(const vkv_gguf *gguf, int64_t i, vkv_gguf_tensor *out);
/* the tensor's bytes in the mapped file */
const void *vkv_gguf_tensor_data(const vkv_gguf *gguf, int64_t i);

/* The model's hyperparameters as the reference populates them from the
 * metadata (src/voxtral.cpp:1066-1113): each key overrides the default of
 * include/voxtral.h when present; is_offline = (general.architecture ==
 * "voxtral"); encoder causality and ada conditioning default to !is_offline. */
typedef struct vkv_hparams {
    int32_t is_offline;
    int32_t enc_dim, enc_layers, enc_heads, enc_head_dim, enc_hidden, enc_kv_heads, enc_causal;
    float enc_norm_eps, enc_rope_theta;
    int32_t dec_dim, dec_layers, dec_heads, dec_head_dim, dec_hidden, dec_kv_heads;
    float dec_norm_eps, dec_rope_theta;
    int32_t ada_t_cond, vocab_size, downsample_factor;
    int32_t tok_bos, tok_eos, tok_audio, tok_begin_audio;
} vkv_hparams;

vkv_status vkv_gguf_hparams(const vkv_gguf *gguf, vkv_hparams *out);

/* ---------------------------------------------------------------------------
 * A model in device memory: every tensor of the file at its data-section
 * offset in one device allocation (the file's bytes unchanged, so Q4_K/Q6_K
 * or Q8_0 rows are what the kernels read), and the description the entry points take,
 * by the reference's tensor names (src/voxtral.cpp:1193-1265).  Streamed from
 * the file through pinned staging buffers on the given HIP stream (host
 * copies on up to 8 threads); the call
 * returns when the upload is complete.  MODEL_ERROR when a tensor the
 * realtime model requires is missing or has an unsupported type (matrices:
 * Q4_K, Q6_K or Q8_0, a layer's Q/K/V all Q8_0 or none, W1 and W3 alike).
 * ------------------------------------------------------------------------- */
typedef struct vkv_model vkv_model;

typedef struct vkv_model_view {
    vkv_hparams hp;
    vkv_enc_model enc;             /* layers: the model's own array */
    vkv_dec_model dec;             /* ada_scale of every layer NULL (session input) */
    vkv_adapter adapter;
    const void *conv0_w, *conv1_w; /* f16 [out][in][3] */
    const float *conv0_b, *conv1_b;
    const float *mel_filters;      /* audio.mel_filters or NULL */
    uint64_t device_bytes;         /* the allocation holding every tensor */
} vkv_model_view;

vkv_status vkv_model_load(const char *path, int32_t device, void *hip_stream, vkv_model **out);
vkv_status vkv_model_free(vkv_model *model);
vkv_status vkv_model_get_view(const vkv_model *model, vkv_model_view *out);
/* device address of a tensor by name, NULL when absent; info may be NULL */
const void *vkv_model_tensor(const vkv_model *model, const char *name, vkv_gguf_tensor *info);
/* Every decoder layer's ada scale (vkv_ada_scale with the layer's
 * dec.blk.N.ada0 / ada2 weights) at time value t into scales [n_layers][dim]
 * (caller's device memory, kept by the model's view from then on:
 * dec.layers[l].ada_scale = scales + l * dim).  A model without ada
 * conditioning leaves the view alone. */
vkv_status vkv_model_set_ada(vkv_model *model, float t, float *scales, void *hip_stream);

/* ---------------------------------------------------------------------------
 * Seeded synthetic rows (integer Irwin-Hall N(0,1), bit-identical to the CPU
 * generator used by the tests).  Row (s, l, p) = key(seed, tag, s0+i, l0+j,
 * p0+k) is written at dst + (i*s_stride + j*l_stride + k*p_stride) * row_len.
 * ------------------------------------------------------------------------- */
vkv_status vkv_synth_rows(float *dst, int32_t row_len, uint64_t seed, uint32_t tag, int64_t s0,
                          int32_t ns, int64_t s_stride, int64_t l0, int32_t nl, int64_t l_stride,
                          int64_t p0, int32_t np, int64_t p_stride, void *hip_stream);

/* ---------------------------------------------------------------------------
 * Diagnostics.
 * ------------------------------------------------------------------------- */
uint32_t vkv_api_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char *vkv_last_error(void);
/* hipError_t of the last BACKEND_ERROR on this thread (0 if none). */
int32_t vkv_last_backend_code(void);

#ifdef __cplusplus
}
#endif
#endif
