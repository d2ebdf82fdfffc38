// gfx950 matrix-vector products of the decoder step on ggml k-quant weights.
//
// ggml_mul_mat(W, x) with one token (src/voxtral.cpp:2656-2659 Q/K/V, :2857
// O-projection, :2878-2882 SwiGLU FFN) on Q4_K / Q6_K rows
// (src/voxtral-quantize.cpp:148-159), computed the way ggml's CPU path does:
// x is quantized to Q8_K (f32 scale per 256, int8 codes, 16-element sums) and
// each row is an integer dot product per block, scaled by fp16(d) * d_x (and
// for Q4_K minus fp16(dmin) * d_x * sum of mins x 32-element sums).  Q8_0
// rows (the files src/voxtral-quantize.cpp:95-96 writes) take a q8_0 image of
// x instead (ggml's x86 quantize_row_q8_0: fp16 d per 32 elements, codes
// rint(x * 127 / amax)), and each 32-weight block contributes its integer
// dot times fp16(d_w) * d_x.
//
//   k_matvec     -- one launch for up to four matrices that read the same x:
//                   prologue = optional RMSNorm x weight (x (1 + ada)) and the
//                   Q8_K quantization, into LDS, while the first weight loads
//                   are in flight; body = each wave streams whole rows, each
//                   lane one quarter of a 256-weight block (64 weights) with
//                   v_dot4_i32_i8, the row sum by a wave reduction; epilogue =
//                   store, residual add, or silu(W0 x) * (W1 x).
//   k_q8k_quant  -- the same prologue alone, to global memory in ggml's
//                   block_q8_K layout.
//   k_kq_dequant -- ggml dequantize_row_q4_K / _q6_K / _q8_0 (get_rows on the token
//                   embedding table, src/voxtral.cpp:3008, + the audio
//                   embedding, :3019).
//   k_argmax     -- ggml_argmax of the logits (src/voxtral.cpp:2970).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "vkv_internal.h"

namespace vkv {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));

constexpr int kQ4Bytes = 144;
constexpr int kQ6Bytes = 210;
constexpr int kQ8Bytes = 34;                   // one block_q8_0: fp16 d, 32 int8
constexpr int kQ8Per256 = 8 * kQ8Bytes;        // bytes of 256 Q8_0 weights

// the weight format a work group streams (one per work group)
enum WKind { kWQ4 = 0, kWQ6 = 1, kWQ8 = 2 };
constexpr uint32_t kOob = 0xFFFFFF00u;   // buffer offset past every resource: loads read 0

// Q8_K image of the input vector, per work group (q8_0 image for Q8_0 rows:
// xq and, in bs32, the f32 value of each 32-element block's fp16 d).
struct ActSmem {
    int8_t xq[kMvMaxIn];                 // codes
    int32_t bs32[kMvMaxIn / 32];         // sums of 32 codes (Q4_K sub-blocks)
    int32_t bs16[kMvMaxIn / 16];         // sums of 16 codes, order [b][n][h][g] (Q6_K)
    float dx[kMvMaxIn / 256];            // block scales
    double ss[kMvMaxIn / 256];           // per-block sums of squares (the norm)
};

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Cross-lane reductions by DPP inside each 16-lane row (0xB1 / 0x4E = quad
// xor 1 / 2, 0x141 = half-row mirror, 0x140 = row mirror) and readlane across
// the four rows: no LDS traffic, a uniform result.
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, dppi<CTRL>(__builtin_bit_cast(int, v)));
}
template <int CTRL>
__device__ __forceinline__ double dppd(double v) {
    int2 p = __builtin_bit_cast(int2, v);
    p.x = dppi<CTRL>(p.x);
    p.y = dppi<CTRL>(p.y);
    return __builtin_bit_cast(double, p);
}
__device__ __forceinline__ int lane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, lane_i(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double lane_d(double v, int l) {
    int2 p = __builtin_bit_cast(int2, v);
    return __builtin_bit_cast(double, int2{lane_i(p.x, l), lane_i(p.y, l)});
}

__device__ __forceinline__ double wave_sum_d(double v) {
    v += dppd<0xB1>(v);
    v += dppd<0x4E>(v);
    v += dppd<0x141>(v);
    v += dppd<0x140>(v);
    return (lane_d(v, 0) + lane_d(v, 16)) + (lane_d(v, 32) + lane_d(v, 48));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    v += dppf<0x141>(v);
    v += dppf<0x140>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Max over the 16 lanes of a DPP row (every lane of the row receives it).
__device__ __forceinline__ uint32_t row_max_u(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)dppi<0xB1>(x));
    x = (int)max((uint32_t)x, (uint32_t)dppi<0x4E>(x));
    x = (int)max((uint32_t)x, (uint32_t)dppi<0x141>(x));
    x = (int)max((uint32_t)x, (uint32_t)dppi<0x140>(x));
    return (uint32_t)x;
}

// One Q8_K block held by a 16-lane row, lane l with elements 16l..16l+15:
// the codes packed 4 per dword, the sum of the lane's 16 codes, of 32 codes
// (lanes 2k, 2k+1 hold the same) and d.  The same arithmetic as q8k_block
// (ggml quantize_row_q8_K_ref).  The first element of largest |h|: each lane
// keeps its own first one (strict >, in element order), the row maximum of
// |h| picks the value, and the row maximum of a key that orders the lanes
// holding it by smallest lane (lane l holds elements before lane l + 1's)
// carries the element's sign.
struct QBlock16 {
    uint32_t packed[4];
    int s16, s32;
    float d;
};
__device__ __forceinline__ QBlock16 q8k_block16(const float (&e)[16], int l) {
#pragma clang fp contract(off)
    float mv = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) mv = fabsf(e[k]) > fabsf(mv) ? e[k] : mv;
    const uint32_t amb = __builtin_bit_cast(uint32_t, fabsf(mv));
    const uint32_t mxa = row_max_u(amb);
    const uint32_t key = (amb == mxa && mxa != 0u)
                             ? ((uint32_t)(16 - l) << 1) | (__builtin_bit_cast(uint32_t, mv) >> 31)
                             : 0u;
    const uint32_t kmax = row_max_u(key);
    int q[16];
    QBlock16 r;
    r.d = 0.0f;
    if (mxa != 0u) {
        const float mx = __builtin_bit_cast(float, mxa | (kmax & 1u) << 31);
        const float iscale = -127.0f / mx;
#pragma unroll
        for (int k = 0; k < 16; ++k) q[k] = min(127, (int)__builtin_rintf(iscale * e[k]));
        r.d = 1.0f / iscale;
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) q[k] = 0;
    }
    int sum = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        r.packed[w] = (uint32_t)(q[4 * w] & 255) | (uint32_t)(q[4 * w + 1] & 255) << 8 |
                      (uint32_t)(q[4 * w + 2] & 255) << 16 | (uint32_t)(q[4 * w + 3] & 255) << 24;
        sum += (q[4 * w] + q[4 * w + 1]) + (q[4 * w + 2] + q[4 * w + 3]);
    }
    r.s16 = sum;
    r.s32 = sum + dppi<0xB1>(sum);
    return r;
}

// One ggml block_q8_0 of the input held by lanes 2k, 2k + 1 of a 16-lane
// row, 16 elements each: quantize_row_q8_0 as ggml's x86 CPU backend computes
// it -- amax over the 32 elements, d = amax / 127 rounded to fp16 (nearest
// even), codes rint(x * (127 / amax)) (one f32 product, half to even).
struct QBlock0 {
    uint32_t packed[4];
    float d;   // f32 value of the fp16 d
};
__device__ __forceinline__ QBlock0 q8_0_block16(const float (&e)[16]) {
#pragma clang fp contract(off)
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) am = fmaxf(am, fabsf(e[k]));
    am = fmaxf(am, dppf<0xB1>(am));   // the partner lane's half
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    QBlock0 r;
    r.d = (float)(_Float16)(am / 127.0f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        int q[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = (int)__builtin_rintf(e[4 * w + t] * id);
        r.packed[w] = (uint32_t)(q[0] & 255) | (uint32_t)(q[1] & 255) << 8 |
                      (uint32_t)(q[2] & 255) << 16 | (uint32_t)(q[3] & 255) << 24;
    }
    return r;
}

// Q8_K quantization of rms_norm(x) * norm_w (* (1 + ada)), or of x itself
// (norm_w == nullptr).  In round k a wave holds 4 blocks, one per 16-lane
// row: lane (row r, l) has elements [16 l, 16 l + 16) of block 16 k + 4 w +
// r, so every reduction over a block stays inside a DPP row and the wave's
// blocks are quantized side by side.  Rounding follows the CPU path step by
// step: the squares are f32 products summed in double, mean = f32(sum / n),
// scale = 1 / sqrtf(mean + eps), h = (x * scale) * w, then h + h * ada;
// iscale = -127 / (first element of largest |h|), code = min(127,
// rint(iscale * h)), d = 1 / iscale.
//
// Split in two so that a caller can issue its own loads between them: the
// input loads of act_load retire first (vmcnt counts in issue order), and
// act_finish then waits for them alone.  NBW = 4 x rounds (float4 per lane);
// with NORM_EARLY the norm weights (and the ada row) are loaded up front too,
// with BIAS_EARLY the norm's bias as well (absent vectors read x instead:
// one load path, unused).  Q80: the q8_0 image instead of Q8_K (codes in xq,
// the blocks' d in bs32; the same rounding of the normed input).
template <int NBW, bool NORM_EARLY, bool BIAS_EARLY = false>
struct ActRegs {
    float4 x[NBW];
    float4 w[NORM_EARLY ? NBW : 1];
    float4 a[NORM_EARLY ? NBW : 1];
    float4 b[BIAS_EARLY ? NBW : 1];
};

template <int NBW, bool NE, bool NB>
__device__ __forceinline__ void act_load(ActRegs<NBW, NE, NB> &r, const float *__restrict__ x,
                                         int n, const float *__restrict__ nw,
                                         const float *__restrict__ ada,
                                         const float *__restrict__ nbias = nullptr) {
    const int lane = threadIdx.x & 63, nb = n >> 8;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float *wp = nw ? nw : x, *ap = ada ? ada : x, *bp = nbias ? nbias : x;
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
        const int bb = 16 * (i >> 2) + 4 * wave + (lane >> 4);
        const int b = bb < nb ? bb : 0;   // rows past the last block read block 0, unused
        const int e0 = 256 * b + 16 * (lane & 15) + 4 * (i & 3);
        r.x[i] = *reinterpret_cast<const float4 *>(x + e0);
        if (NE) {
            r.w[i] = *reinterpret_cast<const float4 *>(wp + e0);
            r.a[i] = *reinterpret_cast<const float4 *>(ap + e0);
        }
        if (NB) r.b[i] = *reinterpret_cast<const float4 *>(bp + e0);
    }
}

template <int NBW, bool NE, bool NB, bool Q80 = false>
__device__ __forceinline__ void act_finish(const ActRegs<NBW, NE, NB> &r, int n,
                                           const float *__restrict__ nw,
                                           const float *__restrict__ ada, float eps, ActSmem &sm,
                                           uint8_t *__restrict__ gout,
                                           const float *__restrict__ nbias = nullptr) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x, lane = tid & 63, nb = n >> 8;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = lane & 15;
    float scale = 1.0f;
    if (nw) {
        // Sum of squares per block (the 16 lanes' f32 products summed in
        // double, the lanes by DPP, lane 0's sum kept), then over the blocks
        // in block order: the fused-input products' order, so both images of
        // a row are equal bit for bit.
#pragma unroll
        for (int k = 0; k < NBW / 4; ++k) {
            if (16 * k + 4 * wave >= nb) break;
            const int bb = 16 * k + 4 * wave + (lane >> 4);
            double s = 0.0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = r.x[4 * k + j];
                s += (double)(v.x * v.x);
                s += (double)(v.y * v.y);
                s += (double)(v.z * v.z);
                s += (double)(v.w * v.w);
            }
            s += dppd<0xB1>(s);
            s += dppd<0x4E>(s);
            s += dppd<0x141>(s);
            s += dppd<0x140>(s);
            if (bb < nb && l == 0) sm.ss[bb] = s;
        }
        __syncthreads();
        double tot = 0.0;
        for (int b = 0; b < nb; ++b) tot += sm.ss[b];
        const float mean = (float)(tot / (double)n);
        scale = 1.0f / sqrtf(mean + eps);
    }
#pragma unroll
    for (int k = 0; k < NBW / 4; ++k) {
        if (16 * k + 4 * wave >= nb) break;   // no block of this wave in this round
        const int bb = 16 * k + 4 * wave + (lane >> 4);
        const bool valid = bb < nb;           // rows past the last block compute, store nothing
        const int b = valid ? bb : 0;
        float e[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 v = r.x[4 * k + j];
            e[4 * j] = v.x;
            e[4 * j + 1] = v.y;
            e[4 * j + 2] = v.z;
            e[4 * j + 3] = v.w;
        }
        if (nw) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e0 = 256 * b + 16 * l + 4 * j;
                const float4 w4 = NE ? r.w[4 * k + j] : *reinterpret_cast<const float4 *>(nw + e0);
                const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    e[4 * j + t] = e[4 * j + t] * scale;
                    e[4 * j + t] = e[4 * j + t] * w[t];
                }
                if (nbias) {
                    // + the norm's bias (the encoder's norms, src/voxtral.cpp:1855-1861)
                    const float4 b4 = NB ? r.b[4 * k + j] : *reinterpret_cast<const float4 *>(nbias + e0);
                    e[4 * j] = e[4 * j] + b4.x;
                    e[4 * j + 1] = e[4 * j + 1] + b4.y;
                    e[4 * j + 2] = e[4 * j + 2] + b4.z;
                    e[4 * j + 3] = e[4 * j + 3] + b4.w;
                }
                if (ada) {
                    const float4 a4 =
                        NE ? r.a[4 * k + j] : *reinterpret_cast<const float4 *>(ada + e0);
                    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const float tt = e[4 * j + t] * av[t];
                        e[4 * j + t] = e[4 * j + t] + tt;
                    }
                }
            }
        }
        if constexpr (Q80) {
            const QBlock0 qb = q8_0_block16(e);
            if (!valid) continue;
            *reinterpret_cast<u32x4_t *>(&sm.xq[256 * b + 16 * l]) =
                u32x4_t{qb.packed[0], qb.packed[1], qb.packed[2], qb.packed[3]};
            if ((l & 1) == 0) sm.bs32[8 * b + (l >> 1)] = __builtin_bit_cast(int32_t, qb.d);
            continue;
        }
        const QBlock16 qb = q8k_block16(e, l);
        if (!valid) continue;
        if (gout) {
            uint8_t *blk = gout + (size_t)b * 292;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                *reinterpret_cast<uint32_t *>(blk + 4 + 16 * l + 4 * w) = qb.packed[w];
            *reinterpret_cast<int16_t *>(blk + 260 + 2 * l) = (int16_t)qb.s16;
            if (l == 0) *reinterpret_cast<float *>(blk) = qb.d;
        } else {
            *reinterpret_cast<u32x4_t *>(&sm.xq[256 * b + 16 * l]) =
                u32x4_t{qb.packed[0], qb.packed[1], qb.packed[2], qb.packed[3]};
            // 16-group l of the block, in the Q6_K order [b][n][h][g]
            sm.bs16[16 * b + 8 * (l >> 3) + 4 * (l & 1) + ((l >> 1) & 3)] = qb.s16;
            if ((l & 1) == 0) sm.bs32[8 * b + (l >> 1)] = qb.s32;
            if (l == 0) sm.dx[b] = qb.d;
        }
    }
    __syncthreads();
}

// Raw bytes of one lane's quarter block.  Q4_K: a, b = 32 code bytes, c = the
// 16-byte header (d, dmin, scales).  Q6_K (blocks are only 2-byte aligned):
// a, b, c = 16 bytes of ql (low), ql (high), qh read from the dword-aligned
// address below, with one more dword each in ax, bx, cx; s = 12 bytes
// covering the lane's 8 scales; dh = fp16 d.
struct FragQ4 {
    u32x4_t a, b, c;
};
struct FragQ6 {
    u32x4_t a, b, c;
    uint32_t ax, bx, cx;
    u32x2_t s01;
    uint32_t s2, dh;
};

__device__ __forceinline__ FragQ4 load_q4(__amdgpu_buffer_rsrc_t rs, uint32_t off, int c) {
    FragQ4 f;
    f.a = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 + 32 * c, 0, 0));
    f.b = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32 + 32 * c, 0, 0));
    f.c = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    return f;
}

__device__ __forceinline__ FragQ6 load_q6(__amdgpu_buffer_rsrc_t rs, uint32_t off, int n, int h) {
    FragQ6 f;
    const uint32_t al = off & ~3u;     // off is even: al = off or off - 2
    const uint32_t o0 = al + 64 * n + 16 * h, o1 = o0 + 32, oh = al + 128 + 32 * n + 16 * h;
    const uint32_t os = al + 192 + 8 * n;
    f.a = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, o0, 0, 0));
    f.ax = __builtin_amdgcn_raw_buffer_load_b32(rs, o0 + 16, 0, 0);
    f.b = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, o1, 0, 0));
    f.bx = __builtin_amdgcn_raw_buffer_load_b32(rs, o1 + 16, 0, 0);
    f.c = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, oh, 0, 0));
    f.cx = __builtin_amdgcn_raw_buffer_load_b32(rs, oh + 16, 0, 0);
    f.s01 = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, os, 0, 0));
    f.s2 = __builtin_amdgcn_raw_buffer_load_b32(rs, os + 8, 0, 0);
    f.dh = __builtin_amdgcn_raw_buffer_load_b16(rs, off + 208, 0, 0);
    return f;
}

// Q8_0: a lane task is two consecutive 34-byte blocks (64 weights) at byte
// 68 t of the row, 4-byte aligned (rows are multiples of 272 bytes): 17 dwords.
struct FragQ8 {
    u32x4_t a, b, c, e;
    uint32_t x;
};

__device__ __forceinline__ FragQ8 load_q8(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    FragQ8 f;
    f.a = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    f.b = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0));
    f.c = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32, 0, 0));
    f.e = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 48, 0, 0));
    f.x = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 64, 0, 0);
    return f;
}

// The activation side of one lane's task for a step (same for every row).
struct XFrag {
    i32x4_t x[4];     // 64 codes
    int32_t bs[4];    // Q4_K: bs[0..1] = sums of sub-blocks 2c, 2c+1; Q6_K: g = 0..3
    float dx;
};

__device__ __forceinline__ XFrag x_q4(const ActSmem &sm, int t) {
    const int b = t >> 2, c = t & 3;
    XFrag f;
    const i32x4_t *p = reinterpret_cast<const i32x4_t *>(&sm.xq[256 * b + 64 * c]);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.x[i] = p[i];
    const u32x2_t s = *reinterpret_cast<const u32x2_t *>(&sm.bs32[8 * b + 2 * c]);
    f.bs[0] = (int32_t)s.x;
    f.bs[1] = (int32_t)s.y;
    f.bs[2] = f.bs[3] = 0;
    f.dx = sm.dx[b];
    return f;
}

__device__ __forceinline__ XFrag x_q6(const ActSmem &sm, int t) {
    const int b = t >> 2, n = (t >> 1) & 1, h = t & 1;
    XFrag f;
#pragma unroll
    for (int g = 0; g < 4; ++g)
        f.x[g] = *reinterpret_cast<const i32x4_t *>(&sm.xq[256 * b + 128 * n + 32 * g + 16 * h]);
    const i32x4_t s = *reinterpret_cast<const i32x4_t *>(&sm.bs16[16 * b + 8 * n + 4 * h]);
    f.bs[0] = s.x;
    f.bs[1] = s.y;
    f.bs[2] = s.z;
    f.bs[3] = s.w;
    f.dx = sm.dx[b];
    return f;
}

// q8_0 image: the task's 64 codes and its two blocks' d (f32 bits in bs[0..1])
__device__ __forceinline__ XFrag x_q8(const ActSmem &sm, int t) {
    XFrag f;
    const i32x4_t *p = reinterpret_cast<const i32x4_t *>(&sm.xq[64 * t]);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.x[i] = p[i];
    const u32x2_t s = *reinterpret_cast<const u32x2_t *>(&sm.bs32[2 * t]);
    f.bs[0] = (int32_t)s.x;
    f.bs[1] = (int32_t)s.y;
    f.bs[2] = f.bs[3] = 0;
    f.dx = 0.0f;
    return f;
}

__device__ __forceinline__ int dot16(const uint32_t (&w)[4], const i32x4_t &x, int acc) {
    acc = __builtin_amdgcn_sdot4((int)w[0], x.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w[1], x.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w[2], x.z, acc, false);
    return __builtin_amdgcn_sdot4((int)w[3], x.w, acc, false);
}

__device__ __forceinline__ float compute_q4(const FragQ4 &f, const XFrag &x, int c) {
    const uint32_t u0 = f.c.y, u1 = f.c.z, u2 = f.c.w;
    const uint32_t sc_lo = u0 & 0x3f3f3f3fu, mn_lo = u1 & 0x3f3f3f3fu;
    const uint32_t sc_hi = (u2 & 0x0f0f0f0fu) | ((u0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((u2 >> 4) & 0x0f0f0f0fu) | ((u1 >> 2) & 0x30303030u);
    const uint32_t scw = c < 2 ? sc_lo : sc_hi, mnw = c < 2 ? mn_lo : mn_hi;
    const uint32_t sh = 16u * (uint32_t)(c & 1);
    const int sc_a = (int)((scw >> sh) & 255u), sc_b = (int)((scw >> (sh + 8)) & 255u);
    const int m_a = (int)((mnw >> sh) & 255u), m_b = (int)((mnw >> (sh + 8)) & 255u);
    const uint32_t w[8] = {f.a.x, f.a.y, f.a.z, f.a.w, f.b.x, f.b.y, f.b.z, f.b.w};
    uint32_t lo[2][4], hi[2][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i >> 2][i & 3] = w[i] & 0x0f0f0f0fu;
        hi[i >> 2][i & 3] = (w[i] >> 4) & 0x0f0f0f0fu;
    }
    const int dot_a = dot16(lo[1], x.x[1], dot16(lo[0], x.x[0], 0));
    const int dot_b = dot16(hi[1], x.x[3], dot16(hi[0], x.x[2], 0));
    const int isum = sc_a * dot_a + sc_b * dot_b;
    const int imin = m_a * x.bs[0] + m_b * x.bs[1];
    const float d = h2f(f.c.x & 0xffffu) * x.dx, dmin = h2f(f.c.x >> 16) * x.dx;
    // one explicit fma (not left to contraction, which may fuse either
    // product depending on the kernel instantiation)
    return fmaf(d, (float)isum, -(dmin * (float)imin));
}

__device__ __forceinline__ float compute_q6(const FragQ6 &f, const XFrag &x, uint32_t mis, int h) {
    uint32_t l0[4], l1[4], qh[4];
    const uint32_t a[5] = {f.a.x, f.a.y, f.a.z, f.a.w, f.ax};
    const uint32_t b[5] = {f.b.x, f.b.y, f.b.z, f.b.w, f.bx};
    const uint32_t c[5] = {f.c.x, f.c.y, f.c.z, f.c.w, f.cx};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        l0[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], mis);
        l1[i] = __builtin_amdgcn_alignbyte(b[i + 1], b[i], mis);
        qh[i] = __builtin_amdgcn_alignbyte(c[i + 1], c[i], mis);
    }
    const uint32_t s_lo = __builtin_amdgcn_alignbyte(f.s01.y, f.s01.x, mis);
    const uint32_t s_hi = __builtin_amdgcn_alignbyte(f.s2, f.s01.y, mis);
    uint32_t q[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[0][i] = (l0[i] & 0x0f0f0f0fu) | ((qh[i] << 4) & 0x30303030u);
        q[1][i] = (l1[i] & 0x0f0f0f0fu) | ((qh[i] << 2) & 0x30303030u);
        q[2][i] = ((l0[i] >> 4) & 0x0f0f0f0fu) | (qh[i] & 0x30303030u);
        q[3][i] = ((l1[i] >> 4) & 0x0f0f0f0fu) | ((qh[i] >> 2) & 0x30303030u);
    }
    const uint32_t hs = 8u * (uint32_t)h;
    const int sc[4] = {(int)(int8_t)(s_lo >> hs), (int)(int8_t)(s_lo >> (hs + 16)),
                       (int)(int8_t)(s_hi >> hs), (int)(int8_t)(s_hi >> (hs + 16))};
    int isum = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) isum += sc[g] * (dot16(q[g], x.x[g], 0) - 32 * x.bs[g]);
    return (h2f(f.dh) * x.dx) * (float)isum;
}
// Two Q8_0 blocks: block 2t's d is the first half of dword 0 and its codes
// bytes 2..33 (realigned by 2), block 2t + 1's d the second half of dword 8
// and its codes dwords 9..16; each block's integer dot times fp16(d_w) * d_x
// (ggml_vec_dot_q8_0_q8_0's per-block term).  The two terms meet in one
// explicit fma: left to contraction, which product fuses depended on the
// kernel instantiation, and the fused-argmax logits differed from the plain
// ones in the last bit.
__device__ __forceinline__ float compute_q8(const FragQ8 &f, const XFrag &x) {
#pragma clang fp contract(off)
    const uint32_t w[17] = {f.a.x, f.a.y, f.a.z, f.a.w, f.b.x, f.b.y, f.b.z, f.b.w, f.c.x,
                            f.c.y, f.c.z, f.c.w, f.e.x, f.e.y, f.e.z, f.e.w, f.x};
    uint32_t q0[2][4], q1[2][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q0[i >> 2][i & 3] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        q1[i >> 2][i & 3] = w[9 + i];
    }
    const int s0 = dot16(q0[1], x.x[1], dot16(q0[0], x.x[0], 0));
    const int s1 = dot16(q1[1], x.x[3], dot16(q1[0], x.x[2], 0));
    const float d0 = h2f(w[0] & 0xffffu) * __builtin_bit_cast(float, x.bs[0]);
    const float d1 = h2f(w[8] >> 16) * __builtin_bit_cast(float, x.bs[1]);
    return fmaf((float)s1, d1, (float)s0 * d0);
}

template <int WK>
__device__ __forceinline__ XFrag xfrag(const ActSmem &sm, int t) {
    if constexpr (WK == kWQ4) return x_q4(sm, t);
    else if constexpr (WK == kWQ8) return x_q8(sm, t);
    else return x_q6(sm, t);
}

// Where unit u of a wave reads its weights.  The buffer descriptor is built
// per load from a uniform pointer and size (a select between two descriptors
// is lowered through scratch memory).  Units past the wave's last one read
// zeros (an offset past the buffer), so every load is unconditional.
struct UnitMap {
    const uint8_t *w0, *w1;
    uint32_t n0, n1;
    int row0;
    uint32_t rbytes, bbytes;
    int tasks, lane, mats, units;
    bool swiglu;

    template <int S, int WK>
    __device__ __forceinline__ auto load(int u) const {
        const int step = u % S;
        const bool second = swiglu && ((u / S) & 1);
        const int row = row0 + u / (S * mats);
        const int t = 64 * step + lane;
        // a Q8_0 task's two blocks are 68 bytes from the previous task's
        const uint32_t toff = WK == kWQ8 ? (uint32_t)t * (2 * kQ8Bytes) : (uint32_t)(t >> 2) * bbytes;
        const uint32_t off = t < tasks && u < units ? (uint32_t)row * rbytes + toff : kOob;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(second ? w1 : w0), (short)0, (int)(second ? n1 : n0), 0x00020000);
        if constexpr (WK == kWQ4) return load_q4(rs, off, t & 3);
        else if constexpr (WK == kWQ8) return load_q8(rs, off);
        else return load_q6(rs, off, (t >> 1) & 1, t & 1);
    }
};

// a.out[k] for a uniform k without indexing the kernel-argument array (a
// dynamic index makes the compiler copy the array to scratch)
__device__ __forceinline__ MvOut out_at(const MvArgs &a, int k) {
    MvOut o = a.out[0];
    if (k == 1) o = a.out[1];
    if (k == 2) o = a.out[2];
    if (k == 3) o = a.out[3];
    return o;
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// The fused argmax's end: the work group's best key (waves through LDS) is
// maxed into *a.amax with one 64-bit atomic; the work group that finishes last
// (the counter) reads the result, writes the row, and clears both words.  The
// counter add is issued only after the max has returned, so every earlier
// work group's max is in place when the last one reads.  Keys order values
// as floats (sign-flipped bits) and, between equal values, the larger row
// wins: ggml_vec_argmax_f32's last index of the maximum.
__device__ __forceinline__ void argmax_publish(const MvArgs &a, unsigned long long best) {
    __shared__ unsigned long long wbest[4];
    __shared__ int last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wbest[0];
        for (int w = 1; w < 4; ++w) b = wbest[w] > b ? wbest[w] : b;
        const unsigned long long prev = atomicMax(a.amax, b);
        asm volatile("" ::"v"(prev));   // the max has returned before the count
        const unsigned int done = atomicAdd(a.amax_count, 1u);
        last = done == gridDim.x - 1;
    }
    __syncthreads();
    if (last && threadIdx.x == 0) {
        const unsigned long long k = atomicMax(a.amax, 0ull);
        a.amax_out[0] = (int32_t)(uint32_t)(k & 0xffffffffull);
        atomicExch(a.amax, 0ull);
        atomicExch(a.amax_count, 0u);
    }
}

// Unit u of a wave = (row, step): step s of a row covers lane tasks
// [64 s, 64 s + 64) of the row's 4 * nb quarter blocks.  With SWIGLU the rows
// alternate between the two matrices: u -> (pair u / 2S, matrix (u / S) & 1).
// WK (the work group's weight format) is a template parameter so that every
// load writes its final registers (a load feeding a merge of two paths would
// be copied, and the copy waits for the load).  Q8_0 rows keep D6 units in
// flight (17 dwords a task against Q6_K's 19).
template <int S, int D4, int D6, bool ONE, int WK, bool AMAX, bool NE>
__device__ __forceinline__ void matvec_body(const MvArgs &a, const MvOut &o0, const MvOut &ob,
                                            int row0, int nrow, ActSmem &sm) {
    const int lane = threadIdx.x & 63;
    const bool swiglu = a.swiglu != 0;
    const int mats = swiglu ? 2 : 1;
    const int units = nrow * S * mats;
    const int nb = a.n_in >> 8, tasks = 4 * nb;
    const uint32_t bbytes = WK == kWQ4 ? kQ4Bytes : WK == kWQ8 ? kQ8Per256 : kQ6Bytes;
    const uint32_t rbytes = (uint32_t)nb * bbytes;
    const UnitMap um{o0.w, ob.w, rbytes * (uint32_t)o0.n_rows, rbytes * (uint32_t)ob.n_rows, row0,
                     rbytes, bbytes, tasks, lane, mats, units, swiglu};

    constexpr int D = WK == kWQ4 ? D4 : D6;   // units in flight per dtype
    constexpr int NBW = S == 1 ? 4 : 4 * S;   // n_in <= 4096 / 12288
    ActRegs<NBW, NE> ar;
    act_load(ar, a.x, a.n_in, a.norm_w, a.ada);
    using Frag = std::conditional_t<WK == kWQ4, FragQ4, std::conditional_t<WK == kWQ8, FragQ8, FragQ6>>;
    // Every weight load is unconditional (units past the end read zeros):
    // a load issued on one path only makes the compiler's wait counts assume
    // it absent, and the input quantization then waited for all of them.
    // The loads stay in unit order (scheduling barriers): the unit loop's
    // waits hold for its first pass too, and a unit requested last there
    // made every pass wait for all of them.
    Frag f[D];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < D; ++k) {
        f[k] = um.load<S, WK>(k);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The residual of the wave's rows (lane l: row row0 + l; a wave has at
    // most 64 rows), requested up front: loaded at a row's end it waited for
    // every weight load in flight.  Without a residual it reads y, unused.
    const float *ap = o0.add ? o0.add : o0.y;
    const float addv = ap[min(row0 + min(lane, max(nrow - 1, 0)), o0.n_rows - 1)];
    __builtin_amdgcn_sched_barrier(0);
    act_finish<NBW, NE, false, WK == kWQ8>(ar, a.n_in, a.norm_w, a.ada, a.eps, sm, nullptr);

    const XFrag xr = xfrag<WK>(sm, min(lane, tasks - 1));   // the only step when S == 1

    float acc = 0.0f, first = 0.0f;
    unsigned long long best = 0;   // argmax key: order key of the value << 32 | row
    // unit u (fragment fr): its share of the row's sum, and the row's end
    auto unit = [&](const Frag &fr, int u) __attribute__((always_inline)) {
        const int step = u % S, m = swiglu ? (u / S) & 1 : 0;
        const int row = row0 + u / (S * mats);
        const int t = 64 * step + lane;
        const XFrag xf = S == 1 ? xr : xfrag<WK>(sm, min(t, tasks - 1));
        float c;
        if constexpr (WK == kWQ4) {
            c = compute_q4(fr, xf, t & 3);
        } else if constexpr (WK == kWQ8) {
            c = compute_q8(fr, xf);
        } else {
            // Q6_K block (row, b) starts at 210 (row nb + b): 2 mod 4 when odd
            const uint32_t mis = 2u * (uint32_t)((row * nb + (t >> 2)) & 1);
            c = compute_q6(fr, xf, mis, t & 1);
        }
        acc += t < tasks ? c : 0.0f;
        if (step == S - 1 && u < units) {
            const float r = wave_sum(acc);
            acc = 0.0f;
            if (!swiglu) {
                const float res = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, addv), u / (S * mats)));
                const float yv = a.gelu ? gelu_erf(r) : o0.add ? res + r : r;
                if (lane == 0) o0.y[row] = yv;
                if constexpr (AMAX) {
                    const uint32_t b = __builtin_bit_cast(uint32_t, yv);
                    const uint32_t ok = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
                    const unsigned long long key = ((unsigned long long)ok << 32) | (uint32_t)row;
                    best = key > best ? key : best;
                }
            } else if (m == 0) {
                first = r;
            } else if (lane == 0) {
                o0.y[row] = silu(first) * r;
            }
        }
    };
    if constexpr (ONE) {
        // every unit was requested above (the launch checked units <= D):
        // no refills, and each unit waits for its own loads only
#pragma unroll
        for (int k = 0; k < D; ++k)
            if (k < units) unit(f[k], k);
    } else {
        for (int u0 = 0; u0 < units; u0 += D) {
#pragma unroll
            for (int k = 0; k < D; ++k) {
                unit(f[k], u0 + k);
                // the next load into this slot once its fragment is consumed,
                // so it can write the slot's own registers (a load into other
                // registers is copied back at the loop's end, and the copy
                // waits for it)
                f[k] = um.load<S, WK>(u0 + k + D);
            }
        }
    }
    if constexpr (AMAX) argmax_publish(a, best);
}

// D4 / D6: a wave's units in flight for Q4_K / Q6_K (and Q8_0) rows; ONE: every wave's
// units fit (the launch picks it from the units per wave, so that a decoder
// product's wave requests all its weights at once and streams nothing).
template <int S, int D4, int D6, bool ONE, bool AMAX>
__global__ void __launch_bounds__(256) k_matvec(MvArgs a) {
    __shared__ ActSmem sm;
    // wave-uniform (readfirstlane): the row range and the unit loop follow
    // from it, and a per-lane wave makes the loop divergent
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int seg = 0;
#pragma unroll
    for (int k = 1; k < kMvMaxOuts; ++k)
        if (k < a.n_outs && (int)blockIdx.x >= a.out[k].wg0) seg = k;
    const MvOut o0 = out_at(a, seg);
    const MvOut ob = a.swiglu ? a.out[1] : o0;
    const int row0 = ((int)blockIdx.x - o0.wg0) * a.rows_per_wg + wave * (a.rows_per_wg >> 2);
    const int nrow = max(0, min(a.rows_per_wg >> 2, o0.n_rows - row0));
    // With a norm (S == 1: the inputs of up to 4096), its weights (and the ada
    // row) are requested together with x, so the norm costs one round trip.
    if (S == 1 && a.norm_w) {
        if (o0.dtype == VKV_DTYPE_Q4_K) matvec_body<S, D4, D6, ONE, kWQ4, AMAX, true>(a, o0, ob, row0, nrow, sm);
        else if (o0.dtype == VKV_DTYPE_Q8_0) matvec_body<S, D4, D6, ONE, kWQ8, AMAX, true>(a, o0, ob, row0, nrow, sm);
        else matvec_body<S, D4, D6, ONE, kWQ6, AMAX, true>(a, o0, ob, row0, nrow, sm);
    } else {
        if (o0.dtype == VKV_DTYPE_Q4_K) matvec_body<S, D4, D6, ONE, kWQ4, AMAX, false>(a, o0, ob, row0, nrow, sm);
        else if (o0.dtype == VKV_DTYPE_Q8_0) matvec_body<S, D4, D6, ONE, kWQ8, AMAX, false>(a, o0, ob, row0, nrow, sm);
        else matvec_body<S, D4, D6, ONE, kWQ6, AMAX, false>(a, o0, ob, row0, nrow, sm);
    }
}

__global__ void __launch_bounds__(256) k_q8k_quant(const float *x, int n, const float *nw,
                                                   const float *ada, float eps, uint8_t *out) {
    __shared__ ActSmem sm;
    ActRegs<kMvMaxIn / 1024, false> r;
    act_load(r, x, n, nw, ada);
    act_finish(r, n, nw, ada, eps, sm, out);
}

// ggml dequantize_row_q4_K / _q6_K / _q8_0 of elements i8 .. i8 + 7 of a row
__device__ __forceinline__ void kq_dequant8(int dtype, const uint8_t *__restrict__ src, int64_t i8,
                                            float out[8]) {
#pragma clang fp contract(off)
    const int64_t b = i8 >> 8;
    const int e0 = (int)(i8 & 255);
    if (dtype == VKV_DTYPE_Q4_K) {
        const uint8_t *blk = src + b * kQ4Bytes;
        const float d = h2f(blk[0] | blk[1] << 8), dmin = h2f(blk[2] | blk[3] << 8);
        const uint8_t *s = blk + 4;
        const int j = e0 >> 5;
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63;
            m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t *qs = blk + 16 + 32 * (j >> 1) + (e0 & 31);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = (j & 1) ? (qs[i] >> 4) : (qs[i] & 15);
            out[i] = d1 * (float)q - m1;
        }
    } else if (dtype == VKV_DTYPE_Q8_0) {
        // dequantize_row_q8_0: code * f32(d), a block per 32 elements
        const uint8_t *blk = src + (i8 >> 5) * kQ8Bytes;
        const float d = h2f(blk[0] | blk[1] << 8);
        const int8_t *qs = reinterpret_cast<const int8_t *>(blk + 2 + (i8 & 31));
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = (float)qs[i] * d;
    } else {
        const uint8_t *blk = src + b * kQ6Bytes;
        const float d = h2f(blk[208] | blk[209] << 8);
        const int n2 = e0 >> 7, g = (e0 >> 5) & 3, l0 = e0 & 31;
        const float ds = d * (float)(int8_t)blk[192 + 8 * n2 + 2 * g + (l0 >> 4)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int l = l0 + i;
            const uint8_t lo = blk[64 * n2 + 32 * (g & 1) + l];
            const int nib = g < 2 ? (lo & 15) : (lo >> 4);
            const int q = nib | (((blk[128 + 32 * n2 + l] >> (2 * g)) & 3) << 4);
            out[i] = ds * (float)(q - 32);
        }
    }
}

// ggml dequantize_row_q4_K / _q6_K / _q8_0, plus add[i] when add is given (the
// token embedding + audio embedding sum); one thread per 8 elements.
__global__ void __launch_bounds__(256) k_kq_dequant(int dtype, const uint8_t *__restrict__ src,
                                                    int64_t n, const float *__restrict__ add,
                                                    float *__restrict__ y,
                                                    unsigned long long *zero_words) {
#pragma clang fp contract(off)
    const int64_t i8 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    // the decoder token's argmax words start each token at zero
    if (zero_words && blockIdx.x == 0 && threadIdx.x < 2) zero_words[threadIdx.x] = 0ull;
    if (i8 >= n) return;
    float out[8];
    kq_dequant8(dtype, src, i8, out);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i8 + i] = add ? out[i] + add[i8 + i] : out[i];
}

// get_rows of up to kEmbedChunk token rows of a Q4_K / Q6_K / Q8_0 table, each plus
// its audio row when add is given (build_decoder_prefill_graph's tok_emb +
// audio_emb): row p = blockIdx.y is table row tok.id[p] into y row p, the
// audio row at (add_row0 + p) % add_ring of a ring (add_ring > 0) or row p.
// The host checked every id against the table's rows.
__global__ void __launch_bounds__(256) k_embed_rows(int dtype, const uint8_t *__restrict__ table,
                                                    int64_t row_bytes, EmbedTokens tok, int64_t n,
                                                    const float *__restrict__ add, int add_ring,
                                                    int add_row0, float *__restrict__ y,
                                                    unsigned long long *zero_words) {
#pragma clang fp contract(off)
    const int p = blockIdx.y;
    const int64_t i8 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (zero_words && blockIdx.x == 0 && p == 0 && threadIdx.x < 2) zero_words[threadIdx.x] = 0ull;
    if (i8 >= n) return;
    float out[8];
    kq_dequant8(dtype, table + (int64_t)tok.id[p] * row_bytes, i8, out);
    float *yr = y + (int64_t)p * n;
    if (add) {
        const float *ar = add + (int64_t)(add_ring > 0 ? (add_row0 + p) % add_ring : p) * n;
#pragma unroll
        for (int i = 0; i < 8; ++i) yr[i8 + i] = out[i] + ar[i8 + i];
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) yr[i8 + i] = out[i];
    }
}

// rms_norm(x_p) * w (+ b) per row, f32 out (the encoder's final norm,
// enc_apply_norm at src/voxtral.cpp:2368): the CPU path's rounding -- squares
// summed in double, mean rounded to f32, scale = 1/sqrtf(mean + eps),
// (x * scale) * w, then + b.  One work group per row.
__global__ void __launch_bounds__(256) k_rms_norm_rows(const float *__restrict__ x, int n,
                                                       const float *__restrict__ w,
                                                       const float *__restrict__ b, float eps,
                                                       float *y, int y_ring, int y_row0) {
#pragma clang fp contract(off)
    __shared__ double red[4];
    const int p = blockIdx.x;
    const float *xr = x + (int64_t)p * n;
    float *yr = y + (int64_t)(y_ring > 0 ? (y_row0 + p) % y_ring : p) * n;
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) s += (double)(xr[i] * xr[i]);
    s = wave_sum_d(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float mean = (float)(tot / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = xr[i] * scale;
        v = v * w[i];
        if (b) v = v + b[i];
        yr[i] = v;
    }
}

// y[r] = sum_k W[r][k] x[k] for a small f16, f32 or Q8_0 matrix (the ada
// MLP's second layer, [dim][ada_dim] with ada_dim = 32): the CPU path's
// vec-dot type for an f16 matrix is f16, so x is rounded to f16 and every
// product is exact in f32; f32 matrices take x as it is.  One wave per row,
// lanes over k.  Q8_0 rows (a Q8_0 file): x quantized per 32-element block
// as ggml's x86 quantize_row_q8_0 does, each block's integer dot times
// fp16(d_w) * d_x, the row by one lane (n_in is a few blocks).
__global__ void __launch_bounds__(256) k_rows_small(const void *__restrict__ w, int w_type,
                                                    const float *__restrict__ x, int n_in,
                                                    int n_rows, float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    if (w_type == VKV_DTYPE_Q8_0) {
#pragma clang fp contract(off)
        if (lane != 0) return;
        const uint8_t *wr = reinterpret_cast<const uint8_t *>(w) + (int64_t)row * (n_in / 32) * kQ8Bytes;
        float acc = 0.0f;
        for (int b = 0; b < n_in / 32; ++b) {
            const float *xb = x + 32 * b;
            const uint8_t *blk = wr + b * kQ8Bytes;
            float am = 0.0f;
            for (int k = 0; k < 32; ++k) am = fmaxf(am, fabsf(xb[k]));
            const float dx = (float)(_Float16)(am / 127.0f);
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            int s = 0;
            for (int k = 0; k < 32; ++k)
                s += (int)(int8_t)blk[2 + k] * (int)__builtin_rintf(xb[k] * id);
            acc = fmaf((float)s, h2f(blk[0] | blk[1] << 8) * dx, acc);
        }
        y[row] = acc;
        return;
    }
    const bool w_f16 = w_type == VKV_DTYPE_F16;
    float acc = 0.0f;
    for (int k = lane; k < n_in; k += 64) {
        if (w_f16) {
            const _Float16 a = reinterpret_cast<const _Float16 *>(w)[(int64_t)row * n_in + k];
            acc += (float)a * (float)(_Float16)x[k];
        } else {
            acc += reinterpret_cast<const float *>(w)[(int64_t)row * n_in + k] * x[k];
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// ggml_argmax of f32 (ggml_vec_argmax_f32: the running max MAX(max, x[i]) and
// idx = i whenever x[i] equals it), i.e. for finite input the last index of
// the maximum.  One work group; (value, index) pairs reduce by larger value,
// then larger index, so the visiting order does not matter.
__global__ void __launch_bounds__(1024) k_argmax(const float *__restrict__ x, int n,
                                                 int32_t *__restrict__ out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -INFINITY;
    int bi = -1;
    auto take = [&](float v, int i) {
        if (v > bv || (v == bv && i > bi)) {
            bv = v;
            bi = i;
        }
    };
    const int n4 = n >> 2;
    for (int j = threadIdx.x; j < n4; j += 1024) {
        const float4 v = reinterpret_cast<const float4 *>(x)[j];
        take(v.x, 4 * j);
        take(v.y, 4 * j + 1);
        take(v.z, 4 * j + 2);
        take(v.w, 4 * j + 3);
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += 1024) take(x[i], i);
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        take(ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < 16; ++w) take(sv[w], si[w]);
        out[0] = bi < 0 ? 0 : bi;
    }
}

// ---------------------------------------------------------------------------
// Products with several input rows (the encoder's P frames per chunk,
// src/voxtral.cpp:2147-2370; the decoder prefill): Y[p][r] = sum_k W[r][k] h_p[k]
// in the CPU path's arithmetic (each h_p quantized to Q8_K, integer block
// sums), on the matrix cores.
//
//   k_q8k_rows -- the Q8_K image of every input row (one work group per row,
//                 same input side as k_matvec), to global memory: codes
//                 [p][K], block scales [p][K/256], 32-element sums [p][K/32] (int16);
//                 for Q8_0 weights the q8_0 image: codes and the fp16 d of
//                 each 32-element block in the sums' place.
//   k_gemm_kq  -- a work group owns 16 weight rows x 16 (or 32) input rows;
//                 its 8 (or 16) waves split the 256-blocks of K and meet in LDS.
//                 A wave holds one block's fragments (about 100 VGPRs), so
//                 two work groups share a CU and hide each other's load
//                 latency.  One
//                 v_mfma_i32_16x16x32_i8 per 32 weights: A = 16 rows' codes
//                 (lane (kg, r): row r, k = 8kg..8kg+7), B = 16 input rows'
//                 Q8_K codes, C = exact int32 sums, row m = 4kg + i of lane
//                 (kg, n) for input n.  Q4_K: one MFMA per sub-block, then its
//                 6-bit scale and min; Q6_K: codes recentred to int8 (q - 32),
//                 one MFMA per 16-element scale group (the other half of the
//                 k window zeroed); Q8_0: one MFMA per 34-byte block against
//                 the q8_0 image, times fp16(d_w) * fp16(d_x).
// ---------------------------------------------------------------------------
// NE: inputs of up to 4096 (one round of 16-lane rows), with the norm's
// weight, ada and bias requested together with the input (one round trip)
template <int NBW, bool NE, bool Q80>
__global__ void __launch_bounds__(256) k_q8k_rows(const float *__restrict__ x, int64_t x_stride,
                                                  int x_ring, int x_row0, int n, const float *nw,
                                                  const float *nbias, const float *ada, float eps,
                                                  int8_t *__restrict__ codes, float *__restrict__ xd,
                                                  int16_t *__restrict__ bs16) {
    __shared__ ActSmem sm;
    const int p = blockIdx.x;
    const int src = x_ring > 0 ? (x_row0 + p) % x_ring : p;
    ActRegs<NBW, NE, NE> r;
    act_load(r, x + (int64_t)src * x_stride, n, nw, ada, nbias);
    act_finish<NBW, NE, NE, Q80>(r, n, nw, ada, eps, sm, nullptr, nbias);
    // codes in the products' lane order: within each 256-block, the 16 bytes
    // at 64 q + 16 kg hold the codes k = 32 j + 8 kg + e of j = 2q, 2q + 1
    // (e = 0..7): lane group kg's MFMA B operands, and one 16-byte load per q
    // reads 64 contiguous bytes of each input row
    int4 *dst = reinterpret_cast<int4 *>(codes + (int64_t)p * n);
    const uint64_t *src8 = reinterpret_cast<const uint64_t *>(sm.xq);
    for (int i = threadIdx.x; i < n / 16; i += 256) {
        const int base = (i >> 4) * 32, kg = i & 3, j0 = 2 * ((i >> 2) & 3);
        const uint64_t lo = src8[base + 4 * j0 + kg], hi = src8[base + 4 * (j0 + 1) + kg];
        dst[i] = make_int4((int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi,
                           (int)(uint32_t)(hi >> 32));
    }
    if constexpr (Q80) {
        // the fp16 d of each 32-element block (held as its f32 value)
        for (int i = threadIdx.x; i < n / 32; i += 256)
            bs16[(int64_t)p * (n / 32) + i] = __builtin_bit_cast(
                int16_t, (_Float16)__builtin_bit_cast(float, sm.bs32[i]));
    } else {
        for (int i = threadIdx.x; i < n / 256; i += 256) xd[(int64_t)p * (n / 256) + i] = sm.dx[i];
        // (a sum of 32 codes fits in 16 bits: |s| <= 32 * 127)
        for (int i = threadIdx.x; i < n / 32; i += 256) bs16[(int64_t)p * (n / 32) + i] = (int16_t)sm.bs32[i];
    }
}

// 8 bytes at an even byte offset of a buffer (Q6_K blocks are 2-byte
// aligned): one 8-byte load when the offset is 4-aligned, else 12 bytes from
// 2 below, realigned -- never past off + 10
__device__ __forceinline__ uint64_t ld8_even(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    // one load path for both alignments (a value merged from two loads is
    // copied, and the copy waits for its load)
    const u32x3_t w = __builtin_amdgcn_raw_buffer_load_b96(rs, off & ~3u, 0, 0);
    const uint32_t lo = __builtin_amdgcn_alignbyte(w.y, w.x, off & 3u);
    const uint32_t hi = __builtin_amdgcn_alignbyte(w.z, w.y, off & 3u);
    return ((uint64_t)hi << 32) | lo;
}

// 6-bit codes c (one per byte) -> c - 32 as int8: t = c ^ 0x20 is c - 32 when
// c >= 32 and c + 32 (bit 5 set) when c < 32; the latter needs bits 6 and 7
// set as well (x6 moves 0x20 to 0xC0 inside each byte)
__device__ __forceinline__ uint32_t recentre6(uint32_t c) {
    const uint32_t t = c ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 6u);
}

__device__ __forceinline__ i32x4_t mfma_i8(uint64_t a, uint64_t b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((int64_t)a, (int64_t)b, c, 0, 0, 0);
}

__device__ __forceinline__ MmOut mm_out_at(const MmArgs &a, int k) {
    MmOut o = a.out[0];
    if (k == 1) o = a.out[1];
    if (k == 2) o = a.out[2];
    if (k == 3) o = a.out[3];
    return o;
}

// One 256-block of one matrix for a lane: the loads (a set of registers per
// block in flight) and the arithmetic that adds the block to acc[i] (weight
// row 4kg + i of the tile, input row n = lane & 15).
struct GFragQ4 {
    uint64_t qs[4];   // codes of sub-blocks 2c / 2c+1 (low / high nibbles), k = 8kg..8kg+7
    u32x4_t h;        // the lane's row header: d|dmin, scales[12]
};
struct GFragQ6 {
    uint64_t ql[2][2], qh[2];   // [half n][low / high ql], [half n], k = 8kg..8kg+7
    uint64_t s0, s1;            // the row's 16 int8 scales
    uint32_t dh;                // fp16 d
};
struct GFragQ8 {
    uint64_t qs[8];   // codes of the 256-block's Q8_0 blocks j = 0..7, k = 8kg..8kg+7
    uint32_t dh[4];   // fp16 d of blocks 2i (low half) and 2i + 1 (high half)
};
struct GFragX {
    uint64_t xb[8];   // Q8_K codes of input row n, k window 32j + 8kg
    int32_t bsx[8];   // their 32-element sums (Q4_K mins); q8_0 image: fp16 d of block j
    float dx;
};

// ALLH: every lane loads the block header (scales, d); otherwise only the
// lanes that pass it on (kg = 0) do, and the others' zeros merge with the
// loaded value, which waits for the load there.  The fused-input kernels
// request a block before the input quantization and must not wait for it;
// the others issue fewer loads without it.
template <int WK, bool ALLH>
__device__ __forceinline__ auto gemm_load_w(__amdgpu_buffer_rsrc_t rs, uint32_t boff, int kg) {
    if constexpr (WK == kWQ8) {
        // block j's codes 8kg..8kg+7 start 2 mod 4 (j even) or 0 mod 4 (j odd)
        // bytes into the row (boff is a multiple of 272); for kg = 0 and j
        // even the realigning load starts at the block, so its first half
        // word is d; odd blocks' d take a load of their own
        GFragQ8 f;
        uint32_t de[4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t off = boff + kQ8Bytes * j + 2 + 8 * kg;
            const u32x3_t w = __builtin_amdgcn_raw_buffer_load_b96(rs, off & ~3u, 0, 0);
            const uint32_t lo = __builtin_amdgcn_alignbyte(w.y, w.x, off & 3u);
            const uint32_t hi = __builtin_amdgcn_alignbyte(w.z, w.y, off & 3u);
            f.qs[j] = ((uint64_t)hi << 32) | lo;
            if ((j & 1) == 0) de[j >> 1] = w.x & 0xffffu;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t dodd = 0;
            if (ALLH || kg == 0)
                dodd = __builtin_amdgcn_raw_buffer_load_b16(rs, boff + kQ8Bytes * (2 * i + 1), 0, 0);
            f.dh[i] = de[i] | dodd << 16;
        }
        return f;
    } else if constexpr (WK == kWQ4) {
        GFragQ4 f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const u32x2_t v = __builtin_bit_cast(
                u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, boff + 16 + 32 * c + 8 * kg, 0, 0));
            f.qs[c] = ((uint64_t)v.y << 32) | v.x;
        }
        // the header is only read by the lanes that pass it on (kg = 0)
        if (ALLH) {
            f.h = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, boff, 0, 0));
        } else {
            f.h = u32x4_t{0, 0, 0, 0};
            if (kg == 0) f.h = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, boff, 0, 0));
        }
        return f;
    } else {
        GFragQ6 f;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            f.ql[n][0] = ld8_even(rs, boff + 64 * n + 8 * kg);
            f.ql[n][1] = ld8_even(rs, boff + 64 * n + 32 + 8 * kg);
            f.qh[n] = ld8_even(rs, boff + 128 + 32 * n + 8 * kg);
        }
        // scales and d are only read by the lanes that pass them on (kg = 0)
        if (ALLH) {
            f.s0 = ld8_even(rs, boff + 192);
            f.s1 = ld8_even(rs, boff + 200);
            f.dh = __builtin_amdgcn_raw_buffer_load_b16(rs, boff + 208, 0, 0);
        } else {
            f.s0 = f.s1 = 0;
            f.dh = 0;
            if (kg == 0) {
                f.s0 = ld8_even(rs, boff + 192);
                f.s1 = ld8_even(rs, boff + 200);
                f.dh = __builtin_amdgcn_raw_buffer_load_b16(rs, boff + 208, 0, 0);
            }
        }
        return f;
    }
}

// The input image: a.xq / a.xd / a.xbs in global memory, or (fused input)
// the work group's own columns in LDS, column col - col0 of the same layout.
struct XImage {
    const int8_t *xq;
    const float *xd;
    const int16_t *xbs;
    int col0;
};

template <int WK>
__device__ __forceinline__ GFragX gemm_load_x(const MmArgs &a, const XImage &im, int col, int b,
                                              int kg) {
    GFragX x;
    const int K = a.n_in;
    col -= im.col0;
    // the image's lane order: 16 bytes per lane group at 64 q + 16 kg
    const int4 *xc = reinterpret_cast<const int4 *>(im.xq + (int64_t)col * K + 256 * b + 16 * kg);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int4 v = xc[4 * q];
        x.xb[2 * q] = ((uint64_t)(uint32_t)v.y << 32) | (uint32_t)v.x;
        x.xb[2 * q + 1] = ((uint64_t)(uint32_t)v.w << 32) | (uint32_t)v.z;
    }
    if constexpr (WK == kWQ4 || WK == kWQ8) {
        // the block's eight 16-bit sums (q8_0: fp16 d) in one 16-byte load
        const int4 v = *reinterpret_cast<const int4 *>(im.xbs + (int64_t)col * (K / 32) + 8 * b);
        const int w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (WK == kWQ4) {
                x.bsx[2 * i] = (int)(int16_t)(w4[i] & 0xffff);
                x.bsx[2 * i + 1] = w4[i] >> 16;
            } else {
                x.bsx[2 * i] = w4[i] & 0xffff;
                x.bsx[2 * i + 1] = (int)((uint32_t)w4[i] >> 16);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x.bsx[j] = 0;
    }
    x.dx = WK == kWQ8 ? 0.0f : im.xd[(int64_t)col * (K >> 8) + b];
    return x;
}

// Fused input: the Q8_K image of input rows [col0, col0 + ncol) in LDS, in
// the products' layout (codes of row c at c n_in, lane order within each
// 256-block; block scales; 32-element sums as int16), by the same arithmetic
// as k_q8k_rows (ggml's rms_norm then quantize_row_q8_K_ref): task (row c,
// block b) is one 16-lane DPP row, lane l holding elements [16 l, 16 l +
// 16) of the block, and a group takes at most kFqRounds tasks, all loaded up
// front (the host routes larger calls to k_q8k_rows).  With a norm, each
// task's sum of squares (f32 products summed in double, the row's 16 lanes
// by DPP) goes to LDS and a row's scale is taken from its block sums in block
// order, so a row's codes do not depend on the work group or the number of
// rows in the call.
constexpr int kFqRounds = 2;
// The norm's vectors (weight, bias, ada) reach the fused quantizer through
// LDS, each thread loading at most kFqNormPer elements of each (the host
// fuses a normed call only when n_in <= kFqNormPer * 64 * waves).
constexpr int kFqNormPer = 4;

// pre() is called once the input rows (and the norm's vectors) have been
// requested and before anything waits for them: the caller requests its
// first weights there, so their round trip overlaps the input's.
template <int W, bool Q80, class Pre>
__device__ __forceinline__ void gemm_quant_cols(const MmArgs &a, int col0, int ncol, int8_t *cq,
                                                float *cd, int16_t *cs, double *ss, float *nv,
                                                Pre &&pre) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l = lane & 15;
    const int K = a.n_in, nb = K >> 8, tasks = ncol * nb;
    const int gi = 4 * wave + (lane >> 4);   // this 16-lane group
    // Only the groups with a task in a round load its input: with few input
    // rows most groups have none (4 rows x 8 blocks: 32 of 2 x 64), and their
    // loads held the work group's waves at the issue of their own for ~2 us
    // (the last waves reached the barrier ~2 us after the first).  A group
    // past the last task leaves its values unused.
    float e[kFqRounds][16];
#pragma unroll
    for (int r = 0; r < kFqRounds; ++r) {
#pragma unroll
        for (int k = 0; k < 16; ++k) e[r][k] = 0.0f;
        const int t = gi + 4 * W * r;
        if (t < tasks) {
            const int c = t / nb, b = t % nb;
            const int p = col0 + c;
            const int src = a.x_ring > 0 ? (a.x_row0 + p) % a.x_ring : p;
            const float4 *xp =
                reinterpret_cast<const float4 *>(a.x + (int64_t)src * a.x_stride + 256 * b + 16 * l);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = xp[j];
                e[r][4 * j] = v.x;
                e[r][4 * j + 1] = v.y;
                e[r][4 * j + 2] = v.z;
                e[r][4 * j + 3] = v.w;
            }
        }
    }
    float nvr[3][kFqNormPer];
    if (a.norm_w) {
#pragma unroll
        for (int k = 0; k < kFqNormPer; ++k) {
            const int i = (int)threadIdx.x + 64 * W * k;
            nvr[0][k] = i < K ? a.norm_w[i] : 0.0f;
            nvr[1][k] = a.norm_b && i < K ? a.norm_b[i] : 0.0f;
            nvr[2][k] = a.ada && i < K ? a.ada[i] : 0.0f;
        }
    }
    pre();
    if (a.norm_w) {
#pragma unroll
        for (int k = 0; k < kFqNormPer; ++k) {
            const int i = (int)threadIdx.x + 64 * W * k;
            if (i < K) {
                nv[i] = nvr[0][k];
                nv[K + i] = nvr[1][k];
                nv[2 * K + i] = nvr[2][k];
            }
        }
#pragma unroll
        for (int r = 0; r < kFqRounds; ++r) {
            const int t = gi + 4 * W * r;
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < 16; ++k) s += (double)(e[r][k] * e[r][k]);
            s += dppd<0xB1>(s);
            s += dppd<0x4E>(s);
            s += dppd<0x141>(s);
            s += dppd<0x140>(s);
            if (t < tasks && l == 0) ss[t] = s;
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < kFqRounds; ++r) {
        const int t = gi + 4 * W * r;
        if (t >= tasks) break;
        const int c = t / nb, b = t % nb;
        if (a.norm_w) {
            double tot = 0.0;
            for (int k = 0; k < nb; ++k) tot += ss[c * nb + k];
            const float mean = (float)(tot / (double)K);
            const float scale = 1.0f / sqrtf(mean + a.eps);
            const int e0 = 256 * b + 16 * l;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 w4 = *reinterpret_cast<const float4 *>(nv + e0 + 4 * j);
                const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    e[r][4 * j + u] = e[r][4 * j + u] * scale;
                    e[r][4 * j + u] = e[r][4 * j + u] * w[u];
                }
                if (a.norm_b) {
                    const float4 b4 = *reinterpret_cast<const float4 *>(nv + K + e0 + 4 * j);
                    e[r][4 * j] = e[r][4 * j] + b4.x;
                    e[r][4 * j + 1] = e[r][4 * j + 1] + b4.y;
                    e[r][4 * j + 2] = e[r][4 * j + 2] + b4.z;
                    e[r][4 * j + 3] = e[r][4 * j + 3] + b4.w;
                }
                if (a.ada) {
                    const float4 a4 = *reinterpret_cast<const float4 *>(nv + 2 * K + e0 + 4 * j);
                    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float tt = e[r][4 * j + u] * av[u];
                        e[r][4 * j + u] = e[r][4 * j + u] + tt;
                    }
                }
            }
        }
        uint32_t packed[4];
        int16_t s32 = 0;
        float dq = 0.0f;
        if constexpr (Q80) {
            // the q8_0 image: the 32-element block's fp16 d in the sums' place
            const QBlock0 q = q8_0_block16(e[r]);
#pragma unroll
            for (int w = 0; w < 4; ++w) packed[w] = q.packed[w];
            s32 = __builtin_bit_cast(int16_t, (_Float16)q.d);
        } else {
            const QBlock16 q = q8k_block16(e[r], l);
#pragma unroll
            for (int w = 0; w < 4; ++w) packed[w] = q.packed[w];
            s32 = (int16_t)q.s32;
            dq = q.d;
        }
        // codes 32 j + 8 kg + e at byte 64 q + 16 kg + 8 (j & 1) + e of the
        // block (q = j / 2): lane l holds j = l / 2, kg = 2 (l & 1) + h
        int8_t *blk = cq + (int64_t)c * K + 256 * b;
        const int jj = (l >> 1) & 1, qq = l >> 2;
#pragma unroll
        for (int h = 0; h < 2; ++h)
            *reinterpret_cast<uint2 *>(blk + 64 * qq + 16 * (2 * (l & 1) + h) + 8 * jj) =
                make_uint2(packed[2 * h], packed[2 * h + 1]);
        if ((l & 1) == 0) cs[(int64_t)c * (K / 32) + 8 * b + (l >> 1)] = s32;
        if (l == 0) cd[(int64_t)c * nb + b] = dq;
    }
    __syncthreads();
}

// The weight codes through an empty asm: what is derived from them (nibbles,
// recentred 6-bit codes) is derived again instead of held in registers.
__device__ __forceinline__ void opaque_codes(GFragQ4 &f) {
#pragma unroll
    for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(f.qs[c]));
}
__device__ __forceinline__ void opaque_codes(GFragQ8 &f) {
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(f.qs[j]));
}
__device__ __forceinline__ void opaque_codes(GFragQ6 &f) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        asm volatile("" : "+v"(f.ql[n][0]));
        asm volatile("" : "+v"(f.ql[n][1]));
        asm volatile("" : "+v"(f.qh[n]));
    }
}

// The block headers of the lane's four accumulator rows 4kg + i (d|dmin and
// the 6-bit scales and mins one per byte for Q4_K; d and the 16 int8 scales
// for Q6_K), passed between the wave's lanes through LDS: lanes kg = 0 hold
// row rr's header.  A wave's LDS accesses complete in order, so the rows'
// headers are in place when read back.
__device__ __forceinline__ void gemm_hdr(const GFragQ4 &f, uint32_t (*hdr)[6], int kg, int rr,
                                         uint32_t (&hd)[4][5]) {
    if (kg == 0) {
        hdr[rr][0] = f.h.x;
        hdr[rr][1] = f.h.y & 0x3f3f3f3fu;
        hdr[rr][2] = (f.h.w & 0x0f0f0f0fu) | ((f.h.y >> 2) & 0x30303030u);
        hdr[rr][3] = f.h.z & 0x3f3f3f3fu;
        hdr[rr][4] = ((f.h.w >> 4) & 0x0f0f0f0fu) | ((f.h.z >> 2) & 0x30303030u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 5; ++w) hd[i][w] = hdr[4 * kg + i][w];
}

__device__ __forceinline__ void gemm_hdr(const GFragQ6 &f, uint32_t (*hdr)[6], int kg, int rr,
                                         uint32_t (&hd)[4][5]) {
    if (kg == 0) {
        hdr[rr][0] = f.dh;
        hdr[rr][1] = (uint32_t)f.s0;
        hdr[rr][2] = (uint32_t)(f.s0 >> 32);
        hdr[rr][3] = (uint32_t)f.s1;
        hdr[rr][4] = (uint32_t)(f.s1 >> 32);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 5; ++w) hd[i][w] = hdr[4 * kg + i][w];
}

__device__ __forceinline__ void gemm_hdr(const GFragQ8 &f, uint32_t (*hdr)[6], int kg, int rr,
                                         uint32_t (&hd)[4][5]) {
    if (kg == 0) {
#pragma unroll
        for (int w = 0; w < 4; ++w) hdr[rr][w] = f.dh[w];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int w = 0; w < 4; ++w) hd[i][w] = hdr[4 * kg + i][w];
        hd[i][4] = 0;
    }
}

// Q8_0: block j's exact integer sums, times fp16(d_w) * fp16(d_x) (ggml's
// per-block term of vec_dot_q8_0_q8_0)
__device__ __forceinline__ void gemm_dot(const GFragQ8 &f, const GFragX &x, const uint32_t (&hd)[4][5],
                                         int kg, float (&acc)[4]) {
    const i32x4_t z = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const i32x4_t c = mfma_i8(f.qs[j], x.xb[j], z);
        const float dx = h2f((uint32_t)x.bsx[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float dw = h2f((hd[i][j >> 1] >> (16 * (j & 1))) & 0xffffu);
            acc[i] = fmaf((float)c[i], dw * dx, acc[i]);
        }
    }
}

__device__ __forceinline__ void gemm_dot(const GFragQ4 &f, const GFragX &x, const uint32_t (&hd)[4][5],
                                         int kg, float (&acc)[4]) {
    const i32x4_t z = {0, 0, 0, 0};
    int isum[4] = {0, 0, 0, 0}, imin[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint64_t q = (j & 1) ? (f.qs[j >> 1] >> 4) & 0x0f0f0f0f0f0f0f0full
                                   : f.qs[j >> 1] & 0x0f0f0f0f0f0f0f0full;
        const i32x4_t c = mfma_i8(q, x.xb[j], z);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t sh = 8 * (j & 3);
            const int sc = (int)(((j < 4 ? hd[i][1] : hd[i][2]) >> sh) & 255u);
            const int mn = (int)(((j < 4 ? hd[i][3] : hd[i][4]) >> sh) & 255u);
            isum[i] += sc * c[i];
            imin[i] += mn * x.bsx[j];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float d = h2f(hd[i][0] & 0xffffu) * x.dx, dmin = h2f(hd[i][0] >> 16) * x.dx;
        acc[i] += d * (float)isum[i] - dmin * (float)imin[i];
    }
}

__device__ __forceinline__ void gemm_dot(const GFragQ6 &f, const GFragX &x, const uint32_t (&hd)[4][5],
                                         int kg, float (&acc)[4]) {
    const i32x4_t z = {0, 0, 0, 0};
    int isum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint64_t lo = f.ql[n][g & 1];
            const uint64_t nib = g < 2 ? lo & 0x0f0f0f0f0f0f0f0full : (lo >> 4) & 0x0f0f0f0f0f0f0f0full;
            const uint64_t hb = ((f.qh[n] >> (2 * g)) & 0x0303030303030303ull) << 4;
            const uint64_t cc = nib | hb;
            const uint64_t q = ((uint64_t)recentre6((uint32_t)(cc >> 32)) << 32) | recentre6((uint32_t)cc);
            // the window's two 16-element scale groups: lanes kg < 2 hold the first
            const i32x4_t c0 = mfma_i8(kg < 2 ? q : 0ull, x.xb[4 * n + g], z);
            const i32x4_t c1 = mfma_i8(kg < 2 ? 0ull : q, x.xb[4 * n + g], z);
            const int t = 8 * n + 2 * g;   // scale index of the first group
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s0 = (int)(int8_t)(hd[i][1 + (t >> 2)] >> (8 * (t & 3)));
                const int s1 = (int)(int8_t)(hd[i][1 + ((t + 1) >> 2)] >> (8 * ((t + 1) & 3)));
                isum[i] += s0 * c0[i] + s1 * c1[i];
            }
        }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += (h2f(hd[i][0]) * x.dx) * (float)isum[i];
}

// RoPE (ggml mode 0) of one element of a pair in the products' epilogue,
// with vkv_rope's arithmetic: the angle pos * ts^pair by the running f32
// product, cos/sin in double rounded to f32, no contraction
__device__ __forceinline__ float rope_elem(float self, float partner, bool odd, int pair, float pos,
                                           float ts) {
#pragma clang fp contract(off)
    float theta = pos;
    for (int i = 0; i < pair; ++i) theta *= ts;
    const float c = (float)cos((double)theta), sn = (float)sin((double)theta);
    return odd ? partner * sn + self * c : self * c - partner * sn;
}

// Waves per work group: 8, or 16 when a call has few 16-row tiles (the
// 1280-row products of the encoder are 80 tiles): more waves split the same
// K, so each walks a shorter chain of blocks.  CT column tiles (16
// input rows each) per work group: a wave loads each weight block once and
// applies it to every column tile, so the weights are read once per 16 CT
// input rows.
template <int WK, int W, int CT, bool ALLH, class GF>
__device__ __forceinline__ void gemm_body(const MmArgs &a, const MmOut &o0, const MmOut &o1,
                                          uint32_t (*hdr)[16][6], float (*red)[W][16][17],
                                          const XImage &im, const GF &w_first) {
    // the wave index through readfirstlane: the per-wave descriptor select
    // below is then scalar (a per-lane one puts every load in a loop over
    // the descriptor's values)
    const int lane = threadIdx.x & 63, kg = lane >> 4, rr = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool swiglu = a.swiglu != 0;
    const int nb = a.n_in >> 8;
    const uint32_t bbytes = WK == kWQ4 ? kQ4Bytes : WK == kWQ8 ? kQ8Per256 : kQ6Bytes;
    const uint32_t rbytes = (uint32_t)nb * bbytes;
    const int row0 = ((int)blockIdx.x - o0.tile0) * 16, col0 = (int)blockIdx.y * 16 * CT;
    const int row = min(row0 + rr, o0.n_rows - 1);
    // column tiles holding input rows (uniform over the work group)
    const int n_ct = min(CT, (a.n_cols - col0 + 15) / 16);
    const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(o0.w), (short)0, (int)(rbytes * (uint32_t)o0.n_rows), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(o1.w), (short)0, (int)(rbytes * (uint32_t)o1.n_rows), 0x00020000);
    // SwiGLU: waves 0..W/2-1 take W1, the others W3; otherwise all W waves
    // split K.  A wave holds one matrix's registers either way.
    const int kw = swiglu ? W / 2 : W;
    const int m = swiglu ? wave / kw : 0, wm = wave - m * kw;
    const __amdgpu_buffer_rsrc_t rs = m ? rs1 : rs0;
    float acc[CT][4];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][i] = 0.0f;
    // The epilogue's inputs (residual, biases), requested before the blocks:
    // loaded at the end they waited for a memory round trip of their own.
    // A thread has at most one output (ot = its index: column tile, input
    // row, row); indices clamp into the matrix and absent vectors read y
    // (unused), so the loads are unconditional.
    static_assert(64 * W >= 256 * CT, "one output per thread");
    const int ot = threadIdx.x;
    const int ot_r = ot & 15, ot_row = min(row0 + ot_r, o0.n_rows - 1);
    const int ot_col = min(col0 + 16 * (ot >> 8) + ((ot >> 4) & 15), a.n_cols - 1);
    const int64_t ot_at =
        (int64_t)(a.y_ring > 0 ? (a.y_row0 + ot_col) % a.y_ring : ot_col) * o0.n_rows + ot_row;
    const float e_b0 = (o0.bias ? o0.bias : o0.y)[ot_row];
    // the second input: W3's bias (SwiGLU), the pair row's bias (RoPE) or
    // the residual
    const float *e2p = swiglu ? (o1.bias ? o1.bias : o0.y)
                       : o0.rope ? (o0.bias ? o0.bias : o0.y)
                                 : (o0.add ? o0.add : o0.y);
    const int64_t e2i = swiglu ? ot_row : o0.rope ? min(row0 + (ot_r ^ 1), o0.n_rows - 1) : ot_at;
    const float e_2 = e2p[e2i];
    // the wave's blocks b, b + kw, b + 2 kw, ...: one block's fragments at a
    // time (occupancy, not a second register set, covers the load latency);
    // the first block's (w_first) were requested by the caller
    auto block = [&](GF w, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            if (c < n_ct) {
                const GFragX x =
                    gemm_load_x<WK>(a, im, min(col0 + 16 * c + rr, a.n_cols - 1), b, kg);
                // with several column tiles the codes pass through an empty
                // asm before each use, so what is derived from them (nibbles,
                // recentred codes, scales) is derived again instead of held
                // in registers
                if (CT > 1) opaque_codes(w);
                uint32_t hd[4][5];
                gemm_hdr(w, hdr[wave], kg, rr, hd);
                gemm_dot(w, x, hd, kg, acc[c]);
            }
            if (CT > 1) __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (wm < nb) block(w_first, wm);
    for (int b = wm + kw; b < nb; b += kw)
        block(gemm_load_w<WK, ALLH>(rs, (uint32_t)row * rbytes + (uint32_t)b * bbytes, kg), b);
    // the waves' partial sums meet in LDS: red[column tile][wave][row][input row]
    // (SwiGLU: waves m kw .. m kw + kw - 1 hold matrix m)
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[c][wave][4 * kg + i][rr] = acc[c][i];
    __syncthreads();
    // outputs: 16 consecutive rows per input row, one per thread
    if (ot < 256 * n_ct) {
        const int ct = ot >> 8, c = (ot >> 4) & 15, r = ot & 15;
        const int orow = row0 + r, ocol = col0 + 16 * ct + c;
        if (orow < o0.n_rows && ocol < a.n_cols) {
            float v0 = 0.0f, v1 = 0.0f;
            for (int w = 0; w < kw; ++w) v0 += red[ct][w][r][c];
            if (o0.bias) v0 = v0 + e_b0;
            float y;
            if (swiglu) {
                for (int w = 0; w < kw; ++w) v1 += red[ct][kw + w][r][c];
                if (o1.bias) v1 = v1 + e_2;
                y = silu(v0) * v1;
            } else if (a.gelu) {
                y = gelu_erf(v0);
            } else if (o0.rope) {
                // the pair's other row is in this tile: its sum and bias
                const int pr = r ^ 1;
                float vp = 0.0f;
                for (int w = 0; w < kw; ++w) vp += red[ct][w][pr][c];
                if (o0.bias) vp = vp + e_2;
                y = rope_elem(v0, vp, (orow & 1) != 0, (orow % a.rope_hd) >> 1,
                              (float)(a.rope_pos0 + ocol), a.rope_ts);
            } else {
                y = o0.add ? e_2 + v0 : v0;
            }
            o0.y[ot_at] = y;
        }
    }
}

// (the body is in the kernel itself: a reference to the by-value kernel
// argument passed through one more inlined function made the compiler copy
// the argument to scratch memory)
// Fused input image in dynamic LDS: codes, block scales, 32-element sums,
// per-task sums of squares (the norm's first pass).
__host__ __device__ constexpr size_t al16(size_t b) { return (b + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t fused_lds_bytes(int cols, int n_in, bool norm) {
    return al16((size_t)cols * n_in) + al16((size_t)cols * (n_in / 256) * 4) +
           al16((size_t)cols * (n_in / 32) * 2) + al16((size_t)cols * (n_in / 256) * 8) +
           (norm ? (size_t)3 * n_in * 4 : 0);
}

template <int W, int CT, bool FQ>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(4))) k_gemm_kq(MmArgs a) {
    __shared__ uint32_t hdr[W][16][6];
    __shared__ float red[CT][W][16][17];
    int seg = 0;
#pragma unroll
    for (int k = 1; k < kMvMaxOuts; ++k)
        if (k < a.n_outs && (int)blockIdx.x >= a.out[k].tile0) seg = k;
    const MmOut o0 = mm_out_at(a, seg);
    const MmOut o1 = a.swiglu ? a.out[1] : o0;
    // one weight dtype per work group (both SwiGLU matrices share it)
    auto run = [&](auto wk) __attribute__((always_inline)) {
        constexpr int WK = decltype(wk)::value;
        // the wave's first weight block (gemm_body's decomposition), requested
        // before the fused input quantization waits for anything; the block
        // index is clamped so the request is unconditional (a wave without a
        // block does not use it)
        const int lane = threadIdx.x & 63, kg = lane >> 4, rr = lane & 15;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int nb = a.n_in >> 8;
        const uint32_t bbytes = WK == kWQ4 ? kQ4Bytes : WK == kWQ8 ? kQ8Per256 : kQ6Bytes;
        const uint32_t rbytes = (uint32_t)nb * bbytes;
        const int row = min(((int)blockIdx.x - o0.tile0) * 16 + rr, o0.n_rows - 1);
        const int kw = a.swiglu ? W / 2 : W;
        const int m = a.swiglu ? wave / kw : 0, wm = wave - m * kw;
        const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(o0.w), (short)0, (int)(rbytes * (uint32_t)o0.n_rows), 0x00020000);
        const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(o1.w), (short)0, (int)(rbytes * (uint32_t)o1.n_rows), 0x00020000);
        const __amdgpu_buffer_rsrc_t rs = m ? rs1 : rs0;
        using GF = std::conditional_t<WK == kWQ4, GFragQ4,
                                      std::conditional_t<WK == kWQ8, GFragQ8, GFragQ6>>;
        GF wf;
        // (a wave without a block -- more waves than blocks -- reads past the
        // buffer: zeros, no memory traffic; 4 KiB below the top, so no
        // fragment offset wraps into the buffer)
        auto pre = [&]() __attribute__((always_inline)) {
            wf = gemm_load_w<WK, FQ>(
                rs, wm < nb ? (uint32_t)row * rbytes + (uint32_t)wm * bbytes : 0xFFFFF000u, kg);
        };
        XImage im{a.xq, a.xd, a.xbs, 0};
        if constexpr (FQ) {
            extern __shared__ __align__(16) uint8_t fq_lds[];
            const int col0 = (int)blockIdx.y * 16 * CT;
            const int ncol = min(16 * CT, a.n_cols - col0);
            const int K = a.n_in, cols = 16 * CT;
            int8_t *cq = reinterpret_cast<int8_t *>(fq_lds);
            float *cd = reinterpret_cast<float *>(fq_lds + al16((size_t)cols * K));
            int16_t *cs = reinterpret_cast<int16_t *>(reinterpret_cast<uint8_t *>(cd) +
                                                      al16((size_t)cols * nb * 4));
            double *ss = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(cs) +
                                                    al16((size_t)cols * (K / 32) * 2));
            float *nv = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(ss) +
                                                  al16((size_t)cols * nb * 8));
            gemm_quant_cols<W, WK == kWQ8>(a, col0, ncol, cq, cd, cs, ss, nv, pre);
            im = XImage{cq, cd, cs, col0};
            if (blockIdx.x == 0 && a.xq) {
                // the first row tile's work groups leave their rows' image in
                // the caller's workspace too (the separate quantization's
                // output), read by nothing in the call
                const int4 *src = reinterpret_cast<const int4 *>(cq);
                int4 *dst = reinterpret_cast<int4 *>(const_cast<int8_t *>(a.xq) + (int64_t)col0 * K);
                for (int i = threadIdx.x; i < ncol * K / 16; i += 64 * W) dst[i] = src[i];
                float *xd = const_cast<float *>(a.xd) + (int64_t)col0 * nb;
                for (int i = threadIdx.x; i < ncol * nb; i += 64 * W) xd[i] = cd[i];
                int16_t *xb = const_cast<int16_t *>(a.xbs) + (int64_t)col0 * (K / 32);
                for (int i = threadIdx.x; i < ncol * (K / 32); i += 64 * W) xb[i] = cs[i];
            }
        } else {
            pre();
        }
        gemm_body<WK, W, CT, FQ>(a, o0, o1, hdr, red, im, wf);
    };
    if (o0.dtype == VKV_DTYPE_Q4_K) run(std::integral_constant<int, kWQ4>{});
    else if (o0.dtype == VKV_DTYPE_Q8_0) run(std::integral_constant<int, kWQ8>{});
    else run(std::integral_constant<int, kWQ6>{});
}

}  // namespace

hipError_t launch_matvec(const MvArgs &a, int n_wg, hipStream_t st) {
    const int S = (a.n_in / 256 * 4 + 63) / 64;
    // the fused argmax only serves the logits (one step per row)
    if (a.amax && S != 1) return hipErrorInvalidValue;
    // A wave's units: its rows x steps x (2 under SwiGLU).  When they fit in
    // one request for every dtype of the call (6 Q4_K or 3 Q6_K units: the
    // decoder's products), the wave requests them all up front; otherwise 3
    // Q4_K / 2 Q6_K units stream, single-step rows 4 / 4 (the 131072-row Q6_K
    // logits: 2, 3, 5, 6 were 0.2-1.2% slower per token; the W1/W3 pair at
    // one work group per CU: 4 Q4_K units 10.4 against 11.2 us with 3).
    const int units = (a.rows_per_wg >> 2) * S * (a.swiglu ? 2 : 1);
    bool q4 = false, q6 = false;
    // (Q8_0 rows take the Q6_K counts)
    for (int k = 0; k < a.n_outs; ++k) (a.out[k].dtype == VKV_DTYPE_Q4_K ? q4 : q6) = true;
    auto fits = [&](int d4, int d6) { return (!q4 || units <= d4) && (!q6 || units <= d6); };
    const bool one = fits(6, 3);
    if (a.amax) k_matvec<1, 3, 4, false, true><<<n_wg, 256, 0, st>>>(a);
    else if (S == 1 && fits(3, 2)) k_matvec<1, 3, 2, true, false><<<n_wg, 256, 0, st>>>(a);
    else if (S == 1 && one) k_matvec<1, 6, 3, true, false><<<n_wg, 256, 0, st>>>(a);
    else if (S == 1) k_matvec<1, 4, 4, false, false><<<n_wg, 256, 0, st>>>(a);
    else if (S == 2 && fits(2, 2)) k_matvec<2, 2, 2, true, false><<<n_wg, 256, 0, st>>>(a);
    else if (S == 2 && one) k_matvec<2, 6, 3, true, false><<<n_wg, 256, 0, st>>>(a);
    else if (S == 2) k_matvec<2, 2, 2, false, false><<<n_wg, 256, 0, st>>>(a);
    else if (one) k_matvec<3, 6, 3, true, false><<<n_wg, 256, 0, st>>>(a);
    else k_matvec<3, 2, 2, false, false><<<n_wg, 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_q8k_quant(const float *x, int n, const float *norm_w, const float *ada, float eps,
                            uint8_t *out, hipStream_t st) {
    k_q8k_quant<<<1, 256, 0, st>>>(x, n, norm_w, ada, eps, out);
    return hipGetLastError();
}

hipError_t launch_kq_dequant(int dtype, const uint8_t *src, int64_t n, const float *add, float *y,
                             hipStream_t st, unsigned long long *zero_words) {
    const int64_t threads = n / 8;
    k_kq_dequant<<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(dtype, src, n, add, y,
                                                                    zero_words);
    return hipGetLastError();
}

hipError_t launch_embed_rows(int dtype, const uint8_t *table, int64_t row_bytes,
                             const EmbedTokens &tok, int n_rows, int64_t n, const float *add,
                             int add_ring, int add_row0, float *y, hipStream_t st,
                             unsigned long long *zero_words) {
    if (n_rows < 1 || n_rows > kEmbedChunk) return hipErrorInvalidValue;
    const int64_t threads = n / 8;
    k_embed_rows<<<dim3((unsigned)((threads + 255) / 256), (unsigned)n_rows), 256, 0, st>>>(
        dtype, table, row_bytes, tok, n, add, add_ring, add_row0, y, zero_words);
    return hipGetLastError();
}

hipError_t launch_q8k_rows(const float *x, int64_t x_stride, int x_ring, int x_row0, int n_rows,
                           int n, const float *norm_w, const float *norm_b, const float *ada,
                           float eps, int8_t *codes, float *xd, int16_t *bs16, bool q80,
                           hipStream_t st) {
    auto go = [&](auto kq) {
        constexpr bool Q80 = decltype(kq)::value;
        if (n <= 4096)
            k_q8k_rows<4, true, Q80><<<n_rows, 256, 0, st>>>(x, x_stride, x_ring, x_row0, n, norm_w,
                                                              norm_b, ada, eps, codes, xd, bs16);
        else
            k_q8k_rows<kMvMaxIn / 1024, false, Q80><<<n_rows, 256, 0, st>>>(
                x, x_stride, x_ring, x_row0, n, norm_w, norm_b, ada, eps, codes, xd, bs16);
    };
    if (q80) go(std::true_type{});
    else go(std::false_type{});
    return hipGetLastError();
}

hipError_t launch_gemm_kq(MmArgs a, int n_col_tiles, hipStream_t st) {
    // the 16-row tiles of each matrix are consecutive work groups
    int tiles = 0;
    for (int k = 0; k < a.n_outs; ++k) {
        if (a.swiglu && k == 1) {
            a.out[1].tile0 = 0x7fffffff;   // W3 rides with W1's tiles
            continue;
        }
        a.out[k].tile0 = tiles;
        tiles += (a.out[k].n_rows + 15) / 16;
    }
    for (int k = a.n_outs; k < kMvMaxOuts; ++k) a.out[k].tile0 = 0x7fffffff;
    // The waves per work group follow from the call's matrices alone, never
    // from its number of input rows: an output's reduction order (the K split
    // over the waves and their sum) then is the same whether its input row
    // comes in a run of 4 or of 128, so a streamed encoder matches its batch
    // run bit for bit.  16 waves (one column tile per work group: their
    // 128-register budget has no room for a second set of accumulators) when
    // the call has fewer than 128 row tiles; else 8 waves with two column
    // tiles (32 input rows) per work group at most: a third set of
    // accumulators spills at four waves per SIMD, and measured slower.
    // A fused-input call (a.x) quantizes each work group's input rows into
    // dynamic LDS (the caller checked gemm_fused_lds).
    const bool fq = a.x != nullptr;
    const int cols = gemm_cols_per_wg(a, n_col_tiles);
    const size_t lds = fq ? fused_lds_bytes(cols, a.n_in, a.norm_w != nullptr) : 0;
    if (tiles < 128) {
        const dim3 g((unsigned)tiles, (unsigned)n_col_tiles);
        if (fq) k_gemm_kq<16, 1, true><<<g, 1024, lds, st>>>(a);
        else k_gemm_kq<16, 1, false><<<g, 1024, 0, st>>>(a);
    } else if (n_col_tiles == 1) {
        const dim3 g((unsigned)tiles, 1u);
        if (fq) k_gemm_kq<8, 1, true><<<g, 512, lds, st>>>(a);
        else k_gemm_kq<8, 1, false><<<g, 512, 0, st>>>(a);
    } else {
        const dim3 g((unsigned)tiles, (unsigned)((n_col_tiles + 1) / 2));
        if (fq) k_gemm_kq<8, 2, true><<<g, 512, lds, st>>>(a);
        else k_gemm_kq<8, 2, false><<<g, 512, 0, st>>>(a);
    }
    return hipGetLastError();
}

int gemm_cols_per_wg(const MmArgs &a, int n_col_tiles) {
    int tiles = 0;
    for (int k = 0; k < a.n_outs; ++k)
        if (!(a.swiglu && k == 1)) tiles += (a.out[k].n_rows + 15) / 16;
    return (tiles < 128 || n_col_tiles == 1) ? 16 : 32;
}

// Whether the call's input image is quantized inside its work groups: every
// 16-lane group then has at most kFqRounds (row, block) tasks (the realtime
// encoder's 4-frame chunks, single adapter groups), and the image fits in LDS
// beside the product's own.  Measured on MI355X: 16-frame encoder chunks
// and 38-row prompts, with 3 to 12 tasks per group, run slower fused than
// with the separate k_q8k_rows launch (2.68 vs 2.23 ms, 6.65 vs 3.40 ms).
bool gemm_fused_ok(const MmArgs &a, int n_col_tiles) {
    int tiles = 0;
    for (int k = 0; k < a.n_outs; ++k)
        if (!(a.swiglu && k == 1)) tiles += (a.out[k].n_rows + 15) / 16;
    const int waves = tiles < 128 ? 16 : 8;
    const int cols = gemm_cols_per_wg(a, n_col_tiles);
    const int rows = std::min(cols, a.n_cols);
    return rows * (a.n_in / 256) <= kFqRounds * 4 * waves &&
           (!a.norm_w || a.n_in <= kFqNormPer * 64 * waves) &&
           fused_lds_bytes(cols, a.n_in, a.norm_w != nullptr) <= 128 * 1024;
}

hipError_t launch_rms_norm_rows(const float *x, int n_rows, int n, const float *w, const float *b,
                                float eps, float *y, int y_ring, int y_row0, hipStream_t st) {
    k_rms_norm_rows<<<n_rows, 256, 0, st>>>(x, n, w, b, eps, y, y_ring, y_row0);
    return hipGetLastError();
}

hipError_t launch_rows_small(const void *w, int w_type, const float *x, int n_in, int n_rows,
                             float *y, hipStream_t st) {
    k_rows_small<<<(unsigned)((n_rows + 3) / 4), 256, 0, st>>>(w, w_type, x, n_in, n_rows, y);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int n, int32_t *out, hipStream_t st) {
    k_argmax<<<1, 1024, 0, st>>>(x, n, out);
    return hipGetLastError();
}

}  // namespace vkv
