// gfx950 (MI355X, CDNA4, wave64) kernels of the voxtral.cpp KV-cache hot path.
//
//   k_append    -- ggml_set_rows / ggml_cpy of projected K/V rows into the ring
//                  (src/voxtral.cpp:2682-2713, 2166-2185); f32 -> f16 RNE, f32
//                  copy, or q8_0 block quantization, 8 elements per lane.
//   k_gather    -- logical-window copy of <=2 read segments (src/voxtral.cpp:
//                  2774-2799, 2285-2331), 16-byte vector copies.
//   k_decode    -- single-query GQA decode attention (ggml_flash_attn_ext at
//                  src/voxtral.cpp:2749-2819), split over slot chunks:
//                  16 lanes x 16 B cover one 256-byte K/V head row, the 4 query
//                  heads of a GQA group share every K/V load, QK partials and
//                  softmax maxima are reduced with DPP / cross-lane shuffles,
//                  online softmax in exp2 domain; optional fused append of the
//                  step's new row (run_decoder_step's SET_ROWS, :2682-2694).
//   k_combine   -- merge of the per-chunk (max, sum, unnormalised output).
//   k_window    -- multi-query causal / sliding-window attention for the
//                  encoder window (src/voxtral.cpp:2201-2284) and the decoder
//                  prefill (:2893-2961).
//   k_q8_pack / k_q8_unpack, k_fill_zero, k_synth.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "vkv_internal.h"

namespace vkv {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// DPP row-local lane exchange; CTRL: 0xB1 = quad xor1, 0x4E = quad xor2,
// 0x141 = row_half_mirror, 0x140 = row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane receives the total.
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x;
}

// Max over the 4 lanes of a quad.
__device__ __forceinline__ float quad_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum / max over lanes l and l ^ 16, and over lanes l and l ^ 32, with the
// gfx950 row-swap permutes (VALU, no LDS round trip).  permlane16_swap
// exchanges the odd 16-lane rows of its first operand with the even rows of
// its second, permlane32_swap the upper half of the first with the lower
// half of the second; with both operands the same value, the two results
// hold the lane's own value and its partner's, which every lane combines in
// the same order (v[lo] op v[hi]).
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Max / sum over the 64 lanes of a wave, every lane receiving the result: a
// DPP butterfly inside each 16-lane row, then the two row-swap permutes.
// The sum's association is fixed, so every caller summing the same lane
// values gets the same bits in every lane.  Its input is made opaque first:
// with contraction on, the compiler otherwise fuses a caller's product into
// the first butterfly add (fma(a, b, partner's rounded product)), and the
// two lanes of a pair then round differently.
__device__ __forceinline__ float wave_max64(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return xor32_max(xor16_max(x));
}
__device__ __forceinline__ float wave_sum64(float x) {
    asm volatile("" : "+v"(x));
    return xor32_sum(xor16_sum(row_sum16(x)));
}

// Round half away from zero.  Contraction stays off: the quantizer rounds the
// product x*id first, exactly like the CPU quantizer.
__device__ __forceinline__ float round_half_away(float v) {
#pragma clang fp contract(off)
    float t = truncf(v);
    float r = v - t;
    if (r >= 0.5f) t += 1.0f;
    else if (r <= -0.5f) t -= 1.0f;
    return t;
}

// Global loads; NT = non-temporal (streaming) hint.  The decode kernels read
// every K/V byte once per step, and on MI355X the streaming hint lifts the
// sustained read rate of that pattern by ~10% of peak (it keeps the window's
// lines from displacing reusable data in L2 and the MALL).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    const u32x4_t *q = reinterpret_cast<const u32x4_t *>(p);
    const u32x4_t r = NT ? __builtin_nontemporal_load(q) : *q;
    return make_uint4(r.x, r.y, r.z, r.w);
}
template <bool NT, class T>
__device__ __forceinline__ T ldw(const T *p) {
    return NT ? __builtin_nontemporal_load(p) : *p;
}

__device__ __forceinline__ int slot_of(const SegPair &sp, int idx) {
    return idx < sp.n0 ? sp.s0 + idx : sp.s1 + (idx - sp.n0);
}

// ---------------------------------------------------------------------------
// Storage formats.  A fragment is the 8 consecutive elements [e, e+8) of a row
// held by one lane (e is a multiple of 8).
// ---------------------------------------------------------------------------

struct FmtF16 {
    struct Frag { uint32_t w[4]; };
    struct QFrag { uint32_t w[4]; };
    template <bool NT = false>
    static __device__ __forceinline__ Frag load(const uint8_t *row, int e) {
        const uint4 x = ld16<NT>(row + (int64_t)e * 2);
        return Frag{{x.x, x.y, x.z, x.w}};
    }
    static __device__ __forceinline__ void store(uint8_t *row, int e, const Frag &f) {
        *reinterpret_cast<uint4 *>(row + (int64_t)e * 2) = make_uint4(f.w[0], f.w[1], f.w[2], f.w[3]);
    }
    // IEEE binary16 round-to-nearest-even (v_cvt_f16_f32 in the default mode).
    static __device__ __forceinline__ Frag from_f32(const float *x) {
        Frag f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            half2_t h;
            h.x = (_Float16)x[2 * i];
            h.y = (_Float16)x[2 * i + 1];
            f.w[i] = as_u32(h);
        }
        return f;
    }
    static __device__ __forceinline__ QFrag make_q(const float *x) {
        Frag f = from_f32(x);
        return QFrag{{f.w[0], f.w[1], f.w[2], f.w[3]}};
    }
    using KPrep = Frag;
    static __device__ __forceinline__ const Frag &prep(const Frag &k) { return k; }
    static __device__ __forceinline__ float dot(const Frag &k, const QFrag &q) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_fdot2(as_h2(k.w[i]), as_h2(q.w[i]), s, false);
        return s;
    }
    static __device__ __forceinline__ void to_f32(const Frag &v, float *o) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            half2_t h = as_h2(v.w[i]);
            o[2 * i] = (float)h.x;
            o[2 * i + 1] = (float)h.y;
        }
    }
};

struct FmtF32 {
    struct Frag { float x[8]; };
    struct QFrag { float x[8]; };
    template <bool NT = false>
    static __device__ __forceinline__ Frag load(const uint8_t *row, int e) {
        const uint8_t *p = row + (int64_t)e * 4;
        const uint4 a = ld16<NT>(p), b = ld16<NT>(p + 16);
        return Frag{{__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                     __uint_as_float(a.w), __uint_as_float(b.x), __uint_as_float(b.y),
                     __uint_as_float(b.z), __uint_as_float(b.w)}};
    }
    static __device__ __forceinline__ void store(uint8_t *row, int e, const Frag &f) {
        float4 *p = reinterpret_cast<float4 *>(row + (int64_t)e * 4);
        p[0] = make_float4(f.x[0], f.x[1], f.x[2], f.x[3]);
        p[1] = make_float4(f.x[4], f.x[5], f.x[6], f.x[7]);
    }
    static __device__ __forceinline__ Frag from_f32(const float *x) {
        Frag f;
#pragma unroll
        for (int i = 0; i < 8; ++i) f.x[i] = x[i];
        return f;
    }
    static __device__ __forceinline__ QFrag make_q(const float *x) {
        QFrag f;
#pragma unroll
        for (int i = 0; i < 8; ++i) f.x[i] = x[i];
        return f;
    }
    using KPrep = Frag;
    static __device__ __forceinline__ const Frag &prep(const Frag &k) { return k; }
    static __device__ __forceinline__ float dot(const Frag &k, const QFrag &q) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = fmaf(k.x[i], q.x[i], s);
        return s;
    }
    static __device__ __forceinline__ void to_f32(const Frag &v, float *o) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = v.x[i];
    }
};

// ggml block_q8_0 {fp16 d; int8 qs[32]} (34 bytes).  Element e lives in block
// e/32 at byte 34*(e/32) + 2 + e%32.  A lane's 8 quants start 2 bytes into a
// dword or on a dword boundary; they are read as three aligned dwords and
// funnel-shifted (every cache allocation carries a 256-byte tail pad so the
// third dword never leaves it).  Quantization spans the 4 lanes of a quad
// (amax), so callers keep quads converged.
struct FmtQ8 {
    struct Frag { uint32_t lo, hi; float d; };
    // The query in ggml's q8_0 arithmetic for a q8_0 K: quantized per
    // 32-element block as the cache is (d kept in f16)
    struct QFrag { uint32_t lo, hi; float d; };
    // Rows start 4-byte aligned (row_bytes = 34 * kv_dim/32 with kv_dim % 64
    // == 0 is a multiple of 4); offsets stay integers so the loads keep the
    // global address space.
    // The streaming hint is not applied: the three dword loads and the scale
    // load of neighbouring lanes share cache lines, which must stay resident
    // between those instructions.
    template <bool NT = false>
    static __device__ __forceinline__ Frag load(const uint8_t *row, int e) {
        const int bo = (e >> 5) * 34;
        const int qo = bo + 2 + (e & 31);
        const uint32_t sh = (uint32_t)(qo & 3);   // 0 or 2
        const uint16_t dh = *reinterpret_cast<const uint16_t *>(row + bo);
        const uint32_t *w = reinterpret_cast<const uint32_t *>(row + (qo - (int)sh));
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
        Frag f;
        f.lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
        f.hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
        f.d = (float)__builtin_bit_cast(_Float16, dh);
        return f;
    }
    // Quantize 8 values; the quad holding one block cooperates on amax, so
    // every lane of the quad must call this (no early exit before it).
    static __device__ __forceinline__ Frag from_f32(const float *x) {
#pragma clang fp contract(off)
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
        amax = quad_max(amax);
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) b[i] = (uint32_t)((int)round_half_away(x[i] * id)) & 0xffu;
        Frag f;
        f.lo = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        f.hi = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
        f.d = (float)(_Float16)d;   // the stored scale, exactly
        return f;
    }
    static __device__ __forceinline__ void store(uint8_t *row, int e, const Frag &f) {
        uint8_t *b = row + (int64_t)(e >> 5) * 34;
        uint16_t *qs = reinterpret_cast<uint16_t *>(b + 2 + (e & 31));
        qs[0] = (uint16_t)f.lo;
        qs[1] = (uint16_t)(f.lo >> 16);
        qs[2] = (uint16_t)f.hi;
        qs[3] = (uint16_t)(f.hi >> 16);
        if ((e & 31) == 0)
            *reinterpret_cast<uint16_t *>(b) = __builtin_bit_cast(uint16_t, (_Float16)f.d);
    }
    static __device__ __forceinline__ QFrag make_q(const float *x) {
        const Frag f = from_f32(x);   // quad-cooperative, like the cache's rows
        return QFrag{f.lo, f.hi, f.d};
    }
    // int8 pair -> exact half2: bias to unsigned, splice under the f16
    // exponent of 1024 (ulp 1), subtract 1024+128.
    static __device__ __forceinline__ half2_t i8x2_to_h2(uint32_t biased, uint32_t sel) {
        const half2_t t = as_h2(__builtin_amdgcn_perm(0x64646464u, biased, sel));
        const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
        return t - off;
    }
    // QK in ggml's q8_0 x q8_0 arithmetic: the block's integer sum (the 4
    // lanes of a quad hold its 32 quants) scaled by d_k d_q; the quad's
    // first lane carries the block's term, the others 0, so the caller's
    // sum over the 16 lanes adds the 4 blocks' terms.
    typedef Frag KPrep;
    static __device__ __forceinline__ KPrep prep(const Frag &k) { return k; }
    static __device__ __forceinline__ float dot(const KPrep &k, const QFrag &q) {
        int s = __builtin_amdgcn_sdot4((int)k.lo, (int)q.lo, 0, false);
        s = __builtin_amdgcn_sdot4((int)k.hi, (int)q.hi, s, false);
        s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);   // quad xor 1
        s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);   // quad xor 2
        return (threadIdx.x & 3) == 0 ? (float)s * (k.d * q.d) : 0.0f;
    }
    static __device__ __forceinline__ void to_f32(const Frag &v, float *o) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[i] = (float)(int8_t)(v.lo >> (8 * i)) * v.d;
            o[4 + i] = (float)(int8_t)(v.hi >> (8 * i)) * v.d;
        }
    }
};

// Word-wise select between two fragments (constant indices only, so the
// fragment arrays stay in registers).
template <class T>
__device__ __forceinline__ T select_frag(bool c, const T &a, const T &b) {
    static_assert(sizeof(T) % 4 == 0, "fragments are whole dwords");
    uint32_t wa[sizeof(T) / 4], wb[sizeof(T) / 4];
    __builtin_memcpy(wa, &a, sizeof(T));
    __builtin_memcpy(wb, &b, sizeof(T));
#pragma unroll
    for (unsigned i = 0; i < sizeof(T) / 4; ++i) wa[i] = c ? wa[i] : wb[i];
    T r;
    __builtin_memcpy(&r, wa, sizeof(T));
    return r;
}

// Convert 8 new f32 elements (called by every lane: Q8 quantization is
// quad-cooperative) and store them when `ok`.
template <class F>
__device__ __forceinline__ typename F::Frag store_new(uint8_t *row, int e, const float *x, bool ok) {
    const typename F::Frag f = F::from_f32(x);
    if (ok) F::store(row, e, f);
    return f;
}

// ---------------------------------------------------------------------------
// Append.  Thread t converts elements [8t, 8t+8) of the flattened
// [n_rows][kv_dim] source of one (layer, K|V).
// ---------------------------------------------------------------------------
template <class F>
__global__ void __launch_bounds__(256) k_append(AppendArgs a) {
    const int layer = blockIdx.y;
    const int which = blockIdx.z;
    const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    const int64_t total = (int64_t)a.n_rows * a.kv_dim;
    const bool ok = e0 < total;
    const int row = ok ? (int)(e0 / a.kv_dim) : 0;
    const int col = ok ? (int)(e0 % a.kv_dim) : 0;
    float x[8];
    if (ok) {
        const float *src = (which ? a.v_src : a.k_src) + (int64_t)layer * a.src_lstride +
                           (int64_t)row * a.kv_dim + col;
        const float4 p0 = reinterpret_cast<const float4 *>(src)[0];
        const float4 p1 = reinterpret_cast<const float4 *>(src)[1];
        x[0] = p0.x; x[1] = p0.y; x[2] = p0.z; x[3] = p0.w;
        x[4] = p1.x; x[5] = p1.y; x[6] = p1.z; x[7] = p1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.0f;
    }
    const int slot = slot_of(a.seg, row);
    uint8_t *dst = (which ? a.v : a.k) + (int64_t)layer * a.layer_bytes + (int64_t)slot * a.row_bytes;
    store_new<F>(dst, col, x, ok);
}

// ---------------------------------------------------------------------------
// Gather: logical window rows -> contiguous rows, bit-exact.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) k_gather(const uint8_t *src, int64_t row_bytes, SegPair seg,
                                                uint8_t *dst) {
    const int64_t per_row = row_bytes / (int64_t)sizeof(T);
    const int64_t total = (int64_t)(seg.n0 + seg.n1) * per_row;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * 256) {
        const int row = (int)(t / per_row);
        const int64_t w = t % per_row;
        const int slot = slot_of(seg, row);
        reinterpret_cast<T *>(dst)[t] =
            reinterpret_cast<const T *>(src + (int64_t)slot * row_bytes)[w];
    }
}


// Transposing sum over the 16 lanes of a DPP row: lane c holds 16 partials
// v[0..15]; on return it holds sum over the row of v[c].  Each step pairs lanes
// that differ in one bit (row_mirror, row_half_mirror, quad reverse, xor 1):
// the lane keeps the half of its list selected by that bit and adds the
// partner's copy of it.  8+4+2+1 exchanges instead of 16x4.
__device__ __forceinline__ float transpose_sum16(const float *v, int c) {
    float a8[8], a4[4], a2[2];
    const bool b3 = c & 8, b2 = c & 4, b1 = c & 2, b0 = c & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float keep = b3 ? v[k + 8] : v[k];
        const float send = b3 ? v[k] : v[k + 8];
        a8[k] = keep + dpp<0x140>(send);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float keep = b2 ? a8[k + 4] : a8[k];
        const float send = b2 ? a8[k] : a8[k + 4];
        a4[k] = keep + dpp<0x141>(send);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float keep = b1 ? a4[k + 2] : a4[k];
        const float send = b1 ? a4[k] : a4[k + 2];
        a2[k] = keep + dpp<0x1B>(send);
    }
    const float keep = b0 ? a2[1] : a2[0];
    const float send = b0 ? a2[0] : a2[1];
    return keep + dpp<0xB1>(send);
}

// acc[j][i] += sum_u p[u][j] * v_u[i].  F16: slot pairs (u, u+1) are packed
// into half2 lanes and accumulated with v_dot2_f32_f16 (f32 accumulation);
// other formats use f32 FMAs on the dequantised values.
template <class F>
__device__ __forceinline__ void pv_accumulate(float (&acc)[4][8], const typename F::Frag (&vf)[4],
                                              const float4 (&pw)[4]) {
    float vv[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) F::to_f32(vf[u], vv[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float pu[4] = {pw[u].x, pw[u].y, pw[u].z, pw[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[j][i] = fmaf(pu[j], vv[u][i], acc[j][i]);
    }
}

template <>
__device__ __forceinline__ void pv_accumulate<FmtF16>(float (&acc)[4][8], const FmtF16::Frag (&vf)[4],
                                                      const float4 (&pw)[4]) {
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
        const float p0[4] = {pw[u].x, pw[u].y, pw[u].z, pw[u].w};
        const float p1[4] = {pw[u + 1].x, pw[u + 1].y, pw[u + 1].z, pw[u + 1].w};
        half2_t pp[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            pp[j].x = (_Float16)p0[j];
            pp[j].y = (_Float16)p1[j];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // (v_u[2i], v_u+1[2i]) and (v_u[2i+1], v_u+1[2i+1])
            const half2_t lo = as_h2(__builtin_amdgcn_perm(vf[u + 1].w[i], vf[u].w[i], 0x05040100u));
            const half2_t hi = as_h2(__builtin_amdgcn_perm(vf[u + 1].w[i], vf[u].w[i], 0x07060302u));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[j][2 * i] = __builtin_amdgcn_fdot2(lo, pp[j], acc[j][2 * i], false);
                acc[j][2 * i + 1] = __builtin_amdgcn_fdot2(hi, pp[j], acc[j][2 * i + 1], false);
            }
        }
    }
}

// q8_0: the generic f32 path, as ggml's CPU flash attention takes a q8_0 V
// (each value dequantised to f32 exactly, q * d, and accumulated with the
// f32 softmax weight); rounding p * d to f16 for a packed product moved the
// output by up to 5e-4 from that arithmetic on short windows.

// RoPE as ggml computes it on the CPU (mode 0: pairs (2i, 2i+1) of a head),
// for the 4 pairs [pair0, pair0+4) held in x[8]: theta starts at the position
// and is multiplied by theta_scale once per pair in f32 (ggml's running
// product, so theta_i carries i roundings); cos/sin are evaluated in double
// and rounded to f32; no contraction in the rotation.
__device__ __forceinline__ void rope8(float (&x)[8], int pair0, float pos, float theta_scale) {
#pragma clang fp contract(off)
    float theta = pos;
    for (int i = 0; i < pair0; ++i) theta *= theta_scale;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float c = (float)cos((double)theta);
        const float sn = (float)sin((double)theta);
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        x[2 * j] = x0 * c - x1 * sn;
        x[2 * j + 1] = x0 * sn + x1 * c;
        theta *= theta_scale;
    }
}

// The same angles once per work group: lane i of wave 0 computes pair i's
// (cos, sin) with i steps of the running product (64 pairs = head_dim 128),
// or copies them from the host's table (rope_host, one stream); the caller
// synchronises before reading tab.
__device__ __forceinline__ void rope_table(float2 *tab, float pos, float theta_scale) {
#pragma clang fp contract(off)
    if (threadIdx.x < 64) {
        float theta = pos;
        for (int i = 0; i < (int)threadIdx.x; ++i) theta *= theta_scale;
        tab[threadIdx.x] = make_float2((float)cos((double)theta), (float)sin((double)theta));
    }
}

__device__ __forceinline__ void decode_rope_table(float2 *tab, const DecodeArgs &a, int s) {
    if (a.rope_host) {
        if (threadIdx.x < 64) tab[threadIdx.x] = a.rope_tab[threadIdx.x];
    } else {
        rope_table(tab, a.rope_pos[s], a.rope_theta_scale);
    }
}

// Rotation of the 4 pairs [pair0, pair0+4) held in x[8] by a rope_table.
__device__ __forceinline__ void rope8_tab(float (&x)[8], int pair0, const float2 *tab) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float2 cs = tab[pair0 + j];
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        x[2 * j] = x0 * cs.x - x1 * cs.y;
        x[2 * j + 1] = x0 * cs.y + x1 * cs.x;
    }
}

// A lane's 4 (cos, sin) pairs [pair0, pair0 + 4) of the host-evaluated table
// (rope_host): two 16-byte loads, straight into registers.
struct RopePairs {
    float2 cs[4];
};
__device__ __forceinline__ RopePairs rope_pairs_host(const DecodeArgs &a, int pair0) {
    const float4 *t = reinterpret_cast<const float4 *>(a.rope_tab + pair0);
    const float4 x = t[0], y = t[1];
    return RopePairs{{make_float2(x.x, x.y), make_float2(x.z, x.w), make_float2(y.x, y.y),
                      make_float2(y.z, y.w)}};
}
__device__ __forceinline__ RopePairs rope_pairs_lds(const float2 *tab, int pair0) {
    return RopePairs{{tab[pair0], tab[pair0 + 1], tab[pair0 + 2], tab[pair0 + 3]}};
}
// rope8_tab's rotation with the pairs in registers
__device__ __forceinline__ void rope8_pairs(float (&x)[8], const RopePairs &r) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float2 cs = r.cs[j];
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        x[2 * j] = x0 * cs.x - x1 * cs.y;
        x[2 * j + 1] = x0 * cs.y + x1 * cs.x;
    }
}

__global__ void __launch_bounds__(256) k_rope(float *x, int64_t n_outer, int64_t n_rows,
                                              int32_t row_len, int32_t head_dim, int64_t pos0,
                                              float theta_scale) {
    const int64_t per_row = row_len / 8;
    const int64_t total = n_outer * n_rows * per_row;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * 256) {
        const int64_t row = (t / per_row) % n_rows;
        const int e = (int)(t % per_row) * 8;
        float v[8];
        float4 *p = reinterpret_cast<float4 *>(x + (t / per_row) * row_len + e);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        rope8(v, (e % head_dim) / 2, (float)(pos0 + row), theta_scale);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// Work item of a decode work group: (stream s, layer, kv head g, chunk).
struct DecodeItem {
    int g, chunk, layer, s;
};

__device__ __forceinline__ DecodeItem decode_item(const DecodeArgs &a) {
    int item = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (a.xcd_swizzle) {
        // Work groups go round-robin over the 8 XCDs (linear id i runs on XCD
        // i % 8), each with its own L2.  Give the 8 kv heads of one (stream,
        // layer, chunk) -- neighbouring segments of the same rows -- to one
        // XCD, back to back, so lines two heads share are fetched once.
        // (Host-checked: 8 kv heads, work-group count a multiple of 64.)
        const int xcd = item & 7, k = item >> 3;
        item = (((k >> 3) << 3) + xcd) * 8 + (k & 7);
    }
    DecodeItem it;
    it.g = item % a.n_kv_heads;
    it.chunk = (item / a.n_kv_heads) % a.n_chunks;
    it.layer = (item / (a.n_kv_heads * a.n_chunks)) % a.n_layers;
    it.s = item / (a.n_kv_heads * a.n_chunks * a.n_layers);
    return it;
}

// Fused append of the step's new row (run_decoder_step's SET_ROWS,
// src/voxtral.cpp:2682-2694).  The new row is the newest logical index
// n_kv-1; lane group 0 of wave 0 in the work group whose chunk holds it
// converts head g's part once and stores it into the ring.  The caller's
// barrier then makes it visible to every wave, which reads it back like any
// other slot; other work groups never touch the slot.
template <class F>
__device__ __forceinline__ void fused_append(const DecodeArgs &a, const SegPair &sp, int s,
                                             int layer, int64_t base, int e, int i_begin,
                                             int i_end, bool leader, const RopePairs &rp) {
    const int n_kv = sp.n0 + sp.n1;
    if (n_kv >= 1 && n_kv - 1 >= i_begin && n_kv - 1 < i_end && leader) {
        const int slot = slot_of(sp, n_kv - 1);
        const float *kn = a.k_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
        const float *vn = a.v_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
        float xk[8], xv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { xk[i] = kn[i]; xv[i] = vn[i]; }
        if (a.rope) rope8_pairs(xk, rp);   // pairs (e & 127) / 2 = 4c
        store_new<F>(a.k_w + base + (int64_t)slot * a.row_bytes, e, xk, true);
        store_new<F>(a.v_w + base + (int64_t)slot * a.row_bytes, e, xv, true);
    }
}

// Merge of the W waves of a decode work group through LDS, then the
// normalised output (one chunk) or this chunk's partial.
template <int W, int GQA>
struct MergeSmem {
    float m[W][GQA], l[W][GQA];
    float o[W][GQA][128];
};

template <int W, int GQA>
__device__ __forceinline__ void decode_merge_finish(const DecodeArgs &a, const DecodeItem &it,
                                                    const MergeSmem<W, GQA> &sm) {
    constexpr int D = 128;
    __syncthreads();
    const int64_t head0 =
        ((int64_t)it.s * a.n_layers + it.layer) * a.n_q_heads + (int64_t)it.g * GQA;
    for (int t = threadIdx.x; t < GQA * D; t += W * 64) {
        const int j = t / D;
        const int d = t % D;
        float M = sm.m[0][j];
#pragma unroll
        for (int w = 1; w < W; ++w) M = fmaxf(M, sm.m[w][j]);
        float O = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float sc_w = fast_exp2(sm.m[w][j] - M);
                O = fmaf(sm.o[w][j][d], sc_w, O);
                L = fmaf(sm.l[w][j], sc_w, L);
            }
        }
        if (a.n_chunks == 1) {
            a.out[(head0 + j) * D + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            const int64_t pidx = (head0 + j) * a.n_chunks + it.chunk;
            a.part_o[pidx * D + d] = O;
            if (d == 0) {
                a.part_ml[pidx * 2] = M;
                a.part_ml[pidx * 2 + 1] = L;
            }
        }
    }
}

// Lanes 0..15 hold acc[j][8*lane .. +8) (summed over the lane groups) and
// lanes 0..3 the running max m and sum l of head `lane`.
template <int W, int GQA>
__device__ __forceinline__ void decode_merge(const DecodeArgs &a, const DecodeItem &it, int wave,
                                             int lane, float m, float l,
                                             const float (&acc)[GQA][8]) {
    __shared__ MergeSmem<W, GQA> sm;
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < GQA; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) sm.o[wave][j][lane * 8 + i] = acc[j][i];
        if (lane < GQA) {
            sm.m[wave][lane] = m;
            sm.l[wave][lane] = l;
        }
    }
    decode_merge_finish<W, GQA>(a, it, sm);
}

// ---------------------------------------------------------------------------
// Decode attention.  Workgroup = W waves on (stream, layer, kv head g, chunk
// of `chunk` logical slots).  Lane (grp = lane/16, c = lane%16) holds elements
// [8c, 8c+8) of one slot's head row; a wave covers 4 slots per load, 16 slots
// per batch (4 loads of K and of V in flight per lane), and the 4 query heads
// of the GQA group share every K/V load.  With one chunk per (stream, layer,
// kv head) the work group owns the whole window and writes the normalised
// output itself; otherwise it writes a (max, sum, unnormalised output)
// partial for k_combine.  Q (and the host's RoPE pairs) are requested before
// any K/V batch: the vector-memory counter retires loads in order, so waiting
// for Q never waits for K/V.
// ---------------------------------------------------------------------------
template <class F, int GQA, bool FUSE, int W, int NS>
__global__ void __launch_bounds__(W * 64) k_decode(DecodeArgs a) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    // wave index as a scalar: loop bounds derived from it stay uniform
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4;
    const int c = lane & 15;
    const DecodeItem it = decode_item(a);
    const int g = it.g, chunk = it.chunk, layer = it.layer, s = it.s;
    const SegPair sp = a.seg[s];
    const int n_kv = sp.n0 + sp.n1;
    const int64_t base = (int64_t)s * a.stream_bytes + (int64_t)layer * a.layer_bytes;
    const uint8_t *kl = a.k + base;
    const uint8_t *vl = a.v + base;
    const int e = g * D + c * 8;
    const uint32_t row_bytes24 = (uint32_t)a.row_bytes;
    const int i_begin = chunk * a.chunk;
    const int i_end = min(i_begin + a.chunk, n_kv);
    auto load_batch = [&](int b, typename F::Frag (&kf)[4], typename F::Frag (&vf)[4])
                          __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // past the chunk end: reload the last valid slot (masked later);
            // an empty chunk reads slot 0 (unused)
            const int ix = min(b + u * 4 + grp, i_end - 1);
            const int slot = i_begin < i_end ? slot_of(sp, ix) : 0;
            // slot < 2^24 and row_bytes < 2^24 (host-checked): 24-bit multiply
            const uint32_t off = __umul24((uint32_t)slot, row_bytes24);
            kf[u] = F::template load<true>(kl + off, e);
            vf[u] = F::template load<true>(vl + off, e);
        }
    };
    typename F::Frag kf[NS][4], vf[NS][4];
    constexpr int kStep = W * 16;   // slots covered by one batch of all waves
    int b0 = i_begin + wave * 16;

    // Q first, then the host's RoPE pairs of this lane (pairs [4c, 4c+4):
    // the same for its Q elements and its new-K elements)
    float4 qraw[GQA][2];
    {
        const float *qp = a.q + (int64_t)s * a.q_sstride + (int64_t)layer * a.q_lstride +
                          (int64_t)(g * GQA) * D + c * 8;
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
            qraw[j][0] = reinterpret_cast<const float4 *>(qp + j * D)[0];
            qraw[j][1] = reinterpret_cast<const float4 *>(qp + j * D)[1];
        }
    }
    RopePairs rp{};
    if (a.rope && a.rope_host) rp = rope_pairs_host(a, 4 * c);

    // The first batches are requested before the prologue (RoPE table, Q,
    // fused append), unconditionally: a load issued on one path only makes
    // the compiler's wait counts assume it absent, and Q's RoPE then waited
    // for the whole first batch, so the second was requested only after it
    // had arrived.  A work group whose first batches can hold the step's new
    // row (the newest logical index n_kv-1, not yet appended) requests them
    // again after the append.
    const bool early = !FUSE || i_begin + (NS - 1) * kStep <= n_kv - 1;
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) load_batch(b0 + p * kStep, kf[p], vf[p]);
    __shared__ float2 sm_rope[64];
    if (a.rope && !a.rope_host) {
        decode_rope_table(sm_rope, a, s);
        __syncthreads();
        rp = rope_pairs_lds(sm_rope, 4 * c);
    }

    typename F::QFrag qf[GQA];
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
        float qv[8] = {qraw[j][0].x, qraw[j][0].y, qraw[j][0].z, qraw[j][0].w,
                       qraw[j][1].x, qraw[j][1].y, qraw[j][1].z, qraw[j][1].w};
        if (a.rope) rope8_pairs(qv, rp);
        qf[j] = F::make_q(qv);
    }

    static_assert(GQA == 4, "the score transposition maps 4 slots x 4 heads onto 16 lanes");
    // Running softmax state.  After the score transposition lane c of a group
    // owns slot-of-batch u = c>>2 and query head j = c&3: m and l are that
    // head's running max and (partial) sum.  acc[j][i] is the unnormalised
    // output of head j at dimension 8c+i over this lane group's slots.
    const int hj = c & 3;
    const int hu = c >> 2;
    float m = -INFINITY, l = 0.0f;
    float acc[GQA][8];
#pragma unroll
    for (int j = 0; j < GQA; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = 0.0f;
    __shared__ float4 sm_p[W][16];   // per wave: p[slot of batch][head]

    // (always inlined: the fragment arrays must stay in registers)
    auto process = [&](typename F::Frag (&kf)[4], typename F::Frag (&vf)[4], const int b0)
                       __attribute__((always_inline)) {
        // QK partials over this lane's 8 dimensions, then a transposing
        // reduction over the 16 lanes of the group: lane c ends with the full
        // score of (slot u = c>>2, head j = c&3).
        float part[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const typename F::KPrep kp = F::prep(kf[u]);
#pragma unroll
            for (int j = 0; j < GQA; ++j) part[u * 4 + j] = F::dot(kp, qf[j]);
        }
        const int my_idx = b0 + hu * 4 + grp;
        float sc = transpose_sum16(part, c) * a.scale_log2;
        if (my_idx >= i_end) sc = -INFINITY;

        // batch max of head j: lanes {j, j+4, j+8, j+12} of the row, then groups
        float bm = fmaxf(sc, dpp<0x124>(sc));
        bm = fmaxf(bm, dpp<0x128>(bm));
        bm = xor16_max(bm);
        bm = xor32_max(bm);
        // Lazy rescale: the reference max only moves when a head's batch max
        // exceeds it by more than 2^8, so p <= 256 and rescaling is rare.
        if (__any(bm > m + 8.0f)) {
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fast_exp2(m - mn);
            l *= alpha;
            float al[GQA];
            al[0] = dpp<0x00>(alpha);    // quad broadcast of head 0..3's alpha
            al[1] = dpp<0x55>(alpha);
            al[2] = dpp<0xAA>(alpha);
            al[3] = dpp<0xFF>(alpha);
#pragma unroll
            for (int j = 0; j < GQA; ++j)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[j][i] *= al[j];
            m = mn;
        }
        const float p = sc == -INFINITY ? 0.0f : fast_exp2(sc - m);
        l += p;
        // hand every lane of the group the 4 heads' weights of each of its slots
        reinterpret_cast<float *>(&sm_p[wave][hu * 4 + grp])[hj] = p;
        __builtin_amdgcn_wave_barrier();
        float4 pw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) pw[u] = sm_p[wave][u * 4 + grp];
        __builtin_amdgcn_wave_barrier();
        pv_accumulate<F>(acc, vf, pw);
    };

    if (FUSE) {
        fused_append<F>(a, sp, s, layer, base, e, i_begin, i_end, wave == 0 && grp == 0, rp);
        __syncthreads();
    }
    // Software pipeline over NS register sets (no copies, so the wave never
    // waits on a batch it has just requested): while batch p is reduced, the
    // loads of the next NS-1 batches are in flight.  The loop body always
    // handles NS batches and the prefetches are unconditional (indices clamp
    // to the last valid slot, an L2 hit; batches past the end are fully
    // masked), so the wait counts stay exact.
    if (!early && i_begin < i_end) {   // the first batches again, after the append
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) load_batch(b0 + p * kStep, kf[p], vf[p]);
    }
    for (; b0 < i_end; b0 += NS * kStep) {
#pragma unroll
        for (int p = 0; p < NS; ++p) {
            load_batch(b0 + (p + NS - 1) * kStep, kf[(p + NS - 1) % NS], vf[(p + NS - 1) % NS]);
            process(kf[p], vf[p], b0 + p * kStep);
        }
    }

    // Merge the 4 lane groups (they share m): every lane of head j sums l
    // over its row and the groups; acc over the groups.
    l += dpp<0x124>(l);
    l += dpp<0x128>(l);
    l = xor16_sum(l);
    l = xor32_sum(l);
#pragma unroll
    for (int j = 0; j < GQA; ++j) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = xor32_sum(xor16_sum(acc[j][i]));
    }

    decode_merge<W, GQA>(a, it, wave, lane, m, l, acc);
}

// ---------------------------------------------------------------------------
// Decode attention by whole rows (F16, 8 kv heads x 128, 4 query heads each).
// Work group = 8 waves on (stream, layer, chunk of `chunk` logical slots);
// wave w reads half h = w & 1 of each row (kv heads 4h..4h+3, 1 KiB, one
// load instruction of 16 B per lane) for the slots of sub-stream sw = w >> 1:
// per round the 4 sub-streams take 16 consecutive slots, 4 each, and both
// halves read the same slots, so the work group consumes whole rows.  Lane
// (grp, c) holds dims [8c, 8c+8) of kv head 4h + grp; the 16 lanes of a group
// are that head's, so the score transposition, the running max and sum and
// the P.V accumulation are k_decode's with one head per lane group.  The 4
// sub-streams of each head meet in LDS; one chunk writes the output, several
// write partials for k_combine.
// ---------------------------------------------------------------------------
template <bool FUSE, int NS>
__global__ void __launch_bounds__(512) k_decode_rows(DecodeArgs a) {
    using F = FmtF16;
    constexpr int D = 128, GQA = 4, NH = 32;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = wave & 1, sw = wave >> 1;
    const int grp = lane >> 4, c = lane & 15;
    const int g = 4 * h + grp;
    const int chunk = blockIdx.x, layer = blockIdx.y, s = blockIdx.z;
    const SegPair sp = a.seg[s];
    const int n_kv = sp.n0 + sp.n1;
    const int64_t base = (int64_t)s * a.stream_bytes + (int64_t)layer * a.layer_bytes;
    const uint8_t *kl = a.k + base;
    const uint8_t *vl = a.v + base;
    const int e = g * D + c * 8;
    const uint32_t row_bytes24 = (uint32_t)a.row_bytes;
    const int i_begin = chunk * a.chunk;
    const int i_end = min(i_begin + a.chunk, n_kv);
    auto load_batch = [&](int b, F::Frag (&kf)[4], F::Frag (&vf)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // past the chunk end: reload the last valid slot (masked later)
            const int ix = min(b + u, i_end - 1);
            const uint32_t off = __umul24((uint32_t)slot_of(sp, ix), row_bytes24);
            kf[u] = F::load<true>(kl + off, e);
            vf[u] = F::load<true>(vl + off, e);
        }
    };
    F::Frag kf[NS][4], vf[NS][4];
    constexpr int kStep = 16;   // slots per round of the 4 sub-streams
    int b0 = i_begin + 4 * sw;
    const bool early = !FUSE || i_begin + (NS - 1) * kStep <= n_kv - 1;
    if (early && i_begin < i_end) {
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) load_batch(b0 + p * kStep, kf[p], vf[p]);
    }
    __shared__ float2 sm_rope[64];
    if (a.rope) {
        decode_rope_table(sm_rope, a, s);
        __syncthreads();
    }
    F::QFrag qf[GQA];
    {
        const float *qp = a.q + (int64_t)s * a.q_sstride + (int64_t)layer * a.q_lstride +
                          (int64_t)(g * GQA) * D + c * 8;
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
            const float4 q0 = reinterpret_cast<const float4 *>(qp + j * D)[0];
            const float4 q1 = reinterpret_cast<const float4 *>(qp + j * D)[1];
            float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            if (a.rope) rope8_tab(qv, 4 * c, sm_rope);
            qf[j] = F::make_q(qv);
        }
    }
    const int hj = c & 3;
    const int hu = c >> 2;
    float m = -INFINITY, l = 0.0f;
    float acc[GQA][8];
#pragma unroll
    for (int j = 0; j < GQA; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = 0.0f;
    __shared__ float4 sm_p[8][16];   // per wave: p[slot u * 4 + group][head]

    auto process = [&](F::Frag (&kf)[4], F::Frag (&vf)[4], const int b) __attribute__((always_inline)) {
        float part[16];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < GQA; ++j) part[u * 4 + j] = F::dot(kf[u], qf[j]);
        float sc = transpose_sum16(part, c) * a.scale_log2;   // (slot u = hu, head j = hj)
        if (b + hu >= i_end) sc = -INFINITY;
        // batch max of head j over the group's 4 slots (lanes j, j+4, j+8, j+12)
        float bm = fmaxf(sc, dpp<0x124>(sc));
        bm = fmaxf(bm, dpp<0x128>(bm));
        if (__any(bm > m + 8.0f)) {
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fast_exp2(m - mn);
            l *= alpha;
            float al[GQA];
            al[0] = dpp<0x00>(alpha);
            al[1] = dpp<0x55>(alpha);
            al[2] = dpp<0xAA>(alpha);
            al[3] = dpp<0xFF>(alpha);
#pragma unroll
            for (int j = 0; j < GQA; ++j)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[j][i] *= al[j];
            m = mn;
        }
        const float p = sc == -INFINITY ? 0.0f : fast_exp2(sc - m);
        l += p;
        reinterpret_cast<float *>(&sm_p[wave][hu * 4 + grp])[hj] = p;
        __builtin_amdgcn_wave_barrier();
        float4 pw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) pw[u] = sm_p[wave][u * 4 + grp];
        __builtin_amdgcn_wave_barrier();
        pv_accumulate<F>(acc, vf, pw);
    };
    if (FUSE) {
        // the step's new row (the newest logical index): the two sub-stream-0
        // waves of the work group that holds it write both halves
        if (n_kv >= 1 && n_kv - 1 >= i_begin && n_kv - 1 < i_end && sw == 0) {
            const int slot = slot_of(sp, n_kv - 1);
            const float *kn = a.k_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
            const float *vn = a.v_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
            float xk[8], xv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) { xk[i] = kn[i]; xv[i] = vn[i]; }
            if (a.rope) rope8_tab(xk, (e & 127) >> 1, sm_rope);
            store_new<F>(a.k_w + base + (int64_t)slot * a.row_bytes, e, xk, true);
            store_new<F>(a.v_w + base + (int64_t)slot * a.row_bytes, e, xv, true);
        }
        __syncthreads();
    }
    if (!early && i_begin < i_end) {
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) load_batch(b0 + p * kStep, kf[p], vf[p]);
    }
    for (; b0 < i_end; b0 += NS * kStep) {
#pragma unroll
        for (int p = 0; p < NS; ++p) {
            load_batch(b0 + (p + NS - 1) * kStep, kf[(p + NS - 1) % NS], vf[(p + NS - 1) % NS]);
            process(kf[p], vf[p], b0 + p * kStep);
        }
    }
    // the head's sum over its 4 slot lanes (the max is shared already)
    l += dpp<0x124>(l);
    l += dpp<0x128>(l);

    // the 4 sub-streams of each head meet in LDS
    __shared__ float sm_m[4][NH], sm_l[4][NH];
    __shared__ float sm_o[4][NH][D];
    if (c < GQA) {
        sm_m[sw][g * GQA + c] = m;   // lane c < 4: head j = c (slot 0's lanes)
        sm_l[sw][g * GQA + c] = l;
    }
#pragma unroll
    for (int j = 0; j < GQA; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) sm_o[sw][g * GQA + j][c * 8 + i] = acc[j][i];
    __syncthreads();
    const int64_t head0 = ((int64_t)s * a.n_layers + layer) * a.n_q_heads;
    for (int t = threadIdx.x; t < NH * D; t += 512) {
        const int hh = t / D, d = t % D;
        float M = sm_m[0][hh];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, sm_m[w][hh]);
        float O = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float sc_w = fast_exp2(sm_m[w][hh] - M);
                O = fmaf(sm_o[w][hh][d], sc_w, O);
                L = fmaf(sm_l[w][hh], sc_w, L);
            }
        }
        if (a.n_chunks == 1) {
            a.out[(head0 + hh) * D + d] = L > 0.0f ? O / L : 0.0f;
        } else {
            const int64_t pidx = (head0 + hh) * a.n_chunks + chunk;
            a.part_o[pidx * D + d] = O;
            if (d == 0) {
                a.part_ml[pidx * 2] = M;
                a.part_ml[pidx * 2 + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode attention over a q8_0 cache on the matrix cores, in ggml's q8_0
// arithmetic for QK: Q is quantized per 32-element block with the cache's own
// quantizer and each v_mfma_i32_16x16x32_i8 contracts exactly one block, so
// the block sums are exact integers; score = sum_t sumi_t * d_k[t] * d_q[t].
// Per 16-slot batch of a wave:
//   - K and V rows arrive with k_decode's q8_0 loads (lane group kg holds
//     slots 4kg + u, lane r quants [8r, 8r+8) of the head and their block
//     scale; one address computation serves both), and are written to
//     per-wave LDS tiles with the quants de-interleaved from the scales
//     (128 contiguous quant bytes per slot).
//   - QK: A = K quants (lane (kg, r): block t quants [8kg, +8) of slot r, one
//     ds_read_b64), B = Q quants (heads as columns 0..3).  Lane (kg, n < 4)
//     receives slots 4kg + i (i = 0..3) of head n.
//   - P.V: O^T[d][head] += V^T[d][slot] P^T[slot][head] with
//     v_mfma_f32_16x16x16f16 per 16-dim tile.  B = p * d_v in f16 -- exactly
//     the score lanes' layout, so p never leaves registers.  A = V^T comes
//     from ds_read_b64_tr_b8: within each 16-lane group, output lane j byte k
//     is byte j%8 of source lane 2k + j/8, so one transpose read hands every
//     lane the 4 slots x 2 tiles of int8 values it needs for a block; they
//     are spliced into f16 exactly (1024 + 128 + q under the f16 exponent).
// ---------------------------------------------------------------------------
typedef int int4v_t __attribute__((ext_vector_type(4)));
typedef int int2v_t __attribute__((ext_vector_type(2)));
typedef float float4v_t __attribute__((ext_vector_type(4)));
typedef _Float16 half4v_t __attribute__((ext_vector_type(4)));

// 4 int8 values (one per byte) -> exact f16x4
__device__ __forceinline__ half4v_t i8x4_to_h4(uint32_t x) {
    const uint32_t b = x ^ 0x80808080u;
    const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const half2_t lo = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x05010400u)) - off;
    const half2_t hi = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x05030402u)) - off;
    return half4v_t{lo.x, lo.y, hi.x, hi.y};
}

// q8_0 fragment loads through a buffer resource: the layer base sits in the
// descriptor (SGPRs) and each lane adds a 32-bit offset, so no 64-bit address
// arithmetic per load.  Lane-constant part of element e's offsets:
struct Q8LaneOff {
    uint32_t q;    // first dword holding the 8 quants
    uint32_t d;    // the block scale
    uint32_t sh;   // byte shift of the quants in that dword (0 or 2)
};
__device__ __forceinline__ Q8LaneOff q8_lane_off(int e) {
    const uint32_t bo = (uint32_t)(e >> 5) * 34u;
    const uint32_t qo = bo + 2u + (uint32_t)(e & 31);
    return Q8LaneOff{qo & ~3u, bo, qo & 3u};
}
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
__device__ __forceinline__ FmtQ8::Frag q8_load_buf(__amdgpu_buffer_rsrc_t rs, uint32_t row_off,
                                                   const Q8LaneOff &lo) {
    const u32x3_t w = __builtin_amdgcn_raw_buffer_load_b96(rs, row_off + lo.q, 0, 0);
    const uint16_t dh = __builtin_amdgcn_raw_buffer_load_b16(rs, row_off + lo.d, 0, 0);
    FmtQ8::Frag f;
    f.lo = __builtin_amdgcn_alignbyte(w.y, w.x, lo.sh);
    f.hi = __builtin_amdgcn_alignbyte(w.z, w.y, lo.sh);
    f.d = (float)__builtin_bit_cast(_Float16, dh);
    return f;
}

template <bool FUSE, int NS, int SB>
__global__ void __launch_bounds__(256) k_decode_q8mfma(DecodeArgs a) {
    constexpr int D = 128, GQA = 4, W = 4;
    constexpr int QS = D + 8;             // LDS row stride of the quant tiles (bytes)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kg = lane >> 4;
    const int r = lane & 15;
    const DecodeItem it = decode_item(a);
    const int g = it.g, layer = it.layer, s = it.s;
    const SegPair sp = a.seg[s];
    const int n_kv = sp.n0 + sp.n1;
    const int64_t base = (int64_t)s * a.stream_bytes + (int64_t)layer * a.layer_bytes;
    const uint8_t *kl = a.k + base;
    const uint8_t *vl = a.v + base;
    const int e = g * D + r * 8;          // quants [8r, 8r+8) of head g
    const bool score_lane = r < GQA;
    // Buffer descriptors of this (stream, layer)'s K and V: the records
    // extend 256 bytes past the layer (the next layer, or the allocation's
    // tail pad), covering the third quant dword of the last row.
    const uint32_t n_rec = (uint32_t)min<int64_t>(a.layer_bytes + 256, (int64_t)UINT32_MAX);
    const __amdgpu_buffer_rsrc_t k_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)kl, (short)0, (int)n_rec, 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)vl, (short)0, (int)n_rec, 0x00020000);
    const Q8LaneOff qlo = q8_lane_off(e);
    const uint32_t row_bytes24 = (uint32_t)a.row_bytes;
    const int i_begin = it.chunk * a.chunk;
    const int i_end = min(i_begin + a.chunk, n_kv);
    // A step of a wave covers SB sub-batches of 16 slots: [b, b + 16 SB).
    using Frags = FmtQ8::Frag[SB][4];
    auto load_step = [&](int b, Frags &kf, Frags &vf) __attribute__((always_inline)) {
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                // past the chunk end: reload the last valid slot (masked later)
                const int ix = min(b + 16 * sb + 4 * kg + u, i_end - 1);
                const uint32_t off = __umul24((uint32_t)slot_of(sp, ix), row_bytes24);
                kf[sb][u] = q8_load_buf(k_rs, off, qlo);
                vf[sb][u] = q8_load_buf(v_rs, off, qlo);
            }
    };
    Frags kf[NS], vf[NS];
    constexpr int kStep = W * 16 * SB;
    int b0 = i_begin + wave * 16 * SB;
    // The first steps are requested before the prologue (RoPE table, Q,
    // fused append) whenever none of them can hold the step's new row, the
    // newest logical index n_kv-1; clamped indices then stay below it too.
    const bool early = !FUSE || i_begin + (NS - 1) * kStep <= n_kv - 1;
    if (early && i_begin < i_end) {   // i_end >= 1: every clamped index is a valid slot
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) load_step(b0 + p * kStep, kf[p], vf[p]);
    }
    __shared__ float2 sm_rope[64];
    if (a.rope) {
        decode_rope_table(sm_rope, a, s);
        __syncthreads();
    }

    // Q of head r, block t, quants [8kg, 8kg+8): the B operand of QK,
    // quantized as the cache is (d = amax/127, id = 1/d, round half away from
    // zero, d kept in f16); the block's amax spans the 4 lane groups.
    int64_t qb[4];
    float dq[4];
    {
        const float *qp = a.q + (int64_t)s * a.q_sstride + (int64_t)layer * a.q_lstride +
                          (int64_t)(g * GQA + (score_lane ? r : 0)) * D + kg * 8;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma clang fp contract(off)
            float x[8];
            const float4 q0 = score_lane ? reinterpret_cast<const float4 *>(qp + 32 * t)[0]
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 q1 = score_lane ? reinterpret_cast<const float4 *>(qp + 32 * t)[1]
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
            x[0] = q0.x; x[1] = q0.y; x[2] = q0.z; x[3] = q0.w;
            x[4] = q1.x; x[5] = q1.y; x[6] = q1.z; x[7] = q1.w;
            if (a.rope) rope8_tab(x, 16 * t + 4 * kg, sm_rope);
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
            amax = fmaxf(amax, __shfl_xor(amax, 16));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint64_t w = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                w |= (uint64_t)((uint32_t)((int)round_half_away(x[i] * id)) & 0xffu) << (8 * i);
            qb[t] = (int64_t)w;
            dq[t] = (float)(_Float16)d;
        }
    }

    // Score lanes (r < 4): running max m and partial sum l of head r, and
    // o[T] = O^T tile T: dims 16T + 4kg + i of head r.
    float m = -INFINITY, l = 0.0f;
    float4v_t o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = float4v_t{0.0f, 0.0f, 0.0f, 0.0f};
    __shared__ __align__(16) uint8_t sm_kq[W][SB][16 * QS];
    __shared__ __align__(16) uint8_t sm_vq[W][SB][16 * QS];
    __shared__ float4 sm_dk[W][SB][16];  // per wave: d_k[slot][block]
    __shared__ float4 sm_dv[W][SB][16];  // per wave: d_v[slot][block]

    // The sub-batches are independent up to the softmax, which takes one
    // joint max (one cross-lane chain) and one rescale decision per step.
    auto process = [&](const Frags &kf, const Frags &vf, const int b0)
                       __attribute__((always_inline)) {
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int row = (4 * kg + u) * QS + 8 * r;
                *reinterpret_cast<uint2 *>(sm_kq[wave][sb] + row) = make_uint2(kf[sb][u].lo, kf[sb][u].hi);
                *reinterpret_cast<uint2 *>(sm_vq[wave][sb] + row) = make_uint2(vf[sb][u].lo, vf[sb][u].hi);
                // the 4 lanes of a block write the same scale
                reinterpret_cast<float *>(&sm_dk[wave][sb][4 * kg + u])[r >> 2] = kf[sb][u].d;
                reinterpret_cast<float *>(&sm_dv[wave][sb][4 * kg + u])[r >> 2] = vf[sb][u].d;
            }
        __builtin_amdgcn_wave_barrier();
        // QK: one MFMA per block t
        int4v_t ci[SB][4];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint2 ka =
                    *reinterpret_cast<const uint2 *>(sm_kq[wave][sb] + r * QS + 32 * t + 8 * kg);
                ci[sb][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                    (int64_t)(((uint64_t)ka.y << 32) | ka.x), qb[t], int4v_t{0, 0, 0, 0}, 0, 0, 0);
            }
        // V^T operands, block P: lane 2k+h of a group reads quants
        // [32P + 16(k>>2) + 8h, +8) of slot 4kg + (k&3)
        int2v_t vt8[SB][4];
        {
            const int k = r >> 1, h = r & 1;
            const int src = (4 * kg + (k & 3)) * QS + 16 * (k >> 2) + 8 * h;
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int P = 0; P < 4; ++P)
                    vt8[sb][P] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                        (__attribute__((address_space(3))) int2v_t *)(sm_vq[wave][sb] + src + 32 * P));
        }
        float sc[SB][4];
        float bm = -INFINITY;
        float4 dvs[SB][4];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 dk = sm_dk[wave][sb][4 * kg + i];
                dvs[sb][i] = sm_dv[wave][sb][4 * kg + i];
                float x = 0.0f;
                x = fmaf((float)ci[sb][0][i], dk.x * dq[0], x);
                x = fmaf((float)ci[sb][1][i], dk.y * dq[1], x);
                x = fmaf((float)ci[sb][2][i], dk.z * dq[2], x);
                x = fmaf((float)ci[sb][3][i], dk.w * dq[3], x);
                const bool ok = score_lane && b0 + 16 * sb + 4 * kg + i < i_end;
                sc[sb][i] = ok ? x * a.scale_log2 : -INFINITY;
                bm = fmaxf(bm, sc[sb][i]);
            }
        __builtin_amdgcn_wave_barrier();
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        // Lazy rescale: the reference max only moves when a head's batch max
        // exceeds it by more than 2^8, so p <= 256 and rescaling is rare.
        if (__any(bm > m + 8.0f)) {
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fast_exp2(m - mn);
            l *= alpha;
            m = mn;
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t] *= alpha;
        }
        float p[SB][4];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[sb][i] = sc[sb][i] == -INFINITY ? 0.0f : fast_exp2(sc[sb][i] - m);
                l += p[sb][i];
            }
        // P.V per block P: B = p * d_v[.][P] (f16), two 16-dim tiles; the
        // sub-batches alternate so that dependent MFMAs are 8 apart
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int P = 0; P < 4; ++P) {
                const half4v_t pb = {
                    (_Float16)(p[sb][0] * reinterpret_cast<const float *>(&dvs[sb][0])[P]),
                    (_Float16)(p[sb][1] * reinterpret_cast<const float *>(&dvs[sb][1])[P]),
                    (_Float16)(p[sb][2] * reinterpret_cast<const float *>(&dvs[sb][2])[P]),
                    (_Float16)(p[sb][3] * reinterpret_cast<const float *>(&dvs[sb][3])[P])};
                o[2 * P] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    i8x4_to_h4((uint32_t)vt8[sb][P].x), pb, o[2 * P], 0, 0, 0);
                o[2 * P + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    i8x4_to_h4((uint32_t)vt8[sb][P].y), pb, o[2 * P + 1], 0, 0, 0);
            }
    };
    if (FUSE) {
        fused_append<FmtQ8>(a, sp, s, layer, base, e, i_begin, i_end, wave == 0 && kg == 0,
                            a.rope ? rope_pairs_lds(sm_rope, (e & 127) >> 1) : RopePairs{});
        __syncthreads();
    }

    if (!early && i_begin < i_end) {
#pragma unroll
        for (int p = 0; p < NS - 1; ++p) load_step(b0 + p * kStep, kf[p], vf[p]);
    }
    for (; b0 < i_end; b0 += NS * kStep) {
#pragma unroll
        for (int p = 0; p < NS; ++p) {
            load_step(b0 + (p + NS - 1) * kStep, kf[(p + NS - 1) % NS], vf[(p + NS - 1) % NS]);
            process(kf[p], vf[p], b0 + p * kStep);
        }
    }

    // l over the 4 lane groups of each head; publish O^T (score lanes) for
    // the merge of the waves
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    __shared__ MergeSmem<W, GQA> msm;
    if (score_lane) {
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) msm.o[wave][r][16 * t + 4 * kg + i] = o[t][i];
        if (kg == 0) {
            msm.m[wave][r] = m;
            msm.l[wave][r] = l;
        }
    }
    decode_merge_finish<W, GQA>(a, it, msm);
}

// ---------------------------------------------------------------------------
// q8_0 decode by whole rows (8 kv heads x 128, 4 query heads each).  Work
// group = 8 waves on (stream, layer, chunk of `chunk` logical slots); wave g
// owns kv head g over the whole chunk, so no merge between waves.  Per stage
// of 16 slots the K and V rows (2 x 16 x 1088 bytes, contiguous within a
// ring segment) arrive as flat 16-byte streaming loads, NR stages ahead in
// registers, and are stored raw into LDS -- whole rows per load instruction,
// the pattern that streams fastest (the per-head kernel's 12-byte fragments,
// 4 slots x 136 bytes per instruction, read each shared line twice).  Each
// wave then feeds the matrix cores straight from its head's 136-byte segment
// of the raw rows, with no re-pack:
//   - QK on v_mfma_i32_16x16x32_i8 with the segment's bytes as the
//     contraction index: MFMA m, lane (kg, r) supplies bytes [40kg + 8m, +8)
//     of slot r's segment (8-byte aligned; m = 0..4 covers 160 >= 136
//     bytes), and lane (kg, c) of B supplies, for column c = (query head h
//     of the group, block t), Q_h's q8_0 code where that byte is quant q of
//     block t and 0 elsewhere (block scales, other blocks, the next
//     segment).  C[slot][(h, t)] is block t's exact integer sum (ggml's
//     sumi); the score sum_t sumi_t d_k[t] d_q[t] meets across the 4 lanes
//     of a quad.  Q is quantized as the cache is (d = amax/127, round half
//     away, d kept in f16).
//   - P.V on v_mfma_f32_16x16x16f16 over the segment's nine 16-byte
//     windows: A = V^T[byte][slot] from ds_read_b64_tr_b8 (the int8 codes
//     spliced into f16 exactly), B column (h, P) = p_h * d_v[.][P] in f16.
//     Output row x of window w is dim 32P + q of head h when byte 16w + x
//     is quant q of block P, so every dim lands in exactly one (window, row,
//     column) and the other outputs are never read.
// ---------------------------------------------------------------------------
// Work-group barrier that orders LDS accesses only: global loads in flight
// stay in flight (__syncthreads' release would wait for them too).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool FUSE, int NR>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_decode_q8rows(DecodeArgs a) {
    constexpr int D = 128, GQA = 4, NQ = 32, SL = 16;
    constexpr int RB = 1088;                  // q8_0 row: 32 blocks x 34 bytes
    constexpr int RS = RB + 16;               // LDS row stride (a multiple of 8)
    constexpr int SEGB = 136;                 // one kv head's bytes in a row
    // V rows follow the K rows; reads past the last segment (up to 24
    // bytes: the fifth QK step, the ninth window's pair) stay in the slack
    constexpr int KVO = SL * RS + 32;
    constexpr int NW = 9;                     // 16-byte windows of a segment
    constexpr uint32_t kOobOff = 0xFFFFFF00u; // past every descriptor: loads read 0
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int g = __builtin_amdgcn_readfirstlane(tid >> 6);   // this wave's kv head
    const int kg = lane >> 4;
    const int r = lane & 15;
    const int hc = r >> 2, tc = r & 3;        // this lane's column: query head hc, block tc
    const int chunk = blockIdx.x, layer = blockIdx.y, s = blockIdx.z;
    const SegPair sp = a.seg[s];
    const int n_kv = sp.n0 + sp.n1;
    const int64_t base = (int64_t)s * a.stream_bytes + (int64_t)layer * a.layer_bytes;
    const uint8_t *kl = a.k + base;
    const uint8_t *vl = a.v + base;
    const int i_begin = chunk * a.chunk;
    const int i_end = min(i_begin + a.chunk, n_kv);
    const int seg = SEGB * g;

    __shared__ __align__(16) uint8_t sm_raw[2][2 * KVO];
    __shared__ __align__(16) uint8_t sm_qc[NQ][D];   // Q's q8_0 codes
    __shared__ float sm_dq[NQ][4];                   // their block scales
    __shared__ float2 sm_rope[64];

    // Stage loads: K (or V) unit u of a stage is bytes [16 (u % 68), +16) of
    // its row u / 68.  Thread tid takes the K and V units tid and tid + 512;
    // the last 64 units of K go to wave 0 and those of V to wave 1 (the
    // other waves' fifth load reads past its descriptor: zeros, no memory
    // access).  Every load is issued with no branch around it, so the wait
    // counts stay exact; slots past the chunk's end reload its last valid
    // one (slot 0 for an empty window), masked in the scores.
    const uint32_t n_rec = (uint32_t)min<int64_t>(a.layer_bytes + 256, (int64_t)UINT32_MAX);
    const __amdgpu_buffer_rsrc_t k_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)kl, (short)0, (int)n_rec, 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)vl, (short)0, (int)n_rec, 0x00020000);
    const __amdgpu_buffer_rsrc_t x_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(g == 1 ? vl : kl), (short)0, (int)n_rec, 0x00020000);
    const int u0 = tid, u1 = tid + 512, u2 = 1024 + lane;
    const int j0 = u0 / 68, j1 = u1 / 68, j2 = u2 / 68;
    const uint32_t c0 = 16u * (uint32_t)(u0 % 68), c1 = 16u * (uint32_t)(u1 % 68),
                   c2 = 16u * (uint32_t)(u2 % 68);
    const bool x_load = g < 2;
    typedef u32x4_t Stage[5];
    auto row_off = [&](int b, int j) __attribute__((always_inline)) {
        const int ix = max(min(b + j, i_end - 1), 0);
        return __umul24((uint32_t)slot_of(sp, ix), (uint32_t)RB);
    };
    auto load_stage = [&](int b, Stage &dst) __attribute__((always_inline)) {
        const uint32_t o0 = row_off(b, j0) + c0, o1 = row_off(b, j1) + c1;
        const uint32_t o2 = x_load ? row_off(b, j2) + c2 : kOobOff;
        dst[0] = __builtin_amdgcn_raw_buffer_load_b128(k_rs, o0, 0, 2);
        dst[1] = __builtin_amdgcn_raw_buffer_load_b128(k_rs, o1, 0, 2);
        dst[2] = __builtin_amdgcn_raw_buffer_load_b128(v_rs, o0, 0, 2);
        dst[3] = __builtin_amdgcn_raw_buffer_load_b128(v_rs, o1, 0, 2);
        dst[4] = __builtin_amdgcn_raw_buffer_load_b128(x_rs, o2, 0, 2);
    };
    const uint32_t s0 = (uint32_t)(j0 * RS) + c0, s1 = (uint32_t)(j1 * RS) + c1,
                   s2 = (uint32_t)(j2 * RS) + c2 + (g == 1 ? (uint32_t)KVO : 0u);
    auto store_stage = [&](const Stage &src, uint8_t *raw) __attribute__((always_inline)) {
        *reinterpret_cast<u32x4_t *>(raw + s0) = src[0];
        *reinterpret_cast<u32x4_t *>(raw + s1) = src[1];
        *reinterpret_cast<u32x4_t *>(raw + KVO + s0) = src[2];
        *reinterpret_cast<u32x4_t *>(raw + KVO + s1) = src[3];
        if (x_load) *reinterpret_cast<u32x4_t *>(raw + s2) = src[4];
    };

    if (a.rope) {
        decode_rope_table(sm_rope, a, s);
        lds_barrier();
    }
    // Q: thread tid quantizes elements [8 (tid & 3), +8) of block (tid >> 2)
    // & 3 of query head tid >> 4 (requested before the stage loads, so that
    // its first use waits for these loads alone)
    const int qh = tid >> 4, qt = (tid >> 2) & 3, qp = tid & 3;
    float qx[8];
    {
        const float *qsrc = a.q + (int64_t)s * a.q_sstride + (int64_t)layer * a.q_lstride +
                            (int64_t)qh * D + 32 * qt + 8 * qp;
        const float4 q0 = reinterpret_cast<const float4 *>(qsrc)[0];
        const float4 q1 = reinterpret_cast<const float4 *>(qsrc)[1];
        qx[0] = q0.x; qx[1] = q0.y; qx[2] = q0.z; qx[3] = q0.w;
        qx[4] = q1.x; qx[5] = q1.y; qx[6] = q1.z; qx[7] = q1.w;
    }
    // The work group whose chunk holds the step's new row (the newest logical
    // index n_kv - 1) stores it first: lanes (kg = 0, r) of wave g quantize
    // quants [8r, 8r + 8) of head g (quads = blocks) with the block scales;
    // the barrier's release orders those global stores before the loads.
    if (FUSE && n_kv >= 1 && n_kv - 1 >= i_begin && n_kv - 1 < i_end) {
        if (kg == 0) {
            const int slot = slot_of(sp, n_kv - 1);
            const int e = g * D + r * 8;
            const float *kn = a.k_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
            const float *vn = a.v_new + (int64_t)s * a.new_sstride + (int64_t)layer * a.new_lstride + e;
            float xk[8], xv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) { xk[i] = kn[i]; xv[i] = vn[i]; }
            if (a.rope) rope8_tab(xk, (e & 127) >> 1, sm_rope);
            store_new<FmtQ8>(a.k_w + base + (int64_t)slot * a.row_bytes, e, xk, true);
            store_new<FmtQ8>(a.v_w + base + (int64_t)slot * a.row_bytes, e, xv, true);
        }
        __syncthreads();
    }
    Stage stg[NR];
#pragma unroll
    for (int p = 0; p < NR; ++p) load_stage(i_begin + p * SL, stg[p]);

    {
#pragma clang fp contract(off)
        if (a.rope) rope8_tab(qx, 16 * qt + 4 * qp, sm_rope);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(qx[i]));
        amax = quad_max(amax);
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= ((uint32_t)((int)round_half_away(qx[i] * id)) & 0xffu) << (8 * i);
            w1 |= ((uint32_t)((int)round_half_away(qx[4 + i] * id)) & 0xffu) << (8 * i);
        }
        *reinterpret_cast<uint2 *>(&sm_qc[qh][32 * qt + 8 * qp]) = make_uint2(w0, w1);
        if (qp == 0) sm_dq[qh][qt] = (float)(_Float16)d;
    }
    lds_barrier();
    // B of QK step m: byte x = 40 kg + 8 m + i of the segment is quant
    // x - 34 tc - 2 of block tc when that lies in [0, 32)
    int64_t qb[5];
    {
        const uint8_t *qc = sm_qc[g * GQA + hc];
#pragma unroll
        for (int m = 0; m < 5; ++m) {
            uint64_t w = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = 40 * kg + 8 * m + i - 34 * tc - 2;
                const uint32_t c = (q >= 0 && q < 32) ? (uint32_t)qc[32 * tc + min(max(q, 0), 31)] : 0u;
                w |= (uint64_t)c << (8 * i);
            }
            qb[m] = (int64_t)w;
        }
    }
    const float dqc = sm_dq[g * GQA + hc][tc];

    // Column (hc, tc): running max m and sum l of query head hc (the quad's
    // 4 lanes hold the same values), o[w] = the P.V outputs of window w,
    // rows 4 kg + i.
    float m = -INFINITY, l = 0.0f;
    float4v_t o[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) o[w] = float4v_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto stage = [&](const uint8_t *raw, const int b) __attribute__((always_inline)) {
        const uint8_t *rk = raw;
        const uint8_t *rv = raw + KVO;
        // QK: C[slot r][column] over the segment's bytes
        int4v_t ci = {0, 0, 0, 0};
#pragma unroll
        for (int mm = 0; mm < 5; ++mm) {
            const uint2 ka = *reinterpret_cast<const uint2 *>(rk + r * RS + seg + 40 * kg + 8 * mm);
            ci = __builtin_amdgcn_mfma_i32_16x16x32_i8((int64_t)(((uint64_t)ka.y << 32) | ka.x),
                                                       qb[mm], ci, 0, 0, 0);
        }
        // V^T windows: lane 2k + h of a 16-lane group reads bytes
        // [16 (w + (k >> 2)) + 8h, +8) of slot 4 kg + (k & 3): output lane j
        // then holds bytes 16w + j and 16(w + 1) + j of slots 4kg .. 4kg + 3
        int2v_t vt8[5];
        {
            const int k = r >> 1, h = r & 1;
            const uint8_t *src = rv + (4 * kg + (k & 3)) * RS + seg + 16 * (k >> 2) + 8 * h;
#pragma unroll
            for (int w2 = 0; w2 < 5; ++w2)
                vt8[w2] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                    (__attribute__((address_space(3))) int2v_t *)(src + 32 * w2));
        }
        // block tc's scales of slots 4 kg + i
        float dk[4], dv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int off = (4 * kg + i) * RS + seg + 34 * tc;
            dk[i] = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(rk + off));
            dv[i] = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(rv + off));
        }
        float sc[4];
        float bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // no contraction: a product fused into the first quad add would
            // round differently in the quad's lanes, and they must agree bit
            // for bit (each carries the head's running max for its column)
#pragma clang fp contract(off)
            float x = (float)ci[i] * (dk[i] * dqc);
            x += dpp<0xB1>(x);
            x += dpp<0x4E>(x);
            const bool ok = b + 4 * kg + i < i_end;
            sc[i] = ok ? x * a.scale_log2 : -INFINITY;
            bm = fmaxf(bm, sc[i]);
        }
        bm = xor32_max(xor16_max(bm));
        // lazy rescale: the reference max moves only when a head's batch max
        // exceeds it by more than 2^8 (p <= 256)
        if (__any(bm > m + 8.0f)) {
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.0f : fast_exp2(m - mn);
            l *= alpha;
            m = mn;
#pragma unroll
            for (int w = 0; w < NW; ++w) o[w] *= alpha;
        }
        half4v_t pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = sc[i] == -INFINITY ? 0.0f : fast_exp2(sc[i] - m);
            l += p;
            pb[i] = (_Float16)(p * dv[i]);
        }
#pragma unroll
        for (int w2 = 0; w2 < 5; ++w2) {
            o[2 * w2] = __builtin_amdgcn_mfma_f32_16x16x16f16(i8x4_to_h4((uint32_t)vt8[w2].x), pb,
                                                               o[2 * w2], 0, 0, 0);
            if (2 * w2 + 1 < NW)
                o[2 * w2 + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    i8x4_to_h4((uint32_t)vt8[w2].y), pb, o[2 * w2 + 1], 0, 0, 0);
        }
    };
    // One barrier per stage: stage n's raw rows go to buffer n & 1, which
    // every wave last read (stage n - 2) before it reached stage n - 1's
    // barrier.
    for (int b0 = i_begin, n = 0; b0 < i_end; b0 += NR * SL, n += NR) {
#pragma unroll
        for (int p = 0; p < NR; ++p) {
            const int b = b0 + p * SL;
            uint8_t *raw = sm_raw[(n + p) & 1];
            store_stage(stg[p], raw);                // waits for this stage's loads only
            load_stage(b + NR * SL, stg[p]);
            lds_barrier();                           // raw rows complete
            if (b < i_end) stage(raw, b);
        }
    }

    // l over the 4 lane groups (slots); the quad's lanes are copies
    l = xor32_sum(xor16_sum(l));
    const int64_t head = ((int64_t)s * a.n_layers + layer) * a.n_q_heads + g * GQA + hc;
    const bool direct = a.n_chunks == 1;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float *op = direct ? a.out + head * D : a.part_o + (head * a.n_chunks + chunk) * D;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = 16 * w + 4 * kg + i - 34 * tc - 2;   // quant of block tc
            if (q >= 0 && q < 32) op[32 * tc + q] = direct ? o[w][i] * inv : o[w][i];
        }
    if (!direct && kg == 0 && tc == 0) {
        const int64_t pidx = head * a.n_chunks + chunk;
        a.part_ml[pidx * 2] = m;
        a.part_ml[pidx * 2 + 1] = l;
    }
}

// One work group of head_dim (128) threads per (stream, layer, query head):
// the chunk maxima, weights exp2(m_c - M) and the weighted sum of l_c are
// reduced once for the group; each thread then accumulates its dimension over
// the chunks with the partial loads batched (they do not depend on each
// other), 128 chunk weights at a time through LDS.
constexpr int kCombineRegs = 32;   // chunks merged from registers in one round trip

__global__ void __launch_bounds__(128) k_combine(CombineArgs a) {
    __shared__ float sw[128];
    __shared__ float red[2][2];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int64_t head = ((int64_t)blockIdx.z * a.n_layers + blockIdx.y) * a.n_q_heads + blockIdx.x;
    const int64_t p0 = head * a.n_chunks;
    const float *ml = a.part_ml + p0 * 2;
    const float *po = a.part_o + p0 * a.head_dim + t;
    const int n = a.n_chunks;
    if (n <= kCombineRegs) {
        // One round trip: the chunk maxima and sums are requested first,
        // then every partial of this thread's dimension, all unconditionally
        // (indices clamp to the last chunk; a load merged with a value of
        // another path is waited for at once), so the two reductions run
        // while the partials are in flight.
        const float mc0 = ml[2 * min(t, n - 1)], lc0 = ml[2 * min(t, n - 1) + 1];
        float v[kCombineRegs];
#pragma unroll
        for (int c = 0; c < kCombineRegs; ++c) v[c] = po[(int64_t)min(c, n - 1) * a.head_dim];
        const float mc = t < n ? mc0 : -INFINITY;
        const float lc = t < n ? lc0 : 0.0f;
        const float m = wave_max64(mc);
        if (lane == 0) red[0][wave] = m;
        __syncthreads();
        const float M = fmaxf(red[0][0], red[0][1]);
        if (M == -INFINITY) {
            a.out[head * a.head_dim + t] = 0.0f;
            return;
        }
        const float w = t < n ? fast_exp2(mc - M) : 0.0f;
        const float l = wave_sum64(lc * w);
        sw[t] = w;
        if (lane == 0) red[1][wave] = l;
        __syncthreads();
        // all kCombineRegs slots, unconditionally, so no partial load is held
        // back behind a condition on n: past the last chunk the weight is 0
        // (sw[t] = 0 for t >= n) on a clamped, finite partial
        float O = 0.0f;
#pragma unroll
        for (int c = 0; c < kCombineRegs; ++c) O = fmaf(v[c], sw[c], O);
        const float L = red[1][0] + red[1][1];
        a.out[head * a.head_dim + t] = L > 0.0f ? O / L : 0.0f;
        return;
    }
    float m = -INFINITY;
    for (int c = t; c < n; c += 128) m = fmaxf(m, ml[2 * c]);
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[0][wave] = m;
    __syncthreads();
    const float M = fmaxf(red[0][0], red[0][1]);
    if (M == -INFINITY) {
        a.out[head * a.head_dim + t] = 0.0f;
        return;
    }
    float O = 0.0f, l = 0.0f;
    for (int c0 = 0; c0 < n; c0 += 128) {
        const int c = c0 + t;
        float w = 0.0f;
        if (c < n) {
            w = fast_exp2(ml[2 * c] - M);
            l = fmaf(ml[2 * c + 1], w, l);
        }
        sw[t] = w;
        __syncthreads();
        const int cn = min(128, n - c0);
        int j = 0;
        for (; j + 8 <= cn; j += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = po[(int64_t)(c0 + j + u) * a.head_dim];
#pragma unroll
            for (int u = 0; u < 8; ++u) O = fmaf(v[u], sw[j + u], O);
        }
        for (; j < cn; ++j) O = fmaf(po[(int64_t)(c0 + j) * a.head_dim], sw[j], O);
        __syncthreads();
    }
    for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    if (lane == 0) red[1][wave] = l;
    __syncthreads();
    const float L = red[1][0] + red[1][1];
    a.out[head * a.head_dim + t] = L > 0.0f ? O / L : 0.0f;
}

// ---------------------------------------------------------------------------
// Window attention (one wave per (query, head, layer)): two passes over the
// allowed keys -- max, then exp-weights through LDS and a lane-per-dimension
// P.V accumulation.
// ---------------------------------------------------------------------------
template <class F>
__global__ void __launch_bounds__(64) k_window(WindowArgs a) {
    const int lane = threadIdx.x;
    const int qi = blockIdx.x / a.n_q_heads;
    const int h = blockIdx.x % a.n_q_heads;
    const int layer = blockIdx.y;
    const int g = h / (a.n_q_heads / a.n_kv_heads);
    const int D = a.head_dim;
    const int n_keys = a.seg.n0 + a.seg.n1;
    const int64_t q_abs = a.q_pos0 + qi;
    const uint8_t *kl = a.k + (int64_t)layer * a.layer_bytes;
    const uint8_t *vl = a.v + (int64_t)layer * a.layer_bytes;
    __shared__ float sq[256];
    __shared__ float sp[64];
    const float *qp = a.q + (int64_t)layer * a.q_lstride + ((int64_t)qi * a.n_q_heads + h) * D;
    for (int d = lane; d < D; d += 64) sq[d] = qp[d];
    __syncthreads();

    // allowed keys form one contiguous logical range [j_lo, j_hi)
    const int64_t lo = a.window > 0 ? q_abs - (a.window - 1) : -((int64_t)1 << 62);
    const int64_t j_lo64 = lo - a.key_pos0;
    const int64_t j_hi64 = q_abs - a.key_pos0 + 1;
    const int j_lo = (int)max<int64_t>(0, j_lo64);
    const int j_hi = (int)min<int64_t>(n_keys, j_hi64);

    auto score = [&](int j) -> float {
        const uint8_t *row = kl + (int64_t)slot_of(a.seg, j) * a.row_bytes;
        float s = 0.0f;
        for (int e0 = 0; e0 < D; e0 += 8) {
            float kv[8];
            F::to_f32(F::load(row, g * D + e0), kv);
#pragma unroll
            for (int i = 0; i < 8; ++i) s = fmaf(kv[i], sq[e0 + i], s);
        }
        return s * a.scale_log2;
    };

    float M = -INFINITY;
    for (int j = j_lo + lane; j < j_hi; j += 64) M = fmaxf(M, score(j));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));

    float o0 = 0.0f, o1 = 0.0f, L = 0.0f;
    for (int jb = j_lo; jb < j_hi; jb += 64) {
        const int j = jb + lane;
        const float p = j < j_hi ? fast_exp2(score(j) - M) : 0.0f;
        __syncthreads();
        sp[lane] = p;
        __syncthreads();
        const int nb = min(64, j_hi - jb);
        for (int kk = 0; kk < nb; ++kk) {
            const float pk = sp[kk];
            L += pk;
            const uint8_t *row = vl + (int64_t)slot_of(a.seg, jb + kk) * a.row_bytes;
            // lane holds dims lane and lane+64 (D <= 128)
            float vv[8];
            const int d0 = lane;
            if (d0 < D) {
                F::to_f32(F::load(row, g * D + (d0 & ~7)), vv);
                o0 = fmaf(pk, vv[d0 & 7], o0);
            }
            const int d1 = lane + 64;
            if (d1 < D) {
                F::to_f32(F::load(row, g * D + (d1 & ~7)), vv);
                o1 = fmaf(pk, vv[d1 & 7], o1);
            }
        }
    }
    float *op = a.out + (int64_t)layer * a.q_lstride + ((int64_t)qi * a.n_q_heads + h) * D;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (lane < D) op[lane] = o0 * inv;
    if (lane + 64 < D) op[lane + 64] = o1 * inv;
}

// ---------------------------------------------------------------------------
// Window attention on the matrix cores (F16 cache): the encoder's 16-query
// block against its sliding window (src/voxtral.cpp:2201-2284) and the
// decoder's causal prefill (:2893-2961).  Work group = W waves on (layer,
// kv head g, tile of 16 query rows); a query row is (token, head of the GQA
// group).  The waves split the window's 16-key blocks round-robin.  W = 4,
// but 8 for the per-layer calls of the encoder chunk (head_dim 64, one
// layer's 32 heads: 32 work groups), where each wave then walks half as
// many blocks (measured on MI355X: 12.3 against 13.2 us per call; 16 waves
// took 14.2).
//
// Per key block, with v_mfma_f32_16x16x16f16:
//   S^T[key][row] = K[key][:] . Q[row][:]   A = K (keys as M, loaded straight
//                   from the ring), B = Q^T (registers); the head dimension is
//                   permuted so each lane reads one contiguous D/4 run of a key.
//   O^T[d][row]  += V^T[d][key] P^T[key][row]   A = V^T (through a padded LDS
//                   tile: the one transpose), B = P^T -- exactly S^T's output
//                   layout, so P never leaves registers and each lane's
//                   online-softmax rescale is its own row's.
// ---------------------------------------------------------------------------
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// HG > 1: one work group takes HG neighbouring kv heads (HG x W waves, wave
// (hh, w) = head g0 + hh, key blocks as wave w of the one-head tile), so the
// HG heads' segments of a row -- HG x 128 contiguous bytes at D = 64 -- are
// requested from one CU at about the same time.  Every output is computed
// exactly as by the one-head tile.
// SPL > 1: the keys are split over SPL work groups per (head, tile)
// (blockIdx.z): the absolute block grid has W x SPL virtual waves and work
// group s runs virtual waves [sW, sW + W); it writes its merged (O, M, L)
// as a partial, which k_window_merge combines in split order.  Only for
// GQA 1 (a partial per (query row, head, split)).
template <int D, int W, int HG = 1, int SPL = 1>
__global__ void __launch_bounds__(64 * W * HG) k_window_mfma(WindowArgs a) {
    constexpr int KB = D / 16;          // k-blocks of the QK product, d-tiles of PV
    constexpr int DL = D / 4;           // contiguous head dims per lane
    constexpr int VS = 2 * D + 8;       // padded LDS row stride of the V tile (bytes)
    constexpr int NWV = W * HG;         // waves per work group
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wk = wave % W;            // the wave's place among its head's W waves
    const int lg = lane >> 4;           // lane group 0..3
    const int lr = lane & 15;
    const int gqa = a.n_q_heads / a.n_kv_heads;
    const int n_groups = a.n_kv_heads / HG;
    const int g0 = (blockIdx.x % n_groups) * HG;
    const int g = g0 + wave / W;
    const int tile = a.tile0 + (int)(blockIdx.x / n_groups);
    const int split = SPL > 1 ? (int)blockIdx.z : 0;
    constexpr int VW = W * SPL;         // virtual waves of the absolute block grid
    const int layer = blockIdx.y;
    const int n_rows = a.n_q * gqa;
    const int n_keys = a.seg.n0 + a.seg.n1;
    const uint8_t *kl = a.k + (int64_t)layer * a.layer_bytes;
    const uint8_t *vl = a.v + (int64_t)layer * a.layer_bytes;

    __shared__ __align__(16) uint8_t sm_v[NWV][16 * VS];   // VS % 8 == 0
    __shared__ float sm_o[NWV][16][D + 1];
    __shared__ float sm_m[NWV][16], sm_l[NWV][16];

    // ---- Q^T operand: lane holds row lr, dims [DL*lg, DL*lg + DL) as f16 ----
    const int row = tile * 16 + lr;
    const bool row_ok = row < n_rows;
    const int tok = row_ok ? row / gqa : 0;
    const int64_t q_abs = a.q_pos0 + tok;
    // Q first (rows past the tile's last read a valid row, unused), then the
    // wave's first key block, then the fused ring write: every request is
    // unconditional and in the order it is waited for, so the three first
    // touches of the launch are in flight together (one after another they
    // were three round trips before the first product).
    float4 qraw[KB];
    {
        const float *qp = a.q + (int64_t)layer * a.q_lstride +
                          ((int64_t)tok * a.n_q_heads + g * gqa + (row_ok ? row % gqa : 0)) * D + DL * lg;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) qraw[kb] = reinterpret_cast<const float4 *>(qp)[kb];
    }
    half4_t qb[KB];   // Q as f16, formed after the ring write

    // ---- the key range any row of this tile may attend ----
    const int row0 = tile * 16;
    const int row1 = min(row0 + 16, n_rows) - 1;
    const int64_t qa_lo = a.q_pos0 + row0 / gqa;
    const int64_t qa_hi = a.q_pos0 + row1 / gqa;
    const int64_t lo = a.window > 0 ? qa_lo - (a.window - 1) : -((int64_t)1 << 62);
    const int j_lo = (int)max<int64_t>(0, lo - a.key_pos0);
    const int j_hi = (int)min<int64_t>(n_keys, qa_hi - a.key_pos0 + 1);
    const int64_t my_lo = a.window > 0 ? q_abs - (a.window - 1) : -((int64_t)1 << 62);

    float m = -INFINITY, l = 0.0f;
    float4_t o[KB];
#pragma unroll
    for (int t = 0; t < KB; ++t) o[t] = float4_t{0, 0, 0, 0};

    // Software pipeline over two register sets: the next key block's K/V
    // loads are in flight while the current one is reduced; indices clamp
    // into [j_lo, j_hi) (keys outside it are masked).
    auto load_kv = [&](int jb, uint4 (&kr)[DL / 8], uint4 (&vr)[DL / 8])
                       __attribute__((always_inline)) {
        // K and V of key jb+lr, dims [DL*lg, +DL): one contiguous run per lane
        const int jk = max(min(jb + lr, j_hi - 1), j_lo);
        // an empty key range reads slot 0 (unused)
        const uint32_t off = (uint32_t)(j_lo < j_hi ? slot_of(a.seg, jk) : 0) * (uint32_t)a.row_bytes +
                             (uint32_t)(g * D + DL * lg) * 2u;
#pragma unroll
        for (int t = 0; t < DL / 8; ++t) {
            kr[t] = reinterpret_cast<const uint4 *>(kl + off)[t];
            vr[t] = reinterpret_cast<const uint4 *>(vl + off)[t];
        }
    };
    auto process = [&](const uint4 (&kr)[DL / 8], const uint4 (&vr)[DL / 8], int jb)
                       __attribute__((always_inline)) {
        // V rows into this wave's LDS tile (row lr, bytes [2*DL*lg, +2*DL));
        // the padded stride keeps rows 8-byte aligned: 8-byte stores
#pragma unroll
        for (int t = 0; t < DL / 8; ++t) {
            uint2 *dst = reinterpret_cast<uint2 *>(&sm_v[wave][lr * VS + 2 * DL * lg + 16 * t]);
            dst[0] = make_uint2(vr[t].x, vr[t].y);
            dst[1] = make_uint2(vr[t].z, vr[t].w);
        }

        // S^T = K Q^T, even and odd 16-dim steps in two accumulators (a
        // shorter chain of dependent MFMAs; summed at the end)
        float4_t s2[2] = {float4_t{0, 0, 0, 0}, float4_t{0, 0, 0, 0}};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const uint32_t w0 = (&kr[0].x)[2 * kb], w1 = (&kr[0].x)[2 * kb + 1];
            const half4_t ka = __builtin_bit_cast(half4_t, (uint64_t)w0 | ((uint64_t)w1 << 32));
            s2[kb & 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qb[kb], s2[kb & 1], 0, 0, 0);
        }
        const float4_t st = s2[0] + s2[1];
        // lane holds keys jb + 4*lg + i (i = 0..3) for row lr
        float sc[4];
        float bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = jb + 4 * lg + i;
            const int64_t kabs = a.key_pos0 + j;
            const bool ok = row_ok && j >= j_lo && j < j_hi && kabs <= q_abs && kabs >= my_lo;
            sc[i] = ok ? st[i] * a.scale_log2 : -INFINITY;
            bm = fmaxf(bm, sc[i]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        // lazy rescale, per row: a row's running max moves only when its own
        // block max passes it by 2^8 (rows that do not move scale by 1)
        const bool grow = bm > m + 8.0f;
        if (__any(grow)) {
            const float alpha = grow && m != -INFINITY ? fast_exp2(m - bm) : 1.0f;
            l *= alpha;
#pragma unroll
            for (int t = 0; t < KB; ++t) o[t] *= alpha;
            m = grow ? bm : m;
        }
        half4_t pb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = sc[i] == -INFINITY ? 0.0f : fast_exp2(sc[i] - m);
            l += p;
            pb[i] = (_Float16)p;
        }
        // V^T operand: lane (lg, lr) needs V[key 4lg+i][d = 16t + lr], i =
        // 0..3.  ds_read_b64_tr_b16 gives output lane j of a 16-lane group
        // element k = element j%4 of source lane 4k + j/4, so source lane
        // (lg, 4i+q) reads V[key 4lg+i][16t + 4q, +4).
        __builtin_amdgcn_wave_barrier();
        {
            const uint8_t *vsrc = &sm_v[wave][(4 * lg + (lr >> 2)) * VS + 8 * (lr & 3)];
#pragma unroll
            for (int t = 0; t < KB; ++t) {
                typedef short short4_t __attribute__((ext_vector_type(4)));
                const half4_t va = __builtin_bit_cast(
                    half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                 (__attribute__((address_space(3))) short4_t *)(vsrc + 32 * t)));
                o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[t], 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();
        };
    uint4 ka_[DL / 8], va_[DL / 8], kb_[DL / 8], vb_[DL / 8];
    // The block grid is absolute: wave w takes the 16-key blocks starting at
    // key positions = 16 w (mod 16 W), whatever the run's first query, so a
    // row meets its keys in the same blocks, waves and order under every
    // chunking of the stream (schedule-invariant results, bit for bit).
    int jb0 = j_lo - (int)((a.key_pos0 + j_lo) & (16 * VW - 1)) + (split * W + wk) * 16;
    load_kv(jb0, ka_, va_);
    // Fused ring write (the encoder step's and the prefill's append): this
    // work group converts its kv heads' part of the n_new new rows (F16 RNE)
    // and stores them through the write segments; the barrier makes them
    // visible to its waves, which attend them like any other key.  Several
    // tiles of one head (GQA prefill) store identical bytes.  A wave whose
    // first block holds a new row (the newest n_new keys) requests it again
    // after the barrier.
    if (a.k_new) {
        const int kv_dim = a.n_kv_heads * D;
        const int64_t src0 = (int64_t)layer * a.n_new * kv_dim;
        uint8_t *kw = a.k_w + (int64_t)layer * a.layer_bytes;
        uint8_t *vw = a.v_w + (int64_t)layer * a.layer_bytes;
        for (int t = threadIdx.x; t < a.n_new * HG * (D / 8); t += 64 * NWV) {
            const int row = t / (HG * D / 8);
            // split tiles: each new row is written by the work group whose
            // key blocks hold it, the only one that reads it
            if (SPL > 1 &&
                (int)(((a.key_pos0 + n_keys - a.n_new + row) >> 4) % VW) / W != split)
                continue;
            const int col = g0 * D + (t % (HG * D / 8)) * 8;
            const int64_t so = src0 + (int64_t)row * kv_dim + col;
            const int64_t dst = (int64_t)slot_of(a.wseg, row) * a.row_bytes;
            float xk[8], xv[8];
            const float4 k0 = reinterpret_cast<const float4 *>(a.k_new + so)[0];
            const float4 k1 = reinterpret_cast<const float4 *>(a.k_new + so)[1];
            const float4 v0 = reinterpret_cast<const float4 *>(a.v_new + so)[0];
            const float4 v1 = reinterpret_cast<const float4 *>(a.v_new + so)[1];
            xk[0] = k0.x; xk[1] = k0.y; xk[2] = k0.z; xk[3] = k0.w;
            xk[4] = k1.x; xk[5] = k1.y; xk[6] = k1.z; xk[7] = k1.w;
            xv[0] = v0.x; xv[1] = v0.y; xv[2] = v0.z; xv[3] = v0.w;
            xv[4] = v1.x; xv[5] = v1.y; xv[6] = v1.z; xv[7] = v1.w;
            FmtF16::store(kw + dst, col, FmtF16::from_f32(xk));
            FmtF16::store(vw + dst, col, FmtF16::from_f32(xv));
        }
        __syncthreads();
    }

    // (its largest index read: clamped into [j_lo, j_hi))
    if (a.k_new && max(j_lo, min(jb0 + 15, j_hi - 1)) >= n_keys - a.n_new) load_kv(jb0, ka_, va_);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const float4 v4 = row_ok ? qraw[kb] : make_float4(0, 0, 0, 0);
        qb[kb] = half4_t{(_Float16)v4.x, (_Float16)v4.y, (_Float16)v4.z, (_Float16)v4.w};
    }
    // Two blocks per trip while both are in range, the odd last block after
    // the loop: with an exit between the halves the compiled loop drained
    // every load at the top of each trip (batched F16 chunk 36.9 -> 36.3 us).
    for (; jb0 + 16 * VW < j_hi; jb0 += 32 * VW) {
        load_kv(jb0 + 16 * VW, kb_, vb_);
        process(ka_, va_, jb0);
        load_kv(jb0 + 32 * VW, ka_, va_);
        process(kb_, vb_, jb0 + 16 * VW);
    }
    if (jb0 < j_hi) process(ka_, va_, jb0);

    // row sums over the 4 lane groups (they share m)
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    // O^T tile t: lane holds d = 16*t + 4*lg + i of row lr
#pragma unroll
    for (int t = 0; t < KB; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[wave][lr][16 * t + 4 * lg + i] = o[t][i];
    if (lg == 0) {
        sm_m[wave][lr] = m;
        sm_l[wave][lr] = l;
    }
    __syncthreads();
    // head g0 + hh's W waves merge in a fixed order
    for (int t = threadIdx.x; t < HG * 16 * D; t += 64 * NWV) {
        const int hh = t / (16 * D);
        const int r = (t / D) % 16;
        const int d = t % D;
        const int rr = tile * 16 + r;
        if (rr >= n_rows) continue;
        const int w0 = hh * W;
        float M = fmaxf(fmaxf(sm_m[w0][r], sm_m[w0 + 1][r]), fmaxf(sm_m[w0 + 2][r], sm_m[w0 + 3][r]));
#pragma unroll
        for (int w = 4; w < W; ++w) M = fmaxf(M, sm_m[w0 + w][r]);
        float O = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float f = fast_exp2(sm_m[w0 + w][r] - M);
                O = fmaf(sm_o[w0 + w][r][d], f, O);
                L = fmaf(sm_l[w0 + w][r], f, L);
            }
        }
        if constexpr (SPL > 1) {
            const int64_t pv =
                ((int64_t)(rr - 16 * a.tile0) * a.n_q_heads + g0 + hh) * SPL + split;
            a.part_o[pv * D + d] = O;
            if (d == 0) {
                a.part_ml[pv * 2] = M;
                a.part_ml[pv * 2 + 1] = L;
            }
        } else {
            const int tk = rr / gqa;
            float *op = a.out + (int64_t)layer * a.q_lstride +
                        ((int64_t)tk * a.n_q_heads + (g0 + hh) * gqa + rr % gqa) * D + d;
            *op = L > 0.0f ? O / L : 0.0f;
        }
    }
}

// The split tile's partials of n_vec (query row, head) vectors, merged in
// split order: one thread per output element.
template <int SPL>
__global__ void __launch_bounds__(256) k_window_merge(const float *part_o, const float *part_ml,
                                                      float *out, int64_t n_vec, int D) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_vec * D) return;
    const int64_t v = i / D;
    const int d = (int)(i - v * D);
    float m[SPL], l[SPL], o[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
        m[s] = part_ml[(v * SPL + s) * 2];
        l[s] = part_ml[(v * SPL + s) * 2 + 1];
        o[s] = part_o[(v * SPL + s) * D + d];
    }
    float M = m[0];
#pragma unroll
    for (int s = 1; s < SPL; ++s) M = fmaxf(M, m[s]);
    float O = 0.0f, L = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const float f = fast_exp2(m[s] - M);
            O = fmaf(o[s], f, O);
            L = fmaf(l[s], f, L);
        }
    }
    out[i] = L > 0.0f ? O / L : 0.0f;
}

// ---------------------------------------------------------------------------
// Window attention on the matrix cores over an F32 cache (the reference's
// default encoder ring, src/voxtral.cpp:100-105, :3955-3984), in f32
// throughout with v_mfma_f32_16x16x4_f32.  Same decomposition as
// k_window_mfma: work group = 4 waves on (layer, kv head g, 16 query rows),
// the waves split the window's 16-key blocks.  Per key block:
//   S^T[key][row] = K . Q^T   A lane (lg, r) = K[key r][DL lg + s] (16..32
//                   contiguous dims per lane, one float per MFMA step s),
//                   B lane (lg, c) = Q[row c][DL lg + s] (registers);
//   O^T[d][row]  += V^T[d][key] P^T[key][row] with step s contracting keys
//                   4 lg + s, so B = the lane's own softmax weight of key
//                   4 lg + s, and A = V^T from a padded LDS tile (V rows
//                   written transposed, stride 17 floats).
// The fused ring write copies the new rows (F32 cache: no conversion).
// ---------------------------------------------------------------------------
// SPL > 1: keys split over SPL work groups per (head, tile), as in
// k_window_mfma (partials merged by k_window_merge; GQA 1 only).
template <int D, int W, int SPL = 1>
__device__ __forceinline__ void window_mfma_f32(const WindowArgs &a) {
    constexpr int DL = D / 4;           // contiguous head dims per lane
    constexpr int NT = D / 16;          // 16-dim tiles of P.V
    constexpr int VS = 17;              // LDS stride of the V^T tile (floats)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lg = lane >> 4;
    const int lr = lane & 15;
    const int gqa = a.n_q_heads / a.n_kv_heads;
    const int g = blockIdx.x % a.n_kv_heads;
    const int tile = a.tile0 + (int)(blockIdx.x / a.n_kv_heads);
    const int split = SPL > 1 ? (int)blockIdx.z : 0;
    constexpr int VW = W * SPL;         // virtual waves of the absolute block grid
    const int layer = blockIdx.y;
    const int n_rows = a.n_q * gqa;
    const int n_keys = a.seg.n0 + a.seg.n1;
    const uint8_t *kl = a.k + (int64_t)layer * a.layer_bytes;
    const uint8_t *vl = a.v + (int64_t)layer * a.layer_bytes;

    __shared__ float sm_vt[W][D * VS];   // per wave: V^T[d][key]
    __shared__ float sm_o[W][16][D + 1];
    __shared__ float sm_m[W][16], sm_l[W][16];

    // ---- Q^T operand: lane holds row lr, dims [DL lg, DL lg + DL) ----
    const int row = tile * 16 + lr;
    const bool row_ok = row < n_rows;
    const int tok = row_ok ? row / gqa : 0;
    const int64_t q_abs = a.q_pos0 + tok;
    // Q first (rows past the tile's last read a valid row, unused), then the
    // wave's first key block, then the fused ring write: every request is
    // unconditional and in the order it is waited for, so the three first
    // touches of the launch are in flight together.
    float4 qraw[DL / 4];
    {
        const float *qp = a.q + (int64_t)layer * a.q_lstride +
                          ((int64_t)tok * a.n_q_heads + g * gqa + (row_ok ? row % gqa : 0)) * D + DL * lg;
#pragma unroll
        for (int t = 0; t < DL / 4; ++t) qraw[t] = reinterpret_cast<const float4 *>(qp)[t];
    }
    float qf[DL];   // formed after the ring write

    // ---- the key range any row of this tile may attend ----
    const int row0 = tile * 16;
    const int row1 = min(row0 + 16, n_rows) - 1;
    const int64_t qa_lo = a.q_pos0 + row0 / gqa;
    const int64_t qa_hi = a.q_pos0 + row1 / gqa;
    const int64_t lo = a.window > 0 ? qa_lo - (a.window - 1) : -((int64_t)1 << 62);
    const int j_lo = (int)max<int64_t>(0, lo - a.key_pos0);
    const int j_hi = (int)min<int64_t>(n_keys, qa_hi - a.key_pos0 + 1);
    const int64_t my_lo = a.window > 0 ? q_abs - (a.window - 1) : -((int64_t)1 << 62);

    float m = -INFINITY, l = 0.0f;
    float4_t o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = float4_t{0, 0, 0, 0};
    float *vt = sm_vt[wave];

    // K and V of key jb + lr, dims [DL lg, +DL): one contiguous run per lane;
    // indices clamp into [j_lo, j_hi) (keys outside it are masked)
    auto load_kv = [&](int jb, float4 (&kr)[DL / 4], float4 (&vr)[DL / 4]) __attribute__((always_inline)) {
        const int jk = max(min(jb + lr, j_hi - 1), j_lo);
        // an empty key range reads slot 0 (unused)
        const uint32_t off = (uint32_t)(j_lo < j_hi ? slot_of(a.seg, jk) : 0) * (uint32_t)a.row_bytes +
                             (uint32_t)(g * D + DL * lg) * 4u;
#pragma unroll
        for (int t = 0; t < DL / 4; ++t) {
            kr[t] = reinterpret_cast<const float4 *>(kl + off)[t];
            vr[t] = reinterpret_cast<const float4 *>(vl + off)[t];
        }
    };
    auto process = [&](const float4 (&kr)[DL / 4], const float4 (&vr)[DL / 4], int jb) __attribute__((always_inline)) {
        // V^T tile: this lane's key lr, dims DL lg + x
#pragma unroll
        for (int t = 0; t < DL / 4; ++t) {
            vt[(DL * lg + 4 * t + 0) * VS + lr] = vr[t].x;
            vt[(DL * lg + 4 * t + 1) * VS + lr] = vr[t].y;
            vt[(DL * lg + 4 * t + 2) * VS + lr] = vr[t].z;
            vt[(DL * lg + 4 * t + 3) * VS + lr] = vr[t].w;
        }
        // S^T = K Q^T, one MFMA per dim step, into four independent
        // accumulators (dims = 0, 1, 2, 3 mod 4) summed at the end: one
        // chain of DL dependent MFMAs per block cost 5% of the launch
        float4_t sa[4] = {float4_t{0, 0, 0, 0}, float4_t{0, 0, 0, 0}, float4_t{0, 0, 0, 0},
                          float4_t{0, 0, 0, 0}};
#pragma unroll
        for (int t = 0; t < DL / 4; ++t) {
            sa[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[t].x, qf[4 * t], sa[0], 0, 0, 0);
            sa[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[t].y, qf[4 * t + 1], sa[1], 0, 0, 0);
            sa[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[t].z, qf[4 * t + 2], sa[2], 0, 0, 0);
            sa[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[t].w, qf[4 * t + 3], sa[3], 0, 0, 0);
        }
        const float4_t st = (sa[0] + sa[1]) + (sa[2] + sa[3]);
        // lane holds keys jb + 4 lg + i (i = 0..3) for row lr
        float sc[4];
        float bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = jb + 4 * lg + i;
            const int64_t kabs = a.key_pos0 + j;
            const bool ok = row_ok && j >= j_lo && j < j_hi && kabs <= q_abs && kabs >= my_lo;
            sc[i] = ok ? st[i] * a.scale_log2 : -INFINITY;
            bm = fmaxf(bm, sc[i]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        // lazy rescale, per row: a row's running max moves only when its own
        // block max passes it by 2^8 (rows that do not move scale by 1)
        const bool grow = bm > m + 8.0f;
        if (__any(grow)) {
            const float alpha = grow && m != -INFINITY ? fast_exp2(m - bm) : 1.0f;
            l *= alpha;
#pragma unroll
            for (int t = 0; t < NT; ++t) o[t] *= alpha;
            m = grow ? bm : m;
        }
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = sc[i] == -INFINITY ? 0.0f : fast_exp2(sc[i] - m);
            l += p[i];
        }
        __builtin_amdgcn_wave_barrier();
        // O^T tile T += V^T[16 T + lr][key 4 lg + s] p_s
#pragma unroll
        for (int T = 0; T < NT; ++T)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                o[T] = __builtin_amdgcn_mfma_f32_16x16x4f32(vt[(16 * T + lr) * VS + 4 * lg + s], p[s],
                                                             o[T], 0, 0, 0);
        __builtin_amdgcn_wave_barrier();
    };
    float4 ka_[DL / 4], va_[DL / 4], kb_[DL / 4], vb_[DL / 4];
    // The block grid is absolute: wave w takes the 16-key blocks starting at
    // key positions = 16 w (mod 16 W), whatever the run's first query, so a
    // row meets its keys in the same blocks, waves and order under every
    // chunking of the stream (schedule-invariant results, bit for bit).
    int jb0 = j_lo - (int)((a.key_pos0 + j_lo) & (16 * VW - 1)) + (split * W + wave) * 16;
    load_kv(jb0, ka_, va_);
    // Fused ring write of kv head g's part of the n_new new rows.  A wave
    // whose first block holds a new row (the newest n_new keys; its largest
    // index read, clamped into [j_lo, j_hi)) requests it again after it.
    if (a.k_new) {
        const int kv_dim = a.n_kv_heads * D;
        const int64_t src0 = (int64_t)layer * a.n_new * kv_dim;
        uint8_t *kw = a.k_w + (int64_t)layer * a.layer_bytes;
        uint8_t *vw = a.v_w + (int64_t)layer * a.layer_bytes;
        for (int t = threadIdx.x; t < a.n_new * (D / 4); t += 64 * W) {
            const int row = t / (D / 4);
            // split tiles: each new row is written by the work group whose
            // key blocks hold it, the only one that reads it
            if (SPL > 1 &&
                (int)(((a.key_pos0 + n_keys - a.n_new + row) >> 4) % VW) / W != split)
                continue;
            const int col = g * D + (t % (D / 4)) * 4;
            const int64_t so = src0 + (int64_t)row * kv_dim + col;
            const int64_t dst = (int64_t)slot_of(a.wseg, row) * a.row_bytes + (int64_t)col * 4;
            *reinterpret_cast<float4 *>(kw + dst) = *reinterpret_cast<const float4 *>(a.k_new + so);
            *reinterpret_cast<float4 *>(vw + dst) = *reinterpret_cast<const float4 *>(a.v_new + so);
        }
        __syncthreads();
    }

    if (a.k_new && max(j_lo, min(jb0 + 15, j_hi - 1)) >= n_keys - a.n_new) load_kv(jb0, ka_, va_);
#pragma unroll
    for (int t = 0; t < DL / 4; ++t) {
        const float4 v4 = row_ok ? qraw[t] : make_float4(0, 0, 0, 0);
        qf[4 * t] = v4.x; qf[4 * t + 1] = v4.y; qf[4 * t + 2] = v4.z; qf[4 * t + 3] = v4.w;
    }
    // (the F32 tile keeps the exit between the halves: the straight-line
    // form ran 94.9 against 92.4 us per 32-layer chunk)
    for (; jb0 < j_hi; jb0 += 32 * VW) {
        load_kv(jb0 + 16 * VW, kb_, vb_);
        process(ka_, va_, jb0);
        if (jb0 + 16 * VW >= j_hi) break;
        load_kv(jb0 + 32 * VW, ka_, va_);
        process(kb_, vb_, jb0 + 16 * VW);
    }

    // row sums over the 4 lane groups (they share m)
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    // O^T tile T: lane holds d = 16 T + 4 lg + i of row lr
#pragma unroll
    for (int T = 0; T < NT; ++T)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[wave][lr][16 * T + 4 * lg + i] = o[T][i];
    if (lg == 0) {
        sm_m[wave][lr] = m;
        sm_l[wave][lr] = l;
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * D; t += 64 * W) {
        const int r = t / D;
        const int d = t % D;
        const int rr = tile * 16 + r;
        if (rr >= n_rows) continue;
        float M = fmaxf(fmaxf(sm_m[0][r], sm_m[1][r]), fmaxf(sm_m[2][r], sm_m[3][r]));
#pragma unroll
        for (int w = 4; w < W; ++w) M = fmaxf(M, sm_m[w][r]);
        float O = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float f = fast_exp2(sm_m[w][r] - M);
                O = fmaf(sm_o[w][r][d], f, O);
                L = fmaf(sm_l[w][r], f, L);
            }
        }
        if constexpr (SPL > 1) {
            const int64_t pv = ((int64_t)(rr - 16 * a.tile0) * a.n_q_heads + g) * SPL + split;
            a.part_o[pv * D + d] = O;
            if (d == 0) {
                a.part_ml[pv * 2] = M;
                a.part_ml[pv * 2 + 1] = L;
            }
        } else {
            const int tk = rr / gqa;
            float *op = a.out + (int64_t)layer * a.q_lstride +
                        ((int64_t)tk * a.n_q_heads + g * gqa + rr % gqa) * D + d;
            *op = L > 0.0f ? O / L : 0.0f;
        }
    }
}

// head_dim 64 (the encoder): at most 128 VGPRs, so four 4-wave work groups
// share a CU and the 32 heads x 32 layers of a chunk fit in one round of the
// 256 CUs (at 139 VGPRs, three per CU, a third of them ran in a second round)
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
k_window_mfma_f32_64(WindowArgs a) {
    window_mfma_f32<64, 4>(a);
}
__global__ void __launch_bounds__(256) k_window_mfma_f32_128(WindowArgs a) {
    window_mfma_f32<128, 4>(a);
}
// the per-layer encoder call, split over kWinSplit work groups per head
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4)))
k_window_mfma_f32_64_split(WindowArgs a) {
    window_mfma_f32<64, 4, kWinSplit>(a);
}

// ---------------------------------------------------------------------------
// q8_0 pack / unpack of flat f32 arrays (n % 32 == 0); 8 elements per lane.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_q8_pack(const float *x, uint8_t *blocks, int64_t n) {
    const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    const bool ok = e0 < n;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ok ? x[e0 + i] : 0.0f;
    store_new<FmtQ8>(blocks + (e0 >> 5) * 34, (int)(e0 & 31), v, ok);
}

__global__ void __launch_bounds__(256) k_q8_unpack(const uint8_t *blocks, float *y, int64_t n) {
    const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (e0 >= n) return;
    const FmtQ8::Frag f = FmtQ8::load(blocks + (e0 >> 5) * 34, (int)(e0 & 31));
    float o[8];
    FmtQ8::to_f32(f, o);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[e0 + i] = o[i];
}

__global__ void __launch_bounds__(256) k_fill_zero(uint8_t *dst, int64_t bytes) {
    const int64_t n16 = bytes / 16;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n16; t += (int64_t)gridDim.x * 256)
        reinterpret_cast<uint4 *>(dst)[t] = make_uint4(0u, 0u, 0u, 0u);
    const int64_t tail = bytes - n16 * 16;
    if (blockIdx.x == 0 && threadIdx.x < tail) dst[n16 * 16 + threadIdx.x] = 0;
}

// ---------------------------------------------------------------------------
// Seeded synthetic N(0,1): splitmix64 output function, twelve 16-bit uniforms
// summed (integer Irwin-Hall), exact in f32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

struct SynthArgs {
    float *dst;
    uint64_t seed;
    uint32_t tag;
    int32_t row_len, ns, nl, np;
    int64_t s0, l0, p0, s_stride, l_stride, p_stride;
};

__global__ void __launch_bounds__(256) k_synth(SynthArgs a) {
    const int64_t rows = (int64_t)a.ns * a.nl * a.np;
    const int64_t total = rows * a.row_len;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * 256) {
        const int64_t r = t / a.row_len;
        const int64_t i = t % a.row_len;
        const int64_t kp = r % a.np;
        const int64_t jl = (r / a.np) % a.nl;
        const int64_t is = r / ((int64_t)a.np * a.nl);
        uint64_t key = mix64(a.seed ^ ((uint64_t)a.tag << 32));
        key = mix64(key ^ (uint64_t)(a.s0 + is));
        key = mix64(key ^ (uint64_t)(a.l0 + jl));
        key = mix64(key ^ (uint64_t)(a.p0 + kp));
        const uint64_t b = key ^ ((uint64_t)i * 0xD1B54A32D192ED03ull);
        int32_t sum = 0;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const uint64_t hsh = mix64(b + (uint64_t)k * 0x9E3779B97F4A7C15ull);
            sum += (int32_t)(hsh & 0xffffu) + (int32_t)((hsh >> 16) & 0xffffu) +
                   (int32_t)((hsh >> 32) & 0xffffu) + (int32_t)(hsh >> 48);
        }
        const int64_t drow = is * a.s_stride + jl * a.l_stride + kp * a.p_stride;
        a.dst[drow * a.row_len + i] = (float)(sum - 393210) * (1.0f / 65536.0f);
    }
}

inline unsigned grid_for(int64_t work, int64_t per_block, int64_t cap = 1 << 20) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
hipError_t launch_append(int dtype, const AppendArgs &a, int n_layers, hipStream_t st) {
    const int64_t threads = ((int64_t)a.n_rows * a.kv_dim + 7) / 8;
    dim3 grid(grid_for(threads, 256, INT32_MAX), (unsigned)n_layers, 2);
    switch (dtype) {
    case VKV_DTYPE_F16: hipLaunchKernelGGL(k_append<FmtF16>, grid, dim3(256), 0, st, a); break;
    case VKV_DTYPE_F32: hipLaunchKernelGGL(k_append<FmtF32>, grid, dim3(256), 0, st, a); break;
    case VKV_DTYPE_Q8_0: hipLaunchKernelGGL(k_append<FmtQ8>, grid, dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gather(const uint8_t *src, int64_t row_bytes, SegPair seg, uint8_t *dst,
                         hipStream_t st) {
    const int64_t rows = seg.n0 + seg.n1;
    if (rows == 0) return hipSuccess;
    if (row_bytes % 16 == 0 && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0) {
        hipLaunchKernelGGL(k_gather<uint4>, dim3(grid_for(rows * row_bytes / 16, 256, 65536)),
                           dim3(256), 0, st, src, row_bytes, seg, dst);
    } else {
        hipLaunchKernelGGL(k_gather<uint16_t>, dim3(grid_for(rows * row_bytes / 2, 256, 65536)),
                           dim3(256), 0, st, src, row_bytes, seg, dst);
    }
    return hipGetLastError();
}

template <class F, int GQA, int W, int NS>
static void launch_decode_w(bool fuse, dim3 grid, const DecodeArgs &a, hipStream_t st) {
    if (fuse) hipLaunchKernelGGL((k_decode<F, GQA, true, W, NS>), grid, dim3(W * 64), 0, st, a);
    else hipLaunchKernelGGL((k_decode<F, GQA, false, W, NS>), grid, dim3(W * 64), 0, st, a);
}

template <class F, int GQA>
static bool launch_decode_fmt(int waves, int stages, bool fuse, dim3 grid, const DecodeArgs &a,
                              hipStream_t st) {
    switch (waves * 16 + stages) {
    case 4 * 16 + 2: launch_decode_w<F, GQA, 4, 2>(fuse, grid, a, st); return true;
    case 4 * 16 + 3: launch_decode_w<F, GQA, 4, 3>(fuse, grid, a, st); return true;
    case 4 * 16 + 4: launch_decode_w<F, GQA, 4, 4>(fuse, grid, a, st); return true;
    case 8 * 16 + 2: launch_decode_w<F, GQA, 8, 2>(fuse, grid, a, st); return true;
    case 8 * 16 + 3: launch_decode_w<F, GQA, 8, 3>(fuse, grid, a, st); return true;
    default: return false;
    }
}

hipError_t launch_decode(int dtype, int gqa, int waves, int stages, bool mfma, bool fuse_append,
                         int n_streams, const DecodeArgs &a, hipStream_t st) {
    dim3 grid((unsigned)(a.n_chunks * a.n_kv_heads), (unsigned)a.n_layers, (unsigned)n_streams);
    if (gqa != 4) return hipErrorInvalidValue;
    if (mfma && dtype == VKV_DTYPE_Q8_0 && waves == 4) {
        // one 16-slot sub-batch per step (two measured 1.5% slower)
        if (stages >= 3) {
            if (fuse_append) hipLaunchKernelGGL((k_decode_q8mfma<true, 3, 1>), grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_decode_q8mfma<false, 3, 1>), grid, dim3(256), 0, st, a);
        } else {
            if (fuse_append) hipLaunchKernelGGL((k_decode_q8mfma<true, 2, 1>), grid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_decode_q8mfma<false, 2, 1>), grid, dim3(256), 0, st, a);
        }
        return hipGetLastError();
    }
    bool ok = false;
    switch (dtype) {
    case VKV_DTYPE_F16:
        ok = launch_decode_fmt<FmtF16, 4>(waves, stages, fuse_append, grid, a, st);
        break;
    case VKV_DTYPE_F32:
        ok = launch_decode_fmt<FmtF32, 4>(waves, stages, fuse_append, grid, a, st);
        break;
    case VKV_DTYPE_Q8_0:
        ok = launch_decode_fmt<FmtQ8, 4>(waves, stages, fuse_append, grid, a, st);
        break;
    default: break;
    }
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_decode_rows(bool fuse_append, int n_streams, const DecodeArgs &a, hipStream_t st) {
    if (a.n_kv_heads != 8 || a.n_q_heads != 32) return hipErrorInvalidValue;
    dim3 grid((unsigned)a.n_chunks, (unsigned)a.n_layers, (unsigned)n_streams);
    // two batches in flight per wave (three or four measured 1-2% slower)
    if (fuse_append) hipLaunchKernelGGL((k_decode_rows<true, 2>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((k_decode_rows<false, 2>), grid, dim3(512), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_decode_q8rows(bool fuse_append, int n_streams, const DecodeArgs &a,
                               hipStream_t st) {
    if (a.n_kv_heads != 8 || a.n_q_heads != 32 || a.row_bytes != 1088 || a.chunk % 16 != 0)
        return hipErrorInvalidValue;
    dim3 grid((unsigned)a.n_chunks, (unsigned)a.n_layers, (unsigned)n_streams);
    // two stages in flight (the loads of a third cost registers, not time)
    if (fuse_append) hipLaunchKernelGGL((k_decode_q8rows<true, 2>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((k_decode_q8rows<false, 2>), grid, dim3(512), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs &a, int n_streams, hipStream_t st) {
    dim3 grid((unsigned)a.n_q_heads, (unsigned)a.n_layers, (unsigned)n_streams);
    hipLaunchKernelGGL(k_combine, grid, dim3(128), 0, st, a);
    return hipGetLastError();
}

// valu: the scalar-ALU kernel instead of the matrix-core tile (cross-check and
// A/B measurement)
hipError_t launch_window(int dtype, bool valu, const WindowArgs &a_in, hipStream_t st) {
    const bool mfma = (dtype == VKV_DTYPE_F16 || dtype == VKV_DTYPE_F32) && !valu &&
                      (a_in.head_dim == 64 || a_in.head_dim == 128);
    WindowArgs a = a_in;
    // Every query tile of a kv head stores that head's new rows in the fused
    // write, so its bytes grow with tiles x rows: keep it for calls with few
    // tiles per head (the encoder's 16-frame chunk is one tile, a 38-token
    // prompt ten) and append in a launch of its own above that.
    constexpr int kMaxFusedTiles = 16;
    const int tiles_per_head = (a.n_q * (a.n_q_heads / a.n_kv_heads) + 15) / 16;
    if (a.k_new && (!mfma || tiles_per_head > kMaxFusedTiles)) {
        // the scalar-ALU kernel has no fused write: append first
        AppendArgs ap{};
        ap.k = a.k_w;
        ap.v = a.v_w;
        ap.layer_bytes = a.layer_bytes;
        ap.row_bytes = a.row_bytes;
        ap.k_src = a.k_new;
        ap.v_src = a.v_new;
        ap.kv_dim = a.n_kv_heads * a.head_dim;
        ap.n_rows = a.n_new;
        ap.src_lstride = (int64_t)a.n_new * ap.kv_dim;
        ap.seg = a.wseg;
        hipError_t e = launch_append(dtype, ap, a.n_layers, st);
        if (e != hipSuccess) return e;
        a.k_new = nullptr;
        a.v_new = nullptr;
        a.n_new = 0;
    }
    if (mfma) {
        const int gqa = a.n_q_heads / a.n_kv_heads;
        const int tiles = (a.n_q * gqa + 15) / 16;
        dim3 g2((unsigned)(tiles * a.n_kv_heads), (unsigned)a.n_layers);
        // A per-layer encoder call (one layer, head_dim 64, GQA 1): one
        // layer's 32 heads are 32 work groups per tile, each streaming its
        // head's whole window from one CU.  Split over kWinSplit work groups
        // per head (key blocks of the absolute grid, 4 waves each) and merged
        // by a second launch, the work groups stream the layer from every CU
        // (F16 ring: encoder chunk 1.893 -> 1.803 ms).  Every such call takes
        // this path, whatever its number of frames, in groups of tiles that
        // fit the partials: the outputs do not depend on how the frames were
        // cut into calls.
        const bool split = a.n_layers == 1 && a.head_dim == 64 && gqa == 1 &&
                           a.split_vecs >= (int64_t)16 * a.n_q_heads * kWinSplit;
        if (split) {
            const int tg = (int)std::min<int64_t>(
                tiles, a.split_vecs / ((int64_t)16 * a.n_q_heads * kWinSplit));
            const int n_rows = a.n_q * gqa;
            for (int t0 = 0; t0 < tiles; t0 += tg) {
                WindowArgs b = a;
                b.tile0 = t0;
                if (t0 > 0) {   // the first launch stored the new rows
                    b.k_new = nullptr;
                    b.v_new = nullptr;
                    b.n_new = 0;
                }
                const int nt = std::min(tg, tiles - t0);
                const dim3 gs((unsigned)(nt * a.n_kv_heads), 1u, (unsigned)kWinSplit);
                if (dtype == VKV_DTYPE_F32)
                    hipLaunchKernelGGL(k_window_mfma_f32_64_split, gs, dim3(256), 0, st, b);
                else
                    hipLaunchKernelGGL((k_window_mfma<64, 4, 1, kWinSplit>), gs, dim3(256), 0, st, b);
                const int64_t n_vec = (int64_t)std::min(16 * nt, n_rows - 16 * t0) * a.n_q_heads;
                hipLaunchKernelGGL(k_window_merge<kWinSplit>,
                                   dim3((unsigned)((n_vec * 64 + 255) / 256)), dim3(256), 0, st,
                                   (const float *)a.part_o, (const float *)a.part_ml,
                                   a.out + (int64_t)16 * t0 * a.n_q_heads * 64, n_vec, 64);
            }
        } else if (dtype == VKV_DTYPE_F32) {
            // (8 waves for the per-layer calls, as the F16 tile takes, measured
            // slower here: 18.3 against 17.6 us per 4-frame call)
            if (a.head_dim == 64) hipLaunchKernelGGL(k_window_mfma_f32_64, g2, dim3(256), 0, st, a);
            else hipLaunchKernelGGL(k_window_mfma_f32_128, g2, dim3(256), 0, st, a);
        } else if (a.n_layers == 1 && a.head_dim == 64) {
            // a per-layer call without room for the split partials: 32 work
            // groups of 8 waves
            hipLaunchKernelGGL((k_window_mfma<64, 8>), g2, dim3(512), 0, st, a);
        } else if (a.head_dim == 64 && a.n_kv_heads % 4 == 0 &&
                   (int64_t)tiles * a.n_layers * (a.n_kv_heads / 4) >= 256) {
            // several layers (the batched encoder window): 4 kv heads per
            // work group, their 128-byte segments of a row read together
            // (32 layers x 32 heads: 256 work groups of 16 waves)
            dim3 g4((unsigned)(tiles * (a.n_kv_heads / 4)), (unsigned)a.n_layers);
            hipLaunchKernelGGL((k_window_mfma<64, 4, 4>), g4, dim3(1024), 0, st, a);
        } else {
            if (a.head_dim == 64) hipLaunchKernelGGL((k_window_mfma<64, 4>), g2, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((k_window_mfma<128, 4>), g2, dim3(256), 0, st, a);
        }
        return hipGetLastError();
    }
    dim3 grid((unsigned)(a.n_q * a.n_q_heads), (unsigned)a.n_layers);
    switch (dtype) {
    case VKV_DTYPE_F16: hipLaunchKernelGGL(k_window<FmtF16>, grid, dim3(64), 0, st, a); break;
    case VKV_DTYPE_F32: hipLaunchKernelGGL(k_window<FmtF32>, grid, dim3(64), 0, st, a); break;
    case VKV_DTYPE_Q8_0: hipLaunchKernelGGL(k_window<FmtQ8>, grid, dim3(64), 0, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rope(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                       int64_t pos0, float theta_scale, hipStream_t st) {
    const int64_t n = n_outer * n_rows * (row_len / 8);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3(grid_for(n, 256, 65536)), dim3(256), 0, st, x, n_outer, n_rows,
                       row_len, head_dim, pos0, theta_scale);
    return hipGetLastError();
}

hipError_t launch_q8_0_pack(const float *x, uint8_t *blocks, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_q8_pack, dim3(grid_for(n / 8, 256, INT32_MAX)), dim3(256), 0, st, x,
                       blocks, n);
    return hipGetLastError();
}

hipError_t launch_q8_0_unpack(const uint8_t *blocks, float *y, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_q8_unpack, dim3(grid_for(n / 8, 256, INT32_MAX)), dim3(256), 0, st,
                       blocks, y, n);
    return hipGetLastError();
}

hipError_t launch_fill_zero(void *dst, int64_t bytes, hipStream_t st) {
    if (bytes <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_zero, dim3(grid_for(bytes / 16 + 1, 256, 65536)), dim3(256), 0, st,
                       (uint8_t *)dst, bytes);
    return hipGetLastError();
}

hipError_t launch_synth(float *dst, int32_t row_len, uint64_t seed, uint32_t tag, int64_t s0,
                        int32_t ns, int64_t s_stride, int64_t l0, int32_t nl, int64_t l_stride,
                        int64_t p0, int32_t np, int64_t p_stride, hipStream_t st) {
    SynthArgs a{dst, seed, tag, row_len, ns, nl, np, s0, l0, p0, s_stride, l_stride, p_stride};
    const int64_t total = (int64_t)ns * nl * np * row_len;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_synth, dim3(grid_for(total, 256, 65536)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace vkv
