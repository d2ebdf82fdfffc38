// Host side of the gfx950 KV-cache hot path: ring planners, cache ownership,
// argument validation and the decoder/encoder step drivers behind vkv.h.
//
// The planners restate the reference's integer ring arithmetic
// (src/voxtral.cpp:1590-1656 decoder, :3636-3692 encoder); the step drivers
// keep run_decoder_step's contract (src/voxtral.cpp:5219-5360): plan first,
// reject an invalid plan before any device work, launch, then commit.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <new>
#include <string>
#include <vector>

#include "vkv.h"
#include "vkv_internal.h"

using namespace vkv;

struct vkv_cache {
    vkv_cache_params p{};
    int64_t row_bytes = 0;
    int64_t layer_bytes = 0;
    int64_t stream_bytes = 0;
    int64_t total_bytes = 0;
    uint8_t *k = nullptr;
    uint8_t *v = nullptr;
    // split-K workspace: partial outputs and (max, sum) per work group/head
    float *part_o = nullptr;
    float *part_ml = nullptr;
    int64_t part_heads_budget = 0;   // capacity of part_ml in (head, chunk) units
    int32_t n_cus = 256;             // compute units of the cache's device
};

namespace {

thread_local std::string g_last_error;
thread_local int32_t g_last_backend = 0;

vkv_status fail(vkv_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    if (st != VKV_STATUS_BACKEND_ERROR) g_last_backend = 0;
    return st;
}

vkv_status hip_fail(hipError_t e, const char *what) {
    g_last_backend = (int32_t)e;
    return fail(VKV_STATUS_BACKEND_ERROR, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

vkv_status ok() {
    g_last_error.clear();
    g_last_backend = 0;
    return VKV_STATUS_OK;
}

// Run device work on the cache's device; restores the caller's device.
struct DeviceGuard {
    int prev = -1;
    bool changed = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
            changed = hipSetDevice(dev) == hipSuccess;
        }
    }
    ~DeviceGuard() {
        if (changed) (void)hipSetDevice(prev);
    }
};

int64_t row_bytes_for(int dtype, int64_t n) {
    switch (dtype) {
    case VKV_DTYPE_F32: return n * 4;
    case VKV_DTYPE_F16: return n * 2;
    case VKV_DTYPE_Q8_0: return (n / 32) * 34;
    default: return -1;
    }
}

// <=2 physical segments of [abs_start, abs_start+len) modulo capacity
// (src/voxtral.cpp:1604-1613 and :3642-3651 apply the same rule).
int32_t ring_segments(int64_t abs_start, int32_t len, int32_t capacity, vkv_seg out[2]) {
    if (len <= 0) return 0;
    const int32_t slot = (int32_t)(abs_start % capacity);
    const int32_t first = std::min(len, capacity - slot);
    out[0] = {slot, first};
    if (first >= len) return 1;
    out[1] = {0, len - first};
    return 2;
}

SegPair seg_pair(const vkv_seg *segs, int32_t nseg) {
    SegPair sp{0, 0, 0, 0};
    if (nseg >= 1) { sp.s0 = segs[0].slot; sp.n0 = segs[0].len; }
    if (nseg >= 2) { sp.s1 = segs[1].slot; sp.n1 = segs[1].len; }
    return sp;
}

vkv_status check_segs(const vkv_cache *c, const vkv_seg *segs, int32_t nseg, const char *what) {
    if (nseg < 0 || nseg > 2) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: nseg=%d", what, nseg);
    if (nseg > 0 && !segs) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: null segments", what);
    int64_t total = 0;
    for (int32_t i = 0; i < nseg; ++i) {
        if (segs[i].len < 0 || segs[i].slot < 0 ||
            (int64_t)segs[i].slot + segs[i].len > c->p.capacity)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: segment %d [%d,+%d) outside capacity %d",
                        what, i, segs[i].slot, segs[i].len, c->p.capacity);
        total += segs[i].len;
    }
    if (total > c->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: %lld rows exceed capacity %d", what,
                    (long long)total, c->p.capacity);
    return VKV_STATUS_OK;
}

vkv_status check_cache(const vkv_cache *c, const char *what) {
    if (!c) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: null cache", what);
    return VKV_STATUS_OK;
}

vkv_status check_span(const vkv_cache *c, int32_t s0, int32_t ns, int32_t l0, int32_t nl,
                      const char *what) {
    if (s0 < 0 || ns < 1 || (int64_t)s0 + ns > c->p.n_streams)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: streams [%d,+%d) outside [0,%d)", what, s0,
                    ns, c->p.n_streams);
    if (l0 < 0 || nl < 1 || (int64_t)l0 + nl > c->p.n_layers)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: layers [%d,+%d) outside [0,%d)", what, l0,
                    nl, c->p.n_layers);
    return VKV_STATUS_OK;
}

vkv_status check_heads(const vkv_cache *c, int32_t n_q_heads, const char *what) {
    if (n_q_heads < c->p.n_kv_heads || n_q_heads % c->p.n_kv_heads != 0 ||
        n_q_heads > c->p.n_q_heads)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "%s: n_q_heads=%d must be a multiple of n_kv_heads=%d and <= %d", what,
                    n_q_heads, c->p.n_kv_heads, c->p.n_q_heads);
    return VKV_STATUS_OK;
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Device f32 arrays read with 16-byte vector loads must be 16-byte aligned.
vkv_status check_aligned(const char *what, std::initializer_list<const void *> ptrs) {
    for (const void *p : ptrs)
        if (p && !aligned16(p))
            return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: device arrays must be 16-byte aligned", what);
    return VKV_STATUS_OK;
}

uint8_t *stream_layer_base(const vkv_cache *c, uint8_t *base, int32_t stream, int32_t layer) {
    return base + (int64_t)stream * c->stream_bytes + (int64_t)layer * c->layer_bytes;
}

vkv_status do_append(vkv_cache *c, int32_t stream, int32_t layer0, int32_t n_layers,
                     const vkv_seg *segs, int32_t nseg, const float *k, const float *v,
                     int64_t layer_stride, hipStream_t st) {
    AppendArgs a{};
    a.k = stream_layer_base(c, c->k, stream, layer0);
    a.v = stream_layer_base(c, c->v, stream, layer0);
    a.layer_bytes = c->layer_bytes;
    a.row_bytes = c->row_bytes;
    a.k_src = k;
    a.v_src = v;
    a.kv_dim = c->p.n_kv_heads * c->p.head_dim;
    a.seg = seg_pair(segs, nseg);
    a.n_rows = a.seg.n0 + a.seg.n1;
    a.src_lstride = layer_stride ? layer_stride : (int64_t)a.n_rows * a.kv_dim;
    if (a.n_rows == 0) return VKV_STATUS_OK;
    hipError_t e = launch_append(c->p.dtype, a, n_layers, st);
    if (e != hipSuccess) return hip_fail(e, "append launch");
    return VKV_STATUS_OK;
}

bool has_flag(const vkv_cache *c, int32_t flag) { return (c->p.kernel_flags & flag) != 0; }

// Chunk size (logical slots per work group) for decode attention.
//
// One pass: when the (stream, layer, kv head) units number between 3/4 of the
// CUs and the CUs, one work group per unit owns the whole window (no split,
// no merge kernel) and each lands on a CU of its own.  Measured on MI355X at
// 26 layers x 8 kv heads x 8192 slots (208 units): the window streams at ~85%
// of HBM peak against ~81% for 1024-slot chunks, and the partials and the
// merge launch go away.  With more units than CUs the last round of such
// long work groups would leave most CUs idle, so the window is split.
//
// Split: the largest of 2048..64 that still gives >= 1536 work groups (about
// two waves of work groups over 256 CUs at 3 per CU), within the workspace.
// Measured on MI355X at 8 streams x 26 layers x 8192 slots (q8_0): 2048-slot
// chunks beat 1024 by 3% (the per-work-group prologue and merge amortise
// over more batches) and 4096 by 8% (too few work groups per CU).
int32_t pick_chunk(const vkv_cache *c, int64_t units, int32_t n_kv_max, int32_t gqa,
                   int32_t *n_chunks_out) {
    const int32_t forced_chunk = c->p.decode_chunk;
    if (!forced_chunk && 4 * units >= 3 * (int64_t)c->n_cus && units <= c->n_cus) {
        *n_chunks_out = 1;
        return std::max(n_kv_max, 1);
    }
    // the largest chunk (2048 .. 64 slots) that still gives every CU a work
    // group: fewer, longer chunks amortise each work group's prologue and
    // leave less to merge
    int32_t chunk = 2048;
    while (chunk > 64 && units * ((n_kv_max + chunk - 1) / chunk) < c->n_cus) chunk /= 2;
    if (forced_chunk) chunk = forced_chunk;
    for (;;) {
        const int32_t nc = std::max(1, (n_kv_max + chunk - 1) / chunk);
        if (units * nc * gqa <= c->part_heads_budget || chunk >= (1 << 30)) {
            *n_chunks_out = nc;
            return chunk;
        }
        chunk *= 2;
    }
}

// ggml's RoPE frequency step: powf(freq_base, -2/n_dims) (host libm, as the
// reference's CPU path evaluates it)
float rope_theta_scale(float theta, int32_t head_dim) {
    return std::pow(theta, -2.0f / (float)head_dim);
}

// The 64 (cos, sin) pairs of ggml's RoPE angles at one position, as the
// kernels' rope_table forms them: theta_i by the f32 running product (i
// multiplications by theta_scale, no contraction), cos/sin in double rounded
// to f32.  Kept per thread for the last position, so the layers of one
// token evaluate them once.
void host_rope_table(float pos, float theta_scale, float2 *tab) {
    struct Cached {
        bool valid = false;
        float pos = 0.0f, ts = 0.0f;
        float2 tab[64];
    };
    thread_local Cached cached;
    if (!cached.valid || cached.pos != pos || cached.ts != theta_scale) {
        volatile float theta = pos;   // one f32 rounding per step, as on the device
        for (int i = 0; i < 64; ++i) {
            const double t = (double)theta;
            cached.tab[i] = make_float2((float)std::cos(t), (float)std::sin(t));
            theta = theta * theta_scale;
        }
        cached.valid = true;
        cached.pos = pos;
        cached.ts = theta_scale;
    }
    std::memcpy(tab, cached.tab, sizeof(cached.tab));
}

// The merge of a split decode's chunk partials (k_combine), launched after it.
vkv_status merge_launch(const vkv_cache *c, const DecodeArgs &a, int32_t n_streams,
                        hipStream_t st) {
    if (a.n_chunks == 1) return VKV_STATUS_OK;
    CombineArgs cb{};
    cb.part_o = c->part_o;
    cb.part_ml = c->part_ml;
    cb.out = a.out;
    cb.n_chunks = a.n_chunks;
    cb.n_q_heads = a.n_q_heads;
    cb.n_layers = a.n_layers;
    cb.head_dim = c->p.head_dim;
    hipError_t e = launch_combine(cb, n_streams, st);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return VKV_STATUS_OK;
}

vkv_status do_decode(vkv_cache *c, int32_t stream0, int32_t n_streams, int32_t layer0,
                     int32_t n_layers, const SegPair *segs, const float *q, float *out,
                     int32_t n_q_heads, float scale, const float *k_new, const float *v_new,
                     hipStream_t st, const float *rope_theta = nullptr,
                     const int64_t *rope_pos = nullptr) {
    const int32_t D = c->p.head_dim;
    const int32_t G = c->p.n_kv_heads;
    const int32_t gqa = n_q_heads / G;
    // the kernel forms slot offsets with a 24x24-bit multiply into 32 bits
    if (c->row_bytes >= (1 << 24) || c->p.capacity >= (1 << 24) ||
        c->layer_bytes > (int64_t)UINT32_MAX)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "decode attention: rows or capacity beyond 2^24, or a layer beyond 4 GiB");
    if (D != 128 || gqa != 4)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "decode attention supports head_dim 128 and 4 query heads per KV head "
                    "(got head_dim %d, group %d)", D, gqa);
    int32_t n_kv_max = 0;
    for (int32_t s = 0; s < n_streams; ++s) n_kv_max = std::max(n_kv_max, segs[s].n0 + segs[s].n1);
    DecodeArgs a{};
    a.k = stream_layer_base(c, c->k, stream0, layer0);
    a.v = stream_layer_base(c, c->v, stream0, layer0);
    a.k_w = stream_layer_base(c, c->k, stream0, layer0);
    a.v_w = stream_layer_base(c, c->v, stream0, layer0);
    a.stream_bytes = c->stream_bytes;
    a.layer_bytes = c->layer_bytes;
    a.row_bytes = c->row_bytes;
    a.q = q;
    a.q_lstride = (int64_t)n_q_heads * D;
    a.q_sstride = (int64_t)n_layers * a.q_lstride;
    a.part_o = c->part_o;
    a.part_ml = c->part_ml;
    a.n_layers = n_layers;
    a.n_kv_heads = G;
    a.n_q_heads = n_q_heads;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.k_new = k_new;
    a.v_new = v_new;
    a.new_lstride = (int64_t)G * D;
    a.new_sstride = (int64_t)n_layers * a.new_lstride;
    for (int32_t s = 0; s < n_streams; ++s) a.seg[s] = segs[s];
    if (rope_theta) {
        a.rope = 1;
        a.rope_theta_scale = rope_theta_scale(*rope_theta, D);
        for (int32_t s = 0; s < n_streams; ++s) a.rope_pos[s] = (float)rope_pos[s];
        if (n_streams == 1) {
            host_rope_table(a.rope_pos[0], a.rope_theta_scale, a.rope_tab);
            a.rope_host = 1;
        }
    }
    const int64_t units = (int64_t)n_streams * n_layers * G;
    a.chunk = pick_chunk(c, units, n_kv_max, gqa, &a.n_chunks);
    a.out = out;
    // F16 by whole rows (k_decode_rows): a work group per (stream, layer,
    // chunk of at most 1024 slots) reads 2 KiB rows, which stream faster than
    // one head's 256-byte segments (measured on MI355X at 26 layers x 8192
    // slots: 135.4 against 140.0 us per step with the merge launch included).
    // Used when its grid at 1024-slot chunks holds between 3/4 of the CUs and
    // the CUs, as the one-pass k_decode; the cache's VKV_KERNEL_DECODE_HEADS
    // / _ROWS flags override.
    {
        const int32_t rows_chunk = c->p.decode_chunk ? c->p.decode_chunk : 1024;
        const int32_t nc = std::max(1, (n_kv_max + rows_chunk - 1) / rows_chunk);
        const int64_t groups = (int64_t)n_streams * n_layers * nc;
        const bool shape_ok = c->p.dtype == VKV_DTYPE_F16 && G == 8 && n_q_heads == 32 &&
                              (nc == 1 || units * nc * gqa <= c->part_heads_budget);
        const bool want = has_flag(c, VKV_KERNEL_DECODE_ROWS) ||
                          (!has_flag(c, VKV_KERNEL_DECODE_HEADS) &&
                           4 * groups >= 3 * (int64_t)c->n_cus && groups <= c->n_cus);
        if (shape_ok && want) {
            // As many chunks per (stream, layer) as leave every work group a
            // CU of its own: each reads less of the window.  Measured on
            // MI355X at 26 layers x 8192 slots: 9 chunks of 912 slots (234
            // work groups) 135.7 us per step against 8 of 1024 (208) 139.8;
            // 10 chunks (260 work groups, 4 of them doubled up) 158 us.
            int32_t chunk = rows_chunk;
            if (!c->p.decode_chunk && nc > 1) {
                const int64_t row_units = (int64_t)n_streams * n_layers;
                const int32_t cpl = (int32_t)std::max<int64_t>(1, c->n_cus / row_units);
                chunk = std::min(rows_chunk, ((n_kv_max + cpl - 1) / cpl + 15) / 16 * 16);
            }
            a.chunk = chunk;
            a.n_chunks = std::max(1, (n_kv_max + chunk - 1) / chunk);
            if (units * a.n_chunks * gqa > c->part_heads_budget) {
                a.chunk = rows_chunk;
                a.n_chunks = nc;
            }
            hipError_t e = launch_decode_rows(k_new != nullptr, n_streams, a, st);
            if (e != hipSuccess) return hip_fail(e, "decode launch");
            return merge_launch(c, a, n_streams, st);
        }
    }
    // q8_0 by whole rows (k_decode_q8rows): 1088-byte rows read as flat
    // 16-byte streams into LDS, the matrix cores fed from the raw rows.  Its
    // HBM reads are ~1.01x the algorithmic bytes against ~1.2x for the
    // per-head kernel (whose 136-byte head segments share lines between work
    // groups); at 8 streams x 26 layers x 8192 slots it measured 638 us per
    // step against 730 us.  Used when 1024-slot chunks give every CU a work
    // group (the multi-stream and all-layer calls); a per-layer call of one
    // stream (8 row units) keeps the per-head kernel's 8x more work groups.
    // The cache's VKV_KERNEL_DECODE_HEADS / _ROWS / _VALU flags override.
    // Chunk: the largest of 1024..64 slots (a multiple of the 16-slot stage)
    // that gives every CU a work group, within the partials workspace.
    const int64_t q8_row_units = (int64_t)n_streams * n_layers;
    const bool q8_rows_want =
        has_flag(c, VKV_KERNEL_DECODE_ROWS) ||
        (!has_flag(c, VKV_KERNEL_DECODE_HEADS) && !has_flag(c, VKV_KERNEL_DECODE_VALU) &&
         q8_row_units * ((n_kv_max + 1023) / 1024) >= (int64_t)c->n_cus);
    // (its loads form 32-bit offsets within a layer, with one past every
    // layer's descriptor for the idle waves' fifth load)
    if (c->p.dtype == VKV_DTYPE_Q8_0 && G == 8 && n_q_heads == 32 && c->row_bytes == 1088 &&
        c->layer_bytes + 256 < (int64_t)0xFFFFFF00 && q8_rows_want) {
        const int64_t row_units = (int64_t)n_streams * n_layers;
        int32_t chunk = 1024;
        while (chunk > 64 && row_units * ((n_kv_max + chunk - 1) / chunk) < (int64_t)c->n_cus)
            chunk /= 2;
        if (c->p.decode_chunk) chunk = c->p.decode_chunk;
        int32_t nc = std::max(1, (n_kv_max + chunk - 1) / chunk);
        while (nc > 1 && units * nc * gqa > c->part_heads_budget) {
            chunk *= 2;
            nc = std::max(1, (n_kv_max + chunk - 1) / chunk);
        }
        a.chunk = chunk;
        a.n_chunks = nc;
        hipError_t e = launch_decode_q8rows(k_new != nullptr, n_streams, a, st);
        if (e != hipSuccess) return hip_fail(e, "decode launch");
        return merge_launch(c, a, n_streams, st);
    }
    // XCD-grouped order: q8_0 head segments (136 B) share cache lines with
    // their neighbours.  The cache's XCD flags override.
    const int64_t n_wg = units * a.n_chunks;
    const bool sw_want = has_flag(c, VKV_KERNEL_XCD_SWIZZLE) ||
                         (!has_flag(c, VKV_KERNEL_NO_XCD_SWIZZLE) && c->p.dtype == VKV_DTYPE_Q8_0);
    a.xcd_swizzle = (sw_want && G == 8 && n_wg % 64 == 0) ? 1 : 0;
    const int32_t waves = c->p.decode_waves ? c->p.decode_waves : 4;
    const int32_t stages = std::min(c->p.decode_stages ? c->p.decode_stages : 2, waves == 8 ? 3 : 4);
    // q8_0: the matrix-core kernel when a work group streams more than 1024
    // slots, the VALU kernel (ggml's q8_0 arithmetic throughout) for chunks
    // of at most 1024 slots -- the per-layer call, and every short window
    // (26 one-layer calls per token at 8192 slots measured 389 against 460 us
    // with 256-slot chunks, 671 against 685 at 1024, and 1104 against 1006
    // at 2048); VKV_KERNEL_DECODE_VALU forces the VALU one.
    const bool short_chunks = a.chunk <= 1024;
    const bool mfma = !has_flag(c, VKV_KERNEL_DECODE_VALU) && !short_chunks;
    hipError_t e = launch_decode(c->p.dtype, gqa, waves, stages, mfma, k_new != nullptr,
                                 n_streams, a, st);
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return merge_launch(c, a, n_streams, st);
}

// Window attention of n_q queries; with k_new, the n_q new rows are first
// written through wsegs (fused into the matrix-core kernel).
vkv_status do_window(vkv_cache *c, int32_t stream, int32_t layer0, int32_t n_layers,
                     const vkv_seg *segs, int32_t nseg, int64_t key_pos0, int64_t q_pos0,
                     int32_t n_q, int32_t window, const float *q, float *out, int32_t n_q_heads,
                     float scale, hipStream_t st, const float *k_new = nullptr,
                     const float *v_new = nullptr, const vkv_seg *wsegs = nullptr,
                     int32_t wnseg = 0) {
    if (c->p.head_dim % 8 != 0 || c->p.head_dim > 128)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "window attention: head_dim %d unsupported",
                    c->p.head_dim);
    // the kernels form slot offsets in 32 bits
    if (c->layer_bytes > (int64_t)UINT32_MAX)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "window attention: a layer beyond 4 GiB");
    if (n_q <= 0) return VKV_STATUS_OK;
    WindowArgs a{};
    a.k = stream_layer_base(c, c->k, stream, layer0);
    a.v = stream_layer_base(c, c->v, stream, layer0);
    a.layer_bytes = c->layer_bytes;
    a.row_bytes = c->row_bytes;
    a.q = q;
    a.out = out;
    a.q_lstride = (int64_t)n_q * n_q_heads * c->p.head_dim;
    a.n_q = n_q;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = c->p.n_kv_heads;
    a.head_dim = c->p.head_dim;
    a.n_layers = n_layers;
    a.q_pos0 = q_pos0;
    a.key_pos0 = key_pos0;
    a.window = window;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.seg = seg_pair(segs, nseg);
    a.k_w = stream_layer_base(c, c->k, stream, layer0);
    a.v_w = stream_layer_base(c, c->v, stream, layer0);
    if (k_new) {
        a.k_new = k_new;
        a.v_new = v_new;
        a.n_new = n_q;
        a.wseg = seg_pair(wsegs, wnseg);
    }
    // this stream's share of the partials workspace (split window tiles)
    a.split_vecs = c->part_heads_budget / c->p.n_streams;
    a.part_o = c->part_o + (int64_t)stream * a.split_vecs * c->p.head_dim;
    a.part_ml = c->part_ml + (int64_t)stream * a.split_vecs * 2;
    hipError_t e = launch_window(c->p.dtype, has_flag(c, VKV_KERNEL_WINDOW_VALU), a, st);
    if (e != hipSuccess) return hip_fail(e, "window attention launch");
    return VKV_STATUS_OK;
}

}  // namespace

namespace vkv {
vkv_status host_fail(vkv_status st, const char *msg) { return fail(st, "%s", msg); }
vkv_status host_hip_fail(hipError_t e, const char *what) { return hip_fail(e, what); }
vkv_status host_ok() { return ok(); }
int cache_device(const vkv_cache *c) { return c->p.device; }
}  // namespace vkv

extern "C" {

uint32_t vkv_api_version(void) { return VKV_API_VERSION; }

const char *vkv_last_error(void) { return g_last_error.c_str(); }

int32_t vkv_last_backend_code(void) { return g_last_backend; }

// src/voxtral.cpp:1615-1644
vkv_status vkv_decoder_plan(const vkv_ring *ring, int64_t absolute_start, int32_t n_new,
                            vkv_plan *out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder plan: null out");
    std::memset(out, 0, sizeof(*out));
    if (!ring) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder plan: null ring");
    if (ring->capacity <= 0 || ring->capacity > INT32_MAX || ring->used < 0 ||
        ring->used > ring->capacity || ring->oldest_absolute_position < 0 ||
        ring->next_absolute_position < 0 ||
        ring->oldest_absolute_position + ring->used != ring->next_absolute_position)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder plan: inconsistent ring metadata");
    if (absolute_start != ring->next_absolute_position)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "decoder plan: invalid absolute position %lld (next=%lld)",
                    (long long)absolute_start, (long long)ring->next_absolute_position);
    if (n_new <= 0 || n_new > ring->capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder plan: n_new=%d outside (0, %lld]", n_new,
                    (long long)ring->capacity);
    const int32_t cap = (int32_t)ring->capacity;
    out->absolute_start = absolute_start;
    out->n_new = n_new;
    out->write_nseg = ring_segments(absolute_start, n_new, cap, out->write_seg);
    out->next_after = absolute_start + n_new;
    out->used_after = std::min<int64_t>(ring->capacity, ring->used + n_new);
    out->oldest_after = out->next_after - out->used_after;
    out->evicted = std::max<int64_t>(0, ring->used + n_new - ring->capacity);
    out->read_nseg = ring_segments(out->oldest_after, (int32_t)out->used_after, cap, out->read_seg);
    // A wrap is a crossing of a capacity cycle boundary by the appended span,
    // including the single-token write exactly at slot zero.
    const int64_t previous_cycle = absolute_start == 0 ? 0 : (absolute_start - 1) / ring->capacity;
    const int64_t newest_cycle = (out->next_after - 1) / ring->capacity;
    out->wrapped = newest_cycle > previous_cycle;
    return ok();
}

// src/voxtral.cpp:1646-1656
vkv_status vkv_decoder_commit(vkv_ring *ring, const vkv_plan *plan) {
    if (!ring || !plan) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder commit: null argument");
    ring->used = plan->used_after;
    ring->oldest_absolute_position = plan->oldest_after;
    ring->next_absolute_position = plan->next_after;
    ring->evictions += plan->evicted;
    if (plan->wrapped) ++ring->wraps;
    return ok();
}

// src/voxtral.cpp:1590-1602
vkv_status vkv_decoder_clear(vkv_ring *ring, int64_t capacity) {
    if (!ring) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder clear: null ring");
    std::memset(ring, 0, sizeof(*ring));
    ring->capacity = capacity;
    return ok();
}

// src/voxtral.cpp:3636-3638
int32_t vkv_enc_mask_allows(int64_t kv_abs, int64_t q_abs, int32_t window) {
    return kv_abs <= q_abs && kv_abs >= q_abs - (int64_t)(window - 1);
}

// src/voxtral.cpp:104-111
int32_t vkv_enc_normalize_physical(int32_t rows) {
    for (int32_t p = 4; p <= 64; p *= 2)
        if (rows <= p) return p;
    return VKV_ENC_MAX_NEW;
}

// src/voxtral.cpp:125-154; arguments <= 0 stand for unset variables
vkv_status vkv_enc_schedule_make(int32_t throughput, int32_t grid, int32_t logical,
                                 int32_t physical, vkv_enc_schedule *out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder schedule: null out");
    vkv_enc_schedule sc{4, 4};
    if (throughput) {
        sc.logical = sc.physical = VKV_ENC_MAX_NEW;
        *out = sc;
        return ok();
    }
    if (grid > 0) {   // the legacy grid knob: logical rows, a full grid from 32 up
        sc.logical = std::min(grid, VKV_ENC_MAX_NEW);
        if (grid >= 32) sc.physical = vkv_enc_normalize_physical(grid);
    }
    sc.logical = std::min(logical > 0 ? logical : sc.logical, VKV_ENC_MAX_NEW);
    sc.physical = vkv_enc_normalize_physical(physical > 0 ? physical : sc.physical);
    sc.logical = std::max(1, sc.logical);
    // a physical block holds a whole number of logical batches
    if (sc.logical > sc.physical || sc.physical % sc.logical != 0) {
        sc.logical = std::min(sc.logical, sc.physical);
        while (sc.logical > 1 && sc.physical % sc.logical != 0) --sc.logical;
    }
    *out = sc;
    return ok();
}

// src/voxtral.cpp:3700-3702
int64_t vkv_enc_frames_realizable(int64_t mel_frames) {
    return mel_frames < 2 ? 0 : (mel_frames - 2) / 2 + 1;
}

// src/voxtral.cpp:4379-4426, one iteration of the loop
vkv_status vkv_enc_drive_next(int64_t emitted, int64_t target, int32_t final,
                              const vkv_enc_schedule *schedule, int32_t finish_physical,
                              int32_t batch_terminal, vkv_enc_run *out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder drive: null out");
    std::memset(out, 0, sizeof(*out));
    if (!schedule || schedule->logical <= 0 || schedule->physical <= 0 || emitted < 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder drive: bad schedule or position");
    if (emitted >= target) return ok();   // done
    const int64_t rem = target - emitted;
    if (emitted == 0) {
        // the 128-frame startup block runs once, as soon as it is realizable;
        // nothing runs before it during feed
        if (target >= VKV_ENC_MAX_NEW) {
            out->q0 = 0;
            out->n = VKV_ENC_MAX_NEW;
            out->physical = VKV_ENC_MAX_NEW;
            out->warmup = 1;
            return ok();
        }
        if (!final) return ok();
    }
    if (!final && rem < schedule->logical) return ok();   // wait for a full logical batch
    const bool terminal = final && batch_terminal;
    const int32_t physical = terminal ? finish_physical : schedule->physical;
    const int32_t logical = terminal ? finish_physical : schedule->logical;
    if (physical <= 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder drive: finish block %d", physical);
    const int32_t room = physical - (int32_t)(emitted % physical);
    const int32_t n = (int32_t)std::min<int64_t>(std::min(logical, room), rem);
    if (n <= 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder drive: empty run");
    out->q0 = emitted;
    out->n = n;
    out->physical = physical;
    return ok();
}

// src/voxtral.cpp:3653-3692
vkv_status vkv_enc_plan_build(int64_t q_start, int32_t n_new, int32_t capacity, int32_t window,
                              vkv_enc_plan *out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder plan: null out");
    std::memset(out, 0, sizeof(*out));
    if (n_new <= 0 || capacity <= 0 || window <= 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder plan: n_new=%d capacity=%d window=%d",
                    n_new, capacity, window);
    if (n_new > capacity - window)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder plan: n_new=%d exceeds headroom %d",
                    n_new, capacity - window);
    if (q_start < 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder plan: q_start < 0");
    out->q_start = q_start;
    out->n_new = n_new;
    out->win_start = std::max<int64_t>(0, q_start - (int64_t)(window - 1));
    out->win_end = q_start + n_new;
    out->win_len = (int32_t)(out->win_end - out->win_start);
    out->read_nseg = ring_segments(out->win_start, out->win_len, capacity, out->read_seg);
    out->read_wraps = out->read_nseg > 1;
    out->write_nseg = ring_segments(q_start, n_new, capacity, out->write_seg);
    out->write_wraps = out->write_nseg > 1;
    out->conv_mel_start = std::max<int64_t>(0, 2 * (q_start - 2));
    out->conv_mel_end = 2 * (q_start + n_new);
    out->conv_slice_start = (int32_t)(q_start - out->conv_mel_start / 2);
    const int64_t old_lo = std::max<int64_t>(0, q_start - (int64_t)window);
    const int64_t new_lo = std::max<int64_t>(0, out->win_end - (int64_t)window);
    out->evicted = new_lo - old_lo;
    return ok();
}

vkv_status vkv_cache_create(const vkv_cache_params *params, vkv_cache **out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: null out");
    *out = nullptr;
    // Callers built against the parameter block that ends at `device` get the
    // automatic kernel selection (the later fields read as zero).
    constexpr size_t kBaseSize = offsetof(vkv_cache_params, kernel_flags);
    if (!params || params->struct_size < kBaseSize)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: params missing or struct_size too small");
    vkv_cache_params p{};
    std::memcpy(&p, params, std::min<size_t>(params->struct_size, sizeof(vkv_cache_params)));
    p.struct_size = sizeof(vkv_cache_params);
    if ((p.kernel_flags & ~VKV_KERNEL_FLAGS_ALL) != 0 ||
        ((p.kernel_flags & VKV_KERNEL_DECODE_HEADS) && (p.kernel_flags & VKV_KERNEL_DECODE_ROWS)) ||
        ((p.kernel_flags & VKV_KERNEL_XCD_SWIZZLE) && (p.kernel_flags & VKV_KERNEL_NO_XCD_SWIZZLE)))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: kernel_flags 0x%x invalid",
                    (unsigned)p.kernel_flags);
    if ((p.decode_chunk != 0 && (p.decode_chunk < 16 || p.decode_chunk % 16 != 0)) ||
        (p.decode_waves != 0 && p.decode_waves != 4 && p.decode_waves != 8) ||
        (p.decode_stages != 0 && (p.decode_stages < 2 || p.decode_stages > 4)))
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "cache create: decode_chunk %d / waves %d / stages %d out of range",
                    p.decode_chunk, p.decode_waves, p.decode_stages);
    if (p.n_streams < 1 || p.n_layers < 1 || p.capacity < 1 || p.n_kv_heads < 1 ||
        p.head_dim < 8 || p.head_dim % 8 != 0 || p.n_q_heads < p.n_kv_heads ||
        p.n_q_heads % p.n_kv_heads != 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: invalid shape");
    const int64_t kv_dim = (int64_t)p.n_kv_heads * p.head_dim;
    if (p.dtype != VKV_DTYPE_F32 && p.dtype != VKV_DTYPE_F16 && p.dtype != VKV_DTYPE_Q8_0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: dtype %d unsupported", p.dtype);
    if (p.dtype == VKV_DTYPE_Q8_0 && p.head_dim % 32 != 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: q8_0 needs head_dim %% 32 == 0");
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess) return hip_fail(e, "cache create: hipGetDeviceCount");
    if (p.device < 0 || p.device >= ndev)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache create: device %d not in [0,%d)", p.device, ndev);

    vkv_cache *c = new (std::nothrow) vkv_cache();
    if (!c) return fail(VKV_STATUS_OUT_OF_MEMORY, "cache create: host allocation");
    c->p = p;
    c->row_bytes = row_bytes_for(p.dtype, kv_dim);
    c->layer_bytes = c->row_bytes * p.capacity;
    c->stream_bytes = c->layer_bytes * p.n_layers;
    c->total_bytes = c->stream_bytes * p.n_streams;
    // decode workspace: every (stream, layer, kv head) at 256-slot chunks, and
    // at least 8192 work groups for small jobs; per work group GQA heads.
    const int64_t gqa = p.n_q_heads / p.n_kv_heads;
    const int64_t units = (int64_t)p.n_streams * p.n_layers * p.n_kv_heads;
    const int64_t wg = std::max<int64_t>(units * ((p.capacity + 255) / 256), 8192);
    c->part_heads_budget = wg * gqa;
    // the split per-layer encoder window (head_dim 64, GQA 1): per stream, 8
    // query tiles of 16 rows x n_q_heads x kWinSplit partials
    if (p.head_dim == 64 && p.n_q_heads == p.n_kv_heads)
        c->part_heads_budget = std::max<int64_t>(
            c->part_heads_budget, (int64_t)p.n_streams * 8 * 16 * p.n_q_heads * kWinSplit);

    DeviceGuard guard(p.device);
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p.device) ==
                hipSuccess && cus > 0)
            c->n_cus = cus;
    }
    // 256-byte tail pad: vector loads of the last q8_0 row may read a few
    // bytes past its end (never used).
    if ((e = hipMalloc(&c->k, (size_t)c->total_bytes + 256)) != hipSuccess ||
        (e = hipMalloc(&c->v, (size_t)c->total_bytes + 256)) != hipSuccess ||
        (e = hipMalloc(&c->part_o, (size_t)(c->part_heads_budget * p.head_dim * 4))) != hipSuccess ||
        (e = hipMalloc(&c->part_ml, (size_t)(c->part_heads_budget * 2 * 4))) != hipSuccess) {
        const bool oom = e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation;
        vkv_cache_destroy(c);
        if (oom) return fail(VKV_STATUS_OUT_OF_MEMORY, "cache create: device allocation failed");
        return hip_fail(e, "cache create: hipMalloc");
    }
    // Zero once at allocation (src/voxtral.cpp:1456-1464); never per stream.
    if ((e = launch_fill_zero(c->k, c->total_bytes, nullptr)) != hipSuccess ||
        (e = launch_fill_zero(c->v, c->total_bytes, nullptr)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        vkv_cache_destroy(c);
        return hip_fail(e, "cache create: zero fill");
    }
    *out = c;
    return ok();
}

vkv_status vkv_cache_destroy(vkv_cache *cache) {
    if (!cache) return ok();
    DeviceGuard guard(cache->p.device);
    hipError_t first = hipSuccess;
    for (void *p : {(void *)cache->k, (void *)cache->v, (void *)cache->part_o,
                    (void *)cache->part_ml}) {
        if (!p) continue;
        hipError_t e = hipFree(p);
        if (e != hipSuccess && first == hipSuccess) first = e;
    }
    delete cache;
    if (first != hipSuccess) return hip_fail(first, "cache destroy: hipFree");
    return ok();
}

vkv_status vkv_cache_get_layout(const vkv_cache *cache, vkv_cache_layout *out) {
    if (!out) return fail(VKV_STATUS_INVALID_ARGUMENT, "cache layout: null out");
    std::memset(out, 0, sizeof(*out));
    if (vkv_status st = check_cache(cache, "cache layout")) return st;
    out->row_bytes = (uint64_t)cache->row_bytes;
    out->layer_bytes = (uint64_t)cache->layer_bytes;
    out->stream_bytes = (uint64_t)cache->stream_bytes;
    out->total_bytes = (uint64_t)cache->total_bytes;
    out->k_base = cache->k;
    out->v_base = cache->v;
    return ok();
}

vkv_status vkv_cache_read_rows(const vkv_cache *cache, int32_t which, int32_t stream,
                               int32_t layer, int32_t slot0, int32_t n_slots, void *host_dst,
                               size_t dst_bytes) {
    if (vkv_status st = check_cache(cache, "cache read")) return st;
    if (which != 0 && which != 1) return fail(VKV_STATUS_INVALID_ARGUMENT, "cache read: which=%d", which);
    if (vkv_status st = check_span(cache, stream, 1, layer, 1, "cache read")) return st;
    if (slot0 < 0 || n_slots < 0 || (int64_t)slot0 + n_slots > cache->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "cache read: slots [%d,+%d) outside capacity", slot0, n_slots);
    const size_t bytes = (size_t)n_slots * (size_t)cache->row_bytes;
    if (!host_dst && bytes) return fail(VKV_STATUS_INVALID_ARGUMENT, "cache read: null destination");
    if (dst_bytes < bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "cache read: need %zu bytes, have %zu", bytes, dst_bytes);
    if (!bytes) return ok();
    DeviceGuard guard(cache->p.device);
    const uint8_t *src = stream_layer_base(cache, which ? cache->v : cache->k, stream, layer) +
                         (int64_t)slot0 * cache->row_bytes;
    hipError_t e = hipMemcpy(host_dst, src, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "cache read: hipMemcpy");
    return ok();
}

vkv_status vkv_cache_zero(vkv_cache *cache, void *hip_stream) {
    if (vkv_status st = check_cache(cache, "cache zero")) return st;
    DeviceGuard guard(cache->p.device);
    hipError_t e;
    if ((e = launch_fill_zero(cache->k, cache->total_bytes, as_stream(hip_stream))) != hipSuccess ||
        (e = launch_fill_zero(cache->v, cache->total_bytes, as_stream(hip_stream))) != hipSuccess)
        return hip_fail(e, "cache zero");
    return ok();
}

vkv_status vkv_append(vkv_cache *cache, int32_t stream, int32_t layer0, int32_t n_layers,
                      const vkv_seg *write_seg, int32_t write_nseg, const float *k_src,
                      const float *v_src, int64_t layer_stride, void *hip_stream) {
    if (vkv_status st = check_cache(cache, "append")) return st;
    if (vkv_status st = check_span(cache, stream, 1, layer0, n_layers, "append")) return st;
    if (vkv_status st = check_segs(cache, write_seg, write_nseg, "append")) return st;
    if (!k_src || !v_src) return fail(VKV_STATUS_INVALID_ARGUMENT, "append: null source");
    if (layer_stride < 0 || layer_stride % 4 != 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "append: layer stride must be a non-negative multiple of 4");
    if (!aligned16(k_src) || !aligned16(v_src))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "append: sources must be 16-byte aligned");
    DeviceGuard guard(cache->p.device);
    if (vkv_status st = do_append(cache, stream, layer0, n_layers, write_seg, write_nseg, k_src,
                                  v_src, layer_stride, as_stream(hip_stream)))
        return st;
    return ok();
}

vkv_status vkv_gather(const vkv_cache *cache, int32_t stream, int32_t layer,
                      const vkv_seg *read_seg, int32_t read_nseg, void *k_dst, void *v_dst,
                      void *hip_stream) {
    if (vkv_status st = check_cache(cache, "gather")) return st;
    if (vkv_status st = check_span(cache, stream, 1, layer, 1, "gather")) return st;
    if (vkv_status st = check_segs(cache, read_seg, read_nseg, "gather")) return st;
    if (!k_dst && !v_dst) return fail(VKV_STATUS_INVALID_ARGUMENT, "gather: null destinations");
    DeviceGuard guard(cache->p.device);
    const SegPair sp = seg_pair(read_seg, read_nseg);
    hipError_t e = hipSuccess;
    if (k_dst)
        e = launch_gather(stream_layer_base(cache, cache->k, stream, layer), cache->row_bytes, sp,
                          (uint8_t *)k_dst, as_stream(hip_stream));
    if (e == hipSuccess && v_dst)
        e = launch_gather(stream_layer_base(cache, cache->v, stream, layer), cache->row_bytes, sp,
                          (uint8_t *)v_dst, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "gather launch");
    return ok();
}

vkv_status vkv_decode_attn(vkv_cache *cache, int32_t stream0, int32_t n_streams, int32_t layer0,
                           int32_t n_layers, const vkv_plan *plans, const float *q, float *out,
                           int32_t n_q_heads, float scale, void *hip_stream) {
    if (vkv_status st = check_cache(cache, "decode attention")) return st;
    if (vkv_status st = check_span(cache, stream0, n_streams, layer0, n_layers, "decode attention"))
        return st;
    if (n_streams > kMaxStreams)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decode attention: at most %d streams per call", kMaxStreams);
    if (vkv_status st = check_heads(cache, n_q_heads, "decode attention")) return st;
    if (!plans || !q || !out) return fail(VKV_STATUS_INVALID_ARGUMENT, "decode attention: null argument");
    if (vkv_status st = check_aligned("decode attention", {q, out})) return st;
    if (!std::isfinite(scale)) return fail(VKV_STATUS_INVALID_ARGUMENT, "decode attention: scale");
    SegPair segs[kMaxStreams];
    for (int32_t s = 0; s < n_streams; ++s) {
        if (vkv_status st = check_segs(cache, plans[s].read_seg, plans[s].read_nseg, "decode attention"))
            return st;
        segs[s] = seg_pair(plans[s].read_seg, plans[s].read_nseg);
    }
    DeviceGuard guard(cache->p.device);
    if (vkv_status st = do_decode(cache, stream0, n_streams, layer0, n_layers, segs, q, out,
                                  n_q_heads, scale, nullptr, nullptr, as_stream(hip_stream)))
        return st;
    return ok();
}

namespace {
// Checks shared by the planned decode steps: the cache span, heads, pointers,
// scale and the RoPE arguments.
vkv_status check_step_args(vkv_cache *cache, int32_t stream0, int32_t n_streams, int32_t layer0,
                           int32_t n_layers, const float *q, const float *k, const float *v,
                           float *out, int32_t n_q_heads, float scale, const float *rope_theta,
                           const int64_t *positions, const char *what) {
    if (vkv_status st = check_cache(cache, what)) return st;
    if (vkv_status st = check_span(cache, stream0, n_streams, layer0, n_layers, what)) return st;
    if (n_streams > kMaxStreams)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: at most %d streams per call", what, kMaxStreams);
    if (vkv_status st = check_heads(cache, n_q_heads, what)) return st;
    if (!positions || !q || !k || !v || !out)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: null argument", what);
    if (vkv_status st = check_aligned(what, {q, k, v, out})) return st;
    if (!std::isfinite(scale)) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: scale", what);
    if (rope_theta) {
        if (!(std::isfinite(*rope_theta) && *rope_theta > 0.0f))
            return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: rope theta", what);
        for (int32_t s = 0; s < n_streams; ++s)
            if (positions[s] < 0 || positions[s] >= (1 << 24))
                return fail(VKV_STATUS_INVALID_ARGUMENT,
                            "%s: rope position %lld outside [0, 2^24)", what,
                            (long long)positions[s]);
    }
    return VKV_STATUS_OK;
}

// The read window of a one-row plan, checked to end at the appended row.
vkv_status planned_window(const vkv_cache *cache, const vkv_plan &plan, SegPair *seg,
                          const char *what) {
    if (plan.n_new != 1 || plan.write_nseg != 1 || plan.write_seg[0].len != 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: the plan must append exactly one row", what);
    if (vkv_status st = check_segs(cache, plan.read_seg, plan.read_nseg, what)) return st;
    if (plan.write_seg[0].slot < 0 || plan.write_seg[0].slot >= cache->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: write slot outside the cache", what);
    *seg = seg_pair(plan.read_seg, plan.read_nseg);
    const int32_t n_kv = seg->n0 + seg->n1;
    const int32_t newest = n_kv - 1 < seg->n0 ? seg->s0 + n_kv - 1 : seg->s1 + (n_kv - 1 - seg->n0);
    if (n_kv < 1 || newest != plan.write_seg[0].slot)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: plan window does not end at the new row", what);
    return VKV_STATUS_OK;
}

vkv_status decoder_step_impl(vkv_cache *cache, int32_t stream0, int32_t n_streams,
                             vkv_ring *rings, const int64_t *positions, int32_t layer0,
                             int32_t n_layers, const float *q, const float *k, const float *v,
                             float *out, int32_t n_q_heads, float scale, const float *rope_theta,
                             vkv_plan *plans_out, void *hip_stream) {
    if (plans_out && n_streams > 0) std::memset(plans_out, 0, sizeof(vkv_plan) * (size_t)n_streams);
    if (vkv_status st = check_step_args(cache, stream0, n_streams, layer0, n_layers, q, k, v, out,
                                        n_q_heads, scale, rope_theta, positions, "decoder step"))
        return st;
    if (!rings) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder step: null argument");
    vkv_plan plans[kMaxStreams];
    SegPair segs[kMaxStreams];
    for (int32_t s = 0; s < n_streams; ++s) {
        if (rings[s].capacity > cache->p.capacity)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder step: ring capacity %lld exceeds backing %d",
                        (long long)rings[s].capacity, cache->p.capacity);
        if (vkv_status st = vkv_decoder_plan(&rings[s], positions[s], 1, &plans[s])) {
            char msg[600];
            std::snprintf(msg, sizeof(msg), "decoder step (stream %d): %s", stream0 + s, g_last_error.c_str());
            return fail(st, "%s", msg);
        }
        if (planned_window(cache, plans[s], &segs[s], "decoder step"))
            return fail(VKV_STATUS_INTERNAL_ERROR, "decoder step: plan window does not end at the new row");
    }
    DeviceGuard guard(cache->p.device);
    if (vkv_status st = do_decode(cache, stream0, n_streams, layer0, n_layers, segs, q, out,
                                  n_q_heads, scale, k, v, as_stream(hip_stream), rope_theta,
                                  positions))
        return st;
    for (int32_t s = 0; s < n_streams; ++s) {
        vkv_decoder_commit(&rings[s], &plans[s]);
        if (plans_out) plans_out[s] = plans[s];
    }
    return ok();
}
}  // namespace

vkv_status vkv_decoder_step(vkv_cache *cache, int32_t stream0, int32_t n_streams, vkv_ring *rings,
                            const int64_t *positions, int32_t layer0, int32_t n_layers,
                            const float *q, const float *k, const float *v, float *out,
                            int32_t n_q_heads, float scale, vkv_plan *plans_out,
                            void *hip_stream) {
    return decoder_step_impl(cache, stream0, n_streams, rings, positions, layer0, n_layers, q, k,
                             v, out, n_q_heads, scale, nullptr, plans_out, hip_stream);
}

// src/voxtral.cpp:2667-2671 (RoPE of q and k) through :2854 (attention)
vkv_status vkv_decoder_step_rope(vkv_cache *cache, int32_t stream0, int32_t n_streams,
                                 vkv_ring *rings, const int64_t *positions, int32_t layer0,
                                 int32_t n_layers, const float *q, const float *k, const float *v,
                                 float *out, int32_t n_q_heads, float scale, float rope_theta,
                                 vkv_plan *plans_out, void *hip_stream) {
    return decoder_step_impl(cache, stream0, n_streams, rings, positions, layer0, n_layers, q, k,
                             v, out, n_q_heads, scale, &rope_theta, plans_out, hip_stream);
}

// build_decoder_layer's RoPE, SET_ROWS and attention (src/voxtral.cpp:2667-2854)
// for a layer range under a plan made once for the token (run_decoder_step,
// :5227-5232); the caller commits after the last layer (:5358).
vkv_status vkv_decoder_layer_step(vkv_cache *cache, int32_t stream, const vkv_plan *plan,
                                  int64_t position, int32_t layer0, int32_t n_layers,
                                  const float *q, const float *k, const float *v, float *out,
                                  int32_t n_q_heads, float scale, float rope_theta,
                                  void *hip_stream) {
    const float *theta = rope_theta > 0.0f ? &rope_theta : nullptr;
    if (!(rope_theta <= 0.0f || std::isfinite(rope_theta)))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder layer step: rope theta");
    if (vkv_status st = check_step_args(cache, stream, 1, layer0, n_layers, q, k, v, out, n_q_heads,
                                        scale, theta, &position, "decoder layer step"))
        return st;
    if (!plan) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder layer step: null plan");
    SegPair seg;
    if (vkv_status st = planned_window(cache, *plan, &seg, "decoder layer step")) return st;
    if (plan->absolute_start != position)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder layer step: position %lld is not the plan's %lld",
                    (long long)position, (long long)plan->absolute_start);
    DeviceGuard guard(cache->p.device);
    if (vkv_status st = do_decode(cache, stream, 1, layer0, n_layers, &seg, q, out, n_q_heads, scale,
                                  k, v, as_stream(hip_stream), theta, &position))
        return st;
    return ok();
}

// ggml_rope_ext mode 0 (src/voxtral.cpp:2667-2671) on f32 rows in place
vkv_status vkv_rope(float *x, int64_t n_outer, int64_t n_rows, int32_t row_len, int32_t head_dim,
                    int64_t pos0, float theta, void *hip_stream) {
    if (n_outer < 0 || n_rows < 0 || row_len <= 0 || head_dim <= 0 || head_dim % 8 != 0 ||
        row_len % head_dim != 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "rope: shape (row_len %d, head_dim %d)", row_len,
                    head_dim);
    if (!(std::isfinite(theta) && theta > 0.0f))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "rope: theta");
    if (pos0 < 0 || pos0 + n_rows > (1 << 24))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "rope: positions beyond exact f32 (2^24)");
    if (n_outer == 0 || n_rows == 0) return ok();
    if (!x || (reinterpret_cast<uintptr_t>(x) & 15) != 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "rope: null or unaligned rows");
    hipError_t e = launch_rope(x, n_outer, n_rows, row_len, head_dim, pos0,
                               rope_theta_scale(theta, head_dim), as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "rope launch");
    return ok();
}

vkv_status vkv_decoder_prefill(vkv_cache *cache, int32_t stream, vkv_ring *ring, int32_t layer0,
                               int32_t n_layers, int32_t n_tokens, const float *q, const float *k,
                               const float *v, float *out, int32_t n_q_heads, float scale,
                               void *hip_stream) {
    if (vkv_status st = check_cache(cache, "decoder prefill")) return st;
    if (vkv_status st = check_span(cache, stream, 1, layer0, n_layers, "decoder prefill")) return st;
    if (vkv_status st = check_heads(cache, n_q_heads, "decoder prefill")) return st;
    if (!ring || !q || !k || !v || !out)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prefill: null argument");
    if (vkv_status st = check_aligned("decoder prefill", {q, k, v, out})) return st;
    if (ring->capacity > cache->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prefill: ring capacity exceeds backing");
    vkv_plan plan;
    if (vkv_status st = vkv_decoder_plan(ring, ring->next_absolute_position, n_tokens, &plan))
        return st;
    if (plan.read_nseg != 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "decoder prefill: the post-append window must be one segment (got %d)", plan.read_nseg);
    DeviceGuard guard(cache->p.device);
    hipStream_t st = as_stream(hip_stream);
    if (vkv_status s = do_window(cache, stream, layer0, n_layers, plan.read_seg, plan.read_nseg,
                                 plan.oldest_after, plan.absolute_start, n_tokens, 0, q, out,
                                 n_q_heads, scale, st, k, v, plan.write_seg, plan.write_nseg))
        return s;
    vkv_decoder_commit(ring, &plan);
    return ok();
}

vkv_status vkv_enc_step(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                        int32_t window, int32_t layer0, int32_t n_layers, const float *q,
                        const float *k, const float *v, float *out, int32_t n_q_heads,
                        float scale, void *hip_stream) {
    if (vkv_status st = check_cache(cache, "encoder step")) return st;
    if (vkv_status st = check_span(cache, stream, 1, layer0, n_layers, "encoder step")) return st;
    if (vkv_status st = check_heads(cache, n_q_heads, "encoder step")) return st;
    if (!plan || !q || !k || !v || !out)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder step: null argument");
    if (vkv_status st = check_aligned("encoder step", {q, k, v, out})) return st;
    if (window <= 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder step: window %d", window);
    if (vkv_status st = check_segs(cache, plan->write_seg, plan->write_nseg, "encoder step write"))
        return st;
    if (vkv_status st = check_segs(cache, plan->read_seg, plan->read_nseg, "encoder step read"))
        return st;
    if (plan->write_seg[0].len + (plan->write_nseg > 1 ? plan->write_seg[1].len : 0) != plan->n_new)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder step: write segments do not cover n_new");
    DeviceGuard guard(cache->p.device);
    hipStream_t st = as_stream(hip_stream);
    if (vkv_status s = do_window(cache, stream, layer0, n_layers, plan->read_seg, plan->read_nseg,
                                 plan->win_start, plan->q_start, plan->n_new, window, q, out,
                                 n_q_heads, scale, st, k, v, plan->write_seg, plan->write_nseg))
        return s;
    return ok();
}

vkv_status vkv_window_attn(vkv_cache *cache, int32_t stream, int32_t layer0, int32_t n_layers,
                           const vkv_seg *read_seg, int32_t read_nseg, int64_t key_pos0,
                           int64_t q_pos0, int32_t n_q, int32_t window, const float *q, float *out,
                           int32_t n_q_heads, float scale, void *hip_stream) {
    if (vkv_status st = check_cache(cache, "window attention")) return st;
    if (vkv_status st = check_span(cache, stream, 1, layer0, n_layers, "window attention")) return st;
    if (vkv_status st = check_heads(cache, n_q_heads, "window attention")) return st;
    if (vkv_status st = check_segs(cache, read_seg, read_nseg, "window attention")) return st;
    if (n_q < 0 || (n_q > 0 && (!q || !out)))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "window attention: bad queries");
    if (vkv_status st = check_aligned("window attention", {q, out})) return st;
    DeviceGuard guard(cache->p.device);
    if (vkv_status s = do_window(cache, stream, layer0, n_layers, read_seg, read_nseg, key_pos0,
                                 q_pos0, n_q, window, q, out, n_q_heads, scale,
                                 as_stream(hip_stream)))
        return s;
    return ok();
}

vkv_status vkv_q8_0_pack(const float *x, void *blocks, int64_t n, void *hip_stream) {
    if (n < 0 || n % 32 != 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "q8_0 pack: n %% 32 != 0");
    if (n == 0) return ok();
    if (!x || !blocks) return fail(VKV_STATUS_INVALID_ARGUMENT, "q8_0 pack: null argument");
    hipError_t e = launch_q8_0_pack(x, (uint8_t *)blocks, n, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "q8_0 pack launch");
    return ok();
}

vkv_status vkv_q8_0_unpack(const void *blocks, float *y, int64_t n, void *hip_stream) {
    if (n < 0 || n % 32 != 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "q8_0 unpack: n %% 32 != 0");
    if (n == 0) return ok();
    if (!blocks || !y) return fail(VKV_STATUS_INVALID_ARGUMENT, "q8_0 unpack: null argument");
    hipError_t e = launch_q8_0_unpack((const uint8_t *)blocks, y, n, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "q8_0 unpack launch");
    return ok();
}

// ---- decoder projections on k-quant weights ----

namespace {

int device_cus() {
    // per device, filled on first use (threads may race to store the same value)
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int cus = cached[dev].load(std::memory_order_relaxed);
    if (cus <= 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

// bytes of 256 weights of a product's weight format (Q8_0: 8 blocks of 34)
int64_t kq_block_bytes(int32_t dtype) {
    return dtype == VKV_DTYPE_Q4_K ? 144 : dtype == VKV_DTYPE_Q6_K ? 210 : dtype == VKV_DTYPE_Q8_0 ? 272 : 0;
}

vkv_status check_mv_input(const char *what, const float *x, int64_t n_in, const float *norm_w,
                          const float *ada) {
    if (n_in < 256 || n_in % 256 != 0 || n_in > VKV_MV_MAX_IN)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: n_in=%lld must be a multiple of 256 in [256, %d]",
                    what, (long long)n_in, VKV_MV_MAX_IN);
    if (!x) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: null input", what);
    if (ada && !norm_w) return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: ada requires norm_w", what);
    return check_aligned(what, {x, norm_w, ada});
}

}  // namespace

namespace {
// vkv_matvec; with amax (one matrix, no SwiGLU) the argmax of its output is
// fused into the same launch (amax: two zeroed 8-byte words, see k_matvec)
vkv_status matvec_impl(const float *x, int64_t n_in, const float *norm_w, const float *ada,
                       float eps, const vkv_mv_out *outs, int32_t n_outs, int32_t epilogue,
                       void *hip_stream, unsigned long long *amax, int32_t *amax_out) {
    if (vkv_status st = check_mv_input("matvec", x, n_in, norm_w, ada)) return st;
    if (!outs || n_outs < 1 || n_outs > VKV_MV_MAX_OUTS)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: n_outs=%d outside [1, %d]", n_outs,
                    VKV_MV_MAX_OUTS);
    if (epilogue != VKV_MV_STORE && epilogue != VKV_MV_SWIGLU && epilogue != VKV_MV_GELU)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: unknown epilogue %d", epilogue);
    const bool swiglu = epilogue == VKV_MV_SWIGLU, gelu = epilogue == VKV_MV_GELU;
    if (swiglu && (n_outs != 2 || outs[0].n_rows != outs[1].n_rows ||
                   outs[0].dtype != outs[1].dtype))
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "matvec: SwiGLU takes two matrices of equal rows and dtype");
    int64_t total = 0;
    for (int32_t k = 0; k < n_outs; ++k) {
        const vkv_mv_out &o = outs[k];
        const int64_t bb = kq_block_bytes(o.dtype);
        if (!bb) return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: weight dtype %d", o.dtype);
        if (!o.w || (!o.y && !(swiglu && k == 1)) || o.n_rows < 1)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: matrix %d: null pointer or no rows", k);
        if ((int64_t)o.n_rows * (n_in / 256) * bb > (int64_t)0xFFFFFE00)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: matrix %d exceeds 4 GiB", k);
        if (reinterpret_cast<uintptr_t>(o.w) & 3u)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: weights must be 4-byte aligned");
        if ((swiglu || gelu) && o.add)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: SwiGLU and GELU have no residual add");
        total += o.n_rows;
    }
    if (swiglu) total = outs[0].n_rows;
    // Rows per wave: about 4 work groups per CU for the decoder's calls of
    // several matrices (Q/K/V: 1152 or more work groups repeat the input's
    // Q8_K prologue too often, 512 leave its latency exposed), one per CU for
    // a single matrix or a SwiGLU pair (3072 .. 9216 rows: each work group
    // streams more rows behind one prologue), 2 for the logits (131072 rows:
    // 64 rows per wave stream best).  Measured on MI355X with cold weights:
    // Q/K/V 7.8 us at 4 per CU (8.7 at one), the O projection 4.5 against
    // 5.0 us, W1/W3 10.4 against 11.2-12.6 us, W2 11.3 us either way.
    const int cus = device_cus();
    const int64_t per_cu = total > 32768 ? 8 : (n_outs == 1 || swiglu) ? 4 : 16;
    int64_t rpw = (total + per_cu * cus - 1) / (per_cu * cus);
    // at most 64 rows per wave: a lane holds each row's residual
    rpw = std::max<int64_t>(1, std::min<int64_t>(rpw, 64));
    MvArgs a{};
    a.x = x;
    a.norm_w = norm_w;
    a.ada = ada;
    a.eps = eps;
    a.n_in = (int32_t)n_in;
    a.n_outs = n_outs;
    a.rows_per_wg = (int32_t)(4 * rpw);
    a.swiglu = swiglu ? 1 : 0;
    a.gelu = gelu ? 1 : 0;
    int64_t wg = 0;
    for (int32_t k = 0; k < n_outs; ++k) {
        a.out[k] = MvOut{(const uint8_t *)outs[k].w, outs[k].y, outs[k].add, outs[k].dtype,
                         outs[k].n_rows, (int32_t)wg};
        if (!swiglu || k == 0) wg += (outs[k].n_rows + a.rows_per_wg - 1) / a.rows_per_wg;
    }
    if (swiglu) a.out[1].wg0 = 0x7fffffff;
    for (int32_t k = n_outs; k < VKV_MV_MAX_OUTS; ++k) a.out[k].wg0 = 0x7fffffff;
    if (wg > 0x7fffffff) return fail(VKV_STATUS_INVALID_ARGUMENT, "matvec: grid too large");
    if (amax) {
        a.amax = amax;
        a.amax_count = reinterpret_cast<unsigned int *>(amax + 1);
        a.amax_out = amax_out;
    }
    hipError_t e = launch_matvec(a, (int)wg, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "matvec launch");
    return ok();
}
}  // namespace

vkv_status vkv_matvec(const float *x, int64_t n_in, const float *norm_w, const float *ada,
                      float eps, const vkv_mv_out *outs, int32_t n_outs, int32_t epilogue,
                      void *hip_stream) {
    return matvec_impl(x, n_in, norm_w, ada, eps, outs, n_outs, epilogue, hip_stream, nullptr,
                       nullptr);
}

namespace {
struct MmImage {
    int8_t *codes;
    float *xd;
    int16_t *bs16;
    size_t bytes;
};
MmImage mm_image(int32_t n_cols, int64_t n_in, uint8_t *base) {
    MmImage im{};
    size_t off = 0;
    auto take = [&](size_t b) {
        uint8_t *p = base ? base + off : nullptr;
        off += (b + 255) & ~(size_t)255;
        return p;
    };
    im.codes = (int8_t *)take((size_t)n_cols * n_in);
    im.xd = (float *)take((size_t)n_cols * (n_in / 256) * 4);
    im.bs16 = (int16_t *)take((size_t)n_cols * (n_in / 32) * 2);
    im.bytes = off;
    return im;
}

// Where input / output row p of a product lives: row (row0 + p) % ring of a
// ring buffer when ring > 0, else row p.
struct RowMap {
    int32_t ring = 0, row0 = 0;
};

// RoPE of the outputs whose bit is set in mask (ggml mode 0, head_dim-wide
// heads, position pos0 + input row), fused into the products' epilogue
struct MmRope {
    uint32_t mask = 0;
    int32_t head_dim = 0;
    int64_t pos0 = 0;
    float theta = 0.0f;
};

vkv_status matmul_impl(const float *x, int32_t n_cols, int64_t n_in, const float *norm_w,
                       const float *norm_b, const float *ada, float eps, const vkv_mm_out *outs,
                       int32_t n_outs, int32_t epilogue, void *workspace, size_t workspace_bytes,
                       void *hip_stream, RowMap in_rows, RowMap out_rows, MmRope rope = MmRope{});
}  // namespace

size_t vkv_matmul_workspace(int32_t n_cols, int64_t n_in) {
    if (n_cols < 1 || n_in < 256 || n_in % 256 || n_in > VKV_MV_MAX_IN) return 0;
    return mm_image(n_cols, n_in, nullptr).bytes;
}

vkv_status vkv_matmul(const float *x, int32_t n_cols, int64_t n_in, const float *norm_w,
                      const float *norm_b, const float *ada, float eps, const vkv_mm_out *outs,
                      int32_t n_outs, int32_t epilogue, void *workspace, size_t workspace_bytes,
                      void *hip_stream) {
    return matmul_impl(x, n_cols, n_in, norm_w, norm_b, ada, eps, outs, n_outs, epilogue, workspace,
                       workspace_bytes, hip_stream, RowMap{}, RowMap{});
}

namespace {
vkv_status matmul_impl(const float *x, int32_t n_cols, int64_t n_in, const float *norm_w,
                       const float *norm_b, const float *ada, float eps, const vkv_mm_out *outs,
                       int32_t n_outs, int32_t epilogue, void *workspace, size_t workspace_bytes,
                       void *hip_stream, RowMap in_rows, RowMap out_rows, MmRope rope) {
    if (vkv_status st = check_mv_input("matmul", x, n_in, norm_w, ada)) return st;
    if (norm_b && !norm_w) return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: norm_b requires norm_w");
    if (vkv_status st = check_aligned("matmul", {norm_b})) return st;
    if (n_cols < 1 || n_cols > 65535 * 16)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: n_cols=%d", n_cols);
    if (!outs || n_outs < 1 || n_outs > VKV_MV_MAX_OUTS)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: n_outs=%d outside [1, %d]", n_outs,
                    VKV_MV_MAX_OUTS);
    if (epilogue != VKV_MV_STORE && epilogue != VKV_MV_SWIGLU && epilogue != VKV_MV_GELU)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: unknown epilogue %d", epilogue);
    const bool swiglu = epilogue == VKV_MV_SWIGLU, gelu = epilogue == VKV_MV_GELU;
    if (swiglu && (n_outs != 2 || outs[0].n_rows != outs[1].n_rows || outs[0].dtype != outs[1].dtype))
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "matmul: SwiGLU takes two matrices of equal rows and dtype");
    int64_t tiles = 0;
    MmArgs a{};
    for (int32_t k = 0; k < n_outs; ++k) {
        const vkv_mm_out &o = outs[k];
        const int64_t bb = kq_block_bytes(o.dtype);
        if (!bb) return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: weight dtype %d", o.dtype);
        // one input image per call: q8_0 for Q8_0 rows, Q8_K for the k-quants
        if ((o.dtype == VKV_DTYPE_Q8_0) != (outs[0].dtype == VKV_DTYPE_Q8_0))
            return fail(VKV_STATUS_INVALID_ARGUMENT,
                        "matmul: Q8_0 matrices cannot share a call with Q4_K / Q6_K ones");
        if (!o.w || (!o.y && !(swiglu && k == 1)) || o.n_rows < 1)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: matrix %d: null pointer or no rows", k);
        if ((int64_t)o.n_rows * (n_in / 256) * bb > (int64_t)0xFFFFFE00)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: matrix %d exceeds 4 GiB", k);
        if (reinterpret_cast<uintptr_t>(o.w) & 3u)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: weights must be 4-byte aligned");
        if ((swiglu || gelu) && o.add)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: SwiGLU and GELU have no residual add");
        a.out[k] = MmOut{(const uint8_t *)o.w, o.y, o.add, o.bias, o.dtype, o.n_rows, 0};
        if (!swiglu || k == 0) tiles += (o.n_rows + 15) / 16;
    }
    if (tiles > 0x7fffffff) return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: grid too large");
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: workspace null or not 256-byte aligned");
    const MmImage im = mm_image(n_cols, n_in, (uint8_t *)workspace);
    if (workspace_bytes < im.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "matmul: workspace %zu < %zu bytes", workspace_bytes,
                    im.bytes);
    a.n_in = (int32_t)n_in;
    a.n_cols = n_cols;
    a.n_outs = n_outs;
    a.swiglu = swiglu ? 1 : 0;
    // The input's Q8_K image: quantized inside the product's work groups for
    // calls with few input rows (no launch of its own: one dependent launch
    // less, ~4.5 us, per product), else by k_q8k_rows into the workspace.
    // An output that overlaps the input rows (in place) takes the separate
    // quantization: the products' work groups would otherwise read rows that
    // others have already overwritten.
    hipError_t e = hipSuccess;
    const int n_col_tiles = (n_cols + 15) / 16;
    const uintptr_t x_lo = reinterpret_cast<uintptr_t>(x);
    const uintptr_t x_hi = x_lo + (uintptr_t)(in_rows.ring > 0 ? in_rows.ring : n_cols) * n_in * 4;
    bool in_place = false;
    for (int32_t k = 0; k < n_outs; ++k)
        for (const float *p : {(const float *)outs[k].y, outs[k].add}) {
            if (!p) continue;
            const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
            const uintptr_t hi =
                lo + (uintptr_t)(out_rows.ring > 0 ? out_rows.ring : n_cols) * outs[k].n_rows * 4;
            in_place = in_place || (lo < x_hi && x_lo < hi);
        }
    // The norm's vectors are set before the fused check: its guard on the
    // input width and its LDS size both depend on whether a norm is applied.
    a.norm_w = norm_w;
    a.norm_b = norm_b;
    a.ada = ada;
    if (!in_place && gemm_fused_ok(a, n_col_tiles)) {
        a.x = x;
        a.x_stride = n_in;
        a.x_ring = in_rows.ring;
        a.x_row0 = in_rows.row0;
        a.eps = eps;
        a.xq = im.codes;   // (the image is also left in the workspace)
        a.xd = im.xd;
        a.xbs = im.bs16;
    } else {
        a.norm_w = a.norm_b = a.ada = nullptr;   // applied by the separate quantization
        e = launch_q8k_rows(x, n_in, in_rows.ring, in_rows.row0, n_cols, (int)n_in, norm_w, norm_b,
                            ada, eps, im.codes, im.xd, im.bs16, outs[0].dtype == VKV_DTYPE_Q8_0,
                            as_stream(hip_stream));
        if (e != hipSuccess) return hip_fail(e, "matmul input launch");
        a.xq = im.codes;
        a.xd = im.xd;
        a.xbs = im.bs16;
    }
    a.gelu = gelu ? 1 : 0;
    a.y_ring = out_rows.ring;
    a.y_row0 = out_rows.row0;
    if (rope.mask) {
        if (epilogue != VKV_MV_STORE || rope.head_dim < 2 || rope.head_dim % 2 || rope.head_dim > 16 * 1024)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: RoPE takes plain outputs and an even head_dim");
        for (int32_t k = 0; k < n_outs; ++k) {
            if (!(rope.mask >> k & 1u)) continue;
            if (outs[k].add || outs[k].n_rows % rope.head_dim)
                return fail(VKV_STATUS_INVALID_ARGUMENT, "matmul: RoPE output %d shape", k);
            a.out[k].rope = 1;
        }
        a.rope_ts = rope_theta_scale(rope.theta, rope.head_dim);
        a.rope_hd = rope.head_dim;
        a.rope_pos0 = rope.pos0;
    }
    e = launch_gemm_kq(a, n_col_tiles, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "matmul launch");
    return ok();
}
}  // namespace

size_t vkv_ada_scale_workspace(int32_t dim, int32_t ada_dim) {
    if (dim < 256 || dim % 256 || dim > VKV_MV_MAX_IN || ada_dim < 1 || ada_dim > VKV_MV_MAX_IN)
        return 0;
    return ((size_t)dim * 4 + 255) / 256 * 256 + ((size_t)ada_dim * 4 + 255) / 256 * 256;
}

vkv_status vkv_ada_scale(const void *w0, int32_t w0_type, const void *w2, int32_t w2_type,
                         int32_t dim, int32_t ada_dim, float t, float *out, void *workspace,
                         size_t workspace_bytes, void *hip_stream) {
    const size_t need = vkv_ada_scale_workspace(dim, ada_dim);
    if (!need) return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: dim=%d ada_dim=%d", dim, ada_dim);
    if (!w0 || !w2 || !out || !workspace)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: null argument");
    if (!kq_block_bytes(w0_type) ||
        (w2_type != VKV_DTYPE_F16 && w2_type != VKV_DTYPE_F32 && w2_type != VKV_DTYPE_Q8_0))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: weight dtypes %d / %d", w0_type, w2_type);
    if (w2_type == VKV_DTYPE_Q8_0 && ada_dim % 32)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: Q8_0 W2 needs ada_dim %% 32 == 0");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: workspace not 256-byte aligned");
    if (workspace_bytes < need)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "ada scale: workspace %zu < %zu bytes", workspace_bytes, need);
    if ((reinterpret_cast<uintptr_t>(w2) & (w2_type == VKV_DTYPE_F32 ? 3u : 1u)) ||
        (reinterpret_cast<uintptr_t>(out) & 3u))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ada scale: misaligned w2 or out");
    // the time embedding as the reference computes it on the host
    // (compute_time_embedding, src/voxtral.cpp:729-740)
    std::vector<float> emb((size_t)dim);
    const int32_t half = dim / 2;
    for (int32_t i = 0; i < half; ++i) {
        const float inv_freq = expf(-logf(10000.0f) * (float)i / (float)half);
        const float angle = t * inv_freq;
        emb[(size_t)i] = cosf(angle);
        emb[(size_t)(i + half)] = sinf(angle);
    }
    float *e_dev = (float *)workspace;
    float *hidden = (float *)((uint8_t *)workspace + ((size_t)dim * 4 + 255) / 256 * 256);
    hipStream_t st = as_stream(hip_stream);
    hipError_t e = hipMemcpyAsync(e_dev, emb.data(), (size_t)dim * 4, hipMemcpyHostToDevice, st);
    // the host vector must outlive the copy
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "ada scale: time embedding upload");
    const vkv_mv_out h[1] = {{w0, w0_type, ada_dim, hidden, nullptr}};
    if (vkv_status s = matvec_impl(e_dev, dim, nullptr, nullptr, 0.0f, h, 1, VKV_MV_GELU, hip_stream,
                                   nullptr, nullptr))
        return s;
    e = launch_rows_small(w2, w2_type, hidden, ada_dim, dim, out, st);
    if (e != hipSuccess) return hip_fail(e, "ada scale: second product launch");
    return ok();
}

vkv_status vkv_quantize_q8_k(const float *x, int64_t n, const float *norm_w, const float *ada,
                             float eps, void *blocks, void *hip_stream) {
    if (vkv_status st = check_mv_input("q8_K quantize", x, n, norm_w, ada)) return st;
    if (!blocks || (reinterpret_cast<uintptr_t>(blocks) & 3u))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "q8_K quantize: output null or not 4-byte aligned");
    hipError_t e = launch_q8k_quant(x, (int)n, norm_w, ada, eps, (uint8_t *)blocks,
                                    as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "q8_K quantize launch");
    return ok();
}

vkv_status vkv_dequantize(int32_t dtype, const void *blocks, int64_t n, float *y,
                          void *hip_stream) {
    if (!kq_block_bytes(dtype)) return fail(VKV_STATUS_INVALID_ARGUMENT, "dequantize: dtype %d", dtype);
    if (n < 0 || n % 256 != 0) return fail(VKV_STATUS_INVALID_ARGUMENT, "dequantize: n %% 256 != 0");
    if (n == 0) return ok();
    if (!blocks || !y) return fail(VKV_STATUS_INVALID_ARGUMENT, "dequantize: null argument");
    if (n / 8 > (int64_t)0x7fffffff * 256)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "dequantize: n too large");
    hipError_t e = launch_kq_dequant(dtype, (const uint8_t *)blocks, n, nullptr, y,
                                     as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return ok();
}

vkv_status vkv_embed(int32_t dtype, const void *table, int32_t n_rows, int64_t n_cols,
                     int32_t token, const float *add, float *y, void *hip_stream) {
    const int64_t bb = kq_block_bytes(dtype);
    if (!bb) return fail(VKV_STATUS_INVALID_ARGUMENT, "embed: dtype %d", dtype);
    if (n_cols < 256 || n_cols % 256 != 0 || n_cols > ((int64_t)1 << 30))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "embed: n_cols=%lld", (long long)n_cols);
    if (token < 0 || token >= n_rows)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "embed: token %d outside [0, %d)", token, n_rows);
    if (!table || !y) return fail(VKV_STATUS_INVALID_ARGUMENT, "embed: null argument");
    const uint8_t *row = (const uint8_t *)table + (int64_t)token * (n_cols / 256) * bb;
    hipError_t e = launch_kq_dequant(dtype, row, n_cols, add, y, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "embed launch");
    return ok();
}

vkv_status vkv_argmax(const float *x, int64_t n, int32_t *out, void *hip_stream) {
    if (n < 1 || n > 0x7fffffff) return fail(VKV_STATUS_INVALID_ARGUMENT, "argmax: n=%lld", (long long)n);
    if (!x || !out) return fail(VKV_STATUS_INVALID_ARGUMENT, "argmax: null argument");
    if (vkv_status st = check_aligned("argmax", {x})) return st;
    hipError_t e = launch_argmax(x, (int)n, out, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    return ok();
}

// ---- one decoder token ----

namespace {

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct TokenBuffers {
    float *x, *q, *k, *v, *attn, *ffn;
    unsigned long long *amax;   // fused argmax: key + finished-work-group count
    size_t bytes;
};

TokenBuffers token_buffers(const vkv_dec_model &m, uint8_t *base) {
    TokenBuffers t{};
    size_t off = 0;
    auto take = [&](size_t n) {
        float *p = base ? reinterpret_cast<float *>(base + off) : nullptr;
        off += align256(n * sizeof(float));
        return p;
    };
    const size_t qd = (size_t)m.n_q_heads * m.head_dim, kd = (size_t)m.n_kv_heads * m.head_dim;
    t.x = take((size_t)m.dim);
    t.q = take(qd);
    t.k = take(kd);
    t.v = take(kd);
    t.attn = take(qd);
    t.ffn = take((size_t)m.hidden);
    t.amax = reinterpret_cast<unsigned long long *>(take(4));
    t.bytes = off;
    return t;
}

vkv_status check_row_ring(const vkv_row_ring *r, const char *what) {
    if (!r || !r->rows || r->capacity < 1 || r->width < 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: null ring or empty shape", what);
    if ((int64_t)r->capacity * r->width > ((int64_t)1 << 40))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "%s: ring too large", what);
    return check_aligned(what, {r->rows});
}

vkv_status check_model(const vkv_dec_model *m) {
    if (!m || !m->layers || m->n_layers < 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: null model or no layers");
    if (m->dim < 256 || m->dim % 256 || m->hidden < 256 || m->hidden % 256 || m->head_dim < 8 ||
        m->n_q_heads < 1 || m->n_kv_heads < 1 || m->vocab < 1 ||
        (int64_t)m->n_q_heads * m->head_dim % 256)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: model dimensions");
    if (!m->tok_embeddings || !m->output || !m->out_norm)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: null embedding/output/norm");
    for (int32_t l = 0; l < m->n_layers; ++l) {
        const vkv_dec_layer &L = m->layers[l];
        if (!L.attn_norm || !L.ffn_norm || !L.attn_q || !L.attn_k || !L.attn_v || !L.attn_o ||
            !L.ffn_w1 || !L.ffn_w2 || !L.ffn_w3)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: layer %d has a null tensor", l);
    }
    return VKV_STATUS_OK;
}

}  // namespace

size_t vkv_decoder_token_workspace(const vkv_dec_model *model) {
    if (check_model(model)) return 0;
    return token_buffers(*model, nullptr).bytes;
}

vkv_status vkv_decoder_token(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                             const vkv_dec_model *model, int32_t token, const float *audio_emb,
                             float *logits, int32_t *token_out, void *workspace,
                             size_t workspace_bytes, vkv_plan *plan_out, void *hip_stream) {
    if (plan_out) std::memset(plan_out, 0, sizeof(*plan_out));
    if (vkv_status st = check_model(model)) return st;
    const vkv_dec_model &m = *model;
    if (vkv_status st = check_cache(cache, "decoder token")) return st;
    if (m.n_layers != cache->p.n_layers || m.n_kv_heads != cache->p.n_kv_heads ||
        m.head_dim != cache->p.head_dim || m.n_q_heads > cache->p.n_q_heads)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: model and cache shapes differ");
    if (!ring || !logits || !token_out || !workspace)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: null argument");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: workspace not 256-byte aligned");
    const TokenBuffers t = token_buffers(m, (uint8_t *)workspace);
    if (workspace_bytes < t.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "decoder token: workspace %zu < %zu bytes",
                    workspace_bytes, t.bytes);
    if (ring->capacity > cache->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: ring capacity exceeds the cache");
    const int64_t pos = ring->next_absolute_position;
    vkv_plan plan;
    if (vkv_status st = vkv_decoder_plan(ring, pos, 1, &plan)) return st;
    const int32_t qd = m.n_q_heads * m.head_dim, kd = m.n_kv_heads * m.head_dim;
    const float scale = 1.0f / std::sqrt((float)m.head_dim);
    void *st = hip_stream;
    if (token < 0 || token >= m.vocab)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: token %d outside [0, %d)", token,
                    m.vocab);
    {
        // embedding row + audio; its first work group also clears the argmax words
        const int64_t bb = kq_block_bytes(m.tok_embeddings_type);
        if (!bb) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token: embedding dtype");
        const uint8_t *row = (const uint8_t *)m.tok_embeddings + (int64_t)token * (m.dim / 256) * bb;
        hipError_t e = launch_kq_dequant(m.tok_embeddings_type, row, m.dim, audio_emb, t.x,
                                         as_stream(st), t.amax);
        if (e != hipSuccess) return hip_fail(e, "decoder token: embedding launch");
    }
    for (int32_t l = 0; l < m.n_layers; ++l) {
        const vkv_dec_layer &L = m.layers[l];
        const vkv_mv_out qkv[3] = {{L.attn_q, L.attn_q_type, qd, t.q, nullptr},
                                   {L.attn_k, L.attn_k_type, kd, t.k, nullptr},
                                   {L.attn_v, L.attn_v_type, kd, t.v, nullptr}};
        if (vkv_status s = vkv_matvec(t.x, m.dim, L.attn_norm, nullptr, m.norm_eps, qkv, 3,
                                      VKV_MV_STORE, st))
            return s;
        if (vkv_status s = vkv_decoder_layer_step(cache, stream, &plan, pos, l, 1, t.q, t.k, t.v,
                                                  t.attn, m.n_q_heads, scale, m.rope_theta, st))
            return s;
        const vkv_mv_out o[1] = {{L.attn_o, L.attn_o_type, m.dim, t.x, t.x}};
        if (vkv_status s = vkv_matvec(t.attn, qd, nullptr, nullptr, m.norm_eps, o, 1, VKV_MV_STORE, st))
            return s;
        const vkv_mv_out gu[2] = {{L.ffn_w1, L.ffn_w1_type, m.hidden, t.ffn, nullptr},
                                  {L.ffn_w3, L.ffn_w3_type, m.hidden, nullptr, nullptr}};
        if (vkv_status s = vkv_matvec(t.x, m.dim, L.ffn_norm, L.ada_scale, m.norm_eps, gu, 2,
                                      VKV_MV_SWIGLU, st))
            return s;
        const vkv_mv_out down[1] = {{L.ffn_w2, L.ffn_w2_type, m.dim, t.x, t.x}};
        if (vkv_status s = vkv_matvec(t.ffn, m.hidden, nullptr, nullptr, m.norm_eps, down, 1,
                                      VKV_MV_STORE, st))
            return s;
    }
    const vkv_mv_out head[1] = {{m.output, m.output_type, m.vocab, logits, nullptr}};
    if (vkv_status s = matvec_impl(t.x, m.dim, m.out_norm, nullptr, m.norm_eps, head, 1,
                                   VKV_MV_STORE, st, t.amax, token_out))
        return s;
    vkv_decoder_commit(ring, &plan);
    if (plan_out) *plan_out = plan;
    return ok();
}

// ---- the decoder prefill of a prompt ----

namespace {

struct PromptBuffers {
    float *x, *q, *k, *v, *attn, *ffn;
    unsigned long long *amax;
    void *image;
    size_t image_bytes, bytes;
};

PromptBuffers prompt_buffers(const vkv_dec_model &m, int32_t n, uint8_t *base) {
    PromptBuffers t{};
    size_t off = 0;
    auto take = [&](size_t b) {
        uint8_t *p = base ? base + off : nullptr;
        off += align256(b);
        return p;
    };
    const size_t qd = (size_t)m.n_q_heads * m.head_dim, kd = (size_t)m.n_kv_heads * m.head_dim;
    t.x = (float *)take((size_t)n * m.dim * 4);
    t.q = (float *)take((size_t)n * qd * 4);
    t.k = (float *)take((size_t)n * kd * 4);
    t.v = (float *)take((size_t)n * kd * 4);
    t.attn = (float *)take((size_t)n * qd * 4);
    t.ffn = (float *)take((size_t)n * m.hidden * 4);
    t.amax = (unsigned long long *)take(16);
    // the products' Q8_K input image, sized for the widest input
    t.image_bytes = vkv_matmul_workspace(n, std::max<int64_t>(std::max<int64_t>(m.dim, m.hidden), qd));
    t.image = take(t.image_bytes);
    t.bytes = off;
    return t;
}

}  // namespace

size_t vkv_decoder_prompt_workspace(const vkv_dec_model *model, int32_t n_tokens) {
    if (check_model(model) || n_tokens < 1 || n_tokens > 65535 * 16) return 0;
    return prompt_buffers(*model, n_tokens, nullptr).bytes;
}

vkv_status vkv_decoder_prompt(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                              const vkv_dec_model *model, const int32_t *tokens, int32_t n_tokens,
                              const vkv_row_ring *audio_emb, float *logits, int32_t *token_out,
                              void *workspace, size_t workspace_bytes, vkv_plan *plan_out,
                              void *hip_stream) {
    if (plan_out) std::memset(plan_out, 0, sizeof(*plan_out));
    if (vkv_status st = check_model(model)) return st;
    const vkv_dec_model &m = *model;
    if (vkv_status st = check_cache(cache, "decoder prompt")) return st;
    if (vkv_status st = check_span(cache, stream, 1, 0, m.n_layers, "decoder prompt")) return st;
    if (m.n_layers != cache->p.n_layers || m.n_kv_heads != cache->p.n_kv_heads ||
        m.head_dim != cache->p.head_dim || m.n_q_heads > cache->p.n_q_heads)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: model and cache shapes differ");
    if (vkv_status st = check_heads(cache, m.n_q_heads, "decoder prompt")) return st;
    if (!ring || !tokens || !logits || !token_out || !workspace)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: null argument");
    if (n_tokens < 1 || n_tokens > 65535 * 16)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: n_tokens=%d", n_tokens);
    for (int32_t i = 0; i < n_tokens; ++i)
        if (tokens[i] < 0 || tokens[i] >= m.vocab)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: token %d (%d) outside [0, %d)",
                        i, tokens[i], m.vocab);
    if (audio_emb) {
        if (vkv_status st = check_row_ring(audio_emb, "decoder prompt")) return st;
        if (audio_emb->width != m.dim)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: audio rows of width %d, not %d",
                        audio_emb->width, m.dim);
    }
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: workspace not 256-byte aligned");
    const PromptBuffers t = prompt_buffers(m, n_tokens, (uint8_t *)workspace);
    if (workspace_bytes < t.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "decoder prompt: workspace %zu < %zu bytes",
                    workspace_bytes, t.bytes);
    if (ring->capacity > cache->p.capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: ring capacity exceeds the cache");
    const int64_t pos0 = ring->next_absolute_position;
    vkv_plan plan;
    if (vkv_status st = vkv_decoder_plan(ring, pos0, n_tokens, &plan)) return st;
    if (plan.read_nseg != 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "decoder prompt: the post-append window must be one segment (got %d)", plan.read_nseg);
    if (pos0 + n_tokens > (1 << 24))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: rope position beyond 2^24");
    const int64_t bb = kq_block_bytes(m.tok_embeddings_type);
    if (!bb) return fail(VKV_STATUS_INVALID_ARGUMENT, "decoder prompt: embedding dtype");
    const int32_t qd = m.n_q_heads * m.head_dim, kd = m.n_kv_heads * m.head_dim;
    const float scale = 1.0f / std::sqrt((float)m.head_dim);
    DeviceGuard guard(cache->p.device);
    void *hs = hip_stream;
    hipStream_t st = as_stream(hs);
    // token rows + audio rows, kEmbedChunk tokens per launch (ids in the
    // kernel arguments); the first launch also clears the argmax words
    for (int32_t c0 = 0; c0 < n_tokens; c0 += kEmbedChunk) {
        const int32_t nc = std::min<int32_t>(kEmbedChunk, n_tokens - c0);
        EmbedTokens tok{};
        std::memcpy(tok.id, tokens + c0, (size_t)nc * sizeof(int32_t));
        const int add_ring = audio_emb ? audio_emb->capacity : 0;
        const int add_row0 = audio_emb ? (int)((pos0 + c0) % audio_emb->capacity) : 0;
        hipError_t e = launch_embed_rows(m.tok_embeddings_type, (const uint8_t *)m.tok_embeddings,
                                         (m.dim / 256) * bb, tok, nc, m.dim,
                                         audio_emb ? audio_emb->rows : nullptr, add_ring, add_row0,
                                         t.x + (size_t)c0 * m.dim, st, c0 == 0 ? t.amax : nullptr);
        if (e != hipSuccess) return hip_fail(e, "decoder prompt: embedding launch");
    }
    for (int32_t l = 0; l < m.n_layers; ++l) {
        const vkv_dec_layer &L = m.layers[l];
        const vkv_mm_out qkv[3] = {{L.attn_q, L.attn_q_type, qd, t.q, nullptr, nullptr},
                                   {L.attn_k, L.attn_k_type, kd, t.k, nullptr, nullptr},
                                   {L.attn_v, L.attn_v_type, kd, t.v, nullptr, nullptr}};
        MmRope rope;
        rope.mask = 3u;
        rope.head_dim = m.head_dim;
        rope.pos0 = pos0;
        rope.theta = m.rope_theta;
        if (vkv_status s = matmul_impl(t.x, n_tokens, m.dim, L.attn_norm, nullptr, nullptr,
                                       m.norm_eps, qkv, 3, VKV_MV_STORE, t.image, t.image_bytes, hs,
                                       RowMap{}, RowMap{}, rope))
            return s;
        // causal attention over the retained keys, appending this layer's rows
        if (vkv_status s = do_window(cache, stream, l, 1, plan.read_seg, plan.read_nseg,
                                     plan.oldest_after, plan.absolute_start, n_tokens, 0, t.q, t.attn,
                                     m.n_q_heads, scale, st, t.k, t.v, plan.write_seg,
                                     plan.write_nseg))
            return s;
        const vkv_mm_out o[1] = {{L.attn_o, L.attn_o_type, m.dim, t.x, t.x, nullptr}};
        if (vkv_status s = vkv_matmul(t.attn, n_tokens, qd, nullptr, nullptr, nullptr, m.norm_eps, o,
                                      1, VKV_MV_STORE, t.image, t.image_bytes, hs))
            return s;
        const vkv_mm_out gu[2] = {{L.ffn_w1, L.ffn_w1_type, m.hidden, t.ffn, nullptr, nullptr},
                                  {L.ffn_w3, L.ffn_w3_type, m.hidden, nullptr, nullptr, nullptr}};
        if (vkv_status s = vkv_matmul(t.x, n_tokens, m.dim, L.ffn_norm, nullptr, L.ada_scale,
                                      m.norm_eps, gu, 2, VKV_MV_SWIGLU, t.image, t.image_bytes, hs))
            return s;
        const vkv_mm_out down[1] = {{L.ffn_w2, L.ffn_w2_type, m.dim, t.x, t.x, nullptr}};
        if (vkv_status s = vkv_matmul(t.ffn, n_tokens, m.hidden, nullptr, nullptr, nullptr,
                                      m.norm_eps, down, 1, VKV_MV_STORE, t.image, t.image_bytes, hs))
            return s;
    }
    // the final norm and the logits of the last token only (:2950-2955)
    const vkv_mv_out head[1] = {{m.output, m.output_type, m.vocab, logits, nullptr}};
    if (vkv_status s = matvec_impl(t.x + (size_t)(n_tokens - 1) * m.dim, m.dim, m.out_norm, nullptr,
                                   m.norm_eps, head, 1, VKV_MV_STORE, hs, t.amax, token_out))
        return s;
    vkv_decoder_commit(ring, &plan);
    if (plan_out) *plan_out = plan;
    return ok();
}

// ---- the encoder conv stem ----

namespace {

// compute_causal_conv1d_dims (src/voxtral.cpp:1670-1687)
struct ConvDims {
    int32_t pad_left, pad_right, padded_len, out_len;
};
ConvDims causal_conv1d_dims(int32_t in_len, int32_t kernel, int32_t stride) {
    ConvDims d{0, 0, 0, 0};
    if (in_len <= 0 || kernel <= 0 || stride <= 0) return d;
    const int32_t padding_total = kernel - stride;
    const float n_frames = ((float)(in_len - kernel + padding_total) / (float)stride) + 1.0f;
    const int32_t target = ((int32_t)std::ceil(n_frames) - 1) * stride + (kernel - padding_total);
    d.pad_left = padding_total;
    d.pad_right = std::max<int32_t>(0, target - in_len);
    d.padded_len = in_len + d.pad_left + d.pad_right;
    d.out_len = (d.padded_len - kernel) / stride + 1;
    return d;
}

struct ConvBuffers {
    void *cols0;
    float *y0;
    void *cols1;
    size_t bytes;
};
ConvBuffers conv_buffers(int32_t conv_len, int32_t n_mel, int32_t dim, int32_t n_new, uint8_t *base) {
    ConvBuffers b{};
    size_t off = 0;
    auto take = [&](size_t n) {
        uint8_t *p = base ? base + off : nullptr;
        off += (n + 255) & ~(size_t)255;
        return p;
    };
    b.cols0 = take((size_t)conv_len * n_mel * 3 * 2);
    b.y0 = (float *)take((size_t)conv_len * dim * 4);
    b.cols1 = take((size_t)n_new * dim * 3 * 2);
    b.bytes = off;
    return b;
}

}  // namespace

size_t vkv_enc_conv_stem_workspace(int32_t conv_len, int32_t n_mel, int32_t dim, int32_t n_new) {
    if (conv_len < 1 || n_mel < 1 || dim < 1 || n_new < 1) return 0;
    return conv_buffers(conv_len, n_mel, dim, n_new, nullptr).bytes;
}

vkv_status vkv_enc_conv_stem(const float *mel, int32_t n_mel, const vkv_enc_plan *plan,
                             const void *conv0_w, const float *conv0_b, const void *conv1_w,
                             const float *conv1_b, int32_t dim, float *x, void *workspace,
                             size_t workspace_bytes, void *hip_stream) {
    if (!mel || !plan || !conv0_w || !conv0_b || !conv1_w || !conv1_b || !x || !workspace)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "conv stem: null argument");
    if (n_mel < 1 || (n_mel * 3) % 32 || dim < 16 || (dim * 3) % 32 || dim % 16)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "conv stem: n_mel %d / dim %d unsupported", n_mel, dim);
    const int64_t conv_len64 = plan->conv_mel_end - plan->conv_mel_start;
    if (conv_len64 < 1 || conv_len64 > (1 << 20) || plan->n_new < 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "conv stem: empty or oversized Mel window");
    const int32_t conv_len = (int32_t)conv_len64, n = plan->n_new;
    const ConvDims d0 = causal_conv1d_dims(conv_len, 3, 1);
    const ConvDims d1 = causal_conv1d_dims(d0.out_len, 3, 2);
    if (plan->conv_slice_start < 0 || plan->conv_slice_start + n > d1.out_len)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "conv stem: frames [%d, +%d) outside the %d conv outputs of the window",
                    plan->conv_slice_start, n, d1.out_len);
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "conv stem: workspace not 256-byte aligned");
    if ((reinterpret_cast<uintptr_t>(conv0_w) | reinterpret_cast<uintptr_t>(conv1_w)) & 15u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "conv stem: weights must be 16-byte aligned");
    const ConvBuffers b = conv_buffers(conv_len, n_mel, dim, n, (uint8_t *)workspace);
    if (workspace_bytes < b.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "conv stem: workspace %zu < %zu bytes",
                    workspace_bytes, b.bytes);
    hipStream_t st = as_stream(hip_stream);
    hipError_t e;
    // conv0 over the whole window: Mel is [bin][frame]
    if ((e = launch_im2col_f16(mel, conv_len, 1, conv_len, n_mel, 1, d0.pad_left, 0, d0.out_len,
                               b.cols0, st)) != hipSuccess ||
        (e = launch_gemm_f16(conv0_w, b.cols0, conv0_b, b.y0, dim, d0.out_len, n_mel * 3, true, st)) !=
            hipSuccess)
        return hip_fail(e, "conv stem: conv0 launch");
    // conv1 at the sliced frames only: y0 is [frame][channel]
    if ((e = launch_im2col_f16(b.y0, 1, dim, d0.out_len, dim, 2, d1.pad_left, plan->conv_slice_start, n,
                               b.cols1, st)) != hipSuccess ||
        (e = launch_gemm_f16(conv1_w, b.cols1, conv1_b, x, dim, n, dim * 3, true, st)) != hipSuccess)
        return hip_fail(e, "conv stem: conv1 launch");
    return ok();
}

// ---- one encoder chunk ----

namespace {

struct EncBuffers {
    float *qk, *v, *attn, *ffn;   // qk: q rows [n_new][qd] then k rows [n_new][kvd]
    uint8_t *image;               // vkv_matmul workspace
    size_t image_bytes, bytes;
};

EncBuffers enc_buffers(const vkv_enc_model &m, int32_t kvd, int32_t n_new, uint8_t *base) {
    EncBuffers t{};
    size_t off = 0;
    auto take = [&](size_t b) {
        uint8_t *p = base ? base + off : nullptr;
        off += (b + 255) & ~(size_t)255;
        return p;
    };
    const size_t rows = (size_t)n_new, qd = (size_t)m.n_heads * m.head_dim;
    t.qk = (float *)take(rows * (qd + (size_t)kvd) * 4);
    t.v = (float *)take(rows * (size_t)kvd * 4);
    t.attn = (float *)take(rows * qd * 4);
    t.ffn = (float *)take(rows * m.hidden * 4);
    t.image_bytes = std::max({vkv_matmul_workspace(n_new, m.dim), vkv_matmul_workspace(n_new, (int64_t)qd),
                              vkv_matmul_workspace(n_new, m.hidden)});
    t.image = take(t.image_bytes);
    t.bytes = off;
    return t;
}

vkv_status check_enc_model(const vkv_enc_model *m) {
    if (!m || !m->layers || m->n_layers < 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: null model or no layers");
    const int64_t qd = (int64_t)m->n_heads * m->head_dim;
    if (m->dim < 256 || m->dim % 256 || m->hidden < 256 || m->hidden % 256 ||
        m->hidden > VKV_MV_MAX_IN || m->dim > VKV_MV_MAX_IN || m->n_heads < 1 ||
        m->head_dim < 8 || qd % 256 || qd > VKV_MV_MAX_IN)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: model dimensions");
    if (!m->out_norm) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: null output norm");
    for (int32_t l = 0; l < m->n_layers; ++l) {
        const vkv_enc_layer &L = m->layers[l];
        if (!L.attn_norm || !L.ffn_norm || !L.attn_q || !L.attn_k || !L.attn_v || !L.attn_o ||
            !L.ffn_w1 || !L.ffn_w2 || !L.ffn_w3)
            return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: layer %d has a null tensor", l);
    }
    return VKV_STATUS_OK;
}

}  // namespace

size_t vkv_encoder_chunk_workspace(const vkv_enc_model *model, int32_t n_new) {
    if (check_enc_model(model) || n_new < 1) return 0;
    // the K/V width is the cache's; an MHA encoder's equals the query width
    return enc_buffers(*model, model->n_heads * model->head_dim, n_new, nullptr).bytes;
}

namespace {

// vkv_encoder_chunk; with out_ring the final norm's rows go to its logical
// rows q_start.. instead of x
vkv_status encoder_chunk_impl(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                              int32_t window, const vkv_enc_model *model, float *x,
                              vkv_row_ring *out_ring, void *workspace, size_t workspace_bytes,
                              void *hip_stream) {
    if (vkv_status st = check_enc_model(model)) return st;
    const vkv_enc_model &m = *model;
    if (vkv_status st = check_cache(cache, "encoder chunk")) return st;
    if (!plan || !x || !workspace)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: null argument");
    const int32_t qd = m.n_heads * m.head_dim, kvd = cache->p.n_kv_heads * cache->p.head_dim;
    if (m.n_layers != cache->p.n_layers || m.head_dim != cache->p.head_dim ||
        m.n_heads > cache->p.n_q_heads || kvd % 256 || kvd > qd)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: model and cache shapes differ");
    const int32_t N = plan->n_new;
    if (N < 1) return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: empty plan");
    if (plan->q_start + N > (1 << 24))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: rope position beyond 2^24");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: workspace not 256-byte aligned");
    if (vkv_status st = check_aligned("encoder chunk", {x})) return st;
    const EncBuffers t = enc_buffers(m, kvd, N, (uint8_t *)workspace);
    if (workspace_bytes < t.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "encoder chunk: workspace %zu < %zu bytes",
                    workspace_bytes, t.bytes);
    const float scale = 1.0f / std::sqrt((float)m.head_dim);
    float *q = t.qk, *k = t.qk + (size_t)N * qd;
    for (int32_t l = 0; l < m.n_layers; ++l) {
        const vkv_enc_layer &L = m.layers[l];
        const vkv_mm_out qkv[3] = {{L.attn_q, L.attn_q_type, qd, q, nullptr, L.attn_q_b},
                                   {L.attn_k, L.attn_k_type, kvd, k, nullptr, nullptr},
                                   {L.attn_v, L.attn_v_type, kvd, t.v, nullptr, L.attn_v_b}};
        // RoPE of the q and k rows at positions q_start + r, in the
        // products' epilogue (vkv_rope's arithmetic, so the same bits)
        MmRope rope;
        rope.mask = 3u;
        rope.head_dim = m.head_dim;
        rope.pos0 = plan->q_start;
        rope.theta = m.rope_theta;
        if (vkv_status s = matmul_impl(x, N, m.dim, L.attn_norm, L.attn_norm_b, nullptr, m.norm_eps,
                                       qkv, 3, VKV_MV_STORE, t.image, t.image_bytes, hip_stream,
                                       RowMap{}, RowMap{}, rope))
            return s;
        if (vkv_status s = vkv_enc_step(cache, stream, plan, window, l, 1, q, k, t.v, t.attn,
                                        m.n_heads, scale, hip_stream))
            return s;
        const vkv_mm_out o[1] = {{L.attn_o, L.attn_o_type, m.dim, x, x, L.attn_o_b}};
        if (vkv_status s = vkv_matmul(t.attn, N, qd, nullptr, nullptr, nullptr, m.norm_eps, o, 1,
                                      VKV_MV_STORE, t.image, t.image_bytes, hip_stream))
            return s;
        const vkv_mm_out gu[2] = {{L.ffn_w1, L.ffn_w1_type, m.hidden, t.ffn, nullptr, nullptr},
                                  {L.ffn_w3, L.ffn_w3_type, m.hidden, nullptr, nullptr, nullptr}};
        if (vkv_status s = vkv_matmul(x, N, m.dim, L.ffn_norm, L.ffn_norm_b, nullptr, m.norm_eps, gu,
                                      2, VKV_MV_SWIGLU, t.image, t.image_bytes, hip_stream))
            return s;
        const vkv_mm_out down[1] = {{L.ffn_w2, L.ffn_w2_type, m.dim, x, x, L.ffn_w2_b}};
        if (vkv_status s = vkv_matmul(t.ffn, N, m.hidden, nullptr, nullptr, nullptr, m.norm_eps,
                                      down, 1, VKV_MV_STORE, t.image, t.image_bytes, hip_stream))
            return s;
    }
    if (vkv_status st = check_aligned("encoder chunk", {m.out_norm, m.out_norm_b})) return st;
    hipError_t e = out_ring ? launch_rms_norm_rows(x, N, m.dim, m.out_norm, m.out_norm_b, m.norm_eps,
                                                   out_ring->rows, out_ring->capacity,
                                                   (int)(plan->q_start % out_ring->capacity),
                                                   as_stream(hip_stream))
                            : launch_rms_norm_rows(x, N, m.dim, m.out_norm, m.out_norm_b, m.norm_eps,
                                                   x, 0, 0, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "encoder chunk: final norm launch");
    return ok();
}
}  // namespace

vkv_status vkv_encoder_chunk(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                             int32_t window, const vkv_enc_model *model, float *x,
                             void *workspace, size_t workspace_bytes, void *hip_stream) {
    return encoder_chunk_impl(cache, stream, plan, window, model, x, nullptr, workspace,
                              workspace_bytes, hip_stream);
}

vkv_status vkv_encoder_chunk_ring(vkv_cache *cache, int32_t stream, const vkv_enc_plan *plan,
                                  int32_t window, const vkv_enc_model *model, float *x,
                                  vkv_row_ring *enc_out, void *workspace, size_t workspace_bytes,
                                  void *hip_stream) {
    if (vkv_status st = check_row_ring(enc_out, "encoder chunk")) return st;
    if (model && enc_out->width != model->dim)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "encoder chunk: ring width %d != dim %d",
                    enc_out->width, model->dim);
    if (plan && (plan->n_new > enc_out->capacity || plan->q_start < 0))
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "encoder chunk: %d new frames do not fit a ring of %d rows", plan->n_new,
                    enc_out->capacity);
    return encoder_chunk_impl(cache, stream, plan, window, model, x, enc_out, workspace,
                              workspace_bytes, hip_stream);
}

// ---- the realtime rows rings and the adapter ----

vkv_status vkv_row_ring_write(vkv_row_ring *ring, int64_t row_start, const float *src,
                              int32_t n_rows, void *hip_stream) {
    if (vkv_status st = check_row_ring(ring, "ring write")) return st;
    if (!src || row_start < 0 || n_rows < 0 || n_rows > ring->capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ring write: rows [%lld, +%d) on a ring of %d",
                    (long long)row_start, n_rows, ring->capacity);
    const size_t rb = (size_t)ring->width * sizeof(float);
    int32_t done = 0;
    while (done < n_rows) {
        const int32_t slot = (int32_t)((row_start + done) % ring->capacity);
        const int32_t seg = std::min(n_rows - done, ring->capacity - slot);
        hipError_t e = hipMemcpyAsync((uint8_t *)ring->rows + (size_t)slot * rb,
                                      (const uint8_t *)src + (size_t)done * rb, (size_t)seg * rb,
                                      hipMemcpyDefault, as_stream(hip_stream));
        if (e != hipSuccess) return hip_fail(e, "ring write copy");
        done += seg;
    }
    return ok();
}

vkv_status vkv_row_ring_read(const vkv_row_ring *ring, int64_t row_start, int32_t n_rows,
                             float *dst, void *hip_stream) {
    if (vkv_status st = check_row_ring(ring, "ring read")) return st;
    if (!dst || row_start < 0 || n_rows < 1 || n_rows > ring->capacity)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "ring read: rows [%lld, +%d) on a ring of %d",
                    (long long)row_start, n_rows, ring->capacity);
    const size_t rb = (size_t)ring->width * sizeof(float);
    int32_t done = 0;
    while (done < n_rows) {
        const int32_t slot = (int32_t)((row_start + done) % ring->capacity);
        const int32_t seg = std::min(n_rows - done, ring->capacity - slot);
        hipError_t e = hipMemcpyAsync((uint8_t *)dst + (size_t)done * rb,
                                      (const uint8_t *)ring->rows + (size_t)slot * rb,
                                      (size_t)seg * rb, hipMemcpyDefault, as_stream(hip_stream));
        if (e != hipSuccess) return hip_fail(e, "ring read copy");
        done += seg;
    }
    hipError_t e = hipStreamSynchronize(as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "ring read synchronize");
    return ok();
}

namespace {
// groups per product launch; longer commits run in pieces
constexpr int32_t kAdapterRun = 256;

struct AdapterBuffers {
    float *hidden;     // gelu(W0 x) rows [run][dec_dim]
    uint8_t *image;    // the Q8_K image of either product's input
    size_t image_bytes, bytes;
};

AdapterBuffers adapter_buffers(const vkv_adapter &ad, int32_t run, uint8_t *base) {
    AdapterBuffers t{};
    size_t off = 0;
    auto take = [&](size_t b) {
        uint8_t *p = base ? base + off : nullptr;
        off += (b + 255) & ~(size_t)255;
        return p;
    };
    t.hidden = (float *)take((size_t)run * ad.dec_dim * 4);
    t.image_bytes = run > 1 ? std::max(vkv_matmul_workspace(run, (int64_t)ad.enc_dim * ad.downsample),
                                       vkv_matmul_workspace(run, ad.dec_dim))
                            : 0;
    t.image = t.image_bytes ? take(t.image_bytes) : nullptr;
    t.bytes = off;
    return t;
}

vkv_status check_adapter(const vkv_adapter *ad) {
    if (!ad || !ad->w0 || !ad->w2)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: null weights");
    const int64_t n_in = (int64_t)ad->enc_dim * ad->downsample;
    if (ad->downsample < 1 || ad->enc_dim < 1 || n_in % 256 || n_in > VKV_MV_MAX_IN ||
        ad->dec_dim < 256 || ad->dec_dim % 256 || ad->dec_dim > VKV_MV_MAX_IN)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: dimensions");
    if (!kq_block_bytes(ad->w0_type) || !kq_block_bytes(ad->w2_type))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: weight dtypes %d / %d", ad->w0_type,
                    ad->w2_type);
    return VKV_STATUS_OK;
}
}  // namespace

size_t vkv_adapter_workspace(const vkv_adapter *adapter, int32_t n_groups) {
    if (check_adapter(adapter) || n_groups < 1) return 0;
    return adapter_buffers(*adapter, std::min(n_groups, kAdapterRun), nullptr).bytes;
}

vkv_status vkv_adapter_commit(const vkv_adapter *adapter, const vkv_row_ring *enc_out,
                              vkv_row_ring *audio_emb, int64_t group_start, int32_t n_groups,
                              void *workspace, size_t workspace_bytes, void *hip_stream) {
    if (vkv_status st = check_adapter(adapter)) return st;
    const vkv_adapter &ad = *adapter;
    if (vkv_status st = check_row_ring(enc_out, "adapter")) return st;
    if (vkv_status st = check_row_ring(audio_emb, "adapter")) return st;
    if (enc_out->width != ad.enc_dim || audio_emb->width != ad.dec_dim)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: ring widths %d / %d, model %d / %d",
                    enc_out->width, audio_emb->width, ad.enc_dim, ad.dec_dim);
    if (enc_out->capacity % ad.downsample)
        return fail(VKV_STATUS_INVALID_ARGUMENT,
                    "adapter: encoder ring capacity %d is not a multiple of %d", enc_out->capacity,
                    ad.downsample);
    if (group_start < 0 || n_groups < 1)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: groups [%lld, +%d)",
                    (long long)group_start, n_groups);
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return fail(VKV_STATUS_INVALID_ARGUMENT, "adapter: workspace null or not 256-byte aligned");
    const int32_t run_max = std::min(n_groups, kAdapterRun);
    const AdapterBuffers t = adapter_buffers(ad, run_max, (uint8_t *)workspace);
    if (workspace_bytes < t.bytes)
        return fail(VKV_STATUS_BUFFER_TOO_SMALL, "adapter: workspace %zu < %zu bytes",
                    workspace_bytes, t.bytes);
    // a group's frames are one contiguous row of enc_dim * downsample floats;
    // the encoder ring holds capacity / downsample of them
    const int32_t n_in = ad.enc_dim * ad.downsample, g_ring = enc_out->capacity / ad.downsample;
    int32_t done = 0;
    while (done < n_groups) {
        // a run writes distinct rows of the audio ring, so no two of its
        // groups race for one row (later groups win across runs)
        const int32_t run = std::min({n_groups - done, kAdapterRun, audio_emb->capacity});
        const int64_t g0 = group_start + done;
        const int32_t in_row = (int32_t)(g0 % g_ring), out_row = (int32_t)(g0 % audio_emb->capacity);
        if (run == 1) {
            // one group: two single-row products, input quantization fused
            const vkv_mv_out h[1] = {{ad.w0, ad.w0_type, ad.dec_dim, t.hidden, nullptr}};
            if (vkv_status s = matvec_impl(enc_out->rows + (size_t)in_row * n_in, n_in, nullptr,
                                           nullptr, 0.0f, h, 1, VKV_MV_GELU, hip_stream, nullptr,
                                           nullptr))
                return s;
            const vkv_mv_out y[1] = {{ad.w2, ad.w2_type, ad.dec_dim,
                                      audio_emb->rows + (size_t)out_row * ad.dec_dim, nullptr}};
            if (vkv_status s = matvec_impl(t.hidden, ad.dec_dim, nullptr, nullptr, 0.0f, y, 1,
                                           VKV_MV_STORE, hip_stream, nullptr, nullptr))
                return s;
        } else {
            const vkv_mm_out h[1] = {{ad.w0, ad.w0_type, ad.dec_dim, t.hidden, nullptr, nullptr}};
            if (vkv_status s = matmul_impl(enc_out->rows, run, n_in, nullptr, nullptr, nullptr, 0.0f,
                                           h, 1, VKV_MV_GELU, t.image, t.image_bytes, hip_stream,
                                           RowMap{g_ring, in_row}, RowMap{}))
                return s;
            const vkv_mm_out y[1] = {{ad.w2, ad.w2_type, ad.dec_dim, audio_emb->rows, nullptr, nullptr}};
            if (vkv_status s = matmul_impl(t.hidden, run, ad.dec_dim, nullptr, nullptr, nullptr, 0.0f,
                                           y, 1, VKV_MV_STORE, t.image, t.image_bytes, hip_stream,
                                           RowMap{}, RowMap{audio_emb->capacity, out_row}))
                return s;
        }
        done += run;
    }
    return ok();
}

vkv_status vkv_synth_rows(float *dst, int32_t row_len, uint64_t seed, uint32_t tag, int64_t s0,
                          int32_t ns, int64_t s_stride, int64_t l0, int32_t nl, int64_t l_stride,
                          int64_t p0, int32_t np, int64_t p_stride, void *hip_stream) {
    if (row_len < 0 || ns < 0 || nl < 0 || np < 0)
        return fail(VKV_STATUS_INVALID_ARGUMENT, "synth: negative extent");
    if ((int64_t)row_len * ns * nl * np == 0) return ok();
    if (!dst) return fail(VKV_STATUS_INVALID_ARGUMENT, "synth: null destination");
    hipError_t e = launch_synth(dst, row_len, seed, tag, s0, ns, s_stride, l0, nl, l_stride, p0, np,
                                p_stride, as_stream(hip_stream));
    if (e != hipSuccess) return hip_fail(e, "synth launch");
    return ok();
}

}  // extern "C"
