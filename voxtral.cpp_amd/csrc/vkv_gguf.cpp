// GGUF model files: the reader behind voxtral_model_load_from_file
// (src/voxtral.cpp:1035-1316) and the model's upload into one device
// allocation.
//
// The format is GGUF v2/v3 as ggml's gguf reader (ggml @ 5cecdad6,
// gguf.cpp; not in the reference tree) accepts it and as
// tools/convert_voxtral_to_gguf.py:839-905 writes it: "GGUF", u32 version,
// u64 tensor count, u64 key count, typed key/value pairs, tensor infos
// (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset), then
// the data section at the alignment (general.alignment, default 32), every
// tensor at the running packed offset rounded up to the alignment.  The
// checks are ggml's: version 1 and versions above 3 rejected, duplicate keys
// and tensor names rejected, at most 4 dims, ne[0] a multiple of the type's
// block, offsets equal to the packed layout, everything inside the file.
//
// The model is uploaded as the data section verbatim: one device allocation,
// each tensor at its file offset (32-byte aligned there, so every f32 vector
// is 16-byte aligned and every weight row starts where the kernels expect),
// streamed through three pinned staging buffers so that reading the file
// (several host threads) and the host-to-device copies overlap.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "vkv.h"
#include "vkv_internal.h"

namespace {

vkv_status gfail(vkv_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return vkv::host_fail(st, buf);
}

// ggml type -> (elements per block, bytes per block); 0 for types a voxtral
// file never holds
struct TypeSize {
    int64_t blck, bytes;
};
TypeSize type_size(uint32_t t) {
    switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 9: return {32, 36};     // Q8_1
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 24: return {1, 1};      // I8
    case 25: return {1, 2};      // I16
    case 26: return {1, 4};      // I32
    case 27: return {1, 8};      // I64
    case 28: return {1, 8};      // F64
    case 30: return {1, 2};      // BF16
    default: return {0, 0};
    }
}

int64_t scalar_size(uint32_t t) {
    switch (t) {
    case VKV_GGUF_UINT8: case VKV_GGUF_INT8: case VKV_GGUF_BOOL: return 1;
    case VKV_GGUF_UINT16: case VKV_GGUF_INT16: return 2;
    case VKV_GGUF_UINT32: case VKV_GGUF_INT32: case VKV_GGUF_FLOAT32: return 4;
    case VKV_GGUF_UINT64: case VKV_GGUF_INT64: case VKV_GGUF_FLOAT64: return 8;
    default: return 0;
    }
}

struct KV {
    std::string key;
    uint32_t type = 0, arr_type = 0;
    uint64_t n = 0;                  // array length
    const uint8_t *val = nullptr;    // scalar / array elements in the file
    std::string str;                 // string value
    std::vector<std::string> strs;   // string array
};

struct TensorInfo {
    std::string name;
    vkv_gguf_tensor t{};
};

// bounds-checked little-endian reader over the mapped file
struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    bool take(void *dst, size_t n) {
        if (!ok || (size_t)(end - p) < n) return ok = false;
        std::memcpy(dst, p, n);
        p += n;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    bool str(std::string &s) {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t)(end - p)) return ok = false;
        s.assign((const char *)p, (size_t)n);
        p += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!ok || n > (uint64_t)(end - p)) return ok = false;
        p += n;
        return true;
    }
};

}  // namespace

struct vkv_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0, data_size = 0;
    std::vector<KV> kv;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, int64_t> kv_index, tensor_index;
    ~vkv_gguf() {
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

vkv_status parse(vkv_gguf &g) {
    Cursor c{g.map, g.map + g.size};
    char magic[4];
    if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0)
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: bad magic");
    g.version = c.get<uint32_t>();
    if (!c.ok) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated header");
    if (g.version == 1) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: version 1 is not supported");
    if (g.version == 0 || g.version > 3)
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: unknown version %u", g.version);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated header");
    // every key/value takes at least 12 bytes and every tensor info 24
    if (n_kv > g.size / 12 || n_tensors > g.size / 24)
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: %llu keys / %llu tensors exceed the file",
                     (unsigned long long)n_kv, (unsigned long long)n_tensors);
    g.kv.resize(n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        KV &kv = g.kv[i];
        if (!c.str(kv.key)) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated key %llu", (unsigned long long)i);
        kv.type = c.get<uint32_t>();
        if (!c.ok) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated key %s", kv.key.c_str());
        if (kv.type == VKV_GGUF_STRING) {
            if (!c.str(kv.str)) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated value of %s", kv.key.c_str());
        } else if (kv.type == VKV_GGUF_ARRAY) {
            kv.arr_type = c.get<uint32_t>();
            kv.n = c.get<uint64_t>();
            if (!c.ok) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated array %s", kv.key.c_str());
            if (kv.arr_type == VKV_GGUF_STRING) {
                if (kv.n > (uint64_t)(c.end - c.p) / 8)
                    return gfail(VKV_STATUS_MODEL_ERROR, "gguf: array %s exceeds the file", kv.key.c_str());
                kv.strs.resize(kv.n);
                for (uint64_t j = 0; j < kv.n; ++j)
                    if (!c.str(kv.strs[j]))
                        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated array %s", kv.key.c_str());
            } else {
                const int64_t es = scalar_size(kv.arr_type);
                if (!es) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: array %s of type %u", kv.key.c_str(), kv.arr_type);
                if (kv.n > (uint64_t)(c.end - c.p) / (uint64_t)es)
                    return gfail(VKV_STATUS_MODEL_ERROR, "gguf: array %s exceeds the file", kv.key.c_str());
                kv.val = c.p;
                c.skip(kv.n * (uint64_t)es);
            }
        } else {
            const int64_t es = scalar_size(kv.type);
            if (!es) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: key %s has type %u", kv.key.c_str(), kv.type);
            kv.val = c.p;
            if (!c.skip((uint64_t)es)) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated value of %s", kv.key.c_str());
        }
        if (!g.kv_index.emplace(kv.key, (int64_t)i).second)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: duplicate key %s", kv.key.c_str());
    }
    auto al = g.kv_index.find("general.alignment");
    if (al != g.kv_index.end()) {
        const KV &kv = g.kv[al->second];
        uint32_t a = 0;
        if (kv.type != VKV_GGUF_UINT32) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: general.alignment is not a u32");
        std::memcpy(&a, kv.val, 4);
        if (a == 0 || (a & (a - 1)) != 0)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: alignment %u is not a power of two", a);
        g.alignment = a;
    }
    g.tensors.resize(n_tensors);
    uint64_t packed = 0;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo &ti = g.tensors[i];
        if (!c.str(ti.name)) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated tensor info %llu", (unsigned long long)i);
        if (ti.name.size() >= 64)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor name %s longer than 63 bytes", ti.name.c_str());
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd > 4) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s has %u dims", ti.name.c_str(), nd);
        ti.t.n_dims = (int32_t)nd;
        int64_t elems = 1;
        for (int d = 0; d < 4; ++d) ti.t.ne[d] = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t ne = c.get<uint64_t>();
            if (ne > (uint64_t)INT64_MAX) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s dim %u", ti.name.c_str(), d);
            ti.t.ne[d] = (int64_t)ne;
            if (ne != 0 && elems > INT64_MAX / (int64_t)ne)
                return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s too large", ti.name.c_str());
            elems *= (int64_t)ne;
        }
        const uint32_t type = c.get<uint32_t>();
        const uint64_t off = c.get<uint64_t>();
        if (!c.ok) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: truncated tensor info %s", ti.name.c_str());
        const TypeSize ts = type_size(type);
        if (!ts.blck) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s has ggml type %u", ti.name.c_str(), type);
        if (ti.t.ne[0] % ts.blck)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s: ne[0]=%lld not a multiple of %lld",
                         ti.name.c_str(), (long long)ti.t.ne[0], (long long)ts.blck);
        ti.t.type = (int32_t)type;
        ti.t.offset = off;
        // sizes checked before every product and sum, so a tensor claiming
        // ~2^62 elements cannot wrap its byte count, its padding or the end
        // check below
        const uint64_t nblocks = (uint64_t)(elems / ts.blck);
        if (nblocks > (UINT64_MAX - g.alignment) / (uint64_t)ts.bytes)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s too large", ti.name.c_str());
        ti.t.nbytes = nblocks * (uint64_t)ts.bytes;
        if (off != packed)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s has offset %llu, expected %llu",
                         ti.name.c_str(), (unsigned long long)off, (unsigned long long)packed);
        const uint64_t padded = (ti.t.nbytes + g.alignment - 1) / g.alignment * g.alignment;
        if (padded > UINT64_MAX - packed) return gfail(VKV_STATUS_MODEL_ERROR, "gguf: data section too large");
        packed += padded;
        if (!g.tensor_index.emplace(ti.name, (int64_t)i).second)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: duplicate tensor %s", ti.name.c_str());
    }
    for (auto &ti : g.tensors) ti.t.name = ti.name.c_str();
    const uint64_t meta_end = (uint64_t)(c.p - g.map);
    g.data_offset = (meta_end + g.alignment - 1) / g.alignment * g.alignment;
    g.data_size = packed;
    // every tensor's bytes inside the file (the last one may end unpadded)
    for (const auto &ti : g.tensors)
        if (g.data_offset > g.size || ti.t.offset > g.size - g.data_offset ||
            ti.t.nbytes > g.size - g.data_offset - ti.t.offset)
            return gfail(VKV_STATUS_MODEL_ERROR, "gguf: tensor %s extends past the end of the file",
                         ti.name.c_str());
    return VKV_STATUS_OK;
}

const KV *kv_at(const vkv_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->kv.size()) return nullptr;
    return &g->kv[(size_t)i];
}

template <class T>
vkv_status get_scalar(const vkv_gguf *g, int64_t i, uint32_t type, T *out, const char *what) {
    const KV *kv = kv_at(g, i);
    if (!kv || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: %s: no key %lld", what, (long long)i);
    if (kv->type != type)
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: %s: key %s has type %u", what, kv->key.c_str(), kv->type);
    std::memcpy(out, kv->val, sizeof(T));
    return vkv::host_ok();
}

}  // namespace

extern "C" {

vkv_status vkv_gguf_open(const char *path, vkv_gguf **out) {
    if (out) *out = nullptr;
    if (!path || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: null argument");
    vkv_gguf *g = new (std::nothrow) vkv_gguf();
    if (!g) return gfail(VKV_STATUS_OUT_OF_MEMORY, "gguf: out of memory");
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st {};
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        delete g;
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: cannot open %s", path);
    }
    g->size = (size_t)st.st_size;
    if (g->size < 24) {
        delete g;
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: %s is too short (%zu bytes)", path, (size_t)st.st_size);
    }
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return gfail(VKV_STATUS_MODEL_ERROR, "gguf: cannot map %s", path);
    }
    g->map = (const uint8_t *)m;
    if (vkv_status s = parse(*g)) {
        delete g;
        return s;
    }
    *out = g;
    return vkv::host_ok();
}

vkv_status vkv_gguf_close(vkv_gguf *gguf) {
    delete gguf;
    return vkv::host_ok();
}

uint32_t vkv_gguf_version(const vkv_gguf *g) { return g ? g->version : 0; }
uint64_t vkv_gguf_alignment(const vkv_gguf *g) { return g ? g->alignment : 0; }
uint64_t vkv_gguf_data_offset(const vkv_gguf *g) { return g ? g->data_offset : 0; }
int64_t vkv_gguf_n_kv(const vkv_gguf *g) { return g ? (int64_t)g->kv.size() : 0; }

int64_t vkv_gguf_find_key(const vkv_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : it->second;
}

const char *vkv_gguf_key(const vkv_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return kv ? kv->key.c_str() : nullptr;
}

int32_t vkv_gguf_kv_type(const vkv_gguf *g, int64_t i) {
    const KV *kv = kv_at(g, i);
    return kv ? (int32_t)kv->type : -1;
}

vkv_status vkv_gguf_get_i32(const vkv_gguf *g, int64_t i, int32_t *out) {
    return get_scalar(g, i, VKV_GGUF_INT32, out, "get_i32");
}
vkv_status vkv_gguf_get_u32(const vkv_gguf *g, int64_t i, uint32_t *out) {
    return get_scalar(g, i, VKV_GGUF_UINT32, out, "get_u32");
}
vkv_status vkv_gguf_get_i64(const vkv_gguf *g, int64_t i, int64_t *out) {
    return get_scalar(g, i, VKV_GGUF_INT64, out, "get_i64");
}
vkv_status vkv_gguf_get_f32(const vkv_gguf *g, int64_t i, float *out) {
    return get_scalar(g, i, VKV_GGUF_FLOAT32, out, "get_f32");
}
vkv_status vkv_gguf_get_f64(const vkv_gguf *g, int64_t i, double *out) {
    return get_scalar(g, i, VKV_GGUF_FLOAT64, out, "get_f64");
}
vkv_status vkv_gguf_get_bool(const vkv_gguf *g, int64_t i, int32_t *out) {
    uint8_t b = 0;
    if (!out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_bool: null output");
    if (vkv_status s = get_scalar(g, i, VKV_GGUF_BOOL, &b, "get_bool")) return s;
    *out = b != 0;
    return VKV_STATUS_OK;
}

vkv_status vkv_gguf_get_scalar(const vkv_gguf *g, int64_t i, void *out, uint64_t out_bytes) {
    const KV *kv = kv_at(g, i);
    if (!kv || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_scalar: no key %lld", (long long)i);
    const int64_t n = scalar_size(kv->type);
    if (!n || kv->type == VKV_GGUF_ARRAY)
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_scalar: key %s is not a scalar", kv->key.c_str());
    if (out_bytes < (uint64_t)n)
        return gfail(VKV_STATUS_BUFFER_TOO_SMALL, "gguf: get_scalar: %llu < %lld bytes",
                     (unsigned long long)out_bytes, (long long)n);
    std::memcpy(out, kv->val, (size_t)n);
    return vkv::host_ok();
}

vkv_status vkv_gguf_get_str(const vkv_gguf *g, int64_t i, const char **out, uint64_t *len) {
    const KV *kv = kv_at(g, i);
    if (!kv || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_str: no key %lld", (long long)i);
    if (kv->type != VKV_GGUF_STRING)
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_str: key %s has type %u", kv->key.c_str(), kv->type);
    *out = kv->str.c_str();
    if (len) *len = kv->str.size();
    return vkv::host_ok();
}

vkv_status vkv_gguf_get_arr(const vkv_gguf *g, int64_t i, int32_t *elem_type, uint64_t *n,
                            const void **data) {
    const KV *kv = kv_at(g, i);
    if (!kv) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_arr: no key %lld", (long long)i);
    if (kv->type != VKV_GGUF_ARRAY)
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_arr: key %s has type %u", kv->key.c_str(), kv->type);
    if (elem_type) *elem_type = (int32_t)kv->arr_type;
    if (n) *n = kv->n;
    if (data) *data = kv->arr_type == VKV_GGUF_STRING ? nullptr : kv->val;
    return vkv::host_ok();
}

vkv_status vkv_gguf_get_arr_str(const vkv_gguf *g, int64_t i, uint64_t j, const char **out,
                                uint64_t *len) {
    const KV *kv = kv_at(g, i);
    if (!kv || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_arr_str: no key %lld", (long long)i);
    if (kv->type != VKV_GGUF_ARRAY || kv->arr_type != VKV_GGUF_STRING)
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_arr_str: key %s is not a string array", kv->key.c_str());
    if (j >= kv->n) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: get_arr_str: index %llu of %llu",
                                 (unsigned long long)j, (unsigned long long)kv->n);
    *out = kv->strs[j].c_str();
    if (len) *len = kv->strs[j].size();
    return vkv::host_ok();
}

int64_t vkv_gguf_n_tensors(const vkv_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t vkv_gguf_find_tensor(const vkv_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : it->second;
}

vkv_status vkv_gguf_tensor_info(const vkv_gguf *g, int64_t i, vkv_gguf_tensor *out) {
    if (out) std::memset(out, 0, sizeof(*out));
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size())
        return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: tensor_info: no tensor %lld", (long long)i);
    *out = g->tensors[(size_t)i].t;
    return vkv::host_ok();
}

const void *vkv_gguf_tensor_data(const vkv_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
    return g->map + g->data_offset + g->tensors[(size_t)i].t.offset;
}

vkv_status vkv_gguf_hparams(const vkv_gguf *g, vkv_hparams *out) {
    if (out) std::memset(out, 0, sizeof(*out));
    if (!g || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "gguf: hparams: null argument");
    vkv_hparams hp{};
    // defaults: include/voxtral.h:38-78
    hp.enc_dim = 1280; hp.enc_layers = 32; hp.enc_heads = 32; hp.enc_head_dim = 64;
    hp.enc_hidden = 5120; hp.enc_kv_heads = 32; hp.enc_norm_eps = 1e-5f; hp.enc_rope_theta = 1000000.0f;
    hp.dec_dim = 3072; hp.dec_layers = 26; hp.dec_heads = 32; hp.dec_head_dim = 128;
    hp.dec_hidden = 9216; hp.dec_kv_heads = 8; hp.dec_norm_eps = 1e-5f; hp.dec_rope_theta = 1000000.0f;
    hp.vocab_size = 131072; hp.downsample_factor = 4;
    hp.tok_bos = 1; hp.tok_eos = 2; hp.tok_audio = 24; hp.tok_begin_audio = 25;
    // a key of another type than the reader expects is a model error here
    // (ggml's gguf_get_val_* assert on it)
    vkv_status st = VKV_STATUS_OK;
    auto typed = [&](const char *k, uint32_t type) -> int64_t {
        const int64_t i = vkv_gguf_find_key(g, k);
        if (i < 0 || st) return -1;
        if (g->kv[(size_t)i].type != type) {
            st = gfail(VKV_STATUS_MODEL_ERROR, "gguf: key %s has type %u, expected %u", k,
                       g->kv[(size_t)i].type, type);
            return -1;
        }
        return i;
    };
    auto gi32 = [&](const char *k, int32_t &dst) {
        const int64_t i = typed(k, VKV_GGUF_INT32);
        if (i >= 0) std::memcpy(&dst, g->kv[(size_t)i].val, 4);
    };
    auto gf32 = [&](const char *k, float &dst) {
        const int64_t i = typed(k, VKV_GGUF_FLOAT32);
        if (i >= 0) std::memcpy(&dst, g->kv[(size_t)i].val, 4);
    };
    auto gbool = [&](const char *k, int32_t &dst) {
        const int64_t i = typed(k, VKV_GGUF_BOOL);
        if (i >= 0) dst = g->kv[(size_t)i].val[0] != 0;
    };
    const int64_t arch = typed("general.architecture", VKV_GGUF_STRING);
    if (st) return st;
    if (arch >= 0) hp.is_offline = g->kv[(size_t)arch].str == "voxtral";
    gi32("voxtral.encoder.dim", hp.enc_dim);
    gi32("voxtral.encoder.n_layers", hp.enc_layers);
    gi32("voxtral.encoder.n_heads", hp.enc_heads);
    gi32("voxtral.encoder.head_dim", hp.enc_head_dim);
    gi32("voxtral.encoder.hidden_dim", hp.enc_hidden);
    gi32("voxtral.encoder.n_kv_heads", hp.enc_kv_heads);
    gf32("voxtral.encoder.norm_eps", hp.enc_norm_eps);
    gf32("voxtral.encoder.rope_theta", hp.enc_rope_theta);
    hp.enc_causal = !hp.is_offline;
    gbool("voxtral.encoder.causal", hp.enc_causal);
    gbool("voxtral.params.multimodal.whisper_model_args.encoder_args.causal", hp.enc_causal);
    gi32("voxtral.decoder.dim", hp.dec_dim);
    gi32("voxtral.decoder.n_layers", hp.dec_layers);
    gi32("voxtral.decoder.n_heads", hp.dec_heads);
    gi32("voxtral.decoder.head_dim", hp.dec_head_dim);
    gi32("voxtral.decoder.hidden_dim", hp.dec_hidden);
    gi32("voxtral.decoder.n_kv_heads", hp.dec_kv_heads);
    gf32("voxtral.decoder.norm_eps", hp.dec_norm_eps);
    gf32("voxtral.decoder.rope_theta", hp.dec_rope_theta);
    hp.ada_t_cond = !hp.is_offline;
    gbool("voxtral.ada_rms_norm_t_cond", hp.ada_t_cond);
    gi32("voxtral.vocab_size", hp.vocab_size);
    gi32("voxtral.audio.downsample_factor", hp.downsample_factor);
    gi32("voxtral.token.bos", hp.tok_bos);
    gi32("voxtral.token.eos", hp.tok_eos);
    gi32("voxtral.token.audio", hp.tok_audio);
    gi32("voxtral.token.begin_audio", hp.tok_begin_audio);
    if (st) return st;
    *out = hp;
    return vkv::host_ok();
}

}  // extern "C"

// ---- the model in device memory ----

struct vkv_model {
    vkv_gguf *g = nullptr;
    int device = 0;
    uint8_t *base = nullptr;   // the data section, one allocation
    uint8_t *ada_ws = nullptr; // vkv_ada_scale's workspace, on first use
    vkv_model_view view{};
    std::vector<vkv_enc_layer> enc_layers;
    std::vector<vkv_dec_layer> dec_layers;
    ~vkv_model() {
        if (base) {
            int prev = -1;
            (void)hipGetDevice(&prev);
            (void)hipSetDevice(device);
            (void)hipFree(base);
            if (ada_ws) (void)hipFree(ada_ws);
            if (prev >= 0) (void)hipSetDevice(prev);
        }
        delete g;   // not vkv_gguf_close: a failed load keeps its error message
    }
};

namespace {

constexpr int32_t kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4K = 12, kQ6K = 14;

// Resolves the reference's tensor names against the file; the first problem
// is kept as the load's error.
struct Mapper {
    vkv_model &m;
    std::string err;
    const TensorInfo *info(const std::string &name) {
        const int64_t i = vkv_gguf_find_tensor(m.g, name.c_str());
        return i < 0 ? nullptr : &m.g->tensors[(size_t)i];
    }
    const void *dev(const TensorInfo *ti) { return m.base + ti->t.offset; }
    void miss(const std::string &what) {
        if (err.empty()) err = what;
    }
    // an f32 vector of n elements; optional ones may be absent
    const float *vec(const std::string &name, int64_t n, bool optional = false) {
        const TensorInfo *ti = info(name);
        if (!ti) {
            if (!optional) miss("tensor '" + name + "' not found");
            return nullptr;
        }
        if (ti->t.type != kF32 || ti->t.ne[0] != n || ti->t.nbytes != (uint64_t)n * 4) {
            miss("tensor '" + name + "' is not f32 [" + std::to_string(n) + "]");
            return nullptr;
        }
        return (const float *)dev(ti);
    }
    // a Q4_K / Q6_K / Q8_0 matrix [rows][n_in] (the Q4_K_M mix, or a Q8_0
    // file: src/voxtral-quantize.cpp:95-96)
    const void *mat(const std::string &name, int64_t rows, int64_t n_in, int32_t *type) {
        const TensorInfo *ti = info(name);
        if (!ti) {
            miss("tensor '" + name + "' not found");
            return nullptr;
        }
        if (ti->t.type != kQ4K && ti->t.type != kQ6K && ti->t.type != kQ8_0) {
            miss("tensor '" + name + "' has ggml type " + std::to_string(ti->t.type) +
                 "; the device products take Q4_K, Q6_K and Q8_0");
            return nullptr;
        }
        if (ti->t.n_dims != 2 || ti->t.ne[0] != n_in || ti->t.ne[1] != rows) {
            miss("tensor '" + name + "' is not [" + std::to_string(n_in) + ", " + std::to_string(rows) + "]");
            return nullptr;
        }
        *type = ti->t.type;
        return dev(ti);
    }
    const void *conv(const std::string &name, int64_t in, int64_t out) {
        const TensorInfo *ti = info(name);
        if (!ti) {
            miss("tensor '" + name + "' not found");
            return nullptr;
        }
        if (ti->t.type != kF16 || ti->t.ne[0] != 3 || ti->t.ne[1] != in || ti->t.ne[2] != out) {
            miss("tensor '" + name + "' is not f16 [3, " + std::to_string(in) + ", " + std::to_string(out) + "]");
            return nullptr;
        }
        return dev(ti);
    }
};

vkv_status map_model(vkv_model &m) {
    const vkv_hparams &hp = m.view.hp;
    if (hp.is_offline)
        return gfail(VKV_STATUS_MODEL_ERROR,
                     "model: the offline architecture (LayerNorm + GELU encoder) is not on the device path");
    if (hp.enc_layers < 1 || hp.dec_layers < 1 || hp.enc_dim < 1 || hp.dec_dim < 1 ||
        hp.enc_heads < 1 || hp.dec_heads < 1 || hp.dec_kv_heads < 1 || hp.enc_head_dim < 1 ||
        hp.dec_head_dim < 1 || hp.vocab_size < 1 || hp.downsample_factor < 1 ||
        hp.enc_layers > 4096 || hp.dec_layers > 4096)
        return gfail(VKV_STATUS_MODEL_ERROR, "model: hyperparameters out of range");
    Mapper mp{m, {}};
    char nm[96];
    auto name = [&](const char *fmt, int l) {
        std::snprintf(nm, sizeof(nm), fmt, l);
        return std::string(nm);
    };
    vkv_model_view &v = m.view;
    const int64_t ed = hp.enc_dim, eq = (int64_t)hp.enc_heads * hp.enc_head_dim,
                  ekv = (int64_t)hp.enc_kv_heads * hp.enc_head_dim, eh = hp.enc_hidden;
    // conv stem: ggml [3, in, out] f16 = [out][in][3]
    const TensorInfo *c0 = mp.info("enc.conv0.weight");
    const int64_t n_mel = c0 ? c0->t.ne[1] : 0;
    v.conv0_w = mp.conv("enc.conv0.weight", n_mel, ed);
    v.conv0_b = mp.vec("enc.conv0.bias", ed);
    v.conv1_w = mp.conv("enc.conv1.weight", ed, ed);
    v.conv1_b = mp.vec("enc.conv1.bias", ed);
    m.enc_layers.assign((size_t)hp.enc_layers, vkv_enc_layer{});
    for (int l = 0; l < hp.enc_layers; ++l) {
        vkv_enc_layer &L = m.enc_layers[(size_t)l];
        L.attn_norm = mp.vec(name("enc.blk.%d.attn_norm.weight", l), ed);
        L.attn_norm_b = mp.vec(name("enc.blk.%d.attn_norm.bias", l), ed, true);
        L.attn_q = mp.mat(name("enc.blk.%d.attn_q.weight", l), eq, ed, &L.attn_q_type);
        L.attn_q_b = mp.vec(name("enc.blk.%d.attn_q.bias", l), eq);
        L.attn_k = mp.mat(name("enc.blk.%d.attn_k.weight", l), ekv, ed, &L.attn_k_type);
        L.attn_v = mp.mat(name("enc.blk.%d.attn_v.weight", l), ekv, ed, &L.attn_v_type);
        L.attn_v_b = mp.vec(name("enc.blk.%d.attn_v.bias", l), ekv);
        L.attn_o = mp.mat(name("enc.blk.%d.attn_o.weight", l), ed, eq, &L.attn_o_type);
        L.attn_o_b = mp.vec(name("enc.blk.%d.attn_o.bias", l), ed);
        L.ffn_norm = mp.vec(name("enc.blk.%d.ffn_norm.weight", l), ed);
        L.ffn_norm_b = mp.vec(name("enc.blk.%d.ffn_norm.bias", l), ed, true);
        L.ffn_w1 = mp.mat(name("enc.blk.%d.ffn_w1.weight", l), eh, ed, &L.ffn_w1_type);
        L.ffn_w2 = mp.mat(name("enc.blk.%d.ffn_w2.weight", l), ed, eh, &L.ffn_w2_type);
        L.ffn_w2_b = mp.vec(name("enc.blk.%d.ffn_w2.bias", l), ed);
        L.ffn_w3 = mp.mat(name("enc.blk.%d.ffn_w3.weight", l), eh, ed, &L.ffn_w3_type);
    }
    v.enc = vkv_enc_model{hp.enc_layers, hp.enc_dim, hp.enc_hidden, hp.enc_heads, hp.enc_head_dim,
                          hp.enc_norm_eps, hp.enc_rope_theta, mp.vec("enc.norm.weight", ed),
                          mp.vec("enc.norm.bias", ed, true), m.enc_layers.data()};
    const int64_t dd = hp.dec_dim, dq = (int64_t)hp.dec_heads * hp.dec_head_dim,
                  dkv = (int64_t)hp.dec_kv_heads * hp.dec_head_dim, dh = hp.dec_hidden;
    v.adapter.enc_dim = hp.enc_dim;
    v.adapter.dec_dim = hp.dec_dim;
    v.adapter.downsample = hp.downsample_factor;
    v.adapter.w0 = mp.mat("adapter.0.weight", dd, ed * hp.downsample_factor, &v.adapter.w0_type);
    v.adapter.w2 = mp.mat("adapter.2.weight", dd, dd, &v.adapter.w2_type);
    m.dec_layers.assign((size_t)hp.dec_layers, vkv_dec_layer{});
    for (int l = 0; l < hp.dec_layers; ++l) {
        vkv_dec_layer &L = m.dec_layers[(size_t)l];
        L.attn_norm = mp.vec(name("dec.blk.%d.attn_norm.weight", l), dd);
        L.attn_q = mp.mat(name("dec.blk.%d.attn_q.weight", l), dq, dd, &L.attn_q_type);
        L.attn_k = mp.mat(name("dec.blk.%d.attn_k.weight", l), dkv, dd, &L.attn_k_type);
        L.attn_v = mp.mat(name("dec.blk.%d.attn_v.weight", l), dkv, dd, &L.attn_v_type);
        L.attn_o = mp.mat(name("dec.blk.%d.attn_o.weight", l), dd, dq, &L.attn_o_type);
        L.ffn_norm = mp.vec(name("dec.blk.%d.ffn_norm.weight", l), dd);
        L.ada_scale = nullptr;
        L.ffn_w1 = mp.mat(name("dec.blk.%d.ffn_w1.weight", l), dh, dd, &L.ffn_w1_type);
        L.ffn_w2 = mp.mat(name("dec.blk.%d.ffn_w2.weight", l), dd, dh, &L.ffn_w2_type);
        L.ffn_w3 = mp.mat(name("dec.blk.%d.ffn_w3.weight", l), dh, dd, &L.ffn_w3_type);
        if (hp.ada_t_cond) {
            // the ada MLP's weights stay available by name (vkv_model_tensor)
            if (!mp.info(name("dec.blk.%d.ada0.weight", l)) || !mp.info(name("dec.blk.%d.ada2.weight", l)))
                mp.miss(name("tensor 'dec.blk.%d.ada0/ada2.weight' not found", l));
        }
    }
    int32_t tok_type = 0, out_type = 0;
    const void *tok = mp.mat("tok_embeddings.weight", hp.vocab_size, dd, &tok_type);
    const void *out = tok;
    out_type = tok_type;
    if (mp.info("output.weight")) out = mp.mat("output.weight", hp.vocab_size, dd, &out_type);
    v.dec = vkv_dec_model{hp.dec_layers, hp.dec_dim, hp.dec_hidden, hp.dec_heads, hp.dec_kv_heads,
                          hp.dec_head_dim, hp.vocab_size, hp.dec_norm_eps, hp.dec_rope_theta, tok,
                          tok_type, mp.vec("norm.weight", dd), out, out_type, m.dec_layers.data()};
    const TensorInfo *mf = mp.info("audio.mel_filters");
    v.mel_filters = mf && mf->t.type == kF32 ? (const float *)mp.dev(mf) : nullptr;
    // Matrices that share one product call read one input image (q8_0 for
    // Q8_0 rows, Q8_K for the k-quants): a layer's Q/K/V are one call, and
    // a SwiGLU pair takes one dtype.
    auto q8 = [](int32_t t) { return t == kQ8_0; };
    for (int l = 0; l < hp.enc_layers && mp.err.empty(); ++l) {
        const vkv_enc_layer &L = m.enc_layers[(size_t)l];
        if (q8(L.attn_q_type) != q8(L.attn_k_type) || q8(L.attn_q_type) != q8(L.attn_v_type) ||
            L.ffn_w1_type != L.ffn_w3_type)
            mp.miss(name("encoder layer %d mixes Q8_0 and k-quant matrices within one product", l));
    }
    for (int l = 0; l < hp.dec_layers && mp.err.empty(); ++l) {
        const vkv_dec_layer &L = m.dec_layers[(size_t)l];
        if (q8(L.attn_q_type) != q8(L.attn_k_type) || q8(L.attn_q_type) != q8(L.attn_v_type) ||
            L.ffn_w1_type != L.ffn_w3_type)
            mp.miss(name("decoder layer %d mixes Q8_0 and k-quant matrices within one product", l));
    }
    if (!mp.err.empty()) return gfail(VKV_STATUS_MODEL_ERROR, "model: %s", mp.err.c_str());
    return VKV_STATUS_OK;
}

// memcpy split over host threads: one thread reads the page cache at
// ~10 GB/s, below what the host link takes
void parallel_copy(void *dst, const void *src, size_t n) {
    static const unsigned kThreads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    if (n < (8u << 20) || kThreads == 1) {
        std::memcpy(dst, src, n);
        return;
    }
    std::vector<std::thread> pool;
    const size_t part = (n / kThreads + 4095) & ~(size_t)4095;
    for (unsigned t = 1; t < kThreads; ++t) {
        const size_t a = std::min(n, part * t), b = std::min(n, part * (t + 1));
        if (a < b)
            pool.emplace_back([=] { std::memcpy((uint8_t *)dst + a, (const uint8_t *)src + a, b - a); });
    }
    std::memcpy(dst, src, std::min(n, part));
    for (auto &th : pool) th.join();
}

// the data section, file -> device, through pinned buffers in turn: the
// host copies into one overlap the device copies out of the others
vkv_status upload(vkv_model &m, hipStream_t st) {
    const vkv_gguf &g = *m.g;
    const uint64_t total = g.data_size;
    if (total == 0) return VKV_STATUS_OK;
    constexpr size_t kChunk = 64u << 20;
    constexpr int kBufs = 3;
    void *pin[kBufs] = {};
    hipEvent_t done[kBufs] = {};
    vkv_status rs = VKV_STATUS_OK;
    hipError_t e = hipSuccess;
    for (int b = 0; b < kBufs && e == hipSuccess; ++b) {
        e = hipHostMalloc(&pin[b], kChunk, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[b], hipEventDisableTiming);
    }
    if (e != hipSuccess) rs = vkv::host_hip_fail(e, "model: staging buffers");
    // bytes of the data section present in the file (the last tensor's
    // padding may be missing)
    const uint64_t in_file = std::min<uint64_t>(total, g.size - g.data_offset);
    bool used[kBufs] = {};
    for (uint64_t off = 0, i = 0; off < in_file && !rs; off += kChunk, ++i) {
        const int b = (int)(i % kBufs);
        const size_t n = (size_t)std::min<uint64_t>(kChunk, in_file - off);
        if (used[b] && (e = hipEventSynchronize(done[b])) != hipSuccess) {
            rs = vkv::host_hip_fail(e, "model: staging wait");
            break;
        }
        parallel_copy(pin[b], g.map + g.data_offset + off, n);
        if ((e = hipMemcpyAsync(m.base + off, pin[b], n, hipMemcpyHostToDevice, st)) != hipSuccess ||
            (e = hipEventRecord(done[b], st)) != hipSuccess) {
            rs = vkv::host_hip_fail(e, "model: upload");
            break;
        }
        used[b] = true;
    }
    if (!rs && (e = hipStreamSynchronize(st)) != hipSuccess) rs = vkv::host_hip_fail(e, "model: upload");
    if (rs) (void)hipStreamSynchronize(st);
    for (int b = 0; b < kBufs; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (pin[b]) (void)hipHostFree(pin[b]);
    }
    return rs;
}

}  // namespace

extern "C" {

vkv_status vkv_model_load(const char *path, int32_t device, void *hip_stream, vkv_model **out) {
    if (out) *out = nullptr;
    if (!path || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "model: null argument");
    vkv_model *m = new (std::nothrow) vkv_model();
    if (!m) return gfail(VKV_STATUS_OUT_OF_MEMORY, "model: out of memory");
    m->device = device;
    // the file first: a bad file is a model error whatever the device
    vkv_status s = vkv_gguf_open(path, &m->g);
    if (!s) s = vkv_gguf_hparams(m->g, &m->view.hp);
    int n_dev = 0;
    if (!s && (hipGetDeviceCount(&n_dev) != hipSuccess || device < 0 || device >= n_dev))
        s = gfail(VKV_STATUS_INVALID_ARGUMENT, "model: device %d of %d", device, n_dev);
    int prev = -1;
    (void)hipGetDevice(&prev);
    if (!s && hipSetDevice(device) != hipSuccess)
        s = gfail(VKV_STATUS_BACKEND_ERROR, "model: cannot select device %d", device);
    if (!s) {
        // the whole data section, padded so the last tensor's padding is mapped too
        const size_t bytes = (size_t)((m->g->data_size + 255) & ~(uint64_t)255);
        hipError_t e = hipMalloc((void **)&m->base, std::max<size_t>(bytes, 256));
        if (e != hipSuccess) {
            m->base = nullptr;
            s = e == hipErrorOutOfMemory ? gfail(VKV_STATUS_OUT_OF_MEMORY, "model: %zu bytes of device memory", bytes)
                                         : vkv::host_hip_fail(e, "model: device allocation");
        }
        m->view.device_bytes = bytes;
    }
    if (!s) s = map_model(*m);
    if (!s) s = upload(*m, (hipStream_t)hip_stream);
    if (prev >= 0) (void)hipSetDevice(prev);
    if (s) {
        delete m;
        return s;
    }
    *out = m;
    return vkv::host_ok();
}

vkv_status vkv_model_free(vkv_model *model) {
    delete model;
    return vkv::host_ok();
}

vkv_status vkv_model_get_view(const vkv_model *model, vkv_model_view *out) {
    if (out) std::memset(out, 0, sizeof(*out));
    if (!model || !out) return gfail(VKV_STATUS_INVALID_ARGUMENT, "model: null argument");
    *out = model->view;
    return vkv::host_ok();
}

vkv_status vkv_model_set_ada(vkv_model *model, float t, float *scales, void *hip_stream) {
    if (!model || !scales) return gfail(VKV_STATUS_INVALID_ARGUMENT, "model: null argument");
    const vkv_hparams &hp = model->view.hp;
    if (!hp.ada_t_cond) return vkv::host_ok();
    int prev = -1;
    (void)hipGetDevice(&prev);
    if (hipSetDevice(model->device) != hipSuccess)
        return gfail(VKV_STATUS_BACKEND_ERROR, "model: cannot select device %d", model->device);
    vkv_status s = VKV_STATUS_OK;
    char nm[96];
    int64_t ada_dim = 0;
    std::vector<std::pair<const TensorInfo *, const TensorInfo *>> w((size_t)hp.dec_layers);
    for (int l = 0; l < hp.dec_layers && !s; ++l) {
        std::snprintf(nm, sizeof(nm), "dec.blk.%d.ada0.weight", l);
        const int64_t i0 = vkv_gguf_find_tensor(model->g, nm);
        std::snprintf(nm, sizeof(nm), "dec.blk.%d.ada2.weight", l);
        const int64_t i2 = vkv_gguf_find_tensor(model->g, nm);
        if (i0 < 0 || i2 < 0) {
            s = gfail(VKV_STATUS_MODEL_ERROR, "model: layer %d has no ada weights", l);
            break;
        }
        const TensorInfo &a0 = model->g->tensors[(size_t)i0], &a2 = model->g->tensors[(size_t)i2];
        if (l == 0) ada_dim = a0.t.ne[1];
        if (a0.t.n_dims != 2 || a0.t.ne[0] != hp.dec_dim || a0.t.ne[1] != ada_dim ||
            (a0.t.type != kQ4K && a0.t.type != kQ6K && a0.t.type != kQ8_0) || a2.t.n_dims != 2 ||
            a2.t.ne[0] != ada_dim || a2.t.ne[1] != hp.dec_dim ||
            (a2.t.type != kF16 && a2.t.type != kF32 && a2.t.type != kQ8_0))
            s = gfail(VKV_STATUS_MODEL_ERROR, "model: layer %d ada weights have unexpected shapes or types", l);
        w[(size_t)l] = {&a0, &a2};
    }
    const size_t wsb = s ? 0 : vkv_ada_scale_workspace(hp.dec_dim, (int32_t)ada_dim);
    if (!s && !wsb) s = gfail(VKV_STATUS_MODEL_ERROR, "model: ada dimension %lld", (long long)ada_dim);
    if (!s && !model->ada_ws) {
        hipError_t e = hipMalloc((void **)&model->ada_ws, wsb);
        if (e != hipSuccess) {
            model->ada_ws = nullptr;
            s = vkv::host_hip_fail(e, "model: ada workspace");
        }
    }
    for (int l = 0; l < hp.dec_layers && !s; ++l)
        s = vkv_ada_scale(model->base + w[(size_t)l].first->t.offset, w[(size_t)l].first->t.type,
                          model->base + w[(size_t)l].second->t.offset, w[(size_t)l].second->t.type,
                          hp.dec_dim, (int32_t)ada_dim, t, scales + (size_t)l * hp.dec_dim,
                          model->ada_ws, wsb, hip_stream);
    if (!s)
        for (int l = 0; l < hp.dec_layers; ++l)
            model->dec_layers[(size_t)l].ada_scale = scales + (size_t)l * hp.dec_dim;
    if (prev >= 0) (void)hipSetDevice(prev);
    return s ? s : vkv::host_ok();
}

const void *vkv_model_tensor(const vkv_model *model, const char *name, vkv_gguf_tensor *info) {
    if (info) std::memset(info, 0, sizeof(*info));
    if (!model || !name) return nullptr;
    const int64_t i = vkv_gguf_find_tensor(model->g, name);
    if (i < 0) return nullptr;
    if (info) *info = model->g->tensors[(size_t)i].t;
    return model->base + model->g->tensors[(size_t)i].t.offset;
}

}  // extern "C"
