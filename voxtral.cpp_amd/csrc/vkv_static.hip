// The decoder token without a workspace argument, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The token's scratch -- the residual
// stream, q/k/v, the attention output, the FFN hidden row and the fused
// argmax words -- lives in `scratch`, a file-scope device array of
// VKV_TOKEN_SCRATCH_BYTES: one copy per GPU, held until the process ends.
//
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): the device address of each GPU's copy is
// resolved once, with that GPU current, by hipGetSymbolAddress, and only
// that address is handed to the kernels.  Every call on a GPU shares its
// copy, which keeps the last call's bytes: the token writes every region
// before reading it, and its first kernel clears the argmax words; calls
// that overlap on one GPU (other streams, other threads) race on it.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "vkv.h"
#include "vkv_internal.h"

namespace {

static __device__ __align__(256) uint8_t scratch[VKV_TOKEN_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on `device`, resolved on the device's first
// call with that device current (the caller's device is restored).
vkv_status scratch_address(int device, void **out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return vkv::host_fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token (no alloc): device ordinal");
    void *p = g_scratch_addr[device].load(std::memory_order_acquire);
    if (p) {
        *out = p;
        return VKV_STATUS_OK;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[device].load(std::memory_order_relaxed);
    if (!p) {
        int prev = -1;
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return vkv::host_hip_fail(e, "decoder token (no alloc): hipGetDevice");
        if (prev != device && (e = hipSetDevice(device)) != hipSuccess)
            return vkv::host_hip_fail(e, "decoder token (no alloc): hipSetDevice");
        void *addr = nullptr;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (prev != device) (void)hipSetDevice(prev);
        if (e != hipSuccess || !addr)
            return vkv::host_hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                      "decoder token (no alloc): hipGetSymbolAddress(scratch)");
        p = addr;
        g_scratch_addr[device].store(p, std::memory_order_release);
    }
    *out = p;
    return VKV_STATUS_OK;
}

}  // namespace

extern "C" vkv_status vkv_decoder_token_noalloc(vkv_cache *cache, int32_t stream, vkv_ring *ring,
                                                const vkv_dec_model *model, int32_t token,
                                                const float *audio_emb, float *logits,
                                                int32_t *token_out, vkv_plan *plan_out,
                                                void *hip_stream) {
    if (plan_out) std::memset(plan_out, 0, sizeof(*plan_out));
    const size_t need = vkv_decoder_token_workspace(model);
    if (need == 0)
        return vkv::host_fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token (no alloc): invalid model");
    if (need > (size_t)VKV_TOKEN_SCRATCH_BYTES) {
        char msg[160];
        std::snprintf(msg, sizeof(msg),
                      "decoder token (no alloc): the model needs %zu bytes of workspace, the "
                      "library's static scratch holds %u",
                      need, (unsigned)VKV_TOKEN_SCRATCH_BYTES);
        return vkv::host_fail(VKV_STATUS_BUFFER_TOO_SMALL, msg);
    }
    if (!cache) return vkv::host_fail(VKV_STATUS_INVALID_ARGUMENT, "decoder token (no alloc): null cache");
    void *ws = nullptr;
    if (vkv_status st = scratch_address(vkv::cache_device(cache), &ws)) return st;
    return vkv_decoder_token(cache, stream, ring, model, token, audio_emb, logits, token_out, ws,
                             (size_t)VKV_TOKEN_SCRATCH_BYTES, plan_out, hip_stream);
}
