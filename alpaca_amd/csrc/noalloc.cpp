// ahip_attention_decode_noalloc: the single-query split-K attention of
// ahip_op_attention (the same two kernels, attn_decode_split + attn_merge) on
// device buffers, for callers that cannot allocate device memory (code under
// HIP graph capture, fixed serving loops, harnesses that forbid hipMalloc).
// It has no counterpart in the reference.
//
// The split partials, the only memory the kernels use beyond their inputs and
// output, live in `scratch`, a file-scope device array of a fixed size that
// each GPU holds until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address is resolved with
// hipGetSymbolAddress once per device (ahip_context_create, with that device
// current) and only that address is passed to kernels.  Every call on a GPU
// shares that GPU's array, so calls that overlap on one GPU (on different
// streams, or from several threads) race; nothing in it needs to start at
// zero, since the merge reads only partials its own call's split kernel wrote.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/alpaca_hip.h"
#include "common.h"
#include "host.h"

namespace {

constexpr size_t kScratchFloats = 655360;  // 2.5 MiB: heads * splits * (head_dim + 2) floats at most
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_lock;
float* g_scratch[kMaxDevices] = {nullptr};

}  // namespace

int noalloc_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "device index out of range");
    std::lock_guard<std::mutex> g(g_lock);
    if (g_scratch[device]) return AHIP_OK;
    float* p = nullptr;
    const hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        hipGetLastError();
        return ahip_fail(AHIP_ERR_COMMAND_FAILED, std::string("scratch address: ") + hipGetErrorString(e));
    }
    g_scratch[device] = p;
    return AHIP_OK;
}

extern "C" int ahip_attention_decode_noalloc(ahip_context* ctx, const float* q, const void* k_cache,
                                             const void* v_cache, int kv_precision, int capacity, int heads,
                                             int kv_heads, int head_dim, int length, float* out, ahip_stream* stream) {
    if (!ctx || !q || !k_cache || !v_cache || !out) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (kv_precision != AHIP_KV_F16 && kv_precision != AHIP_KV_F32)
        return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "bad kv precision");
    if (heads <= 0 || kv_heads <= 0 || capacity <= 0 || length <= 0 || length > capacity)
        return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "attention shapes");
    if (stream && stream->device != ctx->device)
        return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "stream and context belong to different devices");
    if (hipSetDevice(ctx->device) != hipSuccess) return ahip_fail(AHIP_ERR_COMMAND_FAILED, "hipSetDevice");
    // the split length ahip_op_attention takes for one query
    const int sl = attention_decode_supported(heads, kv_heads, head_dim)
                       ? attention_decode_session_split_len(capacity, heads, kv_heads) : 0;
    if (sl <= 0) return ahip_fail(AHIP_ERR_UNSUPPORTED, "head_dim 64 or 128, at most 16 query heads per KV head");
    const int splits = (length + sl - 1) / sl;
    const size_t need = (size_t)heads * splits * (head_dim + 2);
    if (need > kScratchFloats)
        return ahip_fail(AHIP_ERR_INVALID_ARGUMENT,
                         "split partials need " + std::to_string(need) + " floats, more than the " +
                             std::to_string(kScratchFloats) + "-float scratch array holds");
    float* part = nullptr;
    {
        std::lock_guard<std::mutex> g(g_lock);
        part = g_scratch[ctx->device];
    }
    if (!part) return ahip_fail(AHIP_ERR_COMMAND_FAILED, "scratch array not resolved for this device");
    hipStream_t st = stream ? stream->st : ctx->stream;
    hipError_t e = launch_attention_decode(q, k_cache, v_cache, kv_precision == AHIP_KV_F16, capacity, heads, kv_heads,
                                           head_dim, length, nullptr, sl, splits, part, st);
    if (e == hipSuccess) e = launch_attention_merge(part, heads, head_dim, splits, out, st);
    if (e != hipSuccess) {
        hipGetLastError();
        return ahip_fail(AHIP_ERR_COMMAND_FAILED, std::string("kernel launch: ") + hipGetErrorString(e));
    }
    return AHIP_OK;
}
