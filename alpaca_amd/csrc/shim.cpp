// The thin HIP shim of the C ABI: streams, events, pinned host memory,
// asynchronous copies and code-object modules with a launch wrapper.  This is
// the surface a Swift C target wraps to drive HIP directly, the counterpart of
// what the Metal backend takes from Metal itself:
//   MTLCommandQueue / MTLCommandBuffer (MetalContext.swift:48-57,
//   MetalLlamaModel.swift:214-215)       -> ahip_stream (own HIP stream)
//   commit / waitUntilCompleted          -> ahip_stream_synchronize
//   gpuStartTime / gpuEndTime (MetalOps.swift:18-28,
//   MetalLlamaModel.swift:255-260)       -> ahip_event record / elapsed
//   makeBuffer(length:) / (copying:) (MetalContext.swift:113-125)
//                                        -> ahip_malloc / ahip_host_alloc +
//                                           ahip_memcpy_*_async
//   makeLibrary + pipeline(name) (MetalContext.swift:59-111)
//                                        -> ahip_module_load + ahip_module_launch
// Every stream is created at the default priority.
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "../../include/alpaca_hip.h"
#include "host.h"

struct ahip_event {
    int device = 0;
    hipEvent_t ev = nullptr;
};

struct ahip_module {
    int device = 0;
    hipModule_t mod = nullptr;
    std::mutex lock;
    std::map<std::string, hipFunction_t> fns;  // looked up once per name
};

namespace {

// A failed HIP call also becomes the thread's last HIP error, which the
// library's kernel launches read back (hipGetLastError) to detect launch
// failures: every failure path of the shim clears it once reported.
int hip_fail(hipError_t e, const char* what) {
    hipGetLastError();
    return ahip_fail(AHIP_ERR_COMMAND_FAILED, std::string(what) + ": " + hipGetErrorString(e));
}

#define SHIM_OR(expr, what)                      \
    do {                                         \
        hipError_t e_ = (expr);                  \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

int bad(const char* msg) { return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, msg); }

}  // namespace

// ------------------------------------------------------------------ streams

extern "C" int ahip_stream_create(ahip_context* ctx, ahip_stream** out) {
    if (!ctx || !out) return bad("null argument");
    SHIM_OR(hipSetDevice(ctx->device), "hipSetDevice");
    auto* s = new ahip_stream();
    s->device = ctx->device;
    if (hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking) != hipSuccess) {
        hipGetLastError();
        delete s;
        return ahip_fail(AHIP_ERR_COMMAND_FAILED, "hipStreamCreate failed");
    }
    *out = s;
    return AHIP_OK;
}

extern "C" int ahip_stream_destroy(ahip_stream* s) {
    if (!s) return AHIP_OK;
    hipSetDevice(s->device);
    hipStreamSynchronize(s->st);
    hipStreamDestroy(s->st);
    delete s;
    return AHIP_OK;
}

extern "C" int ahip_stream_synchronize(ahip_stream* s) {
    if (!s) return bad("null stream");
    SHIM_OR(hipStreamSynchronize(s->st), "hipStreamSynchronize");
    return AHIP_OK;
}

extern "C" int ahip_stream_wait_event(ahip_stream* s, ahip_event* e) {
    if (!s || !e) return bad("null argument");
    SHIM_OR(hipStreamWaitEvent(s->st, e->ev, 0), "hipStreamWaitEvent");
    return AHIP_OK;
}

// ------------------------------------------------------------------ events

extern "C" int ahip_event_create(ahip_context* ctx, ahip_event** out) {
    if (!ctx || !out) return bad("null argument");
    SHIM_OR(hipSetDevice(ctx->device), "hipSetDevice");
    auto* e = new ahip_event();
    e->device = ctx->device;
    if (hipEventCreate(&e->ev) != hipSuccess) {
        hipGetLastError();
        delete e;
        return ahip_fail(AHIP_ERR_COMMAND_FAILED, "hipEventCreate failed");
    }
    *out = e;
    return AHIP_OK;
}

extern "C" int ahip_event_destroy(ahip_event* e) {
    if (!e) return AHIP_OK;
    hipSetDevice(e->device);
    hipEventDestroy(e->ev);
    delete e;
    return AHIP_OK;
}

extern "C" int ahip_event_record(ahip_event* e, ahip_stream* s) {
    if (!e || !s) return bad("null argument");
    SHIM_OR(hipEventRecord(e->ev, s->st), "hipEventRecord");
    return AHIP_OK;
}

extern "C" int ahip_event_synchronize(ahip_event* e) {
    if (!e) return bad("null event");
    SHIM_OR(hipEventSynchronize(e->ev), "hipEventSynchronize");
    return AHIP_OK;
}

extern "C" int ahip_event_elapsed_ms(const ahip_event* start, const ahip_event* end, float* ms) {
    if (!start || !end || !ms) return bad("null argument");
    SHIM_OR(hipEventElapsedTime(ms, start->ev, end->ev), "hipEventElapsedTime");
    return AHIP_OK;
}

// ------------------------------------------------------------------ memory

extern "C" int ahip_host_alloc(ahip_context* ctx, int64_t bytes, void** ptr) {
    if (!ctx || !ptr || bytes < 0) return bad("bad argument");
    SHIM_OR(hipSetDevice(ctx->device), "hipSetDevice");
    if (hipHostMalloc(ptr, bytes > 0 ? (size_t)bytes : 16, hipHostMallocDefault) != hipSuccess) {
        hipGetLastError();
        *ptr = nullptr;
        return ahip_fail(AHIP_ERR_ALLOC, "failed to allocate " + std::to_string(bytes) + " bytes of pinned host memory");
    }
    return AHIP_OK;
}

extern "C" int ahip_host_free(ahip_context* ctx, void* ptr) {
    if (!ctx) return bad("null context");
    if (ptr) SHIM_OR(hipHostFree(ptr), "hipHostFree");
    return AHIP_OK;
}

extern "C" int ahip_memcpy_htod_async(void* dst, const void* src, int64_t bytes, ahip_stream* s) {
    if (!s || bytes < 0 || (bytes && (!dst || !src))) return bad("bad argument");
    SHIM_OR(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, s->st), "hipMemcpyAsync");
    return AHIP_OK;
}

extern "C" int ahip_memcpy_dtoh_async(void* dst, const void* src, int64_t bytes, ahip_stream* s) {
    if (!s || bytes < 0 || (bytes && (!dst || !src))) return bad("bad argument");
    SHIM_OR(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, s->st), "hipMemcpyAsync");
    return AHIP_OK;
}

extern "C" int ahip_memcpy_dtod_async(void* dst, const void* src, int64_t bytes, ahip_stream* s) {
    if (!s || bytes < 0 || (bytes && (!dst || !src))) return bad("bad argument");
    SHIM_OR(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, s->st), "hipMemcpyAsync");
    return AHIP_OK;
}

// ------------------------------------------------------------------ modules

extern "C" int ahip_module_load(ahip_context* ctx, const char* path, ahip_module** out) {
    if (!ctx || !path || !out) return bad("null argument");
    SHIM_OR(hipSetDevice(ctx->device), "hipSetDevice");
    hipModule_t mod = nullptr;
    const hipError_t e = hipModuleLoad(&mod, path);
    if (e != hipSuccess) {
        hipGetLastError();
        return ahip_fail(AHIP_ERR_MODULE_LOAD, std::string("cannot load code object ") + path + ": " + hipGetErrorString(e));
    }
    auto* m = new ahip_module();
    m->device = ctx->device;
    m->mod = mod;
    *out = m;
    return AHIP_OK;
}

extern "C" int ahip_module_load_data(ahip_context* ctx, const void* image, ahip_module** out) {
    if (!ctx || !image || !out) return bad("null argument");
    SHIM_OR(hipSetDevice(ctx->device), "hipSetDevice");
    hipModule_t mod = nullptr;
    const hipError_t e = hipModuleLoadData(&mod, image);
    if (e != hipSuccess) {
        hipGetLastError();
        return ahip_fail(AHIP_ERR_MODULE_LOAD, std::string("cannot load code object image: ") + hipGetErrorString(e));
    }
    auto* m = new ahip_module();
    m->device = ctx->device;
    m->mod = mod;
    *out = m;
    return AHIP_OK;
}

extern "C" int ahip_module_unload(ahip_module* m) {
    if (!m) return AHIP_OK;
    hipSetDevice(m->device);
    hipModuleUnload(m->mod);
    delete m;
    return AHIP_OK;
}

static int module_function(ahip_module* m, const char* name, hipFunction_t* fn) {
    std::lock_guard<std::mutex> g(m->lock);
    auto it = m->fns.find(name);
    if (it != m->fns.end()) {
        *fn = it->second;
        return AHIP_OK;
    }
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, m->mod, name) != hipSuccess || !f) {
        hipGetLastError();
        return ahip_fail(AHIP_ERR_MISSING_KERNEL, std::string("no kernel named ") + name + " in the module");
    }
    m->fns.emplace(name, f);
    *fn = f;
    return AHIP_OK;
}

extern "C" int ahip_module_has_kernel(ahip_module* m, const char* name, int* found) {
    if (!m || !name || !found) return bad("null argument");
    hipFunction_t f = nullptr;
    *found = module_function(m, name, &f) == AHIP_OK;
    return AHIP_OK;
}

extern "C" int ahip_module_launch(ahip_module* m, const char* kernel, const uint32_t grid[3], const uint32_t block[3],
                                  uint32_t shared_bytes, ahip_stream* s, void** args) {
    if (!m || !kernel || !grid || !block || !s) return bad("null argument");
    for (int d = 0; d < 3; d++)
        if (grid[d] == 0 || block[d] == 0) return bad("grid and block dimensions must be positive");
    if ((uint64_t)block[0] * block[1] * block[2] > 1024) return bad("more than 1024 threads per workgroup");
    if (s->device != m->device) return bad("stream and module belong to different devices");
    hipFunction_t f = nullptr;
    if (int rc = module_function(m, kernel, &f)) return rc;
    SHIM_OR(hipModuleLaunchKernel(f, grid[0], grid[1], grid[2], block[0], block[1], block[2], shared_bytes, s->st, args,
                                  nullptr),
            "hipModuleLaunchKernel");
    return AHIP_OK;
}
