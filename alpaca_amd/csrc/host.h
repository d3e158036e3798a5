// Host-side types shared by the library's C++ sources (runtime.cpp, shim.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

// MetalContext (Sources/AlpacaMetal/Backend/MetalContext.swift:37-57): one
// device and the stream the op-level calls and the shim's synchronous copies
// run on.
struct ahip_context {
    int device = 0;
    hipStream_t stream = nullptr;
};

// A stream of the thin shim (ahip_stream_create), default priority.
struct ahip_stream {
    int device = 0;
    hipStream_t st = nullptr;
};

// Resolves, once per device and with that device current, the address of the
// no-allocation entry point's scratch array (noalloc.cpp); called by
// ahip_context_create.  Returns an ahip_status.
int noalloc_scratch_init(int device);

// Sets the thread-local message ahip_last_error() returns; returns `code`.
int ahip_fail(int code, const std::string& msg);
