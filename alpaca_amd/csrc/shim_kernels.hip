// Kernels of the shim's module-launch test, built as a stand-alone gfx950
// code object (alpaca_amd/shim_kernels.hsaco) that ahip_module_load reads
// from disk, as the Swift side would load the library's kernels by name
// (MetalContext.pipeline, Sources/AlpacaMetal/Backend/MetalContext.swift:102-111).
#include <hip/hip_runtime.h>

// y[i] = a * x[i] + y[i] for i < n.
extern "C" __global__ void ahip_shim_axpy(float a, const float* __restrict__ x, float* __restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a * x[i] + y[i];
}

// out[i] = value for i < n.
extern "C" __global__ void ahip_shim_fill_u32(unsigned* __restrict__ out, unsigned value, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = value;
}
