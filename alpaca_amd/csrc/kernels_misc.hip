// Small HBM-bound kernels of the forward pass: elementwise ops, RMSNorm,
// embedding gather, dequantisation, RoPE + KV-cache store and the greedy
// arg-max.  Semantics follow the reference's CPU ops
// (Sources/AlpacaCore/Operations/CPUOps.swift) cited per kernel.
#include "common.h"

#include <float.h>
#include <limits.h>

namespace {

constexpr int kBlock = 256;

inline int grid_for(int64_t n, int per_block = kBlock) {
    int64_t g = (n + per_block - 1) / per_block;
    return (int)(g < 65535 * 16 ? g : 65535 * 16);
}

// CPUOps.add / mul / silu (CPUOps.swift:29-53) and the SwiGLU gate product.
__global__ void add_kernel(const float* a, const float* b, float* o, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        o[i] = a[i] + b[i];
}
__global__ void mul_kernel(const float* a, const float* b, float* o, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        o[i] = a[i] * b[i];
}
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__global__ void silu_kernel(const float* x, float* o, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        o[i] = silu_f(x[i]);
}
__global__ void silu_mul_kernel(const float* g, const float* u, float* o, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        o[i] = silu_f(g[i]) * u[i];
}
// hi = f16(v) to o, and with ol the remainder lo = f16(v - hi): hi + lo holds v
// to ~2^-22 relative (the two-term activations of the MFMA prefill).
__device__ __forceinline__ void store_terms(f16* o, f16* ol, int64_t i, float v) {
    const f16 h = (f16)v;
    o[i] = h;
    if (ol) ol[i] = (f16)(v - (float)h);
}
__global__ void f32_to_f16_kernel(const float* x, f16* o, f16* ol, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        store_terms(o, ol, i, x[i]);
}

// CPUOps.rmsNorm (CPUOps.swift:144-159): y = x * (1/sqrt(mean(x^2) + eps)) * w,
// one block per row, optionally writing f16 for the MFMA GEMM.
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const float* x, const float* w, float* of, f16* oh,
                                                         f16* ol, int dim, float eps, int lo_row0) {
    if ((int)blockIdx.x < lo_row0) ol = nullptr;
    __shared__ float red[16];
    const float* xr = x + (int64_t)blockIdx.x * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kBlock) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += kBlock) {
        float y = (xr[i] * scale) * w[i];
        if (of) of[(int64_t)blockIdx.x * dim + i] = y;
        if (oh) store_terms(oh, ol, (int64_t)blockIdx.x * dim + i, y);
    }
}

// The same, one wave per row (4 rows per block) with the row in registers as
// float4 (dim % 4 == 0, dim <= 64 * 4 * kNormV4): one read of x, 16-byte loads,
// 8-byte f16 stores, and no block barrier.
constexpr int kNormV4 = 8;
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_kernel(const float* x, const float* w, float* of, f16* oh,
                                                              f16* ol, int rows, int dim, float eps, int lo_row0) {
    const int row = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole waves leave together
    if (row < lo_row0) ol = nullptr;
    const int n4 = dim >> 2;
    const float4* xr = (const float4*)(x + (int64_t)row * dim);
    const float4* wr = (const float4*)w;
    // the gains load with the row, not after the reduction
    float4 v[kNormV4], gv[kNormV4];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kNormV4; k++) {
        const int i = lane + 64 * k;
        v[k] = i < n4 ? xr[i] : float4{0.f, 0.f, 0.f, 0.f};
        gv[k] = i < n4 ? wr[i] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < kNormV4; k++) {
        ss += v[k].x * v[k].x;
        ss += v[k].y * v[k].y;
        ss += v[k].z * v[k].z;
        ss += v[k].w * v[k].w;
    }
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < kNormV4; k++) {
        const int i = lane + 64 * k;
        if (i >= n4) break;
        const float4 g = gv[k];
        const float4 y = {(v[k].x * scale) * g.x, (v[k].y * scale) * g.y, (v[k].z * scale) * g.z,
                          (v[k].w * scale) * g.w};
        if (of) ((float4*)(of + (int64_t)row * dim))[i] = y;
        if (oh) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            const h4 hi = {(f16)y.x, (f16)y.y, (f16)y.z, (f16)y.w};
            ((h4*)(oh + (int64_t)row * dim))[i] = hi;
            if (ol)
                ((h4*)(ol + (int64_t)row * dim))[i] = h4{(f16)(y.x - (float)hi[0]), (f16)(y.y - (float)hi[1]),
                                                         (f16)(y.z - (float)hi[2]), (f16)(y.w - (float)hi[3])};
        }
    }
}

// Element k of row r of a resident matrix, dequantised exactly (d * q is exact
// in float32), Quantization.swift:9-35.
__device__ __forceinline__ float load_elem(const DevMatrix& m, int64_t r, int k) {
    if (m.dtype == DT_F16) return (float)((const f16*)m.q)[r * m.cols + k];
    int nb = m.cols / 32;
    float d = (float)m.s[r * nb + k / 32];
    if (m.dtype == DT_Q8_0) return d * (float)(int)((const int8_t*)m.q)[r * m.cols + k];
    int j = k & 31;
    uint8_t byte = m.q[(r * nb + k / 32) * 16 + (j & 15)];
    int nib = j < 16 ? (byte & 15) : (byte >> 4);
    return d * (float)(nib - 8);
}

// CPUOps.embed (CPUOps.swift:279-290): rows of the table selected by tokens.
// Token ids are validated on the host before launch.
__global__ __launch_bounds__(kBlock) void embed_kernel(const int32_t* tokens, DevMatrix m, float* out) {
    int64_t r = tokens[blockIdx.x];
    for (int k = threadIdx.x; k < m.cols; k += kBlock) out[(int64_t)blockIdx.x * m.cols + k] = load_elem(m, r, k);
}

__global__ void dequant_kernel(DevMatrix m, float* out) {
    int64_t n = (int64_t)m.rows * m.cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = load_elem(m, i / m.cols, (int)(i % m.cols));
}

// Half copy of a quantised matrix for the prefill weight cache: each weight
// d*q (exact in float32) rounded once to f16 (MetalLlamaModel.buildPrefillCache,
// MetalLlamaModel.swift:97-120).  One thread per 8 consecutive weights of a row.
__global__ void dequant_f16_kernel(DevMatrix m, f16* out) {
    const int64_t groups = (int64_t)m.rows * (m.cols / 8);
    for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < groups; g += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = g / (m.cols / 8);
        const int k0 = (int)(g % (m.cols / 8)) * 8;
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (f16)load_elem(m, r, k0 + e);
        *(h8*)(out + r * m.cols + k0) = v;
    }
}

// Greedy arg-max: largest logit, lowest index on ties, NaN never wins
// (Sampler.argmax, Sampler.swift:100-108; all-NaN input yields 0).  Writes the
// next input token and emitted[slot].  One block of 1024 threads.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int n, int32_t* chain, int32_t* emitted,
                                                      int slot, int* pos_dev) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float v = -INFINITY;
    int idx = INT_MAX;
    // 16-byte loads, sixteen in flight per thread (a 64K-entry vocabulary in
    // one batch; indices past the end clamped to the last quad and their
    // values skipped, so the loads go out unconditionally); each thread visits
    // its indices in increasing order, so it keeps the first of equal maxima
    const int n4 = ((uintptr_t)logits & 15) ? 0 : n / 4;
    const float4* l4 = (const float4*)logits;
    for (int base = threadIdx.x; base < n4; base += 16 * 1024) {
        float4 x[16];
#pragma unroll
        for (int u = 0; u < 16; u++) x[u] = l4[min(base + u * 1024, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int i = 4 * (base + u * 1024);
            if (i < 4 * n4) {
                if (x[u].x > v) { v = x[u].x; idx = i; }
                if (x[u].y > v) { v = x[u].y; idx = i + 1; }
                if (x[u].z > v) { v = x[u].z; idx = i + 2; }
                if (x[u].w > v) { v = x[u].w; idx = i + 3; }
            }
        }
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += 1024) {
        float x = logits[i];
        if (x > v) { v = x; idx = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float v2 = __shfl_xor(v, o, 64);
        int i2 = __shfl_xor(idx, o, 64);
        if (v2 > v || (v2 == v && i2 < idx)) { v = v2; idx = i2; }
    }
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) { sv[w] = v; si[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = sv[0];
        int bi = si[0];
        for (int i = 1; i < 16; i++)
            if (sv[i] > bv || (sv[i] == bv && si[i] < bi)) { bv = sv[i]; bi = si[i]; }
        int token = bi == INT_MAX ? 0 : bi;
        if (chain) chain[0] = token;
        if (pos_dev) {
            const int p = *pos_dev;
            if (emitted) emitted[p] = token;
            *pos_dev = p + 1;
        } else if (emitted) {
            emitted[slot] = token;
        }
    }
}

// CPUOps.rope (CPUOps.swift:184-212) fused with the KV-cache append
// (KVCache.write, KVCache.swift:44-63).  cos/sin come from a table built on
// the host in double precision and rounded once, as the CPU reference does,
// and the rotation is evaluated without contraction, so q/k match the CPU
// bit for bit on the same inputs.
template <typename KV>
__global__ __launch_bounds__(kBlock) void rope_store_kernel(float* qkv, int ld, int heads, int kv_heads, int hd,
                                                            int start, const float2* table, int interleaved,
                                                            int write_q, f16* q16, f16* q16lo, KV* kc, KV* vc,
                                                            int capacity) {
#pragma clang fp contract(off)
    int t = blockIdx.x;
    int half = hd / 2;
    int pos = start + t;
    int ny = heads + (kc ? kv_heads : 0);
    float* row = qkv + (int64_t)t * ld;
    for (int idx = threadIdx.x; idx < ny * half; idx += kBlock) {
        int y = idx / half, i = idx - y * half;
        float2 cs = table[(int64_t)pos * half + i];
        int ia = interleaved ? 2 * i : i;
        int ib = interleaved ? 2 * i + 1 : i + half;
        if (y < heads) {
            float* p = row + y * hd;
            float a = p[ia], b = p[ib];
            float ac = a * cs.x, bs = b * cs.y, as = a * cs.y, bc = b * cs.x;
            float ra = ac - bs, rb = as + bc;
            if (write_q) { p[ia] = ra; p[ib] = rb; }
            if (q16) {
                const int64_t o = ((int64_t)t * heads + y) * hd;
                store_terms(q16, q16lo, o + ia, ra);
                store_terms(q16, q16lo, o + ib, rb);
            }
        } else {
            int h = y - heads;
            const float* k = row + heads * hd + h * hd;
            const float* v = row + heads * hd + kv_heads * hd + h * hd;
            float a = k[ia], b = k[ib];
            float ac = a * cs.x, bs = b * cs.y, as = a * cs.y, bc = b * cs.x;
            int64_t dst = ((int64_t)h * capacity + pos) * hd;
            kc[dst + ia] = (KV)(ac - bs);
            kc[dst + ib] = (KV)(as + bc);
            vc[dst + ia] = (KV)v[ia];
            vc[dst + ib] = (KV)v[ib];
        }
    }
}

}  // namespace

hipError_t launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t st) {
    if (n > 0) add_kernel<<<grid_for(n), kBlock, 0, st>>>(a, b, out, n);
    return hipGetLastError();
}
hipError_t launch_mul(const float* a, const float* b, float* out, int64_t n, hipStream_t st) {
    if (n > 0) mul_kernel<<<grid_for(n), kBlock, 0, st>>>(a, b, out, n);
    return hipGetLastError();
}
hipError_t launch_silu(const float* x, float* out, int64_t n, hipStream_t st) {
    if (n > 0) silu_kernel<<<grid_for(n), kBlock, 0, st>>>(x, out, n);
    return hipGetLastError();
}
hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st) {
    if (n > 0) silu_mul_kernel<<<grid_for(n), kBlock, 0, st>>>(g, u, out, n);
    return hipGetLastError();
}
hipError_t launch_f32_to_f16(const float* x, f16* out, f16* out_lo, int64_t n, hipStream_t st) {
    if (n > 0) f32_to_f16_kernel<<<grid_for(n), kBlock, 0, st>>>(x, out, out_lo, n);
    return hipGetLastError();
}
hipError_t launch_rmsnorm(const float* x, const float* w, float* of, f16* oh, f16* ol, int rows, int dim, float eps,
                          hipStream_t st, int lo_row0) {
    if (rows <= 0) return hipSuccess;
    const bool vec = dim % 4 == 0 && dim <= 64 * 4 * kNormV4 && !((uintptr_t)x & 15) && !((uintptr_t)w & 15) &&
                     !((uintptr_t)of & 15) && !((uintptr_t)oh & 7) && !((uintptr_t)ol & 7);
    if (vec) rmsnorm_rows_kernel<<<(rows + 3) / 4, kBlock, 0, st>>>(x, w, of, oh, ol, rows, dim, eps, lo_row0);
    else rmsnorm_kernel<<<rows, kBlock, 0, st>>>(x, w, of, oh, ol, dim, eps, lo_row0);
    return hipGetLastError();
}
hipError_t launch_embed(const int32_t* tokens, int count, const DevMatrix& table, float* out, hipStream_t st) {
    if (count > 0) embed_kernel<<<count, kBlock, 0, st>>>(tokens, table, out);
    return hipGetLastError();
}
hipError_t launch_dequant(const DevMatrix& m, float* out, hipStream_t st) {
    int64_t n = (int64_t)m.rows * m.cols;
    if (n > 0) dequant_kernel<<<grid_for(n), kBlock, 0, st>>>(m, out);
    return hipGetLastError();
}
hipError_t launch_dequant_f16(const DevMatrix& m, f16* out, hipStream_t st) {
    if (m.cols % 8) return hipErrorInvalidValue;
    const int64_t groups = (int64_t)m.rows * (m.cols / 8);
    if (groups > 0) dequant_f16_kernel<<<grid_for(groups), kBlock, 0, st>>>(m, out);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, int32_t* chain, int32_t* emitted, int slot, int* pos_dev,
                         hipStream_t st) {
    argmax_kernel<<<1, 1024, 0, st>>>(logits, n, chain, emitted, slot, pos_dev);
    return hipGetLastError();
}
hipError_t launch_rope_store(float* qkv, int ld, int tokens, int heads, int kv_heads, int hd, int start,
                             const float2* table, int interleaved, int write_q_f32, f16* q_f16, f16* q_f16_lo,
                             void* kcache, void* vcache, int kv_f16, int capacity, hipStream_t st) {
    if (tokens <= 0) return hipSuccess;
    if (kv_f16)
        rope_store_kernel<f16><<<tokens, kBlock, 0, st>>>(qkv, ld, heads, kv_heads, hd, start, table, interleaved,
                                                          write_q_f32, q_f16, q_f16_lo, (f16*)kcache, (f16*)vcache,
                                                          capacity);
    else
        rope_store_kernel<float><<<tokens, kBlock, 0, st>>>(qkv, ld, heads, kv_heads, hd, start, table,
                                                            interleaved, write_q_f32, q_f16, q_f16_lo, (float*)kcache,
                                                            (float*)vcache, capacity);
    return hipGetLastError();
}
