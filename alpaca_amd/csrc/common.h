// Shared device helpers and launch declarations for the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { DT_F32 = 0, DT_F16 = 1, DT_Q8_0 = 2, DT_Q4_0 = 3 };

// A weight matrix [rows, cols] resident in HBM.  Quantised formats are split
// into a quant stream and a scale stream so every row starts 16-byte aligned:
//   Q8_0: q = int8 [rows][cols],             s = f16 [rows][cols/32]
//   Q4_0: q = uint8 [rows][cols/32][16]      s = f16 [rows][cols/32]
//         (byte j of a block: low nibble = element j, high = element j+16)
//   F16:  q = f16 [rows][cols],              s = null
struct DevMatrix {
    int dtype = DT_F16;
    int rows = 0, cols = 0;
    const uint8_t* q = nullptr;
    const f16* s = nullptr;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum over blockDim.x (a multiple of 64, at most 1024) threads.
__device__ __forceinline__ float block_sum(float v, float* red /* >= 16 floats of LDS */) {
    v = wave_sum(v);
    int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    int nw = blockDim.x >> 6;
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// ---------------------------------------------------------------- launchers
// Every launcher enqueues on `st` and returns hipGetLastError().

// elementwise / norm / embed / sampling (kernels_misc.hip)
hipError_t launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t st);
hipError_t launch_mul(const float* a, const float* b, float* out, int64_t n, hipStream_t st);
hipError_t launch_silu(const float* x, float* out, int64_t n, hipStream_t st);
hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st);
hipError_t launch_f32_to_f16(const float* x, f16* out, int64_t n, hipStream_t st);
hipError_t launch_rmsnorm(const float* x, const float* w, float* out_f32, f16* out_f16, int rows, int dim,
                          float eps, hipStream_t st);
hipError_t launch_embed(const int32_t* tokens, int count, const DevMatrix& table, float* out, hipStream_t st);
hipError_t launch_dequant(const DevMatrix& m, float* out, hipStream_t st);
// Greedy arg-max.  Writes the token to *chain_token and emitted[slot] (slot =
// *pos_dev when pos_dev is set, which is then advanced by one).
hipError_t launch_argmax(const float* logits, int n, int32_t* chain_token, int32_t* emitted, int slot,
                         int* pos_dev, hipStream_t st);
// RoPE with a host-built (cos, sin) table [positions][hd/2]; q rotated in
// place (q_f32) and/or written as f16 (q_f16); k rotated and v copied into the
// caches at rows start..start+tokens-1.  k/v may be null (q-only RoPE).
hipError_t launch_rope_store(float* qkv, int ld, int tokens, int heads, int kv_heads, int hd, int start,
                             const float2* table, int interleaved, int write_q_f32, f16* q_f16, void* kcache,
                             void* vcache, int kv_f16, int capacity, hipStream_t st);

// decode GEMV (kernels_gemv.hip)
enum { GEMV_STORE = 0, GEMV_ADD = 1, GEMV_SWIGLU = 2, GEMV_QKV_ROPE = 3 };
// Input row: x, RMS-normalised x (norm != null), or the merge of split-K
// decode-attention partials [heads][splits][hd+2] (partials != null; with
// pos_dev set, only the splits covering positions 0..*pos_dev are read).
struct GemvInput {
    const float* x = nullptr;
    const float* norm = nullptr;
    float eps = 0.f;
    const float* partials = nullptr;
    int heads = 0, splits = 0, hd = 0, split_len = 0;
    const int* pos_dev = nullptr;
};
// QKV epilogue: rows [q | k | v] (q/k in adjacent RoPE pairs); q is rotated
// into out[0..QW), k rotated and v copied into the caches at row pos (taken
// from *pos_dev when set).
struct GemvRope {
    const float2* table = nullptr;
    int heads = 0, kv_heads = 0, hd = 0, capacity = 0, pos = 0;
    const int* pos_dev = nullptr;
    void* kc = nullptr;
    void* vc = nullptr;
    int kv_f16 = 1;
};
hipError_t launch_gemv_ex(const DevMatrix& w, const DevMatrix* w_up, const GemvInput& in, const GemvRope* rope,
                          float* out, int mode, hipStream_t st);
hipError_t launch_gemv(const DevMatrix& w, const DevMatrix* w_up, const float* x, const float* norm, float eps,
                       float* out, int mode, hipStream_t st);

// prefill GEMM (kernels_gemm.hip)
enum { GEMM_STORE = 0, GEMM_ACC = 1, GEMM_SWIGLU = 2 };
// fast: x f16 [m][k] (row stride ldx); MFMA f16 with f32 accumulate.
//   STORE/ACC write y f32 (row stride ldy); SWIGLU writes yh f16 (row stride ldy).
hipError_t launch_gemm_mfma(const f16* x, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up, float* y,
                            f16* yh, int ldy, int mode, hipStream_t st);
// exact: x f32; float32 FMA in the reference's per-block order.  SWIGLU writes y f32.
hipError_t launch_gemm_f32(const float* x, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up, float* y,
                           int ldy, int mode, hipStream_t st);

// attention (kernels_attention.hip).  Cache layout [kv_heads][capacity][hd].
// q rows are [tokens][heads][hd] with row stride ldq (elements).
hipError_t launch_flash_attention(const f16* q, int ldq, const f16* kc, const f16* vc, int capacity, int tokens,
                                  int heads, int kv_heads, int hd, int start, float* out_f32, f16* out_f16,
                                  hipStream_t st);
// Generic online-softmax attention, any hd <= 256, f16 or f32 cache, keys
// split into `splits` ranges merged by a second kernel when splits > 1.
int attention_splits(int length, int heads, int tokens);
size_t attention_partial_floats(int heads, int tokens, int splits, int hd);
// Decode (one query token at position length-1): split-K over the context,
// one workgroup per (KV head, split) for all query heads of the group; writes
// per-split partials [heads][splits][hd+2] merged by launch_attention_merge or
// by the Wo GEMV prologue.  Needs hd 64/128, heads/kv_heads <= 16.
// Context length = *pos_dev + 1 when pos_dev is set (device-side position),
// else `length`; `splits` workgroups of split_len positions (<= 256) each.
bool attention_decode_supported(int heads, int kv_heads, int hd);
int attention_decode_split_len(int capacity);
int attention_decode_max_split_len();
hipError_t launch_attention_decode(const float* q, const void* kc, const void* vc, int kv_f16, int capacity,
                                   int heads, int kv_heads, int hd, int length, const int* pos_dev, int split_len,
                                   int splits, float* partials, hipStream_t st);
hipError_t launch_attention_merge(const float* partials, int heads, int hd, int splits, float* out, hipStream_t st);
hipError_t launch_attention_generic(const float* q, int ldq, const void* kc, const void* vc, int kv_f16,
                                    int capacity, int tokens, int heads, int kv_heads, int hd, int start,
                                    int splits, float* partials, float* out, hipStream_t st);
