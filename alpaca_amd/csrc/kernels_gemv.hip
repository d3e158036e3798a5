// Decode (single-token) dequant-GEMV for gfx950.
//
// Replaces the reference's fused decode mat-vecs (dec_f16 / dec_q8_0 /
// dec_q4_0, host side KernelEncoder.swift:358-399): out (+)= W * norm?(x),
// optionally silu(Wg x) * (Wu x).  The CPU semantics are CPUOps.linear / dot
// (CPUOps.swift:77-139) and CPUOps.rmsNorm (:144-159).
//
// Layout: each row of the quant stream is 16-byte aligned (DevMatrix), so a
// lane reads whole 16-byte chunks with one global_load_dwordx4:
//   Q8_0 chunk = 16 weights (half a block), Q4_0 chunk = 32 weights (one
//   block), F16 chunk = 8 weights.
// A group of LPR lanes owns one output row and strides over its chunks; each
// lane issues up to 4 chunk loads before consuming any, to keep enough bytes
// in flight per CU for HBM.  The (normalised) input row is staged once per
// workgroup in LDS and read back as float4.  Partial sums are combined with
// cross-lane shuffles; lane 0 of the group applies the epilogue.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;

struct GemvArgs {
    DevMatrix w, u;
    const float* x;
    const float* norm;
    float eps;
    float* out;
};

template <int FMT>
__device__ __forceinline__ int chunks_of(int K) {
    return FMT == DT_Q8_0 ? K >> 4 : FMT == DT_Q4_0 ? K >> 5 : K >> 3;
}

template <int FMT>
__device__ __forceinline__ void load_chunk(const DevMatrix& m, int64_t row, int K, int c, int4& q, float& d) {
    if (FMT == DT_Q8_0) {
        q = *(const int4*)(m.q + row * K + 16 * c);
        d = (float)m.s[row * (K >> 5) + (c >> 1)];
    } else if (FMT == DT_Q4_0) {
        q = *(const int4*)(m.q + row * (K >> 1) + 16 * c);
        d = (float)m.s[row * (K >> 5) + c];
    } else {
        q = *(const int4*)(m.q + (row * K + 8 * c) * 2);
        d = 1.f;
    }
}

template <int FMT>
__device__ __forceinline__ float chunk_dot(const int4& q, float d, int c, const float* xs) {
    const int32_t* w = (const int32_t*)&q;
    float s = 0.f;
    if (FMT == DT_Q8_0) {
        const float4* xv = (const float4*)(xs + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 x = xv[i];
            int32_t v = w[i];
            s += (float)(int8_t)(v) * x.x;
            s += (float)(int8_t)(v >> 8) * x.y;
            s += (float)(int8_t)(v >> 16) * x.z;
            s += (float)(int8_t)(v >> 24) * x.w;
        }
        return d * s;
    } else if (FMT == DT_Q4_0) {
        const float4* lo = (const float4*)(xs + 32 * c);
        const float4* hi = (const float4*)(xs + 32 * c + 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 xl = lo[i], xh = hi[i];
            uint32_t v = (uint32_t)w[i];
            s += (float)((int)(v & 15u) - 8) * xl.x;
            s += (float)((int)((v >> 4) & 15u) - 8) * xh.x;
            s += (float)((int)((v >> 8) & 15u) - 8) * xl.y;
            s += (float)((int)((v >> 12) & 15u) - 8) * xh.y;
            s += (float)((int)((v >> 16) & 15u) - 8) * xl.z;
            s += (float)((int)((v >> 20) & 15u) - 8) * xh.z;
            s += (float)((int)((v >> 24) & 15u) - 8) * xl.w;
            s += (float)((int)(v >> 28) - 8) * xh.w;
        }
        return d * s;
    } else {
        const f16* h = (const f16*)&q;
        const float4* xv = (const float4*)(xs + 8 * c);
        float4 x0 = xv[0], x1 = xv[1];
        s = (float)h[0] * x0.x + (float)h[1] * x0.y + (float)h[2] * x0.z + (float)h[3] * x0.w;
        s += (float)h[4] * x1.x + (float)h[5] * x1.y + (float)h[6] * x1.z + (float)h[7] * x1.w;
        return s;
    }
}

template <int FMT, int LPR>
__device__ __forceinline__ float row_dot(const DevMatrix& m, int64_t row, int K, const float* xs, int li) {
    const int nch = chunks_of<FMT>(K);
    float acc = 0.f;
    for (int c0 = li; c0 < nch; c0 += kUnroll * LPR) {
        int4 q[kUnroll];
        float d[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            int c = c0 + u * LPR;
            if (c < nch) load_chunk<FMT>(m, row, K, c, q[u], d[u]);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            int c = c0 + u * LPR;
            if (c < nch) acc += chunk_dot<FMT>(q[u], d[u], c, xs);
        }
    }
    return acc;
}

template <int FMT, int LPR, int MODE, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ float xs[];
    __shared__ float red[16];
    const int K = a.w.cols;
    float scale = 1.f;
    if (NORM) {
        float ss = 0.f;
        for (int i = threadIdx.x; i < K; i += kThreads) ss += a.x[i] * a.x[i];
        ss = block_sum(ss, red);
        scale = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = NORM ? (a.x[i] * scale) * a.norm[i] : a.x[i];
    __syncthreads();

    constexpr int kRowsPerWave = 64 / LPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane % LPR;
    const int64_t row = ((int64_t)blockIdx.x * kWaves + wave) * kRowsPerWave + lane / LPR;
    const bool valid = row < a.w.rows;
    float acc = 0.f, acc2 = 0.f;
    if (valid) {
        acc = row_dot<FMT, LPR>(a.w, row, K, xs, li);
        if (MODE == GEMV_SWIGLU) acc2 = row_dot<FMT, LPR>(a.u, row, K, xs, li);
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
        acc += __shfl_xor(acc, o, 64);
        if (MODE == GEMV_SWIGLU) acc2 += __shfl_xor(acc2, o, 64);
    }
    if (valid && li == 0) {
        if (MODE == GEMV_STORE) a.out[row] = acc;
        else if (MODE == GEMV_ADD) a.out[row] += acc;
        else a.out[row] = (acc / (1.0f + expf(-acc))) * acc2;
    }
}

template <int FMT, int MODE, bool NORM>
hipError_t dispatch(int lpr, const GemvArgs& a, hipStream_t st) {
    const int rows_per_block = kWaves * (64 / lpr);
    const int grid = (a.w.rows + rows_per_block - 1) / rows_per_block;
    const size_t lds = (size_t)a.w.cols * sizeof(float);
    switch (lpr) {
    case 16: gemv_kernel<FMT, 16, MODE, NORM><<<grid, kThreads, lds, st>>>(a); break;
    case 32: gemv_kernel<FMT, 32, MODE, NORM><<<grid, kThreads, lds, st>>>(a); break;
    default: gemv_kernel<FMT, 64, MODE, NORM><<<grid, kThreads, lds, st>>>(a); break;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t dispatch_fmt(int lpr, int mode, bool norm, const GemvArgs& a, hipStream_t st) {
    if (mode == GEMV_STORE) return norm ? dispatch<FMT, GEMV_STORE, true>(lpr, a, st) : dispatch<FMT, GEMV_STORE, false>(lpr, a, st);
    if (mode == GEMV_ADD) return norm ? dispatch<FMT, GEMV_ADD, true>(lpr, a, st) : dispatch<FMT, GEMV_ADD, false>(lpr, a, st);
    return norm ? dispatch<FMT, GEMV_SWIGLU, true>(lpr, a, st) : dispatch<FMT, GEMV_SWIGLU, false>(lpr, a, st);
}

}  // namespace

// Lanes per row: enough workgroups to cover the chip for tall matrices, whole
// waves per row for short ones (the decode matrices of small models are
// latency-bound, so more rows in flight matter more than lane utilisation).
static int pick_lpr(int rows) {
    if ((rows + 15) / 16 >= 1024) return 16;
    if ((rows + 7) / 8 >= 1024) return 32;
    return 64;
}

hipError_t launch_gemv(const DevMatrix& w, const DevMatrix* w_up, const float* x, const float* norm, float eps,
                       float* out, int mode, hipStream_t st) {
    GemvArgs a;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.x = x;
    a.norm = norm;
    a.eps = eps;
    a.out = out;
    const int lpr = pick_lpr(w.rows);
    const bool nrm = norm != nullptr;
    switch (w.dtype) {
    case DT_Q8_0: return dispatch_fmt<DT_Q8_0>(lpr, mode, nrm, a, st);
    case DT_Q4_0: return dispatch_fmt<DT_Q4_0>(lpr, mode, nrm, a, st);
    default: return dispatch_fmt<DT_F16>(lpr, mode, nrm, a, st);
    }
}
