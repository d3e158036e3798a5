// Weight-chunk helpers shared by the decode GEMV kernels.
//
// A lane moves one 16-byte chunk of a row of a resident matrix (DevMatrix)
// with one global_load_dwordx4: 16 Q8_0 weights (half a block), one Q4_0
// block (32 weights), or 8 f16 weights.  chunk_dot multiplies the integer
// quants (or f16 values) by the float32 input staged in LDS and scales the
// chunk sum by the block's d once, so a Q8_0 or Q4_0 product enters the sum
// exactly as CPUOps.dot forms it (CPUOps.swift:106-139) up to float32
// summation order.
#pragma once

#include "common.h"

namespace gemv {

template <int FMT>
__device__ __forceinline__ int chunks_of(int K) {
    return FMT == DT_Q8_0 ? K >> 4 : FMT == DT_Q4_0 ? K >> 5 : K >> 3;
}

// The chunk's quants and its block scale, the scale kept as the f16 it is
// stored as: converting it where it is loaded made the compiler wait for each
// scale load before issuing the next quant load, which held a prefetched row
// back by a memory round trip.
template <int FMT>
__device__ __forceinline__ void load_chunk(const DevMatrix& m, int64_t row, int K, int c, int4& q, f16& d) {
    if (FMT == DT_Q8_0) {
        q = gload_i4(m.q + row * K + 16 * c);
        d = *gptr(m.s + row * (K >> 5) + (c >> 1));
    } else if (FMT == DT_Q4_0) {
        q = gload_i4(m.q + row * (K >> 1) + 16 * c);
        d = *gptr(m.s + row * (K >> 5) + c);
    } else {
        q = gload_i4(m.q + (row * K + 8 * c) * 2);
        d = (f16)1.0f;
    }
}

// Byte offsets of row `row`'s chunk c in the quant stream and of its scale
// (f16) in the scale stream.  With the matrix's base pointers wave-uniform,
// loads through load_q / load_s become global loads with the base in SGPRs,
// one 32-bit VGPR offset and an immediate: the chunks c0 + u * LPR of a row
// share one offset VGPR.  (With 64-bit per-load addresses, the compiler reused
// the address registers of loads still in flight as destinations of later
// loads and waited for those loads to retire first, which held the row's quant
// loads back behind its scale loads.)  Every operand spans less than 4 GiB.
template <int FMT>
__device__ __forceinline__ uint32_t chunk_qoff(int64_t row, int K, int c) {
    return FMT == DT_Q8_0   ? (uint32_t)(row * K + 16 * c)
           : FMT == DT_Q4_0 ? (uint32_t)(row * (K >> 1) + 16 * c)
                            : (uint32_t)(row * K * 2 + 16 * c);
}
template <int FMT>
__device__ __forceinline__ uint32_t chunk_soff(int64_t row, int K, int c) {
    return FMT == DT_Q8_0 ? (uint32_t)(2 * (row * (K >> 5) + (c >> 1))) : (uint32_t)(2 * (row * (K >> 5) + c));
}
// Byte steps between chunk c and chunk c + LPR (LPR even).
template <int FMT, int LPR>
constexpr uint32_t chunk_qstep() {
    return 16 * LPR;
}
template <int FMT, int LPR>
constexpr uint32_t chunk_sstep() {
    return FMT == DT_Q8_0 ? LPR : 2 * LPR;
}
__device__ __forceinline__ int4 load_q(const void* base, uint32_t off) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = *(const AS_GLOBAL v4i*)((const AS_GLOBAL char*)base + off);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ f16 load_s(const void* base, uint32_t off) {
    return *(const AS_GLOBAL f16*)((const AS_GLOBAL char*)base + off);
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

// One row's dot product, with the first batch of loads already in registers.
// Loads are issued unconditionally (a chunk index past the row is clamped to
// its last chunk and the value ignored) so that a batch leaves as back-to-back
// instructions rather than one branch, and one wait, per load.
template <int FMT, int LPR, int kUnroll = 4>
struct RowStream {
    int4 q[kUnroll];
    f16 d[kUnroll];
    __device__ __forceinline__ void prefetch(const DevMatrix& m, int64_t row, int K, int li) {
        const int nch = chunks_of<FMT>(K);
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int c = li + u * LPR;
            load_chunk<FMT>(m, row, K, c < nch ? c : nch - 1, q[u], d[u]);
        }
    }
    __device__ __forceinline__ float finish(const DevMatrix& m, int64_t row, int K, int li, const float* xs) {
        const int nch = chunks_of<FMT>(K);
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int c = li + u * LPR;
            if (c < nch) acc += chunk_dot<FMT>(q[u], (float)d[u], c, xs);
        }
        for (int c0 = li + kUnroll * LPR; c0 < nch; c0 += kUnroll * LPR) {
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int c = c0 + u * LPR;
                load_chunk<FMT>(m, row, K, c < nch ? c : nch - 1, q[u], d[u]);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int c = c0 + u * LPR;
                if (c < nch) acc += chunk_dot<FMT>(q[u], (float)d[u], c, xs);
            }
        }
        return acc;
    }
};


}  // namespace gemv
