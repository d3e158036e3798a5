// Prefill dequant-GEMMs for gfx950: Y[M tokens, N rows] (+)= X[M,K] * W[N,K]^T.
//
// Replaces the reference's batched projections: the fast tensor-op GEMMs
// (gemm_tensor_half_w[_acc], gemm_tensor_gateup_silu, tensor_gemm.metal) and
// the exact simdgroup GEMM (mm_*, matmul.metal), host side
// KernelEncoder.swift:192-280.  CPU semantics: CPUOps.linear / dot
// (CPUOps.swift:77-139).
//
// Fast path (f16 MFMA): quantised weights enter as their integer quants in f16
// (exact) with the per-block f16 scale kept in float32; one
// v_mfma_f32_16x16x32_f16 covers one 32-weight block and its result is scaled
// by d before accumulation.  The activations enter either as one f16 term
// (TT = false: the only input rounding is float32 -> f16, 2^-11 relative) or
// as two, hi = f16(x) and lo = f16(x - hi) (TT = true), which carry x to
// ~2^-22: both terms are multiplied by the same exact quants and summed in the
// block's float32 result before the scaling, so the product keeps float32
// accuracy at twice the MFMA work.  (Rounding half(d*q) as the reference's
// tensor-op path does moves C1 prefill logits past the 2e-3 bound against the
// CPU reference; single-term activations keep C1 inside it but not the larger
// configurations.)
//   dgemm_kernel: global -> LDS DMA, three stages in flight (the default).
//   gemm_mfma_kernel: register-staged, double-buffered; shapes the DMA kernel
//   does not take.
// Epilogues: store f32, accumulate into the f32 residual, or SwiGLU
// (silu(x Wg^T) * (x Wu^T) from two accumulator sets) written as f16.
//
// gemm_f32_kernel (exact): float32 SIMT tiles 64x64, BK = 32 = one block.
// Inside a block the products are summed in the CPU reference's order and the
// block sum is scaled once (acc += d * s), with FP contraction off, so each
// output equals the CPU reference's float32 result.
#include "common.h"

#include <type_traits>

#include <cstdlib>
#include <cstring>

namespace {

// ------------------------------------------------------------------ MFMA path
constexpr int BK = 64;
constexpr int LDT = BK + 8;  // LDS row pitch in halves (144 B: staggers banks)

struct GemmArgs {
    const f16* x;
    const f16* xlo = nullptr;  // the activations' second term (two-term kernels)
    int ldx, M;
    DevMatrix w, u;
    float* y;
    f16* yh;
    f16* yhlo = nullptr;  // f16 outputs' second term, written for rows >= lo_out_row0
    int ldy;
    // Two-term kernels: tiles holding a row >= lo_row0 or a column >= lo_col0
    // take the activations' second term, the others one term; the second term
    // of f16 outputs is written for rows >= lo_out_row0 only.
    int lo_row0 = 0, lo_out_row0 = 0, lo_col0 = 1 << 30;
    // Tiles in row groups of group_m row blocks, column by column inside a
    // group (0: row by row); set per launch by run_dgemm.
    int group_m = 0;
    QkvRope qkv;  // GEMM_QKV_ROPE only (yh = qkv.qh, ldy = heads * hd)
};

template <int FMT>
struct BUnit {
    int4 q0, q1;
    float d;
};

// Load 16 consecutive weights (row n, columns k..k+15) of one matrix.
template <int FMT>
__device__ __forceinline__ void b_load(const DevMatrix& m, int n, int k, int K, BUnit<FMT>& u) {
    const int nb = K >> 5;
    if (FMT == DT_Q8_0) {
        u.q0 = *(const int4*)(m.q + (int64_t)n * K + k);
        u.d = (float)m.s[(int64_t)n * nb + (k >> 5)];
    } else if (FMT == DT_Q4_0) {
        u.q0 = *(const int4*)(m.q + ((int64_t)n * nb + (k >> 5)) * 16);
        u.d = (float)m.s[(int64_t)n * nb + (k >> 5)];
    } else {
        const int4* p = (const int4*)(m.q + ((int64_t)n * K + k) * 2);
        u.q0 = p[0];
        u.q1 = p[1];
    }
}

// Stores a unit as 16 halves.  Quantised formats store the integer quants
// (q for Q8_0, nib-8 for Q4_0), which f16 holds exactly; the block scale d is
// kept in float32 and applied to each block's MFMA result, so the weights
// enter the product without rounding.  F16 weights are stored as they are.
template <int FMT>
__device__ __forceinline__ void b_store(const BUnit<FMT>& u, int k, f16* dst, float* dscale) {
    f16x8 h0, h1;
    if (FMT == DT_Q8_0) {
        const int8_t* q = (const int8_t*)&u.q0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            h0[j] = (f16)(float)q[j];
            h1[j] = (f16)(float)q[8 + j];
        }
    } else if (FMT == DT_Q4_0) {
        const uint8_t* q = (const uint8_t*)&u.q0;
        const int sh = (k & 16) ? 4 : 0;  // low nibbles: elements 0..15 of the block, high: 16..31
#pragma unroll
        for (int j = 0; j < 8; j++) {
            h0[j] = (f16)(float)((int)((q[j] >> sh) & 15) - 8);
            h1[j] = (f16)(float)((int)((q[8 + j] >> sh) & 15) - 8);
        }
    } else {
        h0 = *(const f16x8*)&u.q0;
        h1 = *(const f16x8*)&u.q1;
    }
    *(f16x8*)dst = h0;
    *(f16x8*)(dst + 8) = h1;
    if (FMT != DT_F16 && (k & 16) == 0) *dscale = u.d;
}

template <int FMT, int BM, int BN, int MODE, bool TT>
__global__ __launch_bounds__(256, 2) void gemm_mfma_kernel(GemmArgs p) {
    constexpr int NB = MODE == GEMM_SWIGLU ? 2 : 1;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16;
    constexpr int SA = BM * (BK / 8) / 256;  // 16-byte A segments per thread
    constexpr int UB = BN * (BK / 16) / 256; // 16-weight B units per thread per matrix
    static_assert(SA >= 1 && UB >= 1, "tile too small for 256 threads");

    constexpr bool kQuant = FMT != DT_F16;
    __shared__ __attribute__((aligned(16))) f16 As[2][BM][LDT];
    __shared__ __attribute__((aligned(16))) f16 Al[TT ? 2 : 1][TT ? BM : 1][LDT];  // second term
    __shared__ __attribute__((aligned(16))) f16 Bs[2][NB][BN][LDT];
    __shared__ float Ds[2][NB][BN][BK / 32];  // block scales of the stage

    const int K = p.w.cols, N = p.w.rows, M = p.M;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (K + BK - 1) / BK;
    // Tiles before lo_row0 take one term: their second-term rows are not read
    // (they may hold stale data) and enter as zeros, which add nothing.
    const bool use_lo = m0 + BM > p.lo_row0;

    int4 ra[SA], rl[TT ? SA : 1];
    BUnit<FMT> rb[NB][UB];

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < SA; i++) {
            const int seg = tid + 256 * i, r = seg >> 3, c = (seg & 7) * 8;
            int4 v = {0, 0, 0, 0}, vl = {0, 0, 0, 0};
            if (m0 + r < M && k0 + c < K) {
                v = *(const int4*)(p.x + (int64_t)(m0 + r) * p.ldx + k0 + c);
                if constexpr (TT)
                    if (use_lo) vl = *(const int4*)(p.xlo + (int64_t)(m0 + r) * p.ldx + k0 + c);
            }
            ra[i] = v;
            if constexpr (TT) rl[i] = vl;
        }
#pragma unroll
        for (int mat = 0; mat < NB; mat++)
#pragma unroll
            for (int i = 0; i < UB; i++) {
                const int unit = tid + 256 * i, r = unit >> 2, k = k0 + (unit & 3) * 16;
                if (n0 + r < N && k < K) {
                    b_load<FMT>(mat ? p.u : p.w, n0 + r, k, K, rb[mat][i]);
                } else {
                    rb[mat][i].q0 = int4{0, 0, 0, 0};
                    rb[mat][i].q1 = int4{0, 0, 0, 0};
                    rb[mat][i].d = 0.f;
                }
            }
    };
    auto sstore = [&](int buf, int kt) {
#pragma unroll
        for (int i = 0; i < SA; i++) {
            const int seg = tid + 256 * i, r = seg >> 3, c = (seg & 7) * 8;
            *(int4*)&As[buf][r][c] = ra[i];
            if constexpr (TT) *(int4*)&Al[buf][r][c] = rl[i];
        }
#pragma unroll
        for (int mat = 0; mat < NB; mat++)
#pragma unroll
            for (int i = 0; i < UB; i++) {
                const int unit = tid + 256 * i, r = unit >> 2, kk = (unit & 3) * 16;
                b_store<FMT>(rb[mat][i], kt * BK + kk, &Bs[buf][mat][r][kk], &Ds[buf][mat][r][kk >> 5]);
            }
    };

    f32x4 acc[NB][TM][TN];
#pragma unroll
    for (int mat = 0; mat < NB; mat++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[mat][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    gload(0);
    sstore(0, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 32; kk++) {
            f16x8 af[TM], al[TT ? TM : 1];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                af[i] = *(const f16x8*)&As[cur][wm * WM + 16 * i + (lane & 15)][32 * kk + 8 * (lane >> 4)];
                if constexpr (TT) al[i] = *(const f16x8*)&Al[cur][wm * WM + 16 * i + (lane & 15)][32 * kk + 8 * (lane >> 4)];
            }
#pragma unroll
            for (int mat = 0; mat < NB; mat++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int br = wn * WN + 16 * j + (lane & 15);
                    f16x8 bf = *(const f16x8*)&Bs[cur][mat][br][32 * kk + 8 * (lane >> 4)];
                    if (kQuant) {
                        // One 16x16x32 MFMA spans exactly one quant block: exact integer
                        // products summed in float32, then scaled once by the block's d.
                        const float d = Ds[cur][mat][br][kk];
#pragma unroll
                        for (int i = 0; i < TM; i++) {
                            f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            if constexpr (TT) t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf, t, 0, 0, 0);
                            acc[mat][i][j] += d * t;
                        }
                        // keep one column tile of block results live at a time (register budget)
                        __builtin_amdgcn_sched_barrier(0);
                    } else {
#pragma unroll
                        for (int i = 0; i < TM; i++) {
                            acc[mat][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[mat][i][j], 0, 0, 0);
                            if constexpr (TT)
                                acc[mat][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf, acc[mat][i][j], 0, 0, 0);
                        }
                    }
                }
        }
        if (kt + 1 < nk) sstore(cur ^ 1, kt + 1);
        __syncthreads();
    }

    // C layout of 16x16 MFMA: lane holds rows 4*(lane/16)+r, column lane%16.
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WN + 16 * j + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
                if (m >= M) continue;
                const int64_t o = (int64_t)m * p.ldy + n;
                if (MODE == GEMM_STORE) {
                    p.y[o] = acc[0][i][j][r];
                } else if (MODE == GEMM_ACC) {
                    p.y[o] += acc[0][i][j][r];
                } else {
                    const float g = acc[0][i][j][r], u = acc[NB - 1][i][j][r];
                    const float v = (g / (1.0f + __expf(-g))) * u;
                    const f16 hv = (f16)v;
                    p.yh[o] = hv;
                    if (p.yhlo && m >= p.lo_out_row0) p.yhlo[o] = (f16)(v - (float)hv);
                }
            }
        }
}

template <int FMT, int BM, int BN, bool TT>
hipError_t run_mfma(const GemmArgs& a, int mode, hipStream_t st) {
    dim3 grid((a.M + BM - 1) / BM, (a.w.rows + BN - 1) / BN);
    if (mode == GEMM_STORE) gemm_mfma_kernel<FMT, BM, BN, GEMM_STORE, TT><<<grid, 256, 0, st>>>(a);
    else if (mode == GEMM_ACC) gemm_mfma_kernel<FMT, BM, BN, GEMM_ACC, TT><<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

template <int FMT, int BM, int BN, bool TT>
hipError_t run_mfma_swiglu(const GemmArgs& a, hipStream_t st) {
    dim3 grid((a.M + BM - 1) / BM, (a.w.rows + BN - 1) / BN);
    gemm_mfma_kernel<FMT, BM, BN, GEMM_SWIGLU, TT><<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

// Tiles: 64x64 for short batches and for SwiGLU (two accumulator sets);
// otherwise 128 tokens x 64 rows (quantised formats keep two waves per SIMD
// there: the per-block scaling holds a second set of MFMA results in
// registers), and 128x128 for F16 weights when the grid covers the chip twice.
template <int FMT, bool TT>
hipError_t pick_tile(const GemmArgs& a, int mode, hipStream_t st) {
    const int M = a.M, N = a.w.rows;
    if (mode == GEMM_SWIGLU) return run_mfma_swiglu<FMT, 64, 64, TT>(a, st);
    if (M <= 64) return run_mfma<FMT, 64, 64, TT>(a, mode, st);
    const long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if constexpr (FMT == DT_F16) {
        if (big >= 512) return run_mfma<FMT, 128, 128, TT>(a, mode, st);
    }
    return run_mfma<FMT, 128, 64, TT>(a, mode, st);
}

template <int FMT>
hipError_t pick_tile_terms(const GemmArgs& a, int mode, hipStream_t st) {
    return a.xlo ? pick_tile<FMT, true>(a, mode, st) : pick_tile<FMT, false>(a, mode, st);
}

// ------------------------------------------------------------------ exact path
constexpr int FB = 64;       // tile edge (tokens and rows)
constexpr int FK = 32;       // one quant block per stage
constexpr int FP = FB + 4;   // LDS pitch in floats

struct GemmF32Args {
    const float* x;
    int ldx, M;
    DevMatrix w, u;
    float* y;
    int ldy;
};

// Weight (row n, column k) as an unscaled value: q for Q8_0, nib-8 for Q4_0,
// the f16 value for F16.  The block scale is applied once per block sum.
template <int FMT>
__device__ __forceinline__ float w_raw(const DevMatrix& m, int n, int k, int K) {
    if (FMT == DT_Q8_0) return (float)((const int8_t*)m.q)[(int64_t)n * K + k];
    if (FMT == DT_Q4_0) {
        const int j = k & 31;
        const uint8_t b = m.q[((int64_t)n * (K >> 5) + (k >> 5)) * 16 + (j & 15)];
        return (float)((int)(j < 16 ? (b & 15) : (b >> 4)) - 8);
    }
    return (float)((const f16*)m.q)[(int64_t)n * K + k];
}

template <int FMT, int MODE>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32Args p) {
#pragma clang fp contract(off)
    constexpr int NB = MODE == GEMM_SWIGLU ? 2 : 1;
    constexpr bool kQuant = FMT != DT_F16;
    __shared__ float Xs[FK][FP];
    __shared__ float Ws[NB][FK][FP];
    __shared__ float Ds[NB][FB];

    const int K = p.w.cols, N = p.w.rows, M = p.M;
    const int m0 = blockIdx.x * FB, n0 = blockIdx.y * FB;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;

    float acc[NB][4][4];
#pragma unroll
    for (int mat = 0; mat < NB; mat++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[mat][i][j] = 0.f;

    const int lr = tid >> 2, lk = (tid & 3) * 8;
    for (int k0 = 0; k0 < K; k0 += FK) {
        {
            const int m = m0 + lr;
#pragma unroll
            for (int j = 0; j < 8; j++) Xs[lk + j][lr] = m < M ? p.x[(int64_t)m * p.ldx + k0 + lk + j] : 0.f;
        }
#pragma unroll
        for (int mat = 0; mat < NB; mat++) {
            const DevMatrix& w = mat ? p.u : p.w;
            const int n = n0 + lr;
#pragma unroll
            for (int j = 0; j < 8; j++) Ws[mat][lk + j][lr] = n < N ? w_raw<FMT>(w, n, k0 + lk + j, K) : 0.f;
            if (kQuant && lk == 0) Ds[mat][lr] = n < N ? (float)w.s[(int64_t)n * (K >> 5) + (k0 >> 5)] : 0.f;
        }
        __syncthreads();
        if (kQuant) {
            float blk[NB][4][4];
#pragma unroll
            for (int mat = 0; mat < NB; mat++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) blk[mat][i][j] = 0.f;
            // CPU order inside a block: Q8_0 k = 0..31; Q4_0 k = j, j+16 for j = 0..15.
#pragma unroll 4
            for (int s = 0; s < FK; s++) {
                const int k = FMT == DT_Q4_0 ? ((s & 1) ? 16 + (s >> 1) : (s >> 1)) : s;
                const float4 xv = *(const float4*)&Xs[k][ty * 4];
                const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int mat = 0; mat < NB; mat++) {
                    const float4 wv = *(const float4*)&Ws[mat][k][tx * 4];
                    const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float t = wa[j] * xa[i];
                            blk[mat][i][j] += t;
                        }
                }
            }
#pragma unroll
            for (int mat = 0; mat < NB; mat++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float d = Ds[mat][tx * 4 + j];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float t = d * blk[mat][i][j];
                        acc[mat][i][j] += t;
                    }
                }
        } else {
#pragma unroll 4
            for (int k = 0; k < FK; k++) {
                const float4 xv = *(const float4*)&Xs[k][ty * 4];
                const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int mat = 0; mat < NB; mat++) {
                    const float4 wv = *(const float4*)&Ws[mat][k][tx * 4];
                    const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float t = wa[j] * xa[i];
                            acc[mat][i][j] += t;
                        }
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + tx * 4 + j;
            if (n >= N) continue;
            const int64_t o = (int64_t)m * p.ldy + n;
            if (MODE == GEMM_STORE) {
                p.y[o] = acc[0][i][j];
            } else if (MODE == GEMM_ACC) {
                p.y[o] = p.y[o] + acc[0][i][j];
            } else {
                const float g = acc[0][i][j];
                const float e = expf(-g);
                const float den = 1.0f + e;
                p.y[o] = (g / den) * acc[NB - 1][i][j];
            }
        }
    }
}

template <int FMT>
hipError_t run_f32(const GemmF32Args& a, int mode, hipStream_t st) {
    dim3 grid((a.M + FB - 1) / FB, (a.w.rows + FB - 1) / FB);
    if (mode == GEMM_STORE) gemm_f32_kernel<FMT, GEMM_STORE><<<grid, 256, 0, st>>>(a);
    else if (mode == GEMM_ACC) gemm_f32_kernel<FMT, GEMM_ACC><<<grid, 256, 0, st>>>(a);
    else gemm_f32_kernel<FMT, GEMM_SWIGLU><<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace

// Register-staged kernel: shapes the LDS-DMA kernel does not take (K not a
// multiple of 64, activation rows not 16-byte aligned).
static hipError_t launch_gemm_mfma_staged(const f16* x, const f16* xlo, int ldx, int m, const DevMatrix& w,
                                         const DevMatrix* w_up, float* y, f16* yh, f16* yhlo, int ldy, int mode,
                                         hipStream_t st, int lo_row0, int lo_out_row0) {
    if (m <= 0) return hipSuccess;
    GemmArgs a;
    a.x = x;
    a.xlo = xlo;
    a.yhlo = yhlo;
    a.ldx = ldx;
    a.M = m;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.y = y;
    a.yh = yh;
    a.ldy = ldy;
    a.lo_row0 = lo_row0;
    a.lo_out_row0 = lo_out_row0;
    switch (w.dtype) {
    case DT_Q8_0: return pick_tile_terms<DT_Q8_0>(a, mode, st);
    case DT_Q4_0: return pick_tile_terms<DT_Q4_0>(a, mode, st);
    default: return pick_tile_terms<DT_F16>(a, mode, st);
    }
}

hipError_t launch_gemm_f32(const float* x, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up, float* y,
                           int ldy, int mode, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    GemmF32Args a;
    a.x = x;
    a.ldx = ldx;
    a.M = m;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.y = y;
    a.ldy = ldy;
    switch (w.dtype) {
    case DT_Q8_0: return run_f32<DT_Q8_0>(a, mode, st);
    case DT_Q4_0: return run_f32<DT_Q4_0>(a, mode, st);
    default: return run_f32<DT_F16>(a, mode, st);
    }
}

// ------------------------------------------------------------------ LDS-DMA pipelined GEMM
//
// Same arithmetic as gemm_mfma_kernel (integer quants exact in f16, f16
// activations, one v_mfma_f32_16x16x32_f16 per 32-weight block whose float32
// result is scaled by the block's d and accumulated), built for latency: the
// prefill projections are thin (K = 576..8192, a few hundred tiles on 256
// CUs), so each workgroup keeps several K stages of loads in flight.  Stages
// are 64 wide in K (two quant blocks) and move global -> LDS with
// global_load_lds_dwordx4 (no VGPR staging, no LDS store instructions): stage
// kt+2 is in flight while stage kt is multiplied; three LDS buffers, one
// barrier per stage.  The DMA writes 64 lanes x 16 bytes contiguously, so the
// LDS layout is fixed per instruction and the lane -> global-address map does
// the swizzling:
//   A / F16 weights: rows of 128 B (8 chunks of 16 B), chunk c of row r at
//     slot c ^ swz_a(r), swz_a(r) = (r & 7) ^ ((r >> 1) & 4), which puts the
//     16 rows one MFMA fragment read touches in 16 distinct 16-byte bank groups;
//   Q8_0 quants: rows of 64 B (4 chunks), slot c ^ ((r >> 2) & 3);
//   Q4_0 nibbles: rows of 32 B (2 blocks), slot c ^ ((r >> 3) & 1);
//   scales: the stage's 2 f16 per row, from the stage-major copy (s2).
// Quants become f16 per MFMA fragment after the LDS read (8 bytes -> 8 halves
// with a byte permute and a packed-f16 subtract: 0x64xx is 1024 + xx, so
// (1024 + q + 128) - 1152 = q exactly).  Tiles are taken in an XCD-major
// order so that tiles sharing A rows run on one XCD and share its L2.
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// 4 signed bytes -> 2 dwords holding the 4 quants as f16 pairs (exact).
__device__ __forceinline__ void int8x4_to_f16(uint32_t w, uint32_t& o0, uint32_t& o1) {
    const uint32_t u = w ^ 0x80808080u;  // q + 128 in each byte
    const h2 bias = {(f16)1152.0f, (f16)1152.0f};
    o0 = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    o1 = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}
// 4 nibbles (one per byte, already masked) -> nib - 8 as f16 pairs (exact).
__device__ __forceinline__ void nib4_to_f16(uint32_t nib, uint32_t& o0, uint32_t& o1) {
    const h2 bias = {(f16)1032.0f, (f16)1032.0f};
    o0 = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u)) - bias);
    o1 = as_u32(as_h2(__builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u)) - bias);
}

constexpr int DBK = 64;  // K per stage

__device__ __forceinline__ int swz_a(int r) { return (r & 7) ^ ((r >> 1) & 4); }
__device__ __forceinline__ int swz_q8(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int swz_q4(int r) { return (r >> 3) & 1; }

// Byte layout of one stage buffer: A rows (the second term's A rows after
// them, two-term kernels), then each matrix's weight rows, then each matrix's
// scales.
template <int FMT, int BM, int BN, int NB, bool TT>
struct DStage {
    static constexpr int BROW = FMT == DT_Q8_0 ? 64 : FMT == DT_Q4_0 ? 32 : 128;  // weight bytes per row
    static constexpr int SROW = FMT == DT_F16 ? 0 : 4;                             // scale bytes per row
    static constexpr int A_LO = BM * DBK * 2;
    static constexpr int B_OFF = BM * DBK * 2 * (TT ? 2 : 1);
    static constexpr int S_OFF = B_OFF + NB * BN * BROW;
    static constexpr int BYTES = S_OFF + NB * BN * SROW + 16;
};

template <int FMT, int BM, int BN, int WM, int WN, int MODE, bool TT>
struct DGemm {
    static constexpr int NB = MODE == GEMM_SWIGLU ? 2 : 1;
    static constexpr int TM = WM / 16, TN = WN / 16;
    // waves per workgroup: four (one per SIMD) or eight (two per SIMD, so that
    // one wave's VALU work can issue while the other's MFMAs run)
    static constexpr int NW = (BM / WM) * (BN / WN);
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    // DMA instructions per wave per stage (A rows: 8 of 128 B per instruction; twice with two terms)
    static constexpr int A_I = BM / (8 * NW);
    static constexpr bool Q4_16 = (BN / 8) % (4 * NW) == 0;
    static constexpr int B_I = FMT == DT_Q8_0   ? BN / (16 * NW)
                               : FMT == DT_Q4_0 ? (Q4_16 ? BN / (32 * NW) : BN / (8 * NW))
                                                : BN / (8 * NW);
    static constexpr int S_I = FMT == DT_F16 ? 0 : 1;  // 1/NW of the tile's scale pairs per wave
    static constexpr int PER = A_I * (TT ? 2 : 1) + NB * (B_I + S_I);
    static_assert(A_I >= 1 && B_I >= 1 && BM % (8 * NW) == 0 && BN % (16 * NW) == 0 && BN / (4 * NW) <= 64,
                  "tile shape");
};

// Epilogues that read memory (GEMM_ACC reads the residual rows, GEMM_QKV_ROPE
// the RoPE table) work in 16-row groups (i) of the lane's C fragments and load
// group i+1 before storing group i.  The vector memory counter retires in
// order, so a load issued after a store waits for that store too; and the
// compiler cannot reorder y[m*ldy+n] loads over stores it cannot prove
// disjoint.  Written per element, every element would cost a full round trip.
// Loads of rows or columns past the edge are clamped to the last valid one and
// their results never stored.

// GEMM_ACC: y += acc.  A wave whose fragments lie inside the matrix (the
// usual case) stores without per-element edge tests.
template <int TM, int TN>
__device__ __forceinline__ void acc_epilogue(const GemmArgs& p, const f32x4 (&acc)[TM][TN], int mb, int nb, int M,
                                             int N, int lane) {
    const bool full = mb + 16 * TM <= M && nb + 16 * TN <= N;  // wave-uniform
    float cur[TN][4], nxt[TN][4];
    auto load = [&](int i, float (&v)[TN][4]) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = min(nb + 16 * j + (lane & 15), N - 1);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = min(mb + 16 * i + 4 * (lane >> 4) + r, M - 1);
                v[j][r] = p.y[(int64_t)m * p.ldy + n];
            }
        }
    };
    auto run = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        load(0, cur);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if (i + 1 < TM) load(i + 1, nxt);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nb + 16 * j + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mb + 16 * i + 4 * (lane >> 4) + r;
                    if (FULL || (n < N && m < M)) p.y[(int64_t)m * p.ldy + n] = cur[j][r] + acc[i][j][r];
                }
            }
            if (i + 1 < TM) {
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) cur[j][r] = nxt[j][r];
            }
        }
    };
    if (full) run(std::true_type{});
    else run(std::false_type{});
}

// GEMM_QKV_ROPE.  Columns [0, QW) are q, [QW, QW+KW) k, then v.  A 16-column
// fragment never straddles a head (hd % 16 == 0), so its region (q, k or v),
// head and destination are wave-uniform and each element is one select chain
// and one store.  Interleaved RoPE pairs (columns 2i, 2i+1) sit in
// neighbouring lanes of the C layout: each lane takes its partner's value
// with a DPP quad swap (every lane, before any edge test).  The (cos, sin)
// rows of the tile's positions are one contiguous block of the table; the
// workgroup copies it into the idle stage buffers with one batch of 16-byte
// loads and lanes read their pairs from LDS.  The rotation is evaluated
// without contraction as own*c + partner*(odd ? s : -s): for an even lane
// (a = own, b = partner) that is a*c + (-(b*s)) == a*c - b*s exactly, for an
// odd lane (b = own, a = partner) b*c + a*s == a*s + b*c, so q/k are bit for
// bit those of rope_store_kernel (CPUOps.rope, CPUOps.swift:184-212;
// KVCache.write, KVCache.swift:44-63).  smem holds at least BM * hd/2 float2.
template <int BM, int TM, int TN, bool TT>
__device__ __forceinline__ void qkv_rope_epilogue(const GemmArgs& p, const f32x4 (&acc)[TM][TN], uint8_t* smem,
                                                  int m0, int mb, int nb, int M, int N, int lane, bool active = true) {
#pragma clang fp contract(off)
    const QkvRope& o = p.qkv;
    const int hd = o.hd, half = hd / 2, QW = o.heads * hd, KW = o.kv_heads * hd;
    {
        const int total = min(BM, M - m0) * half / 2;  // float4 = two (cos, sin) pairs
        const float4* src = (const float4*)(o.rope + (int64_t)(o.pos + m0) * half);
        float4* dst = (float4*)smem;
        const int nt = blockDim.x;
        for (int base = 0; base < total; base += 8 * nt) {
            float4 v[8];  // loads clamped to the last element (valid memory), stores guarded
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = src[min(base + (int)threadIdx.x + nt * u, total - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int k = base + threadIdx.x + nt * u;
                if (k < total) dst[k] = v[u];
            }
        }
        __syncthreads();
    }
    if (!active) return;
    const float2* cs_rows = (const float2*)smem;
    const bool full = mb + 16 * TM <= M;  // wave-uniform
    const bool odd = lane & 1;
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int g0 = __builtin_amdgcn_readfirstlane(nb + 16 * j);  // first column of the fragment
        if (g0 >= N) break;                                           // N % 16 == 0: whole fragments
        const int region = g0 < QW ? 0 : g0 < QW + KW ? 1 : 2;
        const int cn0 = g0 - (region == 0 ? 0 : region == 1 ? QW : QW + KW);
        const int h = cn0 / hd, d = cn0 - h * hd + (lane & 15);
        // element (m, column) lives at dst + m * stride (a 32-bit offset: m < M, stride <= heads * hd)
        f16* dst;
        f16* dlo = nullptr;  // q's second term (two-term kernels)
        int stride;
        if (region == 0) {
            dst = p.yh + g0 + (lane & 15);
            if (p.yhlo) dlo = p.yhlo + g0 + (lane & 15);
            stride = p.ldy;
        } else {
            dst = (region == 1 ? o.kc : o.vc) + ((int64_t)h * o.capacity + o.pos) * hd + d;
            stride = hd;
        }
        const float2* cs_col = cs_rows + d / 2;
        auto run = [&](auto full_c, auto rot_c) {
            constexpr bool FULL = decltype(full_c)::value, ROT = decltype(rot_c)::value;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                float pv[4];
                if constexpr (ROT) {
#pragma unroll
                    for (int r = 0; r < 4; r++) pv[r] = dpp_mov<0xB1>(acc[i][j][r]);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mb + 16 * i + 4 * (lane >> 4) + r;
                    float out = acc[i][j][r];
                    if constexpr (ROT) {
                        const float2 cs = cs_col[(m - m0) * half];
                        const float t1 = out * cs.x, t2 = pv[r] * (odd ? cs.y : -cs.y);
                        out = t1 + t2;
                    }
                    if (FULL || m < M) {
                        const f16 ho = (f16)out;
                        dst[m * stride] = ho;
                        if (dlo && m >= p.lo_out_row0) dlo[m * stride] = (f16)(out - (float)ho);
                    }
                }
            }
        };
        if (full) {
            if (region != 2) run(std::true_type{}, std::true_type{});
            else run(std::true_type{}, std::false_type{});
        } else {
            if (region != 2) run(std::false_type{}, std::true_type{});
            else run(std::false_type{}, std::false_type{});
        }
    }
}

// RH: for GEMM_QKV_ROPE, the largest head dim the RoPE staging holds (64 or
// 128); 0 for the other modes.
// KS sets of NW waves each take a contiguous share of the K stages (their own
// stage buffers) and add their accumulators through LDS at the end: on grids
// of about one workgroup per CU, twice the waves per CU and half the
// sequential stage loop per workgroup.  (The split changes the float32
// summation order of each output, so a KS = 2 tile agrees with the others to
// rounding, not bit for bit.)
// TAIL (one-term kernels): the tiles holding rows from p.lo_row0 on (a
// multiple of BM) make a second pass over K with the activations' second term
// as A, adding x_lo * W to the accumulators: the two-term result of those
// rows, in the one-term kernel's LDS footprint and occupancy.  They take the
// first blockIdx values, one tile per workgroup, so they spread over the
// XCDs and start before the other tiles (which follow in XCD-major order).
template <int FMT, int BM, int BN, int WM, int WN, int MODE, int RH, bool TT, int KS = 1, bool TAIL = false>
__global__ __launch_bounds__(64 * (BM / WM) * (BN / WN) * KS) void dgemm_kernel(GemmArgs p) {
    static_assert(!(TT && TAIL), "the second pass belongs to one-term kernels");
    using G = DGemm<FMT, BM, BN, WM, WN, MODE, TT>;
    using L = DStage<FMT, BM, BN, G::NB, TT>;
    constexpr int NB = G::NB, TM = G::TM, TN = G::TN, NW = G::NW;
    static_assert(KS == 1 || KS == 2, "one or two K sets");
    // The stage buffers, in one array that the GEMM_QKV_ROPE epilogue reuses
    // for the tile's RoPE rows (BM positions x RH/2 pairs of 8 bytes: 32 KB at
    // head dim 64, so a 128x64 QKV tile keeps the two-stage footprint).
    // 128x64 and 64x64 tiles pipeline two stages deep (two and three workgroups
    // per CU with two activation terms), the others three.
    constexpr int NSTAGE = BN == 64 && BM <= 128 ? 2 : 3;
    constexpr int kStages = NSTAGE * L::BYTES;  // one K set's stage buffers
    constexpr int kRope = MODE == GEMM_QKV_ROPE ? BM * RH * 4 : 0;
    // the second K set's accumulators go past the first set's stage buffers
    constexpr int kRed = KS > 1 ? NB * TM * TN * 4 * 64 * NW * 4 : 0;
    constexpr int kSet = KS * kStages > kStages + kRed ? KS * kStages : kStages + kRed;
    constexpr int kSmem = kRope > kSet ? kRope : kSet;
    __shared__ __attribute__((aligned(16))) uint8_t smem[kSmem];
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kset = wave_all / NW;  // K set of this wave
    uint8_t* const st0 = smem + kset * kStages;
    uint8_t* const st1 = st0 + L::BYTES;
    uint8_t* const st2 = st0 + (NSTAGE > 2 ? 2 : 0) * L::BYTES;

    const int K = p.w.cols, N = p.w.rows, M = p.M, nb = K >> 5, spitch = stage_scale_pitch(N);
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int main_m = tiles_m, b = blockIdx.x, t = 0;
    bool tail_tile = false;
    if constexpr (TAIL) {
        // blockIdx [0, pad): the tail tiles (grid padded to a multiple of 8
        // there, so the others keep blockIdx % 8 as their XCD)
        main_m = min(tiles_m, p.lo_row0 / BM);
        const int ntail = (tiles_m - main_m) * tiles_n, pad = (ntail + 7) & ~7;
        if (b < pad) {
            if (b >= ntail) return;  // padding
            tail_tile = true;
            t = main_m * tiles_n + b;
        } else {
            b -= pad;
        }
    }
    int tm_i = t / tiles_n, tn_i = t % tiles_n;
    if (!tail_tile) {
        const int tiles = main_m * tiles_n, xcd = b % 8, q = tiles / 8, rem = tiles % 8;
        t = xcd * q + min(xcd, rem) + b / 8;  // XCD-major tile order (bijective)
        tm_i = t / tiles_n;
        tn_i = t % tiles_n;
        if (p.group_m > 0) {
            // a group holds rows [g * group_m, + gr) x every column, taken
            // column by column (the last group may have fewer rows; bijective)
            const int gsz = p.group_m * tiles_n, g = t / gsz, r = t - g * gsz;
            const int gr = min(p.group_m, main_m - g * p.group_m);
            tm_i = g * p.group_m + r % gr;
            tn_i = r / gr;
        }
    }
    const int m0 = tm_i * BM, n0 = tn_i * BN;
    const int lane = threadIdx.x & 63;
    const int wave = wave_all % NW;  // within the K set
    const int wm = wave / (BN / WN), wn = wave % (BN / WN);
    const int nk = K / DBK;
    // This set's stages: [k0s, k0s + cnt); every set runs `per` steps (the
    // same barriers), reloading its last stage past its end without using it.
    const int per = (nk + KS - 1) / KS, k0s = kset * per, cnt = max(0, min(nk - k0s, per));
    auto ktc = [&](int i) { return min(k0s + min(i, max(cnt, 1) - 1), nk - 1); };

    // Per-lane byte offsets of the DMA rows (loop-invariant, 32-bit: the host
    // checks that every operand spans less than 4 GiB); each stage adds its K
    // offset to the wave-uniform base pointers instead.
    uint32_t aoff[G::A_I], boff[NB][G::B_I], soff = 0;
#pragma unroll
    for (int i = 0; i < G::A_I; i++) {
        const int r = (i * NW + wave) * 8 + (lane >> 3), c = (lane & 7) ^ swz_a(r);
        aoff[i] = (uint32_t)((min(m0 + r, M - 1) * p.ldx + c * 8) * 2);
    }
#pragma unroll
    for (int mat = 0; mat < NB; mat++)
#pragma unroll
        for (int i = 0; i < G::B_I; i++) {
            if constexpr (FMT == DT_Q8_0) {
                const int r = (i * NW + wave) * 16 + (lane >> 2), c = (lane & 3) ^ swz_q8(r);
                boff[mat][i] = (uint32_t)(min(n0 + r, N - 1) * K + c * 16);
            } else if constexpr (FMT == DT_Q4_0) {
                if constexpr (G::Q4_16) {
                    const int r = (i * NW + wave) * 32 + (lane >> 1), c = (lane & 1) ^ swz_q4(r);
                    boff[mat][i] = (uint32_t)((min(n0 + r, N - 1) * nb + c) * 16);
                } else {
                    const int r = (i * NW + wave) * 8 + (lane >> 3), c = ((lane >> 2) & 1) ^ swz_q4(r);
                    boff[mat][i] = (uint32_t)((min(n0 + r, N - 1) * nb + c) * 16 + (lane & 3) * 4);
                }
            } else {
                const int r = (i * NW + wave) * 8 + (lane >> 3), c = (lane & 7) ^ swz_a(r);
                boff[mat][i] = (uint32_t)((min(n0 + r, N - 1) * K + c * 8) * 2);
            }
        }
    if constexpr (FMT != DT_F16) soff = (uint32_t)((n0 + wave * (BN / NW) + lane * 4) * 4);

    f32x4 acc[NB][TM][TN];
#pragma unroll
    for (int mat = 0; mat < NB; mat++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[mat][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The K loop, with the activations' second term (T2) or without it.  A
    // two-term kernel takes the second term only in tiles holding a row at or
    // past p.lo_row0 (the workgroup's choice, so each loop keeps its own DMA
    // counts and LDS layout); the other tiles multiply one f16 term.
    const f16* abase = p.x;  // the A plane of the pass
    auto kloop = [&](auto tt_c) {
        constexpr bool T2 = decltype(tt_c)::value;
        using L2 = DStage<FMT, BM, BN, NB, T2>;
        constexpr int PER2 = DGemm<FMT, BM, BN, WM, WN, MODE, T2>::PER;
        auto issue = [&](uint32_t sg, int kt) {  // sg: LDS byte address of the stage buffer
            const int k0 = kt * DBK;
    #pragma unroll
            for (int i = 0; i < G::A_I; i++) {
                const int r0 = (i * NW + wave) * 8;
                dma16s(abase + k0, aoff[i], sg + r0 * DBK * 2);
                if constexpr (T2) dma16s(p.xlo + k0, aoff[i], sg + L2::A_LO + r0 * DBK * 2);
            }
    #pragma unroll
            for (int mat = 0; mat < NB; mat++) {
                const DevMatrix& w = mat ? p.u : p.w;
                const uint32_t bq = sg + L2::B_OFF + mat * BN * L2::BROW;
    #pragma unroll
                for (int i = 0; i < G::B_I; i++) {
                    if constexpr (FMT == DT_Q8_0) {
                        dma16s(w.q + k0, boff[mat][i], bq + (i * NW + wave) * 16 * 64);
                    } else if constexpr (FMT == DT_Q4_0) {
                        if constexpr (G::Q4_16) dma16s(w.q + kt * 32, boff[mat][i], bq + (i * NW + wave) * 32 * 32);
                        else dma4s(w.q + kt * 32, boff[mat][i], bq + (i * NW + wave) * 8 * 32);
                    } else {
                        dma16s(w.q + k0 * 2, boff[mat][i], bq + (i * NW + wave) * 8 * 128);
                    }
                }
                if constexpr (FMT != DT_F16) {
                    // The tile's BN scale pairs are contiguous in s2: each wave moves
                    // 1/NW of them, 16 bytes (4 rows) per active lane.
                    if (lane < BN / (4 * NW))
                        dma16s(w.s2 + (int64_t)kt * spitch, soff, sg + L2::S_OFF + mat * BN * 4 + wave * (BN / NW) * 4);
                }
            }
        };

        const int jj = lane >> 4;  // which 8 of the fragment's 32 k values this lane holds
        // Quantised weights, one 32-weight block (kk) of a stage: each MFMA result
        // is scaled by the block's d before it is accumulated.  The MFMAs of column
        // j+1 are issued before the scaling of column j, so the VALU work of one
        // column runs under the MFMAs of the next instead of waiting on them.
        auto compute_block_quant = [&](const uint8_t* sg, int kk, const f16x8 (&af)[TM], const f16x8 (&al)[T2 ? TM : 1]) {
            // The raw quants of every column are read first; each becomes f16 just
            // before its MFMAs (8 bytes live per column instead of 16).
            uint2 raw[NB * TN];
            float d[NB * TN];
    #pragma unroll
            for (int c = 0; c < NB * TN; c++) {
                const int mat = c / TN, j = c % TN;
                const int r = wn * WN + 16 * j + (lane & 15);
                const uint8_t* bq = sg + L2::B_OFF + mat * BN * L2::BROW;
                if constexpr (FMT == DT_Q8_0) {
                    const int u = 4 * kk + jj;
                    raw[c] = *(const uint2*)(bq + r * 64 + ((u >> 1) ^ swz_q8(r)) * 16 + (u & 1) * 8);
                } else {
                    raw[c] = *(const uint2*)(bq + r * 32 + (kk ^ swz_q4(r)) * 16 + (jj & 1) * 8);
                }
                d[c] = (float)*(const f16*)(sg + L2::S_OFF + mat * BN * 4 + r * 4 + kk * 2);
            }
            auto bfrag = [&](int c) {
                uint32_t o[4];
                if constexpr (FMT == DT_Q8_0) {
                    int8x4_to_f16(raw[c].x, o[0], o[1]);
                    int8x4_to_f16(raw[c].y, o[2], o[3]);
                } else {
                    const int sh = (jj >> 1) * 4;
                    nib4_to_f16((raw[c].x >> sh) & 0x0F0F0F0Fu, o[0], o[1]);
                    nib4_to_f16((raw[c].y >> sh) & 0x0F0F0F0Fu, o[2], o[3]);
                }
                return __builtin_bit_cast(f16x8, make_uint4(o[0], o[1], o[2], o[3]));
            };
            f32x4 prev[TM], cur[TM];
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            // the block's product: both activation terms times the exact quants, summed in float32
            auto block = [&](int i, const f16x8& b) {
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], b, zero, 0, 0, 0);
                if constexpr (T2) t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b, t, 0, 0, 0);
                return t;
            };
            {
                const f16x8 b0 = bfrag(0);
    #pragma unroll
                for (int i = 0; i < TM; i++) prev[i] = block(i, b0);
            }
    #pragma unroll
            for (int c = 1; c <= NB * TN; c++) {
                if (c < NB * TN) {
                    const f16x8 bc = bfrag(c);
    #pragma unroll
                    for (int i = 0; i < TM; i++) cur[i] = block(i, bc);
                }
                const int pc = c - 1, mat = pc / TN, j = pc % TN;
    #pragma unroll
                for (int i = 0; i < TM; i++) acc[mat][i][j] += d[pc] * prev[i];
    #pragma unroll
                for (int i = 0; i < TM; i++) prev[i] = cur[i];
            }
        };
        auto compute = [&](const uint8_t* sg) {
    #pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                f16x8 af[TM], al[T2 ? TM : 1];
    #pragma unroll
                for (int i = 0; i < TM; i++) {
                    const int r = wm * WM + 16 * i + (lane & 15);
                    const int o = r * DBK * 2 + ((4 * kk + jj) ^ swz_a(r)) * 16;
                    af[i] = *(const f16x8*)(sg + o);
                    if constexpr (T2) al[i] = *(const f16x8*)(sg + L2::A_LO + o);
                }
    #pragma unroll
                for (int mat = 0; mat < NB; mat++)
    #pragma unroll
                    for (int j = 0; j < TN; j++) {
                        const int r = wn * WN + 16 * j + (lane & 15);
                        const uint8_t* bq = sg + L2::B_OFF + mat * BN * L2::BROW;
                        if constexpr (FMT == DT_F16) {
                            const f16x8 bf = *(const f16x8*)(bq + r * 128 + ((4 * kk + jj) ^ swz_a(r)) * 16);
    #pragma unroll
                            for (int i = 0; i < TM; i++) {
                                acc[mat][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[mat][i][j], 0, 0, 0);
                                if constexpr (T2)
                                    acc[mat][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf, acc[mat][i][j], 0, 0, 0);
                            }
                        }
                    }
                if constexpr (FMT != DT_F16) compute_block_quant(sg, kk, af, al);
            }
        };

        // One step: wait for stage kt (stage kt+1 stays in flight), barrier, refill
        // the buffer consumed by the previous step with stage kt+2, multiply stage
        // kt.  Past the end the refill reloads the last stage into a buffer that is
        // never read again, so every step has the same wait count.
        auto step = [&](const uint8_t* cur, uint8_t* refill, int i) {
            wait_stage_barrier<PER2>();
            issue(lds_addr(refill), ktc(i + 2));
            if (i < cnt) compute(cur);
        };
        if constexpr (NSTAGE == 3) {
            issue(lds_addr(st0), ktc(0));
            issue(lds_addr(st1), ktc(1));
            for (int i = 0; i < per; i += 3) {
                step(st0, st2, i);
                if (i + 1 < per) step(st1, st0, i + 1);
                if (i + 2 < per) step(st2, st1, i + 2);
            }
        } else {
            // wait for the stage (nothing else in flight), barrier (every wave is
            // done with the other buffer), refill it with the next stage, multiply
            auto step2 = [&](const uint8_t* cur, uint8_t* refill, int i) {
                wait_stage_barrier<0>();
                issue(lds_addr(refill), ktc(i + 1));
                if (i < cnt) compute(cur);
            };
            issue(lds_addr(st0), ktc(0));
            for (int i = 0; i < per; i += 2) {
                step2(st0, st1, i);
                if (i + 1 < per) step2(st1, st0, i + 1);
            }
        }
        // No DMA may still be writing this workgroup's LDS when its waves end.
        wait_stage_barrier<0>();
    };
    if constexpr (TT) {
        if (m0 + BM > p.lo_row0 || n0 + BN > p.lo_col0) kloop(std::true_type{});
        else kloop(std::false_type{});
    } else {
        kloop(std::false_type{});
        if constexpr (TAIL) {
            if (tail_tile) {  // every stage buffer is free: the loop ends on a full wait and barrier
                abase = p.xlo;
                kloop(std::false_type{});
            }
        }
    }
    if constexpr (KS > 1) {
        // The second set hands its accumulators to the first through its own
        // (idle) stage buffers; the first adds them and runs the epilogue.
        float* red = (float*)(smem + kStages) + wave * 64 + lane;
        if (kset == 1) {
#pragma unroll
            for (int mat = 0; mat < NB; mat++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) red[(((mat * TM + i) * TN + j) * 4 + r) * 64 * NW] = acc[mat][i][j][r];
        }
        __syncthreads();
        if (kset == 0) {
#pragma unroll
            for (int mat = 0; mat < NB; mat++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[mat][i][j][r] += red[(((mat * TM + i) * TN + j) * 4 + r) * 64 * NW];
        }
        // The RoPE epilogue's table copy writes smem from offset 0, which can
        // reach into `red` (single-term stages at head dim 128 are smaller than
        // the table): every wave of the first set must be done reading first.
        if constexpr (MODE == GEMM_QKV_ROPE && kRope > kStages) __syncthreads();
    }
    if constexpr (MODE == GEMM_QKV_ROPE) {
        // (every wave joins the epilogue's table copy and barrier; only the
        // first K set stores)
        qkv_rope_epilogue<BM, TM, TN, TT>(p, acc[0], smem, m0, m0 + wm * WM, n0 + wn * WN, M, N, lane, kset == 0);
        return;
    }
    if (kset != 0) return;
    if constexpr (MODE == GEMM_ACC) {
        acc_epilogue<TM, TN>(p, acc[0], m0 + wm * WM, n0 + wn * WN, M, N, lane);
        return;
    }

    // C layout of the 16x16 MFMA: lane holds rows 4*(lane/16)+r, column lane%16.
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WN + 16 * j + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
                if (m >= M) continue;
                const int64_t o = (int64_t)m * p.ldy + n;
                if (MODE == GEMM_STORE) {
                    p.y[o] = acc[0][i][j][r];
                } else if (MODE == GEMM_ACC) {
                    p.y[o] += acc[0][i][j][r];
                } else {
                    const float g = acc[0][i][j][r], u = acc[NB - 1][i][j][r];
                    const float v = (g / (1.0f + __expf(-g))) * u;
                    const f16 hv = (f16)v;
                    p.yh[o] = hv;
                    if (p.yhlo && m >= p.lo_out_row0) p.yhlo[o] = (f16)(v - (float)hv);
                }
            }
        }
}

// Row groups of the tile order.  Each XCD takes a contiguous range of tiles;
// row by row, the tiles it runs at once cover one or two row blocks and a wide
// band of columns, so where the weights exceed its 4 MB L2 it streams every
// weight column again for each of its row blocks.  In groups of four row
// blocks, taken column by column, the tiles running at once share each weight
// column four times.  Measured over 4,096-token prefills (us per layer, row by
// row against groups of 2 / 4 / 8 / 16): at the 1.7B shape (weights 4.5-36 MB
// per GEMM) QKV 243 -> 240 / 236 / 238 / 241, gate+up 390 -> 385 / 381 / 385
// / 389, down 212 -> 209 / 206 / 211 / 213 (165k -> 169k tok/s with 4); at
// the 135M and 360M shapes (weights of 0.35-2.8 MB, which every XCD's L2
// holds) no change.  ALPACA_HIP_GEMM_GROUP=<rows> forces the group (0: row by
// row; tuning and tests; read on every launch).
int gemm_group_rows(const GemmArgs& a, int mats) {
    if (const char* e = std::getenv("ALPACA_HIP_GEMM_GROUP")) return std::max(0, std::atoi(e));
    const DevMatrix& w = a.w;
    const int64_t per = (int64_t)w.rows * w.cols;
    const int64_t bytes = (w.dtype == DT_Q8_0 ? per * 34 / 32 : w.dtype == DT_Q4_0 ? per * 18 / 32 : per * 2) * mats;
    return bytes >= (int64_t)4 << 20 ? 4 : 0;
}

template <int FMT, int BM, int BN, int WM, int WN, int MODE, int RH, bool TT, int KS = 1, bool TAIL = false>
hipError_t run_dgemm(const GemmArgs& args, hipStream_t st) {
    const int tm = (args.M + BM - 1) / BM, tn = (args.w.rows + BN - 1) / BN;
    GemmArgs a = args;
    a.group_m = gemm_group_rows(a, MODE == GEMM_SWIGLU ? 2 : 1);
    int grid = tm * tn;
    if constexpr (TAIL) {
        if (a.lo_row0 % BM) return hipErrorInvalidValue;  // tail tiles start at lo_row0
        const int main_m = std::min(tm, a.lo_row0 / BM);
        grid = ((tm - main_m) * tn + 7) / 8 * 8 + main_m * tn;
    }
    dgemm_kernel<FMT, BM, BN, WM, WN, MODE, RH, TT, KS, TAIL><<<grid, 64 * (BM / WM) * (BN / WN) * KS, 0, st>>>(a);
    return hipGetLastError();
}

// ALPACA_HIP_GEMM_TILE=256 | 128x128 | 128x64 | 128x256 | 64x64 forces a tile
// family (tuning and tests; read on every launch); 256 means 256x128 (256x64
// per matrix for SwiGLU), 128x256 means 128x128 per matrix for SwiGLU, 64x64
// is per matrix for SwiGLU too.
int forced_tile() {
    const char* e = std::getenv("ALPACA_HIP_GEMM_TILE");
    if (!e) return 0;
    if (!std::strcmp(e, "256")) return 1;
    if (!std::strcmp(e, "128x128")) return 2;
    if (!std::strcmp(e, "128x64")) return 3;
    if (!std::strcmp(e, "128x256")) return 4;
    if (!std::strcmp(e, "64x64")) return 5;
    if (!std::strcmp(e, "64x64k2")) return 9;
    return 0;
}

// Compute units of the current device (cached per device id).
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        cus[dev] = n > 0 ? n : 256;
    }
    return cus[dev];
}

// Resident workgroups per CU of one instantiation (registers and LDS as
// compiled), asked once per process.
template <int FMT, int BM, int BN, int WM, int WN, int MODE, int RH, bool TT>
int resident_per_cu() {
    static const int v = [] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, dgemm_kernel<FMT, BM, BN, WM, WN, MODE, RH, TT>,
                                                         64 * (BM / WM) * (BN / WN), 0) !=
                hipSuccess || n < 1) {
            hipGetLastError();
            return 1;
        }
        return n;
    }();
    return v;
}

// Tile choice, counted in rounds of resident workgroups over the device's CUs.
template <int FMT, int MODE, int RH, bool TT, bool TAIL = false>
hipError_t pick_dgemm(const GemmArgs& a, hipStream_t st) {
    const int M = a.M, N = a.w.rows, cus = device_cus();
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    // Wide tiles (one workgroup per CU) pay off in whole rounds or where the
    // last partial round is a small part of the grid.
    auto wide_fits = [&](int t) { return t >= cus && (t % cus == 0 || t >= 3 * cus); };
    const int f = forced_tile();
    // The 256-row tiles hold more accumulators than the 256 architectural VGPRs
    // (344-353 with AGPR spills) and are slower wherever measured; they stay
    // reachable through ALPACA_HIP_GEMM_TILE=256 (single-term activations only:
    // with two terms they do not fit LDS).  With two activation terms a
    // 128x64 tile moves 36 KB per 64-wide K stage for 2 MFLOP and is bound by
    // the global->LDS rate; 128x256 tiles (128x128 per matrix for SwiGLU,
    // three stages, 147 KB of LDS, one workgroup per CU) halve the bytes per
    // MFMA and are taken on grids of whole rounds.  They run eight waves of
    // 64x64 (64x32 per matrix), two per SIMD, so that one wave's VALU work
    // (block scaling, quant conversion) issues while the other's MFMAs run:
    // at the 1.7B shape 4-7% faster than four waves of 64x128.  Single-term
    // activations stay on the narrower tiles, where the wide ones measured
    // slower: 128x64 tiles (two LDS stages) while their grid fits in one round
    // of the workgroups the device holds at once, else 128x128.  With two
    // terms, small grids (at most 1.6 tiles of 128x64 per CU, 3 for SwiGLU,
    // whose 128x64 tiles run one per CU) take 64x64 tiles (two LDS stages,
    // three workgroups per CU with quantised weights): at the 135M shape over
    // 2,048 rows the four GEMMs went 90 -> 75 us, and with f16 weights (the
    // prefill weight cache) the 4,096-token prefill 812k -> 864k tok/s; above
    // those counts, and at the 1.7B shape, they measured slower.  Where the
    // 64x64 grid is at most one tile per CU, QKV, Wo and down split each
    // tile's K stages over two sets of four waves (C1 at 1,024 rows: QKV 13.2
    // -> 12.2 us, Wo 10.9 -> 10.1, down 18.0 -> 15.1; C4 Wo 15.2 -> 13.1, down
    // 28.9 -> 22.9; slower on larger grids and for SwiGLU).  The other modes
    // then choose between 128x64 and 128x256 by the cost below.
    if (f == 5) return run_dgemm<FMT, 64, 64, 32, 32, MODE, RH, TT, 1, TAIL>(a, st);
    if (f == 9) return run_dgemm<FMT, 64, 64, 32, 32, MODE, RH, TT, 2, TAIL>(a, st);
    auto small_grid = [&](double per_cu) {
        return f == 0 && TT && tiles(128, 64) <= per_cu * cus;
    };
    if constexpr (MODE == GEMM_SWIGLU) {
        if constexpr (!TT)
            if (f == 1) return run_dgemm<FMT, 256, 64, 128, 32, MODE, RH, TT, 1, TAIL>(a, st);
        if constexpr (FMT != DT_F16)  // (f16 weight stages are 4x larger: no third stage fits)
            if (f == 4 || (f == 0 && TT && wide_fits(tiles(128, 128))))
                return run_dgemm<FMT, 128, 128, 64, 32, MODE, RH, TT, 1, TAIL>(a, st);
        if constexpr (TT)
            if (small_grid(3.0)) return run_dgemm<FMT, 64, 64, 32, 32, MODE, RH, TT, 1, TAIL>(a, st);
        return run_dgemm<FMT, 128, 64, 64, 32, MODE, RH, TT, 1, TAIL>(a, st);
    } else {
        if constexpr (!TT)
            if (f == 1) return run_dgemm<FMT, 256, 128, 128, 64, MODE, RH, TT, 1, TAIL>(a, st);
        const int slots = resident_per_cu<FMT, 128, 64, 64, 32, MODE, RH, TT>() * cus;
        if constexpr (TT)
            if (small_grid(1.6)) {
                // at most one 64x64 tile per CU (quantised weights): two K sets
                if (FMT != DT_F16 && tiles(64, 64) <= cus) return run_dgemm<FMT, 64, 64, 32, 32, MODE, RH, TT, 2, TAIL>(a, st);
                return run_dgemm<FMT, 64, 64, 32, 32, MODE, RH, TT, 1, TAIL>(a, st);
            }
        if constexpr (FMT != DT_F16) {
            if (f == 4) return run_dgemm<FMT, 128, 256, 64, 64, MODE, RH, TT, 1, TAIL>(a, st);
            if (f == 0 && TT) {
                // Two terms: 128x64 tiles (two per CU) or 128x256 (one per CU),
                // by a cost in rounds of resident workgroups.  A 128x64 round
                // costs 1; a last round of at most one tile per CU 0.6 (a tile
                // alone on its CU runs faster); a 128x256 round W = 1.32 at
                // K <= 960 and 1.87 at K = 2048, as measured over prompts of
                // 1,024-4,096 rows at the 135M, 360M and 1.7B shapes (128x128
                // tiles, one per CU, were never the fastest there).
                const int t64 = tiles(128, 64), rem = t64 % slots;
                const double c64 = t64 / slots + (rem ? (rem <= cus ? 0.6 : 1.0) : 0.0);
                const double cw = ((tiles(128, 256) + cus - 1) / cus) * (a.w.cols >= 1536 ? 1.87 : 1.32);
                if (cw < c64) return run_dgemm<FMT, 128, 256, 64, 64, MODE, RH, TT, 1, TAIL>(a, st);
                return run_dgemm<FMT, 128, 64, 64, 32, MODE, RH, TT, 1, TAIL>(a, st);
            }
        }
        if (f == 2 || (f == 0 && tiles(128, 64) > slots)) return run_dgemm<FMT, 128, 128, 64, 64, MODE, RH, TT, 1, TAIL>(a, st);
        return run_dgemm<FMT, 128, 64, 64, 32, MODE, RH, TT, 1, TAIL>(a, st);
    }
}

template <int FMT, bool TT>
hipError_t dgemm_mode_terms(const GemmArgs& a, int mode, hipStream_t st) {
    if (mode == GEMM_STORE) return pick_dgemm<FMT, GEMM_STORE, 0, TT>(a, st);
    if (mode == GEMM_ACC) return pick_dgemm<FMT, GEMM_ACC, 0, TT>(a, st);
    if (mode == GEMM_QKV_ROPE) {
        if (a.qkv.hd <= 64) return pick_dgemm<FMT, GEMM_QKV_ROPE, 64, TT>(a, st);
        return pick_dgemm<FMT, GEMM_QKV_ROPE, 128, TT>(a, st);
    }
    return pick_dgemm<FMT, GEMM_SWIGLU, 0, TT>(a, st);
}

// Second terms of the activations for the rows from lo_row0 on only: the
// one-term kernel with a second pass over the tail tiles.
template <int FMT>
hipError_t dgemm_mode_tail(const GemmArgs& a, int mode, hipStream_t st) {
    if (mode == GEMM_STORE) return pick_dgemm<FMT, GEMM_STORE, 0, false, true>(a, st);
    if (mode == GEMM_ACC) return pick_dgemm<FMT, GEMM_ACC, 0, false, true>(a, st);
    if (mode == GEMM_SWIGLU) return pick_dgemm<FMT, GEMM_SWIGLU, 0, false, true>(a, st);
    return hipErrorNotSupported;
}

// With the second term on the rows from lo_row0 on only, two forms: the
// one-term kernel with a second K pass over the tail tiles (dispatched first),
// or the two-term kernel taking the second term tile by tile.  The second pass
// doubles a tail tile's time, which a grid of one round of resident
// workgroups waits for in full, while over a longer grid the tail tiles
// overlap the later rounds and the other tiles run at the one-term kernel's
// occupancy and tile shape.  Measured per call at 4,096 rows (us, second pass
// against per tile): 1.7B shape Wo 67 / 70, gate+up 390 / 446, down 238 / 246
// (1.3-5.3 rounds); 135M shape Wo 18.6 / 15.1, gate+up 37.7 / 36.6, down
// 34.7 / 25.6 (0.4-1.0 rounds).  So the second pass is taken where the
// one-term grid of 128x64 tiles exceeds one round.  ALPACA_HIP_LO_PASS=tile |
// tail (read per launch) forces one form.
template <int FMT>
bool tail_pass_pays(const GemmArgs& a, int mode) {
    const char* e = std::getenv("ALPACA_HIP_LO_PASS");
    if (e && !std::strcmp(e, "tile")) return false;
    if (e && !std::strcmp(e, "tail")) return true;
    const int cus = device_cus(), rows = (a.M + 127) / 128, cols = (a.w.rows + 63) / 64;
    const int per_cu = mode == GEMM_SWIGLU ? resident_per_cu<FMT, 128, 64, 64, 32, GEMM_SWIGLU, 0, false>()
                       : mode == GEMM_ACC  ? resident_per_cu<FMT, 128, 64, 64, 32, GEMM_ACC, 0, false>()
                                           : resident_per_cu<FMT, 128, 64, 64, 32, GEMM_STORE, 0, false>();
    return (int64_t)rows * cols > (int64_t)per_cu * cus;
}

template <int FMT>
hipError_t dgemm_mode(const GemmArgs& a, int mode, hipStream_t st) {
    if (a.xlo && a.lo_row0 > 0 && mode != GEMM_QKV_ROPE && tail_pass_pays<FMT>(a, mode))
        return dgemm_mode_tail<FMT>(a, mode, st);
    return a.xlo ? dgemm_mode_terms<FMT, true>(a, mode, st) : dgemm_mode_terms<FMT, false>(a, mode, st);
}

}  // namespace

namespace {
// The DMA kernel addresses activations and weights with 32-bit signed byte
// offsets from per-stage base pointers.
bool dma_offsets_fit(int m, int ldx, const DevMatrix& w) {
    const int64_t lim = INT32_MAX;
    const int64_t wbytes = w.dtype == DT_Q8_0   ? (int64_t)w.rows * w.cols
                           : w.dtype == DT_Q4_0 ? (int64_t)w.rows * (w.cols / 32) * 16
                                                : (int64_t)w.rows * w.cols * 2;
    return (int64_t)m * ldx * 2 < lim && wbytes < lim;
}
}  // namespace

// Whether an m-row prefill chunk whose QKV GEMM is n columns wide is worth
// running as two halves on two streams: that GEMM's grid of 128x64 tiles is at
// most two rounds of two workgroups per CU, so each half's kernels leave CUs
// idle at their tails for the other half to fill.  (At the 1.7B shape the
// grids are larger and the halves only contend: 2,048 rows 123k tok/s on one
// stream, 116k split.)
bool prefill_split_pays(int m, int n) {
    return (int64_t)((m + 127) / 128) * ((n + 63) / 64) <= 4 * (int64_t)device_cus();
}

hipError_t launch_gemm_mfma(const f16* x, const f16* xlo, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up,
                            float* y, f16* yh, f16* yhlo, int ldy, int mode, hipStream_t st, int lo_row0,
                            int lo_out_row0) {
    if (m <= 0) return hipSuccess;
    // The DMA kernel needs 64-wide K stages, 16-byte aligned activation rows and,
    // for quantised weights, the stage-major scales.
    const bool quant = w.dtype != DT_F16;
    if (w.cols % DBK || ldx % 8 || ((uintptr_t)x & 15) || ((uintptr_t)xlo & 15) ||
        (quant && (!w.s2 || (w_up && !w_up->s2))) || !dma_offsets_fit(m, ldx, w))
        return launch_gemm_mfma_staged(x, xlo, ldx, m, w, w_up, y, yh, yhlo, ldy, mode, st, lo_row0, lo_out_row0);
    GemmArgs a;
    a.x = x;
    a.xlo = xlo;
    a.yhlo = yhlo;
    a.ldx = ldx;
    a.M = m;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.y = y;
    a.yh = yh;
    a.ldy = ldy;
    a.lo_row0 = lo_row0;
    a.lo_out_row0 = lo_out_row0;
    switch (w.dtype) {
    case DT_Q8_0: return dgemm_mode<DT_Q8_0>(a, mode, st);
    case DT_Q4_0: return dgemm_mode<DT_Q4_0>(a, mode, st);
    default: return dgemm_mode<DT_F16>(a, mode, st);
    }
}

hipError_t launch_gemm_qkv_rope(const f16* x, const f16* xlo, int ldx, int m, const DevMatrix& w, const QkvRope& o,
                                hipStream_t st, int lo_row0, int lo_out_row0, int lo_col0) {
    if (m <= 0) return hipSuccess;
    const bool quant = w.dtype != DT_F16;
    // the pipelined kernel's conditions (as in launch_gemm_mfma); RoPE pairs and
    // 16-column lane groups must not straddle a head; two-term in, two-term q out
    if (w.cols % DBK || ldx % 8 || ((uintptr_t)x & 15) || ((uintptr_t)xlo & 15) || (quant && !w.s2) ||
        !dma_offsets_fit(m, ldx, w) || o.hd % 16 ||
        o.hd > 128 || o.heads <= 0 || o.kv_heads <= 0 || w.rows != (o.heads + 2 * o.kv_heads) * o.hd || !o.rope ||
        !o.qh || !o.kc || !o.vc)
        return hipErrorNotSupported;
    GemmArgs a;
    a.x = x;
    a.xlo = xlo;
    a.yhlo = o.qlo;
    a.ldx = ldx;
    a.M = m;
    a.w = w;
    a.u = w;
    a.y = nullptr;
    a.yh = o.qh;
    a.ldy = o.heads * o.hd;
    a.qkv = o;
    a.lo_row0 = lo_row0;
    a.lo_out_row0 = lo_out_row0;
    a.lo_col0 = lo_col0;
    switch (w.dtype) {
    case DT_Q8_0: return dgemm_mode<DT_Q8_0>(a, GEMM_QKV_ROPE, st);
    case DT_Q4_0: return dgemm_mode<DT_Q4_0>(a, GEMM_QKV_ROPE, st);
    default: return dgemm_mode<DT_F16>(a, GEMM_QKV_ROPE, st);
    }
}

// Stage-major scale pairs for the prefill GEMM (layout in DevMatrix::s2).
__global__ void stage_scales_kernel(const f16* __restrict__ s, uint32_t* __restrict__ s2, int rows, int cols) {
    const int nst = cols / 64, nb = cols / 32, pitch = stage_scale_pitch(rows);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * nst) return;
    const int n = (int)(i / nst), kt = (int)(i % nst);
    const uint32_t* src = (const uint32_t*)(s + (int64_t)n * nb + 2 * kt);  // nb even: 4-byte aligned
    s2[(int64_t)kt * pitch + n] = *src;
}

hipError_t launch_stage_scales(const f16* s, uint32_t* s2, int rows, int cols, hipStream_t st) {
    const int64_t n = (int64_t)rows * (cols / 64);
    if (n <= 0) return hipSuccess;
    stage_scales_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(s, s2, rows, cols);
    return hipGetLastError();
}
