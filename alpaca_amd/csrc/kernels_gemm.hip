// Prefill dequant-GEMMs for gfx950: Y[M tokens, N rows] (+)= X[M,K] * W[N,K]^T.
//
// Replaces the reference's batched projections: the fast tensor-op GEMMs
// (gemm_tensor_half_w[_acc], gemm_tensor_gateup_silu, tensor_gemm.metal) and
// the exact simdgroup GEMM (mm_*, matmul.metal), host side
// KernelEncoder.swift:192-280.  CPU semantics: CPUOps.linear / dot
// (CPUOps.swift:77-139).
//
// gemm_mfma_kernel (fast): f16 activations; quantised weights staged in LDS as
// their integer quants in f16 (exact) with the per-block f16 scale kept in
// float32; one v_mfma_f32_16x16x32_f16 covers one 32-weight block and its
// result is scaled by d before accumulation, so the only rounding on the
// inputs is the activations' (float32 -> f16).  256 threads = 2x2 waves; BK = 64 (two quant
// blocks) per LDS stage, double-buffered: the next stage's global loads are in
// registers while the current stage is multiplied, one barrier per stage.
// Epilogues: store f32, accumulate into the f32 residual, or SwiGLU
// (silu(x Wg^T) * (x Wu^T) from two accumulator sets) written as f16.
//
// gemm_f32_kernel (exact): float32 SIMT tiles 64x64, BK = 32 = one block.
// Inside a block the products are summed in the CPU reference's order and the
// block sum is scaled once (acc += d * s), with FP contraction off, so each
// output equals the CPU reference's float32 result.
#include "common.h"

namespace {

// ------------------------------------------------------------------ MFMA path
constexpr int BK = 64;
constexpr int LDT = BK + 8;  // LDS row pitch in halves (144 B: staggers banks)

struct GemmArgs {
    const f16* x;
    int ldx, M;
    DevMatrix w, u;
    float* y;
    f16* yh;
    int ldy;
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

template <int FMT, int BM, int BN, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_mfma_kernel(GemmArgs p) {
    constexpr int NB = MODE == GEMM_SWIGLU ? 2 : 1;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16;
    constexpr int SA = BM * (BK / 8) / 256;  // 16-byte A segments per thread
    constexpr int UB = BN * (BK / 16) / 256; // 16-weight B units per thread per matrix
    static_assert(SA >= 1 && UB >= 1, "tile too small for 256 threads");

    constexpr bool kQuant = FMT != DT_F16;
    __shared__ __attribute__((aligned(16))) f16 As[2][BM][LDT];
    __shared__ __attribute__((aligned(16))) f16 Bs[2][NB][BN][LDT];
    __shared__ float Ds[2][NB][BN][BK / 32];  // block scales of the stage

    const int K = p.w.cols, N = p.w.rows, M = p.M;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (K + BK - 1) / BK;

    int4 ra[SA];
    BUnit<FMT> rb[NB][UB];

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < SA; i++) {
            const int seg = tid + 256 * i, r = seg >> 3, c = (seg & 7) * 8;
            int4 v = {0, 0, 0, 0};
            if (m0 + r < M && k0 + c < K) v = *(const int4*)(p.x + (int64_t)(m0 + r) * p.ldx + k0 + c);
            ra[i] = v;
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
            f16x8 af[TM];
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[i] = *(const f16x8*)&As[cur][wm * WM + 16 * i + (lane & 15)][32 * kk + 8 * (lane >> 4)];
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
                            const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            acc[mat][i][j] += d * t;
                        }
                        // keep one column tile of block results live at a time (register budget)
                        __builtin_amdgcn_sched_barrier(0);
                    } else {
#pragma unroll
                        for (int i = 0; i < TM; i++)
                            acc[mat][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[mat][i][j], 0, 0, 0);
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
                    p.yh[o] = (f16)((g / (1.0f + __expf(-g))) * u);
                }
            }
        }
}

template <int FMT, int BM, int BN>
hipError_t run_mfma(const GemmArgs& a, int mode, hipStream_t st) {
    dim3 grid((a.M + BM - 1) / BM, (a.w.rows + BN - 1) / BN);
    if (mode == GEMM_STORE) gemm_mfma_kernel<FMT, BM, BN, GEMM_STORE><<<grid, 256, 0, st>>>(a);
    else if (mode == GEMM_ACC) gemm_mfma_kernel<FMT, BM, BN, GEMM_ACC><<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

template <int FMT, int BM, int BN>
hipError_t run_mfma_swiglu(const GemmArgs& a, hipStream_t st) {
    dim3 grid((a.M + BM - 1) / BM, (a.w.rows + BN - 1) / BN);
    gemm_mfma_kernel<FMT, BM, BN, GEMM_SWIGLU><<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

// Tiles: 64x64 for short batches and for SwiGLU (two accumulator sets);
// otherwise 128 tokens x 64 rows (quantised formats keep two waves per SIMD
// there: the per-block scaling holds a second set of MFMA results in
// registers), and 128x128 for F16 weights when the grid covers the chip twice.
template <int FMT>
hipError_t pick_tile(const GemmArgs& a, int mode, hipStream_t st) {
    const int M = a.M, N = a.w.rows;
    if (mode == GEMM_SWIGLU) return run_mfma_swiglu<FMT, 64, 64>(a, st);
    if (M <= 64) return run_mfma<FMT, 64, 64>(a, mode, st);
    const long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if constexpr (FMT == DT_F16) {
        if (big >= 512) return run_mfma<FMT, 128, 128>(a, mode, st);
    }
    return run_mfma<FMT, 128, 64>(a, mode, st);
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

hipError_t launch_gemm_mfma(const f16* x, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up, float* y,
                            f16* yh, int ldy, int mode, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    GemmArgs a;
    a.x = x;
    a.ldx = ldx;
    a.M = m;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.y = y;
    a.yh = yh;
    a.ldy = ldy;
    switch (w.dtype) {
    case DT_Q8_0: return pick_tile<DT_Q8_0>(a, mode, st);
    case DT_Q4_0: return pick_tile<DT_Q4_0>(a, mode, st);
    default: return pick_tile<DT_F16>(a, mode, st);
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
