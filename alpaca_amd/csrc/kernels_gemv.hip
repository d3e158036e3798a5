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
// A group of LPR lanes owns one output row and strides over its chunks.  The
// first batch of up to 4 chunk loads per lane is issued before the input row
// is staged, so the weight stream is in flight while the workgroup computes
// the RMSNorm (or merges attention partials) into LDS.  Partial sums are
// combined with cross-lane shuffles; lane 0 of the group applies the epilogue.
//
// Input stagers: x (optionally RMS-normalised with gain g), or the merge of
// split-K decode-attention partials (max, sum, unnormalised output) per head,
// which folds the attention merge into the Wo projection.
// Epilogues: store, residual add, SwiGLU, or (QKV projection) RoPE on q and k
// with k and v appended to the KV cache at position pos.
#include "common.h"
#include "gemv_chunks.h"

#include <algorithm>
#include <cstdlib>

namespace {

using gemv::RowStream;
using gemv::chunks_of;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;
constexpr int kMaxRowsPerBlock = kWaves * 64 / 16;

struct GemvArgs {
    DevMatrix w, u;
    GemvInput in;
    GemvRope rope;
    float* out;
};

enum { IN_X = 0, IN_NORM = 1, IN_MERGE = 2 };

// Stages the input row (K floats) into LDS.
template <int INP>
__device__ __forceinline__ void stage_input(const GemvInput& in, int K, float* xs, float* red) {
    if constexpr (INP == IN_MERGE) {
        // Merge split-K attention partials: per head h, weights w_s = exp(m_s - M),
        // x = sum_s w_s o_s / sum_s w_s l_s (attention_decode.metal:117-133).
        __shared__ float mh[256];
        __shared__ float wsp[4096];
        const int H = in.heads, S = in.splits, hd = in.hd;
        const int live = in.pos_dev ? min(S, (*in.pos_dev + in.split_len) / in.split_len) : S;
        for (int h = threadIdx.x; h < H; h += kThreads) {
            float m = -INFINITY;
            for (int s = 0; s < live; s++) m = fmaxf(m, in.partials[((int64_t)h * S + s) * (hd + 2)]);
            mh[h] = m;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < H * live; i += kThreads) {
            const int h = i / live, s = i - h * live;
            const float ms = in.partials[((int64_t)h * S + s) * (hd + 2)];
            wsp[h * live + s] = ms == -INFINITY ? 0.f : expf(ms - mh[h]);
        }
        __syncthreads();
        for (int h = threadIdx.x; h < H; h += kThreads) {
            float l = 0.f;
            for (int s = 0; s < live; s++) l += wsp[h * live + s] * in.partials[((int64_t)h * S + s) * (hd + 2) + 1];
            mh[h] = 1.0f / l;
        }
        __syncthreads();
        for (int k = threadIdx.x; k < K; k += kThreads) {
            const int h = k / hd, dd = k - h * hd;
            const float* pp = in.partials + (int64_t)h * S * (hd + 2) + 2 + dd;
            float acc = 0.f;
            for (int s = 0; s < live; s++) acc += wsp[h * live + s] * pp[(int64_t)s * (hd + 2)];
            xs[k] = acc * mh[h];
        }
    } else if constexpr (INP == IN_NORM) {
        float ss = 0.f;
        for (int i = threadIdx.x; i < K; i += kThreads) ss += in.x[i] * in.x[i];
        ss = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(ss / (float)K + in.eps);
        for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = (in.x[i] * scale) * in.norm[i];
    } else {
        for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = in.x[i];
    }
    __syncthreads();
}

template <int FMT, int LPR, int MODE, int INP>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ float xs[];
    __shared__ float red[16];
    __shared__ float rowbuf[kMaxRowsPerBlock];
    const int K = a.w.cols;
    constexpr int kRowsPerWave = 64 / LPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int li = lane % LPR;
    const int local = wave * kRowsPerWave + lane / LPR;
    const int64_t row = (int64_t)blockIdx.x * kWaves * kRowsPerWave + local;
    const bool valid = row < a.w.rows;

    RowStream<FMT, LPR> s0, s1;
    if (valid) {
        s0.prefetch(a.w, row, K, li);
        if (MODE == GEMV_SWIGLU) s1.prefetch(a.u, row, K, li);
    }
    stage_input<INP>(a.in, K, xs, red);
    float acc = 0.f, acc2 = 0.f;
    if (valid) {
        acc = s0.finish(a.w, row, K, li, xs);
        if (MODE == GEMV_SWIGLU) acc2 = s1.finish(a.u, row, K, li, xs);
    }
    acc = lane_sum<LPR>(acc);
    if (MODE == GEMV_SWIGLU) acc2 = lane_sum<LPR>(acc2);
    if (MODE == GEMV_QKV_ROPE) {
        // Rows come in aligned (even, odd) pairs inside a block: RoPE pairs.
        if (li == 0) rowbuf[local] = acc;
        __syncthreads();
        const GemvRope& r = a.rope;
        const int pos = r.pos_dev ? *r.pos_dev : r.pos;
        const int half = r.hd / 2;
        const int pairs = kWaves * kRowsPerWave / 2;
        for (int pi = threadIdx.x; pi < pairs; pi += kThreads) {
            const int64_t r0 = (int64_t)blockIdx.x * kWaves * kRowsPerWave + 2 * pi;
            if (r0 >= a.w.rows) break;
            const float v0 = rowbuf[2 * pi], v1 = rowbuf[2 * pi + 1];
            const int qw = r.heads * r.hd, kw = r.kv_heads * r.hd;
            if (r0 < qw + kw) {
                const int d = (int)(r0 % r.hd);
                const float2 cs = r.table[(int64_t)pos * half + d / 2];
                float ac = v0 * cs.x, bs = v1 * cs.y, as = v0 * cs.y, bc = v1 * cs.x;
                const float ra = ac - bs, rb = as + bc;
                if (r0 < qw) {
                    a.out[r0] = ra;
                    a.out[r0 + 1] = rb;
                } else {
                    const int64_t dst = ((int64_t)((r0 - qw) / r.hd) * r.capacity + pos) * r.hd + d;
                    if (r.kv_f16) {
                        ((f16*)r.kc)[dst] = (f16)ra;
                        ((f16*)r.kc)[dst + 1] = (f16)rb;
                    } else {
                        ((float*)r.kc)[dst] = ra;
                        ((float*)r.kc)[dst + 1] = rb;
                    }
                }
            } else {
                const int d = (int)((r0 - qw - kw) % r.hd);
                const int64_t dst = ((int64_t)((r0 - qw - kw) / r.hd) * r.capacity + pos) * r.hd + d;
                if (r.kv_f16) {
                    ((f16*)r.vc)[dst] = (f16)v0;
                    ((f16*)r.vc)[dst + 1] = (f16)v1;
                } else {
                    ((float*)r.vc)[dst] = v0;
                    ((float*)r.vc)[dst + 1] = v1;
                }
            }
        }
        return;
    }
    if (valid && li == 0) {
        if (MODE == GEMV_STORE) a.out[row] = acc;
        else if (MODE == GEMV_ADD) a.out[row] += acc;
        else a.out[row] = (acc / (1.0f + expf(-acc))) * acc2;
    }
}

// Tall matrices (the logits, large FFN matrices): a grid of resident
// workgroups walks tiles of kWaves * 64 / LPR rows.  LPR lanes own a row and
// each takes CPL chunks of it (LPR * CPL covers the row with few clamped
// extra loads), so one batch of CPL 16-byte loads per lane holds the whole
// tile; the batch of the workgroup's next tile is issued before the current
// one is multiplied, so every wave keeps a batch in flight while it computes,
// and the input row is staged once per workgroup instead of once per tile.
template <int FMT, int LPR, int CPL, int MODE, int INP>
__global__ __launch_bounds__(kThreads) void gemv_tall_kernel(GemvArgs a, int tiles) {
    extern __shared__ float xs[];
    __shared__ float red[16];
    constexpr int RPW = 64 / LPR, RT = kWaves * RPW;
    const int K = a.w.cols, nch = chunks_of<FMT>(K), rows = a.w.rows;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane % LPR;
    const int rin = wave * RPW + lane / LPR;  // this lane group's row within a tile
    constexpr int NM = MODE == GEMV_SWIGLU ? 2 : 1;
    int4 q[2][NM][CPL];
    float d[2][NM][CPL];
    auto load = [&](int t, int b) {
        const int64_t row = min((int64_t)t * RT + rin, (int64_t)rows - 1);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int u = 0; u < CPL; u++) {
                const int c = li + u * LPR;
                gemv::load_chunk<FMT>(m ? a.u : a.w, row, K, c < nch ? c : nch - 1, q[b][m][u], d[b][m][u]);
            }
    };
    int t = blockIdx.x;
    if (t < tiles) load(t, 0);
    stage_input<INP>(a.in, K, xs, red);
    auto step = [&](int b) {
        const int nt = t + gridDim.x;
        if (nt < tiles) load(nt, b ^ 1);
        float acc[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            acc[m] = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; u++) {
                const int c = li + u * LPR;
                if (c < nch) acc[m] += gemv::chunk_dot<FMT>(q[b][m][u], d[b][m][u], c, xs);
            }
            acc[m] = lane_sum<LPR>(acc[m]);
        }
        const int64_t row = (int64_t)t * RT + rin;
        if (row < rows && li == 0) {
            if (MODE == GEMV_STORE) a.out[row] = acc[0];
            else if (MODE == GEMV_ADD) a.out[row] += acc[0];
            else a.out[row] = (acc[0] / (1.0f + expf(-acc[0]))) * acc[NM - 1];
        }
        t = nt;
    };
    // the two register sets alternate; the loop is unrolled over both so they stay in registers
    while (t < tiles) {
        step(0);
        if (t >= tiles) break;
        step(1);
    }
}

// (LPR, CPL) for a row of nch chunks: the fewest lanes per row whose batch of
// at most 8 chunks per lane covers the row (tiles of more rows, more loads per
// lane in flight), CPL then as small as that allows.
struct TallShape {
    int lpr = 0, cpl = 0;
};
inline TallShape tall_shape(int nch) {
    for (int lpr = 4; lpr <= 64; lpr *= 2) {
        const int cpl = (nch + lpr - 1) / lpr;
        if (cpl <= 8) return {lpr, cpl <= 4 ? 4 : cpl <= 5 ? 5 : 8};
    }
    return {};
}

template <int FMT, int LPR, int CPL, int MODE, int INP>
hipError_t run_tall(const GemvArgs& a, hipStream_t st) {
    static int per_cu[64] = {0};
    int dev = 0;
    hipGetDevice(&dev);
    const size_t lds = (size_t)a.w.cols * sizeof(float);
    int& occ = per_cu[dev & 63];
    if (!occ) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_tall_kernel<FMT, LPR, CPL, MODE, INP>, kThreads,
                                                         lds) != hipSuccess || n < 1) {
            hipGetLastError();
            n = 1;
        }
        occ = n;
    }
    int cus = 0;
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int rt = kWaves * (64 / LPR), tiles = (a.w.rows + rt - 1) / rt;
    const int grid = std::min(tiles, std::max(1, cus) * occ);
    gemv_tall_kernel<FMT, LPR, CPL, MODE, INP><<<grid, kThreads, lds, st>>>(a, tiles);
    return hipGetLastError();
}

template <int FMT, int MODE, int INP>
hipError_t dispatch_tall(const TallShape& ts, const GemvArgs& a, hipStream_t st) {
#define TALL(L, CP) \
    if (ts.lpr == L && ts.cpl == CP) return run_tall<FMT, L, CP, MODE, INP>(a, st);
    TALL(4, 4) TALL(4, 5) TALL(4, 8) TALL(8, 4) TALL(8, 5) TALL(8, 8) TALL(16, 4) TALL(16, 5) TALL(16, 8)
    TALL(32, 4) TALL(32, 5) TALL(32, 8) TALL(64, 4) TALL(64, 5) TALL(64, 8)
#undef TALL
    return hipErrorInvalidValue;
}

template <int FMT, int MODE, int INP>
hipError_t dispatch(int lpr, const GemvArgs& a, hipStream_t st) {
    const int rows_per_block = kWaves * (64 / lpr);
    const int grid = (a.w.rows + rows_per_block - 1) / rows_per_block;
    const size_t lds = (size_t)a.w.cols * sizeof(float);
    switch (lpr) {
    case 16: gemv_kernel<FMT, 16, MODE, INP><<<grid, kThreads, lds, st>>>(a); break;
    case 32: gemv_kernel<FMT, 32, MODE, INP><<<grid, kThreads, lds, st>>>(a); break;
    default: gemv_kernel<FMT, 64, MODE, INP><<<grid, kThreads, lds, st>>>(a); break;
    }
    return hipGetLastError();
}

// The (epilogue, input) pairs the forward pass uses.
template <int FMT>
hipError_t dispatch_fmt(int lpr, int mode, int inp, const GemvArgs& a, hipStream_t st) {
    if (mode == GEMV_STORE) return inp == IN_NORM ? dispatch<FMT, GEMV_STORE, IN_NORM>(lpr, a, st)
                                                  : dispatch<FMT, GEMV_STORE, IN_X>(lpr, a, st);
    if (mode == GEMV_ADD) return inp == IN_MERGE ? dispatch<FMT, GEMV_ADD, IN_MERGE>(lpr, a, st)
                                                 : dispatch<FMT, GEMV_ADD, IN_X>(lpr, a, st);
    if (mode == GEMV_SWIGLU) return inp == IN_NORM ? dispatch<FMT, GEMV_SWIGLU, IN_NORM>(lpr, a, st)
                                                   : dispatch<FMT, GEMV_SWIGLU, IN_X>(lpr, a, st);
    return dispatch<FMT, GEMV_QKV_ROPE, IN_NORM>(lpr, a, st);
}

}  // namespace

template <int FMT>
constexpr int gemv_nch(int K) {
    return FMT == DT_Q8_0 ? K / 16 : FMT == DT_Q4_0 ? K / 32 : K / 8;
}

// Lanes per row: enough workgroups to cover the chip for tall matrices, whole
// waves per row for short ones (the decode matrices of small models are
// latency-bound, so more rows in flight matter more than lane utilisation).
static int pick_lpr(int rows) {
    if ((rows + 15) / 16 >= 1024) return 16;
    if ((rows + 7) / 8 >= 1024) return 32;
    return 64;
}

// Whether a matrix takes the tall kernel: at least 4 MB of weights, and a row
// that one batch of at most 8 chunks per lane on 64 lanes covers.
static bool tall_pays(const DevMatrix& w) {
    const int64_t bytes = w.dtype == DT_Q8_0   ? (int64_t)w.rows * w.cols / 32 * 34
                          : w.dtype == DT_Q4_0 ? (int64_t)w.rows * w.cols / 32 * 18
                                               : (int64_t)w.rows * w.cols * 2;
    const int nch = w.dtype == DT_Q8_0 ? w.cols / 16 : w.dtype == DT_Q4_0 ? w.cols / 32 : w.cols / 8;
    const char* e = std::getenv("ALPACA_HIP_GEMV_TALL");  // tuning: 0 keeps the one-tile-per-workgroup kernel
    if (e && e[0] == '0') return false;
    return bytes >= (4 << 20) && nch <= 64 * 8;
}

template <int FMT>
hipError_t dispatch_tall_fmt(int mode, int inp, const GemvArgs& a, hipStream_t st) {
    const TallShape ts = tall_shape(gemv_nch<FMT>(a.w.cols));
    if (mode == GEMV_STORE) return inp == IN_NORM ? dispatch_tall<FMT, GEMV_STORE, IN_NORM>(ts, a, st)
                                                  : dispatch_tall<FMT, GEMV_STORE, IN_X>(ts, a, st);
    if (mode == GEMV_ADD) return dispatch_tall<FMT, GEMV_ADD, IN_X>(ts, a, st);
    return inp == IN_NORM ? dispatch_tall<FMT, GEMV_SWIGLU, IN_NORM>(ts, a, st)
                          : dispatch_tall<FMT, GEMV_SWIGLU, IN_X>(ts, a, st);
}

hipError_t launch_gemv_ex(const DevMatrix& w, const DevMatrix* w_up, const GemvInput& in, const GemvRope* rope,
                          float* out, int mode, hipStream_t st) {
    const int inp = in.partials ? IN_MERGE : in.norm ? IN_NORM : IN_X;
    if (inp == IN_MERGE && ((long)in.heads * in.splits > 4096 || in.heads > 256 || mode != GEMV_ADD))
        return hipErrorInvalidValue;
    if (mode == GEMV_QKV_ROPE && (!rope || inp != IN_NORM)) return hipErrorInvalidValue;
    if (inp == IN_NORM && mode == GEMV_ADD) return hipErrorInvalidValue;
    GemvArgs a;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.in = in;
    if (rope) a.rope = *rope;
    a.out = out;
    if (mode != GEMV_QKV_ROPE && inp != IN_MERGE && tall_pays(w)) {
        switch (w.dtype) {
        case DT_Q8_0: return dispatch_tall_fmt<DT_Q8_0>(mode, inp, a, st);
        case DT_Q4_0: return dispatch_tall_fmt<DT_Q4_0>(mode, inp, a, st);
        default: return dispatch_tall_fmt<DT_F16>(mode, inp, a, st);
        }
    }
    const int lpr = pick_lpr(w.rows);
    switch (w.dtype) {
    case DT_Q8_0: return dispatch_fmt<DT_Q8_0>(lpr, mode, inp, a, st);
    case DT_Q4_0: return dispatch_fmt<DT_Q4_0>(lpr, mode, inp, a, st);
    default: return dispatch_fmt<DT_F16>(lpr, mode, inp, a, st);
    }
}

hipError_t launch_gemv(const DevMatrix& w, const DevMatrix* w_up, const float* x, const float* norm, float eps,
                       float* out, int mode, hipStream_t st) {
    GemvInput in;
    in.x = x;
    in.norm = norm;
    in.eps = eps;
    return launch_gemv_ex(w, w_up, in, nullptr, out, mode, st);
}
