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
    f16* outh = nullptr;  // GEMV_SWIGLU with f16 output: the two terms of each value
    f16* outl = nullptr;
};

enum { IN_X = 0, IN_NORM = 1, IN_MERGE = 2, IN_PAIR = 3 };

// out[row] = silu(g) * u, as float32 or (outh set) as two f16 terms.
__device__ __forceinline__ void swiglu_store(const GemvArgs& a, int64_t row, float g, float u) {
    const float v = (g / (1.0f + expf(-g))) * u;
    if (a.outh) {
        const f16 hi = (f16)v;
        a.outh[row] = hi;
        a.outl[row] = (f16)(v - (float)hi);
    } else {
        a.out[row] = v;
    }
}

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
    } else if constexpr (INP == IN_PAIR) {
        for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = (float)in.xh[i] + (float)in.xl[i];
    } else {
        for (int i = threadIdx.x; i < K; i += kThreads) xs[i] = in.x[i];
    }
    __syncthreads();
}

// QKV epilogue for the row pair (r0, r0 + 1) of the stacked [q | k | v]
// matrix: q rows rotated into out, k rows rotated and v rows copied into the
// caches at the step's position (CPUOps.rope, CPUOps.swift:184-212, and
// KVCache.write, KVCache.swift:44-63).
__device__ __forceinline__ void rope_pair_store(const GemvRope& r, int64_t r0, float v0, float v1, float* out) {
#pragma clang fp contract(off)
    const int pos = r.pos_dev ? *r.pos_dev : r.pos;
    const int half = r.hd / 2;
    const int qw = r.heads * r.hd, kw = r.kv_heads * r.hd;
    if (r0 < qw + kw) {
        const int d = (int)(r0 % r.hd);
        const float2 cs = r.table[(int64_t)pos * half + d / 2];
        float ac = v0 * cs.x, bs = v1 * cs.y, as = v0 * cs.y, bc = v1 * cs.x;
        const float ra = ac - bs, rb = as + bc;
        if (r0 < qw) {
            out[r0] = ra;
            out[r0 + 1] = rb;
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
        const int pairs = kWaves * kRowsPerWave / 2;
        for (int pi = threadIdx.x; pi < pairs; pi += kThreads) {
            const int64_t r0 = (int64_t)blockIdx.x * kWaves * kRowsPerWave + 2 * pi;
            if (r0 >= a.w.rows) break;
            rope_pair_store(a.rope, r0, rowbuf[2 * pi], rowbuf[2 * pi + 1], a.out);
        }
        return;
    }
    if (valid && li == 0) {
        if (MODE == GEMV_STORE) a.out[row] = acc;
        else if (MODE == GEMV_ADD) a.out[row] += acc;
        else swiglu_store(a, row, acc, acc2);
    }
}

// ---------------------------------------------------------------- streamed GEMV
// Large matrices (the logits, and every projection of a large model's decode
// step): a grid of resident workgroups walks tiles of kWaves * 64 / LPR rows.
// LPR lanes own a row and each takes CPL chunks of it (LPR * CPL covers the
// row with few clamped extra loads), so one batch of CPL 16-byte loads per
// lane holds the whole tile; the batch of the workgroup's next tile is issued
// before the current one is multiplied, and the input row is staged once per
// workgroup.
//
// The input row sits in LDS as float4 quads with each weight chunk's quads
// rotated by c / (8 / QPC) (QPC quads per chunk).  One ds_read_b128 serves 8
// lanes per clock, and the lanes of a row group read one quad index of
// consecutive chunks: the rotation puts those 8 reads on 8 distinct 16-byte
// bank groups, where the plain layout put 4 (Q8_0) or 8 (Q4_0) of them on one.
template <int FMT>
constexpr int quads_per_chunk() {
    return FMT == DT_Q8_0 ? 4 : FMT == DT_Q4_0 ? 8 : 2;
}
template <int FMT>
__device__ __forceinline__ int xq_slot(int c, int q) {
    constexpr int QPC = quads_per_chunk<FMT>(), CPB = 8 / QPC;
    return c * QPC + ((q + c / CPB) & (QPC - 1));
}
// Slot of logical quad Q (input elements 4Q .. 4Q + 3).
template <int FMT>
__device__ __forceinline__ int xq_slot_of(int Q) {
    constexpr int QPC = quads_per_chunk<FMT>();
    return xq_slot<FMT>(Q / QPC, Q % QPC);
}

// gemv::chunk_dot over the rotated layout (same products, same order).
template <int FMT>
__device__ __forceinline__ float chunk_dot_rot(const int4& q, float d, int c, const float4* xq) {
    const int32_t* w = (const int32_t*)&q;
    float s = 0.f;
    if constexpr (FMT == DT_Q8_0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 x = xq[xq_slot<FMT>(c, i)];
            const int32_t v = w[i];
            s += (float)(int8_t)(v) * x.x;
            s += (float)(int8_t)(v >> 8) * x.y;
            s += (float)(int8_t)(v >> 16) * x.z;
            s += (float)(int8_t)(v >> 24) * x.w;
        }
        return d * s;
    } else if constexpr (FMT == DT_Q4_0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 xl = xq[xq_slot<FMT>(c, i)], xh = xq[xq_slot<FMT>(c, 4 + i)];
            const uint32_t v = (uint32_t)w[i];
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
        const float4 x0 = xq[xq_slot<FMT>(c, 0)], x1 = xq[xq_slot<FMT>(c, 1)];
        s = (float)h[0] * x0.x + (float)h[1] * x0.y + (float)h[2] * x0.z + (float)h[3] * x0.w;
        s += (float)h[4] * x1.x + (float)h[5] * x1.y + (float)h[6] * x1.z + (float)h[7] * x1.w;
        return s;
    }
}

// Input row (IN_X) or RMS-normalised input row (IN_NORM) into the rotated LDS
// layout.  issue() loads the thread's XQ quads of x (and of the gain) and is
// called before the weight loads, so that finish(), which waits for them,
// leaves the weight loads in flight: the vector memory counter retires loads
// in issue order.  Every load is issued unconditionally (indices past the row
// clamped to its last quad, their values unused), so that the compiler's wait
// counts stay exact; a load inside a branch makes it wait for every load at
// the join.
template <int FMT, int INP, int XQ>
struct StageRow {
    float4 xv[XQ], gv[XQ];
    uint2 ph[INP == IN_PAIR ? XQ : 1], pl[INP == IN_PAIR ? XQ : 1];  // IN_PAIR: the quad's two f16 terms
    __device__ __forceinline__ void issue(const GemvInput& in, int nq) {
#pragma unroll
        for (int i = 0; i < XQ; i++) {
            const int Q = min((int)threadIdx.x + i * kThreads, nq - 1);
            if constexpr (INP == IN_PAIR) {
                ph[i] = ((const uint2*)in.xh)[Q];
                pl[i] = ((const uint2*)in.xl)[Q];
            } else {
                xv[i] = ((const float4*)in.x)[Q];
            }
            if constexpr (INP == IN_NORM) gv[i] = ((const float4*)in.norm)[Q];
        }
    }
    __device__ __forceinline__ void finish(const GemvInput& in, int K, int nq, float4* xq, float* red) {
        float scale = 1.f;
        if constexpr (INP == IN_NORM) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < XQ; i++)
                if (threadIdx.x + i * kThreads < nq)
                    ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
            ss = block_sum(ss, red);
            scale = 1.0f / sqrtf(ss / (float)K + in.eps);
        }
#pragma unroll
        for (int i = 0; i < XQ; i++) {
            const int Q = threadIdx.x + i * kThreads;
            if (Q < nq) {
                float4 v;
                if constexpr (INP == IN_PAIR) {
                    const f16* h = (const f16*)&ph[i];
                    const f16* l = (const f16*)&pl[i];
                    v = make_float4((float)h[0] + (float)l[0], (float)h[1] + (float)l[1], (float)h[2] + (float)l[2],
                                    (float)h[3] + (float)l[3]);
                } else {
                    v = xv[i];
                }
                if constexpr (INP == IN_NORM) {
                    v.x = (v.x * scale) * gv[i].x;
                    v.y = (v.y * scale) * gv[i].y;
                    v.z = (v.z * scale) * gv[i].z;
                    v.w = (v.w * scale) * gv[i].w;
                }
                xq[xq_slot_of<FMT>(Q)] = v;
            }
        }
    }
};

// Weights per 16-byte chunk, and the input quads per thread that a row of
// LPR * CPL chunks needs (at most kMaxStageQuads).
template <int FMT>
constexpr int weights_per_chunk() {
    return FMT == DT_Q8_0 ? 16 : FMT == DT_Q4_0 ? 32 : 8;
}
constexpr int kMaxStageQuads = 8;
template <int FMT, int LPR, int CPL>
constexpr int stage_quads() {
    const int q = (LPR * CPL * weights_per_chunk<FMT>() / 4 + kThreads - 1) / kThreads;
    return q < kMaxStageQuads ? q : kMaxStageQuads;
}

template <int FMT, int LPR, int CPL, int MODE, int INP>
__global__ __launch_bounds__(kThreads) void gemv_stream_kernel(GemvArgs a, int tiles) {
    extern __shared__ float4 xq[];
    __shared__ float red[16];
    constexpr int RPW = 64 / LPR, RT = kWaves * RPW;
    constexpr int NM = MODE == GEMV_SWIGLU ? 2 : 1;
    const int K = a.w.cols, nch = chunks_of<FMT>(K), rows = a.w.rows;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane % LPR;
    const int rin = wave * RPW + lane / LPR;  // this lane group's row within a tile
    int4 q[2][NM][CPL];
    f16 d[2][NM][CPL];
    // Chunk indices past the row are clamped to its last chunk (their values
    // unused), rows past the matrix to its last row; the loads go out
    // unconditionally (see StageRow).
    auto load = [&](int t, int b) {
        const int64_t row = min((int64_t)t * RT + rin, (int64_t)rows - 1);
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const void* wq = m ? a.u.q : a.w.q;
            const void* ws = m ? a.u.s : a.w.s;
#pragma unroll
            for (int u = 0; u < CPL; u++) {
                const int c = min(li + u * LPR, nch - 1);
                q[b][m][u] = gemv::load_q(wq, gemv::chunk_qoff<FMT>(row, K, c));
                if constexpr (FMT != DT_F16) d[b][m][u] = gemv::load_s(ws, gemv::chunk_soff<FMT>(row, K, c));
            }
        }
    };
    int t = blockIdx.x;  // < tiles: the grid is at most one workgroup per tile
    {
        StageRow<FMT, INP, stage_quads<FMT, LPR, CPL>()> sr;
        sr.issue(a.in, K / 4);
        asm volatile("" ::: "memory");  // (keeps the input loads ahead of the weight loads)
        load(t, 0);
        sr.finish(a.in, K, K / 4, xq, red);
    }
    __syncthreads();
    auto compute = [&](int b) {
        float acc[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            acc[m] = 0.f;
#pragma unroll
            for (int u = 0; u < CPL; u++) {
                const int c = li + u * LPR;
                if (c < nch) acc[m] += chunk_dot_rot<FMT>(q[b][m][u], FMT == DT_F16 ? 1.f : (float)d[b][m][u], c, xq);
            }
            acc[m] = lane_sum<LPR>(acc[m]);
        }
        const int64_t row = (int64_t)t * RT + rin;
        if constexpr (MODE == GEMV_QKV_ROPE) {
            // rows (2i, 2i + 1) are neighbouring lane groups of one wave
            const float odd = __shfl_xor(acc[0], LPR, 64);
            if (li == 0 && ((lane / LPR) & 1) == 0 && row < rows) rope_pair_store(a.rope, row, acc[0], odd, a.out);
        } else if (row < rows && li == 0) {
            if (MODE == GEMV_STORE) a.out[row] = acc[0];
            else if (MODE == GEMV_ADD) a.out[row] += acc[0];
            else swiglu_store(a, row, acc[0], acc[NM - 1]);
        }
    };
    // The next tile's loads go out before this tile is multiplied; the two
    // register sets alternate (the loop is unrolled over both, so they stay in
    // registers), and the last tile takes a path with no loads behind it.
    for (;;) {
        int nt = t + gridDim.x;
        if (nt >= tiles) {
            compute(0);
            break;
        }
        load(nt, 1);
        compute(0);
        t = nt;
        nt = t + gridDim.x;
        if (nt >= tiles) {
            compute(1);
            break;
        }
        load(nt, 0);
        compute(1);
        t = nt;
    }
}

// (LPR, CPL) for a row of nch chunks: the fewest lanes per row whose batch of
// at most 8 chunks per lane covers the row (tiles of more rows, more loads per
// lane in flight), CPL then as small as that allows.
struct TallShape {
    int lpr = 0, cpl = 0;
};
inline TallShape tall_shape(int nch) {
    // four chunks per lane where that covers the row with at most 1/8 to spare
    // (at the 1.7B shape's K = 2,048, 32 lanes x 4 chunks: gate+up 9.4 -> 8.7 us,
    // QKV 6.5 -> 6.2, logits 21.7 -> 20.2 against 16 x 8)
    for (int lpr = 4; lpr <= 64; lpr *= 2)
        if ((nch + lpr - 1) / lpr <= 4 && 8 * (4 * lpr - nch) <= nch) return {lpr, 4};
    for (int lpr = 4; lpr <= 64; lpr *= 2) {
        const int cpl = (nch + lpr - 1) / lpr;
        if (cpl <= 8) return {lpr, cpl <= 4 ? 4 : cpl <= 5 ? 5 : 8};
    }
    return {};
}
// The same, widened to more lanes per row (while a lane keeps at least 4
// chunks) until the grid has a tile for every CU.
inline TallShape stream_shape(int nch, int rows, int cus, int max_lpr = 64) {
    TallShape ts = tall_shape(nch);
    const char* e = std::getenv("ALPACA_HIP_STREAM_LPR");  // tuning: lanes per row (4..64)
    if (e && std::atoi(e) >= 4 && std::atoi(e) <= max_lpr) {
        const int lpr = std::atoi(e), cpl = (nch + lpr - 1) / lpr;
        if (cpl <= 8) return {lpr, cpl <= 4 ? 4 : cpl <= 5 ? 5 : 8};
    }
    while (ts.lpr && ts.lpr < max_lpr && (int64_t)(rows + 4 * 64 / ts.lpr - 1) / (4 * 64 / ts.lpr) < cus &&
           (nch + 2 * ts.lpr - 1) / (2 * ts.lpr) >= 4) {
        ts.lpr *= 2;
        const int cpl = (nch + ts.lpr - 1) / ts.lpr;
        ts.cpl = cpl <= 4 ? 4 : cpl <= 5 ? 5 : 8;
    }
    return ts;
}

template <int FMT, int LPR, int CPL, int MODE, int INP>
hipError_t run_stream(const GemvArgs& a, hipStream_t st) {
    static int per_cu[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipGetLastError();
    const size_t lds = (size_t)a.w.cols * sizeof(float);
    int& occ = per_cu[dev & 63];
    if (!occ) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_stream_kernel<FMT, LPR, CPL, MODE, INP>, kThreads,
                                                         lds) != hipSuccess || n < 1) {
            (void)hipGetLastError();
            n = 1;
        }
        occ = n;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return hipGetLastError();
    const int rt = kWaves * (64 / LPR), tiles = (a.w.rows + rt - 1) / rt;
    int per = occ;
    // tuning: ALPACA_HIP_STREAM_OCC caps the workgroups per CU
    if (const char* e = std::getenv("ALPACA_HIP_STREAM_OCC")) per = std::max(1, std::min(occ, std::atoi(e)));
    const int grid = std::min(tiles, std::max(1, cus) * per);
    gemv_stream_kernel<FMT, LPR, CPL, MODE, INP><<<grid, kThreads, lds, st>>>(a, tiles);
    return hipGetLastError();
}

template <int FMT, int MODE, int INP>
hipError_t dispatch_stream(const TallShape& ts, const GemvArgs& a, hipStream_t st) {
#define STREAM(L, CP) \
    if (ts.lpr == L && ts.cpl == CP) return run_stream<FMT, L, CP, MODE, INP>(a, st);
    STREAM(4, 4) STREAM(4, 5) STREAM(4, 8) STREAM(8, 4) STREAM(8, 5) STREAM(8, 8) STREAM(16, 4) STREAM(16, 5)
    STREAM(16, 8) STREAM(32, 4) STREAM(32, 5) STREAM(32, 8)
    if constexpr (MODE != GEMV_QKV_ROPE) {  // (RoPE pairs need two rows per wave)
        STREAM(64, 4) STREAM(64, 5) STREAM(64, 8)
    }
#undef STREAM
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
    if (mode == GEMV_ADD) return inp == IN_MERGE  ? dispatch<FMT, GEMV_ADD, IN_MERGE>(lpr, a, st)
                                 : inp == IN_PAIR ? dispatch<FMT, GEMV_ADD, IN_PAIR>(lpr, a, st)
                                                  : dispatch<FMT, GEMV_ADD, IN_X>(lpr, a, st);
    if (mode == GEMV_SWIGLU) return inp == IN_NORM   ? dispatch<FMT, GEMV_SWIGLU, IN_NORM>(lpr, a, st)
                                    : inp == IN_PAIR ? dispatch<FMT, GEMV_SWIGLU, IN_PAIR>(lpr, a, st)
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

// Whether a launch takes the streamed kernel: at least 4 MB of weights, a row
// that one batch of at most 8 chunks per lane on 64 lanes covers and that the
// stager's quads cover, a plain or RMS-normalised input row (the merge of
// attention partials runs as its own kernel in front of a large Wo), 16-byte
// aligned input rows, and for the RoPE epilogue two rows per wave.
// ALPACA_HIP_GEMV_STREAM=0 keeps gemv_kernel (tuning).
static bool stream_pays(const DevMatrix& w, const GemvInput& in, int mode, int inp) {
    const int64_t bytes = w.dtype == DT_Q8_0   ? (int64_t)w.rows * w.cols / 32 * 34
                          : w.dtype == DT_Q4_0 ? (int64_t)w.rows * w.cols / 32 * 18
                                               : (int64_t)w.rows * w.cols * 2;
    const int nch = w.dtype == DT_Q8_0 ? w.cols / 16 : w.dtype == DT_Q4_0 ? w.cols / 32 : w.cols / 8;
    const char* e = std::getenv("ALPACA_HIP_GEMV_STREAM");
    if (e && e[0] == '0') return false;
    if (bytes < (4 << 20) || nch > 64 * 8 || w.cols % 4 || w.cols / 4 > kMaxStageQuads * kThreads) return false;
    if (inp == IN_MERGE || ((uintptr_t)in.x & 15) || (inp == IN_NORM && ((uintptr_t)in.norm & 15)) ||
        (inp == IN_PAIR && (((uintptr_t)in.xh | (uintptr_t)in.xl) & 7)))
        return false;
    return mode != GEMV_QKV_ROPE || tall_shape(nch).lpr <= 32;
}

template <int FMT>
hipError_t dispatch_stream_fmt(int mode, int inp, const GemvArgs& a, hipStream_t st) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return hipGetLastError();
    // (RoPE pairs need two rows per wave: at most 32 lanes per row)
    const TallShape ts = stream_shape(gemv_nch<FMT>(a.w.cols), a.w.rows, cus, mode == GEMV_QKV_ROPE ? 32 : 64);
    if (mode == GEMV_QKV_ROPE && ts.lpr > 32) return hipErrorInvalidValue;
    if (mode == GEMV_STORE) return inp == IN_NORM ? dispatch_stream<FMT, GEMV_STORE, IN_NORM>(ts, a, st)
                                                  : dispatch_stream<FMT, GEMV_STORE, IN_X>(ts, a, st);
    if (mode == GEMV_ADD) return inp == IN_PAIR ? dispatch_stream<FMT, GEMV_ADD, IN_PAIR>(ts, a, st)
                                                : dispatch_stream<FMT, GEMV_ADD, IN_X>(ts, a, st);
    if (mode == GEMV_SWIGLU) return inp == IN_NORM   ? dispatch_stream<FMT, GEMV_SWIGLU, IN_NORM>(ts, a, st)
                                    : inp == IN_PAIR ? dispatch_stream<FMT, GEMV_SWIGLU, IN_PAIR>(ts, a, st)
                                                     : dispatch_stream<FMT, GEMV_SWIGLU, IN_X>(ts, a, st);
    return dispatch_stream<FMT, GEMV_QKV_ROPE, IN_NORM>(ts, a, st);
}

hipError_t launch_gemv_ex(const DevMatrix& w, const DevMatrix* w_up, const GemvInput& in, const GemvRope* rope,
                          float* out, int mode, hipStream_t st) {
    const int inp = in.partials ? IN_MERGE : in.norm ? IN_NORM : in.xh ? IN_PAIR : IN_X;
    if (inp == IN_PAIR && (!in.xl || (mode != GEMV_ADD && mode != GEMV_SWIGLU))) return hipErrorInvalidValue;
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
    if (stream_pays(w, in, mode, inp)) {
        switch (w.dtype) {
        case DT_Q8_0: return dispatch_stream_fmt<DT_Q8_0>(mode, inp, a, st);
        case DT_Q4_0: return dispatch_stream_fmt<DT_Q4_0>(mode, inp, a, st);
        default: return dispatch_stream_fmt<DT_F16>(mode, inp, a, st);
        }
    }
    const int lpr = pick_lpr(w.rows);
    switch (w.dtype) {
    case DT_Q8_0: return dispatch_fmt<DT_Q8_0>(lpr, mode, inp, a, st);
    case DT_Q4_0: return dispatch_fmt<DT_Q4_0>(lpr, mode, inp, a, st);
    default: return dispatch_fmt<DT_F16>(lpr, mode, inp, a, st);
    }
}

bool gemv_streams(const DevMatrix& w) {
    GemvInput in;
    return stream_pays(w, in, GEMV_ADD, IN_X);
}

hipError_t launch_gemv(const DevMatrix& w, const DevMatrix* w_up, const float* x, const float* norm, float eps,
                       float* out, int mode, hipStream_t st) {
    GemvInput in;
    in.x = x;
    in.norm = norm;
    in.eps = eps;
    return launch_gemv_ex(w, w_up, in, nullptr, out, mode, st);
}

hipError_t launch_gemv_pair(const DevMatrix& w, const DevMatrix* w_up, const f16* xh, const f16* xl, float* out,
                            f16* outh, f16* outl, int mode, hipStream_t st) {
    if (!xh || !xl || (mode == GEMV_SWIGLU && (!w_up || !outh || !outl)) || (mode == GEMV_ADD && !out) ||
        (mode != GEMV_ADD && mode != GEMV_SWIGLU))
        return hipErrorInvalidValue;
    GemvInput in;
    in.xh = xh;
    in.xl = xl;
    GemvArgs a;
    a.w = w;
    a.u = w_up ? *w_up : w;
    a.in = in;
    a.out = out;
    a.outh = outh;
    a.outl = outl;
    if (stream_pays(w, in, mode, IN_PAIR)) {
        switch (w.dtype) {
        case DT_Q8_0: return dispatch_stream_fmt<DT_Q8_0>(mode, IN_PAIR, a, st);
        case DT_Q4_0: return dispatch_stream_fmt<DT_Q4_0>(mode, IN_PAIR, a, st);
        default: return dispatch_stream_fmt<DT_F16>(mode, IN_PAIR, a, st);
        }
    }
    const int lpr = pick_lpr(w.rows);
    switch (w.dtype) {
    case DT_Q8_0: return dispatch_fmt<DT_Q8_0>(lpr, mode, IN_PAIR, a, st);
    case DT_Q4_0: return dispatch_fmt<DT_Q4_0>(lpr, mode, IN_PAIR, a, st);
    default: return dispatch_fmt<DT_F16>(lpr, mode, IN_PAIR, a, st);
    }
}
