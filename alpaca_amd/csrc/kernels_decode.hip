// Persistent single-token decode for gfx950: one launch runs a
// whole decode step of the Llama forward pass (every layer, the logits and the
// greedy arg-max) for one token.
//
// Replaces the reference's fused decode dispatch chain (MetalLlamaModel.swift:
// 344-356 and the greedy chain at :234-270: decodeQKV, ropeQKVStore, split-K
// attention + merge, decodeProjection(wo, add), decodeGateUp,
// decodeProjection(wDown, add), then norm + logits and argmax_logits).  The
// CPU semantics are LlamaCPUModel.forward for one token
// (LlamaCPUModel.swift:24-61).
//
// Why one launch: at these model sizes each projection streams 0.3-2 MB, a
// fraction of a microsecond of HBM time, while a kernel boundary costs several
// microseconds.  Here the phases of a layer hand results to each other inside
// one launch:
//
//   P1 QKV      rows of the stacked [q|k|v] matrix with the RMSNorm prologue and
//               the RoPE epilogue; k/v rows also go to the KV cache.
//   P2 attn     split-K attention: item (KV head, split of the context) serves
//               the G query heads of that KV head; writes (max, sum, output).
//   P3 merge    one item per query head merges its splits into the context row.
//   P4 Wo       rows of Wo plus the residual.
//   P5 gate/up  rows of gate and up with the RMSNorm prologue, SwiGLU epilogue.
//   P6 down     rows of down plus the residual.
//   then P7 logits (final norm + output rows + a per-workgroup arg-max) and
//   P8 the arg-max reduction in workgroup 0.
//
// Hand-off: every value a phase produces is written as an 8-byte exchange word,
// (launch tag << 32) | f32 bits, with one agent-scope atomic store; a consumer
// polls the words themselves with agent-scope atomic loads until every tag
// equals this launch's tag.  The barrier and the data transfer are one memory
// round trip, and a consumer waits only for the words it reads.  Each phase
// has its own words per layer, so no word is written twice in a launch; the
// tag (a per-session counter advanced by every launch) separates launches.
//
// Before waiting, a workgroup issues the loads of its weight rows (and, in P2,
// of its cached K/V rows), so HBM latency overlaps the wait.  Rows written to
// the KV cache in this launch are read by attention only through the exchange
// words; cache rows of earlier positions come from earlier launches, whose
// completion makes them visible.
//
// A wait copies words into LDS as they arrive, thread by thread.  When the
// destination is a buffer the previous phase read (xn, the input row of QKV
// and of gate/up), a workgroup barrier precedes the wait, so the waves of a
// workgroup that finish their rows first (or have none) cannot overwrite the
// row under the waves still reading it.  A wait into xres needs none: the
// residual epilogue reads xres[r] before it publishes word r, and the next
// phase writes xres[r] only once word r has arrived.
//
// The launch parameters and the current layer's table sit in LDS, so every
// phase reads them with ds_read rather than with dependent memory loads.
// Every phase is inlined into the kernel (a call would save and restore the
// callee-saved registers through scratch memory on each phase); to keep the
// build parallel, this file is compiled once per (weight format, head dim)
// with DECODE_FMT / DECODE_HD / DECODE_ENTRY set, each object holding the
// kernels for its group sizes, and once without them for the host side.
//
// Every wait is bounded: past `timeout_ticks` of the wall clock, or when any
// workgroup has raised the shared abort word, a workgroup raises the abort
// word and the mapped status word and returns, so a launch always drains.  The
// grid is one workgroup per CU, all resident at once on a device that no other
// long-lived grid holds (the host orders persistent launches one at a time).
#include "common.h"
#include "gemv_chunks.h"

#include <limits.h>

namespace {

constexpr int kT = 256;  // threads per workgroup
constexpr int kWaves = kT / 64;
constexpr int kMaxSplitLen = 256;  // positions per attention item (one per thread)
constexpr int kMinSplitLen = 64;
constexpr int kRedFloats = 32;

// Attention decomposition for a context of `len` positions: split length in
// [64, 256] aiming at `target` items over all KV heads.
__device__ __host__ inline int split_len_for(int len, int kv_heads, int target) {
    int sl = (len * kv_heads + target - 1) / target;
    sl = (sl + kMinSplitLen - 1) / kMinSplitLen * kMinSplitLen;
    return sl < kMinSplitLen ? kMinSplitLen : (sl > kMaxSplitLen ? kMaxSplitLen : sl);
}

// Item `it` of the attention phase: KV head j, split s.  Items over full splits
// come first (head-major) and the last split of every head, which holds the
// context's remainder, after them, so the workgroups that run one item more than
// the others run a short one.
__device__ inline void item_split(int it, int S, int kv_heads, int& j, int& s) {
    const int per = S - 1, full = kv_heads * per;
    if (it < full) {
        j = it / per;
        s = it - j * per;
    } else {
        j = it - full;
        s = per;
    }
}

// Group-size bucket: the kernel variant sized for G query heads per KV head.
__host__ __device__ inline int group_bucket(int g) { return g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : g <= 8 ? 8 : 16; }

// Output rows the logits phase stages in LDS: the rows' quants (or f16 values)
// exactly as they lie in HBM, padded to whole 1 KB DMA instructions, then, for
// quantised formats, their f16 scales padded to whole 256-byte instructions.
// They sit past every other phase's LDS (byte offset out_lds_off), so the copy
// can be issued layers before the logits phase reads it.
__host__ __device__ inline int staged_row_bytes(int fmt, int K) {
    return fmt == DT_Q8_0 ? K : fmt == DT_Q4_0 ? K / 2 : 2 * K;
}
__host__ __device__ inline int staged_q_bytes(int fmt, int K, int n) {
    return (n * staged_row_bytes(fmt, K) + 1023) / 1024 * 1024;
}
__host__ __device__ inline int staged_s_bytes(int fmt, int K, int n) {
    return fmt == DT_F16 ? 0 : (n * (K / 32) * 2 + 255) / 256 * 256;
}
// Layers over whose QKV phases the copy is spread (a slice per layer, issued
// before the phase's wait, where it overlaps the hand-off).
constexpr int kStageLayers = 8;

}  // namespace

#ifdef DECODE_FMT

namespace {

using gemv::RowStream;
typedef unsigned long long u64;

// ------------------------------------------------------------------ LDS
// Launch parameters and the current layer's table (copied by every workgroup).
// Sizes rounded to 16 bytes: the dynamic LDS placed after these arrays is read
// with 128-bit accesses, which lose their alignment (and most of their speed)
// otherwise.
__shared__ __attribute__((aligned(16))) unsigned char lds_params[(sizeof(DecodeParams) + 15) & ~size_t(15)];
__shared__ __attribute__((aligned(16))) unsigned char lds_layer[(sizeof(DecLayer) + 15) & ~size_t(15)];
__device__ __forceinline__ const DecodeParams& P() { return *reinterpret_cast<const DecodeParams*>(lds_params); }
__device__ __forceinline__ const DecLayer& LY() { return *reinterpret_cast<const DecLayer*>(lds_layer); }

// Dynamic LDS: [0, 32) reductions; xres [hidden], the residual row of the
// current half-layer; xn [stage], the normalised or staged input row; then
// scratch.
extern __shared__ __attribute__((aligned(16))) float dyn_lds[];
struct Shared {
    float* red;
    float* xres;
    float* xn;
    float* scr;
};
__device__ __forceinline__ Shared lds_of() {
    Shared l;
    l.red = dyn_lds;
    l.xres = dyn_lds + kRedFloats;
    l.xn = l.xres + P().hidden;
    l.scr = l.xn + P().stage;
    return l;
}


// ------------------------------------------------------------------ exchange words
__device__ __forceinline__ u64 ld_word(const u64* p) {
    return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put_word(u64* p, float v, unsigned tag) {
    __hip_atomic_store(gptr(p), ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_flag(const unsigned* p) {
    return __hip_atomic_load(gptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Ctl {
    unsigned tag;
    unsigned* abort_word;
    int* status;
    long long timeout;
    unsigned long long* sub;  // profiling: the sub-point stamps, or null
};

// Profiling: thread 0 stamps sub-point k of the attention phase (the points
// after the phase-end stamps; each layer overwrites the previous layer's).
// The pointer travels in Ctl (registers), so an untraced launch pays one
// scalar test per point.
__device__ __forceinline__ void substamp(const Ctl& c, int k) {
    if (c.sub && threadIdx.x == 0) *gptr(c.sub + (int64_t)k * gridDim.x + blockIdx.x) = wall_clock64();
}

__device__ __noinline__ void raise_abort(Ctl c) {
    __hip_atomic_store(gptr(c.abort_word), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c.status) *(volatile int*)c.status = 1;
}

// Waits until the n words src(0..n-1) carry this launch's tag and copies their
// values to dst[0..n-1] (LDS).  Called by every thread of the workgroup;
// returns false (for every thread) when the launch is aborting.  All of a
// thread's pending words are re-polled together, so a wait costs one round
// trip once the data is there.  Indices past n are clamped to word n-1 for
// loading (never stored).  With keep, thread t also returns in keep[k] the
// value of word t + 256k (k < 8; undefined past n).
template <class Src>
__device__ __forceinline__ bool wait_words_at(Src src, int n, float* dst, const Ctl& c, float* keep = nullptr) {
    constexpr int B = 8;
    int bad = 0;
    for (int base = 0; base < n && !bad; base += B * kT) {
        u64 w[B];
        unsigned pend = 0;
#pragma unroll
        for (int k = 0; k < B; k++) {
            const int i = base + threadIdx.x + k * kT;
            w[k] = ld_word(src(i < n ? i : n - 1));
            if (i < n) pend |= 1u << k;
        }
        long long t0 = 0;
        int it = 0;
        while (true) {
#pragma unroll
            for (int k = 0; k < B; k++)
                if (((pend >> k) & 1u) && (unsigned)(w[k] >> 32) == c.tag) {
                    dst[base + threadIdx.x + k * kT] = __uint_as_float((unsigned)w[k]);
                    pend &= ~(1u << k);
                }
            if (!pend) break;
            if ((it++ & 31) == 0) {
                const long long now = wall_clock64();
                if (t0 == 0) t0 = now;
                if (now - t0 > c.timeout || ld_flag(c.abort_word)) {
                    bad = 1;
                    break;
                }
            }
#pragma unroll
            for (int k = 0; k < B; k++) {
                const int i = base + threadIdx.x + k * kT;
                if ((pend >> k) & 1u) w[k] = ld_word(src(i < n ? i : n - 1));
            }
        }
        if (keep && base == 0) {
#pragma unroll
            for (int k = 0; k < B; k++) keep[k] = __uint_as_float((unsigned)w[k]);
        }
    }
    if (bad) raise_abort(c);
    return !__syncthreads_or(bad);
}
__device__ __forceinline__ bool wait_words(const u64* src, int n, float* dst, const Ctl& c) {
    return wait_words_at([src](int i) { return src + i; }, n, dst, c);
}

// Block-wide sum over the 256 threads (result in every thread).
__device__ __forceinline__ float block_sum4(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Element k of row r of a resident matrix, dequantised exactly (Quantization.swift:9-35).
__device__ __forceinline__ float matrix_elem(const DevMatrix& m, int64_t r, int k) {
    if (m.dtype == DT_F16) return (float)*gptr((const f16*)m.q + r * m.cols + k);
    const int nb = m.cols / 32;
    const float d = (float)*gptr(m.s + r * nb + k / 32);
    if (m.dtype == DT_Q8_0) return d * (float)(int)*gptr((const int8_t*)m.q + r * m.cols + k);
    const int j = k & 31;
    const uint8_t b = *gptr(m.q + (r * nb + k / 32) * 16 + (j & 15));
    return d * (float)((int)(j < 16 ? (b & 15) : (b >> 4)) - 8);
}

// The gain vector of an RMSNorm, loaded before the wait that precedes the
// norm: the first kNormRegs*256 entries in registers, any rest from memory.
constexpr int kNormRegs = 8;
struct NormGain {
    const float* w;
    float r[kNormRegs];
    __device__ __forceinline__ void load(const float* gain, int n) {
        w = gain;
#pragma unroll
        for (int k = 0; k < kNormRegs; k++) {
            const int i = threadIdx.x + k * kT;
            r[k] = *gptr(gain + (i < n ? i : 0));
        }
    }
};

// x (LDS, n floats) -> out = (x * (1/sqrt(mean(x^2) + eps))) * w  (CPUOps.rmsNorm, CPUOps.swift:144-159).
// The thread's first kNormRegs values are read once, unconditionally (index
// clamped, value unused past n), so the reads are in flight together.
__device__ __forceinline__ void rmsnorm_lds(const float* x, const NormGain& g, int n, float eps, float* out,
                                            float* red) {
    float xv[kNormRegs];
#pragma unroll
    for (int k = 0; k < kNormRegs; k++) {
        const int i = threadIdx.x + k * kT;
        xv[k] = x[i < n ? i : 0];
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kNormRegs; k++)
        if (threadIdx.x + k * kT < n) ss += xv[k] * xv[k];
    for (int i = threadIdx.x + kNormRegs * kT; i < n; i += kT) ss += x[i] * x[i];
    ss = block_sum4(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int k = 0; k < kNormRegs; k++) {
        const int i = threadIdx.x + k * kT;
        if (i < n) out[i] = (xv[k] * scale) * g.r[k];
    }
    for (int i = threadIdx.x + kNormRegs * kT; i < n; i += kT) out[i] = (x[i] * scale) * *gptr(g.w + i);
    __syncthreads();
}

// wait_words of an RMSNorm's input row into x, then the norm into out exactly
// as rmsnorm_lds computes it, with the values a thread polled taken from its
// registers instead of being read back from LDS.
__device__ __forceinline__ bool wait_rmsnorm(const u64* src, int n, float* x, const NormGain& g, float eps,
                                             float* out, float* red, const Ctl& c) {
    static_assert(kNormRegs == 8, "one register per word of the first wait pass");
    float v[kNormRegs];
    if (!wait_words_at([src](int i) { return src + i; }, n, x, c, v)) return false;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kNormRegs; k++)
        if (threadIdx.x + k * kT < n) ss += v[k] * v[k];
    for (int i = threadIdx.x + kNormRegs * kT; i < n; i += kT) ss += x[i] * x[i];
    ss = block_sum4(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int k = 0; k < kNormRegs; k++) {
        const int i = threadIdx.x + k * kT;
        if (i < n) out[i] = (v[k] * scale) * g.r[k];
    }
    for (int i = threadIdx.x + kNormRegs * kT; i < n; i += kT) out[i] = (x[i] * scale) * *gptr(g.w + i);
    __syncthreads();
    return true;
}

// ------------------------------------------------------------------ GEMV rows
// Rows [r0, r1) of one or two matrices (same shape) against xs in LDS, LPR
// lanes per row, kWaves*64/LPR rows per pass.  The first pass's weights are
// loaded by prefetch(); later passes are double-buffered (the next pass's
// loads are in flight while the current pass is reduced).  Rows past r1 are
// clamped to r1-1 for loading and never used.  epi(row, a0, a1) runs on the
// row's first lane.
template <int FMT, int LPR, bool TWO>
struct Rows {
    static constexpr int RPB = kWaves * (64 / LPR);
    RowStream<FMT, LPR> a0, a1, b0, b1;
    int li, local;
    __device__ __forceinline__ Rows() {
        const int lane = threadIdx.x & 63;
        li = lane % LPR;
        local = (threadIdx.x >> 6) * (64 / LPR) + lane / LPR;
    }
    __device__ __forceinline__ void load(RowStream<FMT, LPR>& s0, RowStream<FMT, LPR>& s1, const DevMatrix& w0,
                                         const DevMatrix& w1, int base, int r1) {
        const int r = min(base + local, r1 - 1);
        s0.prefetch(w0, r, w0.cols, li);
        if (TWO) s1.prefetch(w1, r, w0.cols, li);
    }
    __device__ __forceinline__ void prefetch(const DevMatrix& w0, const DevMatrix& w1, int r0, int r1) {
        if (r0 < r1) load(a0, a1, w0, w1, r0, r1);
    }
    template <typename Epi>
    __device__ __forceinline__ void pass(RowStream<FMT, LPR>& s0, RowStream<FMT, LPR>& s1, const DevMatrix& w0,
                                         const DevMatrix& w1, int base, int r1, const float* xs, Epi& epi) {
        const int r = base + local;
        float v0 = 0.f, v1 = 0.f;
        if (r < r1) {
            v0 = s0.finish(w0, r, w0.cols, li, xs);
            if (TWO) v1 = s1.finish(w1, r, w0.cols, li, xs);
        }
        v0 = lane_sum<LPR>(v0);
        if (TWO) v1 = lane_sum<LPR>(v1);
        if (r < r1 && li == 0) epi(r, v0, v1);
    }
    // Pairs (even row, odd row) for LPR <= 32: the two rows of a pair are
    // neighbouring lane groups of one wave, so their sums meet with one
    // shuffle; epi2(even_row, even_sum, odd_sum) runs on the even row's first lane.
    template <typename Epi2>
    __device__ __forceinline__ void pass_pairs(RowStream<FMT, LPR>& s0, const DevMatrix& w0, int base, int r1,
                                               const float* xs, Epi2& epi2) {
        static_assert(LPR <= 32, "a row pair must sit in one wave");
        const int r = base + local;
        float v = 0.f;
        if (r < r1) v = s0.finish(w0, r, w0.cols, li, xs);
        v = lane_sum<LPR>(v);
        float partner;
        if constexpr (LPR == 16) partner = xor_partner16(v);
        else if constexpr (LPR == 32) partner = xor_partner32(v);
        else partner = __shfl_xor(v, LPR, 64);
        if (r < r1 && li == 0 && (local & 1) == 0) epi2(r, v, partner);
    }
    template <typename Epi2>
    __device__ __forceinline__ void run_pairs(const DevMatrix& w0, int r0, int r1, const float* xs, Epi2 epi2) {
        for (int base = r0; base < r1;) {
            int nxt = base + RPB;
            if (nxt < r1) load(b0, b1, w0, w0, nxt, r1);
            pass_pairs(a0, w0, base, r1, xs, epi2);
            base = nxt;
            if (base >= r1) break;
            nxt = base + RPB;
            if (nxt < r1) load(a0, a1, w0, w0, nxt, r1);
            pass_pairs(b0, w0, base, r1, xs, epi2);
            base = nxt;
        }
    }
    template <typename Epi>
    __device__ __forceinline__ void run(const DevMatrix& w0, const DevMatrix& w1, int r0, int r1, const float* xs,
                                        Epi epi) {
        for (int base = r0; base < r1;) {
            int nxt = base + RPB;
            if (nxt < r1) load(b0, b1, w0, w1, nxt, r1);
            pass(a0, a1, w0, w1, base, r1, xs, epi);
            base = nxt;
            if (base >= r1) break;
            nxt = base + RPB;
            if (nxt < r1) load(a0, a1, w0, w1, nxt, r1);
            pass(b0, b1, w0, w1, base, r1, xs, epi);
            base = nxt;
        }
    }
};

// The rows of a projection handled by this workgroup.
__device__ __forceinline__ void my_rows(int rows_per_wg, int total, int& r0, int& r1) {
    r0 = min(total, (int)blockIdx.x * rows_per_wg);
    r1 = min(total, r0 + rows_per_wg);
}

// Runs `f.template go<LPR>()` with the lanes-per-row suited to a row count.
template <typename F>
__device__ __forceinline__ bool with_lpr(int rows, F& f) {
    if (rows <= kWaves) return f.template go<64>();
    if (rows <= 2 * kWaves) return f.template go<32>();
    return f.template go<16>();
}

// ------------------------------------------------------------------ phases

// P1: QKV rows with RMSNorm prologue and RoPE epilogue.  On return xres holds
// the layer's input row (kept for the Wo residual).  At most 32 lanes per
// row, so each RoPE pair (rows 2i, 2i+1: q and k rows come in adjacent pairs)
// is completed inside one wave.
template <int FMT>
struct PhaseQKV {
    const u64* xin;  // previous layer's xf words, or null for layer 0
    u64* out;        // this layer's qkv words
    int pos, token;
    Ctl c;
    template <int LPR_>
    __device__ bool go() {
        constexpr int LPR = LPR_ > 32 ? 32 : LPR_;
        const DecodeParams& p = P();
        const DecLayer& L = LY();
        const Shared sh = lds_of();
        const DevMatrix W = L.qkv;
        const int hd = p.hd, QW = p.heads * hd, KW = p.kv_heads * hd, half = hd / 2, cap = p.capacity;
        int r0, r1;
        my_rows(p.rows_qkv, W.rows, r0, r1);
        Rows<FMT, LPR, false> rw;
        rw.prefetch(W, W, r0, r1);
        const int H = p.hidden;
        NormGain gain;
        gain.load(L.attn_norm, H);
        // (cos, sin) of this lane's first pair (CPUOps.rope angle table, CPUOps.swift:196-201)
        const float2* rope = p.rope;
        const int rfirst = min(r0 + (rw.local & ~1), W.rows - 2);
        const float2 cs0 = gload_f2(rope + (int64_t)pos * half + (rfirst % hd) / 2);
        if (xin) {
            if (!wait_words(xin, H, sh.xres, c)) return false;
        } else {
            const DevMatrix E = p.embed;
            for (int k = threadIdx.x; k < H; k += kT) sh.xres[k] = matrix_elem(E, token, k);
            __syncthreads();
        }
        rmsnorm_lds(sh.xres, gain, H, p.eps, sh.xn, sh.red);
        // RoPE on the pair, f16 rounding of k/v as the cache stores them, cache
        // append at row pos (KVCache.write, KVCache.swift:44-63), publication.
        f16* kc = (f16*)L.kc;
        f16* vc = (f16*)L.vc;
        const unsigned tag = c.tag;
        u64* o = out;
        rw.run_pairs(W, r0, r1, sh.xn, [&](int r, float v0, float v1) {
#pragma clang fp contract(off)
            const int d = r % hd;
            if (r < QW + KW) {
                const float2 cs = r == rfirst ? cs0 : gload_f2(rope + (int64_t)pos * half + d / 2);
                const float ac = v0 * cs.x, bs = v1 * cs.y, as = v0 * cs.y, bc = v1 * cs.x;
                v0 = ac - bs;
                v1 = as + bc;
            }
            if (r >= QW) {
                const bool isk = r < QW + KW;
                const int h = (r - (isk ? QW : QW + KW)) / hd;
                const f16 h0 = (f16)v0, h1 = (f16)v1;
                f16* cache = (isk ? kc : vc) + ((int64_t)h * cap + pos) * hd + d;
                *gptr(cache) = h0;
                *gptr(cache + 1) = h1;
                v0 = (float)h0;
                v1 = (float)h1;
            }
            put_word(o + r, v0, tag);
            put_word(o + r + 1, v1, tag);
        });
        return true;
    }
};

// V rows in LDS: 16-byte chunk c of row r sits at slot c ^ vt_swz(r), the
// swizzle of the prefill flash kernel (kernels_attention.hip): the transpose
// reads (8 bytes from chunks 2d, 2d+1 of 4 consecutive rows per 16 lanes) and
// the row stores (whole rows) do not conflict.
__device__ __forceinline__ int vt_swz(int r) {
    return (((r ^ (r >> 3)) & 1) | (((r ^ (r >> 2)) & 1) << 1) | (((r >> 1) & 1) << 2));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Eight floats from 16-byte-aligned LDS, as two 16-byte reads.
struct float8 {
    float v[8];
};
__device__ __forceinline__ float8 ld_f8(const float* p) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    return float8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i % 4) of the 4 halves addressed by lane 4j + i/4, for j = 0..3.  When
// lanes 4j..4j+3 address V row R_j at dims d0, d0+4, d0+8, d0+12, lane i gets
// V[R_0..R_3][d0 + i]: a V^T fragment read from row-major V.
__device__ __forceinline__ f16x4 vt_read_tr(const uint8_t* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(f16x4, v);
}

// P2: split-K attention over the f16 cache.  Item (j, s): KV head j, context
// positions [s*SL, min((s+1)*SL, len)), SL <= 256, cut into 32-position
// chunks; chunk ch belongs to wave ch % 4.  The scores are computed transposed
// with v_mfma_f32_16x16x32_f16, S^T = K Q^T: the A operand is a K row fragment
// loaded straight from the cache into registers (16 bytes per lane, prefetched
// before the query arrives), the B operand the G query rows of the group
// (columns past G are zero).  Each query value enters as two f16 terms,
// hi = f16(q) and lo = f16(q - hi), which carry q to ~2^-22, so with K exact in
// f16 and float32 accumulation the scores keep float32 accuracy.  A lane then
// holds one query column at 4 positions of each 16-position tile: the B
// operand layout of O^T += V^T P^T once the position order inside a
// 32-position step is permuted identically on both operands.  P = 2^(s - max)
// enters as hi + lo of P * 2^14 (scaled so that lo stays out of the f16
// subnormals); V^T fragments come from LDS transpose reads of the V rows, which
// move global -> LDS by DMA (no registers; a workgroup with several items
// requests the next item's K rows once the current scores are reduced and its V
// rows once the current P.V is done).  Writes,
// per query head g of the group, the words
// [max (base-2 units), sum, unnormalised output[HD]] of the split
// (attention_decode.metal:27-116 computes the same triple).
template <int HD, int GM>
__device__ __forceinline__ bool attention_phase(const u64* qkv, u64* part, int pos, Ctl c) {
    constexpr int KC = HD / 32;                      // 32-dim steps of a score tile
    constexpr int DT = HD / 16;                      // 16-dim tiles of the output
    constexpr int NCH = kMaxSplitLen / 32 / kWaves;  // 32-position chunks per wave
    constexpr int ROWB = HD * 2;                     // bytes per V row in LDS
    constexpr float kPScale = 16384.f, kPUnscale = 1.f / 16384.f;
    const DecodeParams& p = P();
    const DecLayer& L = LY();
    float* scr = lds_of().scr;
    const int heads = p.heads, kvh = p.kv_heads, G = heads / kvh, QW = heads * HD, KW = kvh * HD;
    const int cap = p.capacity, max_splits = p.max_splits;
    const int len = pos + 1;
    const int SL = split_len_for(len, kvh, p.target_items);
    const int S = (len + SL - 1) / SL, items = kvh * S;
    const f16* kcache = (const f16*)L.kc;
    const f16* vcache = (const f16*)L.vc;
    float* qs = scr;                                   // [G][HD] query rows, then k and v of the current position
    float* kcur = qs + G * HD;                         // [HD]
    float* vcur = kcur + HD;                           // [HD]
    float* red = scr + GM * HD + 2 * HD;               // [GM][8]: per-wave max, then sum
    float* ws = red + GM * 8;                          // [kWaves][GM][HD]
    uint8_t* vt = (uint8_t*)(ws + kWaves * GM * HD);   // [kMaxSplitLen][HD] f16 V rows, chunk-swizzled
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, q4 = lane >> 4;         // MFMA layout: column / row group
    const float sl2 = 1.4426950408889634f / sqrtf((float)HD);
    auto fmax2 = [](float x, float y) { return fmaxf(x, y); };
    auto add2 = [](float x, float y) { return x + y; };
    auto sub = [&](int k) { substamp(c, k); };
    // An item's cached K rows (cache rows past nc are loaded from row 0 of the
    // split, valid memory, and never used).  A workgroup with several items loads
    // the next item's K rows (every chunk) as soon as the current scores are
    // reduced, and its V rows once the current P.V is done, so those loads
    // overlap the current item's softmax, P.V and publication.
    int4 kr[NCH][2][KC];
    auto rows_of = [&](int t, int64_t& base, int& ncached, int& nrows) {
        int jt, st;
        item_split(t, S, kvh, jt, st);
        const int q0 = st * SL, q1 = min(q0 + SL, len);
        ncached = min(q1, pos) - q0;
        nrows = q1 - q0;
        base = ((int64_t)jt * cap + q0) * HD;
    };
    auto load_k = [&](int t, bool all) {
        int64_t base;
        int ncached, nrows;
        rows_of(t, base, ncached, nrows);
#pragma unroll
        for (int ci = 0; ci < NCH; ci++) {
            if (!all && 32 * (wave + kWaves * ci) >= nrows) continue;  // uniform across the wave
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int r = 32 * (wave + kWaves * ci) + 16 * u + c16;
                const f16* row = kcache + base + (int64_t)(r < ncached ? r : 0) * HD + 8 * q4;
#pragma unroll
                for (int kc = 0; kc < KC; kc++) kr[ci][u][kc] = gload_i4(row + 32 * kc);
            }
        }
    };
    // V rows go global -> LDS by DMA (no registers): one global_load_lds_dwordx4
    // moves RPI whole rows, lane L filling slot L % CH of row L / CH with the
    // cache chunk that the swizzle puts there.  Every row of the 32-row chunks
    // the item covers is written; rows past the cached ones load row 0 of the
    // split (valid memory) and are overwritten before use.  Issued only when the
    // previous item's P.V reads of vt are over (after a barrier).
    auto dma_v = [&](int t) {
        constexpr int CH = HD / 8, RPI = 64 / CH;
        int64_t base;
        int ncached, nrows;
        rows_of(t, base, ncached, nrows);
        const int ninst = ((nrows + 31) & ~31) / RPI;
        const uint32_t vt_lds = __builtin_amdgcn_readfirstlane(lds_addr(vt));  // uniform: m0 takes an SGPR
        for (int i = wave; i < ninst; i += kWaves) {
            const int r = i * RPI + lane / CH, chunk = (lane % CH) ^ vt_swz(r);
            dma16(vcache + base + (int64_t)(r < ncached ? r : 0) * HD + chunk * 8, vt_lds + i * RPI * ROWB);
        }
    };
    if (blockIdx.x < items) {
        load_k(blockIdx.x, false);
        dma_v(blockIdx.x);
    }
    for (int it = blockIdx.x; it < items; it += gridDim.x) {
        sub(0);
        int j, s;
        item_split(it, S, kvh, j, s);
        const int p0 = s * SL, p1 = min(p0 + SL, len), n = p1 - p0;
        const int nc = min(p1, pos) - p0;  // positions read from the cache
        const bool has_cur = p1 == len;    // then position nc (the last) is the current one
        const int next = it + (int)gridDim.x;
        sub(1);
        // the query rows, and for the split holding the current position its k
        // and v rows, in one round trip
        {
            const int nq = G * HD, qo = j * G * HD, dk = QW + j * HD - nq - qo, dv = KW - HD;
            const u64* qb = qkv + qo;
            // sums of selects, not a chained select (which the compiler may turn into a stack lookup)
            auto src = [qb, nq, dk, dv](int i) { return qb + i + (i >= nq ? dk : 0) + (i >= nq + HD ? dv : 0); };
            if (!wait_words_at(src, has_cur ? nq + 2 * HD : nq, qs, c)) return false;
        }
        sub(2);
        sub(3);
        // B operand: column c16 = query head of the group, dims 32kc + 8q4 .. +7,
        // in base-2 exponent units, as hi + lo
        // (read unconditionally from a valid row and scaled by 0 past G: no branches)
        f16x8 qh[KC], ql[KC];
        {
            const float* qrow = qs + (c16 < G ? c16 : 0) * HD + 8 * q4;
            const float qm = c16 < G ? sl2 : 0.f;
#pragma unroll
            for (int kc = 0; kc < KC; kc++) {
                const float8 q8 = ld_f8(qrow + 32 * kc);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float x = q8.v[e] * qm;
                    const f16 h = (f16)x;
                    qh[kc][e] = h;
                    ql[kc][e] = (f16)(x - (float)h);
                }
            }
        }
        // S^T tiles: sacc[ci][u][r] = score(position 32ch + 16u + 4q4 + r, query column c16)
        f32x4 sacc[NCH][2];
        float mx = -INFINITY;
#pragma unroll
        for (int ci = 0; ci < NCH; ci++) {
            const int ch = wave + kWaves * ci;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                sacc[ci][u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
                if (32 * ch >= n) continue;  // uniform across the wave
                f16x8 kf[KC];
#pragma unroll
                for (int kc = 0; kc < KC; kc++) kf[kc] = __builtin_bit_cast(f16x8, kr[ci][u][kc]);
                if (has_cur && 32 * ch + 16 * u + c16 == nc) {  // the current position's k row
#pragma unroll
                    for (int kc = 0; kc < KC; kc++) {
                        const float8 k8 = ld_f8(kcur + 32 * kc + 8 * q4);
#pragma unroll
                        for (int e = 0; e < 8; e++) kf[kc][e] = (f16)k8.v[e];
                    }
                }
                f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < KC; kc++) {
                    a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kc], qh[kc], a, 0, 0, 0);
                    a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kc], ql[kc], a, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float v = 32 * ch + 16 * u + 4 * q4 + r < n ? a[r] : -INFINITY;
                    sacc[ci][u][r] = v;
                    mx = fmaxf(mx, v);
                }
            }
        }
        mx = xor32_combine(xor16_combine(mx, fmax2), fmax2);
        if (q4 == 0 && c16 < G) red[c16 * 8 + wave] = mx;
        // The V rows are in LDS once this wave's DMA has landed (the barrier
        // below then covers every wave's).  Rows past the cached ones are
        // rewritten: the current position's v row, and zeros past the split
        // (they get P = 0 but still enter the MFMA: no uninitialised value may
        // enter, 0 * NaN).  Each wave rewrites only rows its own DMA wrote, so
        // the rewrite cannot be overtaken by another wave's DMA.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        {
            constexpr int CH = HD / 8, RPI = 64 / CH;
            const int end = (n + 31) & ~31;
            for (int i = lane; i < (end - nc) * CH; i += 64) {
                const int r = nc + i / CH, slot = i % CH, chunk = slot ^ vt_swz(r);
                if ((r / RPI) % kWaves != wave) continue;
                f16x8 h;
                if (r < n) {  // r == nc: the current position
                    const float8 v8 = ld_f8(vcur + chunk * 8);
#pragma unroll
                    for (int e = 0; e < 8; e++) h[e] = (f16)v8.v[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) h[e] = (f16)0.f;
                }
                *(f16x8*)(vt + r * ROWB + slot * 16) = h;
            }
        }
        __syncthreads();
        // kr is free: the next item's K rows load during this item's softmax and P.V
        if (next < items) load_k(next, true);
        sub(4);
        const int gq = c16 < G ? c16 : 0;
        const float mg = fmaxf(fmaxf(red[gq * 8 + 0], red[gq * 8 + 1]), fmaxf(red[gq * 8 + 2], red[gq * 8 + 3]));
        // P in the B-operand layout: slot 4u + r of chunk ci is position 32ch + 16u + 4q4 + r
        f16x8 ph[NCH], pl[NCH];
        float ls = 0.f;
#pragma unroll
        for (int ci = 0; ci < NCH; ci++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = exp2f(sacc[ci][u][r] - mg);  // 0 for masked positions
                    ls += e;
                    const float x = e * kPScale;
                    const f16 h = (f16)x;
                    ph[ci][4 * u + r] = h;
                    pl[ci][4 * u + r] = (f16)(x - (float)h);
                }
        ls = xor32_combine(xor16_combine(ls, add2), add2);
        if (q4 == 0 && c16 < G) red[c16 * 8 + 4 + wave] = ls;
        sub(5);
        // O^T += V^T P^T: oacc[dt][r] = output(dim 16dt + 4q4 + r, query column c16) * 2^14
        f32x4 oacc[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ci = 0; ci < NCH; ci++) {
            const int ch = wave + kWaves * ci;
            if (32 * ch >= n) continue;  // uniform across the wave
            const int ra = 32 * ch + 4 * q4 + (c16 >> 2), rb = ra + 16;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int cb = 2 * dt + ((c16 & 3) >> 1), hb = (c16 & 1) * 8;
                const f16x4 lo = vt_read_tr(vt + ra * ROWB + ((cb ^ vt_swz(ra)) * 16) + hb);
                const f16x4 hi = vt_read_tr(vt + rb * ROWB + ((cb ^ vt_swz(rb)) * 16) + hb);
                const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[ci], oacc[dt], 0, 0, 0);
                oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[ci], oacc[dt], 0, 0, 0);
            }
        }
        if (c16 < G) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
                *(f32x4*)&ws[(wave * GM + c16) * HD + 16 * dt + 4 * q4] = oacc[dt];
        }
        __syncthreads();
        if (next < items) dma_v(next);  // every wave is done with vt: the next item's V rows
        sub(6);
        for (int i = tid; i < G * (HD + 2); i += kT) {
            const int g = i / (HD + 2), e = i - g * (HD + 2);
            float v;
            if (e == 0) {
                v = fmaxf(fmaxf(red[g * 8 + 0], red[g * 8 + 1]), fmaxf(red[g * 8 + 2], red[g * 8 + 3]));
            } else if (e == 1) {
                v = (red[g * 8 + 4] + red[g * 8 + 5]) + (red[g * 8 + 6] + red[g * 8 + 7]);
            } else {
                const int d = e - 2;
                v = ((ws[(0 * GM + g) * HD + d] + ws[(1 * GM + g) * HD + d]) +
                     (ws[(2 * GM + g) * HD + d] + ws[(3 * GM + g) * HD + d])) *
                    kPUnscale;
            }
            put_word(part + ((int64_t)(j * G + g) * max_splits + s) * (HD + 2) + e, v, c.tag);
        }
        __syncthreads();
        sub(7);
    }
    return true;
}

// P3: query head h merges its splits: w_s = 2^(m_s - M), out = sum_s w_s o_s / sum_s w_s l_s
// (attention_decode.metal:117-133 merges the same triples).
template <int HD>
__device__ __forceinline__ bool merge_phase(const u64* part, u64* ctx, int pos, Ctl c) {
    const DecodeParams& p = P();
    const Shared sh = lds_of();
    float* scr = sh.scr;
    float* red = sh.red;
    const int len = pos + 1, heads = p.heads, max_splits = p.max_splits;
    const int SL = split_len_for(len, p.kv_heads, p.target_items);
    const int S = (len + SL - 1) / SL;
    float* wsplit = scr + S * (HD + 2);
    for (int h = blockIdx.x; h < heads; h += gridDim.x) {
        if (!wait_words(part + (int64_t)h * max_splits * (HD + 2), S * (HD + 2), scr, c)) return false;
        float m = -INFINITY;
        for (int s = threadIdx.x; s < S; s += kT) m = fmaxf(m, scr[s * (HD + 2)]);
        m = wave_max(m);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float l = 0.f;
        for (int s = threadIdx.x; s < S; s += kT) {
            const float w = exp2f(scr[s * (HD + 2)] - M);
            wsplit[s] = w;
            l += w * scr[s * (HD + 2) + 1];
        }
        l = block_sum4(l, red + 4);
        const float inv = 1.0f / l;
        // QPD neighbouring lanes per output dim, lane q summing the splits
        // s = q mod QPD, so the whole workgroup shares the loop over the splits
        constexpr int QPD = kT / HD;
        const int d = threadIdx.x / QPD, q = threadIdx.x % QPD;
        float o = 0.f;
#pragma unroll 4
        for (int s = q; s < S; s += QPD) o += wsplit[s] * scr[s * (HD + 2) + 2 + d];
        o = lane_sum<QPD>(o);
        if (q == 0) put_word(ctx + h * HD + d, o * inv, c.tag);
        __syncthreads();
    }
    return true;
}

// P4 / P6: rows of a projection over a staged input row plus the residual.
template <int FMT>
struct PhaseResidual {
    int which;      // 0: Wo, 1: down
    const u64* in;  // input words (W.cols of them)
    u64* out;       // output words (W.rows)
    Ctl c;
    template <int LPR>
    __device__ bool go() {
        const DecodeParams& p = P();
        const Shared sh = lds_of();
        const DevMatrix W = which ? LY().down : LY().wo;
        int r0, r1;
        my_rows(which ? p.rows_down : p.rows_wo, W.rows, r0, r1);
        Rows<FMT, LPR, false> rw;
        rw.prefetch(W, W, r0, r1);
        // The wait below fills xn, which the previous phase (QKV, or gate/up)
        // reads as its input row: a wave that finished its rows early (or had
        // none) must not overwrite it while another wave of this workgroup is
        // still reading.  Attention and merge items end with a barrier, but a
        // workgroup that has none goes straight from QKV to here.
        __syncthreads();
        if (!wait_words(in, W.cols, sh.xn, c)) return false;
        const unsigned tag = c.tag;
        const float* xres = sh.xres;
        u64* o = out;
        rw.run(W, W, r0, r1, sh.xn, [&](int r, float v, float) { put_word(o + r, xres[r] + v, tag); });
        return true;
    }
};

// P5: gate and up rows with RMSNorm prologue and SwiGLU epilogue.  On return
// xres holds the row after attention (kept for the down residual).
template <int FMT>
struct PhaseGateUp {
    const u64* in;  // xa words
    u64* out;       // ffn words
    Ctl c;
    template <int LPR>
    __device__ bool go() {
        const DecodeParams& p = P();
        const DecLayer& L = LY();
        const Shared sh = lds_of();
        const DevMatrix Wg = L.gate, Wu = L.up;
        int r0, r1;
        my_rows(p.rows_ffn, Wg.rows, r0, r1);
        Rows<FMT, LPR, true> rw;
        rw.prefetch(Wg, Wu, r0, r1);
        NormGain gain;
        gain.load(L.ffn_norm, p.hidden);
        if (!wait_rmsnorm(in, p.hidden, sh.xres, gain, p.eps, sh.xn, sh.red, c)) return false;
        const unsigned tag = c.tag;
        u64* o = out;
        rw.run(Wg, Wu, r0, r1, sh.xn,
               [&](int r, float g, float u) { put_word(o + r, (g / (1.0f + expf(-g))) * u, tag); });
        return true;
    }
};

// Slice `part` of `parts` of the copy of rows [r0, r0 + n) of W (quants, then
// scales) into LDS at sq / ss, by DMA (global_load_lds: no registers).  A row
// share is one contiguous byte range of each stream, so instruction i of the
// copy moves bytes [1024 i, 1024 i + 1024) of the quants (256-byte pieces of
// the scales); lanes past the end re-read the range's last bytes (in bounds)
// into the padding.  A slice is a contiguous run of instructions, dealt to the
// waves in turn; they stay this wave's outstanding loads until its next wait.
template <int FMT>
__device__ __forceinline__ void stage_rows(const DevMatrix& W, int r0, int n, uint8_t* sq, uint8_t* ss, int part,
                                           int parts) {
    const int K = W.cols, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the LDS address goes to m0
    const int qbytes = n * staged_row_bytes(FMT, K), nq = (qbytes + 1023) / 1024;
    const uint8_t* qsrc = W.q + (int64_t)r0 * staged_row_bytes(FMT, K);
    const uint32_t lq = __builtin_amdgcn_readfirstlane(lds_addr(sq));
    for (int i = nq * part / parts + wave; i < nq * (part + 1) / parts; i += kWaves) {
        const int off = min(i * 1024 + 16 * lane, qbytes - 16);
        dma16(qsrc + off, lq + i * 1024);
    }
    if constexpr (FMT != DT_F16) {
        const int sbytes = n * (K / 32) * 2, ns = (sbytes + 255) / 256;
        const uint8_t* ssrc = (const uint8_t*)W.s + (int64_t)r0 * (K / 32) * 2;
        const uint32_t ls = __builtin_amdgcn_readfirstlane(lds_addr(ss));
        for (int i = ns * part / parts + wave; i < ns * (part + 1) / parts; i += kWaves) {
            const int off = min(i * 256 + 4 * lane, sbytes - 4);
            dma4(ssrc + off, ls + i * 256);
        }
    }
}
// The staged region of this workgroup's output rows and its row range.
struct Staged {
    uint8_t *sq, *ss;
    int r0, n;
};
__device__ __forceinline__ Staged staged_of(const DecodeParams& p) {
    Staged g;
    g.sq = (uint8_t*)dyn_lds + p.out_lds_off;
    g.ss = g.sq + staged_q_bytes(p.out.dtype, p.out.cols, p.out_lds_rows);
    g.r0 = min(p.out.rows, (int)blockIdx.x * p.rows_out);
    g.n = max(0, min(p.out.rows, g.r0 + p.out_lds_rows) - g.r0);
    return g;
}

// Rows [0, n) staged by stage_rows against xs (LDS), with the lanes-per-row
// mapping, chunk order and lane reduction of Rows::run (so each row's sum is
// the one the register path forms, bit for bit); epi(rbase + row, sum) runs on
// the row's first lane, rows ascending within a lane.
template <int FMT, int LPR, typename Epi>
__device__ __forceinline__ void run_staged(const uint8_t* sq, const uint8_t* ss, int K, int rbase, int n,
                                           const float* xs, Epi& epi) {
    constexpr int RPB = kWaves * (64 / LPR);
    const int lane = threadIdx.x & 63, li = lane % LPR;
    const int local = (threadIdx.x >> 6) * (64 / LPR) + lane / LPR;
    const int nch = gemv::chunks_of<FMT>(K), rb = staged_row_bytes(FMT, K), nb = K >> 5;
    const f16* sc = (const f16*)ss;
    for (int base = 0; base < n; base += RPB) {
        const int r = base + local;
        float v = 0.f;
        if (r < n) {
            for (int c = li; c < nch; c += LPR) {
                const int4 q = *(const int4*)(sq + r * rb + 16 * c);
                const float d = FMT == DT_Q8_0 ? (float)sc[r * nb + (c >> 1)] : FMT == DT_Q4_0 ? (float)sc[r * nb + c] : 1.f;
                v += gemv::chunk_dot<FMT>(q, d, c, xs);
            }
        }
        v = lane_sum<LPR>(v);
        if (r < n && li == 0) epi(rbase + r, v, 0.f);
    }
}

// P7: final RMSNorm, output rows (logits) and this workgroup's arg-max, which
// it publishes as two words (value, index bits).  The first out_lds_rows rows of
// the workgroup's share were staged in LDS by DMA during the last layers (a
// slice before each of their QKV waits); the rest stream through registers as
// in the other phases.
template <int FMT>
struct PhaseLogits {
    const u64* in;  // last layer's xf words
    u64* cand;      // [2 * gridDim.x]
    Ctl c;
    template <int LPR>
    __device__ bool go() {
        const DecodeParams& p = P();
        const Shared sh = lds_of();
        const DevMatrix W = p.out;
        int r0, r1;
        my_rows(p.rows_out, W.rows, r0, r1);
        const Staged g = staged_of(p);
        const int rs = r0 + g.n;  // rows [r0, rs) staged in LDS
        Rows<FMT, LPR, false> rw;
        rw.prefetch(W, W, rs, r1);
        NormGain gain;
        gain.load(p.out_norm, p.hidden);
        if (!wait_words(in, p.hidden, sh.xres, c)) return false;
        rmsnorm_lds(sh.xres, gain, p.hidden, p.eps, sh.xn, sh.red);
        float best = -INFINITY;
        int bi = INT_MAX;
        float* logits = p.logits;
        auto epi = [&](int r, float v, float) {
            if (logits) *gptr(logits + r) = v;
            if (v > best) {  // rows ascend within a lane, so ties keep the lower index; NaN never wins
                best = v;
                bi = r;
            }
        };
        if (rs > r0) {
            wait_stage_barrier<0>();  // every wave's DMA has landed
            run_staged<FMT, LPR>(g.sq, g.ss, W.cols, r0, g.n, sh.xn, epi);
        }
        rw.run(W, W, rs, r1, sh.xn, epi);
        wave_argmax(best, bi);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) {
            sh.scr[threadIdx.x >> 6] = best;
            ((int*)sh.scr)[8 + (threadIdx.x >> 6)] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float bv = sh.scr[0];
            int bx = ((int*)sh.scr)[8];
            for (int w = 1; w < kWaves; w++) {
                const float v2 = sh.scr[w];
                const int i2 = ((int*)sh.scr)[8 + w];
                if (v2 > bv || (v2 == bv && i2 < bx)) {
                    bv = v2;
                    bx = i2;
                }
            }
            put_word(cand + 2 * blockIdx.x, bv, c.tag);
            put_word(cand + 2 * blockIdx.x + 1, __int_as_float(bx), c.tag);
        }
        return true;
    }
};

template <int FMT>
__device__ __forceinline__ bool qkv_phase(const u64* xin, u64* out, int pos, int token, Ctl c) {
    PhaseQKV<FMT> ph{xin, out, pos, token, c};
    return with_lpr(P().rows_qkv, ph);
}
template <int FMT>
__device__ __forceinline__ bool residual_phase(int which, const u64* in, u64* out, Ctl c) {
    PhaseResidual<FMT> ph{which, in, out, c};
    return with_lpr(which ? P().rows_down : P().rows_wo, ph);
}
template <int FMT>
__device__ __forceinline__ bool gate_up_phase(const u64* in, u64* out, Ctl c) {
    PhaseGateUp<FMT> ph{in, out, c};
    return with_lpr(P().rows_ffn, ph);
}
template <int FMT>
__device__ __forceinline__ bool logits_phase(const u64* in, u64* cand, Ctl c) {
    PhaseLogits<FMT> ph{in, cand, c};
    return with_lpr(P().rows_out, ph);
}


// Copies `bytes` (a multiple of 4) from global memory into LDS, then syncs.
__device__ __forceinline__ void copy_to_lds(unsigned char* dst, const void* src, int bytes) {
    __syncthreads();
    for (int i = threadIdx.x; i < bytes / 4; i += kT) ((unsigned*)dst)[i] = *gptr((const unsigned*)src + i);
    __syncthreads();
}

template <int FMT, int HD, int GM>
__global__ __launch_bounds__(kT) void decode_step_kernel(DecodeParams kp) {
    for (int i = threadIdx.x; i < (int)(sizeof(DecodeParams) / 4); i += kT)
        ((unsigned*)lds_params)[i] = ((const unsigned*)&kp)[i];
    __syncthreads();
    const Shared sh = lds_of();
    float* red = sh.red;
    Ctl c;
    c.tag = *(volatile unsigned*)kp.epoch;
    c.abort_word = kp.abort_word;
    c.status = kp.status;
    c.timeout = kp.timeout_ticks;
    c.sub = kp.trace ? kp.trace + (int64_t)decode_trace_points(kp.n_layers) * gridDim.x : nullptr;
    const int pos = *(volatile int*)kp.pos;
    const int token = *(volatile int*)kp.chain;
    const int n_layers = kp.n_layers, layer_words = kp.layer_words;
    const int off_part = kp.off_part, off_ctx = kp.off_ctx, off_xa = kp.off_xa, off_ffn = kp.off_ffn,
              off_xf = kp.off_xf;

    // optional timeline: thread 0 stamps the wall clock when its workgroup ends a phase
    unsigned long long* trace = kp.trace;
    int point = 0;
    auto stamp = [&]() {
        if (trace && threadIdx.x == 0) *gptr(trace + (int64_t)point * gridDim.x + blockIdx.x) = wall_clock64();
        point++;
    };
    stamp();
    const u64* xprev = nullptr;
    for (int l = 0; l < n_layers; l++) {
        if (l == kp.abort_at_layer && blockIdx.x == 0) {
            // Failure-path tests only: the other workgroups then wait for rows this workgroup
            // never publishes and leave through the abort word.
            if (threadIdx.x == 0) raise_abort(c);
            return;
        }
        copy_to_lds(lds_layer, kp.layers + l, (int)sizeof(DecLayer));
        if (kp.out_lds_rows > 0) {
            // slice of the staged output rows (the logits phase reads them after a wait)
            const int parts = min(kStageLayers, n_layers), part = l - (n_layers - parts);
            if (part >= 0) {
                const Staged g = staged_of(P());
                if (g.n > 0) {
                    switch (kp.out.dtype) {
                    case DT_Q8_0: stage_rows<DT_Q8_0>(kp.out, g.r0, g.n, g.sq, g.ss, part, parts); break;
                    case DT_Q4_0: stage_rows<DT_Q4_0>(kp.out, g.r0, g.n, g.sq, g.ss, part, parts); break;
                    default: stage_rows<DT_F16>(kp.out, g.r0, g.n, g.sq, g.ss, part, parts); break;
                    }
                }
            }
        }
        u64* X = kp.xbuf + (int64_t)l * layer_words;
        if (!qkv_phase<FMT>(xprev, X, pos, token, c)) return;
        stamp();
        if (!attention_phase<HD, GM>(X, X + off_part, pos, c)) return;
        stamp();
        if (!merge_phase<HD>(X + off_part, X + off_ctx, pos, c)) return;
        stamp();
        if (!residual_phase<FMT>(0, X + off_ctx, X + off_xa, c)) return;
        stamp();
        if (!gate_up_phase<FMT>(X + off_xa, X + off_ffn, c)) return;
        stamp();
        if (!residual_phase<FMT>(1, X + off_ffn, X + off_xf, c)) return;
        stamp();
        xprev = X + off_xf;
    }
    u64* cand = kp.xbuf + kp.off_cand;
    bool ok;
    switch (kp.out.dtype) {
    case DT_Q8_0: ok = logits_phase<DT_Q8_0>(xprev, cand, c); break;
    case DT_Q4_0: ok = logits_phase<DT_Q4_0>(xprev, cand, c); break;
    default: ok = logits_phase<DT_F16>(xprev, cand, c); break;
    }
    if (!ok) return;
    stamp();
    if (blockIdx.x != 0) return;
    // P8: arg-max over the workgroups' candidates (Sampler.argmax, Sampler.swift:100-108:
    // lowest index on ties; NaN never wins; an all-NaN row yields token 0).
    const int nc = gridDim.x;
    if (!wait_words(cand, 2 * nc, sh.scr, c)) return;
    float best = -INFINITY;
    int bi = INT_MAX;
    for (int w = threadIdx.x; w < nc; w += kT) {
        const float v = sh.scr[2 * w];
        const int i = __float_as_int(sh.scr[2 * w + 1]);
        if (v > best || (v == best && i < bi)) {
            best = v;
            bi = i;
        }
    }
    wave_argmax(best, bi);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = best;
        ((int*)red)[8 + (threadIdx.x >> 6)] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = red[0];
        int bx = ((int*)red)[8];
        for (int w = 1; w < kWaves; w++)
            if (red[w] > bv || (red[w] == bv && ((int*)red)[8 + w] < bx)) {
                bv = red[w];
                bx = ((int*)red)[8 + w];
            }
        const int tok = bx == INT_MAX ? 0 : bx;
        *gptr(kp.chain) = tok;
        if (kp.emitted) *(volatile int32_t*)(kp.emitted + pos) = tok;
        *gptr(kp.pos) = pos + 1;
        *gptr(kp.epoch) = c.tag + 1;
        if (trace) *gptr(trace + (int64_t)point * gridDim.x) = wall_clock64();
    }
}

}  // namespace

// The kernel of this variant for group-size bucket gm.
const void* DECODE_ENTRY(int gm) {
    switch (gm) {
    case 1: return (const void*)decode_step_kernel<DECODE_FMT, DECODE_HD, 1>;
    case 2: return (const void*)decode_step_kernel<DECODE_FMT, DECODE_HD, 2>;
    case 4: return (const void*)decode_step_kernel<DECODE_FMT, DECODE_HD, 4>;
    default: return DECODE_HD == 64 ? (const void*)decode_step_kernel<DECODE_FMT, DECODE_HD, 8> : nullptr;
    }
}

#else  // host side

// Kernels of the (format, head dim) variants, one object each.
const void* decode_kernel_q8_hd64(int gm);
const void* decode_kernel_q8_hd128(int gm);
const void* decode_kernel_q4_hd64(int gm);
const void* decode_kernel_q4_hd128(int gm);
const void* decode_kernel_f16_hd64(int gm);
const void* decode_kernel_f16_hd128(int gm);

namespace {
const void* kernel_for(int fmt, int hd, int heads, int kv_heads) {
    const int gm = group_bucket(heads / kv_heads);
    if (hd == 64) {
        switch (fmt) {
        case DT_Q8_0: return decode_kernel_q8_hd64(gm);
        case DT_Q4_0: return decode_kernel_q4_hd64(gm);
        default: return decode_kernel_f16_hd64(gm);
        }
    }
    switch (fmt) {
    case DT_Q8_0: return decode_kernel_q8_hd128(gm);
    case DT_Q4_0: return decode_kernel_q4_hd128(gm);
    default: return decode_kernel_f16_hd128(gm);
    }
}
}  // namespace

bool decode_kernel_supported(int fmt, int hd, int heads, int kv_heads) {
    // query heads per KV head: up to 8 at head_dim 64, up to 4 at 128
    return (fmt == DT_Q8_0 || fmt == DT_Q4_0 || fmt == DT_F16) && (hd == 64 || hd == 128) && kv_heads > 0 &&
           heads % kv_heads == 0 && heads / kv_heads <= (hd == 64 ? 8 : 4);
}

int decode_attention_max_splits(int capacity, int kv_heads, int target_items) {
    int m = 1;
    for (int len = 1; len <= capacity; len++) {
        const int sl = split_len_for(len, kv_heads, target_items);
        const int s = (len + sl - 1) / sl;
        if (s > m) m = s;
    }
    return m;
}

size_t decode_lds_bytes(const DecodeParams& p, int grid) {
    const int G = p.heads / p.kv_heads, GM = group_bucket(G), HD = p.hd;
    size_t scr = 0;
    auto need = [&](size_t floats) { scr = floats > scr ? floats : scr; };
    need((size_t)p.rows_qkv);                                                    // QKV row buffer
    need((size_t)GM * HD + 2 * HD + GM * 8 + (size_t)kWaves * GM * HD + (size_t)kMaxSplitLen * HD / 2);  // attention
    need((size_t)p.max_splits * (HD + 2) + p.max_splits);                         // merge
    need(16);                                                                     // logits arg-max
    need((size_t)2 * grid);                                                       // candidates
    const size_t phases = ((size_t)kRedFloats + p.hidden + p.stage + scr) * sizeof(float);
    if (p.out_lds_rows <= 0) return phases;
    return (size_t)p.out_lds_off + staged_q_bytes(p.out.dtype, p.out.cols, p.out_lds_rows) +
           staged_s_bytes(p.out.dtype, p.out.cols, p.out_lds_rows);
}

size_t decode_logits_stage_offset(const DecodeParams& p, int grid) {
    DecodeParams q = p;
    q.out_lds_rows = 0;
    return (decode_lds_bytes(q, grid) + 15) & ~size_t(15);
}

int decode_logits_stage_rows(const DecodeParams& p, size_t lds_limit) {
    const int fmt = p.out.dtype, K = p.out.cols;
    const size_t base = (size_t)p.out_lds_off;
    int n = 0;
    while (n < p.rows_out &&
           base + staged_q_bytes(fmt, K, n + 1) + staged_s_bytes(fmt, K, n + 1) <= lds_limit)
        n++;
    return n;
}

size_t decode_static_lds(int fmt, int hd, int heads, int kv_heads) {
    const void* f = kernel_for(fmt, hd, heads, kv_heads);
    hipFuncAttributes a;
    if (!f || hipFuncGetAttributes(&a, f) != hipSuccess) {
        hipGetLastError();
        return 0;
    }
    return a.sharedSizeBytes;
}

hipError_t decode_kernel_occupancy(int fmt, int hd, int heads, int kv_heads, size_t lds, int* blocks_per_cu) {
    const void* f = kernel_for(fmt, hd, heads, kv_heads);
    if (!f) return hipErrorInvalidValue;
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, f, kT, lds);
}

hipError_t launch_decode_step(int fmt, const DecodeParams& p, int grid, size_t lds, int cooperative, hipStream_t st) {
    const void* f = kernel_for(fmt, p.hd, p.heads, p.kv_heads);
    if (!f) return hipErrorInvalidValue;
    DecodeParams a = p;
    void* args[] = {&a};
    if (cooperative) return hipLaunchCooperativeKernel(f, dim3(grid), dim3(kT), args, (unsigned)lds, st);
    return hipLaunchKernel(f, dim3(grid), dim3(kT), args, lds, st);
}

#endif  // DECODE_FMT
