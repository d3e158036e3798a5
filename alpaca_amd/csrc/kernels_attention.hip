// Causal grouped-query attention for gfx950.
//
// Semantics: CPUOps.attentionScores / softmax / attentionApply
// (CPUOps.swift:162-175, :222-274): query token t sits at absolute position
// start+t, sees cache rows 0..start+t, query head h reads KV head
// h / (heads/kv_heads), scores scaled by 1/sqrt(hd).  Cache layout here is
// [kv_heads][capacity][hd] (f16, or f32 in exact mode).
//
// flash_attn_kernel (prefill, f16 cache, hd 64/128): replaces the reference's
// tensor-op and simdgroup prefill attention (tensor_attention.metal,
// attention_prefill.metal).  A workgroup takes 64 queries of one head (16 per
// wave; at head dim 64 and on small grids two sets of four waves split the key
// range) and walks 64-key blocks that move global -> LDS by DMA, K one block
// ahead of V, both row-major; V^T fragments come from LDS transpose reads.
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16,
// so each lane owns one query column: the online-softmax max/sum need only
// two cross-lane shuffles, and the probabilities already sit in the B-operand
// layout of O^T += V^T P^T (the key order inside a 32-key MFMA step is
// permuted identically on both operands).  V enters MFMA as f16 (it is f16
// in the cache); Q and P enter either as one f16 term each, or (TT, the
// default prefill) as two, hi = f16(x) and lo = f16(x - hi), which carry them
// to ~2^-22 so that scores and P.V keep float32 accuracy at twice the MFMA
// work; P enters as P * 2^14, which keeps small probabilities (and the second
// term) out of the f16 subnormals.  Accumulation and the softmax statistics
// are float32.  Q's and P's term counts are chosen independently per launch
// (PT: two-term P), and the f16 output's second term is written only where the
// caller asks for it (the next GEMM takes two terms).
//
// attn_generic_kernel: one wave per (query, head, key split) with an online
// softmax in float32 over an f16 or f32 cache; splits are merged by
// attn_merge_kernel.  Used for decode (split-K over the context, as the
// reference's attn_decode_split + attn_decode_merge, attention_decode.metal)
// and for the exact / f32-KV / odd head-dim cases (attention.metal).
#include "common.h"

#include <algorithm>

#include <cstdlib>
#include <type_traits>

namespace {

struct FlashArgs {
    const f16* q;
    const f16* qlo;  // second term of q (TT)
    int ldq;
    const f16* kc;
    const f16* vc;
    int cap, T, H, KVH, start;
    float scale_log2;
    float* out32;
    f16* out16;
    f16* out16lo;  // second term of the f16 output (rows >= lo_out0), or null
    // two-term launches: query blocks holding a row >= lo_q0 take the second
    // terms of Q and P
    int lo_q0, lo_out0;
    // exact_last: the last query row (T - 1) is computed in float32 by the
    // first last_splits rows of workgroups (last_keys keys each; per head a
    // counter last_arrive, zero between launches, and last_splits x (hd + 2)
    // floats of last_part), q as its two f16 terms; the query blocks do not
    // write it
    int exact_last, last_splits, last_keys;
    unsigned* last_arrive;
    float* last_part;
};

constexpr int BQ = 64, BKV = 64;
constexpr int kFlashLastSplits = 64;  // key splits of the float32 last row (FlashArgs.exact_last)

// Chunk swizzle of the K and V blocks in LDS: 16-byte chunk c of key row r
// sits at slot c ^ kv_swz(r), kv_swz(r) = (r0^r3, r0^r2, r1) (bits of r).
// K fragment reads (one chunk from each of 16 consecutive rows): kv_swz takes
// 8 distinct values over any 8 consecutive rows and over the 8 even (and the 8
// odd) rows of 16, so 16 lanes x 16 bytes cover 64 banks once at head dim 64
// (rows of 128 bytes: even and odd rows fall in different bank halves).  V
// transpose reads (8 bytes from chunks 2d, 2d+1 of 4 consecutive rows): the
// two rows of one parity select different chunk pairs.  Found by exhaustive
// search over 3x4 XOR matrices against both bank models (64 banks / 16 lanes,
// 32 banks / 8 lanes); the former swizzle left the K reads 2-way conflicted and
// SQ_LDS_BANK_CONFLICT at half of SQ_LDS_IDX_ACTIVE.
__device__ __forceinline__ int kv_swz(int r) {
    return (((r ^ (r >> 3)) & 1) | (((r ^ (r >> 2)) & 1) << 1) | (((r >> 1) & 1) << 2));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i % 4) of the 4 halves addressed by lane 4j + i/4, for j = 0..3.  When
// lanes 4j..4j+3 address key row R_j at dims d0, d0+4, d0+8, d0+12, lane i
// gets V[R_0..R_3][d0 + i]: a V^T fragment read from row-major V.
__device__ __forceinline__ f16x4 lds_read_tr(const uint8_t* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(f16x4, v);
}

// Two floats -> an f16 pair, each rounded to nearest even (v_cvt_pk_f16_f32).
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){a, b}, f16x2v));
}
// e - (float)half, with the half read straight from the low (or high) 16 bits
// of a packed pair by the mixed-precision FMA (exact: the difference of a float
// and its own f16 rounding is representable).
__device__ __forceinline__ float minus_f16_lo(uint32_t pk, float e) {
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(pk), "v"(e));
    return d;
}
__device__ __forceinline__ float minus_f16_hi(uint32_t pk, float e) {
    float d;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(pk), "v"(e));
    return d;
}

// IEEE max of floats that are never signalling NaNs (plain v_max / v_max3).
__device__ __forceinline__ float vmax(float a, float b) {
    float d;
    asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// NSET wave-sets per workgroup.  With NSET = 2 or 4 (head dim 64) the sets of
// four waves take consecutive ranges of the key blocks of the same 64 queries,
// dividing the sequential walk of the longest (causal) query blocks by NSET;
// the ranges merge at the end.  It costs LDS (32 KB per set: two workgroups
// per CU with two sets, one with four), so the launcher uses it only when
// one-set workgroups would not fill the chip.
template <int HD, int NSET>
struct FlashLds {
    // with several sets the pipeline is two stages deep, with one three
    static constexpr int BYTES = NSET * (NSET > 1 ? 2 : 3) * 2 * (BKV * HD * 2);
};

template <int HD, int NSET, bool OUT16, bool TT, bool PT>
__device__ __forceinline__ void flash_attn_body(const FlashArgs& a, uint8_t* stage_lds) {
    static_assert(NSET == 1 || ((NSET == 2 || NSET == 4) && HD == 64), "several wave-sets fit LDS at head dim 64 only");
    constexpr int KS = HD / 32, DT = HD / 16;
    constexpr int ROWB = HD * 2;          // bytes per key row
    constexpr int CH = HD / 8;            // 16-byte chunks per row
    constexpr int RPI = 1024 / ROWB;      // key rows per DMA instruction
    constexpr int TILE = BKV * ROWB;      // bytes of one K (or V) block
    constexpr int PERW = TILE / 1024 / 4; // DMA instructions per wave per block and matrix
    constexpr int PER = 2 * PERW;
    // Stage buffers per set, each K block then V block, both row-major and
    // swizzled.  With several sets the pipeline is two stages deep (32 KB per
    // set); with one set, three (48 KB, three workgroups per CU).
    constexpr int NSTAGE = NSET > 1 ? 2 : 3;
    static_assert(FlashLds<HD, NSET>::BYTES == NSET * NSTAGE * 2 * TILE, "stage buffer size");

    const int h = blockIdx.x;
    const int qb = gridDim.y - 1 - blockIdx.y;  // longest (latest) query blocks first (after the exact_last rows)
    const int kvh = h / (a.H / a.KVH);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int set = wave / 4, wl = wave % 4;  // wave-set, and the wave's 16 queries within the block
    const int g = lane >> 4, c16 = lane & 15;
    const int qi = qb * BQ + wl * 16 + c16;
    const int qc = qi < a.T ? qi : a.T - 1;
    const int pos_q = a.start + qc;
    // Positions of this wave's first and last query (clamped like qc).
    const int wpos_lo = a.start + min(qb * BQ + wl * 16, a.T - 1);
    const int wpos_hi = a.start + min(qb * BQ + wl * 16 + 15, a.T - 1);
    uint8_t* const st0 = stage_lds + (set * NSTAGE) * 2 * TILE;  // this set's K buffers, then its V buffers

    // P enters the MFMA scaled by 2^14 (P <= 1 becomes <= 2^14): over long key
    // ranges most probabilities lie below f16's smallest normal (2^-14) and
    // would otherwise lose relative precision, as would the second term of the
    // two-term form; the output's normalisation undoes the scale.
    constexpr float kLog2PScale = 14.f;
    f16x8 qf[KS], ql[TT ? KS : 1];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int64_t qo = (int64_t)qc * a.ldq + h * HD + 32 * ks + 8 * g;
        qf[ks] = *(const f16x8*)(a.q + qo);
        if constexpr (TT) ql[ks] = *(const f16x8*)(a.qlo + qo);
    }

    const int last_q = (qb + 1) * BQ < a.T ? (qb + 1) * BQ : a.T;
    const int kend = a.start + last_q;  // keys [0, kend) cover every query of this block
    const int nkb = (kend + BKV - 1) / BKV;
    // Key blocks of this set: [first, first + count); both sets run `steps` steps.
    const int steps = (nkb + NSET - 1) / NSET;
    const int first = set * steps, count = max(0, min(nkb - first, steps));
    const f16* kbase = a.kc + (int64_t)kvh * a.cap * HD;
    const f16* vbase = a.vc + (int64_t)kvh * a.cap * HD;

    // K (or V) rows of this set's j-th key block into a stage buffer at LDS
    // address dst.  Past the set's last block (or for a set with none) the load
    // repeats a valid block that is never used, so every step waits on the
    // same count; rows past kend repeat row kend-1 (in bounds; masked or unused).
    // The block's first row is a wave-uniform base (SGPRs); each lane's byte
    // offset within the block (its row and swizzled chunk) is fixed, so only a
    // block that reaches past kend needs per-lane clamping.
    uint32_t lane_off[PERW];
#pragma unroll
    for (int jj = 0; jj < PERW; jj++) {
        const int r = (jj * 4 + wl) * RPI + lane / CH;
        lane_off[jj] = r * ROWB + ((lane % CH) ^ kv_swz(r)) * 16;
    }
    auto issue = [&](const f16* base, uint32_t dst, int j) {
        const int key0 = min(first + min(j, max(count, 1) - 1), nkb - 1) * BKV;
        const f16* src = base + (int64_t)key0 * HD;
        const int lim = kend - 1 - key0;  // last row of the block that exists
        if (lim >= BKV - 1) {
#pragma unroll
            for (int jj = 0; jj < PERW; jj++) dma16s(src, lane_off[jj], dst + (jj * 4 + wl) * RPI * ROWB);
        } else {
#pragma unroll
            for (int jj = 0; jj < PERW; jj++) {
                const int r0 = (jj * 4 + wl) * RPI, r = r0 + lane / CH, c = (lane % CH) ^ kv_swz(r);
                dma16s(src, min(r, lim) * ROWB + c * 16, dst + r0 * ROWB);
            }
        }
    };
    // Block j of the set is this wave's when it exists and some key of it lies
    // at or before the wave's last query (a prefix of the set's blocks).
    auto mine = [&](int j) { return j < count && (first + j) * BKV <= wpos_hi; };

    float m = -INFINITY;
    // O^T accumulators, and lacc: the row sums of P (every element of lacc is
    // the sum for the lane's query), from an MFMA with an all-ones A operand
    // on the same f16 terms of P that O^T takes.
    f32x4 oacc[DT], lacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < DT; d++) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f16x8 ones = {(f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f};

    // S^T tiles of one key block: sacc[t][r] = score(key0 + 16t + 4g + r, query qi)
    auto qk = [&](const uint8_t* Kt, f32x4* sacc) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            sacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int r = 16 * t + c16;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const f16x8 kf = *(const f16x8*)(Kt + r * ROWB + (((4 * ks + g) ^ kv_swz(r)) * 16));
                sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], sacc[t], 0, 0, 0);
                if constexpr (TT) sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], sacc[t], 0, 0, 0);
            }
        }
    };
    // Masking only where some key of the block lies past some query of the wave.
    auto mask = [&](f32x4* sacc, int kb) {
        const int key0 = kb * BKV;
        if (key0 + BKV - 1 > wpos_lo) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (key0 + 16 * t + 4 * g + r > pos_q) sacc[t][r] = -INFINITY;
        }
    };
    // Online softmax of one block's (masked) scores, then O^T += V^T P^T.
    // V^T fragment (dims 16d.., keys of 32-key step s) from row-major V in LDS.
    auto v_frag = [&](const uint8_t* Vt, int s, int d) {
        const int ra = 32 * s + 4 * g + (c16 >> 2), rb = ra + 16;
        const int cb = 2 * d + ((c16 & 3) >> 1), hb = (c16 & 1) * 8;
        const f16x4 lo = lds_read_tr(Vt + ra * ROWB + ((cb ^ kv_swz(ra)) * 16) + hb);
        const f16x4 hi = lds_read_tr(Vt + rb * ROWB + ((cb ^ kv_swz(rb)) * 16) + hb);
        return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // With one set (three waves per SIMD, registers to spare) the block's V^T
    // fragments are read before the softmax, so their LDS latency overlaps it.
    constexpr bool kEarlyV = NSET == 1 && HD == 64;
    // The exponentials are pinned ahead of the rescale branch (below) with two
    // sets (C1's attention per layer 41.4-41.8 -> 40.7-41.1 us), not with one,
    // three waves per SIMD (C5's 104.0 -> 105.9 us).
    constexpr bool kPinExp = NSET == 2;
    auto softmax_pv = [&](const f32x4* sacc, const uint8_t* Vt) {
        f16x8 vpre[kEarlyV ? 2 : 1][kEarlyV ? DT : 1];
        if constexpr (kEarlyV) {
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int d = 0; d < DT; d++) vpre[s][d] = v_frag(Vt, s, d);
        }
        // Running max in log2 units (m, mn): the scale is positive, so the max
        // of the raw scores scales to the max of the scaled ones.
        // (v_max3 without the compiler's signalling-NaN quieting of every
        // operand: MFMA results and -inf are never signalling NaNs)
        const float m0 = vmax3(sacc[0][0], sacc[0][1], sacc[0][2]), m1 = vmax3(sacc[0][3], sacc[1][0], sacc[1][1]);
        const float m2 = vmax3(sacc[1][2], sacc[1][3], sacc[2][0]), m3 = vmax3(sacc[2][1], sacc[2][2], sacc[2][3]);
        const float m4 = vmax3(sacc[3][0], sacc[3][1], sacc[3][2]);
        float mx = vmax(vmax3(m0, m1, sacc[3][3]), vmax3(m2, m3, m4));
        mx = xor32_combine(xor16_combine(mx, vmax), vmax);  // the 4 lanes of this query
        const float mn = fmaxf(m, mx * a.scale_log2);
        // -inf while every key seen so far is masked (possible past the first
        // set); referencing 0 then keeps alpha and P at exactly 0.
        const float mref = mn == -INFINITY ? 0.f : mn;
        // v_exp_f32 without the library's denormal-result path: values below
        // 2^-126 become 0, as they do anyway once P is rounded to f16.
        const float alpha = __builtin_amdgcn_exp2f(m - mref);
        // P * 2^14 straight from the exponent (the scale is exact); the row sums
        // take the same terms, so they carry the scale too and the final
        // normalisation cancels it.  P enters the MFMA as f16 (hi, and lo with
        // two terms).
        const float eref = kLog2PScale - mref;
        // f16 pairs (keys r = 0,1 and 2,3 of tile t): hi = RNE(P), lo = RNE(P - hi)
        uint32_t ph[4][2], pl[PT ? 4 : 1][2];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                const float e0 = __builtin_amdgcn_exp2f(fmaf(sacc[t][2 * pr], a.scale_log2, eref));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(sacc[t][2 * pr + 1], a.scale_log2, eref));
                const uint32_t h = pack_f16x2(e0, e1);
                ph[t][pr] = h;
                if constexpr (PT) pl[t][pr] = pack_f16x2(minus_f16_lo(h, e0), minus_f16_hi(h, e1));
            }
        // The exponentials are computed here, ahead of the rescale branch,
        // where they can issue among the next block's score MFMAs (left to
        // itself the compiler sinks them past the branch, to their use).
        if constexpr (kPinExp) {
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int pr = 0; pr < 2; pr++) asm volatile("" : "+v"(ph[t][pr]));
        }
        // alpha is exactly 1 in every lane whose running max did not move (the
        // usual case past the first blocks): the wave then skips the rescale.
        if (__builtin_amdgcn_ballot_w64(m != mn)) {
#pragma unroll
            for (int d = 0; d < DT; d++) oacc[d] *= alpha;
            lacc *= alpha;
        }
        // O^T += V^T P^T.  Key order inside a 32-key step, identical on both
        // operands: slot e < 4 is key 32s + 4g + e, slot e >= 4 is 32s + 16 + 4g + e - 4.
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const f16x8 pf = __builtin_bit_cast(f16x8, make_uint4(ph[2 * s][0], ph[2 * s][1], ph[2 * s + 1][0],
                                                                  ph[2 * s + 1][1]));
            f16x8 plf;
            if constexpr (PT)
                plf = __builtin_bit_cast(f16x8, make_uint4(pl[2 * s][0], pl[2 * s][1], pl[2 * s + 1][0],
                                                           pl[2 * s + 1][1]));
            lacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf, lacc, 0, 0, 0);
            if constexpr (PT) lacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, plf, lacc, 0, 0, 0);
#pragma unroll
            for (int d = 0; d < DT; d++) {
                f16x8 vf;
                if constexpr (kEarlyV) vf = vpre[s][d];
                else vf = v_frag(Vt, s, d);
                oacc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, oacc[d], 0, 0, 0);
                if constexpr (PT) oacc[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, plf, oacc[d], 0, 0, 0);
            }
        }
        m = mn;
    };

    // Pipeline, K one block ahead of V: step i multiplies the scores of block
    // i+1 (K) while it runs the softmax and P.V of block i, so a wave's MFMAs
    // and its softmax VALU work are independent within a step.  NSTAGE buffers
    // each for K and V; before step i the loads of K(i+1) and V(i) have been
    // issued NSTAGE-2 steps earlier.  Step i: wait for them, barrier (every
    // wave is done with K(i) and V(i-1)), refill those two buffers with
    // K(i+NSTAGE) and V(i+NSTAGE-1), compute.
    uint8_t* const kbuf = st0;
    uint8_t* const vbuf = st0 + NSTAGE * TILE;
    issue(kbase, lds_addr(kbuf), 0);
#pragma unroll
    for (int j = 0; j + 1 < NSTAGE; j++) {
        issue(kbase, lds_addr(kbuf + (j + 1) * TILE), j + 1);
        issue(vbase, lds_addr(vbuf + j * TILE), j);
    }
    wait_stage_barrier<(NSTAGE - 1) * PER>();  // K(0)
    // Scores of the current and the next block alternate between sa and sb
    // (the loop is unrolled over both parities, so no copies).
    f32x4 sa[4], sb[4];
    qk(kbuf, sa);
    if (mine(0)) mask(sa, first);
    auto step = [&](auto uc, int i, f32x4* scur, f32x4* snext) {
        constexpr int R = decltype(uc)::value % NSTAGE;  // i % NSTAGE
        wait_stage_barrier<(NSTAGE - 2) * PER>();
        issue(kbase, lds_addr(kbuf + R * TILE), i + NSTAGE);
        issue(vbase, lds_addr(vbuf + ((R + NSTAGE - 1) % NSTAGE) * TILE), i + NSTAGE - 1);
        if (mine(i)) {
            qk(kbuf + ((R + 1) % NSTAGE) * TILE, snext);
            softmax_pv(scur, vbuf + R * TILE);
            if (mine(i + 1)) mask(snext, first + i + 1);
        }
    };
    using std::integral_constant;
    for (int i = 0; i < steps; i += 2 * NSTAGE) {
        step(integral_constant<int, 0>(), i, sa, sb);
        if (i + 1 >= steps) break;
        step(integral_constant<int, 1>(), i + 1, sb, sa);
        if (i + 2 >= steps) break;
        step(integral_constant<int, 2>(), i + 2, sa, sb);
        if (i + 3 >= steps) break;
        step(integral_constant<int, 3>(), i + 3, sb, sa);
        if constexpr (NSTAGE > 2) {
            if (i + 4 >= steps) break;
            step(integral_constant<int, 4>(), i + 4, sa, sb);
            if (i + 5 >= steps) break;
            step(integral_constant<int, 5>(), i + 5, sb, sa);
        }
    }
    wait_stage_barrier<0>();  // no DMA may still be writing LDS past this point

    float lsum = lacc[0];
    if constexpr (NSET > 1) {
        // Every other set hands (m, lsum, O) to the first through LDS (its own
        // stage buffers, idle now: its DMA has landed); the first merges the
        // sets in order and writes the output.
        static_assert(4 * DT * 4 * 64 * 4 <= 2 * TILE && 4 * 2 * 64 * 4 <= 2 * TILE, "merge scratch");
        auto xo_of = [&](int s) { return (float*)(stage_lds + (s * NSTAGE) * 2 * TILE) + wl * DT * 4 * 64; };
        auto xml_of = [&](int s) { return (float*)(stage_lds + (s * NSTAGE + 1) * 2 * TILE) + wl * 2 * 64; };
        if (set) {
            float* xo = xo_of(set);  // O: 4 KB per wave
            float* xml = xml_of(set);  // m, lsum
#pragma unroll
            for (int d = 0; d < DT; d++)
#pragma unroll
                for (int r = 0; r < 4; r++) xo[(d * 4 + r) * 64 + lane] = oacc[d][r];
            xml[lane] = m;
            xml[64 + lane] = lsum;
        }
        __syncthreads();
        if (set) return;
        float ms[NSET];
        ms[0] = m;
        float mt = m;  // finite: the first set saw key 0
#pragma unroll
        for (int s = 1; s < NSET; s++) {
            ms[s] = xml_of(s)[lane];
            mt = fmaxf(mt, ms[s]);
        }
        const float a0 = __builtin_amdgcn_exp2f(m - mt);
        lsum *= a0;
#pragma unroll
        for (int d = 0; d < DT; d++) oacc[d] *= a0;
#pragma unroll
        for (int s = 1; s < NSET; s++) {
            const float as = __builtin_amdgcn_exp2f(ms[s] - mt);
            const float* xo = xo_of(s);
            lsum = fmaf(xml_of(s)[64 + lane], as, lsum);
#pragma unroll
            for (int d = 0; d < DT; d++)
#pragma unroll
                for (int r = 0; r < 4; r++) oacc[d][r] = fmaf(xo[(d * 4 + r) * 64 + lane], as, oacc[d][r]);
        }
    }
    if (qi >= a.T - a.exact_last) return;
    const float inv = 1.0f / lsum;  // lsum and O both carry the 2^14
    // oacc[d][r] = O(query qi, dim 16d + 4g + r)
#pragma unroll
    for (int d = 0; d < DT; d++) {
        const int64_t o = ((int64_t)qi * a.H + h) * HD + 16 * d + 4 * g;
        if (OUT16) {
            const float o0 = oacc[d][0] * inv, o1 = oacc[d][1] * inv, o2 = oacc[d][2] * inv, o3 = oacc[d][3] * inv;
            const f16x4 v = {(f16)o0, (f16)o1, (f16)o2, (f16)o3};
            *(f16x4*)(a.out16 + o) = v;
            if (a.out16lo && qi >= a.lo_out0)
                *(f16x4*)(a.out16lo + o) = f16x4{(f16)(o0 - (float)v[0]), (f16)(o1 - (float)v[1]),
                                                 (f16)(o2 - (float)v[2]), (f16)(o3 - (float)v[3])};
        } else {
            *(float4*)(a.out32 + o) = make_float4(oacc[d][0] * inv, oacc[d][1] * inv, oacc[d][2] * inv,
                                                  oacc[d][3] * inv);
        }
    }
}

// The last query row (T - 1, the row whose logits a prefill returns) of head
// blockIdx.x in float32, split over the keys: workgroup blockIdx.y takes keys
// [y * last_keys, (y + 1) * last_keys) in chunks of NT / KT keys (KT threads
// per key, 64 dims each), q = hi + lo (its two f16 terms), scores, running max
// and P.V (HD / 8 threads per V row) in float32; each chunk's K and V rows are
// loaded together (V does not wait for the scores).  The split's (max, sum,
// output) go out as agent-scope stores (written through to the device's point
// of coherence) and the last split workgroup of the head to arrive (a counter
// per head, which it returns to zero) merges them with agent-scope loads and
// writes the row as the kernel writes every row.  These workgroups come first
// in dispatch order and walk at most two chunks each, so they end long before
// the kernel's critical path, the longest query block (whose second terms of
// Q and P this replaces: C1's attention per layer 48.9 -> 40.1-41.0 us).
template <int HD, int NT, bool OUT16>
__device__ __forceinline__ void flash_last_row(const FlashArgs& a, uint8_t* lds) {
    constexpr int KT = HD / 64, CK = NT / KT;  // threads per key, keys per chunk
    constexpr int TPR = HD / 8, RPP = NT / TPR, VR = CK / RPP;  // P.V: threads per row, rows per pass, passes
    constexpr int WV = NT / 64;
    static_assert(VR * RPP == CK && KT * 64 == HD, "shape");
    float* qs = (float*)lds;  // HD, scaled by scale_log2
    float* ps = qs + HD;      // CK probabilities of the chunk
    float* red = ps + CK;     // 2 * WV
    float* ws = red + 2 * WV; // WV x HD partial outputs
    const int h = blockIdx.x, sp = blockIdx.y, S = a.last_splits;
    const int kvh = h / (a.H / a.KVH), tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = a.T - 1, kend = a.start + a.T;  // keys [0, kend)
    const int k0 = sp * a.last_keys, k1 = min(k0 + a.last_keys, kend);  // k0 < kend (the launcher's split count)
    const f16* kbase = a.kc + (int64_t)kvh * a.cap * HD;
    const f16* vbase = a.vc + (int64_t)kvh * a.cap * HD;
    if (tid < HD) {
        const int64_t o = (int64_t)row * a.ldq + h * HD + tid;
        const float v = a.qlo ? (float)a.q[o] + (float)a.qlo[o] : (float)a.q[o];
        qs[tid] = v * a.scale_log2;
    }
    __syncthreads();
    const int kl = tid / KT, kp = tid % KT;   // the thread's key in the chunk, its 64-dim part
    const int tr = tid % TPR, rq = tid / TPR;  // P.V: dims 8 tr .. 8 tr + 7 of rows rq + i RPP
    float m = -INFINITY, l = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c0 = k0; c0 < k1; c0 += CK) {
        // q is read from LDS at every use (not held in 64 registers across chunks)
        asm volatile("" ::: "memory");
        // K and V rows past k1 are clamped to row k1 - 1 (loaded, unused)
        int4 kr[8], vr[VR];
        const f16* krow = kbase + (int64_t)min(c0 + kl, k1 - 1) * HD + kp * 64;
#pragma unroll
        for (int j = 0; j < 8; j++) kr[j] = *(const int4*)(krow + 8 * j);
#pragma unroll
        for (int i = 0; i < VR; i++) vr[i] = *(const int4*)(vbase + (int64_t)min(c0 + rq + i * RPP, k1 - 1) * HD + tr * 8);
        float sc = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f16* kv = (const f16*)&kr[j];
#pragma unroll
            for (int e = 0; e < 8; e++) sc = fmaf(qs[kp * 64 + 8 * j + e], (float)kv[e], sc);
        }
        if constexpr (KT == 2) sc += __shfl_xor(sc, 1, 64);
        if (c0 + kl >= k1) sc = -INFINITY;
        const float wm = wave_max(sc);
        if (lane == 0) red[wave] = wm;
        __syncthreads();
        float mc = red[0];
#pragma unroll
        for (int w = 1; w < WV; w++) mc = fmaxf(mc, red[w]);
        const float mn = fmaxf(m, mc);  // finite: the chunk holds key c0 < k1
        const float alpha = exp2f(m - mn);
        const float pk = exp2f(sc - mn);
        if (kp == 0) ps[kl] = pk;
        const float wsum = wave_sum(kp == 0 ? pk : 0.f);
        if (lane == 0) red[WV + wave] = wsum;
        __syncthreads();
        float lc = 0.f;
#pragma unroll
        for (int w = 0; w < WV; w++) lc += red[WV + w];
        l = l * alpha + lc;
        m = mn;
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] *= alpha;
#pragma unroll
        for (int i = 0; i < VR; i++) {
            const float p = ps[rq + i * RPP];  // 0 past k1
            const f16* v = (const f16*)&vr[i];
#pragma unroll
            for (int j = 0; j < 8; j++) acc[j] = fmaf(p, (float)v[j], acc[j]);
        }
        __syncthreads();  // ps and red are rewritten by the next chunk
    }
    // sum the rows of a wave (lanes with one tr), then the waves
#pragma unroll
    for (int o = TPR; o < 64; o <<= 1)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] += __shfl_xor(acc[j], o, 64);
    if (lane < TPR)
#pragma unroll
        for (int j = 0; j < 8; j++) ws[wave * HD + tr * 8 + j] = acc[j];
    __syncthreads();
    float* pp = a.last_part + ((int64_t)h * S + sp) * (HD + 2);
    if (tid < HD) {
        float o = ws[tid];
#pragma unroll
        for (int w = 1; w < WV; w++) o += ws[w * HD + tid];
        __hip_atomic_store(pp + 2 + tid, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (tid == 0) {
            __hip_atomic_store(pp, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // Each thread waits for its stores to be acknowledged before the barrier,
    // so the arrival counted after it follows them.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned* last_s = (unsigned*)(ws + WV * HD);
    if (tid == 0)
        *last_s = __hip_atomic_fetch_add(a.last_arrive + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (unsigned)(S - 1);
    __syncthreads();
    if (!*last_s) return;
    if (tid == 0) __hip_atomic_store(a.last_arrive + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the merge: the first wave takes the splits' maxima and sums (S <= 64),
    // then thread groups of HD take every G-th split's outputs, added through LDS
    auto ld = [](const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    const float* hp = a.last_part + (int64_t)h * S * (HD + 2);
    float* wts = ps;  // S weights
    float* part = ws; // NT partial sums
    if (tid < 64) {
        const int j = min(tid, S - 1);
        const float mj = ld(hp + j * (HD + 2)), lj = ld(hp + j * (HD + 2) + 1);
        const float mt = wave_max(tid < S ? mj : -INFINITY);
        const float w = tid < S ? exp2f(mj - mt) : 0.f;
        wts[tid] = w;
        const float lt = wave_sum(w * lj);
        if (tid == 0) red[0] = lt;
    }
    __syncthreads();
    constexpr int G = NT / HD;
    {
        const int d = tid % HD, grp = tid / HD;
        float o = 0.f;
        for (int j = grp; j < S; j += G) o = fmaf(ld(hp + j * (HD + 2) + 2 + d), wts[j], o);
        part[tid] = o;
    }
    __syncthreads();
    if (tid < HD) {
        float o = part[tid];
#pragma unroll
        for (int g = 1; g < G; g++) o += part[g * HD + tid];
        o /= red[0];
        const int64_t oi = ((int64_t)row * a.H + h) * HD + tid;
        if constexpr (OUT16) {
            const f16 hi = (f16)o;
            a.out16[oi] = hi;
            if (a.out16lo && row >= a.lo_out0) a.out16lo[oi] = (f16)(o - (float)hi);
        } else {
            a.out32[oi] = o;
        }
    }
}

// Query blocks holding a row at or past a.lo_q0 take Q and P as TT / PT
// terms; the others (of a two-term launch) as one f16 term each.  With
// a.exact_last the first row of workgroups computes the last query row
// (flash_last_row) and the query blocks follow.
template <int HD, int NSET, bool OUT16, bool TT, bool PT>
__global__ __launch_bounds__(256 * NSET) void flash_attn_kernel(FlashArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t stage_lds[FlashLds<HD, NSET>::BYTES];
    if constexpr (!TT && !PT && NSET == 2) {
        if (a.exact_last && (int)blockIdx.y < a.last_splits) {
            flash_last_row<HD, 256 * NSET, OUT16>(a, stage_lds);
            return;
        }
    }
    if constexpr (TT || PT) {
        const int qb = gridDim.y - 1 - blockIdx.y;
        if ((qb + 1) * BQ > a.lo_q0) flash_attn_body<HD, NSET, OUT16, TT, PT>(a, stage_lds);
        else flash_attn_body<HD, NSET, OUT16, false, false>(a, stage_lds);
    } else {
        flash_attn_body<HD, NSET, OUT16, false, false>(a, stage_lds);
    }
}

// ------------------------------------------------------------------ generic
constexpr int kMaxHD = 256;
constexpr int kSplitMin = 64;

template <typename KV>
__global__ __launch_bounds__(64) void attn_generic_kernel(const float* q, int ldq, const KV* kc, const KV* vc,
                                                          int cap, int H, int KVH, int hd, int start,
                                                          int split_len, int splits, float* partials, float* out,
                                                          float scale) {
    __shared__ float qs[kMaxHD];
    const int sp = blockIdx.x, h = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
    const int kvh = h / (H / KVH);
    const int len = start + t + 1;
    const int p0 = sp * split_len;
    const int p1 = (p0 + split_len < len) ? p0 + split_len : len;
    for (int d = lane; d < hd; d += 64) qs[d] = q[(int64_t)t * ldq + h * hd + d];
    __syncthreads();

    const KV* kb = kc + (int64_t)kvh * cap * hd;
    const KV* vb = vc + (int64_t)kvh * cap * hd;
    float m = -INFINITY, l = 0.f;
    float o[kMaxHD / 64] = {0.f, 0.f, 0.f, 0.f};
    for (int c = p0; c < p1; c += 64) {
        const int p = c + lane;
        const bool valid = p < p1;
        float s = -INFINITY;
        if (valid) {
            const KV* kr = kb + (int64_t)p * hd;
            float acc = 0.f;
            for (int d = 0; d < hd; d++) acc += qs[d] * (float)kr[d];
            s = acc * scale;
        }
        const float mn = fmaxf(m, wave_max(s));  // lane 0 is always valid
        const float alpha = expf(m - mn);
        const float e = valid ? expf(s - mn) : 0.f;
        l = l * alpha + wave_sum(e);
#pragma unroll
        for (int i = 0; i < kMaxHD / 64; i++) o[i] *= alpha;
        const int nv = p1 - c < 64 ? p1 - c : 64;
        for (int j = 0; j < nv; j++) {
            const float ej = __shfl(e, j, 64);
            const KV* vr = vb + (int64_t)(c + j) * hd;
#pragma unroll
            for (int i = 0; i < kMaxHD / 64; i++) {
                const int d = lane + 64 * i;
                if (d < hd) o[i] += ej * (float)vr[d];
            }
        }
        m = mn;
    }
    if (splits == 1) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int i = 0; i < kMaxHD / 64; i++) {
            const int d = lane + 64 * i;
            if (d < hd) out[((int64_t)t * H + h) * hd + d] = o[i] * inv;
        }
    } else {
        float* pp = partials + (((int64_t)t * H + h) * splits + sp) * (hd + 2);
        if (lane == 0) { pp[0] = m; pp[1] = l; }
#pragma unroll
        for (int i = 0; i < kMaxHD / 64; i++) {
            const int d = lane + 64 * i;
            if (d < hd) pp[2 + d] = o[i];
        }
    }
}

// Merges per-split (max, sum, unnormalised output) triples (at most 64
// splits): the first wave takes one split per lane for the weights
// exp(m_s - M) and the weighted sum of the row sums, so the splits' statistics
// load in parallel; then each thread sums its output element over the splits
// with the weights from LDS, several splits' loads in flight at a time.
__global__ void attn_merge_kernel(const float* partials, int H, int hd, int splits, float* out) {
    __shared__ float wsh[64];
    __shared__ float lsh;
    const int th = blockIdx.x;  // t * H + h
    const float* pp = partials + (int64_t)th * splits * (hd + 2);
    if (threadIdx.x < 64) {
        const int s = threadIdx.x;
        const float ms = s < splits ? pp[s * (hd + 2)] : -INFINITY;
        const float ls = s < splits ? pp[s * (hd + 2) + 1] : 0.f;
        const float mx = wave_max(ms);
        const float w = ms == -INFINITY ? 0.f : expf(ms - mx);
        wsh[s] = w;
        const float l = wave_sum(ls * w);
        if (s == 0) lsh = l;
    }
    __syncthreads();
    const float l = lsh;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
#pragma unroll 8
        for (int s = 0; s < splits; s++) acc += pp[s * (hd + 2) + 2 + d] * wsh[s];
        out[(int64_t)th * hd + d] = acc / l;
    }
}

// The same merge for up to kMergePer splits per thread: a workgroup of 256
// threads per query head, thread t taking dim t % hd of the splits s = t / hd
// (mod 256 / hd).  Every load (the splits' max and sum, the thread's outputs)
// goes out before the first wait, so the merge costs one round trip to the
// partials rather than one per batch of splits; the groups' sums are added
// through LDS.
constexpr int kMergePer = 16;
__global__ __launch_bounds__(256) void attn_merge_wide_kernel(const float* partials, int hd, int splits, float* out) {
    __shared__ float wsh[64];
    __shared__ float part[256];
    __shared__ float lsh;
    const int th = blockIdx.x;
    const float* pp = partials + (int64_t)th * splits * (hd + 2);
    const int groups = 256 / hd, t = threadIdx.x, d = t % hd, grp = min(t / hd, groups - 1);
    // unconditional loads (indices clamped, surplus values unused)
    const int sm = min(t, splits - 1);
    const float m_raw = pp[sm * (hd + 2)], l_raw = pp[sm * (hd + 2) + 1];
    float o[kMergePer];
#pragma unroll
    for (int i = 0; i < kMergePer; i++) o[i] = pp[min(grp + i * groups, splits - 1) * (hd + 2) + 2 + d];
    if (t < 64) {
        const float ms = t < splits ? m_raw : -INFINITY;
        const float ls = t < splits ? l_raw : 0.f;
        const float mx = wave_max(ms);
        const float w = ms == -INFINITY ? 0.f : expf(ms - mx);
        wsh[t] = w;
        const float l = wave_sum(ls * w);
        if (t == 0) lsh = l;
    }
    __syncthreads();
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kMergePer; i++) {
        const int s = grp + i * groups;
        if (s < splits) acc += o[i] * wsh[s];
    }
    if (t < groups * hd) part[t] = acc;
    __syncthreads();
    if (t < hd) {
        float sum = 0.f;
        for (int g = 0; g < groups; g++) sum += part[g * hd + t];
        out[(int64_t)th * hd + t] = sum / lsh;
    }
}

// ------------------------------------------------------------------ decode split-K
// One workgroup per (KV head, split of the context) serves all G query heads
// of that KV head, so every cached K/V row is read once per token.  Scores:
// one thread per position (a 16-byte-vectorised K row each); probabilities go
// to LDS; P.V: hd/8 threads per V row with 16-byte loads, partial sums
// reduced across rows with shuffles and LDS.  With an f16 cache the thread's
// K row and its first V rows are loaded before anything else (after its q
// values, which are needed first), so the workgroup waits for HBM once rather
// than for K and then for V.  Writes the split's (max, sum, unnormalised
// output) per query head; the Wo projection merges the splits
// (attention_decode.metal:27-133 does split + merge kernels).
constexpr int kDecThreads = 256;
constexpr int kMaxSplitLen = 256;     // positions per workgroup of kDecThreads threads
constexpr int kMaxSplitLenWide = 512;  // with 512-thread workgroups (groups of at most 2 query heads)
constexpr int kMaxGroup = 16;

// NT threads, one position each: split_len <= NT.
template <int HD, int GM, typename KV, int NT = kDecThreads>
__global__ __launch_bounds__(NT) void attn_decode_split_kernel(const float* q, const KV* kc, const KV* vc,
                                                                        int cap, int H, int KVH, int length,
                                                                        const int* pos_dev, int split_len,
                                                                        float scale_log2, float* partials) {
    constexpr int VEC = 16 / sizeof(KV);    // elements per 16-byte load
    constexpr int TPR = HD / 8;             // threads per V row (8 dims each)
    constexpr int WV = NT / 64;             // waves
    constexpr int RPP = NT / TPR;           // V rows in flight per pass
    constexpr bool PRE = sizeof(KV) == 2;   // f16 cache: K row and first V rows loaded up front
    constexpr int KCH = HD / VEC;           // 16-byte chunks per K row
    constexpr int VPF = PRE ? (NT / RPP < 8 ? NT / RPP : 8) : 1;  // V rows per thread up front
    constexpr int QPT = (GM * HD + NT - 1) / NT;                  // q values per thread
    __shared__ float qs[GM][HD];
    __shared__ float es[GM][NT];
    __shared__ float red[GM][2 * WV];
    __shared__ float ws[WV][GM][HD];
    const int G = H / KVH;
    const int sp = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    if (pos_dev) length = *pos_dev + 1;
    const int p0 = sp * split_len;
    const int p1 = min(p0 + split_len, length);
    const int n = p1 - p0;
    const int tr = tid % TPR, rowq = tid / TPR;
    float qv[QPT];
#pragma unroll
    for (int j = 0; j < QPT; j++) {  // (clamped index: an unconditional load)
        const int i = min(tid + j * NT, G * HD - 1);
        qv[j] = q[(kvh * G + i / HD) * HD + i % HD];
    }
    // the q loads stay ahead of the K/V loads: waiting for them then leaves the
    // K/V loads in flight (loads retire in issue order)
    asm volatile("" ::: "memory");
    int4 kraw[PRE ? KCH : 1];
    int4 vpre[VPF];
    // f16 cache: KCH lanes share a K row (lane kj takes its 16-byte chunk kj), so a
    // load instruction reads 64 / KCH whole rows; the lane's KCH loads cover rows
    // kr0 + i * (NT / KCH)
    constexpr int KRP = NT / KCH;  // K rows per load instruction
    const int kj = tid % KCH, kr0 = tid / KCH;
    if constexpr (PRE) {
        // rows past the split's end are clamped to its last row (to its first
        // when it is empty, p0 < cap), so every load goes out unconditionally and
        // the compiler's wait counts stay exact; their values are unused
        const int last = max(n - 1, 0);
#pragma unroll
        for (int i = 0; i < KCH; i++) {
            const int r = min(kr0 + i * KRP, last);
            kraw[i] = *(const int4*)(kc + ((int64_t)kvh * cap + p0 + r) * HD + kj * VEC);
        }
#pragma unroll
        for (int k = 0; k < VPF; k++) {
            const int r = min(rowq + k * RPP, last);
            vpre[k] = *(const int4*)(vc + ((int64_t)kvh * cap + p0 + r) * HD + tr * 8);
        }
    }
#pragma unroll
    for (int j = 0; j < QPT; j++) {
        const int i = tid + j * NT;
        if (i < G * HD) qs[i / HD][i % HD] = qv[j] * scale_log2;
    }
    __syncthreads();

    // scores in base-2 exponent units; thread `tid` ends with the scores of
    // position `pr` (a permutation of 0..255)
    float sc[GM];
    int pr = tid;
    if constexpr (PRE) {
        // Each lane's partial dot products over its 8 dims for its KCH rows are
        // summed over the KCH lanes of the row group by a reduce-scatter: at
        // every step a lane keeps half of its rows and adds the partner's sums
        // for them, so lane kj ends with row i = kj complete.
        pr = kr0 + kj * KRP;
#pragma unroll
        for (int g = 0; g < GM; g++) {
            float part[KCH];
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const KV* kv = (const KV*)&kraw[i];
                float a = 0.f;
#pragma unroll
                for (int e = 0; e < VEC; e++) a += qs[g < G ? g : 0][kj * VEC + e] * (float)kv[e];
                part[i] = a;
            }
#pragma unroll
            for (int h = KCH / 2; h >= 1; h >>= 1) {
                const bool hi = kj & h;
#pragma unroll
                for (int i = 0; i < h; i++) {
                    const float keep = hi ? part[i + h] : part[i], give = hi ? part[i] : part[i + h];
                    part[i] = keep + __shfl_xor(give, h, 64);
                }
            }
            sc[g] = (pr < n && g < G) ? part[0] : -INFINITY;
        }
    } else {
#pragma unroll
        for (int g = 0; g < GM; g++) sc[g] = (tid < n && g < G) ? 0.f : -INFINITY;
        if (tid < n) {
            const KV* kr = kc + ((int64_t)kvh * cap + p0 + tid) * HD;
#pragma unroll
            for (int c = 0; c < HD / VEC; c++) {
                const int4 raw = *(const int4*)(kr + c * VEC);
                const KV* kv = (const KV*)&raw;
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const float kf = (float)kv[j];
#pragma unroll
                    for (int g = 0; g < GM; g++)
                        if (g < G) sc[g] += qs[g][c * VEC + j] * kf;
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < GM; g++) {
        const float m = wave_max(sc[g]);
        if (lane == 0) red[g][wave] = m;
    }
    __syncthreads();
    float mloc[GM];
#pragma unroll
    for (int g = 0; g < GM; g++) {
        mloc[g] = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
#pragma unroll
        for (int w = 4; w < WV; w++) mloc[g] = fmaxf(mloc[g], red[g][w]);
    }
#pragma unroll
    for (int g = 0; g < GM; g++) {
        const float e = (pr < n && g < G) ? exp2f(sc[g] - mloc[g]) : 0.f;
        es[g][pr] = e;
        const float sum = wave_sum(e);
        if (lane == 0) red[g][WV + wave] = sum;
    }
    __syncthreads();

    // P.V: TPR threads per V row, RPP rows per pass
    float acc[GM][8];
#pragma unroll
    for (int g = 0; g < GM; g++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[g][j] = 0.f;
    auto add_row = [&](int r, const float* vf) {
#pragma unroll
        for (int g = 0; g < GM; g++) {
            const float e = es[g][r];
#pragma unroll
            for (int j = 0; j < 8; j++) acc[g][j] += e * vf[j];
        }
    };
    int r0 = rowq;
    if constexpr (PRE) {
#pragma unroll
        for (int k = 0; k < VPF; k++) {
            const int r = rowq + k * RPP;
            if (r < n) {
                const KV* v = (const KV*)&vpre[k];
                float vf[8];
#pragma unroll
                for (int j = 0; j < 8; j++) vf[j] = (float)v[j];
                add_row(r, vf);
            }
        }
        r0 = rowq + VPF * RPP;
    }
    for (int r = r0; r < n; r += RPP) {
        const KV* vr = vc + ((int64_t)kvh * cap + p0 + r) * HD + tr * 8;
        float vf[8];
        if constexpr (sizeof(KV) == 2) {
            const int4 raw = *(const int4*)vr;
            const KV* v = (const KV*)&raw;
#pragma unroll
            for (int j = 0; j < 8; j++) vf[j] = (float)v[j];
        } else {
            const int4 r0v = *(const int4*)vr, r1v = *(const int4*)(vr + 4);
            const float* a = (const float*)&r0v;
            const float* b = (const float*)&r1v;
#pragma unroll
            for (int j = 0; j < 4; j++) { vf[j] = a[j]; vf[4 + j] = b[j]; }
        }
        add_row(r, vf);
    }
    // reduce the rows held by one wave (lane bits >= log2(TPR)), then the 4 waves
#pragma unroll
    for (int o = TPR; o < 64; o <<= 1)
#pragma unroll
        for (int g = 0; g < GM; g++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[g][j] += __shfl_xor(acc[g][j], o, 64);
    if (lane < TPR)
#pragma unroll
        for (int g = 0; g < GM; g++)
#pragma unroll
            for (int j = 0; j < 8; j++) ws[wave][g][tr * 8 + j] = acc[g][j];
    __syncthreads();
    for (int i = tid; i < G * HD; i += NT) {
        const int g = i / HD, d = i % HD;
        float* pp = partials + ((int64_t)(kvh * G + g) * gridDim.x + sp) * (HD + 2);
        float o = ws[0][g][d];
#pragma unroll
        for (int w = 1; w < WV; w++) o += ws[w][g][d];
        pp[2 + d] = o;
        if (d == 0) {
            // the running max is kept in base-2 units; partials carry natural-log units
            float l = red[g][WV];
#pragma unroll
            for (int w = 1; w < WV; w++) l += red[g][WV + w];
            pp[0] = n > 0 ? mloc[g] * 0.69314718055994531f : -INFINITY;
            pp[1] = l;
        }
    }
}

template <int HD, typename KV>
hipError_t decode_dispatch(int G, dim3 grid, hipStream_t st, const float* q, const void* kc, const void* vc, int cap,
                           int H, int KVH, int length, const int* pos_dev, int split_len, float sl2, float* partials) {
    const KV* k = (const KV*)kc;
    const KV* v = (const KV*)vc;
    if (split_len > kMaxSplitLen) {  // (the launcher allows this for groups of at most 2 heads only)
        if (G <= 1) attn_decode_split_kernel<HD, 1, KV, 512><<<grid, 512, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
        else attn_decode_split_kernel<HD, 2, KV, 512><<<grid, 512, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
        return hipGetLastError();
    }
    if (G <= 1) attn_decode_split_kernel<HD, 1, KV><<<grid, kDecThreads, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
    else if (G <= 2) attn_decode_split_kernel<HD, 2, KV><<<grid, kDecThreads, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
    else if (G <= 4) attn_decode_split_kernel<HD, 4, KV><<<grid, kDecThreads, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
    else if (G <= 8) attn_decode_split_kernel<HD, 8, KV><<<grid, kDecThreads, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
    else attn_decode_split_kernel<HD, 16, KV><<<grid, kDecThreads, 0, st>>>(q, k, v, cap, H, KVH, length, pos_dev, split_len, sl2, partials);
    return hipGetLastError();
}

}  // namespace

// Wave-sets per workgroup at head dim 64 (ALPACA_HIP_FLASH_SETS = 1 or 2,
// read per launch, forces a count).  One-set workgroups (48 KB of LDS) run
// three per CU, two-set ones two: below four query blocks per CU the causal
// critical path dominates and two sets win (attention per layer, one set ->
// two: 360M shape at 3,584 and 4,096 rows, 840 and 960 workgroups, 56.8 ->
// 49.8 and 66.4 -> 60.0 us; 1.7B shape at 1,536 rows, 768 workgroups, 29.0 ->
// 27.7; 1,024 workgroups 38.2 either way; 1,280 and 1,536 workgroups 2-3%
// slower).  Four sets (one 1024-thread workgroup per CU) were slower at every
// measured shape: the kernel is bound by the SIMDs' issue, not by the
// longest query block's walk.
static int flash_sets(dim3 grid) {
    const char* e = std::getenv("ALPACA_HIP_FLASH_SETS");
    const int forced = e ? std::atoi(e) : 0;
    if (forced == 1 || forced == 2) return forced;
    return (int64_t)grid.x * grid.y < 4 * 256 ? 2 : 1;
}

template <int NSET, bool TT, bool PT>
void flash_launch64(const FlashArgs& a, dim3 grid, bool out16, hipStream_t st) {
    if (out16) flash_attn_kernel<64, NSET, true, TT, PT><<<grid, 256 * NSET, 0, st>>>(a);
    else flash_attn_kernel<64, NSET, false, TT, PT><<<grid, 256 * NSET, 0, st>>>(a);
}

template <bool TT, bool PT>
hipError_t flash_dispatch(const FlashArgs& a, dim3 grid, int hd, bool out16, hipStream_t st) {
    if (hd == 64) {
        switch (flash_sets(grid)) {
        case 2: flash_launch64<2, TT, PT>(a, grid, out16, st); break;
        default: flash_launch64<1, TT, PT>(a, grid, out16, st); break;
        }
    } else if (hd == 128) {
        if (out16) flash_attn_kernel<128, 1, true, TT, PT><<<grid, 256, 0, st>>>(a);
        else flash_attn_kernel<128, 1, false, TT, PT><<<grid, 256, 0, st>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_flash_attention(const f16* q, const f16* qlo, int ldq, const f16* kc, const f16* vc, int capacity,
                                  int tokens, int heads, int kv_heads, int hd, int start, float* out_f32, f16* out_f16,
                                  f16* out_f16_lo, hipStream_t st, int p_terms, int lo_q0, int lo_out0,
                                  unsigned* last_arrive, float* last_part) {
    if (tokens <= 0) return hipSuccess;
    FlashArgs a;
    a.q = q;
    a.qlo = qlo;
    a.ldq = ldq;
    a.kc = kc;
    a.vc = vc;
    a.cap = capacity;
    a.T = tokens;
    a.H = heads;
    a.KVH = kv_heads;
    a.start = start;
    a.scale_log2 = 1.4426950408889634f / sqrtf((float)hd);
    a.out32 = out_f32;
    a.out16 = out_f16;
    a.out16lo = out_f16_lo;
    a.lo_q0 = lo_q0;
    a.lo_out0 = lo_out0;
    // The float32 last row pays where the query blocks run as two wave-sets
    // (small grids: the two-term last block is then the kernel's critical path);
    // on larger grids (one set) the last block's second terms cost less than the
    // extra workgroups, and the launch takes lo_q0 as given.
    const dim3 qgrid(heads, (tokens + BQ - 1) / BQ);
    a.exact_last = last_arrive && last_part && hd == 64 && flash_sets(qgrid) == 2 ? 1 : 0;
    a.last_arrive = last_arrive;
    a.last_part = last_part;
    a.last_splits = 0;
    a.last_keys = 0;
    if (a.exact_last) {
        // two chunks of 512 keys per split workgroup, at most kFlashLastSplits splits
        const int ck = 512, kend = start + tokens;
        a.last_splits = std::min(kFlashLastSplits, (kend + 2 * ck - 1) / (2 * ck));
        a.last_keys = (kend + a.last_splits - 1) / a.last_splits;
        a.last_splits = (kend + a.last_keys - 1) / a.last_keys;  // every split holds a key
    }
    dim3 grid(heads, (tokens + BQ - 1) / BQ + a.last_splits);
    if (a.exact_last) {
        // (two sets, as for the query grid alone)
        flash_launch64<2, false, false>(a, grid, out_f16, st);
        return hipGetLastError();
    }
    const bool pt = p_terms ? p_terms == 2 : qlo != nullptr;
    if (!qlo) return pt ? flash_dispatch<false, true>(a, grid, hd, out_f16, st)
                        : flash_dispatch<false, false>(a, grid, hd, out_f16, st);
    return pt ? flash_dispatch<true, true>(a, grid, hd, out_f16, st) : flash_dispatch<true, false>(a, grid, hd, out_f16, st);
}

size_t flash_last_part_floats(int heads, int hd) { return (size_t)heads * kFlashLastSplits * (hd + 2); }

// Splits for the generic kernel: decode spreads the context over >= 64-key
// splits (up to 64 of them); batched queries already fill the chip.
hipError_t launch_attention_decode(const float* q, const void* kc, const void* vc, int kv_f16, int capacity,
                                   int heads, int kv_heads, int hd, int length, const int* pos_dev, int split_len,
                                   int splits, float* partials, hipStream_t st) {
    const int G = heads / kv_heads;
    if (split_len < 1 || split_len > (G <= 2 ? kMaxSplitLenWide : kMaxSplitLen) || G > kMaxGroup || heads % kv_heads ||
        (hd != 64 && hd != 128))
        return hipErrorInvalidValue;
    const float sl2 = 1.4426950408889634f / sqrtf((float)hd);
    dim3 grid(splits, kv_heads);
    if (hd == 64)
        return kv_f16 ? decode_dispatch<64, f16>(G, grid, st, q, kc, vc, capacity, heads, kv_heads, length, pos_dev, split_len, sl2, partials)
                      : decode_dispatch<64, float>(G, grid, st, q, kc, vc, capacity, heads, kv_heads, length, pos_dev, split_len, sl2, partials);
    return kv_f16 ? decode_dispatch<128, f16>(G, grid, st, q, kc, vc, capacity, heads, kv_heads, length, pos_dev, split_len, sl2, partials)
                  : decode_dispatch<128, float>(G, grid, st, q, kc, vc, capacity, heads, kv_heads, length, pos_dev, split_len, sl2, partials);
}

hipError_t launch_attention_merge(const float* partials, int heads, int hd, int splits, float* out, hipStream_t st) {
    if (splits < 1 || splits > 64) return hipErrorInvalidValue;  // one split per lane of a wave
    if (hd <= 256 && splits <= (256 / hd) * kMergePer) {
        attn_merge_wide_kernel<<<heads, 256, 0, st>>>(partials, hd, splits, out);
        return hipGetLastError();
    }
    int bt = hd < 64 ? 64 : (hd > 256 ? 256 : (hd + 63) / 64 * 64);
    attn_merge_kernel<<<heads, bt, 0, st>>>(partials, heads, hd, splits, out);
    return hipGetLastError();
}

// A session's split length: 64 to 256 positions (512 for groups of at most
// two query heads), a multiple of 32, aiming at no more than two workgroups
// per CU over all KV heads at full capacity, and at most 64 splits (0: none
// fits).  More workgroups than that put a third on some CUs, which then set
// the kernel's time: 128-position splits gave the 1.7B shape (32 KV heads,
// 4,176 positions) 1,056 workgroups and 256-position splits 544; 288-position
// splits give 480.
int attention_decode_session_split_len(int capacity, int heads, int kv_heads) {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        cus[dev] = n;
    }
    const int most = kv_heads > 0 && heads / kv_heads <= 2 ? kMaxSplitLenWide : kMaxSplitLen;
    const int64_t target = 2 * (int64_t)cus[dev];
    int l = (int)(((int64_t)capacity * kv_heads + target - 1) / target);
    const int fewest = (capacity + 63) / 64;  // at most 64 splits
    l = std::max(std::max(l, fewest), 64);
    l = (l + 31) / 32 * 32;
    if (l <= most) return l;
    return fewest <= most ? most : 0;
}

bool attention_decode_supported(int heads, int kv_heads, int hd) {
    return (hd == 64 || hd == 128) && heads % kv_heads == 0 && heads / kv_heads <= kMaxGroup;
}

int attention_splits(int length, int heads, int tokens) {
    (void)heads;
    if (tokens > 1) return 1;
    int s = (length + kSplitMin - 1) / kSplitMin;
    return s < 1 ? 1 : (s > 64 ? 64 : s);
}

size_t attention_partial_floats(int heads, int tokens, int splits, int hd) {
    return (size_t)tokens * heads * splits * (hd + 2);
}

hipError_t launch_attention_generic(const float* q, int ldq, const void* kc, const void* vc, int kv_f16,
                                    int capacity, int tokens, int heads, int kv_heads, int hd, int start,
                                    int splits, float* partials, float* out, hipStream_t st) {
    if (tokens <= 0) return hipSuccess;
    if (hd > kMaxHD || splits < 1 || splits > 64) return hipErrorInvalidValue;
    const int max_len = start + tokens;
    int split_len = (max_len + splits - 1) / splits;
    split_len = (split_len + 63) / 64 * 64;
    const float scale = 1.0f / sqrtf((float)hd);
    dim3 grid(splits, heads, tokens);
    if (kv_f16)
        attn_generic_kernel<f16><<<grid, 64, 0, st>>>(q, ldq, (const f16*)kc, (const f16*)vc, capacity, heads,
                                                      kv_heads, hd, start, split_len, splits, partials, out, scale);
    else
        attn_generic_kernel<float><<<grid, 64, 0, st>>>(q, ldq, (const float*)kc, (const float*)vc, capacity,
                                                        heads, kv_heads, hd, start, split_len, splits, partials,
                                                        out, scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    int bt = hd < 64 ? 64 : (hd > 256 ? 256 : (hd + 63) / 64 * 64);
    attn_merge_kernel<<<tokens * heads, bt, 0, st>>>(partials, heads, hd, splits, out);
    return hipGetLastError();
}
