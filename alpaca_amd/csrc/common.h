// Shared device helpers and launch declarations for the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Address-space casts: pointers read from structs are generic to the
// compiler, which then emits flat instructions (counted against both the
// vector-memory and the LDS wait counters).  Loads through gptr() are
// global_load instructions.
#define AS_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const AS_GLOBAL T* gptr(const T* p) {
    return (const AS_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ AS_GLOBAL T* gptr(T* p) {
    return (AS_GLOBAL T*)p;
}
// 16- and 8-byte global loads into HIP's vector classes (through the native
// vector types, which address-space-qualified loads accept).
__device__ __forceinline__ int4 gload_i4(const void* p) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    const v4i v = *(const AS_GLOBAL v4i*)p;
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float2 gload_f2(const void* p) {
    typedef float v2f __attribute__((ext_vector_type(2)));
    const v2f v = *(const AS_GLOBAL v2f*)p;
    return make_float2(v.x, v.y);
}

enum { DT_F32 = 0, DT_F16 = 1, DT_Q8_0 = 2, DT_Q4_0 = 3 };

// A weight matrix [rows, cols] resident in HBM.  Quantised formats are split
// into a quant stream and a scale stream so every row starts 16-byte aligned:
//   Q8_0: q = int8 [rows][cols],             s = f16 [rows][cols/32]
//   Q4_0: q = uint8 [rows][cols/32][16]      s = f16 [rows][cols/32]
//         (byte j of a block: low nibble = element j, high = element j+16)
//   F16:  q = f16 [rows][cols],              s = null
// ------------------------------------------------------------------ LDS DMA
// global -> LDS DMA of 16 (or 4) bytes per lane: lane l writes LDS bytes
// [lds + size*l, lds + size*(l+1)).  Issued through asm so that the only waits on
// these loads are the explicit ones in wait_stage_barrier (the compiler's own
// tracking of LDS DMA falls back to waiting for every outstanding load before
// each LDS read, which would serialise the pipeline).  The asm sets m0, which
// nothing else in these kernels uses; one wait state separates the m0 write from
// the load that reads it (the compiler puts the same s_nop after its own m0
// writes for LDS DMA).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte
// offset: one VGPR per load instead of a 64-bit address pair.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// Wait until at most N of this wave's global loads are outstanding, and for
// its LDS reads, then barrier.  The "memory" clobber keeps LDS accesses on
// their side of the barrier.
template <int N>
__device__ __forceinline__ void wait_stage_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

struct DevMatrix {
    int dtype = DT_F16;
    int rows = 0, cols = 0;
    const uint8_t* q = nullptr;
    const f16* s = nullptr;
    // Quantised matrices with cols % 64 == 0 also hold their scales stage-major
    // for the prefill GEMM: s2[kt * stage_scale_pitch(rows) + n] packs the two
    // f16 scales of row n for K columns [64 kt, 64 kt + 64).
    const uint32_t* s2 = nullptr;
};
__host__ __device__ inline int stage_scale_pitch(int rows) { return (rows + 63) & ~63; }
// u32 elements of the s2 buffer, including 128 elements of slack that a tile
// hanging over the last rows of the last stage may read.
inline int64_t stage_scale_elems(int rows, int cols) { return (int64_t)(cols / 64) * stage_scale_pitch(rows) + 128; }
hipError_t launch_stage_scales(const f16* s, uint32_t* s2, int rows, int cols, hipStream_t st);
// Whether an M x N two-term prefill GEMM runs the wide (128x256) tiles.
bool prefill_split_pays(int m, int n);

// Cross-lane moves.  DPP controls (gfx9) act inside 16-lane rows without the
// LDS crossbar: quad_perm [1,0,3,2] = 0xB1 and [2,3,0,1] = 0x4E swap lanes
// xor 1 and xor 2; row_half_mirror (0x141) pairs the two quads of each
// 8-lane half, row_mirror (0x140) the two halves of a row; row_ror:8 (0x128)
// is xor 8.  Xor 16 is a ds_swizzle in bit-mask mode (and 0x1F, xor 0x10)
// and xor 32 a ds_bpermute.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swizzle_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
// Butterflies across 16-lane rows without the LDS crossbar (gfx950):
// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even
// rows of b, so with a = b = v the two results hold {v[l], v[l ^ 16]};
// v_permlane32_swap likewise {v[l], v[l ^ 32]}.  The two results are copied
// out as integers before reinterpretation (a bit cast of an element of the
// returned vector reads element 0).  op must be commutative.
template <typename Op>
__device__ __forceinline__ float xor16_combine(float v, Op op) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const unsigned a = p[0], b = p[1];
    return op(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
template <typename Op>
__device__ __forceinline__ float xor32_combine(float v, Op op) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const unsigned a = p[0], b = p[1];
    return op(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
// Reduction over aligned groups of N lanes (N a power of two up to 64); every
// lane of a group gets the result.  All lanes combine in the same tree, so the
// result is identical across the group.
template <int N, typename Op>
__device__ __forceinline__ float lane_reduce(float v, Op op) {
    if (N >= 2) v = op(v, dpp_mov<0xB1>(v));
    if (N >= 4) v = op(v, dpp_mov<0x4E>(v));
    if (N >= 8) v = op(v, dpp_mov<0x141>(v));
    if (N >= 16) v = op(v, dpp_mov<0x140>(v));
    if (N >= 32) v = xor16_combine(v, op);
    if (N >= 64) v = xor32_combine(v, op);
    return v;
}
// The value of lane l ^ 16 (XOR = 16) or l ^ 32 (XOR = 32), from one permlane
// swap: even rows find the partner in the second result, odd rows in the first.
template <int XOR>
__device__ __forceinline__ unsigned xor_partner(unsigned u) {
    static_assert(XOR == 16 || XOR == 32, "permlane swap partners");
    const int lane = __lane_id();
    if constexpr (XOR == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        const unsigned a = p[0], b = p[1];
        return (lane & 16) ? a : b;
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        const unsigned a = p[0], b = p[1];
        return (lane & 32) ? a : b;
    }
}
__device__ __forceinline__ float xor_partner16(float v) { return __builtin_bit_cast(float, xor_partner<16>(__builtin_bit_cast(unsigned, v))); }
__device__ __forceinline__ float xor_partner32(float v) { return __builtin_bit_cast(float, xor_partner<32>(__builtin_bit_cast(unsigned, v))); }
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
// Wave-wide arg-max over (value, index): the larger value wins, ties go to the
// lower index.  The combine is symmetric, so every lane ends with the result.
__device__ __forceinline__ void wave_argmax(float& best, int& bi) {
    auto take = [&](float v2, int i2) {
        if (v2 > best || (v2 == best && i2 < bi)) {
            best = v2;
            bi = i2;
        }
    };
    take(dpp_mov<0xB1>(best), dpp_mov_i<0xB1>(bi));
    take(dpp_mov<0x4E>(best), dpp_mov_i<0x4E>(bi));
    take(dpp_mov<0x141>(best), dpp_mov_i<0x141>(bi));
    take(dpp_mov<0x140>(best), dpp_mov_i<0x140>(bi));
    take(xor_partner16(best), (int)xor_partner<16>((unsigned)bi));
    take(xor_partner32(best), (int)xor_partner<32>((unsigned)bi));
}
struct AddOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
template <int N>
__device__ __forceinline__ float lane_sum(float v) { return lane_reduce<N>(v, AddOp()); }
__device__ __forceinline__ float wave_sum(float v) { return lane_reduce<64>(v, AddOp()); }
__device__ __forceinline__ float wave_max(float v) { return lane_reduce<64>(v, MaxOp()); }

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
// f16 outputs with a second-term pointer (lo) write hi = f16(v) and, when lo is
// set, lo = f16(v - hi): the two-term activations of the MFMA prefill.
hipError_t launch_f32_to_f16(const float* x, f16* out, f16* out_lo, int64_t n, hipStream_t st);
// With out_f16_lo, the second term is written for rows >= lo_row0.
hipError_t launch_rmsnorm(const float* x, const float* w, float* out_f32, f16* out_f16, f16* out_f16_lo, int rows,
                          int dim, float eps, hipStream_t st, int lo_row0 = 0);
hipError_t launch_embed(const int32_t* tokens, int count, const DevMatrix& table, float* out, hipStream_t st);
hipError_t launch_dequant(const DevMatrix& m, float* out, hipStream_t st);
// f16 copy of a matrix (the prefill weight cache): f16(d*q) per weight, cols % 8 == 0.
hipError_t launch_dequant_f16(const DevMatrix& m, f16* out, hipStream_t st);
// Greedy arg-max.  Writes the token to *chain_token and emitted[slot] (slot =
// *pos_dev when pos_dev is set, which is then advanced by one).
// Sampler.sample for a draw u (kernels_sample.hip): one workgroup; out[0] the
// token, out[1] 1 when the logits hold a NaN; cand_idx / cand_p scratch of n.
hipError_t launch_sample(const float* logits, int n, float temperature, int top_k, float top_p, double u,
                         int32_t* out, int* status, uint32_t* cand_idx, double* cand_p, hipStream_t st);
hipError_t launch_argmax(const float* logits, int n, int32_t* chain_token, int32_t* emitted, int slot,
                         int* pos_dev, hipStream_t st);
// RoPE with a host-built (cos, sin) table [positions][hd/2]; q rotated in
// place (q_f32) and/or written as f16 (q_f16); k rotated and v copied into the
// caches at rows start..start+tokens-1.  k/v may be null (q-only RoPE).
hipError_t launch_rope_store(float* qkv, int ld, int tokens, int heads, int kv_heads, int hd, int start,
                             const float2* table, int interleaved, int write_q_f32, f16* q_f16, f16* q_f16_lo,
                             void* kcache, void* vcache, int kv_f16, int capacity, hipStream_t st);

// decode GEMV (kernels_gemv.hip)
enum { GEMV_STORE = 0, GEMV_ADD = 1, GEMV_SWIGLU = 2, GEMV_QKV_ROPE = 3 };
// Input row: x, RMS-normalised x (norm != null), or the merge of split-K
// decode-attention partials [heads][splits][hd+2] (partials != null; with
// pos_dev set, only the splits covering positions 0..*pos_dev are read).
struct GemvInput {
    const float* x = nullptr;
    // or the row as two f16 terms (x = xh + xl): the last row of a prefill GEMM
    const f16* xh = nullptr;
    const f16* xl = nullptr;
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
// The last row of a prefill GEMM in float32 from its two f16 terms (x = xh +
// xl): GEMV_ADD adds W x to out (the residual row); GEMV_SWIGLU writes
// silu(Wg x) * (Wu x) as two f16 terms (outh, outl), the down projection's
// input row.
hipError_t launch_gemv_pair(const DevMatrix& w, const DevMatrix* w_up, const f16* xh, const f16* xl, float* out,
                            f16* outh, f16* outl, int mode, hipStream_t st);
// Whether w's decode products take the streamed GEMV (large matrices).
bool gemv_streams(const DevMatrix& w);

// prefill GEMM (kernels_gemm.hip)
enum { GEMM_STORE = 0, GEMM_ACC = 1, GEMM_SWIGLU = 2, GEMM_QKV_ROPE = 3 };
// fast: x f16 [m][k] (row stride ldx); MFMA f16 with f32 accumulate.  With
// xlo (the activations' second term, same layout) the tiles holding a row at
// or past lo_row0 take the activations as x + xlo (two-term: float32-grade
// inputs at twice the MFMA work), the others x alone; xlo must hold valid
// second terms for those tiles' rows (a tile's first row is a multiple of its
// height, at most 256, so rows from (lo_row0 / 256) * 256 on suffice).
//   STORE/ACC write y f32 (row stride ldy); SWIGLU writes yh f16 (row stride
//   ldy), and when yhlo is set its second term for rows >= lo_out_row0.
hipError_t launch_gemm_mfma(const f16* x, const f16* xlo, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up,
                            float* y, f16* yh, f16* yhlo, int ldy, int mode, hipStream_t st, int lo_row0 = 0,
                            int lo_out_row0 = 0);
// The stacked [q|k|v] projection of m tokens at positions pos.. with the RoPE
// (interleaved pairs) and KV-cache append in its epilogue: q rotated to qh f16
// [m][heads*hd], k rotated and v copied to the f16 caches [kv_heads][capacity][hd].
// Bit for bit the result of GEMM_STORE followed by launch_rope_store.
// hipErrorNotSupported when the pipelined GEMM cannot take the shapes.
struct QkvRope {
    const float2* rope = nullptr;  // (cos, sin) [positions][hd/2]
    f16* qh = nullptr;
    f16* qlo = nullptr;  // q's second term, written for rows >= lo_out_row0
    f16* kc = nullptr;
    f16* vc = nullptr;
    int heads = 0, kv_heads = 0, hd = 0, pos = 0, capacity = 0;
};
// With xlo, the tiles holding a row >= lo_row0 or a column >= lo_col0 take
// the second term (tiles are 16-column aligned: lo_col0 = heads * hd leaves q
// one-term before lo_row0 and k, v two-term throughout).
hipError_t launch_gemm_qkv_rope(const f16* x, const f16* xlo, int ldx, int m, const DevMatrix& w, const QkvRope& o,
                                hipStream_t st, int lo_row0 = 0, int lo_out_row0 = 0, int lo_col0 = 1 << 30);
// exact: x f32; float32 FMA in the reference's per-block order.  SWIGLU writes y f32.
hipError_t launch_gemm_f32(const float* x, int ldx, int m, const DevMatrix& w, const DevMatrix* w_up, float* y,
                           int ldy, int mode, hipStream_t st);

// persistent single-token decode (kernels_decode.hip)
//
// One launch computes one token: every decoder layer, the logits
// and the greedy arg-max.  Phases hand data to each other through exchange
// words (8 bytes: f32 value in the low half, the launch's tag in the high
// half) written and polled with agent-scope atomics; see kernels_decode.hip.
struct DecLayer {
    DevMatrix qkv, wo, gate, up, down;
    const float* attn_norm = nullptr;
    const float* ffn_norm = nullptr;
    void* kc = nullptr;  // f16 [kv_heads][capacity][head_dim]
    void* vc = nullptr;
};
struct DecodeParams {
    const DecLayer* layers = nullptr;  // device array [n_layers]
    int n_layers = 0, hidden = 0, heads = 0, kv_heads = 0, hd = 0, ffn = 0, vocab = 0, capacity = 0;
    float eps = 0.f;
    const float2* rope = nullptr;  // (cos, sin) [positions][hd/2]
    DevMatrix embed, out;
    const float* out_norm = nullptr;
    int32_t* chain = nullptr;      // device word: input token, replaced by the arg-max
    int* pos = nullptr;            // device word: position of the input token, advanced by one
    unsigned* epoch = nullptr;     // device word: tag of this launch's exchange words, advanced by one
    int32_t* emitted = nullptr;    // mapped host [capacity] (arg-max at emitted[pos]) or null
    int* status = nullptr;         // mapped host word, set non-zero if the launch aborted
    unsigned* abort_word = nullptr;  // device word shared by all workgroups of a launch
    unsigned long long* xbuf = nullptr;  // exchange words
    float* logits = nullptr;       // device [vocab] or null
    unsigned long long* trace = nullptr;  // [decode_trace_points][grid] wall-clock stamps, or null
    long long timeout_ticks = 0;   // bound on every wait, in wall-clock ticks
    int abort_at_layer = -1;       // failure-path tests: workgroup 0 aborts the launch at this layer
    int target_items = 96;         // attention work items to aim for
    int max_splits = 1;            // splits per head the partial buffer holds
    int stage = 0;                 // floats of the LDS staging row
    // exchange-word offsets within one layer's block, and the block size
    int off_part = 0, off_ctx = 0, off_xa = 0, off_ffn = 0, off_xf = 0, layer_words = 0, off_cand = 0;
    // rows per workgroup of each projection (even)
    int rows_qkv = 0, rows_wo = 0, rows_ffn = 0, rows_down = 0, rows_out = 0;
    // leading rows of a workgroup's output-matrix share that the logits phase
    // stages in LDS by DMA before its wait (the rest stream through registers)
    int out_lds_rows = 0;
    int out_lds_off = 0;  // their byte offset in dynamic LDS (past every phase's use)
};
// Phase-end stamps per launch: [0] start, 6 per layer (qkv, attention, merge,
// wo, gate/up, down), then logits and the arg-max (workgroup 0 only).
__host__ __device__ inline int decode_trace_points(int layers) { return 3 + 6 * layers; }
// After those points, kDecodeAttnSubPoints stamps inside the attention phase
// of the last layer (the last value written wins): entry, loads issued, q
// ready, current k/v ready, scores, softmax, P.V, published.
constexpr int kDecodeAttnSubPoints = 8;
// Support, shared-memory size and launch of the persistent decode kernel.
bool decode_kernel_supported(int fmt, int hd, int heads, int kv_heads);
int decode_attention_max_splits(int capacity, int kv_heads, int target_items);
size_t decode_lds_bytes(const DecodeParams& p, int grid);
// Static LDS of the kernel variant (launch parameters and layer table).
size_t decode_static_lds(int fmt, int hd, int heads, int kv_heads);
// Byte offset of the staged output rows in dynamic LDS (past every phase's
// use), and the most rows of a share of `rows_out` that fit below `lds_limit`
// bytes from there (p.out_lds_off set).
size_t decode_logits_stage_offset(const DecodeParams& p, int grid);
int decode_logits_stage_rows(const DecodeParams& p, size_t lds_limit);
hipError_t decode_kernel_occupancy(int fmt, int hd, int heads, int kv_heads, size_t lds, int* blocks_per_cu);
// cooperative = 1 launches the grid with hipLaunchCooperativeKernel, 0 as an
// ordinary kernel (the default; the host orders persistent launches one at a
// time).  Residency of all workgroups is then not checked by the runtime: a
// workgroup that never starts makes the others' bounded waits expire, so the
// launch still ends, with an error.
hipError_t launch_decode_step(int fmt, const DecodeParams& p, int grid, size_t lds, int cooperative, hipStream_t st);

// attention (kernels_attention.hip).  Cache layout [kv_heads][capacity][hd].
// q rows are [tokens][heads][hd] with row stride ldq (elements).
// q (and with qlo its second term: two-term Q, float32-grade scores) f16
// [tokens][heads*hd]; P enters as p_terms f16 terms (0: two with qlo, else
// one); writes out_f32, or out_f16 (and, when out_f16_lo is set, its second
// term for rows >= lo_out0).  The second terms of Q and P are taken only in
// the 64-query blocks holding a row >= lo_q0 (qlo must be valid there).
hipError_t launch_flash_attention(const f16* q, const f16* qlo, int ldq, const f16* kc, const f16* vc, int capacity,
                                  int tokens, int heads, int kv_heads, int hd, int start, float* out_f32, f16* out_f16,
                                  f16* out_f16_lo, hipStream_t st, int p_terms = 0, int lo_q0 = 0, int lo_out0 = 0,
                                  unsigned* last_arrive = nullptr, float* last_part = nullptr);
// With last_arrive and last_part the flash launch computes the last query row
// in float32 (key splits merged by the last split workgroup of each head):
// last_arrive holds `heads` counters, zero between launches; last_part
// flash_last_part_floats(heads, hd) floats.
size_t flash_last_part_floats(int heads, int hd);
// Generic online-softmax attention, any hd <= 256, f16 or f32 cache, keys
// split into `splits` ranges merged by a second kernel when splits > 1.
int attention_splits(int length, int heads, int tokens);
size_t attention_partial_floats(int heads, int tokens, int splits, int hd);
// Decode (one query token at position length-1): split-K over the context,
// one workgroup per (KV head, split) for all query heads of the group; writes
// per-split partials [heads][splits][hd+2] merged by launch_attention_merge or
// by the Wo GEMV prologue.  Needs hd 64/128, heads/kv_heads <= 16.
// Context length = *pos_dev + 1 when pos_dev is set (device-side position),
// else `length`; `splits` workgroups of split_len positions each (<= 256, or
// <= 512 for at most 2 query heads per KV head).
// attention_decode_session_split_len: the split length sessions and the
// single-query ops take for a cache of `capacity` rows (0: unsupported).
bool attention_decode_supported(int heads, int kv_heads, int hd);
int attention_decode_session_split_len(int capacity, int heads, int kv_heads);
hipError_t launch_attention_decode(const float* q, const void* kc, const void* vc, int kv_f16, int capacity,
                                   int heads, int kv_heads, int hd, int length, const int* pos_dev, int split_len,
                                   int splits, float* partials, hipStream_t st);
hipError_t launch_attention_merge(const float* partials, int heads, int hd, int splits, float* out, hipStream_t st);
hipError_t launch_attention_generic(const float* q, int ldq, const void* kc, const void* vc, int kv_f16,
                                    int capacity, int tokens, int heads, int kv_heads, int hd, int start,
                                    int splits, float* partials, float* out, hipStream_t st);
