// Host runtime of the gfx950 backend: the C ABI declared in include/alpaca_hip.h.
//
// Mirrors the reference's Metal host code (Sources/AlpacaMetal/Backend):
// MetalLlamaModel (weights uploaded once), MetalLlamaSession (KV cache and
// scratch per session, chunked prefill, fused single-token decode, GPU greedy
// chain, stage profiling) and MetalOps (tensor-in / tensor-out kernel API).
// Every kernel runs on the session's own HIP stream; the host only enqueues,
// waits and copies logits / emitted tokens through pinned memory.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/alpaca_hip.h"
#include "common.h"
#include "host.h"

// ------------------------------------------------------------------ errors

static thread_local std::string g_err;

static int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

// A failed HIP call is also the thread's last HIP error, which later kernel
// launches read back (hipGetLastError) to detect their own failure; both
// macros clear it once the failure is reported.
#define HIP_OR(expr, what)                                                                             \
    do {                                                                                               \
        hipError_t e_ = (expr);                                                                        \
        if (e_ != hipSuccess) {                                                                        \
            hipGetLastError();                                                                         \
            return fail(AHIP_ERR_COMMAND_FAILED, std::string(what) + ": " + hipGetErrorString(e_));    \
        }                                                                                              \
    } while (0)

#define LAUNCH(expr)                                                                                   \
    do {                                                                                               \
        hipError_t e_ = (expr);                                                                        \
        if (e_ != hipSuccess) {                                                                        \
            hipGetLastError();                                                                         \
            return fail(AHIP_ERR_COMMAND_FAILED, std::string("kernel launch: ") + hipGetErrorString(e_)); \
        }                                                                                              \
    } while (0)

extern "C" const char* ahip_last_error(void) { return g_err.c_str(); }

// Kernel launches report their failure through hipGetLastError(), which also
// returns an error left by an earlier, unrelated HIP call of this thread
// (a failed teardown call, say).  Entry points that launch work start from a
// clean state.
static inline void drop_stale_error() { (void)hipGetLastError(); }

// For the library's other host sources (gguf.cpp).
int ahip_fail(int code, const std::string& msg) { return fail(code, msg); }

extern "C" const char* ahip_version(void) {
    return "alpaca_hip gfx950 (hand-written HIP; MFMA f16 prefill, dequant GEMV decode)";
}

// ------------------------------------------------------------------ host f16

// IEEE binary32 -> binary16, round to nearest even.
static uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t man = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);
        uint32_t q = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((((ax >> 23) - 112u)) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu, bits;
    if (e == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int s = -1;
            do { s++; man <<= 1; } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(112 - s) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

static int block_elems(int dt) { return dt == AHIP_Q8_0 || dt == AHIP_Q4_0 ? 32 : 1; }
static int block_bytes(int dt) { return dt == AHIP_F32 ? 4 : dt == AHIP_F16 ? 2 : dt == AHIP_Q8_0 ? 34 : 18; }
static int64_t raw_bytes(int dt, int64_t elements) { return elements / block_elems(dt) * block_bytes(dt); }
static bool valid_dtype(int dt) { return dt >= AHIP_F32 && dt <= AHIP_Q4_0; }

// ------------------------------------------------------------------ quantiser

template <typename F>
static void parallel_for(int64_t n, F f) {
    const int64_t kMin = 1 << 16;
    unsigned hw = std::thread::hardware_concurrency();
    int nt = (int)std::min<int64_t>(std::max(1u, std::min(hw, 16u)), std::max<int64_t>(1, n / kMin));
    if (nt <= 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> th;
    const int64_t per = (n + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        const int64_t a = t * per, b = std::min(n, a + per);
        if (a < b) th.emplace_back([=] { f(a, b); });
    }
    for (auto& t : th) t.join();
}


// Quantization.swift:39-73 (ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref).
extern "C" int ahip_quantize(int dtype, const float* v, int64_t count, void* out) {
    if (dtype != AHIP_Q8_0 && dtype != AHIP_Q4_0) return fail(AHIP_ERR_INVALID_ARGUMENT, "quantize target must be q8_0 or q4_0");
    if (count < 0 || count % 32 != 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "element count is not a multiple of 32");
    if (count && (!v || !out)) return fail(AHIP_ERR_INVALID_ARGUMENT, "null buffer");
    uint8_t* dst = (uint8_t*)out;
    parallel_for(count / 32, [&](int64_t b0, int64_t b1) {
    for (int64_t b = b0; b < b1; b++) {
        const float* x = v + b * 32;
        if (dtype == AHIP_Q8_0) {
            uint8_t* p = dst + b * 34;
            float amax = 0.f;
            for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
            const float d = amax / 127.0f;
            const float id = d != 0.f ? 1.0f / d : 0.f;
            const uint16_t dh = f32_to_f16_bits(d);
            std::memcpy(p, &dh, 2);
            for (int j = 0; j < 32; j++) {
                volatile float t = x[j] * id;  // one rounding, then round half away from zero
                p[2 + j] = (uint8_t)(int8_t)std::round((float)t);
            }
        } else {
            uint8_t* p = dst + b * 18;
            float maxv = 0.f, amax = 0.f;
            for (int j = 0; j < 32; j++)
                if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); maxv = x[j]; }
            const float d = maxv / -8.0f;
            const float id = d != 0.f ? 1.0f / d : 0.f;
            const uint16_t dh = f32_to_f16_bits(d);
            std::memcpy(p, &dh, 2);
            for (int j = 0; j < 16; j++) {
                volatile float tl = x[j] * id;
                volatile float th = x[j + 16] * id;
                volatile float sl = tl + 8.5f;
                volatile float sh = th + 8.5f;
                const int lo = std::min(15, (int)sl), hi = std::min(15, (int)sh);
                p[2 + j] = (uint8_t)((uint8_t)lo | ((uint8_t)hi << 4));
            }
        }
    }
    });
    return AHIP_OK;
}

// ------------------------------------------------------------------ synthetic inputs

static inline uint64_t splitmix_at(uint64_t seed, uint64_t step) {
    // State after `step` calls of next(): seed + step * gamma (Sampler.swift:30-40).
    uint64_t z = seed + step * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

extern "C" int ahip_synth_uniform(uint64_t seed, uint64_t offset, int64_t n, float lo, float hi, float* out) {
    if (n < 0 || (n && !out)) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad buffer");
    parallel_for(n, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; i++) {
            const double u = (double)(splitmix_at(seed, offset + i + 1) >> 11) * 0x1.0p-53;
            out[i] = (float)(lo + (double)(hi - lo) * u);
        }
    });
    return AHIP_OK;
}

extern "C" int ahip_synth_normal(uint64_t seed, uint64_t offset, int64_t n, float stdv, float* out) {
    if (n < 0 || (n && !out)) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad buffer");
    if (offset % 2) return fail(AHIP_ERR_INVALID_ARGUMENT, "normal stream offset must be even");
    const int64_t pairs = (n + 1) / 2;
    parallel_for(pairs, [&](int64_t a, int64_t b) {
        for (int64_t j = a; j < b; j++) {
            const uint64_t s = offset + 2 * j;
            const double u1 = (double)(splitmix_at(seed, s + 1) >> 11) * 0x1.0p-53;
            const double u2 = (double)(splitmix_at(seed, s + 2) >> 11) * 0x1.0p-53;
            const double r = std::sqrt(-2.0 * std::log(1.0 - u1));
            const double th = 6.283185307179586 * u2;
            out[2 * j] = (float)(r * std::cos(th) * stdv);
            if (2 * j + 1 < n) out[2 * j + 1] = (float)(r * std::sin(th) * stdv);
        }
    });
    return AHIP_OK;
}

extern "C" int ahip_synth_ints(uint64_t seed, uint64_t offset, int64_t n, uint64_t range, int64_t bias, int32_t* out) {
    if (n < 0 || (n && !out) || range == 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad arguments");
    parallel_for(n, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; i++) out[i] = (int32_t)((int64_t)(splitmix_at(seed, offset + i + 1) % range) + bias);
    });
    return AHIP_OK;
}

// ------------------------------------------------------------------ device

extern "C" int ahip_device_count(int* count) {
    if (!count) return fail(AHIP_ERR_INVALID_ARGUMENT, "null count");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return AHIP_OK;
}

extern "C" int ahip_context_create(int device, ahip_context** out) {
    if (!out) return fail(AHIP_ERR_INVALID_ARGUMENT, "null out");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(AHIP_ERR_NO_DEVICE, "no HIP device is available");
    if (device < 0 || device >= n) return fail(AHIP_ERR_INVALID_ARGUMENT, "device index out of range");
    HIP_OR(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    HIP_OR(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(AHIP_ERR_MODULE_LOAD, std::string("library is built for gfx950, device is ") + prop.gcnArchName);
    if (int rc = noalloc_scratch_init(device)) return rc;
    auto* c = new ahip_context();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(AHIP_ERR_COMMAND_FAILED, "hipStreamCreate failed");
    }
    *out = c;
    return AHIP_OK;
}

extern "C" int ahip_context_destroy(ahip_context* c) {
    if (!c) return AHIP_OK;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    hipStreamDestroy(c->stream);
    delete c;
    drop_stale_error();
    return AHIP_OK;
}

// RAII device allocation.
struct DevBuf {
    void* p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) hipFree(p);
    }
    int alloc(size_t bytes) {
        if (hipMalloc(&p, std::max<size_t>(bytes, 256)) != hipSuccess) {
            p = nullptr;
            return fail(AHIP_ERR_ALLOC, "failed to allocate a " + std::to_string(bytes) + "-byte device buffer");
        }
        return AHIP_OK;
    }
    template <typename T>
    T* as() const { return (T*)p; }
};

static int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return std::atoi(v);
}

// Operands of the two-term fast prefill that carry the second f16 term
// (lo = f16(x - f16(x))): the inputs of the QKV, Wo, gate/up and down GEMMs,
// and attention's Q and P.  An operand without it enters its MFMAs as one f16
// term (half the MFMA work and, for the GEMM inputs, half the activation
// bytes), and its producer writes no second plane.
enum : int { kLoQkv = 1, kLoWo = 2, kLoGateUp = 4, kLoDown = 8, kLoQ = 16, kLoP = 32, kLoAll = 63 };

// The second-term operands of a model's two-term prefill.  ALPACA_HIP_LO_TERMS
// (a kLo* bit mask, read at session creation) overrides the choice;
// ALPACA_HIP_FLASH_P_TERMS=1 takes P single-term.
static int lo_terms_for(const ahip_llama_config& c) {
    (void)c;
    int lo = env_int("ALPACA_HIP_LO_TERMS", kLoAll) & kLoAll;
    if (env_int("ALPACA_HIP_FLASH_P_TERMS", 2) == 1) lo &= ~kLoP;
    return lo;
}

// A weight matrix uploaded in the split quant/scale layout of DevMatrix.
struct OwnedMatrix {
    DevMatrix m;
    DevBuf q, s, s2;
    int64_t bytes = 0;
};

// Repack raw GGUF blocks of `rows` x `cols` into quant and scale streams.
static void repack_host(int dt, const uint8_t* raw, int64_t rows, int64_t cols, std::vector<uint8_t>& q,
                        std::vector<uint16_t>& s) {
    if (dt == AHIP_F16) {
        q.assign(raw, raw + rows * cols * 2);
        s.clear();
        return;
    }
    const int64_t nb = cols / 32, bb = block_bytes(dt), qb = dt == AHIP_Q8_0 ? 32 : 16;
    q.resize(rows * nb * qb);
    s.resize(rows * nb);
    for (int64_t b = 0; b < rows * nb; b++) {
        const uint8_t* p = raw + b * bb;
        std::memcpy(&s[b], p, 2);
        std::memcpy(&q[b * qb], p + 2, qb);
    }
}

// Rows of a [heads*hd, cols] projection reordered from split-half RoPE pairs
// (i, i+hd/2) to adjacent pairs (2i, 2i+1).  q.k is unchanged when q and k
// share the permutation, so attention results are identical while every
// kernel can rotate adjacent pairs.
static std::vector<uint8_t> interleave_rows(int dt, const void* raw, int64_t rows, int64_t cols, int hd) {
    const int64_t rb = raw_bytes(dt, cols);
    std::vector<uint8_t> out((size_t)(rows * rb));
    const uint8_t* src = (const uint8_t*)raw;
    for (int64_t r = 0; r < rows; r++) {
        const int64_t h = r / hd, d = r % hd, half = hd / 2;
        const int64_t from = h * hd + (d % 2 == 0 ? d / 2 : d / 2 + half);
        std::memcpy(&out[(size_t)(r * rb)], src + from * rb, (size_t)rb);
    }
    return out;
}

// Uploads one or more matrices with equal dtype and cols stacked in row space.
static int upload_matrix(int dt, const std::vector<std::pair<const void*, int64_t>>& parts, int64_t cols,
                         OwnedMatrix& out, hipStream_t st) {
    int64_t rows = 0;
    for (auto& p : parts) rows += p.second;
    const int64_t qbytes = dt == AHIP_F16 ? rows * cols * 2 : dt == AHIP_Q8_0 ? rows * cols : rows * cols / 2;
    const int64_t sbytes = dt == AHIP_F16 ? 0 : rows * (cols / 32) * 2;
    if (int rc = out.q.alloc(qbytes)) return rc;
    if (sbytes)
        if (int rc = out.s.alloc(sbytes)) return rc;
    int64_t qoff = 0, soff = 0;
    std::vector<uint8_t> q;
    std::vector<uint16_t> s;
    for (auto& p : parts) {
        repack_host(dt, (const uint8_t*)p.first, p.second, cols, q, s);
        HIP_OR(hipMemcpyAsync(out.q.as<uint8_t>() + qoff, q.data(), q.size(), hipMemcpyHostToDevice, st), "upload");
        if (!s.empty())
            HIP_OR(hipMemcpyAsync(out.s.as<uint8_t>() + soff, s.data(), s.size() * 2, hipMemcpyHostToDevice, st),
                   "upload");
        HIP_OR(hipStreamSynchronize(st), "upload");  // host staging is reused
        qoff += q.size();
        soff += s.size() * 2;
    }
    out.m.dtype = dt;
    out.m.rows = (int)rows;
    out.m.cols = (int)cols;
    out.m.q = out.q.as<uint8_t>();
    out.m.s = sbytes ? out.s.as<f16>() : nullptr;
    out.bytes = qbytes + sbytes;
    if (sbytes && cols % 64 == 0) {
        const int64_t s2bytes = stage_scale_elems((int)rows, (int)cols) * 4;
        if (int rc = out.s2.alloc(s2bytes)) return rc;
        HIP_OR(hipMemsetAsync(out.s2.p, 0, s2bytes, st), "stage scales");
        LAUNCH(launch_stage_scales(out.m.s, out.s2.as<uint32_t>(), (int)rows, (int)cols, st));
        HIP_OR(hipStreamSynchronize(st), "stage scales");
        out.m.s2 = out.s2.as<uint32_t>();
        out.bytes += s2bytes;
    }
    return AHIP_OK;
}

// The prefill weight cache's f16 copy of a quantised matrix
// (MetalLlamaModel.buildPrefillCache, MetalLlamaModel.swift:97-120); an F16
// matrix needs none and gets an empty copy.
static int half_copy(const OwnedMatrix& w, OwnedMatrix& h, hipStream_t st) {
    if (w.m.dtype == AHIP_F16) return AHIP_OK;
    const int64_t bytes = (int64_t)w.m.rows * w.m.cols * 2;
    if (int rc = h.q.alloc(bytes)) return rc;
    LAUNCH(launch_dequant_f16(w.m, h.q.as<f16>(), st));
    h.m = DevMatrix{};
    h.m.dtype = AHIP_F16;
    h.m.rows = w.m.rows;
    h.m.cols = w.m.cols;
    h.m.q = h.q.as<uint8_t>();
    h.bytes = bytes;
    return AHIP_OK;
}

// RoPE (cos, sin) for positions [0, positions): frequencies and angles in
// double, rounded once to float (CPUOps.rope, CPUOps.swift:196-201).
static std::vector<float2> rope_table(int positions, int hd, float theta) {
    const int half = hd / 2;
    std::vector<float2> t((size_t)positions * half);
    std::vector<double> freq(half);
    for (int i = 0; i < half; i++) freq[i] = std::pow((double)theta, -2.0 * (double)i / (double)hd);
    for (int p = 0; p < positions; p++)
        for (int i = 0; i < half; i++) {
            const double a = (double)p * freq[i];
            t[(size_t)p * half + i] = make_float2((float)std::cos(a), (float)std::sin(a));
        }
    return t;
}

// ------------------------------------------------------------------ model

struct ahip_model {
    // The creator's reference plus one per live session: a model outlives its
    // sessions (MetalLlamaSession holds its MetalLlamaModel), whatever order the
    // caller destroys them in.
    std::atomic<int> refs{1};
    ahip_context* ctx = nullptr;
    int device = 0;  // kept so destruction never touches a destroyed context
    ahip_llama_config c{};
    struct Layer {
        DevBuf attn_norm, ffn_norm;
        OwnedMatrix qkv, wo, gate, up, down;
        // prefill weight cache: f16 copies of the quantised projections (else empty)
        OwnedMatrix qkv16, wo16, gate16, up16, down16;
        // the matrices the fast (f16 MFMA) prefill multiplies by
        const DevMatrix& pre(const OwnedMatrix& w, const OwnedMatrix& h) const { return h.m.q ? h.m : w.m; }
    };
    std::vector<std::unique_ptr<Layer>> layers;
    OwnedMatrix embed, output;
    bool tied = false;
    DevBuf output_norm, rope;
    int64_t weight_bytes = 0;
    int64_t prefill_cache_bytes = 0;
    const DevMatrix& out_matrix() const { return tied ? embed.m : output.m; }
};

// LlamaConfig.validate (LlamaConfig.swift:30-43) plus what these kernels need
// (MetalLlamaModel.swift:44-46: head_dim a multiple of 32 up to 256).
static int validate_config(const ahip_llama_config* c) {
    if (!c) return fail(AHIP_ERR_INVALID_ARGUMENT, "null config");
    if (c->vocab_size <= 0 || c->hidden_size <= 0 || c->layer_count <= 0 || c->head_count <= 0 ||
        c->kv_head_count <= 0 || c->head_dim <= 0 || c->feed_forward_size <= 0 || c->context_length <= 0)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "all dimensions must be positive");
    if (c->head_count % c->kv_head_count) return fail(AHIP_ERR_INVALID_ARGUMENT, "headCount is not a multiple of kvHeadCount");
    if (c->head_dim % 2) return fail(AHIP_ERR_INVALID_ARGUMENT, "RoPE needs an even headDim");
    if (!(c->rms_norm_eps > 0) || !(c->rope_theta > 0)) return fail(AHIP_ERR_INVALID_ARGUMENT, "rmsNormEps and ropeTheta must be positive");
    const int64_t lim = 1 << 28;
    if (c->vocab_size > lim || c->hidden_size > lim || c->feed_forward_size > lim || c->layer_count > lim ||
        c->context_length > lim)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "implausibly large dimension");
    if (c->head_dim % 32 || c->head_dim > 256)
        return fail(AHIP_ERR_UNSUPPORTED, "head dimension must be a multiple of 32 up to 256");
    const int qw = c->head_count * c->head_dim;
    for (int k : {c->hidden_size, qw, c->feed_forward_size})
        if (k % 32 || k > 12288) return fail(AHIP_ERR_UNSUPPORTED, "input widths must be multiples of 32 up to 12288");
    return AHIP_OK;
}

int ahip_validate_config(const ahip_llama_config* c) { return validate_config(c); }

extern "C" int ahip_model_create(ahip_context* ctx, const ahip_llama_config* config, const ahip_tensor_desc* tensors,
                                 int count, int prefill_weight_cache, ahip_model** out) {
    if (!ctx || !out || (count && !tensors)) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    drop_stale_error();
    if (int rc = validate_config(config)) return rc;
    const ahip_llama_config& c = *config;
    std::map<std::string, const ahip_tensor_desc*> byname;
    for (int i = 0; i < count; i++) {
        if (!tensors[i].name) return fail(AHIP_ERR_INVALID_ARGUMENT, "tensor without a name");
        if (!byname.emplace(tensors[i].name, &tensors[i]).second)
            return fail(AHIP_ERR_INVALID_ARGUMENT, std::string("duplicate tensor ") + tensors[i].name);
    }
    auto get = [&](const std::string& n, int64_t rows, int64_t cols, bool norm, const ahip_tensor_desc** d) -> int {
        auto it = byname.find(n);
        if (it == byname.end()) return fail(AHIP_ERR_INVALID_ARGUMENT, "missing tensor " + n);
        const ahip_tensor_desc* t = it->second;
        const bool shape_ok = norm ? (t->rows * t->cols == cols && (t->rows == 1 || t->cols == 1))
                                   : (t->rows == rows && t->cols == cols);
        if (!shape_ok)
            return fail(AHIP_ERR_INVALID_ARGUMENT, n + ": expected shape [" + std::to_string(rows) + ", " +
                                                       std::to_string(cols) + "]");
        if (!valid_dtype(t->dtype)) return fail(AHIP_ERR_INVALID_ARGUMENT, n + ": unknown dtype");
        if (norm && t->dtype != AHIP_F32) return fail(AHIP_ERR_INVALID_ARGUMENT, n + ": norm weights must be f32");
        if (!norm && t->dtype == AHIP_F32)
            return fail(AHIP_ERR_UNSUPPORTED, n + ": f32 projection matrices (use f16, q8_0 or q4_0)");
        if (!t->data || t->bytes != raw_bytes(t->dtype, t->rows * t->cols))
            return fail(AHIP_ERR_INVALID_ARGUMENT, n + ": byte count does not match shape and dtype");
        *d = t;
        return AHIP_OK;
    };
    const int H = c.hidden_size, QW = c.head_count * c.head_dim, KW = c.kv_head_count * c.head_dim,
              F = c.feed_forward_size, V = c.vocab_size;
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    auto m = std::make_unique<ahip_model>();
    m->ctx = ctx;
    m->device = ctx->device;
    m->c = c;
    hipStream_t st = ctx->stream;
    const ahip_tensor_desc *te, *tn, *to = nullptr;
    if (int rc = get("token_embd", V, H, false, &te)) return rc;
    if (int rc = get("output_norm", 1, H, true, &tn)) return rc;
    if (byname.count("output"))
        if (int rc = get("output", V, H, false, &to)) return rc;
    if (int rc = upload_matrix(te->dtype, {{te->data, V}}, H, m->embed, st)) return rc;
    m->weight_bytes += m->embed.bytes;
    m->tied = to == nullptr;
    if (to) {
        if (int rc = upload_matrix(to->dtype, {{to->data, V}}, H, m->output, st)) return rc;
        m->weight_bytes += m->output.bytes;
    }
    auto upload_norm = [&](const ahip_tensor_desc* t, DevBuf& b) -> int {
        if (int rc = b.alloc(H * 4)) return rc;
        HIP_OR(hipMemcpy(b.p, t->data, H * 4, hipMemcpyHostToDevice), "upload norm");
        m->weight_bytes += H * 4;
        return AHIP_OK;
    };
    if (int rc = upload_norm(tn, m->output_norm)) return rc;
    for (int i = 0; i < c.layer_count; i++) {
        auto L = std::make_unique<ahip_model::Layer>();
        const std::string p = "blk." + std::to_string(i) + ".";
        const ahip_tensor_desc *an, *fn, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
        if (int rc = get(p + "attn_norm", 1, H, true, &an)) return rc;
        if (int rc = get(p + "attn_q", QW, H, false, &wq)) return rc;
        if (int rc = get(p + "attn_k", KW, H, false, &wk)) return rc;
        if (int rc = get(p + "attn_v", KW, H, false, &wv)) return rc;
        if (int rc = get(p + "attn_output", H, QW, false, &wo)) return rc;
        if (int rc = get(p + "ffn_norm", 1, H, true, &fn)) return rc;
        if (int rc = get(p + "ffn_gate", F, H, false, &wg)) return rc;
        if (int rc = get(p + "ffn_up", F, H, false, &wu)) return rc;
        if (int rc = get(p + "ffn_down", H, F, false, &wd)) return rc;
        if (wq->dtype != wk->dtype || wq->dtype != wv->dtype)
            return fail(AHIP_ERR_UNSUPPORTED, p + "attn_q/k/v must share one format (they are stacked into one matrix)");
        if (wg->dtype != wu->dtype) return fail(AHIP_ERR_UNSUPPORTED, p + "ffn_gate/up must share one format");
        if (int rc = upload_norm(an, L->attn_norm)) return rc;
        if (int rc = upload_norm(fn, L->ffn_norm)) return rc;
        const void* qd = wq->data;
        const void* kd = wk->data;
        std::vector<uint8_t> qperm, kperm;
        if (!c.rope_interleaved) {
            qperm = interleave_rows(wq->dtype, wq->data, QW, H, c.head_dim);
            kperm = interleave_rows(wk->dtype, wk->data, KW, H, c.head_dim);
            qd = qperm.data();
            kd = kperm.data();
        }
        if (int rc = upload_matrix(wq->dtype, {{qd, QW}, {kd, KW}, {wv->data, KW}}, H, L->qkv, st)) return rc;
        if (int rc = upload_matrix(wo->dtype, {{wo->data, H}}, QW, L->wo, st)) return rc;
        if (int rc = upload_matrix(wg->dtype, {{wg->data, F}}, H, L->gate, st)) return rc;
        if (int rc = upload_matrix(wu->dtype, {{wu->data, F}}, H, L->up, st)) return rc;
        if (int rc = upload_matrix(wd->dtype, {{wd->data, H}}, F, L->down, st)) return rc;
        m->weight_bytes += L->qkv.bytes + L->wo.bytes + L->gate.bytes + L->up.bytes + L->down.bytes;
        m->layers.push_back(std::move(L));
    }
    if (prefill_weight_cache)
        for (auto& L : m->layers)
            for (auto [w, h] : {std::pair{&L->qkv, &L->qkv16}, {&L->wo, &L->wo16}, {&L->gate, &L->gate16},
                                {&L->up, &L->up16}, {&L->down, &L->down16}}) {
                if (int rc = half_copy(*w, *h, st)) return rc;
                m->prefill_cache_bytes += h->bytes;
            }
    auto table = rope_table(c.context_length, c.head_dim, c.rope_theta);
    if (int rc = m->rope.alloc(table.size() * sizeof(float2))) return rc;
    HIP_OR(hipMemcpy(m->rope.p, table.data(), table.size() * sizeof(float2), hipMemcpyHostToDevice), "upload rope table");
    HIP_OR(hipStreamSynchronize(st), "model upload");
    *out = m.release();
    return AHIP_OK;
}

static void model_release(ahip_model* m) {
    if (m->refs.fetch_sub(1) != 1) return;
    hipSetDevice(m->device);
    delete m;
    drop_stale_error();
}

extern "C" int ahip_model_destroy(ahip_model* m) {
    if (!m) return AHIP_OK;
    model_release(m);
    return AHIP_OK;
}

extern "C" int ahip_model_weight_bytes(const ahip_model* m, int64_t* bytes) {
    if (!m || !bytes) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *bytes = m->weight_bytes;
    return AHIP_OK;
}

extern "C" int ahip_model_prefill_cache_bytes(const ahip_model* m, int64_t* bytes) {
    if (!m || !bytes) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *bytes = m->prefill_cache_bytes;
    return AHIP_OK;
}

// ------------------------------------------------------------------ session

struct SessionSizes {
    int64_t kv_per_layer, x, qkv, q16, ctx, ffn, partials, logits;
    int64_t total;
};

static constexpr int kMaxSplits = 65;

static SessionSizes session_sizes(const ahip_llama_config& c, int capacity, int max_batch, int kv_f16) {
    SessionSizes s{};
    const int64_t B = max_batch, QW = (int64_t)c.head_count * c.head_dim, KW = (int64_t)c.kv_head_count * c.head_dim;
    s.kv_per_layer = (int64_t)capacity * KW * (kv_f16 ? 2 : 4);
    s.x = B * c.hidden_size;
    s.qkv = B * (QW + 2 * KW);
    s.q16 = B * QW;
    s.ctx = B * QW;
    s.ffn = B * c.feed_forward_size;
    s.partials = (int64_t)c.head_count * kMaxSplits * (c.head_dim + 2);
    s.logits = c.vocab_size;
    // the f16 activation buffers hold two planes (the two-term activations' hi and lo)
    s.total = 2 * c.layer_count * s.kv_per_layer + 4 * (2 * s.x + s.qkv + s.ctx + s.ffn + s.partials + s.logits) +
              4 * (s.x + s.q16 + s.ctx + s.ffn) + 4 * ((int64_t)capacity + 9 + capacity);
    return s;
}

extern "C" int ahip_session_byte_count(const ahip_llama_config* config, int capacity, int max_batch, int kv_precision,
                                       int64_t* bytes) {
    if (!config || !bytes || capacity <= 0 || max_batch <= 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    *bytes = session_sizes(*config, capacity, max_batch, kv_precision == AHIP_KV_F16).total;
    return AHIP_OK;
}

struct StageMark {
    std::string label;
    hipEvent_t start, end;
    int dispatches;
};

static void split_stream_release(int device);  // below, with the split prefill

struct ahip_session {
    ahip_model* m = nullptr;
    int capacity = 0, max_batch = 0, kv_f16 = 1, fast = 1;
    int two_term = 1;  // fast prefill with two-term activations (AHIP_GEMM_FAST); 0: one f16 term (FAST_F16)
    int lo_terms = 0;  // with two_term: which operands carry the second term (kLo* bits)
    bool lo_all_rows = false;  // second terms on every row, not only the last row's tiles
    bool qkv_lo_all = false;   // the QKV GEMM's q columns take the second term on every row too
    int fuse_qkv_rope = 1;  // ALPACA_HIP_FUSE_QKV_ROPE at creation; 0: RoPE + KV append as their own kernel
    int exact_last_row = 1;  // ALPACA_HIP_EXACT_LAST_ROW at creation; 0: two-term last query block instead
    DevBuf last_arrive, last_part;  // the float32 last row of the flash launch: counters per head, split partials
    // Numerics diagnostics, read at creation: ALPACA_HIP_PREFILL_ATTENTION=generic runs the fast prefill's
    // attention as the float32 kernel the exact prefill uses; ALPACA_HIP_PREFILL_GEMM=f32 its projections as
    // the exact float32 GEMMs.
    int prefill_generic_attention = 0, prefill_f32_gemm = 0;
    bool logits_ready = false;  // `logits` holds the last forward's logits (for ahip_session_sample)
    DevBuf sample_idx, sample_p, sample_out;  // sampler scratch, allocated on first use
    hipStream_t stream = nullptr;
    // Streams of a split prefill (part 0 on `stream`, the other part on the
    // device's split stream, shared by all sessions) and this session's events:
    // part_start orders the parts after the session stream's earlier work,
    // part_qkv[k] marks part k's K/V rows of the current layer in the cache,
    // part_done[k] joins part k back.  Set up on the first split.
    static constexpr int kMaxParts = 2;  // three and four parts measured slower (C1 4096: 466k / 494k tok/s)
    hipStream_t part_stream[kMaxParts] = {};
    hipEvent_t part_start = nullptr, part_qkv[kMaxParts] = {}, part_done[kMaxParts] = {};
    std::vector<std::unique_ptr<DevBuf>> kc, vc;
    DevBuf x, xn, xh, qkv, qh, ctx, ctxh, ffn, ffnh, partials, logits, tokens, chain, dpos;
    float* logits_host = nullptr;
    int32_t* emitted_host = nullptr;   // pinned, mapped: the arg-max kernel writes tokens here
    int32_t* emitted_mapped = nullptr; // device address of emitted_host
    bool dec_split = false;            // split-K decode attention (else the generic kernel)
    int dec_split_len = 0, dec_splits = 0;
    hipGraphExec_t greedy_graph = nullptr;
    bool graph_failed = false;
    // persistent single-token decode (kernels_decode.hip): one launch per token
    bool pdec = false;
    int pdec_fmt = 0, pdec_grid = 0, pdec_coop = 0;
    size_t pdec_lds = 0;
    DecodeParams pdec_params;
    DevBuf pdec_layers, pdec_xbuf, pdec_ctl;  // ctl: [0] epoch, [1] abort word
    hipEvent_t pdec_peer = nullptr;          // recorded on another session's stream to order after it
    int64_t pdec_xbuf_bytes = 0;
    int* pdec_status = nullptr;              // mapped host word, set by an aborting launch
    uint64_t pdec_launches = 0;
    int pdec_clock_khz = 0;                  // wall-clock rate of the trace stamps
    DevBuf pdec_trace;                       // phase-end stamps of the last launch (profiling)
    std::vector<unsigned long long> pdec_trace_host;
    std::map<std::string, std::pair<double, int>> pdec_stages;
    int32_t* tokens_host = nullptr;
    int length = 0;
    std::atomic<int> busy{0};
    double last_gpu = 0, last_encode = 0;
    bool profiling = false;
    std::vector<hipEvent_t> event_pool;
    size_t events_used = 0;
    std::vector<StageMark> marks;
    std::vector<ahip_stage> profile;
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;

    ~ahip_session() {
        if (stream) hipStreamSynchronize(stream);
        for (auto e : event_pool) hipEventDestroy(e);
        if (ev_begin) hipEventDestroy(ev_begin);
        if (ev_end) hipEventDestroy(ev_end);
        if (greedy_graph) hipGraphExecDestroy(greedy_graph);
        if (logits_host) hipHostFree(logits_host);
        if (emitted_host) hipHostFree(emitted_host);
        if (tokens_host) hipHostFree(tokens_host);
        if (pdec_status) hipHostFree(pdec_status);
        if (pdec_peer) hipEventDestroy(pdec_peer);
        // (a split's work on the shared split stream ends in part_done, which the
        // session stream waits for, so syncing the session stream covers it)
        if (part_stream[1]) split_stream_release(m->device);
        if (part_start) hipEventDestroy(part_start);
        for (int k = 0; k < kMaxParts; k++) {
            if (part_qkv[k]) hipEventDestroy(part_qkv[k]);
            if (part_done[k]) hipEventDestroy(part_done[k]);
        }
        if (stream) hipStreamDestroy(stream);
    }

    hipEvent_t next_event() {
        if (events_used == event_pool.size()) {
            hipEvent_t e;
            hipEventCreate(&e);
            event_pool.push_back(e);
        }
        return event_pool[events_used++];
    }
    // Opens a labelled stage (EncoderProvider.stage, MetalLlamaModel.swift:431-447).
    void stage(const char* label) {
        if (!profiling) return;
        if (!marks.empty() && marks.back().label == label) {
            marks.back().dispatches++;
            return;
        }
        hipEvent_t e = next_event();
        hipEventRecord(e, stream);
        if (!marks.empty()) marks.back().end = e;
        marks.push_back({label, e, nullptr, 1});
    }
    void stage_end() {
        if (!profiling || marks.empty() || marks.back().end) return;
        hipEvent_t e = next_event();
        hipEventRecord(e, stream);
        marks.back().end = e;
    }
    void collect_profile() {
        profile.clear();
        if (!profiling) return;
        std::map<std::string, size_t> index;
        for (auto& mk : marks) {
            float ms = 0;
            if (mk.end) hipEventElapsedTime(&ms, mk.start, mk.end);
            auto it = index.find(mk.label);
            if (it == index.end()) {
                ahip_stage s{};
                std::snprintf(s.label, sizeof s.label, "%s", mk.label.c_str());
                index[mk.label] = profile.size();
                profile.push_back(s);
                it = index.find(mk.label);
            }
            profile[it->second].seconds += ms * 1e-3;
            profile[it->second].dispatches += mk.dispatches;
        }
    }
    void begin_call() {
        events_used = 0;
        marks.clear();
    }
};


// Shortest prefill chunk that may run as two halves on two streams
// (encode_split_prefill); ALPACA_HIP_SPLIT_MIN (read per call) overrides it.
constexpr int kSplitPrefillMin = 1536;

// The second-half stream of split prefills, one per device, shared by the
// sessions that split a prefill: created on the first such split, destroyed
// when the last of those sessions is (nothing HIP owns is left to the runtime's
// exit-time teardown, under which a leftover stream crashed the profiled
// process in exit handlers).  It must not share a hardware
// queue with the sessions' streams (the halves would then run one after the
// other, with an inter-stream barrier per layer: measured 30% slower than one
// stream).  The runtime deals its few hardware queues (GPU_MAX_HW_QUEUES) out
// to ordinary streams as it sees fit, while a stream created with a CU mask
// gets a queue of its own; the mask enables every CU.  One per device rather
// than one per session, because every extra active queue is another one for
// the hardware scheduler to time-slice: with a masked stream per session the
// bench's fourth session prefilled at 442k instead of 790k tok/s.
namespace {
struct SplitStream {
    std::mutex lock;
    hipStream_t st = nullptr;
    int users = 0;  // sessions holding it
};
SplitStream g_split_stream[64];
}  // namespace

// A reference to the device's split stream (created if none exists), or null.
static hipStream_t split_stream_acquire(int device) {
    SplitStream& g = g_split_stream[device & 63];
    std::lock_guard<std::mutex> l(g.lock);
    if (!g.st) {
        int cus = 0;
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        std::vector<uint32_t> all((size_t)std::max(1, (cus + 31) / 32), 0xFFFFFFFFu);
        if (hipExtStreamCreateWithCUMask(&g.st, (uint32_t)all.size(), all.data()) != hipSuccess) {
            hipGetLastError();
            g.st = nullptr;
        }
    }
    if (g.st) g.users++;
    return g.st;
}

// Drops a session's reference; the last one synchronises and destroys the stream.
static void split_stream_release(int device) {
    SplitStream& g = g_split_stream[device & 63];
    std::lock_guard<std::mutex> l(g.lock);
    if (g.users > 0 && --g.users == 0 && g.st) {
        hipStreamSynchronize(g.st);
        hipStreamDestroy(g.st);
        g.st = nullptr;
    }
}

// Persistent decode launches of all sessions on one device run one at a time.
// Each launch needs every one of its workgroups resident at once (one per CU),
// so two launches on two sessions' streams could each hold part
// of the chip and spin in their bounded waits until both abort.  The device
// remembers the stream of its last persistent launch; a launch from another
// session first records an event at the tail of that stream and makes its own
// stream wait for it (on the GPU; the host never blocks).  Consecutive launches
// of one session are ordered by its stream alone and record nothing.
namespace {
struct PdecOrder {
    std::mutex lock;
    const ahip_session* last = nullptr;  // session of the device's last persistent launch
    hipStream_t last_stream = nullptr;   // its stream
};
PdecOrder g_pdec_order[64];
}  // namespace

// ------------------------------------------------------------------ persistent decode setup

// Clears the exchange words and restarts the launch tag at 1 (session
// creation, tag wrap-around, and recovery after an aborted launch).
static int pdec_reset_words(ahip_session* s) {
    HIP_OR(hipMemsetAsync(s->pdec_xbuf.p, 0, (size_t)s->pdec_xbuf_bytes, s->stream), "clear exchange words");
    const unsigned init[2] = {1u, 0u};
    HIP_OR(hipMemcpyAsync(s->pdec_ctl.p, init, sizeof init, hipMemcpyHostToDevice, s->stream), "reset decode tag");
    HIP_OR(hipStreamSynchronize(s->stream), "reset decode tag");
    *(volatile int*)s->pdec_status = 0;
    s->pdec_launches = 0;
    return AHIP_OK;
}

// Chooses the persistent decode kernel when the model and device allow it:
// f16 KV cache, one weight format for every layer matrix, head_dim 64/128,
// cooperative launch support and enough LDS, and layers whose matrices are
// below the streamed GEMV's size.  Where every projection of a layer streams
// (each at least 4 MB: the 1.7B shape), the multi-kernel step (streamed GEMVs,
// split-K attention and merge, one HIP graph per greedy step) moves more bytes
// per microsecond than the persistent kernel's one workgroup per CU: 1.7B
// shape at context 4,096, 942 against 1,172 us per token.
// ALPACA_HIP_PERSISTENT_DECODE=0 turns the persistent kernel off, =2 takes it
// for large layers too; ALPACA_HIP_DECODE_WGS sets the workgroup count (default: one
// per CU); ALPACA_HIP_DECODE_ITEMS the attention items aimed for;
// ALPACA_HIP_DECODE_TIMEOUT_US the bound on each wait inside the kernel;
// ALPACA_HIP_DECODE_ABORT_LAYER (failure-path tests) makes every launch abort
// at that layer; ALPACA_HIP_DECODE_COOPERATIVE=1 launches it with
// hipLaunchCooperativeKernel instead of an ordinary launch.
//
// Ordinary launches are the default.  What residency needs is that no other
// long-lived grid holds CUs while a step runs: persistent launches of every
// session of this process are ordered one after another on the GPU
// (PdecOrder), every other kernel of the library ends on its own, and every
// wait inside the persistent kernel is bounded, so a workgroup that cannot get
// a CU for the whole bound (another process's long grid) ends the launch with
// AHIP_ERR_COMMAND_FAILED rather than a hang.  A cooperative launch adds the
// runtime's own occupancy check and exclusion against other processes'
// cooperative grids, at 12-18 us per token on MI355X (C1 602 against 588 us).
static int setup_persistent_decode(ahip_session* s) {
    ahip_model* m = s->m;
    const ahip_llama_config& c = m->c;
    const int mode = env_int("ALPACA_HIP_PERSISTENT_DECODE", 1);
    if (!mode || !s->kv_f16) return AHIP_OK;
    {
        const ahip_model::Layer& L0 = *m->layers[0];
        bool streams = s->dec_split;
        for (const OwnedMatrix* om : {&L0.qkv, &L0.wo, &L0.gate, &L0.up, &L0.down}) streams = streams && gemv_streams(om->m);
        if (streams && mode != 2) return AHIP_OK;
    }
    const int fmt = m->layers[0]->qkv.m.dtype;
    for (auto& L : m->layers)
        for (const OwnedMatrix* om : {&L->qkv, &L->wo, &L->gate, &L->up, &L->down})
            if (om->m.dtype != fmt) return AHIP_OK;
    if (!decode_kernel_supported(fmt, c.head_dim, c.head_count, c.kv_head_count)) return AHIP_OK;
    int coop = 0, cus = 0, clock_khz = 0;
    hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, m->device);
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->device);
    hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, m->device);
    if (!coop || cus <= 0 || clock_khz <= 0) return AHIP_OK;

    const int H = c.hidden_size, QW = c.head_count * c.head_dim, KW = c.kv_head_count * c.head_dim,
              F = c.feed_forward_size, V = c.vocab_size, hd = c.head_dim;
    DecodeParams p;
    p.n_layers = c.layer_count;
    p.hidden = H;
    p.heads = c.head_count;
    p.kv_heads = c.kv_head_count;
    p.hd = hd;
    p.ffn = F;
    p.vocab = V;
    p.capacity = s->capacity;
    p.eps = c.rms_norm_eps;
    p.rope = m->rope.as<float2>();
    p.embed = m->embed.m;
    p.out = m->out_matrix();
    p.out_norm = m->output_norm.as<float>();
    p.target_items = std::max(1, env_int("ALPACA_HIP_DECODE_ITEMS", 96));
    p.max_splits = decode_attention_max_splits(s->capacity, c.kv_head_count, p.target_items);
    p.stage = std::max(H, std::max(QW, F));
    p.off_part = QW + 2 * KW;
    p.off_ctx = p.off_part + c.head_count * p.max_splits * (hd + 2);
    p.off_xa = p.off_ctx + QW;
    p.off_ffn = p.off_xa + H;
    p.off_xf = p.off_ffn + F;
    p.layer_words = p.off_xf + H;
    p.off_cand = c.layer_count * p.layer_words;

    int grid = env_int("ALPACA_HIP_DECODE_WGS", cus);
    grid = std::max(1, std::min(grid, 4096));
    auto even_share = [&](int rows) { int r = (rows + grid - 1) / grid; return r + (r & 1); };
    p.rows_qkv = even_share(QW + 2 * KW);
    p.rows_wo = even_share(H);
    p.rows_ffn = even_share(F);
    p.rows_down = even_share(H);
    p.rows_out = even_share(V);
    size_t lds = decode_lds_bytes(p, grid);
    int max_lds = 0;
    hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, m->device);
    if (lds > (size_t)max_lds) return AHIP_OK;
    int per_cu = 0;
    if (decode_kernel_occupancy(fmt, hd, c.head_count, c.kv_head_count, lds, &per_cu) != hipSuccess || per_cu < 1) {
        hipGetLastError();
        return AHIP_OK;
    }
    grid = std::min(grid, per_cu * cus);
    // the row shares depend on the grid; recompute if the grid shrank
    p.rows_qkv = even_share(QW + 2 * KW);
    p.rows_wo = even_share(H);
    p.rows_ffn = even_share(F);
    p.rows_down = even_share(H);
    p.rows_out = even_share(V);
    // The logits phase stages the leading rows of each workgroup's output share
    // in whatever LDS the device leaves beyond the kernel's static arrays
    // (ALPACA_HIP_DECODE_LOGIT_STAGE_ROWS caps the count; 0 streams every row
    // through registers).  The copy's loads sit ahead of the QKV input polls of
    // the last eight layers in each wave's in-order load queue (C1 0.4 us, C5
    // 0.9 us more per such layer), so by default rows are staged only where at
    // least half of a workgroup's share fits: C4 765 against 771 us per step
    // with all rows staged, C1 even, C5 (a quarter fits) 1,177 against 1,171.
    {
        const size_t stat = decode_static_lds(fmt, hd, c.head_count, c.kv_head_count);
        const size_t limit = (size_t)max_lds > stat ? (size_t)max_lds - stat : 0;
        p.out_lds_off = (int)decode_logits_stage_offset(p, grid);
        const int fit = decode_logits_stage_rows(p, limit);
        p.out_lds_rows = std::max(0, std::min(env_int("ALPACA_HIP_DECODE_LOGIT_STAGE_ROWS",
                                                      2 * fit >= p.rows_out ? fit : 0),
                                              fit));
    }
    lds = decode_lds_bytes(p, grid);
    if (decode_kernel_occupancy(fmt, hd, c.head_count, c.kv_head_count, lds, &per_cu) != hipSuccess ||
        per_cu * cus < grid) {
        hipGetLastError();
        return AHIP_OK;
    }

    std::vector<DecLayer> table(c.layer_count);
    for (int l = 0; l < c.layer_count; l++) {
        const ahip_model::Layer& L = *m->layers[l];
        table[l].qkv = L.qkv.m;
        table[l].wo = L.wo.m;
        table[l].gate = L.gate.m;
        table[l].up = L.up.m;
        table[l].down = L.down.m;
        table[l].attn_norm = L.attn_norm.as<float>();
        table[l].ffn_norm = L.ffn_norm.as<float>();
        table[l].kc = s->kc[l]->p;
        table[l].vc = s->vc[l]->p;
    }
    if (int rc = s->pdec_layers.alloc(table.size() * sizeof(DecLayer))) return rc;
    HIP_OR(hipMemcpy(s->pdec_layers.p, table.data(), table.size() * sizeof(DecLayer), hipMemcpyHostToDevice),
           "upload layer table");
    s->pdec_xbuf_bytes = ((int64_t)p.off_cand + 2 * grid) * 8;
    if (int rc = s->pdec_xbuf.alloc((size_t)s->pdec_xbuf_bytes)) return rc;
    if (int rc = s->pdec_ctl.alloc(256)) return rc;
    if (hipHostMalloc((void**)&s->pdec_status, 64, hipHostMallocMapped) != hipSuccess)
        return fail(AHIP_ERR_ALLOC, "pinned host allocation failed");
    int* status_dev = nullptr;
    HIP_OR(hipHostGetDevicePointer((void**)&status_dev, s->pdec_status, 0), "hipHostGetDevicePointer");
    p.layers = s->pdec_layers.as<DecLayer>();
    p.chain = s->chain.as<int32_t>();
    p.pos = s->dpos.as<int>();
    p.epoch = s->pdec_ctl.as<unsigned>();
    p.abort_word = s->pdec_ctl.as<unsigned>() + 1;
    p.status = status_dev;
    p.xbuf = s->pdec_xbuf.as<unsigned long long>();
    p.emitted = nullptr;
    p.logits = nullptr;
    const long long timeout_us = env_int("ALPACA_HIP_DECODE_TIMEOUT_US", 2000000);
    p.timeout_ticks = std::max(1LL, timeout_us * (long long)clock_khz / 1000);
    p.abort_at_layer = env_int("ALPACA_HIP_DECODE_ABORT_LAYER", -1);  // failure-path tests
    s->pdec_params = p;
    s->pdec_clock_khz = clock_khz;
    s->pdec_coop = env_int("ALPACA_HIP_DECODE_COOPERATIVE", 0);
    s->pdec_fmt = fmt;
    s->pdec_grid = grid;
    s->pdec_lds = lds;
    HIP_OR(hipEventCreateWithFlags(&s->pdec_peer, hipEventDisableTiming), "hipEventCreate");
    if (int rc = pdec_reset_words(s)) return rc;
    s->pdec = true;
    return AHIP_OK;
}


// Enqueues one persistent decode launch: the token in `chain` at position
// *dpos; the arg-max goes to `chain` (and emitted[pos] when `emitted`), the
// logits to the session's logits buffer when `logits`.
static int pdec_launch(ahip_session* s, bool logits, bool emitted) {
    if (s->pdec_launches >= (1ull << 31)) {
        HIP_OR(hipStreamSynchronize(s->stream), "decode tag wrap");
        if (int rc = pdec_reset_words(s)) return rc;
    }
    DecodeParams p = s->pdec_params;
    p.logits = logits ? s->logits.as<float>() : nullptr;
    p.emitted = emitted ? s->emitted_mapped : nullptr;
    if (s->profiling) {
        const size_t n = (size_t)(decode_trace_points(p.n_layers) + kDecodeAttnSubPoints) * s->pdec_grid;
        if (!s->pdec_trace.p)
            if (int rc = s->pdec_trace.alloc(n * 8)) return rc;
        HIP_OR(hipMemsetAsync(s->pdec_trace.p, 0, n * 8, s->stream), "clear trace");
        p.trace = s->pdec_trace.as<unsigned long long>();
    }
    PdecOrder& order = g_pdec_order[s->m->device & 63];
    std::lock_guard<std::mutex> g(order.lock);
    if (order.last && order.last != s) {
        HIP_OR(hipEventRecord(s->pdec_peer, order.last_stream), "hipEventRecord on the previous session's stream");
        HIP_OR(hipStreamWaitEvent(s->stream, s->pdec_peer, 0), "order after another session");
    }
    hipError_t le = launch_decode_step(s->pdec_fmt, p, s->pdec_grid, s->pdec_lds, s->pdec_coop, s->stream);
    if (le != hipSuccess && s->pdec_coop) {
        // Cooperative launches (ALPACA_HIP_DECODE_COOPERATIVE=1): the runtime
        // refuses them in a process while another process on the device holds
        // its cooperative-launch resource (hipErrorIllegalState).  The session
        // then launches the same kernel the ordinary way, the default mode,
        // for the rest of its life.
        hipGetLastError();
        s->pdec_coop = 0;
        le = launch_decode_step(s->pdec_fmt, p, s->pdec_grid, s->pdec_lds, 0, s->stream);
    }
    LAUNCH(le);
    order.last = s;
    order.last_stream = s->stream;
    s->pdec_launches++;
    return AHIP_OK;
}

// Stage labels of the persistent kernel's phases (the multi-kernel path's labels).
static const char* const kPhaseLabels[6] = {"qkv (fused norm)", "attention", "attention merge",
                                            "attn out projection (+residual)", "ffn gate+up+silu (fused norm)",
                                            "ffn down (+residual)"};

// Profiling: after a launch has completed, turns its phase-end stamps into
// per-stage times on the critical path (the last workgroup to end a phase ends
// it) and adds them to the call's stages.
static int pdec_collect_trace(ahip_session* s) {
    const int L = s->m->c.layer_count, P = decode_trace_points(L), G = s->pdec_grid;
    const size_t total = (size_t)(P + kDecodeAttnSubPoints) * G;
    s->pdec_trace_host.resize(total);
    HIP_OR(hipMemcpyAsync(s->pdec_trace_host.data(), s->pdec_trace.p, total * 8, hipMemcpyDeviceToHost,
                          s->stream), "trace download");
    HIP_OR(hipStreamSynchronize(s->stream), "trace download");
    const unsigned long long* t = s->pdec_trace_host.data();
    unsigned long long prev = ~0ull;
    for (int g = 0; g < G; g++)
        if (t[g]) prev = std::min(prev, t[g]);
    const double tick = 1.0 / (1000.0 * s->pdec_clock_khz);
    for (int k = 1; k < P; k++) {
        unsigned long long end = 0;
        const int n = k == P - 1 ? 1 : G;  // the arg-max runs in workgroup 0 only
        for (int g = 0; g < n; g++) end = std::max(end, t[(size_t)k * G + g]);
        const char* label = k == P - 1 ? "sample" : k == P - 2 ? "final norm + logits" : kPhaseLabels[(k - 1) % 6];
        auto& st = s->pdec_stages[label];
        st.first += end > prev ? (double)(end - prev) * tick : 0.0;
        st.second += 1;
        prev = std::max(prev, end);
    }
    return AHIP_OK;
}

// Writes the accumulated persistent-kernel stages into the session profile.
static void pdec_publish_stages(ahip_session* s) {
    s->profile.clear();
    auto add = [&](const char* label) {
        auto it = s->pdec_stages.find(label);
        if (it == s->pdec_stages.end()) return;
        ahip_stage st{};
        std::snprintf(st.label, sizeof st.label, "%s", label);
        st.seconds = it->second.first;
        st.dispatches = it->second.second;
        s->profile.push_back(st);
    };
    for (const char* l : kPhaseLabels) add(l);
    add("final norm + logits");
    add("sample");
    s->pdec_stages.clear();
}

// After the launches of a call have completed: reports an aborted launch (a
// bounded wait inside the kernel expired) and leaves the session usable.
static int pdec_check(ahip_session* s) {
    if (!s->pdec || *(volatile int*)s->pdec_status == 0) return AHIP_OK;
    pdec_reset_words(s);
    return fail(AHIP_ERR_COMMAND_FAILED, "persistent decode launch aborted: a workgroup timed out or aborted");
}

extern "C" int ahip_session_create(ahip_model* m, int capacity, int max_batch, int kv_precision, int gemm_precision,
                                   ahip_session** out) {
    if (!m || !out) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    drop_stale_error();
    if (capacity <= 0 || max_batch <= 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "capacity and maxBatch must be positive");
    if (kv_precision != AHIP_KV_F16 && kv_precision != AHIP_KV_F32) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad kv precision");
    if (gemm_precision != AHIP_GEMM_EXACT && gemm_precision != AHIP_GEMM_FAST && gemm_precision != AHIP_GEMM_FAST_F16)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "bad gemm precision");
    const ahip_llama_config& c = m->c;
    capacity = std::min(capacity, c.context_length);
    max_batch = std::min(max_batch, capacity);
    HIP_OR(hipSetDevice(m->device), "hipSetDevice");
    auto s = std::make_unique<ahip_session>();
    s->m = m;
    s->capacity = capacity;
    s->max_batch = max_batch;
    s->kv_f16 = kv_precision == AHIP_KV_F16;
    s->fast = gemm_precision != AHIP_GEMM_EXACT;
    s->two_term = gemm_precision == AHIP_GEMM_FAST;
    s->lo_terms = s->two_term ? lo_terms_for(c) : 0;
    {
        const char* r = std::getenv("ALPACA_HIP_LO_ROWS");
        s->lo_all_rows = r && !std::strcmp(r, "all");
        const char* q = std::getenv("ALPACA_HIP_QKV_LO");
        s->qkv_lo_all = s->lo_all_rows || !(q && !std::strcmp(q, "kv"));
    }
    s->fuse_qkv_rope = env_int("ALPACA_HIP_FUSE_QKV_ROPE", 1) != 0;
    s->exact_last_row = s->two_term && env_int("ALPACA_HIP_EXACT_LAST_ROW", 1) != 0;
    if (s->exact_last_row) {
        if (int rc = s->last_arrive.alloc((size_t)c.head_count * 4)) return rc;
        if (int rc = s->last_part.alloc(flash_last_part_floats(c.head_count, c.head_dim) * 4)) return rc;
        HIP_OR(hipMemset(s->last_arrive.p, 0, (size_t)c.head_count * 4), "hipMemset");
    }
    {
        const char* a = std::getenv("ALPACA_HIP_PREFILL_ATTENTION");
        const char* g = std::getenv("ALPACA_HIP_PREFILL_GEMM");
        s->prefill_generic_attention = a && !std::strcmp(a, "generic");
        s->prefill_f32_gemm = g && !std::strcmp(g, "f32");
    }
    HIP_OR(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
    const SessionSizes z = session_sizes(c, capacity, max_batch, s->kv_f16);
    for (int l = 0; l < c.layer_count; l++) {
        s->kc.emplace_back(new DevBuf());
        s->vc.emplace_back(new DevBuf());
        if (int rc = s->kc.back()->alloc(z.kv_per_layer)) return rc;
        if (int rc = s->vc.back()->alloc(z.kv_per_layer)) return rc;
    }
    struct A { DevBuf* b; int64_t n; };
    for (A a : {A{&s->x, z.x * 4}, A{&s->xn, z.x * 4}, A{&s->xh, z.x * 4}, A{&s->qkv, z.qkv * 4}, A{&s->qh, z.q16 * 4},
                A{&s->ctx, z.ctx * 4}, A{&s->ctxh, z.ctx * 4}, A{&s->ffn, z.ffn * 4}, A{&s->ffnh, z.ffn * 4},
                A{&s->partials, z.partials * 4}, A{&s->logits, z.logits * 4}, A{&s->tokens, (int64_t)capacity * 4},
                A{&s->chain, 64}, A{&s->dpos, 64}})
        if (int rc = a.b->alloc(a.n)) return rc;
    if (hipHostMalloc((void**)&s->logits_host, (size_t)c.vocab_size * 4, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void**)&s->emitted_host, ((size_t)capacity + 8) * 4, hipHostMallocMapped) != hipSuccess ||
        hipHostMalloc((void**)&s->tokens_host, ((size_t)capacity + 8) * 4, hipHostMallocDefault) != hipSuccess)
        return fail(AHIP_ERR_ALLOC, "pinned host allocation failed");
    HIP_OR(hipHostGetDevicePointer((void**)&s->emitted_mapped, s->emitted_host, 0), "hipHostGetDevicePointer");
    s->dec_split = attention_decode_supported(c.head_count, c.kv_head_count, c.head_dim) &&
                   attention_decode_session_split_len(capacity, c.head_count, c.kv_head_count) > 0;
    if (s->dec_split) {
        s->dec_split_len = attention_decode_session_split_len(capacity, c.head_count, c.kv_head_count);
        s->dec_splits = (capacity + s->dec_split_len - 1) / s->dec_split_len;
    }
    if (int rc = setup_persistent_decode(s.get())) return rc;
    HIP_OR(hipEventCreate(&s->ev_begin), "hipEventCreate");
    HIP_OR(hipEventCreate(&s->ev_end), "hipEventCreate");
    m->refs.fetch_add(1);
    *out = s.release();
    return AHIP_OK;
}

extern "C" int ahip_session_destroy(ahip_session* s) {
    if (!s) return AHIP_OK;
    hipSetDevice(s->m->device);
    {
        PdecOrder& order = g_pdec_order[s->m->device & 63];
        std::lock_guard<std::mutex> g(order.lock);
        if (order.last == s) {
            order.last = nullptr;
            order.last_stream = nullptr;
        }
    }
    ahip_model* m = s->m;
    delete s;
    drop_stale_error();
    model_release(m);
    return AHIP_OK;
}

// Single-flight guard (MetalLlamaModel.swift:235, :275).
struct BusyGuard {
    ahip_session* s;
    bool ok;
    explicit BusyGuard(ahip_session* s_) : s(s_) {
        int expected = 0;
        ok = s->busy.compare_exchange_strong(expected, 1);
    }
    ~BusyGuard() {
        if (ok) s->busy.store(0);
    }
};


// One decoder layer for a single token (the fused decode path,
// MetalLlamaModel.swift:344-356): 5 launches -- QKV GEMV with RMSNorm prologue
// and RoPE + KV-store epilogue; split-K attention; Wo GEMV merging the splits
// and adding the residual; gate/up GEMV with RMSNorm prologue and SwiGLU
// epilogue; down GEMV adding the residual.  The position is `pos`, or *pos_dev
// when pos_dev is set (the greedy chain advances it on the device).
static int encode_decode_layer(ahip_session* s, int li, int pos, const int* pos_dev) {
    ahip_model* m = s->m;
    const ahip_llama_config& c = m->c;
    const int hd = c.head_dim, LDQKV = (c.head_count + 2 * c.kv_head_count) * hd;
    hipStream_t st = s->stream;
    ahip_model::Layer& L = *m->layers[li];
    float* x = s->x.as<float>();
    float* qkv = s->qkv.as<float>();
    void* kc = s->kc[li]->p;
    void* vc = s->vc[li]->p;
    s->stage("qkv (fused norm)");
    GemvInput in;
    in.x = x;
    in.norm = L.attn_norm.as<float>();
    in.eps = c.rms_norm_eps;
    GemvRope rope;
    rope.table = m->rope.as<float2>();
    rope.heads = c.head_count;
    rope.kv_heads = c.kv_head_count;
    rope.hd = hd;
    rope.capacity = s->capacity;
    rope.pos = pos;
    rope.pos_dev = pos_dev;
    rope.kc = kc;
    rope.vc = vc;
    rope.kv_f16 = s->kv_f16;
    LAUNCH(launch_gemv_ex(L.qkv.m, nullptr, in, &rope, qkv, GEMV_QKV_ROPE, st));
    s->stage("attention");
    GemvInput att;
    if (s->dec_split) {
        // eager calls launch only the splits the context covers; graph replays cover the capacity
        const int splits = pos_dev ? s->dec_splits : (pos + s->dec_split_len) / s->dec_split_len;
        LAUNCH(launch_attention_decode(qkv, kc, vc, s->kv_f16, s->capacity, c.head_count, c.kv_head_count, hd, pos + 1,
                                       pos_dev, s->dec_split_len, splits, s->partials.as<float>(), st));
        att.partials = s->partials.as<float>();
        att.heads = c.head_count;
        att.splits = splits;
        att.hd = hd;
        att.split_len = s->dec_split_len;
        att.pos_dev = pos_dev;
    } else {
        if (pos_dev) return fail(AHIP_ERR_UNSUPPORTED, "device-positioned decode needs the split-K attention kernel");
        const int splits = attention_splits(pos + 1, c.head_count, 1);
        LAUNCH(launch_attention_generic(qkv, LDQKV, kc, vc, s->kv_f16, s->capacity, 1, c.head_count, c.kv_head_count,
                                        hd, pos, splits, s->partials.as<float>(), s->ctx.as<float>(), st));
        att.x = s->ctx.as<float>();
    }
    s->stage("attn out projection (+residual)");
    // A Wo large enough for the streamed GEMV takes the merged context row from
    // its own kernel: folded into Wo's input stage, every workgroup would read
    // all heads' partials (the 1.7B shape: 16.2 us against 4.7 + 4.8 us).
    if (att.partials && gemv_streams(L.wo.m)) {
        LAUNCH(launch_attention_merge(att.partials, c.head_count, hd, att.splits, s->ctx.as<float>(), st));
        LAUNCH(launch_gemv(L.wo.m, nullptr, s->ctx.as<float>(), nullptr, 0.f, x, GEMV_ADD, st));
    } else {
        LAUNCH(launch_gemv_ex(L.wo.m, nullptr, att, nullptr, x, GEMV_ADD, st));
    }
    s->stage("ffn gate+up+silu (fused norm)");
    LAUNCH(launch_gemv(L.gate.m, &L.up.m, x, L.ffn_norm.as<float>(), c.rms_norm_eps, s->ffn.as<float>(), GEMV_SWIGLU,
                       st));
    s->stage("ffn down (+residual)");
    LAUNCH(launch_gemv(L.down.m, nullptr, s->ffn.as<float>(), nullptr, 0.f, x, GEMV_ADD, st));
    return AHIP_OK;
}

// Enqueues one chunk of `n` tokens at absolute position `pos` (encodeChunk,
// MetalLlamaModel.swift:307-384).  Tokens are read from device memory.
// One layer of the fast (MFMA) prefill for the n tokens at activation rows
// [row0, row0 + n) and positions [pos, pos + n), on stream st.  after_qkv (if
// set) is recorded once these rows' K/V are in the cache; the attention first
// waits for the n_before events of before_attn (earlier rows' K/V).
// `last`: these rows end with the row whose logits the call returns.
// Which of a layer's Wo, gate/up and down GEMMs over n rows take the returned
// row as a float32 GEMV (encode_mfma_layer): from 2,048 rows, those with at
// least 2M weights (gate and up together).  The GEMV is one more launch of
// 3-10 us in the layer's chain; the tail rows' second terms it replaces cost
// more only on large GEMMs.  Measured 4096-token prefills (two halves of 2,048
// rows at the 135M and 360M shapes, one stream at the 1.7B shape), tok/s with
// no GEMV -> this rule: 360M 520k -> 564-579k, 1.7B 149k -> 163k; every GEMV on
// the 135M shape 1,023-1,035k -> 951-956k, at the 360M shape over 2,048 tokens
// (halves of 1,024 rows) 467-472k -> 406-412k.
// ALPACA_HIP_LAST_ROW_GEMV (read per call): a mask of kSide* bits instead.
enum : int { kSideWo = 1, kSideGateUp = 2, kSideDown = 4 };
static int last_row_gemv_mask(const ahip_model::Layer& L, int n) {
    const int forced = env_int("ALPACA_HIP_LAST_ROW_GEMV", -1);
    if (forced >= 0) return forced & 7;
    if (n < 2048) return 0;
    auto weights = [](const DevMatrix& w) { return (int64_t)w.rows * w.cols; };
    const int64_t lim = 1 << 21;
    return (weights(L.wo.m) >= lim ? kSideWo : 0) |
           (weights(L.gate.m) + weights(L.up.m) >= lim ? kSideGateUp : 0) | (weights(L.down.m) >= lim ? kSideDown : 0);
}

static int encode_mfma_layer(ahip_session* s, int li, int row0, int n, int pos, bool flash, bool last, hipStream_t st,
                             hipEvent_t after_qkv, const hipEvent_t* before_attn = nullptr, int n_before = 0) {
    ahip_model* m = s->m;
    const ahip_llama_config& c = m->c;
    const int H = c.hidden_size, QW = c.head_count * c.head_dim, KW = c.kv_head_count * c.head_dim,
              F = c.feed_forward_size, hd = c.head_dim, LDQKV = QW + 2 * KW;
    const int64_t B = s->max_batch, r = row0;
    ahip_model::Layer& L = *m->layers[li];
    void* kc = s->kc[li]->p;
    void* vc = s->vc[li]->p;
    const float2* rope = m->rope.as<float2>();
    float* x = s->x.as<float>() + r * H;
    float* qkv = s->qkv.as<float>() + r * LDQKV;
    f16* xh = s->xh.as<f16>() + r * H;
    f16* qh = s->qh.as<f16>() + r * QW;
    f16* ctxh = s->ctxh.as<f16>() + r * QW;
    f16* ffnh = s->ffnh.as<f16>() + r * F;
    // Second-term planes of the f16 activation buffers (two-term prefill),
    // after the first planes; null where the operand takes one term (the
    // producer then writes no second term and the consumer reads none).
    // The QKV input keeps its second term on every row: k and v go to the
    // cache, which every later position reads.  The other operands (Wo,
    // gate/up and down inputs, attention's Q and P) carry it only where the
    // returned logits depend on them row by row: on the rows [tail0, n) of a
    // call's last rows, tail0 being the last row rounded down to a multiple of
    // 256.  Tiles (at most 256 rows, starting at multiples of their height)
    // and 64-query blocks then either lie wholly in that range or wholly
    // before it, so the same rows take two terms whatever tile a GEMM picks.
    // With lo_all_rows every row takes them.
    const int lo = s->two_term ? s->lo_terms : 0;
    const bool all = s->lo_all_rows;
    const int tail0 = all ? 0 : last ? (n - 1) / 256 * 256 : n;
    const int lo_tile = tail0;
    auto want = [&](int bit) { return (lo & bit) && (all || last); };
    f16* xhlo_qkv = lo & kLoQkv ? s->xh.as<f16>() + B * H + r * H : nullptr;
    f16* xhlo_ffn = want(kLoGateUp) ? s->xh.as<f16>() + B * H + r * H : nullptr;
    f16* qhlo = want(kLoQ) ? s->qh.as<f16>() + B * QW + r * QW : nullptr;
    f16* ctxhlo = want(kLoWo) ? s->ctxh.as<f16>() + B * QW + r * QW : nullptr;
    f16* ffnhlo = want(kLoDown) ? s->ffnh.as<f16>() + B * F + r * F : nullptr;
    const int p_terms = want(kLoP) ? 2 : 1;
    float* ctx = s->ctx.as<float>() + r * QW;
    s->stage("rmsnorm");
    LAUNCH(launch_rmsnorm(x, L.attn_norm.as<float>(), nullptr, xh, xhlo_qkv, n, H, c.rms_norm_eps, st));
    s->stage("qkv projections");
    hipError_t fused = hipErrorNotSupported;
    if (flash && s->fuse_qkv_rope) {
        // RoPE and the KV append in the GEMM epilogue (q/k/v never reach HBM as f32)
        QkvRope o;
        o.rope = rope;
        o.qh = qh;
        o.qlo = qhlo;
        o.kc = (f16*)kc;
        o.vc = (f16*)vc;
        o.heads = c.head_count;
        o.kv_heads = c.kv_head_count;
        o.hd = hd;
        o.pos = pos;
        o.capacity = s->capacity;
        // k and v take the second term on every row; q too unless ALPACA_HIP_QKV_LO=kv (read at
        // session creation), which keeps it to the tail rows: 1% faster at the 1.7B shape, and
        // the 135M shape's logit error 0.13 -> 0.20 of the bound, so it is off by default
        fused = launch_gemm_qkv_rope(xh, xhlo_qkv, H, n, L.pre(L.qkv, L.qkv16), o, st, s->qkv_lo_all ? 0 : tail0,
                                     tail0, s->qkv_lo_all ? 0 : QW);
        if (fused != hipErrorNotSupported) LAUNCH(fused);
    }
    if (fused == hipErrorNotSupported) {
        LAUNCH(launch_gemm_mfma(xh, xhlo_qkv, H, n, L.pre(L.qkv, L.qkv16), nullptr, qkv, nullptr, nullptr, LDQKV,
                                GEMM_STORE, st));
        s->stage("rope + kv store");
        LAUNCH(launch_rope_store(qkv, LDQKV, n, c.head_count, c.kv_head_count, hd, pos, rope, 1, flash ? 0 : 1,
                                 flash ? qh : nullptr, flash ? qhlo : nullptr, kc, vc, s->kv_f16, s->capacity, st));
    }
    if (after_qkv) HIP_OR(hipEventRecord(after_qkv, st), "hipEventRecord");
    for (int k = 0; k < n_before; k++) HIP_OR(hipStreamWaitEvent(st, before_attn[k], 0), "hipStreamWaitEvent");
    s->stage("attention");
    if (flash) {
        // Past the first 256 rows the last row, whose logits the call returns, is
        // computed in float32 by workgroups of its own (q as its two f16 terms)
        // while the query blocks take one f16 term of Q and P
        // (ALPACA_HIP_EXACT_LAST_ROW=0: instead Q and P take their second terms in
        // the last row's query block, the longest of the causal walk, where the
        // doubled MFMA work sets the kernel's time).  Shorter calls keep the second
        // terms on the whole block: there the other rows of the block are most of
        // the K/V rows later tokens read (a 40-token prompt of a 256-wide model
        // with weights of standard deviation 0.1 then missed the logit bound by a
        // decode step).  With second terms on every row, every block takes them.
        const bool exact_last = !all && qhlo && s->exact_last_row && tail0 > 0;
        LAUNCH(launch_flash_attention(qh, qhlo, QW, (const f16*)kc, (const f16*)vc, s->capacity, n, c.head_count,
                                      c.kv_head_count, hd, pos, nullptr, ctxh, ctxhlo, st, p_terms,
                                      all ? 0 : n - 1, tail0, exact_last ? s->last_arrive.as<unsigned>() : nullptr,
                                      exact_last ? s->last_part.as<float>() : nullptr));
    } else {
        LAUNCH(launch_attention_generic(qkv, LDQKV, kc, vc, s->kv_f16, s->capacity, n, c.head_count, c.kv_head_count,
                                        hd, pos, 1, nullptr, ctx, st));
        LAUNCH(launch_f32_to_f16(ctx, ctxh, ctxhlo, (int64_t)n * QW, st));
    }
    // Wo, gate/up and down: the returned row either takes the second term of
    // its input inside the GEMM (with the tail rows from tail0, whose tiles then
    // run twice the MFMA work), or (last_row_gemv, past the first 256 rows as
    // for attention) the GEMM covers rows [0, n - 1) with one term and the last
    // row is a float32 GEMV over its two f16 terms (launch_gemv_pair): one more
    // launch against the tail tiles' second terms, which set the time of GEMMs
    // over about one round of workgroups and add a sixteenth of the work of
    // larger ones.
    const int side = (!all && last && tail0 > 0) ? last_row_gemv_mask(L, n) : 0;
    const int64_t lr = n - 1;  // the last row
    s->stage("attn out projection (+residual)");
    const DevMatrix& wo = L.pre(L.wo, L.wo16);
    if ((side & kSideWo) && ctxhlo) {
        LAUNCH(launch_gemm_mfma(ctxh, nullptr, QW, n - 1, wo, nullptr, x, nullptr, nullptr, H, GEMM_ACC, st));
        LAUNCH(launch_gemv_pair(wo, nullptr, ctxh + lr * QW, ctxhlo + lr * QW, x + lr * H, nullptr, nullptr, GEMV_ADD,
                                st));
    } else {
        LAUNCH(launch_gemm_mfma(ctxh, ctxhlo, QW, n, wo, nullptr, x, nullptr, nullptr, H, GEMM_ACC, st, lo_tile));
    }
    s->stage("rmsnorm");
    LAUNCH(launch_rmsnorm(x, L.ffn_norm.as<float>(), nullptr, xh, xhlo_ffn, n, H, c.rms_norm_eps, st, tail0));
    s->stage("ffn gate+up+silu");
    const DevMatrix &wg = L.pre(L.gate, L.gate16), &wu = L.pre(L.up, L.up16);
    if ((side & kSideGateUp) && xhlo_ffn && ffnhlo) {
        LAUNCH(launch_gemm_mfma(xh, nullptr, H, n - 1, wg, &wu, nullptr, ffnh, ffnhlo, F, GEMM_SWIGLU, st, 0, tail0));
        LAUNCH(launch_gemv_pair(wg, &wu, xh + lr * H, xhlo_ffn + lr * H, nullptr, ffnh + lr * F, ffnhlo + lr * F,
                                GEMV_SWIGLU, st));
    } else {
        LAUNCH(launch_gemm_mfma(xh, xhlo_ffn, H, n, wg, &wu, nullptr, ffnh, ffnhlo, F, GEMM_SWIGLU, st, lo_tile, tail0));
    }
    s->stage("ffn down (+residual)");
    const DevMatrix& wd = L.pre(L.down, L.down16);
    if ((side & kSideDown) && ffnhlo) {
        LAUNCH(launch_gemm_mfma(ffnh, nullptr, F, n - 1, wd, nullptr, x, nullptr, nullptr, H, GEMM_ACC, st));
        LAUNCH(launch_gemv_pair(wd, nullptr, ffnh + lr * F, ffnhlo + lr * F, x + lr * H, nullptr, nullptr, GEMV_ADD,
                                st));
    } else {
        LAUNCH(launch_gemm_mfma(ffnh, ffnhlo, F, n, wd, nullptr, x, nullptr, nullptr, H, GEMM_ACC, st, lo_tile));
    }
    return AHIP_OK;
}

// A fast prefill chunk of at least kSplitPrefillMin tokens (unprofiled) whose
// QKV GEMM has at most two rounds of 128x64 tiles (prefill_split_pays) runs as
// two halves on two streams: the first half's layers on the session stream,
// the second's on the shared second stream, whose attention of each layer
// waits for the first half's K/V rows of that layer.  The halves' launches
// overlap on the GPU, where one half alone leaves it partly idle (the GEMMs
// and norms of such a chunk keep most waves waiting on memory).  Measured
// (same box, one stream against two): C1 at 2,048 / 3,072 / 4,096 tokens
// 702k / 726k / 795k -> 720k / 857k / 885k tok/s, C4 at 1,536 / 2,048 tokens
// 343k / 389k -> 365k / 417k; below 1,536 tokens the split lost 5-7% at every
// shape, and at the 1.7B shape, whose grids fill the device, it lost 3-6%.
// Each row goes through the same arithmetic, but a half's smaller grids may
// take other tiles than the whole chunk's: the GEMM's two-K-set 64x64 tiles
// (where a half's grid is at most one tile per CU) and the flash kernel's
// other key-range split both change the float32 summation order, so the
// halves agree with one stream to rounding (logits within 1e-5 of the peak),
// not bit for bit.
// ALPACA_HIP_PREFILL_STREAMS=1 (read per call) keeps one stream.

static int encode_split_prefill(ahip_session* s, const int32_t* dtok, int n, int pos, bool logits, bool flash,
                                int parts) {
    ahip_model* m = s->m;
    const ahip_llama_config& c = m->c;
    const int H = c.hidden_size;
    parts = std::max(2, std::min(parts, ahip_session::kMaxParts));
    s->part_stream[0] = s->stream;
    if (!s->part_start) {
        HIP_OR(hipEventCreateWithFlags(&s->part_start, hipEventDisableTiming), "hipEventCreate");
        for (int k = 0; k < ahip_session::kMaxParts; k++) {
            HIP_OR(hipEventCreateWithFlags(&s->part_qkv[k], hipEventDisableTiming), "hipEventCreate");
            HIP_OR(hipEventCreateWithFlags(&s->part_done[k], hipEventDisableTiming), "hipEventCreate");
        }
    }
    // part k: rows [r[k], r[k+1]); every boundary but the last a multiple of
    // 256, so the last part's rows that take the second terms (from the last
    // row rounded down to a multiple of 256) are those of one stream
    int r[ahip_session::kMaxParts + 1];
    for (int k = 0; k < parts; k++) r[k] = (int)((int64_t)n * k / parts / 256 * 256);
    r[parts] = n;
    HIP_OR(hipEventRecord(s->part_start, s->stream), "hipEventRecord");
    float* x = s->x.as<float>();
    int joined = 1;  // parts whose stream has waited on part_start (the session stream's own part needs none)
    auto body = [&]() -> int {
        for (int k = 0; k < parts; k++) {
            hipStream_t st = s->part_stream[k];
            if (k) {
                HIP_OR(hipStreamWaitEvent(st, s->part_start, 0), "hipStreamWaitEvent");
                joined = k + 1;
            }
            LAUNCH(launch_embed(dtok + r[k], r[k + 1] - r[k], m->embed.m, x + (int64_t)r[k] * H, st));
        }
        for (int li = 0; li < c.layer_count; li++)
            for (int k = 0; k < parts; k++)
                if (int rc = encode_mfma_layer(s, li, r[k], r[k + 1] - r[k], pos + r[k], flash,
                                               logits && k + 1 == parts, s->part_stream[k],
                                               k + 1 < parts ? s->part_qkv[k] : nullptr, s->part_qkv, k))
                    return rc;
        if (logits)
            LAUNCH(launch_gemv(m->out_matrix(), nullptr, x + (int64_t)(n - 1) * H, m->output_norm.as<float>(),
                               c.rms_norm_eps, s->logits.as<float>(), GEMV_STORE, s->part_stream[parts - 1]));
        return AHIP_OK;
    };
    const int rc = body();
    // The session stream joins every part stream that took work, also when
    // encoding failed part way: whatever was queued there reads and writes
    // the session's activations and KV cache, so later calls on the session
    // (and its teardown, which synchronises the session stream) must come
    // after it.
    for (int k = 1; k < joined; k++) {
        HIP_OR(hipEventRecord(s->part_done[k], s->part_stream[k]), "hipEventRecord");
        HIP_OR(hipStreamWaitEvent(s->stream, s->part_done[k], 0), "hipStreamWaitEvent");
    }
    return rc;
}

static int encode_chunk(ahip_session* s, const int32_t* dtok, int n, int pos, bool logits,
                        const int* pos_dev = nullptr) {
    ahip_model* m = s->m;
    const ahip_llama_config& c = m->c;
    const int H = c.hidden_size, QW = c.head_count * c.head_dim, KW = c.kv_head_count * c.head_dim,
              F = c.feed_forward_size, hd = c.head_dim, LDQKV = QW + 2 * KW;
    hipStream_t st = s->stream;
    float* x = s->x.as<float>();
    float* qkv = s->qkv.as<float>();
    const float2* rope = m->rope.as<float2>();
    const bool mfma = s->fast && n >= 16 && !s->prefill_f32_gemm;
    const bool flash = s->fast && n >= 16 && !s->prefill_generic_attention && s->kv_f16 && (hd == 64 || hd == 128);
    if (mfma && n >= env_int("ALPACA_HIP_SPLIT_MIN", kSplitPrefillMin) && !s->profiling && env_int("ALPACA_HIP_PREFILL_STREAMS", 2) >= 2 &&
        prefill_split_pays(n, QW + 2 * KW)) {
        if (!s->part_stream[1]) s->part_stream[1] = split_stream_acquire(m->device);
        if (s->part_stream[1])
            return encode_split_prefill(s, dtok, n, pos, logits, flash, env_int("ALPACA_HIP_PREFILL_STREAMS", 2));
    }
    s->stage("embed");
    LAUNCH(launch_embed(dtok, n, m->embed.m, x, st));
    // Second-term planes of the f16 activation buffers (two-term prefill), after the first planes.
    const int64_t B = s->max_batch;
    f16* qhlo = s->two_term && (s->lo_terms & kLoQ) ? s->qh.as<f16>() + B * QW : nullptr;
    for (int li = 0; li < c.layer_count; li++) {
        ahip_model::Layer& L = *m->layers[li];
        void* kc = s->kc[li]->p;
        void* vc = s->vc[li]->p;
        if (n == 1) {
            if (int rc = encode_decode_layer(s, li, pos, pos_dev)) return rc;
        } else if (mfma) {
            if (int rc = encode_mfma_layer(s, li, 0, n, pos, flash, logits, st, nullptr, nullptr)) return rc;
        } else {
            float* xn = s->xn.as<float>();
            s->stage("rmsnorm");
            LAUNCH(launch_rmsnorm(x, L.attn_norm.as<float>(), xn, nullptr, nullptr, n, H, c.rms_norm_eps, st));
            s->stage("qkv projections");
            LAUNCH(launch_gemm_f32(xn, H, n, L.qkv.m, nullptr, qkv, LDQKV, GEMM_STORE, st));
            s->stage("rope + kv store");
            LAUNCH(launch_rope_store(qkv, LDQKV, n, c.head_count, c.kv_head_count, hd, pos, rope, 1, flash ? 0 : 1,
                                     flash ? s->qh.as<f16>() : nullptr, flash ? qhlo : nullptr, kc, vc, s->kv_f16,
                                     s->capacity, st));
            s->stage("attention");
            if (flash) {
                LAUNCH(launch_flash_attention(s->qh.as<f16>(), qhlo, QW, (const f16*)kc, (const f16*)vc, s->capacity,
                                              n, c.head_count, c.kv_head_count, hd, pos, s->ctx.as<float>(), nullptr,
                                              nullptr, st, s->two_term && (s->lo_terms & kLoP) ? 2 : 1));
            } else {
                LAUNCH(launch_attention_generic(qkv, LDQKV, kc, vc, s->kv_f16, s->capacity, n, c.head_count,
                                                c.kv_head_count, hd, pos, 1, nullptr, s->ctx.as<float>(), st));
            }
            s->stage("attn out projection (+residual)");
            LAUNCH(launch_gemm_f32(s->ctx.as<float>(), QW, n, L.wo.m, nullptr, x, H, GEMM_ACC, st));
            s->stage("rmsnorm");
            LAUNCH(launch_rmsnorm(x, L.ffn_norm.as<float>(), xn, nullptr, nullptr, n, H, c.rms_norm_eps, st));
            s->stage("ffn gate+up+silu");
            LAUNCH(launch_gemm_f32(xn, H, n, L.gate.m, &L.up.m, s->ffn.as<float>(), F, GEMM_SWIGLU, st));
            s->stage("ffn down (+residual)");
            LAUNCH(launch_gemm_f32(s->ffn.as<float>(), F, n, L.down.m, nullptr, x, H, GEMM_ACC, st));
        }
    }
    if (logits) {
        // Only the final position's logits: fused norm + GEMV (MetalLlamaModel.swift:373-383).
        s->stage("final norm + logits");
        LAUNCH(launch_gemv(m->out_matrix(), nullptr, x + (int64_t)(n - 1) * H, m->output_norm.as<float>(),
                           c.rms_norm_eps, s->logits.as<float>(), GEMV_STORE, st));
    }
    return AHIP_OK;
}

static int validate_tokens(const ahip_session* s, const int32_t* tokens, int n) {
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= s->m->c.vocab_size)
            return fail(AHIP_ERR_INVALID_ARGUMENT, "token id outside vocabulary of " + std::to_string(s->m->c.vocab_size));
    return AHIP_OK;
}

extern "C" int ahip_session_forward(ahip_session* s, const int32_t* tokens, int n, const float** logits) {
    drop_stale_error();
    if (!s || !logits) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    BusyGuard guard(s);
    if (!guard.ok) return fail(AHIP_ERR_BUSY, "session is already executing a forward pass");
    if (n <= 0 || !tokens) return fail(AHIP_ERR_INVALID_ARGUMENT, "forward called with no tokens");
    if ((int64_t)s->length + n > s->capacity)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "context exhausted: " + std::to_string(s->length) + " cached + " +
                                                   std::to_string(n) + " new > capacity " + std::to_string(s->capacity));
    if (int rc = validate_tokens(s, tokens, n)) return rc;
    HIP_OR(hipSetDevice(s->m->device), "hipSetDevice");
    s->begin_call();
    const auto t0 = std::chrono::steady_clock::now();
    std::memcpy(s->tokens_host, tokens, (size_t)n * 4);
    HIP_OR(hipEventRecord(s->ev_begin, s->stream), "hipEventRecord");
    const bool persistent = n == 1 && s->pdec;
    if (persistent) {
        // one persistent launch: token in `chain`, position in `dpos`
        s->tokens_host[1] = s->length;
        HIP_OR(hipMemcpyAsync(s->chain.p, s->tokens_host, 4, hipMemcpyHostToDevice, s->stream), "token upload");
        HIP_OR(hipMemcpyAsync(s->dpos.p, s->tokens_host + 1, 4, hipMemcpyHostToDevice, s->stream), "position upload");
        if (int rc = pdec_launch(s, true, false)) {
            hipStreamSynchronize(s->stream);
            return rc;
        }
    } else {
        HIP_OR(hipMemcpyAsync(s->tokens.p, s->tokens_host, (size_t)n * 4, hipMemcpyHostToDevice, s->stream),
               "token upload");
        for (int c0 = 0; c0 < n; c0 += s->max_batch) {
            const int cn = std::min(s->max_batch, n - c0);
            if (int rc = encode_chunk(s, s->tokens.as<int32_t>() + c0, cn, s->length + c0, c0 + cn == n)) {
                hipStreamSynchronize(s->stream);
                return rc;
            }
        }
    }
    s->stage_end();
    HIP_OR(hipMemcpyAsync(s->logits_host, s->logits.p, (size_t)s->m->c.vocab_size * 4, hipMemcpyDeviceToHost, s->stream),
           "logits download");
    HIP_OR(hipEventRecord(s->ev_end, s->stream), "hipEventRecord");
    s->last_encode = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    HIP_OR(hipStreamSynchronize(s->stream), "forward");
    if (persistent)
        if (int rc = pdec_check(s)) return rc;
    float ms = 0;
    hipEventElapsedTime(&ms, s->ev_begin, s->ev_end);
    s->last_gpu = ms * 1e-3;
    if (persistent && s->profiling) {
        if (int rc = pdec_collect_trace(s)) return rc;
        pdec_publish_stages(s);
    } else {
        s->collect_profile();
    }
    s->length += n;
    s->logits_ready = true;
    *logits = s->logits_host;
    return AHIP_OK;
}

extern "C" int ahip_session_decode(ahip_session* s, int32_t token, const float** logits) {
    return ahip_session_forward(s, &token, 1, logits);
}

// One greedy step with the position and input token on the device: forward of
// the token in `chain` at position *dpos, logits, arg-max into `chain` and the
// mapped emitted[] buffer, *dpos += 1.
static int encode_greedy_step(ahip_session* s) {
    const int* dpos = s->dpos.as<int>();
    if (int rc = encode_chunk(s, s->chain.as<int32_t>(), 1, 0, true, dpos)) return rc;
    s->stage("sample");
    LAUNCH(launch_argmax(s->logits.as<float>(), s->m->c.vocab_size, s->chain.as<int32_t>(), s->emitted_mapped, 0,
                         s->dpos.as<int>(), s->stream));
    return AHIP_OK;
}

// Captures one greedy step into a HIP graph (kernel nodes only), replayed once
// per token so the host issues one launch per token instead of ~150.
static bool capture_greedy_graph(ahip_session* s) {
    if (s->greedy_graph) return true;
    if (s->graph_failed || !s->dec_split) return false;
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        s->graph_failed = true;
        return false;
    }
    const int rc = encode_greedy_step(s);
    const hipError_t e = hipStreamEndCapture(s->stream, &g);
    if (rc != AHIP_OK || e != hipSuccess || !g) {
        if (g) hipGraphDestroy(g);
        hipGetLastError();
        s->graph_failed = true;
        return false;
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (ie != hipSuccess) {
        hipGetLastError();
        s->graph_failed = true;
        return false;
    }
    s->greedy_graph = ex;
    return true;
}

extern "C" int ahip_session_decode_greedy(ahip_session* s, int32_t start, int max_steps, int depth, ahip_emit_fn emit,
                                          void* user, int* fed_out) {
    if (!s || !emit || !fed_out) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    drop_stale_error();
    BusyGuard guard(s);
    if (!guard.ok) return fail(AHIP_ERR_BUSY, "session is already executing a forward pass");
    *fed_out = 0;
    s->logits_ready = false;  // the chain does not keep its steps' logits
    if (start < 0 || start >= s->m->c.vocab_size)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "token id outside vocabulary of " + std::to_string(s->m->c.vocab_size));
    const int budget = std::min(max_steps, s->capacity - s->length);
    if (budget <= 0) return AHIP_OK;
    depth = std::max(1, std::min(depth, 8));
    if (s->pdec && s->profiling) depth = 1;  // one launch in flight: each trace is read before the next launch
    HIP_OR(hipSetDevice(s->m->device), "hipSetDevice");
    hipStream_t st = s->stream;
    // Eager launches when profiling (stage events between kernels) or when
    // the split-K attention kernel does not apply; otherwise graph replays.
    const bool use_pdec = s->pdec;
    const bool use_graph = !use_pdec && !s->profiling && capture_greedy_graph(s);
    s->begin_call();
    s->tokens_host[0] = start;
    s->tokens_host[1] = s->length;
    HIP_OR(hipMemcpyAsync(s->chain.p, s->tokens_host, 4, hipMemcpyHostToDevice, st), "chain upload");
    HIP_OR(hipMemcpyAsync(s->dpos.p, s->tokens_host + 1, 4, hipMemcpyHostToDevice, st), "position upload");
    HIP_OR(hipEventRecord(s->ev_begin, st), "hipEventRecord");
    std::vector<hipEvent_t> done(budget, nullptr);
    int submitted = 0, fed = 0, rc = AHIP_OK;
    auto submit = [&]() -> int {
        const int i = submitted;
        if (use_pdec) {
            if (int r = pdec_launch(s, false, true)) return r;
        } else if (use_graph) {
            HIP_OR(hipGraphLaunch(s->greedy_graph, st), "hipGraphLaunch");
        } else if (s->dec_split) {
            if (int r = encode_greedy_step(s)) return r;
        } else {
            // generic attention needs host-side positions
            if (int r = encode_chunk(s, s->chain.as<int32_t>(), 1, s->length + i, true)) return r;
            s->stage("sample");
            LAUNCH(launch_argmax(s->logits.as<float>(), s->m->c.vocab_size, s->chain.as<int32_t>(), s->emitted_mapped,
                                 s->length + i, nullptr, st));
        }
        done[i] = s->next_event();
        HIP_OR(hipEventRecord(done[i], st), "hipEventRecord");
        submitted++;
        return AHIP_OK;
    };
    while (submitted < std::min(depth, budget) && rc == AHIP_OK) rc = submit();
    while (rc == AHIP_OK && fed < submitted) {
        hipError_t e = hipEventSynchronize(done[fed]);
        if (e != hipSuccess) {
            rc = fail(AHIP_ERR_COMMAND_FAILED, std::string("decode step: ") + hipGetErrorString(e));
            break;
        }
        if (use_pdec && *(volatile int*)s->pdec_status) {
            rc = AHIP_ERR_COMMAND_FAILED;  // message set by pdec_check after the drain
            break;
        }
        if (use_pdec && s->profiling)
            if ((rc = pdec_collect_trace(s)) != AHIP_OK) break;
        const int32_t token = ((volatile int32_t*)s->emitted_host)[s->length + fed];
        fed++;
        if (!emit(user, token)) break;
        if (submitted < budget) rc = submit();
    }
    s->stage_end();
    HIP_OR(hipEventRecord(s->ev_end, st), "hipEventRecord");
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess && rc == AHIP_OK) rc = fail(AHIP_ERR_COMMAND_FAILED, std::string("drain: ") + hipGetErrorString(e));
    if (use_pdec && e == hipSuccess)
        if (int prc = pdec_check(s)) rc = prc;
    float ms = 0;
    hipEventElapsedTime(&ms, s->ev_begin, s->ev_end);
    s->last_gpu = ms * 1e-3;
    if (use_pdec && s->profiling) pdec_publish_stages(s);
    else s->collect_profile();
    s->length += fed;  // only tokens whose input was consumed (MetalLlamaModel.swift:265-267)
    *fed_out = fed;
    return rc;
}

extern "C" int ahip_session_reset(ahip_session* s) {
    if (!s) return fail(AHIP_ERR_INVALID_ARGUMENT, "null session");
    BusyGuard guard(s);
    if (!guard.ok) return fail(AHIP_ERR_BUSY, "session is busy");
    s->length = 0;
    s->logits_ready = false;
    return AHIP_OK;
}

// ------------------------------------------------------------------ sampling

// SamplingParameters.validate (Sampler.swift:21-25) and the draw's range.
static int check_sampling(float temperature, int top_k, float top_p, double u) {
    if (!std::isfinite(temperature) || temperature < 0)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "temperature must be finite and >= 0");
    if (top_k < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "topK must be >= 0");
    if (!(top_p > 0 && top_p <= 1)) return fail(AHIP_ERR_INVALID_ARGUMENT, "topP must be in (0, 1]");
    if (!(u >= 0 && u < 1)) return fail(AHIP_ERR_INVALID_ARGUMENT, "the draw u must be in [0, 1)");
    return AHIP_OK;
}

// One sample_kernel launch over device logits; the token comes back through a small copy.
static int run_sample(const float* dlogits, int n, float temperature, int top_k, float top_p, double u,
                      DevBuf& idx, DevBuf& prob, DevBuf& out, hipStream_t st, int32_t* token) {
    if (!idx.p)
        if (int rc = idx.alloc((size_t)n * 4)) return rc;
    if (!prob.p)
        if (int rc = prob.alloc((size_t)n * 8)) return rc;
    if (!out.p)
        if (int rc = out.alloc(8)) return rc;
    LAUNCH(launch_sample(dlogits, n, temperature, top_k, top_p, u, out.as<int32_t>(), out.as<int>() + 1,
                         idx.as<uint32_t>(), prob.as<double>(), st));
    int32_t host[2] = {0, 0};
    HIP_OR(hipMemcpyAsync(host, out.p, 8, hipMemcpyDeviceToHost, st), "sample download");
    HIP_OR(hipStreamSynchronize(st), "sample");
    if (host[1] == 1) return fail(AHIP_ERR_INVALID_ARGUMENT, "logits contain NaN");
    *token = host[0];
    return AHIP_OK;
}

extern "C" int ahip_session_sample(ahip_session* s, float temperature, int top_k, float top_p, double u,
                                   int32_t* token) {
    if (!s || !token) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    drop_stale_error();
    if (int rc = check_sampling(temperature, top_k, top_p, u)) return rc;
    BusyGuard guard(s);
    if (!guard.ok) return fail(AHIP_ERR_BUSY, "session is already executing a forward pass");
    if (!s->logits_ready) return fail(AHIP_ERR_INVALID_ARGUMENT, "no logits to sample: call forward or decode first");
    HIP_OR(hipSetDevice(s->m->device), "hipSetDevice");
    return run_sample(s->logits.as<float>(), s->m->c.vocab_size, temperature, top_k, top_p, u, s->sample_idx,
                      s->sample_p, s->sample_out, s->stream, token);
}
extern "C" int ahip_session_length(const ahip_session* s, int* v) {
    if (!s || !v) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *v = s->length;
    return AHIP_OK;
}
extern "C" int ahip_session_capacity(const ahip_session* s, int* v) {
    if (!s || !v) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *v = s->capacity;
    return AHIP_OK;
}
extern "C" int ahip_session_last_gpu_seconds(const ahip_session* s, double* v) {
    if (!s || !v) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *v = s->last_gpu;
    return AHIP_OK;
}
extern "C" int ahip_session_last_encode_seconds(const ahip_session* s, double* v) {
    if (!s || !v) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *v = s->last_encode;
    return AHIP_OK;
}
extern "C" int ahip_session_set_profiling(ahip_session* s, int enabled) {
    if (!s) return fail(AHIP_ERR_INVALID_ARGUMENT, "null session");
    s->profiling = enabled != 0;
    return AHIP_OK;
}
extern "C" int ahip_session_decode_timeline(const ahip_session* s, uint64_t* out, int64_t cap, int64_t* count,
                                            int* workgroups, double* tick_seconds) {
    if (!s || !count || !workgroups || !tick_seconds || (cap > 0 && !out))
        return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    const int64_t n = (int64_t)s->pdec_trace_host.size();
    for (int64_t i = 0; i < n && i < cap; i++) out[i] = s->pdec_trace_host[(size_t)i];
    *count = n;
    *workgroups = s->pdec ? s->pdec_grid : 0;
    *tick_seconds = s->pdec_clock_khz > 0 ? 1.0 / (1000.0 * s->pdec_clock_khz) : 0.0;
    return AHIP_OK;
}

extern "C" int ahip_session_profile(const ahip_session* s, ahip_stage* out, int cap, int* count) {
    if (!s || !count || (cap > 0 && !out)) return fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    const int n = (int)s->profile.size();
    for (int i = 0; i < n && i < cap; i++) out[i] = s->profile[i];
    *count = n;
    return AHIP_OK;
}

// ------------------------------------------------------------------ op-level API (MetalOps)

namespace {

// Runs `body` on the context stream and waits (MetalOps.run, MetalOps.swift:19-32).
struct OpRun {
    ahip_context* ctx;
    explicit OpRun(ahip_context* c) : ctx(c) { hipSetDevice(c->device); }
    int finish() {
        HIP_OR(hipStreamSynchronize(ctx->stream), "op");
        return AHIP_OK;
    }
};

int upload(DevBuf& b, const void* host, size_t bytes, hipStream_t st) {
    if (int rc = b.alloc(bytes)) return rc;
    if (bytes) HIP_OR(hipMemcpyAsync(b.p, host, bytes, hipMemcpyHostToDevice, st), "upload");
    return AHIP_OK;
}

int download(void* host, const DevBuf& b, size_t bytes, hipStream_t st) {
    if (bytes) HIP_OR(hipMemcpyAsync(host, b.p, bytes, hipMemcpyDeviceToHost, st), "download");
    HIP_OR(hipStreamSynchronize(st), "op");
    return AHIP_OK;
}

int check_matrix(int dtype, int k) {
    if (!valid_dtype(dtype)) return fail(AHIP_ERR_INVALID_ARGUMENT, "unknown dtype");
    if (dtype == AHIP_F32) return fail(AHIP_ERR_UNSUPPORTED, "f32 weight matrices (use f16, q8_0 or q4_0)");
    if (k <= 0 || k % 32 || k > 12288) return fail(AHIP_ERR_UNSUPPORTED, "K must be a positive multiple of 32 up to 12288");
    return AHIP_OK;
}

template <typename F>
int with_ctx(ahip_context* ctx, F f) {
    if (!ctx) return fail(AHIP_ERR_INVALID_ARGUMENT, "null context");
    drop_stale_error();
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    return f(ctx->stream);
}

}  // namespace

static int op_binary(ahip_context* ctx, const float* a, const float* b, int64_t n, float* out, int which) {
    if (n < 0 || (n && (!a || !out || (which != 2 && !b)))) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad buffers");
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        DevBuf da, db, dout;
        if (int rc = upload(da, a, n * 4, st)) return rc;
        if (which != 2)
            if (int rc = upload(db, b, n * 4, st)) return rc;
        if (int rc = dout.alloc(n * 4)) return rc;
        if (which == 0) LAUNCH(launch_add(da.as<float>(), db.as<float>(), dout.as<float>(), n, st));
        else if (which == 1) LAUNCH(launch_mul(da.as<float>(), db.as<float>(), dout.as<float>(), n, st));
        else if (which == 2) LAUNCH(launch_silu(da.as<float>(), dout.as<float>(), n, st));
        else LAUNCH(launch_silu_mul(da.as<float>(), db.as<float>(), dout.as<float>(), n, st));
        return download(out, dout, n * 4, st);
    });
}

extern "C" int ahip_op_add(ahip_context* ctx, const float* a, const float* b, int64_t n, float* out) {
    return op_binary(ctx, a, b, n, out, 0);
}
extern "C" int ahip_op_mul(ahip_context* ctx, const float* a, const float* b, int64_t n, float* out) {
    return op_binary(ctx, a, b, n, out, 1);
}
extern "C" int ahip_op_silu(ahip_context* ctx, const float* x, int64_t n, float* out) {
    return op_binary(ctx, x, nullptr, n, out, 2);
}
extern "C" int ahip_op_silu_mul(ahip_context* ctx, const float* g, const float* u, int64_t n, float* out) {
    return op_binary(ctx, g, u, n, out, 3);
}

extern "C" int ahip_op_rmsnorm(ahip_context* ctx, const float* x, const float* w, int rows, int dim, float eps,
                               float* out) {
    if (rows < 0 || dim <= 0 || !(eps > 0) || (rows && (!x || !w || !out)))
        return fail(AHIP_ERR_INVALID_ARGUMENT, "rmsNorm shapes");
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        DevBuf dx, dw, dout;
        if (int rc = upload(dx, x, (size_t)rows * dim * 4, st)) return rc;
        if (int rc = upload(dw, w, (size_t)dim * 4, st)) return rc;
        if (int rc = dout.alloc((size_t)rows * dim * 4)) return rc;
        LAUNCH(launch_rmsnorm(dx.as<float>(), dw.as<float>(), dout.as<float>(), nullptr, nullptr, rows, dim, eps, st));
        return download(out, dout, (size_t)rows * dim * 4, st);
    });
}

static int upload_weight(int dtype, const void* w, int n, int k, OwnedMatrix& om, hipStream_t st) {
    return upload_matrix(dtype, {{w, n}}, k, om, st);
}

// Shared by linear / linear_add / gate_up_silu (MetalOps.swift:50-105):
// m == 1 -> decode GEMV; fast and m >= 16 -> MFMA GEMM on f16 activations;
// otherwise the float32 GEMM.
static int op_project(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* w, const void* wu,
                      int n, int precision, float* y, int mode) {
    if (m <= 0 || n <= 0 || !x || !w || !y || (mode == GEMM_SWIGLU && !wu))
        return fail(AHIP_ERR_INVALID_ARGUMENT, "linear shapes");
    if (precision != AHIP_GEMM_EXACT && precision != AHIP_GEMM_FAST && precision != AHIP_GEMM_FAST_F16)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "bad precision");
    if (int rc = check_matrix(dtype, k)) return rc;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        OwnedMatrix W, U;
        if (int rc = upload_weight(dtype, w, n, k, W, st)) return rc;
        if (mode == GEMM_SWIGLU)
            if (int rc = upload_weight(dtype, wu, n, k, U, st)) return rc;
        DevBuf dx, dy;
        if (int rc = upload(dx, x, (size_t)m * k * 4, st)) return rc;
        if (mode == GEMM_ACC) {
            if (int rc = upload(dy, y, (size_t)m * n * 4, st)) return rc;
        } else if (int rc = dy.alloc((size_t)m * n * 4)) {
            return rc;
        }
        const DevMatrix* up = mode == GEMM_SWIGLU ? &U.m : nullptr;
        if (m == 1) {
            const int gm = mode == GEMM_STORE ? GEMV_STORE : mode == GEMM_ACC ? GEMV_ADD : GEMV_SWIGLU;
            LAUNCH(launch_gemv(W.m, up, dx.as<float>(), nullptr, 0.f, dy.as<float>(), gm, st));
        } else if (precision != AHIP_GEMM_EXACT && m >= 16) {
            // f16 activations: two planes (hi, lo) for the two-term default, one for FAST_F16.
            // ALPACA_HIP_OP_LO_ROW0 (read per call; a multiple of 256) has the GEMM take the
            // second term only from that row on, as the prefill does for a call's last rows.
            const bool tt = precision == AHIP_GEMM_FAST;
            const int lo_row0 = tt ? env_int("ALPACA_HIP_OP_LO_ROW0", 0) : 0;
            DevBuf xh, yh;
            if (int rc = xh.alloc((size_t)m * k * 2 * (tt ? 2 : 1))) return rc;
            f16* xlo = tt ? xh.as<f16>() + (size_t)m * k : nullptr;
            LAUNCH(launch_f32_to_f16(dx.as<float>(), xh.as<f16>(), xlo, (int64_t)m * k, st));
            if (mode == GEMM_SWIGLU) {
                if (int rc = yh.alloc((size_t)m * n * 2 * (tt ? 2 : 1))) return rc;
                f16* ylo = tt ? yh.as<f16>() + (size_t)m * n : nullptr;
                LAUNCH(launch_gemm_mfma(xh.as<f16>(), xlo, k, m, W.m, up, nullptr, yh.as<f16>(), ylo, n, mode, st,
                                        lo_row0, 0));
                // the result as the next GEMM takes it: hi + lo (two-term) or hi
                std::vector<uint16_t> h((size_t)m * n * (tt ? 2 : 1));
                if (int rc = download(h.data(), yh, h.size() * 2, st)) return rc;
                for (size_t i = 0; i < (size_t)m * n; i++)
                    y[i] = f16_bits_to_f32(h[i]) + (tt ? f16_bits_to_f32(h[(size_t)m * n + i]) : 0.f);
                return AHIP_OK;
            }
            LAUNCH(launch_gemm_mfma(xh.as<f16>(), xlo, k, m, W.m, nullptr, dy.as<float>(), nullptr, nullptr, n, mode,
                                    st, lo_row0, 0));
        } else {
            LAUNCH(launch_gemm_f32(dx.as<float>(), k, m, W.m, up, dy.as<float>(), n, mode, st));
        }
        return download(y, dy, (size_t)m * n * 4, st);
    });
}

extern "C" int ahip_op_linear(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* w, int n,
                              int precision, float* y) {
    return op_project(ctx, x, m, k, dtype, w, nullptr, n, precision, y, GEMM_STORE);
}
extern "C" int ahip_op_linear_add(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* w, int n,
                                  int precision, float* residual) {
    return op_project(ctx, x, m, k, dtype, w, nullptr, n, precision, residual, GEMM_ACC);
}
extern "C" int ahip_op_gate_up_silu(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* wg,
                                    const void* wu, int n, int precision, float* out) {
    return op_project(ctx, x, m, k, dtype, wg, wu, n, precision, out, GEMM_SWIGLU);
}

extern "C" int ahip_op_rope(ahip_context* ctx, float* x, int tokens, int heads, int hd, int start, float theta,
                            int interleaved) {
    if (tokens < 0 || heads <= 0 || hd <= 0 || hd % 2 || start < 0 || !(theta > 0) || (tokens && !x))
        return fail(AHIP_ERR_INVALID_ARGUMENT, "rope shape");
    if (tokens == 0) return AHIP_OK;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        auto table = rope_table(start + tokens, hd, theta);
        DevBuf dt, dx;
        if (int rc = upload(dt, table.data(), table.size() * sizeof(float2), st)) return rc;
        const size_t bytes = (size_t)tokens * heads * hd * 4;
        if (int rc = upload(dx, x, bytes, st)) return rc;
        LAUNCH(launch_rope_store(dx.as<float>(), heads * hd, tokens, heads, 0, hd, start, dt.as<float2>(),
                                 interleaved ? 1 : 0, 1, nullptr, nullptr, nullptr, nullptr, 1, 0, st));
        return download(x, dx, bytes, st);
    });
}

extern "C" int ahip_op_attention(ahip_context* ctx, const float* q, int tokens, int heads, int hd, const float* keys,
                                 const float* values, int capacity, int kv_heads, int start, int kv_precision,
                                 int precision, float* out) {
    if (tokens <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || hd <= 0 || start < 0 ||
        start + tokens > capacity || !q || !keys || !values || !out)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "attention shapes");
    if (hd % 32 || hd > 256) return fail(AHIP_ERR_INVALID_ARGUMENT, "head dimension must be a multiple of 32 up to 256");
    const bool f16kv = kv_precision == AHIP_KV_F16;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        // Cache rows [capacity][kv_heads][hd] -> [kv_heads][capacity][hd] in the cache format.
        const size_t ne = (size_t)capacity * kv_heads * hd;
        std::vector<uint8_t> kb(ne * (f16kv ? 2 : 4)), vb(ne * (f16kv ? 2 : 4));
        for (int p = 0; p < capacity; p++)
            for (int h = 0; h < kv_heads; h++)
                for (int d = 0; d < hd; d++) {
                    const size_t src = ((size_t)p * kv_heads + h) * hd + d, dst = ((size_t)h * capacity + p) * hd + d;
                    if (f16kv) {
                        ((uint16_t*)kb.data())[dst] = f32_to_f16_bits(keys[src]);
                        ((uint16_t*)vb.data())[dst] = f32_to_f16_bits(values[src]);
                    } else {
                        ((float*)kb.data())[dst] = keys[src];
                        ((float*)vb.data())[dst] = values[src];
                    }
                }
        DevBuf dk, dv, dout, dq;
        if (int rc = upload(dk, kb.data(), kb.size(), st)) return rc;
        if (int rc = upload(dv, vb.data(), vb.size(), st)) return rc;
        const size_t qn = (size_t)tokens * heads * hd;
        if (int rc = dout.alloc(qn * 4)) return rc;
        if (precision != AHIP_GEMM_EXACT && f16kv && tokens >= 16 && (hd == 64 || hd == 128)) {
            // q as one f16 term (FAST_F16) or two (hi, then lo = f16(q - hi))
            const bool tt = precision == AHIP_GEMM_FAST;
            std::vector<uint16_t> qh(qn * (tt ? 2 : 1));
            for (size_t i = 0; i < qn; i++) {
                qh[i] = f32_to_f16_bits(q[i]);
                if (tt) qh[qn + i] = f32_to_f16_bits(q[i] - f16_bits_to_f32(qh[i]));
            }
            if (int rc = upload(dq, qh.data(), qh.size() * 2, st)) return rc;
            LAUNCH(launch_flash_attention(dq.as<f16>(), tt ? dq.as<f16>() + qn : nullptr, heads * hd, dk.as<f16>(),
                                          dv.as<f16>(), capacity, tokens, heads, kv_heads, hd, start, dout.as<float>(),
                                          nullptr, nullptr, st));
        } else if (tokens == 1 && attention_decode_supported(heads, kv_heads, hd) &&
                   attention_decode_session_split_len(capacity, heads, kv_heads) > 0) {
            if (int rc = upload(dq, q, qn * 4, st)) return rc;
            const int sl = attention_decode_session_split_len(capacity, heads, kv_heads), splits = (start + sl) / sl;
            DevBuf part;
            if (int rc = part.alloc((size_t)heads * splits * (hd + 2) * 4)) return rc;
            LAUNCH(launch_attention_decode(dq.as<float>(), dk.p, dv.p, f16kv, capacity, heads, kv_heads, hd, start + 1,
                                           nullptr, sl, splits, part.as<float>(), st));
            LAUNCH(launch_attention_merge(part.as<float>(), heads, hd, splits, dout.as<float>(), st));
        } else {
            if (int rc = upload(dq, q, qn * 4, st)) return rc;
            const int splits = attention_splits(start + tokens, heads, tokens);
            DevBuf part;
            if (int rc = part.alloc(attention_partial_floats(heads, tokens, splits, hd) * 4)) return rc;
            LAUNCH(launch_attention_generic(dq.as<float>(), heads * hd, dk.p, dv.p, f16kv, capacity, tokens, heads,
                                            kv_heads, hd, start, splits, part.as<float>(), dout.as<float>(), st));
        }
        return download(out, dout, qn * 4, st);
    });
}

extern "C" int ahip_op_embed(ahip_context* ctx, const int32_t* tokens, int count, int dtype, const void* table,
                             int vocab, int dim, float* out) {
    if (count < 0 || vocab <= 0 || dim <= 0 || !table || (count && (!tokens || !out)))
        return fail(AHIP_ERR_INVALID_ARGUMENT, "embedding table");
    if (!valid_dtype(dtype)) return fail(AHIP_ERR_INVALID_ARGUMENT, "unknown dtype");
    if (dtype == AHIP_F32) return fail(AHIP_ERR_UNSUPPORTED, "f32 embedding tables");
    if (dim % 32) return fail(AHIP_ERR_UNSUPPORTED, "embedding width must be a multiple of 32");
    for (int i = 0; i < count; i++)
        if (tokens[i] < 0 || tokens[i] >= vocab) return fail(AHIP_ERR_INVALID_ARGUMENT, "token id outside vocabulary");
    if (count == 0) return AHIP_OK;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        OwnedMatrix T;
        if (int rc = upload_weight(dtype, table, vocab, dim, T, st)) return rc;
        DevBuf dt, dout;
        if (int rc = upload(dt, tokens, (size_t)count * 4, st)) return rc;
        if (int rc = dout.alloc((size_t)count * dim * 4)) return rc;
        LAUNCH(launch_embed(dt.as<int32_t>(), count, T.m, dout.as<float>(), st));
        return download(out, dout, (size_t)count * dim * 4, st);
    });
}

extern "C" int ahip_op_dequantize(ahip_context* ctx, int dtype, const void* src, int64_t elements, float* out) {
    if (!valid_dtype(dtype) || dtype == AHIP_F32) return fail(AHIP_ERR_INVALID_ARGUMENT, "dequantize: f16, q8_0 or q4_0");
    if (elements < 0 || (elements && (!src || !out))) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad buffers");
    if (elements % 32) return fail(AHIP_ERR_INVALID_ARGUMENT, "element count must be a multiple of 32");
    if (elements == 0) return AHIP_OK;
    if (elements / 32 > (int64_t)1 << 30) return fail(AHIP_ERR_UNSUPPORTED, "too many elements");
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        OwnedMatrix M;
        if (int rc = upload_weight(dtype, src, (int)(elements / 32), 32, M, st)) return rc;
        DevBuf dout;
        if (int rc = dout.alloc(elements * 4)) return rc;
        LAUNCH(launch_dequant(M.m, dout.as<float>(), st));
        return download(out, dout, elements * 4, st);
    });
}

extern "C" int ahip_op_sample(ahip_context* ctx, const float* logits, int n, float temperature, int top_k,
                              float top_p, double u, int32_t* token) {
    if (n <= 0 || !logits || !token) return fail(AHIP_ERR_INVALID_ARGUMENT, "cannot sample from empty logits");
    if (int rc = check_sampling(temperature, top_k, top_p, u)) return rc;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        DevBuf dl, idx, prob, out;
        if (int rc = upload(dl, logits, (size_t)n * 4, st)) return rc;
        return run_sample(dl.as<float>(), n, temperature, top_k, top_p, u, idx, prob, out, st, token);
    });
}

extern "C" int ahip_op_argmax(ahip_context* ctx, const float* logits, int n, int32_t* index) {
    if (n <= 0 || !logits || !index) return fail(AHIP_ERR_INVALID_ARGUMENT, "empty logits");
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        DevBuf dl, di;
        if (int rc = upload(dl, logits, (size_t)n * 4, st)) return rc;
        if (int rc = di.alloc(4)) return rc;
        LAUNCH(launch_argmax(dl.as<float>(), n, di.as<int32_t>(), nullptr, 0, nullptr, st));
        return download(index, di, 4, st);
    });
}

// ------------------------------------------------------------------ thin HIP shim

extern "C" int ahip_malloc(ahip_context* ctx, int64_t bytes, void** dptr) {
    if (!ctx || !dptr || bytes < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    if (hipMalloc(dptr, std::max<int64_t>(bytes, 256)) != hipSuccess)
        return fail(AHIP_ERR_ALLOC, "failed to allocate a " + std::to_string(bytes) + "-byte device buffer");
    return AHIP_OK;
}
extern "C" int ahip_free(ahip_context* ctx, void* dptr) {
    if (!ctx) return fail(AHIP_ERR_INVALID_ARGUMENT, "null context");
    if (dptr) HIP_OR(hipFree(dptr), "hipFree");
    return AHIP_OK;
}
extern "C" int ahip_memcpy_htod(ahip_context* ctx, void* dst, const void* src, int64_t bytes) {
    if (!ctx || bytes < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    HIP_OR(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "memcpy");
    HIP_OR(hipStreamSynchronize(ctx->stream), "memcpy");
    return AHIP_OK;
}
extern "C" int ahip_memcpy_dtoh(ahip_context* ctx, void* dst, const void* src, int64_t bytes) {
    if (!ctx || bytes < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    HIP_OR(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "memcpy");
    HIP_OR(hipStreamSynchronize(ctx->stream), "memcpy");
    return AHIP_OK;
}
extern "C" int ahip_memset(ahip_context* ctx, void* dst, int value, int64_t bytes) {
    if (!ctx || bytes < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    HIP_OR(hipMemsetAsync(dst, value, bytes, ctx->stream), "memset");
    HIP_OR(hipStreamSynchronize(ctx->stream), "memset");
    return AHIP_OK;
}
extern "C" int ahip_synchronize(ahip_context* ctx) {
    if (!ctx) return fail(AHIP_ERR_INVALID_ARGUMENT, "null context");
    HIP_OR(hipStreamSynchronize(ctx->stream), "synchronize");
    return AHIP_OK;
}

extern "C" int ahip_dev_pack_weight(ahip_context* ctx, int dtype, const void* host_w, int rows, int cols, void** handle) {
    if (!ctx || !host_w || !handle || rows <= 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    if (int rc = check_matrix(dtype, cols)) return rc;
    return with_ctx(ctx, [&](hipStream_t st) -> int {
        auto om = std::make_unique<OwnedMatrix>();
        if (int rc = upload_weight(dtype, host_w, rows, cols, *om, st)) return rc;
        *handle = om.release();
        return AHIP_OK;
    });
}
extern "C" int ahip_dev_weight_free(ahip_context* ctx, void* handle) {
    if (!ctx) return fail(AHIP_ERR_INVALID_ARGUMENT, "null context");
    hipSetDevice(ctx->device);
    delete (OwnedMatrix*)handle;
    return AHIP_OK;
}

template <typename F>
static int time_launches(ahip_context* ctx, int iters, double* avg, F launch) {
    drop_stale_error();
    hipStream_t st = ctx->stream;
    hipEvent_t a, b;
    HIP_OR(hipEventCreate(&a), "hipEventCreate");
    HIP_OR(hipEventCreate(&b), "hipEventCreate");
    int rc = AHIP_OK;
    hipEventRecord(a, st);
    for (int i = 0; i < iters && rc == AHIP_OK; i++) {
        hipError_t e = launch(st);
        if (e != hipSuccess) rc = fail(AHIP_ERR_COMMAND_FAILED, std::string("kernel launch: ") + hipGetErrorString(e));
    }
    hipEventRecord(b, st);
    hipError_t e = hipEventSynchronize(b);
    if (e != hipSuccess && rc == AHIP_OK) rc = fail(AHIP_ERR_COMMAND_FAILED, hipGetErrorString(e));
    float ms = 0;
    hipEventElapsedTime(&ms, a, b);
    if (avg) *avg = iters > 0 ? ms * 1e-3 / iters : 0.0;
    hipEventDestroy(a);
    hipEventDestroy(b);
    return rc;
}

extern "C" int ahip_dev_gemv(ahip_context* ctx, void* weight, const float* dx, float* dy, int iters, double* avg) {
    if (!ctx || !weight || !dx || !dy || iters < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    const DevMatrix& w = ((OwnedMatrix*)weight)->m;
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    return time_launches(ctx, iters, avg, [&](hipStream_t st) {
        return launch_gemv(w, nullptr, dx, nullptr, 0.f, dy, GEMV_STORE, st);
    });
}

extern "C" int ahip_dev_gemv_cycle(ahip_context* ctx, void* const* weights, int count, const float* dx, float* dy,
                                   int iters, double* avg) {
    if (!ctx || !weights || count <= 0 || !dx || !dy || iters < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    for (int k = 0; k < count; k++)
        if (!weights[k]) return fail(AHIP_ERR_INVALID_ARGUMENT, "null weight");
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    int i = 0;
    return time_launches(ctx, iters, avg, [&](hipStream_t st) {
        const DevMatrix& w = ((OwnedMatrix*)weights[i++ % count])->m;
        return launch_gemv(w, nullptr, dx, nullptr, 0.f, dy, GEMV_STORE, st);
    });
}

extern "C" int ahip_dev_attention_decode(ahip_context* ctx, const float* dq, const void* dkc, const void* dvc,
                                         int capacity, int length, int heads, int kv_heads, int hd, float* dout,
                                         int iters, double* avg) {
    if (!ctx || !dq || !dkc || !dvc || !dout || length <= 0 || length > capacity || kv_heads <= 0 ||
        heads % kv_heads || iters < 0)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    const int sl = attention_decode_supported(heads, kv_heads, hd)
                       ? attention_decode_session_split_len(capacity, heads, kv_heads) : 0;
    if (sl <= 0) return fail(AHIP_ERR_UNSUPPORTED, "decode attention shape");
    const int splits = (length - 1 + sl) / sl;
    DevBuf part;
    if (int rc = part.alloc((size_t)heads * splits * (hd + 2) * 4)) return rc;
    return time_launches(ctx, iters, avg, [&](hipStream_t st) {
        hipError_t e = launch_attention_decode(dq, dkc, dvc, 1, capacity, heads, kv_heads, hd, length, nullptr, sl,
                                               splits, part.as<float>(), st);
        if (e != hipSuccess) return e;
        return launch_attention_merge(part.as<float>(), heads, hd, splits, dout, st);
    });
}

extern "C" int ahip_dev_gemm(ahip_context* ctx, void* weight, const float* dx, int m, float* dy, int precision,
                             int iters, double* avg) {
    if (!ctx || !weight || !dx || !dy || m <= 0 || iters < 0) return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    const DevMatrix& w = ((OwnedMatrix*)weight)->m;
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    if (precision == AHIP_GEMM_FAST || precision == AHIP_GEMM_FAST_F16) {
        const bool tt = precision == AHIP_GEMM_FAST;
        const size_t e = (size_t)m * w.cols;
        DevBuf xh;
        if (int rc = xh.alloc(e * 2 * (tt ? 2 : 1))) return rc;
        f16* xlo = tt ? xh.as<f16>() + e : nullptr;
        LAUNCH(launch_f32_to_f16(dx, xh.as<f16>(), xlo, (int64_t)e, ctx->stream));
        return time_launches(ctx, iters, avg, [&](hipStream_t st) {
            return launch_gemm_mfma(xh.as<f16>(), xlo, w.cols, m, w, nullptr, dy, nullptr, nullptr, w.rows, GEMM_STORE,
                                    st);
        });
    }
    return time_launches(ctx, iters, avg, [&](hipStream_t st) {
        return launch_gemm_f32(dx, w.cols, m, w, nullptr, dy, w.rows, GEMM_STORE, st);
    });
}

extern "C" int ahip_dev_attention(ahip_context* ctx, const void* dq, const void* dk, const void* dv, int tokens,
                                  int heads, int kv_heads, int hd, int start, float* dout, int iters, double* avg) {
    if (!ctx || !dq || !dk || !dv || !dout || tokens <= 0 || kv_heads <= 0 || heads % kv_heads || iters < 0)
        return fail(AHIP_ERR_INVALID_ARGUMENT, "bad argument");
    if (start != 0) return fail(AHIP_ERR_UNSUPPORTED, "device attention timing takes start = 0");
    if (hd != 64 && hd != 128) return fail(AHIP_ERR_UNSUPPORTED, "flash attention needs head_dim 64 or 128");
    HIP_OR(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t st = ctx->stream;
    DevBuf kc, vc;
    const size_t bytes = (size_t)tokens * kv_heads * hd * 2;
    if (int rc = kc.alloc(bytes)) return rc;
    if (int rc = vc.alloc(bytes)) return rc;
    // [tokens][kv_heads][hd] -> [kv_heads][tokens][hd]
    for (int h = 0; h < kv_heads; h++) {
        HIP_OR(hipMemcpy2DAsync(kc.as<uint8_t>() + (size_t)h * tokens * hd * 2, hd * 2,
                                (const uint8_t*)dk + (size_t)h * hd * 2, (size_t)kv_heads * hd * 2, hd * 2, tokens,
                                hipMemcpyDeviceToDevice, st), "cache copy");
        HIP_OR(hipMemcpy2DAsync(vc.as<uint8_t>() + (size_t)h * tokens * hd * 2, hd * 2,
                                (const uint8_t*)dv + (size_t)h * hd * 2, (size_t)kv_heads * hd * 2, hd * 2, tokens,
                                hipMemcpyDeviceToDevice, st), "cache copy");
    }
    return time_launches(ctx, iters, avg, [&](hipStream_t s2) {
        return launch_flash_attention((const f16*)dq, nullptr, heads * hd, kc.as<f16>(), vc.as<f16>(), tokens, tokens,
                                      heads, kv_heads, hd, 0, dout, nullptr, nullptr, s2);
    });
}
