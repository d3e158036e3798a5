/*
 * alpaca_oracle.c -- CPU restatement of AlpacaCore's reference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP backend in
 * alpaca_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it; the product path never does.
 *
 * It restates, in plain C, the arithmetic of the reference's Swift CPU backend
 * (torinriley/alpaca, Sources/AlpacaCore).  Every function cites the Swift
 * lines it follows.  Float32 operations are written in the same order as the
 * Swift source and compiled with -ffp-contract=off so that no fused
 * multiply-add changes a rounding that Swift performs separately.
 *
 * Pinned by (tests/test_oracle_*.py):
 *   - tests/golden/ops.json: the reference's own fixture (numpy / torch / gguf
 *     float64 values) for add, mul, silu, matmul, linear (f32/f16/q8_0/q4_0),
 *     rmsnorm, softmax, rope (both conventions), causal GQA attention,
 *     dequantise (exact), quantise (byte-identical) and embedding;
 *   - tests/golden/tiny_llama.json: Hugging Face float64 logits of two tiny
 *     Llama models in both RoPE layouts (whole forward, KV cache, reset);
 *   - closed forms and invariants (softmax rows sum to one, RoPE preserves
 *     pair norms, Q4_0 nibble order, argmax tie rule, SplitMix64 vectors);
 *   - the sampler: the assertions of the reference's SamplerTests.swift
 *     (frequencies against softmax, top-k and top-p supports, seeds, extreme
 *     logits) and brute-force checks of the inverse-CDF draw.  The mapping of
 *     a SplitMix64 word to Double.random (orc_uniform53) restates the Swift
 *     standard library and cannot be run here: parity unpinned for the exact
 *     token stream of a seed, pinned for the draw given u.
 * Every exported function is covered by at least one of these.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 2, ORC_Q4_0 = 3 };

/* ---------------------------------------------------------------- helpers */

/* IEEE binary16 -> binary32 (exact). Swift `Float(Float16)`. */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { e++; man <<= 1; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE binary32 -> binary16, round to nearest even (Swift `Float16(Float)`). */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0));
    if (absx >= 0x477FF000u) /* rounds to >= 65520: overflow to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (absx < 0x38800000u) { /* below 2^-14: subnormal half (or zero) */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t man = (absx & 0x7FFFFFu) | 0x800000u;
        int e = (int)(absx >> 23); /* biased float exponent, 102..112 */
        int shift = 126 - e; /* value = man * 2^(e-150); half ulp = 2^-24 */
        uint32_t q = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 127 + 15;
    uint32_t man = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++; /* carry may bump exponent: still correct */
    return (uint16_t)(sign | q);
}

static inline float h2f(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2); /* loadUnaligned(as: Float16.self) */
    return orc_half_to_float(h);
}

/* SplitMix64, Sources/AlpacaCore/Runtime/Sampler.swift:30-40. */
uint64_t orc_splitmix_next(uint64_t* state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

int orc_block_elements(int dtype) { return (dtype == ORC_Q8_0 || dtype == ORC_Q4_0) ? 32 : 1; }
int orc_block_bytes(int dtype) {
    /* Tensor/DType.swift:27-34 */
    switch (dtype) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q4_0: return 18;
    }
    return 0;
}
int64_t orc_row_bytes(int dtype, int64_t cols) {
    return cols / orc_block_elements(dtype) * orc_block_bytes(dtype);
}

/* ---------------------------------------------------------------- quant */

/* Operations/Quantization.swift:9-35 */
void orc_dequantize(int dtype, const void* source, int64_t elements, float* dst) {
    const uint8_t* src = (const uint8_t*)source;
    int64_t blocks = elements / 32;
    switch (dtype) {
    case ORC_Q8_0:
        for (int64_t b = 0; b < blocks; b++) {
            const uint8_t* p = src + b * 34;
            float d = h2f(p);
            const int8_t* q = (const int8_t*)(p + 2);
            for (int j = 0; j < 32; j++) dst[b * 32 + j] = d * (float)q[j];
        }
        break;
    case ORC_Q4_0:
        for (int64_t b = 0; b < blocks; b++) {
            const uint8_t* p = src + b * 18;
            float d = h2f(p);
            const uint8_t* q = p + 2;
            for (int j = 0; j < 16; j++) {
                dst[b * 32 + j] = d * (float)((int)(q[j] & 0x0F) - 8);
                dst[b * 32 + j + 16] = d * (float)((int)(q[j] >> 4) - 8);
            }
        }
        break;
    case ORC_F32:
        memcpy(dst, src, (size_t)elements * 4);
        break;
    case ORC_F16:
        for (int64_t i = 0; i < elements; i++) dst[i] = h2f(src + 2 * i);
        break;
    }
}

/* Operations/Quantization.swift:39-73 (ggml quantize_row_q8_0_ref / q4_0_ref).
 * Returns 0 on success, -1 if the target dtype or element count is invalid. */
int orc_quantize(int dtype, const float* values, int64_t count, void* out) {
    if (dtype != ORC_Q8_0 && dtype != ORC_Q4_0) return -1;
    if (count % 32 != 0) return -1;
    uint8_t* dst = (uint8_t*)out;
    int64_t blocks = count / 32;
    for (int64_t b = 0; b < blocks; b++) {
        const float* x = values + b * 32;
        if (dtype == ORC_Q8_0) {
            uint8_t* p = dst + b * 34;
            float amax = 0;
            for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint16_t dh = orc_float_to_half(d);
            memcpy(p, &dh, 2);
            int8_t* q = (int8_t*)(p + 2);
            for (int j = 0; j < 32; j++) {
                float t = x[j] * id;
                q[j] = (int8_t)roundf(t); /* .toNearestOrAwayFromZero */
            }
        } else {
            uint8_t* p = dst + b * 18;
            float maxv = 0, amax = 0;
            for (int j = 0; j < 32; j++)
                if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); maxv = x[j]; }
            float d = maxv / -8.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint16_t dh = orc_float_to_half(d);
            memcpy(p, &dh, 2);
            uint8_t* q = p + 2;
            for (int j = 0; j < 16; j++) {
                float tl = x[j] * id;
                tl = tl + 8.5f;
                float th = x[j + 16] * id;
                th = th + 8.5f;
                int lo = (int)tl, hi = (int)th; /* Int(...) truncates toward zero */
                if (lo > 15) lo = 15;
                if (hi > 15) hi = 15;
                q[j] = (uint8_t)((uint8_t)lo | ((uint8_t)hi << 4));
            }
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- linear */

/* CPUOps.dot, Operations/CPUOps.swift:106-139: per-block partial sum `s`
 * accumulated sequentially, then acc += d * s. */
static float dot_row(int dtype, const uint8_t* row, const float* x, int k) {
    float acc = 0;
    switch (dtype) {
    case ORC_F32: {
        const float* w = (const float*)row;
        for (int i = 0; i < k; i++) { float t = w[i] * x[i]; acc += t; }
        break;
    }
    case ORC_F16:
        for (int i = 0; i < k; i++) { float t = h2f(row + 2 * i) * x[i]; acc += t; }
        break;
    case ORC_Q8_0:
        for (int b = 0; b < k / 32; b++) {
            const uint8_t* p = row + (int64_t)b * 34;
            float d = h2f(p);
            const int8_t* q = (const int8_t*)(p + 2);
            float s = 0;
            for (int j = 0; j < 32; j++) { float t = (float)q[j] * x[b * 32 + j]; s += t; }
            float ds = d * s;
            acc += ds;
        }
        break;
    case ORC_Q4_0:
        for (int b = 0; b < k / 32; b++) {
            const uint8_t* p = row + (int64_t)b * 18;
            float d = h2f(p);
            const uint8_t* q = p + 2;
            float s = 0;
            for (int j = 0; j < 16; j++) {
                float t0 = (float)((int)(q[j] & 0x0F) - 8) * x[b * 32 + j];
                s += t0;
                float t1 = (float)((int)(q[j] >> 4) - 8) * x[b * 32 + j + 16];
                s += t1;
            }
            float ds = d * s;
            acc += ds;
        }
        break;
    }
    return acc;
}

float orc_dot(int dtype, const void* row, const float* x, int k) {
    return dot_row(dtype, (const uint8_t*)row, x, k);
}

static int g_threads = 0;
void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* CPUOps.linear, Operations/CPUOps.swift:77-103: y[M,N] = x[M,K] * W[N,K]^T.
 * Rows are split into chunks of 16 and the chunks run in parallel, token by
 * token (concurrentPerform); each row's dot product is sequential, so the
 * result does not depend on the thread count. */
void orc_linear(const float* x, int m, int k, int dtype, const void* w, int n, float* out) {
    const uint8_t* wb = (const uint8_t*)w;
    int64_t rb = orc_row_bytes(dtype, k);
    int chunks = (n + 15) / 16;
    int threads = orc_get_threads();
    for (int t = 0; t < m; t++) {
        const float* xr = x + (int64_t)t * k;
        float* orow = out + (int64_t)t * n;
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int c = 0; c < chunks; c++) {
            int r1 = (c + 1) * 16 < n ? (c + 1) * 16 : n;
            for (int r = c * 16; r < r1; r++) orow[r] = dot_row(dtype, wb + (int64_t)r * rb, xr, k);
        }
    }
}

/* CPUOps.matmul, Operations/CPUOps.swift:58-72: C[M,N] = A[M,K] * B[K,N]. */
void orc_matmul(const float* a, const float* b, int m, int k, int n, float* c) {
    memset(c, 0, sizeof(float) * (size_t)m * n);
    for (int i = 0; i < m; i++)
        for (int p = 0; p < k; p++) {
            float aip = a[i * k + p];
            for (int j = 0; j < n; j++) { float t = aip * b[p * n + j]; c[i * n + j] += t; }
        }
}

/* ---------------------------------------------------------------- elementwise */

/* CPUOps.add / mul, Operations/CPUOps.swift:29-46 */
void orc_add(const float* a, const float* b, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = a[i] + b[i];
}
void orc_mul(const float* a, const float* b, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = a[i] * b[i];
}
/* CPUOps.silu, Operations/CPUOps.swift:48-53: x / (1 + exp(-x)) */
void orc_silu(const float* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) {
        float e = expf(-x[i]);
        float den = 1.0f + e;
        out[i] = x[i] / den;
    }
}

/* CPUOps.rmsNorm, Operations/CPUOps.swift:144-159 */
void orc_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (int64_t)r * d;
        float ss = 0;
        for (int i = 0; i < d; i++) { float t = xr[i] * xr[i]; ss += t; }
        float mean = ss / (float)d;
        float scale = 1.0f / sqrtf(mean + eps);
        for (int i = 0; i < d; i++) {
            float t = xr[i] * scale;
            out[(int64_t)r * d + i] = t * w[i];
        }
    }
}

/* CPUOps.softmax, Operations/CPUOps.swift:162-175 (in place). */
void orc_softmax(float* v, int64_t rows, int d) {
    for (int64_t r = 0; r < rows; r++) {
        float* p = v + r * d;
        float mx = -INFINITY;
        for (int i = 0; i < d; i++) mx = fmaxf(mx, p[i]);
        float sum = 0;
        for (int i = 0; i < d; i++) { p[i] = expf(p[i] - mx); sum += p[i]; }
        for (int i = 0; i < d; i++) p[i] /= sum;
    }
}

/* CPUOps.rope, Operations/CPUOps.swift:184-212 (in place).  Frequency and
 * angle in double, cos/sin rounded once to float. */
void orc_rope(float* v, int tokens, int heads, int hd, int start, float theta, int interleaved) {
    int half = hd / 2;
    for (int t = 0; t < tokens; t++) {
        double pos = (double)(start + t);
        for (int i = 0; i < half; i++) {
            double freq = pow((double)theta, -2.0 * (double)i / (double)hd);
            double angle = pos * freq;
            float c = (float)cos(angle), s = (float)sin(angle);
            for (int h = 0; h < heads; h++) {
                int64_t base = ((int64_t)t * heads + h) * hd;
                int64_t ia = interleaved ? base + 2 * i : base + i;
                int64_t ib = interleaved ? base + 2 * i + 1 : base + i + half;
                float a = v[ia], b = v[ib];
                float ac = a * c, bs = b * s, as = a * s, bc = b * c;
                v[ia] = ac - bs;
                v[ib] = as + bc;
            }
        }
    }
}

/* CPUOps.attentionScores, Operations/CPUOps.swift:222-249.
 * q [tokens, nHeads, hd]; keys [capacity, nKV, hd]; scores [nHeads, tokens, length]. */
void orc_attention_scores(const float* q, int tokens, int n_heads, int hd, const float* keys, int n_kv,
                          int length, int start, float* scores) {
    int group = n_heads / n_kv;
    float scale = 1.0f / sqrtf((float)hd);
    for (int64_t i = 0; i < (int64_t)n_heads * tokens * length; i++) scores[i] = -INFINITY;
    for (int h = 0; h < n_heads; h++)
        for (int t = 0; t < tokens; t++)
            for (int p = 0; p <= start + t; p++) {
                float acc = 0;
                const float* qb = q + ((int64_t)t * n_heads + h) * hd;
                const float* kb = keys + ((int64_t)p * n_kv + h / group) * hd;
                for (int i = 0; i < hd; i++) { float m = qb[i] * kb[i]; acc += m; }
                scores[((int64_t)h * tokens + t) * length + p] = acc * scale;
            }
}

/* CPUOps.attentionApply, Operations/CPUOps.swift:252-274.
 * probs [nHeads, tokens, length]; values [capacity, nKV, hd]; out [tokens, nHeads, hd]. */
void orc_attention_apply(const float* probs, int n_heads, int tokens, int length, const float* values, int n_kv,
                         int hd, float* out) {
    int group = n_heads / n_kv;
    memset(out, 0, sizeof(float) * (size_t)tokens * n_heads * hd);
    for (int h = 0; h < n_heads; h++)
        for (int t = 0; t < tokens; t++)
            for (int p = 0; p < length; p++) {
                float w = probs[((int64_t)h * tokens + t) * length + p];
                if (w == 0.0f) continue;
                const float* vb = values + ((int64_t)p * n_kv + h / group) * hd;
                float* ob = out + ((int64_t)t * n_heads + h) * hd;
                for (int i = 0; i < hd; i++) { float m = w * vb[i]; ob[i] += m; }
            }
}

/* Full attention = apply(softmax(scores)); scratch sized n_heads*tokens*length. */
void orc_attention(const float* q, int tokens, int n_heads, int hd, const float* keys, const float* values,
                   int n_kv, int length, int start, float* scratch, float* out) {
    orc_attention_scores(q, tokens, n_heads, hd, keys, n_kv, length, start, scratch);
    orc_softmax(scratch, (int64_t)n_heads * tokens, length);
    orc_attention_apply(scratch, n_heads, tokens, length, values, n_kv, hd, out);
}

/* CPUOps.embed, Operations/CPUOps.swift:279-290.  Returns -1 on a bad id. */
int orc_embed(const int32_t* tokens, int count, int dtype, const void* table, int vocab, int dim, float* out) {
    int64_t rb = orc_row_bytes(dtype, dim);
    for (int i = 0; i < count; i++) {
        if (tokens[i] < 0 || tokens[i] >= vocab) return -1;
        orc_dequantize(dtype, (const uint8_t*)table + (int64_t)tokens[i] * rb, dim, out + (int64_t)i * dim);
    }
    return 0;
}

/* Sampler.argmax, Runtime/Sampler.swift:100-108: lowest index wins ties;
 * returns -1 where the Swift code throws on NaN. */
int orc_argmax(const float* logits, int n) {
    int best = 0;
    for (int i = 0; i < n; i++) {
        if (isnan(logits[i])) return -1;
        if (logits[i] > logits[best]) best = i;
    }
    return best;
}

/* Double.random(in: 0..<1, using:) over SplitMix64 as the Swift standard
 * library defines it for Double (53 significand bits): the low 53 bits of
 * next() times 2^-53 (stdlib FloatingPointRandom.swift; the value is never 1). */
double orc_uniform53(uint64_t* state) {
    return (double)(orc_splitmix_next(state) & ((1ull << 53) - 1)) * 0x1p-53;
}

/* Sampler.sample(logits:), Runtime/Sampler.swift:57-93, for a draw u in
 * [0, 1) (the RNG stays with the caller): temperature 0 is the arg-max; NaN
 * returns -1 (the Swift code throws); top-k keeps the k largest logits (ties
 * by lower index); probabilities exp((l - top) / t) in double; top-p keeps the
 * shortest prefix whose cumulative p/sum reaches top_p; the draw walks the
 * kept probabilities in order against u * sum.  Candidates are sorted by
 * logit, descending, index ascending, exactly when top-k or top-p applies. */
static const float* g_sort_logits;
static int cmp_desc(const void* a, const void* b) {
    const int i = *(const int*)a, j = *(const int*)b;
    const float x = g_sort_logits[i], y = g_sort_logits[j];
    if (x != y) return x > y ? -1 : 1;
    return i < j ? -1 : (i > j ? 1 : 0);
}
int orc_sample(const float* logits, int n, float temperature, int top_k, float top_p, double u) {
    if (n <= 0) return -1;
    if (temperature == 0.0f) return orc_argmax(logits, n);
    for (int i = 0; i < n; i++)
        if (isnan(logits[i])) return -1;
    int* cand = (int*)malloc(sizeof(int) * (size_t)n);
    double* probs = (double*)malloc(sizeof(double) * (size_t)n);
    for (int i = 0; i < n; i++) cand[i] = i;
    int count = n;
    const int k = top_k > 0 ? (top_k < n ? top_k : n) : n;
    if (k < n || top_p < 1.0f) {
        g_sort_logits = logits;
        qsort(cand, (size_t)n, sizeof(int), cmp_desc);
        count = k;
    }
    const double t = (double)temperature;
    double top = (double)logits[cand[0]];
    for (int i = 1; i < count; i++)
        if ((double)logits[cand[i]] > top) top = (double)logits[cand[i]];
    double sum = 0.0;
    for (int i = 0; i < count; i++) {
        probs[i] = exp(((double)logits[cand[i]] - top) / t);
        sum += probs[i];
    }
    if (top_p < 1.0f) {
        double cumulative = 0.0;
        int keep = count;
        for (int i = 0; i < count; i++) {
            cumulative += probs[i] / sum;
            if (cumulative >= (double)top_p) {
                keep = i + 1;
                break;
            }
        }
        count = keep;
        sum = 0.0;
        for (int i = 0; i < count; i++) sum += probs[i];
    }
    const double target = u * sum;
    double acc = 0.0;
    int token = cand[count - 1];
    for (int i = 0; i < count; i++) {
        acc += probs[i];
        if (target < acc) {
            token = cand[i];
            break;
        }
    }
    free(cand);
    free(probs);
    return token;
}

/* ---------------------------------------------------------------- model */

/* LlamaConfig, Transformer/LlamaConfig.swift:8-20 */
typedef struct {
    int32_t vocab_size, hidden_size, layer_count, head_count, kv_head_count, head_dim, feed_forward_size,
        context_length;
    float rms_norm_eps, rope_theta;
    int32_t rope_interleaved;
} orc_config;

/* LlamaLayerWeights / LlamaWeights, Transformer/LlamaWeights.swift:5-24.
 * The caller owns every buffer; norms are f32. */
typedef struct {
    const float* attn_norm;
    const void *wq, *wk, *wv, *wo;
    const float* ffn_norm;
    const void *w_gate, *w_up, *w_down;
} orc_layer;

typedef struct {
    orc_config c;
    int dtype; /* one dtype for every projection matrix */
    int emb_dtype, out_dtype;
    const void* token_embd;
    const void* output; /* == token_embd when tied */
    const float* output_norm;
    orc_layer* layers;
} orc_model;

/* KVCache, Transformer/KVCache.swift:10-73 (f32 storage, optional f16 rounding). */
typedef struct {
    int layers, capacity, kv_heads, head_dim, length, rounds_f16;
    float** keys;
    float** values;
} orc_kvcache;

orc_model* orc_model_create(const orc_config* c, int dtype, int emb_dtype, int out_dtype, const void* token_embd,
                            const void* output, const float* output_norm) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->c = *c;
    m->dtype = dtype;
    m->emb_dtype = emb_dtype;
    m->out_dtype = output ? out_dtype : emb_dtype;
    m->token_embd = token_embd;
    m->output = output ? output : token_embd;
    m->output_norm = output_norm;
    m->layers = (orc_layer*)calloc((size_t)c->layer_count, sizeof(orc_layer));
    return m;
}
void orc_model_set_layer(orc_model* m, int i, const float* attn_norm, const void* wq, const void* wk,
                         const void* wv, const void* wo, const float* ffn_norm, const void* w_gate,
                         const void* w_up, const void* w_down) {
    orc_layer* l = &m->layers[i];
    l->attn_norm = attn_norm; l->wq = wq; l->wk = wk; l->wv = wv; l->wo = wo;
    l->ffn_norm = ffn_norm; l->w_gate = w_gate; l->w_up = w_up; l->w_down = w_down;
}
void orc_model_destroy(orc_model* m) {
    if (!m) return;
    free(m->layers);
    free(m);
}

orc_kvcache* orc_kv_create(int layers, int capacity, int kv_heads, int head_dim, int rounds_f16) {
    orc_kvcache* kv = (orc_kvcache*)calloc(1, sizeof(orc_kvcache));
    kv->layers = layers; kv->capacity = capacity; kv->kv_heads = kv_heads; kv->head_dim = head_dim;
    kv->rounds_f16 = rounds_f16;
    kv->keys = (float**)calloc((size_t)layers, sizeof(float*));
    kv->values = (float**)calloc((size_t)layers, sizeof(float*));
    size_t n = (size_t)capacity * kv_heads * head_dim;
    for (int l = 0; l < layers; l++) {
        kv->keys[l] = (float*)calloc(n, sizeof(float));
        kv->values[l] = (float*)calloc(n, sizeof(float));
    }
    return kv;
}
void orc_kv_destroy(orc_kvcache* kv) {
    if (!kv) return;
    for (int l = 0; l < kv->layers; l++) { free(kv->keys[l]); free(kv->values[l]); }
    free(kv->keys); free(kv->values); free(kv);
}
int orc_kv_length(const orc_kvcache* kv) { return kv->length; }
void orc_kv_reset(orc_kvcache* kv) { kv->length = 0; } /* KVCache.swift:71-73 */

/* Benchmark helper (no reference counterpart): marks `length` rows valid and
 * fills them with small deterministic values, so a decode step at a long
 * context can be timed without first prefilling that context. */
int orc_kv_fill(orc_kvcache* kv, int length, uint64_t seed) {
    if (length < 0 || length > kv->capacity) return -1;
    size_t n = (size_t)length * kv->kv_heads * kv->head_dim;
    for (int l = 0; l < kv->layers; l++)
        for (size_t i = 0; i < n; i++) {
            uint64_t st = seed + (uint64_t)l * 0x100000000ull + i;
            float u = (float)((orc_splitmix_next(&st) >> 40) * (1.0 / 16777216.0)) - 0.5f;
            kv->keys[l][i] = u;
            kv->values[l][i] = -u;
        }
    kv->length = length;
    return 0;
}
const float* orc_kv_keys(const orc_kvcache* kv, int layer) { return kv->keys[layer]; }
const float* orc_kv_values(const orc_kvcache* kv, int layer) { return kv->values[layer]; }

/* KVCache.write, KVCache.swift:44-63.  Returns -1 on a bounds violation. */
static int kv_write(orc_kvcache* kv, int layer, int position, const float* k, const float* v, int n) {
    if (layer < 0 || layer >= kv->layers) return -1;
    if (position < 0 || position != kv->length || position + n > kv->capacity) return -1;
    size_t row = (size_t)kv->kv_heads * kv->head_dim;
    float* kd = kv->keys[layer] + (size_t)position * row;
    float* vd = kv->values[layer] + (size_t)position * row;
    memcpy(kd, k, sizeof(float) * row * n);
    memcpy(vd, v, sizeof(float) * row * n);
    if (kv->rounds_f16) {
        for (size_t i = 0; i < row * n; i++) {
            kd[i] = orc_half_to_float(orc_float_to_half(kd[i]));
            vd[i] = orc_half_to_float(orc_float_to_half(vd[i]));
        }
    }
    return 0;
}

/* LlamaCPUModel.forward, Transformer/LlamaCPUModel.swift:24-61.
 * Appends `tokens` to the cache and writes logits: all rows ([n, vocab]) when
 * all_logits != 0, else the last row ([vocab]).  Returns 0, or -1 (empty
 * input / bad geometry), -2 (context exhausted), -3 (bad token id).  A failed
 * call leaves the cache length unchanged. */
int orc_forward(const orc_model* m, orc_kvcache* kv, const int32_t* tokens, int n, int all_logits, float* logits) {
    const orc_config* c = &m->c;
    if (n <= 0) return -1;
    if (kv->layers != c->layer_count || kv->kv_heads != c->kv_head_count || kv->head_dim != c->head_dim) return -1;
    int start = kv->length;
    if (start + n > kv->capacity) return -2;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab_size) return -3;
    int H = c->hidden_size, QW = c->head_count * c->head_dim, KW = c->kv_head_count * c->head_dim;
    int F = c->feed_forward_size, L = start + n;
    float* x = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* h = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* q = (float*)malloc(sizeof(float) * (size_t)n * QW);
    float* k = (float*)malloc(sizeof(float) * (size_t)n * KW);
    float* v = (float*)malloc(sizeof(float) * (size_t)n * KW);
    float* ctx = (float*)malloc(sizeof(float) * (size_t)n * QW);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* gate = (float*)malloc(sizeof(float) * (size_t)n * F);
    float* up = (float*)malloc(sizeof(float) * (size_t)n * F);
    float* scores = (float*)malloc(sizeof(float) * (size_t)c->head_count * n * L);
    orc_embed(tokens, n, m->emb_dtype, m->token_embd, c->vocab_size, H, x);
    for (int li = 0; li < c->layer_count; li++) {
        const orc_layer* l = &m->layers[li];
        orc_rmsnorm(x, l->attn_norm, n, H, c->rms_norm_eps, h);
        orc_linear(h, n, H, m->dtype, l->wq, QW, q);
        orc_linear(h, n, H, m->dtype, l->wk, KW, k);
        orc_linear(h, n, H, m->dtype, l->wv, KW, v);
        orc_rope(q, n, c->head_count, c->head_dim, start, c->rope_theta, c->rope_interleaved);
        orc_rope(k, n, c->kv_head_count, c->head_dim, start, c->rope_theta, c->rope_interleaved);
        kv_write(kv, li, start, k, v, n);
        orc_attention(q, n, c->head_count, c->head_dim, kv->keys[li], kv->values[li], c->kv_head_count, L, start,
                      scores, ctx);
        orc_linear(ctx, n, QW, m->dtype, l->wo, H, tmp);
        orc_add(x, tmp, (int64_t)n * H, x);
        orc_rmsnorm(x, l->ffn_norm, n, H, c->rms_norm_eps, h);
        orc_linear(h, n, H, m->dtype, l->w_gate, F, gate);
        orc_silu(gate, (int64_t)n * F, gate);
        orc_linear(h, n, H, m->dtype, l->w_up, F, up);
        orc_mul(gate, up, (int64_t)n * F, gate);
        orc_linear(gate, n, F, m->dtype, l->w_down, H, tmp);
        orc_add(x, tmp, (int64_t)n * H, x);
    }
    kv->length = L; /* cache.commit */
    if (all_logits) {
        orc_rmsnorm(x, m->output_norm, n, H, c->rms_norm_eps, h);
        orc_linear(h, n, H, m->out_dtype, m->output, c->vocab_size, logits);
    } else {
        orc_rmsnorm(x + (size_t)(n - 1) * H, m->output_norm, 1, H, c->rms_norm_eps, h);
        orc_linear(h, 1, H, m->out_dtype, m->output, c->vocab_size, logits);
    }
    free(x); free(h); free(q); free(k); free(v); free(ctx); free(tmp); free(gate); free(up); free(scores);
    return 0;
}
