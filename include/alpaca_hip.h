/*
 * alpaca_hip.h -- C ABI of the MI355X (gfx950) backend for alpaca.swift.
 *
 * One shared library, libalpaca_hip.so, built from alpaca_amd/csrc/.  It holds
 * the hand-written HIP kernels of the Llama decoder forward pass and the C++
 * runtime that orders them (model upload, sessions with a resident KV cache,
 * chunked prefill, fused decode, device-resident greedy chain, per-stage
 * timing).  Every entry point takes plain pointers and sizes; nothing here
 * names a PyTorch or Swift type.
 *
 * Each declaration cites the reference interface it replaces
 * (torinriley/alpaca, file:line).  All functions return an ahip_status; on a
 * non-zero status ahip_last_error() returns a thread-local message.
 */
#ifndef ALPACA_HIP_H
#define ALPACA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror MetalError (Sources/AlpacaMetal/Backend/MetalContext.swift:7-31). */
typedef enum {
    AHIP_OK = 0,
    AHIP_ERR_NO_DEVICE = 1,        /* MetalError.noDevice */
    AHIP_ERR_MODULE_LOAD = 2,      /* MetalError.shaderCompilation / shaderSourceMissing */
    AHIP_ERR_MISSING_KERNEL = 3,   /* MetalError.missingFunction / pipelineCreation */
    AHIP_ERR_ALLOC = 4,            /* MetalError.bufferAllocation */
    AHIP_ERR_COMMAND_FAILED = 5,   /* MetalError.commandFailed */
    AHIP_ERR_UNSUPPORTED = 6,      /* MetalError.unsupported */
    AHIP_ERR_INVALID_ARGUMENT = 7, /* MetalError.invalidArgument */
    AHIP_ERR_BUSY = 8,             /* re-entrant call on a busy session (MetalLlamaModel.swift:235, :275) */
    AHIP_ERR_GGUF = 9              /* GGUFError (Sources/AlpacaModels/GGUF/GGUFError.swift:5-19); the case
                                      is ahip_gguf_last_error_kind() */
} ahip_status;

/* Element formats, Sources/AlpacaCore/Tensor/DType.swift:8-56.
 * Q8_0: per 32 elements an f16 scale d then 32 int8 q (34 bytes).
 * Q4_0: per 32 elements an f16 scale d then 16 bytes; byte j holds element j
 * in its low nibble and element j+16 in its high nibble; value = d*(nib-8). */
typedef enum { AHIP_F32 = 0, AHIP_F16 = 1, AHIP_Q8_0 = 2, AHIP_Q4_0 = 3 } ahip_dtype;

/* KVPrecision, Sources/AlpacaMetal/Backend/KernelEncoder.swift:9-17. */
typedef enum { AHIP_KV_F16 = 0, AHIP_KV_F32 = 1 } ahip_kv_precision;

/* GEMMPrecision, KernelEncoder.swift:41-48: exact = float32 operands (the
 * SIMT GEMMs and float32 attention); fast = f16 MFMA with float32
 * accumulation, the default: weights enter as their exact quants, activations
 * (and the prefill attention's Q and P) as two f16 terms hi + lo, so prefill
 * logits stay within 2e-3 + 1e-3 relative of the CPU reference at every
 * benchmark configuration; fast_f16 = the same MFMA kernels with one f16 term
 * per activation (the reference's fast-path numerics class: half the MFMA
 * work, 2^-11 relative input rounding). */
typedef enum { AHIP_GEMM_EXACT = 0, AHIP_GEMM_FAST = 1, AHIP_GEMM_FAST_F16 = 2 } ahip_gemm_precision;

/* LlamaConfig, Sources/AlpacaCore/Transformer/LlamaConfig.swift:8-20. */
typedef struct {
    int32_t vocab_size;
    int32_t hidden_size;
    int32_t layer_count;
    int32_t head_count;
    int32_t kv_head_count;
    int32_t head_dim;
    int32_t feed_forward_size;
    int32_t context_length;
    float rms_norm_eps;
    float rope_theta;
    int32_t rope_interleaved; /* 1: adjacent pairs (GGUF); 0: split halves (HF) */
} ahip_llama_config;

/* One weight tensor handed over at model creation, named as in GGUF
 * (Sources/AlpacaModels/Llama/LlamaLoader.swift:43-67, LlamaWeights.swift:
 * "token_embd", "output_norm", "output" (absent = tied), "blk.N.attn_norm",
 * "blk.N.attn_q|attn_k|attn_v|attn_output", "blk.N.ffn_norm",
 * "blk.N.ffn_gate|ffn_up|ffn_down").  `data` is host memory holding `bytes`
 * bytes in `dtype`'s on-disk layout; it may be released after the call. */
typedef struct {
    const char* name;
    int32_t dtype;
    int64_t rows;
    int64_t cols;
    const void* data;
    int64_t bytes;
} ahip_tensor_desc;

typedef struct ahip_context ahip_context;
typedef struct ahip_stream ahip_stream;
typedef struct ahip_model ahip_model;
typedef struct ahip_session ahip_session;

/* Per-stage GPU time of the last profiled call (EncoderProvider profiling,
 * MetalLlamaModel.swift:387-484; lastProfile at :159-160). */
typedef struct {
    char label[48];
    double seconds;
    int32_t dispatches;
} ahip_stage;

/* ------------------------------------------------------------ errors, device */

const char* ahip_last_error(void);
/* Number of visible HIP devices (MetalContext.isAvailable). */
int ahip_device_count(int* count);
/* Library build string (arch and compile flags). */
const char* ahip_version(void);

/* MetalContext.init, MetalContext.swift:37-126: binds one device. */
int ahip_context_create(int device, ahip_context** out);
int ahip_context_destroy(ahip_context* ctx);

/* ------------------------------------------------------------ model */

/* MetalLlamaModel.init(context:config:weights:mappedRegion:keepAlive:
 * prefillWeightCache:), MetalLlamaModel.swift:38-94.  Validates the config
 * and every tensor shape (LlamaConfig.validate, LlamaWeights.validate), then
 * copies all tensors to HBM once, repacking Q8_0/Q4_0 blocks into separate
 * quant and scale streams.  `prefill_weight_cache` also keeps f16 copies of the
 * layer projections for the fast prefill (ahip_model_prefill_cache_bytes). */
int ahip_model_create(ahip_context* ctx, const ahip_llama_config* config, const ahip_tensor_desc* tensors,
                      int count, int prefill_weight_cache, ahip_model** out);
int ahip_model_destroy(ahip_model* model);
/* Bytes of weights resident in HBM (MetalLlamaModel.copiedWeightBytes, :30-32). */
int ahip_model_weight_bytes(const ahip_model* model, int64_t* bytes);
/* Bytes of the prefill weight cache (MetalLlamaModel.prefillCacheBytes, :23-24):
 * with prefill_weight_cache set, every quantised layer projection also gets an
 * f16 copy (each weight d*q rounded once to f16, buildPrefillCache :97-120)
 * that the fast prefill GEMMs multiply by instead of dequantising blocks;
 * decode and the exact prefill keep using the quantised weights.  0 when not
 * requested or when the layers are already F16. */
int ahip_model_prefill_cache_bytes(const ahip_model* model, int64_t* bytes);

/* ------------------------------------------------------------ GGUF files */

/* GGUFError cases (GGUFError.swift:5-19), the kind of the last AHIP_ERR_GGUF
 * raised on this thread. */
typedef enum {
    AHIP_GGUF_CANNOT_OPEN = 1,
    AHIP_GGUF_INVALID_MAGIC = 2,
    AHIP_GGUF_UNSUPPORTED_VERSION = 3,
    AHIP_GGUF_BIG_ENDIAN = 4,
    AHIP_GGUF_TRUNCATED = 5,
    AHIP_GGUF_MALFORMED = 6,
    AHIP_GGUF_LIMIT_EXCEEDED = 7,
    AHIP_GGUF_UNSUPPORTED_TENSOR_TYPE = 8,
    AHIP_GGUF_DUPLICATE_TENSOR = 9,
    AHIP_GGUF_MISSING_METADATA = 10,
    AHIP_GGUF_MISSING_TENSOR = 11,
    AHIP_GGUF_UNSUPPORTED_MODEL = 12,
    AHIP_GGUF_TENSOR_OUT_OF_RANGE = 13,
    AHIP_GGUF_TENSORS_OVERLAP = 14
} ahip_gguf_error;
int ahip_gguf_last_error_kind(void);

/* GGML storage type ids of a GGUF tensor (GGMLType, GGUFTypes.swift:8-12). */
typedef enum {
    AHIP_GGML_F32 = 0, AHIP_GGML_F16 = 1, AHIP_GGML_Q4_0 = 2, AHIP_GGML_Q4_1 = 3, AHIP_GGML_Q5_0 = 6,
    AHIP_GGML_Q5_1 = 7, AHIP_GGML_Q8_0 = 8, AHIP_GGML_Q8_1 = 9, AHIP_GGML_Q2_K = 10, AHIP_GGML_Q3_K = 11,
    AHIP_GGML_Q4_K = 12, AHIP_GGML_Q5_K = 13, AHIP_GGML_Q6_K = 14, AHIP_GGML_Q8_K = 15, AHIP_GGML_BF16 = 30
} ahip_ggml_type;

/* GGUFTensorInfo (GGUFTypes.swift:72-84): dims in GGUF order (dims[0] varies
 * fastest, so a [rows][cols] matrix has dims {cols, rows}); data points into
 * the file's mapping and stays valid until ahip_gguf_close. */
typedef struct {
    const char* name;
    int32_t n_dims;
    int64_t dims[4];
    uint32_t type;
    int64_t file_offset;
    int64_t byte_count;
    const void* data;
} ahip_gguf_tensor;

typedef struct ahip_gguf ahip_gguf;

/* GGUFFile.init(url:), GGUFFile.swift:32-35 and :42-131: maps the file
 * read-only and validates header, metadata and tensor directory without
 * trusting any length field (limits of GGUFFile.Limits, :13-21). */
int ahip_gguf_open(const char* path, ahip_gguf** out);
/* GGUFFile.init(data:), :38-40: validates a private copy of `bytes` bytes. */
int ahip_gguf_open_memory(const void* data, int64_t bytes, ahip_gguf** out);
int ahip_gguf_close(ahip_gguf* g);
/* version, alignment, dataOffset, fileSize (GGUFFile.swift:23-28). */
int ahip_gguf_header(const ahip_gguf* g, uint32_t* version, int64_t* alignment, int64_t* data_offset,
                     int64_t* file_size);
/* Metadata (GGUFFile.metadata, GGUFValue, GGUFTypes.swift:46-70): keys in file
 * order with their GGUF value type id (0-12).  The typed getters follow
 * GGUFValue.asInt / asDouble / asBool / asString; `index` >= 0 reads element
 * `index` of an array value, -1 the value itself.  A missing key or a value of
 * another type is AHIP_GGUF_MISSING_METADATA (GGUFError.missingMetadata). */
int ahip_gguf_meta_count(const ahip_gguf* g, int* count);
int ahip_gguf_meta_key(const ahip_gguf* g, int i, const char** key, uint32_t* type);
int ahip_gguf_meta_int(const ahip_gguf* g, const char* key, int64_t index, int64_t* out);
int ahip_gguf_meta_uint(const ahip_gguf* g, const char* key, int64_t index, uint64_t* out);
int ahip_gguf_meta_float(const ahip_gguf* g, const char* key, int64_t index, double* out);
int ahip_gguf_meta_bool(const ahip_gguf* g, const char* key, int64_t index, int* out);
int ahip_gguf_meta_string(const ahip_gguf* g, const char* key, int64_t index, const char** data, int64_t* length);
int ahip_gguf_meta_array(const ahip_gguf* g, const char* key, uint32_t* elem_type, int64_t* count);
/* GGUFFile.tensors / info(for:) / rawBytes(of:), GGUFFile.swift:176-198. */
int ahip_gguf_tensor_count(const ahip_gguf* g, int* count);
int ahip_gguf_tensor_at(const ahip_gguf* g, int i, ahip_gguf_tensor* out);
int ahip_gguf_find_tensor(const ahip_gguf* g, const char* name, int* index);

/* LoadReport, Sources/AlpacaModels/Llama/LlamaLoader.swift:8-16. */
typedef struct {
    int64_t mapped_weight_bytes;    /* used in their on-disk format (F32, F16, Q8_0, Q4_0) */
    int64_t converted_weight_bytes; /* expanded at load (Q4_1 -> F16) */
    int32_t converted_tensors;
    char notes[2048];               /* one line per converted tensor, truncated to fit */
} ahip_load_report;

/* LlamaLoader.load, configuration half (LlamaLoader.swift:36-72):
 * general.architecture must be "llama"; llama.* keys as the reference reads
 * them, with its defaults (head_dim = hidden / heads, kv heads = heads,
 * eps 1e-5, theta 10000) and its refusals (value_length != key_length,
 * partial rotary, RoPE scaling, experts); vocabulary from token_embd.weight;
 * RoPE pairs interleaved.  The result is also checked as ahip_model_create
 * would. */
int ahip_gguf_llama_config(const ahip_gguf* g, ahip_llama_config* out);
/* LlamaLoader.load, weights half (:74-104), then ahip_model_create: the
 * blk.N.* / token_embd / output_norm / output (absent = tied) tensors go to
 * HBM from the mapping; norms must be F32; Q4_1 tensors are expanded to F16
 * (value = f16(d*q + m), :106-125) and reported; any other type is
 * AHIP_GGUF_UNSUPPORTED_TENSOR_TYPE.  `config_out` and `report` may be null. */
int ahip_model_load_gguf(ahip_context* ctx, const ahip_gguf* g, int prefill_weight_cache, ahip_model** out,
                         ahip_llama_config* config_out, ahip_load_report* report);

/* MetalLlamaModel.sessionByteCount, MetalLlamaModel.swift:123-127. */
int ahip_session_byte_count(const ahip_llama_config* config, int capacity, int max_batch, int kv_precision,
                            int64_t* bytes);

/* ------------------------------------------------------------ session */

/* MetalLlamaModel.makeSession(capacity:maxBatch:kvPrecision:gemmPrecision:),
 * MetalLlamaModel.swift:136-140 / MetalLlamaSession.init :181-217.  capacity
 * is clamped to the model's context length.  Each session owns its KV cache,
 * scratch, a pinned logits buffer and its own HIP stream. */
int ahip_session_create(ahip_model* model, int capacity, int max_batch, int kv_precision, int gemm_precision,
                        ahip_session** out);
int ahip_session_destroy(ahip_session* s);

/* MetalLlamaSession.forward(tokens:), MetalLlamaModel.swift:274-305 and
 * InferenceSession.forward (Sources/Alpaca/LanguageModel.swift:317-328).
 * Appends `n` tokens at positions length..length+n-1 (chunked by max_batch)
 * and points *logits at the last position's vocab_size logits, valid until the
 * next call on `s`.  Fails without advancing length on an empty input, a token
 * outside the vocabulary or a context overflow. */
int ahip_session_forward(ahip_session* s, const int32_t* tokens, int n, const float** logits);

/* MetalLlamaSession.decode(token:), MetalLlamaModel.swift:221-226. */
int ahip_session_decode(ahip_session* s, int32_t token, const float** logits);

/* MetalLlamaSession.decodeGreedy(startToken:maxSteps:depth:emit:),
 * MetalLlamaModel.swift:228-270.  Feeds `start` at position length, takes the
 * arg-max on the GPU (lowest index wins ties, NaN never wins) and feeds it
 * straight back; up to `depth` steps are queued ahead.  `emit` receives each
 * produced token in order and returns 0 to stop; steps already queued are
 * drained and discarded.  *fed = tokens consumed, by which length advances
 * (also on failure). */
typedef int (*ahip_emit_fn)(void* user, int32_t token);
int ahip_session_decode_greedy(ahip_session* s, int32_t start, int max_steps, int depth, ahip_emit_fn emit,
                               void* user, int* fed);

/* MetalLlamaSession.reset / length / capacity / lastGPUSeconds /
 * lastEncodeSeconds (MetalLlamaModel.swift:151-160, :219). */
/* Sampler.sample(logits:) (Sources/AlpacaCore/Runtime/Sampler.swift:57-93)
 * on the device, over the logits of the session's last forward / decode call
 * (they stay in HBM), for a draw `u` in [0, 1) from the caller's sampler RNG
 * (the reference's Sampler owns a SplitMix64 and draws Double.random once per
 * sample).  temperature 0 is the arg-max; top_k 0 disables top-k; top_p 1
 * disables top-p; parameters are checked as SamplingParameters.validate
 * (:21-25).  NaN logits are AHIP_ERR_INVALID_ARGUMENT (the Swift code throws).
 * After a greedy chain or a reset there are no logits to sample. */
int ahip_session_sample(ahip_session* s, float temperature, int top_k, float top_p, double u, int32_t* token);

int ahip_session_reset(ahip_session* s);
int ahip_session_length(const ahip_session* s, int* length);
int ahip_session_capacity(const ahip_session* s, int* capacity);
int ahip_session_last_gpu_seconds(const ahip_session* s, double* seconds);
int ahip_session_last_encode_seconds(const ahip_session* s, double* seconds);

/* profilingEnabled / lastProfile, MetalLlamaModel.swift:156-160: when on,
 * every stage is bracketed by HIP events on the session stream. */
int ahip_session_set_profiling(ahip_session* s, int enabled);
int ahip_session_profile(const ahip_session* s, ahip_stage* out, int capacity, int* count);
/* The wall-clock timeline behind the stages of the last profiled single-token
 * launch of the persistent decode kernel (the GPU timestamps EncoderProvider
 * takes at stage boundaries, MetalLlamaModel.swift:431-447): `count` stamps,
 * laid out [point][workgroup] with `workgroups` columns.  Points: launch start,
 * then six per layer (qkv, attention, merge, wo, gate/up, down), logits, and the
 * arg-max (workgroup 0 only); then eight stamps inside the attention item of
 * the last layer.  A zero stamp was not written.  Copies min(count, capacity). */
int ahip_session_decode_timeline(const ahip_session* s, uint64_t* out, int64_t capacity, int64_t* count,
                                 int* workgroups, double* tick_seconds);

/* ------------------------------------------------------------ op-level API
 * MetalOps, Sources/AlpacaMetal/Backend/MetalOps.swift:11-219: tensor in /
 * tensor out.  Each call uploads its host operands, runs the same kernels the
 * session uses, and copies the result back.  Weights are raw on-disk bytes. */

int ahip_op_add(ahip_context* ctx, const float* a, const float* b, int64_t n, float* out);
int ahip_op_mul(ahip_context* ctx, const float* a, const float* b, int64_t n, float* out);
int ahip_op_silu(ahip_context* ctx, const float* x, int64_t n, float* out);
int ahip_op_silu_mul(ahip_context* ctx, const float* gate, const float* up, int64_t n, float* out);
int ahip_op_rmsnorm(ahip_context* ctx, const float* x, const float* weight, int rows, int dim, float eps,
                    float* out);
/* y[m,n] = x[m,k] * W[n,k]^T (MetalOps.linear, :50-67). */
int ahip_op_linear(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* w, int n,
                   int gemm_precision, float* y);
/* residual[m,n] += x * W^T in place (MetalOps.linearAdd, :69-84). */
int ahip_op_linear_add(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* w, int n,
                       int gemm_precision, float* residual);
/* silu(x*Wg^T) * (x*Wu^T) (MetalOps.gateUpSilu, :86-105). */
int ahip_op_gate_up_silu(ahip_context* ctx, const float* x, int m, int k, int dtype, const void* wg,
                         const void* wu, int n, int gemm_precision, float* out);
/* RoPE in place on x[tokens, heads, hd] (MetalOps.rope, :107-114). */
int ahip_op_rope(ahip_context* ctx, float* x, int tokens, int heads, int head_dim, int start, float theta,
                 int interleaved);
/* Causal GQA attention (MetalOps.attention, :116-148).  q [tokens, heads, hd];
 * keys/values [capacity, kv_heads, hd] f32, stored into the cache format
 * selected by kv_precision; out [tokens, heads, hd]. */
int ahip_op_attention(ahip_context* ctx, const float* q, int tokens, int heads, int head_dim, const float* keys,
                      const float* values, int capacity, int kv_heads, int start, int kv_precision,
                      int gemm_precision, float* out);
/* Embedding gather + dequant (MetalOps.embed, :150-160). */
int ahip_op_embed(ahip_context* ctx, const int32_t* tokens, int count, int dtype, const void* table, int vocab,
                  int dim, float* out);
/* Block dequantisation of `elements` values (Quantization.swift:9-35 on GPU). */
int ahip_op_dequantize(ahip_context* ctx, int dtype, const void* src, int64_t elements, float* out);
/* GPU arg-max, lowest index on ties, NaN never wins (norm_embed.metal:93-121). */
/* The same sampler over host logits (the op-level test API). */
int ahip_op_sample(ahip_context* ctx, const float* logits, int n, float temperature, int top_k, float top_p,
                   double u, int32_t* token);
int ahip_op_argmax(ahip_context* ctx, const float* logits, int n, int32_t* index);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, fixed serving loops, harnesses that
 * forbid hipMalloc): the single-query case of ahip_op_attention (split-K
 * attention over a KV cache, then the merge of the splits) on device buffers,
 * allocating nothing.  q: [heads * head_dim] f32; k_cache / v_cache: the
 * session layout [kv_heads][capacity][head_dim] in f16 (AHIP_KV_F16) or f32;
 * rows 0..length-1 are visible; out: [heads * head_dim] f32.  Queued on
 * `stream` (null: the context stream) without waiting.  The split partials go
 * to a fixed 2.5 MiB device array per GPU (heads * splits * (head_dim + 2)
 * floats, splits = ceil(length / max(128, ceil(capacity / 64) rounded up to
 * 32))); larger shapes are AHIP_ERR_INVALID_ARGUMENT.  All calls on one GPU
 * share that array: calls that overlap on one GPU race. */
int ahip_attention_decode_noalloc(ahip_context* ctx, const float* q, const void* k_cache, const void* v_cache,
                                  int kv_precision, int capacity, int heads, int kv_heads, int head_dim, int length,
                                  float* out, ahip_stream* stream);

/* Host block quantiser, Quantization.swift:39-73 (ggml quantize_row_*_ref):
 * count must be a multiple of 32; writes count/32 blocks into out. */
int ahip_quantize(int dtype, const float* values, int64_t count, void* out);

/* Seeded synthetic inputs (SplitMix64, Sources/AlpacaCore/Runtime/
 * Sampler.swift:30-40).  Element i of a stream uses the generator state after
 * `offset + i` steps (normal: 2 steps per value pair):
 *   uniform   u = (next() >> 11) * 2^-53 in [0,1)
 *   normal    Box-Muller in double on pairs (u1, u2): r = sqrt(-2 ln(1-u1)),
 *             z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), scaled by std
 *   integers  next() % range                                            */
int ahip_synth_uniform(uint64_t seed, uint64_t offset, int64_t n, float lo, float hi, float* out);
int ahip_synth_normal(uint64_t seed, uint64_t offset, int64_t n, float std, float* out);
int ahip_synth_ints(uint64_t seed, uint64_t offset, int64_t n, uint64_t range, int64_t bias, int32_t* out);

/* ------------------------------------------------------------ thin HIP shim
 * The device-memory / stream / event surface the Swift C target wraps
 * (north star: "a SwiftPM C target wrapping hipMalloc, ... streams and
 * events").  Used by the bench harness to time kernels on device-resident
 * inputs. */
int ahip_malloc(ahip_context* ctx, int64_t bytes, void** dptr);
int ahip_free(ahip_context* ctx, void* dptr);
int ahip_memcpy_htod(ahip_context* ctx, void* dst, const void* src, int64_t bytes);
int ahip_memcpy_dtoh(ahip_context* ctx, void* dst, const void* src, int64_t bytes);
int ahip_memset(ahip_context* ctx, void* dst, int value, int64_t bytes);
int ahip_synchronize(ahip_context* ctx);

typedef struct ahip_event ahip_event;

/* Streams: the session's own command queue (MetalLlamaModel.swift:214-215
 * makes one per session; MTLCommandQueue, MetalContext.swift:48-57), at the
 * default priority.  _synchronize is commit + waitUntilCompleted. */
int ahip_stream_create(ahip_context* ctx, ahip_stream** out);
int ahip_stream_destroy(ahip_stream* s);
int ahip_stream_synchronize(ahip_stream* s);
/* Work queued on `s` after this call waits for `e` (command-buffer ordering
 * across queues). */
int ahip_stream_wait_event(ahip_stream* s, ahip_event* e);

/* Events: the command buffer's gpuStartTime / gpuEndTime pair
 * (MetalOps.swift:18-28, MetalLlamaModel.swift:255-260). */
int ahip_event_create(ahip_context* ctx, ahip_event** out);
int ahip_event_destroy(ahip_event* e);
int ahip_event_record(ahip_event* e, ahip_stream* s);
int ahip_event_synchronize(ahip_event* e);
/* Milliseconds between two recorded events. */
int ahip_event_elapsed_ms(const ahip_event* start, const ahip_event* end, float* ms);

/* Pinned host memory for asynchronous copies (the shared-storage MTLBuffers of
 * MetalContext.makeBuffer, MetalContext.swift:113-125, are host-visible). */
int ahip_host_alloc(ahip_context* ctx, int64_t bytes, void** ptr);
int ahip_host_free(ahip_context* ctx, void* ptr);
/* Copies ordered on `s`; host buffers should be pinned (ahip_host_alloc). */
int ahip_memcpy_htod_async(void* dst, const void* src, int64_t bytes, ahip_stream* s);
int ahip_memcpy_dtoh_async(void* dst, const void* src, int64_t bytes, ahip_stream* s);
int ahip_memcpy_dtod_async(void* dst, const void* src, int64_t bytes, ahip_stream* s);

/* Code-object modules (MetalContext.compileLibrary + pipeline(name),
 * MetalContext.swift:59-111): a gfx950 code object from a file or memory,
 * kernels found by name (AHIP_ERR_MISSING_KERNEL = MetalError.missingFunction)
 * and launched with hipModuleLaunchKernel.  `args` holds one pointer per kernel
 * argument, to a value laid out as the kernel declares it.  The library ships
 * one such object, shim_kernels.hsaco next to libalpaca_hip.so
 * (ahip_shim_axpy, ahip_shim_fill_u32), for the shim's own tests. */
typedef struct ahip_module ahip_module;
int ahip_module_load(ahip_context* ctx, const char* path, ahip_module** out);
int ahip_module_load_data(ahip_context* ctx, const void* image, ahip_module** out);
int ahip_module_unload(ahip_module* m);
int ahip_module_has_kernel(ahip_module* m, const char* name, int* found);
int ahip_module_launch(ahip_module* m, const char* kernel, const uint32_t grid[3], const uint32_t block[3],
                       uint32_t shared_bytes, ahip_stream* s, void** args);

/* Device-resident kernel launches on the context stream, timed with HIP events
 * recorded on that stream around `iters` back-to-back launches: *avg_seconds
 * is the mean launch duration.  These run exactly the kernels the session
 * uses, for the bench's roofline figures. */

/* Decode GEMV: y[n] = W[n,k] x[k] with W in the repacked device layout made
 * by ahip_dev_pack_weight. */
int ahip_dev_pack_weight(ahip_context* ctx, int dtype, const void* host_w, int rows, int cols, void** handle);
int ahip_dev_weight_free(ahip_context* ctx, void* handle);
int ahip_dev_gemv(ahip_context* ctx, void* weight, const float* dx, float* dy, int iters, double* avg_seconds);
/* The same GEMV, launch i on weights[i % count]: with copies that together
 * exceed the device's last-level cache (MI355X: 256 MB of Infinity Cache),
 * every launch streams its matrix from HBM. */
int ahip_dev_gemv_cycle(ahip_context* ctx, void* const* weights, int count, const float* dx, float* dy, int iters,
                        double* avg_seconds);
/* Prefill GEMM: y[m,n] = x[m,k] W^T; x given as f32 on device, converted to
 * f16 once before timing (fast path) or used as f32 (exact). */
int ahip_dev_gemm(ahip_context* ctx, void* weight, const float* dx, int m, float* dy, int gemm_precision,
                  int iters, double* avg_seconds);
/* Causal GQA flash attention over device f16 q [t, heads, hd] and a cache
 * filled from device f16 k/v [t, kv_heads, hd]; writes f32 out. */
int ahip_dev_attention(ahip_context* ctx, const void* dq, const void* dk, const void* dv, int tokens, int heads,
                       int kv_heads, int head_dim, int start, float* dout, int iters, double* avg_seconds);
/* Decode attention (attn_decode_split + attn_decode_merge, attention_decode.
 * metal:27-133): one f32 query dq [heads, hd] over the first `length` rows of
 * a device f16 cache dkc / dvc [kv_heads][capacity][hd]; the split-K kernel
 * and its merge timed together; writes f32 dout [heads, hd]. */
int ahip_dev_attention_decode(ahip_context* ctx, const float* dq, const void* dkc, const void* dvc, int capacity,
                              int length, int heads, int kv_heads, int head_dim, float* dout, int iters,
                              double* avg_seconds);

#ifdef __cplusplus
}
#endif

#endif /* ALPACA_HIP_H */
