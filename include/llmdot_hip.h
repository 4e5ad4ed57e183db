/*
 * llmdot_hip.h -- C ABI of libllmdot_hip.so, the MI355X (gfx950) backend for
 * the llmdot decode token loop.
 *
 * Conventions
 *   - Every function returns int32 status: 0 = OK, < 0 = error (LLMDOT_E_*).
 *     llmdot_hip_last_error() returns a thread-local message for the last
 *     failing call on the calling thread.  No C++ exception crosses the ABI.
 *   - Host pointers are borrowed for the duration of the call.  Synchronous
 *     calls return after results are written to host memory.
 *   - Device memory is owned by the context / model handle.
 *   - One context per device; a context and its models are not thread-safe
 *     (the reference engine is single-threaded too).
 *   - Element types use the GgmlType numbering of
 *     src/Llmdot.Core/Loading/GgmlType.cs:3-28 (F32=0, F16=1, Q4_0=2, Q8_0=8,
 *     Q4_K=12, Q5_K=13, Q6_K=14, BF16=25).  Q4_K and Q5_K are the reference's
 *     own block layouts (src/Llmdot.Core/Tensors/Dequantize/DequantizeK.cs:76-140),
 *     not ggml's.
 *
 * References are relative to the cognisoc/dotllm repository root:
 *   ICB = src/Llmdot.Core/Inference/Backends/IComputeBackend.cs
 *   IE  = src/Llmdot.Core/Inference/InferenceEngine.cs
 */
#ifndef LLMDOT_HIP_H
#define LLMDOT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMDOT_OK 0
#define LLMDOT_E_INVALID (-1)      /* bad argument (ArgumentException)            */
#define LLMDOT_E_UNSUPPORTED (-2)  /* unsupported type/shape (NotSupportedException) */
#define LLMDOT_E_NOT_FOUND (-3)    /* unknown weight key (KeyNotFoundException)    */
#define LLMDOT_E_RANGE (-4)        /* position/token out of range (ArgumentOutOfRangeException) */
#define LLMDOT_E_DEVICE (-5)       /* HIP runtime error / no device                */
#define LLMDOT_E_NOMEM (-6)        /* device or host allocation failed             */

typedef struct llmdot_hip_ctx llmdot_hip_ctx;
typedef struct llmdot_hip_model llmdot_hip_model;

/* ---- context (the backend object; replaces `new MetalBackend()` /
 *      BackendFactory.CreateBestAvailable, src/Llmdot.Extensions.AI/BackendFactory.cs:8-39,
 *      and IDisposable.Dispose of ICB:7) ------------------------------------ */
const char* llmdot_hip_last_error(void);
int32_t llmdot_hip_device_count(int32_t* count);
int32_t llmdot_hip_create(int32_t device, llmdot_hip_ctx** out);
/* Releases the context.  With models created on it still alive the release
 * is deferred until the last of them is destroyed (the context accepts no new
 * models meanwhile), so destroy order mistakes leave no dangling handle. */
int32_t llmdot_hip_destroy(llmdot_hip_ctx* ctx);

typedef struct llmdot_hip_device_info {
    char name[64];
    char arch[32];          /* e.g. "gfx950" */
    int32_t compute_units;
    int32_t clock_mhz;
    uint64_t hbm_bytes;
} llmdot_hip_device_info;
int32_t llmdot_hip_get_device_info(llmdot_hip_ctx* ctx, llmdot_hip_device_info* out);

/* ---- persistent weights (the weightKey cache of MatMul, ICB:9; the Metal
 *      backend's UploadPersistentBytes("w_"+name), src/Llmdot.Metal/MetalBackend.cs:92-100).
 *      The bytes are the tensor's GGUF blocks, [rows][ByteCount(type, cols)],
 *      kept in HBM in that native layout.  Uploading an existing key replaces it;
 *      a key a live model reads keeps its buffer: new bytes of the same type and
 *      shape are copied in place, anything else is LLMDOT_E_INVALID. */
int32_t llmdot_hip_upload_weight(llmdot_hip_ctx* ctx, const char* key, uint32_t ggml_type,
                                 const void* bytes, size_t nbytes, int64_t rows, int64_t cols);
/* LLMDOT_E_INVALID while a live model reads the key. */
int32_t llmdot_hip_release_weight(llmdot_hip_ctx* ctx, const char* key);
int32_t llmdot_hip_has_weight(llmdot_hip_ctx* ctx, const char* key, int32_t* present);

/* ---- op level: one entry point per IComputeBackend member on the LLaMA
 *      decode path.  Inputs/outputs are host spans, as in the interface. */

/* ICB:9  MatMul(a, b, result, bType, aCols, bCols, weightKey).
 * result_len = aRows * bCols.  When weight_key names an uploaded weight, b may
 * be NULL and the resident copy is used; otherwise b is uploaded for this call
 * (and kept under weight_key when weight_key is non-NULL).  With aRows > 1
 * (TO:92-111) and a batched kernel for b_type, all rows run as one MFMA GEMM. */
int32_t llmdot_hip_matmul(llmdot_hip_ctx* ctx, const float* a, const void* b, float* result,
                          int64_t result_len, uint32_t b_type, int32_t a_cols, int32_t b_cols,
                          const char* weight_key);
/* ICB:10 MatMulF32(a, b, result, aCols, bCols, weightKey); b is [bCols][aCols] fp32. */
int32_t llmdot_hip_matmul_f32(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result,
                              int64_t result_len, int32_t a_cols, int32_t b_cols,
                              const char* weight_key);
/* ICB:11 RmsNorm(input, weights, output, epsilon) */
int32_t llmdot_hip_rms_norm(llmdot_hip_ctx* ctx, const float* input, const float* weights,
                            float* output, int32_t n, float epsilon);
/* ICB:14 ApplyRoPE(query, key, headDim, position, freqTable); NeoX half split
 * over 2*half_dim dims.  same_span != 0 means query and key alias (rotate once). */
int32_t llmdot_hip_apply_rope(llmdot_hip_ctx* ctx, float* query, float* key, int32_t head_dim,
                              int32_t position, const float* freq_table, int32_t half_dim,
                              int32_t same_span);
/* ICB:13 ApplyRoPE(query, key, headDim, position, freqBase, rotaryDim) */
int32_t llmdot_hip_apply_rope_base(llmdot_hip_ctx* ctx, float* query, float* key, int32_t head_dim,
                                   int32_t position, float freq_base, int32_t rotary_dim,
                                   int32_t same_span);
/* ICB:15 Softmax(input, softcap) in place; has_softcap = 0 for null. */
int32_t llmdot_hip_softmax(llmdot_hip_ctx* ctx, float* input, int32_t n, int32_t has_softcap,
                           float softcap);
/* ICB:16 Silu(input, result) and ICB:17 SiluInPlace(input) (pass input == result). */
int32_t llmdot_hip_silu(llmdot_hip_ctx* ctx, const float* input, float* result, int32_t n);
/* ICB:12 LayerNorm(input, weights, bias, output, epsilon); bias_or_null NULL is
 * the reference's empty bias span. */
int32_t llmdot_hip_layer_norm(llmdot_hip_ctx* ctx, const float* input, const float* weights,
                              const float* bias_or_null, float* output, int32_t n, float epsilon);
/* ICB:18 Gelu(input, result); ICB:19 GeluScalar(x) is the one-element call
 * (a single element takes the scalar form, as in VectorMath.Gelu). */
int32_t llmdot_hip_gelu(llmdot_hip_ctx* ctx, const float* input, float* result, int32_t n);
/* ICB:25 Softcap(input, cap) in place. */
int32_t llmdot_hip_softcap(llmdot_hip_ctx* ctx, float* input, int32_t n, float cap);
/* ICB:26 Conv1D(input, weights, output, kernelSize, inputDim): input and
 * weights are [input_dim][kernel_size], output [input_dim]; bit-exact. */
int32_t llmdot_hip_conv1d(llmdot_hip_ctx* ctx, const float* input, const float* weights, float* output,
                          int32_t kernel_size, int32_t input_dim);
/* ICB:20 Add(a, b) in place (result == a) and ICB:21 Add(a, b, result). */
int32_t llmdot_hip_add(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result, int32_t n);
/* ICB:22/23 Scale(input, scale[, result]) */
int32_t llmdot_hip_scale(llmdot_hip_ctx* ctx, const float* input, float scale, float* result, int32_t n);
/* ICB:24 Mul(a, b, result) */
int32_t llmdot_hip_mul(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result, int32_t n);
/* ICB:27 DequantizeToFloat(src, dst, type, numRows, rowElements); bit-exact. */
int32_t llmdot_hip_dequantize(llmdot_hip_ctx* ctx, const void* src, float* dst, uint32_t ggml_type,
                              int32_t num_rows, int32_t row_elements);
/* ICB:28 ArgMax(input): first index of the strict maximum. */
int32_t llmdot_hip_argmax(llmdot_hip_ctx* ctx, const float* input, int32_t n, int32_t* index);

/* SamplingOptions (src/Llmdot.Core/Sampling/SamplingOptions.cs:7-15) without
 * the seed: the caller draws the uniform values (Random.NextSingle()). */
typedef struct llmdot_hip_sampling {
    float temperature;       /* <= 0: greedy ArgMax */
    int32_t top_k;           /* 0 < top_k < n: top-k path (top_k <= 4096) */
    float top_p;             /* < 1: nucleus, when the top-k path is not taken */
    float repeat_penalty;
    int32_t repeat_window;   /* RepeatPenaltyWindowSize */
} llmdot_hip_sampling;
/* Sampler.Sample(logits, options, ..., recentTokens) (Sampler.cs:24-62) on the
 * device.  recent: the recent-token list (the last repeat_window entries are
 * penalised); r: the uniform draw SampleFromProbabilities makes
 * (Sampler.cs:160-161).  The top-k path reproduces the reference's arithmetic
 * (ties between equal values go to the smaller index); the top-p path matches
 * it except where r or top_p falls within float rounding of a cumulative
 * boundary.  LLMDOT_E_UNSUPPORTED for 4096 < top_k < n. */
int32_t llmdot_hip_sample(llmdot_hip_ctx* ctx, const float* logits, int32_t n, const llmdot_hip_sampling* opt,
                          const int32_t* recent, int32_t n_recent, float r, int32_t* token);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): llmdot_hip_sample over device pointers -- logits_dev [n],
 * recent_dev [n_recent] (may be NULL when n_recent is 0) and token_dev [1] all
 * in HBM -- enqueued on the context's stream (call llmdot_hip_synchronize
 * before reading token_dev).  The same kernels and results as
 * llmdot_hip_sample; their scratch (9 MiB + 768 B: the scaled logits and the
 * top-p selection buffers) is a static array of the library, one per device,
 * so this call allocates nothing.  n is at most
 * 262144 (LLMDOT_E_UNSUPPORTED beyond).  Every call on a device shares that
 * device's scratch: calls that overlap on one device (several contexts or
 * threads) race; calls on one context's stream do not. */
int32_t llmdot_hip_sample_noalloc(llmdot_hip_ctx* ctx, const float* logits_dev, int32_t n,
                                  const llmdot_hip_sampling* opt, const int32_t* recent_dev, int32_t n_recent,
                                  float r, int32_t* token_dev);

/* ---- device-pointer variants (inputs already resident in HBM; used by
 *      harnesses that time kernels without PCIe traffic). ------------------- */
int32_t llmdot_hip_device_alloc(llmdot_hip_ctx* ctx, size_t nbytes, void** dptr);
int32_t llmdot_hip_device_free(llmdot_hip_ctx* ctx, void* dptr);
int32_t llmdot_hip_memcpy_h2d(llmdot_hip_ctx* ctx, void* dst, const void* src, size_t nbytes);
int32_t llmdot_hip_memcpy_d2h(llmdot_hip_ctx* ctx, void* dst, const void* src, size_t nbytes);
int32_t llmdot_hip_synchronize(llmdot_hip_ctx* ctx);
/* y[rows] = W[rows x cols] . x[cols] on the context stream, all pointers in HBM
 * (W padded by the allocator as device_alloc does).  Asynchronous. */
int32_t llmdot_hip_gemv_device(llmdot_hip_ctx* ctx, uint32_t ggml_type, const void* w_dev,
                               const float* x_dev, float* y_dev, int32_t rows, int32_t cols);
/* Elapsed milliseconds of `iters` back-to-back gemv_device launches cycling
 * through n_weights weight copies, timed with HIP events on the context stream. */
int32_t llmdot_hip_time_gemv(llmdot_hip_ctx* ctx, uint32_t ggml_type, const void* const* w_devs,
                             int32_t n_weights, const float* x_dev, float* y_dev, int32_t rows,
                             int32_t cols, int32_t iters, float* ms);
/* Streaming probe (no reference counterpart; calibrates the HBM counters and
 * gives the practical bandwidth ceiling): `iters` launches of a kernel that
 * reads (mode 0) or writes (mode 1) `nbytes` of a fresh device buffer, 16 B
 * per thread; elapsed milliseconds via HIP events. */
int32_t llmdot_hip_stream_bench(llmdot_hip_ctx* ctx, size_t nbytes, int32_t mode, int32_t iters, float* ms);

/* ---- model level: the device-resident decode step (InferenceEngine.ProcessToken,
 *      IE:134-146, LLaMA-like template IE:184-196) and greedy Generate (IE:74-132). */
typedef struct llmdot_hip_model_desc {
    int32_t hidden;          /* TransformerConfig.HiddenSize          */
    int32_t layers;          /* LayerCount                            */
    int32_t heads;           /* HeadCount                             */
    int32_t kv_heads;        /* HeadCountKv                           */
    int32_t head_dim;        /* HeadDim                               */
    int32_t ffn;             /* FfnDim                                */
    int32_t vocab;           /* VocabSize                             */
    int32_t context;         /* KV capacity in positions (ContextLength) */
    int32_t rope_dim;        /* RopeDimensionCount (0 = head_dim)     */
    float eps;               /* NormEpsilon                           */
    float rope_base;         /* RopeFreqBase                          */
    float rope_linear_factor;/* RopeScalingFactor when type is Linear, else 1 */
    int32_t kv_fp16;         /* 1: fp16 KV cache (default), 0: fp32 as the reference */
    int32_t bos;             /* BosTokenId (used when the prompt is empty) */
    int32_t sliding_window;  /* SlidingWindow: attend to the last N positions (IE:385-387); 0 = all */
    /* Weight keys follow GGUF tensor names (src/Llmdot.Core/Loading/TensorNameResolver.cs:22-107):
     * token_embd.weight, output_norm.weight, output.weight (optional: tied to
     * token_embd), blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_output,ffn_norm,
     * ffn_gate,ffn_up,ffn_down}.weight, each optionally prefixed by key_prefix.
     * Fused Q/K/V (QkvLayout.Fused, ArchitectureResolver.cs:145-146): when any
     * layer has blk.N.attn_qkv.weight (heads*head_dim + 2*kv_heads*head_dim
     * rows, Q then K then V), every layer must, and it replaces attn_q/k/v
     * (IE:321-332).  Optional per layer: blk.N.attn_q_norm.weight and
     * blk.N.attn_k_norm.weight (head_dim each), per-head RmsNorm of q and k
     * before RoPE (IE:354-373). */
    const char* key_prefix;  /* may be NULL */
} llmdot_hip_model_desc;

int32_t llmdot_hip_model_create(llmdot_hip_ctx* ctx, const llmdot_hip_model_desc* desc,
                                llmdot_hip_model** out);
int32_t llmdot_hip_model_destroy(llmdot_hip_model* model);
/* KvCache.Reset (src/Llmdot.Core/Inference/KvCache.cs:40). */
int32_t llmdot_hip_model_reset(llmdot_hip_model* model);
/* ProcessToken(token, position): logits_or_null receives vocab floats;
 * argmax_or_null receives ArgMax(logits). */
int32_t llmdot_hip_decode_step(llmdot_hip_model* model, int32_t token, int32_t position,
                               float* logits_or_null, int32_t* argmax_or_null);
/* Prompt processing (the sequential loop of IE:84-88): tokens[i] at position
 * pos0 + i; outputs refer to the last token.  When every projection's type has
 * a batched kernel (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0) and n > 1 the tokens run as
 * chunks of batched MFMA GEMMs with causal attention over the chunk and the
 * cache; otherwise (or with LLMDOT_HIP_SEQ_PREFILL=1) one decode step per token.
 * Either way the KV cache ends as the sequential loop leaves it. */
int32_t llmdot_hip_prefill(llmdot_hip_model* model, const int32_t* tokens, int32_t n, int32_t pos0,
                           float* logits_or_null, int32_t* argmax_or_null);
/* Greedy Generate (IE:74-132, Sampler.cs:26-27): resets the cache, processes the
 * prompt (as llmdot_hip_prefill), then yields max_tokens tokens (stopping after
 * eos when eos >= 0).
 * The decode loop runs on the device (token feedback stays in HBM).
 * logits_out (nullable) receives [max_tokens][vocab]: the logits each token was
 * sampled from. */
int32_t llmdot_hip_generate(llmdot_hip_model* model, const int32_t* prompt, int32_t n_prompt,
                            int32_t max_tokens, int32_t eos, int32_t* tokens_out, int32_t* n_out,
                            float* logits_out);
/* Generate with SamplingOptions (IE:100-130, Sampler.cs:24-170): as
 * llmdot_hip_generate, each token drawn on the device by llmdot_hip_sample's
 * kernels from the logits in HBM, with the recent-token list kept on the device
 * (the prompt, then the generated tokens).  draws[i] is the uniform value token
 * i uses (max_tokens entries; for a seeded reference run, new
 * Random(seed).NextSingle() for every i). */
int32_t llmdot_hip_generate_sampled(llmdot_hip_model* model, const int32_t* prompt, int32_t n_prompt,
                                    int32_t max_tokens, int32_t eos, const llmdot_hip_sampling* opt,
                                    const float* draws, int32_t* tokens_out, int32_t* n_out, float* logits_out);
/* Streaming Generate: the IAsyncEnumerable of IE:74-132, a batch of tokens per
 * call.  begin resets the cache, processes the prompt and computes token 0
 * (greedy when opt_or_null is NULL or Temperature <= 0, else sampled with
 * draws[i] for token i, as llmdot_hip_generate_sampled).  Each next call
 * returns up to max_k (>= 1) further tokens in tokens_out (and, when
 * logits_out_or_null is given, [n][vocab] logits they were taken from), sets
 * *done once max_tokens tokens or eos (included, IE:112-115) have been
 * returned, and enqueues the step for the following token before it returns,
 * so the device computes while the caller consumes.  A caller that stops early
 * (cancellation, stop sequences) simply stops calling.  The last batch before
 * the end of the KV cache returns its tokens with LLMDOT_E_RANGE.  Any other
 * call that changes the model's state (decode_step, prefill, reset, a new
 * begin) ends the session; next then fails with LLMDOT_E_INVALID. */
int32_t llmdot_hip_generate_begin(llmdot_hip_model* model, const int32_t* prompt, int32_t n_prompt,
                                  int32_t max_tokens, int32_t eos, const llmdot_hip_sampling* opt_or_null,
                                  const float* draws_or_null);
int32_t llmdot_hip_generate_next(llmdot_hip_model* model, int32_t max_k, int32_t* tokens_out, int32_t* n_out,
                                 int32_t* done, float* logits_out_or_null);
/* Reads KV slot (layer, position) as fp32, kv_heads*head_dim floats each. */
int32_t llmdot_hip_kv_read(llmdot_hip_model* model, int32_t layer, int32_t position, float* k,
                           float* v);

/* ---- measurement hooks for the decode step --------------------------------
 * per_kernel == 0: runs `steps` greedy decode steps from the current state
 * (token feedback on the device) and returns the elapsed milliseconds measured
 * with HIP events on the model's stream.
 * per_kernel != 0: times the step's dominant kernel alone -- `steps` replays of
 * a graph of every layer's FFN gate/up GEMV, back to back between two HIP
 * events (distinct weights per layer, so nothing is served from cache; the
 * graph keeps host enqueue gaps out) -- and reports the launch count and their
 * algorithmic bytes. */
typedef struct llmdot_hip_step_timing {
    float total_ms;
    float gemv_ms;           /* per_kernel: elapsed time of the gate/up launches */
    int32_t gemv_launches;
    double gemv_bytes;       /* algorithmic bytes of those launches (weights + x + y) */
} llmdot_hip_step_timing;
/* Batched prompt processing of n tokens from pos0 (as llmdot_hip_prefill,
 * including the last token's LM head) timed with HIP events on the model's
 * stream; fails with LLMDOT_E_UNSUPPORTED when the model has no batched path.
 * No reference counterpart (the reference has no batched prompt path). */
int32_t llmdot_hip_model_time_prefill(llmdot_hip_model* model, const int32_t* tokens, int32_t n,
                                      int32_t pos0, float* ms);
int32_t llmdot_hip_model_time_decode(llmdot_hip_model* model, int32_t first_token, int32_t position,
                                     int32_t steps, int32_t per_kernel, llmdot_hip_step_timing* out);
/* Algorithmic HBM bytes of one decode step at `position`: quantized weights read
 * once + the KV rows read + one embedding row. */
int32_t llmdot_hip_model_step_bytes(llmdot_hip_model* model, int32_t position, double* bytes);
/* Fills KV positions [0, n) with seeded values (timing and parity at a given
 * context without running the prompt).  Element e (kv head * head_dim + d) of
 * the K (kind 0) or V (kind 1) row of (layer, pos) is
 *   key = (2 layer + kind) << 44 | pos << 20 | e,  z = SplitMix64 finaliser of
 *   seed + 0x9E3779B97F4A7C15 (key + 1),  value = ((z >> 40) / 2^24 - 0.5) * 3,
 * stored in the cache's element type (fp16: round to nearest even).  No
 * reference counterpart: a test and timing aid. */
int32_t llmdot_hip_model_kv_fill_random(llmdot_hip_model* model, int32_t n, uint64_t seed);

/* ---- GGUF tooling: reference-layout quantizers and seeded synthetic weights
 *      (the reference ships no quantizer).  Host-only; no device needed. */
int32_t llmdot_hip_quantize(uint32_t ggml_type, const float* src, int64_t rows, int64_t cols,
                            void* dst);
/* Fills dst with rows x cols weights ~ N(0, sigma), generated from (seed, element
 * index) so the result is independent of thread count, quantized to ggml_type.
 * ggml_type F32 writes the floats themselves. */
int32_t llmdot_hip_synth_weights(uint32_t ggml_type, int64_t rows, int64_t cols, uint64_t seed,
                                 float sigma, void* dst, int32_t threads);

#ifdef __cplusplus
}
#endif
#endif
