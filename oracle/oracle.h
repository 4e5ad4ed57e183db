/*
 * oracle.h -- CPU restatement of the llmdot ("dotllm") managed decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library computes the expected values for the HIP
 * implementation in dotllm_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only to compute expected
 * values or to time the reference algorithm on the host.  The product never
 * links, loads or calls it.
 *
 * The reference is C#/.NET (unbuildable here: no dotnet toolchain), so every
 * function below restates the reference source line by line in C99 with
 * IEEE binary32 arithmetic and no FMA contraction (-ffp-contract=off), which
 * matches RyuJIT (it never contracts a*b+c).  Citations are relative to the
 * reference repository root:
 *   IE  = src/Llmdot.Core/Inference/InferenceEngine.cs
 *   TO  = src/Llmdot.Core/Tensors/TensorOps.cs
 *   VM  = src/Llmdot.Core/Tensors/Numeric/VectorMath.cs
 *   DK  = src/Llmdot.Core/Tensors/Dequantize/DequantizeK.cs
 *   DB  = src/Llmdot.Core/Tensors/Dequantize/DequantizeBlock.cs
 *   HH  = src/Llmdot.Core/Tensors/Numeric/HalfHelper.cs
 *   KV  = src/Llmdot.Core/Inference/KvCache.cs
 *   GR  = src/Llmdot.Core/Loading/GgufReader.cs
 *   AR  = src/Llmdot.Core/Loading/ArchitectureResolver.cs
 *   TS  = src/Llmdot.Core/Tensors/TensorSize.cs
 *
 * Assumptions that no reference test pins (tolerance-level only, never
 * affecting dequantisation, which has no reductions):
 *   - System.Numerics.Vector<float>.Count == 8 (x86-64 AVX2);
 *   - Vector.Dot(v, One) sums lanes as ((v0+v1)+(v2+v3))+((v4+v5)+(v6+v7));
 *   - MathF.{Exp,Pow,Cos,Sin,Sqrt,Tanh} map to glibc expf/powf/cosf/sinf/...
 */
#ifndef LLMDOT_ORACLE_H
#define LLMDOT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType values (src/Llmdot.Core/Loading/GgmlType.cs:3-28). */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6,
    ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q8_1 = 9, ORC_Q2_K = 10, ORC_Q3_K = 11,
    ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_BF16 = 25
};

/* ---- numerics ---------------------------------------------------------- */
float   orc_half_to_float(uint16_t h);            /* HH:7-34 */
uint16_t orc_float_to_half(float f);              /* IEEE RNE; fp16 KV variant */
int64_t orc_byte_count(uint32_t type, uint64_t elements);   /* TS:7-24; -1 = unsupported */
int     orc_extract6(const uint8_t* src, int base, int bit); /* DK:189-199 */
float   orc_exp_approx(float x);                  /* one lane of VM:137-166 */

int  orc_dequantize(const uint8_t* src, float* dst, uint32_t type,
                    int num_rows, int row_elements);          /* TO:18-56 */
int  orc_matmul(const float* a, const uint8_t* b, float* result, int result_len,
                uint32_t b_type, int a_cols, int b_cols);      /* TO:60-112 */
void orc_matmul_f32(const float* a, const float* b, float* result, int result_len,
                    int a_cols, int b_cols);                   /* TO:437-504 */
void orc_rms_norm(const float* in, const float* w, float* out, int n, float eps); /* VM:308-340 */
void orc_softmax(float* x, int n, int has_softcap, float softcap);           /* VM:215-258 */
void orc_silu(const float* in, float* out, int n);            /* VM:99-116 */
float orc_gelu_scalar(float x);                                /* VM:169-170 */
void orc_gelu(const float* in, float* out, int n);            /* VM:172-193 */
void orc_softcap(float* x, int n, float cap);                 /* VM:286-302 */
void orc_layer_norm(const float* in, const float* w, const float* b, float* out,
                    int n, float eps);                        /* VM:342-405 */
void orc_conv1d(const float* in, const float* w, float* out, int kernel_size,
                int input_dim);                               /* TO:745-775 */
void orc_silu_inplace(float* x, int n);                       /* VM:118-135 */
void orc_add_inplace(float* a, const float* b, int n);        /* VM:27-42 */
void orc_add(const float* a, const float* b, float* out, int n);   /* VM:10-25 */
void orc_scale(const float* in, float s, float* out, int n);  /* VM:44-59 */
void orc_mul(const float* a, const float* b, float* out, int n);   /* VM:78-93 */
void orc_rope_table(float* q, float* k, int head_dim, int position,
                    const float* freq, int half_dim, int same_span);  /* TO:679-743 */
void orc_rope_base(float* q, float* k, int head_dim, int position,
                   float freq_base, int rotary_dim, int same_span);   /* TO:658-677 */
int  orc_argmax(const float* x, int n);                       /* VM:412-425 */
/* Sampler.Sample (Sampler.cs:24-62) with the uniform draw r given. */
int  orc_sample(const float* logits, int n, float temperature, int top_k, float top_p, float penalty, int window,
                const int* recent, int n_recent, float r);
/* aliased = 1: the reference as written (FindNucleus writes into the buffer it
 * reads); 0: FindNucleus with a buffer of its own. */
int  orc_sample_ex(const float* logits, int n, float temperature, int top_k, float top_p, float penalty,
                   int window, const int* recent, int n_recent, float r, int aliased);

void orc_set_threads(int n);   /* row-parallel GEMV/attention; results are bitwise identical */
int  orc_get_threads(void);
/* Reduction order of orc_prefill (and of RmsNorm, Softmax and attention,
 * which it shares with orc_process_token): 0 (default) is the reference's;
 * 1, 2 and 3 are other valid fp32 orders -- 16, 4 and 32 lanes instead of
 * Vector<float>'s 8 (what .NET gives with 512-bit, 128-bit and wider vectors),
 * a partial per 32-, 64- and 16-element group in the scalar K-quant GEMV sums,
 * per-64-, 32- and 128-position partials in the attention's value sum.  They
 * measure how far summation order alone moves the results (the tolerance
 * floor of tests against other implementations); the fused single-row GEMVs
 * of orc_process_token ignore the order. */
void orc_set_order(int order);
int  orc_get_order(void);

/* ---- model ------------------------------------------------------------- */
typedef struct orc_config {
    int hidden, layers, context, vocab, ffn;
    int heads, kv_heads, head_dim, rope_dim;
    int rope_scaling_linear;      /* 1 when rope.scaling.type == "linear" */
    float rope_scaling_factor;
    float eps, rope_base;
    int bos, eos;
    int tied_embeddings;
    int sliding_window;
} orc_config;

typedef struct orc_model orc_model;

/* Parses a GGUF image in memory (the buffer must outlive the model). */
orc_model* orc_model_open_buffer(const uint8_t* buf, size_t len, int kv_fp16,
                                 char* err, int errlen);
orc_model* orc_model_open_file(const char* path, int kv_fp16, char* err, int errlen);
void orc_model_close(orc_model* m);
void orc_model_config(const orc_model* m, orc_config* out);
/* Overrides the KV-cache capacity (ContextLength); 0 keeps the GGUF value. */
int  orc_model_set_context(orc_model* m, int context);

/* ProcessToken (IE:134-146): writes VocabSize logits. */
int orc_process_token(orc_model* m, int token, int position, float* logits);
/* The last token's logits and the KV cache of n sequential ProcessToken calls
 * (tokens[i] at position pos0 + i, IE:84-88), computed with the tokens of a
 * chunk going through each layer together; bitwise identical to the loop.
 * No reference counterpart (test infrastructure for long prompts). */
int orc_prefill(orc_model* m, const int* tokens, int n, int pos0, float* logits);
/* out[r][0..b_cols) = MatMul of activation row r (aRows == 1 each, TO:60-90)
 * for r < rows, through orc_prefill's batched path: bitwise orc_matmul per
 * row (tests pin this for every type). */
int orc_matmul_rows(const float* a, int rows, const uint8_t* b, uint32_t type, int a_cols, int b_cols, float* out);
/* Generate (IE:74-132) with greedy sampling.  tokens_out holds max_tokens
 * entries; logits_out (nullable) holds [max_tokens][vocab]: the logits each
 * sampled token was taken from.  eos < 0 disables the EOS stop. */
int orc_generate(orc_model* m, const int* prompt, int n_prompt, int max_tokens,
                 int eos, int* tokens_out, int* n_out, float* logits_out);
/* Fills KV positions [0, n) with the seeded values llmdot_hip_model_kv_fill_random
 * writes (timing and long-context parity). */
int orc_kv_fill_random(orc_model* m, int n, uint64_t seed);
/* Copies one KV slot (kvDim floats each). */
int orc_kv_read(const orc_model* m, int layer, int position, float* k, float* v);

#ifdef __cplusplus
}
#endif
#endif
