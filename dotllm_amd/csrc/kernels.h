// kernels.h -- host-side launchers for the HIP kernels (all asynchronous on `s`).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmdot {

// ---- dequant.hip ----
// Bit-exact TensorOps.DequantizeToFloat (TO:18-56) of num_rows rows.
hipError_t launch_dequant(const uint8_t* src, float* dst, uint32_t type, int num_rows, int row_elems,
                          hipStream_t s);
// Embedding row (InferenceEngine.GetEmbedding, IE:148-156): row *token_dev of
// the [vocab][hidden] table, bit-exact, into out.  The token id is read on the
// device so that a captured step can take it from the previous argmax.
hipError_t launch_embed(const uint8_t* table, uint32_t type, int hidden, const int32_t* token_dev,
                        float* out, hipStream_t s);

// ---- gemv.hip ----
struct XRec;   // xrec.h
enum GemvEpi : int { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GemvSeg {
    const uint8_t* w;   // [rows][row_bytes] blocks
    const uint8_t* w2;  // EPI_SWIGLU: the up matrix (w is the gate)
    float* out;         // rows outputs
    int rows;
    int groups;         // gemv_groups(rows)
};

struct ArgmaxState {
    float* cand_val;      // per 32-row group
    int32_t* cand_idx;
    uint32_t* counter;    // zero before launch; the last workgroup resets it
    int32_t* token_out;   // argmax result (next token)
    int32_t* pos;         // optional: incremented by the last workgroup
    int32_t* token_log;   // optional: token_log[*step] = argmax while *step < log_cap
    int32_t log_cap;
    int32_t* step;        // optional: incremented by the last workgroup
};

struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    int cols;             // reduction length K
    int splitk;           // K splits per 32-row group (gemv_pick_splitk)
    const float* x;       // fp32 input (the hidden state when norm != 0)
    const float* norm_w;  // RmsNorm weights applied on the fly by the fp32 path
    const XRec* xrec;     // input records (Q4_K path; ssq source when norm != 0)
    int norm;             // apply RmsNorm (1/rms from the records' ssq)
    float eps;
    XRec* rec_out;        // EPI_ADD / EPI_SWIGLU: records of the output vector
    const float* rec_w;   // norm weights of the output's consumer (nullable)
    float* partial;       // split-K scratch [groups][splitk][64]
    uint32_t* counters;   // split-K arrival counters [groups], zero between launches
    ArgmaxState am;       // EPI_ARGMAX
};

bool gemv_supported(uint32_t type);
int gemv_unit_elems(uint32_t type);
int gemv_groups(int rows);
int gemv_pick_splitk(uint32_t type, int cols, int rows_total);
int gemv_grid(const GemvArgs& a);
hipError_t launch_gemv(uint32_t type, int epi, const GemvArgs& a, hipStream_t s);
// Records of x (optionally multiplied by norm weights w) for n elements.
hipError_t launch_make_xrec(const float* x, const float* w, int n, XRec* out, hipStream_t s);

// ---- ops.hip (op-level IComputeBackend members) ----
hipError_t launch_rmsnorm(const float* in, const float* w, float* out, int n, float eps, hipStream_t s);
hipError_t launch_rope(float* q, float* k, const float* cosv, const float* sinv, int half, int same,
                       hipStream_t s);
hipError_t launch_softmax(float* x, int n, int has_softcap, float cap, hipStream_t s);
hipError_t launch_silu(const float* in, float* out, int n, hipStream_t s);
hipError_t launch_binary(int op, const float* a, const float* b, float* out, int n, hipStream_t s);  // 0 add, 1 mul
hipError_t launch_scale(const float* in, float sc, float* out, int n, hipStream_t s);
// ArgMax over n floats; st.cand_* sized for argmax_grid(n) workgroups.
int argmax_grid(int n);
hipError_t launch_argmax(const float* x, int n, const ArgmaxState& st, hipStream_t s);
// Position bookkeeping for a captured decode step.
hipError_t launch_set_scalar(int32_t* dst, int32_t v, hipStream_t s);
hipError_t launch_fill_random_half(void* dst, size_t n, uint64_t seed, int fp16, hipStream_t s);

// ---- attention.hip ----
struct AttnArgs {
    const float* q;         // [heads][head_dim] (pre-RoPE)
    const float* k;         // [kv_heads][head_dim] (pre-RoPE), current token
    const float* v;         // [kv_heads][head_dim], current token
    void* kcache;           // this layer: [kv_heads][context][head_dim], fp16 or fp32
    void* vcache;
    const float* cos_tab;   // [context][rope_half]
    const float* sin_tab;
    const int32_t* pos;     // device position T
    float* scores;          // [heads][context]
    float* chunk_max;       // [heads][max_chunks]
    float* part_out;        // [max_chunks][heads][head_dim]
    float* part_sum;        // [max_chunks][heads]
    uint32_t* counters;     // [kv_heads], zero; the last workgroup of each kv head resets its own
    float* out;             // [heads][head_dim]
    XRec* rec_out;          // records of out (nullable)
    int heads, kv_heads, head_dim, rope_half, context, kv_fp16;
};
int attn_chunk(int heads, int kv_heads);
int attn_max_chunks(int heads, int kv_heads, int context);
bool attn_supported(int heads, int kv_heads, int head_dim);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

}  // namespace llmdot
