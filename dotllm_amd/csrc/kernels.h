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
// device so that a captured step can take it from the previous argmax.  With
// w non-null also packs out for its RmsNorm consumer (see launch_pack_norm).
hipError_t launch_embed(const uint8_t* table, uint32_t type, int hidden, const int32_t* token_dev,
                        float* out, const float* w, float* packed, float* ssq, hipStream_t s);
// Packs x for an RmsNorm consumer: packed[i] = w[i] * x[i], ssq[i/4] = sum of x^2
// over 4 consecutive elements (n a multiple of 8).  The consumer adds the two
// sums of each 8-element group, ssq[2j] + ssq[2j+1].
hipError_t launch_pack_norm(const float* x, const float* w, int n, float* packed, float* ssq, hipStream_t s);

// ---- gemv.hip ----
enum GemvEpi : int { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GemvSeg {
    const uint8_t* w;   // [rows][row_bytes] blocks
    const uint8_t* w2;  // EPI_SWIGLU: the up matrix (w is the gate)
    float* out;         // rows outputs
    int rows;
    int wgs;            // workgroups of this segment (set by launch_gemv)
    uint32_t type;      // ggml type; 0 = the launch's type (Q4_K launches accept Q6_K segments)
};

struct ArgmaxState {
    float* cand_val;      // one candidate per workgroup of the first pass
    int32_t* cand_idx;
    int32_t cap;          // capacity of cand_*
    int32_t* token_out;   // argmax result (next token)
    int32_t* pos;         // optional: incremented by the second pass
    int32_t* token_log;   // optional: token_log[*step] = argmax while *step < log_cap
    int32_t log_cap;
    int32_t* step;        // optional: incremented by the second pass
    // element 0 of the reduced vector: VectorMath.ArgMax (VM:412-425) starts
    // from input[0] and compares with '>', so a NaN there is never replaced
    // and the result is 0; NaN elsewhere never wins (set by the launchers)
    const float* first;
    uint32_t* epoch;      // optional: incremented by the second pass (decode-step counter)
};

struct GemvArgs {
    GemvSeg seg[3];       // up to 3 matrices of the same type and width in one launch
    int nseg;
    int cols;             // reduction length K
    const float* x;       // fp32 input; with norm != 0 it is already w * h (RmsNorm weights applied)
    const float* ssq;     // norm != 0: sums of h^2 over consecutive 4-element groups, K/4 of them
    int norm;             // RmsNorm of the input: row sums are scaled by 1/sqrt(sum(h^2)/K + eps)
    float eps;
    // EPI_ADD: also pack the updated vector for its RmsNorm consumer:
    // pack_out[i] = pack_w[i] * out[i] and pack_ssq[i/4] = sum of out^2 over 4 rows
    const float* pack_w;
    float* pack_out;
    float* pack_ssq;
    ArgmaxState am;       // EPI_ARGMAX
};

bool gemv_supported(uint32_t type);
// Whether rows of `cols` elements fit the kernel (block multiple, <= 16384 wide).
bool gemv_width_ok(uint32_t type, int cols);
// Row batches per workgroup for a launch over rows_total output rows.
int gemv_plan(uint32_t type, int epi, int rows_total, int cols);
int gemv_rows_per_wg(uint32_t type, int epi, int nb);
// Upper bound of the grid (argmax candidate slots) for rows output rows.
int gemv_max_grid(uint32_t type, int epi, int rows, int cols);
hipError_t launch_gemv(uint32_t type, int epi, GemvArgs& a, hipStream_t s);

// ---- ops.hip (op-level IComputeBackend members) ----
hipError_t launch_rmsnorm(const float* in, const float* w, float* out, int n, float eps, hipStream_t s);
// Per-head RmsNorm in place: q [heads][hd] with wq, k [kv_heads][hd] with wk
// (either weight may be null: that side is left as it is).
hipError_t launch_qk_norm(float* q, float* k, const float* wq, const float* wk, int heads, int kv_heads, int hd,
                          float eps, hipStream_t s);
hipError_t launch_rope(float* q, float* k, const float* cosv, const float* sinv, int half, int same,
                       hipStream_t s);
hipError_t launch_softmax(float* x, int n, int has_softcap, float cap, hipStream_t s);
hipError_t launch_silu(const float* in, float* out, int n, hipStream_t s);
hipError_t launch_layernorm(const float* in, const float* w, const float* b, float* out, int n, float eps,
                            hipStream_t s);
hipError_t launch_gelu(const float* in, float* out, int n, hipStream_t s);
hipError_t launch_softcap(float* x, int n, float cap, hipStream_t s);
hipError_t launch_conv1d(const float* in, const float* w, float* out, int kernel_size, int input_dim, hipStream_t s);
hipError_t launch_binary(int op, const float* a, const float* b, float* out, int n, hipStream_t s);  // 0 add, 1 mul
hipError_t launch_scale(const float* in, float sc, float* out, int n, hipStream_t s);
// ArgMax over n floats (two launches); st.cand_* sized for argmax_grid(n).
int argmax_grid(int n);
hipError_t launch_argmax(const float* x, int n, const ArgmaxState& st, hipStream_t s);
// Second pass over ncand candidates: token_out, token_log/step, pos.
hipError_t launch_argmax_finish(const ArgmaxState& st, int ncand, hipStream_t s);
// Streaming probe: reads (mode 0) or writes (mode 1) nbytes (16 B per thread).
hipError_t launch_stream_probe(void* buf, size_t nbytes, int mode, uint32_t* sink, hipStream_t s);
// Position bookkeeping for a captured decode step.
hipError_t launch_set_scalar(int32_t* dst, int32_t v, hipStream_t s);
// Seeded KV contents at positions [0, n) of one cache (kind 0 = K, 1 = V); the values
// depend only on (seed, layer, kind, position, element).
hipError_t launch_kv_fill(uint8_t* cache, int kind, int layers, int kv_heads, int context, int hd, int n,
                          uint64_t seed, int fp16, hipStream_t s);

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
    float* out;             // [heads][head_dim]
    int heads, kv_heads, head_dim, rope_half, context, kv_fp16;
    // One-launch scores and values (fused != 0): the workgroups of a kv head
    // exchange their chunk maxima through tagged 64-bit slots, (tag << 32) |
    // float bits, stored and loaded at system scope (past the per-XCD L2s), so
    // a reader sees an older tag or the whole new pair; tag = epoch * layers +
    // layer + 1 is new for every (decode step, layer).  A wait gives up after
    // spin_max polls and sets *err.
    int fused;
    uint64_t* xmax;         // [kv_heads][group][max_chunks]
    const uint32_t* epoch;  // decode steps so far (advanced by the head's argmax pass)
    int layer, layers, spin_max;
    int32_t* err;
    // One-launch path only: the XCD-local chunk-maximum exchange (kv_heads a
    // multiple of 8): a one-dimensional grid puts every chunk of a kv head on
    // one XCD and the maxima go through that XCD's L2.  A chunk placed on
    // another XCD than the rest of its kv head makes that kv head's wait give
    // up (*err) rather than mix L2s.
    int xcd_exchange;
    // XCD-local form: the chunk partials as tagged words, (tag << 32) | float
    // bits: [max_chunks][heads][head_dim] sums of e.V, then [max_chunks][heads]
    // sums of e (max_chunks = attn_max_chunks)
    uint64_t* xpart;
    // SlidingWindow (IE:385-387): with window > 0 only the last `window`
    // positions attend (one-launch form only); 0 attends to all
    int window;
};
// Whether the XCD-local exchange suits the shape: kv heads a multiple of 8,
// and every live chunk of the kv heads one XCD serves (kv_heads / 8 of them,
// at most attn_max_chunks each) resident at once with a quarter to spare
// (the chunks of a kv head wait for each other); cus = compute units.
bool attn_xcd_fits(int heads, int kv_heads, int head_dim, int context, int kv_fp16, int cus);
// Whether workgroup w of a one-dimensional launch runs on XCD (w + o) mod 8,
// o fixed within the launch (what the XCD-local attention relies on), from a
// 2048-workgroup probe launch.
hipError_t attn_xcd_check(hipStream_t s, bool* ok);
// Slots of AttnArgs::xmax for `heads` q heads.
int attn_xmax_slots(int heads);
int attn_max_chunks(int heads, int kv_heads, int context);
// Whether the one-launch path applies (every chunk maximum of a head fits
// one wavefront's four slots per lane).
bool attn_fused_ok(int heads, int kv_heads, int head_dim, int context);
bool attn_supported(int heads, int kv_heads, int head_dim);
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

// ---- sample.hip (Sampler.Sample on the device) ----
constexpr int SAMPLE_MAX_K = 4096;   // largest top-k handled (TopK >= n takes the top-p path)
struct SampleArgs {
    const float* logits;      // [n]
    int n;
    float inv_temp;           // 1f / Temperature (> 0)
    int top_k;                // 0 < top_k < n: top-k path
    float top_p;              // < 1: nucleus (top-p path only)
    float penalty;            // RepeatPenalty
    int window;               // RepeatPenaltyWindowSize
    const int32_t* hist;      // tokens so far; the draw sees hist[0, hist_base + *step - 1)
    int hist_base;
    const int32_t* step;      // this is draw *step - 1 (the argmax pass has advanced it)
    const float* rvals;       // uniform draws: draw s uses rvals[s]
    float* work;              // [sample_work_floats(n)] scratch: probabilities, then the top-p scratch
    int32_t* token_out;       // the sampled token
    int32_t* token_log;       // optional: token_log[draw] = token while draw < log_cap
    int32_t log_cap;
    int32_t* hist_out;        // optional: hist_out[hist_base + draw] = token
};
bool sample_supported(int n, int top_k);
// Floats of SampleArgs::work for n logits: the probabilities, then (8-byte
// aligned) the top-p slow path's scratch: 3n 64-bit sort slots, n ids, n values.
__host__ __device__ constexpr size_t sample_comp_offset(int n) { return ((size_t)n + 1) & ~(size_t)1; }
__host__ __device__ constexpr size_t sample_work_floats(int n) { return sample_comp_offset(n) + 8 * (size_t)n; }
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);

// ---- prefill.hip (batched prompt processing) ----
// Activation planes of a [M][K] fp32 matrix: xh/xl [M][K] fp16 (x s = xh + xl,
// s a power of two per row), sh/sl [M][K/32] fp16 (group sums of x times s/32),
// xinv [M] = 1/s.
struct PfPlanes {
    _Float16 *xh, *xl, *sh, *sl;
    float* xinv;
};
struct PfAttnArgs {
    const float* q;           // [T][heads*head_dim] projections (pre-RoPE)
    const float* k;           // [T][kv_heads*head_dim]
    const float* v;
    float* qr;                // [T][heads*head_dim] rotated q
    void* kcache;             // this layer: [kv_heads][context][head_dim]
    void* vcache;
    const float* cos_tab;     // [context][rope_half]
    const float* sin_tab;
    float* scores;            // [heads][T][ld_scores]
    float* rowmax;            // [heads][T]
    float* out;               // [T][heads*head_dim]
    int T, pos0, ld_scores, heads, kv_heads, head_dim, rope_half, context, kv_fp16;
    // q, k and v as sums of q_split (k_split, v_split) K parts, q_part elements apart
    int q_split, k_split, v_split;
    int64_t q_part, k_part, v_part;
    // per-head Q/K RmsNorm weights [head_dim] applied before RoPE (null: none)
    // with eps; SlidingWindow (0: every earlier position; fp16 KV path only)
    const float *q_norm, *k_norm;
    float eps;
    int window;
};
bool prefill_gemm_supported(uint32_t type, int cols);
// Optional RmsNorm (norm_w non-null) of each row of x, then its planes.
hipError_t launch_prefill_planes(const float* x, int M, int K, const float* norm_w, float eps, const PfPlanes& p,
                                 hipStream_t s);
// out[M][ldo] (=, += for epi 1, SiLU(gate) * up for epi 2 with w = gate, w2 = up)
// of the planes times the [N][K] weight blocks, transposed.  ksplit > 1 (STORE
// only): K in ksplit parts of whole blocks, part p written at out + p * part_stride.
hipError_t launch_prefill_gemm(uint32_t type, int epi, const PfPlanes& p, const uint8_t* w, const uint8_t* w2, int M,
                               int N, int K, float* out, int ldo, hipStream_t s, int ksplit = 1,
                               int64_t part_stride = 0);
// K parts for an [M x N x K] prefill GEMM: more than 1 only for launches of
// fewer than 128 tiles, so that tiles x parts stays within 512 workgroups.
// (Splitting the 128-tile K/V projections of a 7B-shape 2048-token prompt too
// moved a deep-layer fp16 KV row one ulp past twice the oracle's reorder
// floor.)
int prefill_ksplit(uint32_t type, int M, int N, int K);
// Two STORE products over the same planes in one launch: out[M][ldo] of the
// [N][K] blocks w (N a multiple of 128 rows) and outb[M][ldob] of the [nb][K]
// blocks wb, same type; each output equals launch_prefill_gemm's.
hipError_t launch_prefill_gemm_pair(uint32_t type, const PfPlanes& p, const uint8_t* w, int N, float* out, int ldo,
                                    const uint8_t* wb, int nb, float* outb, int ldob, int M, int K, hipStream_t s);
// h[i] += sum over the nparts parts (stride elements apart) of parts[p][i], i < n.
hipError_t launch_prefill_add_parts(float* h, const float* parts, int nparts, int64_t stride, int64_t n,
                                    hipStream_t s);
hipError_t launch_prefill_rope_kv(const PfAttnArgs& a, hipStream_t s);
hipError_t launch_prefill_attention(const PfAttnArgs& a, hipStream_t s);
// Embedding rows tokens[0..T) (device ids) into out[T][hidden].
hipError_t launch_embed_rows(const uint8_t* table, uint32_t type, int hidden, const int32_t* tokens, int T, float* out,
                             hipStream_t s);

}  // namespace llmdot
