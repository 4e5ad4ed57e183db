// backend.hip -- host side of libllmdot_hip.so: the C ABI declared in
// include/llmdot_hip.h.
//
//   * llmdot_hip_ctx   : one device + one HIP stream + the persistent weight
//                        table keyed like the reference's weightKey cache
//                        (src/Llmdot.Metal/MetalBackend.cs:92-100).
//   * op-level calls   : IComputeBackend members (src/Llmdot.Core/Inference/
//                        Backends/IComputeBackend.cs:7-29) over host spans.
//   * llmdot_hip_model : the decode step of InferenceEngine (IE:134-196) with
//                        weights, KV cache and activations resident in HBM.
//                        One step = embed + per layer [QKV GEMV(+RmsNorm),
//                        attention (2 kernels), O GEMV(+residual), gate/up
//                        GEMV(+RmsNorm, SwiGLU), down GEMV(+residual)] + LM
//                        head GEMV(+final RmsNorm, argmax).  The step reads the
//                        token and position from device memory and the head
//                        writes the next token and position back, so a single
//                        captured HIP graph is replayed for every token and
//                        the greedy loop never returns to the host.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <deque>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/llmdot_hip.h"
#include "common.h"
#include "kernels.h"

using namespace llmdot;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIPCHK(expr)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return fail(LLMDOT_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));       \
    } while (0)

struct Weight {
    uint32_t type = 0;
    int64_t rows = 0, cols = 0;
    size_t nbytes = 0;
    uint8_t* dev = nullptr;
    int pins = 0;   // live models reading it (their captured steps hold dev)
};

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        hipError_t e = hipMalloc(&p, n + WEIGHT_PAD);
        if (e == hipSuccess) cap = n;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

bool env_flag(const char* name) {
    const char* v = getenv(name);
    return v && *v && strcmp(v, "0") != 0;
}
bool env_is_zero(const char* name) {
    const char* v = getenv(name);
    return v && strcmp(v, "0") == 0;
}

}  // namespace

struct llmdot_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::unordered_map<std::string, Weight> weights;
    DevBuf scratch[6];
    DevBuf planes[5];            // batched MatMul: activation planes (xh, xl, sh, sl, xinv)
    int32_t* am_ints = nullptr;  // [0] token_out
    float* am_val = nullptr;
    int32_t* am_idx = nullptr;
    int am_cap = 0;
    // two more streams (default priority) for independent prompt GEMMs, forked
    // from and joined back into `stream` with events
    hipStream_t side[2] = {nullptr, nullptr};
    hipEvent_t fork = nullptr, join[2] = {nullptr, nullptr};
    // models created on this context and not yet destroyed; llmdot_hip_destroy
    // with models alive defers the release to the last model's destroy
    int models = 0;
    bool closing = false;
    // fp32 copies models keep of non-F32 norm weights (LM:63-75): an in-place
    // re-upload of the key converts the new bytes into each of them
    struct NormCopy {
        std::string key;
        float* dst;
        int n;
        const void* owner;
    };
    std::vector<NormCopy> norm_copies;
};

namespace {

int ensure_device(llmdot_hip_ctx* ctx) {
    HIPCHK(hipSetDevice(ctx->device));
    return 0;
}

// Fresh device memory is zeroed, and host bytes are copied in, on the context
// stream, which is then waited for.  A plain hipMemset / hipMemcpy runs on the
// null stream, which the context stream (created non-blocking) and the side
// streams forked from it do not wait for: work enqueued right after could read
// or write the buffer before the zeros or the bytes land.
int zero_fresh(llmdot_hip_ctx* ctx, void* p, size_t n) {
    HIPCHK(hipMemsetAsync(p, 0, n, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}
int copy_in(llmdot_hip_ctx* ctx, void* dst, const void* src, size_t n) {
    HIPCHK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

int ensure_argmax(llmdot_hip_ctx* ctx, int n) {
    if (!ctx->am_ints) {
        HIPCHK(hipMalloc(&ctx->am_ints, 64));
        if (int rc = zero_fresh(ctx, ctx->am_ints, 64)) return rc;
    }
    if (n > ctx->am_cap) {
        if (ctx->am_val) (void)hipFree(ctx->am_val);
        if (ctx->am_idx) (void)hipFree(ctx->am_idx);
        ctx->am_val = nullptr; ctx->am_idx = nullptr; ctx->am_cap = 0;
        HIPCHK(hipMalloc(&ctx->am_val, sizeof(float) * (size_t)n));
        HIPCHK(hipMalloc(&ctx->am_idx, sizeof(int32_t) * (size_t)n));
        ctx->am_cap = n;
    }
    return 0;
}

int upload(llmdot_hip_ctx* ctx, const std::string& key, uint32_t type, const void* bytes, size_t nbytes,
           int64_t rows, int64_t cols, const Weight** out) {
    if (block_elems(type) == 0) return fail(LLMDOT_E_UNSUPPORTED, "unsupported ggml type " + std::to_string(type));
    if (rows <= 0 || cols <= 0 || cols % block_elems(type) != 0)
        return fail(LLMDOT_E_INVALID, "bad shape for weight '" + key + "'");
    const int64_t need = rows * byte_count(type, cols);
    if ((int64_t)nbytes < need)
        return fail(LLMDOT_E_INVALID, "weight '" + key + "' has " + std::to_string(nbytes) + " bytes, needs " +
                                          std::to_string(need));
    auto it = ctx->weights.find(key);
    if (it != ctx->weights.end()) {
        Weight& old = it->second;
        if (old.pins > 0) {   // a model's captured step reads this buffer: new bytes in place only
            if (old.type != type || old.rows != rows || old.cols != cols)
                return fail(LLMDOT_E_INVALID, "weight '" + key + "' is in use by a model with another shape or type");
            HIPCHK(hipStreamSynchronize(ctx->stream));
            if (int rc = copy_in(ctx, old.dev, bytes, (size_t)need)) return rc;
            for (const auto& c : ctx->norm_copies)   // models reading an fp32 copy of this norm
                if (c.key == key) HIPCHK(launch_dequant(old.dev, c.dst, type, 1, c.n, ctx->stream));
            HIPCHK(hipStreamSynchronize(ctx->stream));
            if (out) *out = &old;
            return 0;
        }
        (void)hipFree(old.dev);
        ctx->weights.erase(it);
    }
    Weight w;
    w.type = type; w.rows = rows; w.cols = cols; w.nbytes = (size_t)need;
    HIPCHK(hipMalloc(&w.dev, (size_t)need + WEIGHT_PAD));
    if (int rc = zero_fresh(ctx, w.dev + need, WEIGHT_PAD)) { (void)hipFree(w.dev); return rc; }
    if (int rc = copy_in(ctx, w.dev, bytes, (size_t)need)) { (void)hipFree(w.dev); return rc; }
    auto& slot = ctx->weights[key];
    slot = w;
    if (out) *out = &slot;
    return 0;
}

}  // namespace

// ======================================================= allocation-free ==
// llmdot_hip_sample_noalloc keeps its scratch in this file-scope device array
// instead of allocating: the sampler's work vector (sample_work_floats(n):
// the probabilities and the top-p sort scratch, 9 floats per logit), the
// argmax candidates (one per 4096 logits) and two words (the draw counter and
// the uniform draw).  Each device holds its own copy until the process ends;
// its address is looked up once per device (with that device current) when a
// context is created, and only that address is handed to kernels and copies.
namespace {
constexpr int NOALLOC_MAX_N = 262144;                                  // logits per call
constexpr int NOALLOC_CAND = NOALLOC_MAX_N / 4096;                     // argmax_grid(NOALLOC_MAX_N)
constexpr size_t NOALLOC_WORK = sizeof(float) * (((size_t)NOALLOC_MAX_N + 1) & ~(size_t)1) +
                                sizeof(float) * 8 * (size_t)NOALLOC_MAX_N;  // sample_work_floats(NOALLOC_MAX_N)
static_assert(NOALLOC_WORK == sizeof(float) * sample_work_floats(NOALLOC_MAX_N), "sampler work size");
constexpr size_t NOALLOC_CAND_VAL = NOALLOC_WORK;                      // float[NOALLOC_CAND]
constexpr size_t NOALLOC_CAND_IDX = NOALLOC_CAND_VAL + 4 * NOALLOC_CAND;   // int32[NOALLOC_CAND]
constexpr size_t NOALLOC_INTS = NOALLOC_CAND_IDX + 4 * NOALLOC_CAND;   // [0] draw counter, [1] draw bits
constexpr size_t NOALLOC_BYTES = NOALLOC_INTS + 256;                   // 9 MiB + 768 B
constexpr int NOALLOC_MAX_DEVICES = 64;
// Elements of each prefill K-part buffer: a split keeps tiles (of 128 x 128)
// x parts <= 512 (prefill_ksplit).
constexpr int64_t PF_PARTS_MAX = 512LL * 128 * 128;

__attribute__((used)) __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};
bool g_scratch_done[NOALLOC_MAX_DEVICES] = {};
std::string g_scratch_err[NOALLOC_MAX_DEVICES];

// Once per device, with `device` current: the device address of `scratch`.
void scratch_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) return;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_done[device]) return;
    g_scratch_done[device] = true;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        g_scratch_err[device] = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        (void)hipGetLastError();
        return;
    }
    g_scratch_ptr[device] = static_cast<uint8_t*>(p);
}

uint8_t* scratch_of(int device, std::string* err) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) { *err = "device index beyond the scratch table"; return nullptr; }
    if (!g_scratch_ptr[device]) *err = g_scratch_err[device].empty() ? "scratch not set up" : g_scratch_err[device];
    return g_scratch_ptr[device];
}
}  // namespace

// =============================================================== context ==

extern "C" const char* llmdot_hip_last_error(void) { return g_err.c_str(); }

extern "C" int32_t llmdot_hip_device_count(int32_t* count) {
    if (!count) return fail(LLMDOT_E_INVALID, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) { *count = 0; return fail(LLMDOT_E_DEVICE, std::string("hipGetDeviceCount: ") + hipGetErrorString(e)); }
    *count = n;
    return 0;
}

extern "C" int32_t llmdot_hip_create(int32_t device, llmdot_hip_ctx** out) {
    if (!out) return fail(LLMDOT_E_INVALID, "null out");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(LLMDOT_E_DEVICE, "no HIP device available");
    if (device < 0 || device >= n) return fail(LLMDOT_E_INVALID, "device index out of range");
    auto* ctx = new llmdot_hip_ctx();
    ctx->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(LLMDOT_E_DEVICE, std::string("stream creation failed: ") + hipGetErrorString(e));
    }
    scratch_setup(device);   // llmdot_hip_sample_noalloc reports a failure here
    *out = ctx;
    return 0;
}

namespace {
void ctx_release(llmdot_hip_ctx* ctx) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->weights) (void)hipFree(kv.second.dev);
    for (auto& b : ctx->scratch) b.release();
    for (auto& b : ctx->planes) b.release();
    if (ctx->am_ints) (void)hipFree(ctx->am_ints);
    if (ctx->am_val) (void)hipFree(ctx->am_val);
    if (ctx->am_idx) (void)hipFree(ctx->am_idx);
    for (int i = 0; i < 2; i++) {
        if (ctx->side[i]) {
            (void)hipStreamSynchronize(ctx->side[i]);
            (void)hipStreamDestroy(ctx->side[i]);
        }
        if (ctx->join[i]) (void)hipEventDestroy(ctx->join[i]);
    }
    if (ctx->fork) (void)hipEventDestroy(ctx->fork);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}
}  // namespace

extern "C" int32_t llmdot_hip_destroy(llmdot_hip_ctx* ctx) {
    if (!ctx) return 0;
    if (ctx->models > 0) {   // its models still use the stream and weights
        ctx->closing = true;
        return 0;
    }
    ctx_release(ctx);
    return 0;
}

extern "C" int32_t llmdot_hip_get_device_info(llmdot_hip_ctx* ctx, llmdot_hip_device_info* out) {
    if (!ctx || !out) return fail(LLMDOT_E_INVALID, "null argument");
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, ctx->device));
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s", p.name);
    snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->clock_mhz = p.clockRate / 1000;
    out->hbm_bytes = (uint64_t)p.totalGlobalMem;
    return 0;
}

extern "C" int32_t llmdot_hip_upload_weight(llmdot_hip_ctx* ctx, const char* key, uint32_t type, const void* bytes,
                                            size_t nbytes, int64_t rows, int64_t cols) {
    if (!ctx || !key || !bytes) return fail(LLMDOT_E_INVALID, "null argument");
    if (int rc = ensure_device(ctx)) return rc;
    return upload(ctx, key, type, bytes, nbytes, rows, cols, nullptr);
}

extern "C" int32_t llmdot_hip_release_weight(llmdot_hip_ctx* ctx, const char* key) {
    if (!ctx || !key) return fail(LLMDOT_E_INVALID, "null argument");
    auto it = ctx->weights.find(key);
    if (it == ctx->weights.end()) return fail(LLMDOT_E_NOT_FOUND, std::string("Tensor '") + key + "' not found.");
    if (it->second.pins > 0) return fail(LLMDOT_E_INVALID, std::string("Tensor '") + key + "' is in use by a model.");
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(it->second.dev);
    ctx->weights.erase(it);
    return 0;
}

extern "C" int32_t llmdot_hip_has_weight(llmdot_hip_ctx* ctx, const char* key, int32_t* present) {
    if (!ctx || !key || !present) return fail(LLMDOT_E_INVALID, "null argument");
    *present = ctx->weights.count(key) ? 1 : 0;
    return 0;
}

// ============================================================== op level ==

namespace {

// One GEMV y = W x on the context stream (x, y, W in device memory).
int ctx_gemv(llmdot_hip_ctx* ctx, uint32_t type, const uint8_t* w, const float* x, float* y, int rows, int cols) {
    if (!gemv_width_ok(type, cols))
        return fail(LLMDOT_E_UNSUPPORTED, "GEMV width " + std::to_string(cols) + " not supported for type " + std::to_string(type));
    GemvArgs ga{};
    ga.nseg = 1;
    ga.seg[0] = {w, nullptr, y, rows, 0};
    ga.cols = cols;
    ga.x = x;
    HIPCHK(launch_gemv(type, EPI_STORE, ga, ctx->stream));
    return 0;
}

template <typename T>
int stage_in(llmdot_hip_ctx* ctx, int slot, const T* host, size_t n, T** dev) {
    HIPCHK(ctx->scratch[slot].ensure(sizeof(T) * (n ? n : 1)));
    *dev = reinterpret_cast<T*>(ctx->scratch[slot].p);
    if (n && host) HIPCHK(hipMemcpyAsync(*dev, host, sizeof(T) * n, hipMemcpyHostToDevice, ctx->stream));
    return 0;
}

// Activation-plane buffers for M rows of K elements.
int ctx_planes(llmdot_hip_ctx* ctx, int M, int K, PfPlanes* pl) {
    const size_t n = (size_t)M * K;
    HIPCHK(ctx->planes[0].ensure(2 * n));
    HIPCHK(ctx->planes[1].ensure(2 * n));
    HIPCHK(ctx->planes[2].ensure(2 * (n / 32 + 8)));
    HIPCHK(ctx->planes[3].ensure(2 * (n / 32 + 8)));
    HIPCHK(ctx->planes[4].ensure(4 * (size_t)M));
    pl->xh = (_Float16*)ctx->planes[0].p; pl->xl = (_Float16*)ctx->planes[1].p;
    pl->sh = (_Float16*)ctx->planes[2].p; pl->sl = (_Float16*)ctx->planes[3].p;
    pl->xinv = (float*)ctx->planes[4].p;
    return 0;
}

int copy_out(llmdot_hip_ctx* ctx, void* host, const void* dev, size_t nbytes) {
    HIPCHK(hipMemcpyAsync(host, dev, nbytes, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

int matmul_common(llmdot_hip_ctx* ctx, const float* a, const void* b, float* result, int64_t result_len,
                  uint32_t type, int a_cols, int b_cols, const char* weight_key) {
    if (!ctx || !a || !result) return fail(LLMDOT_E_INVALID, "null argument");
    if (a_cols <= 0 || b_cols <= 0 || result_len < b_cols || result_len % b_cols != 0)
        return fail(LLMDOT_E_INVALID, "bad MatMul shape");
    if (!gemv_supported(type)) return fail(LLMDOT_E_UNSUPPORTED, "MatMul: unsupported weight type " + std::to_string(type));
    if (a_cols % block_elems(type) != 0) return fail(LLMDOT_E_UNSUPPORTED, "MatMul: width not a multiple of the block size");
    if (!gemv_width_ok(type, a_cols)) return fail(LLMDOT_E_UNSUPPORTED, "MatMul: width " + std::to_string(a_cols) + " too large");
    if (int rc = ensure_device(ctx)) return rc;
    const Weight* w = nullptr;
    Weight tmp;
    if (weight_key) {
        auto it = ctx->weights.find(weight_key);
        if (it != ctx->weights.end()) {
            w = &it->second;
            if (w->type != type || w->cols != a_cols || w->rows != b_cols)
                return fail(LLMDOT_E_INVALID, std::string("weight '") + weight_key + "' shape/type mismatch");
        }
    }
    if (!w) {
        if (!b) return fail(LLMDOT_E_NOT_FOUND, std::string("Tensor '") + (weight_key ? weight_key : "") + "' not found.");
        if (weight_key) {
            if (int rc = upload(ctx, weight_key, type, b, (size_t)(b_cols * byte_count(type, a_cols)), b_cols, a_cols, &w)) return rc;
        } else {
            const size_t nb = (size_t)(b_cols * byte_count(type, a_cols));
            HIPCHK(ctx->scratch[5].ensure(nb));
            HIPCHK(hipMemcpyAsync(ctx->scratch[5].p, b, nb, hipMemcpyHostToDevice, ctx->stream));
            HIPCHK(hipMemsetAsync((uint8_t*)ctx->scratch[5].p + nb, 0, WEIGHT_PAD, ctx->stream));
            tmp.type = type; tmp.rows = b_cols; tmp.cols = a_cols; tmp.nbytes = nb;
            tmp.dev = (uint8_t*)ctx->scratch[5].p;
            w = &tmp;
        }
    }
    const int64_t a_rows = result_len / b_cols;
    float *da, *dy;
    if (int rc = stage_in(ctx, 0, a, (size_t)(a_rows * a_cols), &da)) return rc;
    if (int rc = stage_in<float>(ctx, 1, nullptr, (size_t)result_len, &dy)) return rc;
    if (a_rows > 1 && a_rows <= INT32_MAX && prefill_gemm_supported(type, a_cols)) {
        // several activation rows (TO:92-111): one MFMA GEMM over all of them
        PfPlanes pl;
        if (int rc = ctx_planes(ctx, (int)a_rows, a_cols, &pl)) return rc;
        HIPCHK(launch_prefill_planes(da, (int)a_rows, a_cols, nullptr, 0.f, pl, ctx->stream));
        HIPCHK(launch_prefill_gemm(type, 0, pl, w->dev, nullptr, (int)a_rows, b_cols, a_cols, dy, b_cols, ctx->stream));
        return copy_out(ctx, result, dy, sizeof(float) * (size_t)result_len);
    }
    for (int64_t r = 0; r < a_rows; r++)
        if (int rc = ctx_gemv(ctx, type, w->dev, da + r * a_cols, dy + r * b_cols, b_cols, a_cols)) return rc;
    return copy_out(ctx, result, dy, sizeof(float) * (size_t)result_len);
}

}  // namespace

extern "C" int32_t llmdot_hip_matmul(llmdot_hip_ctx* ctx, const float* a, const void* b, float* result,
                                     int64_t result_len, uint32_t b_type, int32_t a_cols, int32_t b_cols,
                                     const char* weight_key) {
    return matmul_common(ctx, a, b, result, result_len, b_type, a_cols, b_cols, weight_key);
}

extern "C" int32_t llmdot_hip_matmul_f32(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result,
                                         int64_t result_len, int32_t a_cols, int32_t b_cols, const char* weight_key) {
    return matmul_common(ctx, a, b, result, result_len, GGML_F32, a_cols, b_cols, weight_key);
}

extern "C" int32_t llmdot_hip_rms_norm(llmdot_hip_ctx* ctx, const float* input, const float* weights, float* output,
                                       int32_t n, float eps) {
    if (!ctx || !input || !weights || !output || n <= 0) return fail(LLMDOT_E_INVALID, "bad RmsNorm arguments");
    if (int rc = ensure_device(ctx)) return rc;
    float *di, *dw, *dy;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &di)) return rc;
    if (int rc = stage_in(ctx, 1, weights, (size_t)n, &dw)) return rc;
    if (int rc = stage_in<float>(ctx, 2, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_rmsnorm(di, dw, dy, n, eps, ctx->stream));
    return copy_out(ctx, output, dy, sizeof(float) * (size_t)n);
}

namespace {
int rope_common(llmdot_hip_ctx* ctx, float* q, float* k, int head_dim, const std::vector<float>& cs,
                const std::vector<float>& sn, int same) {
    const int half = (int)cs.size();
    if (2 * half > head_dim) return fail(LLMDOT_E_INVALID, "rotary dims exceed head_dim");
    float *dq, *dk = nullptr, *dc, *ds;
    if (int rc = ensure_device(ctx)) return rc;
    if (int rc = stage_in(ctx, 0, q, (size_t)head_dim, &dq)) return rc;
    if (!same) { if (int rc = stage_in(ctx, 1, k, (size_t)head_dim, &dk)) return rc; }
    if (int rc = stage_in(ctx, 2, cs.data(), cs.size(), &dc)) return rc;
    if (int rc = stage_in(ctx, 3, sn.data(), sn.size(), &ds)) return rc;
    HIPCHK(launch_rope(dq, same ? dq : dk, dc, ds, half, same, ctx->stream));
    HIPCHK(hipMemcpyAsync(q, dq, sizeof(float) * (size_t)head_dim, hipMemcpyDeviceToHost, ctx->stream));
    if (!same) HIPCHK(hipMemcpyAsync(k, dk, sizeof(float) * (size_t)head_dim, hipMemcpyDeviceToHost, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}
}  // namespace

extern "C" int32_t llmdot_hip_apply_rope(llmdot_hip_ctx* ctx, float* query, float* key, int32_t head_dim, int32_t position,
                                         const float* freq_table, int32_t half_dim, int32_t same_span) {
    if (!ctx || !query || !freq_table || half_dim < 0 || head_dim <= 0) return fail(LLMDOT_E_INVALID, "bad ApplyRoPE arguments");
    const int same = same_span || key == nullptr || key == query;
    std::vector<float> cs((size_t)half_dim), sn((size_t)half_dim);
    for (int i = 0; i < half_dim; i++) {   // TO:688-693: angles and libm cos/sin on the host, as the reference
        float angle = (float)position * freq_table[i];
        cs[i] = cosf(angle);
        sn[i] = sinf(angle);
    }
    return rope_common(ctx, query, key, head_dim, cs, sn, same);
}

extern "C" int32_t llmdot_hip_apply_rope_base(llmdot_hip_ctx* ctx, float* query, float* key, int32_t head_dim,
                                              int32_t position, float freq_base, int32_t rotary_dim, int32_t same_span) {
    if (!ctx || !query || head_dim <= 0) return fail(LLMDOT_E_INVALID, "bad ApplyRoPE arguments");
    const int same = same_span || key == nullptr || key == query;
    const int actual = rotary_dim > 0 ? rotary_dim : head_dim;
    const int half = actual / 2;
    std::vector<float> cs((size_t)half), sn((size_t)half);
    for (int i = 0; i < half; i++) {       // TO:668-674
        float freq = 1.0f / powf(freq_base, 2.0f * (float)i / (float)actual);
        float angle = (float)position * freq;
        cs[i] = cosf(angle);
        sn[i] = sinf(angle);
    }
    return rope_common(ctx, query, key, head_dim, cs, sn, same);
}

extern "C" int32_t llmdot_hip_softmax(llmdot_hip_ctx* ctx, float* input, int32_t n, int32_t has_softcap, float softcap) {
    if (!ctx || (!input && n > 0) || n < 0) return fail(LLMDOT_E_INVALID, "bad Softmax arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float* dx;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    HIPCHK(launch_softmax(dx, n, has_softcap, softcap, ctx->stream));
    return copy_out(ctx, input, dx, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_silu(llmdot_hip_ctx* ctx, const float* input, float* result, int32_t n) {
    if (!ctx || !input || !result || n < 0) return fail(LLMDOT_E_INVALID, "bad Silu arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float *dx, *dy;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    if (int rc = stage_in<float>(ctx, 1, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_silu(dx, dy, n, ctx->stream));
    return copy_out(ctx, result, dy, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_layer_norm(llmdot_hip_ctx* ctx, const float* input, const float* weights,
                                         const float* bias_or_null, float* output, int32_t n, float epsilon) {
    if (!ctx || n < 0 || (n > 0 && (!input || !weights || !output))) return fail(LLMDOT_E_INVALID, "bad LayerNorm arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float *dx, *dw, *db = nullptr, *dy;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    if (int rc = stage_in(ctx, 1, weights, (size_t)n, &dw)) return rc;
    if (bias_or_null)
        if (int rc = stage_in(ctx, 2, bias_or_null, (size_t)n, &db)) return rc;
    if (int rc = stage_in<float>(ctx, 3, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_layernorm(dx, dw, db, dy, n, epsilon, ctx->stream));
    return copy_out(ctx, output, dy, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_gelu(llmdot_hip_ctx* ctx, const float* input, float* result, int32_t n) {
    if (!ctx || n < 0 || (n > 0 && (!input || !result))) return fail(LLMDOT_E_INVALID, "bad Gelu arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float *dx, *dy;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    if (int rc = stage_in<float>(ctx, 1, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_gelu(dx, dy, n, ctx->stream));
    return copy_out(ctx, result, dy, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_softcap(llmdot_hip_ctx* ctx, float* input, int32_t n, float cap) {
    if (!ctx || n < 0 || (n > 0 && !input)) return fail(LLMDOT_E_INVALID, "bad Softcap arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float* dx;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    HIPCHK(launch_softcap(dx, n, cap, ctx->stream));
    return copy_out(ctx, input, dx, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_conv1d(llmdot_hip_ctx* ctx, const float* input, const float* weights, float* output,
                                     int32_t kernel_size, int32_t input_dim) {
    if (!ctx || kernel_size < 1 || input_dim < 0 || (input_dim > 0 && (!input || !weights || !output)))
        return fail(LLMDOT_E_INVALID, "bad Conv1D arguments");
    if ((int64_t)kernel_size * input_dim > INT32_MAX) return fail(LLMDOT_E_RANGE, "Conv1D input too large");
    if (input_dim == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    const size_t n = (size_t)kernel_size * (size_t)input_dim;
    float *dx, *dw, *dy;
    if (int rc = stage_in(ctx, 0, input, n, &dx)) return rc;
    if (int rc = stage_in(ctx, 1, weights, n, &dw)) return rc;
    if (int rc = stage_in<float>(ctx, 2, nullptr, (size_t)input_dim, &dy)) return rc;
    HIPCHK(launch_conv1d(dx, dw, dy, kernel_size, input_dim, ctx->stream));
    return copy_out(ctx, output, dy, sizeof(float) * (size_t)input_dim);
}

namespace {
int binary_common(llmdot_hip_ctx* ctx, int op, const float* a, const float* b, float* result, int n) {
    if (!ctx || !a || !b || !result || n < 0) return fail(LLMDOT_E_INVALID, "bad elementwise arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float *da, *db, *dy;
    if (int rc = stage_in(ctx, 0, a, (size_t)n, &da)) return rc;
    if (int rc = stage_in(ctx, 1, b, (size_t)n, &db)) return rc;
    if (int rc = stage_in<float>(ctx, 2, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_binary(op, da, db, dy, n, ctx->stream));
    return copy_out(ctx, result, dy, sizeof(float) * (size_t)n);
}
}  // namespace

extern "C" int32_t llmdot_hip_add(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result, int32_t n) {
    return binary_common(ctx, 0, a, b, result, n);
}
extern "C" int32_t llmdot_hip_mul(llmdot_hip_ctx* ctx, const float* a, const float* b, float* result, int32_t n) {
    return binary_common(ctx, 1, a, b, result, n);
}
extern "C" int32_t llmdot_hip_scale(llmdot_hip_ctx* ctx, const float* input, float scale, float* result, int32_t n) {
    if (!ctx || !input || !result || n < 0) return fail(LLMDOT_E_INVALID, "bad Scale arguments");
    if (n == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    float *dx, *dy;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    if (int rc = stage_in<float>(ctx, 1, nullptr, (size_t)n, &dy)) return rc;
    HIPCHK(launch_scale(dx, scale, dy, n, ctx->stream));
    return copy_out(ctx, result, dy, sizeof(float) * (size_t)n);
}

extern "C" int32_t llmdot_hip_dequantize(llmdot_hip_ctx* ctx, const void* src, float* dst, uint32_t type, int32_t num_rows,
                                         int32_t row_elements) {
    if (!ctx || !src || !dst || num_rows < 0 || row_elements <= 0) return fail(LLMDOT_E_INVALID, "bad DequantizeToFloat arguments");
    if (block_elems(type) == 0)   // TensorOps.DequantizeGeneric's NotSupportedException (TO:647-648)
        return fail(LLMDOT_E_UNSUPPORTED, "Dequantization for type " + std::to_string(type) + " not yet implemented.");
    if (row_elements % block_elems(type) != 0) return fail(LLMDOT_E_INVALID, "row not a whole number of blocks");
    if (num_rows == 0) return 0;
    if (int rc = ensure_device(ctx)) return rc;
    const size_t nb = (size_t)((int64_t)num_rows * byte_count(type, row_elements));
    uint8_t* ds;
    float* dy;
    if (int rc = stage_in(ctx, 0, reinterpret_cast<const uint8_t*>(src), nb, &ds)) return rc;
    // zeros after the blocks: Q3_K's last q bytes lie 2 bytes past its block
    HIPCHK(hipMemsetAsync(ds + nb, 0, WEIGHT_PAD, ctx->stream));
    if (int rc = stage_in<float>(ctx, 1, nullptr, (size_t)num_rows * row_elements, &dy)) return rc;
    HIPCHK(launch_dequant(ds, dy, type, num_rows, row_elements, ctx->stream));
    return copy_out(ctx, dst, dy, sizeof(float) * (size_t)num_rows * row_elements);
}

extern "C" int32_t llmdot_hip_argmax(llmdot_hip_ctx* ctx, const float* input, int32_t n, int32_t* index) {
    if (!ctx || !input || !index || n <= 0) return fail(LLMDOT_E_INVALID, "bad ArgMax arguments");
    if (int rc = ensure_device(ctx)) return rc;
    if (int rc = ensure_argmax(ctx, argmax_grid(n))) return rc;
    float* dx;
    if (int rc = stage_in(ctx, 0, input, (size_t)n, &dx)) return rc;
    ArgmaxState st{};
    st.cand_val = ctx->am_val; st.cand_idx = ctx->am_idx;
    st.cap = ctx->am_cap; st.token_out = ctx->am_ints;
    HIPCHK(launch_argmax(dx, n, st, ctx->stream));
    return copy_out(ctx, index, ctx->am_ints, sizeof(int32_t));
}

extern "C" int32_t llmdot_hip_sample(llmdot_hip_ctx* ctx, const float* logits, int32_t n, const llmdot_hip_sampling* opt,
                                     const int32_t* recent, int32_t n_recent, float r, int32_t* token) {
    if (!ctx || !logits || !opt || !token || n <= 0 || n_recent < 0 || (n_recent > 0 && !recent))
        return fail(LLMDOT_E_INVALID, "bad Sample arguments");
    if (opt->temperature <= 0.f) return llmdot_hip_argmax(ctx, logits, n, token);   // Sampler.cs:26-27
    if (!sample_supported(n, opt->top_k))
        return fail(LLMDOT_E_UNSUPPORTED, "TopK between " + std::to_string(SAMPLE_MAX_K) + " and the vocabulary size is not supported");
    if (int rc = ensure_device(ctx)) return rc;
    if (int rc = ensure_argmax(ctx, 1)) return rc;
    float *dl, *dr;
    int32_t* dh;
    if (int rc = stage_in(ctx, 0, logits, (size_t)n, &dl)) return rc;
    HIPCHK(ctx->scratch[1].ensure(sizeof(float) * sample_work_floats(n)));
    if (int rc = stage_in(ctx, 2, recent, (size_t)n_recent, &dh)) return rc;
    if (int rc = stage_in(ctx, 3, &r, 1, &dr)) return rc;
    HIPCHK(launch_set_scalar(ctx->am_ints + 1, 1, ctx->stream));   // draw 0
    SampleArgs sa{};
    sa.logits = dl; sa.n = n; sa.inv_temp = 1.0f / opt->temperature;
    sa.top_k = opt->top_k; sa.top_p = opt->top_p; sa.penalty = opt->repeat_penalty; sa.window = opt->repeat_window;
    sa.hist = dh; sa.hist_base = n_recent; sa.step = ctx->am_ints + 1; sa.rvals = dr;
    sa.work = (float*)ctx->scratch[1].p; sa.token_out = ctx->am_ints;
    HIPCHK(launch_sample(sa, ctx->stream));
    return copy_out(ctx, token, ctx->am_ints, sizeof(int32_t));
}

extern "C" int32_t llmdot_hip_sample_noalloc(llmdot_hip_ctx* ctx, const float* logits_dev, int32_t n,
                                             const llmdot_hip_sampling* opt, const int32_t* recent_dev,
                                             int32_t n_recent, float r, int32_t* token_dev) {
    if (!ctx || !logits_dev || !opt || !token_dev || n <= 0 || n_recent < 0 || (n_recent > 0 && !recent_dev))
        return fail(LLMDOT_E_INVALID, "bad Sample arguments");
    if (n > NOALLOC_MAX_N)
        return fail(LLMDOT_E_UNSUPPORTED, "llmdot_hip_sample_noalloc: " + std::to_string(n) +
                                              " logits exceed its scratch of " + std::to_string(NOALLOC_MAX_N));
    const bool sampled = opt->temperature > 0.f;   // Sampler.cs:26-27: greedy otherwise
    if (sampled && !sample_supported(n, opt->top_k))
        return fail(LLMDOT_E_UNSUPPORTED, "TopK between " + std::to_string(SAMPLE_MAX_K) + " and the vocabulary size is not supported");
    if (int rc = ensure_device(ctx)) return rc;
    std::string err;
    uint8_t* base = scratch_of(ctx->device, &err);
    if (!base) return fail(LLMDOT_E_DEVICE, "llmdot_hip_sample_noalloc: " + err);
    float* work = reinterpret_cast<float*>(base);
    int32_t* ints = reinterpret_cast<int32_t*>(base + NOALLOC_INTS);
    if (!sampled) {
        ArgmaxState st{};
        st.cand_val = reinterpret_cast<float*>(base + NOALLOC_CAND_VAL);
        st.cand_idx = reinterpret_cast<int32_t*>(base + NOALLOC_CAND_IDX);
        st.cap = NOALLOC_CAND;
        st.token_out = token_dev;
        HIPCHK(launch_argmax(logits_dev, n, st, ctx->stream));
        return 0;
    }
    // the draw counter (this is draw 0) and the uniform draw, written by kernels
    // so that the call records no memset or host copy
    uint32_t rbits;
    memcpy(&rbits, &r, 4);
    HIPCHK(launch_set_scalar(ints, 1, ctx->stream));
    HIPCHK(launch_set_scalar(ints + 1, (int32_t)rbits, ctx->stream));
    SampleArgs sa{};
    sa.logits = logits_dev; sa.n = n; sa.inv_temp = 1.0f / opt->temperature;
    sa.top_k = opt->top_k; sa.top_p = opt->top_p; sa.penalty = opt->repeat_penalty; sa.window = opt->repeat_window;
    sa.hist = recent_dev; sa.hist_base = n_recent; sa.step = ints; sa.rvals = reinterpret_cast<const float*>(ints + 1);
    sa.work = work; sa.token_out = token_dev;
    HIPCHK(launch_sample(sa, ctx->stream));
    return 0;
}

// ========================================================= device pointers ==

extern "C" int32_t llmdot_hip_device_alloc(llmdot_hip_ctx* ctx, size_t nbytes, void** dptr) {
    if (!ctx || !dptr) return fail(LLMDOT_E_INVALID, "null argument");
    if (int rc = ensure_device(ctx)) return rc;
    hipError_t e = hipMalloc(dptr, nbytes + WEIGHT_PAD);
    if (e != hipSuccess) return fail(LLMDOT_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return zero_fresh(ctx, *dptr, nbytes + WEIGHT_PAD);
}
extern "C" int32_t llmdot_hip_device_free(llmdot_hip_ctx* ctx, void* dptr) {
    if (!ctx) return fail(LLMDOT_E_INVALID, "null ctx");
    if (dptr) { (void)hipStreamSynchronize(ctx->stream); HIPCHK(hipFree(dptr)); }
    return 0;
}
extern "C" int32_t llmdot_hip_memcpy_h2d(llmdot_hip_ctx* ctx, void* dst, const void* src, size_t nbytes) {
    if (!ctx || !dst || !src) return fail(LLMDOT_E_INVALID, "null argument");
    HIPCHK(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}
extern "C" int32_t llmdot_hip_memcpy_d2h(llmdot_hip_ctx* ctx, void* dst, const void* src, size_t nbytes) {
    if (!ctx || !dst || !src) return fail(LLMDOT_E_INVALID, "null argument");
    return copy_out(ctx, dst, src, nbytes);
}
extern "C" int32_t llmdot_hip_synchronize(llmdot_hip_ctx* ctx) {
    if (!ctx) return fail(LLMDOT_E_INVALID, "null ctx");
    HIPCHK(hipStreamSynchronize(ctx->stream));
    return 0;
}

extern "C" int32_t llmdot_hip_gemv_device(llmdot_hip_ctx* ctx, uint32_t type, const void* w_dev, const float* x_dev,
                                          float* y_dev, int32_t rows, int32_t cols) {
    if (!ctx || !w_dev || !x_dev || !y_dev || rows <= 0 || cols <= 0) return fail(LLMDOT_E_INVALID, "bad gemv arguments");
    if (!gemv_supported(type)) return fail(LLMDOT_E_UNSUPPORTED, "unsupported gemv type");
    return ctx_gemv(ctx, type, reinterpret_cast<const uint8_t*>(w_dev), x_dev, y_dev, rows, cols);
}

extern "C" int32_t llmdot_hip_time_gemv(llmdot_hip_ctx* ctx, uint32_t type, const void* const* w_devs, int32_t n_weights,
                                        const float* x_dev, float* y_dev, int32_t rows, int32_t cols, int32_t iters,
                                        float* ms) {
    if (!ctx || !w_devs || n_weights <= 0 || iters <= 0 || !ms) return fail(LLMDOT_E_INVALID, "bad timing arguments");
    if (!gemv_supported(type)) return fail(LLMDOT_E_UNSUPPORTED, "unsupported gemv type");
    if (int rc = ctx_gemv(ctx, type, reinterpret_cast<const uint8_t*>(w_devs[0]), x_dev, y_dev, rows, cols)) return rc;
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipEventRecord(e0, ctx->stream));
    for (int i = 0; i < iters; i++)
        if (int rc = ctx_gemv(ctx, type, reinterpret_cast<const uint8_t*>(w_devs[i % n_weights]), x_dev, y_dev, rows,
                              cols))
            return rc;
    HIPCHK(hipEventRecord(e1, ctx->stream));
    HIPCHK(hipEventSynchronize(e1));
    HIPCHK(hipEventElapsedTime(ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

extern "C" int32_t llmdot_hip_stream_bench(llmdot_hip_ctx* ctx, size_t nbytes, int32_t mode, int32_t iters, float* ms) {
    if (!ctx || !ms || nbytes < 16 || iters <= 0 || (mode != 0 && mode != 1))
        return fail(LLMDOT_E_INVALID, "bad stream_bench arguments");
    if (int rc = ensure_device(ctx)) return rc;
    void* buf = nullptr;
    uint32_t* sink = nullptr;
    hipError_t e = hipMalloc(&buf, nbytes);
    if (e != hipSuccess) return fail(LLMDOT_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    int rc = 0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto run = [&]() -> hipError_t {
        hipError_t r;
        if ((r = hipMalloc(&sink, 4)) != hipSuccess) return r;
        if ((r = hipMemsetAsync(buf, 0, nbytes, ctx->stream)) != hipSuccess) return r;
        if ((r = hipEventCreate(&e0)) != hipSuccess || (r = hipEventCreate(&e1)) != hipSuccess) return r;
        if ((r = launch_stream_probe(buf, nbytes, mode, sink, ctx->stream)) != hipSuccess) return r;   // warm-up
        if ((r = hipEventRecord(e0, ctx->stream)) != hipSuccess) return r;
        for (int i = 0; i < iters; i++)
            if ((r = launch_stream_probe(buf, nbytes, mode, sink, ctx->stream)) != hipSuccess) return r;
        if ((r = hipEventRecord(e1, ctx->stream)) != hipSuccess) return r;
        if ((r = hipEventSynchronize(e1)) != hipSuccess) return r;
        return hipEventElapsedTime(ms, e0, e1);
    };
    e = run();
    if (e != hipSuccess) rc = fail(LLMDOT_E_DEVICE, std::string("stream_bench: ") + hipGetErrorString(e));
    (void)hipStreamSynchronize(ctx->stream);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink) (void)hipFree(sink);
    (void)hipFree(buf);
    return rc;
}

// ================================================================== model ==

namespace {

struct LayerW {
    const Weight *attn_norm, *ffn_norm, *q, *k, *v, *o, *gate, *up, *down;
    float *attn_norm_f, *ffn_norm_f;   // fp32 norm weights on the device
    float *q_norm_f = nullptr, *k_norm_f = nullptr;   // per-head Q/K norms [head_dim] (absent: null)
};

}  // namespace

struct llmdot_hip_model {
    llmdot_hip_ctx* ctx = nullptr;
    std::set<std::string> pinned;   // context weight keys this model reads
    llmdot_hip_model_desc d{};
    std::string prefix;
    std::vector<LayerW> L;
    const Weight *embd = nullptr, *out = nullptr, *out_norm = nullptr;
    float* out_norm_f = nullptr;
    std::vector<void*> owned;          // device allocations owned by the model
    std::deque<Weight> views;          // Q, K and V row ranges of fused attn_qkv tensors
    // activations
    float *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    // h packed for its next RmsNorm consumer: xn = w * h, xssq[i] = sum of h^2 over h[4i .. 4i+3]
    float *xn = nullptr, *xssq = nullptr;
    // KV cache [layer][kv_head][context][head_dim]
    uint8_t *kcache = nullptr, *vcache = nullptr;
    size_t kv_layer_bytes = 0;
    float *cos_tab = nullptr, *sin_tab = nullptr;
    int rope_half = 0;
    // attention scratch
    float *scores = nullptr, *chunk_max = nullptr, *part_out = nullptr, *part_sum = nullptr;
    uint64_t* xmax = nullptr;   // tagged chunk maxima of the one-launch attention
    uint64_t* xpart = nullptr;  // tagged chunk partials of its XCD-local form
    bool attn_fused = false;
    int attn_spin = 1 << 18;
    bool attn_xcd_exchange = false;    // one-launch attention: chunk maxima through the kv head's XCD L2
    // argmax + device-side loop state: ints[0] token, [1] pos, [2] step,
    // [3] epoch (decode steps run, never reset: tags the attention's slots),
    // [4] error flags set by device waits that gave up
    int32_t* ints = nullptr;
    int32_t* token_log = nullptr;
    float* am_val = nullptr;
    int32_t* am_idx = nullptr;
    int am_cap = 0;
    hipGraphExec_t graph = nullptr;
    bool use_graph = true;
    // batched prefill (allocated on first use): chunk of pf_cap tokens
    bool pf_eligible = false;
    int pf_cap = 0;
    float *pf_h = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr, *pf_qr = nullptr, *pf_attn = nullptr,
          *pf_act = nullptr, *pf_scores = nullptr, *pf_rowmax = nullptr;
    // K parts of the narrow projections (prefill_ksplit): Q, then O and down
    // (in stream order) share one buffer; K and V run at the same time as Q
    float *pf_parts_q = nullptr, *pf_parts_k = nullptr, *pf_parts_v = nullptr;
    PfPlanes pf_planes{};
    int32_t* pf_tokens = nullptr;
    // sampled generation (allocated on first use): recent-token history
    // [context + 1], uniform draws [context + 1], sampler scratch [vocab]
    int32_t* s_hist = nullptr;
    float* s_draws = nullptr;
    float* s_work = nullptr;
    // streaming Generate: tokens [0, yielded) returned, [yielded, computed)
    // computed on the device and not yet returned
    struct GenState {
        bool active = false, sampled = false, done = false;
        llmdot_hip_sampling opt{};
        int hist_base = 0, produce = 0, max_tokens = 0, eos = -1, yielded = 0, computed = 0;
    } gen;
};

namespace {

int32_t* m_token(llmdot_hip_model* m) { return m->ints; }
int32_t* m_pos(llmdot_hip_model* m) { return m->ints + 1; }
int32_t* m_step(llmdot_hip_model* m) { return m->ints + 2; }
uint32_t* m_epoch(llmdot_hip_model* m) { return reinterpret_cast<uint32_t*>(m->ints + 3); }
int32_t* m_err(llmdot_hip_model* m) { return m->ints + 4; }

int dalloc(llmdot_hip_model* m, size_t n, void** p) {
    hipError_t e = hipMalloc(p, n + WEIGHT_PAD);
    if (e != hipSuccess) return fail(LLMDOT_E_NOMEM, "device allocation of " + std::to_string(n) + " bytes failed: " + hipGetErrorString(e));
    m->owned.push_back(*p);
    return zero_fresh(m->ctx, *p, n + WEIGHT_PAD);
}

// A context weight the model reads; it stays pinned (no release, no
// reallocation) until the model is destroyed.
const Weight* find_w(llmdot_hip_model* m, const std::string& name) {
    auto it = m->ctx->weights.find(m->prefix + name);
    if (it == m->ctx->weights.end()) return nullptr;
    if (m->pinned.insert(it->first).second) it->second.pins++;
    return &it->second;
}

int need_w(llmdot_hip_model* m, const std::string& name, int64_t rows, int64_t cols, const Weight** out) {
    const Weight* w = find_w(m, name);
    if (!w) return fail(LLMDOT_E_NOT_FOUND, "Tensor '" + m->prefix + name + "' not found.");
    if ((rows >= 0 && w->rows != rows) || (cols >= 0 && w->cols != cols))
        return fail(LLMDOT_E_INVALID, "Tensor '" + name + "' has shape [" + std::to_string(w->rows) + " x " +
                                          std::to_string(w->cols) + "], expected [" + std::to_string(rows) + " x " +
                                          std::to_string(cols) + "]");
    *out = w;
    return 0;
}

// Norm weights as fp32 on the device (LoadedModel.GetDequantizedWeights, LM:63-75).
// F32 norms are read in place; other types are converted into a model-owned
// copy that the context re-converts when the key is re-uploaded in place.
int norm_f32(llmdot_hip_model* m, const Weight* w, int n, float** out) {
    if (w->rows * w->cols != n) return fail(LLMDOT_E_INVALID, "norm weight has wrong size");
    if (w->type == GGML_F32) { *out = reinterpret_cast<float*>(w->dev); return 0; }
    void* p;
    if (int rc = dalloc(m, sizeof(float) * (size_t)n, &p)) return rc;
    HIPCHK(launch_dequant(w->dev, (float*)p, w->type, 1, n, m->ctx->stream));
    for (const auto& kv : m->ctx->weights)
        if (&kv.second == w) m->ctx->norm_copies.push_back({kv.first, (float*)p, n, m});
    *out = (float*)p;
    return 0;
}

int check_gemv_type(const Weight* w, const std::string& name) {
    if (!gemv_supported(w->type)) return fail(LLMDOT_E_UNSUPPORTED, "tensor " + name + ": unsupported type " + std::to_string(w->type));
    if (w->cols % 32 != 0 || !gemv_width_ok(w->type, (int)w->cols))
        return fail(LLMDOT_E_UNSUPPORTED, "tensor " + name + ": width " + std::to_string(w->cols) + " not supported by the GEMV kernel");
    return 0;
}

// GEMV launch on the model stream.
hipError_t step_gemv(llmdot_hip_model* m, uint32_t type, int epi, GemvArgs& a) {
    a.eps = m->d.eps;
    return launch_gemv(type, epi, a, m->ctx->stream);
}

// FFN gate/up over RmsNorm(h), SiLU(gate) * up (IE:190, IE:463-474): the
// step's dominant launch.
hipError_t launch_gate_up(llmdot_hip_model* m, int l) {
    const LayerW& w = m->L[l];
    GemvArgs ga{};
    ga.nseg = 1; ga.seg[0] = {w.gate->dev, w.up->dev, m->act, m->d.ffn, 0};
    ga.cols = m->d.hidden; ga.x = m->xn; ga.ssq = m->xssq; ga.norm = 1;
    return step_gemv(m, w.gate->type, EPI_SWIGLU, ga);
}

// Final RmsNorm + LM head + greedy ArgMax (IE:575-602, Sampler.cs:26-27) over the
// packed xn / xssq; the argmax pass advances the device position and step.
int enqueue_head(llmdot_hip_model* m) {
    const auto& d = m->d;
    GemvArgs ga{};
    ga.nseg = 1; ga.seg[0] = {m->out->dev, nullptr, m->logits, d.vocab, 0};
    ga.cols = d.hidden; ga.x = m->xn; ga.ssq = m->xssq; ga.norm = 1;
    ga.am.cand_val = m->am_val; ga.am.cand_idx = m->am_idx; ga.am.cap = m->am_cap;
    ga.am.token_out = m_token(m); ga.am.pos = m_pos(m);
    ga.am.token_log = m->token_log; ga.am.log_cap = d.context + 1; ga.am.step = m_step(m);
    ga.am.epoch = m_epoch(m);
    HIPCHK(step_gemv(m, m->out->type, EPI_ARGMAX, ga));
    return 0;
}

// Enqueues one decode step on the model stream (token and position on the device).
int enqueue_step(llmdot_hip_model* m) {
    const auto& d = m->d;
    hipStream_t s = m->ctx->stream;
    const int qdim = d.heads * d.head_dim, kvdim = d.kv_heads * d.head_dim;
    HIPCHK(launch_embed(m->embd->dev, m->embd->type, d.hidden, m_token(m), m->h, m->L[0].attn_norm_f, m->xn,
                        m->xssq, s));
    for (int l = 0; l < d.layers; l++) {
        const LayerW& w = m->L[l];
        // Q, K, V projections over RmsNorm(h) (IE:185-186, IE:333-353) in one launch when the
        // types allow (one type, or Q4_K or Q8_0 mixed with Q6_K, as the Q4_K_M and
        // Q6_K/Q8_0 mixes give), else one per type.
        const Weight* mats[3] = {w.q, w.k, w.v};
        float* outs[3] = {m->q, m->k, m->v};
        int rows[3] = {qdim, kvdim, kvdim};
        uint32_t prim = 0;   // the one type other than Q6_K, if Q4_K or Q8_0
        bool mixed_ok = true;
        for (int i = 0; i < 3; i++) {
            const uint32_t t = mats[i]->type;
            if (t == GGML_Q6_K) continue;
            mixed_ok = mixed_ok && (t == GGML_Q4_K || t == GGML_Q8_0) && (prim == 0 || prim == t);
            prim = t;
        }
        mixed_ok = mixed_ok && prim != 0;
        bool done[3] = {false, false, false};
        for (int i = 0; i < 3; i++) {
            if (done[i]) continue;
            GemvArgs ga{};
            ga.cols = d.hidden; ga.x = m->xn; ga.ssq = m->xssq; ga.norm = 1;
            const uint32_t lt = mixed_ok ? prim : mats[i]->type;
            for (int j = i; j < 3; j++)
                if (!done[j] && (mats[j]->type == mats[i]->type || mixed_ok)) {
                    ga.seg[ga.nseg++] = {mats[j]->dev, nullptr, outs[j], rows[j], 0, mats[j]->type};
                    done[j] = true;
                }
            HIPCHK(step_gemv(m, lt, EPI_STORE, ga));
        }
        if (w.q_norm_f || w.k_norm_f)   // per-head Q/K RmsNorm before RoPE (IE:354-359, IE:367-372)
            HIPCHK(launch_qk_norm(m->q, m->k, w.q_norm_f, w.k_norm_f, d.heads, d.kv_heads, d.head_dim, d.eps, s));
        AttnArgs aa{};
        aa.q = m->q; aa.k = m->k; aa.v = m->v;
        aa.kcache = m->kcache + (size_t)l * m->kv_layer_bytes;
        aa.vcache = m->vcache + (size_t)l * m->kv_layer_bytes;
        aa.cos_tab = m->cos_tab; aa.sin_tab = m->sin_tab; aa.pos = m_pos(m);
        aa.scores = m->scores; aa.chunk_max = m->chunk_max; aa.part_out = m->part_out; aa.part_sum = m->part_sum;
        aa.out = m->attn;
        aa.heads = d.heads; aa.kv_heads = d.kv_heads; aa.head_dim = d.head_dim; aa.rope_half = m->rope_half;
        aa.context = d.context; aa.kv_fp16 = d.kv_fp16;
        aa.fused = m->attn_fused ? 1 : 0; aa.xmax = m->xmax; aa.epoch = m_epoch(m);
        aa.layer = l; aa.layers = d.layers; aa.spin_max = m->attn_spin; aa.err = m_err(m);
        aa.xcd_exchange = m->attn_xcd_exchange ? 1 : 0; aa.xpart = m->xpart;
        aa.window = d.sliding_window;
        HIPCHK(launch_attention(aa, s));
        {   // O projection + residual (IE:444-449, IE:189), h packed for the FFN RmsNorm
            GemvArgs ga{};
            ga.nseg = 1; ga.seg[0] = {w.o->dev, nullptr, m->h, d.hidden, 0};
            ga.cols = qdim; ga.x = m->attn;
            ga.pack_w = w.ffn_norm_f; ga.pack_out = m->xn; ga.pack_ssq = m->xssq;
            HIPCHK(step_gemv(m, w.o->type, EPI_ADD, ga));
        }
        HIPCHK(launch_gate_up(m, l));
        {   // down projection + residual (IE:475, IE:195), h packed for the next RmsNorm
            GemvArgs ga{};
            ga.nseg = 1; ga.seg[0] = {w.down->dev, nullptr, m->h, d.hidden, 0};
            ga.cols = d.ffn; ga.x = m->act;
            ga.pack_w = l + 1 < d.layers ? m->L[l + 1].attn_norm_f : m->out_norm_f;
            ga.pack_out = m->xn; ga.pack_ssq = m->xssq;
            HIPCHK(step_gemv(m, w.down->type, EPI_ADD, ga));
        }
    }
    return enqueue_head(m);
}

int build_graph(llmdot_hip_model* m) {
    if (!m->use_graph) return 0;
    hipStream_t s = m->ctx->stream;
    HIPCHK(hipStreamSynchronize(s));
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m);
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return fail(LLMDOT_E_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { m->graph = nullptr; return fail(LLMDOT_E_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e)); }
    return 0;
}

int run_step(llmdot_hip_model* m) {
    if (m->graph) {
        HIPCHK(hipGraphLaunch(m->graph, m->ctx->stream));
        return 0;
    }
    return enqueue_step(m);
}

int set_int(llmdot_hip_model* m, int32_t* dst, int32_t v) {
    HIPCHK(launch_set_scalar(dst, v, m->ctx->stream));
    return 0;
}

// ---- batched prefill ------------------------------------------------------

// Whether every projection of every layer has a batched (MFMA) kernel.
bool prefill_check(const llmdot_hip_model* m) {
    const auto& d = m->d;
    const int qdim = d.heads * d.head_dim;
    for (const auto& w : m->L) {
        // the window is on the fp16 (MFMA) attention only: with an fp32 KV
        // cache a windowed model's prompt runs through the decode step
        if (d.sliding_window > 0 && !d.kv_fp16) return false;
        const Weight* in_h[5] = {w.q, w.k, w.v, w.gate, w.up};
        for (auto* x : in_h)
            if (!prefill_gemm_supported(x->type, d.hidden)) return false;
        if (!prefill_gemm_supported(w.o->type, qdim) || !prefill_gemm_supported(w.down->type, d.ffn)) return false;
    }
    return true;
}

int prefill_chunk_cap(const llmdot_hip_model* m) {
    int cap = 2048;
    if (const char* v = getenv("LLMDOT_HIP_PREFILL_CHUNK")) {
        const int c = atoi(v);
        if (c >= 16) cap = c;
    }
    // fp32 KV: score scratch [heads][cap][context] fp32 within 2 GiB (the
    // fp16-KV attention keeps its scores in registers)
    if (!m->d.kv_fp16) {
        const double per_tok = 4.0 * m->d.heads * (double)m->d.context;
        while (cap > 64 && per_tok * cap > 2147483648.0) cap /= 2;
    }
    return cap;
}

int ensure_side_streams(llmdot_hip_ctx* ctx) {
    if (ctx->fork) return 0;
    for (int i = 0; i < 2; i++) {
        HIPCHK(hipStreamCreateWithFlags(&ctx->side[i], hipStreamNonBlocking));
        HIPCHK(hipEventCreateWithFlags(&ctx->join[i], hipEventDisableTiming));
    }
    HIPCHK(hipEventCreateWithFlags(&ctx->fork, hipEventDisableTiming));
    return 0;
}

int ensure_prefill_ws(llmdot_hip_model* m) {
    if (m->pf_cap) return 0;
    if (int rc = ensure_side_streams(m->ctx)) return rc;
    const auto& d = m->d;
    const int cap = prefill_chunk_cap(m);
    const size_t qdim = (size_t)d.heads * d.head_dim, kvdim = (size_t)d.kv_heads * d.head_dim;
    const size_t kmax = std::max({(size_t)d.hidden, qdim, (size_t)d.ffn});
    void* p;
    auto A = [&](size_t n, void** dst) { return dalloc(m, n, dst); };
    int rc;
    if ((rc = A(4 * cap * (size_t)d.hidden, &p))) return rc; m->pf_h = (float*)p;
    if ((rc = A(4 * cap * qdim, &p))) return rc; m->pf_q = (float*)p;
    if ((rc = A(4 * cap * kvdim, &p))) return rc; m->pf_k = (float*)p;
    if ((rc = A(4 * cap * kvdim, &p))) return rc; m->pf_v = (float*)p;
    if ((rc = A(4 * cap * qdim, &p))) return rc; m->pf_qr = (float*)p;
    if ((rc = A(4 * cap * qdim, &p))) return rc; m->pf_attn = (float*)p;
    if ((rc = A(4 * cap * (size_t)d.ffn, &p))) return rc; m->pf_act = (float*)p;
    // a K split keeps tiles x parts <= 512, so parts x rows x cols <= 512 x 128 x 128
    if ((rc = A(4 * PF_PARTS_MAX, &p))) return rc; m->pf_parts_q = (float*)p;
    if ((rc = A(4 * PF_PARTS_MAX, &p))) return rc; m->pf_parts_k = (float*)p;
    if ((rc = A(4 * PF_PARTS_MAX, &p))) return rc; m->pf_parts_v = (float*)p;
    if (!d.kv_fp16) {
        if ((rc = A(4 * (size_t)d.heads * cap * (size_t)d.context, &p))) return rc;
        m->pf_scores = (float*)p;
    }
    if ((rc = A(4 * (size_t)d.heads * cap, &p))) return rc; m->pf_rowmax = (float*)p;
    if ((rc = A(2 * cap * kmax, &p))) return rc; m->pf_planes.xh = (_Float16*)p;
    if ((rc = A(2 * cap * kmax, &p))) return rc; m->pf_planes.xl = (_Float16*)p;
    if ((rc = A(2 * cap * (kmax / 32), &p))) return rc; m->pf_planes.sh = (_Float16*)p;
    if ((rc = A(2 * cap * (kmax / 32), &p))) return rc; m->pf_planes.sl = (_Float16*)p;
    if ((rc = A(4 * (size_t)cap, &p))) return rc; m->pf_planes.xinv = (float*)p;
    if ((rc = A(4 * (size_t)cap, &p))) return rc; m->pf_tokens = (int32_t*)p;
    m->pf_cap = cap;
    return 0;
}

// One chunk of T prompt tokens at positions pos0 .. pos0+T-1 (tokens already
// in pf_tokens): every layer as batched GEMMs, RoPE + KV write and causal
// attention; leaves the chunk's hidden states in pf_h.
int enqueue_prefill_chunk(llmdot_hip_model* m, int T, int pos0) {
    const auto& d = m->d;
    hipStream_t s = m->ctx->stream;
    const int qdim = d.heads * d.head_dim, kvdim = d.kv_heads * d.head_dim;
    const PfPlanes& pl = m->pf_planes;
    const bool split_ok = !env_flag("LLMDOT_HIP_PF_NO_SPLIT");
    // A STORE projection [T x N] over K columns, in K parts into `parts` when
    // the launch has few tiles; returns the part count (1: written to out).
    auto proj = [&](const Weight* w, int N, int K, float* out, float* parts, hipStream_t st, int* nparts) {
        int sp = split_ok ? prefill_ksplit(w->type, T, N, K) : 1;
        if ((int64_t)sp * T * N > PF_PARTS_MAX) sp = 1;
        *nparts = sp;
        if (sp == 1) return launch_prefill_gemm(w->type, 0, pl, w->dev, nullptr, T, N, K, out, N, st);
        return launch_prefill_gemm(w->type, 0, pl, w->dev, nullptr, T, N, K, parts, N, st, sp, (int64_t)T * N);
    };
    // h += the [T x hidden] projection: in place, or its K parts then their sum
    auto proj_add = [&](const Weight* w, int K) {
        int sp = split_ok ? prefill_ksplit(w->type, T, d.hidden, K) : 1;
        if ((int64_t)sp * T * d.hidden > PF_PARTS_MAX) sp = 1;
        if (sp == 1) return launch_prefill_gemm(w->type, 1, pl, w->dev, nullptr, T, d.hidden, K, m->pf_h, d.hidden, s);
        const int64_t n = (int64_t)T * d.hidden;
        hipError_t e = launch_prefill_gemm(w->type, 0, pl, w->dev, nullptr, T, d.hidden, K, m->pf_parts_q, d.hidden, s,
                                           sp, n);
        return e != hipSuccess ? e : launch_prefill_add_parts(m->pf_h, m->pf_parts_q, sp, n, n, s);
    };
    // Q and K (same type) as one launch where neither would be split in K:
    // their row tiles then share the CUs in one grid instead of K's narrow
    // launch running beside Q's (LLMDOT_HIP_PF_QK_PAIR=0 turns this off)
    const bool pair_ok = !env_is_zero("LLMDOT_HIP_PF_QK_PAIR") && qdim % 128 == 0;
    auto qk_pair = [&](const LayerW& w) {
        return pair_ok && w.q->type == w.k->type && prefill_ksplit(w.q->type, T, qdim, d.hidden) == 1 &&
               prefill_ksplit(w.k->type, T, kvdim, d.hidden) == 1;
    };
    HIPCHK(launch_embed_rows(m->embd->dev, m->embd->type, d.hidden, m->pf_tokens, T, m->pf_h, s));
    for (int l = 0; l < d.layers; l++) {
        const LayerW& w = m->L[l];
        HIPCHK(launch_prefill_planes(m->pf_h, T, d.hidden, w.attn_norm_f, d.eps, pl, s));
        // Q, K and V read the same planes and write separate buffers: V runs
        // on a side stream beside Q and K (one launch where qk_pair allows,
        // else K on the other side stream; K and V alone fill half the CUs)
        llmdot_hip_ctx* c = m->ctx;
        int nq = 1, nk = 1, nv = 1;
        HIPCHK(hipEventRecord(c->fork, s));
        HIPCHK(hipStreamWaitEvent(c->side[1], c->fork, 0));
        HIPCHK(proj(w.v, kvdim, d.hidden, m->pf_v, m->pf_parts_v, c->side[1], &nv));
        HIPCHK(hipEventRecord(c->join[1], c->side[1]));
        if (qk_pair(w)) {   // Q and K in one launch, of 128-token tiles
            HIPCHK(launch_prefill_gemm_pair(w.q->type, pl, w.q->dev, qdim, m->pf_q, qdim, w.k->dev, kvdim, m->pf_k,
                                            kvdim, T, d.hidden, s));
        } else {
            HIPCHK(hipStreamWaitEvent(c->side[0], c->fork, 0));
            HIPCHK(proj(w.k, kvdim, d.hidden, m->pf_k, m->pf_parts_k, c->side[0], &nk));
            HIPCHK(hipEventRecord(c->join[0], c->side[0]));
            HIPCHK(proj(w.q, qdim, d.hidden, m->pf_q, m->pf_parts_q, s, &nq));
            HIPCHK(hipStreamWaitEvent(s, c->join[0], 0));
        }
        HIPCHK(hipStreamWaitEvent(s, c->join[1], 0));
        PfAttnArgs aa{};
        aa.q = nq > 1 ? m->pf_parts_q : m->pf_q;
        aa.k = nk > 1 ? m->pf_parts_k : m->pf_k;
        aa.v = nv > 1 ? m->pf_parts_v : m->pf_v;
        aa.q_split = nq; aa.k_split = nk; aa.v_split = nv;
        aa.q_part = (int64_t)T * qdim; aa.k_part = (int64_t)T * kvdim; aa.v_part = (int64_t)T * kvdim;
        aa.qr = m->pf_qr;
        aa.kcache = m->kcache + (size_t)l * m->kv_layer_bytes;
        aa.vcache = m->vcache + (size_t)l * m->kv_layer_bytes;
        aa.cos_tab = m->cos_tab; aa.sin_tab = m->sin_tab;
        aa.scores = m->pf_scores; aa.rowmax = m->pf_rowmax; aa.out = m->pf_attn;
        aa.T = T; aa.pos0 = pos0; aa.ld_scores = d.context;
        aa.heads = d.heads; aa.kv_heads = d.kv_heads; aa.head_dim = d.head_dim; aa.rope_half = m->rope_half;
        aa.context = d.context; aa.kv_fp16 = d.kv_fp16;
        aa.q_norm = w.q_norm_f; aa.k_norm = w.k_norm_f; aa.eps = d.eps;
        aa.window = d.sliding_window;
        HIPCHK(launch_prefill_rope_kv(aa, s));
        HIPCHK(launch_prefill_attention(aa, s));
        HIPCHK(launch_prefill_planes(m->pf_attn, T, qdim, nullptr, 0.f, pl, s));
        HIPCHK(proj_add(w.o, qdim));
        HIPCHK(launch_prefill_planes(m->pf_h, T, d.hidden, w.ffn_norm_f, d.eps, pl, s));
        HIPCHK(launch_prefill_gemm(w.gate->type, 2, pl, w.gate->dev, w.up->dev, T, d.ffn, d.hidden, m->pf_act, d.ffn, s));
        HIPCHK(launch_prefill_planes(m->pf_act, T, d.ffn, nullptr, 0.f, pl, s));
        HIPCHK(proj_add(w.down, d.ffn));
    }
    return 0;
}

// Batched prompt processing of n tokens from pos0 (the sequential loop of
// IE:84-88 in chunks), then the LM head and argmax of the last token.  The
// device position ends at pos0 + n; with reset_step the argmax is logged as
// token 0 of a Generate call.
int prefill_batched(llmdot_hip_model* m, const int32_t* tokens, int n, int pos0, bool reset_step) {
    if (int rc = ensure_prefill_ws(m)) return rc;
    hipStream_t s = m->ctx->stream;
    int T = 0;
    for (int c0 = 0; c0 < n; c0 += m->pf_cap) {
        T = std::min(m->pf_cap, n - c0);
        HIPCHK(hipMemcpyAsync(m->pf_tokens, tokens + c0, sizeof(int32_t) * (size_t)T, hipMemcpyHostToDevice, s));
        if (int rc = enqueue_prefill_chunk(m, T, pos0 + c0)) return rc;
    }
    const float* h_last = m->pf_h + (size_t)(T - 1) * m->d.hidden;
    HIPCHK(launch_pack_norm(h_last, m->out_norm_f, m->d.hidden, m->xn, m->xssq, s));
    if (int rc = set_int(m, m_pos(m), pos0 + n - 1)) return rc;
    if (reset_step)
        if (int rc = set_int(m, m_step(m), 0)) return rc;
    return enqueue_head(m);
}

bool use_batched_prefill(const llmdot_hip_model* m, int n) {
    return m->pf_eligible && n > 1 && !env_flag("LLMDOT_HIP_SEQ_PREFILL");
}

}  // namespace

extern "C" int32_t llmdot_hip_model_destroy(llmdot_hip_model* m) {
    if (!m) return 0;
    llmdot_hip_ctx* ctx = m->ctx;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    auto& nc = ctx->norm_copies;
    nc.erase(std::remove_if(nc.begin(), nc.end(), [m](const llmdot_hip_ctx::NormCopy& c) { return c.owner == m; }),
             nc.end());
    for (void* p : m->owned) (void)hipFree(p);
    for (const auto& k : m->pinned) {
        auto it = ctx->weights.find(k);
        if (it != ctx->weights.end()) it->second.pins--;
    }
    delete m;
    if (--ctx->models == 0 && ctx->closing) ctx_release(ctx);
    return 0;
}

extern "C" int32_t llmdot_hip_model_create(llmdot_hip_ctx* ctx, const llmdot_hip_model_desc* desc, llmdot_hip_model** out) {
    if (!ctx || !desc || !out) return fail(LLMDOT_E_INVALID, "null argument");
    *out = nullptr;
    const auto& d = *desc;
    if (d.hidden <= 0 || d.layers <= 0 || d.heads <= 0 || d.kv_heads <= 0 || d.head_dim <= 0 || d.ffn <= 0 ||
        d.vocab <= 0 || d.context <= 0 || d.heads % d.kv_heads != 0)
        return fail(LLMDOT_E_INVALID, "invalid model description");
    if (d.hidden % 32 != 0 || d.ffn % 32 != 0 || (d.heads * d.head_dim) % 32 != 0)
        return fail(LLMDOT_E_UNSUPPORTED, "hidden, ffn and heads*head_dim must be multiples of 32");
    if (!attn_supported(d.heads, d.kv_heads, d.head_dim))
        return fail(LLMDOT_E_UNSUPPORTED, "attention shape not supported (head_dim 64/96/128, group 1/2/4/8)");
    if (int rc = ensure_device(ctx)) return rc;
    if (ctx->closing) return fail(LLMDOT_E_INVALID, "the context has been destroyed");
    auto* m = new llmdot_hip_model();
    m->ctx = ctx;
    ctx->models++;   // every path out (llmdot_hip_model_destroy included) balances this
    m->d = d;
    m->prefix = d.key_prefix ? d.key_prefix : "";
    m->d.key_prefix = nullptr;
    m->use_graph = !env_flag("LLMDOT_HIP_NO_GRAPH");
    const int qdim = d.heads * d.head_dim, kvdim = d.kv_heads * d.head_dim;
    int rc = 0;
    auto bail = [&](int code) { llmdot_hip_model_destroy(m); return code; };
    if ((rc = need_w(m, "token_embd.weight", -1, d.hidden, &m->embd))) return bail(rc);
    if (m->embd->rows < d.vocab && !find_w(m, "output.weight"))
        return bail(fail(LLMDOT_E_INVALID, "token_embd has fewer rows than the vocabulary"));
    const Weight* onorm = find_w(m, "output_norm.weight");
    if (!onorm) onorm = find_w(m, "token_embd_norm.weight");
    if (!onorm) return bail(fail(LLMDOT_E_NOT_FOUND, "Tensor 'output_norm.weight' not found."));
    m->out_norm = onorm;
    m->out = find_w(m, "output.weight");
    if (!m->out) m->out = m->embd;   // tied embeddings (IE:585-589)
    if (m->out->cols != d.hidden || m->out->rows != d.vocab)
        return bail(fail(LLMDOT_E_INVALID, "output projection shape does not match hidden x vocab"));
    if ((rc = check_gemv_type(m->out, "output"))) return bail(rc);
    if (!(m->embd->type == GGML_F32 || m->embd->type == GGML_F16 || m->embd->type == GGML_BF16 ||
          m->embd->type == GGML_Q4_0 || m->embd->type == GGML_Q8_0 || m->embd->type == GGML_Q4_K ||
          m->embd->type == GGML_Q5_K || m->embd->type == GGML_Q6_K))
        return bail(fail(LLMDOT_E_UNSUPPORTED, "token_embd type not supported"));
    if ((rc = norm_f32(m, onorm, d.hidden, &m->out_norm_f))) return bail(rc);
    m->L.resize((size_t)d.layers);
    // Fused Q/K/V (QkvLayout.Fused, ArchitectureResolver.cs:145-146: some
    // tensor is an attn_qkv): every layer then has blk.N.attn_qkv.weight
    // (TensorNameResolver.cs:123-126) of qdim + 2 kvdim rows, Q, K, V in that
    // order, and the reference's one product over it split into q, k, v
    // (IE:321-332) equals the three products over its row ranges, each output
    // row being its own dot product: Q, K and V are views of the one tensor.
    bool fused = false;
    for (int l = 0; l < d.layers && !fused; l++)
        fused = m->ctx->weights.count(m->prefix + "blk." + std::to_string(l) + ".attn_qkv.weight") > 0;
    for (int l = 0; l < d.layers; l++) {
        LayerW& w = m->L[l];
        const std::string p = "blk." + std::to_string(l) + ".";
        if ((rc = need_w(m, p + "attn_norm.weight", -1, -1, &w.attn_norm))) return bail(rc);
        w.ffn_norm = find_w(m, p + "ffn_norm.weight");
        if (!w.ffn_norm) w.ffn_norm = w.attn_norm;   // IE:547
        if (fused) {
            const Weight* f = find_w(m, p + "attn_qkv.weight");
            if (!f)
                return bail(fail(LLMDOT_E_NOT_FOUND, "Expected fused QKV tensor '" + m->prefix + p +
                                                         "attn_qkv.weight' for QkvLayout.Fused."));
            if ((rc = need_w(m, p + "attn_qkv.weight", qdim + 2 * kvdim, d.hidden, &f))) return bail(rc);
            const int64_t rb = byte_count(f->type, d.hidden);
            auto view = [&](int64_t r0, int64_t nr) {
                Weight& v = m->views.emplace_back();
                v.type = f->type;
                v.rows = nr;
                v.cols = d.hidden;
                v.nbytes = (size_t)(nr * rb);
                v.dev = f->dev + r0 * rb;
                return (const Weight*)&v;
            };
            w.q = view(0, qdim);
            w.k = view(qdim, kvdim);
            w.v = view(qdim + kvdim, kvdim);
        } else {
            if ((rc = need_w(m, p + "attn_q.weight", qdim, d.hidden, &w.q))) return bail(rc);
            if ((rc = need_w(m, p + "attn_k.weight", kvdim, d.hidden, &w.k))) return bail(rc);
            if ((rc = need_w(m, p + "attn_v.weight", kvdim, d.hidden, &w.v))) return bail(rc);
        }
        if ((rc = need_w(m, p + "attn_output.weight", d.hidden, qdim, &w.o))) return bail(rc);
        if ((rc = need_w(m, p + "ffn_gate.weight", d.ffn, d.hidden, &w.gate))) return bail(rc);
        if ((rc = need_w(m, p + "ffn_up.weight", d.ffn, d.hidden, &w.up))) return bail(rc);
        if ((rc = need_w(m, p + "ffn_down.weight", d.hidden, d.ffn, &w.down))) return bail(rc);
        const Weight* all[7] = {w.q, w.k, w.v, w.o, w.gate, w.up, w.down};
        const char* nm[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
        for (int i = 0; i < 7; i++)
            if ((rc = check_gemv_type(all[i], p + nm[i]))) return bail(rc);
        if (w.gate->type != w.up->type) return bail(fail(LLMDOT_E_UNSUPPORTED, "ffn_gate and ffn_up must share a type"));
        if ((rc = norm_f32(m, w.attn_norm, d.hidden, &w.attn_norm_f))) return bail(rc);
        if ((rc = norm_f32(m, w.ffn_norm, d.hidden, &w.ffn_norm_f))) return bail(rc);
        // optional per-head Q/K norms (attn_q_norm / attn_k_norm, head_dim each)
        if (const Weight* qn = find_w(m, p + "attn_q_norm.weight"))
            if ((rc = norm_f32(m, qn, d.head_dim, &w.q_norm_f))) return bail(rc);
        if (const Weight* kn = find_w(m, p + "attn_k_norm.weight"))
            if ((rc = norm_f32(m, kn, d.head_dim, &w.k_norm_f))) return bail(rc);
    }
    // RoPE tables: PrecomputeRopeFrequencies (IE:57-72) then, per position, the
    // reference's per-call cosf/sinf of position * freq (TO:688-693).
    const int rot = d.rope_dim > 0 ? d.rope_dim : d.head_dim;
    m->rope_half = rot / 2;
    if (2 * m->rope_half > d.head_dim) return bail(fail(LLMDOT_E_INVALID, "rope_dim exceeds head_dim"));
    {
        std::vector<float> freq((size_t)m->rope_half);
        for (int i = 0; i < m->rope_half; i++) {
            float f = 1.0f / powf(d.rope_base, 2.0f * (float)i / (float)rot);
            if (d.rope_linear_factor > 1.0f) f /= d.rope_linear_factor;
            freq[i] = f;
        }
        const size_t n = (size_t)d.context * (size_t)(m->rope_half > 0 ? m->rope_half : 1);
        std::vector<float> cs(n, 1.0f), sn(n, 0.0f);
        for (int t = 0; t < d.context; t++)
            for (int i = 0; i < m->rope_half; i++) {
                float angle = (float)t * freq[i];
                cs[(size_t)t * m->rope_half + i] = cosf(angle);
                sn[(size_t)t * m->rope_half + i] = sinf(angle);
            }
        void *pc, *ps;
        if ((rc = dalloc(m, n * sizeof(float), &pc)) || (rc = dalloc(m, n * sizeof(float), &ps))) return bail(rc);
        m->cos_tab = (float*)pc; m->sin_tab = (float*)ps;
        if ((rc = copy_in(ctx, pc, cs.data(), n * sizeof(float))) || (rc = copy_in(ctx, ps, sn.data(), n * sizeof(float))))
            return bail(rc);
    }
    void* p;
    auto A = [&](size_t n, void** dst) { return dalloc(m, n, dst); };
    if ((rc = A(sizeof(float) * d.hidden, &p))) return bail(rc); m->h = (float*)p;
    if ((rc = A(sizeof(float) * qdim, &p))) return bail(rc); m->q = (float*)p;
    if ((rc = A(sizeof(float) * kvdim, &p))) return bail(rc); m->k = (float*)p;
    if ((rc = A(sizeof(float) * kvdim, &p))) return bail(rc); m->v = (float*)p;
    if ((rc = A(sizeof(float) * qdim, &p))) return bail(rc); m->attn = (float*)p;
    if ((rc = A(sizeof(float) * d.ffn, &p))) return bail(rc); m->act = (float*)p;
    if ((rc = A(sizeof(float) * d.hidden, &p))) return bail(rc); m->xn = (float*)p;
    if ((rc = A(sizeof(float) * (d.hidden / 4), &p))) return bail(rc); m->xssq = (float*)p;
    if ((rc = A(sizeof(float) * d.vocab, &p))) return bail(rc); m->logits = (float*)p;
    const size_t elt = d.kv_fp16 ? 2 : 4;
    m->kv_layer_bytes = (size_t)d.kv_heads * d.context * d.head_dim * elt;
    if ((rc = A(m->kv_layer_bytes * d.layers, &p))) return bail(rc); m->kcache = (uint8_t*)p;
    if ((rc = A(m->kv_layer_bytes * d.layers, &p))) return bail(rc); m->vcache = (uint8_t*)p;
    const int nch = attn_max_chunks(d.heads, d.kv_heads, d.context);
    if ((rc = A(sizeof(float) * (size_t)d.heads * d.context, &p))) return bail(rc); m->scores = (float*)p;
    if ((rc = A(sizeof(float) * (size_t)d.heads * nch, &p))) return bail(rc); m->chunk_max = (float*)p;
    if ((rc = A(sizeof(float) * (size_t)nch * qdim, &p))) return bail(rc); m->part_out = (float*)p;
    if ((rc = A(sizeof(float) * (size_t)nch * d.heads, &p))) return bail(rc); m->part_sum = (float*)p;
    m->attn_fused = attn_fused_ok(d.heads, d.kv_heads, d.head_dim, d.context);
    if (const char* v = getenv("LLMDOT_HIP_ATTN_FUSED")) m->attn_fused = m->attn_fused && strcmp(v, "0") != 0;
    if (const char* v = getenv("LLMDOT_HIP_ATTN_SPIN")) m->attn_spin = atoi(v) >= 0 ? atoi(v) : m->attn_spin;
    if (d.sliding_window < 0) return bail(fail(LLMDOT_E_INVALID, "negative sliding window"));
    if (d.sliding_window > 0 && !m->attn_fused)
        return bail(fail(LLMDOT_E_UNSUPPORTED, "sliding-window attention needs the one-launch attention "
                                               "(at most 16384 positions, LLMDOT_HIP_ATTN_FUSED not 0)"));
    if ((rc = A(sizeof(uint64_t) * (size_t)attn_xmax_slots(d.heads), &p))) return bail(rc); m->xmax = (uint64_t*)p;
    // The XCD-local chunk-maximum exchange where the shape fits it (attn_xcd_fits)
    // and the device deals workgroups to XCDs in turn; LLMDOT_HIP_ATTN_XCD=0 keeps
    // the exchange through the coherence point.
    {
        const char* v = getenv("LLMDOT_HIP_ATTN_XCD");
        int cus = 0;
        HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->ctx->device));
        bool want = m->attn_fused && !(v && strcmp(v, "0") == 0) &&
                    attn_xcd_fits(d.heads, d.kv_heads, d.head_dim, d.context, d.kv_fp16 ? 1 : 0, cus);
        if (want) {
            bool ok = false;
            HIPCHK(attn_xcd_check(m->ctx->stream, &ok));
            want = ok;
        }
        m->attn_xcd_exchange = want;
        if (want && (rc = A(sizeof(uint64_t) * (size_t)nch * d.heads * (d.head_dim + 1), &p))) return bail(rc);
        if (want) m->xpart = (uint64_t*)p;
    }
    if ((rc = A(64, &p))) return bail(rc); m->ints = (int32_t*)p;
    if ((rc = A(sizeof(int32_t) * (size_t)(d.context + 1), &p))) return bail(rc); m->token_log = (int32_t*)p;
    {
        const int g = gemv_max_grid(m->out->type, EPI_ARGMAX, d.vocab, d.hidden);
        m->am_cap = g;
        if ((rc = A(sizeof(float) * (size_t)g, &p))) return bail(rc); m->am_val = (float*)p;
        if ((rc = A(sizeof(int32_t) * (size_t)g, &p))) return bail(rc); m->am_idx = (int32_t*)p;
    }
    m->pf_eligible = prefill_check(m);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return bail(fail(LLMDOT_E_DEVICE, "synchronize failed"));
    if ((rc = build_graph(m))) {
        // fall back to eager launches
        m->use_graph = false;
        if (m->graph) { (void)hipGraphExecDestroy(m->graph); m->graph = nullptr; }
        (void)hipGetLastError();
    }
    *out = m;
    return 0;
}

extern "C" int32_t llmdot_hip_model_reset(llmdot_hip_model* m) {
    if (!m) return fail(LLMDOT_E_INVALID, "null model");
    m->gen.active = false;
    if (int rc = set_int(m, m_pos(m), 0)) return rc;
    if (int rc = set_int(m, m_step(m), 0)) return rc;
    HIPCHK(hipStreamSynchronize(m->ctx->stream));
    return 0;
}

namespace {
int check_token(llmdot_hip_model* m, int32_t token) {
    if (token < 0 || token >= m->embd->rows) return fail(LLMDOT_E_RANGE, "token id out of range");
    return 0;
}
int check_pos(llmdot_hip_model* m, int32_t pos) {
    if (pos < 0 || pos >= m->d.context) return fail(LLMDOT_E_RANGE, "position outside the KV cache");
    return 0;
}
// Device waits that gave up (the attention's chunk-maximum exchange; in the
// XCD-local form also a chunk placed on another XCD than its kv head's) leave
// a flag; it is reported once and cleared.
int check_device_flags(llmdot_hip_model* m) {
    hipStream_t s = m->ctx->stream;
    int32_t err = 0;
    HIPCHK(hipMemcpyAsync(&err, m_err(m), sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIPCHK(hipStreamSynchronize(s));
    if (err) {
        HIPCHK(launch_set_scalar(m_err(m), 0, s));
        HIPCHK(hipStreamSynchronize(s));
        return fail(LLMDOT_E_DEVICE, "decode attention: a workgroup gave up waiting for the chunk maxima of its kv "
                                     "head (spin limit, or with the XCD-local form a chunk on another XCD: "
                                     "LLMDOT_HIP_ATTN_XCD=0 avoids it); the step's results are invalid");
    }
    return 0;
}

int fetch_outputs(llmdot_hip_model* m, float* logits, int32_t* am) {
    hipStream_t s = m->ctx->stream;
    if (logits) HIPCHK(hipMemcpyAsync(logits, m->logits, sizeof(float) * (size_t)m->d.vocab, hipMemcpyDeviceToHost, s));
    if (am) HIPCHK(hipMemcpyAsync(am, m_token(m), sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIPCHK(hipStreamSynchronize(s));
    return check_device_flags(m);
}
}  // namespace

extern "C" int32_t llmdot_hip_decode_step(llmdot_hip_model* m, int32_t token, int32_t position, float* logits, int32_t* am) {
    if (!m) return fail(LLMDOT_E_INVALID, "null model");
    m->gen.active = false;   // the step changes the state a streaming Generate continues from
    if (int rc = check_token(m, token)) return rc;
    if (int rc = check_pos(m, position)) return rc;
    if (int rc = set_int(m, m_token(m), token)) return rc;
    if (int rc = set_int(m, m_pos(m), position)) return rc;
    if (int rc = run_step(m)) return rc;
    return fetch_outputs(m, logits, am);
}

extern "C" int32_t llmdot_hip_prefill(llmdot_hip_model* m, const int32_t* tokens, int32_t n, int32_t pos0, float* logits,
                                      int32_t* am) {
    if (!m || (!tokens && n > 0) || n < 0) return fail(LLMDOT_E_INVALID, "bad prefill arguments");
    m->gen.active = false;
    if (n == 0) return 0;
    if (int rc = check_pos(m, pos0)) return rc;
    if (int rc = check_pos(m, pos0 + n - 1)) return rc;
    for (int i = 0; i < n; i++)
        if (int rc = check_token(m, tokens[i])) return rc;
    if (use_batched_prefill(m, n)) {
        if (int rc = prefill_batched(m, tokens, n, pos0, false)) return rc;
        return fetch_outputs(m, logits, am);
    }
    if (int rc = set_int(m, m_pos(m), pos0)) return rc;
    for (int i = 0; i < n; i++) {
        if (int rc = set_int(m, m_token(m), tokens[i])) return rc;
        if (int rc = run_step(m)) return rc;
    }
    return fetch_outputs(m, logits, am);
}

namespace {

// Draw the token from the logits the head just wrote (after its argmax pass
// advanced the step), replacing the argmax in the token slot and log.
int enqueue_sample(llmdot_hip_model* m, const llmdot_hip_sampling* opt, int hist_base) {
    SampleArgs sa{};
    sa.logits = m->logits; sa.n = m->d.vocab; sa.inv_temp = 1.0f / opt->temperature;
    sa.top_k = opt->top_k; sa.top_p = opt->top_p; sa.penalty = opt->repeat_penalty; sa.window = opt->repeat_window;
    sa.hist = m->s_hist; sa.hist_base = hist_base; sa.step = m_step(m); sa.rvals = m->s_draws;
    sa.work = m->s_work; sa.token_out = m_token(m);
    sa.token_log = m->token_log; sa.log_cap = m->d.context + 1; sa.hist_out = m->s_hist;
    HIPCHK(launch_sample(sa, m->ctx->stream));
    return 0;
}

// Generate up to the first token (IE:79-101, then the first Sample): the cache
// reset, the prompt, and token 0 left in the token log; the session is armed.
int generate_begin(llmdot_hip_model* m, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens, int32_t eos,
                   const llmdot_hip_sampling* opt, const float* draws) {
    if (!m || (!prompt && n_prompt > 0) || n_prompt < 0 || max_tokens < 0)
        return fail(LLMDOT_E_INVALID, "bad Generate arguments");
    m->gen = {};
    const auto& d = m->d;
    const bool sampled = opt && opt->temperature > 0.f;   // Sampler.cs:26-27: greedy otherwise
    if (sampled && !draws && max_tokens > 0) return fail(LLMDOT_E_INVALID, "sampled Generate needs the uniform draws");
    if (sampled && !sample_supported(d.vocab, opt->top_k))
        return fail(LLMDOT_E_UNSUPPORTED, "TopK between " + std::to_string(SAMPLE_MAX_K) + " and the vocabulary size is not supported");
    std::vector<int32_t> pr(prompt, prompt + n_prompt);
    if (pr.empty()) pr.push_back(d.bos > 0 ? d.bos : 0);   // IE:90-95
    const int np = (int)pr.size();
    for (int t : pr)
        if (int rc = check_token(m, t)) return rc;
    if (np > d.context) return fail(LLMDOT_E_RANGE, "prompt longer than the KV cache");
    auto& g = m->gen;
    g.sampled = sampled; g.max_tokens = max_tokens; g.eos = eos; g.hist_base = n_prompt;
    if (sampled) g.opt = *opt;
    if (max_tokens == 0) { g.active = true; g.done = true; return 0; }
    // Token g (0-based) is sampled after position np-1+g; producing it needs
    // np + g steps, and positions stop at context - 1.
    const int fit = d.context - np + 1;
    g.produce = max_tokens < fit ? max_tokens : fit;
    hipStream_t s = m->ctx->stream;
    if (sampled) {
        // recentTokens starts as the prompt (IE:101); draws on the device
        if (!m->s_hist) {
            void *h, *r, *w;
            if (int rc = dalloc(m, sizeof(int32_t) * (size_t)(d.context + 1), &h)) return rc;
            if (int rc = dalloc(m, sizeof(float) * (size_t)(d.context + 1), &r)) return rc;
            if (int rc = dalloc(m, sizeof(float) * sample_work_floats(d.vocab), &w)) return rc;
            m->s_hist = (int32_t*)h; m->s_draws = (float*)r; m->s_work = (float*)w;
        }
        if (n_prompt > 0)
            HIPCHK(hipMemcpyAsync(m->s_hist, prompt, sizeof(int32_t) * (size_t)n_prompt, hipMemcpyHostToDevice, s));
        HIPCHK(hipMemcpyAsync(m->s_draws, draws, sizeof(float) * (size_t)g.produce, hipMemcpyHostToDevice, s));
    }
    if (use_batched_prefill(m, np)) {
        if (int rc = prefill_batched(m, pr.data(), np, 0, true)) return rc;   // KvCache.Reset (IE:79) + prompt
    } else {
        if (int rc = set_int(m, m_pos(m), 0)) return rc;   // KvCache.Reset (IE:79)
        for (int i = 0; i < np; i++) {
            if (i == np - 1)
                if (int rc = set_int(m, m_step(m), 0)) return rc;
            if (int rc = set_int(m, m_token(m), pr[i])) return rc;
            if (int rc = run_step(m)) return rc;
        }
    }
    if (sampled)
        if (int rc = enqueue_sample(m, &g.opt, g.hist_base)) return rc;
    g.computed = 1;
    g.active = true;
    return 0;
}

// One more token on the device: the step that consumes the last computed
// token (ProcessToken, IE:127), then its Sample.
int generate_advance(llmdot_hip_model* m) {
    if (int rc = run_step(m)) return rc;
    if (m->gen.sampled)
        if (int rc = enqueue_sample(m, &m->gen.opt, m->gen.hist_base)) return rc;
    m->gen.computed++;
    return 0;
}

// Returns up to max_k further tokens (and, when logits_out is given, the
// logits each was taken from).  On entry token `yielded` is computed and its
// logits are the model's current ones.  After the tokens are copied out, the
// step for the next token is enqueued (not waited for), so the device works
// while the caller handles these tokens.
int generate_next(llmdot_hip_model* m, int32_t max_k, int32_t* tokens_out, int32_t* n_out, int32_t* done,
                  float* logits_out) {
    if (!m || !n_out || !done || max_k < 1 || !tokens_out) return fail(LLMDOT_E_INVALID, "bad Generate arguments");
    *n_out = 0;
    *done = 0;
    auto& g = m->gen;
    if (!g.active) return fail(LLMDOT_E_INVALID, "no Generate in progress on this model");
    if (g.done) { *done = 1; return 0; }
    const auto& d = m->d;
    hipStream_t s = m->ctx->stream;
    const int want = std::min(max_k, g.produce - g.yielded);
    if (logits_out) HIPCHK(hipMemcpyAsync(logits_out, m->logits, sizeof(float) * d.vocab, hipMemcpyDeviceToHost, s));
    for (int i = 1; i < want; i++) {
        if (g.computed < g.yielded + i + 1)
            if (int rc = generate_advance(m)) return rc;
        if (logits_out)
            HIPCHK(hipMemcpyAsync(logits_out + (size_t)i * d.vocab, m->logits, sizeof(float) * d.vocab,
                                  hipMemcpyDeviceToHost, s));
    }
    HIPCHK(hipMemcpyAsync(tokens_out, m->token_log + g.yielded, sizeof(int32_t) * (size_t)want, hipMemcpyDeviceToHost, s));
    HIPCHK(hipStreamSynchronize(s));
    if (int rc = check_device_flags(m)) { g.active = false; return rc; }
    int n = want;
    bool eos_hit = false;
    if (g.eos >= 0)
        for (int i = 0; i < want; i++)
            if (tokens_out[i] == g.eos) { n = i + 1; eos_hit = true; break; }   // IE:112-115
    *n_out = n;
    g.yielded += n;
    if (eos_hit || g.yielded == g.produce) {
        g.done = true;
        *done = 1;
        if (!eos_hit && g.produce < g.max_tokens) return fail(LLMDOT_E_RANGE, "generation reached the end of the KV cache");
        return 0;
    }
    return generate_advance(m);   // the next call's first token
}

int generate_impl(llmdot_hip_model* m, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens, int32_t eos,
                  const llmdot_hip_sampling* opt, const float* draws, int32_t* tokens_out, int32_t* n_out,
                  float* logits_out) {
    if (!n_out || (!tokens_out && max_tokens > 0)) return fail(LLMDOT_E_INVALID, "bad Generate arguments");
    *n_out = 0;
    if (int rc = generate_begin(m, prompt, n_prompt, max_tokens, eos, opt, draws)) return rc;
    int32_t done = 0;
    int rc = max_tokens > 0 ? generate_next(m, max_tokens, tokens_out, n_out, &done, logits_out) : 0;
    m->gen.active = false;
    return rc;
}

}  // namespace

extern "C" int32_t llmdot_hip_generate(llmdot_hip_model* m, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens,
                                       int32_t eos, int32_t* tokens_out, int32_t* n_out, float* logits_out) {
    return generate_impl(m, prompt, n_prompt, max_tokens, eos, nullptr, nullptr, tokens_out, n_out, logits_out);
}

extern "C" int32_t llmdot_hip_generate_sampled(llmdot_hip_model* m, const int32_t* prompt, int32_t n_prompt,
                                               int32_t max_tokens, int32_t eos, const llmdot_hip_sampling* opt,
                                               const float* draws, int32_t* tokens_out, int32_t* n_out,
                                               float* logits_out) {
    if (!opt) return fail(LLMDOT_E_INVALID, "null sampling options");
    return generate_impl(m, prompt, n_prompt, max_tokens, eos, opt, draws, tokens_out, n_out, logits_out);
}

extern "C" int32_t llmdot_hip_generate_begin(llmdot_hip_model* m, const int32_t* prompt, int32_t n_prompt,
                                             int32_t max_tokens, int32_t eos, const llmdot_hip_sampling* opt,
                                             const float* draws) {
    return generate_begin(m, prompt, n_prompt, max_tokens, eos, opt, draws);
}

extern "C" int32_t llmdot_hip_generate_next(llmdot_hip_model* m, int32_t max_k, int32_t* tokens_out, int32_t* n_out,
                                            int32_t* done, float* logits_out) {
    return generate_next(m, max_k, tokens_out, n_out, done, logits_out);
}

extern "C" int32_t llmdot_hip_kv_read(llmdot_hip_model* m, int32_t layer, int32_t position, float* k, float* v) {
    if (!m || !k || !v) return fail(LLMDOT_E_INVALID, "null argument");
    if (layer < 0 || layer >= m->d.layers) return fail(LLMDOT_E_RANGE, "layer out of range");
    if (int rc = check_pos(m, position)) return rc;
    const auto& d = m->d;
    const size_t elt = d.kv_fp16 ? 2 : 4;
    std::vector<uint8_t> kb((size_t)d.head_dim * elt), vb((size_t)d.head_dim * elt);
    HIPCHK(hipStreamSynchronize(m->ctx->stream));
    for (int h = 0; h < d.kv_heads; h++) {
        const size_t off = (size_t)layer * m->kv_layer_bytes + (((size_t)h * d.context + position) * d.head_dim) * elt;
        HIPCHK(hipMemcpy(kb.data(), m->kcache + off, kb.size(), hipMemcpyDeviceToHost));
        HIPCHK(hipMemcpy(vb.data(), m->vcache + off, vb.size(), hipMemcpyDeviceToHost));
        for (int i = 0; i < d.head_dim; i++) {
            if (d.kv_fp16) {
                _Float16 hk, hv;
                memcpy(&hk, kb.data() + 2 * i, 2);
                memcpy(&hv, vb.data() + 2 * i, 2);
                k[h * d.head_dim + i] = (float)hk;
                v[h * d.head_dim + i] = (float)hv;
            } else {
                memcpy(&k[h * d.head_dim + i], kb.data() + 4 * i, 4);
                memcpy(&v[h * d.head_dim + i], vb.data() + 4 * i, 4);
            }
        }
    }
    return 0;
}

extern "C" int32_t llmdot_hip_model_step_bytes(llmdot_hip_model* m, int32_t position, double* bytes) {
    if (!m || !bytes) return fail(LLMDOT_E_INVALID, "null argument");
    const auto& d = m->d;
    double b = 0;
    for (const auto& w : m->L) {
        const Weight* all[7] = {w.q, w.k, w.v, w.o, w.gate, w.up, w.down};
        for (auto* x : all) b += (double)x->nbytes;
        b += (double)w.attn_norm->nbytes + (w.ffn_norm != w.attn_norm ? (double)w.ffn_norm->nbytes : 0.0);
    }
    b += (double)m->out->nbytes + (double)m->out_norm->nbytes;
    b += (double)byte_count(m->embd->type, d.hidden);
    const double elt = d.kv_fp16 ? 2.0 : 4.0;
    b += (double)d.layers * 2.0 * (double)(position + 1) * (double)(d.kv_heads * d.head_dim) * elt;
    *bytes = b;
    return 0;
}

extern "C" int32_t llmdot_hip_model_kv_fill_random(llmdot_hip_model* m, int32_t n, uint64_t seed) {
    if (!m) return fail(LLMDOT_E_INVALID, "null model");
    m->gen.active = false;
    if (n < 0 || n > m->d.context) return fail(LLMDOT_E_RANGE, "fill length outside the KV cache");
    const auto& d = m->d;
    HIPCHK(launch_kv_fill(m->kcache, 0, d.layers, d.kv_heads, d.context, d.head_dim, n, seed, d.kv_fp16, m->ctx->stream));
    HIPCHK(launch_kv_fill(m->vcache, 1, d.layers, d.kv_heads, d.context, d.head_dim, n, seed, d.kv_fp16, m->ctx->stream));
    HIPCHK(hipStreamSynchronize(m->ctx->stream));
    return 0;
}

extern "C" int32_t llmdot_hip_model_time_prefill(llmdot_hip_model* m, const int32_t* tokens, int32_t n, int32_t pos0,
                                                 float* ms) {
    if (!m || !tokens || n <= 0 || !ms) return fail(LLMDOT_E_INVALID, "bad prefill timing arguments");
    m->gen.active = false;
    if (!m->pf_eligible) return fail(LLMDOT_E_UNSUPPORTED, "the model's weight types have no batched prefill kernel");
    if (int rc = check_pos(m, pos0)) return rc;
    if (int rc = check_pos(m, pos0 + n - 1)) return rc;
    for (int i = 0; i < n; i++)
        if (int rc = check_token(m, tokens[i])) return rc;
    if (int rc = ensure_prefill_ws(m)) return rc;
    hipStream_t s = m->ctx->stream;
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipStreamSynchronize(s));
    HIPCHK(hipEventRecord(e0, s));
    int rc = prefill_batched(m, tokens, n, pos0, false);
    if (rc == 0) {
        HIPCHK(hipEventRecord(e1, s));
        HIPCHK(hipEventSynchronize(e1));
        HIPCHK(hipEventElapsedTime(ms, e0, e1));
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

extern "C" int32_t llmdot_hip_model_time_decode(llmdot_hip_model* m, int32_t first_token, int32_t position, int32_t steps,
                                                int32_t per_kernel, llmdot_hip_step_timing* out) {
    if (!m || !out || steps <= 0) return fail(LLMDOT_E_INVALID, "bad timing arguments");
    m->gen.active = false;
    if (int rc = check_token(m, first_token)) return rc;
    if (int rc = check_pos(m, position)) return rc;
    if (position + steps > m->d.context) return fail(LLMDOT_E_RANGE, "timed steps run past the KV cache");
    memset(out, 0, sizeof *out);
    hipStream_t s = m->ctx->stream;
    if (int rc = set_int(m, m_token(m), first_token)) return rc;
    if (int rc = set_int(m, m_pos(m), position)) return rc;
    if (int rc = set_int(m, m_step(m), 0)) return rc;
    // the dominant kernel alone: every layer's gate/up launch back to back
    // (distinct weights per layer, past any cache), captured once and replayed
    // so that host enqueue gaps stay out of the timed region
    hipGraphExec_t kg = nullptr;
    if (per_kernel) {
        hipGraph_t g = nullptr;
        HIPCHK(hipStreamSynchronize(s));
        HIPCHK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        hipError_t le = hipSuccess;
        for (int l = 0; l < m->d.layers && le == hipSuccess; l++) le = launch_gate_up(m, l);
        const hipError_t ce = hipStreamEndCapture(s, &g);
        if (le != hipSuccess || ce != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return fail(LLMDOT_E_DEVICE, std::string("gate/up capture: ") + hipGetErrorString(le != hipSuccess ? le : ce));
        }
        const hipError_t ie = hipGraphInstantiate(&kg, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ie != hipSuccess) return fail(LLMDOT_E_DEVICE, std::string("gate/up graph: ") + hipGetErrorString(ie));
    }
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipStreamSynchronize(s));
    HIPCHK(hipEventRecord(e0, s));
    int launches = 0;
    hipError_t re = hipSuccess;
    for (int i = 0; i < steps && re == hipSuccess; i++) {
        if (per_kernel) {
            re = hipGraphLaunch(kg, s);
            launches += m->d.layers;
        } else if (int rc = run_step(m)) {
            if (kg) (void)hipGraphExecDestroy(kg);
            return rc;
        }
    }
    HIPCHK(hipEventRecord(e1, s));
    HIPCHK(hipEventSynchronize(e1));
    if (kg) (void)hipGraphExecDestroy(kg);
    HIPCHK(re);
    float total = 0;
    HIPCHK(hipEventElapsedTime(&total, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (int rc = check_device_flags(m)) return rc;
    const double gemv_ms = per_kernel ? total : 0.0;
    out->total_ms = total;
    out->gemv_ms = (float)gemv_ms;
    out->gemv_launches = launches;
    if (per_kernel && !m->L.empty()) {
        const LayerW& w = m->L[0];
        // weights + the packed RmsNorm input (w*h, one sum of squares per 4
        // elements) + the SwiGLU output
        out->gemv_bytes = (double)launches * ((double)w.gate->nbytes + (double)w.up->nbytes +
                                              4.0 * (m->d.hidden + m->d.hidden / 4.0 + (double)m->d.ffn));
    }
    return 0;
}
