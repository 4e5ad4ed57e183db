// attention.hip -- GQA decode attention over the KV cache for one layer.
//
// Restates InferenceEngine.AttentionForward after the projections
// (src/Llmdot.Core/Inference/InferenceEngine.cs:355-442):
//   RoPE on each q head and on the new k head (TensorOps.ApplyRoPE with the
//   precomputed frequency table, TO:679-743), KV write at slot T (IE:380-381),
//   score_s = (q . K_s) * (1/sqrt(hd)), Softmax (VectorMath.cs:215-258: global
//   max M, ExpApprox(s - M) for s < 8*floor(n/8), expf for the tail), and
//   out = sum_s p_s V_s.  q head h reads kv head h / (H/Hkv).
//
// The reference's ExpApprox is not multiplicative, so an online (rescaling)
// softmax cannot reproduce it; the global max must be known before any
// exponent.  Two kernels therefore split the sequence into chunks of C
// positions per kv head:
//   phase 1: RoPE + KV write + scores of the chunk + per-chunk max (per q head)
//   phase 2: global max from the chunk maxima, exponentials, chunk partial
//            sum(e) and sum(e V); the last workgroup of each kv head combines
//            the chunk partials (out = sum(eV) / sum(e)).
// Each K/V row is read from HBM exactly once per layer.  cos/sin come from a
// host table computed with the same libm calls as the reference, so RoPE is
// bit-exact.
#include "common.h"
#include "kernels.h"

namespace llmdot {

namespace {

constexpr int WG = 256;

__device__ __forceinline__ float load_kv(const void* cache, int64_t idx, int fp16) {
    if (fp16) return (float)reinterpret_cast<const _Float16*>(cache)[idx];
    return reinterpret_cast<const float*>(cache)[idx];
}
__device__ __forceinline__ float store_kv(void* cache, int64_t idx, float v, int fp16) {
    if (fp16) {
        _Float16 h = (_Float16)v;                       // round to nearest even
        reinterpret_cast<_Float16*>(cache)[idx] = h;
        return (float)h;
    }
    reinterpret_cast<float*>(cache)[idx] = v;
    return v;
}

// NeoX rotation of element d of a head (pairs (i, i + half), dims >= 2*half untouched).
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, float c_lo, float s_lo) {
#pragma clang fp contract(off)
    if (d < half) return ((x[d] * c_lo) - (x[d + half] * s_lo));
    if (d < 2 * half) return ((x[d - half] * s_lo) + (x[d] * c_lo));
    return x[d];
}

template <int HD>
__global__ __launch_bounds__(WG) void attn_scores_kernel(AttnArgs a, int C, int G) {
    extern __shared__ float smem[];
    float* q_s = smem;                      // [G][HD]
    float* k_s = smem + G * HD;             // [C][HD + 1]
    __shared__ float red_max[WG / 16];

    const int T = *a.pos, n = T + 1;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int p0 = c * C;
    if (p0 >= n) return;
    const int cnt = min(C, n - p0);
    const int half = a.rope_half;
    const float* cs = a.cos_tab + (int64_t)T * half;
    const float* sn = a.sin_tab + (int64_t)T * half;

    for (int idx = threadIdx.x; idx < G * HD; idx += WG) {
        const int h = idx / HD, d = idx - h * HD;
        const float* qh = a.q + (int64_t)(kvh * G + h) * HD;
        const int i = d < half ? d : d - half;
        const float cv = i < half ? cs[i] : 1.f, sv = i < half ? sn[i] : 0.f;
        q_s[idx] = rope_elem(qh, d, half, cv, sv);
    }
    const int64_t cache_base = (int64_t)kvh * a.context * HD;
    for (int idx = threadIdx.x; idx < cnt * HD; idx += WG) {
        const int p = idx / HD, d = idx - p * HD;
        k_s[p * (HD + 1) + d] = load_kv(a.kcache, cache_base + (int64_t)(p0 + p) * HD + d, a.kv_fp16);
    }
    __syncthreads();
    if (T >= p0 && T < p0 + C) {
        // this workgroup owns the new token: rotate k, store K/V slot T
        const float* kh = a.k + (int64_t)kvh * HD;
        const float* vh = a.v + (int64_t)kvh * HD;
        for (int d = threadIdx.x; d < HD; d += WG) {
            const int i = d < half ? d : d - half;
            const float cv = i < half ? cs[i] : 1.f, sv = i < half ? sn[i] : 0.f;
            float kr = rope_elem(kh, d, half, cv, sv);
            const int64_t slot = cache_base + (int64_t)T * HD + d;
            k_s[(T - p0) * (HD + 1) + d] = store_kv(a.kcache, slot, kr, a.kv_fp16);
            store_kv(a.vcache, slot, vh[d], a.kv_fp16);
        }
        __syncthreads();
    }

    // dot products: TPD threads per (head, position)
    const int TPD = WG / (G * C);
    const int di = threadIdx.x / TPD, sub = threadIdx.x - di * TPD;
    const int h = di / C, p = di - h * C;
    const int per = HD / TPD;
    float s = 0.f;
    if (h < G && p < cnt) {
        const float* qv = q_s + h * HD + sub * per;
        const float* kv = k_s + p * (HD + 1) + sub * per;
        for (int d = 0; d < per; d++) s += qv[d] * kv[d];
    }
    for (int o = 1; o < TPD; o <<= 1) s += __shfl_xor(s, o, 64);
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    float score = (s * inv_sqrt);
    const bool live = h < G && p < cnt && sub == 0;
    if (live) a.scores[(int64_t)(kvh * G + h) * a.context + p0 + p] = score;
    // per-head max over this chunk: head h owns threads [h*C*TPD, (h+1)*C*TPD)
    const int span = C * TPD, width = span < 64 ? span : 64;
    float m = live ? score : -INFINITY;
    for (int o = 1; o < width; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & (width - 1)) == 0) red_max[threadIdx.x / width] = m;
    __syncthreads();
    if (threadIdx.x < G) {
        const int gph = span / width;
        float mm = -INFINITY;
        for (int i = 0; i < gph; i++) mm = fmaxf(mm, red_max[threadIdx.x * gph + i]);
        a.chunk_max[(int64_t)(kvh * G + threadIdx.x) * gridDim.x + c] = mm;
    }
}

template <int HD>
__global__ __launch_bounds__(WG) void attn_pv_kernel(AttnArgs a, int C, int G) {
    extern __shared__ float smem[];
    float* v_s = smem;                      // [C][HD + 1]
    float* p_s = smem + C * (HD + 1);       // [G][C]
    __shared__ float gmax[16];
    __shared__ int is_last;

    const int T = *a.pos, n = T + 1, n8 = n & ~7;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int p0 = c * C;
    if (p0 >= n) return;
    const int cnt = min(C, n - p0);
    const int nch = (n + C - 1) / C;

    if (threadIdx.x < G) {
        const float* cm = a.chunk_max + (int64_t)(kvh * G + threadIdx.x) * gridDim.x;
        float m = -INFINITY;
        for (int i = 0; i < nch; i++) m = fmaxf(m, cm[i]);
        gmax[threadIdx.x] = m;
    }
    const int64_t cache_base = (int64_t)kvh * a.context * HD;
    for (int idx = threadIdx.x; idx < cnt * HD; idx += WG) {
        const int p = idx / HD, d = idx - p * HD;
        v_s[p * (HD + 1) + d] = load_kv(a.vcache, cache_base + (int64_t)(p0 + p) * HD + d, a.kv_fp16);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * C; idx += WG) {
        const int h = idx / C, p = idx - h * C;
        float e = 0.f;
        if (p < cnt) {
            const int sidx = p0 + p;
            const float x = (a.scores[(int64_t)(kvh * G + h) * a.context + sidx] - gmax[h]);
            e = sidx < n8 ? exp_approx(x) : expf(x);
        }
        p_s[idx] = e;
    }
    __syncthreads();
    if (threadIdx.x < G) {
        float z = 0.f;
        for (int p = 0; p < cnt; p++) z += p_s[threadIdx.x * C + p];
        a.part_sum[(int64_t)c * a.heads + kvh * G + threadIdx.x] = z;
    }
    for (int idx = threadIdx.x; idx < G * HD; idx += WG) {
        const int h = idx / HD, d = idx - h * HD;
        float acc = 0.f;
        const float* pr = p_s + h * C;
        for (int p = 0; p < cnt; p++) acc += pr[p] * v_s[p * (HD + 1) + d];
        a.part_out[((int64_t)c * a.heads + kvh * G + h) * HD + d] = acc;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned prev = atomicAdd(a.counters + kvh, 1u);
        is_last = (prev == (unsigned)nch - 1u);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int idx = threadIdx.x; idx < G * HD; idx += WG) {
        const int h = idx / HD, d = idx - h * HD;
        const int hq = kvh * G + h;
        float acc = 0.f, z = 0.f;
        for (int i = 0; i < nch; i++) {
            acc += __builtin_nontemporal_load(a.part_out + ((int64_t)i * a.heads + hq) * HD + d);
            z += __builtin_nontemporal_load(a.part_sum + (int64_t)i * a.heads + hq);
        }
        a.out[(int64_t)hq * HD + d] = acc * (1.0f / z);
    }
    if (threadIdx.x == 0) a.counters[kvh] = 0u;
}

template <int HD>
hipError_t launch_hd(const AttnArgs& a, hipStream_t s) {
    const int G = a.heads / a.kv_heads;
    const int C = attn_chunk(a.heads, a.kv_heads);
    const int nchunks = attn_max_chunks(a.heads, a.kv_heads, a.context);
    dim3 grid(nchunks, a.kv_heads);
    size_t sm1 = sizeof(float) * (size_t)(G * HD + C * (HD + 1));
    size_t sm2 = sizeof(float) * (size_t)(C * (HD + 1) + G * C);
    attn_scores_kernel<HD><<<grid, WG, sm1, s>>>(a, C, G);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_pv_kernel<HD><<<grid, WG, sm2, s>>>(a, C, G);
    return hipGetLastError();
}

}  // namespace

int attn_chunk(int heads, int kv_heads) {
    const int G = heads / kv_heads;
    return G <= 4 ? 64 : WG / G;
}

int attn_max_chunks(int heads, int kv_heads, int context) {
    const int C = attn_chunk(heads, kv_heads);
    return (context + C - 1) / C;
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
    if (a.kv_heads <= 0 || a.heads % a.kv_heads != 0) return hipErrorInvalidValue;
    const int G = a.heads / a.kv_heads;
    if (G > 16) return hipErrorInvalidValue;
    const int C = attn_chunk(a.heads, a.kv_heads);
    if ((WG / (G * C)) < 1 || a.head_dim % (WG / (G * C)) != 0) return hipErrorInvalidValue;
    switch (a.head_dim) {
    case 64: return launch_hd<64>(a, s);
    case 96: return launch_hd<96>(a, s);
    case 128: return launch_hd<128>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmdot
