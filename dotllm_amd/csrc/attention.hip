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
// exponent.  The sequence is split into chunks per kv head (grid = chunks x
// kv heads; chunks past T exit), over three launches (each reads what the
// previous wrote, so no fences or atomics are needed):
//   scores:  64-position chunks: RoPE + KV write + scores + chunk max (per q head).
//            4 threads per position, each loading a quarter of the K row with
//            16-byte loads; every K row is read once for all G q heads.
//   pv:      64-position chunks: global max from the chunk maxima,
//            exponentials, partial sum(e) and sum(e V) (16-byte V loads).
//   combine: out = sum(eV) / sum(e) over the chunks, one q head per workgroup.
// Loads carry no branches (positions past T read a written row and are
// masked), so each thread's loads are all in flight together.
// cos/sin come from a host table built with the same libm calls as the
// reference, so RoPE is bit-exact.
#include "common.h"
#include "kernels.h"

namespace llmdot {

namespace {

constexpr int WG = 256;
constexpr int CH = 64;    // positions per score chunk (scores kernel; one per lane of a wavefront)
constexpr int CHP = 64;   // positions per pv chunk (pv kernel; its partials feed the combine)

// N consecutive cache elements starting at element idx (16-byte aligned) as floats.
template <int N>
__device__ __forceinline__ void load_kv_row(const void* cache, int64_t idx, int fp16, float* out) {
    if (fp16) {
        const _Float16* p = reinterpret_cast<const _Float16*>(cache) + idx;
        if constexpr (N % 8 == 0) {
#pragma unroll
            for (int i = 0; i < N / 8; i++) {
                const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    out[8 * i + 2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xFFFFu));
                    out[8 * i + 2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < N / 2; i++) {
                const uint32_t w = reinterpret_cast<const uint32_t*>(p)[i];
                out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
                out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
            }
        }
    } else {
        const float* p = reinterpret_cast<const float*>(cache) + idx;
        if constexpr (N % 4 == 0) {
#pragma unroll
            for (int i = 0; i < N / 4; i++) {
                const float4 v = reinterpret_cast<const float4*>(p)[i];
                out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; i++) out[i] = p[i];
        }
    }
}

template <int HD, int G>
__global__ __launch_bounds__(WG) void attn_scores_kernel(AttnArgs a) {
    __shared__ float q_s[G * HD];
    __shared__ float knew[HD];
    __shared__ float sc_s[G][CH];   // this chunk's scores (-inf past T) for the maxima
    constexpr int DPT = HD / 4;           // K elements per thread
    const int T = *a.pos, n = T + 1;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int p0 = c * CH;
    if (p0 >= n) return;
    const int half = a.rope_half;
    const float* cs = a.cos_tab + (int64_t)T * half;
    const float* sn = a.sin_tab + (int64_t)T * half;
    const int64_t cache_base = (int64_t)kvh * a.context * HD;

    // this thread's K quarter-row, issued first; positions past T read row p0
    // (always written) and are masked afterwards
    const int t = threadIdx.x, p = t >> 2, sub = t & 3;
    const int pos = p0 + p;
    const bool live = pos < n;
    const bool is_new = pos == T;
    float kv[DPT];
    load_kv_row<DPT>(a.kcache, cache_base + (int64_t)(live && !is_new ? pos : p0) * HD + sub * DPT, a.kv_fp16, kv);

    for (int idx = t; idx < G * HD; idx += WG) {
        const int h = idx / HD, d = idx - h * HD;
        q_s[idx] = rope_elem(a.q + (int64_t)(kvh * G + h) * HD, d, half, cs, sn);
    }
    if (T >= p0 && T < p0 + CH) {   // this workgroup owns the new token: store K/V slot T
        for (int d = t; d < HD; d += WG) {
            const int64_t slot = cache_base + (int64_t)T * HD + d;
            knew[d] = store_kv(a.kcache, slot, rope_elem(a.k + (int64_t)kvh * HD, d, half, cs, sn), a.kv_fp16);
            store_kv(a.vcache, slot, a.v[(int64_t)kvh * HD + d], a.kv_fp16);
        }
    }
    __syncthreads();
    if (is_new) {
#pragma unroll
        for (int d = 0; d < DPT; d++) kv[d] = knew[sub * DPT + d];
    }
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    const int lane = t & 63, wave = t >> 6;
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float* qv = q_s + h * HD + sub * DPT;
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < DPT; d++) s += qv[d] * kv[d];
        s = sum4(s);
        const float score = s * inv_sqrt;
        if (live && sub == 0) a.scores[(int64_t)(kvh * G + h) * a.context + pos] = score;
        if (sub == 0) sc_s[h][p] = live ? score : -INFINITY;
    }
    __syncthreads();
    for (int h = wave; h < G; h += 4) {   // one head per wavefront: its CH positions, one per lane
        const float m = wave_max(sc_s[h][lane]);
        if (lane == 0) a.chunk_max[(int64_t)(kvh * G + h) * gridDim.x + c] = m;
    }
}

template <int HD, int G>
__global__ __launch_bounds__(WG) void attn_pv_kernel(AttnArgs a) {
    constexpr int DPG = HD / 16;                  // V elements per thread and position
    constexpr int PPT = CHP / 16;                 // positions per thread
    constexpr int SPT = (G * CHP + WG - 1) / WG;  // scores per thread
    __shared__ float p_s[G][CHP];
    // partial sums of the 16 position groups: with several heads per kv head
    // through LDS (one padded row per group), for one head by lane exchanges
    // inside each wavefront first (measured faster for each case)
    constexpr int NGR = G > 1 ? 16 : 4;
    __shared__ float red[NGR][G * HD + 4];
    __shared__ float gmax[G];
    const int T = *a.pos, n = T + 1, n8 = n & ~7;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int p0 = c * CHP;
    if (p0 >= n) return;
    const int cnt = min(CHP, n - p0);
    const int nch = (n + CH - 1) / CH;            // score chunks (their maxima)
    const int cm_stride = (a.context + CH - 1) / CH;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int dg = t & 15, pg = t >> 4;
    const int64_t cache_base = (int64_t)kvh * a.context * HD;

    // Every global load is issued before any is used: the V rows of positions
    // pg + 16 i (rows past T read row p0), this chunk's scores, and the chunk
    // maxima of this wavefront's heads.
    float vv[PPT][DPG];
#pragma unroll
    for (int i = 0; i < PPT; i++) {
        const int p = pg + 16 * i;
        load_kv_row<DPG>(a.vcache, cache_base + (int64_t)(p0 + (p < cnt ? p : 0)) * HD + dg * DPG, a.kv_fp16, vv[i]);
    }
    float sc[SPT];
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int idx = min(t + k * WG, G * CHP - 1);
        const int h = idx / CHP, p = idx - h * CHP;
        sc[k] = a.scores[(int64_t)(kvh * G + h) * a.context + p0 + (p < cnt ? p : 0)];
    }
    constexpr int HPW = (G + 3) / 4;              // heads per wavefront for the global max
    float cm[HPW][2];
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        const int h = min(wave + 4 * j, G - 1);
        const float* row = a.chunk_max + (int64_t)(kvh * G + h) * cm_stride;
        cm[j][0] = row[min(lane, nch - 1)];       // repeats of entry nch-1 do not change the max
        cm[j][1] = row[min(lane + 64, nch - 1)];
    }
    // global max of each head's scores (Softmax's max over all n)
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        const int h = wave + 4 * j;
        float m = fmaxf(cm[j][0], cm[j][1]);
        for (int i = lane + 128; i < nch; i += 64) m = fmaxf(m, a.chunk_max[(int64_t)(kvh * G + min(h, G - 1)) * cm_stride + i]);
        m = wave_max(m);
        if (h < G && lane == 0) gmax[h] = m;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int idx = t + k * WG;
        if (idx < G * CHP) {
            const int h = idx / CHP, p = idx - h * CHP;
            const int sidx = p0 + p;
            float e;
            {
#pragma clang fp contract(off)
                const float x = sc[k] - gmax[h];
                // Softmax: ExpApprox on the vector lanes (first 8*floor(n/8)), expf on the tail
                e = sidx < n8 ? exp_approx(x) : expf(x);
            }
            p_s[h][p] = p < cnt ? e : 0.f;
        }
    }
    __syncthreads();
    for (int h = wave; h < G; h += 4) {   // this chunk's sum of exponentials
        float z = 0.f;
#pragma unroll
        for (int k = 0; k < CHP / 64; k++) z += p_s[h][lane + 64 * k];
        z = wave_sum(z);
        if (lane == 0) a.part_sum[(int64_t)c * a.heads + kvh * G + h] = z;
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
        float acc[DPG];
#pragma unroll
        for (int d = 0; d < DPG; d++) acc[d] = 0.f;
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const float pr = p_s[h][pg + 16 * i];
#pragma unroll
            for (int d = 0; d < DPG; d++) acc[d] += pr * vv[i][d];
        }
#pragma unroll
        for (int d = 0; d < DPG; d++) {
            if constexpr (G > 1) {
                red[pg][h * HD + dg * DPG + d] = acc[d];
            } else {
                const float v = xor32_add(xor16_add(acc[d]));
                if (lane < 16) red[wave][h * HD + dg * DPG + d] = v;
            }
        }
    }
    __syncthreads();
    for (int idx = t; idx < G * HD; idx += WG) {
        const int h = idx / HD, d = idx - h * HD;
        float r = 0.f;
#pragma unroll
        for (int q = 0; q < NGR; q += 4) r += (red[q][idx] + red[q + 1][idx]) + (red[q + 2][idx] + red[q + 3][idx]);
        a.part_out[((int64_t)c * a.heads + kvh * G + h) * HD + d] = r;
    }
}

// out = sum_c part_out[c] / sum_c part_sum[c] for one q head per workgroup
// (a separate launch: the chunk partials are visible without fences).  NG
// groups of HD threads each take every NG-th chunk; the group sums are then
// added in group order.
template <int HD>
__global__ __launch_bounds__(1024) void attn_combine_kernel(AttnArgs a) {
    constexpr int NG = 1024 / HD;
    __shared__ float acc_s[NG][HD];
    __shared__ float z_s[NG];
    const int n = *a.pos + 1;
    const int nch = (n + CHP - 1) / CHP;
    const int hq = blockIdx.x, g = threadIdx.x / HD, d = threadIdx.x - g * HD;
    float acc = 0.f, z = 0.f;
#pragma unroll 4
    for (int i = g; i < nch; i += NG) {
        acc += a.part_out[((int64_t)i * a.heads + hq) * HD + d];
        z += a.part_sum[(int64_t)i * a.heads + hq];
    }
    acc_s[g][d] = acc;
    if (d == 0) z_s[g] = z;
    __syncthreads();
    if (g == 0) {
        float at = 0.f, zt = 0.f;
#pragma unroll
        for (int k = 0; k < NG; k++) {
            at += acc_s[k][d];
            zt += z_s[k];
        }
        a.out[(int64_t)hq * HD + d] = at * (1.0f / zt);
    }
}

template <int HD, int G>
hipError_t launch_hg(const AttnArgs& a, hipStream_t s) {
    const int nchunks = attn_max_chunks(a.heads, a.kv_heads, a.context);
    attn_scores_kernel<HD, G><<<dim3(nchunks, a.kv_heads), WG, 0, s>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_pv_kernel<HD, G><<<dim3((a.context + CHP - 1) / CHP, a.kv_heads), WG, 0, s>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_combine_kernel<HD><<<a.heads, (1024 / HD) * HD, 0, s>>>(a);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const AttnArgs& a, hipStream_t s) {
    switch (a.heads / a.kv_heads) {
    case 1: return launch_hg<HD, 1>(a, s);
    case 2: return launch_hg<HD, 2>(a, s);
    case 4: return launch_hg<HD, 4>(a, s);
    case 8: return launch_hg<HD, 8>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int attn_max_chunks(int heads, int kv_heads, int context) {
    (void)heads; (void)kv_heads;
    return (context + CH - 1) / CH;
}

bool attn_supported(int heads, int kv_heads, int head_dim) {
    if (kv_heads <= 0 || heads % kv_heads != 0) return false;
    const int g = heads / kv_heads;
    return (g == 1 || g == 2 || g == 4 || g == 8) && (head_dim == 64 || head_dim == 96 || head_dim == 128);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
    if (!attn_supported(a.heads, a.kv_heads, a.head_dim)) return hipErrorInvalidValue;
    switch (a.head_dim) {
    case 64: return launch_hd<64>(a, s);
    case 96: return launch_hd<96>(a, s);
    case 128: return launch_hd<128>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmdot
