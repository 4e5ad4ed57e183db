// sample.hip -- Sampler.Sample (src/Llmdot.Core/Sampling/Sampler.cs:24-170) on
// the device, for a logits vector already in HBM.
//
//   scale:    work = logits * (1f / Temperature)            (Sampler.cs:30-34)
//   penalty:  the last RepeatPenaltyWindowSize history tokens, applied once per
//             occurrence: x > 0 ? x / p : x * p, then the same scale
//             (ApplyRepeatPenalty, Sampler.cs:64-81)
//   top-k:    (0 < TopK < n, Sampler.cs:36-42) one workgroup: radix select of
//             the k-th largest value, the k winners gathered in index order and
//             sorted by (value desc, index asc), VectorMath.Softmax over them in
//             the reference's summation order, then the sequential draw
//             (SampleFromProbabilities, Sampler.cs:158-170)
//   softmax:  (otherwise) VectorMath.Softmax over all n (same maximum and
//             exponentials; the sum is a workgroup reduction)
//   top-p:    (TopP < 1, Sampler.cs:44-59, FindNucleus 129-156) the nucleus
//             boundary and the draw inside it located by radix descent over
//             the probabilities with fp64 mass sums, so no full sort is needed;
//             without a proper nucleus the draw walks the probabilities in index
//             order (Sampler.cs:61).
//
// The uniform draw r (Random.NextSingle() in the reference, Sampler.cs:160-161)
// is an input, read from rvals[step - 1], so the caller owns the generator.
// Exact ties between values are resolved toward the smaller index.
#include "common.h"
#include "kernels.h"

namespace llmdot {

namespace {

constexpr int SWG = 1024;          // the single-workgroup kernels
constexpr int NWAVE = SWG / 64;

// Order-preserving 32-bit key of a float (larger float, larger key) and back.
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float keyf(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Exclusive prefix sum over the workgroup in thread order; *total gets the sum.
template <typename V>
__device__ V block_excl_scan(V v, V* tmp, V* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    V incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const V u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
    }
    if (lane == 63) tmp[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        V w = lane < NWAVE ? tmp[lane] : V(0);
        V wi = w;
#pragma unroll
        for (int o = 1; o < NWAVE; o <<= 1) {
            const V u = __shfl_up(wi, o, 64);
            if (lane >= o) wi += u;
        }
        if (lane < NWAVE) tmp[NWAVE + lane] = wi - w;   // exclusive offset of each wavefront
        if (lane == NWAVE - 1) tmp[2 * NWAVE] = wi;
    }
    __syncthreads();
    const V r = tmp[NWAVE + wave] + incl - v;
    *total = tmp[2 * NWAVE];
    __syncthreads();
    return r;
}

struct Descent {
    uint32_t key;     // key of the element reached
    double above;     // weight of all elements with a larger key
    int cnt_above;    // how many there are
    int n_eq;         // elements with this key
};

// Radix descent over keys (largest first): the element at which the running
// weight, in (key desc, index asc) order, first reaches T.  MASS: weight = the
// value (non-negative); otherwise weight = 1 per element (a rank).  With T
// beyond the total the last element is reached.  Workgroup-uniform result.
template <bool MASS>
__device__ Descent descend(const float* x, int n, double T) {
    __shared__ int cnt[256];
    __shared__ double wsum[256];
    __shared__ uint32_t s_digit;
    __shared__ double s_above;
    __shared__ int s_cabove, s_neq;
    const int t = threadIdx.x, lane = t & 63;
    uint32_t prefix = 0, mask = 0;
    double above = 0.0;
    int cabove = 0, neq = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = t; i < 256; i += SWG) { cnt[i] = 0; wsum[i] = 0.0; }
        __syncthreads();
        for (int i = t; i < n; i += SWG) {
            const float v = x[i];
            const uint32_t k = fkey(v);
            if ((k & mask) == prefix) {
                const int d = (k >> shift) & 255;
                atomicAdd(&cnt[d], 1);
                if (MASS) atomicAdd(&wsum[d], (double)v);
            }
        }
        __syncthreads();
        if (t < 64) {
            // lane l holds digits 255 - 4l .. 252 - 4l (descending)
            int c[4];
            double w[4], lw = 0.0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int d = 255 - 4 * lane - q;
                c[q] = cnt[d];
                w[q] = MASS ? wsum[d] : (double)c[q];
                lw += w[q];
            }
            double incl = lw;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const double u = __shfl_up(incl, o, 64);
                if (lane >= o) incl += u;
            }
            double run = above + (incl - lw);
            int crun = 0;
            int hit = -1;
            double hit_above = 0.0;
            int hit_c = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (hit < 0 && c[q] > 0 && run + w[q] >= T) { hit = q; hit_above = run; hit_c = crun; }
                run += w[q];
                crun += c[q];
            }
            // counts above this lane's digits
            int ci = crun;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(ci, o, 64);
                if (lane >= o) ci += u;
            }
            const int cexcl = ci - crun;
            const uint64_t found = __ballot(hit >= 0);
            // nonempty digits, for the case T lies beyond the total
            int last_q = -1;
#pragma unroll
            for (int q = 0; q < 4; q++) if (c[q] > 0) last_q = q;
            const uint64_t nonempty = __ballot(last_q >= 0);
            int src;
            if (found) src = __ffsll((unsigned long long)found) - 1;
            else src = 63 - __clzll((long long)nonempty);
            if (lane == src) {
                int q = hit;
                double ab = hit_above;
                int cb = hit_c;
                if (!found) {   // the last nonempty digit, with everything before it above
                    q = last_q;
                    ab = above + (incl - lw);
                    cb = 0;
                    for (int j = 0; j < q; j++) { ab += w[j]; cb += c[j]; }
                }
                s_digit = (uint32_t)(255 - 4 * lane - q);
                s_above = ab;
                s_cabove = cabove + cexcl + cb;
                s_neq = c[q];
            }
        }
        __syncthreads();
        prefix |= s_digit << shift;
        mask |= 255u << shift;
        above = s_above;
        cabove = s_cabove;
        neq = s_neq;
        __syncthreads();
    }
    return Descent{prefix, above, cabove, neq};
}

// Index of the j-th (1-based) element whose key is K, in index order.
__device__ int jth_equal(const float* x, int n, uint32_t K, int j) {
    __shared__ int tmp[2 * NWAVE + 1];
    __shared__ int s_idx;
    const int seg = (n + SWG - 1) / SWG;
    const int b = threadIdx.x * seg, e = min(n, b + seg);
    int c = 0;
    for (int i = b; i < e; i++) c += fkey(x[i]) == K;
    if (threadIdx.x == 0) s_idx = -1;
    int total;
    const int off = block_excl_scan<int>(c, tmp, &total);
    if (off < j && j <= off + c) {
        int r = off;
        for (int i = b; i < e; i++)
            if (fkey(x[i]) == K && ++r == j) { s_idx = i; break; }
    }
    __syncthreads();
    return s_idx;
}

__global__ void samp_scale_kernel(const float* logits, float inv_temp, float* work, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) work[i] = logits[i] * inv_temp;
}

// ApplyRepeatPenalty (Sampler.cs:64-81) on the last `window` history tokens,
// then the temperature scale of those entries.
__global__ void samp_penalty_kernel(SampleArgs a) {
    const int L = a.hist_base + *a.step - 1;   // tokens before this draw
    const int w0 = max(0, L - a.window);
    for (int j = w0 + (int)threadIdx.x; j < L; j += blockDim.x) {
        const int tok = a.hist[j];
        if (tok < 0 || tok >= a.n) continue;
        bool first = true;
        for (int i = w0; i < j; i++)
            if (a.hist[i] == tok) { first = false; break; }
        if (!first) continue;
        int c = 0;
        for (int i = j; i < L; i++) c += a.hist[i] == tok;
        float x = a.logits[tok];
        for (int i = 0; i < c; i++) x = x > 0.f ? x / a.penalty : x * a.penalty;
        a.work[tok] = x * a.inv_temp;
    }
}

__device__ void publish(const SampleArgs& a, int token) {
    const int s = *a.step - 1;
    *a.token_out = token;
    if (a.token_log && s >= 0 && s < a.log_cap) a.token_log[s] = token;
    if (a.hist_out) a.hist_out[a.hist_base + s] = token;
}

// Top-k path: select, gather in index order, sort, softmax, draw.
__global__ __launch_bounds__(SWG) void samp_topk_kernel(SampleArgs a) {
    __shared__ uint64_t cand[SAMPLE_MAX_K];
    __shared__ float pv[SAMPLE_MAX_K];
    __shared__ int tmp[2 * NWAVE + 1];
    __shared__ float s_part[8];
    __shared__ int s_pick;
    const int n = a.n, k = a.top_k, t = threadIdx.x;
    const Descent D = descend<false>(a.work, n, (double)k);
    const uint32_t K = D.key;
    const int need_eq = k - D.cnt_above;   // elements equal to the k-th value that are kept

    // stable gather: thread t walks [t * seg, ...) twice
    const int seg = (n + SWG - 1) / SWG;
    const int b = t * seg, e = min(n, b + seg);
    int ng = 0, ne = 0;
    for (int i = b; i < e; i++) {
        const uint32_t kk = fkey(a.work[i]);
        ng += kk > K;
        ne += kk == K;
    }
    int tot;
    const int eq_off = block_excl_scan<int>(ne, tmp, &tot);
    const int keep_eq = max(0, min(ne, need_eq - eq_off));
    const int out_off = block_excl_scan<int>(ng + keep_eq, tmp, &tot);
    {
        int o = out_off, r = 0;
        for (int i = b; i < e; i++) {
            const uint32_t kk = fkey(a.work[i]);
            const bool take = kk > K || (kk == K && r++ < keep_eq);
            if (take && o < SAMPLE_MAX_K) cand[o++] = ((uint64_t)kk << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
        }
    }
    int P = 1;
    while (P < k) P <<= 1;
    for (int i = k + t; i < P; i += SWG) cand[i] = 0;
    __syncthreads();
    // bitonic sort, descending
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < P / 2; i += SWG) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = cand[lo], y = cand[hi];
                if ((x < y) == desc) { cand[lo] = y; cand[hi] = x; }
            }
            __syncthreads();
        }
    }
    // VectorMath.Softmax over the k sorted values (VM:215-258): max, exponentials,
    // eight interleaved partial sums, their horizontal sum, then the tail
    const float M = keyf((uint32_t)(cand[0] >> 32));
    const int k8 = k & ~7;
    if (t < 8) {
        float vs = 0.f;
        for (int j = t; j < k8; j += 8) {
            float ev;
            {
#pragma clang fp contract(off)
                ev = exp_approx(keyf((uint32_t)(cand[j] >> 32)) - M);
            }
            pv[j] = ev;
            vs += ev;
        }
        s_part[t] = vs;
    }
    __syncthreads();
    if (t == 0) {
        float sum = ((s_part[0] + s_part[1]) + (s_part[2] + s_part[3])) + ((s_part[4] + s_part[5]) + (s_part[6] + s_part[7]));
        for (int j = k8; j < k; j++) {
            float ev;
            {
#pragma clang fp contract(off)
                ev = expf(keyf((uint32_t)(cand[j] >> 32)) - M);
            }
            pv[j] = ev;
            sum += ev;
        }
        const float inv = 1.0f / sum;
        const float r = a.rvals[*a.step - 1];
        float cum = 0.f;
        int pick = k - 1;
        for (int j = 0; j < k; j++) {
#pragma clang fp contract(off)
            const float pj = pv[j] * inv;   // Scale(input, invSum), then the running sum
            cum += pj;
            if (r <= cum) { pick = j; break; }
        }
        s_pick = (int)(0xFFFFFFFFu - (uint32_t)(cand[pick] & 0xFFFFFFFFu));
    }
    __syncthreads();
    if (t == 0) publish(a, s_pick);
}

// VectorMath.Softmax over all n in place (VM:215-258): the same max and
// exponentials (ExpApprox on the first 8 floor(n/8), expf on the tail); the sum
// is a workgroup reduction, so it (and the probabilities) may differ from the
// reference's interleaved sequential sum in the last bits.
__global__ __launch_bounds__(SWG) void samp_softmax_kernel(SampleArgs a) {
    __shared__ float red[NWAVE];
    __shared__ float s_inv;
    const int n = a.n, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float* x = a.work;
    // FindMax (VM:260-284) returns the maximum value whatever the order
    float m = -INFINITY;
    for (int i = t; i < n; i += SWG) m = fmaxf(m, x[i]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < NWAVE; w++) m = fmaxf(m, red[w]);
    const int n8 = n & ~7;
    float sum = 0.f;
    for (int i = t; i < n; i += SWG) {
        float ev;
        {
#pragma clang fp contract(off)
            const float d = x[i] - m;
            ev = i < n8 ? exp_approx(d) : expf(d);
        }
        x[i] = ev;
        sum += ev;
    }
    sum = wave_sum(sum);
    __syncthreads();
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    if (t == 0) {
        float z = 0.f;
        for (int w = 0; w < NWAVE; w++) z += red[w];
        s_inv = 1.0f / z;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = t; i < n; i += SWG) x[i] = x[i] * inv;
}

// Top-p nucleus and the draw (Sampler.cs:44-61) over the probabilities in work.
__global__ __launch_bounds__(SWG) void samp_nucleus_kernel(SampleArgs a) {
    __shared__ double dtmp[2 * NWAVE + 1];
    __shared__ int s_pick;
    const int n = a.n, t = threadIdx.x;
    const float* p = a.work;
    const double r = (double)a.rvals[*a.step - 1];
    bool nucleus = false;
    Descent D1{};
    int j1 = 0, m = n;
    if (a.top_p < 1.f) {
        // FindNucleus: the shortest prefix, by descending probability, whose sum reaches TopP
        const double T1 = (double)a.top_p;
        D1 = descend<true>(p, n, T1);
        const double w1 = (double)keyf(D1.key);
        j1 = D1.n_eq;
        if (w1 > 0.0) {
            const double need = ceil((T1 - D1.above) / w1);
            j1 = (int)fmin(fmax(need, 1.0), (double)D1.n_eq);
        }
        m = D1.cnt_above + j1;
        nucleus = m < n;
    }
    if (nucleus) {
        // renormalised draw inside the nucleus: the element at which the
        // running sum first reaches r * (nucleus sum)
        const double S = D1.above + (double)j1 * (double)keyf(D1.key);
        const Descent D2 = descend<true>(p, n, r * S);
        uint32_t K = D2.key;
        int j = D2.n_eq;
        const double w2 = (double)keyf(D2.key);
        if (w2 > 0.0) j = (int)fmin(fmax(ceil((r * S - D2.above) / w2), 1.0), (double)D2.n_eq);
        if (D2.cnt_above + j > m) {   // past the nucleus (rounding): its last element
            K = D1.key;
            j = j1;
        }
        const int idx = jth_equal(p, n, K, j);
        if (t == 0) s_pick = idx;
    } else {
        // SampleFromProbabilities over all n in index order
        const int seg = (n + SWG - 1) / SWG;
        const int b = t * seg, e = min(n, b + seg);
        double sum = 0.0;
        for (int i = b; i < e; i++) sum += (double)p[i];
        double total;
        const double off = block_excl_scan<double>(sum, dtmp, &total);
        if (t == 0) s_pick = n - 1;
        __syncthreads();
        if (off < r && r <= off + sum) {
            double c = off;
            for (int i = b; i < e; i++) {
                c += (double)p[i];
                if (r <= c) { s_pick = i; break; }
            }
        } else if (t == 0 && r <= 0.0) {
            s_pick = 0;
        }
    }
    __syncthreads();
    if (t == 0) publish(a, s_pick < 0 ? n - 1 : s_pick);
}

}  // namespace

bool sample_supported(int n, int top_k) { return n > 0 && !(top_k > SAMPLE_MAX_K && top_k < n); }

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
    if (!sample_supported(a.n, a.top_k) || a.inv_temp <= 0.f) return hipErrorInvalidValue;
    int g = (a.n + 255) / 256;
    samp_scale_kernel<<<g > 1024 ? 1024 : g, 256, 0, s>>>(a.logits, a.inv_temp, a.work, a.n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.penalty != 1.f && a.window > 0 && a.hist) {
        samp_penalty_kernel<<<1, 256, 0, s>>>(a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (a.top_k > 0 && a.top_k < a.n) {
        samp_topk_kernel<<<1, SWG, 0, s>>>(a);
        return hipGetLastError();
    }
    samp_softmax_kernel<<<1, SWG, 0, s>>>(a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    samp_nucleus_kernel<<<1, SWG, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace llmdot
