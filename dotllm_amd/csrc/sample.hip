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
//   softmax:  (otherwise) VectorMath.Softmax over all n in the reference's
//             summation order: the probabilities bit for bit
//   top-p:    (TopP < 1, Sampler.cs:44-61, FindNucleus 129-156) the reference
//             as written: its selection-sort order (ties included), the values
//             it writes into the buffer it still reads from, the sequential
//             float running sum that closes the nucleus, the renormalised draw,
//             and the fall-through draw over the rewritten buffer that returns
//             a rank; candidates located by fp64 radix descent, so a full sort
//             runs only when they do not suffice
//   no top-p: the draw over the probabilities in index order (Sampler.cs:61),
//             placed with fp64 running sums
//
// The uniform draw r (Random.NextSingle() in the reference, Sampler.cs:160-161)
// is an input, read from rvals[step - 1], so the caller owns the generator.
// In the top-k path exact ties between values are resolved toward the smaller
// index.
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

// VectorMath.Softmax over all n in place (VM:215-258) in the reference's
// order: the maximum (FindMax, VM:260-284: the same value whatever the order),
// the exponentials (ExpApprox on the first 8 floor(n/8), expf on the tail),
// eight lane sums (lane l adds elements l, l + 8, ... in order), their
// horizontal sum ((l0 + l1) + (l2 + l3)) + ((l4 + l5) + (l6 + l7)), the tail
// added in order, then each probability times 1f / sum -- bit for bit the
// reference's probabilities.
__global__ __launch_bounds__(SWG) void samp_softmax_kernel(SampleArgs a) {
    __shared__ float red[NWAVE];
    __shared__ float s_lane[8];
    __shared__ float s_inv;
    const int n = a.n, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float* x = a.work;
    float m = -INFINITY;
    for (int i = t; i < n; i += SWG) m = fmaxf(m, x[i]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < NWAVE; w++) m = fmaxf(m, red[w]);
    const int n8 = n & ~7;
    for (int i = t; i < n; i += SWG) {
        float ev;
        {
#pragma clang fp contract(off)
            const float d = x[i] - m;
            ev = i < n8 ? exp_approx(d) : expf(d);
        }
        x[i] = ev;
    }
    __syncthreads();
    if (t < 8) {
        // lane t's running sum; the loads run ahead of the dependent adds
        float acc = 0.f;
        int j = t;
        for (; j + 8 * 15 < n8; j += 8 * 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = x[j + 8 * u];
#pragma unroll
            for (int u = 0; u < 16; u++) acc += v[u];
        }
        for (; j < n8; j += 8) acc += x[j];
        s_lane[t] = acc;
    }
    __syncthreads();
    if (t == 0) {
        float z = ((s_lane[0] + s_lane[1]) + (s_lane[2] + s_lane[3])) + ((s_lane[4] + s_lane[5]) + (s_lane[6] + s_lane[7]));
        for (int j = n8; j < n; j++) z += x[j];
        s_inv = 1.0f / z;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = t; i < n; i += SWG) x[i] = x[i] * inv;
}

// ---- top-p: FindNucleus (Sampler.cs:129-156) with the reference's buffers ----
//
// The reference sorts token ids by probability with a selection sort (strict
// `>`, so among equal values the first in the array's current order wins) and
// then writes values[i] = probabilities[indices[i]] into the same buffer the
// probabilities live in (Sampler.cs:30, 48-50): a rank i whose id indices[i]
// is below i reads the value rank indices[i] already wrote.  Following
// a = indices[a] while indices[a] < a therefore gives rank i's value,
// p[indices[a]] (each link lowers a, so the chain ends).  The running float sum
// of those values, in rank order, closes the nucleus; when it never reaches
// TopP the fall-through draw walks the rewritten buffer and returns a rank.
//
// Selection order: distinct values leave in descending order.  Equal values
// leave together, in the order of the array positions they hold when the
// first of them is selected; positions change only by the sort's swaps: at
// step s the selected element's old position src[s] receives the element that
// stood at s.  An element e still unselected at step s therefore stands at the
// end of e, src[e], src[src[e]], ... (followed while below s), and the members
// of a run of equal values keep their positions while the run is selected.
//
// Candidates: every element down to the value at which the fp64 mass reaches
// TopP + 1e-4 (whole runs of equal values).  The aliased values are at least
// the true ones and float addition is monotonic, so the aliased running sum
// reaches TopP no later than the true one; if it still has not within the
// candidates the kernel repeats the work over all n (global scratch).

constexpr int NUC_LDS = 4096;   // candidates sorted in LDS (fast path)

// Ascending bitonic sort of a[0, P) (P a power of two) by the whole workgroup.
__device__ void bitonic_asc(uint64_t* a, int P, bool global) {
    const int t = threadIdx.x;
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < P / 2; i += SWG) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t x = a[lo], y = a[hi];
                if ((x > y) == up) { a[lo] = y; a[hi] = x; }
            }
            if (global) __threadfence();
            __syncthreads();
        }
    }
}

// Position at step s of element e (unselected before s).
__device__ __forceinline__ int position_at(const int* src, int e, int s) {
    int q = e;
    while (q < s) q = src[q];
    return q;
}

// The selection-sort order of K candidates whose (~key, id) pairs are sorted
// ascending in comp[0, K): ids[r] = the id selected at step r.  Positions
// (src[r] = where the element selected at step r stood then) are computed up
// to the end of the last run of equal values, the only steps whose order
// depends on positions; comp[K, 3K) is the scratch of the runs' sorts.
__device__ void selection_order(uint64_t* comp, int K, int* ids, int* src, bool global) {
    __shared__ int s_last, s_i, s_i1;
    const int t = threadIdx.x;
    if (t == 0) { s_last = 0; s_i = 0; }
    __syncthreads();
    for (int i = t; i < K; i += SWG) {
        ids[i] = (int)(uint32_t)comp[i];
        if (i + 1 < K && (comp[i] >> 32) == (comp[i + 1] >> 32)) atomicMax(&s_last, i + 2);
    }
    if (global) __threadfence();
    __syncthreads();
    const int R = s_last;   // ranks [0, R) need positions; [R, K) follow the value order
    uint64_t* tmp = comp + K;
    while (R > 0) {
        if (t == 0) {
            // singleton steps in order, up to the next run of equal values
            int i = s_i, i1 = i;
            while (i < R) {
                i1 = i + 1;
                const uint64_t k = comp[i] >> 32;
                while (i1 < K && (comp[i1] >> 32) == k) i1++;
                if (i1 - i > 1) break;
                src[i] = position_at(src, ids[i], i);
                i++;
            }
            s_i = i;
            s_i1 = i1;
        }
        if (global) __threadfence();
        __syncthreads();
        const int i = s_i, i1 = s_i1;
        if (i >= R) break;
        // the run [i, i1): members leave in the order of their positions at step i
        const int g = i1 - i;
        int P = 1;
        while (P < g) P <<= 1;
        for (int j = t; j < P; j += SWG) {
            uint64_t v = ~0ull;
            if (j < g) {
                const int e = ids[i + j];
                v = ((uint64_t)(uint32_t)position_at(src, e, i) << 32) | (uint32_t)e;
            }
            tmp[j] = v;
        }
        if (global) __threadfence();
        __syncthreads();
        bitonic_asc(tmp, P, global);
        for (int j = t; j < g; j += SWG) {
            ids[i + j] = (int)(uint32_t)tmp[j];
            src[i + j] = (int)(tmp[j] >> 32);
        }
        if (global) __threadfence();
        __syncthreads();
        if (t == 0) s_i = i1;
        __syncthreads();
    }
    __syncthreads();
}

// Rank r's value as the reference writes it (the aliased chain), for r < K.
__device__ __forceinline__ float aliased_value(const float* p, const int* ids, int r) {
    int a = r;
    while (ids[a] < a) a = ids[a];
    return p[ids[a]];
}

// FindNucleus over K candidates (comp: (~key, id) pairs sorted in [0, K), 3K
// slots; ids, val: K each), then the draw.  Returns the token (or the rank, when the nucleus spans
// all n), or -1 when the running sum does not reach TopP within K < n.
__device__ int nucleus_draw(const float* p, int n, uint64_t* comp, int K, int* ids, float* val, float top_p, float r,
                            bool global) {
    __shared__ int s_res;
    const int t = threadIdx.x;
    int* src = reinterpret_cast<int*>(val);   // positions first, values after
    selection_order(comp, K, ids, src, global);
    for (int i = t; i < K; i += SWG) val[i] = aliased_value(p, ids, i);
    if (global) __threadfence();
    __syncthreads();
    if (t == 0) {
        // FindNucleus's running sum (Sampler.cs:146-154)
        float cum = 0.f;
        int count = -1;
        for (int i = 0; i < K; i++) {
            cum += val[i];
            if (cum >= top_p) { count = i + 1; break; }
        }
        if (count < 0 && K == n) count = n;
        int res = -1;
        if (count > 0 && count < n) {
            // Sampler.cs:51-57: sum, Scale(1f / sum), the draw over the nucleus
            float sum = 0.f;
            for (int i = 0; i < count; i++) sum += val[i];
            const float f = 1.0f / sum;
            float c2 = 0.f;
            int pick = count - 1;
            for (int i = 0; i < count; i++) {
#pragma clang fp contract(off)
                c2 += val[i] * f;
                if (r <= c2) { pick = i; break; }
            }
            res = ids[pick];
        } else if (count == n) {
            // Sampler.cs:61 over the rewritten buffer: a rank is returned
            float c = 0.f;
            res = n - 1;
            for (int i = 0; i < n; i++) {
                c += val[i];
                if (r <= c) { res = i; break; }
            }
        }
        s_res = res;
    }
    __syncthreads();
    return s_res;
}

// Top-p nucleus and the draw (Sampler.cs:44-61) over the probabilities in
// work[0, n); the rest of work is the slow path's scratch (sample_work_floats).
__global__ __launch_bounds__(SWG) void samp_nucleus_kernel(SampleArgs a) {
    __shared__ double dtmp[2 * NWAVE + 1];
    __shared__ int s_pick, s_cnt;
    __shared__ uint64_t l_comp[3 * NUC_LDS];
    __shared__ int l_ids[NUC_LDS];
    __shared__ float l_val[NUC_LDS];
    const int n = a.n, t = threadIdx.x;
    const float* p = a.work;
    const float rf = a.rvals[*a.step - 1];
    if (a.top_p < 1.f) {
        // candidates: every element at or above the value where the fp64 mass reaches TopP + 1e-4
        const Descent D = descend<true>(p, n, (double)a.top_p + 1e-4);
        const int K = D.cnt_above + D.n_eq;
        int res = -1;
        if (K <= NUC_LDS) {
            if (t == 0) s_cnt = 0;
            __syncthreads();
            for (int i = t; i < n; i += SWG) {
                const uint32_t k = fkey(p[i]);
                if (k >= D.key) {
                    const int o = atomicAdd(&s_cnt, 1);
                    if (o < NUC_LDS) l_comp[o] = ((uint64_t)(~k) << 32) | (uint32_t)i;
                }
            }
            int P = 1;
            while (P < K) P <<= 1;
            __syncthreads();
            for (int i = K + t; i < P; i += SWG) l_comp[i] = ~0ull;
            __syncthreads();
            bitonic_asc(l_comp, P, false);
            res = nucleus_draw(p, n, l_comp, K, l_ids, l_val, a.top_p, rf, false);
        }
        if (res < 0) {
            // all n in global scratch
            int P = 1;
            while (P < n) P <<= 1;
            uint64_t* comp = reinterpret_cast<uint64_t*>(a.work + sample_comp_offset(n));
            int* ids = reinterpret_cast<int*>(a.work + sample_comp_offset(n) + 6 * (size_t)n);
            float* val = a.work + sample_comp_offset(n) + 7 * (size_t)n;
            for (int i = t; i < P; i += SWG)
                comp[i] = i < n ? ((uint64_t)(~fkey(p[i])) << 32) | (uint32_t)i : ~0ull;
            __threadfence();
            __syncthreads();
            bitonic_asc(comp, P, true);
            res = nucleus_draw(p, n, comp, n, ids, val, a.top_p, rf, true);
        }
        if (t == 0) publish(a, res < 0 ? n - 1 : res);
        return;
    }
    // SampleFromProbabilities over all n in index order (Sampler.cs:61)
    const double r = (double)rf;
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
