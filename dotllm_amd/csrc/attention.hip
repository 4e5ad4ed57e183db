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
// exponent.  The sequence is split into 64-position chunks per kv head (grid
// = chunks x kv heads; chunks past T exit).  Up to 16384 positions the
// scores and the values run in one launch (attn_fused_kernel: the workgroups
// of a kv head exchange their chunk maxima through tagged slots).  Where the
// kv heads are a multiple of 8 and a kv head's chunks fit one XCD, they all
// run on one XCD, exchange through its L2 and also sum their partials inside
// the launch; otherwise the exchange goes through the coherence point and the
// combine launch follows.  Beyond 16384 positions, or with
// LLMDOT_HIP_ATTN_FUSED=0, three launches (each reads what the previous
// wrote, so no fences or atomics are needed):
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
constexpr int XSTRIDE = 512;   // tagged chunk-maximum slots per q head (4 KiB apart)

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

// N consecutive cache elements of a row as raw dwords (fp16 pairs or fp32),
// loaded with no branch on the element type so that every load of a thread
// is issued before the first one is waited on; converted at use.
template <int N, bool F16>
struct KvRaw {
    static constexpr int W = F16 ? N / 2 : N;   // dwords
    static constexpr bool V4 = W % 4 == 0 && (N * (F16 ? 2 : 4)) % 16 == 0;
    uint32_t w[W];
    __device__ __forceinline__ void load(const void* cache, int64_t idx) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(cache) +
                                                              idx * (F16 ? 2 : 4));
        if constexpr (V4) {
#pragma unroll
            for (int i = 0; i < W / 4; i++) {
                const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
                w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < W; i++) w[i] = p[i];
        }
    }
    __device__ __forceinline__ float at(int e) const {
        if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
        else return __uint_as_float(w[e]);
    }
};

// Tagged slot: (tag << 32) | float bits, stored and loaded at system scope so
// that the access goes past the per-XCD L2s (which are not coherent with each
// other) and a reader sees either an older tag or the whole new pair.
__device__ __forceinline__ void slot_put(uint64_t* p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t slot_get(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// One poll of the tagged chunk maxima of the G heads of kv head kvh: four
// slots per lane and head.
template <int G>
__device__ __forceinline__ void poll_issue(uint64_t (&v)[G][4], const uint64_t* xmax, int kvh, int lane, int c0,
                                           int nch, int mc) {
#pragma unroll
    for (int j = 0; j < G; j++) {
        const uint64_t* slots = xmax + ((int64_t)kvh * G + j) * mc;
#pragma unroll
        for (int i = 0; i < 4; i++) v[j][i] = slot_get(slots + min(c0 + lane + 64 * i, nch - 1));
    }
}
template <int HW>
__device__ __forceinline__ bool poll_ready(const uint64_t (&v)[HW][4], uint32_t tag) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < HW; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) ok = ok && (uint32_t)(v[j][i] >> 32) == tag;
    return __all(ok) != 0;
}
template <int HW>
__device__ __forceinline__ void poll_max(const uint64_t (&v)[HW][4], float (&res)[HW]) {
#pragma unroll
    for (int j = 0; j < HW; j++) {
        float mm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) mm = fmaxf(mm, __uint_as_float((uint32_t)v[j][i]));
        res[j] = wave_max(mm);
    }
}

// ---- XCD-local chunk-maximum exchange ----
// The dispatcher deals a launch's workgroups to the eight XCDs in turn:
// workgroup w runs on XCD (w + o) mod 8, o fixed for the launch (it varies from
// launch to launch; checked at context creation).  With the kv heads a
// multiple of 8, workgroup w serves kv head (w mod 8) + 8 j, so all chunks of a
// kv head run on one XCD and exchange their maxima through its L2: plain
// stores, and device-scope loads (cache policy sc1: past the CU's L1, served by
// the L2), which see a store from the same XCD ~0.2 us after it completes
// against ~1 us from another XCD (measured).  The partials go out the same
// way, as tagged words, and each chunk sums every chunk's partials for its
// own share of the kv head's outputs (reloading words whose tag is not yet
// this step's), so no combine launch follows.
// Each workgroup folds its own o (from its XCC_ID register) into the tag it
// publishes, so a chunk placed on another XCD never matches: its kv head's
// wait ends at the spin limit with the device error set, instead of mixing
// L2s.

constexpr uint32_t RSRC_W3 = 0x00020000u;   // buffer descriptor word 3 for gfx9 raw loads

__device__ __forceinline__ uint32_t xcc_id() {
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11)) & 0xFu;   // HW_REG_XCC_ID[3:0]
}
// 8 bytes at byte offset off of a buffer, read past the L1 (cache policy sc1);
// the load is not volatile, so a poll loop puts a compiler barrier before it
__device__ __forceinline__ uint64_t l2_load64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 16);
    return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
}

// Scores and values in one launch.  Workgroup (chunk c, kv head k) covers 64
// positions with two pairs of wavefronts: wavefronts 0-1 load the K rows
// (two threads per row), form the scores (RoPE and the new token's KV write
// as attn_scores_kernel), publish the chunk maxima in tagged slots and wait
// until every live chunk of the kv head has published; wavefronts 2-3 load
// the V rows into LDS at the same time.  The wait counter is per wavefront,
// so the exchange waits only for K.  Then all four form the exponentials
// against the global maxima and the chunk partials (as attn_pv_kernel),
// summed by attn_combine_kernel or, in the XCD-local form, inside this launch.  The wait needs the kv head's workgroups to run
// together: workgroups are dispatched in index order and the whole grid (at
// most 256 chunks per kv head, a few workgroups per CU) is resident at once,
// so none of them waits on a workgroup that cannot start; a wait that still
// runs past spin_max polls gives up and sets *err (the host reports it).
template <int HD, int G, bool F16, bool XL>
__global__ __launch_bounds__(WG) void attn_fused_kernel(AttnArgs a) {
    // XL: the XCD-local exchange (one-dimensional grid, see above)
    constexpr int HALF_ROW = HD / 2;              // K / V elements per loading thread
    constexpr int DPG = HD / 16;                  // V elements per thread and position (values)
    constexpr int PPT = CH / 16;                  // positions per thread (values)
    constexpr int NGR = G > 1 ? 16 : 4;
    constexpr int EB = F16 ? 2 : 4;               // bytes per cache element
    constexpr int VBUF = CH * HD * EB;            // V rows of the chunk, raw
    constexpr int RED = NGR * (G * HD + 4) * 4;   // position-group partial sums
    __shared__ float q_s[G * HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ float sc_s[G][CH];                 // scores (-inf past T), then exponentials
    __shared__ float gmax[G];
    __shared__ __align__(16) uint8_t pool[VBUF > RED ? VBUF : RED];   // V rows, then the partial sums
    // Every kernel argument in one round (a load of an argument that waits on
    // another's use adds a scalar round trip to every launch).
    asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.kcache), "s"(a.vcache), "s"(a.cos_tab), "s"(a.sin_tab),
                 "s"(a.pos), "s"(a.epoch), "s"(a.heads), "s"(a.kv_heads), "s"(a.rope_half), "s"(a.context));
    asm volatile("" ::"s"(a.xmax), "s"(a.layer), "s"(a.layers), "s"(a.spin_max), "s"(a.err), "s"(a.out));
    if (XL) asm volatile("" ::"s"(a.xpart));
    __builtin_amdgcn_sched_barrier(0);   // the argument loads go out together, before any use
    int c, kvh;
    if (XL) {   // one-dimensional grid: kv head (w mod 8) + 8 j, chunk c; one XCD per kv head
        const int w = blockIdx.x, per = a.kv_heads >> 3, r = w >> 3;
        kvh = (w & 7) + 8 * (r % per);
        c = r / per;
    } else {
        c = blockIdx.x;
        kvh = blockIdx.y;
    }
    const int half = a.rope_half;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const bool kwave = wave < 2;
    // Loads: the position and the epoch first (each wavefront's wait counter
    // retires loads in issue order, so waiting for them waits for nothing
    // else), then q and the new token's k and v, which do not need the
    // position; after it, the RoPE table rows of the position and the
    // thread's half row of K (wavefronts 0-1) or of V (2-3).  Rows past T read
    // row p0 (written) and are masked; row T is written below by this
    // workgroup and taken from LDS instead.
    const int T = *a.pos;
    const uint32_t epoch = *a.epoch;
    constexpr int QI = (G * HD + WG - 1) / WG;    // q elements per thread
    float qa[QI], qb[QI], qc[QI], qs[QI];
#pragma unroll
    for (int j = 0; j < QI; j++) {
        const int idx = min(t + j * WG, G * HD - 1);
        const int h = idx / HD, d = idx - h * HD;
        const float* x = a.q + (int64_t)(kvh * G + h) * HD;
        qa[j] = x[d];
        qb[j] = x[d < half ? d + half : (d < 2 * half ? d - half : d)];
    }
    // the new token's k pair and v element (read by every workgroup, used by
    // the owner: a load under a branch would be waited on inside it)
    float ka, kb, kc, ks, vn;
    const int dk = t < HD ? t : 0, ik = dk < half ? dk : (dk < 2 * half ? dk - half : 0);
    {
        const float* x = a.k + (int64_t)kvh * HD;
        ka = x[dk];
        kb = x[dk < half ? dk + half : (dk < 2 * half ? dk - half : dk)];
        vn = a.v[(int64_t)kvh * HD + dk];
    }
    // nothing above moves below the exit (a load used only past it would be
    // sunk there, behind the wait for the position)
    asm volatile("" ::: "memory");
    const int p0 = c * CH;
    const int n = T + 1;
    // SlidingWindow (IE:385-387): positions s0 .. T attend, chunks c0 .. nch-1
    // hold them, and the Softmax's vector lanes are the window's first
    // 8 floor(len / 8) positions (without a window: s0 = c0 = 0)
    const int s0 = a.window > 0 ? max(0, n - a.window) : 0, c0 = s0 / CH;
    const int n8 = s0 + ((n - s0) & ~7);
    if (p0 >= n || c < c0) return;
    const int nch = (n + CH - 1) / CH;            // chunks up to the last live one
    const int cnt = min(CH, n - p0);
    const int mc = XSTRIDE;                       // slots per head: one 4 KiB page each
    uint32_t tag = epoch * (uint32_t)a.layers + (uint32_t)a.layer + 1u;
    if (XL) tag = (tag << 3) | ((xcc_id() - blockIdx.x) & 7u);   // the launch's XCD offset, as this workgroup sees it
    const float* cs = a.cos_tab + (int64_t)T * half;
    const float* sn = a.sin_tab + (int64_t)T * half;
    const int64_t cache_base = (int64_t)kvh * a.context * HD;
    const bool owner = T >= p0 && T < p0 + CH;
#pragma unroll
    for (int j = 0; j < QI; j++) {
        const int idx = min(t + j * WG, G * HD - 1);
        const int d = idx % HD, i = d < half ? d : (d < 2 * half ? d - half : 0);
        qc[j] = cs[i];
        qs[j] = sn[i];
    }
    kc = cs[ik];
    ks = sn[ik];
    __builtin_amdgcn_sched_barrier(0);   // the small loads stay ahead of the rows
    const int lt = t & 127, rp = lt >> 1, rh = lt & 1;   // row (position) and half of it
    const int rpos = p0 + rp;
    const bool rlive = rpos < n && rpos >= s0;
    KvRaw<HALF_ROW, F16> row;
    row.load(kwave ? a.kcache : a.vcache,
             cache_base + (int64_t)(rlive && rpos != T ? rpos : p0) * HD + rh * HALF_ROW);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int j = 0; j < QI; j++) {
        const int idx = t + j * WG;
        if (idx < G * HD) q_s[idx] = rope_pair(qa[j], qb[j], qc[j], qs[j], idx % HD, half);
    }
    if (owner && t < HD) {   // this workgroup owns the new token: K/V slot T
        const int64_t slot = cache_base + (int64_t)T * HD + t;
        knew[t] = store_kv(a.kcache, slot, rope_pair(ka, kb, kc, ks, t, half), F16);
        vnew[t] = store_kv(a.vcache, slot, vn, F16);
    }
    __syncthreads();
    if (kwave) {
        // scores: two threads per position, each over half of the row
        float kf[HALF_ROW];
#pragma unroll
        for (int d = 0; d < HALF_ROW; d++) kf[d] = row.at(d);
        if (owner && rpos == T) {   // one branch around the loop, taken in one workgroup
#pragma unroll
            for (int d = 0; d < HALF_ROW; d++) kf[d] = knew[rh * HALF_ROW + d];
        }
        const float inv_sqrt = 1.0f / sqrtf((float)HD);
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float* qv = q_s + h * HD + rh * HALF_ROW;
            float sdot = 0.f;
#pragma unroll
            for (int d = 0; d < HALF_ROW; d++) sdot += qv[d] * kf[d];
            sdot += fx(lane_xor1, sdot);
            if (rh == 0) sc_s[h][rp] = rlive ? sdot * inv_sqrt : -INFINITY;
        }
    } else {
        // V half rows into LDS, raw
        uint32_t* vb = reinterpret_cast<uint32_t*>(pool) + (rp * HD + rh * HALF_ROW) * EB / 4;
#pragma unroll
        for (int i = 0; i < KvRaw<HALF_ROW, F16>::W; i++) vb[i] = row.w[i];
    }
    __syncthreads();
    if (kwave) {
        // Chunk maxima out, global maxima in: wavefronts 0 and 1 publish and
        // gather heads wave, wave + 2, ... (the wavefronts that loaded V have
        // finished with memory and stay out of the polling traffic); each
        // lane polls four slots per head (chunks lane + 64 i, clamped to the
        // last live one).
        for (int h = wave; h < G; h += 2) {
            const float m = wave_max(sc_s[h][lane]);
            if (lane == 0) {
                uint64_t* slot = a.xmax + ((int64_t)kvh * G + h) * mc + c;
                if (XL) __hip_atomic_store(slot, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(m), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);   // a plain store into this XCD's L2
                else slot_put(slot, tag, m);
            }
        }
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            a.xmax, (short)0, (int)((uint32_t)a.heads * XSTRIDE * 8), (int)RSRC_W3);
        if (XL) {   // all of the wavefront's heads in one poll loop
            constexpr int HW = (G + 1) / 2;
            const int nh = (G - wave + 1) / 2;   // heads of this wavefront (none: wavefront 1 when G = 1)
            if (nh > 0) {
                uint64_t v[HW][4];
                float res[HW];
                for (int it = 0;; it++) {
                    asm volatile("" ::: "memory");   // a fresh load every poll
#pragma unroll
                    for (int j = 0; j < HW; j++) {
                        const uint32_t base = (uint32_t)((kvh * G + wave + 2 * min(j, nh - 1)) * mc) * 8;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            v[j][i] = l2_load64(rx, base + 8 * (uint32_t)min(c0 + lane + 64 * i, nch - 1));
                    }
                    if (poll_ready<HW>(v, tag)) break;
                    if (it >= a.spin_max) {
                        if (lane == 0) atomicOr(a.err, 1);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                poll_max<HW>(v, res);
#pragma unroll
                for (int j = 0; j < HW; j++)
                    if (lane == 0 && j < nh) gmax[wave + 2 * j] = res[j];
            }
        } else {
            for (int h = wave; h < G; h += 2) {
                uint64_t v[1][4];
                float res[1];
                for (int it = 0;; it++) {
                    poll_issue<1>(v, a.xmax + ((int64_t)kvh * G + h) * mc, 0, lane, c0, nch, mc);
                    if (poll_ready<1>(v, tag)) break;
                    if (it >= a.spin_max) {
                        if (lane == 0) atomicOr(a.err, 1);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                poll_max<1>(v, res);
                if (lane == 0) gmax[h] = res[0];
            }
        }
    }
    __syncthreads();
    // the values phase: this thread's V slices (positions pg + 16 i, DPG
    // elements from dg * DPG) as floats; the new token's from LDS
    const int dg = t & 15, pg = t >> 4;
    float vv[PPT][DPG];
#pragma unroll
    for (int i = 0; i < PPT; i++) {
        const int e0 = (pg + 16 * i) * HD + dg * DPG;
#pragma unroll
        for (int d = 0; d < DPG; d++) {
            if constexpr (F16) vv[i][d] = (float)reinterpret_cast<const _Float16*>(pool)[e0 + d];
            else vv[i][d] = reinterpret_cast<const float*>(pool)[e0 + d];
        }
    }
    if (owner) {   // the new token's V slice from LDS (its cache row was loaded stale)
#pragma unroll
        for (int i = 0; i < PPT; i++)
            if (p0 + pg + 16 * i == T) {
#pragma unroll
                for (int d = 0; d < DPG; d++) vv[i][d] = vnew[dg * DPG + d];
            }
    }
    for (int idx = t; idx < G * CH; idx += WG) {
        const int h = idx / CH, pp = idx - h * CH;
        const int sidx = p0 + pp;
        float e;
        {
#pragma clang fp contract(off)
            const float x = sc_s[h][pp] - gmax[h];
            // Softmax: ExpApprox on the vector lanes (first 8*floor(len/8) of the window), expf on the tail
            e = sidx < n8 ? exp_approx(x) : expf(x);
        }
        sc_s[h][pp] = pp < cnt && sidx >= s0 ? e : 0.f;
    }
    __syncthreads();   // exponentials visible; the V rows are in registers (pool reused below)
    // XL: the partials go out as tagged 64-bit words, (tag << 32) | float bits,
    // which the kv head's other chunks poll for (no separate "written" flag)
    uint64_t* const xz = XL ? a.xpart + (int64_t)((a.context + CH - 1) / CH) * a.heads * HD : nullptr;   // [chunks][heads]
    for (int h = wave; h < G; h += 4) {   // this chunk's sum of exponentials
        const float z = wave_sum(sc_s[h][lane]);
        if (lane == 0) {
            if (XL) __hip_atomic_store(xz + (int64_t)c * a.heads + kvh * G + h, ((uint64_t)tag << 32) | __float_as_uint(z),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            else a.part_sum[(int64_t)c * a.heads + kvh * G + h] = z;
        }
    }
    float (*red)[G * HD + 4] = reinterpret_cast<float (*)[G * HD + 4]>(pool);
#pragma unroll
    for (int h = 0; h < G; h++) {
        float acc[DPG];
#pragma unroll
        for (int d = 0; d < DPG; d++) acc[d] = 0.f;
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const float pr = sc_s[h][pg + 16 * i];
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
        const int64_t o = ((int64_t)c * a.heads + kvh * G + h) * HD + d;
        if (XL) __hip_atomic_store(a.xpart + o, ((uint64_t)tag << 32) | __float_as_uint(r), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        else a.part_out[o] = r;
    }
    if (XL) {
        // The combine without a launch: each workgroup sums every chunk's
        // partials for its own share of the kv head's G*HD outputs, polling the
        // tagged words until each carries this step's tag (the barrier only
        // frees the LDS pool for reuse).
        __syncthreads();
        constexpr int NCOL = G * HD;                  // outputs of the kv head
        const int nlive = nch - c0;                   // chunks in the window
        const int per = (NCOL + nlive - 1) / nlive;   // outputs per chunk workgroup
        const int j0 = (c - c0) * per, nc = min(NCOL, j0 + per) - j0;
        if (nc <= 0) return;
        // Two lane layouts.  Many chunks (fewer than 64 columns each): columns
        // run fastest over the lanes (padded to a power of two, ncp), so a load
        // instruction reads whole runs of a chunk's columns, and a column's
        // chunk groups meet in an xor tree inside the wavefront, then through
        // at most four LDS partials.  Few chunks (64 or more columns): the
        // chunk groups (at most four) run fastest and their xor tree ends the
        // sum.  Either way ngrp groups (a power of two) each take every
        // ngrp-th chunk, and each column also sums its head's exponent sums
        // over the same chunks (one round of loads for both).
        int ncp = 1;
        while (ncp < nc) ncp *= 2;
        const bool wide = ncp >= 64;
        int ngrp = 1;
        while (2 * ngrp * (wide ? nc : ncp) <= WG && 2 * ngrp <= nlive && 2 * ngrp <= 64) ngrp *= 2;
        const int np = wide ? 1 : (ngrp * ncp + 63) / 64;   // partials per column
        float* cred = reinterpret_cast<float*>(pool);  // [np][ncp] sums of e.V, then [np][ncp] sums of e
        float* zred = cred + np * ncp;
        const uint32_t chunk_bytes = (uint32_t)a.heads * HD * 8;
        const __amdgpu_buffer_rsrc_t ro =
            __builtin_amdgcn_make_buffer_rsrc(a.xpart, (short)0, (int)((uint32_t)nch * chunk_bytes), (int)RSRC_W3);
        const __amdgpu_buffer_rsrc_t rz =
            __builtin_amdgcn_make_buffer_rsrc(xz, (short)0, (int)((uint32_t)nch * a.heads * 8), (int)RSRC_W3);
        // column col over chunks g, g + ngrp, ...: the four chunks' words are
        // loaded again until every live one carries the tag (chunks >= nch
        // read past the buffer's end and count as 0)
        auto column_sum = [&](int col, int g, float& zacc) {
            float acc = 0.f;
            zacc = 0.f;
            const uint32_t off = ((uint32_t)kvh * NCOL + j0 + col) * 8;
            const uint32_t zoff = ((uint32_t)kvh * G + (uint32_t)(j0 + col) / HD) * 8;
            for (int cc = c0 + g; cc < nch; cc += 4 * ngrp) {
                uint64_t v[4], w[4];
                for (int it = 0;; it++) {
                    asm volatile("" ::: "memory");   // a fresh load every poll
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const uint32_t ch = (uint32_t)(cc + u * ngrp);
                        v[u] = l2_load64(ro, off + ch * chunk_bytes);
                        w[u] = l2_load64(rz, zoff + ch * (uint32_t)a.heads * 8);
                    }
                    bool ok = true;
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        ok = ok && (cc + u * ngrp >= nch || ((uint32_t)(v[u] >> 32) == tag && (uint32_t)(w[u] >> 32) == tag));
                    if (ok) break;
                    if (it >= a.spin_max) {
                        atomicOr(a.err, 1);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    acc += __uint_as_float((uint32_t)v[u]);
                    zacc += __uint_as_float((uint32_t)w[u]);
                }
            }
            return acc;
        };
        if (wide) {
            const int g = t & (ngrp - 1), slots = WG / ngrp;
            for (int col = t / ngrp; col < nc; col += slots) {   // the ngrp lanes of a column share the loop
                float z;
                float acc = column_sum(col, g, z);
                for (int o = ngrp >> 1; o > 0; o >>= 1) {
                    acc += __shfl_xor(acc, o, 64);
                    z += __shfl_xor(z, o, 64);
                }
                if (g == 0) {
                    cred[col] = acc;
                    zred[col] = z;
                }
            }
        } else {
            const int col = t & (ncp - 1), g = t / ncp;
            float z = 0.f;
            float acc = g < ngrp && col < nc ? column_sum(col, g, z) : 0.f;
            for (int o = ncp; o < 64; o <<= 1) {   // the wavefront's groups of this column
                acc += __shfl_xor(acc, o, 64);
                z += __shfl_xor(z, o, 64);
            }
            if (lane < ncp && wave < np) {
                cred[wave * ncp + col] = acc;
                zred[wave * ncp + col] = z;
            }
        }
        __syncthreads();
        for (int cl = t; cl < nc; cl += WG) {
            float r = cred[cl], z = zred[cl];
            for (int q = 1; q < np; q++) {
                r += cred[q * ncp + cl];
                z += zred[q * ncp + cl];
            }
            a.out[(int64_t)kvh * NCOL + j0 + cl] = r * (1.0f / z);
        }
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
    const int c0 = a.window > 0 ? max(0, n - a.window) / CHP : 0;   // the window's first chunk
    const int hq = blockIdx.x, g = threadIdx.x / HD, d = threadIdx.x - g * HD;
    float acc = 0.f, z = 0.f;
#pragma unroll 8
    for (int i = c0 + g; i < nch; i += NG) {
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
    if (a.fused) {
        if (!a.xmax || !a.epoch || !a.err || !attn_fused_ok(a.heads, a.kv_heads, a.head_dim, a.context))
            return hipErrorInvalidValue;
        if (a.xcd_exchange) {   // XCD-local exchange: one-dimensional grid
            if (a.kv_heads % 8 || !a.xpart) return hipErrorInvalidValue;
            const dim3 grid(nchunks * a.kv_heads);
            if (a.kv_fp16) attn_fused_kernel<HD, G, true, true><<<grid, WG, 0, s>>>(a);
            else attn_fused_kernel<HD, G, false, true><<<grid, WG, 0, s>>>(a);
        } else {
            if (a.kv_fp16) attn_fused_kernel<HD, G, true, false><<<dim3(nchunks, a.kv_heads), WG, 0, s>>>(a);
            else attn_fused_kernel<HD, G, false, false><<<dim3(nchunks, a.kv_heads), WG, 0, s>>>(a);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || a.xcd_exchange) return e;   // the XCD-local form combines in the launch
        attn_combine_kernel<HD><<<a.heads, (1024 / HD) * HD, 0, s>>>(a);
        return hipGetLastError();
    }
    // the three-launch form attends to every position: a model with a window
    // runs the one-launch form (its creation refuses a window otherwise)
    if (a.window > 0) return hipErrorInvalidValue;
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

int attn_xmax_slots(int heads) { return heads * XSTRIDE; }

namespace {
__global__ void xcc_probe_kernel(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}
}  // namespace

namespace {
template <int HD, int G>
int xl_per_cu(int kv_fp16) {
    int n = 0;
    const hipError_t e = kv_fp16
        ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_fused_kernel<HD, G, true, true>, WG, 0)
        : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_fused_kernel<HD, G, false, true>, WG, 0);
    return e == hipSuccess ? n : 0;
}
template <int HD>
int xl_per_cu_g(int g, int kv_fp16) {
    switch (g) {
    case 1: return xl_per_cu<HD, 1>(kv_fp16);
    case 2: return xl_per_cu<HD, 2>(kv_fp16);
    case 4: return xl_per_cu<HD, 4>(kv_fp16);
    case 8: return xl_per_cu<HD, 8>(kv_fp16);
    default: return 0;
    }
}
}  // namespace

bool attn_xcd_fits(int heads, int kv_heads, int head_dim, int context, int kv_fp16, int cus) {
    if (!attn_fused_ok(heads, kv_heads, head_dim, context) || kv_heads % 8 || cus < 8) return false;
    const int g = heads / kv_heads;
    const int per_cu = head_dim == 64 ? xl_per_cu_g<64>(g, kv_fp16)
                     : head_dim == 96 ? xl_per_cu_g<96>(g, kv_fp16)
                     : xl_per_cu_g<128>(g, kv_fp16);
    const int per_xcd = per_cu * (cus / 8);   // workgroups one XCD holds at once
    return (kv_heads / 8) * attn_max_chunks(heads, kv_heads, context) * 4 <= per_xcd * 3;
}

hipError_t attn_xcd_check(hipStream_t s, bool* ok) {
    constexpr int N = 2048;   // workgroups of the probe launch
    *ok = false;
    uint32_t* d = nullptr;
    hipError_t e = hipMalloc(&d, N * sizeof(uint32_t));
    if (e != hipSuccess) return e;
    uint32_t h[N];
    xcc_probe_kernel<<<N, 64, 0, s>>>(d);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpyAsync(h, d, sizeof h, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(d);
    if (e != hipSuccess) return e;
    bool all = true;
    for (int w = 0; w < N; w++) all = all && ((h[w] - (uint32_t)w) & 7u) == ((h[0] - 0u) & 7u);
    *ok = all;
    return hipSuccess;
}

bool attn_fused_ok(int heads, int kv_heads, int head_dim, int context) {
    return attn_supported(heads, kv_heads, head_dim) && (context + CH - 1) / CH <= 256;
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
