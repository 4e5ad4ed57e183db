// gemv.hip -- fused dequant-GEMV over native GGUF blocks (batch 1).
//
// y[r] = sum_k deq(W)[r][k] * x[k]   (TensorOps.MatMul with aRows == 1,
// src/Llmdot.Core/Tensors/TensorOps.cs:60-90, fused per-type kernels TO:118-431).
// The weight blocks are read once from HBM in their GGUF layout.
//
// Decomposition.  A workgroup (4 wavefronts) owns a group of 32 consecutive
// output rows and a slice of the reduction dimension (split-K); each wavefront
// owns 8 of the rows, processed as 2 tiles of 4 rows (4 tiles of 2 gate + 2 up
// rows for the SwiGLU form).  The 64 lanes stride over the slice in "units" (a
// 32-element sub-block, 64 for Q6_K); a lane's units are fixed for the whole
// workgroup, so its activations are loaded once and stay in registers while
// all rows stream through.  A tile's 4 row sums are reduced across the
// wavefront with a transposing butterfly (7 shuffles).  With split-K the
// per-split partial sums go to a scratch buffer and the last workgroup of the
// group (atomic counter) adds them in split order, so results do not depend
// on scheduling.
//
// Arithmetic.  Q4_K (the reference's own layout) runs on v_dot8_i32_i4 against
// the activation records of xrec.h: weight nibble ^ 8 = q - 8 as int4, four
// dot8 per 8 elements, exact int32; per sub-block the result is scaled by
// (d*sc) and the dmin*m term uses the record's sum.  The other types
// dequantise in registers (v_cvt_f32_ubyte*) and accumulate in fp32.
//
// Epilogues: STORE; ADD (residual h += y, VectorMath.Add VM:27-42, plus the
// records of the new h for the next consumer's RmsNorm); SWIGLU
// (SiluInPlace(gate) * up, IE:463-474, VM:118-135, plus the records of the
// result); ARGMAX (logits plus ArgMax VM:412-425, last-workgroup reduction).
#include "common.h"
#include "kernels.h"
#include "xrec.h"

namespace llmdot {

namespace {

constexpr int WG = 256;
constexpr int GROUP = 32;

__device__ __forceinline__ float h16(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
__device__ __forceinline__ float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sb(uint32_t w, int k) { return (float)(int8_t)(w >> (8 * k)); }

// 6-bit scale and min of sub-block g from the 96-bit LSB-first stream in
// header words y, z, w (DequantizeK.Extract6Bit, DK:189-199).
__device__ __forceinline__ void kscale(uint32_t y, uint32_t z, uint32_t w, int g, float& sc, float& m) {
    const int bit = 12 * g;
    const uint32_t lo = bit < 32 ? y : (bit < 64 ? z : w);
    const uint32_t hi = bit < 32 ? z : (bit < 64 ? w : 0u);
    const uint32_t f = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)(bit & 31));
    sc = (float)(f & 63u);
    m = (float)((f >> 6) & 63u);
}

// ---- integer path (Q4_K) ------------------------------------------------------
struct XI {           // a lane's activation record for one unit (s, sum already times 1/rms)
    uint32_t pl[16];
    float s, sum;
};

__device__ __forceinline__ float q4k_int(const uint8_t* row, int u, const XI& x) {
    const uint8_t* blk = row + (u >> 3) * 144;
    const int g = u & 7;
    const u32x4 h = ld16_a4(blk);
    const u32x4 q = ld16_a4(blk + 16 + 16 * g);
    const uint32_t w[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
    int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        a0 = __builtin_amdgcn_sdot8((int)w[j], (int)x.pl[j], a0, false);
        a1 = __builtin_amdgcn_sdot8((int)w[j], (int)x.pl[4 + j], a1, false);
        a2 = __builtin_amdgcn_sdot8((int)w[j], (int)x.pl[8 + j], a2, false);
        a3 = __builtin_amdgcn_sdot8((int)w[j], (int)x.pl[12 + j], a3, false);
    }
    const int S = a0 + (a1 << 4) + (a2 << 8) + (a3 << 12);
    float sc, m;
    kscale(h.y, h.z, h.w, g, sc, m);
    const float d = h16(h.x & 0xFFFFu), dm = h16(h.x >> 16);
    return (d * sc) * (x.s * (float)S) - (dm * m) * x.sum;
}

// ---- fp32 path decoders ------------------------------------------------------------
// Unit u of a row; x holds the unit's UE activations in the unit's element
// order; xs the NS partial sums the type's offset needs.

struct UQ5K {  // reference Q5_K: 176 B / 256; unit = sub-block g
    static constexpr int UE = 32, NS = 1;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + (u >> 3) * 176;
        const int g = u & 7;
        const u32x4 h = ld16_a4(blk);
        const uint32_t qh = ld4_a4(blk + 16 + 4 * g);
        const u32x4 q = ld16_a4(blk + 48 + 16 * g);
        float sc, m;
        kscale(h.y, h.z, h.w, g, sc, m);
        const float d = h16(h.x & 0xFFFFu), dm = h16(h.x >> 16);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t hb = qh >> (8 * j);
            // bits 0,2,4,6 of hb -> bit 4 of bytes 0..3 (even elements), bits 1,3,5,7 -> odd
            const uint32_t he = ((hb & 0x55u) * 0x410410u) & 0x10101010u;
            const uint32_t ho = (((hb >> 1) & 0x55u) * 0x410410u) & 0x10101010u;
            const uint32_t e = (w[j] & 0x0F0F0F0Fu) | he, o = ((w[j] >> 4) & 0x0F0F0F0Fu) | ho;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x[8 * j + 2 * k] * ub(e, k);
                s1 += x[8 * j + 2 * k + 1] * ub(o, k);
            }
        }
        return (d * sc) * ((s0 + s1) - 16.f * xs[0]) - (dm * m) * xs[0];
    }
};

struct UQ6K {  // Q6_K: 210 B / 256; unit = (half n, l-range l0..l0+15) -> 64 elements
    static constexpr int UE = 64, NS = 4;
    // run t (0..3) of 16 elements: n + l0 + 32 t + [0, 16)
    __device__ static int xoff(int u, int t) {
        const int sub = u & 3;
        return (u >> 2) * 256 + (sub >> 1) * 128 + (sub & 1) * 16 + 32 * t;
    }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + (u >> 2) * 210;
        const int sub = u & 3, n = (sub >> 1) * 128, l0 = (sub & 1) * 16;
        uint32_t A[4], B[4], C[4], S[2], Dw[1];
        ld_realign<4>(blk + n / 2 + l0, A);
        ld_realign<4>(blk + n / 2 + l0 + 32, B);
        ld_realign<4>(blk + 128 + n / 4 + l0, C);
        ld_realign<2>(blk + 192 + n / 16 + l0 / 16, S);
        ld_realign<1>(blk + 208, Dw);
        const float d = h16(Dw[0] & 0xFFFFu);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t q0 = (A[j] & 0x0F0F0F0Fu) | ((C[j] & 0x03030303u) << 4);
            const uint32_t q1 = (B[j] & 0x0F0F0F0Fu) | ((C[j] & 0x0C0C0C0Cu) << 2);
            const uint32_t q2 = ((A[j] >> 4) & 0x0F0F0F0Fu) | (C[j] & 0x30303030u);
            const uint32_t q3 = ((B[j] >> 4) & 0x0F0F0F0Fu) | ((C[j] >> 2) & 0x30303030u);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s[0] += x[0 * 16 + 4 * j + k] * ub(q0, k);
                s[1] += x[1 * 16 + 4 * j + k] * ub(q1, k);
                s[2] += x[2 * 16 + 4 * j + k] * ub(q2, k);
                s[3] += x[3 * 16 + 4 * j + k] * ub(q3, k);
            }
        }
        float r = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++) r += (d * sb(S[t >> 1], 2 * (t & 1))) * (s[t] - 32.f * xs[t]);
        return r;
    }
};

struct UQ8_0 {  // Q8_0: 34 B / 32; unit = block
    static constexpr int UE = 32, NS = 0;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float*) {
        const uint8_t* blk = row + u * 34;
        uint32_t Dw[1], Q[8];
        ld_realign<1>(blk, Dw);
        ld_realign<8>(blk + 2, Q);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x[4 * j + k] * sb(Q[j], k);
                s1 += x[4 * j + 4 + k] * sb(Q[j + 1], k);
            }
        return h16(Dw[0] & 0xFFFFu) * (s0 + s1);
    }
};

struct UQ4_0 {  // Q4_0: 18 B / 32; unit = block; low nibbles -> j, high -> j + 16
    static constexpr int UE = 32, NS = 1;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + u * 18;
        uint32_t Dw[1], Q[4];
        ld_realign<1>(blk, Dw);
        ld_realign<4>(blk + 2, Q);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = Q[j] & 0x0F0F0F0Fu, hi = (Q[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x[4 * j + k] * ub(lo, k);
                s1 += x[16 + 4 * j + k] * ub(hi, k);
            }
        }
        return h16(Dw[0] & 0xFFFFu) * ((s0 + s1) - 8.f * xs[0]);
    }
};

struct UF32 {
    static constexpr int UE = 32, NS = 0;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float*) {
        const float4* p = reinterpret_cast<const float4*>(row + (int64_t)u * 128);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float4 a = p[j], b = p[j + 1];
            s0 += x[4 * j] * a.x + x[4 * j + 1] * a.y + x[4 * j + 2] * a.z + x[4 * j + 3] * a.w;
            s1 += x[4 * j + 4] * b.x + x[4 * j + 5] * b.y + x[4 * j + 6] * b.z + x[4 * j + 7] * b.w;
        }
        return s0 + s1;
    }
};

struct UF16 {
    static constexpr int UE = 32, NS = 0;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float*) {
        const uint8_t* p = row + (int64_t)u * 64;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const u32x4 v = ld16_a4(p + 16 * j);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; k++)
                s += x[8 * j + 2 * k] * h16(w[k] & 0xFFFFu) + x[8 * j + 2 * k + 1] * h16(w[k] >> 16);
        }
        return s;
    }
};

template <uint32_t T> struct UnitOf;
template <> struct UnitOf<GGML_Q5_K> { using type = UQ5K; };
template <> struct UnitOf<GGML_Q6_K> { using type = UQ6K; };
template <> struct UnitOf<GGML_Q8_0> { using type = UQ8_0; };
template <> struct UnitOf<GGML_Q4_0> { using type = UQ4_0; };
template <> struct UnitOf<GGML_F32> { using type = UF32; };
template <> struct UnitOf<GGML_F16> { using type = UF16; };

// Sum of 4 per-lane values for 4 rows: lanes 16 r .. 16 r + 15 end with row r's total.
__device__ __forceinline__ float reduce4(float a0, float a1, float a2, float a3, int lane) {
    const bool hi = lane & 32;
    float k0 = hi ? a2 : a0, k1 = hi ? a3 : a1;
    const float s0 = hi ? a0 : a2, s1 = hi ? a1 : a3;
    k0 += __shfl_xor(s0, 32, 64);
    k1 += __shfl_xor(s1, 32, 64);
    const bool b4 = lane & 16;
    float k = b4 ? k1 : k0;
    const float s = b4 ? k0 : k1;
    k += __shfl_xor(s, 16, 64);
    k += __shfl_xor(k, 8, 64);
    k += __shfl_xor(k, 4, 64);
    k += __shfl_xor(k, 2, 64);
    k += __shfl_xor(k, 1, 64);
    return k;
}

// 1/rms of the vector whose records are xrec[0 .. nrec) (every lane gets it):
// RmsNorm's ss = sum(x^2); ss /= n; ss += eps; inv = 1 / sqrt(ss).
__device__ __forceinline__ float rms_inv_from_records(const XRec* xrec, int nrec, int n, float eps) {
#pragma clang fp contract(off)
    float ss = 0.f;
    for (int i = threadIdx.x & 63; i < nrec; i += 64) ss += xrec[i].ssq;
    ss = wave_sum(ss);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

struct Place {   // this workgroup's segment, row group and K split
    int seg, group, split;
};

__device__ __forceinline__ Place locate(const GemvArgs& a) {
    int b = blockIdx.x, s = 0;
    for (; s < a.nseg - 1; s++) {
        const int nb = a.seg[s].groups * a.splitk;
        if (b < nb) break;
        b -= nb;
    }
    return Place{s, b / a.splitk, b % a.splitk};
}

template <int UPL>
struct Units {   // a lane's units in this split: u0 + lane + 64 i below u1
    int u[UPL];
    bool ok[UPL];
};

// The 8 rows (or 8 gate + 8 up rows) of this wavefront; sums go to
// part_lds[wave*8 + i] (and part_lds[32 + wave*8 + i] for up).
template <int UPL, bool SWIGLU, typename DotFn>
__device__ __forceinline__ void rows_body(const GemvSeg& seg, const Place& pl, int64_t rb, DotFn&& dotfn,
                                          const Units<UPL>& un, float* part_lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row_base = pl.group * GROUP + wave * 8;
    constexpr int TILES = SWIGLU ? 4 : 2;
#pragma unroll
    for (int t = 0; t < TILES; t++) {
        const uint8_t* wr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = SWIGLU ? row_base + 2 * t + (r & 1) : row_base + 4 * t + r;
            const uint8_t* base = (SWIGLU && r >= 2) ? seg.w2 : seg.w;
            wr[r] = base + (int64_t)(row < seg.rows ? row : 0) * rb;
        }
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < UPL; i++)
            if (un.ok[i]) {
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] += dotfn(wr[r], un.u[i], i);
            }
        const float tot = reduce4(acc[0], acc[1], acc[2], acc[3], lane);
        if ((lane & 15) == 0) {
            const int r = lane >> 4;
            if (SWIGLU) part_lds[(r >= 2 ? 32 : 0) + wave * 8 + 2 * t + (r & 1)] = tot;
            else part_lds[wave * 8 + 4 * t + r] = tot;
        }
    }
}

// Split-K combine and epilogue for one 32-row group.
template <int EPI>
__device__ __forceinline__ void finish_group(const GemvArgs& a, const Place& pl, const GemvSeg& seg, float* part_lds) {
    __shared__ int last;
    constexpr int NV = EPI == EPI_SWIGLU ? 64 : 32;
    const int tid = threadIdx.x;
    if (a.splitk > 1) {
        float* slot = a.partial + ((int64_t)pl.group * a.splitk + pl.split) * 64;
        if (tid < NV) slot[tid] = part_lds[tid];
        // One agent-scope release by thread 0 after the barrier publishes the
        // whole workgroup's stores (the barrier orders them before it); the
        // last arrival's acquire likewise covers the reads of all its threads.
        __syncthreads();
        if (tid == 0) {
            __threadfence();
            last = atomicAdd(a.counters + pl.group, 1u) == (unsigned)(a.splitk - 1);
            if (last) __threadfence();
        }
        __syncthreads();
        if (!last) return;
        if (tid < NV) {
            float s = 0.f;
            const float* base = a.partial + (int64_t)pl.group * a.splitk * 64;
            for (int k = 0; k < a.splitk; k++) s += __builtin_nontemporal_load(base + k * 64 + tid);
            part_lds[tid] = s;
        }
        if (tid == 0) a.counters[pl.group] = 0u;
        __syncthreads();
    }
    if (tid >= 64) return;   // wavefront 0 finishes: lane e < 32 owns row group*32 + e
    const int e = tid & 31;
    const int row = pl.group * GROUP + e;
    const bool valid = row < seg.rows && tid < 32;
    const float y = part_lds[e];
    if (EPI == EPI_STORE) {
        if (valid) seg.out[row] = y;
    } else if (EPI == EPI_ADD || EPI == EPI_SWIGLU) {
        float outv = 0.f;
        if (valid) {
#pragma clang fp contract(off)
            if (EPI == EPI_ADD) {
                outv = seg.out[row] + y;      // residual: a[i] + b[i]
            } else {
                const float up = part_lds[32 + e];
                const float sg = row < (seg.rows & ~7) ? silu_ref(y) : y / (1.0f + expf(-y));
                outv = sg * up;
            }
            seg.out[row] = outv;
        }
        if (a.rec_out) {
            float v = outv;
            if (a.rec_w && valid) {
#pragma clang fp contract(off)
                v = a.rec_w[row] * outv;
            }
            build_xrec(v, outv * outv, a.rec_out + pl.group, tid < 32);
        }
    } else if (EPI == EPI_ARGMAX) {
        if (valid) seg.out[row] = y;
        float bv = valid ? y : -INFINITY;
        int bi = valid ? row : 0x7FFFFFFF;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        int is_last = 0;
        if (tid == 0) {
            a.am.cand_val[pl.group] = bv;
            a.am.cand_idx[pl.group] = bi;
            __threadfence();
            is_last = atomicAdd(a.am.counter, 1u) == (unsigned)(seg.groups - 1);
        }
        is_last = __shfl(is_last, 0, 64);
        if (!is_last) return;
        if (tid == 0) __threadfence();
        __builtin_amdgcn_wave_barrier();
        float v = -INFINITY;
        int idx = 0x7FFFFFFF;
        for (int c = tid; c < seg.groups; c += 64) {
            const float cv = __builtin_nontemporal_load(a.am.cand_val + c);
            const int ci = __builtin_nontemporal_load(a.am.cand_idx + c);
            if (cv > v || (cv == v && ci < idx)) { v = cv; idx = ci; }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(v, o, 64);
            const int oi = __shfl_xor(idx, o, 64);
            if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
        }
        if (tid == 0) {
            if (idx == 0x7FFFFFFF) idx = 0;   // all NaN: ArgMax returns 0
            *a.am.token_out = idx;
            if (a.am.token_log && *a.am.step >= 0 && *a.am.step < a.am.log_cap) a.am.token_log[*a.am.step] = idx;
            if (a.am.step) *a.am.step += 1;
            if (a.am.pos) *a.am.pos += 1;
            *a.am.counter = 0u;
        }
    }
}

template <uint32_t T, int EPI>
__global__ __launch_bounds__(WG) void gemv_kernel(GemvArgs a) {
    __shared__ float part_lds[64];
    const Place pl = locate(a);
    const GemvSeg seg = a.seg[pl.seg];
    constexpr bool SWIGLU = EPI == EPI_SWIGLU;
    const int lane = threadIdx.x & 63;
    const int K = a.cols;
    if constexpr (T == GGML_Q4_K) {
        constexpr int UPL = 2;
        const int U = K / 32, per = U / a.splitk;
        const int u0 = pl.split * per, u1 = u0 + per;
        const int64_t rb = (int64_t)(K / 256) * 144;
        const float inv = a.norm ? rms_inv_from_records(a.xrec, U, K, a.eps) : 1.f;
        Units<UPL> un;
        XI xi[UPL];
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            un.u[i] = u0 + lane + 64 * i;
            un.ok[i] = un.u[i] < u1;
            const XRec* r = a.xrec + (un.ok[i] ? un.u[i] : 0);
            const u32x4* p = reinterpret_cast<const u32x4*>(r);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const u32x4 v = p[q];
                xi[i].pl[4 * q] = v.x; xi[i].pl[4 * q + 1] = v.y; xi[i].pl[4 * q + 2] = v.z; xi[i].pl[4 * q + 3] = v.w;
            }
            xi[i].s = r->s * inv;
            xi[i].sum = r->sum * inv;
        }
        auto fn = [&](const uint8_t* row, int u, int i) { return q4k_int(row, u, xi[i]); };
        rows_body<UPL, SWIGLU>(seg, pl, rb, fn, un, part_lds);
    } else {
        using U_ = typename UnitOf<T>::type;
        constexpr int UE = U_::UE;
        constexpr int UPL = UE == 64 ? 1 : 2;
        const int U = K / UE, per = U / a.splitk;
        const int u0 = pl.split * per, u1 = u0 + per;
        const int64_t rb = (int64_t)(K / block_elems(T)) * block_bytes(T);
        const float inv = a.norm ? rms_inv_from_records(a.xrec, K / 32, K, a.eps) : 1.f;
        Units<UPL> un;
        float xv[UPL][UE];
        float xs[UPL][U_::NS > 0 ? U_::NS : 1];
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            un.u[i] = u0 + lane + 64 * i;
            un.ok[i] = un.u[i] < u1;
            const int uu = un.ok[i] ? un.u[i] : 0;
#pragma unroll
            for (int run = 0; run < UE / 16; run++) {
                const int off = U_::xoff(uu, run);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 h = *reinterpret_cast<const float4*>(a.x + off + 4 * q);
                    if (a.norm) {   // VectorMath.RmsNorm vector lanes: (w * x) * inv
#pragma clang fp contract(off)
                        const float4 w = *reinterpret_cast<const float4*>(a.norm_w + off + 4 * q);
                        h.x = (w.x * h.x) * inv; h.y = (w.y * h.y) * inv;
                        h.z = (w.z * h.z) * inv; h.w = (w.w * h.w) * inv;
                    }
                    xv[i][run * 16 + 4 * q] = h.x; xv[i][run * 16 + 4 * q + 1] = h.y;
                    xv[i][run * 16 + 4 * q + 2] = h.z; xv[i][run * 16 + 4 * q + 3] = h.w;
                }
            }
            if constexpr (U_::NS == 1) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < UE; e++) t += xv[i][e];
                xs[i][0] = t;
            } else if constexpr (U_::NS == 4) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    float z = 0.f;
#pragma unroll
                    for (int e = 0; e < 16; e++) z += xv[i][16 * t + e];
                    xs[i][t] = z;
                }
            }
        }
        auto fn = [&](const uint8_t* row, int u, int i) { return U_::dot(row, u, xv[i], xs[i]); };
        rows_body<UPL, SWIGLU>(seg, pl, rb, fn, un, part_lds);
    }
    __syncthreads();
    finish_group<EPI>(a, pl, seg, part_lds);
}

// Records of a plain vector (op-level calls): one 32-lane half-wavefront per unit.
__global__ __launch_bounds__(64) void make_xrec_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        int n, XRec* __restrict__ out) {
    const int unit = blockIdx.x * 2 + (threadIdx.x >> 5);
    const int e = threadIdx.x & 31;
    const int i = unit * 32 + e;
    const bool ok = i < n;
    const float h = ok ? x[i] : 0.f;
    float v = h;
    if (w && ok) {
#pragma clang fp contract(off)
        v = w[i] * h;
    }
    build_xrec(v, h * h, out + unit, unit * 32 < n);
}

// Generic fallback for F32/F16 weights whose width is not a multiple of 32
// (MatMulF32 with small shapes, TO:437-504): one wavefront per output row.
__global__ __launch_bounds__(WG) void gemv_generic_kernel(const uint8_t* w, uint32_t type, const float* x,
                                                          float* y, int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float s = 0.f;
    for (int k = lane; k < cols; k += 64) {
        const float wv = type == GGML_F32 ? reinterpret_cast<const float*>(w)[(int64_t)r * cols + k]
                                          : h16(reinterpret_cast<const uint16_t*>(w)[(int64_t)r * cols + k]);
        s += wv * x[k];
    }
    s = wave_sum(s);
    if (lane == 0) y[r] = s;
}

template <uint32_t T>
hipError_t launch_t(int epi, const GemvArgs& a, int grid, hipStream_t s) {
    switch (epi) {
    case EPI_STORE: gemv_kernel<T, EPI_STORE><<<grid, WG, 0, s>>>(a); break;
    case EPI_ADD: gemv_kernel<T, EPI_ADD><<<grid, WG, 0, s>>>(a); break;
    case EPI_SWIGLU: gemv_kernel<T, EPI_SWIGLU><<<grid, WG, 0, s>>>(a); break;
    case EPI_ARGMAX: gemv_kernel<T, EPI_ARGMAX><<<grid, WG, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_supported(uint32_t type) {
    return type == GGML_Q4_K || type == GGML_Q5_K || type == GGML_Q6_K || type == GGML_Q8_0 ||
           type == GGML_Q4_0 || type == GGML_F32 || type == GGML_F16;
}

int gemv_unit_elems(uint32_t type) { return type == GGML_Q6_K ? 64 : 32; }

int gemv_max_units(uint32_t type) { return 64 * (type == GGML_Q6_K ? 1 : 2); }

int gemv_groups(int rows) { return (rows + GROUP - 1) / GROUP; }

int gemv_pick_splitk(uint32_t type, int cols, int rows_total) {
    if ((type == GGML_F32 || type == GGML_F16) && cols % 32 != 0) return 1;
    const int U = cols / gemv_unit_elems(type);
    const int groups = gemv_groups(rows_total);
    const int maxu = gemv_max_units(type);
    // the smallest split that fits the per-lane unit budget; then keep
    // splitting (at least one unit per lane) until the grid covers 512 workgroups
    int best = 0;
    for (int s = 1; s <= 32; s++) {
        if (U % s) continue;
        const int per = U / s;
        if (per > maxu) continue;
        if (!best) {
            best = s;
            if (groups * s >= 512) break;
            continue;
        }
        if (per < 64) break;
        best = s;
        if (groups * s >= 512) break;
    }
    return best;
}

int gemv_grid(const GemvArgs& a) {
    int g = 0;
    for (int s = 0; s < a.nseg; s++) g += a.seg[s].groups * a.splitk;
    return g;
}

hipError_t launch_make_xrec(const float* x, const float* w, int n, XRec* out, hipStream_t s) {
    const int units = (n + 31) / 32;
    make_xrec_kernel<<<(units + 1) / 2, 64, 0, s>>>(x, w, n, out);
    return hipGetLastError();
}

hipError_t launch_gemv(uint32_t type, int epi, const GemvArgs& a, hipStream_t s) {
    if (a.cols <= 0) return hipErrorInvalidValue;
    if ((type == GGML_F32 || type == GGML_F16) && (a.cols % 32 != 0)) {
        if (epi != EPI_STORE || a.nseg != 1 || a.norm) return hipErrorInvalidValue;
        gemv_generic_kernel<<<(a.seg[0].rows + 3) / 4, WG, 0, s>>>(a.seg[0].w, type, a.x, a.seg[0].out,
                                                                  a.seg[0].rows, a.cols);
        return hipGetLastError();
    }
    if (!gemv_supported(type) || a.cols % gemv_unit_elems(type) != 0 || a.cols % block_elems(type) != 0)
        return hipErrorInvalidValue;
    const int U = a.cols / gemv_unit_elems(type);
    if (a.splitk < 1 || U % a.splitk != 0 || U / a.splitk > gemv_max_units(type)) return hipErrorInvalidValue;
    if (type == GGML_Q4_K && !a.xrec) return hipErrorInvalidValue;
    if (a.norm && !a.xrec) return hipErrorInvalidValue;
    if (a.splitk > 1 && (!a.partial || !a.counters)) return hipErrorInvalidValue;
    if (epi == EPI_SWIGLU && (a.nseg != 1 || !a.seg[0].w2)) return hipErrorInvalidValue;
    if ((epi == EPI_ADD || epi == EPI_SWIGLU) && a.rec_out && a.nseg != 1) return hipErrorInvalidValue;
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].groups != gemv_groups(a.seg[i].rows)) return hipErrorInvalidValue;
    const int grid = gemv_grid(a);
    if (grid <= 0) return hipSuccess;
    switch (type) {
    case GGML_Q4_K: return launch_t<GGML_Q4_K>(epi, a, grid, s);
    case GGML_Q5_K: return launch_t<GGML_Q5_K>(epi, a, grid, s);
    case GGML_Q6_K: return launch_t<GGML_Q6_K>(epi, a, grid, s);
    case GGML_Q8_0: return launch_t<GGML_Q8_0>(epi, a, grid, s);
    case GGML_Q4_0: return launch_t<GGML_Q4_0>(epi, a, grid, s);
    case GGML_F32: return launch_t<GGML_F32>(epi, a, grid, s);
    case GGML_F16: return launch_t<GGML_F16>(epi, a, grid, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmdot
