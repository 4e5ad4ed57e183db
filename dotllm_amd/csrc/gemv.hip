// gemv.hip -- fused dequant-GEMV over native GGUF blocks (batch 1).
//
// y[r] = sum_k deq(W)[r][k] * x[k]   (TensorOps.MatMul with aRows == 1,
// src/Llmdot.Core/Tensors/TensorOps.cs:60-90, and the fused per-type kernels
// TO:118-431).  The weights are read once, straight from their GGUF blocks.
//
// Work decomposition: a workgroup is 4 wavefronts; each wavefront owns 4
// output rows (2 gate + 2 up rows for the SwiGLU form) and its 64 lanes stride
// over the row in "units" (a sub-block of 32 elements, or 64 for Q6_K).  A
// lane loads the activation slice of its unit once and reuses it for all rows
// of the wavefront, dequantises the unit's bytes in registers and accumulates
// in fp32; rows are then reduced across the wavefront with cross-lane shuffles.
//
// Prologue PRO_RMSNORM fuses RmsNorm (VectorMath.cs:308-340): every workgroup
// reduces sum(x^2) itself and forms x_i = (w_i * h_i) * inv on the fly.
// Epilogues: EPI_STORE, EPI_ADD (residual add, VectorMath.Add VM:27-42),
// EPI_SWIGLU (SiluInPlace(gate) then Mul(gate, up), IE:463-474) and
// EPI_ARGMAX (logits plus ArgMax VM:412-425 via a last-workgroup reduction).
#include "common.h"
#include "kernels.h"

namespace llmdot {

namespace {

constexpr int WG = 256;

__device__ __forceinline__ float h16(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
__device__ __forceinline__ float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sb(uint32_t w, int k) { return (float)(int8_t)(w >> (8 * k)); }

// ---- per-type unit decoders ------------------------------------------------
// Unit u of a row; x points at the unit's UE activations (in the unit's own
// element order); xs holds NS partial sums of x needed by the type's offset.

struct UQ4K {  // reference Q4_K: 144 B / 256; unit = sub-block g (32 elements)
    static constexpr int UE = 32, BE = 256, BB = 144, NS = 1;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }  // 2 runs of 16
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + (u >> 3) * 144;
        const int g = u & 7;
        u32x4 h = ld16_a4(blk);
        u32x4 q = ld16_a4(blk + 16 + 16 * g);
        float d = h16(h.x & 0xFFFFu), dm = h16(h.x >> 16);
        uint64_t lo = (uint64_t)h.y | ((uint64_t)h.z << 32), hi = (uint64_t)h.z | ((uint64_t)h.w << 32);
        uint32_t f = g < 5 ? (uint32_t)(lo >> (12 * g)) : (uint32_t)(hi >> (12 * g - 32));
        float sc = (float)(f & 63u), m = (float)((f >> 6) & 63u);
        uint32_t w[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t e = w[j] & 0x0F0F0F0Fu, o = (w[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x[8 * j + 2 * k] * ub(e, k);
                s1 += x[8 * j + 2 * k + 1] * ub(o, k);
            }
        }
        return (d * sc) * ((s0 + s1) - 8.f * xs[0]) - (dm * m) * xs[0];
    }
};

struct UQ5K {  // reference Q5_K: 176 B / 256; unit = sub-block g
    static constexpr int UE = 32, BE = 256, BB = 176, NS = 1;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + (u >> 3) * 176;
        const int g = u & 7;
        u32x4 h = ld16_a4(blk);
        uint32_t qh = ld4_a4(blk + 16 + 4 * g);
        u32x4 q = ld16_a4(blk + 48 + 16 * g);
        float d = h16(h.x & 0xFFFFu), dm = h16(h.x >> 16);
        uint64_t lo = (uint64_t)h.y | ((uint64_t)h.z << 32), hi = (uint64_t)h.z | ((uint64_t)h.w << 32);
        uint32_t f = g < 5 ? (uint32_t)(lo >> (12 * g)) : (uint32_t)(hi >> (12 * g - 32));
        float sc = (float)(f & 63u), m = (float)((f >> 6) & 63u);
        uint32_t w[4] = {q.x, q.y, q.z, q.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t hb = qh >> (8 * j);
            // bits 0,2,4,6 of hb -> bit 4 of bytes 0..3 (even elements), bits 1,3,5,7 -> odd
            uint32_t he = (((hb & 0x55u) * 0x410410u) & 0x10101010u);
            uint32_t ho = ((((hb >> 1) & 0x55u) * 0x410410u) & 0x10101010u);
            uint32_t e = (w[j] & 0x0F0F0F0Fu) | he, o = ((w[j] >> 4) & 0x0F0F0F0Fu) | ho;
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
    static constexpr int UE = 64, BE = 256, BB = 210, NS = 4;
    // run t (0..3) of 16 elements: n + l0 + 32 t + [0, 16)
    __device__ static int xoff(int u, int t) {
        int sub = u & 3;
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
        float d = h16(Dw[0] & 0xFFFFu);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t q0 = (A[j] & 0x0F0F0F0Fu) | ((C[j] & 0x03030303u) << 4);
            uint32_t q1 = (B[j] & 0x0F0F0F0Fu) | ((C[j] & 0x0C0C0C0Cu) << 2);
            uint32_t q2 = ((A[j] >> 4) & 0x0F0F0F0Fu) | (C[j] & 0x30303030u);
            uint32_t q3 = ((B[j] >> 4) & 0x0F0F0F0Fu) | ((C[j] >> 2) & 0x30303030u);
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
        for (int t = 0; t < 4; t++) {
            float sc = sb(S[t >> 1], 2 * (t & 1));
            r += (d * sc) * (s[t] - 32.f * xs[t]);
        }
        return r;
    }
};

struct UQ8_0 {  // Q8_0: 34 B / 32; unit = block
    static constexpr int UE = 32, BE = 32, BB = 34, NS = 0;
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
    static constexpr int UE = 32, BE = 32, BB = 18, NS = 1;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float* xs) {
        const uint8_t* blk = row + u * 18;
        uint32_t Dw[1], Q[4];
        ld_realign<1>(blk, Dw);
        ld_realign<4>(blk + 2, Q);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t lo = Q[j] & 0x0F0F0F0Fu, hi = (Q[j] >> 4) & 0x0F0F0F0Fu;
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
    static constexpr int UE = 32, BE = 1, BB = 4, NS = 0;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float*) {
        const float4* p = reinterpret_cast<const float4*>(row + (int64_t)u * 128);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            float4 a = p[j], b = p[j + 1];
            s0 += x[4 * j] * a.x + x[4 * j + 1] * a.y + x[4 * j + 2] * a.z + x[4 * j + 3] * a.w;
            s1 += x[4 * j + 4] * b.x + x[4 * j + 5] * b.y + x[4 * j + 6] * b.z + x[4 * j + 7] * b.w;
        }
        return s0 + s1;
    }
};

struct UF16 {
    static constexpr int UE = 32, BE = 1, BB = 2, NS = 0;
    __device__ static int xoff(int u, int run) { return u * 32 + run * 16; }
    __device__ static float dot(const uint8_t* row, int u, const float* x, const float*) {
        const uint8_t* p = row + (int64_t)u * 64;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            u32x4 v = ld16_a4(p + 16 * j);
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; k++)
                s += x[8 * j + 2 * k] * h16(w[k] & 0xFFFFu) + x[8 * j + 2 * k + 1] * h16(w[k] >> 16);
        }
        return s;
    }
};

template <uint32_t T> struct UnitOf;
template <> struct UnitOf<GGML_Q4_K> { using type = UQ4K; };
template <> struct UnitOf<GGML_Q5_K> { using type = UQ5K; };
template <> struct UnitOf<GGML_Q6_K> { using type = UQ6K; };
template <> struct UnitOf<GGML_Q8_0> { using type = UQ8_0; };
template <> struct UnitOf<GGML_Q4_0> { using type = UQ4_0; };
template <> struct UnitOf<GGML_F32> { using type = UF32; };
template <> struct UnitOf<GGML_F16> { using type = UF16; };

// sum(h^2) over n with all 256 threads; returns 1 / sqrt(ss / n + eps) to every thread.
__device__ float block_rms_inv(const float* __restrict__ h, int n, float eps, float* red) {
#pragma clang fp contract(off)
    float ss = 0.f;
    const int n4 = n >> 2;
    const float4* h4 = reinterpret_cast<const float4*>(h);
    for (int i = threadIdx.x; i < n4; i += WG) {
        float4 v = h4[i];
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int i = n4 * 4 + threadIdx.x; i < n; i += WG) ss += h[i] * h[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return (1.0f / (sqrtf(((ss / (float)n) + eps))));
}

// x element i for the prologue in use.
template <int PRO>
__device__ __forceinline__ float4 xload4(const GemvArgs& a, int i, float inv, int n8) {
#pragma clang fp contract(off)
    float4 h = *reinterpret_cast<const float4*>(a.x + i);
    if (PRO == PRO_NONE) return h;
    float4 w = *reinterpret_cast<const float4*>(a.norm_w + i);
    float4 r;
    if (i + 4 <= n8) {  // Vector<float> part: (w * x) * inv
        r.x = ((w.x * h.x) * inv); r.y = ((w.y * h.y) * inv);
        r.z = ((w.z * h.z) * inv); r.w = ((w.w * h.w) * inv);
    } else {            // scalar tail: w * (x * inv)
        r.x = (w.x * (h.x * inv)); r.y = (w.y * (h.y * inv));
        r.z = (w.z * (h.z * inv)); r.w = (w.w * (h.w * inv));
    }
    return r;
}

template <uint32_t T, int PRO, int EPI>
__global__ __launch_bounds__(WG) void gemv_kernel(GemvArgs a) {
    using U = typename UnitOf<T>::type;
    constexpr int ROWS_WAVE = (EPI == EPI_SWIGLU) ? 2 : 4;
    constexpr int ROWS_WG = 4 * ROWS_WAVE;
    __shared__ float red[8];
    __shared__ float am_val[4];
    __shared__ int am_idx[4];
    __shared__ int am_last;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = a.cols;
    const int nunits = cols / U::UE;
    const int64_t rb = (int64_t)(cols / U::BE) * U::BB;

    int b = blockIdx.x, s = 0;
    for (; s < a.nseg - 1; s++) {
        int nb = (a.seg[s].rows + ROWS_WG - 1) / ROWS_WG;
        if (b < nb) break;
        b -= nb;
    }
    const GemvSeg seg = a.seg[s];
    const int row0 = b * ROWS_WG + wave * ROWS_WAVE;

    float inv = 1.f;
    if (PRO == PRO_RMSNORM) inv = block_rms_inv(a.x, cols, a.eps, red);
    const int n8 = cols & ~7;

    const uint8_t* wrow[4];
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int rr = (EPI == EPI_SWIGLU) ? row0 + (r & 1) : row0 + r;
        const uint8_t* base = (EPI == EPI_SWIGLU && r >= 2) ? a.seg[1].w : seg.w;
        valid[r] = rr < seg.rows;
        wrow[r] = base + (int64_t)(valid[r] ? rr : 0) * rb;
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid[0]) {
        for (int u = lane; u < nunits; u += 64) {
            float xv[U::UE];
            float xs[U::NS > 0 ? U::NS : 1];
#pragma unroll
            for (int run = 0; run < U::UE / 16; run++) {
                const int off = U::xoff(u, run);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 v = xload4<PRO>(a, off + 4 * q, inv, n8);
                    xv[run * 16 + 4 * q] = v.x; xv[run * 16 + 4 * q + 1] = v.y;
                    xv[run * 16 + 4 * q + 2] = v.z; xv[run * 16 + 4 * q + 3] = v.w;
                }
            }
            if (U::NS == 1) {
                float t = 0.f;
#pragma unroll
                for (int i = 0; i < U::UE; i++) t += xv[i];
                xs[0] = t;
            } else if (U::NS == 4) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    float z = 0.f;
#pragma unroll
                    for (int i = 0; i < 16; i++) z += xv[16 * t + i];
                    xs[t] = z;
                }
            }
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] += U::dot(wrow[r], u, xv, xs);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = wave_sum(acc[r]);

    if (EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_ARGMAX) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (lane == r && valid[r]) {
                float* o = seg.out + row0 + r;
                *o = (EPI == EPI_ADD) ? (*o + acc[r]) : acc[r];
            }
        }
    } else {  // EPI_SWIGLU
        const int f8 = seg.rows & ~7;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            if (lane == r && valid[r]) {
                const int rr = row0 + r;
                float g = acc[r], up = acc[r + 2];
                float sg = rr < f8 ? silu_ref(g) : (g / (1.0f + expf(-g)));
                seg.out[rr] = (sg * up);
            }
        }
    }

    if (EPI == EPI_ARGMAX) {
        // first index of the strict maximum over this workgroup's rows
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int r = 0; r < 4; r++)
            if (valid[r] && (acc[r] > bv)) { bv = acc[r]; bi = row0 + r; }
        if (lane == 0) { am_val[wave] = bv; am_idx[wave] = bi; }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v = am_val[0];
            int i = am_idx[0];
            for (int w = 1; w < 4; w++)
                if (am_val[w] > v || (am_val[w] == v && am_idx[w] < i)) { v = am_val[w]; i = am_idx[w]; }
            a.am.cand_val[blockIdx.x] = v;
            a.am.cand_idx[blockIdx.x] = i;
            __threadfence();
            unsigned prev = atomicAdd(a.am.counter, 1u);
            am_last = (prev == gridDim.x - 1);
        }
        __syncthreads();
        if (am_last) {
            __threadfence();
            float v = -INFINITY;
            int i = 0x7FFFFFFF;
            for (int c = threadIdx.x; c < (int)gridDim.x; c += WG) {
                float cv = __builtin_nontemporal_load(a.am.cand_val + c);
                int ci = __builtin_nontemporal_load(a.am.cand_idx + c);
                if (cv > v || (cv == v && ci < i)) { v = cv; i = ci; }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                float ov = __shfl_xor(v, o, 64);
                int oi = __shfl_xor(i, o, 64);
                if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
            }
            if (lane == 0) { am_val[wave] = v; am_idx[wave] = i; }
            __syncthreads();
            if (threadIdx.x == 0) {
                v = am_val[0]; i = am_idx[0];
                for (int w = 1; w < 4; w++)
                    if (am_val[w] > v || (am_val[w] == v && am_idx[w] < i)) { v = am_val[w]; i = am_idx[w]; }
                if (i == 0x7FFFFFFF) i = 0;  // all NaN: ArgMax returns 0
                *a.am.token_out = i;
                if (a.am.token_log && *a.am.step >= 0 && *a.am.step < a.am.log_cap) a.am.token_log[*a.am.step] = i;
                if (a.am.step) *a.am.step += 1;
                if (a.am.pos) *a.am.pos += 1;
                *a.am.counter = 0u;
            }
        }
    }
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
        float wv = type == GGML_F32 ? reinterpret_cast<const float*>(w)[(int64_t)r * cols + k]
                                    : h16(reinterpret_cast<const uint16_t*>(w)[(int64_t)r * cols + k]);
        s += wv * x[k];
    }
    s = wave_sum(s);
    if (lane == 0) y[r] = s;
}

template <uint32_t T>
hipError_t launch_t(int pro, int epi, const GemvArgs& a, int grid, hipStream_t s) {
#define L(P, E) gemv_kernel<T, P, E><<<grid, WG, 0, s>>>(a)
    if (pro == PRO_NONE) {
        if (epi == EPI_STORE) L(PRO_NONE, EPI_STORE);
        else if (epi == EPI_ADD) L(PRO_NONE, EPI_ADD);
        else return hipErrorInvalidValue;
    } else {
        if (epi == EPI_STORE) L(PRO_RMSNORM, EPI_STORE);
        else if (epi == EPI_SWIGLU) L(PRO_RMSNORM, EPI_SWIGLU);
        else if (epi == EPI_ARGMAX) L(PRO_RMSNORM, EPI_ARGMAX);
        else return hipErrorInvalidValue;
    }
#undef L
    return hipGetLastError();
}

int unit_elems(uint32_t type) { return type == GGML_Q6_K ? 64 : 32; }

}  // namespace

bool gemv_supported(uint32_t type) {
    return type == GGML_Q4_K || type == GGML_Q5_K || type == GGML_Q6_K || type == GGML_Q8_0 ||
           type == GGML_Q4_0 || type == GGML_F32 || type == GGML_F16;
}

int gemv_grid(uint32_t type, int epi, const GemvArgs& a) {
    const int rows_wg = epi == EPI_SWIGLU ? 8 : 16;
    if (epi == EPI_SWIGLU) return (a.seg[0].rows + rows_wg - 1) / rows_wg;
    int g = 0;
    for (int s = 0; s < a.nseg; s++) g += (a.seg[s].rows + rows_wg - 1) / rows_wg;
    return g;
}

hipError_t launch_gemv(uint32_t type, int pro, int epi, const GemvArgs& a, hipStream_t s) {
    if (a.cols <= 0) return hipErrorInvalidValue;
    if ((type == GGML_F32 || type == GGML_F16) && (a.cols % 32 != 0)) {
        if (pro != PRO_NONE || epi != EPI_STORE || a.nseg != 1) return hipErrorInvalidValue;
        gemv_generic_kernel<<<(a.seg[0].rows + 3) / 4, WG, 0, s>>>(a.seg[0].w, type, a.x, a.seg[0].out,
                                                                  a.seg[0].rows, a.cols);
        return hipGetLastError();
    }
    if (a.cols % unit_elems(type) != 0 || a.cols % block_elems(type) != 0) return hipErrorInvalidValue;
    if (epi == EPI_SWIGLU && (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows)) return hipErrorInvalidValue;
    const int grid = gemv_grid(type, epi, a);
    if (grid <= 0) return hipSuccess;
    switch (type) {
    case GGML_Q4_K: return launch_t<GGML_Q4_K>(pro, epi, a, grid, s);
    case GGML_Q5_K: return launch_t<GGML_Q5_K>(pro, epi, a, grid, s);
    case GGML_Q6_K: return launch_t<GGML_Q6_K>(pro, epi, a, grid, s);
    case GGML_Q8_0: return launch_t<GGML_Q8_0>(pro, epi, a, grid, s);
    case GGML_Q4_0: return launch_t<GGML_Q4_0>(pro, epi, a, grid, s);
    case GGML_F32: return launch_t<GGML_F32>(pro, epi, a, grid, s);
    case GGML_F16: return launch_t<GGML_F16>(pro, epi, a, grid, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmdot
