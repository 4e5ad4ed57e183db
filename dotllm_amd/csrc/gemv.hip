// gemv.hip -- fused dequant-GEMV over native GGUF blocks (batch 1).
//
// y[r] = sum_k deq(W)[r][k] * x[k]   (TensorOps.MatMul with aRows == 1,
// src/Llmdot.Core/Tensors/TensorOps.cs:60-90, fused per-type kernels TO:118-431).
// The weight blocks are read once from HBM in their GGUF layout.
//
// Decomposition.  A workgroup owns a few output rows (slabs of 2 to 8
// consecutive rows, interleaved across the workgroups) and the whole
// reduction dimension.  It has ceil(U/64) wavefronts, U being the number of
// 32-element "units" of a row, and lane L of wavefront w owns unit 64w + L in
// every row, so a lane's activations are loaded once and stay in registers
// while the rows stream through.  Rows go in batches (2 to 8 rows by type, half
// gate and half up rows for the SwiGLU form); the loads of batch b+1 are
// issued before batch b is computed, so every wavefront keeps two batches of
// loads in flight.  One launch may cover up to three matrices (segments),
// e.g. Q, K and V, also of two types with equal batch geometry (Q4_K + Q6_K).  A row's lane partials are summed over 16-lane rows with
// DPP rotations, then over quarter-wavefronts and wavefronts through LDS, in a
// fixed order.  The loads carry no branches (lanes past the end of a row read
// unit 0 and contribute 0), so the compiler keeps them all in flight.  Workgroups
// do not communicate (no fences or atomics).
//
// Arithmetic.  Q4_K (the reference's own layout) runs on v_dot8_i32_i4.  Each
// lane quantises its 32 activations v (times the norm weight) to 24 bits,
// X = rint(v / s) with s = max|v| / 4194000, and splits X into six signed-nibble
// planes: X + 0x888888 has the digits t_p + 8, so the planes hold t_p directly
// after an XOR with 8 (X = sum_p 16^p t_p).  The weight nibble ^ 8 is q - 8 as
// an int4, so six dot8 per 8 elements give the plane sums exactly in int32; the
// sub-block result is (d*sc) * s * S - (dmin*m) * sum(v).  The quantisation
// error is at most s/2 = 1.2e-7 max|v| per element, the size of fp32 rounding.  The other types dequantise in registers
// and accumulate in fp32.  RmsNorm of the input (VectorMath.RmsNorm,
// VM:308-340) is folded in: the lanes multiply by the norm weight, the
// workgroup reduces sum(h^2), and each row sum is scaled by 1/rms at the end.
//
// Epilogues: STORE; ADD (residual h += y, VectorMath.Add VM:27-42); SWIGLU
// (SiluInPlace(gate) * up, IE:463-474, VM:118-135); ARGMAX (logits plus
// ArgMax VM:412-425: one candidate per workgroup, reduced by a second launch).
#include "common.h"
#include "kernels.h"

#include <stdlib.h>
#include <string.h>

#include <type_traits>

namespace llmdot {

namespace {

constexpr int MAXW = 8;   // wavefronts per workgroup: U <= 512 units

__device__ __forceinline__ float h16(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
__device__ __forceinline__ float ub(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }
__device__ __forceinline__ float sb(uint32_t w, int k) { return (float)(int8_t)(w >> (8 * k)); }

// fp16 value at a 2-byte-aligned address (it never straddles a dword).
__device__ __forceinline__ uint32_t ld_h16_bits(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
    return (w >> (8 * (a & 2))) & 0xFFFFu;
}

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

struct __attribute__((aligned(4))) u32x3 { uint32_t x, y, z; };

// Dword-aligned raw words covering [p, p + 4N) for a 2-byte-aligned p;
// word i of the span is (*this)[i].
template <int N>
struct RawW {
    uint32_t w[N + 1];
    uint32_t sh;
    __device__ __forceinline__ void load(const uint8_t* p) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
        sh = (uint32_t)(a & 3u);
        if constexpr (N + 1 == 3) {
            const u32x3 v = *reinterpret_cast<const u32x3*>(base);
            w[0] = v.x; w[1] = v.y; w[2] = v.z;
        } else {
#pragma unroll
            for (int i = 0; i + 4 <= N + 1; i += 4) {
                const u32x4 v = ld16_a4(base + 4 * i);
                w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
            }
#pragma unroll
            for (int i = ((N + 1) / 4) * 4; i < N + 1; i++) w[i] = ld4_a4(base + 4 * i);
        }
    }
    __device__ __forceinline__ uint32_t operator[](int i) const { return __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh); }
};

// ---- activations of one lane -----------------------------------------------------

constexpr int XQ_PLANES = 6;            // 24-bit activations
constexpr float XQ_MAX = 4194000.0f;    // |X| < 2^22: exact rint by the 1.5 * 2^23 constant

struct XQ {            // Q4_K path
    uint32_t pl[4 * XQ_PLANES];   // pl[4p + j]: nibble k = digit p of X[8j + k] as a signed int4
    float s, sum;                 // v ~= s * X;  sum = sum(v)
};

// Byte b of Y[0], Y[2], Y[4], Y[6] (or of the odd elements) in one dword.
__device__ __forceinline__ uint32_t gather_bytes(uint32_t y0, uint32_t y2, uint32_t y4, uint32_t y6, int b) {
    const uint32_t sel = b == 0 ? 0x0C0C0400u : (b == 1 ? 0x0C0C0501u : 0x0C0C0602u);
    const uint32_t lo = __builtin_amdgcn_perm(y2, y0, sel);   // [y0.b, y2.b, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(y6, y4, sel);   // [y4.b, y6.b, 0, 0]
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);        // [y0.b, y2.b, y4.b, y6.b]
}

__device__ __forceinline__ void quantize32(const float* v, XQ& q) {
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    const float scale = amax > 0.f ? XQ_MAX / amax : 0.f;
    q.s = amax > 0.f ? amax / XQ_MAX : 0.f;
    q.sum = sum;
    uint32_t Y[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        // rint through the 1.5 * 2^23 constant: the low 23 bits of the sum hold
        // 2^22 + X, so Y = X + 0x888888 lies in [0, 2^24) with digits t_p + 8.
        const float f = v[i] * scale + 12582912.0f;
        Y[i] = __float_as_uint(f) - (0x4B400000u - 0x888888u);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t* y = Y + 8 * j;
#pragma unroll
        for (int b = 0; b < 3; b++) {   // byte b of Y holds digits 2b (low nibble) and 2b + 1
            const uint32_t E = gather_bytes(y[0], y[2], y[4], y[6], b);
            const uint32_t O = gather_bytes(y[1], y[3], y[5], y[7], b);
            const uint32_t m = 0x0F0F0F0Fu;
            q.pl[4 * (2 * b) + j] = ((E & m) | ((O << 4) & ~m)) ^ 0x88888888u;
            q.pl[4 * (2 * b + 1) + j] = (((E >> 4) & m) | (O & ~m)) ^ 0x88888888u;
        }
    }
}

// Q8_0 path: the same 24-bit X as three signed byte digits, X = 65536 d2 +
// 256 d1 + d0 (X + 0x808080 has the bytes d_p + 128), so v_dot4_i32_i8 takes
// the int8 weights against each digit plane.
struct XB {
    uint32_t pl[4 * XQ_PLANES];   // pl[8p + j]: byte k = digit p of X[4j + k] as a signed int8
    float s, sum;                 // v ~= s * X;  sum = sum(v)
};

__device__ __forceinline__ void quantize32_b(const float* v, XB& q) {
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    const float scale = amax > 0.f ? XQ_MAX / amax : 0.f;
    q.s = amax > 0.f ? amax / XQ_MAX : 0.f;
    q.sum = sum;
    uint32_t Y[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {   // as quantize32, with Y = X + 0x808080
        const float f = v[i] * scale + 12582912.0f;
        Y[i] = __float_as_uint(f) - (0x4B400000u - 0x808080u);
    }
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int b = 0; b < 3; b++)
            q.pl[8 * b + j] = gather_bytes(Y[4 * j], Y[4 * j + 1], Y[4 * j + 2], Y[4 * j + 3], b) ^ 0x80808080u;
}

// fp32 path: the unit's 32 activations in its element order, and the sums
// its offsets need.
template <int NS>
struct XF {
    float v[32];
    float s[NS];
};

// ---- per-type row units -----------------------------------------------------------
// RUN: contiguous elements per run of a unit; xoff(u, run) its first element.

struct TQ4K {   // reference Q4_K, 144 B / 256: unit = sub-block g
    // 4 rows per batch keep the kernel near 100 VGPRs (4 wavefronts per SIMD)
    static constexpr int RB = 4, PRE = 2, DEPTH = 2;
    // h: the 16-byte block header (d | dmin << 16, then the 96-bit 6-bit
    // (sc, m) stream), one load shared by the block's 8 lanes; q: the
    // sub-block's 16 nibble bytes.
    struct Raw { u32x4 h; u32x4 q; };
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * 144;
        r.h = ld16_a4(blk);
        r.q = ld16_a4(blk + 16 + 16 * (u & 7));
    }
    __device__ static float dot(const Raw& r, int u, const XQ& x) {
        const uint32_t w[4] = {r.q.x ^ 0x88888888u, r.q.y ^ 0x88888888u, r.q.z ^ 0x88888888u, r.q.w ^ 0x88888888u};
        // S = sum (q-8) X = sum_p 16^p a_p by Horner over the planes.  |S| <=
        // 32 * 8 * 4194000 < 2^31, and int32 wrap-around is exact modulo 2^32,
        // so the result is exact whatever the intermediate values.
        int acc = 0;
#pragma unroll
        for (int p = XQ_PLANES - 1; p >= 0; p--) {
            if (p < XQ_PLANES - 1) acc <<= 4;
#pragma unroll
            for (int j = 0; j < 4; j++) acc = __builtin_amdgcn_sdot8((int)w[j], (int)x.pl[4 * p + j], acc, false);
        }
        const float S = (float)acc;
        float sc, m;
        kscale(r.h.y, r.h.z, r.h.w, u & 7, sc, m);
        const float d = h16(r.h.x & 0xFFFFu), dm = h16(r.h.x >> 16);
        return (d * sc) * (x.s * S) - (dm * m) * x.sum;
    }
};

struct TQ5K {   // reference Q5_K, 176 B / 256: unit = sub-block g
    static constexpr int RB = 8, NS = 1, RUN = 32, PRE = 2, DEPTH = 2;
    struct Raw { u32x4 h, q; uint32_t qh; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * 176;
        const int g = u & 7;
        r.h = ld16_a4(blk);
        r.qh = ld4_a4(blk + 16 + 4 * g);
        r.q = ld16_a4(blk + 48 + 16 * g);
    }
    __device__ static float dot(const Raw& r, int u, const XF<NS>& x) {
        float sc, m;
        kscale(r.h.y, r.h.z, r.h.w, u & 7, sc, m);
        const float d = h16(r.h.x & 0xFFFFu), dm = h16(r.h.x >> 16);
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t hb = r.qh >> (8 * j);
            // bits 0,2,4,6 of hb -> bit 4 of bytes 0..3 (even elements), bits 1,3,5,7 -> odd
            const uint32_t he = ((hb & 0x55u) * 0x410410u) & 0x10101010u;
            const uint32_t ho = (((hb >> 1) & 0x55u) * 0x410410u) & 0x10101010u;
            const uint32_t e = (w[j] & 0x0F0F0F0Fu) | he, o = ((w[j] >> 4) & 0x0F0F0F0Fu) | ho;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x.v[8 * j + 2 * k] * ub(e, k);
                s1 += x.v[8 * j + 2 * k + 1] * ub(o, k);
            }
        }
        return (d * sc) * ((s0 + s1) - 16.f * x.s[0]) - (dm * m) * x.s[0];
    }
};

// Q6_K, 210 B / 256 (ql[128], qh[64], sc[16], d).  Unit u of a block: half
// n = 128 ((u >> 2) & 1), l-range l0 = 8 (u & 3) .. l0 + 7, four runs t = 0..3 of 8
// elements at n + l0 + 32 t (the q1..q4 groups of the reference loop).
struct TQ6K {
    static constexpr int RB = 4, NS = 4, RUN = 8, PRE = 1, DEPTH = 2;   // PRE: batches issued before the activations' arithmetic
    // A, B: ql bytes of runs 0/2 and 1/3; C: qh bytes; S: scales.  A, B, C sit
    // at multiples of 8 from the 2-aligned block start and share one shift.
    struct Raw { uint32_t A[3], B[3], C[3], S[3], d, sh; };
    __device__ static int xoff(int u, int t) { return (u >> 3) * 256 + ((u >> 2) & 1) * 128 + (u & 3) * 8 + 32 * t; }
    __device__ static void ld3(uint32_t* w, const uint8_t* p) {
        const u32x3 v = *reinterpret_cast<const u32x3*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t(3));
        w[0] = v.x; w[1] = v.y; w[2] = v.z;
    }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * 210;
        const int half = (u >> 2) & 1, l0 = (u & 3) * 8;
        const uint8_t* ps = blk + 192 + 8 * half + (l0 >> 4);
        ld3(r.A, blk + 64 * half + l0);
        ld3(r.B, blk + 64 * half + l0 + 32);
        ld3(r.C, blk + 128 + 32 * half + l0);
        ld3(r.S, ps);
        r.d = ld_h16_bits(blk + 208);
        r.sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u) | ((uint32_t)(reinterpret_cast<uintptr_t>(ps) & 3u) << 8);
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        const float d = h16(r.d);
        const uint32_t sa = r.sh & 3u, ss = r.sh >> 8;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t A = __builtin_amdgcn_alignbyte(r.A[j + 1], r.A[j], sa);
            const uint32_t B = __builtin_amdgcn_alignbyte(r.B[j + 1], r.B[j], sa);
            const uint32_t C = __builtin_amdgcn_alignbyte(r.C[j + 1], r.C[j], sa);
            const uint32_t q0 = (A & 0x0F0F0F0Fu) | ((C & 0x03030303u) << 4);
            const uint32_t q1 = (B & 0x0F0F0F0Fu) | ((C & 0x0C0C0C0Cu) << 2);
            const uint32_t q2 = ((A >> 4) & 0x0F0F0F0Fu) | (C & 0x30303030u);
            const uint32_t q3 = ((B >> 4) & 0x0F0F0F0Fu) | ((C >> 2) & 0x30303030u);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s[0] += x.v[0 * 8 + 4 * j + k] * ub(q0, k);
                s[1] += x.v[1 * 8 + 4 * j + k] * ub(q1, k);
                s[2] += x.v[2 * 8 + 4 * j + k] * ub(q2, k);
                s[3] += x.v[3 * 8 + 4 * j + k] * ub(q3, k);
            }
        }
        const uint32_t S0 = __builtin_amdgcn_alignbyte(r.S[1], r.S[0], ss);
        const uint32_t S1 = __builtin_amdgcn_alignbyte(r.S[2], r.S[1], ss);
        const uint32_t S[2] = {S0, S1};
        float res = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++) res += (d * sb(S[t >> 1], 2 * (t & 1))) * (s[t] - 32.f * x.s[t]);
        return res;
    }
};

// Reference Q2_K, 84 B / 256 (DequantizeK.cs:8-41): unit = 32 elements, two
// sub-blocks of 16 with a (scale, min) byte pair each (low nibbles, bytes 4 +
// 4 (u & 7) ..), 2-bit q at byte 20 + 8 (u & 7) + e / 4, shift 2 (e % 4).
// value = d sc (q - 1/2) - dmin mi.  Blocks and rows are 4-byte aligned.
struct TQ2K {
    static constexpr int RB = 8, NS = 2, RUN = 32, PRE = 2, DEPTH = 2;
    struct Raw { uint32_t h, s, q0, q1; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * 84;
        const int g = u & 7;
        r.h = ld4_a4(blk);
        r.s = ld4_a4(blk + 4 + 4 * g);
        r.q0 = ld4_a4(blk + 20 + 8 * g);
        r.q1 = ld4_a4(blk + 24 + 8 * g);
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        const uint32_t Q[2] = {r.q0, r.q1};
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t qt = (Q[h] >> (2 * t)) & 0x03030303u;   // byte k: element 16 h + 4 k + t
#pragma unroll
                for (int k = 0; k < 4; k++) s[h] += x.v[16 * h + 4 * k + t] * ub(qt, k);
            }
        const float d = h16(r.h & 0xFFFFu), dm = h16(r.h >> 16);
        const float sc0 = (float)(r.s & 15u), mi0 = (float)((r.s >> 8) & 15u);
        const float sc1 = (float)((r.s >> 16) & 15u), mi1 = (float)((r.s >> 24) & 15u);
        return ((d * sc0) * (s[0] - 0.5f * x.s[0]) - (dm * mi0) * x.s[0]) +
               ((d * sc1) * (s[1] - 0.5f * x.s[1]) - (dm * mi1) * x.s[1]);
    }
};

// Reference Q3_K, 110 B / 256 (DequantizeK.cs:43-74, TensorOps.cs:331-362):
// unit = 32 elements, two groups of 16 whose 6-bit scales sit at bits 12 (u & 7)
// and 12 (u & 7) + 6 of the stream from byte 4; the high-bit mask at byte 16 +
// 4 (u & 7) (bit e), 2-bit q at byte 48 + 8 (u & 7) + e / 4.  value = q - 4 m,
// scaled by d sc.  The q field of unit 7 ends 2 bytes past the block, in the
// next block (as the reference reads it) or, for the tensor's last block, in
// the device buffer's zero padding.  Blocks are 2-byte aligned.
struct TQ3K {
    static constexpr int RB = 4, NS = 2, RUN = 32, PRE = 2, DEPTH = 2;
    struct Raw { RawW<4> H; RawW<1> M; RawW<2> Q; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + (u >> 3) * 110;
        const int g = u & 7;
        r.H.load(blk);
        r.M.load(blk + 16 + 4 * g);
        r.Q.load(blk + 48 + 8 * g);
    }
    __device__ static float dot(const Raw& r, int u, const XF<NS>& x) {
        float sc0, sc1;
        kscale(r.H[1], r.H[2], r.H[3], u & 7, sc0, sc1);
        const float d = h16(r.H[0] & 0xFFFFu);
        const uint32_t M = r.M[0];
        const uint32_t Q[2] = {r.Q[0], r.Q[1]};
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int k = 0; k < 4; k++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int e = 16 * h + 4 * k + t;
                    const int q = (int)((Q[h] >> (8 * k + 2 * t)) & 3u);
                    const int m = (int)((M >> e) & 1u);
                    s[h] += x.v[e] * (float)(q - (m << 2));
                }
        return d * (sc0 * s[0] + sc1 * s[1]);
    }
};

struct TQ8_0 {   // Q8_0, 34 B / 32: unit = block; int8 weights on v_dot4_i32_i8
    static constexpr int RB = 4, PRE = 2, DEPTH = 2;
    struct Raw { RawW<8> Q; uint32_t d; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + u * 34;
        r.d = ld_h16_bits(blk);
        r.Q.load(blk + 2);
    }
    __device__ static float dot(const Raw& r, int, const XB& x) {
        // S = sum q X exactly in two int32 parts: the top two digits by Horner
        // (|hi| <= 32 * 128 * (64 * 256 + 128) < 2^27), the low digit apart
        // (|lo| <= 2^19); S = 256 hi + lo in fp32.
        int hi = 0, lo = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) hi = __builtin_amdgcn_sdot4((int)r.Q[j], (int)x.pl[16 + j], hi, false);
        hi <<= 8;
#pragma unroll
        for (int j = 0; j < 8; j++) hi = __builtin_amdgcn_sdot4((int)r.Q[j], (int)x.pl[8 + j], hi, false);
#pragma unroll
        for (int j = 0; j < 8; j++) lo = __builtin_amdgcn_sdot4((int)r.Q[j], (int)x.pl[j], lo, false);
        const float S = (float)hi * 256.0f + (float)lo;
        return h16(r.d) * (x.s * S);
    }
};

struct TQ4_0 {   // Q4_0, 18 B / 32: unit = block; low nibbles -> j, high -> j + 16
    static constexpr int RB = 8, NS = 1, RUN = 32, PRE = 1, DEPTH = 2;
    struct Raw { RawW<4> Q; uint32_t d; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + u * 18;
        r.d = ld_h16_bits(blk);
        r.Q.load(blk + 2);
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t q = r.Q[j];
            const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x.v[4 * j + k] * ub(lo, k);
                s1 += x.v[16 + 4 * j + k] * ub(hi, k);
            }
        }
        return h16(r.d) * ((s0 + s1) - 8.f * x.s[0]);
    }
};

// Q4_1 (20 B / 32): d, m, 16 nibble bytes (low -> j, high -> j + 16); d q + m
// (TO:586-603, reached through MatMul's dequantise-then-dot path TO:92-111).
struct TQ4_1 {
    static constexpr int RB = 8, NS = 1, RUN = 32, PRE = 1, DEPTH = 2;
    struct Raw { u32x4 Q; uint32_t h; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* blk = row + u * 20;   // 4-byte aligned (20-byte blocks, 4-aligned rows)
        r.h = ld4_a4(blk);
        r.Q = ld16_a4(blk + 4);
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        const uint32_t q[4] = {r.Q.x, r.Q.y, r.Q.z, r.Q.w};
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t lo = q[j] & 0x0F0F0F0Fu, hi = (q[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x.v[4 * j + k] * ub(lo, k);
                s1 += x.v[16 + 4 * j + k] * ub(hi, k);
            }
        }
        return h16(r.h & 0xFFFFu) * (s0 + s1) + h16(r.h >> 16) * x.s[0];
    }
};

// Q5_0 (22 B / 32, 2-byte aligned) and Q5_1 (24 B / 32): d [, m], the 32 high
// bits qh, 16 nibble bytes; element j < 16 is (nibble | bit j of qh << 4),
// j + 16 the high nibble with bit j + 16; Q5_0: d (x - 16), Q5_1: d x + m
// (TO:604-641).
template <bool ONE>
struct TQ5_01 {
    static constexpr int BB = ONE ? 24 : 22, OQ = ONE ? 8 : 6, OH = ONE ? 4 : 2;
    static constexpr int RB = 8, NS = 1, RUN = 32, PRE = 1, DEPTH = 2;
    struct Raw { RawW<6> W; };   // bytes [0, 24) of the block: header, qh, the 16 quant bytes
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) { r.W.load(row + u * BB); }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        // qh at byte OH, quants at byte OQ (both even): realign by 2 bytes when needed
        const uint32_t w0 = r.W[0];
        const uint32_t qh = OH == 4 ? r.W[1] : __builtin_amdgcn_alignbyte(r.W[1], w0, 2);
        uint32_t q[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            q[j] = OQ == 8 ? r.W[2 + j] : __builtin_amdgcn_alignbyte(r.W[2 + j], r.W[1 + j], 2);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // bits 4j .. 4j + 3 of qh -> bit 4 of bytes 0..3 (low half), bits 16 + 4j .. of qh (high half)
            const uint32_t hl = (((qh >> (4 * j)) & 15u) * 0x00204081u) & 0x01010101u;
            const uint32_t hh = (((qh >> (16 + 4 * j)) & 15u) * 0x00204081u) & 0x01010101u;
            const uint32_t lo = (q[j] & 0x0F0F0F0Fu) | (hl << 4), hi = ((q[j] >> 4) & 0x0F0F0F0Fu) | (hh << 4);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s0 += x.v[4 * j + k] * ub(lo, k);
                s1 += x.v[16 + 4 * j + k] * ub(hi, k);
            }
        }
        const float d = h16(w0 & 0xFFFFu);
        if constexpr (ONE) return d * (s0 + s1) + h16(w0 >> 16) * x.s[0];
        else return d * ((s0 + s1) - 16.f * x.s[0]);
    }
};

struct TF32 {
    static constexpr int RB = 2, NS = 1, RUN = 32, PRE = 2, DEPTH = 2;
    struct Raw { float4 f[8]; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const float4* p = reinterpret_cast<const float4*>(row + (int64_t)u * 128);
#pragma unroll
        for (int j = 0; j < 8; j++) r.f[j] = p[j];
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float4 a = r.f[j], b = r.f[j + 1];
            s0 += x.v[4 * j] * a.x + x.v[4 * j + 1] * a.y + x.v[4 * j + 2] * a.z + x.v[4 * j + 3] * a.w;
            s1 += x.v[4 * j + 4] * b.x + x.v[4 * j + 5] * b.y + x.v[4 * j + 6] * b.z + x.v[4 * j + 7] * b.w;
        }
        return s0 + s1;
    }
};

struct TF16 {
    static constexpr int RB = 4, NS = 1, RUN = 32, PRE = 2, DEPTH = 2;
    struct Raw { u32x4 q[4]; };
    __device__ static int xoff(int u, int) { return u * 32; }
    __device__ static void load(Raw& r, const uint8_t* row, int u) {
        const uint8_t* p = row + (int64_t)u * 64;
#pragma unroll
        for (int j = 0; j < 4; j++) r.q[j] = ld16_a4(p + 16 * j);
    }
    __device__ static float dot(const Raw& r, int, const XF<NS>& x) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w[4] = {r.q[j].x, r.q[j].y, r.q[j].z, r.q[j].w};
#pragma unroll
            for (int k = 0; k < 4; k++)
                s += x.v[8 * j + 2 * k] * h16(w[k] & 0xFFFFu) + x.v[8 * j + 2 * k + 1] * h16(w[k] >> 16);
        }
        return s;
    }
};

template <uint32_t T> struct TypeOf;
template <> struct TypeOf<GGML_Q2_K> { using type = TQ2K; };
template <> struct TypeOf<GGML_Q3_K> { using type = TQ3K; };
template <> struct TypeOf<GGML_Q4_K> { using type = TQ4K; };
template <> struct TypeOf<GGML_Q5_K> { using type = TQ5K; };
template <> struct TypeOf<GGML_Q6_K> { using type = TQ6K; };
template <> struct TypeOf<GGML_Q8_0> { using type = TQ8_0; };
template <> struct TypeOf<GGML_Q4_0> { using type = TQ4_0; };
template <> struct TypeOf<GGML_Q4_1> { using type = TQ4_1; };
template <> struct TypeOf<GGML_Q5_0> { using type = TQ5_01<false>; };
template <> struct TypeOf<GGML_Q5_1> { using type = TQ5_01<true>; };
template <> struct TypeOf<GGML_F32> { using type = TF32; };
template <> struct TypeOf<GGML_F16> { using type = TF16; };

// Sum of v over each row of 16 lanes, in every lane of the row (DPP row
// rotations by 8, 4, 2, 1; all 64 lanes must be active).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
template <int N>
__device__ __forceinline__ void row_sums16(float* v) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f32<0x128>(v[i]);   // row_ror:8
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f32<0x124>(v[i]);   // row_ror:4
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f32<0x122>(v[i]);   // row_ror:2
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_f32<0x121>(v[i]);   // row_ror:1
}

// Raw activations of a lane: the unit's 32 values of x, in the unit's element
// order.  For an RmsNorm consumer x is already w * h (packed by the producer).
struct XRaw {
    float4 h[8];
};

template <int RUN, typename XOff>
__device__ __forceinline__ void issue_x(const GemvArgs& a, XOff&& xoff, XRaw& r) {
#pragma unroll
    for (int run = 0; run < 32 / RUN; run++) {
        const int off = xoff(run);
#pragma unroll
        for (int q = 0; q < RUN / 4; q++) r.h[run * (RUN / 4) + q] = *reinterpret_cast<const float4*>(a.x + off + 4 * q);
    }
}

// The lane's 32 values, 0 past the row end.
__device__ __forceinline__ void finish_x(const XRaw& r, bool has, float* v) {
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const float4 e = r.h[q];
        v[4 * q] = has ? e.x : 0.f; v[4 * q + 1] = has ? e.y : 0.f;
        v[4 * q + 2] = has ? e.z : 0.f; v[4 * q + 3] = has ? e.w : 0.f;
    }
}

template <int NS>
__device__ __forceinline__ void run_sums(XF<NS>& x) {
    constexpr int PER = 32 / NS;
#pragma unroll
    for (int t = 0; t < NS; t++) {
        float z = 0.f;
#pragma unroll
        for (int e = 0; e < PER; e++) z += x.v[PER * t + e];
        x.s[t] = z;
    }
}

// The activation form a row unit takes: 24-bit nibble planes (Q4_K, sdot8),
// 24-bit byte planes (Q8_0, sdot4) or fp32 values with run sums.
template <typename TT> struct ActOf { using type = XF<TT::NS>; static constexpr int kind = 0; };
template <> struct ActOf<TQ4K> { using type = XQ; static constexpr int kind = 1; };
template <> struct ActOf<TQ8_0> { using type = XB; static constexpr int kind = 2; };

// One workgroup's rows.  Issue order: the activations, then the first PRE
// batches of weights; a scheduling barrier keeps the activation arithmetic
// (quantisation) after those issues, so it overlaps the weight loads.  DEPTH
// batches are in flight: each computed batch frees its registers for the
// batch DEPTH ahead.  Every lane
// loads (lanes past the row end read unit 0 and contribute 0): no branches,
// so no load is serialised behind another.  Row i's per-quarter-wavefront
// sums go to red_w[i][0..3].
// HV > 1 (Q4_K only): the workgroup is HV halves over the same units; half 0
// loads and quantises the activations and hands them to the other halves
// through LDS (xq_s), so each activation byte leaves L2 once per HV x rows.
template <typename TT, int NB, int HV = 1, typename RowPtr>
__device__ __forceinline__ void gemv_rows(const GemvArgs& a, int uu, bool has, RowPtr&& row_ptr, float (*red_w)[4],
                                          bool own_x = true, uint32_t* xq_s = nullptr, int units = 0) {
    constexpr int RB = TT::RB;
    constexpr int AK = ActOf<TT>::kind;
    constexpr bool INT = AK != 0;
    static_assert(HV == 1 || INT, "shared activations are quantised ones");
    const int lane = threadIdx.x & 63;
    XRaw xr;
    if (own_x) {
        if constexpr (INT) issue_x<32>(a, [&](int) { return uu * 32; }, xr);
        else issue_x<TT::RUN>(a, [&](int run) { return TT::xoff(uu, run); }, xr);
    }
    constexpr int D = TT::DEPTH;     // batches in flight
    typename TT::Raw buf[D][RB];
#pragma unroll
    for (int k = 0; k < TT::PRE && k < NB && k < D; k++)
#pragma unroll
        for (int i = 0; i < RB; i++) TT::load(buf[k][i], row_ptr(k * RB + i), uu);
    __builtin_amdgcn_sched_barrier(0);
    float v[32];
    if (own_x) finish_x(xr, has, v);
#pragma unroll
    for (int k = TT::PRE; k < NB && k < D; k++)
#pragma unroll
        for (int i = 0; i < RB; i++) TT::load(buf[k][i], row_ptr(k * RB + i), uu);
    typename ActOf<TT>::type x;
    if constexpr (INT) {
        if (own_x) {
            if constexpr (AK == 1) quantize32(v, x);
            else quantize32_b(v, x);
        }
        if constexpr (HV > 1) {
            constexpr int XW = 4 * XQ_PLANES + 2;   // dwords per unit: planes, s, sum
            if (own_x && has) {
#pragma unroll
                for (int j = 0; j < 4 * XQ_PLANES; j++) xq_s[j * units + uu] = x.pl[j];
                xq_s[(XW - 2) * units + uu] = __float_as_uint(x.s);
                xq_s[(XW - 1) * units + uu] = __float_as_uint(x.sum);
            }
            __syncthreads();
            if (!own_x) {
#pragma unroll
                for (int j = 0; j < 4 * XQ_PLANES; j++) x.pl[j] = xq_s[j * units + uu];
                x.s = __uint_as_float(xq_s[(XW - 2) * units + uu]);
                x.sum = __uint_as_float(xq_s[(XW - 1) * units + uu]);
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 32; e++) x.v[e] = v[e];
        run_sums(x);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float dv[RB];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const float d = TT::dot(buf[b % D][i], uu, x);
            dv[i] = has ? d : 0.f;
        }
        row_sums16<RB>(dv);   // all rows level by level: no DPP hazard stalls
        if ((lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++) red_w[b * RB + i][lane >> 4] = dv[i];
        }
        if (b + D < NB) {
#pragma unroll
            for (int i = 0; i < RB; i++) TT::load(buf[b % D][i], row_ptr((b + D) * RB + i), uu);
        }
    }
}

// ---- the kernel -------------------------------------------------------------------
// NB batches of RB dot rows; SwiGLU batches hold RB/2 gate then RB/2 up rows.
// Segments of the second type T2 take NB2 <= NB batches per workgroup.
// HV halves (HV_MAX_UNITS units at most) each take NB batches of the same units.
constexpr int HV_MAX_UNITS = 256;

template <uint32_t T, int EPI, int NB, bool NORM, uint32_t T2 = T, int NB2 = NB, int HV = 1>
__global__ __launch_bounds__(MAXW * 64) void gemv_kernel(GemvArgs a) {
    using TT = typename TypeOf<T>::type;
    using TT2 = typename TypeOf<T2>::type;
    static_assert(TT2::RB == TT::RB, "mixed-type launches need equal batch geometry");
    static_assert(HV == 1 || T2 == T, "halves are for single-type launches");
    constexpr int RB = TT::RB;
    constexpr bool SW = EPI == EPI_SWIGLU;
    constexpr int OPB = SW ? RB / 2 : RB;     // output rows per batch
    constexpr int ROWS_H = NB * OPB;          // output rows per half
    constexpr int ROWS_WG = HV * ROWS_H;
    constexpr int NSUM = NB * RB;
    static_assert(ROWS_WG <= 64, "epilogue uses one wavefront");
    __shared__ float red[MAXW][NSUM][4];
    __shared__ float ssq[MAXW];
    __shared__ uint32_t xq_s[HV > 1 ? (4 * XQ_PLANES + 2) * HV_MAX_UNITS : 1];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x >> 6) / HV;   // waves per half
    const int half = wave / nw, hw = wave - half * nw;
    // Segment and first row of this workgroup.  Every argument is read at once
    // and the segment picked by selects: a search loop made each argument load
    // wait for the one before it (~0.8 us of dependent round trips before the
    // first activation load, measured).
    const GemvSeg s0 = a.seg[0], s1 = a.seg[1], s2 = a.seg[2];
    int blk = blockIdx.x;
    const bool in1 = a.nseg > 1 && blk >= s0.wgs;
    const bool in2 = in1 && a.nseg > 2 && blk >= s0.wgs + s1.wgs;
    blk -= in2 ? s0.wgs + s1.wgs : (in1 ? s0.wgs : 0);
    GemvSeg seg;
    seg.w = in2 ? s2.w : (in1 ? s1.w : s0.w);
    seg.w2 = in2 ? s2.w2 : (in1 ? s1.w2 : s0.w2);
    seg.out = in2 ? s2.out : (in1 ? s1.out : s0.out);
    seg.rows = in2 ? s2.rows : (in1 ? s1.rows : s0.rows);
    seg.wgs = in2 ? s2.wgs : (in1 ? s1.wgs : s0.wgs);
    seg.type = in2 ? s2.type : (in1 ? s1.type : s0.type);
    // the remaining arguments the first loads and the epilogue need, in SGPRs
    // in the same round
    asm volatile("" ::"s"(a.x), "s"(a.ssq), "s"(seg.w), "s"(seg.w2), "s"(seg.out), "s"(a.pack_w), "s"(a.cols));
    if (EPI == EPI_ADD) asm volatile("" ::"s"(a.pack_out), "s"(a.pack_ssq));
    if (NORM) asm volatile("" ::"s"(a.eps));
    if (EPI == EPI_ARGMAX) asm volatile("" ::"s"(a.am.cand_val), "s"(a.am.cand_idx));
    // Output rows in slabs of SLAB: slab j of this workgroup is rows
    // (j * wgs + blk) * SLAB ..., so at any moment the workgroups of a
    // segment stream through one contiguous stretch of each matrix.  The ADD
    // epilogue packs rows in aligned 4s (slabs of 8 where the workgroup's rows
    // allow, else of its 4).
    constexpr int SLAB = EPI == EPI_ADD ? (ROWS_WG % 8 == 0 ? 8 : ROWS_WG) : OPB;
    auto out_row = [&](int o) { return ((o / SLAB) * seg.wgs + blk) * SLAB + o % SLAB; };
    const int K = a.cols;
    const int u = hw * 64 + lane;
    const bool has = u < K / 32;
    const int uu = has ? u : 0;
    const bool second = T2 != T && seg.type == T2;   // uniform per workgroup
    static_assert(NB2 <= NB, "second-type segments take at most NB batches");
    const int rows_wg = second ? NB2 * OPB : ROWS_WG;
    const int b0 = half * NB;   // this half's first batch of the workgroup
    const int64_t rbytes = second ? (int64_t)(K / block_elems(T2)) * block_bytes(T2)
                                  : (int64_t)(K / block_elems(T)) * block_bytes(T);

    auto row_ptr = [&](int i) -> const uint8_t* {   // dot row i of this half
        const int b = b0 + i / RB, k = i % RB;
        const uint8_t* base = seg.w;
        int r;
        if (SW) {
            r = out_row(b * OPB + (k % OPB));
            if (k >= OPB) base = seg.w2;
        } else {
            r = out_row(b * RB + k);
        }
        return base + (int64_t)(r < seg.rows ? r : 0) * rbytes;
    };

    // RmsNorm: the producer's sums of h^2 over 4-element groups, two per
    // 8-element group (K/8 <= 4 groups per thread, threads >= K/32), issued
    // first and summed after the rows
    float2 sq[4];
    if (NORM) {
        const int nq = K >> 3;
#pragma unroll
        for (int k = 0; k < 4; k++)
            sq[k] = reinterpret_cast<const float2*>(a.ssq)[min((int)threadIdx.x + k * (int)blockDim.x, nq - 1)];
    }
    // ADD: the residual and norm weight of this lane's output row, loaded
    // before the rows so the epilogue does not wait on them; unconditional
    // (clamped row, and the output itself standing in for an absent norm
    // weight), so no branch waits on an argument: the epilogue uses them only
    // for valid rows
    float res = 0.f, pw = 0.f;
    if (EPI == EPI_ADD) {
        const int r = min(out_row(min((int)threadIdx.x, rows_wg - 1)), seg.rows - 1);
        res = seg.out[r];
        pw = (a.pack_out ? a.pack_w : seg.out)[r];
    }
    if (T2 != T && second) gemv_rows<TT2, NB2>(a, uu, has, row_ptr, red[wave]);
    else gemv_rows<TT, NB, HV>(a, uu, has, row_ptr, red[wave], half == 0, xq_s, K / 32);
    if (NORM) {
        const int nq = K >> 3;
        float hsq = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) hsq += (int)threadIdx.x + k * (int)blockDim.x < nq ? sq[k].x + sq[k].y : 0.f;
        const float w = wave_sum(hsq);
        if (lane == 0) ssq[wave] = w;   // over every wave: each entry of a.ssq is read by one thread
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;

    // epilogue (wavefront 0): lane t < rows_wg owns output row out_row(t)
    const int t = threadIdx.x;
    float inv = 1.f;
    if (NORM) {
#pragma clang fp contract(off)
        float ss = 0.f;
        for (int w = 0; w < HV * nw; w++) ss += ssq[w];
        inv = 1.0f / sqrtf(ss / (float)K + a.eps);   // RmsNorm: 1 / sqrt(sum/n + eps)
    }
    const int th = t / ROWS_H, tl = t - th * ROWS_H;   // half of output row t, and its row in the half
    auto total = [&](int i) {   // dot i of half th over that half's waves
        float s = 0.f;
        for (int w = th * nw; w < (th + 1) * nw; w++) s += (red[w][i][0] + red[w][i][1]) + (red[w][i][2] + red[w][i][3]);
        return s * inv;
    };
    const int b = tl / OPB, k = tl % OPB;
    const int row = out_row((th * NB + b) * OPB + k);
    const bool valid = t < rows_wg && row < seg.rows;
    if (EPI == EPI_STORE) {
        if (valid) seg.out[row] = total(b * RB + k);
    } else if (EPI == EPI_ADD) {
        float hn = 0.f;
        if (valid) {
            hn = res + total(b * RB + k);   // residual: a[i] + b[i]
            seg.out[row] = hn;
        }
        if (a.pack_out) {   // the updated vector packed for its RmsNorm consumer (rows come in 4s)
            if (valid) {
#pragma clang fp contract(off)
                a.pack_out[row] = pw * hn;
            }
            float q = hn * hn;
            q = sum4(q);
            if (valid && (t & 3) == 0) a.pack_ssq[row >> 2] = q;
        }
    } else if (EPI == EPI_SWIGLU) {
        if (valid) {
#pragma clang fp contract(off)
            const float g = total(b * RB + k), up = total(b * RB + OPB + k);
            // SiluInPlace: vector lanes (ExpApprox) for the first 8*floor(n/8), expf tail
            const float sg = row < (seg.rows & ~7) ? silu_ref(g) : g / (1.0f + expf(-g));
            seg.out[row] = sg * up;
        }
    } else if (EPI == EPI_ARGMAX) {
        const float y = valid ? total(t) : -INFINITY;
        if (valid) seg.out[row] = y;
        // NaN never wins (a NaN logit at index 0 is applied by the second pass)
        const bool cand = valid && !__builtin_isnan(y);
        float bv = cand ? y : -INFINITY;
        int bi = cand ? row : 0x7FFFFFFF;
        wave_argmax(bv, bi);
        if (t == 0) {   // one candidate per workgroup; launch_argmax_finish reduces them
            a.am.cand_val[blockIdx.x] = bv;
            a.am.cand_idx[blockIdx.x] = bi;
        }
    }
}

// Generic fallback for F32/F16 weights whose width is not a multiple of 32
// (MatMulF32 with small shapes, TO:437-504): one wavefront per output row.
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t* w, uint32_t type, const float* x,
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

int type_rb(uint32_t t) {
    switch (t) {
    case GGML_Q6_K: return TQ6K::RB;
    case GGML_Q3_K: return TQ3K::RB;
    case GGML_Q8_0: return TQ8_0::RB;
    case GGML_Q4_K: return TQ4K::RB;
    case GGML_F32: return TF32::RB;
    case GGML_F16: return TF16::RB;
    default: return 8;
    }
}

template <uint32_t T, int EPI, bool NORM, int HV = 1>
hipError_t launch_te(const GemvArgs& a, int nb, int grid, int threads, hipStream_t s) {
    switch (nb) {
    case 1: gemv_kernel<T, EPI, 1, NORM, T, 1, HV><<<grid, threads, 0, s>>>(a); break;
    case 2: gemv_kernel<T, EPI, 2, NORM, T, 2, HV><<<grid, threads, 0, s>>>(a); break;
    case 4: gemv_kernel<T, EPI, 4, NORM, T, 4, HV><<<grid, threads, 0, s>>>(a); break;
    case 8:
        if constexpr (HV * 8 * TypeOf<T>::type::RB <= 64) { gemv_kernel<T, EPI, 8, NORM, T, 8, HV><<<grid, threads, 0, s>>>(a); break; }
        else return hipErrorInvalidValue;
    case 7: gemv_kernel<T, EPI, 7, NORM, T, 7, HV><<<grid, threads, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Instantiated forms: STORE with or without RmsNorm, ADD without, SWIGLU and
// ARGMAX with (the decode step's uses and the op-level MatMul).
template <uint32_t T>
hipError_t launch_t(int epi, const GemvArgs& a, int nb, int grid, int threads, hipStream_t s, int hv = 1) {
    if constexpr (T == GGML_Q4_K) {
        if (hv == 2) {
            if (epi == EPI_ADD) return launch_te<T, EPI_ADD, false, 2>(a, nb, grid, threads, s);
            return hipErrorInvalidValue;
        }
    }
    if (hv != 1) return hipErrorInvalidValue;
    switch (epi) {
    case EPI_STORE:
        return a.norm ? launch_te<T, EPI_STORE, true>(a, nb, grid, threads, s)
                      : launch_te<T, EPI_STORE, false>(a, nb, grid, threads, s);
    case EPI_ADD: return launch_te<T, EPI_ADD, false>(a, nb, grid, threads, s);
    case EPI_SWIGLU: return launch_te<T, EPI_SWIGLU, true>(a, nb, grid, threads, s);
    case EPI_ARGMAX: return launch_te<T, EPI_ARGMAX, true>(a, nb, grid, threads, s);
    default: return hipErrorInvalidValue;
    }
}

bool generic_shape(uint32_t type, int cols) { return (type == GGML_F32 || type == GGML_F16) && cols % 32 != 0; }

}  // namespace

bool gemv_supported(uint32_t type) {
    return type == GGML_Q4_K || type == GGML_Q5_K || type == GGML_Q6_K || type == GGML_Q8_0 ||
           type == GGML_Q4_0 || type == GGML_Q4_1 || type == GGML_Q5_0 || type == GGML_Q5_1 ||
           type == GGML_Q2_K || type == GGML_Q3_K || type == GGML_F32 || type == GGML_F16;
}

bool gemv_width_ok(uint32_t type, int cols) {
    if (!gemv_supported(type) || cols <= 0) return false;
    if (generic_shape(type, cols)) return true;
    return cols % block_elems(type) == 0 && cols / 32 <= MAXW * 64;
}

// Wavefronts a launch should have at least: 6 per CU for workgroups of two or
// more wavefronts, 4 per CU for one-wavefront workgroups (fewer, longer
// workgroups amortise the activation loads; measured: the Phi-3 Q/K/V and
// gate/up launches gained 1.9% of the step at 1536, the 7B launches were
// unchanged, 1B's one-wavefront gate/up lost 0.3%); LLMDOT_GEMV_WAVES
// overrides both.
// LLMDOT_GEMV_HALVES=0 keeps one half per workgroup (A/B timing and tests).
static bool env_halves_off() {
    static const bool off = [] {
        const char* e = getenv("LLMDOT_GEMV_HALVES");
        return e && strcmp(e, "0") == 0;
    }();
    return off;
}

static int target_waves(int nw) {
    static const int w = [] {
        const char* e = getenv("LLMDOT_GEMV_WAVES");
        return e ? atoi(e) : 0;
    }();
    return w > 0 ? w : (nw > 1 ? 1536 : 1024);
}

int gemv_plan(uint32_t type, int epi, int rows_total, int cols) {
    if (generic_shape(type, cols)) return 0;
    const int nw = (cols / 32 + 63) / 64;
    const int opb = epi == EPI_SWIGLU ? type_rb(type) / 2 : type_rb(type);
    // the most rows per workgroup that still gives the target wavefront count
    // SwiGLU: 7 batches when that gives a whole number of workgroups per CU
    // (14336 rows: 1024 workgroups, 4 per CU, instead of 896)
    if (epi == EPI_SWIGLU && rows_total % (7 * opb) == 0 && (rows_total / (7 * opb)) % 256 == 0) return 7;
    int nb = 8;
    while (nb > 1 && ((rows_total + nb * opb - 1) / (nb * opb)) * nw < target_waves(nw)) nb /= 2;
    // the ADD epilogue packs rows in groups of 4 and prefers slabs of 8; but
    // where 8-row slabs leave a fraction of a workgroup per CU (some CUs two,
    // others one) and 4-row workgroups fill the CUs evenly, it takes 4 rows
    // (Phi-3-mini's 3072-row O and down projections: 768 workgroups, not 384)
    if (epi == EPI_ADD) {
        auto wgs = [&](int n) { return (rows_total + n * opb - 1) / (n * opb); };
        while (nb < 8 && (nb * opb) % 8) nb *= 2;
        if (nb > 1 && wgs(nb) % 256 && ((nb / 2) * opb) % 4 == 0 && wgs(nb / 2) % 256 == 0) nb /= 2;
    }
    return nb;
}

// Halves per workgroup: 2 for Q4_K residual-add launches over at most 4096
// columns that keep a workgroup per CU with halves (the 7B attention output
// projection, 4096 x 4096: 6.48 -> 6.16 us).  With fewer workgroups than CUs,
// or wider rows (the 1B shape's 2048 x 8192 down projection), halves measured
// slower, as did the larger STORE / SwiGLU GEMVs.
int gemv_halves(uint32_t type, int epi, int cols, bool mixed, int grid_one_half) {
    const int units = cols / 32;
    if (type != GGML_Q4_K || mixed || epi != EPI_ADD || env_halves_off()) return 1;
    return units <= 128 && grid_one_half >= 2 * 256 ? 2 : 1;
}

int gemv_rows_per_wg(uint32_t type, int epi, int nb) {
    return nb * (epi == EPI_SWIGLU ? type_rb(type) / 2 : type_rb(type));
}

int gemv_max_grid(uint32_t type, int epi, int rows, int cols) {
    if (generic_shape(type, cols)) return (rows + 3) / 4;
    const int rwg = gemv_rows_per_wg(type, epi, gemv_plan(type, epi, rows, cols));
    return (rows + rwg - 1) / rwg + 2;   // segments round up separately (halves only lower the count)
}

hipError_t launch_gemv(uint32_t type, int epi, GemvArgs& a, hipStream_t s) {
    if (a.cols <= 0 || a.nseg < 1 || a.nseg > 3) return hipErrorInvalidValue;
    // segment types: 0 means `type`; a second type is supported for Q4_K + Q6_K
    uint32_t t2 = type;
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].type == 0) a.seg[i].type = type;
        if (a.seg[i].type != type) {
            if (t2 != type && a.seg[i].type != t2) return hipErrorInvalidValue;
            t2 = a.seg[i].type;
        }
    }
    if (t2 != type && !((type == GGML_Q4_K || type == GGML_Q8_0) && t2 == GGML_Q6_K && epi == EPI_STORE && a.norm))
        return hipErrorInvalidValue;
    if (t2 != type && !gemv_width_ok(t2, a.cols)) return hipErrorInvalidValue;
    if (generic_shape(type, a.cols)) {
        if (epi != EPI_STORE || a.nseg != 1 || a.norm) return hipErrorInvalidValue;
        if (a.seg[0].rows <= 0) return hipSuccess;
        gemv_generic_kernel<<<(a.seg[0].rows + 3) / 4, 256, 0, s>>>(a.seg[0].w, type, a.x, a.seg[0].out,
                                                                   a.seg[0].rows, a.cols);
        return hipGetLastError();
    }
    if (!gemv_width_ok(type, a.cols)) return hipErrorInvalidValue;
    if (epi == EPI_SWIGLU && (a.nseg != 1 || !a.seg[0].w2)) return hipErrorInvalidValue;
    if (epi == EPI_ARGMAX && (a.nseg != 1 || !a.am.cand_val || !a.am.cand_idx || !a.am.token_out))
        return hipErrorInvalidValue;
    if (a.norm && (!a.ssq || a.cols % 8)) return hipErrorInvalidValue;
    if (epi == EPI_ADD && a.norm) return hipErrorInvalidValue;
    if (a.pack_out && (epi != EPI_ADD || !a.pack_w || !a.pack_ssq || a.nseg != 1 || a.seg[0].rows % 8))
        return hipErrorInvalidValue;
    if ((epi == EPI_SWIGLU || epi == EPI_ARGMAX) && !a.norm) return hipErrorInvalidValue;
    int rows_total = 0;
    for (int i = 0; i < a.nseg; i++) {
        if (a.seg[i].rows < 0) return hipErrorInvalidValue;
        rows_total += a.seg[i].rows;
    }
    // Q4_K + Q6_K Q/K/V launches: one batch per workgroup (4 rows; the 7B
    // shape's 1536 workgroups measured 0.2% faster than 896 of 8 rows, while
    // the Q8_0 + Q6_K mix lost 3% that way)
    const int nb = t2 != type && type == GGML_Q4_K ? 1 : gemv_plan(type, epi, rows_total, a.cols);
    const int rwg1 = gemv_rows_per_wg(type, epi, nb);
    const int hv = gemv_halves(type, epi, a.cols, t2 != type, (rows_total + rwg1 - 1) / rwg1);
    const int rwg = hv * rwg1;
    // Q6_K segments of a mixed launch: half the batches per workgroup (a Q6_K
    // row costs about twice a Q4_K or Q8_0 row), so their workgroups end with
    // the rest
    const int nb2 = nb > 1 ? nb / 2 : 1;
    const int rwg2 = gemv_rows_per_wg(t2, epi, nb2);
    int grid = 0;
    for (int i = 0; i < a.nseg; i++) {
        const int r = (t2 != type && a.seg[i].type == t2) ? rwg2 : rwg;
        a.seg[i].wgs = (a.seg[i].rows + r - 1) / r;
        grid += a.seg[i].wgs;
    }
    if (grid <= 0) return hipSuccess;
    if (epi == EPI_ARGMAX && a.am.cap < grid) return hipErrorInvalidValue;
    const int threads = hv * 64 * ((a.cols / 32 + 63) / 64);
    hipError_t e;
    if (t2 != type && type == GGML_Q8_0) {   // Q8_0 with Q6_K segments (Q/K/V of the Q6_K/Q8_0 mixes)
        switch (nb) {
        case 1: gemv_kernel<GGML_Q8_0, EPI_STORE, 1, true, GGML_Q6_K, 1><<<grid, threads, 0, s>>>(a); break;
        case 2: gemv_kernel<GGML_Q8_0, EPI_STORE, 2, true, GGML_Q6_K, 1><<<grid, threads, 0, s>>>(a); break;
        case 4: gemv_kernel<GGML_Q8_0, EPI_STORE, 4, true, GGML_Q6_K, 2><<<grid, threads, 0, s>>>(a); break;
        case 8: gemv_kernel<GGML_Q8_0, EPI_STORE, 8, true, GGML_Q6_K, 4><<<grid, threads, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (t2 != type) {   // Q4_K with Q6_K segments (Q/K/V of the Q4_K_M mix)
        switch (nb) {
        case 1: gemv_kernel<GGML_Q4_K, EPI_STORE, 1, true, GGML_Q6_K, 1><<<grid, threads, 0, s>>>(a); break;
        case 2: gemv_kernel<GGML_Q4_K, EPI_STORE, 2, true, GGML_Q6_K, 1><<<grid, threads, 0, s>>>(a); break;
        case 4: gemv_kernel<GGML_Q4_K, EPI_STORE, 4, true, GGML_Q6_K, 2><<<grid, threads, 0, s>>>(a); break;
        case 8: gemv_kernel<GGML_Q4_K, EPI_STORE, 8, true, GGML_Q6_K, 4><<<grid, threads, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (type) {
    case GGML_Q4_K: e = launch_t<GGML_Q4_K>(epi, a, nb, grid, threads, s, hv); break;
    case GGML_Q5_K: e = launch_t<GGML_Q5_K>(epi, a, nb, grid, threads, s); break;
    case GGML_Q6_K: e = launch_t<GGML_Q6_K>(epi, a, nb, grid, threads, s); break;
    case GGML_Q8_0: e = launch_t<GGML_Q8_0>(epi, a, nb, grid, threads, s); break;
    case GGML_Q4_0: e = launch_t<GGML_Q4_0>(epi, a, nb, grid, threads, s); break;
    case GGML_Q4_1: e = launch_t<GGML_Q4_1>(epi, a, nb, grid, threads, s); break;
    case GGML_Q5_0: e = launch_t<GGML_Q5_0>(epi, a, nb, grid, threads, s); break;
    case GGML_Q5_1: e = launch_t<GGML_Q5_1>(epi, a, nb, grid, threads, s); break;
    case GGML_Q2_K: e = launch_t<GGML_Q2_K>(epi, a, nb, grid, threads, s); break;
    case GGML_Q3_K: e = launch_t<GGML_Q3_K>(epi, a, nb, grid, threads, s); break;
    case GGML_F32: e = launch_t<GGML_F32>(epi, a, nb, grid, threads, s); break;
    case GGML_F16: e = launch_t<GGML_F16>(epi, a, nb, grid, threads, s); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || epi != EPI_ARGMAX) return e;
    ArgmaxState am = a.am;
    am.first = a.seg[0].out;   // logits[0]: VectorMath.ArgMax's NaN-at-[0] rule
    return launch_argmax_finish(am, grid, s);
}

}  // namespace llmdot
