// prefill.hip -- batched prompt processing: a chunk of T prompt tokens per
// launch, projections on MFMA.
//
// The reference processes a prompt one ProcessToken call per token
// (src/Llmdot.Core/Inference/InferenceEngine.cs:84-88, IE:134-146); only the
// KV cache and the last token's logits are observable (the logits of the
// other prompt tokens are discarded, IE:86).  Here every projection of a chunk
// is one GEMM Y[T x N] = X[T x K] . W^T on v_mfma_f32_16x16x32_f16 with W's
// GGUF blocks dequantised into LDS tile by tile, and attention is causal over
// the chunk plus the cached positions.
//
// Numerics (fp32-equivalent, not bf16):
//  * Activations: each token row x is scaled by a power of two s (max|x s| in
//    [2^14, 2^15)) and split into two fp16 planes, x s = hi + lo with
//    |x s - hi - lo| <= 2^-23 |x s| -- 22-23 significant bits.
//  * Weights: every supported format is (scale) * (small integer) per block
//    (Q4_K/Q5_K: d * sc_g * (q - 8|16) - dmin * m_g; Q6_K: d * sc_16 * (q - 32);
//    Q8_0: d * q; Q4_0: d * (q - 8), DequantizeK.cs / DequantizeBasic.cs).  The
//    integer part v = sc * (q - c) is exact in fp16 (|v| <= 1008), except Q6_K
//    (|v| <= 4096), which is split into v_hi + v_lo with v_lo in {-1, 0, 1}.
//    Products of fp16 planes are exact in fp32, so a block's partial sum
//    P = sum v x carries only fp32 accumulation error; the block scale (d) is
//    applied once per block: acc += d * P.
//  * The min term of Q4_K/Q5_K, -dmin * sum_g m_g * sum_{k in g} x_k, uses the
//    group sums of x (fp32, split into two fp16 planes) against the 6-bit m_g
//    on v_mfma_f32_16x16x16_f16 (8 groups + 8 zero slots per superblock).
//  So a GEMM output differs from the reference's sequential fp32 dot by
//  rounding-level error, like the decode GEMV.
//
// Tiles: 128 tokens x 128 weight rows per 256-thread workgroup; wave w owns
// tokens 64 (w & 1) .. +63 and rows 64 (w >> 1) .. +63 as 4 x 4 MFMA tiles.
// K advances 32 per step (one MFMA K), the scale chunk is 256 (K-quants) or
// 32 (Q8_0, Q4_0).  Global loads of step s+1 are issued before the MFMAs of
// step s; their dequantisation follows the MFMAs so it overlaps them.
#include "common.h"
#include "kernels.h"

namespace llmdot {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int BM = 128;   // tokens per workgroup
constexpr int BN = 128;   // weight rows per workgroup
constexpr int WG = 256;

// ---------------------------------------------------------------- planes --

// One workgroup per token row: optional RmsNorm (VectorMath.RmsNorm, VM:308-340:
// ss = sum x^2, inv = 1/sqrt(ss/n + eps), y = (w x) inv on the vector lanes,
// w (x inv) on the tail), then the power-of-two scale, the two fp16 planes of
// y s, the group sums of y (scaled by s/32) as two planes, and 1/s.
template <bool NORM>
__global__ __launch_bounds__(WG) void pf_planes_kernel(const float* __restrict__ x, int K, const float* __restrict__ w,
                                                       float eps, _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                       _Float16* __restrict__ sh, _Float16* __restrict__ sl,
                                                       float* __restrict__ xinv) {
    __shared__ float red[WG / 64];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* row = x + (int64_t)t * K;
    float inv = 1.f;
    if (NORM) {
        float ss = 0.f;
        for (int i = tid; i < K; i += WG) {
            const float v = row[i];
            ss += v * v;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < WG / 64; i++) tot += red[i];
        __syncthreads();
        {
#pragma clang fp contract(off)
            inv = 1.0f / sqrtf((tot / (float)K) + eps);
        }
    }
    const int n8 = K & ~7;
    auto yval = [&](int i) -> float {
#pragma clang fp contract(off)
        const float v = row[i];
        if (!NORM) return v;
        return i < n8 ? ((w[i] * v) * inv) : (w[i] * (v * inv));
    };
    float amax = 0.f;
    for (int i = tid; i < K; i += WG) amax = fmaxf(amax, fabsf(yval(i)));
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < WG / 64; i++) m = fmaxf(m, red[i]);
    int e = 0;
    if (m > 0.f) {
        (void)frexpf(m, &e);          // m = f 2^e, f in [0.5, 1)
        e = 15 - e;                   // max |y| 2^e in [2^14, 2^15)
        e = e > 126 ? 126 : (e < -126 ? -126 : e);
    }
    const float s = ldexpf(1.0f, e), s32 = ldexpf(1.0f, e - 5);
    if (tid == 0) xinv[t] = ldexpf(1.0f, -e);
    // 4 consecutive elements per thread; 8 threads cover one 32-element group
    for (int b0 = 0; b0 < K; b0 += 4 * WG) {
        const int base = b0 + 4 * tid;
        const bool ok = base < K;     // K % 32 == 0: a group's 8 lanes agree
        float y[4], g = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            y[j] = ok ? yval(base + j) : 0.f;
            g += y[j];
        }
        g += __shfl_xor(g, 1, 64);
        g += __shfl_xor(g, 2, 64);
        g += __shfl_xor(g, 4, 64);
        if (ok) {
            h4 hv, lv;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float ys = y[j] * s;
                const _Float16 hi = (_Float16)ys;
                hv[j] = hi;
                lv[j] = (_Float16)(ys - (float)hi);
            }
            *reinterpret_cast<h4*>(xh + (int64_t)t * K + base) = hv;
            *reinterpret_cast<h4*>(xl + (int64_t)t * K + base) = lv;
            if ((tid & 7) == 0) {
                const float gs = g * s32;
                const _Float16 hi = (_Float16)gs;
                sh[(int64_t)t * (K / 32) + base / 32] = hi;
                sl[(int64_t)t * (K / 32) + base / 32] = (_Float16)(gs - (float)hi);
            }
        }
    }
}

// ------------------------------------------------------------------ GEMM --

struct PfGemmArgs {
    const _Float16 *xh, *xl, *sh, *sl;   // [M][K], [M][K], [M][K/32] x2
    const float* xinv;                   // [M]
    const uint8_t* w;                    // [N][row bytes] GGUF blocks
    const uint8_t* w2;                   // SWIGLU: the up matrix (w = gate)
    float* out;                          // [M][ldo]
    int M, N, K, ldo;
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Four bytes b0..b3 (each < 1024 - c) -> two fp16 pairs (b - c) * sc, exact:
// 0x6400 | b is the fp16 1024 + b.
__device__ __forceinline__ void bytes_to_h2(uint32_t b, _Float16 c1024, _Float16 sc, uint32_t* out) {
    const h2 off = {c1024, c1024}, scv = {sc, sc};
    const uint32_t p0 = perm(0x64646464u, b, 0x04010400u);
    const uint32_t p1 = perm(0x64646464u, b, 0x04030402u);
    out[0] = as_u((as_h2(p0) - off) * scv);
    out[1] = as_u((as_h2(p1) - off) * scv);
}

// 6-bit field at bit b of the 96-bit scale stream w1:w2:w3 (bytes 4..15 of a
// reference-layout K-quant block, DequantizeK.Extract6Bit, DK:189-199): low
// 12 bits = sc | m << 6 for group b / 12.
__device__ __forceinline__ uint32_t k_field12(uint32_t w1, uint32_t w2, uint32_t w3, int b) {
    const uint32_t lo = b < 32 ? w1 : (b < 64 ? w2 : w3);
    const uint32_t hi = b < 32 ? w2 : (b < 64 ? w3 : 0u);
    return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)(b & 31)) & 0xFFFu;
}

// Per-thread staging registers of one 32-K step: this thread's weight bytes
// (one row half: 16 elements) and the row's scale fields.
struct Stage {
    uint32_t q[4];      // weight payload bytes (Q4_K/Q5_K: q[0..1])
    uint32_t qh[4];     // Q6_K: high bits; Q5_K: qh[0] = 16 high bits
    uint32_t hdr[4];    // Q4_K/Q5_K: the 16-byte block header; others: hdr[0] = fp16 d, hdr[1] = Q6_K scale byte
};

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

template <uint32_t FMT>
struct PfFmt;
template <>
struct PfFmt<GGML_Q4_K> { static constexpr int SB = 8, NP = 1, BSZ = 144, EPB = 256; static constexpr bool MIN = true; };
template <>
struct PfFmt<GGML_Q5_K> { static constexpr int SB = 8, NP = 1, BSZ = 176, EPB = 256; static constexpr bool MIN = true; };
template <>
struct PfFmt<GGML_Q6_K> { static constexpr int SB = 8, NP = 2, BSZ = 210, EPB = 256; static constexpr bool MIN = false; };
template <>
struct PfFmt<GGML_Q8_0> { static constexpr int SB = 1, NP = 1, BSZ = 34, EPB = 32; static constexpr bool MIN = false; };
template <>
struct PfFmt<GGML_Q4_0> { static constexpr int SB = 1, NP = 1, BSZ = 18, EPB = 32; static constexpr bool MIN = false; };

// Global loads of step `st` (K offset 32 st) for this thread's weight row half.
template <uint32_t FMT>
__device__ __forceinline__ void load_w(Stage& S, const uint8_t* rowp, int st, int hf) {
    using F = PfFmt<FMT>;
    if constexpr (FMT == GGML_Q4_K || FMT == GGML_Q5_K) {
        const int sb = st >> 3, g = st & 7;
        const uint8_t* blk = rowp + (int64_t)sb * F::BSZ;
        const u32x4 h = ld16_a4(blk);
        S.hdr[0] = h.x; S.hdr[1] = h.y; S.hdr[2] = h.z; S.hdr[3] = h.w;
        if constexpr (FMT == GGML_Q4_K) {
            const uint2 v = *reinterpret_cast<const uint2*>(blk + 16 + 16 * g + 8 * hf);
            S.q[0] = v.x; S.q[1] = v.y;
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(blk + 48 + 16 * g + 8 * hf);
            S.q[0] = v.x; S.q[1] = v.y;
            S.qh[0] = *reinterpret_cast<const uint16_t*>(blk + 16 + 4 * g + 2 * hf);
        }
    } else if constexpr (FMT == GGML_Q6_K) {
        const int sb = st >> 3, g = st & 7;
        const uint8_t* blk = rowp + (int64_t)sb * F::BSZ;
        const int n = 128 * (g >> 2), qq = g & 3;
        ld_realign<4>(blk + n / 2 + (qq & 1) * 32 + 16 * hf, S.q);
        ld_realign<4>(blk + 128 + n / 4 + 16 * hf, S.qh);
        S.hdr[0] = *reinterpret_cast<const uint16_t*>(blk + 208);
        S.hdr[1] = blk[192 + 2 * g + hf];   // int8 scale of elements 32 g + 16 hf .. +15
    } else {   // Q8_0, Q4_0: one block per step
        const uint8_t* blk = rowp + (int64_t)st * F::BSZ;
        S.hdr[0] = *reinterpret_cast<const uint16_t*>(blk);
        if constexpr (FMT == GGML_Q8_0) ld_realign<4>(blk + 2 + 16 * hf, S.q);
        else ld_realign<4>(blk + 2, S.q);
    }
}

// Dequantises this thread's 16 elements (plane 0, and plane 1 for Q6_K) into
// out[plane][8] words of fp16 pairs in natural element order.
template <uint32_t FMT>
__device__ __forceinline__ void convert_w(const Stage& S, int st, int hf, uint32_t (*out)[8]) {
    if constexpr (FMT == GGML_Q4_K || FMT == GGML_Q5_K) {
        const int g = st & 7;
        const uint32_t f = k_field12(S.hdr[1], S.hdr[2], S.hdr[3], 12 * g);
        const _Float16 sc = (_Float16)(float)(f & 63u);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t w = S.q[j];
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            uint32_t n0 = perm(hi, lo, 0x05010400u);   // elements 8j+0..3 as bytes
            uint32_t n1 = perm(hi, lo, 0x07030602u);   // elements 8j+4..7
            if constexpr (FMT == GGML_Q5_K) {
                const uint32_t hb = S.qh[0] >> (8 * j);
                n0 |= ((((hb & 15u) * 0x00204081u) & 0x01010101u) << 4);
                n1 |= (((((hb >> 4) & 15u) * 0x00204081u) & 0x01010101u) << 4);
                bytes_to_h2(n0, (_Float16)1040.f, sc, &out[0][4 * j]);
                bytes_to_h2(n1, (_Float16)1040.f, sc, &out[0][4 * j + 2]);
            } else {
                bytes_to_h2(n0, (_Float16)1032.f, sc, &out[0][4 * j]);
                bytes_to_h2(n1, (_Float16)1032.f, sc, &out[0][4 * j + 2]);
            }
        }
    } else if constexpr (FMT == GGML_Q6_K) {
        const int g = st & 7, qq = g & 3;
        const int scv = (int)(int8_t)(uint8_t)S.hdr[1];
        const h2 sc2 = {(_Float16)(float)scv, (_Float16)(float)scv};
        const h2 off = {(_Float16)1056.f, (_Float16)1056.f};
        const uint32_t nsh = 4 * (qq >> 1), qsh = 2 * qq;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t qb = ((S.q[j] >> nsh) & 0x0F0F0F0Fu) | (((S.qh[j] >> qsh) & 0x03030303u) << 4);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const uint32_t pr = perm(0x64646464u, qb, p ? 0x04030402u : 0x04010400u);
                const h2 qv = as_h2(pr) - off;                 // q - 32, exact
                const h2 vh = qv * sc2;                        // rounded to fp16
                const h2 vl = __builtin_elementwise_fma(qv, sc2, -vh);   // exact remainder
                out[0][2 * j + p] = as_u(vh);
                out[1][2 * j + p] = as_u(vl);
            }
        }
    } else if constexpr (FMT == GGML_Q8_0) {
#pragma unroll
        for (int j = 0; j < 4; j++) bytes_to_h2(S.q[j] ^ 0x80808080u, (_Float16)1152.f, (_Float16)1.f, &out[0][2 * j]);
    } else {   // Q4_0: half 0 = low nibbles of bytes 0..15, half 1 = high nibbles
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t b = hf ? ((S.q[j] >> 4) & 0x0F0F0F0Fu) : (S.q[j] & 0x0F0F0F0Fu);
            bytes_to_h2(b, (_Float16)1032.f, (_Float16)1.f, &out[0][2 * j]);
        }
    }
}

enum PfEpi : int { PF_STORE = 0, PF_ADD = 1, PF_SWIGLU = 2 };

// Workgroup barrier for LDS hand-offs: waits for this wave's LDS reads and
// writes, then s_barrier.  Unlike __syncthreads() it does not wait for
// outstanding global loads (the prefetched steps stay in flight); the
// activation copies of the step about to be read are complete because the
// wave has waited for the weight registers issued after them.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS rows of 32 halves (64 bytes) hold 4 chunks of 8; chunk c of row r sits
// at position c ^ swz(r), which spreads the 16 rows of an MFMA fragment read
// over distinct banks.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

template <uint32_t FMT, int EPI>
__global__ __launch_bounds__(WG, 2) void pf_gemm_kernel(PfGemmArgs a) {
    using F = PfFmt<FMT>;
    constexpr int NP = F::NP;
    // Activation stages are copied global -> LDS by global_load_lds_dwordx4
    // (no registers); NXB stages give a prefetch distance of NXB - 1 steps.
    // Weight bytes travel through registers at the same distance.
    constexpr int NXB = NP == 2 ? 2 : 3, D = NXB - 1;
    constexpr int XS1 = 2 * BM * 64;                 // one stage: [plane][token][32 halves]
    constexpr int XS_B = NXB * XS1;
    constexpr int WS_B = 2 * NP * BN * 64;           // [buf][plane][row][32 halves]
    constexpr int WD_B = 2 * BN * 4;                 // [buf][row] block scale d
    constexpr int WM_B = F::MIN ? 2 * BN * 4 : 0;    // [sb parity][row] 32 dmin
    constexpr int WQ_B = F::MIN ? 2 * BN * 16 : 0;   // [sb parity][row][8] m_g
    constexpr int SS_B = F::MIN ? 2 * 2 * BM * 16 : 0;   // [sb parity][plane][token][8] group sums
    constexpr int STAGE_B = XS_B + WS_B + WD_B + WM_B + WQ_B + SS_B;
    constexpr int EX_B = 2 * 64 * 65 * 4;            // SWIGLU exchange
    constexpr int SMEM = STAGE_B > EX_B ? STAGE_B : EX_B;
    __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
    unsigned char* const Xb = smem;
    unsigned char* const Wb = smem + XS_B;
    float* const Wd = reinterpret_cast<float*>(smem + XS_B + WS_B);
    float* const Wm = reinterpret_cast<float*>(smem + XS_B + WS_B + WD_B);
    unsigned char* const Wq = smem + XS_B + WS_B + WD_B + WM_B;
    unsigned char* const Ss = smem + XS_B + WS_B + WD_B + WM_B + WQ_B;
    auto xaddr = [&](int buf, int pl, int r, int c) { return Xb + buf * XS1 + (pl * BM + r) * 64 + ((c ^ swz(r)) << 4); };
    auto waddr = [&](int buf, int pl, int r, int c) { return Wb + ((buf * NP + pl) * BN + r) * 64 + ((c ^ swz(r)) << 4); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1, lr = lane & 15, lk = lane >> 4;
    const int m0 = blockIdx.y * BM;
    const int K = a.K, nsteps = K / 32;

    // weight row staged by this thread: rows 0..127 of the tile, two threads per row
    const int srow = tid >> 1, hf = tid & 1;
    int grow;
    const uint8_t* wbase = a.w;
    if (EPI == PF_SWIGLU) {
        grow = blockIdx.x * 64 + (srow & 63);
        if (srow >= 64) wbase = a.w2;
    } else {
        grow = blockIdx.x * BN + srow;
    }
    grow = min(grow, a.N - 1);
    const int64_t rbytes = (int64_t)(K / F::EPB) * F::BSZ;
    const uint8_t* rowp = wbase + (int64_t)grow * rbytes;

    // Activation stage st: wave w's instruction i fills LDS slots (4w + i) * 64 + lane
    // (16 bytes each) of the stage; slot q holds plane q >> 9, token (q >> 2) & 127,
    // position q & 3, i.e. chunk (q & 3) ^ swz(token) of the token's 32 elements.
    auto load_x = [&](int st) __attribute__((always_inline)) {
        unsigned char* base = Xb + (st % NXB) * XS1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = (4 * wave + i) * 64 + lane;
            const int pl = q >> 9, tk = (q >> 2) & 127, c = (q & 3) ^ swz(tk);
            const int tg = min(m0 + tk, a.M - 1);
            const _Float16* src = (pl ? a.xl : a.xh) + (int64_t)tg * K + 32 * st + 8 * c;
            __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)(base + (4 * wave + i) * 1024), 16, 0, 0);
        }
        if (F::MIN && (st & 7) == 0) {   // group sums of the superblock: [plane][token] 16-byte rows
            const int q = wave * 64 + lane;
            const int pl = q >> 7, tk = q & 127;
            const int tg = min(m0 + tk, a.M - 1);
            const _Float16* src = (pl ? a.sl : a.sh) + (int64_t)tg * (K / 32) + 8 * (st >> 3);
            __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)(Ss + ((st >> 3) & 1) * (2 * BM * 16) + wave * 1024),
                                             16, 0, 0);
        }
    };
    // Issues step st's loads: the activation copies first, then the weight
    // registers.  Loads return in issue order, so once a wave has the weight
    // registers of step st its activation copies of step st are in LDS too.
    auto load = [&](Stage& S, int st) __attribute__((always_inline)) {
        load_x(st);
        __builtin_amdgcn_sched_barrier(0);
        load_w<FMT>(S, rowp, st, hf);
    };
    auto store_w = [&](const Stage& S, int st) __attribute__((always_inline)) {
        const int buf = st & 1;
        uint32_t wv[2][8];
        convert_w<FMT>(S, st, hf, wv);
#pragma unroll
        for (int p = 0; p < NP; p++) {
            *reinterpret_cast<v4u*>(waddr(buf, p, srow, 2 * hf)) = v4u{wv[p][0], wv[p][1], wv[p][2], wv[p][3]};
            *reinterpret_cast<v4u*>(waddr(buf, p, srow, 2 * hf + 1)) = v4u{wv[p][4], wv[p][5], wv[p][6], wv[p][7]};
        }
        if (hf == 0) Wd[buf * BN + srow] = (float)__builtin_bit_cast(_Float16, (uint16_t)(S.hdr[0] & 0xFFFFu));
        if constexpr (F::MIN) {
            if ((st & 7) == 0 && hf == 0) {
                const int sp = (st >> 3) & 1;
                Wm[sp * BN + srow] = 32.0f * (float)__builtin_bit_cast(_Float16, (uint16_t)(S.hdr[0] >> 16));
                h8 mv;
#pragma unroll
                for (int gg = 0; gg < 8; gg++)
                    mv[gg] = (_Float16)(float)(k_field12(S.hdr[1], S.hdr[2], S.hdr[3], 12 * gg) >> 6);
                *reinterpret_cast<h8*>(Wq + (sp * BN + srow) * 16) = mv;
            }
        }
    };

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    // One step: issue step st + D's loads, MFMAs on step st, then step st + 1's
    // weights into LDS.  With D == 2, cur (step st, already in LDS) takes step
    // st + 2 and nxt holds step st + 1; with D == 1, nxt takes step st + 1.
    auto step = [&](int st, Stage& cur, Stage& nxt) __attribute__((always_inline)) {
        const int xb = st % NXB, wbuf = st & 1;
        if (st + D < nsteps) load(D == 2 ? cur : nxt, st + D);
        h8 wb[NP][4];
        float d[4];
#pragma unroll
        for (int tj = 0; tj < 4; tj++) {
            const int r = wn * 64 + tj * 16 + lr;
#pragma unroll
            for (int p = 0; p < NP; p++) wb[p][tj] = *reinterpret_cast<const h8*>(waddr(wbuf, p, r, lk));
            d[tj] = Wd[wbuf * BN + r];
        }
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
            const int r = wm * 64 + ti * 16 + lr;
            const h8 x0 = *reinterpret_cast<const h8*>(xaddr(xb, 0, r, lk));
            const h8 x1 = *reinterpret_cast<const h8*>(xaddr(xb, 1, r, lk));
#pragma unroll
            for (int tj = 0; tj < 4; tj++) {
                f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, wb[0][tj], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, wb[0][tj], c, 0, 0, 0);
                if constexpr (NP == 2) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, wb[1][tj], c, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[ti][tj][e] += d[tj] * c[e];
            }
        }
        if constexpr (F::MIN) {
            if ((st & 7) == 7) {   // superblock end: acc -= 32 dmin (sum_g m_g S_g) / 32
                const int sp = (st >> 3) & 1;
#pragma unroll
                for (int tj = 0; tj < 4; tj++) {
                    const int rl = wn * 64 + tj * 16 + lr;
                    const float dm = Wm[sp * BN + rl];
                    h4 mq = h4{0, 0, 0, 0};
                    if (lk < 2) mq = *reinterpret_cast<const h4*>(Wq + (sp * BN + rl) * 16 + 8 * lk);
#pragma unroll
                    for (int ti = 0; ti < 4; ti++) {
                        const int tl = wm * 64 + ti * 16 + lr;
                        h4 s0 = h4{0, 0, 0, 0}, s1 = h4{0, 0, 0, 0};
                        if (lk < 2) {
                            s0 = *reinterpret_cast<const h4*>(Ss + ((sp * 2 + 0) * BM + tl) * 16 + 8 * lk);
                            s1 = *reinterpret_cast<const h4*>(Ss + ((sp * 2 + 1) * BM + tl) * 16 + 8 * lk);
                        }
                        f4 r = __builtin_amdgcn_mfma_f32_16x16x16f16(s0, mq, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        r = __builtin_amdgcn_mfma_f32_16x16x16f16(s1, mq, r, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[ti][tj][e] -= dm * r[e];
                    }
                }
            }
        }
        if (st + 1 < nsteps) store_w(nxt, st + 1);
        lds_barrier();
    };

    Stage S0, S1;
    S0.qh[0] = S0.qh[1] = S0.qh[2] = S0.qh[3] = 0u;
    S1.qh[0] = S1.qh[1] = S1.qh[2] = S1.qh[3] = 0u;
    S0.hdr[1] = S0.hdr[2] = S0.hdr[3] = 0u;
    S1.hdr[1] = S1.hdr[2] = S1.hdr[3] = 0u;
    load(S0, 0);
    if (D == 2 && nsteps > 1) load(S1, 1);
    store_w(S0, 0);
    lds_barrier();
    for (int st = 0; st < nsteps; st += 2) {
        step(st, S0, S1);
        if (st + 1 < nsteps) step(st + 1, S1, S0);
    }

    // epilogue: y = acc / s for token rows; lane holds tokens 4 lk + e of tile ti, row lr of tile tj
    float xi[4][4];
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) xi[ti][e] = a.xinv[min(m0 + wm * 64 + ti * 16 + 4 * lk + e, a.M - 1)];
    if (EPI == PF_SWIGLU) {
        float (*E)[64][65] = reinterpret_cast<float (*)[64][65]>(smem);
        if (wn == 1) {
#pragma unroll
            for (int ti = 0; ti < 4; ti++)
#pragma unroll
                for (int tj = 0; tj < 4; tj++)
#pragma unroll
                    for (int e = 0; e < 4; e++) E[wm][ti * 16 + 4 * lk + e][tj * 16 + lr] = acc[ti][tj][e] * xi[ti][e];
        }
        __syncthreads();
        if (wn == 0) {
            const int n8 = a.N & ~7;
#pragma unroll
            for (int ti = 0; ti < 4; ti++)
#pragma unroll
                for (int tj = 0; tj < 4; tj++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int t = m0 + wm * 64 + ti * 16 + 4 * lk + e;
                        const int row = blockIdx.x * 64 + tj * 16 + lr;
                        if (t < a.M && row < a.N) {
#pragma clang fp contract(off)
                            const float g = acc[ti][tj][e] * xi[ti][e];
                            const float u = E[wm][ti * 16 + 4 * lk + e][tj * 16 + lr];
                            // SiluInPlace then Mul (IE:463-474): ExpApprox on the vector lanes
                            const float sg = row < n8 ? silu_ref(g) : g / (1.0f + expf(-g));
                            a.out[(int64_t)t * a.ldo + row] = sg * u;
                        }
                    }
        }
    } else {
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
            for (int tj = 0; tj < 4; tj++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = m0 + wm * 64 + ti * 16 + 4 * lk + e;
                    const int row = blockIdx.x * BN + wn * 64 + tj * 16 + lr;
                    if (t < a.M && row < a.N) {
                        const float y = acc[ti][tj][e] * xi[ti][e];
                        float* o = a.out + (int64_t)t * a.ldo + row;
                        if (EPI == PF_ADD) {
#pragma clang fp contract(off)
                            *o = *o + y;
                        } else {
                            *o = y;
                        }
                    }
                }
    }
}

// ------------------------------------------------------------ RoPE + KV --

// One workgroup per token of the chunk (position pos0 + t): RoPE on every q
// head (into qr) and k head, K and V written to their cache slots
// (IE:362-381, same per-element arithmetic as the decode path).
__global__ __launch_bounds__(WG) void pf_rope_kv_kernel(PfAttnArgs a) {
    const int t = blockIdx.x, p = a.pos0 + t;
    const int HD = a.head_dim, half = a.rope_half;
    const int qdim = a.heads * HD, kvdim = a.kv_heads * HD;
    const float* cs = a.cos_tab + (int64_t)p * half;
    const float* sn = a.sin_tab + (int64_t)p * half;
    for (int i = threadIdx.x; i < qdim; i += WG) {
        const int h = i / HD, d = i - h * HD;
        a.qr[(int64_t)t * qdim + i] = rope_elem(a.q + (int64_t)t * qdim + h * HD, d, half, cs, sn);
    }
    for (int i = threadIdx.x; i < kvdim; i += WG) {
        const int h = i / HD, d = i - h * HD;
        const int64_t slot = ((int64_t)h * a.context + p) * HD + d;
        store_kv(a.kcache, slot, rope_elem(a.k + (int64_t)t * kvdim + h * HD, d, half, cs, sn), a.kv_fp16);
        store_kv(a.vcache, slot, a.v[(int64_t)t * kvdim + i], a.kv_fp16);
    }
}

// ------------------------------------------------------------- attention --

constexpr int AQ = 64;   // queries per workgroup
constexpr int AK = 64;   // keys per tile

template <int HD>
__device__ __forceinline__ void load_kv_tile(float (*dst)[HD + 4], const void* cache, int64_t base, int j0, int jmax,
                                             int fp16) {
    // AK rows of HD elements, 4 per thread per pass
    for (int c = threadIdx.x; c < AK * HD / 4; c += WG) {
        const int r = c / (HD / 4), q = c - r * (HD / 4);
        const int j = min(j0 + r, jmax);
        const int64_t idx = base + (int64_t)j * HD + 4 * q;
        float4 v;
        if (fp16) {
            const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const _Float16*>(cache) + idx);
            v.x = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x & 0xFFFFu));
            v.y = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x >> 16));
            v.z = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y & 0xFFFFu));
            v.w = (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y >> 16));
        } else {
            v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(cache) + idx);
        }
        *reinterpret_cast<float4*>(&dst[r][4 * q]) = v;
    }
}

// Scores (q . K_j) / sqrt(hd) of 64 queries of one q head against every key
// j <= pos0 + t, into the score scratch, and each query's maximum.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_scores_kernel(PfAttnArgs a) {
    __shared__ __attribute__((aligned(16))) float Qs[AQ][HD + 4];
    __shared__ __attribute__((aligned(16))) float Ks[AK][HD + 4];
    const int t0 = blockIdx.x * AQ, h = blockIdx.y, kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * HD;
    const int tid = threadIdx.x, tq = tid >> 4, tk = tid & 15;
    for (int c = tid; c < AQ * HD / 4; c += WG) {
        const int r = c / (HD / 4), q = c - r * (HD / 4);
        const int t = min(t0 + r, a.T - 1);
        *reinterpret_cast<float4*>(&Qs[r][4 * q]) =
            *reinterpret_cast<const float4*>(a.qr + (int64_t)t * qdim + h * HD + 4 * q);
    }
    const int nkeys = a.pos0 + min(t0 + AQ, a.T);   // keys 0 .. pos0 + last query
    const int64_t kbase = (int64_t)kvh * a.context * HD;
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    float rmax[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int j0 = 0; j0 < nkeys; j0 += AK) {
        __syncthreads();
        load_kv_tile<HD>(Ks, a.kcache, kbase, j0, nkeys - 1, a.kv_fp16);
        __syncthreads();
        float s[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) s[i][j] = 0.f;
#pragma unroll 4
        for (int d = 0; d < HD; d += 4) {
            float4 qv[4], kv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qv[i] = *reinterpret_cast<const float4*>(&Qs[4 * tq + i][d]);
#pragma unroll
            for (int j = 0; j < 4; j++) kv[j] = *reinterpret_cast<const float4*>(&Ks[4 * tk + j][d]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    s[i][j] += qv[i].x * kv[j].x + qv[i].y * kv[j].y + qv[i].z * kv[j].z + qv[i].w * kv[j].w;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 4 * tq + i;
            if (t >= a.T) continue;
            const int p = a.pos0 + t;
            float* srow = a.scores + ((int64_t)h * a.T + t) * a.ld_scores;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int key = j0 + 4 * tk + j;
                if (key <= p) {
                    const float sc = s[i][j] * inv_sqrt;
                    srow[key] = sc;
                    rmax[i] = fmaxf(rmax[i], sc);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float m = rmax[i];
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        const int t = t0 + 4 * tq + i;
        if (tk == 0 && t < a.T) a.rowmax[(int64_t)h * a.T + t] = m;
    }
}

// Softmax (VectorMath.Softmax, VM:215-258: ExpApprox(s - max) on the first
// 8 floor(n/8) scores, expf on the tail) and out = sum_j e_j V_j / sum_j e_j
// for 64 queries of one q head.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_pv_kernel(PfAttnArgs a) {
    constexpr int DPT = HD / 16;
    __shared__ __attribute__((aligned(16))) float Vs[AK][HD + 4];
    __shared__ float Es[AQ][AK + 1];
    __shared__ float Ms[AQ];
    const int t0 = blockIdx.x * AQ, h = blockIdx.y, kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * HD;
    const int tid = threadIdx.x, tq = tid >> 4, td = tid & 15;
    if (tid < AQ) Ms[tid] = a.rowmax[(int64_t)h * a.T + min(t0 + tid, a.T - 1)];
    const int nkeys = a.pos0 + min(t0 + AQ, a.T);
    const int64_t vbase = (int64_t)kvh * a.context * HD;
    float acc[4][DPT], z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int d = 0; d < DPT; d++) acc[i][d] = 0.f;
    for (int j0 = 0; j0 < nkeys; j0 += AK) {
        __syncthreads();
        load_kv_tile<HD>(Vs, a.vcache, vbase, j0, nkeys - 1, a.kv_fp16);
        for (int c = tid; c < AQ * AK; c += WG) {
            const int qi = c >> 6, kj = c & 63;
            const int t = t0 + qi, key = j0 + kj;
            float e = 0.f;
            if (t < a.T) {
                const int n = a.pos0 + t + 1, n8 = n & ~7;
                if (key < n) {
#pragma clang fp contract(off)
                    const float x = a.scores[((int64_t)h * a.T + t) * a.ld_scores + key] - Ms[qi];
                    e = key < n8 ? exp_approx(x) : expf(x);
                }
            }
            Es[qi][kj] = e;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < 4; k++) z[i] += Es[4 * tq + i][4 * td + k];
#pragma unroll 4
        for (int kj = 0; kj < AK; kj++) {
            float ev[4], vv[DPT];
#pragma unroll
            for (int i = 0; i < 4; i++) ev[i] = Es[4 * tq + i][kj];
#pragma unroll
            for (int d = 0; d < DPT; d++) vv[d] = Vs[kj][td * DPT + d];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int d = 0; d < DPT; d++) acc[i][d] += ev[i] * vv[d];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float zz = z[i];
        zz += __shfl_xor(zz, 1, 64);
        zz += __shfl_xor(zz, 2, 64);
        zz += __shfl_xor(zz, 4, 64);
        zz += __shfl_xor(zz, 8, 64);
        const int t = t0 + 4 * tq + i;
        if (t < a.T) {
            const float inv = 1.0f / zz;
#pragma unroll
            for (int d = 0; d < DPT; d++) a.out[(int64_t)t * qdim + h * HD + td * DPT + d] = acc[i][d] * inv;
        }
    }
}

// ---- attention on MFMA (fp16 KV cache) ----
//
// K and V are fp16 in the cache, so they are exact MFMA operands; q (per
// query row and head) and the softmax numerators e are fp32 and enter as two
// fp16 planes each (22-bit significands), with fp32 accumulation, so scores
// and outputs carry fp32-level rounding only.  Wave w of a workgroup owns
// queries t0 + 16 w .. + 15 of one q head; keys advance 64 per tile.

constexpr int KPAD = 8;   // halves of row padding in the K / V^T tiles

// Scores (q . K_j) / sqrt(hd) into the score scratch plus each query's maximum.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_scores_mfma(PfAttnArgs a) {
    constexpr int KS = HD / 32;   // MFMA k-steps over the head dimension
    __shared__ __attribute__((aligned(16))) _Float16 Ks[AK][HD + KPAD];
    const int t0 = blockIdx.x * AQ, h = blockIdx.y, kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lk = lane >> 4;
    // this lane's q elements (query lr of the wave, dims 32 ks + 8 lk .. +7) as two planes
    const int tq = min(t0 + 16 * wave + lr, a.T - 1);
    const float* qrow = a.qr + (int64_t)tq * qdim + h * HD;
    float qv[KS][8];
    float amax = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const float4 u = *reinterpret_cast<const float4*>(qrow + 32 * ks + 8 * lk);
        const float4 v = *reinterpret_cast<const float4*>(qrow + 32 * ks + 8 * lk + 4);
        qv[ks][0] = u.x; qv[ks][1] = u.y; qv[ks][2] = u.z; qv[ks][3] = u.w;
        qv[ks][4] = v.x; qv[ks][5] = v.y; qv[ks][6] = v.z; qv[ks][7] = v.w;
#pragma unroll
        for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(qv[ks][i]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    int e = 0;
    if (amax > 0.f) {
        (void)frexpf(amax, &e);
        e = 15 - e;
        e = e > 126 ? 126 : (e < -126 ? -126 : e);
    }
    const float sq = ldexpf(1.0f, e);
    h8 qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float x = qv[ks][i] * sq;
            const _Float16 hi = (_Float16)x;
            qh[ks][i] = hi;
            ql[ks][i] = (_Float16)(x - (float)hi);
        }
    // output rows are queries 4 lk + r: their scale factors (held by lanes 4 lk + r)
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    float oscale[4];
#pragma unroll
    for (int r = 0; r < 4; r++) oscale[r] = inv_sqrt * ldexpf(1.0f, -__shfl(e, 4 * lk + r, 64));

    const int nkeys = a.pos0 + min(t0 + AQ, a.T);
    const int64_t kbase = (int64_t)kvh * a.context * HD;
    const _Float16* kc = reinterpret_cast<const _Float16*>(a.kcache);
    float rmax[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int j0 = 0; j0 < nkeys; j0 += AK) {
        __syncthreads();
        for (int c = tid; c < AK * HD / 8; c += WG) {   // 16-byte chunks of the K tile
            const int r = c / (HD / 8), q = c - r * (HD / 8);
            const int j = min(j0 + r, nkeys - 1);
            *reinterpret_cast<v4u*>(&Ks[r][8 * q]) = *reinterpret_cast<const v4u*>(kc + kbase + (int64_t)j * HD + 8 * q);
        }
        __syncthreads();
#pragma unroll
        for (int kt = 0; kt < AK / 16; kt++) {
            f4 c = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const h8 kf = *reinterpret_cast<const h8*>(&Ks[kt * 16 + lr][32 * ks + 8 * lk]);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], kf, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[ks], kf, c, 0, 0, 0);
            }
            const int key = j0 + kt * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = t0 + 16 * wave + 4 * lk + r;
                if (t < a.T && key <= a.pos0 + t) {
                    const float sc = c[r] * oscale[r];
                    a.scores[((int64_t)h * a.T + t) * a.ld_scores + key] = sc;
                    rmax[r] = fmaxf(rmax[r], sc);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float m = rmax[r];
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        const int t = t0 + 16 * wave + 4 * lk + r;
        if (lr == 0 && t < a.T) a.rowmax[(int64_t)h * a.T + t] = m;
    }
}

// Softmax numerators (ExpApprox on the first 8 floor(n/8) keys, expf on the
// tail, VM:215-258) and out = sum_j e_j V_j / sum_j e_j.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_pv_mfma(PfAttnArgs a) {
    constexpr int DT = HD / 16;   // 16-wide output tiles over the head dimension
    __shared__ __attribute__((aligned(16))) _Float16 Vt[HD][AK + KPAD];   // V^T tile
    const int t0 = blockIdx.x * AQ, h = blockIdx.y, kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lk = lane >> 4;
    const int tA = t0 + 16 * wave + lr;                 // this lane's A-operand query
    const bool liveA = tA < a.T;
    const int tAc = min(tA, a.T - 1);
    const int nA = a.pos0 + tAc + 1, n8A = nA & ~7;     // keys of that query, vector-lane part
    const float mA = a.rowmax[(int64_t)h * a.T + tAc];
    const float* srow = a.scores + ((int64_t)h * a.T + tAc) * a.ld_scores;
    const int nkeys = a.pos0 + min(t0 + AQ, a.T);
    const int64_t vbase = (int64_t)kvh * a.context * HD;
    const _Float16* vc = reinterpret_cast<const _Float16*>(a.vcache);
    const float P14 = 16384.0f;
    f4 acc[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
    float z = 0.f;
    for (int j0 = 0; j0 < nkeys; j0 += AK) {
        __syncthreads();
        for (int c = tid; c < AK * HD / 8; c += WG) {   // V rows -> V^T; a wave writes 64 consecutive keys
            const int r = c & (AK - 1), q = c / AK;
            const int j = min(j0 + r, nkeys - 1);
            const h8 v = *reinterpret_cast<const h8*>(vc + vbase + (int64_t)j * HD + 8 * q);
#pragma unroll
            for (int i = 0; i < 8; i++) Vt[8 * q + i][r] = v[i];
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < AK / 32; kk++) {
            const int kb = j0 + kk * 32 + 8 * lk;   // this lane's 8 keys
            h8 eh, el;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int key = kb + i;
                float ev = 0.f;
                if (liveA && key < nA) {
#pragma clang fp contract(off)
                    const float x = srow[key] - mA;
                    ev = key < n8A ? exp_approx(x) : expf(x);
                }
                z += ev;
                const float xs = ev * P14;
                const _Float16 hi = (_Float16)xs;
                eh[i] = hi;
                el[i] = (_Float16)(xs - (float)hi);
            }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const h8 vf = *reinterpret_cast<const h8*>(&Vt[dt * 16 + lr][kk * 32 + 8 * lk]);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(eh, vf, acc[dt], 0, 0, 0);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(el, vf, acc[dt], 0, 0, 0);
            }
        }
    }
    z += __shfl_xor(z, 16, 64);
    z += __shfl_xor(z, 32, 64);   // lanes lr, lr+16, ... hold query lr's sum
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int ql = 4 * lk + r;
        const float zq = __shfl(z, ql, 64);
        const int t = t0 + 16 * wave + ql;
        if (t < a.T) {
            const float inv = 1.0f / zq;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
                a.out[(int64_t)t * qdim + h * HD + dt * 16 + lr] = (acc[dt][r] * (1.0f / P14)) * inv;
        }
    }
}

template <uint32_t FMT>
hipError_t launch_gemm_fmt(int epi, const PfGemmArgs& a, hipStream_t s) {
    const dim3 grid(epi == PF_SWIGLU ? (a.N + 63) / 64 : (a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
    switch (epi) {
    case PF_STORE: pf_gemm_kernel<FMT, PF_STORE><<<grid, WG, 0, s>>>(a); break;
    case PF_ADD: pf_gemm_kernel<FMT, PF_ADD><<<grid, WG, 0, s>>>(a); break;
    case PF_SWIGLU: pf_gemm_kernel<FMT, PF_SWIGLU><<<grid, WG, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(const PfAttnArgs& a, hipStream_t s) {
    const dim3 grid((a.T + AQ - 1) / AQ, a.heads);
    if (a.kv_fp16) pf_attn_scores_mfma<HD><<<grid, WG, 0, s>>>(a);
    else pf_attn_scores_kernel<HD><<<grid, WG, 0, s>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.kv_fp16) pf_attn_pv_mfma<HD><<<grid, WG, 0, s>>>(a);
    else pf_attn_pv_kernel<HD><<<grid, WG, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

bool prefill_gemm_supported(uint32_t type, int cols) {
    switch (type) {
    case GGML_Q4_K: case GGML_Q5_K: case GGML_Q6_K: return cols > 0 && cols % 256 == 0;
    case GGML_Q8_0: case GGML_Q4_0: return cols > 0 && cols % 32 == 0;
    default: return false;
    }
}

hipError_t launch_prefill_planes(const float* x, int M, int K, const float* norm_w, float eps, const PfPlanes& p,
                                 hipStream_t s) {
    if (M <= 0 || K <= 0 || K % 32) return hipErrorInvalidValue;
    if (norm_w) pf_planes_kernel<true><<<M, WG, 0, s>>>(x, K, norm_w, eps, p.xh, p.xl, p.sh, p.sl, p.xinv);
    else pf_planes_kernel<false><<<M, WG, 0, s>>>(x, K, nullptr, eps, p.xh, p.xl, p.sh, p.sl, p.xinv);
    return hipGetLastError();
}

hipError_t launch_prefill_gemm(uint32_t type, int epi, const PfPlanes& p, const uint8_t* w, const uint8_t* w2, int M,
                               int N, int K, float* out, int ldo, hipStream_t s) {
    if (M <= 0 || N <= 0 || !prefill_gemm_supported(type, K) || (epi == PF_SWIGLU && !w2) || ldo < N)
        return hipErrorInvalidValue;
    PfGemmArgs a{p.xh, p.xl, p.sh, p.sl, p.xinv, w, w2, out, M, N, K, ldo};
    switch (type) {
    case GGML_Q4_K: return launch_gemm_fmt<GGML_Q4_K>(epi, a, s);
    case GGML_Q5_K: return launch_gemm_fmt<GGML_Q5_K>(epi, a, s);
    case GGML_Q6_K: return launch_gemm_fmt<GGML_Q6_K>(epi, a, s);
    case GGML_Q8_0: return launch_gemm_fmt<GGML_Q8_0>(epi, a, s);
    case GGML_Q4_0: return launch_gemm_fmt<GGML_Q4_0>(epi, a, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prefill_rope_kv(const PfAttnArgs& a, hipStream_t s) {
    if (a.T <= 0) return hipErrorInvalidValue;
    pf_rope_kv_kernel<<<a.T, WG, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PfAttnArgs& a, hipStream_t s) {
    if (a.T <= 0 || a.heads % a.kv_heads) return hipErrorInvalidValue;
    switch (a.head_dim) {
    case 64: return launch_attn_hd<64>(a, s);
    case 96: return launch_attn_hd<96>(a, s);
    case 128: return launch_attn_hd<128>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace llmdot
