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
//    Q8_0: d * q; Q4_0: d * (q - 8), DequantizeK.cs / DequantizeBlock.cs).  The
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
// all 128 tokens and rows 32 w .. 32 w + 31 as 8 x 2 MFMA tiles, so each
// wave dequantises only its own 32 rows.  K advances 32 per step (one MFMA
// K).  Each step's activation planes and raw weight blocks are copied
// global -> LDS by the waves (global_load_lds, no registers) one step ahead
// into two LDS stages; each wave then builds its weight fragments from the
// raw bytes in LDS.  Launches that would have few tiles use 64-token tiles
// (128 to 255 tiles) or split K into parts summed by the next kernel (under
// 128 tiles).
#include "common.h"
#include "kernels.h"

// dma16 below names m0 (the LDS base of global_load_lds) as clobbered; nothing
// else in this file keeps a value in m0.
#pragma clang diagnostic ignored "-Winline-asm"

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
    // The thread's y values, 4 consecutive elements per 1024-element block,
    // read once and kept in registers (K <= 16384), or re-read below.
    constexpr int NB = 16;
    const bool held = K <= NB * 4 * WG;
    float yr[NB][4];
    float amax = 0.f;
    if (held) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int base = b * 4 * WG + 4 * tid;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                yr[b][j] = base < K ? yval(base + j) : 0.f;   // K % 32 == 0: whole quads
                amax = fmaxf(amax, fabsf(yr[b][j]));
            }
        }
    } else {
        for (int i = tid; i < K; i += WG) amax = fmaxf(amax, fabsf(yval(i)));
    }
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
    auto emit = [&](const int base, const float* y) __attribute__((always_inline)) {
        float g = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) g += y[j];
        g = sum8(g);
        if (base < K) {
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
    };
    if (held) {
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (b * 4 * WG < K) emit(b * 4 * WG + 4 * tid, yr[b]);   // uniform: every lane calls sum8
    } else {
        for (int b0 = 0; b0 < K; b0 += 4 * WG) {
            const int base = b0 + 4 * tid;
            float y[4];
#pragma unroll
            for (int j = 0; j < 4; j++) y[j] = base < K ? yval(base + j) : 0.f;
            emit(base, y);
        }
    }
}

// ------------------------------------------------------------------ GEMM --

struct PfGemmArgs {
    const _Float16 *xh, *xl, *sh, *sl;   // [M][K], [M][K], [M][K/32] x2
    const float* xinv;                   // [M]
    const uint8_t* w;                    // [N][row bytes] GGUF blocks
    const uint8_t* w2;                   // SWIGLU: the up matrix (w = gate)
    float* out;                          // [M][ldo]; K part p (split) at out + p * part_stride
    int M, N, K, ldo;
    int tiles_n;                         // weight-row tiles (128 rows; SWIGLU: 64 gate + 64 up)
    int ksplit;                          // K parts (STORE only): each a whole number of blocks
    int64_t part_stride;
    // STORE with a second matrix: row tiles from tn_b on read wb [nb rows]
    // into outb [M][ldob] (tn_b = tiles_n: none)
    const uint8_t* wb;
    float* outb;
    int tn_b, nb, ldob;
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

// Weight formats on the batched path.  Per 32-element step a row contributes
// R 16-byte chunks of raw block bytes.  K-quants (16-byte aligned blocks) keep
// chunk ch of all 128 rows together in LDS ([ch][row]: a fragment read of 16
// rows touches 256 contiguous bytes); the 2-byte aligned formats copy windows
// starting at the block address rounded down to 4 bytes ([row][ch]).
// Every step's partial sum is scaled by the row's block scale d; NP = weight
// planes; NS = LDS stages (prefetch distance NS - 1).  RH > 0: the weights
// are staged once per 4 steps instead, RH chunks per row.  Q6_K: the 4 steps
// of a half superblock read the same qh bytes and pairs of them the same ql
// bytes, which a per-step copy fetched again each time (128 bytes per row and
// step for ~68 used); Q8_0: 4 blocks of 34 bytes in 10 chunks instead of 4
// per block (the last a repeat).
template <uint32_t FMT>
struct PfFmt;
template <>
struct PfFmt<GGML_Q4_K> { static constexpr int BSZ = 144, EPB = 256, R = 2, NP = 1, NS = 2, RH = 0; static constexpr bool MIN = true, KQ = true; };
template <>
struct PfFmt<GGML_Q5_K> { static constexpr int BSZ = 176, EPB = 256, R = 4, NP = 1, NS = 2, RH = 0; static constexpr bool MIN = true, KQ = true; };
template <>
struct PfFmt<GGML_Q6_K> { static constexpr int BSZ = 210, EPB = 256, R = 8, NP = 2, NS = 2, RH = 10; static constexpr bool MIN = false, KQ = false; };
template <>
struct PfFmt<GGML_Q8_0> { static constexpr int BSZ = 34, EPB = 32, R = 4, NP = 1, NS = 2, RH = 10; static constexpr bool MIN = false, KQ = false; };
template <>
struct PfFmt<GGML_Q4_0> { static constexpr int BSZ = 18, EPB = 32, R = 2, NP = 1, NS = 2, RH = 0; static constexpr bool MIN = false, KQ = false; };

// K-quants: byte offset of chunk ch of group g within a superblock.
template <uint32_t FMT>
__device__ __forceinline__ int kq_chunk_off(int ch, int g) {
    if constexpr (FMT == GGML_Q4_K) return ch == 0 ? 0 : 16 + 16 * g;                          // header | quants of g
    else return ch == 0 ? 0 : ch == 1 ? 48 + 16 * g : 16 + 16 * (g >> 2);                   // header | low nibbles | high bits
}
// Q4_0: byte offset (from the row start) of the window that chunk ch of step
// st belongs to, and the chunk's index inside that window.
template <uint32_t FMT>
__device__ __forceinline__ void win_chunk(int st, int ch, int64_t* off, int* k) {
    *off = (int64_t)st * PfFmt<FMT>::BSZ;   // the block
    *k = ch < 2 ? ch : 2;
}

// Q6_K half-superblock stage (steps 4 h .. 4 h + 3 of a superblock share it):
// chunks 0-4 cover the 64 ql bytes at 64 h, 5-7 the 32 qh bytes at 128 + 32 h,
// 8-9 the scales and d at 192; each window starts at its offset rounded down
// to 4 bytes.  Byte offset (from the row start) of chunk ch's window, and the
// chunk's index inside it.
__device__ __forceinline__ void q6_half_chunk(int st, int ch, int64_t* off, int* k) {
    const int h = (st >> 2) & 1;
    const int64_t blk = (int64_t)(st >> 3) * 210;
    *off = blk + (ch < 5 ? 64 * h : ch < 8 ? 128 + 32 * h : 192);
    *k = ch < 5 ? ch : ch < 8 ? ch - 5 : ch - 8;
}

// Q8_0 stage: the 4 blocks of steps 4 j .. 4 j + 3 (136 bytes) in 10 chunks
// from the first block's offset rounded down to 4 bytes.
__device__ __forceinline__ void q8_quad_chunk(int st, int ch, int64_t* off, int* k) {
    *off = (int64_t)(st & ~3) * 34;
    *k = ch;
}

// Stage window of chunk ch for step st (formats with PfFmt::RH > 0).
template <uint32_t FMT>
__device__ __forceinline__ void staged_chunk(int st, int ch, int64_t* off, int* k) {
    if constexpr (FMT == GGML_Q6_K) q6_half_chunk(st, ch, off, k);
    else q8_quad_chunk(st, ch, off, k);
}

// 8 bytes starting at byte offset o (any alignment) of an LDS array, as 2 words.
__device__ __forceinline__ void lds_bytes8(const unsigned char* p, int o, uint32_t* w) {
    const uint32_t* d = reinterpret_cast<const uint32_t*>(p + (o & ~3));
    const uint32_t sh = (uint32_t)(o & 3);
    const uint32_t a = d[0], b = d[1], c = d[2];
    w[0] = __builtin_amdgcn_alignbyte(b, a, sh);
    w[1] = __builtin_amdgcn_alignbyte(c, b, sh);
}

// K-quant B fragment: elements 8 lk .. 8 lk + 7 of group g for the row whose
// header words 1..3 (bytes 4..15, the packed scales) are hw and whose quant
// chunk(s) start at qs (next chunk 2048 bytes further): fp16 sc * (q - 8|16),
// exact.  The header comes from registers: an 8-byte LDS read of it would sit
// at a 4-byte-aligned address for 5 of the 8 groups, which the LDS serves an
// order of magnitude slower than an aligned one.
template <uint32_t FMT>
__device__ __forceinline__ h8 kq_frag(v4u hw, const unsigned char* qs, int g, int lk) {
    const _Float16 sc = (_Float16)(float)(k_field12(hw[1], hw[2], hw[3], 12 * g) & 63u);
    const uint32_t w = reinterpret_cast<const uint32_t*>(qs)[lk];
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    uint32_t n0 = perm(hi, lo, 0x05010400u), n1 = perm(hi, lo, 0x07030602u);
    uint32_t pr[4];
    if constexpr (FMT == GGML_Q5_K) {
        const uint32_t hb = qs[2048 + 4 * (g & 3) + lk];
        n0 |= (((hb & 15u) * 0x00204081u) & 0x01010101u) << 4;
        n1 |= ((((hb >> 4) & 15u) * 0x00204081u) & 0x01010101u) << 4;
        bytes_to_h2(n0, (_Float16)1040.f, sc, &pr[0]);
        bytes_to_h2(n1, (_Float16)1040.f, sc, &pr[2]);
    } else {
        bytes_to_h2(n0, (_Float16)1032.f, sc, &pr[0]);
        bytes_to_h2(n1, (_Float16)1032.f, sc, &pr[2]);
    }
    return __builtin_bit_cast(h8, v4u{pr[0], pr[1], pr[2], pr[3]});
}

// Windowed B fragment for the row whose R chunks start at raw; rowoff = the
// row's byte offset in the tensor (window alignment shifts).
template <uint32_t FMT>
__device__ __forceinline__ void win_frag(const unsigned char* raw, int st, int lk, int64_t rowoff, h8* out, float* d) {
    uint32_t pr[4];
    if constexpr (FMT == GGML_Q6_K) {
        // raw: this row's half-superblock stage (q6_half_chunk)
        const int g = st & 7, h = g >> 2, qq = g & 3;
        const int64_t blk = rowoff + (int64_t)(st >> 3) * 210;
        const int sA = (int)((blk + 64 * h) & 3), sB = (int)((blk + 128 + 32 * h) & 3);
        const int sC = (int)((blk + 192) & 3);
        uint32_t ql[2], qh[2];
        lds_bytes8(raw, sA + (qq & 1) * 32 + 8 * lk, ql);
        lds_bytes8(raw + 80, sB + 8 * lk, qh);
        const int scv = (int)(int8_t)raw[128 + sC + 2 * g + (lk >> 1)];
        const uint32_t dw = reinterpret_cast<const uint32_t*>(raw + 128)[(sC + 16) >> 2];
        *d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw >> (8 * ((sC + 16) & 3))));
        const h2 sc2 = {(_Float16)(float)scv, (_Float16)(float)scv};
        const h2 off = {(_Float16)1056.f, (_Float16)1056.f};
        const uint32_t nsh = 4 * (qq >> 1), qsh = 2 * qq;
        uint32_t ph[4], pl[4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t qb = ((ql[j] >> nsh) & 0x0F0F0F0Fu) | (((qh[j] >> qsh) & 0x03030303u) << 4);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const h2 qv = as_h2(perm(0x64646464u, qb, p ? 0x04030402u : 0x04010400u)) - off;   // q - 32
                const h2 vh = qv * sc2;
                ph[2 * j + p] = as_u(vh);
                pl[2 * j + p] = as_u(__builtin_elementwise_fma(qv, sc2, -vh));
            }
        }
        out[0] = __builtin_bit_cast(h8, v4u{ph[0], ph[1], ph[2], ph[3]});
        out[1] = __builtin_bit_cast(h8, v4u{pl[0], pl[1], pl[2], pl[3]});
    } else if constexpr (FMT == GGML_Q8_0) {   // raw: this row's 4-block stage (q8_quad_chunk)
        const int o = (int)((rowoff + (int64_t)(st & ~3) * 34) & 3) + 34 * (st & 3);   // block start, even
        const uint32_t dw = reinterpret_cast<const uint32_t*>(raw)[o >> 2];
        *d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw >> (8 * (o & 3))));
        uint32_t q[2];
        lds_bytes8(raw, o + 2 + 8 * lk, q);
        bytes_to_h2(q[0] ^ 0x80808080u, (_Float16)1152.f, (_Float16)1.f, &pr[0]);
        bytes_to_h2(q[1] ^ 0x80808080u, (_Float16)1152.f, (_Float16)1.f, &pr[2]);
        out[0] = __builtin_bit_cast(h8, v4u{pr[0], pr[1], pr[2], pr[3]});
    } else {   // Q4_0: window shift s = block offset & 3; d at s, payload at s + 2
        const int sh = (int)((rowoff + (int64_t)st * PfFmt<FMT>::BSZ) & 3);
        const uint32_t dw = reinterpret_cast<const uint32_t*>(raw)[0];
        *d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw >> (8 * sh)));
        uint32_t q[2];
        // elements 0..15: low nibbles of bytes 0..15; 16..31: high nibbles
        lds_bytes8(raw, sh + 2 + 8 * (lk & 1), q);
        const uint32_t sft = lk < 2 ? 0u : 4u;
        bytes_to_h2((q[0] >> sft) & 0x0F0F0F0Fu, (_Float16)1032.f, (_Float16)1.f, &pr[0]);
        bytes_to_h2((q[1] >> sft) & 0x0F0F0F0Fu, (_Float16)1032.f, (_Float16)1.f, &pr[2]);
        out[0] = __builtin_bit_cast(h8, v4u{pr[0], pr[1], pr[2], pr[3]});
    }
}

enum PfEpi : int { PF_STORE = 0, PF_ADD = 1, PF_SWIGLU = 2 };

// 16 bytes per lane from global memory straight into LDS: lane i reads
// base + off_i and writes LDS bytes [lds + 16 i, lds + 16 i + 16) (base and
// lds wave-uniform).  Issued as inline assembly so that the compiler's
// wait-count bookkeeping does not serialise it; completion is awaited
// explicitly with vm_wait below.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
// Waits until at most N of this wave's vector memory operations are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
// Workgroup barrier after this wave's LDS operations (no wait on global loads).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS rows of 32 halves (64 bytes) hold 4 chunks of 8; chunk c of row r sits
// at position c ^ swz(r), swz(r) = (r >> 1) & 3 (the same for rows 16 i + l
// and l).  An MFMA fragment read (16 rows x 4 chunks, lane 16 c + l reading
// chunk c of row l) then takes one LDS pass: measured on gfx950, conflict-free
// like a read of consecutive 16-byte words, where the unswizzled order and
// other XOR patterns take two.  A copy instruction still covers 16 tokens'
// contiguous 64 bytes, 4 lanes each (the chunk-major layout, also
// conflict-free to read, made the copies slower than it saved).
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 3; }

// TM tokens per workgroup: BM, or 64 for launches that would have only 128
// to 255 tiles of BM (all CUs busy; each output's sum runs in the same order).
template <uint32_t FMT, int EPI, int TM = BM>
__global__ __launch_bounds__(WG, 2) void pf_gemm_kernel(PfGemmArgs a) {
    using F = PfFmt<FMT>;
    static_assert(TM == BM || (TM == 64 && EPI != PF_SWIGLU), "64-token tiles: STORE and ADD only");
    constexpr int NP = F::NP, R = F::R, NS = F::NS;
    constexpr int TI = TM / 16, TJ = BN / 16 / 4;    // wave w: all TM tokens x rows 16 TJ w .. +16 TJ - 1
    constexpr bool WH = F::RH > 0;                   // weights staged once per 4 steps
    constexpr int XS1 = 2 * TM * 64;                 // activation stage: [plane][token][32 halves]
    constexpr int WS1 = WH ? 0 : BN * R * 16;        // raw weight stage (per step)
    constexpr int WSH = WH ? BN * F::RH * 16 : 0;    // raw weight stage (per 4 steps), two of them
    constexpr int ST1 = XS1 + WS1;
    constexpr int SS_B = F::MIN ? 2 * 2 * TM * 16 : 0;   // [sb parity][plane][token][8] group sums
    constexpr int STAGE_B = NS * ST1 + SS_B + 2 * WSH;
    constexpr int EX_B = 2 * TM * (16 * TJ + 1) * 4;     // SWIGLU exchange: [gate wave][token][rows + 1]
    constexpr int SMEM = STAGE_B > EX_B ? STAGE_B : EX_B;
    constexpr int NX = TM / 32, NW = WH ? BN * F::RH / 256 : R / 2;   // DMA instructions per wave (weights: per stage)
    constexpr int XPI = TM / 16;                     // activation DMA instructions per plane
    __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
    const uint32_t sm = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    unsigned char* const Ss = smem + NS * ST1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lk = lane >> 4;
    // XCD-aware tile order: workgroup L runs on XCD L % 8, which takes the
    // contiguous tile range [xcd * per, (xcd + 1) * per) in token-tile-major
    // order, so the workgroups resident on one XCD share a token tile and its
    // activation stream stays in that XCD's L2.
    // With a K split, tile = (part * ntm + token tile) * ntn + row tile: the
    // workgroups of one XCD still share one token tile and K range.
    const int ntm = (a.M + TM - 1) / TM, ntn = a.tiles_n, per = (ntm * ntn * a.ksplit + 7) / 8;
    const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (tile >= ntm * ntn * a.ksplit) return;
    const int tn = tile % ntn, m0 = ((tile / ntn) % ntm) * TM, part = tile / (ntn * ntm);
    const int K = a.K, spp = K / 32 / a.ksplit;   // 32-element steps per part
    const int st0 = part * spp, st1 = st0 + spp;
    const int64_t rbytes = (int64_t)(K / F::EPB) * F::BSZ;
    // the matrix this row tile reads (uniform per workgroup): the second one
    // from row tile tn_b on
    const bool segb = EPI == PF_STORE && tn >= a.tn_b;
    const int tnl = segb ? tn - a.tn_b : tn, Nl = segb ? a.nb : a.N;
    const uint8_t* const wseg = segb ? a.wb : a.w;
    auto grow_of = [&](int r) {   // tile row -> weight row (SWIGLU: rows 0..63 gate, 64..127 up)
        const int g = EPI == PF_SWIGLU ? tn * 64 + (r & 63) : tnl * BN + r;
        return min(g, Nl - 1);
    };
    auto wsel = [&](int r) -> const uint8_t* { return EPI == PF_SWIGLU && r >= 64 ? a.w2 : wseg; };

    // DMA sources.  Activations: instruction i of wave wv covers stage slots
    // q = (NX wv + i) 64 + lane: plane q / (4 TM), token (q >> 2) % TM,
    // position q & 3 holding chunk (q & 3) ^ swz(token).
    uint32_t xoff[NX];
#pragma unroll
    for (int i = 0; i < NX; i++) {
        const int q = (NX * wv + i) * 64 + lane;
        const int tk = (q >> 2) & (TM - 1), c = (q & 3) ^ swz(tk);
        xoff[i] = (uint32_t)(((int64_t)min(m0 + tk, a.M - 1) * K + 8 * c) * 2);
    }
    // Weights: K-quants: slot q = ch * 128 + row (ch uniform per instruction);
    // others: slot q = row * R + ch.
    uint32_t woff[NW];
    int64_t wrow[NW];
#pragma unroll
    for (int j = 0; j < NW; j++) {
        const int q = (NW * wv + j) * 64 + lane;
        const int r = F::KQ ? (q & 127) : q / (WH ? F::RH : R);
        wrow[j] = (int64_t)grow_of(r) * rbytes;
        woff[j] = (uint32_t)wrow[j];
    }
    uint32_t soff = 0;
    if (F::MIN) soff = (uint32_t)((int64_t)min(m0 + ((wv * 64 + lane) & (TM - 1)), a.M - 1) * (K / 32) * 2);

    auto issue = [&](int st) __attribute__((always_inline)) {
        const uint32_t lb = sm + (uint32_t)((st % NS) * ST1);
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const char* xb = reinterpret_cast<const char*>((NX * wv + i) >= XPI ? a.xl : a.xh) + 64 * st;
            dma16(xb, xoff[i], lb + (NX * wv + i) * 1024);
        }
#pragma unroll
        for (int j = 0; j < NW; j++) {
            const int q0 = (NW * wv + j) * 64;
            if constexpr (F::KQ) {
                // chunk 0 (the header) is read only at a superblock's first step
                if ((q0 >> 7) != 0 || (st & 7) == 0) {
                    const uint8_t* wb = wsel(q0 & 127) + (int64_t)(st >> 3) * F::BSZ + kq_chunk_off<FMT>(q0 >> 7, st & 7);
                    dma16(wb, woff[j], lb + XS1 + (NW * wv + j) * 1024);
                }
            } else if constexpr (WH) {   // a new stage every 4 steps (and at a part's first step)
                if ((st & 3) == 0 || st == st0) {
                    int64_t off;
                    int k;
                    staged_chunk<FMT>(st, (q0 + lane) % F::RH, &off, &k);
                    const uint32_t o = (uint32_t)(((wrow[j] + off) & ~int64_t(3)) + 16 * k);
                    dma16(wsel(q0 / F::RH), o,
                          sm + (uint32_t)(NS * ST1 + SS_B + ((st >> 2) & 1) * WSH + (NW * wv + j) * 1024));
                }
            } else {
                int64_t off;
                int k;
                win_chunk<FMT>(st, (q0 + lane) % R, &off, &k);
                const uint32_t o = (uint32_t)(((wrow[j] + off) & ~int64_t(3)) + 16 * k);
                dma16(wsel(q0 / R), o, lb + XS1 + (NW * wv + j) * 1024);
            }
        }
        if (F::MIN && (st & 7) == 0 && wv < TM / 32) {   // TM / 32 x 1 KB of group sums
            const char* sbase = reinterpret_cast<const char*>(wv >= TM / 64 ? a.sl : a.sh) + 16 * (st >> 3);
            dma16(sbase, soff, sm + (uint32_t)(NS * ST1 + ((st >> 3) & 1) * (2 * TM * 16) + wv * 1024));
        }
    };
    // fragment addresses: activation rows ti * 16 + lr, weight rows rw[tj]
    const int xo0 = lr * 64 + ((lk ^ swz(lr)) << 4);
    int rw[TJ];
    int64_t frow[TJ];
#pragma unroll
    for (int tj = 0; tj < TJ; tj++) {
        rw[tj] = wv * 16 * TJ + tj * 16 + lr;
        frow[tj] = (int64_t)grow_of(rw[tj]) * rbytes;
    }

    // K-quants carry one scale d per 256-element superblock: their MFMA sums run
    // over the superblock's 8 steps in cs and are scaled into acc once, at its end
    constexpr bool SBD = F::EPB == 256;
    f4 acc[TI][TJ], cs[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = cs[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    v4u hdr[TJ];   // K-quants: the current superblock's 16-byte header per weight row
#pragma unroll
    for (int j = 0; j < TJ; j++) hdr[j] = v4u{0u, 0u, 0u, 0u};

    issue(st0);
    if (NS == 3 && st0 + 1 < st1) issue(st0 + 1);
    for (int st = st0; st < st1; st++) {
        // step st's copies are complete once at most the later step's remain
        if (NS == 3 && st + 1 < st1) {
            if (F::MIN && ((st + 1) & 7) == 0) vm_wait<NX + NW + 1>();
            else vm_wait<NX + NW>();
        } else {
            vm_wait<0>();
        }
        lds_barrier();   // every wave's copies of step st landed; step st - 1's buffers are free
        if (st + NS - 1 < st1) issue(st + NS - 1);
        const unsigned char* sb = smem + (st % NS) * ST1;
        const unsigned char* raw = WH ? smem + NS * ST1 + SS_B + ((st >> 2) & 1) * WSH : sb + XS1;
        h8 wf[TJ][NP];
        float d[TJ];
        if constexpr (F::KQ) {
            // the 16-byte header (d, dmin, packed scales) of the superblock, read
            // aligned once at its first step (every step's stage holds a copy)
            if ((st & 7) == 0) {
#pragma unroll
                for (int tj = 0; tj < TJ; tj++) hdr[tj] = *reinterpret_cast<const v4u*>(raw + rw[tj] * 16);
            }
        }
#pragma unroll
        for (int tj = 0; tj < TJ; tj++) {
            if constexpr (F::KQ) {
                wf[tj][0] = kq_frag<FMT>(hdr[tj], raw + 2048 + rw[tj] * 16, st & 7, lk);
                d[tj] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr[tj][0] & 0xFFFFu));
            } else {
                win_frag<FMT>(raw + rw[tj] * (WH ? F::RH : R) * 16, st, lk, frow[tj], wf[tj], &d[tj]);
            }
        }
        // activation fragments of tile ti + 1 are read while tile ti's MFMAs issue
        h8 xn0 = *reinterpret_cast<const h8*>(sb + xo0), xn1 = *reinterpret_cast<const h8*>(sb + xo0 + TM * 64);
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            const h8 x0 = xn0, x1 = xn1;
            if (ti + 1 < TI) {
                const unsigned char* xr = sb + (ti + 1) * 1024 + xo0;
                xn0 = *reinterpret_cast<const h8*>(xr);
                xn1 = *reinterpret_cast<const h8*>(xr + TM * 64);
            }
#pragma unroll
            for (int tj = 0; tj < TJ; tj++) {
                f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, wf[tj][0], SBD ? cs[ti][tj] : f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, wf[tj][0], c, 0, 0, 0);
                if constexpr (NP == 2) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, wf[tj][1], c, 0, 0, 0);
                if constexpr (SBD) {
                    cs[ti][tj] = c;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[ti][tj][e] += d[tj] * c[e];
                }
            }
        }
        if (SBD && (st & 7) == 7) {   // superblock end: acc += d * (its 8 steps' sums)
#pragma unroll
            for (int ti = 0; ti < TI; ti++)
#pragma unroll
                for (int tj = 0; tj < TJ; tj++) {
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[ti][tj][e] += d[tj] * cs[ti][tj][e];
                    cs[ti][tj] = f4{0.f, 0.f, 0.f, 0.f};
                }
        }
        if constexpr (F::MIN) {
            if ((st & 7) == 7) {   // superblock end: acc -= 32 dmin * (sum_g m_g S_g) / 32
                const int sp = (st >> 3) & 1;
#pragma unroll
                for (int tj = 0; tj < TJ; tj++) {
                    const v4u hw = hdr[tj];
                    const float dm = 32.0f * (float)__builtin_bit_cast(_Float16, (uint16_t)(hw[0] >> 16));
                    h4 mq = h4{0, 0, 0, 0};
                    if (lk < 2) {
                        const uint32_t h1 = hw[1], h2w = hw[2], h3 = hw[3];
#pragma unroll
                        for (int gg = 0; gg < 4; gg++)
                            mq[gg] = (_Float16)(float)(k_field12(h1, h2w, h3, 12 * (4 * lk + gg)) >> 6);
                    }
#pragma unroll
                    for (int ti = 0; ti < TI; ti++) {
                        const int tl = ti * 16 + lr;
                        h4 s0 = h4{0, 0, 0, 0}, s1 = h4{0, 0, 0, 0};
                        if (lk < 2) {
                            s0 = *reinterpret_cast<const h4*>(Ss + ((sp * 2 + 0) * TM + tl) * 16 + 8 * lk);
                            s1 = *reinterpret_cast<const h4*>(Ss + ((sp * 2 + 1) * TM + tl) * 16 + 8 * lk);
                        }
                        f4 rr = __builtin_amdgcn_mfma_f32_16x16x16f16(s0, mq, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        rr = __builtin_amdgcn_mfma_f32_16x16x16f16(s1, mq, rr, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[ti][tj][e] -= dm * rr[e];
                    }
                }
            }
        }
    }
    lds_barrier();   // all waves are done with the stage buffers (SWIGLU reuses them)
    const int wn = wv;

    // epilogue: y = acc / s for token rows; lane holds tokens 4 lk + e of tile ti, row lr of tile tj
    float xi[TI][4];
#pragma unroll
    for (int ti = 0; ti < TI; ti++)
#pragma unroll
        for (int e = 0; e < 4; e++) xi[ti][e] = a.xinv[min(m0 + ti * 16 + 4 * lk + e, a.M - 1)];
    if (EPI == PF_SWIGLU) {
        // waves 2, 3 hold the up rows matching the gate rows of waves 0, 1.
        // The pair splits the tokens: the gate wave finishes the first half
        // (up values through LDS), the up wave the second (gate values
        // through LDS); each value crosses as the same fp32 number.
        float (*E)[TM][16 * TJ + 1] = reinterpret_cast<float (*)[TM][16 * TJ + 1]>(smem);
        const bool gate = wn < 2;
        const int pw = gate ? wn : wn - 2;   // the pair's index
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            if ((ti < TI / 2) == gate) continue;   // the half the other wave finishes
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
#pragma unroll
                for (int e = 0; e < 4; e++) E[pw][ti * 16 + 4 * lk + e][tj * 16 + lr] = acc[ti][tj][e] * xi[ti][e];
        }
        __syncthreads();
        const int n8 = a.N & ~7;
#pragma unroll
        for (int ti = 0; ti < TI; ti++) {
            if ((ti < TI / 2) != gate) continue;
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = m0 + ti * 16 + 4 * lk + e;
                    const int row = tn * 64 + pw * 16 * TJ + tj * 16 + lr;
                    if (t < a.M && row < a.N) {
#pragma clang fp contract(off)
                        const float own = acc[ti][tj][e] * xi[ti][e];
                        const float other = E[pw][ti * 16 + 4 * lk + e][tj * 16 + lr];
                        const float g = gate ? own : other, u = gate ? other : own;
                        // SiluInPlace then Mul (IE:463-474): ExpApprox on the vector lanes
                        const float sg = row < n8 ? silu_ref(g) : g / (1.0f + expf(-g));
                        a.out[(int64_t)t * a.ldo + row] = sg * u;
                    }
                }
        }
    } else {
#pragma unroll
        for (int ti = 0; ti < TI; ti++)
#pragma unroll
            for (int tj = 0; tj < TJ; tj++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = m0 + ti * 16 + 4 * lk + e;
                    const int row = tnl * BN + wn * 16 * TJ + tj * 16 + lr;
                    if (t < a.M && row < Nl) {
                        const float y = acc[ti][tj][e] * xi[ti][e];
                        float* o = segb ? a.outb + (int64_t)t * a.ldob + row
                                        : a.out + part * a.part_stride + (int64_t)t * a.ldo + row;
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
// (IE:362-381, same per-element arithmetic as the decode path).  A projection
// computed in K parts is summed here, parts in order.
__device__ __forceinline__ float sum_parts(const float* x, int64_t idx, int n, int64_t stride) {
    float v = x[idx];
    for (int p = 1; p < n; p++) v += x[p * stride + idx];
    return v;
}

// With per-head Q/K norms (IE:354-359, IE:367-372) one wavefront takes a
// head: the sum of squares of its (summed) row, then VectorMath.RmsNorm's
// vector-lane / tail forms on each element and its rotation partner, then
// the rotation; the decode step's qk_norm_kernel sums in the same order.
__device__ __forceinline__ void pf_norm_rope_heads(const float* x, int split, int64_t part, int64_t row0, int nheads,
                                                   int HD, const float* w, float eps, const float* cs, const float* sn,
                                                   int half, float* qr_out, void* cache, int64_t slot0,
                                                   int64_t head_stride, int fp16) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    auto partner = [&](int d) { return d < half ? d + half : (d < 2 * half ? d - half : d); };
    auto pidx = [&](int d) { return d < half ? d : (d < 2 * half ? d - half : 0); };
    const int n8 = HD & ~7;
    for (int h = wave; h < nheads; h += WG / 64) {
        const int64_t r = row0 + (int64_t)h * HD;
        float ss = 0.f;
        for (int d = lane; d < HD; d += 64) {
            const float v = sum_parts(x, r + d, split, part);
            ss += v * v;
        }
        ss = wave_sum(ss);
        const float inv = (1.0f / (sqrtf(((ss / (float)HD) + eps))));
        auto nrm = [&](int d) {
#pragma clang fp contract(off)
            const float v = sum_parts(x, r + d, split, part);
            return d < n8 ? ((w[d] * v) * inv) : (w[d] * (v * inv));
        };
        for (int d = lane; d < HD; d += 64) {
            const float y = rope_pair(nrm(d), nrm(partner(d)), cs[pidx(d)], sn[pidx(d)], d, half);
            if (qr_out) qr_out[(int64_t)h * HD + d] = y;
            else store_kv(cache, slot0 + (int64_t)h * head_stride + d, y, fp16);
        }
    }
}

__global__ __launch_bounds__(WG) void pf_rope_kv_kernel(PfAttnArgs a) {
    const int t = blockIdx.x, p = a.pos0 + t;
    const int HD = a.head_dim, half = a.rope_half;
    const int qdim = a.heads * HD, kvdim = a.kv_heads * HD;
    const float* cs = a.cos_tab + (int64_t)p * half;
    const float* sn = a.sin_tab + (int64_t)p * half;
    // element d's rotation partner and the pair's table index
    auto partner = [&](int d) { return d < half ? d + half : (d < 2 * half ? d - half : d); };
    auto pidx = [&](int d) { return d < half ? d : (d < 2 * half ? d - half : 0); };
    if (a.q_norm)
        pf_norm_rope_heads(a.q, a.q_split, a.q_part, (int64_t)t * qdim, a.heads, HD, a.q_norm, a.eps, cs, sn, half,
                           a.qr + (int64_t)t * qdim, nullptr, 0, 0, 0);
    if (a.k_norm)
        pf_norm_rope_heads(a.k, a.k_split, a.k_part, (int64_t)t * kvdim, a.kv_heads, HD, a.k_norm, a.eps, cs, sn,
                           half, nullptr, a.kcache, (int64_t)p * HD, (int64_t)a.context * HD, a.kv_fp16);
    for (int i = threadIdx.x; i < qdim && !a.q_norm; i += WG) {
        const int h = i / HD, d = i - h * HD;
        const int64_t r = (int64_t)t * qdim + h * HD;
        const float x = sum_parts(a.q, r + d, a.q_split, a.q_part);
        const float y = sum_parts(a.q, r + partner(d), a.q_split, a.q_part);
        a.qr[(int64_t)t * qdim + i] = rope_pair(x, y, cs[pidx(d)], sn[pidx(d)], d, half);
    }
    for (int i = threadIdx.x; i < kvdim; i += WG) {
        const int h = i / HD, d = i - h * HD;
        const int64_t r = (int64_t)t * kvdim + h * HD;
        const int64_t slot = ((int64_t)h * a.context + p) * HD + d;
        if (!a.k_norm) {
            const float x = sum_parts(a.k, r + d, a.k_split, a.k_part);
            const float y = sum_parts(a.k, r + partner(d), a.k_split, a.k_part);
            store_kv(a.kcache, slot, rope_pair(x, y, cs[pidx(d)], sn[pidx(d)], d, half), a.kv_fp16);
        }
        store_kv(a.vcache, slot, sum_parts(a.v, (int64_t)t * kvdim + i, a.v_split, a.v_part), a.kv_fp16);
    }
}

// h[i] += parts[0][i] + parts[1][i] + ... (in part order) for i < n: the
// residual add of an output projection computed in K parts.
__global__ __launch_bounds__(WG) void pf_add_parts_kernel(float* __restrict__ h, const float* __restrict__ parts,
                                                          int nparts, int64_t stride, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    float y = parts[i];
    for (int p = 1; p < nparts; p++) y += parts[p * stride + i];
    h[i] += y;
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
        m = max16(m);
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
        zz = sum16(zz);
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
//
// Scores are computed transposed, S^T = K q^T (MFMA A = K rows, B = the
// query planes), so a lane holds keys 4 (l >> 4) .. + 3 of each 16-key
// sub-tile for query l & 15: exactly the row layout the e V product needs as
// its A operand (with the keys of a 32-key step taken in the order 4 lk .. +3,
// 16 + 4 lk .. +3, matched in the V^T fragment).  Two passes over the keys:
// the first finds each query's maximum (VectorMath.Softmax needs the exact
// maximum before any ExpApprox, VM:215-258), the second recomputes the same
// scores bit for bit and accumulates e and e V; no score leaves registers.

constexpr int KPAD = 8;   // halves of row padding in the K / V^T tiles

// The lane's query planes (query l & 15 of the wave, dims 32 ks + 8 lk .. +7,
// scaled by a power of two) and the factor that turns an MFMA sum into the
// score (q . K_j) / sqrt(hd).
template <int HD>
struct QFrag {
    static constexpr int KS = HD / 32;
    h8 qh[KS], ql[KS];
    float oscale;
    __device__ void load(const PfAttnArgs& a, int tq, int h, int lk) {
        const float* qrow = a.qr + (int64_t)tq * (a.heads * HD) + h * HD;
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
        amax = fmaxf(amax, fx(lane_xor16, amax));
        amax = fmaxf(amax, fx(lane_xor32, amax));
        int e = 0;
        if (amax > 0.f) {
            (void)frexpf(amax, &e);
            e = 15 - e;
            e = e > 126 ? 126 : (e < -126 ? -126 : e);
        }
        const float sq = ldexpf(1.0f, e);
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = qv[ks][i] * sq;
                const _Float16 hi = (_Float16)x;
                qh[ks][i] = hi;
                ql[ks][i] = (_Float16)(x - (float)hi);
            }
        oscale = (1.0f / sqrtf((float)HD)) * ldexpf(1.0f, -e);
    }
    // scores of keys kt * 16 + 4 lk + r (r = 0..3) of the LDS K tile for this lane's query
    __device__ f4 scores(const _Float16 (*Ks)[HD + KPAD], int kt, int lr, int lk) const {
        f4 c = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const h8 kf = *reinterpret_cast<const h8*>(&Ks[kt * 16 + lr][32 * ks + 8 * lk]);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], c, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) c[r] = c[r] * oscale;
        return c;
    }
};

// 16-byte chunks of a K tile (rows j0 .. j0 + AK - 1, clamped to the last key)
// through registers into LDS.
template <int HD>
struct KTile {
    static constexpr int CH = AK * HD / 8 / WG;
    v4u r[CH];
    __device__ void load(const _Float16* kc, int64_t base, int j0, int nkeys, int tid) {
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int c = tid + k * WG, row = c / (HD / 8), q = c - row * (HD / 8);
            r[k] = *reinterpret_cast<const v4u*>(kc + base + (int64_t)min(j0 + row, nkeys - 1) * HD + 8 * q);
        }
    }
    __device__ void store(_Float16 (*Ks)[HD + KPAD], int tid) const {
#pragma unroll
        for (int k = 0; k < CH; k++) {
            const int c = tid + k * WG, row = c / (HD / 8), q = c - row * (HD / 8);
            *reinterpret_cast<v4u*>(&Ks[row][8 * q]) = r[k];
        }
    }
};

// Query block and head of this workgroup: the causal work grows with the
// block, so the last (heaviest) blocks are dispatched first and the light
// ones fill the CUs as they free up.
__device__ __forceinline__ void attn_block(const PfAttnArgs& a, int& t0, int& h) {
    const int nqb = (a.T + AQ - 1) / AQ;
    const int L = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    h = L % a.heads;
    t0 = (nqb - 1 - L / a.heads) * AQ;
}

// Pass 1: each query's maximum score over its keys, 0 (or its window's
// start) .. pos0 + t.
template <int HD>
__global__ __launch_bounds__(WG) void pf_attn_max_mfma(PfAttnArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][AK][HD + KPAD];
    int t0, h;
    attn_block(a, t0, h);
    const int kvh = h / (a.heads / a.kv_heads);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lk = lane >> 4;
    const int tq = t0 + 16 * wave + lr;
    QFrag<HD> qf;
    qf.load(a, min(tq, a.T - 1), h, lk);
    const int last = tq < a.T ? a.pos0 + tq : -1;      // the query's last key
    // SlidingWindow (IE:385-387): the query's first key, and the block's
    // first tile (its first query's window starts earliest)
    const int first = a.window > 0 ? max(0, last + 1 - a.window) : 0;
    const int jstart = a.window > 0 ? max(0, a.pos0 + t0 + 1 - a.window) / AK * AK : 0;
    const int nkeys = a.pos0 + min(t0 + AQ, a.T);
    const int64_t kbase = (int64_t)kvh * a.context * HD;
    const _Float16* kc = reinterpret_cast<const _Float16*>(a.kcache);
    float m = -INFINITY;
    KTile<HD> kt_regs;
    kt_regs.load(kc, kbase, jstart, nkeys, tid);
    int it = 0;
    for (int j0 = jstart; j0 < nkeys; j0 += AK, it++) {
        const int buf = it & 1;
        kt_regs.store(Ks[buf], tid);   // buffer last read two tiles ago
        __syncthreads();
        if (j0 + AK < nkeys) kt_regs.load(kc, kbase, j0 + AK, nkeys, tid);
#pragma unroll
        for (int kt = 0; kt < AK / 16; kt++) {
            const f4 c = qf.scores(Ks[buf], kt, lr, lk);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = j0 + kt * 16 + 4 * lk + r;
                if (key <= last && key >= first) m = fmaxf(m, c[r]);
            }
        }
    }
    m = fmaxf(m, fx(lane_xor16, m));
    m = fmaxf(m, fx(lane_xor32, m));
    if (lk == 0 && tq < a.T) a.rowmax[(int64_t)h * a.T + tq] = m;
}

// Pass 2: the same scores, softmax numerators (ExpApprox on the first
// 8 floor(n/8) of the query's n keys, expf on the tail, VM:215-258) and
// out = sum_j e_j V_j / sum_j e_j.
template <int HD>
__global__ __launch_bounds__(WG, 3) void pf_attn_pv_mfma(PfAttnArgs a) {
    constexpr int DT = HD / 16;              // 16-wide output tiles over the head dimension
    constexpr int VCH = AK * HD / 8 / WG;    // 16-byte V chunks per thread and tile
    __shared__ __attribute__((aligned(16))) _Float16 Ks[AK][HD + KPAD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[HD][AK + KPAD];   // V^T tile
    int t0, h;
    attn_block(a, t0, h);
    const int kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lk = lane >> 4;
    const int tq = t0 + 16 * wave + lr;
    const int tqc = min(tq, a.T - 1);
    QFrag<HD> qf;
    qf.load(a, tqc, h, lk);
    const int last = tq < a.T ? a.pos0 + tq : -1;
    // the query's window (all earlier keys without one); its first
    // 8 floor(len/8) keys are the Softmax's vector lanes
    const int first = a.window > 0 ? max(0, a.pos0 + tqc + 1 - a.window) : 0;
    const int jstart = a.window > 0 ? max(0, a.pos0 + t0 + 1 - a.window) / AK * AK : 0;
    const int n8 = first + ((a.pos0 + tqc + 1 - first) & ~7);
    const float mq = a.rowmax[(int64_t)h * a.T + tqc];
    const int nkeys = a.pos0 + min(t0 + AQ, a.T);
    const int64_t base = (int64_t)kvh * a.context * HD;
    const _Float16* kc = reinterpret_cast<const _Float16*>(a.kcache);
    const _Float16* vc = reinterpret_cast<const _Float16*>(a.vcache);
    const float P14 = 16384.0f;
    f4 acc[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) acc[i] = f4{0.f, 0.f, 0.f, 0.f};
    float z = 0.f;
    KTile<HD> kr;
    h8 vr[VCH];
    auto load_v = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < VCH; k++) {
            const int c = tid + k * WG, r = c & (AK - 1), q = c / AK;
            vr[k] = *reinterpret_cast<const h8*>(vc + base + (int64_t)min(j0 + r, nkeys - 1) * HD + 8 * q);
        }
    };
    kr.load(kc, base, jstart, nkeys, tid);
    load_v(jstart);
    for (int j0 = jstart; j0 < nkeys; j0 += AK) {
        __syncthreads();   // the previous tile's LDS reads are done
        kr.store(Ks, tid);
#pragma unroll
        for (int k = 0; k < VCH; k++) {   // V rows -> V^T; a wave writes 64 consecutive keys
            const int c = tid + k * WG, r = c & (AK - 1), q = c / AK;
#pragma unroll
            for (int i = 0; i < 8; i++) Vt[8 * q + i][r] = vr[k][i];
        }
        __syncthreads();
        if (j0 + AK < nkeys) {
            kr.load(kc, base, j0 + AK, nkeys, tid);
            load_v(j0 + AK);
        }
#pragma unroll
        for (int p = 0; p < AK / 32; p++) {
            h8 eh, el;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const int kt = 2 * p + half;
                const f4 c = qf.scores(Ks, kt, lr, lk);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = j0 + kt * 16 + 4 * lk + r;
                    float ev = 0.f;
                    if (key <= last && key >= first) {
#pragma clang fp contract(off)
                        const float x = c[r] - mq;
                        ev = key < n8 ? exp_approx(x) : expf(x);
                    }
                    z += ev;
                    const float xs = ev * P14;
                    const _Float16 hi = (_Float16)xs;
                    eh[4 * half + r] = hi;
                    el[4 * half + r] = (_Float16)(xs - (float)hi);
                }
            }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                // keys 32 p + 4 lk .. +3 and 32 p + 16 + 4 lk .. +3, as in eh / el
                const uint2 v0 = *reinterpret_cast<const uint2*>(&Vt[dt * 16 + lr][32 * p + 4 * lk]);
                const uint2 v1 = *reinterpret_cast<const uint2*>(&Vt[dt * 16 + lr][32 * p + 16 + 4 * lk]);
                const h8 vf = __builtin_bit_cast(h8, v4u{v0.x, v0.y, v1.x, v1.y});
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(eh, vf, acc[dt], 0, 0, 0);
                acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(el, vf, acc[dt], 0, 0, 0);
            }
        }
    }
    z = xor32_add(xor16_add(z));   // lanes lr, lr+16, ... hold query lr's sum
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
hipError_t launch_gemm_fmt(int epi, PfGemmArgs a, hipStream_t s) {
    const int tn_a = epi == PF_SWIGLU ? (a.N + 63) / 64 : (a.N + BN - 1) / BN;
    a.tiles_n = tn_a + (a.wb ? (a.nb + BN - 1) / BN : 0);
    a.tn_b = tn_a;
    const int tiles = a.tiles_n * ((a.M + BM - 1) / BM) * a.ksplit;
    // 128 to 255 tiles of BM tokens fill only part of the CUs: 64-token tiles
    // (LLMDOT_HIP_PF_TM64=0 turns this off)
    const char* env = getenv("LLMDOT_HIP_PF_TM64");
    const bool tm64_off = env && env[0] == '0' && env[1] == 0;
    const bool tm64 = !tm64_off && epi != PF_SWIGLU && a.ksplit == 1 && tiles >= 128 && tiles < 256;
    const int t64 = a.tiles_n * ((a.M + 63) / 64);
    const dim3 grid(8 * (((tm64 ? t64 : tiles) + 7) / 8));
    switch (epi) {
    case PF_STORE:
        if (tm64) pf_gemm_kernel<FMT, PF_STORE, 64><<<grid, WG, 0, s>>>(a);
        else pf_gemm_kernel<FMT, PF_STORE><<<grid, WG, 0, s>>>(a);
        break;
    case PF_ADD:
        if (tm64) pf_gemm_kernel<FMT, PF_ADD, 64><<<grid, WG, 0, s>>>(a);
        else pf_gemm_kernel<FMT, PF_ADD><<<grid, WG, 0, s>>>(a);
        break;
    case PF_SWIGLU: pf_gemm_kernel<FMT, PF_SWIGLU><<<grid, WG, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int HD>
hipError_t launch_attn_hd(const PfAttnArgs& a, hipStream_t s) {
    const dim3 grid((a.T + AQ - 1) / AQ, a.heads);
    if (a.kv_fp16) pf_attn_max_mfma<HD><<<grid, WG, 0, s>>>(a);
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

namespace {
hipError_t launch_gemm_type(uint32_t type, int epi, const PfGemmArgs& a, hipStream_t s) {
    switch (type) {
    case GGML_Q4_K: return launch_gemm_fmt<GGML_Q4_K>(epi, a, s);
    case GGML_Q5_K: return launch_gemm_fmt<GGML_Q5_K>(epi, a, s);
    case GGML_Q6_K: return launch_gemm_fmt<GGML_Q6_K>(epi, a, s);
    case GGML_Q8_0: return launch_gemm_fmt<GGML_Q8_0>(epi, a, s);
    case GGML_Q4_0: return launch_gemm_fmt<GGML_Q4_0>(epi, a, s);
    default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t launch_prefill_gemm(uint32_t type, int epi, const PfPlanes& p, const uint8_t* w, const uint8_t* w2, int M,
                               int N, int K, float* out, int ldo, hipStream_t s, int ksplit, int64_t part_stride) {
    if (M <= 0 || N <= 0 || !prefill_gemm_supported(type, K) || (epi == PF_SWIGLU && !w2) || ldo < N)
        return hipErrorInvalidValue;
    // parts of whole blocks (256-element superblocks for the K-quants), STORE only
    const int gran = block_elems(type) == 256 ? 8 : 1;
    if (ksplit < 1 || (ksplit > 1 && (epi != PF_STORE || (K / 32) % (ksplit * gran) != 0 ||
                                      part_stride < (int64_t)(M - 1) * ldo + N)))
        return hipErrorInvalidValue;
    // the kernel addresses activations and weight rows with 32-bit byte offsets
    if ((int64_t)M * K * 2 >= (int64_t)1 << 31 || (int64_t)N * byte_count(type, K) >= ((int64_t)1 << 31) - 65536)
        return hipErrorInvalidValue;
    PfGemmArgs a{p.xh, p.xl, p.sh, p.sl, p.xinv, w, w2, out, M, N, K, ldo, 0, ksplit, part_stride};
    return launch_gemm_type(type, epi, a, s);
}

hipError_t launch_prefill_gemm_pair(uint32_t type, const PfPlanes& p, const uint8_t* w, int N, float* out, int ldo,
                                    const uint8_t* wb, int nb, float* outb, int ldob, int M, int K, hipStream_t s) {
    if (M <= 0 || N <= 0 || nb <= 0 || N % BN || !w || !wb || !prefill_gemm_supported(type, K) || ldo < N ||
        ldob < nb)
        return hipErrorInvalidValue;
    if ((int64_t)M * K * 2 >= (int64_t)1 << 31 ||
        (int64_t)std::max(N, nb) * byte_count(type, K) >= ((int64_t)1 << 31) - 65536)
        return hipErrorInvalidValue;
    PfGemmArgs a{p.xh, p.xl, p.sh, p.sl, p.xinv, w, nullptr, out, M, N, K, ldo, 0, 1, 0, wb, outb, 0, nb, ldob};
    return launch_gemm_type(type, PF_STORE, a, s);
}

hipError_t launch_prefill_rope_kv(const PfAttnArgs& a, hipStream_t s) {
    if (a.T <= 0 || a.q_split < 1 || a.k_split < 1 || a.v_split < 1) return hipErrorInvalidValue;
    pf_rope_kv_kernel<<<a.T, WG, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_prefill_add_parts(float* h, const float* parts, int nparts, int64_t stride, int64_t n, hipStream_t s) {
    if (n <= 0 || nparts < 1 || stride < n) return hipErrorInvalidValue;
    pf_add_parts_kernel<<<(unsigned)((n + WG - 1) / WG), WG, 0, s>>>(h, parts, nparts, stride, n);
    return hipGetLastError();
}

int prefill_ksplit(uint32_t type, int M, int N, int K) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int gran = block_elems(type) == 256 ? 8 : 1;
    int sp = 1;
    if (tiles >= 128) return 1;
    while (sp < 8 && tiles * sp * 2 <= 512 && (K / 32) % (sp * 2 * gran) == 0) sp *= 2;
    return sp;
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
