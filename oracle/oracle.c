/*
 * oracle.c -- CPU restatement of the llmdot managed decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Build with
 *   gcc -O2 -ffp-contract=off -fno-fast-math -fopenmp -shared -fPIC
 * so that every float expression rounds exactly as written, left to right,
 * like the .NET JIT.  Each function names the reference lines it restates.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define VEC 8 /* Vector<float>.Count on x86-64 AVX2 */

static int g_threads = 1;
/* Reduction order: 0 = the reference's; 1, 2, 3 = other valid fp32 orders
 * used only to measure how far summation order alone moves the results (see
 * orc_set_order in oracle.h). */
static int g_order = 0;
#define N_ORDERS 4
/* Per order: lanes of the reductions the reference runs over Vector<float>
 * (its 8; 16 and 32 as 512-bit and wider vectors would give, 4 as 128-bit
 * ones), the element groups of the scalar K-quant sums (order 0: none, one
 * running sum), the positions per partial of the attention's value sum. */
static const int ORD_LANES[N_ORDERS] = {8, 16, 4, 32};
static const int ORD_GROUP[N_ORDERS] = {0, 32, 64, 16};
static const int ORD_PVCH[N_ORDERS] = {0, 64, 32, 128};

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }
void orc_set_order(int order) { g_order = order > 0 && order < N_ORDERS ? order : 0; }
int orc_get_order(void) { return g_order; }

static inline float bits_to_float(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t float_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* Vector.Dot(acc, Vector<float>.One): per-128-bit-lane DPPS, then lane sum. */
static inline float hsum8(const float v[VEC]) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

/* The most lanes any order uses. */
#define VEC_ALT 32
/* Horizontal sum of L lanes (L a power of two >= 4) as halves added pairwise;
 * for L = 8 exactly hsum8. */
static float hsum_lanes(const float* v, int L) {
    if (L == 4) return (v[0] + v[1]) + (v[2] + v[3]);
    return hsum_lanes(v, L / 2) + hsum_lanes(v + L / 2, L / 2);
}

/* Sum of x[0..n) in the lanes-then-tail order of the reference's vector loops:
 * ORD_LANES lanes (8 for order 0), horizontal sum, then the tail in order. */
static float lane_sum(const float* x, int n) {
    const int L = ORD_LANES[g_order];
    float acc[VEC_ALT] = {0};
    int i = 0;
    for (; i <= n - L; i += L)
        for (int l = 0; l < L; l++) acc[l] = acc[l] + x[i + l];
    float s = hsum_lanes(acc, L);
    for (; i < n; i++) s += x[i];
    return s;
}

/* ---------------------------------------------------------------- HH ---- */

/* HalfHelper.HalfToFloat, HH:7-34. */
float orc_half_to_float(uint16_t half) {
    uint32_t sign = (half >> 15) & 0x1u;
    uint32_t exponent = (half >> 10) & 0x1Fu;
    uint32_t mantissa = half & 0x3FFu;
    if (exponent == 0) {
        if (mantissa == 0) return sign ? -0.0f : 0.0f;
        uint32_t normalized = mantissa;
        int shift = 0;
        while ((normalized & 0x400u) == 0) { normalized <<= 1; shift++; }
        uint32_t newExp = (uint32_t)(127 - 14 - shift);
        uint32_t newMantissa = (normalized & 0x3FFu) << 13;
        return bits_to_float((sign << 31) | (newExp << 23) | newMantissa);
    }
    if (exponent == 31) {
        if (mantissa == 0) return sign ? -INFINITY : INFINITY;
        return bits_to_float(0xFFC00000u); /* float.NaN on x86 */
    }
    uint32_t floatExp = exponent - 15 + 127;
    return bits_to_float((sign << 31) | (floatExp << 23) | (mantissa << 13));
}

static inline float h2f_at(const uint8_t* p) {
    return orc_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

/* IEEE binary32 -> binary16, round to nearest even (what a fp16 KV store does). */
uint16_t orc_float_to_half(float f) {
    uint32_t x = float_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);           /* NaN */
    if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* overflow -> inf */
    if (absx >= 0x38800000u) {                                            /* normal half */
        uint32_t mant = absx & 0x7FFFFFu;
        uint32_t exp = (absx >> 23) - 127 + 15;
        uint32_t h = (exp << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (absx < 0x33000000u) return (uint16_t)sign;                       /* < half of min subnormal */
    {   /* subnormal half: value = mant * 2^(e-150) = k * 2^-24 with k = mant >> (126-e) */
        uint32_t e = absx >> 23;                 /* 102 <= e <= 112 */
        uint32_t mant = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t s = 126 - e;                    /* 14 <= s <= 24 */
        uint32_t k = mant >> s;
        uint32_t rem = mant & ((1u << s) - 1u);
        uint32_t halfway = 1u << (s - 1);
        if (rem > halfway || (rem == halfway && (k & 1u))) k++;
        return (uint16_t)(sign | k);
    }
}

/* ---------------------------------------------------------------- TS ---- */

/* TensorSize.ByteCount, TS:7-24. */
int64_t orc_byte_count(uint32_t type, uint64_t n) {
    switch (type) {
    case ORC_F32: return (int64_t)(n * 4);
    case ORC_F16: return (int64_t)(n * 2);
    case ORC_BF16: return (int64_t)(n * 2);
    case ORC_Q4_0: return (int64_t)(n / 32 * 18);
    case ORC_Q4_1: return (int64_t)(n / 32 * 20);
    case ORC_Q5_0: return (int64_t)(n / 32 * 22);
    case ORC_Q5_1: return (int64_t)(n / 32 * 24);
    case ORC_Q8_0: return (int64_t)(n / 32 * 34);
    case ORC_Q8_1: return (int64_t)(n / 32 * 40);
    case ORC_Q2_K: return (int64_t)(n / 256 * 84);
    case ORC_Q3_K: return (int64_t)(n / 256 * 110);
    case ORC_Q4_K: return (int64_t)(n / 256 * 144);
    case ORC_Q5_K: return (int64_t)(n / 256 * 176);
    case ORC_Q6_K: return (int64_t)(n / 256 * 210);
    default: return -1;
    }
}

/* ---------------------------------------------------------------- DK ---- */

/* DequantizeK.Extract6Bit, DK:189-199. */
int orc_extract6(const uint8_t* src, int baseOffset, int bitOffset) {
    int byteIdx = bitOffset / 8;
    int bitShift = bitOffset % 8;
    if (bitShift <= 2) return (src[baseOffset + byteIdx] >> bitShift) & 0x3F;
    return ((src[baseOffset + byteIdx] >> bitShift) |
            (src[baseOffset + byteIdx + 1] << (8 - bitShift))) & 0x3F;
}

/* DK:8-41 */
static void deq_q2_k(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int qk = 256, bsz = 84;
    int bpr = rowElements / qk;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int off = rowOffset + b * bsz;
            float d = h2f_at(src + off), dmin = h2f_at(src + off + 2);
            for (int i = 0; i < qk; i++) {
                int g = i / 64, local = i % 64, sub = local / 16, scIdx = g * 4 + sub;
                int sc = src[off + 4 + scIdx * 2] & 0x0F;
                int mi = src[off + 4 + scIdx * 2 + 1] & 0x0F;
                int q = (src[off + 20 + i / 4] >> ((i % 4) * 2)) & 0x3;
                dst[dstOffset + b * qk + i] = d * (float)sc * ((float)q - 0.5f) - dmin * (float)mi;
            }
        }
    }
}

/* DK:43-74 */
static void deq_q3_k(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int qk = 256, bsz = 110;
    int bpr = rowElements / qk;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int off = rowOffset + b * bsz;
            float d = h2f_at(src + off);
            for (int i = 0; i < qk; i++) {
                int g = i / 16;
                int sc = orc_extract6(src, off + 4, g * 6);
                int q = (src[off + 48 + i / 4] >> ((i % 4) * 2)) & 0x3;
                int m = (src[off + 16 + i / 8] >> (i % 8)) & 0x1;
                int value = q - (m << 2);
                dst[dstOffset + b * qk + i] = d * (float)sc * (float)value;
            }
        }
    }
}

/* Reference-layout Q4_K (not ggml): DK:76-106. */
static void deq_q4_k(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int qk = 256, bsz = 144;
    int bpr = rowElements / qk;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int off = rowOffset + b * bsz;
            float d = h2f_at(src + off), dmin = h2f_at(src + off + 2);
            for (int i = 0; i < qk; i++) {
                int g = i / 32;
                int sc = orc_extract6(src, off + 4, g * 12);
                int mi = orc_extract6(src, off + 4, g * 12 + 6);
                int q = (src[off + 16 + i / 2] >> ((i % 2) * 4)) & 0xF;
                dst[dstOffset + b * qk + i] = d * (float)sc * (float)(q - 8) - dmin * (float)mi;
            }
        }
    }
}

/* Reference-layout Q5_K (not ggml): DK:108-140. */
static void deq_q5_k(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int qk = 256, bsz = 176;
    int bpr = rowElements / qk;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int off = rowOffset + b * bsz;
            float d = h2f_at(src + off), dmin = h2f_at(src + off + 2);
            for (int i = 0; i < qk; i++) {
                int g = i / 32;
                int sc = orc_extract6(src, off + 4, g * 12);
                int mi = orc_extract6(src, off + 4, g * 12 + 6);
                int qLow = (src[off + 48 + i / 2] >> ((i % 2) * 4)) & 0xF;
                int qHigh = (src[off + 16 + i / 8] >> (i % 8)) & 0x1;
                int q5 = qLow + (qHigh << 4);
                dst[dstOffset + b * qk + i] = d * (float)sc * (float)(q5 - 16) - dmin * (float)mi;
            }
        }
    }
}

/* Q6_K (ggml layout): DK:142-187. */
static void deq_q6_k(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int qk = 256, bsz = 210;
    int bpr = rowElements / qk;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int off = rowOffset + b * bsz;
            float d = h2f_at(src + off + 208);
            for (int n = 0; n < qk; n += 128) {
                int qlBase = off + n / 2, qhBase = off + 128 + n / 4, scBase = off + 192 + (n / 16);
                for (int l = 0; l < 32; l++) {
                    int isIdx = l / 16;
                    int q1 = ((src[qlBase + l] & 0xF) | (((src[qhBase + l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((src[qlBase + l + 32] & 0xF) | (((src[qhBase + l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((src[qlBase + l] >> 4) | (((src[qhBase + l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((src[qlBase + l + 32] >> 4) | (((src[qhBase + l] >> 6) & 3) << 4)) - 32;
                    int sc0 = (int8_t)src[scBase + isIdx + 0];
                    int sc2 = (int8_t)src[scBase + isIdx + 2];
                    int sc4 = (int8_t)src[scBase + isIdx + 4];
                    int sc6 = (int8_t)src[scBase + isIdx + 6];
                    int dstBase = dstOffset + b * qk + n;
                    dst[dstBase + l] = d * (float)sc0 * (float)q1;
                    dst[dstBase + l + 32] = d * (float)sc2 * (float)q2;
                    dst[dstBase + l + 64] = d * (float)sc4 * (float)q3;
                    dst[dstBase + l + 96] = d * (float)sc6 * (float)q4;
                }
            }
        }
    }
}

/* ---------------------------------------------------------------- DB ---- */

/* DB:7-34 */
static void deq_q4_0(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int be = 32, bsz = 18;
    int bpr = rowElements / be;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int bo = rowOffset + b * bsz;
            float scale = h2f_at(src + bo);
            for (int j = 0; j < be / 2; j++) {
                int qs = src[bo + 2 + j];
                dst[dstOffset + b * be + j] = (float)((qs & 0x0F) - 8) * scale;
                dst[dstOffset + b * be + j + be / 2] = (float)(((qs >> 4) & 0x0F) - 8) * scale;
            }
        }
    }
}

/* DB:36-59 */
static void deq_q8_0(const uint8_t* src, float* dst, int numRows, int rowElements) {
    const int be = 32, bsz = 34;
    int bpr = rowElements / be;
    for (int r = 0; r < numRows; r++) {
        int rowOffset = r * bpr * bsz, dstOffset = r * rowElements;
        for (int b = 0; b < bpr; b++) {
            int bo = rowOffset + b * bsz;
            float scale = h2f_at(src + bo);
            for (int i = 0; i < be; i++)
                dst[dstOffset + b * be + i] = (float)(int8_t)src[bo + 2 + i] * scale;
        }
    }
}

/* DB:61-67 */
static void deq_f16(const uint8_t* src, float* dst, int count) {
    for (int i = 0; i < count; i++) dst[i] = h2f_at(src + 2 * i);
}

/* DB:69-95 */
static void deq_bf16(const uint8_t* src, float* dst, int count) {
    for (int i = 0; i < count; i++) {
        uint32_t bits = ((uint32_t)src[i * 2 + 1] << 24) | ((uint32_t)src[i * 2] << 16);
        dst[i] = bits_to_float(bits);
    }
}

/* TO:580-652 (Q4_1, Q5_0, Q5_1) */
static int deq_generic(const uint8_t* src, float* dst, uint32_t type, int numRows, int rowElements) {
    const int be = 32;
    int bpr = rowElements / be;
    switch (type) {
    case ORC_Q4_1:
        for (int r = 0; r < numRows; r++)
            for (int b = 0; b < bpr; b++) {
                int off = r * bpr * 20 + b * 20;
                float d = h2f_at(src + off), m = h2f_at(src + off + 2);
                for (int j = 0; j < be / 2; j++) {
                    int qs = src[off + 4 + j];
                    dst[r * rowElements + b * be + j] = d * (float)(qs & 0x0F) + m;
                    dst[r * rowElements + b * be + j + be / 2] = d * (float)((qs >> 4) & 0x0F) + m;
                }
            }
        return 0;
    case ORC_Q5_0:
        for (int r = 0; r < numRows; r++)
            for (int b = 0; b < bpr; b++) {
                int off = r * bpr * 22 + b * 22;
                float d = h2f_at(src + off);
                uint32_t qh;
                memcpy(&qh, src + off + 2, 4);
                for (int j = 0; j < be / 2; j++) {
                    int qs = src[off + 6 + j];
                    int x0 = ((qs & 0x0F) | (int)(((qh >> (j + 0)) << 4) & 0x10u)) - 16;
                    int x1 = (((qs >> 4) & 0x0F) | (int)((qh >> (j + 12)) & 0x10u)) - 16;
                    dst[r * rowElements + b * be + j] = (float)x0 * d;
                    dst[r * rowElements + b * be + j + be / 2] = (float)x1 * d;
                }
            }
        return 0;
    case ORC_Q5_1:
        for (int r = 0; r < numRows; r++)
            for (int b = 0; b < bpr; b++) {
                int off = r * bpr * 24 + b * 24;
                float d = h2f_at(src + off), m = h2f_at(src + off + 2);
                uint32_t qh;
                memcpy(&qh, src + off + 4, 4);
                for (int j = 0; j < be / 2; j++) {
                    int qs = src[off + 8 + j];
                    int x0 = (qs & 0x0F) | (int)(((qh >> (j + 0)) << 4) & 0x10u);
                    int x1 = ((qs >> 4) & 0x0F) | (int)((qh >> (j + 12)) & 0x10u);
                    dst[r * rowElements + b * be + j] = d * (float)x0 + m;
                    dst[r * rowElements + b * be + j + be / 2] = d * (float)x1 + m;
                }
            }
        return 0;
    default:
        return -1; /* NotSupportedException */
    }
}

/* TensorOps.DequantizeToFloat, TO:18-56.  Returns -1 for unsupported types. */
int orc_dequantize(const uint8_t* src, float* dst, uint32_t type, int numRows, int rowElements) {
    switch (type) {
    case ORC_F32: memcpy(dst, src, (size_t)numRows * rowElements * 4); return 0;
    case ORC_F16: deq_f16(src, dst, numRows * rowElements); return 0;
    case ORC_BF16: deq_bf16(src, dst, numRows * rowElements); return 0;
    case ORC_Q4_0: deq_q4_0(src, dst, numRows, rowElements); return 0;
    case ORC_Q8_0: deq_q8_0(src, dst, numRows, rowElements); return 0;
    case ORC_Q2_K: deq_q2_k(src, dst, numRows, rowElements); return 0;
    case ORC_Q3_K: deq_q3_k(src, dst, numRows, rowElements); return 0;
    case ORC_Q4_K: deq_q4_k(src, dst, numRows, rowElements); return 0;
    case ORC_Q5_K: deq_q5_k(src, dst, numRows, rowElements); return 0;
    case ORC_Q6_K: deq_q6_k(src, dst, numRows, rowElements); return 0;
    default: return deq_generic(src, dst, type, numRows, rowElements);
    }
}

/* TensorOps.DequantizeRow, TO:537-574 (BF16 is not in its switch: falls to
 * DequantizeGeneric, which throws). */
static int dequantize_row(const uint8_t* src, float* dst, uint32_t type, int row, int rowElements) {
    int64_t bc = orc_byte_count(type, (uint64_t)rowElements);
    if (bc < 0) return -1;
    const uint8_t* slice = src + (int64_t)row * bc;
    switch (type) {
    case ORC_F32: memcpy(dst, slice, (size_t)rowElements * 4); return 0;
    case ORC_F16: deq_f16(slice, dst, rowElements); return 0;
    case ORC_Q4_0: deq_q4_0(slice, dst, 1, rowElements); return 0;
    case ORC_Q8_0: deq_q8_0(slice, dst, 1, rowElements); return 0;
    case ORC_Q2_K: deq_q2_k(slice, dst, 1, rowElements); return 0;
    case ORC_Q3_K: deq_q3_k(slice, dst, 1, rowElements); return 0;
    case ORC_Q4_K: deq_q4_k(slice, dst, 1, rowElements); return 0;
    case ORC_Q5_K: deq_q5_k(slice, dst, 1, rowElements); return 0;
    case ORC_Q6_K: deq_q6_k(slice, dst, 1, rowElements); return 0;
    default: return deq_generic(slice, dst, type, 1, rowElements);
    }
}

/* ---------------------------------------------------------------- TO ---- */

/* TensorOps.DotProduct, TO:510-531. */
static float dot_product(const float* a, const float* b, int n) {
    float acc[VEC] = {0};
    int i = 0;
    for (; i <= n - VEC; i += VEC)
        for (int l = 0; l < VEC; l++) acc[l] = acc[l] + a[i + l] * b[i + l];
    float dot = hsum8(acc);
    for (; i < n; i++) dot += a[i] * b[i];
    return dot;
}

/* TO:118-173 */
static void mm_fused_q4_0(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int bs = 32, hb = 16, bb = 18;
    int nb = aCols / bs;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        float* fused = (float*)malloc(sizeof(float) * (size_t)aCols);
        int64_t rowOffset = (int64_t)c * nb * bb;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bb;
            float d = h2f_at(p);
            int baseIdx = blk * bs;
            for (int i = 0; i < hb; i++) {
                int qs = p[2 + i];
                fused[baseIdx + i] = a[baseIdx + i] * (((float)(qs & 0x0F) - 8.0f) * d);
                fused[baseIdx + i + hb] = a[baseIdx + i + hb] * (((float)((qs >> 4) & 0x0F) - 8.0f) * d);
            }
        }
        float acc[VEC] = {0};
        int k = 0;
        for (; k <= aCols - VEC; k += VEC)
            for (int l = 0; l < VEC; l++) acc[l] = acc[l] + fused[k + l];
        float dot = hsum8(acc);
        for (; k < aCols; k++) dot += fused[k];
        result[c] = dot;
        free(fused);
    }
}

/* TO:179-224 */
static void mm_fused_q8_0(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int bs = 32, bb = 34;
    int nb = aCols / bs;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        float* fused = (float*)malloc(sizeof(float) * (size_t)aCols);
        int64_t rowOffset = (int64_t)c * nb * bb;
        int fusedIdx = 0;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bb;
            float d = h2f_at(p);
            for (int i = 0; i < bs; i++) {
                fused[fusedIdx] = a[fusedIdx] * ((float)(int8_t)p[2 + i] * d);
                fusedIdx++;
            }
        }
        float acc[VEC] = {0};
        int k = 0;
        for (; k <= aCols - VEC; k += VEC)
            for (int l = 0; l < VEC; l++) acc[l] = acc[l] + fused[k + l];
        float r = hsum8(acc);
        for (; k < aCols; k++) r += fused[k];
        result[c] = r;
        free(fused);
    }
}

/* TO:230-287 */
static void mm_fused_q6_k(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int qk = 256, bsz = 210;
    int nb = aCols / qk;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        float* deqBuf = (float*)malloc(sizeof(float) * (size_t)aCols);
        int64_t rowOffset = (int64_t)c * nb * bsz;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bsz;
            float d = h2f_at(p + 208);
            for (int n = 0; n < qk; n += 128) {
                int dstBase = blk * qk + n;
                const uint8_t* ql = p + n / 2;
                const uint8_t* qh = p + 128 + n / 4;
                const uint8_t* sc = p + 192 + n / 16;
                for (int l = 0; l < 32; l++) {
                    int isIdx = l / 16;
                    int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    int sc0 = (int8_t)sc[isIdx + 0], sc2 = (int8_t)sc[isIdx + 2];
                    int sc4 = (int8_t)sc[isIdx + 4], sc6 = (int8_t)sc[isIdx + 6];
                    deqBuf[dstBase + l] = d * (float)sc0 * (float)q1;
                    deqBuf[dstBase + l + 32] = d * (float)sc2 * (float)q2;
                    deqBuf[dstBase + l + 64] = d * (float)sc4 * (float)q3;
                    deqBuf[dstBase + l + 96] = d * (float)sc6 * (float)q4;
                }
            }
        }
        result[c] = dot_product(a, deqBuf, aCols);
        free(deqBuf);
    }
}

/* TO:293-329 */
static void mm_fused_q2_k(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int qk = 256, bsz = 84;
    int nb = aCols / qk;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        int64_t rowOffset = (int64_t)c * nb * bsz;
        float dot = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bsz;
            float d = h2f_at(p), dmin = h2f_at(p + 2);
            int baseIdx = blk * qk;
            for (int i = 0; i < qk; i++) {
                int g = i / 64, local = i % 64, sub = local / 16, scIdx = g * 4 + sub;
                int sc = p[4 + scIdx * 2] & 0x0F, mi = p[4 + scIdx * 2 + 1] & 0x0F;
                int q = (p[20 + i / 4] >> ((i % 4) * 2)) & 0x3;
                dot += a[baseIdx + i] * (d * (float)sc * ((float)q - 0.5f) - dmin * (float)mi);
            }
        }
        result[c] = dot;
    }
}

/* TO:331-362 */
static void mm_fused_q3_k(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int qk = 256, bsz = 110;
    int nb = aCols / qk;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        int64_t rowOffset = (int64_t)c * nb * bsz;
        float dot = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bsz;
            float d = h2f_at(p);
            int baseIdx = blk * qk;
            for (int i = 0; i < qk; i++) {
                int g = i / 16;
                int sc = orc_extract6(p, 4, g * 6);
                int q = (p[48 + i / 4] >> ((i % 4) * 2)) & 0x3;
                int m = (p[16 + i / 8] >> (i % 8)) & 0x1;
                int value = q - (m << 2);
                dot += a[baseIdx + i] * d * (float)sc * (float)value;
            }
        }
        result[c] = dot;
    }
}

/* TO:364-395: scalar sequential accumulation over the reference Q4_K layout. */
static void mm_fused_q4_k(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int qk = 256, bsz = 144;
    int nb = aCols / qk;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        int64_t rowOffset = (int64_t)c * nb * bsz;
        float dot = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bsz;
            float d = h2f_at(p), dmin = h2f_at(p + 2);
            int baseIdx = blk * qk;
            for (int i = 0; i < qk; i++) {
                int g = i / 32;
                int sc = orc_extract6(p, 4, g * 12);
                int mi = orc_extract6(p, 4, g * 12 + 6);
                int q = (p[16 + i / 2] >> ((i % 2) * 4)) & 0xF;
                dot += a[baseIdx + i] * (d * (float)sc * (float)(q - 8) - dmin * (float)mi);
            }
        }
        result[c] = dot;
    }
}

/* TO:397-431 */
static void mm_fused_q5_k(const float* a, const uint8_t* b, float* result, int aCols, int bCols) {
    const int qk = 256, bsz = 176;
    int nb = aCols / qk;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int c = 0; c < bCols; c++) {
        int64_t rowOffset = (int64_t)c * nb * bsz;
        float dot = 0.0f;
        for (int blk = 0; blk < nb; blk++) {
            const uint8_t* p = b + rowOffset + blk * bsz;
            float d = h2f_at(p), dmin = h2f_at(p + 2);
            int baseIdx = blk * qk;
            for (int i = 0; i < qk; i++) {
                int g = i / 32;
                int sc = orc_extract6(p, 4, g * 12);
                int mi = orc_extract6(p, 4, g * 12 + 6);
                int qLow = (p[48 + i / 2] >> ((i % 2) * 4)) & 0xF;
                int qHigh = (p[16 + i / 8] >> (i % 8)) & 0x1;
                int q5 = qLow + (qHigh << 4);
                dot += a[baseIdx + i] * (d * (float)sc * (float)(q5 - 16) - dmin * (float)mi);
            }
        }
        result[c] = dot;
    }
}

/* TensorOps.MatMul, TO:60-112.  Returns -1 for unsupported weight types. */
int orc_matmul(const float* a, const uint8_t* b, float* result, int result_len,
               uint32_t bType, int aCols, int bCols) {
    int aRows = result_len / bCols;
    if (aRows == 1) {
        switch (bType) {
        case ORC_Q4_0: mm_fused_q4_0(a, b, result, aCols, bCols); return 0;
        case ORC_Q8_0: mm_fused_q8_0(a, b, result, aCols, bCols); return 0;
        case ORC_Q6_K: mm_fused_q6_k(a, b, result, aCols, bCols); return 0;
        case ORC_Q4_K: mm_fused_q4_k(a, b, result, aCols, bCols); return 0;
        case ORC_Q2_K: mm_fused_q2_k(a, b, result, aCols, bCols); return 0;
        case ORC_Q3_K: mm_fused_q3_k(a, b, result, aCols, bCols); return 0;
        case ORC_Q5_K: mm_fused_q5_k(a, b, result, aCols, bCols); return 0;
        default: break;
        }
    }
    if (orc_byte_count(bType, (uint64_t)aCols) < 0 || bType == ORC_BF16) return -1;
    int fail = 0;
    for (int r = 0; r < aRows; r++) {
        const float* aRow = a + (int64_t)r * aCols;
#pragma omp parallel for num_threads(g_threads) schedule(static) reduction(| : fail)
        for (int c = 0; c < bCols; c++) {
            float* tmp = (float*)malloc(sizeof(float) * (size_t)aCols);
            if (dequantize_row(b, tmp, bType, c, aCols) != 0) fail |= 1;
            else result[(int64_t)r * bCols + c] = dot_product(aRow, tmp, aCols);
            free(tmp);
        }
    }
    return fail ? -1 : 0;
}

/* TensorOps.MatMulF32 (+ SingleRow), TO:437-504: both accumulate 8 lanes of
 * a*b then add the scalar tail, so they share one body. */
void orc_matmul_f32(const float* a, const float* b, float* result, int result_len, int aCols, int bCols) {
    int aRows = result_len / bCols;
    for (int r = 0; r < aRows; r++) {
        const float* aRow = a + (int64_t)r * aCols;
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (int c = 0; c < bCols; c++)
            result[(int64_t)r * bCols + c] = dot_product(aRow, b + (int64_t)c * aCols, aCols);
    }
}

/* TO:699-743 */
static void rope_core(float* q, float* k, const float* cosBuf, const float* sinBuf,
                      int halfDim, int sameSpan) {
    /* The vector part and the scalar tail evaluate the same expressions. */
    for (int i = 0; i < halfDim; i++) {
        float c = cosBuf[i], s = sinBuf[i];
        float q0 = q[i], q1 = q[i + halfDim];
        q[i] = q0 * c - q1 * s;
        q[i + halfDim] = q0 * s + q1 * c;
        if (sameSpan) continue;
        float k0 = k[i], k1 = k[i + halfDim];
        k[i] = k0 * c - k1 * s;
        k[i + halfDim] = k0 * s + k1 * c;
    }
}

/* ApplyRoPE(freqTable), TO:679-696 */
void orc_rope_table(float* q, float* k, int head_dim, int position, const float* freq,
                    int halfDim, int sameSpan) {
    (void)head_dim;
    float* cosBuf = (float*)malloc(sizeof(float) * (size_t)(halfDim > 0 ? halfDim : 1));
    float* sinBuf = (float*)malloc(sizeof(float) * (size_t)(halfDim > 0 ? halfDim : 1));
    for (int i = 0; i < halfDim; i++) {
        float angle = (float)position * freq[i];
        cosBuf[i] = cosf(angle);
        sinBuf[i] = sinf(angle);
    }
    rope_core(q, k, cosBuf, sinBuf, halfDim, sameSpan || q == k);
    free(cosBuf);
    free(sinBuf);
}

/* ApplyRoPE(freqBase, rotaryDim), TO:658-677 */
void orc_rope_base(float* q, float* k, int head_dim, int position, float freqBase,
                   int rotaryDim, int sameSpan) {
    int actual = rotaryDim > 0 ? rotaryDim : head_dim;
    int halfDim = actual / 2;
    float* cosBuf = (float*)malloc(sizeof(float) * (size_t)(halfDim > 0 ? halfDim : 1));
    float* sinBuf = (float*)malloc(sizeof(float) * (size_t)(halfDim > 0 ? halfDim : 1));
    for (int i = 0; i < halfDim; i++) {
        float freq = 1.0f / powf(freqBase, 2.0f * (float)i / (float)actual);
        float angle = (float)position * freq;
        cosBuf[i] = cosf(angle);
        sinBuf[i] = sinf(angle);
    }
    rope_core(q, k, cosBuf, sinBuf, halfDim, sameSpan || q == k);
    free(cosBuf);
    free(sinBuf);
}

/* ---------------------------------------------------------------- VM ---- */

void orc_add(const float* a, const float* b, float* out, int n) {      /* VM:10-25 */
    for (int i = 0; i < n; i++) out[i] = a[i] + b[i];
}
void orc_add_inplace(float* a, const float* b, int n) {                /* VM:27-42 */
    for (int i = 0; i < n; i++) a[i] = a[i] + b[i];
}
void orc_scale(const float* in, float s, float* out, int n) {          /* VM:44-76 */
    for (int i = 0; i < n; i++) out[i] = in[i] * s;
}
void orc_mul(const float* a, const float* b, float* out, int n) {      /* VM:78-93 */
    for (int i = 0; i < n; i++) out[i] = a[i] * b[i];
}

/* One lane of ExpApproxVector, VM:137-166.  The range reduction truncates
 * (Vector.ConvertToInt32), so for negative arguments y spans (-1.04, 0.35]
 * and the polynomial 1+y+y^2/2+y^3/6+y^4/10 is far from exp there; this is
 * the reference behaviour that SiLU and the attention softmax inherit. */
float orc_exp_approx(float x) {
    float clamped = x > -87.3f ? x : -87.3f;    /* Vector.Max */
    clamped = clamped < 88.4f ? clamped : 88.4f; /* Vector.Min */
    int k = (int)(clamped * 1.4426950408889634f + 0.5f);
    float kFlt = (float)k;
    float y = clamped - kFlt * 0.693145751953125f - kFlt * 1.42860677e-6f;
    float c = y * y * 0.5f;
    float pade = 1.0f + y + c + c * y * 0.3333333f + c * y * y * 0.2f;
    float scale = bits_to_float((uint32_t)(k + 127) << 23);
    float result = pade * scale;
    if (x < -87.3f) result = 0.0f;
    if (x > 88.4f) result = INFINITY;
    return result;
}

/* VM:99-116 */
void orc_silu(const float* in, float* out, int n) {
    int i = 0;
    for (; i <= n - VEC; i += VEC)
        for (int l = 0; l < VEC; l++) {
            float x = in[i + l];
            out[i + l] = x / (1.0f + orc_exp_approx(-x));
        }
    for (; i < n; i++) {
        float x = in[i];
        out[i] = x / (1.0f + expf(-x));
    }
}

/* VM:118-135 */
void orc_silu_inplace(float* x, int n) { orc_silu(x, x, n); }

/* TanhApproxVector, VM:196-209 */
static float tanh_approx(float x) {
    float x2 = x * x;
    float approx = x * (27.0f + x2) / (27.0f + 9.0f * x2);
    if (fabsf(x) > 4.0f) return x > 0.0f ? 1.0f : -1.0f;
    return approx;
}

/* The GELU constants of VM:170 / VM:178-180: sqrt(2/pi) and the cubic term. */
#define GELU_C 0.7978845608028654f
#define GELU_C3 0.044715f

/* VectorMath.Gelu(float), VM:169-170 (CpuBackend.GeluScalar): the libm tanh. */
float orc_gelu_scalar(float x) {
    return 0.5f * x * (1.0f + tanhf(GELU_C * (x + GELU_C3 * x * x * x)));
}

/* VectorMath.Gelu(input, result), VM:172-193: the vector lanes take
 * TanhApproxVector of x*c*(1 + c3*x*x*x) (grouped as written there: x^3, not
 * GELU's x^2, inside the bracket, so the lanes return x for x <= -4), the
 * tail the scalar form. */
void orc_gelu(const float* in, float* out, int n) {
    int i = 0;
    for (; i <= n - VEC; i += VEC)
        for (int l = 0; l < VEC; l++) {
            const float x = in[i + l];
            const float t = tanh_approx(x * GELU_C * (1.0f + GELU_C3 * x * x * x));
            out[i + l] = 0.5f * x * (1.0f + t);
        }
    for (; i < n; i++) out[i] = orc_gelu_scalar(in[i]);
}

/* VectorMath.Softcap, VM:286-302, in place: cap * tanh(x / cap), the vector
 * lanes through TanhApproxVector(x * (1/cap)). */
void orc_softcap(float* x, int n, float cap) {
    const float inv = 1.0f / cap;
    int i = 0;
    for (; i <= n - VEC; i += VEC)
        for (int l = 0; l < VEC; l++) x[i + l] = cap * tanh_approx(x[i + l] * inv);
    for (; i < n; i++) x[i] = cap * tanhf(x[i] / cap);
}

/* VectorMath.LayerNorm, VM:342-405: mean and variance as lane sums (lanes,
 * horizontal sum, tail), then w * (x - mean) * invStd (+ bias).  bias NULL is
 * the reference's empty bias span. */
void orc_layer_norm(const float* in, const float* w, const float* b, float* out, int n, float eps) {
    float mean = lane_sum(in, n);
    mean /= (float)n;
    float* sq = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int e = 0; e < n; e++) {
        const float d = in[e] - mean;
        sq[e] = d * d;
    }
    float variance = lane_sum(sq, n);
    free(sq);
    variance /= (float)n;
    const float invStd = 1.0f / sqrtf(variance + eps);
    for (int i = 0; i < n; i++) {
        const float val = w[i] * (in[i] - mean) * invStd;
        out[i] = b ? val + b[i] : val;
    }
}

/* TensorOps.Conv1D, TO:745-775: input and weights are [inputDim][kernelSize];
 * kernelSize 1 is the elementwise product, otherwise each channel's dot in
 * lanes, horizontal sum, then the tail. */
void orc_conv1d(const float* in, const float* w, float* out, int ks, int dim) {
    if (ks == 1) {
        for (int i = 0; i < dim; i++) out[i] = in[i] * w[i];
        return;
    }
    for (int c = 0; c < dim; c++) {
        const float* x = in + (size_t)c * ks;
        const float* y = w + (size_t)c * ks;
        float acc[VEC] = {0};
        int k = 0;
        for (; k <= ks - VEC; k += VEC)
            for (int l = 0; l < VEC; l++) acc[l] = acc[l] + x[k + l] * y[k + l];
        float sum = hsum8(acc);
        for (; k < ks; k++) sum += x[k] * y[k];
        out[c] = sum;
    }
}

/* FindMax, VM:260-284 */
static float find_max(const float* in, int n) {
    if (n >= VEC) {
        float vmax[VEC];
        for (int l = 0; l < VEC; l++) vmax[l] = in[l];
        int mi = VEC;
        for (; mi <= n - VEC; mi += VEC)
            for (int l = 0; l < VEC; l++) vmax[l] = in[mi + l] > vmax[l] ? in[mi + l] : vmax[l];
        float max = -INFINITY;
        for (int l = 0; l < VEC; l++) if (vmax[l] > max) max = vmax[l];
        for (; mi < n; mi++) if (in[mi] > max) max = in[mi];
        return max;
    }
    float m = in[0];
    for (int mi = 1; mi < n; mi++) if (in[mi] > m) m = in[mi];
    return m;
}

/* VectorMath.Softmax, VM:215-258 */
void orc_softmax(float* in, int n, int has_softcap, float cap) {
    if (n == 0) return;
    if (has_softcap) {
        float invCap = 1.0f / cap;
        int si = 0;
        for (; si <= n - VEC; si += VEC)
            for (int l = 0; l < VEC; l++) in[si + l] = cap * tanh_approx(in[si + l] * invCap);
        for (; si < n; si++) in[si] = cap * tanhf(in[si] / cap);
    }
    float max = find_max(in, n);
    float vsum[VEC] = {0};
    int j = 0;
    for (; j <= n - VEC; j += VEC)
        for (int l = 0; l < VEC; l++) {
            float v = orc_exp_approx(in[j + l] - max);
            in[j + l] = v;
            vsum[l] = vsum[l] + v;
        }
    float sum = hsum8(vsum);
    for (; j < n; j++) {
        in[j] = expf(in[j] - max);
        sum += in[j];
    }
    if (g_order) sum = lane_sum(in, n);   /* the same exponentials, summed in the other order */
    float invSum = 1.0f / sum;
    for (int i = 0; i < n; i++) in[i] = in[i] * invSum;
}

/* VectorMath.RmsNorm, VM:308-340 */
void orc_rms_norm(const float* in, const float* w, float* out, int n, float eps) {
    float ss;
    int i = 0;
    if (g_order) {
        float* sq = (float*)malloc(sizeof(float) * (size_t)n);
        for (int e = 0; e < n; e++) sq[e] = in[e] * in[e];
        ss = lane_sum(sq, n);
        free(sq);
    } else {
        float ssv[VEC] = {0};
        for (; i <= n - VEC; i += VEC)
            for (int l = 0; l < VEC; l++) ssv[l] = ssv[l] + in[i + l] * in[i + l];
        ss = hsum8(ssv);
        for (; i < n; i++) ss += in[i] * in[i];
    }
    ss /= (float)n;
    ss += eps;
    float invNorm = 1.0f / sqrtf(ss);
    i = 0;
    for (; i <= n - VEC; i += VEC)
        for (int l = 0; l < VEC; l++) out[i + l] = w[i + l] * in[i + l] * invNorm;
    for (; i < n; i++) out[i] = w[i] * (in[i] * invNorm);
}

/* VectorMath.ArgMax, VM:412-425: first index of the strict maximum. */
int orc_argmax(const float* x, int n) {
    int maxIdx = 0;
    float maxVal = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > maxVal) { maxVal = x[i]; maxIdx = i; }
    return maxIdx;
}

/* ========================================================= Sampler ====== */

/* Sampler.ApplyRepeatPenalty, Sampler.cs:64-81 (every occurrence in the
 * window applies once). */
static void apply_repeat_penalty(float* logits, int n, float penalty, int window, const int* recent, int n_recent) {
    if (penalty == 1.0f || n_recent == 0 || window <= 0) return;
    int start = n_recent - window > 0 ? n_recent - window : 0;
    for (int i = start; i < n_recent; i++) {
        int t = recent[i];
        if (t >= 0 && t < n) {
            if (logits[t] > 0) logits[t] = logits[t] / penalty;
            else logits[t] = logits[t] * penalty;
        }
    }
}

/* Sampler.FindTopK, Sampler.cs:83-127: the first k as the running set, each
 * later value replaces the (first) smallest when strictly larger, then a
 * descending insertion sort. */
static void find_top_k(const float* logits, int k, int n, int* idx, float* val) {
    for (int i = 0; i < k; i++) { idx[i] = i; val[i] = logits[i]; }
    for (int i = k; i < n; i++) {
        int minIdx = 0;
        for (int j = 1; j < k; j++) if (val[j] < val[minIdx]) minIdx = j;
        if (logits[i] > val[minIdx]) { idx[minIdx] = i; val[minIdx] = logits[i]; }
    }
    for (int i = 1; i < k; i++) {
        int ki = idx[i];
        float kv = val[i];
        int j = i - 1;
        while (j >= 0 && val[j] < kv) { idx[j + 1] = idx[j]; val[j + 1] = val[j]; j--; }
        idx[j + 1] = ki;
        val[j + 1] = kv;
    }
}

/* Sampler.FindNucleus, Sampler.cs:129-156: selection sort of the indices by
 * probability (descending), then the shortest prefix whose running sum
 * reaches topP. */
static int find_nucleus(const float* p, int n, float topP, int* idx, float* val) {
    for (int i = 0; i < n; i++) idx[i] = i;
    for (int i = 0; i < n - 1; i++) {
        int maxIdx = i;
        for (int j = i + 1; j < n; j++) if (p[idx[j]] > p[idx[maxIdx]]) maxIdx = j;
        if (maxIdx != i) { int tmp = idx[i]; idx[i] = idx[maxIdx]; idx[maxIdx] = tmp; }
    }
    float cumulative = 0.0f;
    int count = 0;
    for (int i = 0; i < n; i++) {
        val[i] = p[idx[i]];
        cumulative += val[i];
        count++;
        if (cumulative >= topP) break;
    }
    return count;
}

/* Sampler.SampleFromProbabilities, Sampler.cs:158-170, with the draw r given
 * (Random.NextSingle(), Sampler.cs:160-161). */
static int sample_from(const float* p, int n, float r) {
    float cumulative = 0.0f;
    for (int i = 0; i < n; i++) {
        cumulative += p[i];
        if (r <= cumulative) return i;
    }
    return n - 1;
}

/* Sampler.Sample, Sampler.cs:24-62.  recent = the recent-token list, r = the
 * uniform draw.
 *
 * aliased = 1 is the reference as written: `scaled` is the first n floats of
 * samplingBuf (Sampler.cs:30) and FindNucleus is handed samplingBuf again as
 * its output `values` (Sampler.cs:48-50), so while it writes the sorted
 * probabilities (values[i] = probabilities[indices[i]], Sampler.cs:150) it
 * overwrites the probabilities it still reads: rank i reads the value already
 * written at rank indices[i] whenever indices[i] < i.  Two consequences: the
 * nucleus can close early with repeated (larger) values, and when it spans all
 * n tokens the fall-through draw (Sampler.cs:61) walks the rewritten buffer --
 * the probabilities in sorted order -- and returns a rank, not a token id.
 * aliased = 0 gives FindNucleus a buffer of its own: the nucleus of the true
 * probabilities, and the fall-through draw over them in token order. */
int orc_sample_ex(const float* logits, int n, float temperature, int top_k, float top_p, float penalty, int window,
                  const int* recent, int n_recent, float r, int aliased) {
    if (temperature <= 0.0f) return orc_argmax(logits, n);
    float* scaled = (float*)malloc(sizeof(float) * (size_t)n);
    float* buf = aliased ? scaled : (float*)malloc(sizeof(float) * (size_t)n);
    int* ibuf = (int*)malloc(sizeof(int) * (size_t)n);
    memcpy(scaled, logits, sizeof(float) * (size_t)n);
    apply_repeat_penalty(scaled, n, penalty, window, recent, n_recent);
    orc_scale(scaled, 1.0f / temperature, scaled, n);
    int result;
    if (top_k > 0 && top_k < n) {
        find_top_k(scaled, top_k, n, ibuf, buf);
        orc_softmax(buf, top_k, 0, 0.0f);
        result = ibuf[sample_from(buf, top_k, r)];
    } else {
        orc_softmax(scaled, n, 0, 0.0f);
        result = -1;
        if (top_p < 1.0f) {
            int m = find_nucleus(scaled, n, top_p, ibuf, buf);
            if (m < n) {
                float sum = 0.0f;
                for (int i = 0; i < m; i++) sum += buf[i];
                orc_scale(buf, 1.0f / sum, buf, m);
                result = ibuf[sample_from(buf, m, r)];
            }
        }
        if (result < 0) result = sample_from(scaled, n, r);
    }
    if (buf != scaled) free(buf);
    free(scaled);
    free(ibuf);
    return result;
}

int orc_sample(const float* logits, int n, float temperature, int top_k, float top_p, float penalty, int window,
               const int* recent, int n_recent, float r) {
    return orc_sample_ex(logits, n, temperature, top_k, top_p, penalty, window, recent, n_recent, r, 1);
}

/* ============================================================ GGUF ====== */

enum { GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR,
       GV_ARR, GV_U64, GV_I64, GV_F64 };

typedef struct {
    const char* key; uint64_t keylen;
    uint32_t type;
    const uint8_t* val;         /* points at the value (for arrays: at the first element) */
    uint32_t arr_type; uint64_t arr_len;
} gg_kv;

typedef struct {
    const char* name; uint64_t namelen;
    uint32_t ndim; uint32_t dims[4];
    uint32_t type; uint64_t offset;
    uint32_t nelem;             /* uint, as GR:113-115 computes it */
    const uint8_t* data; int64_t nbytes;
} gg_tensor;

typedef struct {
    const uint8_t* p; const uint8_t* end; int err;
} cursor;

static uint64_t rd(cursor* c, int n) {
    if (c->err || c->p + n > c->end) { c->err = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)c->p[i] << (8 * i);
    c->p += n;
    return v;
}

static int value_size(uint32_t t) {
    switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;  /* GR:68 reads one byte for Bool */
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: return 8;
    default: return -1;
    }
}

static void skip_value(cursor* c, uint32_t t) {
    if (t == GV_STR) { uint64_t n = rd(c, 8); if (c->p + n > c->end) c->err = 1; else c->p += n; return; }
    if (t == GV_ARR) {
        uint32_t et = (uint32_t)rd(c, 4); uint64_t n = rd(c, 8);
        for (uint64_t i = 0; i < n && !c->err; i++) skip_value(c, et);
        return;
    }
    int s = value_size(t);
    if (s < 0) { c->err = 1; return; }
    if (c->p + s > c->end) c->err = 1; else c->p += s;
}

struct orc_model {
    const uint8_t* buf; size_t len; int mapped;
    gg_kv* kv; uint64_t nkv;
    gg_tensor* t; uint64_t nt;
    orc_config cfg;
    int kv_fp16;
    /* per layer */
    const gg_tensor **attn_norm, **ffn_norm, **wq, **wk, **wv, **wo, **wg, **wu, **wd;
    const gg_tensor** wqkv;     /* fused Q/K/V (QkvLayout.Fused), else NULL */
    float **q_norm_f, **k_norm_f;   /* per-head Q/K RmsNorm weights [head_dim] (NULL entries: none) */
    int ffn_buf_len;            /* InferenceBuffers' FfnBuf length */
    float **attn_norm_f, **ffn_norm_f;
    const gg_tensor *embd, *out, *out_norm;
    float* out_norm_f;
    float* rope_freqs;
    /* KV cache, layer-major [L][ctx][kvDim] (KV:19-20) */
    float *kcache, *vcache;
    int cache_ctx;
    /* buffers (InferenceBuffers.cs:29-62) */
    float *hidden, *norm, *normtmp, *q, *k, *v, *attn_result, *attn_out, *ffn_buf, *ffn_result,
          *scores, *logits;
};

static const gg_kv* find_kv(const orc_model* m, const char* key) {
    size_t kl = strlen(key);
    for (uint64_t i = 0; i < m->nkv; i++)
        if (m->kv[i].keylen == kl && memcmp(m->kv[i].key, key, kl) == 0) return &m->kv[i];
    return NULL;
}

static int kv_number(const gg_kv* kv, double* out) {
    cursor c = {kv->val, kv->val + 8, 0};
    switch (kv->type) {
    case GV_U8: *out = (double)kv->val[0]; return 1;
    case GV_I8: *out = (double)(int8_t)kv->val[0]; return 1;
    case GV_U16: *out = (double)(uint16_t)rd(&c, 2); return 1;
    case GV_I16: *out = (double)(int16_t)rd(&c, 2); return 1;
    case GV_U32: *out = (double)(uint32_t)rd(&c, 4); return 1;
    case GV_I32: *out = (double)(int32_t)rd(&c, 4); return 1;
    case GV_F32: { uint32_t b = (uint32_t)rd(&c, 4); *out = (double)bits_to_float(b); return 1; }
    case GV_BOOL: *out = kv->val[0] != 0; return 1;
    case GV_U64: *out = (double)rd(&c, 8); return 1;
    case GV_I64: *out = (double)(int64_t)rd(&c, 8); return 1;
    case GV_F64: { uint64_t b = rd(&c, 8); double d; memcpy(&d, &b, 8); *out = d; return 1; }
    default: return 0;
    }
}

static int get_int(const orc_model* m, const char* arch, const char* key, int def) {
    char full[256];
    snprintf(full, sizeof full, "%s.%s", arch, key);
    const gg_kv* kv = find_kv(m, full);
    double d;
    if (kv && kv_number(kv, &d)) return (int)d;
    return def;
}

static float get_float(const orc_model* m, const char* arch, const char* key, float def, int* found) {
    char full[256];
    snprintf(full, sizeof full, "%s.%s", arch, key);
    const gg_kv* kv = find_kv(m, full);
    double d;
    if (found) *found = 0;
    if (kv && kv_number(kv, &d)) { if (found) *found = 1; return (float)d; }
    return def;
}

static const gg_tensor* find_tensor(const orc_model* m, const char* name) {
    size_t nl = strlen(name);
    for (uint64_t i = 0; i < m->nt; i++)
        if (m->t[i].namelen == nl && strncasecmp(m->t[i].name, name, nl) == 0 && m->t[i].data)
            return &m->t[i];
    return NULL;
}

static float* dequant_whole(const gg_tensor* t) {
    float* r = (float*)malloc(sizeof(float) * (size_t)t->nelem);
    int rows = t->ndim > 1 ? (int)t->dims[1] : 1;
    if (rows <= 0) rows = 1;
    orc_dequantize(t->data, r, t->type, rows, (int)(t->nelem / (uint32_t)rows));
    return r;
}

static void seterr(char* err, int errlen, const char* msg) {
    if (err && errlen > 0) snprintf(err, (size_t)errlen, "%s", msg);
}

void orc_model_close(orc_model* m) {
    if (!m) return;
    if (m->mapped) munmap((void*)m->buf, m->len);
    free(m->kv); free(m->t);
    free(m->attn_norm); free(m->ffn_norm); free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->wqkv);
    free(m->wg); free(m->wu); free(m->wd);
    if (m->attn_norm_f) for (int l = 0; l < m->cfg.layers; l++) free(m->attn_norm_f[l]);
    if (m->ffn_norm_f) for (int l = 0; l < m->cfg.layers; l++) free(m->ffn_norm_f[l]);
    if (m->q_norm_f) for (int l = 0; l < m->cfg.layers; l++) free(m->q_norm_f[l]);
    if (m->k_norm_f) for (int l = 0; l < m->cfg.layers; l++) free(m->k_norm_f[l]);
    free(m->q_norm_f); free(m->k_norm_f);
    free(m->attn_norm_f); free(m->ffn_norm_f); free(m->out_norm_f); free(m->rope_freqs);
    free(m->kcache); free(m->vcache);
    free(m->hidden); free(m->norm); free(m->normtmp); free(m->q); free(m->k); free(m->v);
    free(m->attn_result); free(m->attn_out); free(m->ffn_buf); free(m->ffn_result);
    free(m->scores); free(m->logits);
    free(m);
}

static int alloc_buffers(orc_model* m) {
    orc_config* c = &m->cfg;
    int kvdim = c->kv_heads * c->head_dim;
    size_t cache = (size_t)c->layers * (size_t)c->context * (size_t)kvdim;
    free(m->kcache); free(m->vcache);
    m->kcache = (float*)calloc(cache ? cache : 1, sizeof(float));
    m->vcache = (float*)calloc(cache ? cache : 1, sizeof(float));
    m->cache_ctx = c->context;
    free(m->scores);
    m->scores = (float*)calloc((size_t)(c->hidden > c->context ? c->hidden : c->context), sizeof(float));
    return m->kcache && m->vcache && m->scores;
}

int orc_model_set_context(orc_model* m, int context) {
    if (context <= 0) return 0;
    m->cfg.context = context;
    return alloc_buffers(m) ? 0 : -1;
}

/* GgufReader.Read (GR:8-42) + ArchitectureResolver.Resolve (AR:14-112) for
 * the LLaMA-like template + LoadedModel.LoadTensors (LM:77-107). */
orc_model* orc_model_open_buffer(const uint8_t* buf, size_t len, int kv_fp16, char* err, int errlen) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->buf = buf; m->len = len; m->kv_fp16 = kv_fp16;
    cursor c = {buf, buf + len, 0};
    if (len < 4 || memcmp(buf, "GGUF", 4) != 0) { seterr(err, errlen, "Invalid GGUF magic. Expected 'GGUF'."); free(m); return NULL; }
    c.p += 4;
    uint32_t version = (uint32_t)rd(&c, 4);
    if (version < 2) { seterr(err, errlen, "Unsupported GGUF version"); free(m); return NULL; }
    m->nt = rd(&c, 8);
    m->nkv = rd(&c, 8);
    if (c.err || m->nkv > (1u << 24) || m->nt > (1u << 24)) { seterr(err, errlen, "truncated GGUF header"); free(m); return NULL; }
    m->kv = (gg_kv*)calloc(m->nkv ? m->nkv : 1, sizeof(gg_kv));
    for (uint64_t i = 0; i < m->nkv && !c.err; i++) {
        uint64_t kl = rd(&c, 8);
        if (c.p + kl > c.end) { c.err = 1; break; }
        m->kv[i].key = (const char*)c.p; m->kv[i].keylen = kl; c.p += kl;
        m->kv[i].type = (uint32_t)rd(&c, 4);
        if (m->kv[i].type == GV_ARR) {
            m->kv[i].arr_type = (uint32_t)rd(&c, 4);
            m->kv[i].arr_len = rd(&c, 8);
            m->kv[i].val = c.p;
            for (uint64_t j = 0; j < m->kv[i].arr_len && !c.err; j++) skip_value(&c, m->kv[i].arr_type);
        } else {
            m->kv[i].val = c.p;
            skip_value(&c, m->kv[i].type);
        }
    }
    m->t = (gg_tensor*)calloc(m->nt ? m->nt : 1, sizeof(gg_tensor));
    for (uint64_t i = 0; i < m->nt && !c.err; i++) {
        gg_tensor* t = &m->t[i];
        uint64_t nl = rd(&c, 8);
        if (c.p + nl > c.end) { c.err = 1; break; }
        t->name = (const char*)c.p; t->namelen = nl; c.p += nl;
        t->ndim = (uint32_t)rd(&c, 4);
        if (t->ndim > 4) { c.err = 1; break; }
        uint32_t ne = t->ndim ? 1u : 0u;
        for (uint32_t d = 0; d < t->ndim; d++) { t->dims[d] = (uint32_t)rd(&c, 8); ne *= t->dims[d]; }
        t->type = (uint32_t)rd(&c, 4);
        t->offset = rd(&c, 8);
        t->nelem = ne;
    }
    if (c.err) { seterr(err, errlen, "truncated GGUF metadata"); orc_model_close(m); return NULL; }
    uint32_t alignment = 32;
    const gg_kv* al = find_kv(m, "general.alignment");
    if (al && al->type == GV_U32) { cursor ac = {al->val, al->val + 4, 0}; alignment = (uint32_t)rd(&ac, 4); }
    uint64_t dataOff = (uint64_t)(c.p - buf);
    dataOff += (alignment - (dataOff % alignment)) % alignment;
    for (uint64_t i = 0; i < m->nt; i++) {
        gg_tensor* t = &m->t[i];
        int64_t bc = orc_byte_count(t->type, t->nelem);
        t->nbytes = bc;
        if (bc <= 0) continue;
        uint64_t off = dataOff + t->offset;
        if (off + (uint64_t)bc > len) continue;      /* LM:87-88: silently skipped */
        t->data = buf + off;
    }

    /* ArchitectureResolver (LLaMA-like subset). */
    const gg_kv* akv = find_kv(m, "general.architecture");
    char arch[64] = {0};
    if (!akv || akv->type != GV_STR) { seterr(err, errlen, "GGUF model missing 'general.architecture' metadata key."); orc_model_close(m); return NULL; }
    {
        cursor sc = {akv->val, buf + len, 0};
        uint64_t sl = rd(&sc, 8);
        if (sl >= sizeof arch) sl = sizeof arch - 1;
        memcpy(arch, sc.p, sl);
    }
    if (strcasecmp(arch, "llama") && strcasecmp(arch, "phi3") && strcasecmp(arch, "qwen2") && strcasecmp(arch, "stablelm")) {
        seterr(err, errlen, "architecture is not LLaMA-like"); orc_model_close(m); return NULL;
    }
    orc_config* cf = &m->cfg;
    cf->hidden = get_int(m, arch, "embedding_length", 0);
    cf->layers = get_int(m, arch, "block_count", 0);
    cf->context = get_int(m, arch, "context_length", 0);
    cf->ffn = get_int(m, arch, "feed_forward_length", 0);
    cf->heads = get_int(m, arch, "attention.head_count", 0);
    {
        char full[256]; snprintf(full, sizeof full, "%s.attention.head_count_kv", arch);
        const gg_kv* hk = find_kv(m, full);
        if (hk && hk->type == GV_ARR && hk->arr_len > 0) {
            int mx = 0; cursor ac = {hk->val, buf + len, 0};
            for (uint64_t j = 0; j < hk->arr_len; j++) {
                int sz = value_size(hk->arr_type); if (sz < 0) break;
                gg_kv tmp = {0}; tmp.type = hk->arr_type; tmp.val = ac.p; double d = 0;
                kv_number(&tmp, &d); ac.p += sz;
                if ((int)d > mx) mx = (int)d;
            }
            cf->kv_heads = mx;
        } else cf->kv_heads = get_int(m, arch, "attention.head_count_kv", cf->heads);
    }
    cf->head_dim = get_int(m, arch, "attention.key_length", cf->hidden / (cf->heads > 1 ? cf->heads : 1));
    {
        const gg_kv* tk = find_kv(m, "tokenizer.ggml.tokens");
        cf->vocab = (tk && tk->type == GV_ARR) ? (int)tk->arr_len : 0;
    }
    int found = 0;
    cf->eps = get_float(m, arch, "attention.layer_norm_rms_epsilon", 0.0f, &found);
    if (!found) { seterr(err, errlen, "No RMS norm epsilon found"); orc_model_close(m); return NULL; }
    cf->rope_base = get_float(m, arch, "rope.freq_base", 10000.0f, NULL);
    cf->rope_dim = get_int(m, arch, "rope.dimension_count", cf->head_dim);
    cf->rope_scaling_factor = get_float(m, arch, "rope.scaling.factor", 1.0f, NULL);
    {
        char full[256]; snprintf(full, sizeof full, "%s.rope.scaling.type", arch);
        const gg_kv* st = find_kv(m, full);
        cf->rope_scaling_linear = 0;
        if (st && st->type == GV_STR) {
            cursor sc = {st->val, buf + len, 0}; uint64_t sl = rd(&sc, 8);
            cf->rope_scaling_linear = (sl == 6 && strncasecmp((const char*)sc.p, "linear", 6) == 0);
        }
    }
    cf->sliding_window = get_int(m, arch, "attention.sliding_window", 0);
    cf->bos = get_int(m, "tokenizer.ggml", "bos_token_id", 1);
    cf->eos = get_int(m, "tokenizer.ggml", "eos_token_id", 2);

    /* Tensors (TensorNameResolver.cs:22-107). */
    int L = cf->layers;
    m->attn_norm = calloc((size_t)L, sizeof(void*)); m->ffn_norm = calloc((size_t)L, sizeof(void*));
    m->wq = calloc((size_t)L, sizeof(void*)); m->wk = calloc((size_t)L, sizeof(void*));
    m->wv = calloc((size_t)L, sizeof(void*)); m->wo = calloc((size_t)L, sizeof(void*));
    m->wg = calloc((size_t)L, sizeof(void*)); m->wu = calloc((size_t)L, sizeof(void*));
    m->wd = calloc((size_t)L, sizeof(void*));
    m->attn_norm_f = calloc((size_t)L, sizeof(float*)); m->ffn_norm_f = calloc((size_t)L, sizeof(float*));
    char name[128];
#define NEED(dst, fmt)                                                           \
    do {                                                                         \
        snprintf(name, sizeof name, fmt, l);                                     \
        dst = find_tensor(m, name);                                              \
        if (!dst) { char e[200]; snprintf(e, sizeof e, "Tensor '%s' not found.", name); \
                    seterr(err, errlen, e); orc_model_close(m); return NULL; }   \
    } while (0)
    /* QkvLayout: Fused when any tensor name contains "attn_qkv"
       (ArchitectureResolver.cs:145-146); then every layer needs its
       blk.N.attn_qkv.weight (TensorNameResolver.cs:123-126). */
    int fused = 0;
    for (uint64_t i = 0; i < m->nt && !fused; i++)
        for (uint64_t j = 0; j + 8 <= m->t[i].namelen && !fused; j++)
            if (memcmp(m->t[i].name + j, "attn_qkv", 8) == 0) fused = 1;
    if (fused) m->wqkv = calloc((size_t)L, sizeof(void*));
    for (int l = 0; l < L; l++) {
        NEED(m->attn_norm[l], "blk.%d.attn_norm.weight");
        if (fused) {
            NEED(m->wqkv[l], "blk.%d.attn_qkv.weight");
        } else {
            NEED(m->wq[l], "blk.%d.attn_q.weight");
            NEED(m->wk[l], "blk.%d.attn_k.weight");
            NEED(m->wv[l], "blk.%d.attn_v.weight");
        }
        NEED(m->wo[l], "blk.%d.attn_output.weight");
        NEED(m->wg[l], "blk.%d.ffn_gate.weight");
        NEED(m->wu[l], "blk.%d.ffn_up.weight");
        NEED(m->wd[l], "blk.%d.ffn_down.weight");
        snprintf(name, sizeof name, "blk.%d.ffn_norm.weight", l);
        m->ffn_norm[l] = find_tensor(m, name);
        if (!m->ffn_norm[l]) m->ffn_norm[l] = m->attn_norm[l];   /* IE:547 */
        m->attn_norm_f[l] = dequant_whole(m->attn_norm[l]);
        m->ffn_norm_f[l] = dequant_whole(m->ffn_norm[l]);
        /* optional per-head Q/K norms (TensorNameResolver: attn_q_norm / attn_k_norm) */
        const gg_tensor* qn; const gg_tensor* kn;
        snprintf(name, sizeof name, "blk.%d.attn_q_norm.weight", l); qn = find_tensor(m, name);
        snprintf(name, sizeof name, "blk.%d.attn_k_norm.weight", l); kn = find_tensor(m, name);
        if ((qn || kn) && !m->q_norm_f) {
            m->q_norm_f = calloc((size_t)L, sizeof(float*));
            m->k_norm_f = calloc((size_t)L, sizeof(float*));
        }
        if (qn) m->q_norm_f[l] = dequant_whole(qn);
        if (kn) m->k_norm_f[l] = dequant_whole(kn);
    }
#undef NEED
    m->embd = find_tensor(m, "token_embd.weight");
    m->out_norm = find_tensor(m, "output_norm.weight");
    if (!m->out_norm) m->out_norm = find_tensor(m, "token_embd_norm.weight");
    m->out = find_tensor(m, "output.weight");
    cf->tied_embeddings = m->out == NULL;
    if (!m->out) m->out = m->embd;
    if (!m->embd || !m->out_norm) { seterr(err, errlen, "missing token_embd/output_norm"); orc_model_close(m); return NULL; }
    m->out_norm_f = dequant_whole(m->out_norm);

    /* PrecomputeRopeFrequencies, IE:57-72 */
    int rot = cf->rope_dim > 0 ? cf->rope_dim : cf->head_dim;
    int half = rot / 2;
    m->rope_freqs = (float*)calloc((size_t)(half > 0 ? half : 1), sizeof(float));
    for (int i = 0; i < half; i++) {
        float freq = 1.0f / powf(cf->rope_base, 2.0f * (float)i / (float)rot);
        if (cf->rope_scaling_linear && cf->rope_scaling_factor > 1.0f) freq /= cf->rope_scaling_factor;
        m->rope_freqs[i] = freq;
    }

    int qdim = cf->heads * cf->head_dim, kvdim = cf->kv_heads * cf->head_dim;
    m->hidden = calloc((size_t)cf->hidden, 4); m->norm = calloc((size_t)cf->hidden, 4);
    m->normtmp = calloc((size_t)cf->hidden, 4);
    m->q = calloc((size_t)qdim, 4); m->k = calloc((size_t)kvdim, 4); m->v = calloc((size_t)kvdim, 4);
    m->attn_result = calloc((size_t)(qdim > cf->hidden ? qdim : cf->hidden), 4);
    m->attn_out = calloc((size_t)cf->hidden, 4);
    int maxInter = 2 * cf->ffn > 3 * cf->hidden ? 2 * cf->ffn : 3 * cf->hidden;
    m->ffn_buf = calloc((size_t)maxInter, 4);
    m->ffn_buf_len = maxInter;
    m->ffn_result = calloc((size_t)cf->hidden, 4);
    m->logits = calloc((size_t)(cf->vocab > 0 ? cf->vocab : 1), 4);
    if (!alloc_buffers(m)) { seterr(err, errlen, "out of memory for KV cache"); orc_model_close(m); return NULL; }
    return m;
}

orc_model* orc_model_open_file(const char* path, int kv_fp16, char* err, int errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { seterr(err, errlen, "cannot open file"); return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); seterr(err, errlen, "cannot stat file"); return NULL; }
    void* p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) { seterr(err, errlen, "mmap failed"); return NULL; }
    orc_model* m = orc_model_open_buffer((const uint8_t*)p, (size_t)st.st_size, kv_fp16, err, errlen);
    if (!m) { munmap(p, (size_t)st.st_size); return NULL; }
    m->mapped = 1;
    return m;
}

void orc_model_config(const orc_model* m, orc_config* out) { *out = m->cfg; }

/* MatMulFromTensor, IE:604-617 */
static int matmul_tensor(orc_model* m, const float* input, const gg_tensor* w, float* out, int cols) {
    int inDim = (int)w->dims[0];
    if (w->type == ORC_F32) {
        orc_matmul_f32(input, (const float*)w->data, out, cols, inDim, cols);
        return 0;
    }
    (void)m;
    return orc_matmul(input, w->data, out, cols, w->type, inDim, cols);
}

static inline float kv_store(const orc_model* m, float x) {
    return m->kv_fp16 ? orc_half_to_float(orc_float_to_half(x)) : x;
}

/* One q head h at `position` over the cached K/V of `layer` (IE:384-442):
 * score_s = (q . K_s) * (1/sqrt(hd)) with 8-lane partial sums, Softmax, then
 * out = sum_s V_s * p_s with s ascending.  q head h reads kv head h / (H/Hkv). */
static void attend_head(const orc_model* m, int layer, int position, int h, const float* qs, float* rs) {
    const orc_config* c = &m->cfg;
    int hd = c->head_dim, H = c->heads, Hkv = c->kv_heads, kvdim = Hkv * hd;
    int seqLen = position + 1;
    int attnStart = c->sliding_window > 0 ? (seqLen - c->sliding_window > 0 ? seqLen - c->sliding_window : 0) : 0;
    int attnLen = seqLen - attnStart;
    const float* keys = m->kcache + (size_t)layer * (size_t)m->cache_ctx * (size_t)kvdim;
    const float* values = m->vcache + (size_t)layer * (size_t)m->cache_ctx * (size_t)kvdim;
    int group = H / Hkv;
    float invSqrt = 1.0f / sqrtf((float)hd);
    int kvH = h / group;
    float* score = (float*)malloc(sizeof(float) * (size_t)attnLen);
    float prod[512];
    for (int s = attnStart; s < seqLen; s++) {
        const float* kr = keys + (size_t)s * kvdim + (size_t)kvH * hd;
        float dot;
        if (g_order) {
            for (int d = 0; d < hd; d++) prod[d] = qs[d] * kr[d];
            dot = lane_sum(prod, hd);
        } else {
            float acc[VEC] = {0};
            int d = 0;
            for (; d <= hd - VEC; d += VEC)
                for (int l = 0; l < VEC; l++) acc[l] = acc[l] + qs[d + l] * kr[d + l];
            dot = hsum8(acc);
            for (; d < hd; d++) dot += qs[d] * kr[d];
        }
        score[s - attnStart] = dot * invSqrt;
    }
    orc_softmax(score, attnLen, 0, 0.0f);
    for (int d = 0; d < hd; d++) rs[d] = 0.0f;
    if (g_order) {   /* other orders: partial sums over ORD_PVCH-position chunks, chunks in order */
        const int ch = ORD_PVCH[g_order];
        for (int s0 = 0; s0 < attnLen; s0 += ch) {
            for (int d = 0; d < hd; d++) prod[d] = 0.0f;
            for (int s = s0; s < attnLen && s < s0 + ch; s++) {
                float sc = score[s];
                const float* vr = values + (size_t)(attnStart + s) * kvdim + (size_t)kvH * hd;
                for (int d = 0; d < hd; d++) prod[d] = prod[d] + vr[d] * sc;
            }
            for (int d = 0; d < hd; d++) rs[d] = rs[d] + prod[d];
        }
    } else {
        for (int s = 0; s < attnLen; s++) {
            float sc = score[s];
            const float* vr = values + (size_t)(attnStart + s) * kvdim + (size_t)kvH * hd;
            for (int d = 0; d < hd; d++) rs[d] = rs[d] + vr[d] * sc;
        }
    }
    free(score);
}

/* AttentionForward, IE:304-450 (separate or fused Q/K/V, optional per-head Q/K norms, no softcap). */
static int attention(orc_model* m, int layer, int position) {
    orc_config* c = &m->cfg;
    int hd = c->head_dim, H = c->heads, Hkv = c->kv_heads;
    int qdim = H * hd, kvdim = Hkv * hd, hidden = c->hidden;
    const float* input = m->norm;
    int rc = 0;
    if (m->wqkv) {
        /* fused: one MatMul into FfnBuf (or a fresh array when it is too
           short), then q, k, v copied out of it (IE:321-332) */
        const int fusedCols = qdim + 2 * kvdim;
        float* fb = fusedCols <= m->ffn_buf_len ? m->ffn_buf : (float*)malloc(sizeof(float) * (size_t)fusedCols);
        if (!fb) return -4;
        rc |= matmul_tensor(m, input, m->wqkv[layer], fb, fusedCols);
        memcpy(m->q, fb, sizeof(float) * (size_t)qdim);
        memcpy(m->k, fb + qdim, sizeof(float) * (size_t)kvdim);
        memcpy(m->v, fb + qdim + kvdim, sizeof(float) * (size_t)kvdim);
        if (fb != m->ffn_buf) free(fb);
    } else {
        rc |= matmul_tensor(m, input, m->wq[layer], m->q, (int)(m->wq[layer]->nelem / (uint32_t)hidden));
        rc |= matmul_tensor(m, input, m->wk[layer], m->k, (int)(m->wk[layer]->nelem / (uint32_t)hidden));
        rc |= matmul_tensor(m, input, m->wv[layer], m->v, (int)(m->wv[layer]->nelem / (uint32_t)hidden));
    }
    if (rc) return rc;
    /* per-head RmsNorm of q and of k before their RoPE (IE:354-359, IE:367-372) */
    if (m->q_norm_f && m->q_norm_f[layer])
        for (int h = 0; h < H; h++) orc_rms_norm(m->q + h * hd, m->q_norm_f[layer], m->q + h * hd, hd, c->eps);
    if (m->k_norm_f && m->k_norm_f[layer])
        for (int h = 0; h < Hkv; h++) orc_rms_norm(m->k + h * hd, m->k_norm_f[layer], m->k + h * hd, hd, c->eps);
    int half = (c->rope_dim > 0 ? c->rope_dim : hd) / 2;
    for (int h = 0; h < H; h++) {
        float* qh = m->q + h * hd;
        orc_rope_table(qh, qh, hd, position, m->rope_freqs, half, 1);
    }
    size_t slot = ((size_t)layer * (size_t)m->cache_ctx + (size_t)position) * (size_t)kvdim;
    for (int h = 0; h < Hkv; h++) {
        float* kh = m->k + h * hd;
        float* vh = m->v + h * hd;
        orc_rope_table(kh, kh, hd, position, m->rope_freqs, half, 1);
        for (int d = 0; d < hd; d++) {
            m->kcache[slot + (size_t)h * hd + d] = kv_store(m, kh[d]);
            m->vcache[slot + (size_t)h * hd + d] = kv_store(m, vh[d]);
        }
    }
    float* result = m->attn_result;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int h = 0; h < H; h++) attend_head(m, layer, position, h, m->q + h * hd, result + h * hd);
    int outCols = (int)(m->wo[layer]->nelem / (uint32_t)(H * hd));
    rc = matmul_tensor(m, result, m->wo[layer], m->attn_out, outCols);
    memcpy(m->attn_result, m->attn_out, sizeof(float) * (size_t)hidden);
    (void)qdim;
    return rc;
}

/* FfnForward SwiGLU branch, IE:452-476 */
static int ffn(orc_model* m, int layer) {
    int hidden = m->cfg.hidden;
    int gateCols = (int)(m->wg[layer]->nelem / (uint32_t)hidden);
    int upCols = (int)(m->wu[layer]->nelem / (uint32_t)hidden);
    int rc = matmul_tensor(m, m->norm, m->wg[layer], m->ffn_buf, gateCols);
    orc_silu_inplace(m->ffn_buf, gateCols);
    rc |= matmul_tensor(m, m->norm, m->wu[layer], m->ffn_buf + gateCols, upCols);
    orc_mul(m->ffn_buf, m->ffn_buf + gateCols, m->ffn_buf, gateCols);
    rc |= matmul_tensor(m, m->ffn_buf, m->wd[layer], m->ffn_result, hidden);
    return rc;
}

/* ProcessToken (IE:134-146) with ProcessLlamaLikeLayer (IE:184-196). */
int orc_process_token(orc_model* m, int token, int position, float* logits) {
    orc_config* c = &m->cfg;
    if (position < 0 || position >= m->cache_ctx) return -2;      /* KV:29-33 slice throws */
    if (token < 0 || (uint32_t)token >= m->embd->dims[1]) return -3;
    /* GetEmbedding, IE:148-156 */
    int64_t rowBytes = orc_byte_count(m->embd->type, (uint64_t)m->embd->dims[0]);
    orc_dequantize(m->embd->data + (int64_t)token * rowBytes, m->hidden, m->embd->type, 1, (int)m->embd->dims[0]);
    int rc = 0;
    for (int l = 0; l < c->layers && !rc; l++) {
        orc_rms_norm(m->hidden, m->attn_norm_f[l], m->norm, c->hidden, c->eps);
        rc |= attention(m, l, position);
        orc_add_inplace(m->hidden, m->attn_result, c->hidden);
        orc_rms_norm(m->hidden, m->ffn_norm_f[l], m->norm, c->hidden, c->eps);
        rc |= ffn(m, l);
        orc_add_inplace(m->hidden, m->ffn_result, c->hidden);
    }
    if (rc) return -1;
    /* ApplyFinalNorm IE:575-581 */
    memcpy(m->normtmp, m->hidden, sizeof(float) * (size_t)c->hidden);
    orc_rms_norm(m->normtmp, m->out_norm_f, m->hidden, c->hidden, c->eps);
    /* ComputeLogits IE:583-602 */
    if (m->out->type == ORC_F32)
        orc_matmul_f32(m->hidden, (const float*)m->out->data, m->logits, c->vocab, c->hidden, c->vocab);
    else if (orc_matmul(m->hidden, m->out->data, m->logits, c->vocab, m->out->type, c->hidden, c->vocab))
        return -1;
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)c->vocab);
    return 0;
}

/* Generate, IE:74-132, greedy (Sampler.cs:26-27). */
int orc_generate(orc_model* m, const int* prompt, int n_prompt, int max_tokens, int eos,
                 int* tokens_out, int* n_out, float* logits_out) {
    orc_config* c = &m->cfg;
    int pos = 0, rc = 0;
    *n_out = 0;
    for (int i = 0; i < n_prompt; i++) {
        if ((rc = orc_process_token(m, prompt[i], i, NULL))) return rc;
        pos++;
    }
    if (n_prompt == 0) {
        int initial = c->bos > 0 ? c->bos : 0;
        if ((rc = orc_process_token(m, initial, 0, NULL))) return rc;
        pos++;
    }
    int generated = 0;
    while (generated < max_tokens) {
        if (logits_out) memcpy(logits_out + (size_t)generated * c->vocab, m->logits, sizeof(float) * (size_t)c->vocab);
        int next = orc_argmax(m->logits, c->vocab);
        tokens_out[generated] = next;
        *n_out = generated + 1;
        if (eos >= 0 && next == eos) break;
        if (generated + 1 == max_tokens) break;   /* the reference's last ProcessToken is unobservable */
        if ((rc = orc_process_token(m, next, pos, NULL))) return rc;
        pos++;
        generated++;
    }
    return 0;
}

/* Seeded KV contents (no reference counterpart; timing and long-context
 * parity): element e of the K (kind 0) or V (kind 1) row of (layer, pos) is a
 * SplitMix64 finaliser of the packed key, 24 bits scaled to [-1.5, 1.5) -- the
 * same values llmdot_hip_model_kv_fill_random writes. */
static float kv_fill_value(uint64_t seed, int layer, int kind, int pos, int e) {
    uint64_t key = ((uint64_t)(2 * layer + kind) << 44) | ((uint64_t)pos << 20) | (uint64_t)e;
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (key + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f) - 0.5f) * 3.0f;
}

int orc_kv_fill_random(orc_model* m, int n, uint64_t seed) {
    if (n < 0 || n > m->cache_ctx) return -2;
    int kvdim = m->cfg.kv_heads * m->cfg.head_dim;
    for (int l = 0; l < m->cfg.layers; l++)
        for (int p = 0; p < n; p++)
            for (int e = 0; e < kvdim; e++) {
                size_t i = ((size_t)l * m->cache_ctx + p) * kvdim + e;
                m->kcache[i] = kv_store(m, kv_fill_value(seed, l, 0, p, e));
                m->vcache[i] = kv_store(m, kv_fill_value(seed, l, 1, p, e));
            }
    return 0;
}

int orc_kv_read(const orc_model* m, int layer, int position, float* k, float* v) {
    if (layer < 0 || layer >= m->cfg.layers || position < 0 || position >= m->cache_ctx) return -2;
    int kvdim = m->cfg.kv_heads * m->cfg.head_dim;
    size_t slot = ((size_t)layer * m->cache_ctx + position) * kvdim;
    memcpy(k, m->kcache + slot, sizeof(float) * (size_t)kvdim);
    memcpy(v, m->vcache + slot, sizeof(float) * (size_t)kvdim);
    return 0;
}

/* ===================================================== prompt batches ====== */
/* Prompt processing with the tokens of a chunk going through each layer
 * together.  No counterpart in the reference (Generate processes the prompt
 * one ProcessToken at a time, IE:84-88): this is test infrastructure that
 * makes long prompts affordable for the expected-value runs.  Every token
 * gets exactly the operations orc_process_token applies at its position, in
 * the same order, so the KV cache and the last token's logits are bitwise
 * those of the sequential loop (tests/test_oracle.py pins this).  The speed
 * comes from dequantising each weight row once per chunk instead of once per
 * token, and from evaluating many tokens' identical scalar recurrences side
 * by side (SIMD across tokens, never across one token's sum). */

/* How TensorOps.MatMul accumulates one activation row (aRows == 1, TO:60-90):
 * Q2_K/Q4_K/Q5_K fused kernels sum a[i] * deq[i] sequentially (TO:293-329,
 * 364-431); Q3_K sums ((a[i] * d) * sc) * value sequentially (TO:331-362);
 * Q4_0/Q8_0 (fused), Q6_K (dequantise, then DotProduct) and every other type
 * (TO:92-111) add a[i] * deq[i] into 8 lanes, then the horizontal sum and the
 * scalar tail (TO:118-287, 510-531).  The per-element dequantised values equal
 * DequantizeRow's bit for bit (same expressions). */
enum { ACC_SEQ = 0, ACC_LANE8 = 1, ACC_Q3K = 2 };
static int acc_mode(uint32_t t) {
    if (t == ORC_Q2_K || t == ORC_Q4_K || t == ORC_Q5_K) return ACC_SEQ;
    if (t == ORC_Q3_K) return ACC_Q3K;
    return ACC_LANE8;
}

#define PF_TB 64   /* tokens per inner block */
#define PF_RB 8    /* weight rows per inner block */

/* out[t * ldo + c] for the T activation rows at[i * T + t] (transposed), rows
 * c of the dequantised block deq[j * K + i]. */
/* Vectorised across tokens only: each (row, token) sum keeps its own order,
 * and without -ffast-math the compiler may not reassociate it. */
__attribute__((target_clones("avx2", "default"), optimize("tree-vectorize")))
static void pf_rows_seq(const float* at, int T, int K, const float* deq, int nr, float* out, int ldo, int c0) {
    for (int t0 = 0; t0 < T; t0 += PF_TB) {
        int tb = T - t0 < PF_TB ? T - t0 : PF_TB;
        float acc[PF_RB][PF_TB];
        memset(acc, 0, sizeof acc);
        if (g_order) {   /* other orders: a partial per ORD_GROUP-element group, groups added in order */
            const int gs = ORD_GROUP[g_order];
            float gp[PF_RB][PF_TB];
            for (int g0 = 0; g0 < K; g0 += gs) {
                memset(gp, 0, sizeof gp);
                for (int i = g0; i < g0 + gs && i < K; i++) {
                    const float* ai = at + (size_t)i * T + t0;
                    for (int j = 0; j < nr; j++) {
                        const float w = deq[(size_t)j * K + i];
                        for (int t = 0; t < tb; t++) gp[j][t] = gp[j][t] + ai[t] * w;
                    }
                }
                for (int j = 0; j < nr; j++)
                    for (int t = 0; t < tb; t++) acc[j][t] = acc[j][t] + gp[j][t];
            }
        } else {
            for (int i = 0; i < K; i++) {
                const float* ai = at + (size_t)i * T + t0;
                for (int j = 0; j < nr; j++) {
                    const float w = deq[(size_t)j * K + i];
                    for (int t = 0; t < tb; t++) acc[j][t] = acc[j][t] + ai[t] * w;
                }
            }
        }
        for (int j = 0; j < nr; j++)
            for (int t = 0; t < tb; t++) out[(size_t)(t0 + t) * ldo + c0 + j] = acc[j][t];
    }
}

__attribute__((target_clones("avx2", "default"), optimize("tree-vectorize")))
static void pf_rows_lane8(const float* at, int T, int K, const float* deq, int nr, float* out, int ldo, int c0) {
    const int L = ORD_LANES[g_order];   /* lanes: the reference's 8, or another order's */
    const int KL = (K / L) * L;
    for (int t0 = 0; t0 < T; t0 += PF_TB) {
        int tb = T - t0 < PF_TB ? T - t0 : PF_TB;
        float acc[PF_RB][VEC_ALT][PF_TB];
        memset(acc, 0, sizeof acc);
        for (int k = 0; k < KL; k += L)
            for (int l = 0; l < L; l++) {
                const float* ai = at + (size_t)(k + l) * T + t0;
                for (int j = 0; j < nr; j++) {
                    const float w = deq[(size_t)j * K + k + l];
                    for (int t = 0; t < tb; t++) acc[j][l][t] = acc[j][l][t] + ai[t] * w;
                }
            }
        for (int j = 0; j < nr; j++)
            for (int t = 0; t < tb; t++) {
                float v[VEC_ALT];
                for (int l = 0; l < L; l++) v[l] = acc[j][l][t];
                float dot = hsum_lanes(v, L);
                for (int i = KL; i < K; i++) dot += at[(size_t)i * T + t0 + t] * deq[(size_t)j * K + i];
                out[(size_t)(t0 + t) * ldo + c0 + j] = dot;
            }
    }
}

/* Q3_K: per element the block scale d, the 6-bit group scale and the signed
 * 3-bit value, applied as ((a * d) * sc) * value (TO:331-362). */
static void pf_rows_q3k(const float* at, int T, int K, const uint8_t* wrow, float* out, int ldo, int c) {
    const int qk = 256, bsz = 110;
    for (int t = 0; t < T; t++) {
        float dot = 0.0f;
        for (int blk = 0; blk < K / qk; blk++) {
            const uint8_t* p = wrow + blk * bsz;
            float d = h2f_at(p);
            for (int i = 0; i < qk; i++) {
                int sc = orc_extract6(p, 4, (i / 16) * 6);
                int q = (p[48 + i / 4] >> ((i % 4) * 2)) & 0x3;
                int mm = (p[16 + i / 8] >> (i % 8)) & 0x1;
                dot += at[(size_t)(blk * qk + i) * T + t] * d * (float)sc * (float)(q - (mm << 2));
            }
        }
        out[(size_t)t * ldo + c] = dot;
    }
}

/* Row r of a Q4_K / Q5_K tensor as DequantizeRow gives it (DK:76-140): the
 * same per-element expression d * sc * (q - c) - dmin * m with the two
 * 6-bit fields extracted once per sub-block instead of once per element;
 * every other type goes through dequantize_row itself. */
static int pf_deq_row(const uint8_t* src, float* dst, uint32_t type, int row, int K) {
    if (type != ORC_Q4_K && type != ORC_Q5_K) return dequantize_row(src, dst, type, row, K);
    const int q5 = type == ORC_Q5_K, bsz = q5 ? 176 : 144;
    const uint8_t* base = src + (int64_t)row * (K / 256) * bsz;
    for (int b = 0; b < K / 256; b++) {
        const uint8_t* p = base + b * bsz;
        const float d = h2f_at(p), dmin = h2f_at(p + 2);
        for (int g = 0; g < 8; g++) {
            const int sc = orc_extract6(p, 4, g * 12), mi = orc_extract6(p, 4, g * 12 + 6);
            for (int i = 32 * g; i < 32 * g + 32; i++) {
                float v;
                if (q5) {
                    int qLow = (p[48 + i / 2] >> ((i % 2) * 4)) & 0xF, qHigh = (p[16 + i / 8] >> (i % 8)) & 0x1;
                    v = d * (float)sc * (float)(qLow + (qHigh << 4) - 16) - dmin * (float)mi;
                } else {
                    int q = (p[16 + i / 2] >> ((i % 2) * 4)) & 0xF;
                    v = d * (float)sc * (float)(q - 8) - dmin * (float)mi;
                }
                dst[b * 256 + i] = v;
            }
        }
    }
    return 0;
}

/* out[t][0..N) = MatMulFromTensor(a[t], w) for t < T (IE:604-617), each row
 * as its own single-row call would compute it. */
static int pf_matmul(const float* a, int T, const gg_tensor* w, float* out, int N) {
    const int K = (int)w->dims[0];
    const uint32_t type = w->type;
    if (type == ORC_BF16 || orc_byte_count(type, (uint64_t)K) < 0) return -1;
    float* at = (float*)malloc(sizeof(float) * (size_t)K * (size_t)T);
    if (!at) return -1;
    for (int t = 0; t < T; t++)
        for (int i = 0; i < K; i++) at[(size_t)i * T + t] = a[(size_t)t * K + i];
    const int mode = type == ORC_F32 ? ACC_LANE8 : acc_mode(type);
    const int64_t rb = orc_byte_count(type, (uint64_t)K);
    int fail = 0;
#pragma omp parallel num_threads(g_threads) reduction(| : fail)
    {
        float* deq = (float*)malloc(sizeof(float) * (size_t)K * PF_RB);   /* one per thread */
#pragma omp for schedule(dynamic, 4)
        for (int c0 = 0; c0 < N; c0 += PF_RB) {
            const int nr = N - c0 < PF_RB ? N - c0 : PF_RB;
            if (mode == ACC_Q3K) {
                for (int j = 0; j < nr; j++) pf_rows_q3k(at, T, K, w->data + (int64_t)(c0 + j) * rb, out, N, c0 + j);
                continue;
            }
            int bad = !deq;
            for (int j = 0; j < nr && !bad; j++)
                if (pf_deq_row(w->data, deq + (size_t)j * K, type, c0 + j, K) != 0) bad = 1;
            if (!bad) {
                if (mode == ACC_SEQ) pf_rows_seq(at, T, K, deq, nr, out, N, c0);
                else pf_rows_lane8(at, T, K, deq, nr, out, N, c0);
            }
            fail |= bad;
        }
        free(deq);
    }
    free(at);
    return fail ? -1 : 0;
}

int orc_matmul_rows(const float* a, int rows, const uint8_t* b, uint32_t type, int a_cols, int b_cols, float* out) {
    gg_tensor w;
    memset(&w, 0, sizeof w);
    w.type = type;
    w.dims[0] = (uint64_t)a_cols;
    w.dims[1] = (uint64_t)b_cols;
    w.data = b;
    return pf_matmul(a, rows, &w, out, b_cols);
}

int orc_prefill(orc_model* m, const int* tokens, int n, int pos0, float* logits) {
    orc_config* c = &m->cfg;
    if (n <= 0) return 0;
    if (pos0 < 0 || pos0 + n > m->cache_ctx) return -2;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= m->embd->dims[1]) return -3;
    const int d = c->hidden, hd = c->head_dim, H = c->heads, Hkv = c->kv_heads;
    const int qdim = H * hd, kvdim = Hkv * hd, F = c->ffn;
    const int half = (c->rope_dim > 0 ? c->rope_dim : hd) / 2;
    const int CH = 512;
    const int cap = n < CH ? n : CH;
    float* X = (float*)malloc(sizeof(float) * (size_t)cap * d);    /* hidden states */
    float* Nn = (float*)malloc(sizeof(float) * (size_t)cap * d);   /* normed */
    float* Q = (float*)malloc(sizeof(float) * (size_t)cap * qdim);
    float* Kb = (float*)malloc(sizeof(float) * (size_t)cap * kvdim);
    float* Vb = (float*)malloc(sizeof(float) * (size_t)cap * kvdim);
    float* A = (float*)malloc(sizeof(float) * (size_t)cap * qdim);  /* attention output */
    float* O = (float*)malloc(sizeof(float) * (size_t)cap * d);
    float* G = (float*)malloc(sizeof(float) * (size_t)cap * F);
    float* U = (float*)malloc(sizeof(float) * (size_t)cap * F);
    int rc = (X && Nn && Q && Kb && Vb && A && O && G && U) ? 0 : -4;
    const int64_t rowBytes = orc_byte_count(m->embd->type, (uint64_t)m->embd->dims[0]);
    for (int c0 = 0; c0 < n && !rc; c0 += cap) {
        const int T = n - c0 < cap ? n - c0 : cap;
        for (int t = 0; t < T; t++)   /* GetEmbedding, IE:148-156 */
            orc_dequantize(m->embd->data + (int64_t)tokens[c0 + t] * rowBytes, X + (size_t)t * d, m->embd->type, 1,
                           (int)m->embd->dims[0]);
        for (int l = 0; l < c->layers && !rc; l++) {
            for (int t = 0; t < T; t++) orc_rms_norm(X + (size_t)t * d, m->attn_norm_f[l], Nn + (size_t)t * d, d, c->eps);
            if (m->wqkv) {   /* fused (IE:321-332): one product, then each token's q, k, v copied out */
                const int fc = qdim + 2 * kvdim;
                float* F3 = (float*)malloc(sizeof(float) * (size_t)T * fc);
                if (!F3) { rc = -4; break; }
                rc |= pf_matmul(Nn, T, m->wqkv[l], F3, fc);
                for (int t = 0; t < T && !rc; t++) {
                    memcpy(Q + (size_t)t * qdim, F3 + (size_t)t * fc, sizeof(float) * (size_t)qdim);
                    memcpy(Kb + (size_t)t * kvdim, F3 + (size_t)t * fc + qdim, sizeof(float) * (size_t)kvdim);
                    memcpy(Vb + (size_t)t * kvdim, F3 + (size_t)t * fc + qdim + kvdim, sizeof(float) * (size_t)kvdim);
                }
                free(F3);
            } else {
                rc |= pf_matmul(Nn, T, m->wq[l], Q, qdim);
                rc |= pf_matmul(Nn, T, m->wk[l], Kb, kvdim);
                rc |= pf_matmul(Nn, T, m->wv[l], Vb, kvdim);
            }
            if (rc) break;
            for (int t = 0; t < T; t++) {   /* Q/K norms, RoPE and the KV write of each token (IE:354-381) */
                const int pos = pos0 + c0 + t;
                float* qt = Q + (size_t)t * qdim;
                float* kt = Kb + (size_t)t * kvdim;
                const float* vt = Vb + (size_t)t * kvdim;
                if (m->q_norm_f && m->q_norm_f[l])
                    for (int h = 0; h < H; h++) orc_rms_norm(qt + h * hd, m->q_norm_f[l], qt + h * hd, hd, c->eps);
                if (m->k_norm_f && m->k_norm_f[l])
                    for (int h = 0; h < Hkv; h++) orc_rms_norm(kt + h * hd, m->k_norm_f[l], kt + h * hd, hd, c->eps);
                for (int h = 0; h < H; h++) orc_rope_table(qt + h * hd, qt + h * hd, hd, pos, m->rope_freqs, half, 1);
                size_t slot = ((size_t)l * (size_t)m->cache_ctx + (size_t)pos) * (size_t)kvdim;
                for (int h = 0; h < Hkv; h++) {
                    float* kh = kt + h * hd;
                    orc_rope_table(kh, kh, hd, pos, m->rope_freqs, half, 1);
                    for (int e = 0; e < hd; e++) {
                        m->kcache[slot + (size_t)h * hd + e] = kv_store(m, kh[e]);
                        m->vcache[slot + (size_t)h * hd + e] = kv_store(m, vt[h * hd + e]);
                    }
                }
            }
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 1)
            for (int th = 0; th < T * H; th++) {
                const int t = th / H, h = th % H;
                attend_head(m, l, pos0 + c0 + t, h, Q + (size_t)t * qdim + h * hd, A + (size_t)t * qdim + h * hd);
            }
            rc |= pf_matmul(A, T, m->wo[l], O, d);
            if (rc) break;
            for (int t = 0; t < T; t++) {
                orc_add_inplace(X + (size_t)t * d, O + (size_t)t * d, d);
                orc_rms_norm(X + (size_t)t * d, m->ffn_norm_f[l], Nn + (size_t)t * d, d, c->eps);
            }
            rc |= pf_matmul(Nn, T, m->wg[l], G, F);
            rc |= pf_matmul(Nn, T, m->wu[l], U, F);
            if (rc) break;
            for (int t = 0; t < T; t++) {   /* FfnForward SwiGLU (IE:457-476) */
                orc_silu_inplace(G + (size_t)t * F, F);
                orc_mul(G + (size_t)t * F, U + (size_t)t * F, G + (size_t)t * F, F);
            }
            rc |= pf_matmul(G, T, m->wd[l], O, d);
            if (rc) break;
            for (int t = 0; t < T; t++) orc_add_inplace(X + (size_t)t * d, O + (size_t)t * d, d);
        }
        if (!rc && c0 + T == n) {   /* the last token: final norm and logits (IE:575-602) */
            memcpy(m->hidden, X + (size_t)(T - 1) * d, sizeof(float) * (size_t)d);
            memcpy(m->normtmp, m->hidden, sizeof(float) * (size_t)d);
            orc_rms_norm(m->normtmp, m->out_norm_f, m->hidden, d, c->eps);
            rc |= pf_matmul(m->hidden, 1, m->out, m->logits, c->vocab);
        }
    }
    free(X); free(Nn); free(Q); free(Kb); free(Vb); free(A); free(O); free(G); free(U);
    if (rc) return rc;
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)c->vocab);
    return 0;
}
