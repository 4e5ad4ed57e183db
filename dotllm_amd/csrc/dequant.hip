// dequant.hip -- bit-exact dequantisation of the reference's block formats.
//
// Every element is produced with the same separately rounded fp32 operations,
// in the same order, as src/Llmdot.Core/Tensors/Dequantize/{DequantizeK,
// DequantizeBlock}.cs (no FMA contraction: __fmul_rn/__fsub_rn/__fadd_rn).
#include "common.h"
#include "kernels.h"

// Reference rounding everywhere in this file: no FMA contraction.
#pragma clang fp contract(off)

namespace llmdot {

__device__ __forceinline__ float h2f_at(const uint8_t* p) { return half_bits_to_float(p[0] | (p[1] << 8)); }

// DequantizeK.Extract6Bit (DK:189-199).
__device__ __forceinline__ int extract6(const uint8_t* src, int bit) {
    int byteIdx = bit >> 3, sh = bit & 7;
    if (sh <= 2) return (src[byteIdx] >> sh) & 0x3F;
    return ((src[byteIdx] >> sh) | (src[byteIdx + 1] << (8 - sh))) & 0x3F;
}

// Element i (0-based within the row) of one row of `type` blocks.
__device__ float deq_elem(uint32_t type, const uint8_t* row, int i) {
    switch (type) {
    case GGML_F32: return reinterpret_cast<const float*>(row)[i];
    case GGML_F16: return h2f_at(row + 2 * i);
    case GGML_BF16: return __uint_as_float(((uint32_t)row[2 * i + 1] << 24) | ((uint32_t)row[2 * i] << 16));
    case GGML_Q4_0: {  // DB:7-34
        const uint8_t* b = row + (i >> 5) * 18;
        int j = i & 31;
        float d = h2f_at(b);
        int qs = b[2 + (j & 15)];
        int q = j < 16 ? (qs & 0x0F) : ((qs >> 4) & 0x0F);
        return ((float)(q - 8) * d);
    }
    case GGML_Q4_1: {  // TO:586-603: d * q + m, low nibbles -> j, high -> j + 16
        const uint8_t* b = row + (i >> 5) * 20;
        int j = i & 31;
        float d = h2f_at(b), m = h2f_at(b + 2);
        int qs = b[4 + (j & 15)];
        int q = j < 16 ? (qs & 0x0F) : ((qs >> 4) & 0x0F);
        return ((d * (float)q) + m);
    }
    case GGML_Q5_0: {  // TO:604-622: (q | high bit from qh) - 16, times d
        const uint8_t* b = row + (i >> 5) * 22;
        int j = i & 31, jj = j & 15;
        float d = h2f_at(b);
        uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        int qs = b[6 + jj];
        int x = j < 16 ? (((qs & 0x0F) | (int)(((qh >> jj) << 4) & 0x10u)) - 16)
                       : ((((qs >> 4) & 0x0F) | (int)((qh >> (jj + 12)) & 0x10u)) - 16);
        return ((float)x * d);
    }
    case GGML_Q5_1: {  // TO:623-641: d * (q | high bit from qh) + m
        const uint8_t* b = row + (i >> 5) * 24;
        int j = i & 31, jj = j & 15;
        float d = h2f_at(b), m = h2f_at(b + 2);
        uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
        int qs = b[8 + jj];
        int x = j < 16 ? ((qs & 0x0F) | (int)(((qh >> jj) << 4) & 0x10u))
                       : (((qs >> 4) & 0x0F) | (int)((qh >> (jj + 12)) & 0x10u));
        return ((d * (float)x) + m);
    }
    case GGML_Q8_0: {  // DB:36-59
        const uint8_t* b = row + (i >> 5) * 34;
        return ((float)(int8_t)b[2 + (i & 31)] * h2f_at(b));
    }
    case GGML_Q2_K: {  // DK:8-41 (the reference's layout: scale/min byte pairs from byte 4, 2-bit q from byte 20)
        const uint8_t* b = row + (i >> 8) * 84;
        int j = i & 255, g = j >> 6, sub = (j & 63) >> 4, scIdx = g * 4 + sub;
        float d = h2f_at(b), dmin = h2f_at(b + 2);
        int sc = b[4 + scIdx * 2] & 0x0F, mi = b[4 + scIdx * 2 + 1] & 0x0F;
        int q = (b[20 + (j >> 2)] >> ((j & 3) * 2)) & 0x3;
        return (((d * (float)sc) * ((float)q - 0.5f)) - (dmin * (float)mi));
    }
    case GGML_Q3_K: {  // DK:43-74: 6-bit group scales from byte 4, high-bit mask from 16, 2-bit q from 48
        // (the q field runs to byte 111 of a 110-byte block: the last 8 elements
        // read the next block's first two bytes, as the reference does; past the
        // tensor's end the device buffer's zero padding)
        const uint8_t* b = row + (i >> 8) * 110;
        int j = i & 255, g = j >> 4;
        float d = h2f_at(b);
        int sc = extract6(b + 4, g * 6);
        int q = (b[48 + (j >> 2)] >> ((j & 3) * 2)) & 0x3;
        int m = (b[16 + (j >> 3)] >> (j & 7)) & 0x1;
        int value = q - (m << 2);
        return ((d * (float)sc) * (float)value);
    }
    case GGML_Q4_K: {  // DK:76-106
        const uint8_t* b = row + (i >> 8) * 144;
        int j = i & 255, g = j >> 5;
        float d = h2f_at(b), dmin = h2f_at(b + 2);
        int sc = extract6(b + 4, g * 12), mi = extract6(b + 4, g * 12 + 6);
        int q = (b[16 + (j >> 1)] >> ((j & 1) * 4)) & 0xF;
        return (((d * (float)sc) * (float)(q - 8)) - (dmin * (float)mi));
    }
    case GGML_Q5_K: {  // DK:108-140
        const uint8_t* b = row + (i >> 8) * 176;
        int j = i & 255, g = j >> 5;
        float d = h2f_at(b), dmin = h2f_at(b + 2);
        int sc = extract6(b + 4, g * 12), mi = extract6(b + 4, g * 12 + 6);
        int ql = (b[48 + (j >> 1)] >> ((j & 1) * 4)) & 0xF;
        int qh = (b[16 + (j >> 3)] >> (j & 7)) & 0x1;
        int q5 = ql + (qh << 4);
        return (((d * (float)sc) * (float)(q5 - 16)) - (dmin * (float)mi));
    }
    case GGML_Q6_K: {  // DK:142-187
        const uint8_t* b = row + (i >> 8) * 210;
        int j = i & 255, n = j & 128, r = j & 127, t = r >> 5, l = r & 31;
        float d = h2f_at(b + 208);
        const uint8_t* ql = b + n / 2;
        const uint8_t* qh = b + 128 + n / 4;
        int lo = (t & 1) ? ql[l + 32] : ql[l];
        int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
        int q = (nib | (((qh[l] >> (2 * t)) & 3) << 4)) - 32;
        int sc = (int8_t)b[192 + n / 16 + (l >> 4) + 2 * t];
        return ((d * (float)sc) * (float)q);
    }
    default: return 0.0f;
    }
}

__global__ void dequant_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst, uint32_t type,
                               int num_rows, int row_elems, int64_t row_bytes) {
    int64_t n = (int64_t)num_rows * row_elems;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = e / row_elems;
        int i = (int)(e - r * row_elems);
        dst[e] = deq_elem(type, src + r * row_bytes, i);
    }
}

// One thread per element; with w set, also the packed input of the first
// RmsNorm consumer (as pack_norm_kernel).
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ table, uint32_t type, int hidden,
                                                    int64_t row_bytes, const int32_t* __restrict__ token,
                                                    float* __restrict__ out, const float* __restrict__ w,
                                                    float* __restrict__ packed, float* __restrict__ ssq) {
    const int tok = *token;
    const uint8_t* row = table + (int64_t)tok * row_bytes;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const float h = i < hidden ? deq_elem(type, row, i) : 0.f;
    if (i < hidden) out[i] = h;
    if (w) {   // uniform
        if (i < hidden) packed[i] = w[i] * h;
        float q = h * h;
        q = sum4(q);
        if ((i & 3) == 0 && i < hidden) ssq[i >> 2] = q;
    }
}

// One thread per element; lanes 4k..4k+3 reduce their squares for ssq[k].
__global__ __launch_bounds__(256) void pack_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                        float* __restrict__ packed, float* __restrict__ ssq) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const float h = i < n ? x[i] : 0.f;
    if (i < n) packed[i] = w[i] * h;   // RmsNorm's vector lanes compute (w * x) * inv
    float q = h * h;
    q = sum4(q);
    if ((i & 3) == 0 && i < n) ssq[i >> 2] = q;
}

hipError_t launch_pack_norm(const float* x, const float* w, int n, float* packed, float* ssq, hipStream_t s) {
    if (n <= 0 || n % 8) return hipErrorInvalidValue;
    pack_norm_kernel<<<(n + 255) / 256, 256, 0, s>>>(x, w, n, packed, ssq);
    return hipGetLastError();
}

// Embedding rows of a token chunk: grid (hidden / 256, T).
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t* __restrict__ table, uint32_t type, int hidden,
                                                         int64_t row_bytes, const int32_t* __restrict__ tokens,
                                                         float* __restrict__ out) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i < hidden) out[(int64_t)t * hidden + i] = deq_elem(type, table + (int64_t)tokens[t] * row_bytes, i);
}

hipError_t launch_embed_rows(const uint8_t* table, uint32_t type, int hidden, const int32_t* tokens, int T, float* out,
                             hipStream_t s) {
    if (T <= 0 || hidden <= 0) return hipErrorInvalidValue;
    embed_rows_kernel<<<dim3((hidden + 255) / 256, T), 256, 0, s>>>(table, type, hidden, byte_count(type, hidden), tokens,
                                                                      out);
    return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* src, float* dst, uint32_t type, int num_rows, int row_elems,
                          hipStream_t s) {
    int64_t rb = byte_count(type, row_elems);
    int64_t n = (int64_t)num_rows * row_elems;
    if (n <= 0) return hipSuccess;
    int grid = (int)((n + 255) / 256);
    if (grid > 65536) grid = 65536;
    dequant_kernel<<<grid, 256, 0, s>>>(src, dst, type, num_rows, row_elems, rb);
    return hipGetLastError();
}

hipError_t launch_embed(const uint8_t* table, uint32_t type, int hidden, const int32_t* token_dev,
                        float* out, const float* w, float* packed, float* ssq, hipStream_t s) {
    if (w && (hidden % 8 || !packed || !ssq)) return hipErrorInvalidValue;
    int64_t rb = byte_count(type, hidden);
    int grid = (hidden + 255) / 256;
    embed_kernel<<<grid, 256, 0, s>>>(table, type, hidden, rb, token_dev, out, w, packed, ssq);
    return hipGetLastError();
}

}  // namespace llmdot
