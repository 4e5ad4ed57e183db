// quantize.cpp -- host quantizers for the block layouts the reference decodes,
// plus a seeded, thread-count-independent synthetic weight generator.
//
// The reference has no quantizer; these write exactly the layouts its
// dequantizers read:
//   Q8_0  DequantizeBlock.cs:36-59        (ggml layout)
//   Q4_0  DequantizeBlock.cs:7-34         (ggml layout)
//   Q4_K  DequantizeK.cs:76-106, 189-199  (reference layout: 6-bit LSB-first
//                                          scale/min stream, sequential nibbles, q-8)
//   Q5_K  DequantizeK.cs:108-140          (reference layout: q5-16)
//   Q6_K  DequantizeK.cs:142-187          (ggml layout)
// (all paths relative to src/Llmdot.Core/Tensors/Dequantize/).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/llmdot_hip.h"

namespace {

enum : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, BF16 = 25 };

inline uint32_t fbits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
inline float bitsf(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }

// binary32 -> binary16, round to nearest even.
uint16_t f2h(float f) {
    uint32_t x = fbits(f), sign = (x >> 16) & 0x8000u, a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a >= 0x38800000u) {
        uint32_t h = (((a >> 23) - 112) << 10) | ((a & 0x7FFFFFu) >> 13), rem = a & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return (uint16_t)sign;
    uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u, s = 126 - e;
    uint32_t k = m >> s, rem = m & ((1u << s) - 1u), hw = 1u << (s - 1);
    if (rem > hw || (rem == hw && (k & 1u))) k++;
    return (uint16_t)(sign | k);
}
// binary16 -> binary32 (exact).
float h2f(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 0) return m == 0 ? bitsf(s) : (s ? -1.0f : 1.0f) * (float)m * 5.9604644775390625e-8f;
    if (e == 31) return bitsf(s | 0x7F800000u | (m << 13));
    return bitsf(s | ((e + 112) << 23) | (m << 13));
}
inline void put_h(uint8_t* p, float v) { uint16_t h = f2h(v); p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }
inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
inline int rnd(float v) { return (int)lroundf(v); }

void quant_q8_0(const float* x, uint8_t* out, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, out += 34) {
        float amax = 0;
        for (int i = 0; i < 32; i++) amax = std::max(amax, fabsf(x[i]));
        uint16_t dh = f2h(amax / 127.0f);
        float d = h2f(dh);
        out[0] = (uint8_t)dh; out[1] = (uint8_t)(dh >> 8);
        for (int i = 0; i < 32; i++)
            out[2 + i] = (uint8_t)(int8_t)(d != 0.0f ? clampi(rnd(x[i] / d), -127, 127) : 0);
    }
}

void quant_q4_0(const float* x, uint8_t* out, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++, x += 32, out += 18) {
        float amax = 0, mx = 0;
        for (int i = 0; i < 32; i++)
            if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); mx = x[i]; }
        uint16_t dh = f2h(mx / -8.0f);
        float d = h2f(dh);
        out[0] = (uint8_t)dh; out[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 16; j++) {
            int q0 = d != 0.0f ? clampi(rnd(x[j] / d) + 8, 0, 15) : 8;
            int q1 = d != 0.0f ? clampi(rnd(x[j + 16] / d) + 8, 0, 15) : 8;
            out[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// Writes a 6-bit value at bit offset `bit` of the LSB-first stream starting at p
// (the inverse of DequantizeK.Extract6Bit).
void put6(uint8_t* p, int bit, int v) {
    for (int k = 0; k < 6; k++) {
        int b = bit + k;
        if ((v >> k) & 1) p[b / 8] |= (uint8_t)(1u << (b % 8));
    }
}

// Shared by the reference Q4_K (nq = 16, offset 8) and Q5_K (nq = 32, offset 16)
// layouts: x = (d*sc)*(q - offset) - dmin*m with sc, m in [0, 63].
void quant_kmin(const float* x, uint8_t* blk, int nq, float* eff_D, float* eff_M, int* sc_out, int* m_out) {
    const int off = nq / 2;
    float D[8], M[8];
    for (int g = 0; g < 8; g++) {
        float mn = x[32 * g], mx = x[32 * g];
        for (int i = 1; i < 32; i++) { mn = std::min(mn, x[32 * g + i]); mx = std::max(mx, x[32 * g + i]); }
        float d = (mx - mn) / (float)(nq - 1);
        float m = -(mn + (float)off * d);
        if (m < 0.0f) { m = 0.0f; d = std::max(mx / (float)(off - 1), -mn / (float)off); }
        D[g] = std::max(d, 0.0f); M[g] = m;
    }
    float dmax = 0, mmax = 0;
    for (int g = 0; g < 8; g++) { dmax = std::max(dmax, D[g]); mmax = std::max(mmax, M[g]); }
    uint16_t dh = f2h(dmax / 63.0f), mh = f2h(mmax / 63.0f);
    float dr = h2f(dh), mr = h2f(mh);
    blk[0] = (uint8_t)dh; blk[1] = (uint8_t)(dh >> 8); blk[2] = (uint8_t)mh; blk[3] = (uint8_t)(mh >> 8);
    memset(blk + 4, 0, 12);
    for (int g = 0; g < 8; g++) {
        int sc = dr > 0.0f ? clampi(rnd(D[g] / dr), 0, 63) : 0;
        if (sc == 0 && D[g] > 0.0f && dr > 0.0f) sc = 1;
        int m = mr > 0.0f ? clampi(rnd(M[g] / mr), 0, 63) : 0;
        put6(blk + 4, 12 * g, sc);
        put6(blk + 4, 12 * g + 6, m);
        sc_out[g] = sc; m_out[g] = m;
        eff_D[g] = dr * (float)sc; eff_M[g] = mr * (float)m;
    }
}

void quant_q4_k(const float* x, uint8_t* out, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++, x += 256, out += 144) {
        float D[8], M[8]; int sc[8], m[8];
        quant_kmin(x, out, 16, D, M, sc, m);
        memset(out + 16, 0, 128);
        for (int i = 0; i < 256; i++) {
            int g = i / 32;
            int q = D[g] > 0.0f ? clampi(rnd((x[i] + M[g]) / D[g]) + 8, 0, 15) : 8;
            out[16 + i / 2] |= (uint8_t)(q << (4 * (i % 2)));
        }
    }
}

void quant_q5_k(const float* x, uint8_t* out, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++, x += 256, out += 176) {
        float D[8], M[8]; int sc[8], m[8];
        quant_kmin(x, out, 32, D, M, sc, m);
        memset(out + 16, 0, 160);
        for (int i = 0; i < 256; i++) {
            int g = i / 32;
            int q = D[g] > 0.0f ? clampi(rnd((x[i] + M[g]) / D[g]) + 16, 0, 31) : 16;
            out[48 + i / 2] |= (uint8_t)((q & 15) << (4 * (i % 2)));
            out[16 + i / 8] |= (uint8_t)(((q >> 4) & 1) << (i % 8));
        }
    }
}

void quant_q6_k(const float* x, uint8_t* out, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++, x += 256, out += 210) {
        float s[16], smax = 0;
        for (int j = 0; j < 16; j++) {
            float amax = 0;
            for (int i = 0; i < 16; i++) amax = std::max(amax, fabsf(x[16 * j + i]));
            s[j] = amax / 31.5f;
            smax = std::max(smax, s[j]);
        }
        uint16_t dh = f2h(smax / 127.0f);
        float d = h2f(dh);
        int q[256];
        for (int j = 0; j < 16; j++) {
            int sc = d > 0.0f ? clampi(rnd(s[j] / d), -128, 127) : 0;
            out[192 + j] = (uint8_t)(int8_t)sc;
            float De = d * (float)sc;
            for (int i = 0; i < 16; i++)
                q[16 * j + i] = De != 0.0f ? clampi(rnd(x[16 * j + i] / De), -32, 31) + 32 : 32;
        }
        memset(out, 0, 192);
        for (int nn = 0; nn < 256; nn += 128) {
            uint8_t* ql = out + nn / 2;
            uint8_t* qh = out + 128 + nn / 4;
            for (int l = 0; l < 32; l++) {
                int q1 = q[nn + l], q2 = q[nn + l + 32], q3 = q[nn + l + 64], q4 = q[nn + l + 96];
                ql[l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        }
        put_h(out + 208, d);
    }
}

int quantize_row(uint32_t type, const float* x, int64_t cols, uint8_t* out) {
    switch (type) {
    case F32: memcpy(out, x, (size_t)cols * 4); return 0;
    case F16:
        for (int64_t i = 0; i < cols; i++) put_h(out + 2 * i, x[i]);
        return 0;
    case BF16:
        for (int64_t i = 0; i < cols; i++) {
            uint32_t b = fbits(x[i]);
            uint32_t r = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
            out[2 * i] = (uint8_t)r; out[2 * i + 1] = (uint8_t)(r >> 8);
        }
        return 0;
    case Q8_0: quant_q8_0(x, out, cols); return 0;
    case Q4_0: quant_q4_0(x, out, cols); return 0;
    case Q4_K: quant_q4_k(x, out, cols); return 0;
    case Q5_K: quant_q5_k(x, out, cols); return 0;
    case Q6_K: quant_q6_k(x, out, cols); return 0;
    default: return LLMDOT_E_UNSUPPORTED;
    }
}

int64_t row_bytes(uint32_t type, int64_t cols) {
    switch (type) {
    case F32: return cols * 4;
    case F16: case BF16: return cols * 2;
    case Q8_0: return cols % 32 ? -1 : cols / 32 * 34;
    case Q4_0: return cols % 32 ? -1 : cols / 32 * 18;
    case Q4_K: return cols % 256 ? -1 : cols / 256 * 144;
    case Q5_K: return cols % 256 ? -1 : cols / 256 * 176;
    case Q6_K: return cols % 256 ? -1 : cols / 256 * 210;
    default: return -1;
    }
}

inline uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element i of the seeded N(0, sigma) stream: Box-Muller on pair i/2.
void gauss_fill(uint64_t seed, int64_t first, int64_t n, float sigma, float* out) {
    const double two_pi = 6.283185307179586;
    uint64_t key = splitmix(seed ^ 0xD1B54A32D192ED03ull);
    for (int64_t i = first; i < first + n;) {
        int64_t p = i >> 1;
        uint64_t r = splitmix(key ^ (uint64_t)p * 0x9E3779B97F4A7C15ull);
        uint64_t r2 = splitmix(r);
        double u1 = ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740993.0);   // (0, 1]
        double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);          // [0, 1)
        double rad = sqrt(-2.0 * log(u1));
        double z[2] = {rad * cos(two_pi * u2), rad * sin(two_pi * u2)};
        for (int k = (int)(i & 1); k < 2 && i < first + n; k++, i++) out[i - first] = (float)(z[k] * sigma);
    }
}

}  // namespace

extern "C" int32_t llmdot_hip_quantize(uint32_t type, const float* src, int64_t rows, int64_t cols, void* dst) {
    int64_t rb = row_bytes(type, cols);
    if (!src || !dst || rows < 0 || cols <= 0) return LLMDOT_E_INVALID;
    if (rb < 0) return LLMDOT_E_UNSUPPORTED;
    for (int64_t r = 0; r < rows; r++) {
        int rc = quantize_row(type, src + r * cols, cols, (uint8_t*)dst + r * rb);
        if (rc) return rc;
    }
    return LLMDOT_OK;
}

extern "C" int32_t llmdot_hip_synth_weights(uint32_t type, int64_t rows, int64_t cols, uint64_t seed,
                                            float sigma, void* dst, int32_t threads) {
    int64_t rb = row_bytes(type, cols);
    if (!dst || rows < 0 || cols <= 0) return LLMDOT_E_INVALID;
    if (rb < 0) return LLMDOT_E_UNSUPPORTED;
    int nt = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
    nt = (int)std::min<int64_t>(nt, std::max<int64_t>(1, rows));
    auto work = [&](int t) {
        std::vector<float> buf((size_t)cols);
        for (int64_t r = t; r < rows; r += nt) {
            gauss_fill(seed, r * cols, cols, sigma, buf.data());
            quantize_row(type, buf.data(), cols, (uint8_t*)dst + r * rb);
        }
    };
    if (nt == 1) { work(0); return LLMDOT_OK; }
    std::vector<std::thread> pool;
    for (int t = 0; t < nt; t++) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
    return LLMDOT_OK;
}
