// xrec.h -- activation records: one per 32-element unit of a GEMV input vector.
//
// The producer of a vector (embedding, residual-add epilogue, SwiGLU epilogue,
// attention combine) writes, next to the fp32 values, one record per 32
// consecutive elements v[32u .. 32u+31]:
//   pl[4p + j]  nibble plane p (weight 16^p) of elements 8j .. 8j+7:
//               nibble k holds digit p of X[8j+k] as a signed int4,
//               where X = round(v / s) in [-30000, 30000] = sum_p 16^p t_p,
//               t_p in [-8, 7]
//   s           max|v| / 30000  (v ~= s * X)
//   sum         sum(v)
//   ssq         sum(h^2) of the unnormalised values (RmsNorm of the consumer)
// When the consumer applies RmsNorm with weights w, v = w * h and the consumer
// multiplies s and sum by 1/rms = 1/sqrt(sum(ssq)/n + eps) (VectorMath.RmsNorm,
// VM:308-340, computes (w*h)*inv; quantising w*h and scaling by inv afterwards
// differs only by the 16-bit quantisation, |err| <= s/2 per element).
//
// A Q4_K GEMV consumes the planes with v_dot8_i32_i4: the weight nibble q
// XOR 8 is q-8 as a signed int4, so sum_i (q_i - 8) X_i is four dot8 per
// 8 elements, exact in int32.
#pragma once

#include "common.h"

namespace llmdot {

struct XRec {
    uint32_t pl[16];
    float s, sum, ssq, pad;
};
static_assert(sizeof(XRec) == 80, "XRec layout");

constexpr float XREC_QMAX = 30000.0f;

// Builds the record of one unit from a 32-lane half-wavefront: lane e (0..31 of
// the half) holds element e's value v (already multiplied by the consumer's
// norm weight when it has one) and h^2 for the ssq.  Both halves of a
// wavefront may build different units at once.  All 64 lanes must call it.
__device__ __forceinline__ void build_xrec(float v, float hsq, XRec* dst, bool active) {
    float amax = fabsf(v), sum = v, ssq = hsq;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        sum += __shfl_xor(sum, o, 64);
        ssq += __shfl_xor(ssq, o, 64);
    }
    const float s = amax > 0.f ? amax / XREC_QMAX : 0.f;
    int X = amax > 0.f ? __float2int_rn(v * (XREC_QMAX / amax)) : 0;
    X = X > 30000 ? 30000 : (X < -30000 ? -30000 : X);
    // Offset-binary digits: Y = X + 0x8888 has nibbles t_p + 8 (no carries).
    const uint32_t Y = (uint32_t)(X + 0x8888);
    const int e = threadIdx.x & 31, k = e & 7;
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        uint32_t nib = (((Y >> (4 * p)) & 15u) ^ 8u) << (4 * k);
        nib |= __shfl_xor(nib, 1, 64);
        nib |= __shfl_xor(nib, 2, 64);
        nib |= __shfl_xor(nib, 4, 64);
        w[p] = nib;
    }
    if (active && k == 0) {
        const int j = e >> 3;
#pragma unroll
        for (int p = 0; p < 4; p++) dst->pl[4 * p + j] = w[p];
    }
    if (active && e == 0) {
        dst->s = s;
        dst->sum = sum;
        dst->ssq = ssq;
        dst->pad = 0.f;
    }
}

}  // namespace llmdot
