// common.h -- shared definitions for the llmdot HIP backend (gfx950 / MI355X).
//
// Weight tensors stay in HBM in their native GGUF block layout, row-major by
// output row: row r of a [rows x cols] tensor is ByteCount(type, cols) bytes
// starting at r * ByteCount(type, cols) (src/Llmdot.Core/Tensors/TensorSize.cs:7-24).
// Every device allocation that holds weights is padded by WEIGHT_PAD bytes so
// that the realigning dword loads below may read up to 8 bytes past a tensor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmdot {

// GgmlType (src/Llmdot.Core/Loading/GgmlType.cs:3-28).
enum GgmlType : uint32_t {
    GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q5_0 = 6, GGML_Q5_1 = 7,
    GGML_Q8_0 = 8, GGML_Q8_1 = 9, GGML_Q2_K = 10, GGML_Q3_K = 11, GGML_Q4_K = 12,
    GGML_Q5_K = 13, GGML_Q6_K = 14, GGML_BF16 = 25
};

constexpr size_t WEIGHT_PAD = 256;

// Block geometry (elements per block, bytes per block); 0 = not supported.
__host__ __device__ inline constexpr int block_elems(uint32_t t) {
    return t == GGML_F32 || t == GGML_F16 || t == GGML_BF16 ? 1
         : t == GGML_Q4_0 || t == GGML_Q4_1 || t == GGML_Q5_0 || t == GGML_Q5_1 || t == GGML_Q8_0 ? 32
         : t == GGML_Q2_K || t == GGML_Q3_K || t == GGML_Q4_K || t == GGML_Q5_K || t == GGML_Q6_K ? 256 : 0;
}
__host__ __device__ inline constexpr int block_bytes(uint32_t t) {
    return t == GGML_F32 ? 4 : t == GGML_F16 || t == GGML_BF16 ? 2
         : t == GGML_Q4_0 ? 18 : t == GGML_Q4_1 ? 20 : t == GGML_Q5_0 ? 22 : t == GGML_Q5_1 ? 24
         : t == GGML_Q8_0 ? 34 : t == GGML_Q2_K ? 84 : t == GGML_Q3_K ? 110
         : t == GGML_Q4_K ? 144 : t == GGML_Q5_K ? 176 : t == GGML_Q6_K ? 210 : 0;
}
// TensorSize.ByteCount (TensorSize.cs:7-24); -1 when unsupported.
inline int64_t byte_count(uint32_t t, int64_t n) {
    int be = block_elems(t), bb = block_bytes(t);
    if (!be) return -1;
    return n / be * bb;
}

// ---- device helpers -------------------------------------------------------

// Bit pattern -> float for fp16 exactly as HalfHelper.HalfToFloat (HH:7-34),
// including the canonical NaN it returns for any NaN payload.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign << 31;
        } else {
            // subnormal: normalise; value = m * 2^-24
            int sh = __builtin_clz(m) - 21;        // shifts until bit 10 is set
            uint32_t nm = (m << sh) & 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(127 - 14 - sh) << 23) | (nm << 13);
        }
    } else if (e == 31) {
        bits = m == 0 ? ((sign << 31) | 0x7F800000u) : 0xFFC00000u;
    } else {
        bits = (sign << 31) | ((e - 15 + 127) << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

// 16 bytes from a 4-byte-aligned address (one global_load_dwordx4).
struct __attribute__((aligned(4))) u32x4 { uint32_t x, y, z, w; };
__device__ __forceinline__ u32x4 ld16_a4(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ uint32_t ld4_a4(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// n*4 bytes starting at a 2-byte-aligned address p, realigned with v_alignbyte:
// loads n+1 dwords from p & ~3 (may read up to 2 bytes past p + 4n).
template <int N>
__device__ __forceinline__ void ld_realign(const uint8_t* p, uint32_t* out) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t)(a & 3u);
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i + 4 <= N + 1; i += 4) {
        u32x4 v = ld16_a4(base + 4 * i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
#pragma unroll
    for (int i = ((N + 1) / 4) * 4; i < N + 1; i++) w[i] = ld4_a4(base + 4 * i);
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

// ---- lane exchanges without the LDS --------------------------------------
// __shfl_xor compiles to ds_bpermute (an LDS round trip per step); these use
// DPP (within 16-lane rows) and gfx950's row-swap permutes (across rows).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t lane_xor1(uint32_t x) { return dpp_u32<0xB1>(x); }   // quad_perm [1,0,3,2]
__device__ __forceinline__ uint32_t lane_xor2(uint32_t x) { return dpp_u32<0x4E>(x); }   // quad_perm [2,3,0,1]
// lane ^ 7 within 8 lanes (row_half_mirror) and lane ^ 15 within 16 (row_mirror):
// once every lane of a quad (of 8 lanes) holds the same value, these act as
// lane ^ 4 (lane ^ 8).
__device__ __forceinline__ uint32_t lane_mirror8(uint32_t x) { return dpp_u32<0x141>(x); }
__device__ __forceinline__ uint32_t lane_mirror16(uint32_t x) { return dpp_u32<0x140>(x); }
// lane ^ 16 / lane ^ 32: the swap leaves each lane's own value in one result
// and its partner's in the other.
__device__ __forceinline__ uint32_t lane_xor16(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t lane_xor32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
}
__device__ __forceinline__ float fx(uint32_t (*f)(uint32_t), float v) { return __uint_as_float(f(__float_as_uint(v))); }

// Sums over each 4 / 8 consecutive lanes (every lane receives its group's sum).
__device__ __forceinline__ float sum4(float v) {
    v += fx(lane_xor1, v);
    return v + fx(lane_xor2, v);
}
__device__ __forceinline__ float sum8(float v) {
    v = sum4(v);
    return v + fx(lane_mirror8, v);
}
__device__ __forceinline__ float sum16(float v) {
    v = sum8(v);
    return v + fx(lane_mirror16, v);
}
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, fx(lane_xor1, v));
    v = fmaxf(v, fx(lane_xor2, v));
    v = fmaxf(v, fx(lane_mirror8, v));
    return fmaxf(v, fx(lane_mirror16, v));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = sum16(v);
    v += fx(lane_xor16, v);
    return v + fx(lane_xor32, v);
}
__device__ __forceinline__ float wave_max(float v) {
    v = max16(v);
    v = fmaxf(v, fx(lane_xor16, v));
    return fmaxf(v, fx(lane_xor32, v));
}
__device__ __forceinline__ float xor16_add(float v) { return v + fx(lane_xor16, v); }
__device__ __forceinline__ float xor32_add(float v) { return v + fx(lane_xor32, v); }

// (value, index) argmax over the wavefront: the larger value, or equal value
// and smaller index (VectorMath.ArgMax keeps the first strict maximum; NaN
// never wins).  Every lane receives the result.
__device__ __forceinline__ void am_pick(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    am_pick(v, i, fx(lane_xor1, v), (int)lane_xor1((uint32_t)i));
    am_pick(v, i, fx(lane_xor2, v), (int)lane_xor2((uint32_t)i));
    am_pick(v, i, fx(lane_mirror8, v), (int)lane_mirror8((uint32_t)i));
    am_pick(v, i, fx(lane_mirror16, v), (int)lane_mirror16((uint32_t)i));
    am_pick(v, i, fx(lane_xor16, v), (int)lane_xor16((uint32_t)i));
    am_pick(v, i, fx(lane_xor32, v), (int)lane_xor32((uint32_t)i));
}

// NeoX rotation of element d of a head (TensorOps.ApplyRoPE, TO:679-743):
// pairs (i, i + half) with the position's cos/sin, dims >= 2*half untouched.
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, const float* cs, const float* sn) {
#pragma clang fp contract(off)
    if (d < half) return x[d] * cs[d] - x[d + half] * sn[d];
    if (d < 2 * half) return x[d - half] * sn[d - half] + x[d] * cs[d - half];
    return x[d];
}

// rope_elem with the operands already loaded: a = x[d], b = its partner
// (x[d + half] below half, x[d - half] above), c/s = cos/sin of the pair.
__device__ __forceinline__ float rope_pair(float a, float b, float c, float s, int d, int half) {
#pragma clang fp contract(off)
    if (d < half) return a * c - b * s;
    if (d < 2 * half) return b * s + a * c;
    return a;
}

// Stores one KV cache element (fp16: round to nearest even) and returns the
// value as later reads see it.
__device__ __forceinline__ float store_kv(void* cache, int64_t idx, float v, int fp16) {
    if (fp16) {
        const _Float16 h = (_Float16)v;
        reinterpret_cast<_Float16*>(cache)[idx] = h;
        return (float)h;
    }
    reinterpret_cast<float*>(cache)[idx] = v;
    return v;
}

// One lane of ExpApproxVector (src/Llmdot.Core/Tensors/Numeric/VectorMath.cs:137-166),
// bit-exact: every operation is a separately rounded fp32 op (contraction is
// switched off in the function body; the __f*_rn spellings alone do not stop it).
__device__ __forceinline__ float exp_approx(float x) {
#pragma clang fp contract(off)
    float c = x > -87.3f ? x : -87.3f;
    c = c < 88.4f ? c : 88.4f;
    int k = (int)((c * 1.4426950408889634f) + 0.5f);   // truncates
    float kf = (float)k;
    float y = ((c - (kf * 0.693145751953125f)) - (kf * 1.42860677e-6f));
    float cc = ((y * y) * 0.5f);
    float cy = (cc * y);
    float pade = ((((1.0f + y) + cc) + (cy * 0.3333333f)) + ((cy * y) * 0.2f));
    float r = (pade * __uint_as_float((uint32_t)(k + 127) << 23));
    if (x < -87.3f) r = 0.0f;
    if (x > 88.4f) r = __uint_as_float(0x7F800000u);
    return r;
}

// Vector lanes of VectorMath.SiluInPlace (VM:118-135): x / (1 + ExpApprox(-x)).
__device__ __forceinline__ float silu_ref(float x) {
#pragma clang fp contract(off)
    return (x / (1.0f + exp_approx(-x)));
}

}  // namespace llmdot
