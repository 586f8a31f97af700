// Device-side helpers for the gfx950 kernels: vector types, MFMA wrappers,
// f16/bf16 bit helpers and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace nnq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16x16x32 f16 MFMA: lane l supplies A[row l%16][8 k-values of group l/16] and
// B[8 k-values of group l/16][col l%16]; lane l receives D[4*(l/16)+i][l%16], i=0..3.
__device__ __forceinline__ floatx4 mfma16x16x32_f16(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ floatx4 mfma16x16x32_bf16(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
// round-to-nearest-even f32 -> bf16 bits (NaN kept quiet); a select, not a branch
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t r = (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
    return (x & 0x7FFFFFFFu) > 0x7F800000u ? ((x >> 16) | 0x40u) : r;
}

// Split x (already scaled into f16 range) into hi + lo f16 parts: x ~= hi + lo with
// |x - hi - lo| <= 2^-25 for |x| < 2^15 (lo may be an f16 subnormal).
__device__ __forceinline__ void split_f16(float x, uint32_t &hi, uint32_t &lo) {
    _Float16 h = (_Float16)x;
    float r = x - (float)h;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)r);
}

// Power-of-two prescale: s = 2^e with amax * s in [2^14, 2^15) (s = 1 for amax = 0)
// and back = 1 / s exactly, both normal f32; a non-finite amax gives NaN for both, so
// NaN / inf activations propagate to the outputs.
__device__ __forceinline__ void f16_prescale(float amax, float &s, float &back) {
    const int eb = (int)((__float_as_uint(amax) >> 23) & 0xFF);  // biased exponent (0 for subnormal)
    int se = 141 - (eb > 1 ? eb : 1);                             // 14 - (eb - 127)
    se = se > 126 ? 126 : (se < -126 ? -126 : se);
    s = __uint_as_float((uint32_t)(127 + se) << 23);
    back = __uint_as_float((uint32_t)(127 - se) << 23);
    if (amax == 0.0f) s = back = 1.0f;
    if (!(amax <= 3.0e38f)) s = back = __uint_as_float(0x7FC00000u);
}

// DPP quad permutations: the value of lane (l ^ 1) / (l ^ 2) within each group of 4.
// All lanes of the wave must be active.
__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Weight loads: every weight byte is read once per call, so they are issued as
// non-temporal (streaming) loads that do not displace the activations in the caches.
__device__ __forceinline__ u32x4 ldg128(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ u32x3 ldg96(const uint8_t *p) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
    return u32x3{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), __builtin_nontemporal_load(q + 2)};
}

// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// DPP row_half_mirror: the value of lane 7 - (l % 8) within each group of 8.
__device__ __forceinline__ float dpp_half_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
}

}  // namespace nnq
