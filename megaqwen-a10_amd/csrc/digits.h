// Exact matrix-core products of fp32 activations with int8 weights: an fp32
// vector over a power-of-two scale becomes a 55-bit fixed-point number held as
// eight 7-bit digits (the top one signed), each digit plane is multiplied by the
// int8 weights on the int8 matrix cores (v_mfma_i32_16x16x64_i8, exact int32
// sums), and the plane sums are recombined in fp64. Shared by the decode-step
// kernel (decode_async.hip) and the prompt-batched prefill (prefill.hip).
#pragma once

#include "common.h"

namespace mq {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Maximum over the wave, uniform: the 16-lane row maxima by DPP, then the four rows'
// read out (a cross-row permlane level costs about twice a DPP level).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, __float_as_uint(partner<1>(__uint_as_float(v))));
    v = max(v, __float_as_uint(partner<2>(__uint_as_float(v))));
    v = max(v, __float_as_uint(partner<4>(__uint_as_float(v))));
    v = max(v, __float_as_uint(partner<8>(__uint_as_float(v))));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t exp_field(float v) { return (__float_as_uint(v) >> 23) & 0xffu; }

// X = trunc(v * 2^(181 - emax)) for fp32 v whose biased exponent is at most emax
// (|X| < 2^55; fixed55), and as its eight digits: X = sum_d dig[d] 2^(49 - 7d), dig[0]
// in [-64, 63], the others in [0, 127] (digits55). Zeros and denormals give X = 0.
__device__ __forceinline__ int64_t fixed55(float v, uint32_t emax) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t e = (b >> 23) & 0xffu;
    const uint64_t m = (uint64_t)((b & 0x7fffffu) | 0x800000u) << 31;
    const uint32_t sh = emax - e;
    const uint64_t X = (e != 0u && sh < 56u) ? (m >> sh) : 0ull;
    return (b >> 31) ? -(int64_t)X : (int64_t)X;
}
__device__ __forceinline__ void digits55(float v, uint32_t emax, int (&dig)[8]) {
    const uint64_t X = (uint64_t)fixed55(v, emax);
    const uint32_t lo = (uint32_t)X, hi = (uint32_t)(X >> 32);
    dig[0] = ((int)(hi << 8)) >> 25;                     // bits 49..55, sign-extended
    dig[1] = (int)((hi >> 10) & 127u);
    dig[2] = (int)((hi >> 3) & 127u);
    dig[3] = (int)(__builtin_amdgcn_alignbit(hi, lo, 28) & 127u);
    dig[4] = (int)((lo >> 21) & 127u);
    dig[5] = (int)((lo >> 14) & 127u);
    dig[6] = (int)((lo >> 7) & 127u);
    dig[7] = (int)(lo & 127u);
}
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

__device__ __forceinline__ i32x4_t mfma_i8(i32x4_t a, i32x4_t b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// Row value of an MFMA output tile: lane n (< 16) holds digit sums 0-3 of row n and lane
// n + 16 sums 4-7; the exact integer sum_d S_d 2^(49 - 7d) is formed from the two 4-digit
// halves (each exact in fp64) with one rounding, then scaled by 2^(emax - 181).
__device__ __forceinline__ double tile_value(i32x4_t c, uint32_t emax) {
    const double half = (double)(((int64_t)c[0] << 21) + ((int64_t)c[1] << 14) + ((int64_t)c[2] << 7) + (int64_t)c[3]);
    const double lo = partner64<16>(half);
    return ldexp(fma(half, 268435456.0, lo), (int)emax - 181);
}

}  // namespace mq
