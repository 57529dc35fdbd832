// Device helpers shared by the gfx950 kernels: bf16 conversion, wave64
// cross-lane reductions (DPP within 16-lane rows, ds_bpermute across rows),
// the int8/bf16 16-byte dot products and the tagged 64-bit exchange words
// the persistent decode kernel synchronises with.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even (quiet NaN preserved).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ---- cross-lane exchange --------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Value held by this lane's partner at level M of a 64-lane butterfly. Every
// level pairs a lane whose bit M is clear with one whose bit M is set, inside
// the same 2M-lane group: xor for M = 32, 16, 2, 1 and the (half-)row mirrors
// for M = 8, 4 (lane i <-> 15-i, lane i <-> 7-i). The xor-32 and xor-16
// exchanges use gfx950's v_permlane32_swap / v_permlane16_swap (VALU, no LDS
// round trip): swapping a register with itself leaves the partner's value in
// one of the two results, chosen by the lane's bit M.
template <int M>
__device__ __forceinline__ float partner(float v) {
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
    }
    else if constexpr (M == 8) return dpp<0x140>(v);   // row_mirror
    else if constexpr (M == 4) return dpp<0x141>(v);   // row_half_mirror
    else if constexpr (M == 2) return dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    else return dpp<0xB1>(v);                           // quad_perm [1,0,3,2]
}

// Sum over the wave, returned uniformly (readlane of the four 16-lane row sums).
__device__ __forceinline__ float wave_sum(float v) {
    v += partner<1>(v);
    v += partner<2>(v);
    v += partner<4>(v);
    v += partner<8>(v);
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, partner<1>(v));
    v = fmaxf(v, partner<2>(v));
    v = fmaxf(v, partner<4>(v));
    v = fmaxf(v, partner<8>(v));
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// One transpose level: N values per lane become N/2; lanes with bit M clear
// keep the lower half of the list, lanes with bit M set the upper half, and
// each adds its partner's copy of the half it keeps.
template <int M, int N>
__device__ __forceinline__ void transpose_level(float* v, int lane) {
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int r = 0; r < N / 2; ++r) {
        float keep = hi ? v[r + N / 2] : v[r];
        float send = hi ? v[r] : v[r + N / 2];
        v[r] = keep + partner<M>(send);
    }
}

// Reduce R per-lane partial sums (R a power of two <= 64) over the wave, with
// G consecutive list entries summed together (G divides R). Afterwards every
// lane of block b = lane / (64*G/R) holds sum over lanes and over
// entries [b*G, b*G+G) of v.
template <int R, int G = 1>
__device__ __forceinline__ float transpose_reduce(float* v, int lane) {
    constexpr int T = R / G;                         // number of distinct results
    if constexpr (T >= 2) transpose_level<32, R>(v, lane);
    if constexpr (T >= 4) transpose_level<16, R / 2>(v, lane);
    if constexpr (T >= 8) transpose_level<8, R / 4>(v, lane);
    if constexpr (T >= 16) transpose_level<4, R / 8>(v, lane);
    if constexpr (T >= 32) transpose_level<2, R / 16>(v, lane);
    if constexpr (T >= 64) transpose_level<1, R / 32>(v, lane);
    float x = v[0];
#pragma unroll
    for (int g = 1; g < G; ++g) x += v[g];
    if constexpr (T < 64) x += partner<1>(x);
    if constexpr (T < 32) x += partner<2>(x);
    if constexpr (T < 16) x += partner<4>(x);
    if constexpr (T < 8) x += partner<8>(x);
    if constexpr (T < 4) x += partner<16>(x);
    if constexpr (T < 2) x += partner<32>(x);
    return x;
}

// ---- fp64 variants ---------------------------------------------------------------------
// The decode kernels accumulate in fp64 and round to fp32 / bf16 only where the
// reference stores a value: int8 x fp32 and bf16 x fp32 products are exact in
// fp64 and CDNA runs fp64 FMA at the (non-packed) fp32 rate, so every stored
// intermediate is the correctly rounded value of its defining expression.
template <int M>
__device__ __forceinline__ double partner64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const float lo = partner<M>(__uint_as_float((uint32_t)u));
    const float hi = partner<M>(__uint_as_float((uint32_t)(u >> 32)));
    return __longlong_as_double((long long)(((uint64_t)__float_as_uint(hi) << 32) | __float_as_uint(lo)));
}

__device__ __forceinline__ double wave_sum64(double v) {
    v += partner64<1>(v);
    v += partner64<2>(v);
    v += partner64<4>(v);
    v += partner64<8>(v);
    v += partner64<16>(v);
    v += partner64<32>(v);
    return v;
}

__device__ __forceinline__ double wave_max64(double v) {
    v = fmax(v, partner64<1>(v));
    v = fmax(v, partner64<2>(v));
    v = fmax(v, partner64<4>(v));
    v = fmax(v, partner64<8>(v));
    v = fmax(v, partner64<16>(v));
    v = fmax(v, partner64<32>(v));
    return v;
}

template <int M, int N>
__device__ __forceinline__ void transpose_level64(double* v, int lane) {
    const bool hi = (lane & M) != 0;
#pragma unroll
    for (int r = 0; r < N / 2; ++r) {
        double keep = hi ? v[r + N / 2] : v[r];
        double send = hi ? v[r] : v[r + N / 2];
        v[r] = keep + partner64<M>(send);
    }
}

// fp64 twin of transpose_reduce.
template <int R, int G = 1>
__device__ __forceinline__ double transpose_reduce64(double* v, int lane) {
    constexpr int T = R / G;
    if constexpr (T >= 2) transpose_level64<32, R>(v, lane);
    if constexpr (T >= 4) transpose_level64<16, R / 2>(v, lane);
    if constexpr (T >= 8) transpose_level64<8, R / 4>(v, lane);
    if constexpr (T >= 16) transpose_level64<4, R / 8>(v, lane);
    if constexpr (T >= 32) transpose_level64<2, R / 16>(v, lane);
    if constexpr (T >= 64) transpose_level64<1, R / 32>(v, lane);
    double x = v[0];
#pragma unroll
    for (int g = 1; g < G; ++g) x += v[g];
    if constexpr (T < 64) x += partner64<1>(x);
    if constexpr (T < 32) x += partner64<2>(x);
    if constexpr (T < 16) x += partner64<4>(x);
    if constexpr (T < 8) x += partner64<8>(x);
    if constexpr (T < 4) x += partner64<16>(x);
    if constexpr (T < 2) x += partner64<32>(x);
    return x;
}

// 16 int8 weights against 16 fp64 activations (exact products, fp64 sum). The
// activations are 8 double2 at x[0], x[S], ..., x[7S]. Four independent
// accumulators keep the dependent fp64 FMA chain short (its latency, not the
// FMA rate, bounds these small dot products).
template <int S = 1>
__device__ __forceinline__ double dot_i8x16_d(uint4 w, const double2* x, double acc) {
    const int8_t* b = reinterpret_cast<const int8_t*>(&w);
    double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const double2 xv = x[j * S];
        s[(2 * j) & 3] = fma((double)(float)b[2 * j], xv.x, s[(2 * j) & 3]);
        s[(2 * j + 1) & 3] = fma((double)(float)b[2 * j + 1], xv.y, s[(2 * j + 1) & 3]);
    }
    return acc + ((s[0] + s[1]) + (s[2] + s[3]));
}

// 8 bf16 weights against 8 fp64 activations (4 double2 at x[0], x[S], ...).
template <int S = 1>
__device__ __forceinline__ double dot_bf16x8_d(uint4 w, const double2* x, double acc) {
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const double2 xv = x[j * S];
        s[(2 * j) & 3] = fma((double)__uint_as_float(wv[j] << 16), xv.x, s[(2 * j) & 3]);
        s[(2 * j + 1) & 3] = fma((double)__uint_as_float(wv[j] & 0xffff0000u), xv.y, s[(2 * j + 1) & 3]);
    }
    return acc + ((s[0] + s[1]) + (s[2] + s[3]));
}

// ---- 16-byte dot products ----------------------------------------------------------------
// int8 x16 against 16 fp32 activations (one v_cvt_f32_i32 with a sign-extended
// byte select plus one FMA per element).
__device__ __forceinline__ float dot_i8x16(uint4 w, const float4* x, float acc) {
    const int8_t* b = reinterpret_cast<const int8_t*>(&w);
    float4 x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
    acc = fmaf((float)b[0], x0.x, acc);  acc = fmaf((float)b[1], x0.y, acc);
    acc = fmaf((float)b[2], x0.z, acc);  acc = fmaf((float)b[3], x0.w, acc);
    acc = fmaf((float)b[4], x1.x, acc);  acc = fmaf((float)b[5], x1.y, acc);
    acc = fmaf((float)b[6], x1.z, acc);  acc = fmaf((float)b[7], x1.w, acc);
    acc = fmaf((float)b[8], x2.x, acc);  acc = fmaf((float)b[9], x2.y, acc);
    acc = fmaf((float)b[10], x2.z, acc); acc = fmaf((float)b[11], x2.w, acc);
    acc = fmaf((float)b[12], x3.x, acc); acc = fmaf((float)b[13], x3.y, acc);
    acc = fmaf((float)b[14], x3.z, acc); acc = fmaf((float)b[15], x3.w, acc);
    return acc;
}

// bf16 x8 against 8 fp32 activations.
__device__ __forceinline__ float dot_bf16x8(uint4 w, const float4* x, float acc) {
    float4 x0 = x[0], x1 = x[1];
    acc = fmaf(__uint_as_float(w.x << 16), x0.x, acc);
    acc = fmaf(__uint_as_float(w.x & 0xffff0000u), x0.y, acc);
    acc = fmaf(__uint_as_float(w.y << 16), x0.z, acc);
    acc = fmaf(__uint_as_float(w.y & 0xffff0000u), x0.w, acc);
    acc = fmaf(__uint_as_float(w.z << 16), x1.x, acc);
    acc = fmaf(__uint_as_float(w.z & 0xffff0000u), x1.y, acc);
    acc = fmaf(__uint_as_float(w.w << 16), x1.z, acc);
    acc = fmaf(__uint_as_float(w.w & 0xffff0000u), x1.w, acc);
    return acc;
}

// Weight element formats: bytes per element, elements per 16-byte lane load,
// and the dot product over one lane load.
struct Int8W {
    static constexpr int kBytes = 1;
    static constexpr int kPerLane = 16;
    __device__ static float dot(uint4 w, const float4* x, float acc) { return dot_i8x16(w, x, acc); }
    template <int S = 1>
    __device__ static double dotd(uint4 w, const double2* x, double acc) { return dot_i8x16_d<S>(w, x, acc); }
};
// 16 FP8 E4M3 codes (OCP E4M3FN, decoded exactly by v_cvt_pk_f32_fp8) against 16 fp32
// activations (x[0..3] hold elements 0-3, 4-7, 8-11, 12-15).
__device__ __forceinline__ float dot_fp8x16(uint4 w, const float4* x, float acc) {
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 xv = x[i];
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[i], false);   // bytes 0, 1
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[i], true);    // bytes 2, 3
        acc = fmaf(lo[0], xv.x, acc);
        acc = fmaf(lo[1], xv.y, acc);
        acc = fmaf(hi[0], xv.z, acc);
        acc = fmaf(hi[1], xv.w, acc);
    }
    return acc;
}
// The same against 16 fp64 activations (8 double2 at x[0], x[S], ...): the decoded codes
// and their products are exact in fp64, as the int8 ones are.
template <int S = 1>
__device__ __forceinline__ double dot_fp8x16_d(uint4 w, const double2* x, double acc) {
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[i], false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[i], true);
        const double2 x0 = x[(2 * i) * S], x1 = x[(2 * i + 1) * S];
        s[0] = fma((double)lo[0], x0.x, s[0]);
        s[1] = fma((double)lo[1], x0.y, s[1]);
        s[2] = fma((double)hi[0], x1.x, s[2]);
        s[3] = fma((double)hi[1], x1.y, s[3]);
    }
    return acc + ((s[0] + s[1]) + (s[2] + s[3]));
}
// FP8 E4M3 weights with per-row scales (the INT8 layout: one byte per element, so every
// path that applies INT8 row scales applies these).
struct Fp8W {
    static constexpr int kBytes = 1;
    static constexpr int kPerLane = 16;
    __device__ static float dot(uint4 w, const float4* x, float acc) { return dot_fp8x16(w, x, acc); }
    template <int S = 1>
    __device__ static double dotd(uint4 w, const double2* x, double acc) { return dot_fp8x16_d<S>(w, x, acc); }
};
struct Bf16W {
    static constexpr int kBytes = 2;
    static constexpr int kPerLane = 8;
    __device__ static float dot(uint4 w, const float4* x, float acc) { return dot_bf16x8(w, x, acc); }
    template <int S = 1>
    __device__ static double dotd(uint4 w, const double2* x, double acc) { return dot_bf16x8_d<S>(w, x, acc); }
};

// ---- activation vector in LDS, laid out per lane --------------------------------------
// A wave-wide 16-byte-per-lane load covers one 1 KB "chunk" of a weight row
// (64*kPerLane elements). Lane l needs elements [chunk*64*P + l*P, +P) of the
// activation vector; they are stored as P/4 float4 values at
// xs[(chunk*(P/4) + j)*64 + l] so that the lanes of a wave read consecutive
// float4s (no bank conflicts).
template <class W>
__device__ __forceinline__ int xs_index(int k) {          // float index of element k
    constexpr int P = W::kPerLane;
    const int chunk = k / (64 * P);
    const int e = k % (64 * P);
    const int lane = e / P;
    const int t = e % P;
    return ((chunk * (P / 4) + (t >> 2)) * 64 + lane) * 4 + (t & 3);
}
template <class W>
__device__ __forceinline__ const float4* xs_frag(const float4* xs, int chunk, int lane) {
    constexpr int P = W::kPerLane;
    return xs + (chunk * (P / 4)) * 64 + lane;           // stride 64 float4 between the P/4 parts
}
template <class W>
__device__ __forceinline__ float dot_frag(uint4 w, const float4* frag, float acc) {
    if constexpr (W::kPerLane == 16) {
        float4 x[4] = {frag[0], frag[64], frag[128], frag[192]};
        return W::dot(w, x, acc);
    } else {
        float4 x[2] = {frag[0], frag[64]};
        return W::dot(w, x, acc);
    }
}

// fp64 activation vector in LDS, per-lane order: lane l's P elements of chunk c
// are P/2 double2 at xd[(c*(P/2) + j)*64 + l].
template <class W>
__device__ __forceinline__ int xd_index(int k) {          // double index of element k
    constexpr int P = W::kPerLane;
    const int chunk = k / (64 * P);
    const int e = k % (64 * P);
    const int lane = e / P;
    const int t = e % P;
    return ((chunk * (P / 2) + (t >> 1)) * 64 + lane) * 2 + (t & 1);
}
template <class W>
__device__ __forceinline__ double dot_fragd(uint4 w, const double2* xd, int chunk, int lane, double acc) {
    constexpr int P = W::kPerLane;
    return W::template dotd<64>(w, xd + (chunk * (P / 2)) * 64 + lane, acc);
}

// Piece-major fp64 activation layout for matvecs whose row segment is split
// into 16-byte weight "pieces" handed to consecutive lanes: element k of the
// segment (piece p = k / EPP, e = k % EPP) is stored as double e of double2
// (e / 2) * NP + p, so the lanes of a wave read consecutive double2 values.
__device__ __forceinline__ int piece_index(int k, int epp, int np) {     // double index of element k
    const int p = k / epp, e = k % epp;
    return ((e >> 1) * np + p) * 2 + (e & 1);
}

// Sum of v over aligned groups of N consecutive lanes (N a power of two <= 64);
// every lane of a group receives its group's sum. Butterfly order, so the
// result is bitwise reproducible.
template <int N>
__device__ __forceinline__ double group_sum64(double v) {
    if constexpr (N >= 2) v += partner64<1>(v);
    if constexpr (N >= 4) v += partner64<2>(v);
    if constexpr (N >= 8) v += partner64<4>(v);
    if constexpr (N >= 16) v += partner64<8>(v);
    if constexpr (N >= 32) v += partner64<16>(v);
    if constexpr (N >= 64) v += partner64<32>(v);
    return v;
}

// Maximum over aligned groups of N lanes (N a power of two <= 64).
template <int N>
__device__ __forceinline__ double group_max64(double v) {
    if constexpr (N >= 2) v = fmax(v, partner64<1>(v));
    if constexpr (N >= 4) v = fmax(v, partner64<2>(v));
    if constexpr (N >= 8) v = fmax(v, partner64<4>(v));
    if constexpr (N >= 16) v = fmax(v, partner64<8>(v));
    if constexpr (N >= 32) v = fmax(v, partner64<16>(v));
    if constexpr (N >= 64) v = fmax(v, partner64<32>(v));
    return v;
}

// Keeps the compiler from moving memory accesses across this point (used to
// issue step-independent loads before a wait instead of where they are used).
__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }

// The value of v, hidden from the optimiser. Taken once per iteration of a long
// loop, it keeps per-lane addresses derived from v from being hoisted out of
// the loop and held (or spilled to scratch) for its whole length: they are
// recomputed at their use with a couple of integer operations instead.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// A prefetched 32-bit value, released for use at this point. Without it the
// compiler converts a loaded value right after its load, and the wait for that
// load (loads return in order, so it also waits for every load issued before
// it, such as a stage's weight prefetch) lands ahead of the exchange the
// prefetch is meant to overlap. Prefetched scalars are therefore kept as raw
// bits and pass through here after the wait.
__device__ __forceinline__ uint32_t after_wait(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ float after_wait_f(uint32_t v) { return __uint_as_float(after_wait(v)); }
__device__ __forceinline__ float after_wait_bf16(uint32_t v) { return bf16_bits_to_f32(after_wait(v)); }

// Global-memory view of a pointer. A pointer the kernel reads from memory (the
// per-layer pointer tables) is generic to the compiler, which then emits flat
// loads; a flat load counts against the LDS counter as well, so every later LDS
// wait would also wait for it and a weight prefetch could not overlap the
// exchange that follows. Loads through this view are global loads.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gview(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// 16-byte global load (gview() for uint4, whose assignment operators take
// generic references only).
__device__ __forceinline__ uint4 ldg16(const void* p) {
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The same with the non-temporal hint, for the layer weights: every step streams
// them once (440 MB at the 0.6B shape, more than the 256 MB last-level cache), so
// they should not displace what is reused from one step to the next there (the
// LM-head matrix, 156 MB, read after every step's layers).
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
// Raw 32-bit load of a float / bf16 value for after_wait().
__device__ __forceinline__ uint32_t ldg_bits(const float* p) { return *gview(reinterpret_cast<const uint32_t*>(p)); }
__device__ __forceinline__ uint32_t ldg_bits(const uint16_t* p) { return *gview(p); }

// ---- tagged exchange words --------------------------------------------------------------
// A 64-bit word holds a 32-bit payload and a 32-bit tag naming the step,
// layer and stage that wrote it. Producers store it with one relaxed
// agent-scope atomic store; consumers poll it with relaxed agent-scope atomic
// loads until the tag matches. Payload and tag travel in one single-copy-atomic
// access, so no fence is needed between them.
__device__ __forceinline__ void ll_put(uint64_t* p, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A packed word: an fp64 value whose lowest mantissa bit is replaced by a
// one-bit tag. A buffer of packed words is written once per use and the tag
// alternates between uses (first use 1, the workspace starts zeroed), so a
// reader tells this use's value from the previous one's. That needs every
// reader of a use to have read before the slot is written again, which the
// writers' data dependencies guarantee where these words are used.
__device__ __forceinline__ uint64_t pack_tagged(double v, uint32_t pbit) {
    return ((uint64_t)__double_as_longlong(v) & ~(uint64_t)1) | (uint64_t)(pbit & 1u);
}
__device__ __forceinline__ void ll_put64(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte agent-coherent reads of an exchange region: one buffer load with
// agent scope (sc1) returns two adjacent 64-bit words, so lanes that read
// consecutive 16-byte chunks coalesce into whole cache lines. A 16-byte access
// is one transaction, so each aligned 8-byte word comes back as one store
// wrote it (a word is checked on its own tag). The base must be the same in
// every lane of the wave (the buffer resource lives in scalar registers); reads
// past `nwords` return zero, which is never a tagged word's tag.
struct XRegion {
    __amdgpu_buffer_rsrc_t rs;
    __device__ __forceinline__ XRegion(const uint64_t* base, uint32_t nwords)
        : rs(__builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base), (short)0, (int)(nwords * 8u),
                                               0x00020000 /* 32-bit data format, no swizzle */)) {}
    // words w and w + 1 (w even)
    __device__ __forceinline__ uint4 load2(uint32_t w) const {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(w * 8u), 0, 16 /* sc1 */);
        return make_uint4(v[0], v[1], v[2], v[3]);
    }
};

// Bounded polling. After `limit` unsuccessful polls of one word, or once any
// workgroup has raised the abort flag, every further wait returns at once, so
// a grid whose producers stalled still drains in bounded time and the host
// reports MQ_ERR_TIMEOUT.
struct Waiter {
    uint32_t* abort_flag;
    uint32_t limit;
    bool dead;

    __device__ Waiter(uint32_t* flag, uint32_t lim) : abort_flag(flag), limit(lim), dead(false) {}

    __device__ __forceinline__ uint32_t get(const uint64_t* p, uint32_t tag) {
        uint64_t w = ll_load(p);
        if ((uint32_t)(w >> 32) == tag || dead) return (uint32_t)w;
        uint32_t n = 0;
        for (;;) {
            __builtin_amdgcn_s_sleep(1);
            w = ll_load(p);
            if ((uint32_t)(w >> 32) == tag) break;
            if (++n >= limit) {
                dead = true;
                __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((n & 127u) == 0 &&
                __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                dead = true;
                break;
            }
        }
        return (uint32_t)w;
    }
    __device__ __forceinline__ float getf(const uint64_t* p, uint32_t tag) { return __uint_as_float(get(p, tag)); }

    // N packed words at p[i * stride] (see pack_tagged): waits until bit 0 of
    // each equals `pbit` and returns the fp64 values with that bit cleared.
    template <int N>
    __device__ __forceinline__ void get_packed(const uint64_t* p, int stride, uint32_t pbit, double (&out)[N]) {
        get_packed_at<N>([&](int i) { return p + i * stride; }, pbit, out);
    }

    // As get_packed, for the N packed words at addr(0) .. addr(N - 1).
    template <int N, class Addr>
    __device__ __forceinline__ void get_packed_at(Addr addr, uint32_t pbit, double (&out)[N]) {
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = ll_load(addr(i));
        uint32_t pending = 0;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if ((uint32_t)(w[i] & 1u) != pbit) pending |= 1u << i;
        uint32_t n = 0;
        while (pending != 0 && !dead) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (pending & (1u << i)) w[i] = ll_load(addr(i));
#pragma unroll
            for (int i = 0; i < N; ++i)
                if ((pending & (1u << i)) && (uint32_t)(w[i] & 1u) == pbit) pending &= ~(1u << i);
            if (pending == 0) break;
            if (++n >= limit) {
                dead = true;
                __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((n & 127u) == 0 &&
                __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
                dead = true;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = __longlong_as_double((long long)(w[i] & ~(uint64_t)1));
    }

    // N words at p[i * stride]: all N loads are issued before any is checked,
    // and every retry re-issues the still-missing ones together, so a wait
    // costs one memory round trip however many words a thread reads.
    // Only the first `count` words are read (count <= N); the rest of `out` is 0.
    template <int N>
    __device__ __forceinline__ void get_strided(const uint64_t* p, int stride, uint32_t tag, float (&out)[N],
                                                int count = N) {
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = i < count ? ll_load(p + i * stride) : ((uint64_t)tag << 32);
        uint32_t pending = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            out[i] = __uint_as_float((uint32_t)w[i]);
            if ((uint32_t)(w[i] >> 32) != tag) pending |= 1u << i;
        }
        if (pending == 0 || dead) return;
        uint32_t n = 0;
        for (;;) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (pending & (1u << i)) w[i] = ll_load(p + i * stride);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if ((pending & (1u << i)) && (uint32_t)(w[i] >> 32) == tag) {
                    out[i] = __uint_as_float((uint32_t)w[i]);
                    pending &= ~(1u << i);
                }
            }
            if (pending == 0) return;
            if (++n >= limit) {
                dead = true;
                __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            if ((n & 127u) == 0 &&
                __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                dead = true;
                return;
            }
        }
    }

    // Chunks of two tagged words: chunk i is words w[i], w[i] + 1 of R (w[i] even),
    // payloads to out[2i], out[2i + 1]. Only the first `count` chunks are read (the
    // rest of `out` is 0); all loads are issued before any check, and every retry
    // re-issues the still-missing chunks together.
    template <int N>
    __device__ __forceinline__ void get_pairs(const XRegion& R, const uint32_t (&w)[N], uint32_t tag,
                                              float (&out)[2 * N], int count = N) {
        get_pairs(R, w, tag, out, count, [] {});
    }
    // The same; `meanwhile()` runs once the first loads are issued and before any of
    // them is waited for (work that overlaps the memory round trip).
    template <int N, class F>
    __device__ __forceinline__ void get_pairs(const XRegion& R, const uint32_t (&w)[N], uint32_t tag,
                                              float (&out)[2 * N], int count, F&& meanwhile) {
        uint4 c[N];
#pragma unroll
        for (int i = 0; i < N; ++i) c[i] = i < count ? R.load2(w[i]) : make_uint4(0, tag, 0, tag);
        asm volatile("" ::: "memory");
        meanwhile();
        uint32_t pending = 0;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (c[i].y != tag || c[i].w != tag) pending |= 1u << i;
        uint32_t n = 0;
        while (pending != 0 && !dead) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (pending & (1u << i)) c[i] = R.load2(w[i]);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if ((pending & (1u << i)) && c[i].y == tag && c[i].w == tag) pending &= ~(1u << i);
            if (pending == 0) break;
            if (++n >= limit) {
                dead = true;
                __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((n & 127u) == 0 &&
                __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
                dead = true;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            out[2 * i] = __uint_as_float(c[i].x);
            out[2 * i + 1] = __uint_as_float(c[i].z);
        }
    }

    // Chunks of two packed words (see pack_tagged), as get_pairs: waits until bit 0
    // of both words of each chunk equals `pbit`; values with that bit cleared.
    template <int N>
    __device__ __forceinline__ void get_packed_pairs(const XRegion& R, const uint32_t (&w)[N], uint32_t pbit,
                                                     double (&out)[2 * N], int count = N) {
        uint4 c[N];
#pragma unroll
        for (int i = 0; i < N; ++i) c[i] = i < count ? R.load2(w[i]) : make_uint4(pbit, 0, pbit, 0);
        uint32_t pending = 0;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if ((c[i].x & 1u) != pbit || (c[i].z & 1u) != pbit) pending |= 1u << i;
        uint32_t n = 0;
        while (pending != 0 && !dead) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if (pending & (1u << i)) c[i] = R.load2(w[i]);
#pragma unroll
            for (int i = 0; i < N; ++i)
                if ((pending & (1u << i)) && (c[i].x & 1u) == pbit && (c[i].z & 1u) == pbit) pending &= ~(1u << i);
            if (pending == 0) break;
            if (++n >= limit) {
                dead = true;
                __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((n & 127u) == 0 &&
                __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
                dead = true;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            out[2 * i] = __longlong_as_double((long long)((((uint64_t)c[i].y) << 32) | (c[i].x & ~1u)));
            out[2 * i + 1] = __longlong_as_double((long long)((((uint64_t)c[i].w) << 32) | (c[i].z & ~1u)));
        }
    }
};

// Order-preserving map fp32 -> uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t ordered_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

}  // namespace mq
