// Other weight formats on gfx950: FP8 E4M3 per-row and INT4 per-group weight-only
// matvecs, and their quantizers from bf16. The reference has INT8 (bench_int8.py:19-24)
// and BF16 weights only; these follow the INT8 quantizer's pattern (symmetric scale
// from the absolute maximum, IEEE division, round half to even) with:
//   FP8  (OCP E4M3FN, decoded by v_cvt_pk_f32_fp8): per row s = fp32(amax) / 448,
//        q = nearest code of fp32(w) / s (ties to the even code, |x| >= 448 -> +-448)
//   INT4 per group of 128 elements of a row: s = bf16(amax / 7), q = clamp(rint(w / s), -8, 7),
//        two's complement nibbles, low nibble = even element
// Matvec y[j] = sum_k dequant(w)[j, k] x[k] with fp32 x and y, fp32 accumulation:
// the structure of the INT8 matvec (one 16-byte load per lane per 1 KB of a row, the
// activation in LDS in per-lane order, R rows per wave item, the same steady-state
// repeat form). FP8: 16 weights per lane per 16-byte load, 8 v_cvt_pk_f32_fp8, the row
// scale applied after the row sum. INT4: 16 weights per lane per 8-byte load (a row of
// 1024 fills all 64 lanes; one group is eight lanes' loads), biased nibbles converted
// with v_cvt_f32_ubyteN, and the lane's partial sum scaled by its group's scale before
// the row sum.
#include "common.h"
#include "internal.h"

#include <algorithm>

namespace mq {

namespace {

constexpr int kFmtThreads = 256;
constexpr int kFmtWaves = kFmtThreads / kWave;
constexpr int kInt4Group = 128;

// ---- quantizers ------------------------------------------------------------------------
__device__ __forceinline__ uint32_t fp8_e4m3_encode(float x) {
    const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = fabsf(x);
    if (!(a < 448.0f)) return sign | 0x7Eu;                       // saturate (and NaN)
    if (a < 0x1p-6f) return sign | (uint32_t)__builtin_rintf(a * 512.0f);   // subnormal: m 2^-9, exact scaling
    const uint32_t u = __float_as_uint(a);
    const uint32_t r = (u + 0x7FFFFu + ((u >> 20) & 1u)) & 0xFFF00000u;      // mantissa to 3 bits, RNE
    const int e = (int)(r >> 23) - 127;
    return sign | ((uint32_t)(e + 7) << 3) | ((r >> 20) & 7u);
}

__device__ __forceinline__ float block_max_abs(float v, float* red) {
    v = wave_max(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kFmtWaves; ++i) m = fmaxf(m, red[i]);
    return m;
}

__global__ void __launch_bounds__(kFmtThreads)
quantize_fp8_rows_kernel(const uint16_t* __restrict__ w, int64_t K, uint8_t* __restrict__ q, float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const uint16_t* wr = w + row * K;
    uint8_t* qr = q + row * K;
    __shared__ float red[kFmtWaves];
    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += kFmtThreads) amax = fmaxf(amax, fabsf(bf16_bits_to_f32(wr[k])));
    const float m = block_max_abs(amax, red);
    const float s = fmaxf(__fdiv_rn(m, 448.0f), 1e-12f);
    if (threadIdx.x == 0) scale[row] = s;
    for (int64_t k = threadIdx.x; k < K; k += kFmtThreads)
        qr[k] = (uint8_t)fp8_e4m3_encode(__fdiv_rn(bf16_bits_to_f32(wr[k]), s));
}

// One workgroup per row; thread t quantizes groups t, t + 256, ... of the row.
__global__ void __launch_bounds__(kFmtThreads)
quantize_int4_groups_kernel(const uint16_t* __restrict__ w, int64_t K, uint8_t* __restrict__ q,
                            float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const int64_t ng = K / kInt4Group;
    for (int64_t gi = threadIdx.x; gi < ng; gi += kFmtThreads) {
        const uint16_t* wg = w + row * K + gi * kInt4Group;
        float amax = 0.0f;
        for (int k = 0; k < kInt4Group; ++k) amax = fmaxf(amax, fabsf(bf16_bits_to_f32(wg[k])));
        const float s = fmaxf(round_bf16(__fdiv_rn(amax, 7.0f)), 1e-12f);
        scale[row * ng + gi] = s;
        uint8_t* qg = q + row * (K / 2) + gi * (kInt4Group / 2);
        for (int k = 0; k < kInt4Group; k += 2) {
            const float r0 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(bf16_bits_to_f32(wg[k]), s)), -8.0f), 7.0f);
            const float r1 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(bf16_bits_to_f32(wg[k + 1]), s)), -8.0f), 7.0f);
            qg[k / 2] = (uint8_t)(((uint32_t)(int)r0 & 15u) | (((uint32_t)(int)r1 & 15u) << 4));
        }
    }
}

// ---- matvecs -----------------------------------------------------------------------------
// P weights per lane per 16-byte load: 16 (FP8) or 32 (INT4).
template <int P>
__device__ __forceinline__ int fmt_xs_index(int k) {              // float index of element k
    const int chunk = k / (64 * P);
    const int e = k % (64 * P);
    const int lane = e / P;
    const int t = e % P;
    return ((chunk * (P / 4) + (t >> 2)) * 64 + lane) * 4 + (t & 3);
}

// 16 FP8 codes against 16 activations (x[i] holds elements 4i .. 4i + 3)
__device__ __forceinline__ float dot_fp8x16_regs(uint4 w, const float4 (&x)[4], float acc) {
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

// 16 INT4 nibbles against 16 activations (x[i] holds elements 4i .. 4i + 3), in
// biased form: each two's complement nibble n XOR 8 is n + 8 in [0, 15]. A word's even
// and odd nibbles masked into bytes convert with one v_cvt_f32_ubyteN each, so a weight
// costs a conversion and an FMA; the caller subtracts 8 * (sum of the 16 activations).
__device__ __forceinline__ float dot_int4x16_biased(uint2 w, const float4 (&x)[4]) {
    const uint32_t wv[2] = {w.x ^ 0x88888888u, w.y ^ 0x88888888u};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t lo = wv[i] & 0x0F0F0F0Fu;            // bytes: elements 0, 2, 4, 6 of the word
        const uint32_t hi = (wv[i] >> 4) & 0x0F0F0F0Fu;     // elements 1, 3, 5, 7
        const float4 x0 = x[2 * i], x1 = x[2 * i + 1];
        acc = fmaf((float)(lo & 0xFFu), x0.x, acc);
        acc = fmaf((float)(hi & 0xFFu), x0.y, acc);
        acc = fmaf((float)((lo >> 8) & 0xFFu), x0.z, acc);
        acc = fmaf((float)((hi >> 8) & 0xFFu), x0.w, acc);
        acc = fmaf((float)((lo >> 16) & 0xFFu), x1.x, acc);
        acc = fmaf((float)((hi >> 16) & 0xFFu), x1.y, acc);
        acc = fmaf((float)(lo >> 24), x1.z, acc);
        acc = fmaf((float)(hi >> 24), x1.w, acc);
    }
    return acc;
}

// kInt4: INT4 per group (scale [M, K / 128]); else FP8 per row (scale [M]).
template <bool kInt4, int R, int CHMAX>
__global__ void __launch_bounds__(kFmtThreads)
fmt_gemv_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w, int64_t copy_stride, int n_copies,
                const float* __restrict__ scale, float* __restrict__ y, int M, int K, int reps) {
    constexpr int P = 16;                            // weights per lane per load (16 or 8 bytes)
    extern __shared__ float4 xs[];
    const int CH = (K + 64 * P - 1) / (64 * P);
    float* xsf = reinterpret_cast<float*>(xs);
    for (int k = threadIdx.x; k < CH * 64 * P; k += kFmtThreads) xsf[fmt_xs_index<P>(k)] = (k < K) ? x[k] : 0.0f;
    __syncthreads();

    const int lane = threadIdx.x % kWave;
    // INT4: 8 x the sum of the lane's 16 activations per chunk (the nibbles' bias)
    float xb[CHMAX];
#pragma unroll
    for (int c = 0; c < CHMAX; ++c) {
        xb[c] = 0.0f;
        if (kInt4 && c < CH) {
            const float4* f = xs + (c * (P / 4)) * 64 + lane;
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < P / 4; ++i) t += (f[i * 64].x + f[i * 64].y) + (f[i * 64].z + f[i * 64].w);
            xb[c] = 8.0f * t;
        }
    }
    const int wave = threadIdx.x / kWave;
    const int total_waves = gridDim.x * kFmtWaves;
    const int nbatch = (M + R - 1) / R;
    const int items = reps * nbatch;                 // < 2^31, checked by the host
    const int64_t rowbytes = kInt4 ? K / 2 : K;
    const int ng = K / kInt4Group;

    for (int it = blockIdx.x * kFmtWaves + wave; it < items; it += total_waves) {
        const int rep = it / nbatch;
        const int row0 = (it - rep * nbatch) * R;
        const int copy = rep % n_copies;
        const uint8_t* const wc = w + (int64_t)copy * copy_stride;
        uint4 wv[R][CHMAX];                          // FP8: 16 bytes; INT4: 8 bytes in .x, .y
        float gs[R][CHMAX];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int c = 0; c < CHMAX; ++c) {
                wv[r][c] = make_uint4(0, 0, 0, 0);
                gs[r][c] = 0.0f;
                const int col = c * 64 * P + lane * P;     // first element of the lane's piece
                if (c < CH && row0 + r < M && col < K) {
                    const uint8_t* p = wc + (int64_t)(row0 + r) * rowbytes + (kInt4 ? col / 2 : col);
                    if constexpr (kInt4) {
                        const uint2 v = *reinterpret_cast<const uint2*>(p);
                        wv[r][c] = make_uint4(v.x, v.y, 0, 0);
                        gs[r][c] = scale[(int64_t)(row0 + r) * ng + col / kInt4Group];
                    } else {
                        wv[r][c] = *reinterpret_cast<const uint4*>(p);
                    }
                }
            }
        }
        // chunk outer, rows inner: the lane's 16 activations of a chunk are read from LDS
        // once and used for all R rows
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < CHMAX; ++c) {
            if (c < CH) {
                const float4* frag = xs + (c * (P / 4)) * 64 + lane;
                const float4 xv[4] = {frag[0], frag[64], frag[128], frag[192]};
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if constexpr (kInt4)
                        acc[r] = fmaf(dot_int4x16_biased(make_uint2(wv[r][c].x, wv[r][c].y), xv) - xb[c], gs[r][c],
                                      acc[r]);
                    else acc[r] = dot_fp8x16_regs(wv[r][c], xv, acc[r]);
                }
            }
        }
        const float s = transpose_reduce<R>(acc, lane);
        constexpr int span = kWave / R;
        const int row = row0 + lane / span;
        if ((lane % span) == 0 && row < M) y[(int64_t)copy * M + row] = kInt4 ? s : s * scale[row];
    }
}

int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

template <bool kInt4, int R, int CHMAX>
int launch_fmt_t(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                 int M, int K, int reps, hipStream_t stream) {
    constexpr int P = 16;
    const int64_t items = (int64_t)reps * ((M + R - 1) / R);
    const int64_t want = (items + kFmtWaves - 1) / kFmtWaves;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(want, 8 * device_cus()));
    const int CH = (K + 64 * P - 1) / (64 * P);
    const size_t lds = (size_t)CH * 64 * P * sizeof(float);
    hipLaunchKernelGGL((fmt_gemv_kernel<kInt4, R, CHMAX>), dim3(grid), dim3(kFmtThreads), lds, stream,
                       x, w, copy_stride, n_copies, scale, y, M, K, reps);
    return check_launch(kInt4 ? "int4_gemv" : "fp8_gemv");
}

// Rows per wave item as in the INT8 matvec: the largest R for the row length that still
// gives every CU at least two workgroups of items. (Twice the rows for INT4, to match the
// INT8 bytes in flight per wave, measured slower: the INT4 loop is bound by its VALU work.)
int fmt_rows_per_item(int M, int CH, int reps) {
    int R = CH <= 1 ? 8 : CH == 2 ? 4 : CH <= 4 ? 2 : 1;
    const int64_t min_waves = (int64_t)2 * kFmtWaves * device_cus();
    while (R > 1 && (int64_t)reps * ((M + R - 1) / R) < min_waves) R /= 2;
    return R;
}

template <bool kInt4, int CHMAX>
int launch_fmt_r(int R, const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                 float* y, int M, int K, int reps, hipStream_t stream) {
    constexpr int RMAX = CHMAX <= 1 ? 8 : CHMAX == 2 ? 4 : CHMAX <= 4 ? 2 : 1;
#define MQ_FMT(RR)                                                                                      \
    if constexpr (RR <= RMAX)                                                                           \
        if (R == RR) return launch_fmt_t<kInt4, RR, CHMAX>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    MQ_FMT(8) MQ_FMT(4) MQ_FMT(2)
#undef MQ_FMT
    return launch_fmt_t<kInt4, 1, CHMAX>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

template <bool kInt4>
int launch_fmt(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
               int M, int K, int reps, hipStream_t stream) {
    constexpr int P = 16;
    const int CH = (K + 64 * P - 1) / (64 * P);
    const int R = fmt_rows_per_item(M, CH, reps);
    if (CH <= 1) return launch_fmt_r<kInt4, 1>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH == 2) return launch_fmt_r<kInt4, 2>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH <= 4) return launch_fmt_r<kInt4, 4>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH <= 8) return launch_fmt_r<kInt4, 8>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    return launch_fmt_r<kInt4, 16>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

}  // namespace

int launch_quantize_fp8(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_fp8_rows_kernel, dim3(M), dim3(kFmtThreads), 0, stream,
                       static_cast<const uint16_t*>(w_bf16), (int64_t)K, q, scale);
    return check_launch("quantize_fp8_rows_kernel");
}

int launch_quantize_int4(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_int4_groups_kernel, dim3(M), dim3(kFmtThreads), 0, stream,
                       static_cast<const uint16_t*>(w_bf16), (int64_t)K, q, scale);
    return check_launch("quantize_int4_groups_kernel");
}

int launch_fp8_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                    int M, int K, int reps, hipStream_t stream) {
    return launch_fmt<false>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

int launch_int4_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                     int M, int K, int reps, hipStream_t stream) {
    return launch_fmt<true>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

}  // namespace mq
