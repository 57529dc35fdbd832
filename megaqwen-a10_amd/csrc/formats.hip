// Other weight formats on gfx950: FP8 E4M3 per-row and INT4 per-group weight-only
// matvecs, and their quantizers from bf16. The reference has INT8 (bench_int8.py:19-24)
// and BF16 weights only; these follow the INT8 quantizer's pattern (symmetric scale
// from the absolute maximum, IEEE division, round half to even) with:
//   FP8  (OCP E4M3FN, decoded by v_cvt_pk_f32_fp8): per row s = fp32(amax) / 448,
//        q = nearest code of fp32(w) / s (ties to the even code, |x| >= 448 -> +-448)
//   INT4 per group of 128 elements of a row: s = bf16(amax / 7), q = clamp(rint(w / s), -8, 7),
//        two's complement nibbles, low nibble = even element
// Matvecs y[j] = sum_k dequant(w)[j, k] x[k], fp32 x and y.
//   FP8: the structure of the INT8 matvec (one 16-byte load per lane per 1 KB of a row, the
//        activation in LDS in per-lane order, R rows per wave item, the same steady-state
//        repeat form), 16 weights per lane per load, 8 v_cvt_pk_f32_fp8, fp32 accumulation,
//        the row scale applied after the row sum.
//   INT4: on the int8 matrix cores, as the decode step's products: x as a 55-bit fixed-point
//        vector in eight digit planes, the biased nibbles as the int8 operand, exact integer
//        sums per group of 128, recombined and scaled in fp64 (int4_gemv_kernel).
#include "common.h"
#include "digits.h"
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
// P weights per lane per 16-byte load (16 FP8 codes).
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

// FP8 per row (scale [M]).
template <int R, int CHMAX>
__global__ void __launch_bounds__(kFmtThreads)
fp8_gemv_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w, int64_t copy_stride, int n_copies,
                const float* __restrict__ scale, float* __restrict__ y, int M, int K, int reps) {
    constexpr int P = 16;                            // weights per lane per 16-byte load
    extern __shared__ float4 xs[];
    const int CH = (K + 64 * P - 1) / (64 * P);
    float* xsf = reinterpret_cast<float*>(xs);
    for (int k = threadIdx.x; k < CH * 64 * P; k += kFmtThreads) xsf[fmt_xs_index<P>(k)] = (k < K) ? x[k] : 0.0f;
    __syncthreads();

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int total_waves = gridDim.x * kFmtWaves;
    const int nbatch = (M + R - 1) / R;
    const int items = reps * nbatch;                 // < 2^31, checked by the host

    for (int it = blockIdx.x * kFmtWaves + wave; it < items; it += total_waves) {
        const int rep = it / nbatch;
        const int row0 = (it - rep * nbatch) * R;
        const int copy = rep % n_copies;
        const uint8_t* const wc = w + (int64_t)copy * copy_stride;
        uint4 wv[R][CHMAX];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int c = 0; c < CHMAX; ++c) {
                wv[r][c] = make_uint4(0, 0, 0, 0);
                const int col = c * 64 * P + lane * P;     // first element of the lane's piece
                if (c < CH && row0 + r < M && col < K)
                    wv[r][c] = *reinterpret_cast<const uint4*>(wc + (int64_t)(row0 + r) * K + col);
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
                for (int r = 0; r < R; ++r) acc[r] = dot_fp8x16_regs(wv[r][c], xv, acc[r]);
            }
        }
        const float s = transpose_reduce<R>(acc, lane);
        constexpr int span = kWave / R;
        const int row = row0 + lane / span;
        if ((lane % span) == 0 && row < M) y[(int64_t)copy * M + row] = s * scale[row];
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

template <int R, int CHMAX>
int launch_fp8_t(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                 int M, int K, int reps, hipStream_t stream) {
    constexpr int P = 16;
    const int64_t items = (int64_t)reps * ((M + R - 1) / R);
    const int64_t want = (items + kFmtWaves - 1) / kFmtWaves;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(want, 8 * device_cus()));
    const int CH = (K + 64 * P - 1) / (64 * P);
    const size_t lds = (size_t)CH * 64 * P * sizeof(float);
    hipLaunchKernelGGL((fp8_gemv_kernel<R, CHMAX>), dim3(grid), dim3(kFmtThreads), lds, stream,
                       x, w, copy_stride, n_copies, scale, y, M, K, reps);
    return check_launch("fp8_gemv");
}

// Rows per wave item as in the INT8 matvec: the largest R for the row length that still
// gives every CU at least two workgroups of items.
int fmt_rows_per_item(int M, int CH, int reps) {
    int R = CH <= 1 ? 8 : CH == 2 ? 4 : CH <= 4 ? 2 : 1;
    const int64_t min_waves = (int64_t)2 * kFmtWaves * device_cus();
    while (R > 1 && (int64_t)reps * ((M + R - 1) / R) < min_waves) R /= 2;
    return R;
}

template <int CHMAX>
int launch_fp8_r(int R, const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                 float* y, int M, int K, int reps, hipStream_t stream) {
    constexpr int RMAX = CHMAX <= 1 ? 8 : CHMAX == 2 ? 4 : CHMAX <= 4 ? 2 : 1;
#define MQ_FMT(RR)                                                                                      \
    if constexpr (RR <= RMAX)                                                                           \
        if (R == RR) return launch_fp8_t<RR, CHMAX>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    MQ_FMT(8) MQ_FMT(4) MQ_FMT(2)
#undef MQ_FMT
    return launch_fp8_t<1, CHMAX>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

// ---- INT4 matvec on the int8 matrix cores ----------------------------------------------------
// y[j] = sum_g s[j, g] sum_{k in g} q[j, k] x[k], with the decode step's exact products: x
// becomes X_k = trunc(x_k 2^(181 - emax)) (emax the largest biased exponent of x; |X_k| <
// 2^55) held as eight 7-bit digit planes in LDS. Each nibble is taken biased, b = n XOR 8 =
// q + 8 in [0, 15], as the int8 operand, so that unpacking is two masks a word. Per group of
// 128 elements two v_mfma_i32_16x16x64_i8 give the exact digit sums sum_k b_k d_p(X_k) of 16
// rows; they are recombined in fp64 (one rounding), corrected by -8 S_g with S_g = sum_{k in
// g} X_k (exact int64, once per workgroup), scaled by s[j, g] and summed over the groups in
// fp64; y = fp32(2^(emax - 181) sum). Besides fp64 roundings the error is x's truncation
// to 55 bits of its largest element (x finite).
//
// Operands. For group g, lane (n, kq) (n = lane % 16, kq = lane / 16) of a wave item (16 rows
// from row0) needs the 16 bytes of row row0 + n holding elements 128 g + 32 kq + [0, 32), as
// words w0..w3 of 8 nibbles. K step h (0, 1) of the group takes {lo(w_2h), hi(w_2h),
// lo(w_2h+1), hi(w_2h+1)} as the B operand (lo: the even nibbles masked into bytes, hi: the
// odd ones), so byte j of the lane's 16 holds element 128 g + 32 kq + 16 h + e(j), e = 0 2 4
// 6 1 3 5 7 8 10 12 14 9 11 13 15. Digit plane p holds its digit of that element at byte
// 128 g + 64 h + 16 kq + j (int4_plane_byte), so the A operand of lane l is 16 contiguous
// bytes of plane (l % 16) & 7. Rows 8-15 of the A operand repeat planes 0-7: their sums land
// in lanes 32-63, which are not read. Planes are K + 16 bytes apart, so that the eight
// planes' reads fall on different LDS banks.
//
// Loads. The rows' bytes come in pairs of groups (128 bytes of a row): load A takes rows 0-7
// of the item, load B rows 8-15, lane l chunk c = kq + 4 ((l >> 3) & 1) (16 bytes) of the pair,
// so that every load instruction reads whole 128-byte lines; one row_ror:8 exchange then
// hands lane (n, kq) chunk kq of row n for the pair's first group and chunk kq + 4 for its
// second. The scales of a row are contiguous and only lanes 0-15 (where the row sums end)
// use them: 16-byte loads of four groups' scales when K / 128 is a multiple of 4. (16 rows of
// 64 bytes per load, and one 4-byte scale load per group, measured 0.50-0.56 of the HBM
// peak at the Qwen3-0.6B shapes; this form 0.69-0.81.)
constexpr int kW4Unroll = 8;                      // groups whose loads are issued together (even)

__device__ __forceinline__ int int4_plane_byte(int k) {
    const int r = k & 127, e = r & 15;
    const int j = (e & 1) ? ((e < 8) ? 4 + (e >> 1) : 12 + ((e - 9) >> 1)) : ((e < 8) ? (e >> 1) : 8 + ((e - 8) >> 1));
    return (k & ~127) + 64 * ((r >> 4) & 1) + 16 * (r >> 5) + j;
}

__global__ void __launch_bounds__(kFmtThreads)
int4_gemv_kernel(const float* __restrict__ x, const uint8_t* __restrict__ w, int64_t copy_stride, int n_copies,
                 const float* __restrict__ scale, float* __restrict__ y, int M, int K, int reps, bool vec_scales) {
    extern __shared__ __align__(16) uint8_t w4lds[];
    __shared__ uint32_t red[kFmtWaves];
    constexpr int U = kW4Unroll;
    const int PS = K + 16;                        // digit plane stride in bytes
    uint8_t* const planes = w4lds;
    double* const sg = reinterpret_cast<double*>(w4lds + 8 * PS);   // S_g of each group
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int ng = K / kInt4Group;

    uint32_t em = 0;
    for (int k = threadIdx.x; k < K; k += kFmtThreads) em = max(em, exp_field(x[k]));
    em = wave_max_u32(em);
    if (lane == 0) red[wave] = em;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kFmtWaves; ++i) em = max(em, red[i]);
    for (int k = threadIdx.x; k < K; k += kFmtThreads) {
        int d[8];
        digits55(x[k], em, d);
        const int at = int4_plane_byte(k);
#pragma unroll
        for (int p = 0; p < 8; ++p) planes[p * PS + at] = (uint8_t)(d[p] & 0xff);
    }
    for (int g = wave; g < ng; g += kFmtWaves) {
        int64_t t = fixed55(x[kInt4Group * g + lane], em) + fixed55(x[kInt4Group * g + 64 + lane], em);
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) t += __shfl_xor(t, o, kWave);
        if (lane == 0) sg[g] = (double)t;
    }
    __syncthreads();

    const int nt = (M + 15) / 16;
    const int items = reps * nt;                  // < 2^31, checked by the host
    const int total_waves = gridDim.x * kFmtWaves;
    const int n = lane & 15, kq = lane >> 4;
    const bool low = (lane & 8) == 0;
    const int c = kq + 4 * ((lane >> 3) & 1);     // the lane's 16-byte chunk of a group pair
    const uint8_t* const arow = planes + (lane & 7) * PS + 16 * kq;
    const int64_t rowbytes = K / 2;
    const bool vec = vec_scales && (ng % 4) == 0;
    const double unit = ldexp(1.0, (int)em - 181);
    for (int it = blockIdx.x * kFmtWaves + wave; it < items; it += total_waves) {
        const int rep = it / nt, tile = it - rep * nt;
        const uint8_t* const wc = w + (int64_t)(rep % n_copies) * copy_stride;
        // rows past M repeat the last one (never stored)
        const int rA = min(16 * tile + (lane & 7), M - 1), rB = min(16 * tile + 8 + (lane & 7), M - 1);
        const uint8_t* const pA = wc + (int64_t)rA * rowbytes + 16 * c;
        const uint8_t* const pB = wc + (int64_t)rB * rowbytes + 16 * c;
        const float* const srow = scale + (int64_t)min(16 * tile + n, M - 1) * ng;
        double acc = 0.0;
        for (int g0 = 0; g0 < ng; g0 += U) {
            uint4 va[U / 2], vb[U / 2];
            float sc[U];
#pragma unroll
            for (int u = 0; u < U / 2; ++u) {
                if (g0 + 2 * u + (c >> 2) < ng) {        // the group this lane's chunk is in
                    va[u] = ldg16_stream(pA + 128 * (g0 / 2 + u));
                    vb[u] = ldg16_stream(pB + 128 * (g0 / 2 + u));
                }
            }
            if (vec && g0 + U <= ng) {
#pragma unroll
                for (int u = 0; u < U; u += 4) {
                    float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (lane < 16) f = *reinterpret_cast<const float4*>(srow + g0 + u);
                    sc[u] = f.x; sc[u + 1] = f.y; sc[u + 2] = f.z; sc[u + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) sc[u] = (g0 + u < ng) ? srow[g0 + u] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (g0 + u < ng) {
                    const int g = g0 + u;
                    // first group of the pair: low lanes keep their A chunk, high lanes take B from
                    // lane - 8; second group: low lanes take A from lane + 8, high lanes keep B
                    const uint4& mine = (u & 1) ? vb[u / 2] : va[u / 2];
                    const uint4& other = (u & 1) ? va[u / 2] : vb[u / 2];
                    const bool keep = (u & 1) ? !low : low;
                    auto pick = [&](uint32_t m, uint32_t o) -> uint32_t {
                        const uint32_t r = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)o, 0x128, 0xF, 0xF, false);
                        return keep ? m : r;                               // 0x128: row_ror:8
                    };
                    const uint32_t q0 = pick(mine.x, other.x) ^ 0x88888888u, q1 = pick(mine.y, other.y) ^ 0x88888888u;
                    const uint32_t q2 = pick(mine.z, other.z) ^ 0x88888888u, q3 = pick(mine.w, other.w) ^ 0x88888888u;
                    const i32x4_t b0 = {(int)(q0 & 0x0F0F0F0Fu), (int)((q0 >> 4) & 0x0F0F0F0Fu),
                                        (int)(q1 & 0x0F0F0F0Fu), (int)((q1 >> 4) & 0x0F0F0F0Fu)};
                    const i32x4_t b1 = {(int)(q2 & 0x0F0F0F0Fu), (int)((q2 >> 4) & 0x0F0F0F0Fu),
                                        (int)(q3 & 0x0F0F0F0Fu), (int)((q3 >> 4) & 0x0F0F0F0Fu)};
                    const uint4 a0 = *reinterpret_cast<const uint4*>(arow + kInt4Group * g);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(arow + kInt4Group * g + 64);
                    i32x4_t cc = mfma_i8(i32x4_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w}, b0, i32x4_t{0, 0, 0, 0});
                    cc = mfma_i8(i32x4_t{(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w}, b1, cc);
                    // lane n: digits 0-3 of row n, lane n + 16: digits 4-7 (each sum < 2^18, exact)
                    const double half = ((double)cc[0] * 2097152.0 + (double)cc[1] * 16384.0) +
                                        ((double)cc[2] * 128.0 + (double)cc[3]);
                    const double v = fma(half, 268435456.0, partner64<16>(half)) - 8.0 * sg[g];
                    acc = fma(v, (double)sc[u], acc);
                }
            }
        }
        if (lane < 16 && 16 * tile + n < M) y[(int64_t)(rep % n_copies) * M + 16 * tile + n] = (float)(acc * unit);
    }
}

int launch_int4_t(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                  int M, int K, int reps, hipStream_t stream) {
    const int64_t items = (int64_t)reps * ((M + 15) / 16);
    const int64_t want = (items + kFmtWaves - 1) / kFmtWaves;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(want, 8 * device_cus()));
    const size_t lds = (size_t)8 * (K + 16) + sizeof(double) * (K / kInt4Group);   // <= 132 KB (K <= 16384)
    if (lds > 65536) {
        static bool raised[64] = {false};          // per device: the limit is the current device's
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
        if (!raised[dev]) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(int4_gemv_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return set_error(MQ_ERR_HIP, "int4_gemv: %zu bytes of LDS: %s", lds, hipGetErrorString(e));
            raised[dev] = true;
        }
    }
    const bool vec_scales = ((uintptr_t)scale % 16) == 0;
    hipLaunchKernelGGL(int4_gemv_kernel, dim3(grid), dim3(kFmtThreads), lds, stream,
                       x, w, copy_stride, n_copies, scale, y, M, K, reps, vec_scales);
    return check_launch("int4_gemv");
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
    constexpr int P = 16;
    const int CH = (K + 64 * P - 1) / (64 * P);
    const int R = fmt_rows_per_item(M, CH, reps);
    if (CH <= 1) return launch_fp8_r<1>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH == 2) return launch_fp8_r<2>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH <= 4) return launch_fp8_r<4>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    if (CH <= 8) return launch_fp8_r<8>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
    return launch_fp8_r<16>(R, x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

int launch_int4_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                     int M, int K, int reps, hipStream_t stream) {
    return launch_int4_t(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream);
}

}  // namespace mq
