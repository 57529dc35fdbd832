// Standalone INT8 weight-only matvec, y[j] = scale[j] * sum_k x[k] * w[j,k]
// (int8_decoder.py:100-115 semantics; fp32 activations as BASELINE config 2).
//
// Layout: one 64-lane wave owns R consecutive rows at a time; each lane reads
// 16 contiguous int8 of a row per 1 KB chunk (one global_load_dwordx4 per
// chunk, a fully coalesced 1 KB row segment per wave instruction), converts
// with v_cvt_f32_i32 on a sign-extended byte and FMAs against the activation
// fragment held in LDS in per-lane order. The R row sums are finished with a
// transpose reduction (R values -> 1 per lane group). Waves stride over row
// batches so the grid stays at a few workgroups per CU.
#include "common.h"
#include "internal.h"

#include <algorithm>

namespace mq {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

template <int R, int CHMAX>
__global__ void __launch_bounds__(kGemvThreads)
int8_gemv_kernel(const float* __restrict__ x, const int8_t* __restrict__ w,
                 const float* __restrict__ scale, float* __restrict__ y, int M, int K) {
    extern __shared__ float4 xs[];
    const int CH = (K + 1023) / 1024;
    float* xsf = reinterpret_cast<float*>(xs);
    for (int k = threadIdx.x; k < CH * 1024; k += kGemvThreads)
        xsf[xs_index<Int8W>(k)] = (k < K) ? x[k] : 0.0f;
    __syncthreads();

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int total_waves = gridDim.x * kGemvWaves;
    const int nbatch = (M + R - 1) / R;
    const int64_t rowbytes = K;

    for (int b = blockIdx.x * kGemvWaves + wave; b < nbatch; b += total_waves) {
        const int row0 = b * R;
        uint4 wv[R][CHMAX];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int c = 0; c < CHMAX; ++c) {
                wv[r][c] = make_uint4(0, 0, 0, 0);
                const int col = c * 1024 + lane * 16;
                if (c < CH && row0 + r < M && col < K)
                    wv[r][c] = *reinterpret_cast<const uint4*>(w + (int64_t)(row0 + r) * rowbytes + col);
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int c = 0; c < CHMAX; ++c)
                if (c < CH) acc[r] = dot_frag<Int8W>(wv[r][c], xs_frag<Int8W>(xs, c, lane), acc[r]);
        }
        const float s = transpose_reduce<R>(acc, lane);
        constexpr int span = kWave / R;
        const int row = row0 + lane / span;
        if ((lane % span) == 0 && row < M) y[row] = s * scale[row];
    }
}

static int device_cu_count() {
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
static int launch_gemv_t(const float* x, const int8_t* w, const float* scale, float* y, int M, int K,
                         hipStream_t stream) {
    const int nbatch = (M + R - 1) / R;
    const int want = (nbatch + kGemvWaves - 1) / kGemvWaves;
    const int grid = std::max(1, std::min(want, 8 * device_cu_count()));
    const int CH = (K + 1023) / 1024;
    const size_t lds = (size_t)CH * 1024 * sizeof(float);
    hipLaunchKernelGGL((int8_gemv_kernel<R, CHMAX>), dim3(grid), dim3(kGemvThreads), lds, stream,
                       x, w, scale, y, M, K);
    return check_launch("int8_gemv_kernel");
}

int launch_int8_gemv(const float* x, const int8_t* w, const float* scale, float* y, int M, int K,
                     hipStream_t stream) {
    const int CH = (K + 1023) / 1024;
    if (CH <= 1) return launch_gemv_t<8, 1>(x, w, scale, y, M, K, stream);
    if (CH == 2) return launch_gemv_t<4, 2>(x, w, scale, y, M, K, stream);
    if (CH <= 4) return launch_gemv_t<2, 4>(x, w, scale, y, M, K, stream);
    if (CH <= 8) return launch_gemv_t<1, 8>(x, w, scale, y, M, K, stream);
    return launch_gemv_t<1, 16>(x, w, scale, y, M, K, stream);
}

}  // namespace mq
