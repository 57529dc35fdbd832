// Standalone INT8 weight-only matvec, y[j] = scale[j] * sum_k x[k] * w[j,k]
// (int8_decoder.py:100-115 semantics; fp32 activations as BASELINE config 2).
//
// Layout: one 64-lane wave owns R consecutive rows at a time; each lane reads
// 16 contiguous int8 of a row per 1 KB chunk (one global_load_dwordx4 per
// chunk, a fully coalesced 1 KB row segment per wave instruction), converts
// with v_cvt_f32_i32 on a sign-extended byte and FMAs against the activation
// fragment held in LDS in per-lane order. The R row sums are finished with a
// transpose reduction (R values -> 1 per lane group). Waves stride over row
// batches; R is chosen per call so that small shapes still spread over every CU.
//
// Repeat mode (steady-state measurement): one launch computes `reps` matvecs,
// rep i against weight copy i % n_copies (copies `copy_stride` bytes apart,
// output row block i % n_copies of y). The items (rep, row batch) are
// independent, so the waves stream weights without a launch or a ramp between
// matvecs; reps = n_copies = 1 is the plain call.
#include "common.h"
#include "internal.h"

#include <algorithm>

namespace mq {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

template <int R, int CHMAX>
__global__ void __launch_bounds__(kGemvThreads)
int8_gemv_kernel(const float* __restrict__ x, const int8_t* __restrict__ w, int64_t copy_stride, int n_copies,
                 const float* __restrict__ scale, float* __restrict__ y, int M, int K, int reps) {
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
    const int items = reps * nbatch;                 // < 2^31, checked by the host
    const int64_t rowbytes = K;

    for (int it = blockIdx.x * kGemvWaves + wave; it < items; it += total_waves) {
        const int rep = it / nbatch;
        const int row0 = (it - rep * nbatch) * R;
        const int copy = rep % n_copies;
        const int8_t* const wc = w + (int64_t)copy * copy_stride;
        uint4 wv[R][CHMAX];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int c = 0; c < CHMAX; ++c) {
                wv[r][c] = make_uint4(0, 0, 0, 0);
                const int col = c * 1024 + lane * 16;
                if (c < CH && row0 + r < M && col < K)
                    wv[r][c] = *reinterpret_cast<const uint4*>(wc + (int64_t)(row0 + r) * rowbytes + col);
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
                const float4* frag = xs_frag<Int8W>(xs, c, lane);
                float4 xv[4] = {frag[0], frag[64], frag[128], frag[192]};
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = Int8W::dot(wv[r][c], xv, acc[r]);
            }
        }
        const float s = transpose_reduce<R>(acc, lane);
        constexpr int span = kWave / R;
        const int row = row0 + lane / span;
        if ((lane % span) == 0 && row < M) y[(int64_t)copy * M + row] = s * scale[row];
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
static int launch_gemv_t(const float* x, const int8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                         float* y, int M, int K, int reps, hipStream_t stream) {
    const int64_t items = (int64_t)reps * ((M + R - 1) / R);
    const int64_t want = (items + kGemvWaves - 1) / kGemvWaves;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(want, 8 * device_cu_count()));
    const int CH = (K + 1023) / 1024;
    const size_t lds = (size_t)CH * 1024 * sizeof(float);
    hipLaunchKernelGGL((int8_gemv_kernel<R, CHMAX>), dim3(grid), dim3(kGemvThreads), lds, stream,
                       x, w, copy_stride, n_copies, scale, y, M, K, reps);
    return check_launch("int8_gemv_kernel");
}

// Rows per wave item: the largest R for the row length (R rows x CH chunks of 16 bytes
// per lane in flight) that still gives every CU at least two workgroups of items; a
// matvec of a few MB (QKV, O, down at the 0.6B shape) is one DRAM round trip, so it
// needs all CUs issuing at once rather than fewer waves each reading more rows.
static int gemv_rows_per_item(int M, int CH, int reps) {
    int R = CH <= 1 ? 8 : CH == 2 ? 4 : CH <= 4 ? 2 : 1;
    const int64_t min_waves = (int64_t)2 * kGemvWaves * device_cu_count();
    while (R > 1 && (int64_t)reps * ((M + R - 1) / R) < min_waves) R /= 2;
    return R;
}

int launch_int8_gemv_repeat(const float* x, const int8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                            float* y, int M, int K, int reps, hipStream_t stream) {
    const int CH = (K + 1023) / 1024;
    const int R = gemv_rows_per_item(M, CH, reps);
#define MQ_GEMV(RR, CC) return launch_gemv_t<RR, CC>(x, w, copy_stride, n_copies, scale, y, M, K, reps, stream)
    if (CH <= 1) {
        if (R == 8) MQ_GEMV(8, 1);
        if (R == 4) MQ_GEMV(4, 1);
        if (R == 2) MQ_GEMV(2, 1);
        MQ_GEMV(1, 1);
    }
    if (CH == 2) {
        if (R == 4) MQ_GEMV(4, 2);
        if (R == 2) MQ_GEMV(2, 2);
        MQ_GEMV(1, 2);
    }
    if (CH <= 4) {
        if (R == 2) MQ_GEMV(2, 4);
        MQ_GEMV(1, 4);
    }
    if (CH <= 8) MQ_GEMV(1, 8);
    MQ_GEMV(1, 16);
#undef MQ_GEMV
}

int launch_int8_gemv(const float* x, const int8_t* w, const float* scale, float* y, int M, int K,
                     hipStream_t stream) {
    return launch_int8_gemv_repeat(x, w, 0, 1, scale, y, M, K, 1, stream);
}

}  // namespace mq
