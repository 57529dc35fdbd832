// Per-output-channel symmetric INT8 quantization of bf16 weights on the GPU
// (bench_int8.py:19-24, quantize_per_channel):
//   amax  = max_k |w[j,k]|                exact in bf16
//   scale = bf16_rne(amax / 127.0f)       the reference divides in bf16
//           widened to fp32, clamped to >= 1e-12f
//   q     = clamp(rint(fp32(w) / scale), -128, 127)   IEEE division, ties to even
// One workgroup per row; each thread reads the row's bf16 elements k = tid, tid + 256, ...
// (2-byte loads; the quantizer runs once at load time, off the decode path).
#include "common.h"
#include "internal.h"

namespace mq {

constexpr int kQuantThreads = 256;

__global__ void __launch_bounds__(kQuantThreads)
quantize_rows_kernel(const uint16_t* __restrict__ w, int64_t K, int8_t* __restrict__ q,
                     float* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const uint16_t* wr = w + row * K;
    int8_t* qr = q + row * K;
    __shared__ float red[kQuantThreads / kWave];

    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += kQuantThreads)
        amax = fmaxf(amax, fabsf(bf16_bits_to_f32(wr[k])));
    amax = wave_max(amax);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) red[wave] = amax;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < kQuantThreads / kWave; ++i) m = fmaxf(m, red[i]);

    float s = round_bf16(__fdiv_rn(m, 127.0f));
    s = fmaxf(s, 1e-12f);
    if (threadIdx.x == 0) scale[row] = s;
    for (int64_t k = threadIdx.x; k < K; k += kQuantThreads) {
        float r = __builtin_rintf(__fdiv_rn(bf16_bits_to_f32(wr[k]), s));
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        qr[k] = (int8_t)(int)r;
    }
}

int launch_quantize(const void* w_bf16, int M, int K, int8_t* q, float* scale, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(M), dim3(kQuantThreads), 0, stream,
                       static_cast<const uint16_t*>(w_bf16), (int64_t)K, q, scale);
    return check_launch("quantize_rows_kernel");
}

}  // namespace mq
