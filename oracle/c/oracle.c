/*
 * oracle.c — plain-C restatement of the byte/integer parts of the decode
 * path (TEST INFRASTRUCTURE: loaded only by the tests to pin the Python
 * oracle and to check the HIP kernels).
 *
 * oracle_quantize_bf16  bench_int8.py:19-24 (quantize_per_channel), written
 *                       from the IEEE definitions rather than torch ops:
 *                       amax exact in bf16; scale = bf16_rne(amax / 127.0f)
 *                       widened to fp32 and clamped to >= 1e-12f;
 *                       q = clamp(rint(fp32(w) / scale), -128, 127) with the
 *                       default round-to-nearest-even mode.
 * oracle_int8_matvec_f64  y[j] = sum_k double(q[j,k]) * double(x[k]) * double(scale[j])
 *                       (the textbook dequantized product; int8_decoder.py:100-115).
 * oracle_bf16_round     fp32 -> bf16 round-to-nearest-even, returned as fp32.
 *
 * Built with -O2 and without -ffast-math so that '/' is the IEEE division.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float bf16_bits_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

static uint16_t f32_to_bf16_bits_rne(float f) {
    uint32_t u = f32_to_bits(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float oracle_bf16_round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits_rne(f)); }

void oracle_quantize_bf16(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, float* scale) {
    for (int64_t j = 0; j < rows; ++j) {
        const uint16_t* row = w + j * cols;
        float amax = 0.0f;
        for (int64_t k = 0; k < cols; ++k) {
            float a = fabsf(bf16_bits_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        float s = oracle_bf16_round(amax / 127.0f);
        if (s < 1e-12f) s = 1e-12f;
        scale[j] = s;
        for (int64_t k = 0; k < cols; ++k) {
            float r = rintf(bf16_bits_to_f32(row[k]) / s);
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            q[j * cols + k] = (int8_t)r;
        }
    }
}

void oracle_int8_matvec_f64(const int8_t* q, const float* scale, const float* x,
                            int64_t rows, int64_t cols, double* y) {
    for (int64_t j = 0; j < rows; ++j) {
        const int8_t* row = q + j * cols;
        double acc = 0.0;
        for (int64_t k = 0; k < cols; ++k) acc += (double)row[k] * (double)x[k];
        y[j] = acc * (double)scale[j];
    }
}
