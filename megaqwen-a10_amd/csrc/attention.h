// Decode attention of one KV head and its two query heads over the bf16 KV
// cache, for one 512-thread workgroup (a10_int8_decode_kernel.cu:165-359):
// QK-RMSNorm and RoPE of the new q/k rows, the bf16 cache write, scores,
// softmax and P @ V. Everything is computed in fp64 and rounded to fp32 / bf16
// only where the reference stores a value (q and k after RoPE, the cache rows,
// the attention output), so the output is the correctly rounded value of the
// reference's expression.
#pragma once

#include "decode_common.h"

namespace mq {

constexpr int kHD = 128;               // head dim

// LDS working set.
struct AttnShared {
    double q[2][kHD];                      // rotated queries (fp32 values)
    uint32_t kv_cur[2][kHD / 2];           // this position's K and V rows (bf16 pairs)
    uint32_t kv_pre[2][kKvLds][kHD / 2];   // K and V rows of the first kKvLds positions
    double p[2][kMaxAttnLen];              // scores
    double pv[kWaves][2 * kHD];            // per-wave partial P @ V
    double wred[4][kWaves];                // per-wave score maxima, then probability sums (2 heads each)
};

// QK-RMSNorm and RoPE (split-half rotation) of the new q and k rows, and the
// bf16 K/V rows of this position. Waves 0 and 1 take the two query heads,
// wave 2 the key, wave 3 the value; `in` holds the q0|q1|k|v projections.
// nw*/c*/s* are raw bf16 bits prefetched by the caller (norm gains, RoPE row).
// The new K/V rows go to the cache when `cache_k` is non-null. Returns with
// the rows in LDS but without a barrier.
__device__ __forceinline__ void attn_qk_rope(AttnShared& at, const float* in, uint32_t nw0, uint32_t nw1,
                                             uint32_t c0, uint32_t s0, uint32_t c1, uint32_t s1,
                                             uint16_t* cache_k, uint16_t* cache_v, float* dbg_q, float* dbg_k,
                                             float* dbg_v, int wave, int lane) {
    if (wave < 3) {
        const float* src = in + wave * kHD;
        const double x0 = src[lane], x1 = src[lane + 64];
        const double ssq = wave_sum64(fma(x0, x0, x1 * x1));
        const double sc = rms_scale(ssq, kHD, kEps);
        const double y0 = x0 * sc * (double)after_wait_bf16(nw0);
        const double y1 = x1 * sc * (double)after_wait_bf16(nw1);
        const double cd0 = after_wait_bf16(c0), sd0 = after_wait_bf16(s0);
        const double cd1 = after_wait_bf16(c1), sd1 = after_wait_bf16(s1);
        const float o0 = (float)(y0 * cd0 - y1 * sd0);
        const float o1 = (float)(y0 * sd1 + y1 * cd1);
        if (wave < 2) {
            at.q[wave][lane] = o0;
            at.q[wave][lane + 64] = o1;
            if (dbg_q) { dbg_q[wave * kHD + lane] = o0; dbg_q[wave * kHD + lane + 64] = o1; }
        } else {
            const uint32_t b0 = f32_to_bf16_bits(o0), b1 = f32_to_bf16_bits(o1);
            if (cache_k) { cache_k[lane] = (uint16_t)b0; cache_k[lane + 64] = (uint16_t)b1; }
            uint16_t* row = reinterpret_cast<uint16_t*>(at.kv_cur[0]);
            row[lane] = (uint16_t)b0;
            row[lane + 64] = (uint16_t)b1;
            if (dbg_k) { dbg_k[lane] = o0; dbg_k[lane + 64] = o1; }
        }
    } else if (wave == 3) {
        const float v0 = in[3 * kHD + lane], v1 = in[3 * kHD + lane + 64];
        const uint32_t b0 = f32_to_bf16_bits(v0), b1 = f32_to_bf16_bits(v1);
        if (cache_v) { cache_v[lane] = (uint16_t)b0; cache_v[lane + 64] = (uint16_t)b1; }
        uint16_t* row = reinterpret_cast<uint16_t*>(at.kv_cur[1]);
        row[lane] = (uint16_t)b0;
        row[lane + 64] = (uint16_t)b1;
        if (dbg_v) { dbg_v[lane] = v0; dbg_v[lane + 64] = v1; }
    }
}

// K row words of position j: this position's row and the first kKvLds rows
// come from LDS, later ones from the cache (kh = the head's cache rows).
__device__ __forceinline__ const uint32_t* attn_k_row_lds(const AttnShared& at, int j, int pos) {
    return j == pos ? at.kv_cur[0] : at.kv_pre[0][j];
}

// Scores of both heads for all n positions with G lanes per position (each
// lane a 128/G-element slice of the head dim), scaled, into at.p; each wave's
// maxima, rounded to fp32, into at.wred[0..1] (the softmax only needs a value
// close to the maximum: exp(s - m) / sum exp(s - m) does not depend on m).
template <int G>
__device__ __forceinline__ void attn_scores(AttnShared& at, const uint16_t* kh, int n, int pos, double scale,
                                            int tid, int lane, int wave) {
    constexpr int EPL = kHD / G;            // elements per lane (a multiple of 8: 16-byte K loads)
    constexpr int P = kThreads / G;         // positions per pass
    static_assert(EPL % 8 == 0, "16-byte K slices");
    const int gi = tid % G;
    const double* q0 = at.q[0] + gi * EPL;
    const double* q1 = at.q[1] + gi * EPL;
    float m0 = -INFINITY, m1 = -INFINITY;
    for (int j0 = 0; j0 < n; j0 += P) {
        const int j = j0 + tid / G;
        double d0[2] = {0.0, 0.0}, d1[2] = {0.0, 0.0};
        if (j < n) {
            uint4 kw[EPL / 8];
            if (j == pos || j < kKvLds) {
                const uint4* kp = reinterpret_cast<const uint4*>(attn_k_row_lds(at, j, pos) + gi * (EPL / 2));
#pragma unroll
                for (int u = 0; u < EPL / 8; ++u) kw[u] = kp[u];
            } else {
                const uint16_t* kp = kh + (int64_t)j * kHD + gi * EPL;
#pragma unroll
                for (int u = 0; u < EPL / 8; ++u) kw[u] = ldg16(kp + 8 * u);
            }
#pragma unroll
            for (int u = 0; u < EPL / 8; ++u) {
                const uint32_t wv[4] = {kw[u].x, kw[u].y, kw[u].z, kw[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = u * 8 + 2 * e;
                    const double klo = __uint_as_float(wv[e] << 16);
                    const double khi = __uint_as_float(wv[e] & 0xffff0000u);
                    d0[e & 1] = fma(q0[k], klo, d0[e & 1]);
                    d0[e & 1] = fma(q0[k + 1], khi, d0[e & 1]);
                    d1[e & 1] = fma(q1[k], klo, d1[e & 1]);
                    d1[e & 1] = fma(q1[k + 1], khi, d1[e & 1]);
                }
            }
        }
        const double s0 = group_sum64<G>(d0[0] + d0[1]) * scale;
        const double s1 = group_sum64<G>(d1[0] + d1[1]) * scale;
        if (j < n) {
            if (gi == 0) { at.p[0][j] = s0; at.p[1][j] = s1; }
            m0 = fmaxf(m0, (float)s0);
            m1 = fmaxf(m1, (float)s1);
        }
    }
    m0 = wave_max(m0);
    m1 = wave_max(m1);
    if (lane == 0) { at.wred[0][wave] = m0; at.wred[1][wave] = m1; }
}

__device__ __forceinline__ double readlane64(double v, int l) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)u, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Scores, softmax and P @ V of both query heads over positions [0, n) (the
// current one, `pos`, from at.kv_cur). at.q / kv_cur / kv_pre must be written
// and visible (barrier) on entry. Calls emit(i, value) for output element
// i = head * 128 + dim on threads tid < 256, then returns without a barrier.
// mark(k) is called after sub-stage k (0 scores, 1 and 2 softmax with P @ V)
// for timing instrumentation.
template <class Emit, class Mark>
__device__ __forceinline__ void attn_core(AttnShared& at, const uint16_t* kh, const uint16_t* vh, int n, int pos,
                                          double scale, int tid, int lane, int wave, Emit emit, Mark mark) {
    // short contexts spread each position over more lanes
    if (n <= 32) attn_scores<16>(at, kh, n, pos, scale, tid, lane, wave);
    else if (n <= 64) attn_scores<8>(at, kh, n, pos, scale, tid, lane, wave);
    else attn_scores<4>(at, kh, n, pos, scale, tid, lane, wave);
    __syncthreads();
    mark(0);
    double M0 = at.wred[0][0], M1 = at.wred[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) { M0 = fmax(M0, at.wred[0][w]); M1 = fmax(M1, at.wred[1][w]); }
    // softmax numerators and P @ V. Wave w takes positions j = w + 8t: lane t
    // computes exp(s_j - m) for its t (64 positions per chunk) and the loop hands
    // the values to every lane with readlane; lane l accumulates dims 2l, 2l+1 of
    // both heads, and the probability sums ride along.
    {
        double a00 = 0.0, a01 = 0.0, a10 = 0.0, a11 = 0.0, l0 = 0.0, l1 = 0.0;
        for (int c0 = wave; c0 < n; c0 += kWaves * kWave) {
            const int jl = c0 + kWaves * lane;
            double p0 = 0.0, p1 = 0.0;
            if (jl < n) {
                p0 = exp(at.p[0][jl] - M0);
                p1 = exp(at.p[1][jl] - M1);
            }
            const int rem = (n - c0 + kWaves - 1) / kWaves;
            const int T = rem < kWave ? rem : kWave;
            for (int t = 0; t < T; ++t) {
                const int j = c0 + kWaves * t;
                const uint32_t vw = j == pos ? at.kv_cur[1][lane]
                                  : j < kKvLds ? at.kv_pre[1][j][lane]
                                               : *gview(reinterpret_cast<const uint32_t*>(vh + (int64_t)j * kHD + 2 * lane));
                const double q0 = readlane64(p0, t), q1 = readlane64(p1, t);
                const double v0 = __uint_as_float(vw << 16);
                const double v1 = __uint_as_float(vw & 0xffff0000u);
                a00 = fma(q0, v0, a00); a01 = fma(q0, v1, a01);
                a10 = fma(q1, v0, a10); a11 = fma(q1, v1, a11);
                l0 += q0;
                l1 += q1;
            }
        }
        at.pv[wave][2 * lane] = a00;
        at.pv[wave][2 * lane + 1] = a01;
        at.pv[wave][kHD + 2 * lane] = a10;
        at.pv[wave][kHD + 2 * lane + 1] = a11;
        if (lane == 0) { at.wred[2][wave] = l0; at.wred[3][wave] = l1; }
    }
    __syncthreads();
    mark(1);
    mark(2);
    if (tid < 2 * kHD) {
        const int h = tid / kHD;
        double o[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) o[w] = at.pv[w][tid];
#pragma unroll
        for (int s2 = kWaves / 2; s2 > 0; s2 /= 2)
#pragma unroll
            for (int w = 0; w < s2; ++w) o[w] += o[w + s2];
        emit(tid, (float)(o[0] * rcp_nr(tree_sum<kWaves>(at.wred[2 + h]))));
    }
}

}  // namespace mq
