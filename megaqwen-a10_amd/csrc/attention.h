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

// LDS working set. Split slices of at most NR positions (a multiple of 32)
// stage their K rows in kst.
template <int NR>
struct AttnShared {
    static constexpr int kNR = NR;
    double q[2][kHD];                      // rotated queries (fp32 values)
    uint16_t qb[8][kHD];                   // the same as bf16 triples: row 4h + p = part p of head h (row 4h + 3 zero)
    uint32_t kv_cur[2][kHD / 2];           // this position's K and V rows (bf16 pairs)
    double p[2][kMaxAttnLen];              // scores
    double wred[4][kWaves];                // per-wave score maxima, then probability sums (2 heads each)
    union {
        struct {
            uint32_t kv_pre[2][kKvLds][kHD / 2];   // K and V rows of the first kKvLds positions of the range
            double pv[kWaves][2 * kHD];            // per-wave partial P @ V
        };
        uint32_t kst[NR][kHD / 2];                 // K rows of a split slice (pv overlays it once read)
    };
};

// QK-RMSNorm and RoPE (split-half rotation) of the new q and k rows, and the
// bf16 K/V rows of this position. Waves 0 and 1 take the two query heads,
// wave 2 the key, wave 3 the value; `in` holds the q0|q1|k|v projections.
// nw*/c*/s* are raw bf16 bits prefetched by the caller (norm gains, RoPE row).
// The new K/V rows go to the cache when `cache_k` is non-null; with `triples`
// the queries also go to at.qb (for attn_scores_mfma). Returns with the rows
// in LDS but without a barrier.
template <class AS>
__device__ __forceinline__ void attn_qk_rope(AS& at, const float* in, uint32_t nw0, uint32_t nw1,
                                             uint32_t c0, uint32_t s0, uint32_t c1, uint32_t s1,
                                             uint16_t* cache_k, uint16_t* cache_v, float* dbg_q, float* dbg_k,
                                             float* dbg_v, int wave, int lane, bool triples = false) {
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
            if (triples) {
                // o = b0 + b1 + b2 exactly with bf16 b_p (each residual is exact
                // in fp32 and the last has at most 8 significant bits)
                float r0 = o0, r1 = o1;
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    const uint32_t u0 = f32_to_bf16_bits(r0), u1 = f32_to_bf16_bits(r1);
                    at.qb[4 * wave + p][lane] = (uint16_t)u0;
                    at.qb[4 * wave + p][lane + 64] = (uint16_t)u1;
                    r0 -= bf16_bits_to_f32(u0);
                    r1 -= bf16_bits_to_f32(u1);
                }
                at.qb[4 * wave + 3][lane] = 0;
                at.qb[4 * wave + 3][lane + 64] = 0;
            }
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

// K row words of position j of a range starting at j0: this position's row
// and the range's first kKvLds rows come from LDS.
template <class AS>
__device__ __forceinline__ const uint32_t* attn_k_row_lds(const AS& at, int j, int j0, int pos) {
    return j == pos ? at.kv_cur[0] : at.kv_pre[0][j - j0];
}

// Scores of both heads for positions [j0, j1) with G lanes per position (each
// lane a 128/G-element slice of the head dim), scaled, into at.p[h][j - j0]; each wave's
// maxima, rounded to fp32, into at.wred[0..1] (the softmax only needs a value
// close to the maximum: exp(s - m) / sum exp(s - m) does not depend on m).
template <int G, class AS>
__device__ __forceinline__ void attn_scores(AS& at, const uint16_t* kh, int j0, int j1, int pos,
                                            double scale, int tid, int lane, int wave) {
    constexpr int EPL = kHD / G;            // elements per lane (a multiple of 8: 16-byte K loads)
    constexpr int P = kThreads / G;         // positions per pass
    static_assert(EPL % 8 == 0, "16-byte K slices");
    const int gi = tid % G;
    const double* q0 = at.q[0] + gi * EPL;
    const double* q1 = at.q[1] + gi * EPL;
    float m0 = -INFINITY, m1 = -INFINITY;
    for (int jb = j0; jb < j1; jb += P) {
        const int j = jb + tid / G;
        double d0[2] = {0.0, 0.0}, d1[2] = {0.0, 0.0};
        if (j < j1) {
            uint4 kw[EPL / 8];
            if (j == pos || j - j0 < kKvLds) {
                const uint4* kp = reinterpret_cast<const uint4*>(attn_k_row_lds(at, j, j0, pos) + gi * (EPL / 2));
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
        if (j < j1) {
            if (gi == 0) { at.p[0][j - j0] = s0; at.p[1][j - j0] = s1; }
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

// Sums the per-wave P @ V accumulators (lane l: dims 2l, 2l+1 of both heads)
// and probability sums over the 8 waves and calls emit(i, acc, l, m) on
// threads tid < 256 (see attn_partial).
template <class AS, class Emit, class Mark>
__device__ __forceinline__ void attn_finish(AS& at, double a00, double a01, double a10, double a11,
                                            double l0, double l1, double M0, double M1, int tid, int lane,
                                            int wave, Emit emit, Mark mark) {
    at.pv[wave][2 * lane] = a00;
    at.pv[wave][2 * lane + 1] = a01;
    at.pv[wave][kHD + 2 * lane] = a10;
    at.pv[wave][kHD + 2 * lane + 1] = a11;
    if (lane == 0) { at.wred[2][wave] = l0; at.wred[3][wave] = l1; }
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
        emit(tid, o[0], tree_sum<kWaves>(at.wred[2 + h]), h == 0 ? M0 : M1);
    }
}

// Softmax-weighted sums of both query heads over positions [j0, j1) (the
// current one, `pos`, from at.kv_cur). at.q / kv_cur / kv_pre must be written
// and visible (barrier) on entry. With m_h the maximum score of head h over the
// range (rounded to fp32), calls emit(i, acc, l, m) on threads tid < 256 for
// output element i = h * 128 + dim: acc = sum_j e^(s_j - m_h) V_j[dim],
// l = sum_j e^(s_j - m_h). An empty range gives acc = l = 0, m = -inf.
// Returns without a barrier. mark(k) is called after sub-stage k (0 scores,
// 1 and 2 softmax with P @ V) for timing instrumentation.
template <bool kBatchTail = false, class AS, class Emit, class Mark>
__device__ __forceinline__ void attn_partial(AS& at, const uint16_t* kh, const uint16_t* vh, int j0, int j1,
                                             int pos, double scale, int tid, int lane, int wave, Emit emit, Mark mark) {
    const int n = j1 - j0;
    // short ranges spread each position over more lanes
    if (n <= 32) attn_scores<16>(at, kh, j0, j1, pos, scale, tid, lane, wave);
    else if (n <= 64) attn_scores<8>(at, kh, j0, j1, pos, scale, tid, lane, wave);
    else attn_scores<4>(at, kh, j0, j1, pos, scale, tid, lane, wave);
    __syncthreads();
    mark(0);
    double M0 = at.wred[0][0], M1 = at.wred[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) { M0 = fmax(M0, at.wred[0][w]); M1 = fmax(M1, at.wred[1][w]); }
    // softmax numerators and P @ V. Wave w takes local positions w + 8t: lane t
    // computes exp(s - m) for its t (64 positions per chunk) and the loop hands
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
            auto vword = [&](int t) -> uint32_t {
                const int j = j0 + c0 + kWaves * t;
                return j == pos ? at.kv_cur[1][lane]
                     : j - j0 < kKvLds ? at.kv_pre[1][j - j0][lane]
                                       : *gview(reinterpret_cast<const uint32_t*>(vh + (int64_t)j * kHD + 2 * lane));
            };
            auto accum = [&](uint32_t vw, int t) {
                const double q0 = readlane64(p0, t), q1 = readlane64(p1, t);
                const double v0 = __uint_as_float(vw << 16);
                const double v1 = __uint_as_float(vw & 0xffff0000u);
                a00 = fma(q0, v0, a00); a01 = fma(q0, v1, a01);
                a10 = fma(q1, v0, a10); a11 = fma(q1, v1, a11);
                l0 += q0;
                l1 += q1;
            };
            if constexpr (kBatchTail) {
                // positions past the kKvLds prefetched rows read their V word from memory: that
                // tail is loaded eight words at a time before use, one round trip per eight
                // positions instead of one per position (same accumulation order)
                const int T_lds = min(T, max(0, (kKvLds - c0 + kWaves - 1) / kWaves));
                for (int t = 0; t < T_lds; ++t) accum(vword(t), t);
                for (int t0 = T_lds; t0 < T; t0 += 8) {
                    uint32_t vw[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) vw[u] = t0 + u < T ? vword(t0 + u) : 0u;
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (t0 + u < T) accum(vw[u], t0 + u);
                }
            } else {
                for (int t = 0; t < T; ++t) accum(vword(t), t);
            }
        }
        attn_finish(at, a00, a01, a10, a11, l0, l1, M0, M1, tid, lane, wave, emit, mark);
    }
}

// ---- split slices of at most NR positions, loaded ahead of use ----
// Position of 16-byte chunk g of the K row at local index r in at.kst (an
// involution: also the chunk stored at position g).
__device__ __forceinline__ int kst_chunk(int g, int r) { return g ^ (r & 15); }

// The K rows go straight from HBM into at.kst (global_load_lds: no registers
// are held while they are in flight, so they can be issued a whole stage
// ahead); for P @ V, lane l of wave w holds the dims 2l, 2l+1 word of V at
// positions j0 + w + 8t.
template <int NR>
struct SliceRegs {
    uint32_t v[NR / kWaves];
};

// K rows of positions [j0, jend) (jend <= the current position, whose row
// comes from at.kv_cur) into at.kst[j - j0], the 16-byte chunks of row r
// permuted (chunk g at g ^ (r % 16), see kst_chunk) so that 16 rows read at the
// same head dims hit 16 different bank groups, issued by NW waves (wave < NW).
// Asynchronous: wait for the loads (vmcnt) and barrier before reading them.
// kAll: every wave issues all of its instructions (rows past jend repeat row
// jend - 1, into rows of at.kst past the slice), so that the number of loads in
// flight is fixed and later waits can count them.
template <int NW = kWaves, bool kAll = false, class AS>
__device__ __forceinline__ void attn_slice_k(AS& at, const uint16_t* kh, int j0, int jend, int lane, int wave) {
    constexpr int PW = AS::kNR / (4 * NW);         // instructions per wave
    static_assert(AS::kNR % (4 * NW) == 0, "whole instructions per wave");
    // wave w moves rows [4 PW w, 4 PW (w + 1)): 4 rows (1 KB) per instruction;
    // each lane's 16 bytes land at the instruction's base + 16 l, i.e. LDS chunk
    // l % 16 of row 4c + l / 16, so lane l fetches the row's chunk (l % 16) ^ r.
    // z (zero, hidden from the optimiser) keeps the per-instruction addresses
    // from being hoisted out of a caller's loop and held in (spilled) registers.
    const int z = opaque(0);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int c = wave * PW + i + z;
        const int r = 4 * c + lane / 16;
        const int j = kAll ? min(j0 + r, jend - 1) : j0 + r;
        if (kAll || (4 * c < jend - j0 && j < jend))
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)(kh + (int64_t)j * kHD + kst_chunk(lane % 16, r) * 8),
                (void __attribute__((address_space(3)))*)(&at.kst[4 * c][0]), 16, 0, 0);
    }
    issue_fence();      // issued here, not moved
}

// V words of positions [j0, jend) in the P @ V layout (jend > j0); the words of
// later positions repeat row jend - 1 (branch-free: attn_softmax_pv never uses them).
template <int NR>
__device__ __forceinline__ void attn_slice_v(SliceRegs<NR>& sr, const uint16_t* vh, int j0, int jend, int lane,
                                             int wave) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(vh) + lane;
#pragma unroll
    for (int t = 0; t < NR / kWaves; ++t) {
        const int j = min(j0 + wave + kWaves * t, jend - 1);
        sr.v[t] = *gview(base + (int64_t)j * (kHD / 2));
    }
    issue_fence();      // all loads issued here, not sunk to their uses
}

// V rows of positions [j0, jend) (jend <= the current position) into vs[j - j0],
// straight from HBM as attn_slice_k does for K, by NW waves (no chunk
// permutation: the P @ V loop reads one 4-byte word per lane of a row).
// Asynchronous, as attn_slice_k.
template <int NR, int NW = kWaves>
__device__ __forceinline__ void attn_slice_v_lds(uint32_t (*vs)[kHD / 2], const uint16_t* vh, int j0, int jend,
                                                 int lane, int wave) {
    constexpr int PW = NR / (4 * NW);
    static_assert(NR % (4 * NW) == 0, "whole instructions per wave");
    const int z = opaque(0);            // as in attn_slice_k
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int c = wave * PW + i + z;
        const int j = j0 + 4 * c + lane / 16;
        if (4 * c < jend - j0 && j < jend)
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)(vh + (int64_t)j * kHD + (lane % 16) * 8),
                (void __attribute__((address_space(3)))*)(&vs[4 * c][0]), 16, 0, 0);
    }
    issue_fence();
}

// Waits for this wave's outstanding vector memory operations (the LDS-direct
// loads above among them); a barrier must follow before other waves' rows
// are read.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Scores of both heads for the positions [j0, j1) of a split slice on the
// matrix cores: D = A B with A (16 x 128) the bf16 query triples (rows 4h + p)
// and B (128 x 16) the bf16 K rows of 16 positions, fp32 accumulation
// (v_mfma_f32_16x16x32_bf16, 4 per 16 positions; lane l holds A[l % 16][8 (l / 16) + e],
// B[8 (l / 16) + e][l % 16] and D[4 (l / 16) + i][l % 16]). The products are exact,
// so the score s_j = sum_p D[4h + p][j] carries only the fp32 accumulation
// error (|error| ~ 2^-24 sum_d |q_d k_d|). Writes at.p and the per-wave fp32
// maxima (at.wred[0..1]); no barrier.
template <class AS>
__device__ __forceinline__ void attn_scores_mfma(AS& at, int j0, int j1, int pos, double scale, int lane,
                                                 int wave) {
    const int n = j1 - j0;
    const int m = lane % 16, kq = lane / 16;
    bf16x8_t a[kHD / 32];
#pragma unroll
    for (int kb = 0; kb < kHD / 32; ++kb) {
        if (m < 8) a[kb] = *reinterpret_cast<const bf16x8_t*>(&at.qb[m][kb * 32 + 8 * kq]);
        else a[kb] = bf16x8_t{};
    }
    float m0 = -INFINITY, m1 = -INFINITY;
    const int tiles = (n + 15) / 16;
    for (int t = wave; t < tiles; t += kWaves) {
        const int jl = 16 * t + m;                 // this lane's B column (local position)
        const bool cur = (j0 + jl == pos);
        const uint4* row = reinterpret_cast<const uint4*>(cur ? at.kv_cur[0] : at.kst[jl]);
        f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < kHD / 32; ++kb) {
            const int g = 4 * kb + kq;             // 16-byte chunk of the row
            const uint4 w = row[cur ? g : kst_chunk(g, jl)];
            bf16x8_t b;
            __builtin_memcpy(&b, &w, 16);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kb], b, c, 0, 0, 0);
        }
        if (kq < 2 && jl < n) {
            const double sv = (((double)c[0] + (double)c[1]) + (double)c[2]) * scale;
            at.p[kq][jl] = sv;
            if (kq == 0) m0 = fmaxf(m0, (float)sv);
            else m1 = fmaxf(m1, (float)sv);
        }
    }
    m0 = wave_max(m0);
    m1 = wave_max(m1);
    if (lane == 0) { at.wred[0][wave] = m0; at.wred[1][wave] = m1; }
}

// Softmax and P @ V of a split slice of n <= TV * 8 positions after
// attn_scores_mfma (and a barrier): wave w takes local positions w + 8t, lane t
// computing exp(s - m) for its t and readlane handing it to every lane; vword(t)
// is lane l's V word (dims 2l, 2l+1) of local position w + 8t, the current
// position's coming from at.kv_cur. The probability sums are wave sums of the
// lanes' own values. Then attn_finish. With kFastExp (for paths checked to a
// tolerance) the numerators are the hardware fp32 2^x of (s - m) log2(e)
// (relative error about 2^-23) instead of the fp64 exp, and the products and
// sums are fp32 (fixed order) instead of fp64.
// kGroups (fp64 path): the P @ V loop tests its bound once per group of 8 slots, for
// callers whose vword(t) is a finite V word for every t < TV (slots past the wave's
// positions carry numerator 0, so they add exact zeros).
template <int TV, bool kFastExp = false, bool kGroups = false, class AS, class VWord, class Emit, class Mark>
__device__ __forceinline__ void attn_softmax_pv(AS& at, VWord vword, int j0, int n, int pos, int tid, int lane,
                                                int wave, Emit emit, Mark mark) {
    static_assert(TV <= kWave, "one P @ V chunk");
    double M0 = at.wred[0][0], M1 = at.wred[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) { M0 = fmax(M0, at.wred[0][w]); M1 = fmax(M1, at.wred[1][w]); }
    const int jl = wave + kWaves * lane;
    // wave-uniform bounds (scalar branches below)
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int T = __builtin_amdgcn_readfirstlane(n > wu ? (n - wu + kWaves - 1) / kWaves : 0);
    const int tc = __builtin_amdgcn_readfirstlane(pos - j0 - wu);   // t of the current position, if this wave has it
    if constexpr (kFastExp) {
        // fp32 numerators, products and sums (fixed order)
        constexpr double kLog2e = 1.4426950408889634;
        float p0 = 0.0f, p1 = 0.0f;
        if (lane < TV && jl < n) {
            p0 = __builtin_amdgcn_exp2f((float)((at.p[0][jl] - M0) * kLog2e));
            p1 = __builtin_amdgcn_exp2f((float)((at.p[1][jl] - M1) * kLog2e));
        }
        float a00 = 0.0f, a01 = 0.0f, a10 = 0.0f, a11 = 0.0f;
#pragma unroll
        for (int t = 0; t < TV; ++t) {
            if (t < T) {
                const uint32_t vw = t * kWaves == tc ? at.kv_cur[1][lane] : vword(t);
                const float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p0), t));
                const float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p1), t));
                const float v0 = __uint_as_float(vw << 16);
                const float v1 = __uint_as_float(vw & 0xffff0000u);
                a00 = fmaf(r0, v0, a00); a01 = fmaf(r0, v1, a01);
                a10 = fmaf(r1, v0, a10); a11 = fmaf(r1, v1, a11);
            }
        }
        attn_finish(at, (double)a00, (double)a01, (double)a10, (double)a11, (double)wave_sum(p0),
                    (double)wave_sum(p1), M0, M1, tid, lane, wave, emit, mark);
    } else {
        double p0 = 0.0, p1 = 0.0;
        if (lane < TV && jl < n) {
            p0 = exp(at.p[0][jl] - M0);
            p1 = exp(at.p[1][jl] - M1);
        }
        double a00 = 0.0, a01 = 0.0, a10 = 0.0, a11 = 0.0;
        // this position's V word, read once (selected per slot without a branch or an LDS read)
        const uint32_t vcur = at.kv_cur[1][lane];
        auto slot = [&](int t) {
            const uint32_t vw = t * kWaves == tc ? vcur : vword(t);
            const double r0 = readlane64(p0, t), r1 = readlane64(p1, t);
            const double v0 = __uint_as_float(vw << 16);
            const double v1 = __uint_as_float(vw & 0xffff0000u);
            a00 = fma(r0, v0, a00); a01 = fma(r0, v1, a01);
            a10 = fma(r1, v0, a10); a11 = fma(r1, v1, a11);
        };
        if constexpr (kGroups) {
#pragma unroll
            for (int tb = 0; tb < TV; tb += 8) {
                if (tb < T) {
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (tb + u < TV) slot(tb + u);
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < TV; ++t)
                if (t < T) slot(t);
        }
        attn_finish(at, a00, a01, a10, a11, wave_sum64(p0), wave_sum64(p1), M0, M1, tid, lane, wave, emit, mark);
    }
}

// attn_partial for a range [j0, j1) of at most NR positions whose K rows and
// V words were loaded by attn_slice_k / attn_slice_v (and waited for, with a
// barrier): scores on the matrix cores, softmax and P @ V in fp64.
template <class AS, int NR, class Emit, class Mark>
__device__ __forceinline__ void attn_partial_regs(AS& at, const SliceRegs<NR>& sr, int j0, int j1, int pos,
                                                  double scale, int tid, int lane, int wave, Emit emit, Mark mark) {
    static_assert(NR == AS::kNR && NR % 16 == 0, "slice capacity");
    attn_scores_mfma(at, j0, j1, pos, scale, lane, wave);
    __syncthreads();
    mark(0);
    attn_softmax_pv<NR / kWaves, false, true>(at, [&](int t) { return sr.v[t]; }, j0, j1 - j0, pos, tid, lane, wave,
                                              emit, mark);
}

// attn_partial for a range [j0, j1) of at most kKvLds positions whose K rows
// are in at.kst (chunks permuted as by kst_chunk) and V rows in at.kv_pre[1]
// (staged from registers loaded during the previous layer).
template <class AS, class Emit, class Mark>
__device__ __forceinline__ void attn_partial_lds(AS& at, int j0, int j1, int pos, double scale, int tid, int lane,
                                                 int wave, Emit emit, Mark mark) {
    static_assert(AS::kNR >= kKvLds, "staging rows");
    attn_scores_mfma(at, j0, j1, pos, scale, lane, wave);
    __syncthreads();
    mark(0);
    attn_softmax_pv<kKvLds / kWaves>(at, [&](int t) { return at.kv_pre[1][wave + kWaves * t][lane]; }, j0, j1 - j0,
                                     pos, tid, lane, wave, emit, mark);
}

// attn_partial for a range [j0, j1) of at most NR positions whose K rows are in
// at.kst (attn_slice_k) and V rows in vs (attn_slice_v_lds), waited for with a
// barrier: scores on the matrix cores, softmax and P @ V in fp64 (numerators as
// attn_softmax_pv's kFastExp says).
template <class AS, int NR, bool kFastExp = false, class Emit, class Mark>
__device__ __forceinline__ void attn_partial_lds_v(AS& at, const uint32_t (*vs)[kHD / 2], int j0, int j1, int pos,
                                                   double scale, int tid, int lane, int wave, Emit emit, Mark mark) {
    static_assert(NR <= AS::kNR && NR % 16 == 0, "slice capacity");
    attn_scores_mfma(at, j0, j1, pos, scale, lane, wave);
    __syncthreads();
    mark(0);
    attn_softmax_pv<NR / kWaves, kFastExp>(at, [&](int t) { return vs[wave + kWaves * t][lane]; }, j0, j1 - j0,
                                           pos, tid, lane, wave, emit, mark);
}

// Attention output of both query heads over positions [0, n) in one workgroup:
// calls emit(i, value) with the fp32 output element i = h * 128 + dim on
// threads tid < 256, then returns without a barrier.
template <bool kBatchTail = false, class AS, class Emit, class Mark>
__device__ __forceinline__ void attn_core(AS& at, const uint16_t* kh, const uint16_t* vh, int n, int pos,
                                          double scale, int tid, int lane, int wave, Emit emit, Mark mark) {
    attn_partial<kBatchTail>(at, kh, vh, 0, n, pos, scale, tid, lane, wave,
                 [&](int i, double acc, double l, double) { emit(i, (float)(acc * rcp_nr(l))); }, mark);
}

}  // namespace mq
