// Persistent batch-1 decode step for Qwen3-shaped models on gfx950.
//
// Computes what a10_int8_decode_kernel.cu:21-815 computes (and, with bf16
// weights and unit scales, a10_decode_kernel.cu:21-755): embedding, L layers of
// [RMSNorm + QKV, QK-norm + RoPE + bf16 KV write, GQA attention, O + residual,
// RMSNorm + gate/up + SwiGLU, down + residual -> bf16], final RMSNorm, LM head
// and greedy argmax — in ONE launch of 256 workgroups x 512 threads.
//
// Work split (per workgroup g, 0 <= g < 256):
//   QKV      rows [16g, 16g+16) of the concatenated q|k|v projection
//   ATTN     workgroups 0..7: KV head g with its two query heads
//   O, DOWN  rows [H/256*g, +H/256) of o_proj and down_proj
//   GATE/UP  channels [I/256*g, +I/256) of gate_proj and up_proj
//   LM HEAD  rows [V*g/256, V*(g+1)/256)
// Every workgroup recomputes the RMSNorms it needs from the full vector, so no
// stage waits for a single "norm" workgroup.
//
// Stages hand vectors to each other through 64-bit words (32-bit value +
// 32-bit tag naming step/layer/stage) written with one relaxed agent-scope
// atomic store and polled with relaxed agent-scope atomic loads (common.h).
// A consumer therefore waits exactly for the words it reads; there is no
// separate grid barrier and no cache write-back/invalidate. Each stage issues
// its own weight loads (registers) before polling its input, so weight-fetch
// latency overlaps the wait for the producers.
//
// The workspace (internal.h: WsHeader + exchange buffers) carries the step
// counter; the last workgroup to finish the LM head publishes the token and
// advances it.
#include "attention.h"

#include <hip/hip_ext.h>

#include <atomic>

#include <algorithm>
#include <climits>

namespace mq {

template <int H, int I, class W, bool kDebug>
__global__ void __launch_bounds__(kThreads, 1) decode_kernel(KArgs a) {
    constexpr int NQ = 16, NKV = 8, D = 128;
    constexpr Layout kLay = layout_for(H, I, NQ, NKV, D);
    constexpr int QD = NQ * D, KVD = NKV * D, QKV = QD + 2 * KVD;
    constexpr int ES = W::kBytes;
    constexpr bool kInt8 = (ES == 1);
    constexpr int ROWS_QKV = QKV / kNWG;
    constexpr int ROWS_H = H / kNWG;
    constexpr int CPW = I / kNWG;
    constexpr int PT = H / kThreads;                  // hidden elements per thread
    constexpr int XMAX = (H > QD ? (H > I ? H : I) : (QD > I ? QD : I));
    static_assert(QKV % kNWG == 0 && H % kNWG == 0 && I % kNWG == 0, "rows must split evenly");
    static_assert(H % kThreads == 0 && QD % kThreads == 0 && I % kThreads == 0, "vectors must split evenly");
    static_assert(ROWS_QKV <= kThreads && CPW <= kThreads, "epilogue threads");
    static_assert(Stage_<W, ROWS_QKV, H>::ITEMS <= 256 && Stage_<W, 2 * CPW, H>::ITEMS <= 256 &&
                  Stage_<W, ROWS_H, QD>::ITEMS <= 256 && Stage_<W, ROWS_H, I>::ITEMS <= 256, "partials fit");

    __shared__ double2 xd[XMAX / 2];                   // fp64 matvec input in per-lane order
    __shared__ float4 xs[H / 4];                       // fp32 LM-head input in per-lane order
    __shared__ double part[256];
    __shared__ double red[2 * kWaves];
    __shared__ float rows_res[ROWS_H];
    __shared__ float att_in[4 * D];
    __shared__ __align__(16) AttnShared<128> at;   // never splits: kst stays inside the kv_pre/pv union
    __shared__ float lm_best_v[kWaves];
    __shared__ int lm_best_i[kWaves];
    __shared__ LayerWeights s_lw[kMaxLayers];
    __shared__ ScalePointers s_sp[kMaxLayers];

    const int g = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    float* xsf = reinterpret_cast<float*>(xs);
    double* xdf = reinterpret_cast<double*>(xd);

    // step-independent reads first: the embedding row and the per-layer pointer tables
    float hv0[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) hv0[i] = bf16_bits_to_f32(gview(a.embed)[(int64_t)a.token * H + tid + i * kThreads]);
    {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.lw);
        uint64_t* dst = reinterpret_cast<uint64_t*>(s_lw);
        for (int i = tid; i < a.L * 11; i += kThreads) dst[i] = src[i];
        if (kInt8) {
            const uint64_t* ssrc = reinterpret_cast<const uint64_t*>(a.sp);
            uint64_t* sdst = reinterpret_cast<uint64_t*>(s_sp);
            for (int i = tid; i < a.L * 7; i += kThreads) sdst[i] = ssrc[i];
        }
    }

    WsHeader* hdr = reinterpret_cast<WsHeader*>(a.ws);
    uint64_t* const hid_x = reinterpret_cast<uint64_t*>(a.ws + kLay.hid);
    uint64_t* const qkv_x = reinterpret_cast<uint64_t*>(a.ws + kLay.qkv);
    uint64_t* const att_x = reinterpret_cast<uint64_t*>(a.ws + kLay.att);
    uint64_t* const act_x = reinterpret_cast<uint64_t*>(a.ws + kLay.act);
    uint64_t* const mlp_x = reinterpret_cast<uint64_t*>(a.ws + kLay.mlp);
    const uint32_t E = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (g == 0 && tid == 0) {
        __hip_atomic_store(&hdr->done[(E + 1) & 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&hdr->best[(E + 1) & 1], (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t tps = 5u * (uint32_t)a.L + 4u;
    // tags end in binary 01 (the XCD-aware kernel's end in 11): no overlap when the
    // two kernels share a workspace
    auto tag = [&](int l, int st) -> uint32_t { return ((E * tps + 5u * (uint32_t)l + (uint32_t)st) << 2) | 1u; };
    Waiter wt(&hdr->abort_flag, a.spin_limit);
    auto trace = [&](int l, int point) {
        if (kDebug && a.trace != nullptr && tid == 0)
            a.trace[((int64_t)l * kTracePoints + point) * kNWG + g] = __builtin_amdgcn_s_memrealtime();
    };

    const int64_t kv_head_stride = (int64_t)a.S * D;
    const int last = a.L - 1;
    const double attn_scale = (double)a.attn_scale;
    __syncthreads();

    const int tid_all = tid;
    for (int l = 0; l < a.L; ++l) {
        const LayerWeights& lw = s_lw[l];
        const ScalePointers& sp = s_sp[l];
        const int tid = opaque(tid_all);
        const int lane = tid % kWave;

        // ---------------- RMSNorm + QKV ----------------
        {
            const int row0 = g * ROWS_QKV;
            const uint8_t* base;
            const float* sc = nullptr;
            int lrow0;
            if (row0 < QD) { base = (const uint8_t*)lw.q_proj_weight; lrow0 = row0; if (kInt8) sc = sp.q_scale; }
            else if (row0 < QD + KVD) { base = (const uint8_t*)lw.k_proj_weight; lrow0 = row0 - QD; if (kInt8) sc = sp.k_scale; }
            else { base = (const uint8_t*)lw.v_proj_weight; lrow0 = row0 - QD - KVD; if (kInt8) sc = sp.v_scale; }
            Stage_<W, ROWS_QKV, H> st;
            st.load([&](int r) { return base + (int64_t)(lrow0 + r) * H * ES; }, wave, lane);
            uint32_t my_scale = 0x3f800000u;            // prefetched raw bits (after_wait at use)
            if (kInt8 && tid < ROWS_QKV) my_scale = ldg_bits(sc + lrow0 + tid);
            const uint16_t* lnw = (const uint16_t*)lw.input_layernorm_weight;
            uint32_t wln[PT];
#pragma unroll
            for (int i = 0; i < PT; ++i) wln[i] = ldg_bits(lnw + tid + i * kThreads);
            issue_fence();

            float hv[PT];
            if (l == 0) {
#pragma unroll
                for (int i = 0; i < PT; ++i) hv[i] = hv0[i];
            } else {
                wt.get_strided<PT>(hid_x + tid, kThreads, tag(l - 1, ST_DOWN), hv);
            }
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < PT; ++i) ss = fma((double)hv[i], (double)hv[i], ss);
            const double tot = block_sum64<kWaves>(ss, red, 0, wave, lane);
            trace(l, 0);
            const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const int k = tid + i * kThreads;
                xdf[xd_index<W>(k)] = (double)(float)((double)hv[i] * rstd * (double)after_wait_bf16(wln[i]));
                const int rr = k - g * ROWS_H;
                if (rr >= 0 && rr < ROWS_H) rows_res[rr] = hv[i];
            }
            __syncthreads();
            st.compute(xd, part, wave, lane);
            __syncthreads();
            if (tid < ROWS_QKV) {
                double v = Stage_<W, ROWS_QKV, H>::row_sum(part, tid);
                if (kInt8) v = v * (double)after_wait_f(my_scale);
                ll_put(&qkv_x[row0 + tid], __float_as_uint((float)v), tag(l, ST_QKV));
            }
            trace(l, 1);
        }

        // ---------------- QK-norm + RoPE + KV write + attention (KV head g) ----------------
        if (g < NKV) {
            const int h = g;
            const int n = a.cache_len;
            const int64_t cache_base = ((int64_t)l * NKV + h) * kv_head_stride;
            const int64_t cur = cache_base + (int64_t)a.pos * D;
            // step-independent inputs: norm gains, the RoPE row, and the K/V rows of
            // earlier positions (up to kKvLds of them) staged through registers
            uint32_t nw0 = 0, nw1 = 0, c0 = 0, s0 = 0, c1 = 0, s1 = 0;
            if (wave < 3) {
                const uint16_t* nw = (const uint16_t*)(wave < 2 ? lw.q_norm_weight : lw.k_norm_weight);
                nw0 = ldg_bits(nw + lane);
                nw1 = ldg_bits(nw + lane + 64);
                const uint16_t* ct = a.cos_t + (int64_t)a.pos * D;
                const uint16_t* stt = a.sin_t + (int64_t)a.pos * D;
                c0 = ldg_bits(ct + lane);
                s0 = ldg_bits(stt + lane);
                c1 = ldg_bits(ct + lane + 64);
                s1 = ldg_bits(stt + lane + 64);
            }
            const int npre = a.pos < kKvLds ? a.pos : kKvLds;   // earlier positions held in LDS
            constexpr int kPreU4 = 2 * kKvLds * (D / 8) / kThreads;
            uint4 pre[kPreU4];
#pragma unroll
            for (int i = 0; i < kPreU4; ++i) {
                const int f = tid + i * kThreads;                 // 16-byte unit: side, position, column
                const int side = f / (kKvLds * (D / 8));
                const int rem = f % (kKvLds * (D / 8));
                const int j = rem / (D / 8), c = rem % (D / 8);
                pre[i] = make_uint4(0, 0, 0, 0);
                if (j < npre) {
                    const uint16_t* src = (side == 0 ? a.kc : a.vc) + cache_base + (int64_t)j * D + c * 8;
                    pre[i] = ldg16(src);
                }
            }
            issue_fence();
            {
                int word;
                if (tid < 2 * D) word = 2 * h * D + tid;
                else if (tid < 3 * D) word = QD + h * D + (tid - 2 * D);
                else word = QD + KVD + h * D + (tid - 3 * D);
                float v1[1];
                wt.get_strided<1>(qkv_x + word, 0, tag(l, ST_QKV), v1);
                att_in[tid] = v1[0];
            }
#pragma unroll
            for (int i = 0; i < kPreU4; ++i) {
                const int f = tid + i * kThreads;
                const int side = f / (kKvLds * (D / 8));
                const int rem = f % (kKvLds * (D / 8));
                const int j = rem / (D / 8), c = rem % (D / 8);
                if (j < npre) *reinterpret_cast<uint4*>(&at.kv_pre[side][j][c * 4]) = pre[i];
            }
            __syncthreads();
            trace(l, 2);
            const bool dbg = kDebug && l == last;
            attn_qk_rope(at, att_in, nw0, nw1, c0, s0, c1, s1, a.kc + cur, a.vc + cur,
                         (dbg && a.dbg_q) ? a.dbg_q + 2 * h * D : nullptr, (dbg && a.dbg_k) ? a.dbg_k + h * D : nullptr,
                         (dbg && a.dbg_v) ? a.dbg_v + h * D : nullptr, wave, lane);
            __syncthreads();
            attn_core(at, a.kc + cache_base, a.vc + cache_base, n, a.pos, attn_scale, tid, lane, wave,
                      [&](int i, float v) {
                          const int word = 2 * h * D + i;
                          ll_put(&att_x[word], __float_as_uint(v), tag(l, ST_ATTN));
                          if (dbg && a.dbg_attn) a.dbg_attn[word] = v;
                      },
                      [](int) {});
            trace(l, 3);
        }

        // ---------------- O projection + residual ----------------
        {
            const int row0 = g * ROWS_H;
            const uint8_t* base = (const uint8_t*)lw.o_proj_weight;
            Stage_<W, ROWS_H, QD> st;
            st.load([&](int r) { return base + (int64_t)(row0 + r) * QD * ES; }, wave, lane);
            uint32_t my_scale = 0x3f800000u;
            if (kInt8 && tid < ROWS_H) my_scale = ldg_bits(sp.o_scale + row0 + tid);
            issue_fence();
            {
                float v[QD / kThreads];
                wt.get_strided<QD / kThreads>(att_x + tid, kThreads, tag(l, ST_ATTN), v);
#pragma unroll
                for (int i = 0; i < QD / kThreads; ++i) xdf[xd_index<W>(tid + i * kThreads)] = v[i];
            }
            __syncthreads();
            trace(l, 4);
            st.compute(xd, part, wave, lane);
            __syncthreads();
            if (tid < ROWS_H) {
                double v = Stage_<W, ROWS_H, QD>::row_sum(part, tid);
                if (kInt8) v = v * (double)after_wait_f(my_scale);
                const float x = (float)(v + (double)rows_res[tid]);
                ll_put(&act_x[row0 + tid], __float_as_uint(x), tag(l, ST_O));
            }
            trace(l, 5);
        }

        // ---------------- RMSNorm + gate/up + SwiGLU ----------------
        {
            const int c0 = g * CPW;
            const uint8_t* gb = (const uint8_t*)lw.gate_proj_weight;
            const uint8_t* ub = (const uint8_t*)lw.up_proj_weight;
            Stage_<W, 2 * CPW, H> st;
            st.load([&](int r) {
                return r < CPW ? gb + (int64_t)(c0 + r) * H * ES : ub + (int64_t)(c0 + r - CPW) * H * ES;
            }, wave, lane);
            uint32_t gsc = 0x3f800000u, usc = 0x3f800000u;
            if (kInt8 && tid < CPW) { gsc = ldg_bits(sp.gate_scale + c0 + tid); usc = ldg_bits(sp.up_scale + c0 + tid); }
            const uint16_t* pnw = (const uint16_t*)lw.post_attn_layernorm_weight;
            uint32_t wpn[PT];
#pragma unroll
            for (int i = 0; i < PT; ++i) wpn[i] = ldg_bits(pnw + tid + i * kThreads);
            issue_fence();
            float av[PT];
            wt.get_strided<PT>(act_x + tid, kThreads, tag(l, ST_O), av);
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < PT; ++i) ss = fma((double)av[i], (double)av[i], ss);
            const double tot = block_sum64<kWaves>(ss, red, 1, wave, lane);
            trace(l, 6);
            const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const int k = tid + i * kThreads;
                const float nv = (float)((double)av[i] * rstd * (double)after_wait_bf16(wpn[i]));
                xdf[xd_index<W>(k)] = nv;
                const int rr = k - g * ROWS_H;
                if (rr >= 0 && rr < ROWS_H) rows_res[rr] = av[i];
                if (kDebug && l == last && g == 0) {
                    if (a.dbg_act) a.dbg_act[k] = nv;
                    if (a.dbg_resid) a.dbg_resid[k] = av[i];
                }
            }
            __syncthreads();
            st.compute(xd, part, wave, lane);
            __syncthreads();
            if (tid < CPW) {
                double gs = Stage_<W, 2 * CPW, H>::row_sum(part, tid);
                double us = Stage_<W, 2 * CPW, H>::row_sum(part, CPW + tid);
                if (kInt8) { gs = gs * (double)after_wait_f(gsc); us = us * (double)after_wait_f(usc); }
                const float m = (float)silu_mul(gs, us);
                ll_put(&mlp_x[c0 + tid], __float_as_uint(m), tag(l, ST_GU));
                if (l == last && kDebug && a.dbg_mlp) a.dbg_mlp[c0 + tid] = m;
            }
            trace(l, 7);
        }

        // ---------------- down projection + residual -> bf16 hidden ----------------
        {
            const int row0 = g * ROWS_H;
            const uint8_t* base = (const uint8_t*)lw.down_proj_weight;
            Stage_<W, ROWS_H, I> st;
            st.load([&](int r) { return base + (int64_t)(row0 + r) * I * ES; }, wave, lane);
            uint32_t my_scale = 0x3f800000u;
            if (kInt8 && tid < ROWS_H) my_scale = ldg_bits(sp.down_scale + row0 + tid);
            issue_fence();
            {
                float v[I / kThreads];
                wt.get_strided<I / kThreads>(mlp_x + tid, kThreads, tag(l, ST_GU), v);
#pragma unroll
                for (int i = 0; i < I / kThreads; ++i) xdf[xd_index<W>(tid + i * kThreads)] = v[i];
            }
            __syncthreads();
            trace(l, 8);
            st.compute(xd, part, wave, lane);
            __syncthreads();
            if (tid < ROWS_H) {
                double v = Stage_<W, ROWS_H, I>::row_sum(part, tid);
                if (kInt8) v = v * (double)after_wait_f(my_scale);
                const uint32_t hb = f32_to_bf16_bits((float)(v + (double)rows_res[tid]));
                ll_put(&hid_x[row0 + tid], __float_as_uint(bf16_bits_to_f32(hb)), tag(l, ST_DOWN));
                if (l == last && kDebug && a.dbg_hidden) a.dbg_hidden[row0 + tid] = (uint16_t)hb;
            }
            trace(l, 9);
        }
    }

    // ---------------- final RMSNorm + LM head + greedy argmax ----------------
    {
        constexpr int CH = H / (64 * W::kPerLane);
        constexpr int RB = CH >= 8 ? 1 : 8 / CH;          // rows per wave batch
        constexpr int R = RB * CH;                         // 1 KB items per batch
        constexpr int span = kWave / RB;
        const int r0 = (int)((int64_t)a.V * g / kNWG);
        const int r1 = (int)((int64_t)a.V * (g + 1) / kNWG);
        const int nb = (r1 - r0 + RB - 1) / RB;
        const int64_t rowbytes = (int64_t)H * ES;

        uint4 cur[R], nxt[R];
        float scur = 0.0f, snxt = 0.0f;
        auto fetch = [&](int b, uint4* dst, float& s) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int row = r0 + b * RB + i / CH;
                dst[i] = make_uint4(0, 0, 0, 0);
                if (row < r1) dst[i] = ldg16(a.lm_w + row * rowbytes + (i % CH) * 1024 + lane * 16);
            }
            const int myrow = r0 + b * RB + lane / span;
            s = 1.0f;
            if (kInt8 && myrow < r1) s = gview(a.lm_s)[myrow];
        };
        // the first LM-head batch and the final norm gains do not depend on this step
        int b = wave;
        if (b < nb) fetch(b, cur, scur);
        uint32_t wfn[PT];
#pragma unroll
        for (int i = 0; i < PT; ++i) wfn[i] = ldg_bits(a.final_norm + tid + i * kThreads);
        issue_fence();

        float hv[PT];
        wt.get_strided<PT>(hid_x + tid, kThreads, tag(last, ST_DOWN), hv);
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < PT; ++i) ss = fma((double)hv[i], (double)hv[i], ss);
        const double tot = block_sum64<kWaves>(ss, red, 0, wave, lane);
        trace(a.L, 0);
        const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int k = tid + i * kThreads;
            const float nv = (float)((double)hv[i] * rstd * (double)after_wait_bf16(wfn[i]));
            xsf[xs_index<W>(k)] = nv;
            if (g == 0 && kDebug && a.dbg_norm) a.dbg_norm[k] = nv;
        }
        __syncthreads();

        float best_v = -INFINITY;
        int best_i = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < R; ++i) nxt[i] = make_uint4(0, 0, 0, 0);
        for (; b < nb; b += kWaves) {
            if (b + kWaves < nb) fetch(b + kWaves, nxt, snxt);
            float acc[R];
#pragma unroll
            for (int i = 0; i < R; ++i) acc[i] = dot_frag<W>(cur[i], xs_frag<W>(xs, i % CH, lane), 0.0f);
            const float s = transpose_reduce<R, CH>(acc, lane);
            const int row = r0 + b * RB + lane / span;
            if ((lane % span) == 0 && row < r1) {
                float v = kInt8 ? s * scur : s;
                // sampling: the Gumbel-max rule (see gumbel_noise)
                if (a.inv_temp > 0.0f) v = v * a.inv_temp + gumbel_noise(a.seed, a.pos, row);
                if (v > best_v) { best_v = v; best_i = row; }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) cur[i] = nxt[i];
            scur = snxt;
        }
        // wave argmax, ties to the lower index
#define MQ_ARGMAX_LEVEL(M)                                                                   \
        {                                                                                    \
            const float ov = partner<M>(best_v);                                             \
            const int oi = __float_as_int(partner<M>(__int_as_float(best_i)));               \
            if (ov > best_v || (ov == best_v && oi < best_i)) { best_v = ov; best_i = oi; }  \
        }
        MQ_ARGMAX_LEVEL(1) MQ_ARGMAX_LEVEL(2) MQ_ARGMAX_LEVEL(4) MQ_ARGMAX_LEVEL(8)
        MQ_ARGMAX_LEVEL(16) MQ_ARGMAX_LEVEL(32)
#undef MQ_ARGMAX_LEVEL
        if (lane == 0) { lm_best_v[wave] = best_v; lm_best_i[wave] = best_i; }
        __syncthreads();
        trace(a.L, 1);
        if (tid == 0) {
            float bv = lm_best_v[0];
            int bi = lm_best_i[0];
            for (int w = 1; w < kWaves; ++w) {
                if (lm_best_v[w] > bv || (lm_best_v[w] == bv && lm_best_i[w] < bi)) { bv = lm_best_v[w]; bi = lm_best_i[w]; }
            }
            if (kDebug && a.dbg_bmax) a.dbg_bmax[g] = bv;
            if (kDebug && a.dbg_bidx) a.dbg_bidx[g] = bi;
            const uint64_t key = ((uint64_t)ordered_key(bv) << 32) | (uint64_t)(~(uint32_t)bi);
            const int slot = E & 1;
            __hip_atomic_fetch_max(&hdr->best[slot], key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t prev = __hip_atomic_fetch_add(&hdr->done[slot], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if (prev == gridDim.x - 1) {
                const uint64_t k = __hip_atomic_load(&hdr->best[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint32_t flag = __hip_atomic_load(&hdr->abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *a.out_token = flag != 0u ? -1 : (int)(~(uint32_t)(k & 0xffffffffu));
                if (a.status_out) *a.status_out = flag;
                __hip_atomic_store(&hdr->epoch, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (kDebug && a.trace != nullptr) a.trace[((int64_t)a.L * kTracePoints + 2) * kNWG] = __builtin_amdgcn_s_memrealtime();
            }
        }
    }
}

// ---------------- host side ----------------

size_t decode_workspace_bytes(const DecodeShape& s) {
    const size_t a = layout_for(s.H, s.I, s.NQ, s.NKV, s.D).total, b = decode_xcd_workspace_bytes(s);
    const size_t c = decode_async_workspace_bytes(s);      // follows the other two regions (0 if unsupported)
    return std::max(std::max(a, b), c);
}

// ---- kernel variant selection ----
// XCD of each workgroup of the placement check (a device array: the check allocates nothing)
static __device__ uint32_t g_xcc_map[kNWG];

__global__ void xcc_map_kernel(uint32_t* out) {
    if (threadIdx.x == 0) {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = v & 0xfu;
    }
}

static std::atomic<int> g_variant{0};
static std::atomic<int> g_xcd_ok[64];     // 0 unknown, 1 placement verified, 2 not usable

int set_decode_variant(int variant) {
    if (variant < 0 || variant > 3) return set_error(MQ_ERR_INVALID_ARGUMENT, "variant %d not in {0,1,2,3}", variant);
    g_variant = variant;
    return MQ_OK;
}

void mark_xcd_unusable() {
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) g_xcd_ok[dev] = 2;
}

// The XCD-aware kernel takes each workgroup's XCD from the hardware and its
// rank from g / 8, which needs the workgroups of one residue class of g mod 8
// to share an XCD and the 8 classes to fill the 8 XCDs; verified once per
// device with a launch of the same shape.
bool xcd_placement_ok() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    int st = g_xcd_ok[dev].load();
    if (st != 0) return st == 1;
    bool ok = false;
    uint32_t* d = nullptr;
    if (hipGetSymbolAddress(reinterpret_cast<void**>(&d), HIP_SYMBOL(g_xcc_map)) == hipSuccess && d != nullptr) {
        hipLaunchKernelGGL(xcc_map_kernel, dim3(kNWG), dim3(kThreads), 0, 0, d);
        uint32_t h[kNWG];
        if (hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
            hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess) {
            bool seen[8] = {false};
            ok = true;
            for (int i = 0; i < 8; ++i) {
                ok = ok && h[i] < 8 && !seen[h[i]];
                if (ok) seen[h[i]] = true;
            }
            for (int i = 8; i < kNWG; ++i) ok = ok && (h[i] == h[i % 8]);
        }
    }
    g_xcd_ok[dev] = ok ? 1 : 2;
    return ok;
}

// The kernel a step of these dims with `cache_len` cached positions uses: the async-wave
// kernel (3) for the INT8 Qwen3-0.6B shape up to 6144 positions (it runs to 10240 when forced;
// past 6144 the XCD-aware kernel is faster), the XCD-aware kernel (2) otherwise when the
// workgroup placement allows, else the single-level kernel (1).
// A refusal returns its status negated (MQ_ERR_UNSUPPORTED is 2, the XCD-aware kernel's
// number, so it must not share the positive range).
int decode_variant_for(const DecodeShape& s, bool int8, int cache_len) {
    const int v = g_variant.load();
    // INT4 weights run on the async-wave kernel only
    if (s.int4) {
        if (v == 1 || v == 2 || !xcd_placement_ok() || !decode_async_supports(s, true, cache_len))
            return -set_error(MQ_ERR_UNSUPPORTED, "INT4 weights run on the async-wave kernel only: hidden 1024 / "
                              "intermediate 3072, up to %d cached positions (cache_len %d, variant %d%s)",
                              decode_async_max_len(), cache_len, v,
                              xcd_placement_ok() ? "" : ", workgroup placement unsupported");
        return 3;
    }
    const bool have_xcd = decode_xcd_kernel_ptr(s, int8, false) != nullptr;
    // FP8 weights run on the XCD-aware kernel only
    if (s.fp8) {
        if (!have_xcd) return -set_error(MQ_ERR_UNSUPPORTED, "no FP8 decode kernel for H=%d I=%d", s.H, s.I);
        if (v == 1 || v == 3 || !xcd_placement_ok())
            return -set_error(MQ_ERR_UNSUPPORTED, "FP8 weights run on the XCD-aware kernel only (variant %d%s)", v,
                             xcd_placement_ok() ? "" : ", workgroup placement unsupported");
        return 2;
    }
    if (v == 1) return 1;
    if (v == 2) return have_xcd ? 2 : -set_error(MQ_ERR_UNSUPPORTED, "no XCD-aware kernel for these dims");
    if (v == 3)
        return decode_async_supports(s, int8, cache_len)
                   ? 3
                   : -set_error(MQ_ERR_UNSUPPORTED, "the async-wave kernel covers INT8 hidden 1024 / intermediate 3072 "
                                                   "up to %d cached positions (cache_len %d)", decode_async_max_len(), cache_len);
    if (!(have_xcd && xcd_placement_ok())) return 1;
    return decode_async_supports(s, int8, cache_len) && cache_len <= decode_async_auto_len() ? 3 : 2;
}

int decode_variant_in_use(const DecodeShape& s, bool int8) { return decode_variant_for(s, int8, 1); }

// All kNWG workgroups wait on each other, so they must be resident at once;
// checked once per (kernel, device) from the occupancy calculator. The kernels
// need co-residency only (their exchanges are their own, no runtime grid
// barrier), so they are launched plainly: on this runtime a cooperative launch
// cost about 10 us more per step. If other work holds CUs when a step starts,
// its bounded waits end the step with MQ_ERR_TIMEOUT instead of hanging.
static std::atomic<int> g_cooperative{0};

int set_cooperative_launch(int on) {
    g_cooperative = on ? 1 : 0;
    return MQ_OK;
}

hipError_t launch_resident(const void* fn, dim3 grid, dim3 block, void** args, hipStream_t stream, hipEvent_t t0,
                           hipEvent_t t1) {
    if (g_cooperative.load() == 0) return hipExtLaunchKernel(fn, grid, block, args, 0, stream, t0, t1, 0);
    hipError_t e = hipSuccess;
    if (t0 != nullptr && (e = hipEventRecord(t0, stream)) != hipSuccess) return e;
    if ((e = hipLaunchCooperativeKernel(fn, grid, block, args, 0, stream)) != hipSuccess) return e;
    if (t1 != nullptr) e = hipEventRecord(t1, stream);
    return e;
}

int check_residency(const void* fn, int threads) {
    // the (device, kernel) pairs that passed, so that alternating kernels (per-step and
    // multi-step decode, prefill) do not repeat the occupancy query
    struct Passed { int dev; const void* fn; };
    static thread_local Passed passed[32];
    static thread_local int n_passed = 0, next = 0;      // entries in use (<= 32), slot written next
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(MQ_ERR_HIP, "hipGetDevice failed");
    for (int i = 0; i < n_passed; ++i)
        if (passed[i].dev == dev && passed[i].fn == fn) return MQ_OK;
    int ncu = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess)
        return set_error(MQ_ERR_HIP, "occupancy query failed");
    if ((int64_t)ncu * per_cu < kNWG)
        return set_error(MQ_ERR_UNSUPPORTED, "device holds %d x %d resident workgroups, the decode kernel needs %d",
                         ncu, per_cu, kNWG);
    passed[next] = Passed{dev, fn};
    next = (next + 1) % 32;
    if (n_passed < 32) ++n_passed;
    return MQ_OK;
}

template <int H, int I, class W>
static int launch_t(const KArgs& ka, bool debug, hipStream_t stream, hipEvent_t t0, hipEvent_t t1) {
    auto fn = debug ? reinterpret_cast<const void*>(&decode_kernel<H, I, W, true>)
                    : reinterpret_cast<const void*>(&decode_kernel<H, I, W, false>);
    int st = check_residency(fn);
    if (st != MQ_OK) return st;
    KArgs copy = ka;
    void* args[] = {&copy};
    // a plain launch (start/stop events when given): see check_residency
    const hipError_t e = launch_resident(fn, dim3(kNWG), dim3(kThreads), args, stream, t0, t1);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "launch(decode): %s", hipGetErrorString(e));
    return MQ_OK;
}

int launch_decode(const mq_decode_args& a, const DecodeShape& s, bool int8, hipStream_t stream, uint32_t* status_out,
                  const GenPlan* plan) {
    if (a.num_layers > kMaxLayers)
        return set_error(MQ_ERR_UNSUPPORTED, "num_layers %d exceeds %d", a.num_layers, kMaxLayers);
    // several steps per launch: the kernel chosen for the longest cache the launch reaches (the
    // async-wave kernel within its range, else the XCD-aware kernel; not the single-level one)
    const int variant = decode_variant_for(s, int8, plan ? a.position + plan->n_steps : a.cache_len);
    if (variant < 0) return -variant;
    if (plan && variant == 1)
        return set_error(MQ_ERR_UNSUPPORTED, "several steps per launch run on the async-wave and XCD-aware kernels, "
                         "not on the single-level kernel");
    // split attention: the XCD kernel with a slice of at most kMaxAttnLen positions per
    // workgroup; the async-wave kernel with slices of at most 64 (its own threshold)
    int split_min = a.attn_split_min == 0 ? kDefaultSplitMin : a.attn_split_min;
    split_min = split_min > 0 ? std::min(split_min, kMaxAttnLen + 1) : INT_MAX;
    if (variant == 3) split_min = decode_async_split_min(a.attn_split_min);
    const int last_len = plan ? a.position + plan->n_steps : a.cache_len;
    const int max_len = variant == 3 ? decode_async_max_len()
                        : (variant == 2 && split_min != INT_MAX) ? kSplitRanks * kMaxAttnLen : kMaxAttnLen;
    if (last_len > max_len)
        return set_error(MQ_ERR_UNSUPPORTED, "cache_len %d exceeds the attention limit %d of the %s kernel%s",
                         last_len, max_len, variant == 3 ? "async-wave" : variant == 2 ? "XCD-aware" : "single-level",
                         variant == 2 && split_min == INT_MAX ? " without split attention" : "");
    KArgs k;
    k.token = a.input_token_id;
    k.out_token = a.output_token_id;
    k.embed = static_cast<const uint16_t*>(a.embed_weight);
    k.lw = a.layer_weights;
    k.sp = a.scales;
    k.final_norm = static_cast<const uint16_t*>(a.final_norm_weight);
    k.lm_w = static_cast<const uint8_t*>(a.lm_head_weight);
    k.lm_s = a.lm_head_scale;
    k.cos_t = static_cast<const uint16_t*>(a.cos_table);
    k.sin_t = static_cast<const uint16_t*>(a.sin_table);
    k.kc = static_cast<uint16_t*>(a.k_cache);
    k.vc = static_cast<uint16_t*>(a.v_cache);
    k.dbg_hidden = static_cast<uint16_t*>(a.hidden_buffer);
    k.dbg_act = static_cast<float*>(a.g_activations);
    k.dbg_resid = static_cast<float*>(a.g_residual);
    k.dbg_q = static_cast<float*>(a.g_q);
    k.dbg_k = static_cast<float*>(a.g_k);
    k.dbg_v = static_cast<float*>(a.g_v);
    k.dbg_attn = static_cast<float*>(a.g_attn_out);
    k.dbg_mlp = static_cast<float*>(a.g_mlp_intermediate);
    k.dbg_norm = static_cast<float*>(a.g_normalized);
    k.dbg_bmax = static_cast<float*>(a.block_max_vals);
    k.dbg_bidx = static_cast<int*>(a.block_max_idxs);
    k.L = a.num_layers;
    k.pos = a.position;
    k.cache_len = a.cache_len;
    k.S = a.max_seq_len;
    k.V = s.V;
    k.split_min = split_min;
    k.attn_scale = a.attn_scale;
    k.spin_limit = a.spin_limit ? a.spin_limit : (1u << 21);
    k.trace = static_cast<uint64_t*>(a.trace);
    k.ws = static_cast<uint8_t*>(a.workspace);
    k.status_out = status_out;
    k.n_steps = plan ? plan->n_steps : 1;
    k.n_forced = plan ? plan->n_forced : 1;
    k.step_tokens = plan ? plan->tokens : nullptr;
    k.tokens_out = plan ? plan->tokens_out : nullptr;
    k.inv_temp = a.temperature > 0.0f ? 1.0f / a.temperature : 0.0f;
    k.seed = a.seed;
    const bool debug = a.hidden_buffer || a.g_activations || a.g_residual || a.g_q || a.g_k || a.g_v ||
                       a.g_attn_out || a.g_mlp_intermediate || a.g_normalized || a.block_max_vals ||
                       a.block_max_idxs || a.trace;

    hipEvent_t t0 = static_cast<hipEvent_t>(a.timing_start), t1 = static_cast<hipEvent_t>(a.timing_stop);
    if (variant == 3) return launch_decode_async(k, debug, s.int4, stream, t0, t1);
    if (variant == 2) return launch_decode_xcd(k, s, int8, debug, stream, t0, t1);
    if (s.H == 1024 && s.I == 3072) {
        return int8 ? launch_t<1024, 3072, Int8W>(k, debug, stream, t0, t1) : launch_t<1024, 3072, Bf16W>(k, debug, stream, t0, t1);
    }
    if (s.H == 2048 && s.I == 6144 && int8) return launch_t<2048, 6144, Int8W>(k, debug, stream, t0, t1);
    return set_error(MQ_ERR_UNSUPPORTED, "no decode kernel compiled for H=%d I=%d (%s)", s.H, s.I,
                     int8 ? "int8" : "bf16");
}

}  // namespace mq
