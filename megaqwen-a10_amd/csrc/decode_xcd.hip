// XCD-aware persistent decode step (the fast path on MI355X).
//
// Same computation as decode.hip (a10_int8_decode_kernel.cu:21-815, and the
// bf16 twin), laid out for 8 XCDs x 32 CUs: workgroup g takes the XCD it runs
// on, x = HW_REG_XCC_ID, as its group and r = g / 8 as its rank there, and KV
// head x with its two query heads belongs to XCD x. The dispatcher deals the
// workgroups of a launch round-robin over the 8 XCDs, so each XCD receives one
// residue class of g mod 8 and (x, r) covers the 8 x 32 roles exactly once,
// whichever XCD the round-robin starts on. Per layer:
//
//   A  QKV      rank r: 16 of XCD x's 512 q|k|v rows          -> XCD-local words
//   B  attn     every rank of XCD x: QK-norm, RoPE, attention over the bf16
//               KV cache for head pair x (redundant; the KV rows are shared
//               through the XCD's L2); rank 0 writes the cache row. From
//               split_min positions on, rank r takes the r-th 1/32 of the
//               positions instead: its softmax partial (max, sum, weighted V)
//               goes to XCD-local words, rank r merges output dims
//               [8r, 8r+8) over the 32 partials, and an XCD-local all-gather
//               hands every rank the 256 outputs
//   C  O        rank r: rows [H/32 r, +H/32) of O[:, 256x : 256x+256]
//                                                             -> cross-XCD partials
//   D  reduce   rank r sums its rows' 8 partials in XCD order, applies the
//               row scale and the residual                    -> XCD-local act
//   E  gate/up  rank r: channels [I/8 x + I/256 r, +I/256), SwiGLU
//                                                             -> XCD-local mlp
//   F  down     rank r: rows [H/32 r, +H/32) of down[:, I/8 x : I/8 (x+1)]
//                                                             -> cross-XCD partials
//   G  reduce   as D, plus bf16 rounding                      -> XCD-local hidden
//
// so each layer has four exchanges inside one XCD (plain stores land in the
// XCD's shared L2; agent-scope loads read it) and two across XCDs
// (agent-scope stores and loads). Words carry a (step, layer, stage) tag as in
// decode.hip. Every reduction sums in a fixed order, so all ranks see identical
// values and results are bitwise reproducible. The LM head is split over all
// 256 workgroups; workgroup (0, 0) reads their 256 maxima in one round.
//
// Each stage's weights (and scales / norm gains) are loaded into registers
// before the preceding wait, so their fetch overlaps the exchange latency.
#include "attention.h"

#include <hip/hip_ext.h>

namespace mq {

// Partial-row matvec piece: 16 bytes of weights against the matching fp32
// activations held contiguously in LDS.
template <class W>
__device__ __forceinline__ float dot_piece(uint4 w, const float* x) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    return W::dot(w, x4, 0.0f);
}

// One wave gathers the N tagged words at base (N a multiple of 128) into dst[0, N):
// 16-byte agent-coherent loads of two words, consecutive lanes on consecutive chunks.
template <int N>
__device__ __forceinline__ void gather_xcd(Waiter& wt, const uint64_t* base, uint32_t tag, float* dst, int lane) {
    static_assert(N % 128 == 0, "whole 128-word rounds");
    constexpr int C = N / 128;
    uint32_t w[C];
#pragma unroll
    for (int i = 0; i < C; ++i) w[i] = 2u * (uint32_t)(lane + 64 * i);
    float v[2 * C];
    wt.get_pairs<C>(XRegion(base, N), w, tag, v);
#pragma unroll
    for (int i = 0; i < C; ++i)
        *reinterpret_cast<float2*>(&dst[2 * (lane + 64 * i)]) = make_float2(v[2 * i], v[2 * i + 1]);
}

// kMulti: a launch's steps in sequence (a.n_steps; step s decodes at position a.pos + s, its
// input token is a.step_tokens[s] for the first a.n_forced steps and the previous step's
// output after them, which workgroup (0, 0) hands to every workgroup through one tagged
// word); otherwise one step, and the step loop disappears.
template <int H, int I, class W, bool kDebug, bool kMulti = false>
__global__ void __launch_bounds__(kThreads, 1) decode_xcd_kernel(KArgs a) {
    constexpr int D = 128;
    constexpr int ES = W::kBytes;
    constexpr bool kInt8 = (ES == 1);
    constexpr XLayout kLay = xlayout_for(H, I);
    constexpr int GR = 4 * D;               // q|k|v rows of one XCD (2 query heads, 1 K, 1 V)
    constexpr int ROWS_A = GR / kGS;        // QKV rows per workgroup
    constexpr int RPW = H / kGS;            // O / down output rows per workgroup
    constexpr int IX = I / kNX;             // intermediate channels per XCD
    constexpr int CPW = IX / kGS;           // gate/up channels per workgroup
    constexpr int PT = H / kThreads;        // hidden elements per thread
    constexpr int AD = 2 * D;               // attention outputs per XCD
    constexpr int EPP = 16 / ES;            // weight elements per 16-byte piece
    // stages C and F: LPR consecutive lanes per output row, each taking every
    // LPR-th 16-byte piece of the row's segment; the row sum is a DPP butterfly
    // inside the lane group
    constexpr int LPR = kThreads / RPW;
    constexpr int PC_O = AD / EPP;          // pieces per O row segment
    constexpr int PPL_O = (PC_O + LPR - 1) / LPR;
    constexpr int PC_D = IX / EPP;          // pieces per down row segment
    constexpr int PPL_D = (PC_D + LPR - 1) / LPR;
    constexpr int MLP_PT = (IX + kThreads - 1) / kThreads;
    static_assert(RPW * LPR == kThreads && (LPR & (LPR - 1)) == 0 && LPR <= kWave, "C/F lane groups");
    static_assert(GR % kGS == 0 && H % kGS == 0 && IX % kGS == 0 && H % kThreads == 0, "even split");
    static_assert(RPW <= kThreads && AD % EPP == 0 && IX % EPP == 0, "shapes");

    __shared__ double2 xd[H / 2];           // fp64 matvec input in per-lane order (QKV, gate/up)
    __shared__ float4 xs[H / 4];            // fp32 LM-head input in per-lane order
    __shared__ __align__(16) float hid[H];  // layer input (bf16 values)
    __shared__ __align__(16) float act[H];                // post-attention residual stream (fp32 values)
    __shared__ double attn_d[AD];           // this XCD's attention outputs (fp32 values), piece-major
    __shared__ double mlp_d[IX];            // this XCD's SwiGLU outputs (fp32 values), piece-major
    __shared__ double part[256];
    __shared__ double red[2 * kWaves];
    __shared__ float att_in[GR];
    __shared__ uint32_t mrg[kGS * 19];      // split attention: the 32 partials of this rank's 8 dims
    // split slices staged in LDS: up to 320 positions (context 10240) at H = 1024,
    // 256 (context 8192) at H = 2048, whose other buffers leave less LDS
    // Split-slice capacity of the register/DMA path (sdma below). The bf16 instantiation
    // has no registers to spare for a slice's V words (they were spilled right after
    // loading, turning the prefetch into a wait), so it has no such path: its slices come
    // from the rows prefetched a layer ahead up to kKvLds positions, and from the cache
    // inside the loop beyond that.
    constexpr bool kSliceRegs = kInt8 && !kMulti;       // (the multi-step form has no registers to spare either)
    constexpr int kSlice = !kSliceRegs ? kKvLds : H <= 1024 ? 320 : 256;
    __shared__ __align__(16) AttnShared<kSlice> at;
    __shared__ float lm_v[kWaves];
    __shared__ int lm_i[kWaves];
    __shared__ uint32_t rope_s[2][D];       // cos / sin row of this step's position (bf16 bits)
    __shared__ LayerWeights s_lw[kMaxLayers];
    __shared__ ScalePointers s_sp[kMaxLayers];

    const int g0 = blockIdx.x;
    const int x0 = (int)hw_xcc_id();
    const int tid0 = threadIdx.x;
    double* xdf = reinterpret_cast<double*>(xd);
    float* xsf = reinterpret_cast<float*>(xs);

    WsHeader* hdr = reinterpret_cast<WsHeader*>(a.ws);

    // step-independent reads first
    int token = (kMulti && a.step_tokens) ? *gview(a.step_tokens) : a.token;
    float hv0[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) hv0[i] = bf16_bits_to_f32(gview(a.embed)[(int64_t)token * H + tid0 + i * kThreads]);
    {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.lw);
        uint64_t* dst = reinterpret_cast<uint64_t*>(s_lw);
        for (int i = tid0; i < a.L * 11; i += kThreads) dst[i] = src[i];
        if (kInt8) {
            const uint64_t* ssrc = reinterpret_cast<const uint64_t*>(a.sp);
            uint64_t* sdst = reinterpret_cast<uint64_t*>(s_sp);
            for (int i = tid0; i < a.L * 7; i += kThreads) sdst[i] = ssrc[i];
        }
    }
    const uint32_t E0 = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t XS0 = __hip_atomic_load(&hdr->xsteps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Waiter wt(&hdr->abort_flag, a.spin_limit);
    // A device with other than 8 XCDs cannot run this kernel: flag it (the waits
    // then end at once and the host switches to the single-level kernel).
    if (x0 >= kNX) {
        if (tid0 == 0) __hip_atomic_store(&hdr->abort_flag, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    const int n_steps = kMulti ? a.n_steps : 1;
    for (int step = 0; step < n_steps; ++step) {
    const int g = g0, x = x0;
    const int r = g / kNX;
    const int64_t kv_head_stride = (int64_t)a.S * D;
    const int last = a.L - 1;
    uint64_t* const qkvx = reinterpret_cast<uint64_t*>(a.ws + kLay.qkvx) + (size_t)x * GR;
    uint64_t* const actx = reinterpret_cast<uint64_t*>(a.ws + kLay.actx) + (size_t)x * H;
    uint64_t* const mlpx = reinterpret_cast<uint64_t*>(a.ws + kLay.mlpx) + (size_t)x * IX;
    uint64_t* const hidx = reinterpret_cast<uint64_t*>(a.ws + kLay.hidx) + (size_t)x * H;
    uint64_t* const lmg = reinterpret_cast<uint64_t*>(a.ws + kLay.lmg);
    uint64_t* const po = reinterpret_cast<uint64_t*>(a.ws + kLay.po);    // packed [8][H]
    uint64_t* const pd = reinterpret_cast<uint64_t*>(a.ws + kLay.pd);    // packed [8][H]
    uint64_t* const attp = reinterpret_cast<uint64_t*>(a.ws + kLay.attp) + (size_t)x * kGS * kAttWords;
    uint64_t* const atto = reinterpret_cast<uint64_t*>(a.ws + kLay.atto) + (size_t)x * AD;
    uint64_t* const tokw = reinterpret_cast<uint64_t*>(a.ws + kLay.tokw);
    const int tid = tid0;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const uint32_t E = E0 + (uint32_t)step;      // the step's epoch (tags) and packed-word step count
    const uint32_t XS = XS0 + (uint32_t)step;
    const uint32_t tps = kXStages * (uint32_t)a.L + 4u;
    // tags end in binary 11 (the single-level kernel's end in 01): no overlap when
    // the two kernels share a workspace
    auto tag = [&](int l, int st) -> uint32_t { return ((E * tps + kXStages * (uint32_t)l + (uint32_t)st) << 2) | 3u; };
    // one-bit tag of the packed cross-XCD words: po and pd are each written once
    // per layer, so their use count is XS * L + l + 1
    auto pbit = [&](int l) -> uint32_t { return (XS * (uint32_t)a.L + (uint32_t)l + 1u) & 1u; };
    auto trace = [&](int l, int point) {
        if (kDebug && a.trace != nullptr && tid == 0)
            a.trace[((int64_t)l * kTracePoints + point) * kNWG + g] = __builtin_amdgcn_s_memrealtime();
    };
    const int pos = a.pos + step;
    const int cache_len = pos + 1;
    if (g == 0 && tid == 0) {
        // keep the header slots the single-level kernel counts on in a known state
        __hip_atomic_store(&hdr->done[(E + 1) & 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&hdr->best[(E + 1) & 1], (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // attention positions of this workgroup: all of them, or the r-th slice
    const bool split = cache_len >= a.split_min;
    const int cs = (cache_len + kGS - 1) / kGS;
    const int sj0 = split ? min(cache_len, r * cs) : 0;
    const int sj1 = split ? min(cache_len, sj0 + cs) : cache_len;
    // split slices of at most kKvLds positions come wholly from the rows
    // prefetched during the previous layer (spre); up to kSlice positions, the
    // K rows go straight to LDS and the V words to registers ahead of the QKV
    // wait (sdma); longer slices read the cache inside the loop
    const bool spre = split && cs <= kKvLds;
    const bool sdma = kSliceRegs && split && !spre && cs <= kSlice;
    // the range's first npre earlier positions prefetched into registers, staged
    // in LDS (the current one comes from the QKV words)
    const int npre = sdma ? 0 : max(0, min(kKvLds, min(sj1, pos) - sj0));
    const int R0 = RPW * r;                 // first O / down row of this workgroup
    const double attn_scale = (double)a.attn_scale;
    __syncthreads();

    // QKV rows of this workgroup: rank < 16 query rows, < 24 key rows, else value rows
    auto qkv_rows = [&](const LayerWeights& lw, const ScalePointers& sp, const uint8_t*& base, const float*& sc,
                        int& mrow0) {
        if (r < 16) { base = (const uint8_t*)lw.q_proj_weight; mrow0 = 2 * x * D + ROWS_A * r; if (kInt8) sc = sp.q_scale; }
        else if (r < 24) { base = (const uint8_t*)lw.k_proj_weight; mrow0 = x * D + ROWS_A * (r - 16); if (kInt8) sc = sp.k_scale; }
        else { base = (const uint8_t*)lw.v_proj_weight; mrow0 = x * D + ROWS_A * (r - 24); if (kInt8) sc = sp.v_scale; }
    };

    Stage_<W, ROWS_A, H, 1> stA;            // wave 0 polls stage G's cross-XCD words
    uint32_t scA = 0x3f800000u;             // prefetched raw bits (after_wait at use)
    uint32_t wln[PT];
    {
        const uint8_t* base; const float* sc = nullptr; int mrow0;
        qkv_rows(s_lw[0], s_sp[0], base, sc, mrow0);
        stA.load([&](int rr) { return base + (int64_t)(mrow0 + rr) * H * ES; }, wave, lane);
        if (kInt8 && tid < ROWS_A) scA = ldg_bits(sc + mrow0 + tid);
        const uint16_t* lnw = (const uint16_t*)s_lw[0].input_layernorm_weight;
#pragma unroll
        for (int i = 0; i < PT; ++i) wln[i] = ldg_bits(lnw + tid + i * kThreads);
#pragma unroll
        for (int i = 0; i < PT; ++i) hid[tid + i * kThreads] = hv0[i];
    }
    __syncthreads();

    // Stage B's step-independent inputs for a layer, loaded one stage ahead of
    // its QKV wait: O weights (consumed in stage C), the O scale, the QK-norm
    // gains and the K/V rows of the range's first npre positions.
    const int crow_s = tid / LPR, clr_s = tid % LPR;   // stages C and F: row, lane in the row's group
    constexpr int kPreU4 = 2 * kKvLds * (D / 8) / kThreads;
    uint4 wo[PPL_O];
    uint4 pre[kPreU4];
    // Where stage B's QK-norm gains and RoPE row live: the int8 instantiations have
    // registers to spare and load the gains a layer ahead (with the O scale) and hold
    // the RoPE row in registers. The bf16 instantiation spills, and a spilled value
    // costs more than it saves: the spill store waits for its load, and the reload
    // waits, in order, behind every weight load issued before it. It keeps the RoPE
    // row in LDS and loads the gains at the start of stage A.
    constexpr bool kLateInputs = !kInt8;
    uint32_t so = 0x3f800000u, nw0 = 0, nw1 = 0;
    auto load_gains = [&](const LayerWeights& lw) {
        if (wave < 3) {
            const uint16_t* nw = (const uint16_t*)(wave < 2 ? lw.q_norm_weight : lw.k_norm_weight);
            nw0 = ldg_bits(nw + lane);
            nw1 = ldg_bits(nw + lane + 64);
        }
    };
    // t: the calling thread's index as the caller holds it (with several steps, rederived per
    // layer, so that the addresses below are not held through the layer loop)
    auto prefetch_b = [&](int ll, int t) {
        const int crow = kMulti ? t / LPR : crow_s, clr = kMulti ? t % LPR : clr_s;
        const LayerWeights& lw = s_lw[ll];
        const uint8_t* ob = (const uint8_t*)lw.o_proj_weight;
#pragma unroll
        for (int k = 0; k < PPL_O; ++k) {
            const int pc = clr + LPR * k;
            wo[k] = make_uint4(0, 0, 0, 0);
            if (pc < PC_O) wo[k] = ldg16_stream(ob + (int64_t)(R0 + crow) * (16 * D) * ES + (int64_t)AD * x * ES + pc * 16);
        }
        if (kInt8 && tid < RPW) so = ldg_bits(s_sp[ll].o_scale + R0 + tid);
        if constexpr (!kLateInputs) load_gains(lw);
        const int64_t cb = ((int64_t)ll * kNX + x) * kv_head_stride + (int64_t)opaque(sj0) * D;
#pragma unroll
        for (int i = 0; i < kPreU4; ++i) {
            // K rows for the first half of the i, V rows for the second: a uniform choice (the
            // thread index is below kThreads, which divides kKvLds * D / 8), so the cache pointer
            // stays a scalar
            static_assert((kKvLds * (D / 8)) % kThreads == 0, "prefetch split");
            const int side = i * kThreads / (kKvLds * (D / 8));
            const int rem = ((kMulti ? t : tid) + i * kThreads) % (kKvLds * (D / 8));
            const int j = rem / (D / 8), c = rem % (D / 8);
            pre[i] = make_uint4(0, 0, 0, 0);
            if (j < npre) pre[i] = ldg16((side == 0 ? a.kc : a.vc) + cb + (int64_t)j * D + c * 8);
        }
    };
    // the RoPE row of this position is the same for every layer (in LDS: stage A's
    // barriers order these writes before the first read)
    uint32_t c0 = 0, s0 = 0, c1 = 0, s1 = 0;
    if constexpr (kLateInputs) {
        if (tid < 2 * D) {
            const uint16_t* row = (tid < D ? a.cos_t : a.sin_t) + (int64_t)pos * D;
            rope_s[tid / D][tid % D] = ldg_bits(row + tid % D);
        }
    } else if (wave < 3) {
        const uint16_t* ct = a.cos_t + (int64_t)pos * D;
        const uint16_t* stt = a.sin_t + (int64_t)pos * D;
        c0 = ldg_bits(ct + lane);
        s0 = ldg_bits(stt + lane);
        c1 = ldg_bits(ct + lane + 64);
        s1 = ldg_bits(stt + lane + 64);
    }
    prefetch_b(0, tid);

    uint32_t wfn[PT];                       // final RMSNorm gains (raw bits, loaded in the last layer)
    const int tid_all = tid;
    for (int l = 0; l < a.L; ++l) {
        const LayerWeights& lw = s_lw[l];
        const ScalePointers& sp = s_sp[l];
        const int tid = opaque(tid_all);
        const int lane = tid % kWave;
        // the wave index too is rederived per layer: held through the loop, the addresses
        // derived from it were spilled to scratch, and each reload (its line evicted from L2
        // by the layer's weight stream) waited for memory
        const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        const int crow = kMulti ? tid / LPR : crow_s, clr = kMulti ? tid % LPR : clr_s;
        // bf16: stage B's QK-norm gains, at the start of stage A (no exchange poll before
        // their use, so the loads overlap stage A's work)
        if constexpr (kLateInputs) load_gains(lw);
        const int64_t cache_base = ((int64_t)l * kNX + x) * kv_head_stride;
        // ---------------- A: RMSNorm + QKV rows -> XCD-local words ----------------
        auto stage_a = [&]() {
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < PT; ++i) { const double v = hid[tid + i * kThreads]; ss = fma(v, v, ss); }
            const double tot = block_sum64_lds<kWaves>(ss, red, 0, wave, lane);
            trace(l, 0);
            const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const int k = tid + i * kThreads;
                xdf[xd_index<W>(k)] = (double)(float)((double)hid[k] * rstd * (double)after_wait_bf16(wln[i]));
            }
            lds_barrier();
            stA.compute(xd, part, wave, lane);
            lds_barrier();
            if (tid < ROWS_A) {
                double v = Stage_<W, ROWS_A, H, 1>::row_sum(part, tid);
                if (kInt8) v = v * (double)after_wait_f(scA);
                ll_put_xcd(&qkvx[ROWS_A * r + tid], __float_as_uint((float)v), tag(l, XS_QKV));
            }
            trace(l, 1);
        };
        // Split slices of up to kSlice positions: their K rows go straight to LDS, issued
        // here so that they stream during stage A, whose barriers wait for LDS data only.
        // The loads stage A consumes (issued a stage ahead) are waited for first, and
        // stage A is compiled a second time for this path: no wait in it then has to
        // count the slice's loads, which stay in flight until stage B.
        if (sdma) {
            wait_vmem();
            attn_slice_k<kWaves, true>(at, a.kc + cache_base, opaque(sj0), min(sj1, pos), lane, wave);
            stage_a();
        } else {
            stage_a();
        }

        // ---------------- B: attention for head pair x (every rank) ----------------
        {
            // this stage's step-independent inputs (O weights, K/V rows of earlier
            // positions, QK-norm gains) were loaded during the previous layer
            // the K/V rows prefetched during the previous layer go to LDS (read
            // after the barrier below); a split slice's K rows with their chunks
            // permuted for the matrix-core reads (kv_pre[0] is kst's first rows)
#pragma unroll
            for (int i = 0; i < kPreU4; ++i) {
                const int f = tid + i * kThreads;
                const int side = f / (kKvLds * (D / 8));
                const int rem = f % (kKvLds * (D / 8));
                const int j = rem / (D / 8), c = rem % (D / 8);
                const int cc = (spre && side == 0) ? kst_chunk(c, j) : c;
                if (j < npre) *reinterpret_cast<uint4*>(&at.kv_pre[side][j][cc * 4]) = pre[i];
            }
            // split slices: the V words (to registers; the K rows were issued at the
            // start of stage A), all in flight at once (opaque offsets keep the addresses
            // from being hoisted out of the layer loop)
            SliceRegs<kSlice> sr;
            if (sdma) attn_slice_v(sr, a.vc + cache_base, opaque(sj0), min(sj1, pos), lane, tid / kWave);
            {
                float v1[1];
                wt.get_strided<1>(qkvx + tid, 0, tag(l, XS_QKV), v1);
                att_in[tid] = v1[0];
            }
            if (sdma) wait_vmem();              // the K rows are in LDS after the barrier
            __syncthreads();
            trace(l, 2);
            const int64_t cur = cache_base + (int64_t)pos * D;
            const bool writer = (r == 0);           // rank 0 writes the cache rows
            const bool dbg = kDebug && writer && l == last;
            if constexpr (kLateInputs) {
                c0 = rope_s[0][lane];
                s0 = rope_s[1][lane];
                c1 = rope_s[0][lane + 64];
                s1 = rope_s[1][lane + 64];
            }
            attn_qk_rope(at, att_in, nw0, nw1, c0, s0, c1, s1, writer ? a.kc + cur : nullptr,
                         writer ? a.vc + cur : nullptr, (dbg && a.dbg_q) ? a.dbg_q + 2 * x * D : nullptr,
                         (dbg && a.dbg_k) ? a.dbg_k + x * D : nullptr, (dbg && a.dbg_v) ? a.dbg_v + x * D : nullptr,
                         wave, lane, spre || sdma);
            __syncthreads();
            if (!split) {
                attn_core(at, a.kc + cache_base, a.vc + cache_base, sj1, pos, attn_scale, tid, lane, wave,
                          [&](int i, float v) {
                              attn_d[piece_index(i, EPP, PC_O)] = v;
                              if (dbg && a.dbg_attn) a.dbg_attn[AD * x + i] = v;
                          },
                          [](int) {});
            } else {
                const uint32_t tp = tag(l, XS_ATP);
                uint64_t* const mine = attp + (size_t)r * kAttWords;
                auto publish = [&](int i, double acc, double psum, double m) {
                    const uint64_t u = (uint64_t)__double_as_longlong(acc);
                    ll_put_xcd(&mine[2 * i], (uint32_t)u, tp);
                    ll_put_xcd(&mine[2 * i + 1], (uint32_t)(u >> 32), tp);
                    if ((i & (D - 1)) == 0) {
                        const int h = i / D;
                        const uint64_t su = (uint64_t)__double_as_longlong(psum);
                        ll_put_xcd(&mine[2 * AD + 3 * h], __float_as_uint((float)m), tp);
                        ll_put_xcd(&mine[2 * AD + 3 * h + 1], (uint32_t)su, tp);
                        ll_put_xcd(&mine[2 * AD + 3 * h + 2], (uint32_t)(su >> 32), tp);
                    }
                };
                if (spre) {
                    attn_partial_lds(at, sj0, sj1, pos, attn_scale, tid, lane, wave, publish, [](int) {});
                } else if (sdma) {
                    attn_partial_regs(at, sr, sj0, sj1, pos, attn_scale, tid, lane, wave, publish, [](int) {});
                } else
                    attn_partial(at, a.kc + cache_base, a.vc + cache_base, sj0, sj1, pos, attn_scale, tid, lane,
                                 wave, publish, [](int) {});
                // merge output dims [8r, 8r+8) (query head r / 16) over the 32
                // partials: thread (s, k) reads word k of rank s's slice, and
                // threads below 96 rank s2's maximum and probability sum
                {
                    const int hh = r / (kGS / 2);
                    const uint64_t* pa = attp + (size_t)(tid >> 4) * kAttWords + 16 * r + (tid & 15);
                    const uint64_t* pb = attp + (size_t)(tid / 3) * kAttWords + 2 * AD + 3 * hh + tid % 3;
                    float w2[2];
                    wt.get_strided<2>(pa, (int)(pb - pa), tp, w2, tid < 3 * kGS ? 2 : 1);
                    mrg[tid] = __float_as_uint(w2[0]);
                    if (tid < 3 * kGS) mrg[16 * kGS + tid] = __float_as_uint(w2[1]);
                }
                __syncthreads();
                if (tid < 8 * kGS) {
                    const int k = tid / kGS, s = tid % kGS;
                    auto word64 = [&](int w) {
                        return __longlong_as_double((long long)(((uint64_t)mrg[w + 1] << 32) | mrg[w]));
                    };
                    const double ms = __uint_as_float(mrg[16 * kGS + 3 * s]);
                    const double ls = word64(16 * kGS + 3 * s + 1);
                    const double acc = word64(16 * s + 2 * k);
                    const double M = group_max64<kGS>(ms);
                    const double c = exp(ms - M);        // 0 for an empty slice (m = -inf)
                    const double num = group_sum64<kGS>(c * acc);
                    const double den = group_sum64<kGS>(c * ls);
                    if (s == 0) {
                        const float o = (float)(num * rcp_nr(den));
                        ll_put_xcd(&atto[8 * r + k], __float_as_uint(o), tag(l, XS_ATO));
                        if (kDebug && l == last && a.dbg_attn) a.dbg_attn[AD * x + 8 * r + k] = o;
                    }
                }
                if (tid < AD) attn_d[piece_index(tid, EPP, PC_O)] = wt.getf(atto + tid, tag(l, XS_ATO));
            }
            __syncthreads();
            trace(l, 3);
        }

        // ---------------- C: O partial over this XCD's 256 attention dims -> cross-XCD ----------------
        {
            double p = 0.0;
#pragma unroll
            for (int k = 0; k < PPL_O; ++k) {
                const int pc = clr + LPR * k;
                if (pc < PC_O) p = W::template dotd<PC_O>(wo[k], reinterpret_cast<const double2*>(attn_d) + pc, p);
            }
            p = group_sum64<LPR>(p);
            if (clr == 0) ll_put64(&po[(size_t)x * H + R0 + crow], pack_tagged(p, pbit(l)));
            trace(l, 4);
        }

        // ---------------- D: reduce O partials -> act rows -> XCD-local all-gather ----------------
        Stage_<W, 2 * CPW, H, 1> stE;       // wave 0 polls stage D's cross-XCD words
        uint32_t sd = 0x3f800000u;
        uint4 wd[PPL_D];                    // stage F's down weights
        uint32_t gsc = 0x3f800000u, usc = 0x3f800000u;
        uint32_t wpn[PT];
        const int c0 = opaque(IX * x + CPW * r);
        {
            // stage E's weights (waves 1-7), scales and norm gains
            const uint8_t* gb = (const uint8_t*)lw.gate_proj_weight;
            const uint8_t* ub = (const uint8_t*)lw.up_proj_weight;
            stE.load([&](int rr) {
                return rr < CPW ? gb + (int64_t)(c0 + rr) * H * ES : ub + (int64_t)(c0 + rr - CPW) * H * ES;
            }, wave, lane);
            if (kInt8 && tid < CPW) { gsc = ldg_bits(sp.gate_scale + c0 + tid); usc = ldg_bits(sp.up_scale + c0 + tid); }
            const uint16_t* pnw = (const uint16_t*)lw.post_attn_layernorm_weight;
#pragma unroll
            for (int i = 0; i < PT; ++i) wpn[i] = ldg_bits(pnw + tid + i * kThreads);
            issue_fence();

            if (tid < RPW) {
                double v8[kNX];
                wt.get_packed<kNX>(po + R0 + tid, H, pbit(l), v8);
                double s = ((v8[0] + v8[1]) + (v8[2] + v8[3])) + ((v8[4] + v8[5]) + (v8[6] + v8[7]));
                if (kInt8) s = s * (double)after_wait_f(so);
                const float av = (float)(s + (double)hid[R0 + tid]);
                ll_put_xcd(&actx[R0 + tid], __float_as_uint(av), tag(l, XS_ACT));
            }

            // wave 0 gathers every residual row: the other waves have stage E's weights in
            // flight, and their polls would return only after those (loads return in order)
            if (wave == 0) gather_xcd<H>(wt, actx, tag(l, XS_ACT), act, lane);
            __syncthreads();
            float av[PT];
#pragma unroll
            for (int i = 0; i < PT; ++i) av[i] = act[tid + i * kThreads];
            trace(l, 5);
            issue_fence();
            {
                // stage F's down weights: issued after the act gather (so that
                // neither exchange waits for them), consumed after stage E
                const uint8_t* db = (const uint8_t*)lw.down_proj_weight;
#pragma unroll
                for (int k = 0; k < PPL_D; ++k) {
                    const int pc = clr + LPR * k;
                    wd[k] = make_uint4(0, 0, 0, 0);
                    if (pc < PC_D) wd[k] = ldg16_stream(db + (int64_t)(R0 + crow) * I * ES + (int64_t)IX * x * ES + pc * 16);
                }
                if (kInt8 && tid < RPW) sd = ldg_bits(sp.down_scale + R0 + tid);
            }

            // ---------------- E: RMSNorm + gate/up + SwiGLU -> XCD-local mlp ----------------
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < PT; ++i) ss = fma((double)av[i], (double)av[i], ss);
            const double tot = block_sum64<kWaves>(ss, red, 1, wave, lane);
            const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const int k = tid + i * kThreads;
                const float nv = (float)((double)av[i] * rstd * (double)after_wait_bf16(wpn[i]));
                xdf[xd_index<W>(k)] = nv;
                if (kDebug && l == last && g == 0) {
                    if (a.dbg_act) a.dbg_act[k] = nv;
                    if (a.dbg_resid) a.dbg_resid[k] = av[i];
                }
            }
            __syncthreads();
            stE.compute(xd, part, wave, lane);
            __syncthreads();
            if (tid < CPW) {
                double gs = Stage_<W, 2 * CPW, H, 1>::row_sum(part, tid);
                double us = Stage_<W, 2 * CPW, H, 1>::row_sum(part, CPW + tid);
                if (kInt8) { gs = gs * (double)after_wait_f(gsc); us = us * (double)after_wait_f(usc); }
                const float m = (float)silu_mul(gs, us);
                ll_put_xcd(&mlpx[CPW * r + tid], __float_as_uint(m), tag(l, XS_MLP));
                if (kDebug && l == last && a.dbg_mlp) a.dbg_mlp[c0 + tid] = m;
            }
            trace(l, 6);
        }

        // ---------------- F: down partial over this XCD's channels -> cross-XCD ----------------
        {

            if (tid < IX) {
                float mv[MLP_PT];
                wt.get_strided<MLP_PT>(mlpx + tid, kThreads, tag(l, XS_MLP), mv, (IX - tid + kThreads - 1) / kThreads);
#pragma unroll
                for (int i = 0; i < MLP_PT; ++i)
                    if (tid + i * kThreads < IX) mlp_d[piece_index(tid + i * kThreads, EPP, PC_D)] = mv[i];
            }
            __syncthreads();
            trace(l, 7);
            double p = 0.0;
#pragma unroll
            for (int k = 0; k < PPL_D; ++k) {
                const int pc = clr + LPR * k;
                if (pc < PC_D) p = W::template dotd<PC_D>(wd[k], reinterpret_cast<const double2*>(mlp_d) + pc, p);
            }
            p = group_sum64<LPR>(p);
            if (clr == 0) ll_put64(&pd[(size_t)x * H + R0 + crow], pack_tagged(p, pbit(l)));
            trace(l, 8);
        }

        // ---------------- G: reduce down partials -> bf16 hidden -> XCD-local all-gather ----------------
        {
            if (l < last) {
                // the next layer's QKV weights (waves 1-7), scales and input-norm gains
                const LayerWeights& nl = s_lw[l + 1];
                const uint8_t* base; const float* sc = nullptr; int mrow0;
                qkv_rows(nl, s_sp[l + 1], base, sc, mrow0);
                stA.load([&](int rr) { return base + (int64_t)(mrow0 + rr) * H * ES; }, wave, lane);
                if (kInt8 && tid < ROWS_A) scA = ldg_bits(sc + mrow0 + tid);
                const uint16_t* lnw = (const uint16_t*)nl.input_layernorm_weight;
#pragma unroll
                for (int i = 0; i < PT; ++i) wln[i] = ldg_bits(lnw + tid + i * kThreads);
                issue_fence();
            } else {
                // the final RMSNorm gains, so that the tail's norm does not wait behind
                // the first LM-head weight batch
#pragma unroll
                for (int i = 0; i < PT; ++i) wfn[i] = ldg_bits(a.final_norm + tid + i * kThreads);
                issue_fence();
            }
            if (tid < RPW) {
                double v8[kNX];
                wt.get_packed<kNX>(pd + R0 + tid, H, pbit(l), v8);
                double s = ((v8[0] + v8[1]) + (v8[2] + v8[3])) + ((v8[4] + v8[5]) + (v8[6] + v8[7]));
                if (kInt8) s = s * (double)after_wait_f(sd);
                const float hf = (float)(s + (double)act[R0 + tid]);
                ll_put_xcd(&hidx[R0 + tid], __float_as_uint(round_bf16(hf)), tag(l, XS_HID));
            }

            // wave 0 gathers every hidden row (the other waves have the next layer's QKV
            // weights in flight)
            if (wave == 0) gather_xcd<H>(wt, hidx, tag(l, XS_HID), hid, lane);
            __syncthreads();
            if (kDebug && l == last && g == 0 && a.dbg_hidden) {
#pragma unroll
                for (int i = 0; i < PT; ++i)
                    a.dbg_hidden[tid + i * kThreads] = (uint16_t)f32_to_bf16_bits(hid[tid + i * kThreads]);
            }
            // the next layer's stage B inputs: after the hidden gather, so that
            // neither exchange waits for them; stage A covers their latency
            issue_fence();
            if (l < last) prefetch_b(l + 1, tid);
            trace(l, 9);
        }
    }

    // ---------------- final RMSNorm + LM head + greedy argmax ----------------
    {
        constexpr int CH = H / (64 * W::kPerLane);
        constexpr int RB = CH >= 8 ? 1 : 8 / CH;
        constexpr int R = RB * CH;
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
        int b = wave;
        if (b < nb) fetch(b, cur, scur);
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const double v = hid[tid + i * kThreads];
            ss = fma(v, v, ss);
        }
        const double tot = block_sum64<kWaves>(ss, red, 0, wave, lane);
        const double rstd = rms_scale(tot, H, kEps);
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const int k = tid + i * kThreads;
            const float nv = (float)((double)hid[k] * rstd * (double)after_wait_bf16(wfn[i]));
            xsf[xs_index<W>(k)] = nv;
            if (kDebug && g == 0 && a.dbg_norm) a.dbg_norm[k] = nv;
        }
        __syncthreads();
        trace(a.L, 0);

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
                if (a.inv_temp > 0.0f) v = v * a.inv_temp + gumbel_noise(a.seed, pos, row);
                if (v > best_v) { best_v = v; best_i = row; }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) cur[i] = nxt[i];
            scur = snxt;
        }
#define MQ_ARGMAX_LEVEL(M)                                                                   \
        {                                                                                    \
            const float ov = partner<M>(best_v);                                             \
            const int oi = __float_as_int(partner<M>(__int_as_float(best_i)));               \
            if (ov > best_v || (ov == best_v && oi < best_i)) { best_v = ov; best_i = oi; }  \
        }
        MQ_ARGMAX_LEVEL(1) MQ_ARGMAX_LEVEL(2) MQ_ARGMAX_LEVEL(4) MQ_ARGMAX_LEVEL(8)
        MQ_ARGMAX_LEVEL(16) MQ_ARGMAX_LEVEL(32)
#undef MQ_ARGMAX_LEVEL
        if (lane == 0) { lm_v[wave] = best_v; lm_i[wave] = best_i; }
        __syncthreads();
        trace(a.L, 1);
        // argmax over the 8 waves; then workgroup (0, 0) reads the maxima of all 256
        // workgroups in one cross-XCD round (4 per lane) and publishes the token
        const uint32_t tag_lm = tag(a.L, 0);
        if (tid == 0) {
            float bv = lm_v[0];
            int bi = lm_i[0];
            for (int w = 1; w < kWaves; ++w)
                if (lm_v[w] > bv || (lm_v[w] == bv && lm_i[w] < bi)) { bv = lm_v[w]; bi = lm_i[w]; }
            if (kDebug && a.dbg_bmax) a.dbg_bmax[g] = bv;
            if (kDebug && a.dbg_bidx) a.dbg_bidx[g] = bi;
            ll_put(&lmg[2 * g], ordered_key(bv), tag_lm);
            ll_put(&lmg[2 * g + 1], (uint32_t)bi, tag_lm);
        }
        if (x == 0 && r == 0 && wave == 0) {
            constexpr int C = kNWG / kWave;
            uint32_t w[C];
#pragma unroll
            for (int i = 0; i < C; ++i) w[i] = 2u * (uint32_t)(lane + kWave * i);
            float v[2 * C];
            wt.get_pairs<C>(XRegion(lmg, 2 * kNWG), w, tag_lm, v);
            uint32_t kv = __float_as_uint(v[0]), iv = __float_as_uint(v[1]);
#pragma unroll
            for (int i = 1; i < C; ++i) {
                const uint32_t ok = __float_as_uint(v[2 * i]), oi = __float_as_uint(v[2 * i + 1]);
                if (ok > kv || (ok == kv && oi < iv)) { kv = ok; iv = oi; }
            }
#define MQ_KEY_LEVEL(M)                                                                      \
            {                                                                                \
                const uint32_t ok = __float_as_uint(partner<M>(__uint_as_float(kv)));        \
                const uint32_t oi = __float_as_uint(partner<M>(__uint_as_float(iv)));        \
                if (ok > kv || (ok == kv && oi < iv)) { kv = ok; iv = oi; }                  \
            }
            MQ_KEY_LEVEL(1) MQ_KEY_LEVEL(2) MQ_KEY_LEVEL(4) MQ_KEY_LEVEL(8) MQ_KEY_LEVEL(16) MQ_KEY_LEVEL(32)
#undef MQ_KEY_LEVEL
            if (lane == 0) {
                const uint32_t flag = __hip_atomic_load(&hdr->abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int chosen = (flag != 0u || wt.dead) ? -1 : (int)iv;
                if constexpr (kMulti) {
                    // the next step's input, for every workgroup (a failed step's -1 becomes 0
                    // there, which keeps the remaining steps' reads in bounds; they report -1)
                    if (step + 1 < n_steps && step + 1 >= a.n_forced) ll_put(tokw, (uint32_t)max(chosen, 0), tag(a.L, 1));
                    if (a.tokens_out != nullptr && step >= a.n_forced - 1) a.tokens_out[step - (a.n_forced - 1)] = chosen;
                }
                if (step == n_steps - 1) {
                    *a.out_token = chosen;
                    if (a.status_out) *a.status_out = flag != 0u ? flag : (wt.dead ? 1u : 0u);
                    __hip_atomic_store(&hdr->xsteps, XS0 + (uint32_t)n_steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&hdr->epoch, E0 + (uint32_t)n_steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (kDebug && a.trace != nullptr)
                        a.trace[((int64_t)a.L * kTracePoints + 2) * kNWG] = __builtin_amdgcn_s_memrealtime();
                }
            }
        }
    }
    if constexpr (kMulti) {
        if (step + 1 < n_steps) {
            // the next step's input token: forced, or this step's output from workgroup (0, 0)
            if (step + 1 < a.n_forced) {
                token = *gview(a.step_tokens + step + 1);
            } else {
                if (tid == 0) lm_i[0] = (int)wt.get(tokw, tag(a.L, 1));
                __syncthreads();
                token = min(max(lm_i[0], 0), a.V - 1);      // an expired wait returns a stale word
            }
            issue_fence();
#pragma unroll
            for (int i = 0; i < PT; ++i)
                hv0[i] = bf16_bits_to_f32(gview(a.embed)[(int64_t)token * H + opaque(tid) + i * kThreads]);
        }
    }
    }
}

// ---------------- host side ----------------

size_t decode_xcd_workspace_bytes(const DecodeShape& s) { return xlayout_for(s.H, s.I).total; }

size_t decode_token_offset(const DecodeShape& s) {
    static_assert(kSplitRanks * kMaxAttnLen == kDecodeMaxForced, "forced-token region");
    return xlayout_for(s.H, s.I).tok;
}

template <int H, int I, class W>
static int launch_xcd_t(const KArgs& ka, bool debug, hipStream_t stream, hipEvent_t t0, hipEvent_t t1) {
    // several steps: the multi-step instantiation (without the debug outputs, which hold one step's values)
    auto fn = ka.n_steps > 1 ? reinterpret_cast<const void*>(&decode_xcd_kernel<H, I, W, false, true>)
              : debug        ? reinterpret_cast<const void*>(&decode_xcd_kernel<H, I, W, true>)
                             : reinterpret_cast<const void*>(&decode_xcd_kernel<H, I, W, false>);
    int st = check_residency(fn);
    if (st != MQ_OK) return st;
    KArgs copy = ka;
    void* args[] = {&copy};
    // a plain launch (start/stop events when given): see check_residency
    const hipError_t e = launch_resident(fn, dim3(kNWG), dim3(kThreads), args, stream, t0, t1);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "launch(decode_xcd): %s", hipGetErrorString(e));
    return MQ_OK;
}

const void* decode_xcd_kernel_ptr(const DecodeShape& s, bool int8, bool debug) {
    if (s.fp8) {
        if (!(int8 && s.H == 1024 && s.I == 3072)) return nullptr;
        return debug ? (const void*)&decode_xcd_kernel<1024, 3072, Fp8W, true> : (const void*)&decode_xcd_kernel<1024, 3072, Fp8W, false>;
    }
    if (s.H == 1024 && s.I == 3072) {
        if (int8) return debug ? (const void*)&decode_xcd_kernel<1024, 3072, Int8W, true> : (const void*)&decode_xcd_kernel<1024, 3072, Int8W, false>;
        return debug ? (const void*)&decode_xcd_kernel<1024, 3072, Bf16W, true> : (const void*)&decode_xcd_kernel<1024, 3072, Bf16W, false>;
    }
    if (s.H == 2048 && s.I == 6144 && int8)
        return debug ? (const void*)&decode_xcd_kernel<2048, 6144, Int8W, true> : (const void*)&decode_xcd_kernel<2048, 6144, Int8W, false>;
    return nullptr;
}

int launch_decode_xcd(const KArgs& k, const DecodeShape& s, bool int8, bool debug, hipStream_t stream,
                      hipEvent_t t0, hipEvent_t t1) {
    if (s.fp8) {
        if (int8 && s.H == 1024 && s.I == 3072) return launch_xcd_t<1024, 3072, Fp8W>(k, debug, stream, t0, t1);
        return set_error(MQ_ERR_UNSUPPORTED, "FP8 weights are compiled for hidden 1024 / intermediate 3072 only "
                         "(H=%d I=%d)", s.H, s.I);
    }
    if (s.H == 1024 && s.I == 3072)
        return int8 ? launch_xcd_t<1024, 3072, Int8W>(k, debug, stream, t0, t1)
                    : launch_xcd_t<1024, 3072, Bf16W>(k, debug, stream, t0, t1);
    if (s.H == 2048 && s.I == 6144 && int8) return launch_xcd_t<2048, 6144, Int8W>(k, debug, stream, t0, t1);
    return set_error(MQ_ERR_UNSUPPORTED, "no XCD decode kernel for H=%d I=%d (%s)", s.H, s.I, int8 ? "int8" : "bf16");
}

}  // namespace mq
