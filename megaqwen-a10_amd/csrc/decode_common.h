// Pieces shared by the two decode kernels (decode.hip: one exchange level
// over all 256 workgroups; decode_xcd.hip: XCD-local exchanges plus two
// cross-XCD reductions per layer): launch shape, kernel arguments, the
// register-staged matvec stage and a workgroup sum.
#pragma once

#include "common.h"
#include "internal.h"

namespace mq {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kNWG = 256;
constexpr int kMaxAttnLen = 1024;     // positions one workgroup attends over (fp64 scores in LDS)
constexpr int kKvLds = 64;            // earlier positions whose K/V rows are prefetched into LDS
constexpr int kSplitRanks = 32;       // XCD kernel: workgroups sharing one KV head's split attention
constexpr int kDefaultSplitMin = 48;  // XCD kernel: default cache_len from which attention is split
constexpr int kMaxLayers = 64;        // per-layer pointer tables cached in LDS
constexpr int kTracePoints = 10;      // timestamps per layer in the optional trace
constexpr double kEps = 1e-6;        // RMSNorm epsilon (config.cuh:40), applied in fp64

enum Stage { ST_QKV = 0, ST_ATTN = 1, ST_O = 2, ST_GU = 3, ST_DOWN = 4 };

struct KArgs {
    int token;
    int* out_token;
    const uint16_t* embed;
    const LayerWeights* lw;
    const ScalePointers* sp;
    const uint16_t* final_norm;
    const uint8_t* lm_w;
    const float* lm_s;
    const uint16_t* cos_t;
    const uint16_t* sin_t;
    uint16_t* kc;
    uint16_t* vc;
    uint16_t* dbg_hidden;
    float* dbg_act;
    float* dbg_resid;
    float* dbg_q;
    float* dbg_k;
    float* dbg_v;
    float* dbg_attn;
    float* dbg_mlp;
    float* dbg_norm;
    float* dbg_bmax;
    int* dbg_bidx;
    int L, pos, cache_len, S, V;
    int split_min;                         // XCD kernel: split attention over the ranks from this cache_len on
    float attn_scale;
    uint32_t spin_limit;
    uint64_t* trace;
    uint8_t* ws;
    uint32_t* status_out;                  // optional: the step's abort flag (0 = completed), stored with the token
    // Steps per launch (async kernel; the others run one): step s decodes at position pos + s,
    // its input token is step_tokens[s] for s < n_forced (token when step_tokens is NULL) and
    // the previous step's output after that; tokens_out[s - (n_forced - 1)] receives the
    // output of every step from the last forced one on, out_token the last step's.
    int n_steps;
    int n_forced;
    const int* step_tokens;
    int* tokens_out;
    float inv_temp;                        // 0: greedy argmax; > 0: sample at temperature 1 / inv_temp
    uint64_t seed;                         // sampling seed
};

// Gumbel noise for sampling at position pos, vocabulary row `row`: 23 bits of
// SplitMix64 (Steele, Lea, Flood 2014) of seed ^ ((pos << 32 | row) * golden ratio)
// give u = (m + 0.5) 2^-23 in (0, 1), exact in fp32, and g = -log(-log(u)). The
// argmax over rows of logit / T + g is a sample of softmax(logits / T) (the
// Gumbel-max identity), and the noise depends only on (seed, position, row), so a
// device-side loop and one launch per step draw the same tokens.
__device__ __forceinline__ float gumbel_noise(uint64_t seed, int pos, int row) {
    uint64_t z = seed ^ ((((uint64_t)(uint32_t)pos << 32) | (uint64_t)(uint32_t)row) * 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const float u = ((float)(uint32_t)(z >> 41) + 0.5f) * 0x1p-23f;
    return -logf(-logf(u));
}

constexpr size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Workspace layout (after the 256-byte header): one 64-bit exchange word per
// element of each handed-over vector, every region 256-byte aligned.
struct Layout {
    size_t hid, qkv, att, act, mlp, total;
};
constexpr Layout layout_for(int H, int I, int NQ, int NKV, int D) {
    Layout o{};
    o.hid = sizeof(WsHeader);
    o.qkv = o.hid + round256((size_t)H * 8);
    o.att = o.qkv + round256(((size_t)NQ * D + 2 * (size_t)NKV * D) * 8);
    o.act = o.att + round256((size_t)NQ * D * 8);
    o.mlp = o.act + round256((size_t)H * 8);
    o.total = o.mlp + round256((size_t)I * 8);
    return o;
}

// ---- XCD-aware kernel (decode_xcd.hip): roles and workspace regions ----
constexpr int kNX = 8;                 // XCDs, one KV head each (the 8-term reductions below assume 8)
constexpr int kGS = kNWG / kNX;        // workgroups per XCD

enum XStage { XS_QKV = 0, XS_PO = 1, XS_ACT = 2, XS_MLP = 3, XS_PD = 4, XS_HID = 5, XS_ATP = 6, XS_ATO = 7 };
constexpr uint32_t kXStages = 8;
// split attention partial of one rank: 256 fp64 weighted sums (low word, high
// word), then per head the fp32 maximum and the fp64 probability sum (3 words)
constexpr int kAttWords = 2 * 256 + 2 * 3;

struct XLayout {
    size_t qkvx, actx, mlpx, hidx, lmg, po, pd, attp, atto, tokw, tok, total;
};
// The regions follow the single-level kernel's (layout_for), so neither kernel
// writes words the other could take for its own: the packed words below carry
// a one-bit tag only.
constexpr XLayout xlayout_for(int H, int I) {
    XLayout o{};
    size_t off = layout_for(H, I, 16, 8, 128).total;
    o.qkvx = off; off += round256((size_t)kNX * 512 * 8);
    o.actx = off; off += round256((size_t)kNX * H * 8);
    o.mlpx = off; off += round256((size_t)kNX * (I / kNX) * 8);
    o.hidx = off; off += round256((size_t)kNX * H * 8);
    o.lmg = off; off += round256((size_t)kNWG * 2 * 8);        // LM-head maxima [workgroup][key, index]
    o.po = off; off += round256((size_t)kNX * H * 8);          // packed fp64 partials [xcd][row]
    o.pd = off; off += round256((size_t)kNX * H * 8);
    o.attp = off; off += round256((size_t)kNX * kGS * kAttWords * 8);
    o.atto = off; off += round256((size_t)kNX * 256 * 8);
    o.tokw = off; off += 256;                                   // a multi-step launch's token word
    o.tok = off; off += round256((size_t)kSplitRanks * kMaxAttnLen * 4);   // a launch's forced input tokens
    o.total = off;
    return o;
}

constexpr size_t xlayout_total(int H, int I) { return xlayout_for(H, I).total; }

constexpr int pow2ceil(int x) { return x <= 1 ? 1 : 2 * pow2ceil((x + 1) / 2); }

// One matvec stage of a workgroup: ROWS rows of K inputs, split into (row,
// 1 KB chunk) items handed round-robin to waves W0..7 (a stage whose wave 0
// polls a cross-XCD exchange leaves it out, so that its polls are not queued
// behind weight loads: loads return in order). Weights are loaded into
// registers by load() ahead of the input wait; compute() leaves one fp64
// partial sum per item in `part` (the input vector is fp64 in per-lane order,
// xd_index()). Items past the end get zero weights, so compute() runs every
// item slot without branches and the FMA chains of the items interleave.
template <class W, int ROWS, int K, int W0 = 0>
struct Stage_ {
    static constexpr int NWV = kWaves - W0;
    static constexpr int CHUNK = 64 * W::kPerLane;
    static constexpr int CH = K / CHUNK;
    static constexpr int ITEMS = ROWS * CH;
    static constexpr int IPW = (ITEMS + NWV - 1) / NWV;
    static constexpr int R = pow2ceil(IPW);
    static_assert(K % CHUNK == 0, "row length must be a whole number of 1 KB chunks");
    uint4 w[IPW];

    template <class RowPtr>
    __device__ __forceinline__ void load(RowPtr rowptr, int wave, int lane) {
        if (wave < W0) return;
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const int it = (wave - W0) + NWV * j;
            w[j] = make_uint4(0, 0, 0, 0);
            if (it < ITEMS) w[j] = ldg16_stream(rowptr(it / CH) + (it % CH) * 1024 + lane * 16);
        }
    }
    __device__ __forceinline__ void compute(const double2* xd, double* part, int wave, int lane) const {
        if (wave < W0) return;
        double acc[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int it = (wave - W0) + NWV * j;
            acc[j] = j < IPW ? dot_fragd<W>(w[j], xd, it % CH, lane, 0.0) : 0.0;
        }
        const double s = transpose_reduce64<R>(acc, lane);
        constexpr int span = kWave / R;
        const int j = lane / span;
        if ((lane % span) == 0 && j < IPW) {
            const int it = (wave - W0) + NWV * j;
            if (it < ITEMS) part[it] = s;
        }
    }
    __device__ __forceinline__ static double row_sum(const double* part, int row) {
        double s = 0.0;
#pragma unroll
        for (int c = 0; c < CH; ++c) s += part[row * CH + c];
        return s;
    }
};

// Sum of N doubles held in LDS, as a fixed pairwise tree (3 levels for 8).
template <int N>
__device__ __forceinline__ double tree_sum(const double* r) {
    double t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = r[i];
#pragma unroll
    for (int s = N / 2; s > 0; s /= 2)
#pragma unroll
        for (int i = 0; i < s; ++i) t[i] += t[i + s];
    return t[0];
}

// Workgroup sum in fp64: wave sums, then a fixed tree over the N wave sums
// (every thread gets the same value). `red` holds 2N doubles; consecutive
// calls use different halves (`half`), so the previous call's readers are
// ordered by that call's barrier and no leading barrier is needed.
template <int N>
__device__ __forceinline__ double block_sum64(double v, double* red, int half, int wave, int lane) {
    v = wave_sum64(v);
    double* r = red + half * N;
    if (lane == 0) r[wave] = v;
    __syncthreads();
    return tree_sum<N>(r);
}

// Workgroup barrier for data in LDS only: this wave's LDS operations complete, then
// s_barrier. __syncthreads (a workgroup-scope release fence) also waits for every
// outstanding global load, LDS-direct loads among them; loads issued before this
// barrier stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// block_sum64 with lds_barrier
template <int N>
__device__ __forceinline__ double block_sum64_lds(double v, double* red, int half, int wave, int lane) {
    v = wave_sum64(v);
    double* r = red + half * N;
    if (lane == 0) r[wave] = v;
    lds_barrier();
    return tree_sum<N>(r);
}

// 1/sqrt(v) for v > 0 in fp64: the hardware estimate refined by two Newton
// steps y <- y (3/2 - v/2 y^2). Each step squares the relative error, so the
// result is within about an ulp of the correctly rounded value (the estimate's
// error is far below 2^-14), with 7 dependent operations instead of the ~25 of
// an IEEE sqrt followed by an IEEE division.
__device__ __forceinline__ double rsqrt_nr(double v) {
    double y = __builtin_amdgcn_rsq(v);
    const double h = 0.5 * v;
#pragma unroll
    for (int i = 0; i < 2; ++i) y = fma(y, fma(-h * y, y, 0.5), y);
    return y;
}

// XCD-local exchange store. A wavefront-scope relaxed atomic store is a plain
// global_store (no cache-scope bits): the CU's L1 is write-through, so the word
// lands in this XCD's shared L2, where the other ranks' agent-scope loads (which
// bypass their own L1) read it about twice as fast as an agent-scope store
// (measured on MI355X: 0.27 us vs 0.52 us one-way). It is not visible to other
// XCDs, which never read these buffers.
__device__ __forceinline__ void ll_put_xcd(uint64_t* p, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__device__ __forceinline__ uint32_t hw_xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xfu;
}

// 1/v for finite v > 0: hardware estimate and two Newton steps r <- r (2 - v r).
__device__ __forceinline__ double rcp_nr(double v) {
    double r = __builtin_amdgcn_rcp(v);
#pragma unroll
    for (int i = 0; i < 2; ++i) r = fma(r, fma(-v, r, 1.0), r);
    return r;
}

// SiLU(g) * u = g / (1 + e^-g) * u in fp64 (config.cuh:81-83); 0 where e^-g overflows.
__device__ __forceinline__ double silu_mul(double g, double u) {
    const double e = exp(-g);
    return e == INFINITY ? 0.0 : g * rcp_nr(1.0 + e) * u;
}

// RMSNorm scale 1/sqrt(mean + eps) in fp64.
__device__ __forceinline__ double rms_scale(double sumsq, int n, double eps) {
    return rsqrt_nr(sumsq / (double)n + eps);
}


// All kNWG workgroups wait on each other, so they must be resident at once:
// checked once per (kernel, device) with the occupancy calculator.
int check_residency(const void* fn, int threads = kThreads);
// Launch of a kernel whose workgroups wait on each other: a plain launch (start/stop events
// recorded by the dispatch when given), or with set_cooperative_launch(1) a cooperative one,
// which the runtime starts only when every workgroup can be resident at once (events then
// recorded around it on the stream).
hipError_t launch_resident(const void* fn, dim3 grid, dim3 block, void** args, hipStream_t stream,
                           hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);

// Async-wave kernel (decode_async.hip): INT8 Qwen3-0.6B shape, cache_len <= 2048 (split
// attention past 64).
size_t decode_async_workspace_bytes(const DecodeShape& s);
bool decode_async_supports(const DecodeShape& s, bool int8, int cache_len);
int decode_async_auto_len();
int launch_decode_async(const KArgs& k, bool debug, bool int4, hipStream_t stream, hipEvent_t t0, hipEvent_t t1);

// XCD-aware kernel (decode_xcd.hip).
size_t decode_xcd_workspace_bytes(const DecodeShape& s);
const void* decode_xcd_kernel_ptr(const DecodeShape& s, bool int8, bool debug);
int launch_decode_xcd(const KArgs& k, const DecodeShape& s, bool int8, bool debug, hipStream_t stream,
                      hipEvent_t t0, hipEvent_t t1);

}  // namespace mq
