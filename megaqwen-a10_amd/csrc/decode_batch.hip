// Batched INT8 decode step: B <= 16 independent sequences share one pass over
// the weights (the reference has no batched path, its
// semantics are B copies of a10_int8_decode_kernel.cu:621-815).
//
// Same XCD roles as decode_xcd.hip: workgroup g runs on XCD x = HW_REG_XCC_ID
// as rank r = g / 8 of 32; KV head x belongs to XCD x, and rank r of every XCD
// owns hidden rows [64r, 64r + 64) of every sequence. Per layer:
//
//   A  QKV, K-sliced   rank r = 8q + s: rows [128q, +128) of XCD x's 512 q|k|v
//                      rows x hidden elements [256s, +256) (gathered from the 4
//                      ranks owning them, times the input-norm gains) -> XCD-
//                      local partials
//   B  attention       rank b < B: sequence b -- sums its 512 rows over the 8
//                      slices, applies the RMSNorm and row scales, then QK-norm,
//                      RoPE, cache write, softmax over its KV cache (attention.h)
//   C  O, row-split    rank r: rows [64r, +64) x XCD x's 256 attention dims
//                                                             -> cross-XCD partials
//   D  reduce          rank r: its 64 rows over the 8 XCDs, scale, residual
//                                                             -> XCD-local rows
//   E  gate/up, K-sliced  as A over XCD x's 768 channels (1536 rows, 384 per
//                      row group); rank r reduces channels [24r, +24), SwiGLU
//                                                             -> XCD-local
//   F  down, row-split rank r: rows [64r, +64) x XCD x's 768 channels -> cross-XCD
//   G  reduce          rank r: its 64 rows, scale, residual, bf16 -> XCD-local rows
//
// The products run on the matrix cores (v_mfma_i32_16x16x64_i8): the int8
// weights are the B operand straight from HBM, and each activation vector
// x (one per sequence) becomes four int8 digits over a power-of-two scale 2^e
// (e with max |x| < 2^e): X = trunc(x 2^(28-e)) = d0 2^21 + d1 2^14 + d2 2^7 + d3,
// d0 in [-128, 127], d1..d3 in [0, 127]. The A operand holds the digit rows
// (4 sequences x 4 digits per 16-row tile), so the result lane of a (sequence,
// weight row) pair holds its four digit sums and recombines them exactly in
// fp64 (integer sums, no rounding). Approximations: x is truncated to 28 bits
// below its vector's maximum, and in stages A and E (whose K slices are local)
// x is the product of the hidden value and the norm gain, the RMSNorm scale
// being applied after the reduction -- the reference rounds the normalised
// value to fp32 first. Projections therefore differ from the single-sequence
// path by ~1e-8 relative, which can flip an occasional bf16 rounding.
#include "attention.h"

#include <hip/hip_ext.h>

namespace mq {

namespace {

constexpr int kBMax = 16;               // sequences per step
constexpr int kBX = 8;                  // XCDs
constexpr int kBG = kNWG / kBX;         // ranks per XCD
constexpr int kSl = 64;                 // hidden elements per rank
constexpr int kD = 128;                 // head dim
constexpr int kSliceB = 192;            // longest sequence whose K/V rows stage B loads straight into LDS
constexpr int kLmTiles = 5;             // LM-head 16-row tiles per wave
constexpr int kLmRowsPerWG = 16 * kLmTiles * kWaves;

enum BStage { BS_ATT = 1, BS_MLP = 2, BS_ACT = 3, BS_HID = 4 };    // tag stages (0 unused)
constexpr uint32_t kBStages = 5;
constexpr int kKS = 256;                // stages A and E: K slice of a rank
constexpr int kNSl = 8;                 // K slices (rank r takes slice r % 8, row group r / 8)

typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct BArgs {
    int tok[kBMax];
    int pos[kBMax];
    int* out;
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
    int B, L, S, V;
    float attn_scale;
    uint32_t spin_limit;
    uint8_t* ws;
    uint16_t* dbg_hidden;                // optional bf16 [B][H]
    float* dbg_attn;                     // optional fp32 [B][16 * 128]
    float* dbg_act;                      // optional fp32 [B][H]
    float* dbg_mlp;                      // optional fp32 [B][I]
    float* dbg_qkv;                      // optional fp32 [B][8][512] (this XCD's q|k|v rows before RoPE)
    uint64_t* trace;                     // optional [(L + 1) * kTracePoints * kNWG] timeline
};

// Exchange regions (64-bit words). "Packed" buffers hold fp64 values with a
// one-bit parity tag (pack_tagged), written exactly once per layer; the others
// carry a 32-bit payload and a (step, layer, stage) tag.
struct BLayout {
    size_t qp, qss, atto, po, actx, ep, ess, mlpx, pd, hidx, lme, lmd, lmx, lmc, total;
};
// Every layout puts the index that consecutive lanes of the writer and of the
// reader step through last (coalesced stores and loads).
constexpr BLayout blayout_for(int H, int I) {
    const int IX = I / kBX;
    BLayout o{};
    size_t off = 256;
    o.qp = off;   off += round256((size_t)kBX * kNSl * kBMax * 512 * 8);     // [x][slice][b][row 512]
    o.qss = off;  off += round256((size_t)kBX * kBMax * kNSl * 8);           // [x][b][slice]
    o.atto = off; off += round256((size_t)kBX * kBMax * 256 * 8);            // [x][b][dim 256]
    o.po = off;   off += round256((size_t)kBX * kBMax * H * 8);              // [xcd][b][row]
    o.actx = off; off += round256((size_t)kBX * kBMax * H * 8);              // [x][b][row]
    o.ep = off;   off += round256((size_t)kBX * kNSl * kBMax * 2 * IX * 8);  // [x][slice][b][row 2 IX]
    o.ess = off;  off += round256((size_t)kBX * kBMax * kNSl * 8);           // [x][b][slice]
    o.mlpx = off; off += round256((size_t)kBX * kBMax * IX * 8);             // [x][b][channel]
    o.pd = off;   off += round256((size_t)kBX * kBMax * H * 8);              // [xcd][b][row]
    o.hidx = off; off += round256((size_t)kBX * kBMax * H * 8);              // [x][b][row]
    o.lme = off;  off += round256((size_t)kBX * kBMax * kBG * 8);           // [x][b][src]
    o.lmd = off;  off += round256((size_t)kBX * kBG * 64 * 16 * 8);         // [x][src][digit row][word]
    o.lmx = off;  off += round256((size_t)kBX * kBG * kBMax * 2 * 8);       // [x][rank][b][2]
    o.lmc = off;  off += round256((size_t)kBX * kBMax * 2 * 8);             // [x][b][2]
    o.total = off;
    return o;
}

// Exponent e with |v| < 2^e for every |v| <= mx (0 for mx = 0).
__device__ __forceinline__ int digit_exp(double mx) {
    int e = 0;
    if (mx > 0.0) (void)frexp(mx, &e);
    return e;
}

// X = trunc(v 2^(28-e)), |X| < 2^28 for |v| < 2^e (the scaling is exact).
__device__ __forceinline__ int fixed28(double v, int e) { return (int)ldexp(v, 28 - e); }

// The four digit bytes of X0..X3 packed per digit: out[d] holds digit d of
// X0 | X1 << 8 | X2 << 16 | X3 << 24. Digit d of X is byte 3 - d of X << (3 - d)
// (bits 21 - 7d .. 28 - 7d of X), masked to 7 bits for d > 0.
__device__ __forceinline__ void digit_words(const int* X, uint32_t* out) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const int sh = 3 - d;
        const uint32_t y0 = (uint32_t)X[0] << sh, y1 = (uint32_t)X[1] << sh;
        const uint32_t y2 = (uint32_t)X[2] << sh, y3 = (uint32_t)X[3] << sh;
        // byte sh of each y into bytes 0..3 (v_perm_b32 picks byte i of {src0:src1} for
        // selector value i, src1 holding bytes 0-3)
        const uint32_t sel = 0x0c0c0400u + 0x0101u * (uint32_t)sh;
        const uint32_t t01 = __builtin_amdgcn_perm(y1, y0, sel);
        const uint32_t t23 = __builtin_amdgcn_perm(y3, y2, sel);
        const uint32_t w = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
        out[d] = d == 0 ? w : (w & 0x7f7f7f7fu);
    }
}

// Value of a (sequence, row) pair from its four digit sums (exact in fp64).
__device__ __forceinline__ double digit_value(i32x4_t c, int e) {
    const double v = ((double)c[0] * 2097152.0 + (double)c[1] * 16384.0) + ((double)c[2] * 128.0 + (double)c[3]);
    return ldexp(v, e - 28);
}

__device__ __forceinline__ i32x4_t as_i32x4(uint4 u) {
    i32x4_t v;
    __builtin_memcpy(&v, &u, 16);
    return v;
}

__device__ __forceinline__ i32x4_t mfma8(i32x4_t a, i32x4_t b, i32x4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ double sum_tree(double (&v)[N]) {
#pragma unroll
    for (int s = N / 2; s > 0; s /= 2)
#pragma unroll
        for (int i = 0; i < s; ++i) v[i] += v[i + s];
    return v[0];
}

// Chunked vector layout of the gathers: lane c (0..31) of a sequence's 32-lane
// group holds elements 2 (c + 32 j) and 2 (c + 32 j) + 1 for j = 0, 1, ..., so
// every 16-byte exchange read (two words) of the group is contiguous with its
// neighbours'. The bf16 pairs at those elements of p, as 4 words (j = 0..3).
__device__ __forceinline__ uint4 slice_pairs(const uint16_t* p, int c) {
    const __attribute__((address_space(1))) uint32_t* q = gview(reinterpret_cast<const uint32_t*>(p));
    return make_uint4(q[c], q[c + 32], q[c + 64], q[c + 96]);
}

// Digit rows of 8 chunked values (two groups of 4: v[4h..4h+3] are chunks 2h and
// 2h + 1): digit d of chunk j goes to the 16-bit slot c + 32 j of row d.
__device__ __forceinline__ void put_digit_chunks(uint8_t* row0, int pitch, int c, const int (&X)[4], int h) {
    uint32_t dw[4];
    digit_words(X, dw);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint16_t* row = reinterpret_cast<uint16_t*>(row0 + d * pitch);
        row[c + 32 * (2 * h)] = (uint16_t)dw[d];
        row[c + 32 * (2 * h + 1)] = (uint16_t)(dw[d] >> 16);
    }
}

// Sums of v[0..15] over the 8 lanes of each aligned lane octet, transposed:
// afterwards v[0], v[1] of lane j (j = lane % 8) hold the octet's sums of
// entries 2j and 2j + 1 (three halving exchange levels, lane bits 4, 2, 1).
__device__ __forceinline__ void xcd_transpose_sum(double (&v)[kBMax], int lane) {
    transpose_level64<4, 16>(v, lane);
    transpose_level64<2, 8>(v, lane);
    transpose_level64<1, 4>(v, lane);
}

}  // namespace

template <int H, int I>
__global__ void __launch_bounds__(kThreads, 1) decode_batch_kernel(BArgs a) {
    constexpr int IX = I / kBX;              // gate/up channels of one XCD
    constexpr int RPW = H / kBG;             // O / down rows of one rank (= kSl)
    constexpr int KC = 2 * kD;               // attention dims of one XCD (stage C's K)
    constexpr int KPC = KC + 16;             // digit row pitch in bytes (stage C), padded against bank conflicts
    constexpr int KPF = IX + 16;             // same for stage F
    constexpr int KSC = KC / 64, KSF = IX / 64;        // k-steps of stages C and F
    constexpr int KPA = kKS + 16;            // digit row pitch, stages A and E
    constexpr int NTE = 2 * IX / 4 / 16 / kWaves;      // stage E weight tiles per wave (per row group)
    constexpr BLayout kLay = blayout_for(H, I);
    static_assert(RPW == kSl && H == kBG * kSl && H == kNSl * kKS, "hidden slices");
    static_assert(IX == kBG * 24 && IX % 64 == 0 && 2 * IX == 4 * 16 * kWaves * NTE, "gate/up split");
    static_assert(512 == 4 * 16 * kWaves, "QKV split: 16 rows per wave and row group");
    static_assert(RPW / 16 * 2 == kWaves && KSC % 2 == 0 && KSF % 2 == 0, "row-split stages: 2 waves per tile");
    static_assert(kKS == 64 * 4 && KC == 64 * 4 && IX == 64 * 12, "chunked gathers: 4, 4 and 12 chunks per lane");
    static_assert(RPW == 64 && kBX == 8 && kWaves == 8 && kWave == 64, "D/G reductions: 8 XCDs x 32 row pairs x 2 sequences per pass");

    // LDS
    __shared__ LayerWeights s_lw[kMaxLayers];
    __shared__ ScalePointers s_sp[kMaxLayers];
    __shared__ float hid_s[kBMax][kSl];       // this rank's hidden rows (bf16 values)
    __shared__ float act_s[kBMax][kSl];       // this rank's post-attention residual rows
    __shared__ int es[kBMax];                 // digit exponents of the current matvec input
    __shared__ double rs[kBMax];              // RMSNorm scales
    __shared__ float att_in[512];
    __shared__ float lm_v[kWaves][kBMax];
    __shared__ int lm_i[kWaves][kBMax];
    __shared__ uint32_t rope_s[2][kD];        // attention rank: cos / sin row of its position (bf16 bits)
    __shared__ __align__(16) uint32_t vsl[kSliceB][kD / 2];   // attention rank, short sequences: V rows
    constexpr size_t kBigF = (size_t)64 * KPF + (size_t)4 * 4 * 64 * 16;          // F digits + pair partials
    constexpr size_t kBigLM = (size_t)8 * 64 * 64;                                  // 8 k-steps of LM digits
    constexpr size_t kBig0 = sizeof(AttnShared<kSliceB>) > kBigF ? sizeof(AttnShared<kSliceB>) : kBigF;
    constexpr size_t kBig = kBig0 > kBigLM ? kBig0 : kBigLM;
    __shared__ __align__(16) uint8_t big[kBig];
    AttnShared<kSliceB>& at = *reinterpret_cast<AttnShared<kSliceB>*>(big);
    uint8_t* const dg = big;                                      // digit rows
    i32x4_t* const cred = reinterpret_cast<i32x4_t*>(big + (size_t)64 * KPF);   // pair partials [nt][mg][lane]
    double* const gu = reinterpret_cast<double*>(big + 64 * KPA); // stage E reducer sums [48][16]

    const int g = blockIdx.x;
    const int x = (int)hw_xcc_id();
    const int r = g / kBX;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int B = a.B;
    const int MG = (B + 3) / 4;               // 16-row digit tiles (4 sequences each)

    WsHeader* hdr = reinterpret_cast<WsHeader*>(a.ws);
    uint64_t* const qp = reinterpret_cast<uint64_t*>(a.ws + kLay.qp) + (size_t)x * kNSl * kBMax * 512;
    uint64_t* const qss = reinterpret_cast<uint64_t*>(a.ws + kLay.qss) + (size_t)x * kBMax * kNSl;
    uint64_t* const atto = reinterpret_cast<uint64_t*>(a.ws + kLay.atto) + (size_t)x * kBMax * 256;
    uint64_t* const po = reinterpret_cast<uint64_t*>(a.ws + kLay.po);
    uint64_t* const ep = reinterpret_cast<uint64_t*>(a.ws + kLay.ep) + (size_t)x * kNSl * kBMax * 2 * IX;
    uint64_t* const ess = reinterpret_cast<uint64_t*>(a.ws + kLay.ess) + (size_t)x * kBMax * kNSl;
    uint64_t* const actx = reinterpret_cast<uint64_t*>(a.ws + kLay.actx) + (size_t)x * kBMax * H;
    uint64_t* const hidx = reinterpret_cast<uint64_t*>(a.ws + kLay.hidx) + (size_t)x * kBMax * H;
    uint64_t* const mlpx = reinterpret_cast<uint64_t*>(a.ws + kLay.mlpx) + (size_t)x * kBMax * IX;
    uint64_t* const pd = reinterpret_cast<uint64_t*>(a.ws + kLay.pd);
    uint64_t* const lme = reinterpret_cast<uint64_t*>(a.ws + kLay.lme) + (size_t)x * kBMax * kBG;
    uint64_t* const lmd = reinterpret_cast<uint64_t*>(a.ws + kLay.lmd) + (size_t)x * kBG * 64 * 16;
    uint64_t* const lmx = reinterpret_cast<uint64_t*>(a.ws + kLay.lmx) + (size_t)x * kBG * kBMax * 2;
    uint64_t* const lmc = reinterpret_cast<uint64_t*>(a.ws + kLay.lmc);

    // step-independent reads first
    {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.lw);
        uint64_t* dst = reinterpret_cast<uint64_t*>(s_lw);
        for (int i = tid; i < a.L * 11; i += kThreads) dst[i] = src[i];
        const uint64_t* ssrc = reinterpret_cast<const uint64_t*>(a.sp);
        uint64_t* sdst = reinterpret_cast<uint64_t*>(s_sp);
        for (int i = tid; i < a.L * 7; i += kThreads) sdst[i] = ssrc[i];
        for (int i = tid; i < kBMax * kSl; i += kThreads) {
            const int b = i / kSl, k = i % kSl;
            hid_s[b][k] = b < B ? bf16_bits_to_f32(gview(a.embed)[(int64_t)a.tok[b] * H + kSl * r + k]) : 0.0f;
        }
    }
    const uint32_t E = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t BS = __hip_atomic_load(&hdr->bsteps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t hb = __hip_atomic_load(&hdr->batch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t tps = kBStages * (uint32_t)a.L + 4u;
    auto tag = [&](int l, int st) -> uint32_t { return ((E * tps + kBStages * (uint32_t)l + (uint32_t)st) << 2) | 2u; };
    auto pbit = [&](int l) -> uint32_t { return (BS * (uint32_t)a.L + (uint32_t)l + 1u) & 1u; };
    Waiter wt(&hdr->abort_flag, a.spin_limit);
    auto trace = [&](int l, int point) {
        if (a.trace != nullptr && threadIdx.x == 0)
            a.trace[((int64_t)l * kTracePoints + point) * kNWG + g] = __builtin_amdgcn_s_memrealtime();
    };
    // a device with other than 8 XCDs, or a workspace last used with another batch
    // size, cannot run this step: flag it (the waits then end at once)
    if (x >= kBX || (hb != 0u && hb != (uint32_t)B)) {
        if (tid == 0) __hip_atomic_store(&hdr->abort_flag, x >= kBX ? 2u : 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int last = a.L - 1;
    const int64_t head_stride = (int64_t)a.S * kD;                 // one KV head of one layer
    const int64_t seq_stride = (int64_t)a.L * 8 * head_stride;     // one sequence's cache

    // stage-B inputs of the attention rank (sequence r): the RoPE row of its
    // position (in LDS for the whole step) and the K/V rows of the first kKvLds
    // earlier positions (prefetched a layer ahead); the QK-norm gains are loaded
    // in stage B with the query gather
    const bool attn = r < B;
    const int apos = attn ? a.pos[r] : 0;
    // a sequence of at most kSliceB positions has all its earlier K and V rows loaded straight into
    // LDS at the start of stage B (at.kst, vsl) and its scores taken on the matrix cores; a longer
    // one uses the rows prefetched a layer ahead and reads the rest inside the attention loops
    const bool sliced = attn && apos < kSliceB;
    if (attn && tid < 2 * kD) {
        const uint16_t* row = (tid < kD ? a.cos_t : a.sin_t) + (int64_t)apos * kD;
        rope_s[tid / kD][tid % kD] = ldg_bits(row + tid % kD);
    }
    constexpr int kPreU4 = 2 * kKvLds * (kD / 8) / kThreads;
    uint4 pre[kPreU4];
    const int npre = (attn && !sliced) ? min(apos, kKvLds) : 0;
    auto prefetch_attn = [&](int ll) {
        if (!attn) return;
        const int64_t cb = (int64_t)r * seq_stride + ((int64_t)ll * 8 + x) * head_stride;
#pragma unroll
        for (int i = 0; i < kPreU4; ++i) {
            const int f = tid + i * kThreads;
            const int side = f / (kKvLds * (kD / 8));
            const int rem = f % (kKvLds * (kD / 8));
            const int j = rem / (kD / 8), c = rem % (kD / 8);
            pre[i] = make_uint4(0, 0, 0, 0);
            if (j < npre) pre[i] = ldg16((side == 0 ? a.kc : a.vc) + cb + (int64_t)j * kD + c * 8);
        }
    };

    // XCD-local QKV row m (0..511): 2 query heads, then K, then V of KV head x
    auto qkv_row = [&](const LayerWeights& lw, const ScalePointers& sp, int m, const uint8_t*& w, const float*& sc) {
        if (m < 256) { w = (const uint8_t*)lw.q_proj_weight + (int64_t)(256 * x + m) * H; sc = sp.q_scale + 256 * x + m; }
        else if (m < 384) { w = (const uint8_t*)lw.k_proj_weight + (int64_t)(128 * x + m - 256) * H; sc = sp.k_scale + 128 * x + m - 256; }
        else { w = (const uint8_t*)lw.v_proj_weight + (int64_t)(128 * x + m - 384) * H; sc = sp.v_scale + 128 * x + m - 384; }
    };
    // stages A and E: this rank's K slice and row group
    const int sl = r % kNSl, rg = r / kNSl;
    // stage A weights: wave w takes rows 128 rg + 16 w + lane % 16 of XCD x's 512, the 16
    // bytes at k = 256 sl + 64 ks + 16 (lane / 16) for k-step ks
    //
    // Only weights are loaded ahead. A stage's scales and norm gains are loaded just
    // before the exchange poll that precedes their use: a value loaded ahead would be
    // live across stages and may be spilled, and a spill store waits for its load,
    // which (loads returning in order) waits for the whole weight batch before it.
    uint4 wA[4];
    auto load_a = [&](int ll) {
        const uint8_t* w; const float* sc;
        qkv_row(s_lw[ll], s_sp[ll], 128 * rg + 16 * wave + lane % 16, w, sc);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) wA[ks] = ldg16(w + kKS * sl + 64 * ks + 16 * (lane / 16));
    };
    // stage C weights: wave w, O rows 64 r + 16 (w / 2) + lane % 16, k-steps 2 (w % 2) + s
    uint4 wC[2];
    // stages D and G: thread t reduces rows 2 cD, 2 cD + 1 of the rank's 64 (see stage D)
    const int cD = ((tid & 63) >> 3) + 8 * ((tid >> 6) & 3);
    auto load_c = [&](int ll) {
        const uint8_t* ob = (const uint8_t*)s_lw[ll].o_proj_weight;
        const int row = RPW * r + 16 * (wave >> 1) + lane % 16;
#pragma unroll
        for (int s = 0; s < 2; ++s)
            wC[s] = ldg16(ob + (int64_t)row * (16 * kD) + KC * x + 64 * (2 * (wave & 1) + s) + 16 * (lane / 16));
    };
    // stage E weights: wave w, tiles j: rows 384 rg + 16 (NTE w + j) + lane % 16 of XCD x's
    // gate (< IX) / up rows, k-steps as in stage A
    uint4 wE[NTE * 4];
    auto load_e = [&](int ll) {
        const LayerWeights& lw = s_lw[ll];
#pragma unroll
        for (int j = 0; j < NTE; ++j) {
            const int m = 2 * IX / 4 * rg + 16 * (NTE * wave + j) + lane % 16;
            const uint8_t* w = m < IX ? (const uint8_t*)lw.gate_proj_weight + (int64_t)(IX * x + m) * H
                                      : (const uint8_t*)lw.up_proj_weight + (int64_t)(IX * x + m - IX) * H;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) wE[4 * j + ks] = ldg16(w + kKS * sl + 64 * ks + 16 * (lane / 16));
        }
    };
    // stage F weights: wave w, down rows 64 r + 16 (w / 2) + lane % 16, k-steps 6 (w % 2) + s
    uint4 wF[KSF / 2];
    auto load_f = [&](int ll) {
        const uint8_t* db = (const uint8_t*)s_lw[ll].down_proj_weight;
        const int row = RPW * r + 16 * (wave >> 1) + lane % 16;
#pragma unroll
        for (int s = 0; s < KSF / 2; ++s)
            wF[s] = ldg16(db + (int64_t)row * I + IX * x + 64 * ((KSF / 2) * (wave & 1) + s) + 16 * (lane / 16));
    };

    // Digits of v = h * gain for the K slice [256 sl, +256) of every sequence: thread
    // t: sequence t / 32, the 8 slice elements of chunks j = 0..3 of lane t % 32
    // (slice_pairs) with values hv and gains g8. Writes digit rows 4b + d (pitch KPA)
    // and es[b]; returns the thread's group sum of h^2 over the slice (32 lanes).
    auto slice_digits = [&](const float (&hv)[8], uint4 g8) -> double {
        const int b = tid >> 5, c = tid & 31;
        const uint32_t gw[4] = {g8.x, g8.y, g8.z, g8.w};
        double v[8], ss = 0.0, mx = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const double h = b < B ? (double)hv[j] : 0.0;
            const uint32_t gb = (j & 1) ? (gw[j >> 1] >> 16) : (gw[j >> 1] & 0xffffu);
            ss = fma(h, h, ss);
            v[j] = h * (double)bf16_bits_to_f32(gb);
            mx = fmax(mx, fabs(v[j]));
        }
        mx = group_max64<32>(mx);
        ss = group_sum64<32>(ss);
        const int e = digit_exp(mx);
        if (b < 4 * MG) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int X[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) X[j] = b < B ? fixed28(v[4 * h + j], e) : 0;
                put_digit_chunks(dg + 4 * b * KPA, KPA, c, X, h);
            }
        }
        if (b < B && (tid & 31) == 0) es[b] = e;
        return ss;
    };

    const int tid_all = tid;
    // every wave reads the pointer tables that all waves copied into LDS above
    __syncthreads();
    load_a(0);
    prefetch_attn(0);
    __syncthreads();

    for (int l = 0; l < a.L; ++l) {
        const int tid = opaque(tid_all);
        const int lane = tid % kWave;
        // the wave index too is rederived per layer: held through the loop, the addresses
        // derived from it were spilled to scratch, and a reload in stage B (its line evicted
        // from L2 by the layer's weight stream) waited about 2 us for memory
        const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        const LayerWeights& lw = s_lw[l];
        const ScalePointers& sp = s_sp[l];
        const uint32_t pb = pbit(l);

        // ---------------- A: QKV partials over the hidden slice [256 sl, +256) ----------------
        trace(l, 0);
        {
            // the slice of every sequence's layer input (the embedding rows at layer 0)
            const int b = tid >> 5, c = tid & 31;
            const uint4 win8 = slice_pairs((const uint16_t*)lw.input_layernorm_weight + kKS * sl, c);
            float hv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (b < B) {
                if (l == 0) {
                    const uint4 e8 = slice_pairs(a.embed + (int64_t)a.tok[b] * H + kKS * sl, c);
                    const uint32_t ew[4] = {e8.x, e8.y, e8.z, e8.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) hv[j] = bf16_bits_to_f32((j & 1) ? (ew[j >> 1] >> 16) : (ew[j >> 1] & 0xffffu));
                } else {
                    uint32_t w[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)(b * H + kKS * sl + 2 * (c + 32 * j));
                    wt.get_pairs<4>(XRegion(hidx, kBMax * H), w, tag(l - 1, BS_HID), hv);
                }
            }
            const double ss = slice_digits(hv, win8);
            if (b < B && (tid & 31) == 0 && rg == 0) ll_put64(&qss[b * kNSl + sl], pack_tagged(ss, pb));
            __syncthreads();
            // stage C's weights (consumed after the attention exchange; issued behind this
            // stage's stores they arrive too late)
            load_c(l);
            issue_fence();
            {
                const int m = 128 * rg + 16 * wave + lane % 16;
#pragma unroll
                for (int mg = 0; mg < 4; ++mg) {
                    if (mg < MG) {
                        i32x4_t c = i32x4_t{0, 0, 0, 0};
#pragma unroll
                        for (int ks = 0; ks < 4; ++ks) {
                            const i32x4_t av = *reinterpret_cast<const i32x4_t*>(dg + (16 * mg + lane % 16) * KPA + 64 * ks + 16 * (lane / 16));
                            c = mfma8(av, as_i32x4(wA[ks]), c);
                        }
                        const int bb = 4 * mg + lane / 16;
                        if (bb < B) ll_put64(&qp[((size_t)sl * kBMax + bb) * 512 + m], pack_tagged(digit_value(c, es[bb]), pb));
                    }
                }
            }
            trace(l, 1);
            // every wave has read the digit rows and es (stage B / C write them next)
            __syncthreads();
        }

        trace(l, 2);
        // ---------------- B: attention of sequence r (ranks r < B) ----------------
        if (attn) {
            const int64_t cache_base = (int64_t)r * seq_stride + ((int64_t)l * 8 + x) * head_stride;
            // a short sequence: waves 4-7 first load its earlier K and V rows straight into LDS.
            // Loads return in order per wave, so only these waves' gather polls come back after
            // them (about when stage A's partials are complete anyway); waves 0-3 poll at once.
            // Stage A's last barrier ordered every read of the LDS they overwrite.
            const bool loader = sliced && __builtin_amdgcn_readfirstlane(wave) >= 4;   // wave-uniform branch
            // (every LDS access of a wave after its LDS-direct loads waits for them, so the pointer
            // tables are read and the row scale is requested first, and the RMSNorm scale is
            // broadcast with a lane read)
            uint32_t scA;
            {
                const uint8_t* w; const float* sc;
                qkv_row(lw, sp, tid, w, sc);
                scA = ldg_bits(sc);
            }
            uint32_t nw0 = 0, nw1 = 0;
            if (wave < 3) {
                const uint16_t* nw = (const uint16_t*)(wave < 2 ? lw.q_norm_weight : lw.k_norm_weight);
                nw0 = ldg_bits(nw + lane);
                nw1 = ldg_bits(nw + lane + 64);
            }
            issue_fence();
            if (loader) {
                const int ln = opaque(lane);    // per-lane offsets are recomputed, not held across layers
                // (from layer 1 on, the K and V rows were loaded at the end of the previous
                // layer's stage F)
                if (l == 0) {
                    attn_slice_k<4>(at, a.kc + cache_base, 0, apos, ln, wave - 4);
                    attn_slice_v_lds<kSliceB, 4>(vsl, a.vc + cache_base, 0, apos, ln, wave - 4);
                }
            }
            {
                // this sequence's 512 q|k|v rows straight from stage A's partials: thread t sums
                // row t over the 8 K slices (written by all 32 ranks of the XCD), times the
                // RMSNorm scale from the slices' sums of squares (lanes 0..7 of every wave) and
                // the row scale
                double qv = 0.0;
                if (lane < kNSl) {
                    double v1[1];
                    wt.get_packed<1>(&qss[r * kNSl + lane], 1, pb, v1);
                    qv = v1[0];
                }
                qv = group_sum64<kNSl>(qv);
                const double rsb = rms_scale(readlane64(qv, 0), H, kEps);
                double v8[kNSl];
                wt.get_packed<kNSl>(&qp[(size_t)r * 512 + tid], kBMax * 512, pb, v8);
                const float y = (float)(sum_tree(v8) * rsb * (double)after_wait_f(scA));
                att_in[tid] = y;
                if (l == last && a.dbg_qkv != nullptr) a.dbg_qkv[((int64_t)r * 8 + x) * 512 + tid] = y;
            }
            if (loader) wait_vmem();            // the slice rows are in LDS after the barrier below
#pragma unroll
            for (int i = 0; i < kPreU4; ++i) {
                const int f = tid + i * kThreads;
                const int side = f / (kKvLds * (kD / 8));
                const int rem = f % (kKvLds * (kD / 8));
                const int j = rem / (kD / 8), c = rem % (kD / 8);
                if (j < npre) *reinterpret_cast<uint4*>(&at.kv_pre[side][j][c * 4]) = pre[i];
            }
            __syncthreads();
            const int64_t cur = cache_base + (int64_t)apos * kD;
            attn_qk_rope(at, att_in, nw0, nw1, rope_s[0][lane], rope_s[1][lane], rope_s[0][lane + 64],
                         rope_s[1][lane + 64], a.kc + cur, a.vc + cur, nullptr, nullptr, nullptr, wave, lane, sliced);
            __syncthreads();
            auto emit = [&](int i, float v) {
                ll_put_xcd(&atto[r * 256 + i], __float_as_uint(v), tag(l, BS_ATT));
                if (l == last && a.dbg_attn != nullptr) a.dbg_attn[(int64_t)r * 2048 + 256 * x + i] = v;
            };
            if (sliced) {
                attn_partial_lds_v<AttnShared<kSliceB>, kSliceB, true>(
                    at, vsl, 0, apos + 1, apos, (double)a.attn_scale, tid, lane, wave,
                    [&](int i, double acc, double l1, double) { emit(i, (float)(acc * rcp_nr(l1))); }, [](int) {});
            } else {
                // up to 1024 positions, most of them read from memory
                attn_core<true>(at, a.kc + cache_base, a.vc + cache_base, apos + 1, apos, (double)a.attn_scale, tid,
                                lane, wave, emit, [](int) {});
            }
            __syncthreads();
        }

        trace(l, 3);
        // ---------------- C: O partials, rows [64r, +64) x XCD x's attention dims ----------------
        {
            // gather: thread t: sequence t / 32, the dims of chunks j = 0..3 of lane t % 32
            const int b = tid >> 5, c = tid & 31;
            float v8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (b < B) {
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) w[j] = (uint32_t)(b * 256 + 2 * (c + 32 * j));
                wt.get_pairs<4>(XRegion(atto, kBMax * 256), w, tag(l, BS_ATT), v8);
            }
            double mx = 0.0;
#pragma unroll
            for (int j = 0; j < 8; ++j) mx = fmax(mx, fabs((double)v8[j]));
            mx = group_max64<32>(mx);
            const int e = digit_exp(mx);
            if (b < 4 * MG) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    int X[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) X[j] = b < B ? fixed28(v8[4 * h + j], e) : 0;
                    put_digit_chunks(dg + 4 * b * KPC, KPC, c, X, h);
                }
            }
            if (b < B && (tid & 31) == 0) es[b] = e;
            __syncthreads();
            const int nt = wave >> 1;
            i32x4_t cm[4];
#pragma unroll
            for (int mg = 0; mg < 4; ++mg) {
                cm[mg] = i32x4_t{0, 0, 0, 0};
                if (mg < MG) {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const int ks = 2 * (wave & 1) + s;
                        const i32x4_t av = *reinterpret_cast<const i32x4_t*>(dg + (16 * mg + lane % 16) * KPC + 64 * ks + 16 * (lane / 16));
                        cm[mg] = mfma8(av, as_i32x4(wC[s]), cm[mg]);
                    }
                }
            }
            if (wave & 1) {
#pragma unroll
                for (int mg = 0; mg < 4; ++mg)
                    if (mg < MG) cred[(nt * 4 + mg) * kWave + lane] = cm[mg];
            }
            __syncthreads();
            if (!(wave & 1)) {
#pragma unroll
                for (int mg = 0; mg < 4; ++mg) {
                    const int bb = 4 * mg + lane / 16;
                    if (mg < MG && bb < B) {
                        const i32x4_t c = cm[mg] + cred[(nt * 4 + mg) * kWave + lane];
                        const int row = RPW * r + 16 * nt + lane % 16;
                        ll_put64(&po[((size_t)x * kBMax + bb) * H + row], pack_tagged(digit_value(c, es[bb]), pb));
                    }
                }
            }
            // stage E's weights, behind this stage's stores: a weight batch fills the CU's
            // memory pipeline for microseconds, and the stores are on the critical path
            issue_fence();
            load_e(l);
            issue_fence();
        }

        trace(l, 4);
        // ---------------- D: O rows [64r, +64) over the 8 XCDs, scale, residual ----------------
        {
            // thread t: the partials of XCD xs = t % 8 for rows 2 cD, 2 cD + 1 of sequences
            // t / 256 + 2 i, one 16-byte chunk each (a wave reads 8 runs of 128 bytes). A
            // transpose-reduction over the 8 lanes of a row pair (one per XCD) leaves lane xs
            // with both rows' sums of sequence t / 256 + 2 xs.
            const int xs = lane & 7, b0 = wave >> 2;
            const int nb = (B - b0 + 1) >> 1;                 // sequences of this wave
            uint32_t w[kBMax / 2];
#pragma unroll
            for (int i = 0; i < kBMax / 2; ++i) w[i] = (uint32_t)((xs * kBMax + b0 + 2 * i) * H + RPW * r + 2 * cD);
            const uint32_t soD0 = ldg_bits(sp.o_scale + RPW * r + 2 * cD);
            const uint32_t soD1 = ldg_bits(sp.o_scale + RPW * r + 2 * cD + 1);
            double v[kBMax];
            wt.get_packed_pairs<kBMax / 2>(XRegion(po, kBX * kBMax * H), w, pb, v, nb);
            xcd_transpose_sum(v, lane);
            if (xs < nb) {
                const int b = b0 + 2 * xs;
                const double sv[2] = {v[0] * (double)after_wait_f(soD0), v[1] * (double)after_wait_f(soD1)};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int rl = 2 * cD + h;
                    const float av = (float)(sv[h] + (double)hid_s[b][rl]);
                    act_s[b][rl] = av;
                    ll_put_xcd(&actx[b * H + RPW * r + rl], __float_as_uint(av), tag(l, BS_ACT));
                    if (l == last && x == 0 && a.dbg_act != nullptr) a.dbg_act[(int64_t)b * H + RPW * r + rl] = av;
                }
            }
        }
        __syncthreads();
        trace(l, 5);
        // ---------------- E: gate/up partials over the slice [256 sl, +256) ----------------
        {
            const int b = tid >> 5, c = tid & 31;
            const uint4 wpost8 = slice_pairs((const uint16_t*)lw.post_attn_layernorm_weight + kKS * sl, c);
            float hv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (b < B) {
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) w[j] = (uint32_t)(b * H + kKS * sl + 2 * (c + 32 * j));
                wt.get_pairs<4>(XRegion(actx, kBMax * H), w, tag(l, BS_ACT), hv);
            }
            const double ss = slice_digits(hv, wpost8);
            if (b < B && (tid & 31) == 0 && rg == 0) ll_put64(&ess[b * kNSl + sl], pack_tagged(ss, pb));
            __syncthreads();
#pragma unroll
            for (int mg = 0; mg < 4; ++mg) {
                if (mg < MG) {
                    i32x4_t av[4];
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks)
                        av[ks] = *reinterpret_cast<const i32x4_t*>(dg + (16 * mg + lane % 16) * KPA + 64 * ks + 16 * (lane / 16));
                    const int bb = 4 * mg + lane / 16;
#pragma unroll
                    for (int j = 0; j < NTE; ++j) {
                        i32x4_t c = i32x4_t{0, 0, 0, 0};
#pragma unroll
                        for (int ks = 0; ks < 4; ++ks) c = mfma8(av[ks], as_i32x4(wE[4 * j + ks]), c);
                        const int m = 2 * IX / 4 * rg + 16 * (NTE * wave + j) + lane % 16;
                        if (bb < B)
                            ll_put64(&ep[((size_t)sl * kBMax + bb) * (2 * IX) + m], pack_tagged(digit_value(c, es[bb]), pb));
                    }
                }
            }
            trace(l, 6);
            // reduce channels [24r, +24) (gate rows 24 r + c, up rows IX + 24 r + c) over the 8 slices
            const uint32_t gsc = ldg_bits(sp.gate_scale + IX * x + 24 * r + tid % 24);
            const uint32_t usc = ldg_bits(sp.up_scale + IX * x + 24 * r + tid % 24);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int p = tid + kThreads * i;
                const int rsel = p % 48, bb = p / 48;
                if (bb < B) {
                    const int m = rsel < 24 ? 24 * r + rsel : IX + 24 * r + rsel - 24;
                    double v8[kNSl];
                    wt.get_packed<kNSl>(&ep[(size_t)bb * (2 * IX) + m], kBMax * 2 * IX, pb, v8);
                    gu[rsel * kBMax + bb] = sum_tree(v8);
                }
            }
            {
                const int b2 = tid >> 3, s2 = tid & 7;
                double qv = 0.0;
                if (tid < 128 && b2 < B) {
                    double v1[1];
                    wt.get_packed<1>(&ess[b2 * kNSl + s2], 1, pb, v1);
                    qv = v1[0];
                }
                qv = group_sum64<kNSl>(qv);
                if (tid < 128 && s2 == 0 && b2 < B) rs[b2] = rms_scale(qv, H, kEps);
            }
            __syncthreads();
            if (tid < 24 * B) {
                const int c = tid % 24, bb = tid / 24;
                const double gs = gu[c * kBMax + bb] * rs[bb] * (double)after_wait_f(gsc);
                const double us = gu[(24 + c) * kBMax + bb] * rs[bb] * (double)after_wait_f(usc);
                const float m = (float)silu_mul(gs, us);
                ll_put_xcd(&mlpx[bb * IX + 24 * r + c], __float_as_uint(m), tag(l, BS_MLP));
                if (l == last && a.dbg_mlp != nullptr) a.dbg_mlp[(int64_t)bb * I + IX * x + 24 * r + c] = m;
            }
            // stage F's weights, behind this stage's stores (its K-slice reduction polls
            // must not queue behind them)
            issue_fence();
            load_f(l);
            issue_fence();
        }

        trace(l, 7);
        // ---------------- F: down partials, rows [64r, +64) x XCD x's channels ----------------
        {
            // gather: thread t: sequence t / 32, the channels of chunks j = 0..11 of lane t % 32
            const int b = tid >> 5, c = tid & 31;
            float v24[24];
#pragma unroll
            for (int j = 0; j < 24; ++j) v24[j] = 0.0f;
            if (b < B) {
                uint32_t w[12];
#pragma unroll
                for (int j = 0; j < 12; ++j) w[j] = (uint32_t)(b * IX + 2 * (c + 32 * j));
                wt.get_pairs<12>(XRegion(mlpx, kBMax * IX), w, tag(l, BS_MLP), v24);
            }
            double mx = 0.0;
#pragma unroll
            for (int j = 0; j < 24; ++j) mx = fmax(mx, fabs((double)v24[j]));
            mx = group_max64<32>(mx);
            const int e = digit_exp(mx);
            __syncthreads();                  // gu (overlaying dg) read above
            if (b < 4 * MG) {
#pragma unroll
                for (int h = 0; h < 6; ++h) {
                    int X[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) X[j] = b < B ? fixed28(v24[4 * h + j], e) : 0;
                    put_digit_chunks(dg + 4 * b * KPF, KPF, c, X, h);
                }
            }
            if (b < B && (tid & 31) == 0) es[b] = e;
            __syncthreads();
            const int nt = wave >> 1;
            i32x4_t cm[4];
#pragma unroll
            for (int mg = 0; mg < 4; ++mg) {
                cm[mg] = i32x4_t{0, 0, 0, 0};
                if (mg < MG) {
#pragma unroll
                    for (int s = 0; s < KSF / 2; ++s) {
                        const int ks = (KSF / 2) * (wave & 1) + s;
                        const i32x4_t av = *reinterpret_cast<const i32x4_t*>(dg + (16 * mg + lane % 16) * KPF + 64 * ks + 16 * (lane / 16));
                        cm[mg] = mfma8(av, as_i32x4(wF[s]), cm[mg]);
                    }
                }
            }
            if (wave & 1) {
#pragma unroll
                for (int mg = 0; mg < 4; ++mg)
                    if (mg < MG) cred[(nt * 4 + mg) * kWave + lane] = cm[mg];
            }
            __syncthreads();
            if (!(wave & 1)) {
#pragma unroll
                for (int mg = 0; mg < 4; ++mg) {
                    const int bb = 4 * mg + lane / 16;
                    if (mg < MG && bb < B) {
                        const i32x4_t c = cm[mg] + cred[(nt * 4 + mg) * kWave + lane];
                        const int row = RPW * r + 16 * nt + lane % 16;
                        ll_put64(&pd[((size_t)x * kBMax + bb) * H + row], pack_tagged(digit_value(c, es[bb]), pb));
                    }
                }
            }
            // the next layer's stage A weights and, on an attention rank, its first K/V rows,
            // behind the stores
            if (l < last) {
                issue_fence();
                load_a(l + 1);
                prefetch_attn(l + 1);
                issue_fence();
                if (sliced) {
                    // a short sequence's K and V rows of the next layer, straight into LDS (its
                    // stage B waits for them): at.kst overlays this stage's pair partials, so
                    // every wave's reads of them come first; vsl is stage B's alone, and stages
                    // G and A do not touch at.kst
                    __syncthreads();
                    if (__builtin_amdgcn_readfirstlane(wave) >= 4) {
                        const int ln = opaque(lane);
                        const int64_t nb = (int64_t)r * seq_stride + ((int64_t)(l + 1) * 8 + x) * head_stride;
                        attn_slice_k<4>(at, a.kc + nb, 0, apos, ln, wave - 4);
                        attn_slice_v_lds<kSliceB, 4>(vsl, a.vc + nb, 0, apos, ln, wave - 4);
                    }
                }
            }
        }

        trace(l, 8);
        // ---------------- G: down rows [64r, +64) over the 8 XCDs, scale, residual, bf16 ----------------
        {
            // as stage D
            const int xs = lane & 7, b0 = wave >> 2;
            const int nb = (B - b0 + 1) >> 1;
            uint32_t w[kBMax / 2];
#pragma unroll
            for (int i = 0; i < kBMax / 2; ++i) w[i] = (uint32_t)((xs * kBMax + b0 + 2 * i) * H + RPW * r + 2 * cD);
            const uint32_t sdG0 = ldg_bits(sp.down_scale + RPW * r + 2 * cD);
            const uint32_t sdG1 = ldg_bits(sp.down_scale + RPW * r + 2 * cD + 1);
            double v[kBMax];
            wt.get_packed_pairs<kBMax / 2>(XRegion(pd, kBX * kBMax * H), w, pb, v, nb);
            xcd_transpose_sum(v, lane);
            if (xs < nb) {
                const int b = b0 + 2 * xs;
                const double sv[2] = {v[0] * (double)after_wait_f(sdG0), v[1] * (double)after_wait_f(sdG1)};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int rl = 2 * cD + h;
                    const float hf = round_bf16((float)(sv[h] + (double)act_s[b][rl]));
                    hid_s[b][rl] = hf;
                    if (l < last) ll_put_xcd(&hidx[b * H + RPW * r + rl], __float_as_uint(hf), tag(l, BS_HID));
                    if (l == last && x == 0 && a.dbg_hidden != nullptr)
                        a.dbg_hidden[(int64_t)b * H + RPW * r + rl] = (uint16_t)f32_to_bf16_bits(hf);
                }
            }
        }
        __syncthreads();
        trace(l, 9);
        (void)lw;
        (void)sp;
    }
    trace(a.L, 0);

    // ---------------- final RMSNorm + LM head + greedy argmax per sequence ----------------
    {
        const uint32_t tl0 = tag(a.L, 0), tl1 = tag(a.L, 1), tl2 = tag(a.L, 2), tl3 = tag(a.L, 3);
        // digits of n = hid * w_final over the whole hidden vector of each sequence:
        // the exponent is the maximum of the 32 slices' exponents (the positive RMSNorm
        // scale does not change the argmax, so it is not applied)
        const int b = tid >> 4, k0 = 4 * (tid & 15);
        double v[4] = {0.0, 0.0, 0.0, 0.0}, mx = 0.0;
        if (b < B) {
            const uint16_t* fw = a.final_norm + kSl * r + k0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = (double)hid_s[b][k0 + j] * (double)bf16_bits_to_f32(gview(fw)[j]);
                mx = fmax(mx, fabs(v[j]));
            }
        }
        mx = group_max64<16>(mx);
        if (b < B && (tid & 15) == 0) ll_put_xcd(&lme[b * kBG + r], (uint32_t)(digit_exp(mx) + 4096), tl0);
        {
            const int b2 = tid >> 5, src = tid & 31;
            int ee = 0;
            if (b2 < B) ee = (int)wt.get(&lme[b2 * kBG + src], tl0) - 4096;
#pragma unroll
            for (int m = 1; m < 32; m <<= 1) ee = max(ee, __shfl_xor(ee, m, kWave));
            if (src == 0 && b2 < B) es[b2] = ee;
        }
        __syncthreads();
        if (b < 4 * MG) {
            int X[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) X[j] = b < B ? fixed28(v[j], es[b]) : 0;
            uint32_t dw[4];
            digit_words(X, dw);
#pragma unroll
            for (int d = 0; d < 4; ++d) ll_put_xcd(&lmd[((size_t)r * 64 + 4 * b + d) * 16 + (k0 >> 2)], dw[d], tl1);
        }

        // this workgroup's LM rows; wave w takes 16-row tiles w, w + 8, ...
        const int r0 = (int)((int64_t)a.V * g / kNWG);
        const int r1 = (int)((int64_t)a.V * (g + 1) / kNWG);
        const int ntl = (r1 - r0 + 15) / 16;
        constexpr int TPW = kLmTiles;
        i32x4_t acc[TPW][4];
#pragma unroll
        for (int i = 0; i < TPW; ++i)
#pragma unroll
            for (int mg = 0; mg < 4; ++mg) acc[i][mg] = i32x4_t{0, 0, 0, 0};
        auto lm_load = [&](int ks, uint4* dst) {
#pragma unroll
            for (int i = 0; i < TPW; ++i) {
                const int row = r0 + 16 * (wave + kWaves * i) + lane % 16;
                dst[i] = make_uint4(0, 0, 0, 0);
                if (row < r1) dst[i] = ldg16(a.lm_w + (int64_t)row * H + 64 * ks + 16 * (lane / 16));
            }
        };
        // weights two k-steps ahead: wb0 holds even k-steps, wb1 odd ones (k-step ks + 2
        // is loaded into the buffer ks has just used)
        uint4 wb0[TPW], wb1[TPW];
        lm_load(0, wb0);
        lm_load(1, wb1);
        for (int q = 0; q < kBG / 8; ++q) {
            // digit rows of k-steps 8q .. 8q + 7 (hidden slices of ranks 8q ..): 8 x 64 rows x 16 words
            __syncthreads();                  // the previous chunk's digits are consumed
            {
                // wave s8 takes k-step 8q + s8: lane l reads words 2 (l % 8), +1 of digit rows
                // 8 i + l / 8 (rows < 16 MG are in use), a contiguous 1 KB per i and wave
                const int s8 = tid >> 6, pr = lane & 7;
                uint32_t w[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) w[i] = (uint32_t)(((8 * q + s8) * 64 + 8 * i + (lane >> 3)) * 16 + 2 * pr);
                float v16[16];
                wt.get_pairs<8>(XRegion(lmd, kBG * 64 * 16), w, tl1, v16, 2 * MG);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (i < 2 * MG) {
                        uint2* dst = reinterpret_cast<uint2*>(dg + ((size_t)s8 * 64 + 8 * i + (lane >> 3)) * 64 + 8 * pr);
                        *dst = make_uint2(__float_as_uint(v16[2 * i]), __float_as_uint(v16[2 * i + 1]));
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int ks = 8 * q + s;
                uint4 (&wcur)[TPW] = (s & 1) ? wb1 : wb0;
#pragma unroll
                for (int mg = 0; mg < 4; ++mg) {
                    if (mg < MG) {
                        const i32x4_t av = *reinterpret_cast<const i32x4_t*>(dg + ((size_t)s * 64 + 16 * mg + lane % 16) * 64 + 16 * (lane / 16));
#pragma unroll
                        for (int i = 0; i < TPW; ++i)
                            if (wave + kWaves * i < ntl) acc[i][mg] = mfma8(av, as_i32x4(wcur[i]), acc[i][mg]);
                    }
                }
                if (ks + 2 < kBG) lm_load(ks + 2, wcur);
            }
        }
        trace(a.L, 1);
        // per lane: best (logit, row) of sequence 4 mg + lane / 16 over its tiles
        float bv[4];
        int bi[4];
#pragma unroll
        for (int mg = 0; mg < 4; ++mg) {
            bv[mg] = -INFINITY;
            bi[mg] = 0x7fffffff;
            const int bb = 4 * mg + lane / 16;
#pragma unroll
            for (int i = 0; i < TPW; ++i) {
                const int row = r0 + 16 * (wave + kWaves * i) + lane % 16;
                if (mg < MG && bb < B && wave + kWaves * i < ntl && row < r1) {
                    const float lv = (float)(digit_value(acc[i][mg], es[bb]) * (double)gview(a.lm_s)[row]);
                    if (lv > bv[mg]) { bv[mg] = lv; bi[mg] = row; }
                }
            }
            // across the 16 lanes of this sequence (lanes with equal lane / 16)
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) {
                const float ov = __shfl_xor(bv[mg], m, kWave);
                const int oi = __shfl_xor(bi[mg], m, kWave);
                if (ov > bv[mg] || (ov == bv[mg] && oi < bi[mg])) { bv[mg] = ov; bi[mg] = oi; }
            }
            if ((lane % 16) == 0 && mg < MG && bb < B) { lm_v[wave][bb] = bv[mg]; lm_i[wave][bb] = bi[mg]; }
        }
        __syncthreads();
        if (tid < B) {
            float v0 = lm_v[0][tid];
            int i0 = lm_i[0][tid];
            for (int w = 1; w < kWaves; ++w)
                if (lm_v[w][tid] > v0 || (lm_v[w][tid] == v0 && lm_i[w][tid] < i0)) { v0 = lm_v[w][tid]; i0 = lm_i[w][tid]; }
            ll_put_xcd(&lmx[((size_t)r * kBMax + tid) * 2], ordered_key(v0), tl2);
            ll_put_xcd(&lmx[((size_t)r * kBMax + tid) * 2 + 1], (uint32_t)i0, tl2);
        }
        // per XCD (rank 0): thread t: sequence t / 32, rank t % 32
        if (r == 0) {
            const int b2 = tid >> 5, src = tid & 31;
            uint32_t kv = 0, iv = 0x7fffffffu;
            if (b2 < B) {
                kv = wt.get(&lmx[((size_t)src * kBMax + b2) * 2], tl2);
                iv = wt.get(&lmx[((size_t)src * kBMax + b2) * 2 + 1], tl2);
            }
#pragma unroll
            for (int m = 1; m < 32; m <<= 1) {
                const uint32_t ok = (uint32_t)__shfl_xor((int)kv, m, kWave);
                const uint32_t oi = (uint32_t)__shfl_xor((int)iv, m, kWave);
                if (ok > kv || (ok == kv && oi < iv)) { kv = ok; iv = oi; }
            }
            if (src == 0 && b2 < B) {
                ll_put(&lmc[((size_t)x * kBMax + b2) * 2], kv, tl3);
                ll_put(&lmc[((size_t)x * kBMax + b2) * 2 + 1], iv, tl3);
            }
            if (x == 0) {
                // thread t < 8 B: sequence t / 8, XCD t % 8
                const int b3 = tid >> 3, xs = tid & 7;
                uint32_t k2 = 0, i2 = 0x7fffffffu;
                if (b3 < B) {
                    k2 = wt.get(&lmc[((size_t)xs * kBMax + b3) * 2], tl3);
                    i2 = wt.get(&lmc[((size_t)xs * kBMax + b3) * 2 + 1], tl3);
                }
#pragma unroll
                for (int m = 1; m < 8; m <<= 1) {
                    const uint32_t ok = (uint32_t)__shfl_xor((int)k2, m, kWave);
                    const uint32_t oi = (uint32_t)__shfl_xor((int)i2, m, kWave);
                    if (ok > k2 || (ok == k2 && oi < i2)) { k2 = ok; i2 = oi; }
                }
                const bool aborted = __hip_atomic_load(&hdr->abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
                if (xs == 0 && b3 < B) a.out[b3] = (aborted || wt.dead) ? -1 : (int)i2;
                __syncthreads();
                if (tid == 0) {
                    __hip_atomic_store(&hdr->batch, (uint32_t)B, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&hdr->bsteps, BS + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&hdr->epoch, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

// ---------------- host side ----------------

size_t decode_batch_workspace_bytes(const DecodeShape& s) {
    if (s.H == 2048 && s.I == 6144) return blayout_for(2048, 6144).total;
    return 0;
}

int launch_decode_batch(const mq_batch_args& a, const DecodeShape& s, hipStream_t stream) {
    if (!(s.H == 2048 && s.I == 6144 && s.NQ == 16 && s.NKV == 8 && s.D == kD))
        return set_error(MQ_ERR_UNSUPPORTED, "no batched decode kernel for H=%d I=%d heads %d/%d x %d", s.H, s.I,
                         s.NQ, s.NKV, s.D);
    if (a.batch < 1 || a.batch > kBMax)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "batch %d not in [1, %d]", a.batch, kBMax);
    if (a.num_layers < 1 || a.num_layers > kMaxLayers)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "num_layers %d not in [1, %d]", a.num_layers, kMaxLayers);
    if (s.V < kNWG || s.V > kNWG * kLmRowsPerWG)
        return set_error(MQ_ERR_UNSUPPORTED, "vocab_size %d outside [%d, %d]", s.V, kNWG, kNWG * kLmRowsPerWG);
    for (int b = 0; b < a.batch; ++b) {
        if (a.input_token_ids[b] < 0 || a.input_token_ids[b] >= s.V)
            return set_error(MQ_ERR_INVALID_ARGUMENT, "sequence %d: token %d outside [0, %d)", b, a.input_token_ids[b], s.V);
        if (a.positions[b] < 0 || a.positions[b] >= a.max_seq_len || a.positions[b] >= kMaxAttnLen)
            return set_error(MQ_ERR_INVALID_ARGUMENT, "sequence %d: position %d outside [0, min(%d, %d))", b,
                             a.positions[b], a.max_seq_len, kMaxAttnLen);
    }
    if (!a.output_token_ids || !a.embed_weight || !a.layer_weights || !a.scales || !a.final_norm_weight ||
        !a.lm_head_weight || !a.lm_head_scale || !a.cos_table || !a.sin_table || !a.k_cache || !a.v_cache)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "null pointer argument");
    const size_t need = decode_batch_workspace_bytes(s);
    if (!a.workspace || a.workspace_bytes < need)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed", need);
    if (!xcd_placement_ok())
        return set_error(MQ_ERR_UNSUPPORTED, "the batched kernel needs each residue class g mod 8 on one XCD");

    BArgs k{};
    for (int b = 0; b < kBMax; ++b) {
        k.tok[b] = b < a.batch ? a.input_token_ids[b] : 0;
        k.pos[b] = b < a.batch ? a.positions[b] : 0;
    }
    k.out = a.output_token_ids;
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
    k.B = a.batch;
    k.L = a.num_layers;
    k.S = a.max_seq_len;
    k.V = s.V;
    k.attn_scale = a.attn_scale;
    k.spin_limit = a.spin_limit ? a.spin_limit : (1u << 21);
    k.ws = static_cast<uint8_t*>(a.workspace);
    k.dbg_hidden = static_cast<uint16_t*>(a.hidden_out);
    k.dbg_qkv = static_cast<float*>(a.qkv_out);
    k.dbg_attn = static_cast<float*>(a.attn_out);
    k.dbg_act = static_cast<float*>(a.act_out);
    k.dbg_mlp = static_cast<float*>(a.mlp_out);
    k.trace = static_cast<uint64_t*>(a.trace);

    const void* fn = reinterpret_cast<const void*>(&decode_batch_kernel<2048, 6144>);
    int st = check_residency(fn);
    if (st != MQ_OK) return st;
    void* args[] = {&k};
    hipEvent_t t0 = static_cast<hipEvent_t>(a.timing_start), t1 = static_cast<hipEvent_t>(a.timing_stop);
    // a plain launch (start/stop events when given): see check_residency
    const hipError_t e = launch_resident(fn, dim3(kNWG), dim3(kThreads), args, stream, t0, t1);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "launch(decode_batch): %s", hipGetErrorString(e));
    return MQ_OK;
}

}  // namespace mq
