// Asynchronous-wave persistent decode step: the INT8 Qwen3-0.6B shape (hidden
// 1024, intermediate 3072, 16 / 8 heads of 128) up to 10240 cached positions.
//
// Same computation (a10_int8_decode_kernel.cu:21-815) and the same work split
// over workgroups as decode_xcd.hip: workgroup g runs on XCD x = HW_REG_XCC_ID
// with rank r = g / 8; XCD x owns KV head x and its two query heads; rank r owns
// 16 of the XCD's 512 q|k|v rows, O and down rows [32r, +32) and gate/up
// channels [384x + 12r, +12). What differs is how a workgroup runs a layer.
// Measured on MI355X, a workgroup barrier costs about 135 ns, an LDS
// store-then-load round trip 57 ns, an fp64 wave sum 106 ns and a workgroup
// fp64 sum 300 ns, so a layer built from barrier-separated stages spends most
// of its time synchronising. Here:
//
//  * Waves 0-3 (compute waves) run the layer's critical path. They issue no
//    weight loads (a wave's loads return in order, so a poll behind a weight
//    batch would wait for the whole batch) and never meet at an s_barrier:
//    they synchronise through LDS counters, and a sum over the four waves is
//    finished by whichever arrives last.
//  * Waves 4-7 (loader waves) load each layer's weights, scales, norm gains and
//    cached K/V rows into registers while the compute waves run the previous
//    layer's attention, write each slot into LDS as soon as the compute waves are
//    done with the previous layer's contents of it, and raise that slot's ready
//    counter.
//  * The products run on the int8 matrix cores (v_mfma_i32_16x16x64_i8). A
//    compute wave writes its slice of the activation vector as a 55-bit fixed
//    point number (scale from the slice's largest exponent) in eight 7-bit
//    digits, the top one signed; the digit sums are exact integers, recombined
//    in fp64, so every stored value is the correctly rounded value of the
//    reference's expression, as in the fp64 kernels.
//  * Attention runs on the four compute waves: each takes both query heads over
//    a block of consecutive positions (scores, softmax numerators and P V in
//    fp64), and the blocks are merged with their log-sum-exp weights. Up to 64
//    cached positions every workgroup attends over all of them from its LDS
//    slot; past that (to 10240) rank r takes slice r of 32 (<= 320 positions,
//    streamed through its slot in chunks of 64 by the KV loader, one chunk in
//    flight while the compute waves attend over the one before it), publishes
//    its fp64 partial (max, denominator, numerators) as
//    tagged XCD-local words, merges output dims [8r, +8) over the 32 partials,
//    and the merged 256 outputs come back through one more XCD-local exchange.
//
// Per layer, compute wave c:
//   A  hidden slice [256c, +256) (polled) and the sum of squares from the 32
//      partial sums the hidden rows' producers published; RMSNorm, digits, 4
//      MFMA steps over the rank's 16 q|k|v rows       -> last arriver: XCD-local words
//   B  attention of both heads over the wave's block of positions; the four
//      waves meet in LDS, and wave c merges attention dims [64c, +64)
//      (with split attention: the rank's partial, the 32-rank merge, the gather)
//   C  those dims x O rows [32r, +32), 2 MFMAs         -> last arriver: cross-XCD packed partials
//   D  wave 0: the 8-XCD sum of its 32 rows, scale, residual
//                                                      -> XCD-local act words + sum of squares
//   E  act slice [256c, +256), RMSNorm, digits, 8 MFMAs over the 24 gate|up rows
//                                                      -> last arriver: SwiGLU, XCD-local words
//   F  c < 3: SwiGLU outputs [384x + 128c, +128) x down rows [32r, +32)
//                                                      -> last arriver: cross-XCD packed partials
//   G  wave 0: the 8-XCD sum, scale, residual, bf16    -> XCD-local hidden words + sum of squares
// Then all eight waves run the final RMSNorm, the LM head and the argmax as in
// decode_xcd.hip.
#include "attention.h"
#include "digits.h"

#include <hip/hip_ext.h>


namespace mq {

namespace {

constexpr int kAH = 1024, kAI = 3072, kAD = 128;
constexpr int kAX = 8;                     // XCDs
constexpr int kAIX = kAI / kAX;            // intermediate channels per XCD
constexpr int kAMaxLen = 64;               // positions one workgroup holds in LDS (slot B): one chunk
constexpr int kAMaxChunks = 5;             // chunks of a rank's slice, streamed through slot B in turn
constexpr int kARanks = kNWG / kAX;        // workgroups (ranks) per XCD
constexpr int kASplitLen = kARanks * kAMaxLen * kAMaxChunks;   // longest cache_len: 32 slices of <= 320
constexpr int kAPart = 4 + 2 * kAD;        // a rank's attention partial: (max, denominator) per head, numerators
constexpr int kCW = 4;                     // compute waves
// digit plane pitch in words: 68, not 64, so that the 8 planes one A-operand read
// touches start in different LDS banks
constexpr int kPlane = 68;

enum AStage { AS_QKV = 0, AS_ATT = 1, AS_ACT = 2, AS_MLP = 4, AS_HID = 5 };
constexpr uint32_t kAStages = 8;

// LDS counters (sync[]): ready and consumed per loader slot, arrival per combine
enum ASlot { SL_A = 0, SL_B = 1, SL_C = 2, SL_E = 3, SL_F = 4, kSlots = 5 };
constexpr int kReady = 0, kConsumed = 5, kArrive = 10;   // + slot / stage
constexpr int kWindow = 15;          // layers whose attention compute wave 0 has begun
enum AArr { AR_A = 0, AR_B = 1, AR_C = 2, AR_E = 3, AR_F = 4 };

// An XCD's hidden (or act) block: the 1024 row words, then the 32 ranks' partial sums
// of squares (low and high word each), so that one buffer load reaches both.
constexpr int kVecWords = kAH + 64;
struct ALayout {
    size_t qkvx, hidx, actx, mlpx, po, pd, lmg, apart, amrg, total;
};
// After the other two kernels' regions, so that the three can alternate on one workspace.
constexpr ALayout alayout_for(size_t base) {
    ALayout o{};
    size_t off = base;
    o.qkvx = off; off += round256((size_t)kAX * 512 * 8);
    o.hidx = off; off += round256((size_t)kAX * kVecWords * 8);
    o.actx = off; off += round256((size_t)kAX * kVecWords * 8);
    o.mlpx = off; off += round256((size_t)kAX * kAIX * 8);
    o.po = off; off += round256((size_t)kAX * kAH * 8);        // packed fp64 partials [xcd][row]
    o.pd = off; off += round256((size_t)kAX * kAH * 8);
    o.lmg = off; off += round256((size_t)kNWG * 2 * 8);
    o.apart = off; off += round256((size_t)kAX * kARanks * kAPart * 2 * 8);   // split attention partials (fp64 as two tagged words)
    o.amrg = off; off += round256((size_t)kAX * 2 * kAD * 8);             // merged outputs [xcd][dim]
    o.total = off;
    return o;
}

struct __align__(16) AsyncLds {
    // loader slots: layer l's data, written while the compute waves run layer l - 1
    uint4 wA[kCW][4][kWave];               // QKV: [wave][K step][lane] of the MFMA B operand
    uint4 wC[kCW][2][kWave];               // O: [wave][row tile][lane]
    uint4 wE[kCW][4][2][kWave];            // gate|up: [wave][K step][row tile][lane]
    uint4 wF[3][2][2][kWave];              // down: [wave][K step][row tile][lane]
    __align__(16) uint16_t kvk[kAMaxLen][kAD];           // cached K rows of positions [0, pos) (bf16)
    __align__(16) uint16_t kvv[kAMaxLen][kAD];           // cached V rows
    __align__(16) uint16_t lnA[kAH];                     // input RMSNorm gains
    __align__(16) uint16_t lnE[kAH];                     // post-attention RMSNorm gains
    uint16_t qkn[2][kAD];                  // q / k norm gains
    float scA[16], scC[32], scE[24], scF[32];     // row scales (1 with INT4 weights)
    // INT4 weights: the scales of each row's groups of 128 inputs that this workgroup's
    // products touch (A: 16 rows x 8 groups; C: 32 O rows x the XCD's 2 groups of
    // attention dims; E: 24 gate|up rows x 8; F: 32 down rows x the XCD's 3 groups)
    float gsA[16][8], gsC[32][2], gsE[24][8], gsF[32][3];
    uint16_t rope[2][kAD];                 // cos / sin at this position (once per step)
    uint16_t fnorm[kAH];                   // final RMSNorm gains (once per step)
    // compute waves
    __align__(16) uint32_t dig[kCW][8][kPlane];          // digit planes of each wave's slice (byte k of plane d)
    double qa[kCW][2][kAD];                // each wave's copy of the two rotated queries
    double pacc[kCW][2][kAD];              // P V partials of each wave's block, both heads
    double pml[kCW][2][2];                 // (max score, numerator sum) per wave and head
    __align__(16) double pw[kCW][16][2];   // softmax numerators of each wave's block [position][head]
    __align__(16) float hs[kAH];                         // the layer's input (bf16 values): stage D's residual
    double part[4][kCW][32];               // per-wave row partials of the combines A, C, E, F
    uint32_t sync[16];
    // tail
    __align__(16) float4 xs[kAH / 4];                    // final normalized vector, per-lane layout
    double fss;                            // final sum of squares
    float lm_v[kWaves];
    int lm_i[kWaves];
    int next_tok;                          // the step's token (every workgroup reduces it)
};

// ---- LDS synchronisation --------------------------------------------------------------
__device__ __forceinline__ uint32_t lds_load(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Compiler-level ordering only: LDS operations of one wave complete in order, so data
// written before a counter update is in LDS when another wave sees the update.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// Spins until *p >= target. Bounded: after `limit` polls it raises the abort flag and
// returns (the step then reports MQ_ERR_TIMEOUT, as the exchange waits do).
__device__ __forceinline__ void lds_wait(const uint32_t* p, uint32_t target, uint32_t limit, uint32_t* abort_flag) {
    uint32_t n = 0;
    while (lds_load(p) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (++n >= limit) {
            __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    lds_order();
}
__device__ __forceinline__ void lds_add(uint32_t* p, int lane) {
    lds_order();
    if (lane == 0) __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Arrival of one of the kCW compute waves at a combine; true for the last of the four.
__device__ __forceinline__ bool last_arrival(uint32_t* p, int lane) {
    lds_order();
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    lds_order();
    return (old % kCW) == kCW - 1;
}

// ---- exchange layout of the q|k|v rows ------------------------------------------------
// Word of q|k|v row m (q heads 2x, 2x + 1: rows 0-255, k: 256-383, v: 384-511). Within
// each 128-row q or k block, dims i and i + 64 (a RoPE rotation pair) share one 16-byte
// chunk, so lane l of a consumer reads both with one load; v rows stay in order (lane l
// reads dims 2l, 2l + 1, the word layout of a cache row).
__device__ __forceinline__ int qkv_word(int m) {
    if (m >= 384) return m;
    const int i = m & 127;
    return (m & ~127) + 2 * (i & 63) + (i >> 6);
}

// ---- cross-lane fp64 ------------------------------------------------------------------
// Value of lane l ^ 8 (DPP row rotation by 8) and of lane l ^ 4 (half-row mirror, l ^ 7,
// then the quad reversal, l ^ 3), for fp64 values.
template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double xor8_64(double v) { return dpp64<0x128>(v); }
__device__ __forceinline__ double xor4_64(double v) { return dpp64<0x1B>(dpp64<0x141>(v)); }
// Transposed pair sums across lane bit 5 (bit 4): lanes with the bit clear get
// lo(self) + lo(partner), lanes with it set hi(self) + hi(partner). One
// v_permlane32_swap (v_permlane16_swap) per 32-bit word exchanges the halves the
// partner keeps, so no lane selects are needed; with lo == hi this is a plain
// butterfly sum.
__device__ __forceinline__ double tsum32(double lo, double hi) {
    const uint64_t a = (uint64_t)__double_as_longlong(lo), b = (uint64_t)__double_as_longlong(hi);
    const auto w0 = __builtin_amdgcn_permlane32_swap((uint32_t)a, (uint32_t)b, false, false);
    const auto w1 = __builtin_amdgcn_permlane32_swap((uint32_t)(a >> 32), (uint32_t)(b >> 32), false, false);
    const double x = __longlong_as_double((long long)(((uint64_t)w1[0] << 32) | w0[0]));
    const double y = __longlong_as_double((long long)(((uint64_t)w1[1] << 32) | w0[1]));
    return x + y;
}
__device__ __forceinline__ double tsum16(double lo, double hi) {
    const uint64_t a = (uint64_t)__double_as_longlong(lo), b = (uint64_t)__double_as_longlong(hi);
    const auto w0 = __builtin_amdgcn_permlane16_swap((uint32_t)a, (uint32_t)b, false, false);
    const auto w1 = __builtin_amdgcn_permlane16_swap((uint32_t)(a >> 32), (uint32_t)(b >> 32), false, false);
    const double x = __longlong_as_double((long long)(((uint64_t)w1[0] << 32) | w0[0]));
    const double y = __longlong_as_double((long long)(((uint64_t)w1[1] << 32) | w0[1]));
    return x + y;
}
// max(self, lane ^ 32) and max(self, lane ^ 16), the same way
__device__ __forceinline__ double xmax32(double v) {
    const uint64_t a = (uint64_t)__double_as_longlong(v);
    const auto w0 = __builtin_amdgcn_permlane32_swap((uint32_t)a, (uint32_t)a, false, false);
    const auto w1 = __builtin_amdgcn_permlane32_swap((uint32_t)(a >> 32), (uint32_t)(a >> 32), false, false);
    return fmax(__longlong_as_double((long long)(((uint64_t)w1[0] << 32) | w0[0])),
                __longlong_as_double((long long)(((uint64_t)w1[1] << 32) | w0[1])));
}
__device__ __forceinline__ double xmax16(double v) {
    const uint64_t a = (uint64_t)__double_as_longlong(v);
    const auto w0 = __builtin_amdgcn_permlane16_swap((uint32_t)a, (uint32_t)a, false, false);
    const auto w1 = __builtin_amdgcn_permlane16_swap((uint32_t)(a >> 32), (uint32_t)(a >> 32), false, false);
    return fmax(__longlong_as_double((long long)(((uint64_t)w1[0] << 32) | w0[0])),
                __longlong_as_double((long long)(((uint64_t)w1[1] << 32) | w0[1])));
}
// Sum over each 16-lane row (every lane of the row receives it): four DPP levels.
__device__ __forceinline__ double row_sum64(double v) {
    v += partner64<1>(v);
    v += partner64<2>(v);
    v += partner64<4>(v);
    v += partner64<8>(v);
    return v;
}
__device__ __forceinline__ double row_max64(double v) {
    v = fmax(v, partner64<1>(v));
    v = fmax(v, partner64<2>(v));
    v = fmax(v, partner64<4>(v));
    v = fmax(v, partner64<8>(v));
    return v;
}
// Sum over the wave, the same value in every lane: row sums by DPP, then the four
// row sums read out and added in a fixed order (the cross-row permlane levels of a
// full butterfly cost twice a DPP level).
__device__ __forceinline__ double wave_sum64_u(double v) {
    v = row_sum64(v);
    return (readlane64(v, 0) + readlane64(v, 16)) + (readlane64(v, 32) + readlane64(v, 48));
}

// ---- digits ---------------------------------------------------------------------------
// Digit planes of a wave's slice, four consecutive elements per lane (element 4 lane + i).
__device__ __forceinline__ void put_digits4(uint32_t (*planes)[kPlane], const float (&v)[4], uint32_t emax, int lane) {
    int d[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) digits55(v[i], emax, d[i]);
#pragma unroll
    for (int p = 0; p < 8; ++p) planes[p][lane] = pack4(d[0][p], d[1][p], d[2][p], d[3][p]);
}
// Two consecutive elements per lane (element 2 lane + i).
__device__ __forceinline__ void put_digits2(uint32_t (*planes)[kPlane], const float (&v)[2], uint32_t emax, int lane) {
    int d[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i) digits55(v[i], emax, d[i]);
#pragma unroll
    for (int p = 0; p < 8; ++p)
        reinterpret_cast<uint16_t*>(planes[p])[lane] = (uint16_t)(pack4(d[0][p], d[1][p], 0, 0) & 0xffffu);
}
// One element per lane (element lane).
__device__ __forceinline__ void put_digits1(uint32_t (*planes)[kPlane], float v, uint32_t emax, int lane) {
    int d[8];
    digits55(v, emax, d);
#pragma unroll
    for (int p = 0; p < 8; ++p) reinterpret_cast<uint8_t*>(planes[p])[lane] = (uint8_t)(d[p] & 0xff);
}
// MFMA A operand of K step s: lane l holds digit plane l % 16 (zero past plane 7) at
// elements [64 s + 16 (l / 16), +16). Every lane reads (lanes past plane 7 the same
// words as lane l - 8, a broadcast) and the zero is a select, so that a stage's
// operand reads carry no branch and issue together ahead of its MFMAs.
__device__ __forceinline__ i32x4_t a_frag(const uint32_t (*planes)[kPlane], int s, int lane) {
    const int p = lane % 16;
    const uint4 w = *reinterpret_cast<const uint4*>(&planes[p & 7][16 * s + 4 * (lane / 16)]);
    const bool z = p >= 8;
    return i32x4_t{z ? 0 : (int)w.x, z ? 0 : (int)w.y, z ? 0 : (int)w.z, z ? 0 : (int)w.w};
}
__device__ __forceinline__ i32x4_t b_frag(const uint4& w) { return i32x4_t{(int)w.x, (int)w.y, (int)w.z, (int)w.w}; }
// The operands a stage's MFMAs read, all in registers at this point: their LDS reads
// are then issued together and waited for once (left to itself the scheduler reuses
// registers and waits for each MFMA's two reads in turn, one LDS round trip each).
template <int N>
__device__ __forceinline__ void operands_ready(i32x4_t (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
// ---- INT4 weights -----------------------------------------------------------------------
// 16 two's complement nibbles (8 bytes, the low nibble of a byte the even element) as 16
// int8 values in element order: the MFMA B operand the int8 path reads from LDS.
__device__ __forceinline__ uint32_t sext_nibble_bytes(uint32_t v) {
    return v | ((v & 0x08080808u) * 0x1Eu);        // bytes 8-15 -> 0xF8-0xFF (v - 16)
}
__device__ __forceinline__ uint4 nibbles_to_i8(uint2 p) {
    uint32_t o[4];
    const uint32_t w[2] = {p.x, p.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t lo = sext_nibble_bytes(w[i] & 0x0F0F0F0Fu);          // elements 0, 2, 4, 6 of the word
        const uint32_t hi = sext_nibble_bytes((w[i] >> 4) & 0x0F0F0F0Fu);   // elements 1, 3, 5, 7
        o[2 * i] = (lo & 0xFFu) | ((hi & 0xFFu) << 8) | ((lo & 0xFF00u) << 8) | ((hi & 0xFF00u) << 16);
        o[2 * i + 1] = ((lo >> 16) & 0xFFu) | ((hi >> 8) & 0xFF00u) | ((lo >> 8) & 0xFF0000u) | (hi & 0xFF000000u);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}
// 8-byte weight load with the non-temporal hint (INT4 rows: 16 elements)
__device__ __forceinline__ uint2 ldg8_stream(const void* p) {
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x2_t*)p);
    return make_uint2(v.x, v.y);
}

// ---- polls ----------------------------------------------------------------------------
// One round of polls over an XCD's vector block (kVecWords words at `block`, one tag):
// elements [256 slice + 4 lane, +4) into v, and the 32 fp64 partial sums of squares
// (lanes < 32 one each), returned summed in a fixed order (the same value in every lane).
// `meanwhile()` runs while the first round of loads is in flight.
template <class F>
__device__ __forceinline__ double poll_slice(Waiter& wt, const uint64_t* block, uint32_t tag, int slice, int lane,
                                             float (&v)[4], F&& meanwhile) {
    uint32_t w[3] = {2u * (uint32_t)(128 * slice + 2 * lane), 2u * (uint32_t)(128 * slice + 2 * lane) + 2u,
                     (uint32_t)kAH + 2u * (uint32_t)(lane & 31)};
    float o[6];
    wt.get_pairs<3>(XRegion(block, kVecWords), w, tag, o, lane < 32 ? 3 : 2, meanwhile);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = o[i];
    double s = lane < 32 ? __longlong_as_double((long long)(((uint64_t)__float_as_uint(o[5]) << 32) |
                                                            __float_as_uint(o[4])))
                         : 0.0;
    // lanes 32-63 hold 0: the two 16-lane row sums of lanes 0-31 by DPP, then added from
    // lanes 0 and 16 (the same value in every lane; a cross-row permlane level costs
    // about twice a DPP level)
    s = row_sum64(s);
    return readlane64(s, 0) + readlane64(s, 16);
}

}  // namespace

// The launch's arguments read afresh from the kernel-argument segment (a volatile
// view): used for what only the LM head needs, so that with several steps per launch
// it is not held in registers through every layer. (Reading the by-value parameter
// through its address instead would copy the arguments to scratch memory.)
__device__ __forceinline__ const volatile KArgs* kargs() {
    return (const volatile KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}

// kMulti: several steps per launch (a.n_steps); otherwise one, and the step loop
// disappears (held across a loop back-edge, the kernel's long-lived values would
// cost register spills in the one-step kernel too).
// kW4: the layer projections are INT4 per group of 128 inputs (packed nibbles [out, in / 2],
// scales [out, in / 128]); the LM head stays INT8 per row.
// kDeep: a rank's slice may take several slot-B chunks (cache_len past 2048); without it the
// kernel holds every slice in one chunk and the host launches it only up to 2048 positions.
template <bool kDebug, bool kMulti, bool kW4 = false, bool kDeep = false>
__global__ void __launch_bounds__(kThreads, 1) decode_async_kernel(KArgs a) {
    constexpr int H = kAH, D = kAD;
    constexpr ALayout kLay = alayout_for(xlayout_total(kAH, kAI));
    __shared__ AsyncLds S;

    const int g = blockIdx.x;
    const int x = (int)hw_xcc_id();
    const int r = g / kAX;
    const int tid0 = threadIdx.x;
    const int lane0 = tid0 % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid0 / kWave);   // uniform: scalar registers

    WsHeader* hdr = reinterpret_cast<WsHeader*>(a.ws);
    uint64_t* const qkvx = reinterpret_cast<uint64_t*>(a.ws + kLay.qkvx) + (size_t)x * 512;
    uint64_t* const hidx = reinterpret_cast<uint64_t*>(a.ws + kLay.hidx) + (size_t)x * kVecWords;
    uint64_t* const hss = hidx + H;
    uint64_t* const actx = reinterpret_cast<uint64_t*>(a.ws + kLay.actx) + (size_t)x * kVecWords;
    uint64_t* const ass = actx + H;
    uint64_t* const mlpx = reinterpret_cast<uint64_t*>(a.ws + kLay.mlpx) + (size_t)x * kAIX;
    uint64_t* const po = reinterpret_cast<uint64_t*>(a.ws + kLay.po);     // packed [8][H]
    uint64_t* const pd = reinterpret_cast<uint64_t*>(a.ws + kLay.pd);
    uint64_t* const lmg = reinterpret_cast<uint64_t*>(a.ws + kLay.lmg);
    uint64_t* const apart = reinterpret_cast<uint64_t*>(a.ws + kLay.apart) + (size_t)x * kARanks * kAPart * 2;
    uint64_t* const amrg = reinterpret_cast<uint64_t*>(a.ws + kLay.amrg) + (size_t)x * 2 * kAD;

    const uint32_t E0 = __hip_atomic_load(&hdr->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t AS0 = __hip_atomic_load(&hdr->asteps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t E = E0, AS = AS0;              // the step's epoch (tags) and packed-word step count
    const uint32_t tps = kAStages * (uint32_t)a.L + 4u;
    // tags end in binary 10 (the other kernels' in 01 and 11)
    auto tag = [&](int l, int st) -> uint32_t { return ((E * tps + kAStages * (uint32_t)l + (uint32_t)st) << 2) | 2u; };
    // one-bit tag of the packed cross-XCD words (po and pd are each written once per layer)
    auto pbit = [&](int l) -> uint32_t { return (AS * (uint32_t)a.L + (uint32_t)l + 1u) & 1u; };
    Waiter wt(&hdr->abort_flag, a.spin_limit);
    const uint32_t lds_limit = a.spin_limit * 8u;
    auto trace = [&](int l, int point) {
        if (kDebug && a.trace != nullptr && tid0 == 0)
            a.trace[((int64_t)l * kTracePoints + point) * kNWG + g] = __builtin_amdgcn_s_memrealtime();
    };
    // The positions [s0, s0 + ns) of cache_len p + 1 this rank attends over: all of them up to
    // kAMaxLen (below the split threshold), else slice r of 32 (<= kAMaxLen each); true when split.
    const int split_min = a.split_min;
    auto attn_slice = [&](int p, int& s0, int& ns) -> bool {
        const int n = p + 1;
        if (n <= kAMaxLen && n < split_min) {
            s0 = 0;
            ns = n;
            return false;
        }
        const int cs = (n + kARanks - 1) / kARanks;
        s0 = min(n, r * cs);
        ns = min(n, s0 + cs) - s0;
        return true;
    };
    // Slot-B chunks of this rank's positions at cache_len p + 1: ceil(ns / kAMaxLen), at least 1
    // (the first carries the QK-norm gains and, in layer 0, the RoPE row). Slot B's ready and
    // consumed counters count chunks over the launch: chunk k of layer l of a step is number
    // cbase + l nch + k, cbase being the chunks of the launch's earlier steps.
    auto chunks_at = [&](int p) -> int {
        int s0, ns;
        attn_slice(p, s0, ns);
        return max(1, (ns + kAMaxLen - 1) / kAMaxLen);
    };
    uint32_t cbase = 0;
    int nch = 1;
    if (x >= kAX) {
        if (tid0 == 0) __hip_atomic_store(&hdr->abort_flag, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (tid0 < 16) S.sync[tid0] = 0u;
    const int last = a.L - 1;
    const int64_t kv_head_stride = (int64_t)a.S * D;
    if (wave == kCW + 3) {
        // the final norm gains, once per launch
        uint32_t fw[H / 128];
#pragma unroll
        for (int i = 0; i < H / 128; ++i) fw[i] = *gview(reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(a.final_norm) + 256 * i + 4 * lane0));
#pragma unroll
        for (int i = 0; i < H / 128; ++i) reinterpret_cast<uint32_t*>(S.fnorm)[64 * i + lane0] = fw[i];
    }
    __syncthreads();

    // Steps: step s decodes at position a.pos + s (cache_len = position + 1 <= kASplitLen,
    // checked by the host); its input token is a.step_tokens[s] for the first n_forced
    // steps (a.token when there is no list) and the previous step's output after them.
    // The LDS counters count layers over the whole launch (gl = s L + l).
    int pos = a.pos;
    int token = a.step_tokens ? (int)__builtin_amdgcn_readfirstlane(*gview(a.step_tokens)) : a.token;
    const int n_steps = kMulti ? kargs()->n_steps : 1;
    for (int step = 0; step < n_steps; ++step) {
    // lane-derived addresses are rederived every step (hidden from the optimiser): held
    // across the step loop they would be live in the LM head too and be spilled
    issue_fence();                          // loads (kernel arguments among them) are redone per step
    const int tid = opaque(tid0);
    const int lane = opaque(lane0);
    E = E0 + (uint32_t)step;
    AS = AS0 + (uint32_t)step;
    pos = a.pos + step;
    if (kDeep) {
        if (step > 0) cbase += (uint32_t)(a.L * nch);
        nch = chunks_at(pos);
    }

    if (wave >= kCW) {
        // ================================ loader waves ================================
        // Loader d loads its share of layer l into registers once compute wave 0 has begun
        // layer l - 1's attention (the compute waves then have no exchange poll in flight
        // for a while, and a poll queued behind these loads would wait for them), writes
        // each slot into LDS when the compute waves have released the previous layer's
        // contents of it, and raises the slot's ready counter:
        //   d = 0: slot A (the rank's q|k|v rows, input norm gains, row scales)
        //   d = 1: slots C and F (O and down rows, their scales)
        //   d = 2: slot E (gate|up rows, post-attention norm gains, scales)
        //   d = 3: slot B (cached K and V rows of positions [0, pos), QK-norm gains; past 2048
        //          positions a rank's slice in chunks of 64, one after another), and
        //          once per step this position's RoPE row and the final norm gains; it also
        //          stores the position's new K and V rows into the cache (store_row)
        const int d = wave - kCW;
        auto await_free = [&](int slot, int l) {
            lds_wait(&S.sync[kConsumed + slot], (uint32_t)(kCW * l), lds_limit, &hdr->abort_flag);
        };
        auto raise = [&](int slot, int l) {
            lds_order();
            if (lane == 0)
                __hip_atomic_store(&S.sync[kReady + slot], (uint32_t)(l + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        auto ld32 = [&](const void* q) -> uint32_t { return *gview(static_cast<const uint32_t*>(q)); };
        auto put32 = [&](void* base, int word, uint32_t v) { static_cast<uint32_t*>(base)[word] = v; };
        // The cache row of this step's position in layer ll: the owner compute wave put it in
        // slot B (K chunks permuted); one rank per XCD stores it from there once the compute
        // waves have released the slot (rank 0, or with split attention the rank whose slice
        // holds the position). The store is issued here rather than by the owner wave: a
        // compute wave's stores count against the same counter as its exchange polls, and
        // the owner's store held its rank's attention back by about 0.75 us per layer.
        auto store_row = [&](int ll) {
            int s0, ns;
            const bool sp_ = attn_slice(pos, s0, ns);
            if (!(sp_ ? (pos >= s0 && pos < s0 + ns) : r == 0)) return;
            const int pl = pos - s0 - kAMaxLen * (nch - 1);       // its row in the last chunk
            const int ls = opaque(lane);
            const int64_t row = ((int64_t)ll * kAX + x) * kv_head_stride + (int64_t)pos * D;
            if (ls < 16) {
                const uint4 kw = reinterpret_cast<const uint4*>(S.kvk[pl])[ls ^ (pl % 16)];
                *reinterpret_cast<uint4*>(a.kc + row + 8 * ls) = kw;
            } else if (ls < 32) {
                const uint4 vw = reinterpret_cast<const uint4*>(S.kvv[pl])[ls - 16];
                *reinterpret_cast<uint4*>(a.vc + row + 8 * (ls - 16)) = vw;
            }
        };
        for (int l = 0; l < a.L; ++l) {
            const int gl = step * a.L + l;
            if (gl > 0) lds_wait(&S.sync[kWindow], (uint32_t)gl, lds_limit, &hdr->abort_flag);
            const LayerWeights lw = a.lw[l];
            const ScalePointers sp = a.sp[l];
            if (d == 0) {
                const uint8_t* base;
                const float* sc;
                int mrow0;
                if (r < 16) { base = (const uint8_t*)lw.q_proj_weight; sc = sp.q_scale; mrow0 = 2 * x * D + 16 * r; }
                else if (r < 24) { base = (const uint8_t*)lw.k_proj_weight; sc = sp.k_scale; mrow0 = x * D + 16 * (r - 16); }
                else { base = (const uint8_t*)lw.v_proj_weight; sc = sp.v_scale; mrow0 = x * D + 16 * (r - 24); }
                // lane: row mrow0 + lane % 16, inputs [256 c + 64 s + 16 (lane / 16), +16) of K step
                // (c, s) = (i / 4, i % 4)
                uint4 w[kW4 ? 1 : 16];
                uint2 w4[kW4 ? 16 : 1];
                if constexpr (kW4) {
                    const uint8_t* rowp = base + (int64_t)(mrow0 + lane % 16) * (H / 2) + 8 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 16; ++i) w4[i] = ldg8_stream(rowp + 128 * (i / 4) + 32 * (i % 4));
                } else {
                    const uint8_t* rowp = base + (int64_t)(mrow0 + lane % 16) * H + 16 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 16; ++i) w[i] = ldg16_stream(rowp + 256 * (i / 4) + 64 * (i % 4));
                }
                uint32_t gw[H / 128];
#pragma unroll
                for (int i = 0; i < H / 128; ++i) gw[i] = ld32(static_cast<const uint8_t*>(lw.input_layernorm_weight) + 256 * i + 4 * lane);
                // INT4: the 16 rows' 8 group scales (rows mrow0.. are contiguous: 128 floats)
                const uint32_t scv = kW4 ? 0x3F800000u : lane < 16 ? ld32(sc + mrow0 + lane) : 0u;
                const uint32_t gs0 = kW4 ? ld32(sc + (int64_t)mrow0 * 8 + 2 * lane) : 0u;
                const uint32_t gs1 = kW4 ? ld32(sc + (int64_t)mrow0 * 8 + 2 * lane + 1) : 0u;
                await_free(SL_A, gl);
#pragma unroll
                for (int i = 0; i < 16; ++i) S.wA[i / 4][i % 4][lane] = kW4 ? nibbles_to_i8(w4[i]) : w[i];
#pragma unroll
                for (int i = 0; i < H / 128; ++i) put32(S.lnA, 64 * i + lane, gw[i]);
                if (lane < 16) put32(S.scA, lane, scv);
                if (kW4) {
                    put32(S.gsA, 2 * lane, gs0);
                    put32(S.gsA, 2 * lane + 1, gs1);
                }
                raise(SL_A, gl);
            } else if (d == 1) {
                // O: lane row 32 r + 16 t + lane % 16, inputs 256 x + 64 c + 16 (lane / 16) (i = 2 c + t);
                // down: row 32 r + 16 t + lane % 16, inputs 384 x + 64 (2 c + s) + 16 (lane / 16)
                uint4 wc[kW4 ? 1 : 8], wf[kW4 ? 1 : 12];
                uint2 wc4[kW4 ? 8 : 1], wf4[kW4 ? 12 : 1];
                uint32_t so, sdv, gc = 0u, gf0 = 0u, gf1 = 0u;
                if constexpr (kW4) {
                    const uint8_t* ob = (const uint8_t*)lw.o_proj_weight + (int64_t)(32 * r + lane % 16) * 1024 + 128 * x +
                                        8 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 8; ++i) wc4[i] = ldg8_stream(ob + (int64_t)16 * (i % 2) * 1024 + 32 * (i / 2));
                    const uint8_t* db = (const uint8_t*)lw.down_proj_weight + (int64_t)(32 * r + lane % 16) * (kAI / 2) +
                                        (kAIX / 2) * x + 8 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 12; ++i)             // i = (2 c + s) * 2 + t
                        wf4[i] = ldg8_stream(db + (int64_t)16 * (i % 2) * (kAI / 2) + 32 * (i / 2));
                    so = sdv = 0x3F800000u;
                    // group scales: O rows 32 r.. x groups 2 x, 2 x + 1 of 16; down rows x groups 3 x.. of 24
                    gc = ld32(sp.o_scale + (int64_t)(32 * r + lane / 2) * 16 + 2 * x + lane % 2);
                    gf0 = ld32(sp.down_scale + (int64_t)(32 * r + lane / 3) * 24 + 3 * x + lane % 3);
                    gf1 = lane < 32 ? ld32(sp.down_scale + (int64_t)(32 * r + (lane + 64) / 3) * 24 + 3 * x + (lane + 64) % 3)
                                    : 0u;
                } else {
                    const uint8_t* ob = (const uint8_t*)lw.o_proj_weight + (int64_t)(32 * r + lane % 16) * 2048 + 256 * x +
                                        16 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 8; ++i) wc[i] = ldg16_stream(ob + (int64_t)16 * (i % 2) * 2048 + 64 * (i / 2));
                    const uint8_t* db = (const uint8_t*)lw.down_proj_weight + (int64_t)(32 * r + lane % 16) * kAI + kAIX * x +
                                        16 * (lane / 16);
#pragma unroll
                    for (int i = 0; i < 12; ++i)             // i = (2 c + s) * 2 + t
                        wf[i] = ldg16_stream(db + (int64_t)16 * (i % 2) * kAI + 64 * (i / 2));
                    so = lane < 32 ? ld32(sp.o_scale + 32 * r + lane) : 0u;
                    sdv = lane < 32 ? ld32(sp.down_scale + 32 * r + lane) : 0u;
                }
                await_free(SL_C, gl);
#pragma unroll
                for (int i = 0; i < 8; ++i) S.wC[i / 2][i % 2][lane] = kW4 ? nibbles_to_i8(wc4[i]) : wc[i];
                if (lane < 32) put32(S.scC, lane, so);
                if (kW4) put32(S.gsC, lane, gc);
                raise(SL_C, gl);
                await_free(SL_F, gl);
#pragma unroll
                for (int i = 0; i < 12; ++i) S.wF[i / 4][(i / 2) % 2][i % 2][lane] = kW4 ? nibbles_to_i8(wf4[i]) : wf[i];
                if (lane < 32) put32(S.scF, lane, sdv);
                if (kW4) {
                    put32(S.gsF, lane, gf0);
                    if (lane < 32) put32(S.gsF, 64 + lane, gf1);
                }
                raise(SL_F, gl);
            } else if (d == 2) {
                const int c0 = kAIX * x + 12 * r;
                uint4 we[kW4 ? 1 : 32];                        // i = (4 c + s) * 2 + t; tile rows 24-31 zero
                uint2 we4[kW4 ? 32 : 1];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int j = 16 * t + lane % 16;
                    if constexpr (kW4) {
                        const uint8_t* rowp = (j < 12 ? (const uint8_t*)lw.gate_proj_weight + (int64_t)(c0 + j) * (H / 2)
                                                      : (const uint8_t*)lw.up_proj_weight + (int64_t)(c0 + min(j, 23) - 12) * (H / 2)) +
                                              8 * (lane / 16);
#pragma unroll
                        for (int k = 0; k < 16; ++k) {
                            we4[2 * k + t] = make_uint2(0, 0);
                            if (j < 24) we4[2 * k + t] = ldg8_stream(rowp + 32 * k);
                        }
                    } else {
                        const uint8_t* rowp = (j < 12 ? (const uint8_t*)lw.gate_proj_weight + (int64_t)(c0 + j) * H
                                                      : (const uint8_t*)lw.up_proj_weight + (int64_t)(c0 + min(j, 23) - 12) * H) +
                                              16 * (lane / 16);
#pragma unroll
                        for (int k = 0; k < 16; ++k) {
                            we[2 * k + t] = make_uint4(0, 0, 0, 0);
                            if (j < 24) we[2 * k + t] = ldg16_stream(rowp + 64 * k);
                        }
                    }
                }
                uint32_t gw[H / 128];
#pragma unroll
                for (int i = 0; i < H / 128; ++i)
                    gw[i] = ld32(static_cast<const uint8_t*>(lw.post_attn_layernorm_weight) + 256 * i + 4 * lane);
                const uint32_t scv = kW4 ? 0x3F800000u
                                   : lane < 12 ? ld32(sp.gate_scale + c0 + lane)
                                   : lane < 24 ? ld32(sp.up_scale + c0 + lane - 12) : 0u;
                // INT4: 24 rows (gate 0-11, up 12-23) x 8 group scales, entry 64 m + lane
                uint32_t ge[3] = {0u, 0u, 0u};
                if constexpr (kW4) {
#pragma unroll
                    for (int m = 0; m < 3; ++m) {
                        const int idx = 64 * m + lane, j = idx / 8, grp = idx % 8;
                        ge[m] = ld32(j < 12 ? sp.gate_scale + (int64_t)(c0 + j) * 8 + grp
                                            : sp.up_scale + (int64_t)(c0 + j - 12) * 8 + grp);
                    }
                }
                await_free(SL_E, gl);
#pragma unroll
                for (int k = 0; k < 16; ++k)
#pragma unroll
                    for (int t = 0; t < 2; ++t) S.wE[k / 4][k % 4][t][lane] = kW4 ? nibbles_to_i8(we4[2 * k + t]) : we[2 * k + t];
#pragma unroll
                for (int i = 0; i < H / 128; ++i) put32(S.lnE, 64 * i + lane, gw[i]);
                if (lane < 24) put32(S.scE, lane, scv);
                if (kW4) {
#pragma unroll
                    for (int m = 0; m < 3; ++m) put32(S.gsE, 64 * m + lane, ge[m]);
                }
                raise(SL_E, gl);
            }
            if (d == 3) {
                // K rows keep their 16-byte chunks XOR-permuted by row (chunk g of row j at
                // g ^ (j % 16)), so that lanes reading the same chunk of different rows hit
                // different banks; V rows are read whole by every lane and stay in order
                // (the lane is rederived per layer, so that its row addresses are not held
                // through the layer loop alongside the 128 registers of rows)
                // Slot row jl of chunk k holds position s0 + kAMaxLen k + jl of this rank's positions
                // (all of them, or its slice with split attention); rows before pos come from the
                // cache. Chunk 0 is loaded once compute wave 0 has begun the previous layer's
                // attention, each later one as soon as the one before it is in the slot, so that
                // it is in flight while the compute waves attend over that one. (Loader 0 taking
                // every other chunk, so that two were in flight, measured slower: 563 against
                // 547 us per step at depth 4096.)
                const int64_t cb = ((int64_t)l * kAX + x) * kv_head_stride;
                int s0, ns;
                attn_slice(pos, s0, ns);
                const uint32_t qn = ld32(static_cast<const uint8_t*>(lw.q_norm_weight) + 4 * opaque(lane));
                const uint32_t kn = ld32(static_cast<const uint8_t*>(lw.k_norm_weight) + 4 * opaque(lane));
                // this step's RoPE row rides with layer 0's first chunk (slot B is free once the
                // previous step's last attention is done)
                const uint32_t cw = l == 0 ? ld32(a.cos_t + (int64_t)pos * D + 2 * opaque(lane)) : 0u;
                const uint32_t sw = l == 0 ? ld32(a.sin_t + (int64_t)pos * D + 2 * opaque(lane)) : 0u;
                auto put_gains = [&](int ls) {
                    put32(S.qkn[0], ls, qn);
                    put32(S.qkn[1], ls, kn);
                    if (l == 0) {
                        put32(S.rope[0], ls, cw);
                        put32(S.rope[1], ls, sw);
                    }
                };
                if constexpr (!kDeep) {
                    const int ln = opaque(lane);
                    const int lim = min(ns, pos - s0);
                    uint4 rk[kAMaxLen / 4], rv[kAMaxLen / 4];
#pragma unroll
                    for (int i = 0; i < kAMaxLen / 4; ++i) {
                        const int jl = 4 * i + ln / 16;
                        rk[i] = make_uint4(0, 0, 0, 0);
                        rv[i] = make_uint4(0, 0, 0, 0);
                        if (jl < lim) {
                            rk[i] = ldg16(a.kc + cb + (int64_t)(s0 + jl) * D + 8 * (ln % 16));
                            rv[i] = ldg16(a.vc + cb + (int64_t)(s0 + jl) * D + 8 * (ln % 16));
                        }
                    }
                    await_free(SL_B, gl);
                    if (l > 0) store_row(l - 1);
                    const int ls = opaque(ln);
#pragma unroll
                    for (int i = 0; i < kAMaxLen / 4; ++i) {
                        const int jl = 4 * i + ls / 16;
                        if (jl < lim) {
                            reinterpret_cast<uint4*>(S.kvk[jl])[(ls % 16) ^ (jl % 16)] = rk[i];
                            reinterpret_cast<uint4*>(S.kvv[jl])[ls % 16] = rv[i];
                        }
                    }
                    put_gains(ls);
                    raise(SL_B, gl);
                } else {
                    // chunk k's rows, each chunk loaded as soon as the one before it is in the slot
                    const int lim_all = min(ns, pos - s0);
                    const uint32_t ci0 = cbase + (uint32_t)(l * nch);
                    for (int k = 0; k < nch; ++k) {
                        const int ln = opaque(lane);
                        const int lim = min(lim_all - kAMaxLen * k, kAMaxLen);   // rows from the cache
                        const int64_t kb0 = cb + (int64_t)(s0 + kAMaxLen * k) * D;
                        uint4 rk[kAMaxLen / 4], rv[kAMaxLen / 4];
#pragma unroll
                        for (int i = 0; i < kAMaxLen / 4; ++i) {
                            const int jl = 4 * i + ln / 16;
                            rk[i] = make_uint4(0, 0, 0, 0);
                            rv[i] = make_uint4(0, 0, 0, 0);
                            if (jl < lim) {
                                rk[i] = ldg16(a.kc + kb0 + (int64_t)jl * D + 8 * (ln % 16));
                                rv[i] = ldg16(a.vc + kb0 + (int64_t)jl * D + 8 * (ln % 16));
                            }
                        }
                        await_free(SL_B, (int)(ci0 + k));
                        if (l > 0 && k == 0) store_row(l - 1);
                        const int ls = opaque(ln);
#pragma unroll
                        for (int i = 0; i < kAMaxLen / 4; ++i) {
                            const int jl = 4 * i + ls / 16;
                            if (jl < lim) {
                                reinterpret_cast<uint4*>(S.kvk[jl])[(ls % 16) ^ (jl % 16)] = rk[i];
                                reinterpret_cast<uint4*>(S.kvv[jl])[ls % 16] = rv[i];
                            }
                        }
                        if (k == 0) put_gains(ls);
                        raise(SL_B, (int)(ci0 + k));
                    }
                }
            }
        }
        if (d == 3) {
            // the step's last layer, once its attention has released slot B
            await_free(SL_B, kDeep ? (int)(cbase + (uint32_t)(a.L * nch)) : (step + 1) * a.L);
            store_row(a.L - 1);
        }
    } else {
        // =============================== compute waves ================================
        const int c = wave;
        float act_reg = 0.0f;                   // wave 0: this rank's residual row (lane % 32) from stage D
        for (int l = 0; l < a.L; ++l) {
            const int gl = step * a.L + l;
            // ---------------- A: RMSNorm + QKV ----------------
            // The loader slots of this layer are filled a layer ahead: A checks those of
            // stages A-C and E (while its hidden-slice loads are in flight) and E the
            // one of F, so that no later stage waits an LDS round trip for its slot.
            // (slot B: its first chunk of the layer)
            const uint32_t ci0 = kDeep ? cbase + (uint32_t)(l * nch) : (uint32_t)gl;
            auto slots_ready = [&](uint32_t mask) {
                uint32_t v[kSlots];
#pragma unroll
                for (int k = 0; k < kSlots; ++k) v[k] = (mask & (1u << k)) ? lds_load(&S.sync[kReady + k]) : 0u;
#pragma unroll
                for (int k = 0; k < kSlots; ++k) {
                    const uint32_t want = k == SL_B ? ci0 + 1u : (uint32_t)(gl + 1);
                    if ((mask & (1u << k)) && v[k] < want) lds_wait(&S.sync[kReady + k], want, lds_limit, &hdr->abort_flag);
                }
                lds_order();
            };
            constexpr uint32_t kSlotsA = (1u << SL_A) | (1u << SL_B) | (1u << SL_C) | (1u << SL_E);
            float hv[4];
            double ssq;
            if (l == 0) {
                typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
                const u32x2_t e4 = *(const __attribute__((address_space(1))) u32x2_t*)(a.embed + (int64_t)token * H +
                                                                                        256 * c + 4 * lane);
                hv[0] = bf16_bits_to_f32(e4.x & 0xffffu); hv[1] = bf16_bits_to_f32(e4.x >> 16);
                hv[2] = bf16_bits_to_f32(e4.y & 0xffffu); hv[3] = bf16_bits_to_f32(e4.y >> 16);
                const uint4* er = reinterpret_cast<const uint4*>(a.embed + (int64_t)token * H);
                const uint4 u0 = ldg16(er + 2 * lane), u1 = ldg16(er + 2 * lane + 1);
                const uint32_t wv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
                double s = 0.0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const double lo = bf16_bits_to_f32(wv[i] & 0xffffu), hi = bf16_bits_to_f32(wv[i] >> 16);
                    s = fma(lo, lo, s);
                    s = fma(hi, hi, s);
                }
                ssq = wave_sum64(s);
                slots_ready(kSlotsA);
            } else {
                ssq = poll_slice(wt, hidx, tag(l - 1, AS_HID), c, lane, hv, [&] { slots_ready(kSlotsA); });
            }
            *reinterpret_cast<float4*>(&S.hs[256 * c + 4 * lane]) = make_float4(hv[0], hv[1], hv[2], hv[3]);
            trace(l, 0);
            const double rstd = rms_scale(ssq, H, kEps);
            float nv[4];
            {
                const uint2 gw = *reinterpret_cast<const uint2*>(&S.lnA[256 * c + 4 * lane]);
                const float gl[4] = {bf16_bits_to_f32(gw.x & 0xffffu), bf16_bits_to_f32(gw.x >> 16),
                                     bf16_bits_to_f32(gw.y & 0xffffu), bf16_bits_to_f32(gw.y >> 16)};
#pragma unroll
                for (int i = 0; i < 4; ++i) nv[i] = (float)((double)hv[i] * rstd * (double)gl[i]);
            }
            {
                uint32_t em = max(max(exp_field(nv[0]), exp_field(nv[1])), max(exp_field(nv[2]), exp_field(nv[3])));
                em = wave_max_u32(em);
                put_digits4(S.dig[c], nv, em, lane);
                lds_order();
                i32x4_t op[8];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    op[2 * s] = a_frag(S.dig[c], s, lane);
                    op[2 * s + 1] = b_frag(S.wA[c][s][lane]);
                }
                operands_ready(op);
                double v;
                if constexpr (kW4) {
                    // K steps 0-1 and 2-3 are the slice's two groups of 128: one sum each, scaled
                    i32x4_t a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        a0 = mfma_i8(op[2 * s], op[2 * s + 1], a0);
                        a1 = mfma_i8(op[2 * s + 4], op[2 * s + 5], a1);
                    }
                    const int row = lane % 16;
                    v = tile_value(a0, em) * (double)S.gsA[row][2 * c] + tile_value(a1, em) * (double)S.gsA[row][2 * c + 1];
                } else {
                    i32x4_t acc = {0, 0, 0, 0};
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc = mfma_i8(op[2 * s], op[2 * s + 1], acc);
                    v = tile_value(acc, em);
                }
                if (lane < 16) S.part[0][c][lane] = v;
            }
            if (last_arrival(&S.sync[kArrive + AR_A], lane)) {
                if (lane < 16) {
                    const double* P = &S.part[0][0][lane];
                    const double v = ((P[0] + P[32]) + (P[64] + P[96])) *
                                     (double)S.scA[lane];
                    ll_put_xcd(&qkvx[qkv_word(16 * r + lane)], __float_as_uint((float)v), tag(l, AS_QKV));
                }
            }
            lds_add(&S.sync[kConsumed + SL_A], lane);
            trace(l, 1);

            // ---------------- B: attention ----------------
            // Every compute wave takes both query heads over its block of q0 = ceil(n / 4)
            // consecutive positions, so each cached K and V word is converted once for the
            // two heads. Lane l holds dims l and l + 64 of the queries (and of k), the
            // rotation pairs of RoPE; v dims 2l, 2l + 1 (the word layout of a cache row).
            float ao;
            {
                int s0, ns;
                const bool split = attn_slice(pos, s0, ns);
                // The slice runs as nch chunks of <= kAMaxLen positions through slot B; in chunk k
                // wave c takes the block of its q0 = ceil(nk / 4) consecutive positions. The owner
                // of this position (one wave of one workgroup per XCD when split) is the wave whose
                // block of the last chunk holds it.
                const int c_last = kAMaxLen * (nch - 1);                // the last chunk's first slice row
                const int n_last = ns - c_last;
                const int q_last = (n_last + kCW - 1) / kCW;
                const bool owner = s0 + c_last + min(n_last, c * q_last) <= pos && pos < s0 + c_last + min(n_last, c * q_last + q_last);
                float qv[2][2], kv2[2], vv[2];
                {
                    const uint32_t w[4] = {2u * (uint32_t)lane, 128u + 2u * (uint32_t)lane, 256u + 2u * (uint32_t)lane,
                                           384u + 2u * (uint32_t)lane};
                    float o[8];
                    wt.get_pairs<4>(XRegion(qkvx, 512), w, tag(l, AS_QKV), o, owner ? 4 : 2);
                    qv[0][0] = o[0]; qv[0][1] = o[1];
                    qv[1][0] = o[2]; qv[1][1] = o[3];
                    kv2[0] = o[4]; kv2[1] = o[5];
                    vv[0] = o[6]; vv[1] = o[7];
                }
                if (c == 0) {
                    trace(l, 2);
                    if (lane == 0)
                        __hip_atomic_store(&S.sync[kWindow], (uint32_t)(gl + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
                // QK-norm and RoPE: out[i] = y[i] cos[i] - y[i+64] sin[i],
                // out[i+64] = y[i] sin[i+64] + y[i+64] cos[i+64] (i = lane)
                const double cl = bf16_bits_to_f32(S.rope[0][lane]), ch = bf16_bits_to_f32(S.rope[0][lane + 64]);
                const double sl = bf16_bits_to_f32(S.rope[1][lane]), sh = bf16_bits_to_f32(S.rope[1][lane + 64]);
                const double gq0 = bf16_bits_to_f32(S.qkn[0][lane]), gq1 = bf16_bits_to_f32(S.qkn[0][lane + 64]);
                const double ssq0 = wave_sum64_u(fma((double)qv[0][0], (double)qv[0][0], (double)qv[0][1] * (double)qv[0][1]));
                const double ssq1 = wave_sum64_u(fma((double)qv[1][0], (double)qv[1][0], (double)qv[1][1] * (double)qv[1][1]));
                const double ssk = owner ? wave_sum64_u(fma((double)kv2[0], (double)kv2[0], (double)kv2[1] * (double)kv2[1]))
                                         : 1.0;
                auto rope = [&](double sc, const float (&in)[2], double g0, double g1, float (&out)[2]) {
                    const double y0 = (double)in[0] * sc * g0, y1 = (double)in[1] * sc * g1;
                    out[0] = (float)(y0 * cl - y1 * sl);
                    out[1] = (float)(y0 * sh + y1 * ch);
                };
                float qr[2][2];
                rope(rms_scale(ssq0, D, kEps), qv[0], gq0, gq1, qr[0]);
                rope(rms_scale(ssq1, D, kEps), qv[1], gq0, gq1, qr[1]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    S.qa[c][h][lane] = qr[h][0];
                    S.qa[c][h][lane + 64] = qr[h][1];
                }
                const bool dbg = kDebug && r == 0 && l == last;
                if (dbg && c == 0 && a.dbg_q) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        a.dbg_q[(2 * x + h) * D + lane] = qr[h][0];
                        a.dbg_q[(2 * x + h) * D + lane + 64] = qr[h][1];
                    }
                }
                uint32_t own_k = 0u, own_v = 0u;
                if (owner) {
                    // this position's K and V rows, into the LDS copies the loops below read (K
                    // chunks permuted as the loader stores them; with several chunks, into the last
                    // one once it is in the slot), from where the KV loader of one rank per XCD
                    // stores them into the cache
                    float kr[2];
                    rope(rms_scale(ssk, D, kEps), kv2, bf16_bits_to_f32(S.qkn[1][lane]),
                         bf16_bits_to_f32(S.qkn[1][lane + 64]), kr);
                    const uint32_t k0 = f32_to_bf16_bits(kr[0]), k1 = f32_to_bf16_bits(kr[1]);
                    const uint32_t vw = f32_to_bf16_bits(vv[0]) | (f32_to_bf16_bits(vv[1]) << 16);
                    if constexpr (kDeep) {
                        own_k = k0 | (k1 << 16);
                        own_v = vw;
                    } else {
                        const int pl = pos - s0, p16 = pl % 16;
                        S.kvk[pl][8 * ((lane >> 3) ^ p16) + (lane & 7)] = (uint16_t)k0;
                        S.kvk[pl][8 * (((lane + 64) >> 3) ^ p16) + (lane & 7)] = (uint16_t)k1;
                        reinterpret_cast<uint32_t*>(S.kvv[pl])[lane] = vw;
                    }
                    // (the KV loader stores the row into the cache from this slot: store_row)
                    if (split || r == 0) {
                        const bool dbgkv = kDebug && l == last;
                        if (dbgkv && a.dbg_k) { a.dbg_k[x * D + lane] = kr[0]; a.dbg_k[x * D + lane + 64] = kr[1]; }
                        if (dbgkv && a.dbg_v) { a.dbg_v[x * D + 2 * lane] = vv[0]; a.dbg_v[x * D + 2 * lane + 1] = vv[1]; }
                    }
                }
                // Running softmax state over the chunks: shift mh and numerator sum lh of head
                // (lane >> 3) & 1, P V sums pa (dims 2 lane, 2 lane + 1 of both heads, even and
                // odd positions).
                double mh = -INFINITY, lh = 0.0;
                double pa[2][2][2];                      // (zeroed where its sums begin)
                const int jj = lane & 3, d16 = lane >> 2;
                // (the kDeep kernel keeps a running shift over the chunks; the other holds one chunk)
                {
                    constexpr bool kMC = kDeep;
                    // several chunks: the sums run over all of them; one chunk: zeroed just before
                    // P V, so that they are not live through the scores
                    if constexpr (kMC) {
#pragma unroll
                        for (int u = 0; u < 8; ++u) (&pa[0][0][0])[u] = 0.0;
                    }
                    for (int k = 0; k < (kMC ? nch : 1); ++k) {
                        const int ck = kAMaxLen * k, nk = min(ns - ck, kAMaxLen);
                        const int q0 = (nk + kCW - 1) / kCW;                    // <= 16
                        const int jb = min(nk, c * q0);                           // the wave's first slot row
                        const int np = max(0, min(nk, c * q0 + q0) - jb);
                        if (kMC && k > 0)
                            lds_wait(&S.sync[kReady + SL_B], ci0 + (uint32_t)k + 1u, lds_limit, &hdr->abort_flag);
                        if (kDeep && owner && k == nch - 1) {
                            const int pl = pos - s0 - ck, p16 = pl % 16;
                            S.kvk[pl][8 * ((lane >> 3) ^ p16) + (lane & 7)] = (uint16_t)(own_k & 0xffffu);
                            S.kvk[pl][8 * (((lane + 64) >> 3) ^ p16) + (lane & 7)] = (uint16_t)(own_k >> 16);
                            reinterpret_cast<uint32_t*>(S.kvv[pl])[lane] = own_v;
                        }
                        lds_order();
                        // Scores. Lane = jj + 4 d16: jj (bits 0-1) takes the slot rows jb + 4p + jj of
                        // passes p < ceil(np / 4), d16 (bits 2-5) the dims [8 d16, +8), both heads.
                        if (np > 0) {
                            const int passes = (np + 3) >> 2;    // <= 4
                            double2 qd[2][4];
                            uint4 kc[4];
#pragma unroll
                            for (int h = 0; h < 2; ++h)
#pragma unroll
                                for (int t = 0; t < 4; ++t) qd[h][t] = reinterpret_cast<const double2*>(&S.qa[c][h][8 * d16])[t];
#pragma unroll
                            for (int p = 0; p < 4; ++p) {
                                const int rl = jb + min(4 * p + jj, np - 1);            // slot row
                                kc[p] = reinterpret_cast<const uint4*>(S.kvk[rl])[d16 ^ (rl & 15)];
                            }
                            double E[8];                         // entry 2p + h: partial score over the 8 dims
                            // passes in pairs without a bound check (rows past the block are its last
                            // row; their scores are masked below), so that the four accumulation
                            // chains of a pair interleave
                            auto pass = [&](int p) {
                                double s0 = 0.0, s1 = 0.0;
                                const uint32_t k4[4] = {kc[p].x, kc[p].y, kc[p].z, kc[p].w};
#pragma unroll
                                for (int t = 0; t < 4; ++t) {
                                    const double klo = bf16_bits_to_f32(k4[t] & 0xffffu);
                                    const double khi = __uint_as_float(k4[t] & 0xffff0000u);
                                    s0 = fma(qd[0][t].x, klo, s0);
                                    s0 = fma(qd[0][t].y, khi, s0);
                                    s1 = fma(qd[1][t].x, klo, s1);
                                    s1 = fma(qd[1][t].y, khi, s1);
                                }
                                E[2 * p] = s0;
                                E[2 * p + 1] = s1;
                            };
                            pass(0);
                            pass(1);
                            if (passes > 2) {
                                pass(2);
                                pass(3);
                            } else {
#pragma unroll
                                for (int k = 4; k < 8; ++k) E[k] = 0.0;
                            }
                            // sum over d16 (lane bits 5, 4, 3, 2), transposed: the lane keeps entry
                            // 4 b5 + 2 b4 + b3, i.e. pass pe = 2 b5 + b4, head he = b3
#pragma unroll
                            for (int k = 0; k < 4; ++k) E[k] = tsum32(E[k], E[k + 4]);
#pragma unroll
                            for (int k = 0; k < 2; ++k) E[k] = tsum16(E[k], E[k + 2]);
                            {
                                const bool u3 = (lane & 8) != 0;
                                const double keep = u3 ? E[1] : E[0], send = u3 ? E[0] : E[1];
                                E[0] = keep + xor8_64(send);
                                E[0] += xor4_64(E[0]);
                            }
                            const int pe = 2 * ((lane >> 5) & 1) + ((lane >> 4) & 1);
                            const bool valid = 4 * pe + jj < np;
                            const double sc = valid ? E[0] * (double)a.attn_scale : -INFINITY;
                            // Softmax numerators e^s without the running maximum (m = 0) unless a valid
                            // score of this wave's block exceeds 600 in magnitude: then e^(s - m) with
                            // the block's maximum m per head (over the lanes of the same head, bits 0,
                            // 1, 4, 5). Within 600 no sum of up to 10240 terms e^s |v| (|v| up to the
                            // bf16 maximum, e^89) leaves fp64's range and e^-600 is a normal number, so
                            // both forms equal the exact softmax to fp64 rounding whatever keys the cache
                            // holds (rows written elsewhere included); each block's m travels with its
                            // partials, and the merges below rescale only blocks whose m differs from
                            // the largest.
                            const bool shift = __any(valid && fabs(sc) > 600.0);
                            double m = 0.0;
                            if (shift) {
                                m = sc;
                                m = fmax(m, partner64<1>(m));
                                m = fmax(m, partner64<2>(m));
                                m = fmax(m, xmax16(m));
                                m = fmax(m, xmax32(m));
                            }
                            // onto the running shift: M = max(mh, m); earlier chunks' sums scale by
                            // e^(mh - M), this chunk's numerators by e^(m - M) (1 unless a shift moved it)
                            // (no earlier chunk with a valid key: its sums are 0, any factor will do; the
                            // exponentials only when a shift moved, behind a wave-uniform branch)
                            const double Mn = kMC ? fmax(mh, m) : m;
                            double fo = 1.0, fn = 1.0;
                            if (kMC && __any(m != Mn || (mh != Mn && mh != -INFINITY))) {
                                fo = (mh == Mn || mh == -INFINITY) ? 1.0 : exp(mh - Mn);
                                fn = m == Mn ? 1.0 : exp(m - Mn);
                            }
                            const double pv = valid ? (kMC ? exp(sc - m) * fn : exp(sc - m)) : 0.0;
                            double ls = pv + partner64<1>(pv);
                            ls += partner64<2>(ls);
                            ls = tsum16(ls, ls);
                            ls = tsum32(ls, ls);
                            if (kMC && __any(fo != 1.0)) {
                                const double f0 = readlane64(fo, 0), f1 = readlane64(fo, 8);   // heads 0 and 1
#pragma unroll
                                for (int u = 0; u < 2; ++u) {
                                    pa[u][0][0] *= f0; pa[u][0][1] *= f0;
                                    pa[u][1][0] *= f1; pa[u][1][1] *= f1;
                                }
                            }
                            mh = Mn;
                            lh = kMC ? lh * fo + ls : ls;
                            // numerators to LDS: position 4 pe + jj, head he (one lane of each pair);
                            // all 16 entries, zero past the block, so that P V runs without bounds
                            if ((lane & 4) == 0) S.pw[c][4 * pe + jj][(lane >> 3) & 1] = pv;
                        }
                        // P V: lane l accumulates dims 2l, 2l + 1 of both heads over the wave's block, in
                        // rounds of 8 positions without bounds checks (numerators past the block are 0,
                        // their V row is the block's last); two accumulator sets, even and odd positions
                        lds_order();
                        if constexpr (!kMC) {
#pragma unroll
                            for (int u = 0; u < 8; ++u) (&pa[0][0][0])[u] = 0.0;
                        }
                        if (np > 0) {
                            const uint32_t* const vrow = reinterpret_cast<const uint32_t*>(S.kvv[jb]) + lane;
                            const int rounds = (np + 7) >> 3;               // <= 2
                            for (int t0 = 0; t0 < 8 * rounds; t0 += 8) {
                                double2 pp[8];
                                uint32_t vw[8];
#pragma unroll
                                for (int u = 0; u < 8; ++u) {
                                    pp[u] = *reinterpret_cast<const double2*>(S.pw[c][t0 + u]);
                                    vw[u] = vrow[(kAD / 2) * min(t0 + u, np - 1)];
                                }
#pragma unroll
                                for (int u = 0; u < 8; ++u) {
                                    const double vlo = bf16_bits_to_f32(vw[u] & 0xffffu), vhi = __uint_as_float(vw[u] & 0xffff0000u);
                                    double (&A)[2][2] = pa[u & 1];
                                    A[0][0] = fma(pp[u].x, vlo, A[0][0]);
                                    A[0][1] = fma(pp[u].x, vhi, A[0][1]);
                                    A[1][0] = fma(pp[u].y, vlo, A[1][0]);
                                    A[1][1] = fma(pp[u].y, vhi, A[1][1]);
                                }
                            }
                        }
                        lds_add(&S.sync[kConsumed + SL_B], lane);     // this chunk's slot rows are read
                    }
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<double2*>(&S.pacc[c][h][2 * lane]) =
                        make_double2(pa[0][h][0] + pa[1][h][0], pa[0][h][1] + pa[1][h][1]);
                if ((lane & ~8) == 0) {
                    S.pml[c][lane >> 3][0] = mh;
                    S.pml[c][lane >> 3][1] = lh;
                }
                // all four waves' partials in LDS
                lds_add(&S.sync[kArrive + AR_B], lane);
                lds_wait(&S.sync[kArrive + AR_B], (uint32_t)(kCW * (gl + 1)), lds_limit, &hdr->abort_flag);
                // merge: wave c takes attention dims [64c, +64) (head c / 2) from the four blocks;
                // lane w < 4 computes block w's weight e^(m_w - M), the others read it (weight 1
                // for blocks at the largest m, which is every block when none shifted, so that
                // the exponential is not evaluated at all then; an empty block weighs 0)
                const int hh = c >> 1, dim = 64 * (c & 1) + lane;
                double M = -INFINITY;
#pragma unroll
                for (int w = 0; w < kCW; ++w) M = fmax(M, S.pml[w][hh][0]);
                const double mine = S.pml[lane & 3][hh][0];
                double ew = mine == -INFINITY ? 0.0 : 1.0;
                if (mine != M && mine != -INFINITY) ew = exp(mine - M);
                double num = 0.0, den = 0.0;
#pragma unroll
                for (int w = 0; w < kCW; ++w) {
                    const double e = readlane64(ew, w);
                    num = fma(e, S.pacc[w][hh][dim], num);
                    den = fma(e, S.pml[w][hh][1], den);
                }
                if (!split) {
                    ao = (float)(num * rcp_nr(den));
                } else {
                    // This rank's partial over its slice: (max, denominator) of head hh and the
                    // numerators of dims [64c, +64), fp64 as two tagged XCD-local words each.
                    const uint32_t ta = tag(l, AS_ATT);
                    auto put_d = [&](int k, double v) {
                        const uint64_t u = (uint64_t)__double_as_longlong(v);
                        ll_put_xcd(&apart[((size_t)r * kAPart + k) * 2], (uint32_t)u, ta);
                        ll_put_xcd(&apart[((size_t)r * kAPart + k) * 2 + 1], (uint32_t)(u >> 32), ta);
                    };
                    put_d(4 + 64 * c + lane, num);
                    if ((c & 1) == 0 && lane == 0) {
                        put_d(2 * hh, M == -INFINITY ? -1e300 : M);          // an empty slice weighs 0
                        put_d(2 * hh + 1, den);
                    }
                    // merge: this rank's output dims D0, D0 + 1 (wave c) over the 32 partials;
                    // lane s < 32 reads rank s's (max, denominator) and numerators
                    const int D0 = 8 * r + 2 * c, hm = D0 >> 7;
                    const int sr = lane & 31;
                    const uint32_t w4[4] = {(uint32_t)((sr * kAPart + 2 * hm) * 2), (uint32_t)((sr * kAPart + 2 * hm + 1) * 2),
                                            (uint32_t)((sr * kAPart + 4 + D0) * 2), (uint32_t)((sr * kAPart + 5 + D0) * 2)};
                    float o8[8];
                    wt.get_pairs<4>(XRegion(apart, kARanks * kAPart * 2), w4, ta, o8, lane < 32 ? 4 : 0);
                    auto dv = [&](int i) {
                        return __longlong_as_double((long long)(((uint64_t)__float_as_uint(o8[2 * i + 1]) << 32) |
                                                                __float_as_uint(o8[2 * i])));
                    };
                    // slice weights e^(M_s - max M): 1 for the slices at the largest maximum (all
                    // of them when none shifted), 0 for empty ones
                    const double Ms = lane < 32 ? dv(0) : -1e300;
                    double Mx = Ms;
                    Mx = fmax(Mx, partner64<1>(Mx));
                    Mx = fmax(Mx, partner64<2>(Mx));
                    Mx = fmax(Mx, partner64<4>(Mx));
                    Mx = fmax(Mx, partner64<8>(Mx));
                    Mx = fmax(Mx, partner64<16>(Mx));                    // lanes 0-31: max over the ranks
                    double wgt = (lane < 32 && Ms != -1e300) ? 1.0 : 0.0;
                    if (lane < 32 && Ms != Mx && Ms != -1e300) wgt = exp(Ms - Mx);
                    double sd = wgt * (lane < 32 ? dv(1) : 0.0);
                    double s0n = wgt * (lane < 32 ? dv(2) : 0.0), s1n = wgt * (lane < 32 ? dv(3) : 0.0);
#define MQ_SPLIT_LEVEL(Mk)                                                                    \
                    sd += partner64<Mk>(sd);                                                  \
                    s0n += partner64<Mk>(s0n);                                                \
                    s1n += partner64<Mk>(s1n);
                    MQ_SPLIT_LEVEL(1) MQ_SPLIT_LEVEL(2) MQ_SPLIT_LEVEL(4) MQ_SPLIT_LEVEL(8) MQ_SPLIT_LEVEL(16)
#undef MQ_SPLIT_LEVEL
                    if (lane == 0) {
                        const double rd = rcp_nr(sd);
                        ll_put_xcd(&amrg[D0], __float_as_uint((float)(s0n * rd)), ta);
                        ll_put_xcd(&amrg[D0 + 1], __float_as_uint((float)(s1n * rd)), ta);
                    }
                    // gather dims [64c, +64) of the 256 merged outputs (8 ranks' words)
                    const uint32_t wg[1] = {(uint32_t)(64 * c + 2 * (lane >> 1))};
                    float o2[2];
                    wt.get_pairs<1>(XRegion(amrg, 2 * kAD), wg, ta, o2);
                    ao = o2[lane & 1];
                }
                if (kDebug && r == 0 && l == last && a.dbg_attn) a.dbg_attn[2 * D * x + 64 * c + lane] = ao;
            }
            if (c == 0) trace(l, 3);

            // ---------------- C: O partial over this XCD's attention dims ----------------
            {
                const uint32_t em = wave_max_u32(exp_field(ao));
                put_digits1(S.dig[c], ao, em, lane);
                lds_order();
                const i32x4_t af = a_frag(S.dig[c], 0, lane);
                const i32x4_t t0 = mfma_i8(af, b_frag(S.wC[c][0][lane]), i32x4_t{0, 0, 0, 0});
                const i32x4_t t1 = mfma_i8(af, b_frag(S.wC[c][1][lane]), i32x4_t{0, 0, 0, 0});
                double v0 = tile_value(t0, em), v1 = tile_value(t1, em);
                if constexpr (kW4) {      // the wave's 64 dims lie in the XCD's group c / 2
                    v0 *= (double)S.gsC[lane % 16][c / 2];
                    v1 *= (double)S.gsC[16 + lane % 16][c / 2];
                }
                if (lane < 16) { S.part[1][c][lane] = v0; S.part[1][c][16 + lane] = v1; }
            }
            if (last_arrival(&S.sync[kArrive + AR_C], lane)) {
                if (lane < 32) {
                    const double* P = &S.part[1][0][lane];
                    const double v = (P[0] + P[32]) + (P[64] + P[96]);
                    ll_put64(&po[(size_t)x * H + 32 * r + lane], pack_tagged(v, pbit(l)));
                }
            }
            if (c != 0) lds_add(&S.sync[kConsumed + SL_C], lane);
            if (c == 0) trace(l, 4);

            // ---------------- D (wave 0): reduce the O partials -> residual rows ----------------
            if (c == 0) {
                const int rr = lane % 32, q = lane / 32;
                double v4[4];
                wt.get_packed<4>(po + (size_t)(4 * q) * H + 32 * r + rr, H, pbit(l), v4);
                const double s4 = (v4[0] + v4[1]) + (v4[2] + v4[3]);
                const double tot = s4 + partner64<32>(s4);
                act_reg = (float)(tot * (double)S.scC[rr] + (double)S.hs[32 * r + rr]);
                lds_add(&S.sync[kConsumed + SL_C], lane);
                if (lane < 32) ll_put_xcd(&actx[32 * r + lane], __float_as_uint(act_reg), tag(l, AS_ACT));
                double ss = lane < 32 ? (double)act_reg * (double)act_reg : 0.0;
                ss += partner64<1>(ss);
                ss += partner64<2>(ss);
                ss += partner64<4>(ss);
                ss += partner64<8>(ss);
                ss += partner64<16>(ss);
                if (lane == 0) {
                    const uint64_t u = (uint64_t)__double_as_longlong(ss);
                    ll_put_xcd(&ass[2 * r], (uint32_t)u, tag(l, AS_ACT));
                    ll_put_xcd(&ass[2 * r + 1], (uint32_t)(u >> 32), tag(l, AS_ACT));
                }
                trace(l, 5);
            }

            // ---------------- E: RMSNorm + gate/up + SwiGLU ----------------
            {
                float av[4];
                const double ss = poll_slice(wt, actx, tag(l, AS_ACT), c, lane, av,
                                             [&] { slots_ready(1u << SL_F); });
                const double rstd2 = rms_scale(ss, H, kEps);
                const uint2 gw = *reinterpret_cast<const uint2*>(&S.lnE[256 * c + 4 * lane]);
                const float gl[4] = {bf16_bits_to_f32(gw.x & 0xffffu), bf16_bits_to_f32(gw.x >> 16),
                                     bf16_bits_to_f32(gw.y & 0xffffu), bf16_bits_to_f32(gw.y >> 16)};
                float nv2[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) nv2[i] = (float)((double)av[i] * rstd2 * (double)gl[i]);
                if (kDebug && g == 0 && l == last) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (a.dbg_act) a.dbg_act[256 * c + 4 * lane + i] = nv2[i];
                        if (a.dbg_resid) a.dbg_resid[256 * c + 4 * lane + i] = av[i];
                    }
                }
                uint32_t em = max(max(exp_field(nv2[0]), exp_field(nv2[1])), max(exp_field(nv2[2]), exp_field(nv2[3])));
                em = wave_max_u32(em);
                put_digits4(S.dig[c], nv2, em, lane);
                lds_order();
                i32x4_t op[12];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    op[3 * s] = a_frag(S.dig[c], s, lane);
                    op[3 * s + 1] = b_frag(S.wE[c][s][0][lane]);
                    op[3 * s + 2] = b_frag(S.wE[c][s][1][lane]);
                }
                operands_ready(op);
                double v0, v1;
                if constexpr (kW4) {
                    // one sum per tile and group of 128 (K steps 0-1, 2-3), scaled
                    i32x4_t t0[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}}, t1[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        t0[s / 2] = mfma_i8(op[3 * s], op[3 * s + 1], t0[s / 2]);
                        t1[s / 2] = mfma_i8(op[3 * s], op[3 * s + 2], t1[s / 2]);
                    }
                    const int j0 = lane % 16, j1 = min(16 + lane % 16, 23);      // tile rows 24-31 are zero
                    v0 = tile_value(t0[0], em) * (double)S.gsE[j0][2 * c] + tile_value(t0[1], em) * (double)S.gsE[j0][2 * c + 1];
                    v1 = tile_value(t1[0], em) * (double)S.gsE[j1][2 * c] + tile_value(t1[1], em) * (double)S.gsE[j1][2 * c + 1];
                } else {
                    i32x4_t t0 = {0, 0, 0, 0}, t1 = {0, 0, 0, 0};
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        t0 = mfma_i8(op[3 * s], op[3 * s + 1], t0);
                        t1 = mfma_i8(op[3 * s], op[3 * s + 2], t1);
                    }
                    v0 = tile_value(t0, em);
                    v1 = tile_value(t1, em);
                }
                if (lane < 16) { S.part[2][c][lane] = v0; S.part[2][c][16 + lane] = v1; }
            }
            if (last_arrival(&S.sync[kArrive + AR_E], lane)) {
                if (lane < 12) {
                    const double* P = &S.part[2][0][lane];
                    const double gs = ((P[0] + P[32]) + (P[64] + P[96])) * (double)S.scE[lane];
                    const double us = ((P[12] + P[44]) + (P[76] + P[108])) * (double)S.scE[12 + lane];
                    const float m = (float)silu_mul(gs, us);
                    ll_put_xcd(&mlpx[12 * r + lane], __float_as_uint(m), tag(l, AS_MLP));
                    if (kDebug && l == last && a.dbg_mlp) a.dbg_mlp[kAIX * x + 12 * r + lane] = m;
                }
            }
            lds_add(&S.sync[kConsumed + SL_E], lane);
            if (c == 0) trace(l, 6);

            // ---------------- F: down partial over this XCD's channels ----------------
            if (c < 3) {
                float mv[2];
                uint32_t w[1] = {2u * (uint32_t)(64 * c + lane)};
                wt.get_pairs<1>(XRegion(mlpx, kAIX), w, tag(l, AS_MLP), mv);
                if (c == 0) trace(l, 7);
                const uint32_t em = wave_max_u32(max(exp_field(mv[0]), exp_field(mv[1])));
                put_digits2(S.dig[c], mv, em, lane);
                lds_order();
                i32x4_t op[6];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    op[3 * s] = a_frag(S.dig[c], s, lane);
                    op[3 * s + 1] = b_frag(S.wF[c][s][0][lane]);
                    op[3 * s + 2] = b_frag(S.wF[c][s][1][lane]);
                }
                operands_ready(op);
                i32x4_t t0 = {0, 0, 0, 0}, t1 = {0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    t0 = mfma_i8(op[3 * s], op[3 * s + 1], t0);
                    t1 = mfma_i8(op[3 * s], op[3 * s + 2], t1);
                }
                double v0 = tile_value(t0, em), v1 = tile_value(t1, em);
                if constexpr (kW4) {      // the wave's 128 channels are the XCD's group c
                    v0 *= (double)S.gsF[lane % 16][c];
                    v1 *= (double)S.gsF[16 + lane % 16][c];
                }
                if (lane < 16) { S.part[3][c][lane] = v0; S.part[3][c][16 + lane] = v1; }
            }
            if (last_arrival(&S.sync[kArrive + AR_F], lane)) {      // wave 3 has no F slice: waves 0-2 sum
                if (lane < 32) {
                    const double* P = &S.part[3][0][lane];
                    const double v = (P[0] + P[32]) + P[64];
                    ll_put64(&pd[(size_t)x * H + 32 * r + lane], pack_tagged(v, pbit(l)));
                }
            }
            if (c != 0) lds_add(&S.sync[kConsumed + SL_F], lane);
            if (c == 0) trace(l, 8);

            // ---------------- G (wave 0): reduce the down partials -> hidden rows ----------------
            if (c == 0) {
                const int rr = lane % 32, q = lane / 32;
                double v4[4];
                wt.get_packed<4>(pd + (size_t)(4 * q) * H + 32 * r + rr, H, pbit(l), v4);
                const double s4 = (v4[0] + v4[1]) + (v4[2] + v4[3]);
                const double tot = s4 + partner64<32>(s4);
                const float hb = round_bf16((float)(tot * (double)S.scF[rr] + (double)act_reg));
                lds_add(&S.sync[kConsumed + SL_F], lane);
                if (lane < 32) ll_put_xcd(&hidx[32 * r + lane], __float_as_uint(hb), tag(l, AS_HID));
                double ss = lane < 32 ? (double)hb * (double)hb : 0.0;
                ss += partner64<1>(ss);
                ss += partner64<2>(ss);
                ss += partner64<4>(ss);
                ss += partner64<8>(ss);
                ss += partner64<16>(ss);
                if (lane == 0) {
                    const uint64_t u = (uint64_t)__double_as_longlong(ss);
                    ll_put_xcd(&hss[2 * r], (uint32_t)u, tag(l, AS_HID));
                    ll_put_xcd(&hss[2 * r + 1], (uint32_t)(u >> 32), tag(l, AS_HID));
                }
                trace(l, 9);
            }
        }
        // the final hidden vector and its sum of squares
        {
            float hv[4];
            const double ssq = poll_slice(wt, hidx, tag(last, AS_HID), c, lane, hv, [] {});
            *reinterpret_cast<float4*>(&S.hs[256 * c + 4 * lane]) = make_float4(hv[0], hv[1], hv[2], hv[3]);
            if (c == 0 && lane == 0) S.fss = ssq;
            if (kDebug && g == 0 && a.dbg_hidden) {
#pragma unroll
                for (int i = 0; i < 4; ++i) a.dbg_hidden[256 * c + 4 * lane + i] = (uint16_t)f32_to_bf16_bits(hv[i]);
            }
        }
    }

    // ================= final RMSNorm + LM head + greedy argmax (all waves) =================
    {
        constexpr int CH = H / (64 * 16);   // 1 KB chunks per row
        constexpr int RB = 8 / CH;
        constexpr int R = RB * CH;
        constexpr int span = kWave / RB;
        const int V = kargs()->V;
        const uint8_t* const lm_w = kargs()->lm_w;
        const float* const lm_s = kargs()->lm_s;
        const int r0 = (int)((int64_t)V * g / kNWG);
        const int r1 = (int)((int64_t)V * (g + 1) / kNWG);
        const int nb = (r1 - r0 + RB - 1) / RB;
        const int64_t rowbytes = H;
        uint4 cur[R], nxt[R];
        float scur = 0.0f, snxt = 0.0f;
        auto fetch = [&](int b, uint4* dst, float& s) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int row = r0 + b * RB + i / CH;
                dst[i] = make_uint4(0, 0, 0, 0);
                if (row < r1) dst[i] = ldg16(lm_w + row * rowbytes + (i % CH) * 1024 + lane * 16);
            }
            const int myrow = r0 + b * RB + lane / span;
            s = 1.0f;
            if (myrow < r1) s = gview(lm_s)[myrow];
        };
        int b = wave;
        if (b < nb) fetch(b, cur, scur);
        __syncthreads();                    // final hidden vector and sum of squares in LDS; loaders done
        const double rstd = rms_scale(S.fss, H, kEps);
        float* xsf = reinterpret_cast<float*>(S.xs);
#pragma unroll
        for (int i = 0; i < H / kThreads; ++i) {
            const int k = tid + i * kThreads;
            const float nv = (float)((double)S.hs[k] * rstd * (double)bf16_bits_to_f32(S.fnorm[k]));
            xsf[xs_index<Int8W>(k)] = nv;
            if (kDebug && g == 0 && a.dbg_norm) a.dbg_norm[k] = nv;
        }
        __syncthreads();
        trace(a.L, 0);

        const float inv_temp = kargs()->inv_temp;
        const uint64_t seed = kargs()->seed;
        float best_v = -INFINITY;
        int best_i = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < R; ++i) nxt[i] = make_uint4(0, 0, 0, 0);
        for (; b < nb; b += kWaves) {
            if (b + kWaves < nb) fetch(b + kWaves, nxt, snxt);
            float accv[R];
#pragma unroll
            for (int i = 0; i < R; ++i) accv[i] = dot_frag<Int8W>(cur[i], xs_frag<Int8W>(S.xs, i % CH, lane), 0.0f);
            const float s = transpose_reduce<R, CH>(accv, lane);
            const int row = r0 + b * RB + lane / span;
            if ((lane % span) == 0 && row < r1) {
                float v = s * scur;
                // sampling (temperature T > 0): argmax of logit / T + Gumbel noise draws the
                // token with probability softmax(logits / T) (the Gumbel-max identity)
                if (inv_temp > 0.0f) v = v * inv_temp + gumbel_noise(seed, pos, row);
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
        if (lane == 0) { S.lm_v[wave] = best_v; S.lm_i[wave] = best_i; }
        __syncthreads();
        trace(a.L, 1);
        const uint32_t tag_lm = tag(a.L, 0);
        if (tid == 0) {
            float bv = S.lm_v[0];
            int bi = S.lm_i[0];
            for (int w = 1; w < kWaves; ++w)
                if (S.lm_v[w] > bv || (S.lm_v[w] == bv && S.lm_i[w] < bi)) { bv = S.lm_v[w]; bi = S.lm_i[w]; }
            if (kDebug && a.dbg_bmax) a.dbg_bmax[g] = bv;
            if (kDebug && a.dbg_bidx) a.dbg_bidx[g] = bi;
            ll_put(&lmg[2 * g], ordered_key(bv), tag_lm);
            ll_put(&lmg[2 * g + 1], (uint32_t)bi, tag_lm);
        }
        // every workgroup reduces the 256 partial maxima itself: the step's token is then in
        // every workgroup for the next step's embedding, with no broadcast exchange
        if (wave == 0) {
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
                S.next_tok = chosen;
                if (g == 0) {
                    const int n_forced = kargs()->n_forced;
                    int* const tokens_out = kargs()->tokens_out;
                    if (tokens_out != nullptr && step >= n_forced - 1) tokens_out[step - (n_forced - 1)] = chosen;
                    if (step == n_steps - 1) {
                        *kargs()->out_token = chosen;
                        uint32_t* const status_out = kargs()->status_out;
                        if (status_out) *status_out = flag != 0u ? flag : (wt.dead ? 1u : 0u);
                        __hip_atomic_store(&hdr->asteps, AS0 + (uint32_t)n_steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(&hdr->epoch, E0 + (uint32_t)n_steps, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (kDebug && a.trace != nullptr)
                            a.trace[((int64_t)a.L * kTracePoints + 2) * kNWG] = __builtin_amdgcn_s_memrealtime();
                    }
                }
            }
        }
        __syncthreads();
        // the next step's input: a forced token, else this step's output (a failed step's
        // -1 becomes 0, which keeps the remaining steps' reads in bounds; they report -1)
        if (step + 1 < kargs()->n_forced) token = (int)__builtin_amdgcn_readfirstlane(*gview(kargs()->step_tokens + step + 1));
        else token = max(S.next_tok, 0);
    }
    }
}

// ---------------- host side ----------------

size_t decode_async_workspace_bytes(const DecodeShape& s) {
    if (s.H != kAH || s.I != kAI) return 0;
    return alayout_for(xlayout_total(kAH, kAI)).total;
}

bool decode_async_supports(const DecodeShape& s, bool int8, int cache_len) {
    return int8 && !s.fp8 && s.H == kAH && s.I == kAI && s.NQ == 16 && s.NKV == 8 && s.D == kAD &&
           cache_len <= kASplitLen;
}

// The cache_len from which this kernel splits attention over the 32 ranks of an XCD:
// past kAMaxLen always; `attn_split_min` > 0 lowers that (0 = default, < 0 = only when required).
int decode_async_split_min(int attn_split_min) {
    return attn_split_min > 0 ? std::min(attn_split_min, kAMaxLen + 1) : kAMaxLen + 1;
}

template <bool kW4, bool kDeep>
static const void* async_kernel_ptr(const KArgs& ka, bool debug) {
    if (ka.n_steps > 1) return reinterpret_cast<const void*>(&decode_async_kernel<false, true, kW4, kDeep>);
    if (debug) return reinterpret_cast<const void*>(&decode_async_kernel<true, false, kW4, kDeep>);
    return reinterpret_cast<const void*>(&decode_async_kernel<false, false, kW4, kDeep>);
}

int launch_decode_async(const KArgs& ka, bool debug, bool int4, hipStream_t stream, hipEvent_t t0, hipEvent_t t1) {
    // the launch's last step attends over cache_len pos + n_steps; past one chunk per slice
    // (32 x 64 positions) it needs the chunked instantiation
    const int steps = ka.n_steps > 1 ? ka.n_steps : 1;
    const bool deep = ka.pos + steps > kARanks * kAMaxLen;
    const void* fn = int4 ? (deep ? async_kernel_ptr<true, true>(ka, debug) : async_kernel_ptr<true, false>(ka, debug))
                          : (deep ? async_kernel_ptr<false, true>(ka, debug) : async_kernel_ptr<false, false>(ka, debug));
    int st = check_residency(fn);
    if (st != MQ_OK) return st;
    KArgs copy = ka;
    void* args[] = {&copy};
    const hipError_t e = launch_resident(fn, dim3(kNWG), dim3(kThreads), args, stream, t0, t1);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "launch(decode_async): %s", hipGetErrorString(e));
    return MQ_OK;
}

int decode_async_max_len() { return kASplitLen; }

// The longest cache_len for which the automatic choice takes this kernel: rank slices of up to
// three 64-position chunks. Past 2048 positions each further chunk of a rank's slice costs ~2 us
// per layer (it is loaded while the chunk before it is attended over, and written once all four
// compute waves are done with that one); measured against the XCD-aware kernel (kernel us per
// step, 64 steps from each depth): 4608: 560 vs 600; 5120: 565 vs 604; 5632: 574 vs 608; 6144
// (the steps reach a fourth chunk): 628 vs 618; 7168: 645 vs 631; 8192: 703 vs 649.
int decode_async_auto_len() { return kARanks * 192; }

}  // namespace mq
