// Prompt-batched prefill: the KV-cache rows of P prompt positions, each layer's
// weights passed over once for all P positions, on the int8 matrix cores.
//
// The reference prefills one decode step per prompt token (a10_decode.py:367-368,
// verify_correctness_a10.py:326-328); the cache rows a step writes are those of
// a10_int8_decode_kernel.cu:143-241. Here the P positions of a chunk go through a
// layer together, as matrix products of P activation rows with each weight matrix.
// The arithmetic is the decode-step kernels' (every stored value is the correctly
// rounded value of the reference's expression, up to fp64 rounding of the sums):
// each activation row becomes a 55-bit fixed-point number over its own
// power-of-two scale (digits.h), the products are exact int32 digit-plane sums
// on the int8 matrix cores recombined in fp64, and attention runs in fp64. So the
// cache rows equal those of P decode steps, apart from fp32 roundings that the
// fp64 summation order can move once in about 2^20 values.
//
// One persistent launch per chunk (a workgroup per compute unit, all resident); per layer
// nine phases over the chunk's P positions, separated by grid barriers:
//   digits      RMSNorm of the layer input (the embedding rows in layer 0), its
//               digit planes                                 one workgroup per position
//   QKV         q|k|v rows on the matrix cores; the epilogue runs QK-norm and RoPE
//               and writes this layer's K/V cache rows and the rotated queries
//               (a 128-row tile is one head, so the norm and the rotation pairs
//               are inside one wave)                        tiles of 32 positions x 128 rows
//   attention   causal, fp64 on the matrix cores, per (KV head, 8 positions) its 16
//               queries over cache rows [0, pos0 + p]; a workgroup takes one such
//               item or two of complementary length, its key blocks cut evenly over
//               the four waves
//   digits      of the attention output
//   O           + residual (the layer input)                 32 positions x 64 rows
//   digits      post-attention RMSNorm
//   gate|up     64 channels' gate and up rows per tile; SwiGLU in the epilogue
//   digits      of the SwiGLU output
//   down        + residual, bf16: the next layer's input
// The last layer stops after its cache rows. The first generated token comes from
// the decode step of the last prompt token, as in the reference's loop. A phase's work
// items (positions or product tiles) are dealt round-robin over the workgroups.
#include <algorithm>

#include "attention.h"
#include "digits.h"

namespace mq {

namespace {

constexpr int kFH = 1024, kFI = 3072, kFD = 128, kFQ = 2048, kFNKV = 8;
constexpr int kFKB = kFI / 64;             // most 64-element K blocks of a product (down: 3072)
constexpr int kTileP = 32;                 // positions per product tile: 4 waves x 4 pairs
constexpr int kFThreads = 256;

// Chunk workspace for Pp positions (a multiple of kTileP). Digit planes are laid out
// [K block][position][plane][64 bytes], so that the MFMA A operand of a position pair
// and K block (16 rows of 64 bytes) is 1 KB of contiguous memory.
struct PfLayout {
    size_t sync, hid, x, q, m, dig, emax, tok, total;
};
constexpr PfLayout pf_layout(size_t Pp) {
    PfLayout o{};
    size_t off = 0;
    o.sync = off; off += 1024;                         // grid-barrier counters, abort flag
    o.hid = off; off += round256(Pp * kFH * 2);        // layer input, bf16
    o.x = off; off += round256(Pp * kFH * 4);          // post-attention residual, fp32
    o.q = off; off += round256(Pp * kFQ * 4);          // rotated queries, fp32
    o.m = off; off += round256(Pp * kFI * 4);          // SwiGLU output, fp32
    o.dig = off; off += round256(Pp * kFKB * 512);     // digit planes of the current product's input
    o.emax = off; off += round256(Pp * 4);             // their exponents, one per position
    o.tok = off; off += round256(Pp * 4);              // the chunk's tokens
    o.total = off;
    return o;
}
constexpr size_t kPfPerPos = pf_layout(1024).total / 1024 + 1;

struct PfArgs {
    const uint16_t* embed;
    const LayerWeights* lw;
    const ScalePointers* sp;
    const uint16_t* cos_t;
    const uint16_t* sin_t;
    uint16_t* kc;
    uint16_t* vc;
    int layer, P, Pp, pos0, S, L;
    float attn_scale;
    uint32_t spin_limit;
    uint8_t* ws;
    uint64_t* trace;                       // optional phase timeline (kPfTracePoints per layer)
};

// Grid-barrier state. Counters are cumulative over a launch (zeroed before it), each on a
// 64-byte line of its own.
constexpr int kPfXcd = 8;
constexpr int kPfTracePoints = 18;            // phase k (9 per layer): 2 k phase done, 2 k + 1 barrier passed
struct PfSync {
    uint32_t count;                        // XCD leaders that reached the current barrier
    uint32_t abort;                        // set when a barrier wait expired
    uint32_t pad0[14];
    struct {
        uint32_t arrived;                  // workgroups of the XCD that reached the current barrier
        uint32_t released;                 // the last barrier the XCD's leader has passed
        uint32_t pad[14];
    } xcd[kPfXcd];
};
static_assert(sizeof(PfSync) <= 1024, "barrier state");

// LDS of a workgroup, shared by the phases
struct PfShared {
    double am[3][kWave][34];               // attention: parts handed to an item's leader wave (m, denominator, outputs)
    uint4 gb[2][8][kWave];                 // products: a K block's weight operands (B), shared by the waves
    double reds[4];
    uint32_t rede[4];
};

enum PfSrc { SRC_EMBED = 0, SRC_HID = 1, SRC_X = 2, SRC_M = 3, SRC_A = 4 };
enum PfEpi { EPI_QKV = 0, EPI_O = 1, EPI_GU = 2, EPI_DOWN = 3 };

// The kernel runs every phase of every layer in one body. Values that depend only on the
// thread or workgroup index are the same in every layer, and the compiler would otherwise
// compute them once, before the layer loop, and keep them all live through every phase (more
// than the register file holds). Reading the index through an empty volatile asm makes it
// new in each phase, so each phase computes what it needs at its start.
__device__ __forceinline__ int pf_fresh(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ int pf_fresh_uniform(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

template <class T>
__device__ __forceinline__ T* pf_buf(const PfArgs& a, size_t off) {
    return reinterpret_cast<T*>(a.ws + off);
}

// Digit planes of v (4 consecutive elements k0 .. k0 + 3 of position p) into the
// chunk's plane buffer.
__device__ __forceinline__ void store_digits4(uint8_t* dig, int Pp, int p, int k0, const float (&v)[4], uint32_t emax) {
    int d[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) digits55(v[i], emax, d[i]);
    uint8_t* base = dig + ((size_t)(k0 / 64) * Pp + p) * 512 + (k0 % 64);
#pragma unroll
    for (int pl = 0; pl < 8; ++pl)
        *reinterpret_cast<uint32_t*>(base + 64 * pl) = pack4(d[0][pl], d[1][pl], d[2][pl], d[3][pl]);
}

// Largest exponent field over a workgroup of kFThreads threads (uniform result).
__device__ __forceinline__ uint32_t block_max_u32(uint32_t e, uint32_t* red, int wave, int lane, int nwaves) {
    e = wave_max_u32(e);
    if (lane == 0) red[wave] = e;
    __syncthreads();
    uint32_t r = red[0];
    for (int w = 1; w < nwaves; ++w) r = max(r, red[w]);
    return r;
}

// ---- row -> (RMSNorm) -> digit planes ------------------------------------------------
// One work item per position. SRC_EMBED / SRC_HID: the layer input (bf16; in layer 0
// the embedding row of the token, also stored as the layer input), input RMSNorm.
// SRC_X: the post-attention residual, post-attention RMSNorm. SRC_M: the SwiGLU
// output, SRC_A: the attention output (in the query buffer), no norm. The normalized value is fp32(r * rstd * gain) as in the decode
// step (a10_int8_decode_kernel.cu:54-84, :421-457).
template <int K, int SRC>
__device__ void pf_digits(const PfArgs& a, int p, PfShared& sh) {
    constexpr int G = K / 1024;            // groups of 4 consecutive elements per thread
    static_assert(SRC == SRC_M || SRC == SRC_A || G == 1, "the normed rows are hidden-sized");
    double* const reds = sh.reds;
    uint32_t* const rede = sh.rede;
    const PfLayout L = pf_layout((size_t)a.Pp);
    const int t = pf_fresh(threadIdx.x), lane = t % kWave, wave = t / kWave;
    float v[G][4];
    if constexpr (SRC == SRC_EMBED || SRC == SRC_HID) {
        uint16_t* hid = pf_buf<uint16_t>(a, L.hid) + (size_t)p * kFH;
        const uint16_t* row = hid;
        if constexpr (SRC == SRC_EMBED) row = a.embed + (size_t)pf_buf<int>(a, L.tok)[p] * kFH;
        const uint2 u = *reinterpret_cast<const uint2*>(row + 4 * t);
        if constexpr (SRC == SRC_EMBED) *reinterpret_cast<uint2*>(hid + 4 * t) = u;
        v[0][0] = bf16_bits_to_f32(u.x & 0xffffu);
        v[0][1] = bf16_bits_to_f32(u.x >> 16);
        v[0][2] = bf16_bits_to_f32(u.y & 0xffffu);
        v[0][3] = bf16_bits_to_f32(u.y >> 16);
    } else {
        const float* row = SRC == SRC_X ? pf_buf<float>(a, L.x) + (size_t)p * kFH
                         : SRC == SRC_A ? pf_buf<float>(a, L.q) + (size_t)p * kFQ : pf_buf<float>(a, L.m) + (size_t)p * K;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float4 f = *reinterpret_cast<const float4*>(row + 1024 * g + 4 * t);
            v[g][0] = f.x; v[g][1] = f.y; v[g][2] = f.z; v[g][3] = f.w;
        }
    }
    float n[G][4];
    if constexpr (SRC != SRC_M && SRC != SRC_A) {
        double ss = 0.0;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) ss = fma((double)v[g][i], (double)v[g][i], ss);
        ss = wave_sum64(ss);
        if (lane == 0) reds[wave] = ss;
        __syncthreads();
        const double rstd = rms_scale((reds[0] + reds[1]) + (reds[2] + reds[3]), K, kEps);
        const LayerWeights lw = a.lw[a.layer];
        const uint16_t* gain = static_cast<const uint16_t*>(SRC == SRC_X ? lw.post_attn_layernorm_weight
                                                                         : lw.input_layernorm_weight);
        const uint2 gu = *reinterpret_cast<const uint2*>(gain + 4 * t);
        const float gv[4] = {bf16_bits_to_f32(gu.x & 0xffffu), bf16_bits_to_f32(gu.x >> 16),
                             bf16_bits_to_f32(gu.y & 0xffffu), bf16_bits_to_f32(gu.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i) n[0][i] = (float)((double)v[0][i] * rstd * (double)gv[i]);
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) n[g][i] = v[g][i];
    }
    uint32_t e = 0;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) e = max(e, exp_field(n[g][i]));
    e = block_max_u32(e, rede, wave, lane, kFThreads / kWave);
    uint8_t* dig = pf_buf<uint8_t>(a, L.dig);
#pragma unroll
    for (int g = 0; g < G; ++g) store_digits4(dig, a.Pp, p, 1024 * g + 4 * t, n[g], e);
    if (t == 0) pf_buf<uint32_t>(a, L.emax)[p] = e;
}

// ---- products on the int8 matrix cores -------------------------------------------------
// Work item (row tile rt, position tile pt) of a workgroup of kFThreads threads: wave w takes positions
// [32 pt + 8 w, +8) (four pairs) and the tile's NT row blocks of 16. Per 64-element K block
// a wave loads its four A operands (a pair's 8 + 8 digit planes: 1 KB contiguous) and NT B
// operands (16 weight rows x 64 bytes) and issues 4 NT MFMAs, with the next block's operands
// in flight. The output tile of pair j, block t: lane l (bit 4 clear) ends with the value of
// position 2j + l / 32 and weight row 16 t + l % 16 (tile_value).
//
// Row tiles: QKV 32 x 128 rows (q heads 0-15, k heads 0-7, v heads 0-7); O and down
// 16 x 64 rows; gate|up 48 tiles of 64 channels, blocks 0-3 gate rows, 4-7 up rows.
template <int EPI>
struct GemmShape {
    static constexpr int K = EPI == EPI_O ? kFQ : EPI == EPI_DOWN ? kFI : kFH;
    static constexpr int NT = (EPI == EPI_QKV || EPI == EPI_GU) ? 8 : 4;
    static constexpr int NRT = EPI == EPI_QKV ? 32 : EPI == EPI_GU ? 48 : 16;
};

template <int EPI>
__device__ void pf_gemm(const PfArgs& a, int tile, PfShared& sh) {
    using GS = GemmShape<EPI>;
    constexpr int K = GS::K, NT = GS::NT, NK = K / 64;
    const PfLayout L = pf_layout((size_t)a.Pp);
    const int tid = pf_fresh(threadIdx.x), lane = tid % kWave, w = tid / kWave;
    const int rt = tile % GS::NRT, pt = tile / GS::NRT;
    const int p0 = kTileP * pt + 8 * w;
    const int l16 = lane % 16;
    const LayerWeights lw = a.lw[a.layer];
    const ScalePointers sp = a.sp[a.layer];

    // the lane's weight row of each block, and its scale
    const int8_t* wrow[NT];
    const float* srow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int8_t* base;
        const float* sc;
        int row;
        if constexpr (EPI == EPI_QKV) {
            if (rt < 16) { base = (const int8_t*)lw.q_proj_weight; sc = sp.q_scale; row = 128 * rt; }
            else if (rt < 24) { base = (const int8_t*)lw.k_proj_weight; sc = sp.k_scale; row = 128 * (rt - 16); }
            else { base = (const int8_t*)lw.v_proj_weight; sc = sp.v_scale; row = 128 * (rt - 24); }
            row += 16 * t + l16;
        } else if constexpr (EPI == EPI_GU) {
            base = (const int8_t*)(t < 4 ? lw.gate_proj_weight : lw.up_proj_weight);
            sc = t < 4 ? sp.gate_scale : sp.up_scale;
            row = 64 * rt + 16 * (t % 4) + l16;
        } else {
            base = (const int8_t*)(EPI == EPI_O ? lw.o_proj_weight : lw.down_proj_weight);
            sc = EPI == EPI_O ? sp.o_scale : sp.down_scale;
            row = 64 * rt + 16 * t + l16;
        }
        wrow[t] = base + (size_t)row * K + 16 * (lane / 16);
        srow[t] = sc + row;
    }
    const uint8_t* abase = pf_buf<uint8_t>(a, L.dig) + (size_t)p0 * 512 + l16 * 64 + 16 * (lane / 16);
    const size_t kstride = (size_t)a.Pp * 512;

    i32x4_t acc[4][NT];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[j][t] = i32x4_t{0, 0, 0, 0};
    // Each wave loads a quarter of a K block's weight tile (NB of the NT row blocks) and
    // shares it through LDS: the four waves would otherwise each load the whole tile, and
    // those loads (16 rows x 64 bytes per instruction) were most of a product's time.
    constexpr int NB = NT / 4;
    auto load = [&](int kb, i32x4_t (&A)[4], uint4 (&Bs)[NB]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 u = ldg16(abase + kb * kstride + 1024 * j);
            A[j] = i32x4_t{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) Bs[u] = ldg16(wrow[NB * w + u] + 64 * kb);
    };
    // three K blocks' operands in registers (stage kb % 3): block kb + 3's loads go into the
    // registers block kb has just used, so each load has three blocks of work to arrive in
    i32x4_t A0[4], A1[4], A2[4];
    uint4 B0[NB], B1[NB], B2[NB];
    load(0, A0, B0);
    __builtin_amdgcn_sched_barrier(0);
    if (NK > 1) load(1, A1, B1);
    __builtin_amdgcn_sched_barrier(0);
    if (NK > 2) load(2, A2, B2);
    __builtin_amdgcn_sched_barrier(0);
    auto step = [&](int kb, i32x4_t (&A)[4], uint4 (&Bs)[NB]) {
        // the wave's share into LDS buffer kb % 2; after the barrier every wave has finished
        // block kb - 1, whose buffer kb + 1 will overwrite
        uint4 (*gb)[kWave] = sh.gb[kb % 2];
#pragma unroll
        for (int u = 0; u < NB; ++u) gb[NB * w + u][lane] = Bs[u];
        __syncthreads();
        i32x4_t B[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint4 u = gb[t][lane];
            B[t] = i32x4_t{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[j][t] = mfma_i8(A[j], B[t], acc[j][t]);
        if (kb + 3 < NK) load(kb + 3, A, Bs);
        // kept in this order: left to itself the scheduler moves later blocks' MFMAs up to
        // the loads and waits for nearly every load in flight before the first of them
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int kb = 0; kb < NK; kb += 3) {
        step(kb, A0, B0);
        if (kb + 1 < NK) step(kb + 1, A1, B1);
        if (kb + 2 < NK) step(kb + 2, A2, B2);
    }
    __syncthreads();                        // the last blocks' buffers are read before the next tile writes them

    // ---- epilogue ----
    // Every global value the epilogue reads is requested first, for all four pairs, so that
    // they come back in one memory round trip (issued pair by pair, each pair waited for
    // its own: four round trips per tile).
    const bool owner = (lane & 16) == 0;       // after tile_value: lanes 0-15 (even pair member), 32-47 (odd)
    const uint32_t* emax = pf_buf<uint32_t>(a, L.emax);
    int pj[4];
    uint32_t exv[4];
    float scv[NT];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pj[j] = p0 + 2 * j + (lane >> 5);                  // chunk position of this lane's values (< Pp)
        exv[j] = emax[pj[j]];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) scv[t] = *srow[t];
    // QKV: QK-norm gains and the positions' RoPE rows (bf16, rows clamped into the table);
    // O / down: the residual rows
    uint32_t gnv[8], cs[4][16];
    float res[4][NT];
    if constexpr (EPI == EPI_QKV) {
        if (rt < 24) {
            const uint16_t* gn = static_cast<const uint16_t*>(rt < 16 ? lw.q_norm_weight : lw.k_norm_weight);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                gnv[t] = gn[16 * t + l16];
                gnv[t + 4] = gn[16 * t + l16 + 64];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int pos = min(a.pos0 + pj[j], a.S - 1);
                const uint16_t* cr = a.cos_t + (size_t)pos * kFD;
                const uint16_t* sr = a.sin_t + (size_t)pos * kFD;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int i = 16 * t + l16;
                    cs[j][t] = cr[i];
                    cs[j][4 + t] = cr[i + 64];
                    cs[j][8 + t] = sr[i];
                    cs[j][12 + t] = sr[i + 64];
                }
            }
        }
    } else if constexpr (EPI == EPI_O || EPI == EPI_DOWN) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int n = 64 * rt + 16 * t + l16;
                if constexpr (EPI == EPI_O) res[j][t] = bf16_bits_to_f32(pf_buf<uint16_t>(a, L.hid)[(size_t)pj[j] * kFH + n]);
                else res[j][t] = pf_buf<float>(a, L.x)[(size_t)pj[j] * kFH + n];
            }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = pj[j];
        double val[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) val[t] = tile_value(acc[j][t], exv[j]);
        const bool store = owner && p < a.P;
        const int pos = a.pos0 + p;
        if constexpr (EPI == EPI_QKV) {
            if (rt < 24) {
                // q or k head: fp32 value, QK RMSNorm over the head's 128 dims (8 blocks in the
                // lane, 16 lanes of the row), RoPE on the pairs (i, i + 64) = blocks (t, t + 4)
                float y[8];
                double ss = 0.0;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    y[t] = (float)(val[t] * (double)scv[t]);
                    ss = fma((double)y[t], (double)y[t], ss);
                }
                ss += partner64<1>(ss);
                ss += partner64<2>(ss);
                ss += partner64<4>(ss);
                ss += partner64<8>(ss);
                if (store) {
                    const double rs = rms_scale(ss, kFD, kEps);
                    const int64_t crow = rt < 16 ? 0 : (((int64_t)a.layer * kFNKV + (rt - 16)) * a.S + pos) * kFD;
                    float* qrow = pf_buf<float>(a, L.q) + (size_t)p * kFQ + 128 * rt;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 16 * t + l16;
                        const double y0 = (double)y[t] * rs * (double)bf16_bits_to_f32(gnv[t]);
                        const double y1 = (double)y[t + 4] * rs * (double)bf16_bits_to_f32(gnv[t + 4]);
                        const double cl = bf16_bits_to_f32(cs[j][t]), ch = bf16_bits_to_f32(cs[j][4 + t]);
                        const double sl = bf16_bits_to_f32(cs[j][8 + t]), sh = bf16_bits_to_f32(cs[j][12 + t]);
                        const float o0 = (float)(y0 * cl - y1 * sl);
                        const float o1 = (float)(y0 * sh + y1 * ch);
                        if (rt < 16) {
                            qrow[i] = o0;
                            qrow[i + 64] = o1;
                        } else {
                            a.kc[crow + i] = (uint16_t)f32_to_bf16_bits(o0);
                            a.kc[crow + i + 64] = (uint16_t)f32_to_bf16_bits(o1);
                        }
                    }
                }
            } else if (store) {
                const int64_t crow = (((int64_t)a.layer * kFNKV + (rt - 24)) * a.S + pos) * kFD;
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    a.vc[crow + 16 * t + l16] = (uint16_t)f32_to_bf16_bits((float)(val[t] * (double)scv[t]));
            }
        } else if constexpr (EPI == EPI_O) {
            if (store) {
                float* x = pf_buf<float>(a, L.x) + (size_t)p * kFH;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int n = 64 * rt + 16 * t + l16;
                    x[n] = (float)(val[t] * (double)scv[t] + (double)res[j][t]);
                }
            }
        } else if constexpr (EPI == EPI_GU) {
            if (store) {
                float* m = pf_buf<float>(a, L.m) + (size_t)p * kFI;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const double gs = val[t] * (double)scv[t];
                    const double us = val[t + 4] * (double)scv[t + 4];
                    m[64 * rt + 16 * t + l16] = (float)silu_mul(gs, us);
                }
            }
        } else {
            if (store) {
                uint16_t* hid = pf_buf<uint16_t>(a, L.hid) + (size_t)p * kFH;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int n = 64 * rt + 16 * t + l16;
                    hid[n] = (uint16_t)f32_to_bf16_bits((float)(val[t] * (double)scv[t] + (double)res[j][t]));
                }
            }
        }
    }
}

// ---- causal attention on the fp64 matrix cores -------------------------------------------
// Work item (KV head x, tile of 8 positions p0..p0+7): its 16 queries (lane
// column q = lane % 16: position p0 + q % 8, query head 2x + q / 8) attend over the cache
// rows [0, pos0 + p], 16 keys per block, with v_mfma_f64_16x16x4f64 (A: lane l holds
// A[l % 16][l / 16]; B: B[l / 16][l % 16]; D: register i of lane l holds D[4 i + l / 16]
// [l % 16]). Both products are transposed so that each lane works for its own query:
//   scores S^T = K Q^T: A = K (key rows x dim slots), B = Q^T; instruction j's slot g is
//     dim 32 g + j, so lane l reads 32 contiguous dims of key row l % 16 and of its query;
//     register i of lane l then holds key 4 i + g (g = l / 16) of query q;
//   outputs O^T = V^T P^T: A = V^T, B = P^T; instruction j's slot g is key 4 j + g, which
//     is register j of the lane's own scores, and row c of tile t is dim 8 c + t, so lane
//     l reads 8 contiguous dims of V row 4 j + g; register i of tile t then holds dim
//     32 i + 8 g + t of query q.
// Softmax in fp64: e = exp(s - m) with the query's shift m raised only when a block's
// maximum exceeds it by more than 2^8 (then the accumulators are rescaled), so e stays
// below e^256; the lane's partial denominator covers its keys and the four lane groups'
// are added at the end. Each K and V row is read once per item (8 positions share it),
// where the per-position form read it once per position. The outputs (fp32, as the
// reference stores them) replace the item's queries in the query buffer.
typedef double f64x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f64x4_t mfma_f64(double a, double b, f64x4_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// The key blocks [b0, b1) (16 keys each) of item (x, p0) in one wave: the partial softmax
// state of the lane's query over them (shift m, partial denominator lsum, outputs acc, not
// yet divided). An empty range leaves m = -inf, lsum = 0, acc = 0.
__device__ __forceinline__ void pf_attn_blocks(const PfArgs& a, int x, int p0, int b0, int b1, double& m, double& lsum,
                                               f64x4_t (&acc)[8]) {
    const PfLayout L = pf_layout((size_t)a.Pp);
    const int lane = pf_fresh(threadIdx.x) % kWave;
    const int q = lane % 16, g = lane / 16;
    const int pq = p0 + q % 8;                              // chunk position of the lane's query
    const bool qvalid = pq < a.P;
    const int qpos = a.pos0 + pq;                           // its cache position: keys [0, qpos]
    const int klast = a.pos0 + min(p0 + 7, a.P - 1);        // the item's last key
    const double sc = (double)a.attn_scale;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f64x4_t{0.0, 0.0, 0.0, 0.0};
    m = -INFINITY;
    lsum = 0.0;
    if (b0 >= b1) return;
    const float* const qrow = pf_buf<float>(a, L.q) + (size_t)min(pq, a.P - 1) * kFQ + 256 * x + 128 * (q / 8);
    double qd[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 f = qvalid ? reinterpret_cast<const float4*>(qrow + 32 * g)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        qd[4 * j] = f.x; qd[4 * j + 1] = f.y; qd[4 * j + 2] = f.z; qd[4 * j + 3] = f.w;
    }
    const int64_t head = ((int64_t)a.layer * kFNKV + x) * a.S * kFD;
    const uint16_t* kb = a.kc + head;
    const uint16_t* vb = a.vc + head;
    // K row k0 + q (dims 32 g..), V rows k0 + 4 j + g (dims 8 q..), clamped into the cache;
    // the next block's are in flight while a block is computed
    uint4 kw[4], vw[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) kw[j] = ldg16(reinterpret_cast<const uint4*>(kb + (size_t)min(k0 + q, klast) * kFD + 32 * g) + j);
#pragma unroll
        for (int j = 0; j < 4; ++j) vw[j] = ldg16(vb + (size_t)min(k0 + 4 * j + g, klast) * kFD + 8 * q);
    };
    load(16 * b0);
    for (int bk = b0; bk < b1; ++bk) {
        const int k0 = 16 * bk;
        const uint4 kc[4] = {kw[0], kw[1], kw[2], kw[3]};
        const uint4 vc[4] = {vw[0], vw[1], vw[2], vw[3]};
        if (bk + 1 < b1) load(k0 + 16);
        f64x4_t sa = {0.0, 0.0, 0.0, 0.0}, sb = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint4 w4 = kc[j / 8];
            const uint32_t w = (j % 8) < 2 ? w4.x : (j % 8) < 4 ? w4.y : (j % 8) < 6 ? w4.z : w4.w;
            const double kv = (j % 2) ? (double)__uint_as_float(w & 0xffff0000u) : (double)bf16_bits_to_f32(w & 0xffffu);
            if (j % 2) sb = mfma_f64(kv, qd[j], sb);
            else sa = mfma_f64(kv, qd[j], sa);
        }
        double e[4], mb = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = k0 + 4 * i + g;
            e[i] = (qvalid && key <= qpos) ? (sa[i] + sb[i]) * sc : -INFINITY;
            mb = fmax(mb, e[i]);
        }
        mb = fmax(mb, partner64<16>(mb));
        mb = fmax(mb, partner64<32>(mb));
        // raise the shift when the block's maximum exceeds it by more than 2^8 (always on
        // the first block with a valid key); the same decision in the query's four lanes
        const bool raise = mb > m + 256.0;
        if (__any(raise)) {
            const double alpha = raise ? exp(m - mb) : 1.0;      // 0 while m is -inf
            lsum *= alpha;
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] *= alpha;
            m = raise ? mb : m;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            e[i] = e[i] == -INFINITY ? 0.0 : exp(e[i] - m);
            lsum += e[i];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t vv[4] = {vc[j].x, vc[j].y, vc[j].z, vc[j].w};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t w = vv[t / 2];
                const double v = (t % 2) ? (double)__uint_as_float(w & 0xffff0000u) : (double)bf16_bits_to_f32(w & 0xffffu);
                acc[t] = mfma_f64(v, e[j], acc[t]);
            }
        }
    }
}

// Number of 16-key blocks of item (x, p0): keys [0, pos0 + min(p0 + 7, P - 1)].
__device__ __forceinline__ int pf_attn_nblocks(const PfArgs& a, int p0) {
    return (a.pos0 + min(p0 + 7, a.P - 1)) / 16 + 1;
}

// One attention unit on the workgroup's four waves: item A = (KV head x, positions pa ..
// pa + 7) and, if pb >= 0, item B = (x, pb .. pb + 7). The unit's T = nA + nB key blocks (A's,
// then B's) are cut into four contiguous ranges [T w / 4, T (w + 1) / 4), one per wave w, so
// a wave's range may hold the end of A and the start of B. Wave 0 merges A's partial states
// and writes A's outputs, wave 3 does the same for B. The other parts go through LDS: A's part
// of wave w (w > 0) to slot w - 1, B's part of wave w (w < 3) to slot w (slot k cannot hold
// both: A's part of wave k + 1 needs T (k + 1) / 4 < nA, B's part of wave k needs it > nA).
// A leader computes its own part last, so that it stays in registers. Both workgroup
// barriers are reached by every wave.
__device__ void pf_attention_unit(const PfArgs& a, int x, int pa, int pb, PfShared& sh) {
    const int w = __builtin_amdgcn_readfirstlane(pf_fresh(threadIdx.x) / kWave);
    const int lane = pf_fresh(threadIdx.x) % kWave;
    const int nA = pf_attn_nblocks(a, pa), nB = pb >= 0 ? pf_attn_nblocks(a, pb) : 0, T = nA + nB;
    auto cut = [&](int i) { return (T * i) / 4; };
    // the wave's parts, leader part last: (item, first block, end block, slot or -1 to keep)
    int part_p[2], part_b0[2], part_b1[2], part_slot[2];
    {
        const int r0 = cut(w), r1 = cut(w + 1);
        const int a0 = r0, a1 = min(r1, nA);                   // A's blocks of the range
        const int c0 = max(r0, nA) - nA, c1 = r1 - nA;         // B's blocks of the range
        if (w == 0) {
            part_p[0] = pb; part_b0[0] = c0; part_b1[0] = nB > 0 ? c1 : c0; part_slot[0] = 0;
            part_p[1] = pa; part_b0[1] = a0; part_b1[1] = a1; part_slot[1] = -1;
        } else if (w == 3 && nB > 0) {
            part_p[0] = pa; part_b0[0] = a0; part_b1[0] = a1; part_slot[0] = 2;
            part_p[1] = pb; part_b0[1] = c0; part_b1[1] = c1; part_slot[1] = -1;
        } else {
            part_p[0] = pa; part_b0[0] = a0; part_b1[0] = a1; part_slot[0] = w - 1;
            part_p[1] = pb; part_b0[1] = c0; part_b1[1] = nB > 0 ? c1 : c0; part_slot[1] = w;
        }
    }
    double m = -INFINITY, lsum = 0.0;
    f64x4_t acc[8];
#pragma unroll 1
    for (int k = 0; k < 2; ++k) {
        const int pk = __builtin_amdgcn_readfirstlane(k == 0 ? part_p[0] : part_p[1]);
        const int b0 = __builtin_amdgcn_readfirstlane(k == 0 ? part_b0[0] : part_b0[1]);
        const int b1 = __builtin_amdgcn_readfirstlane(k == 0 ? part_b1[0] : part_b1[1]);
        const int sl = __builtin_amdgcn_readfirstlane(k == 0 ? part_slot[0] : part_slot[1]);
        if (sl >= 0 && b0 >= b1) continue;                     // no part to hand over
        pf_attn_blocks(a, x, pk, b0, b1, m, lsum, acc);
        if (sl >= 0) {
            double* const slot = sh.am[sl][lane];
            slot[0] = m;
            slot[1] = lsum;
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) slot[2 + 4 * t + i] = acc[t][i];
        }
    }
    __syncthreads();
    const bool leadA = w == 0, leadB = w == 3 && nB > 0;
    if (leadA || leadB) {
        // the other waves' parts of this item: wave i's is in slot i - 1 (item A) or i (item B)
        auto has = [&](int i) {
            return leadA ? (i > 0 && cut(i) < min(cut(i + 1), nA)) : (i < 3 && max(cut(i), nA) < cut(i + 1));
        };
        double mm = m;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (has(i)) mm = fmax(mm, sh.am[leadA ? max(i - 1, 0) : min(i, 2)][lane][0]);
        const double f0 = m == -INFINITY ? 0.0 : exp(m - mm);
        lsum *= f0;
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] *= f0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (!has(i)) continue;
            const double* const slot = sh.am[leadA ? max(i - 1, 0) : min(i, 2)][lane];
            const double mj = slot[0];
            const double fj = mj == -INFINITY ? 0.0 : exp(mj - mm);
            lsum += slot[1] * fj;
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][j] += slot[2 + 4 * t + j] * fj;
        }
        lsum += partner64<16>(lsum);        // the query's four lanes: all valid or all not
        lsum += partner64<32>(lsum);
        const double r = rcp_nr(lsum);
        const int p0 = leadA ? pa : pb;
        const int q = lane % 16, g = lane / 16;
        const int pq = p0 + q % 8;
        if (pq < a.P) {
            float* const orow = pf_buf<float>(a, pf_layout((size_t)a.Pp).q) + (size_t)pq * kFQ + 256 * x + 128 * (q / 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float o[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) o[t] = (float)(acc[t][i] * r);
                float4* dst = reinterpret_cast<float4*>(orow + 32 * i + 8 * g);
                dst[0] = make_float4(o[0], o[1], o[2], o[3]);
                dst[1] = make_float4(o[4], o[5], o[6], o[7]);
            }
        }
    }
    __syncthreads();                        // the slots are read before the next unit writes them
}

// ---- grid barrier ----------------------------------------------------------------------
// Two levels. A workgroup's results are in its XCD's L2 once it reaches the barrier (the
// workgroup barrier first waits for its stores). The last workgroup of an XCD to arrive is
// that XCD's leader: its agent-scope release writes the XCD's L2 back to memory (once per XCD
// and barrier: one write-back per workgroup, 32 per XCD, cost 26-90 us per barrier), then it
// arrives at the grid counter, waits for the other seven leaders, drops stale lines of the
// L2 (acquire) and releases its XCD's workgroups, which drop their own stale lines. Barrier
// number b completes when the counters reach b times their arrivals. A wait that expires
// sets the abort flag, and every later wait of the launch then returns at once, so the
// grid always drains (the host reports MQ_ERR_TIMEOUT, mq_prefill_check). Needs the
// workgroups dealt round-robin over the 8 XCDs (checked by the host).
__device__ __forceinline__ bool pf_wait_ge(const uint32_t* p, uint32_t target, PfSync* sy, uint32_t limit) {
    uint32_t n = 0;
    while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        if (__hip_atomic_load(&sy->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return false;
        __builtin_amdgcn_s_sleep(2);
        if (++n >= limit) {
            __hip_atomic_store(&sy->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    return true;
}

__device__ __forceinline__ void pf_grid_barrier(PfSync* sy, uint32_t b, uint32_t limit) {
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t x = hw_xcc_id() % kPfXcd;
        const uint32_t per_xcd = gridDim.x / kPfXcd;
        const uint32_t old = __hip_atomic_fetch_add(&sy->xcd[x].arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == b * per_xcd - 1u) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_fetch_add(&sy->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pf_wait_ge(&sy->count, b * kPfXcd, sy, limit);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __hip_atomic_store(&sy->xcd[x].released, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            pf_wait_ge(&sy->xcd[x].released, b, sy, limit);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
}

// The whole chunk in one launch: every layer's eight phases, each phase's work items dealt
// over the workgroups: product tiles round-robin as rt + NRT pt (with NRT a multiple of 8 a
// row tile's position tiles all run on one XCD and share its L2 copy of the weights),
// attention items in units of even length (pf_attention_unit).
__global__ void __launch_bounds__(kFThreads, 1) pf_chunk_kernel(PfArgs a) {
    __shared__ PfShared sh;
    const PfLayout L0 = pf_layout((size_t)a.Pp);
    PfSync* const sy = pf_buf<PfSync>(a, L0.sync);
    const int G = (int)gridDim.x, g = (int)blockIdx.x;
    const int PT = (a.P + kTileP - 1) / kTileP;
    uint32_t nb = 0;
    int l = 0;
    auto stamp = [&](int point) {
        if (a.trace != nullptr && threadIdx.x == 0)
            a.trace[((size_t)l * kPfTracePoints + point) * G + g] = __builtin_amdgcn_s_memrealtime();
    };
    auto barrier = [&](int k) {
        stamp(2 * k);
        pf_grid_barrier(sy, ++nb, a.spin_limit);
        stamp(2 * k + 1);
    };
    for (l = 0; l < a.L; ++l) {
        PfArgs b = a;
        b.layer = l;
        for (int p = pf_fresh_uniform(g); p < a.P; p += G) {
            if (l == 0) pf_digits<kFH, SRC_EMBED>(b, p, sh);
            else pf_digits<kFH, SRC_HID>(b, p, sh);
        }
        barrier(0);
        for (int t = pf_fresh_uniform(g); t < GemmShape<EPI_QKV>::NRT * PT; t += G) pf_gemm<EPI_QKV>(b, t, sh);
        if (l == a.L - 1) { stamp(2); break; }                 // the last layer contributes its cache rows only
        barrier(1);
        {
            // attention units, one per workgroup: a chunk of at most G items (KV head, tile of 8
            // positions) gives each workgroup one item; a longer one pairs tile j with tile
            // np - 1 - j of the same head, so that every unit holds about as many key blocks.
            // Unit u runs KV head u % 8, on the XCD whose L2 then holds that head's rows.
            const int np = (a.P + 7) / 8, items = kFNKV * np;
            const bool paired = items > G;
            const int units = paired ? kFNKV * ((np + 1) / 2) : items;
            for (int u = pf_fresh_uniform(g); u < units; u += G) {
                const int j = u / kFNKV, jb = np - 1 - j;
                pf_attention_unit(b, u % kFNKV, 8 * j, paired && jb > j ? 8 * jb : -1, sh);
            }
        }
        barrier(2);
        for (int p = pf_fresh_uniform(g); p < a.P; p += G) pf_digits<kFQ, SRC_A>(b, p, sh);
        barrier(3);
        for (int t = pf_fresh_uniform(g); t < GemmShape<EPI_O>::NRT * PT; t += G) pf_gemm<EPI_O>(b, t, sh);
        barrier(4);
        for (int p = pf_fresh_uniform(g); p < a.P; p += G) pf_digits<kFH, SRC_X>(b, p, sh);
        barrier(5);
        for (int t = pf_fresh_uniform(g); t < GemmShape<EPI_GU>::NRT * PT; t += G) pf_gemm<EPI_GU>(b, t, sh);
        barrier(6);
        for (int p = pf_fresh_uniform(g); p < a.P; p += G) pf_digits<kFI, SRC_M>(b, p, sh);
        barrier(7);
        for (int t = pf_fresh_uniform(g); t < GemmShape<EPI_DOWN>::NRT * PT; t += G) pf_gemm<EPI_DOWN>(b, t, sh);
        barrier(8);
    }
}

__global__ void pf_sync_reset_kernel(PfSync* sy) {
    sy->count = 0u;
    sy->abort = 0u;
    for (int x = 0; x < kPfXcd; ++x) {
        sy->xcd[x].arrived = 0u;
        sy->xcd[x].released = 0u;
    }
}

__global__ void pf_sync_status_kernel(const PfSync* sy, uint32_t* out) { *out = sy->abort; }

}  // namespace

size_t prefill_workspace_bytes(int max_tokens) {
    if (max_tokens < 1) return 0;
    const size_t Pp = (size_t)(max_tokens + kTileP - 1) / kTileP * kTileP;
    return pf_layout(Pp).total;
}

// Positions one chunk holds in `bytes` of workspace (a multiple of kTileP), 0 if none.
int prefill_capacity(size_t bytes) {
    size_t Pp = bytes / kPfPerPos / kTileP * kTileP;
    while (Pp >= (size_t)kTileP && pf_layout(Pp).total > bytes) Pp -= kTileP;
    return (int)std::min(Pp, (size_t)1 << 20);
}

// The chunk kernel's grid: one workgroup per compute unit (its barriers need every workgroup
// resident; checked with the occupancy calculator).
static int prefill_grid(int* grid) {
    static thread_local int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(MQ_ERR_HIP, "hipGetDevice failed");
    if (cached[dev] == 0) {
        int ncu = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&pf_chunk_kernel),
                                                         kFThreads, 0) != hipSuccess)
            return set_error(MQ_ERR_HIP, "occupancy query failed");
        if (ncu < kPfXcd || ncu % kPfXcd != 0 || per_cu < 1 || !xcd_placement_ok())
            return set_error(MQ_ERR_UNSUPPORTED, "the prefill kernel needs its workgroups dealt round-robin over "
                             "8 XCDs (%d compute units)", ncu);
        cached[dev] = ncu;
    }
    *grid = cached[dev];
    return MQ_OK;
}

int launch_prefill(const mq_decode_args& d, const int* tokens, int n_tokens, void* ws, size_t ws_bytes,
                   hipStream_t stream) {
    const int cap = prefill_capacity(ws_bytes);
    if (cap < kTileP) return set_error(MQ_ERR_INVALID_ARGUMENT, "prefill workspace of %zu bytes holds no chunk", ws_bytes);
    int grid = 0;
    int st = prefill_grid(&grid);
    if (st != MQ_OK) return st;
    PfArgs a{};
    a.embed = static_cast<const uint16_t*>(d.embed_weight);
    a.lw = d.layer_weights;
    a.sp = d.scales;
    a.cos_t = static_cast<const uint16_t*>(d.cos_table);
    a.sin_t = static_cast<const uint16_t*>(d.sin_table);
    a.kc = static_cast<uint16_t*>(d.k_cache);
    a.vc = static_cast<uint16_t*>(d.v_cache);
    a.S = d.max_seq_len;
    a.L = d.num_layers;
    a.attn_scale = d.attn_scale;
    a.spin_limit = d.spin_limit ? d.spin_limit : (1u << 21);
    a.ws = static_cast<uint8_t*>(ws);
    a.trace = static_cast<uint64_t*>(d.trace);
    a.Pp = cap;
    const PfLayout L = pf_layout((size_t)cap);
    PfSync* sy = reinterpret_cast<PfSync*>(a.ws + L.sync);
    for (int c0 = 0; c0 < n_tokens; c0 += cap) {
        a.P = std::min(cap, n_tokens - c0);
        a.pos0 = d.position + c0;
        const hipError_t e = hipMemcpyAsync(a.ws + L.tok, tokens + c0, (size_t)a.P * sizeof(int),
                                            hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return set_error(MQ_ERR_HIP, "hipMemcpyAsync(prefill tokens): %s", hipGetErrorString(e));
        // a fill kernel, not a memset, so that the launch sequence can be captured in a graph
        pf_sync_reset_kernel<<<1, 1, 0, stream>>>(sy);
        void* args[] = {&a};
        const hipError_t le = launch_resident(reinterpret_cast<const void*>(&pf_chunk_kernel), dim3(grid),
                                              dim3(kFThreads), args, stream);
        if (le != hipSuccess) return set_error(MQ_ERR_HIP, "launch(prefill): %s", hipGetErrorString(le));
        st = check_launch("prefill");
        if (st != MQ_OK) return st;
    }
    return MQ_OK;
}

int prefill_check(void* ws, size_t ws_bytes, hipStream_t stream) {
    const int cap = prefill_capacity(ws_bytes);
    if (cap < kTileP) return set_error(MQ_ERR_INVALID_ARGUMENT, "prefill workspace of %zu bytes holds no chunk", ws_bytes);
    uint32_t* flag = nullptr;
    if (hipHostMalloc(reinterpret_cast<void**>(&flag), sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
        return set_error(MQ_ERR_HIP, "hipHostMalloc failed");
    *flag = 0u;
    const PfLayout L = pf_layout((size_t)cap);
    pf_sync_status_kernel<<<1, 1, 0, stream>>>(reinterpret_cast<const PfSync*>(static_cast<uint8_t*>(ws) + L.sync), flag);
    int st = check_launch("prefill check");
    if (st == MQ_OK && hipStreamSynchronize(stream) != hipSuccess) st = set_error(MQ_ERR_HIP, "hipStreamSynchronize failed");
    const uint32_t v = *flag;
    (void)hipHostFree(flag);
    if (st != MQ_OK) return st;
    return v ? set_error(MQ_ERR_TIMEOUT, "a grid barrier of the prefill expired (were all compute units free?)") : MQ_OK;
}

}  // namespace mq
