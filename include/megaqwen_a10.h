/*
 * megaqwen_a10.h — C ABI of the MI355X (gfx950) batch-1 decode library.
 *
 * Plain C: pointers, sizes and status codes; no torch or HIP C++ types.
 * Every device pointer is a HIP device allocation on the current device.
 * Weight matrices are row-major [out_features, in_features] (the HF layout),
 * int8 for the quantized path and bf16 (raw uint16 bits) for the bf16 path.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   launch_a10_int8_decode   a10_int8_decode_kernel.cu:821-842 (declared again at bench_int8.py:97-117)
 *   launch_a10_decode        a10_decode_kernel.cu:761-780       (declared again at a10_decode.py:66-85)
 *   LayerWeights             config.cuh:45-57, bench_int8.py:73-85
 *   ScalePointers            config.cuh:59-67, bench_int8.py:87-95
 *   mq_int8_gemv             int8_decoder.py:100-115 (int8_gemv: y[j] = scale[j] * sum_i x[i] * w[j,i])
 *   mq_quantize_per_channel_bf16   bench_int8.py:19-24 (quantize_per_channel)
 */
#ifndef MEGAQWEN_A10_H
#define MEGAQWEN_A10_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same opaque handle type as HIP's own hip_runtime_api.h typedef. */
typedef struct ihipStream_t* hipStream_t;

/* Status codes returned by every mq_* entry point. */
enum {
    MQ_OK = 0,
    MQ_ERR_INVALID_ARGUMENT = 1, /* bad pointer, shape, token id, position ... (nothing launched) */
    MQ_ERR_UNSUPPORTED = 2,      /* model dims / device not supported by a compiled kernel        */
    MQ_ERR_HIP = 3,              /* a HIP runtime call failed                                      */
    MQ_ERR_TIMEOUT = 4,          /* a kernel's bounded wait expired; the workspace must be re-initialised */
    MQ_ERR_OUT_OF_MEMORY = 5
};

/* 11 pointers per layer, field order fixed by config.cuh:45-57 (sizeof == 88). */
typedef struct LayerWeights {
    const void* input_layernorm_weight;     /* bf16 [H]                         */
    const void* q_proj_weight;              /* int8|bf16 [NQ*D, H]             */
    const void* k_proj_weight;              /* int8|bf16 [NKV*D, H]            */
    const void* v_proj_weight;              /* int8|bf16 [NKV*D, H]            */
    const void* q_norm_weight;              /* bf16 [D]                         */
    const void* k_norm_weight;              /* bf16 [D]                         */
    const void* o_proj_weight;              /* int8|bf16 [H, NQ*D]             */
    const void* post_attn_layernorm_weight; /* bf16 [H]                         */
    const void* gate_proj_weight;           /* int8|bf16 [I, H]                */
    const void* up_proj_weight;             /* int8|bf16 [I, H]                */
    const void* down_proj_weight;           /* int8|bf16 [H, I]                */
} LayerWeights;

/* 7 per-output-channel fp32 scale vectors per layer, config.cuh:59-67 (sizeof == 56). */
typedef struct ScalePointers {
    float* q_scale;
    float* k_scale;
    float* v_scale;
    float* o_scale;
    float* gate_scale;
    float* up_scale;
    float* down_scale;
} ScalePointers;

/* Model dimensions. A NULL dims pointer means the Qwen3-0.6B shape
 * (H=1024, I=3072, 16 Q heads, 8 KV heads, head_dim 128, vocab 151936).
 * Compiled kernels exist for (H, I) = (1024, 3072) and (2048, 6144) with
 * 16/8 heads of 128; vocab_size is free (>= 1). */
typedef struct mq_model_dims {
    int hidden_size;
    int intermediate_size;
    int num_q_heads;
    int num_kv_heads;
    int head_dim;
    int vocab_size;
} mq_model_dims;

/* Arguments of one decode step (one token, batch 1). */
typedef struct mq_decode_args {
    int input_token_id;               /* 0 <= id < vocab_size                               */
    int* output_token_id;             /* device int32[1]: greedy argmax (lowest index on ties) */
    const void* embed_weight;         /* bf16 [V, H]                                         */
    const LayerWeights* layer_weights;/* DEVICE array [num_layers]                           */
    const ScalePointers* scales;      /* DEVICE array [num_layers]; NULL on the bf16 path    */
    const void* final_norm_weight;    /* bf16 [H]                                            */
    const void* lm_head_weight;       /* int8|bf16 [V, H]                                    */
    const float* lm_head_scale;       /* fp32 [V]; NULL on the bf16 path                     */
    const void* cos_table;            /* bf16 [max_seq_len, D]                               */
    const void* sin_table;            /* bf16 [max_seq_len, D]                               */
    void* k_cache;                    /* bf16 [num_layers, NKV, max_seq_len, D]              */
    void* v_cache;                    /* bf16 [num_layers, NKV, max_seq_len, D]              */
    /* Optional per-stage outputs (may be NULL). After a step they hold the
     * last layer's values, as the reference's scratch buffers do:
     * hidden bf16[H], activations fp32[H] (post-attn RMSNorm output),
     * residual fp32[H] (post-attn residual), q fp32[NQ*D] and k fp32[NKV*D]
     * after QK-norm+RoPE, v fp32[NKV*D], attn_out fp32[NQ*D],
     * mlp_intermediate fp32[I], normalized fp32[H] (final RMSNorm output),
     * block_max_vals fp32[>=256] / block_max_idxs int32[>=256] (per-workgroup LM-head maxima). */
    void* hidden_buffer;
    void* g_activations;
    void* g_residual;
    void* g_q;
    void* g_k;
    void* g_v;
    void* g_attn_out;
    void* g_mlp_intermediate;
    void* g_normalized;
    void* block_max_vals;
    void* block_max_idxs;
    int num_layers;
    int position;                     /* 0 <= position < max_seq_len                         */
    int cache_len;                    /* must equal position + 1                              */
    int max_seq_len;
    float attn_scale;                 /* 1/sqrt(head_dim) in the reference                    */
    const mq_model_dims* dims;        /* NULL: Qwen3-0.6B                                     */
    void* workspace;                  /* device memory of mq_decode_workspace_bytes(dims)     */
    size_t workspace_bytes;
    unsigned int spin_limit;          /* bound on each in-kernel wait (polls); 0 = default    */
    /* Optional hipEvent_t pair, recorded at the kernel's own start and end
     * (exact kernel time). Steps are dispatched with hipExtLaunchKernel. All
     * 256 workgroups must be co-resident, which the library checks once per
     * device from the kernel's occupancy; if other work holds compute units when
     * a step starts, its bounded waits end it with MQ_ERR_TIMEOUT. */
    void* timing_start;
    void* timing_stop;
    /* Optional per-stage timeline: uint64 [(num_layers + 1) * 10 * 256], written
     * when non-NULL with the 100 MHz real-time counter. Entry
     * [(l * 10 + p) * 256 + g] is when workgroup g passed point p of layer l.
     * Single-level kernel: p = 0/1 QKV input ready/output written, 2/3
     * attention (workgroups 0-7), 4/5 O projection, 6/7 gate/up, 8/9 down.
     * XCD-aware kernel: p = 0/1 QKV input ready/output written, 2/3 attention
     * inputs ready/output in LDS (every workgroup), 4 O partial written,
     * 5 residual rows gathered, 6 gate/up output written, 7 SwiGLU outputs
     * gathered, 8 down partial written, 9 hidden rows gathered.
     * Layer num_layers holds p = 0 final-norm input ready, p = 1 LM head done,
     * and [(L*10 + 2) * 256] the token publication.
     * mq_int8_prefill: uint64 [num_layers * 18 * G], G = the prefill grid
     * (one workgroup per compute unit, 256 on MI355X); entry
     * [(l * 18 + 2 k + e) * G + g] is when workgroup g finished phase k of
     * layer l (e = 0) or passed the grid barrier after it (e = 1); phases
     * 0 input digit planes, 1 QKV, 2 attention, 3 attention-output digit
     * planes, 4 O, 5 post-attention digit planes, 6 gate/up, 7 SwiGLU digit
     * planes, 8 down; the last layer writes points 0-2 only. A prefill of several chunks leaves the last
     * chunk's timeline. */
    void* trace;
    /* Attention split (XCD-aware kernel): from cache_len >= attn_split_min on,
     * each of the 32 workgroups sharing a KV head attends over 1/32 of the
     * positions and the softmax partials are merged (log-sum-exp), which lifts
     * the context limit from 1024 to 32768 positions. 0 = library default
     * (48), > 1025 is taken as 1025, < 0 = never split. The single-level
     * kernel never splits (cache_len <= 1024). */
    int attn_split_min;
    /* Sampling (no counterpart in the reference, whose generate() accepts a
     * temperature and ignores it, a10_decode.py:358): 0 = greedy argmax; > 0 =
     * the token is drawn from softmax(logits / temperature) by the Gumbel-max
     * rule, argmax over rows of logit / temperature + g, with the noise g keyed
     * by (seed, position, vocabulary row): a given seed gives the same tokens
     * one launch per step and in mq_int8_decode_generate. */
    float temperature;
    unsigned long long seed;
} mq_decode_args;

/* ---- device-side generation loop (no counterpart in the reference) --------
 * Runs n_forced + n_generate - 1 decode steps in ONE launch, each step handing
 * its token to the next on the device (a10_decode.py:358-393 and
 * bench_int8.py:218 launch one step per token and read each token back).
 * Step i, at position args->position + i, takes prompt_tokens[i] for
 * i < n_forced (the prefill) and the previous step's output after that;
 * output_tokens[j] receives the output of step n_forced - 1 + j (the last
 * prefill step's output is the first generated token, the convention of
 * verify_correctness_a10.py:323-339) and args->output_token_id the last one.
 * args->input_token_id must equal prompt_tokens[0] and cache_len position + 1.
 * A loop over the one-step entry point of the same weight format gives the
 * same tokens and KV cache, sampled tokens included. */
typedef struct mq_generate_args {
    const int* prompt_tokens;         /* HOST int32[n_forced], each in [0, vocab_size)        */
    int n_forced;                     /* >= 1                                                 */
    int n_generate;                   /* >= 1                                                 */
    int* output_tokens;               /* device or pinned host int32[n_generate]              */
} mq_generate_args;

/* ---- batched INT8 decode (no counterpart in the reference) ---------------
 * B <= MQ_MAX_BATCH independent sequences share one pass over the weights per
 * step; each has its own KV cache slice and position. The semantics are B
 * copies of mq_int8_decode_step's; the matrix products run on the int8 matrix
 * cores with each activation vector split into four int8 digits (per-sequence
 * power-of-two scale, 28 significant bits) and the RMSNorm scale applied after
 * the product, so projections differ from the single-sequence path by ~1e-8
 * relative and an occasional bf16 rounding (K/V rows, hidden state) lands one
 * ulp apart: agreement is within bf16 tolerance, not bitwise. Only the
 * Qwen3-1.7B layer shapes (hidden 2048, intermediate 6144, 16 / 8 heads of
 * 128) are compiled. */
#define MQ_MAX_BATCH 16
typedef struct mq_batch_args {
    int batch;                        /* 1..MQ_MAX_BATCH; the same for every step on a workspace */
    int input_token_ids[MQ_MAX_BATCH];/* per sequence, 0 <= id < vocab_size                   */
    int positions[MQ_MAX_BATCH];      /* per sequence, 0 <= position < min(max_seq_len, 1024) */
    int* output_token_ids;            /* device int32[batch]: greedy argmax per sequence        */
    const void* embed_weight;         /* bf16 [V, H]                                           */
    const LayerWeights* layer_weights;/* DEVICE array [num_layers] (int8 projections)          */
    const ScalePointers* scales;      /* DEVICE array [num_layers]                              */
    const void* final_norm_weight;    /* bf16 [H]                                              */
    const void* lm_head_weight;       /* int8 [V, H]                                           */
    const float* lm_head_scale;       /* fp32 [V]                                              */
    const void* cos_table;            /* bf16 [max_seq_len, D]                                 */
    const void* sin_table;            /* bf16 [max_seq_len, D]                                 */
    void* k_cache;                    /* bf16 [batch, num_layers, NKV, max_seq_len, D]         */
    void* v_cache;                    /* bf16 [batch, num_layers, NKV, max_seq_len, D]         */
    int num_layers;
    int max_seq_len;
    float attn_scale;
    const mq_model_dims* dims;        /* NULL: Qwen3-1.7B                                      */
    void* workspace;                  /* device memory of mq_batch_workspace_bytes(dims)       */
    size_t workspace_bytes;
    unsigned int spin_limit;          /* bound on each in-kernel wait (polls); 0 = default     */
    void* timing_start;               /* optional hipEvent_t pair, as in mq_decode_args        */
    void* timing_stop;
    /* Optional per-sequence values of the last layer (NULL: not written):
     * hidden_out bf16 [batch, H] (layer output), qkv_out fp32 [batch, NKV, 512]
     * (each KV head's two query heads, key and value projections before QK-norm),
     * attn_out fp32 [batch, NQ * D], act_out fp32 [batch, H] (post-attention
     * residual), mlp_out fp32 [batch, I] (SwiGLU output). */
    void* hidden_out;
    void* qkv_out;
    void* attn_out;
    void* act_out;
    void* mlp_out;
    /* Optional timeline, uint64 [(num_layers + 1) * 10 * 256] of the 100 MHz
     * real-time counter: [(l * 10 + p) * 256 + g] is when workgroup g passed
     * point p of layer l: 0 layer start, 1 QKV partials written, 2 QKV rows
     * reduced, 3 attention done, 4 O partials written, 5 O rows reduced, 6
     * gate/up partials written, 7 SwiGLU outputs written, 8 down partials
     * written, 9 layer done; layer num_layers: 0 LM head start, 1 LM products done. */
    void* trace;
} mq_batch_args;

/* ---- library information ------------------------------------------------ */
int mq_abi_version(void);
/* Message of the last failing mq_* call on this host thread ("" if none). */
const char* mq_last_error(void);

/* ---- decode (persistent workgroup pipeline) ----------------------------- */
size_t mq_decode_workspace_bytes(const mq_model_dims* dims);
/* Zero the workspace and reset its step counter. Required once after
 * allocation and again after any MQ_ERR_TIMEOUT. */
int mq_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream);
/* One INT8 weight-only decode step (all linears and the LM head int8 with
 * per-row fp32 scales). Replaces launch_a10_int8_decode. Asynchronous on
 * `stream`; the token lands in *output_token_id. */
int mq_int8_decode_step(const mq_decode_args* args, hipStream_t stream);
/* Same with bf16 weights (scales and lm_head_scale ignored). Replaces launch_a10_decode. */
int mq_bf16_decode_step(const mq_decode_args* args, hipStream_t stream);
/* Same with FP8 E4M3 weights: every linear and the LM head as codes from
 * mq_quantize_fp8_rows_bf16 (uint8 [out, in]) with their per-row fp32 scales,
 * in the INT8 layout and packing order. No counterpart in the reference (INT8
 * and BF16 only). Hidden 1024 / intermediate 3072, on the XCD-aware kernel
 * (MQ_ERR_UNSUPPORTED for other dims or when its workgroup placement does not
 * hold). Every stored intermediate is the correctly rounded value of the
 * dequantized weights' expression, as for INT8. */
int mq_fp8_decode_step(const mq_decode_args* args, hipStream_t stream);
/* Same with INT4 weights per group of 128 inputs for the seven layer
 * projections: codes from mq_quantize_int4_groups_bf16 (two's complement
 * nibbles, uint8 [out, in / 2], the low nibble the even element) with their
 * fp32 group scales [out, in / 128] in place of the per-row scales (same
 * packing order); the LM head stays INT8 per row (lm_head_weight,
 * lm_head_scale). No counterpart in the reference. Hidden 1024 / intermediate
 * 3072 up to 10240 cached positions, on the async-wave kernel (MQ_ERR_UNSUPPORTED
 * otherwise): each group's exact digit-plane sum is scaled by its group scale
 * in fp64, so every stored intermediate is the correctly rounded value of the
 * dequantized weights' expression. */
int mq_int4_decode_step(const mq_decode_args* args, hipStream_t stream);
/* Allocation-free variant of mq_int8_decode_step. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * args->workspace is ignored: the step uses a library-held static device array
 * of 4 MiB per device (every compiled dims fits: at most 1.8 MB), cleared by a
 * fill kernel on `stream` at the start of every call, so no state carries over
 * from one call to the next. The call allocates nothing (no hipMalloc, no
 * library allocation). Every call on a device shares that device's array:
 * calls that overlap on one device (other streams, other threads) race. */
int mq_int8_decode_step_noalloc(const mq_decode_args* args, hipStream_t stream);
/* Several steps per launch (see mq_generate_args): INT8, bf16 and FP8 weights.
 * The async-wave kernel runs the launch within its range (INT8 Qwen3-0.6B shape,
 * position + steps <= 6144; 10240 when forced), the XCD-aware kernel's multi-step form otherwise
 * (every compiled shape and format, up to 32768 positions with split attention);
 * MQ_ERR_UNSUPPORTED on the single-level kernel. */
int mq_int8_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream);
int mq_bf16_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream);
int mq_fp8_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream);
/* INT4 layer weights (see mq_int4_decode_step): the async-wave kernel only. */
int mq_int4_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream);
/* Prompt-batched prefill. The reference prefills a prompt one decode step per
 * token (a10_decode.py:367-368, verify_correctness_a10.py:326-328, each step
 * a10_int8_decode_kernel.cu:821-842); this writes the same K/V cache rows with
 * each layer's weights read once for the whole prompt. tokens: HOST array of
 * n_tokens ids (validated before anything is launched), prefilled at positions
 * args->position + i (0 <= i < n_tokens <= max_seq_len - position); no logits
 * and no token are produced: the decode step of the next token (the prompt's
 * last, as in the reference's loop) gives the first generated token.
 * args->input_token_id, output_token_id, cache_len and workspace are not used.
 * INT8 Qwen3-0.6B shape only (MQ_ERR_UNSUPPORTED otherwise). workspace: device
 * memory of mq_prefill_workspace_bytes(dims, m) bytes, 16-byte aligned; a
 * longer prompt runs in chunks of m positions (m rounded up to a multiple of
 * 32), one persistent launch per chunk (one workgroup per compute unit, grid
 * barriers between its phases). Asynchronous on `stream`. */
size_t mq_prefill_workspace_bytes(const mq_model_dims* dims, int max_tokens);
int mq_int8_prefill(const mq_decode_args* args, const int* tokens, int n_tokens, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);
/* After mq_int8_prefill: synchronises `stream`; MQ_ERR_TIMEOUT if the prefill's
 * grid-wide waits expired (its launch needs every compute unit; args->spin_limit
 * bounds each wait), else MQ_OK. The cache rows are then unusable: prefill again. */
int mq_prefill_check(void* workspace, size_t workspace_bytes, hipStream_t stream);
/* Host-side wait for a token the kernel stores into host memory (pinned, e.g.
 * hipHostMalloc): spins until *token differs from `sentinel`, which the
 * caller wrote before the launch. MQ_OK, or MQ_ERR_TIMEOUT after timeout_us
 * microseconds (then synchronise the stream and call mq_decode_check). The
 * kernel stores the token last, so this returns as the step ends, without the
 * stream synchronisation's wake-up. No counterpart in the reference, which
 * copies the token back with .item(). */
int mq_wait_host_token(const volatile int* token, int sentinel, unsigned int timeout_us);
/* After a completed step: MQ_ERR_TIMEOUT if a bounded wait of that step expired, else MQ_OK.
 * Synchronises `stream`. */
int mq_decode_check(void* workspace, hipStream_t stream);

/* Batched decode: workspace size for any batch up to MQ_MAX_BATCH (0 for
 * unsupported dims), and one step of `batch` sequences (mq_batch_args).
 * Initialise the workspace with mq_workspace_init; a workspace serves one
 * batch size (re-initialise it to change the size). Needs the XCD-aware
 * workgroup placement (mq_decode_variant() == 2). */
size_t mq_batch_workspace_bytes(const mq_model_dims* dims);
int mq_int8_decode_batch_step(const mq_batch_args* args, hipStream_t stream);

/* Kernel variant for all following steps in this process: 0 = automatic
 * (default: the async-wave kernel for INT8 steps of the Qwen3-0.6B shape up to
 * 6144 cached positions, otherwise the XCD-aware kernel, when the workgroups of
 * each residue class g mod 8 share one XCD and the 8 classes cover the 8 XCDs,
 * checked once per device), 1 = single-level exchange kernel, 2 = XCD-aware,
 * 3 = async-wave (INT8 Qwen3-0.6B shape, cache_len <= 10240 only). */
int mq_decode_set_variant(int variant);
/* Launch mode of the persistent kernels (decode steps, generation, batched
 * steps, prefill chunks) for all following calls in this process. 0 (default):
 * plain launches; every workgroup must be resident at once, which is checked
 * with the occupancy calculator but not guaranteed when other work holds compute
 * units (the step's bounded waits then end it with MQ_ERR_TIMEOUT). 1:
 * cooperative launches, which the runtime starts only when all workgroups can
 * be resident (about 10 us more per launch; timing events are recorded around
 * the launch instead of by the dispatch). No counterpart in the reference,
 * whose launchers are cooperative. */
int mq_decode_set_cooperative(int enable);
/* The variant a short-context step (cache_len 1) with these dims would use now
 * (1, 2 or 3), or -status. */
int mq_decode_variant(const mq_model_dims* dims, int int8);
/* The same for a step that attends over `cache_len` cached positions (the choice can depend
 * on the context length); minus MQ_ERR_INVALID_ARGUMENT for cache_len < 1. No counterpart in the
 * reference. */
int mq_decode_variant_at(const mq_model_dims* dims, int int8, int cache_len);

/* ---- reference-signature entry points (drop-in for the CUDA launchers) --- */
/* a10_int8_decode_kernel.cu:821-842. Uses a library-owned workspace per
 * device (allocated on first use): calls that overlap on one device race.
 * The block_max_* buffers need >= 256 entries. Errors are reported through
 * mq_last_error() since the reference signature returns void. A step that
 * fails inside the kernel (expired bounded wait) stores token -1; the next
 * call on that device then re-initialises the workspace before launching and
 * reports the earlier failure through mq_last_error() (the reference's caller
 * reads every token back, bench_int8.py:218, so the failure is known by then).
 * The vocabulary and layer shapes are those of mq_reference_set_dims (default
 * Qwen3-0.6B); the embedding, LM head, caches and tables are checked on the host
 * against the device allocations that hold them, where the runtime can tell. */
void launch_a10_int8_decode(
    int input_token_id, int* output_token_id,
    const void* embed_weight, const LayerWeights* layer_weights,
    const void* final_norm_weight, const void* lm_head_weight, const float* lm_head_scale,
    const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache,
    void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, void* block_max_vals, void* block_max_idxs,
    int num_layers, int position, int cache_len, int max_seq_len, float attn_scale,
    const ScalePointers* scales, hipStream_t stream);

/* a10_decode_kernel.cu:761-780 (bf16 weights, no scales). */
void launch_a10_decode(
    int input_token_id, int* output_token_id,
    const void* embed_weight, const LayerWeights* layer_weights,
    const void* final_norm_weight, const void* lm_head_weight,
    const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache,
    void* hidden_buffer, void* g_activations, void* g_residual,
    void* g_q, void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate,
    void* g_normalized, void* block_max_vals, void* block_max_idxs,
    int num_layers, int position, int cache_len, int max_seq_len, float attn_scale,
    hipStream_t stream);

/* Bound on each in-kernel wait (polls) of the steps the two launchers above
 * run; 0 = library default. No counterpart in the reference (for tests that
 * force the failure path from the host). */
void mq_reference_set_spin_limit(unsigned int polls);
/* Model dims the two launchers above assume from now on (NULL = Qwen3-0.6B,
 * vocab 151936). The reference compiles its dims in (config.cuh:15-43); its
 * launchers' signature carries none, so another model (e.g. a smaller
 * vocabulary) must be declared here first. Returns a status code. */
int mq_reference_set_dims(const mq_model_dims* dims);

/* ---- standalone kernels ------------------------------------------------- */
/* int8_decoder.py:100-115: y[j] = scale[j] * sum_k x[k] * w[j,k].
 * x fp32 [K], w int8 [M,K] row-major (16-byte aligned rows: K % 16 == 0),
 * scale fp32 [M], y fp32 [M]. 1 <= K <= 16384. */
int mq_int8_gemv(const float* x, const int8_t* w, const float* scale, float* y,
                 int M, int K, hipStream_t stream);
/* Steady-state form of mq_int8_gemv (no counterpart in the reference, whose
 * microbenchmark int8_decoder.py:351-434 times isolated calls): one launch
 * computes `reps` matvecs, rep i against weight copy i % n_copies at
 * w + (i % n_copies) * copy_stride bytes, into y + (i % n_copies) * M. The
 * matvecs are independent, so the launch streams weights without a launch gap
 * or ramp between them; per-matvec time = launch time / reps. y fp32
 * [n_copies, M]; copy_stride a multiple of 16 and >= M * K when n_copies > 1;
 * reps * M < 2^31. reps = n_copies = 1 is mq_int8_gemv. */
int mq_int8_gemv_repeat(const float* x, const int8_t* w, int64_t copy_stride, int n_copies,
                        const float* scale, float* y, int M, int K, int reps, hipStream_t stream);

/* ---- other weight formats (no counterpart in the reference, which has INT8
 * and BF16 weights only; its one other-format figure is llama.cpp Q4_K_M,
 * README.md:19). The quantizers follow mq_quantize_per_channel_bf16's pattern:
 *   FP8 E4M3 (OCP E4M3FN: bias 7, subnormals m * 2^-9, 0x7F / 0xFF NaN, max 448),
 *     per row:   s = fp32(amax) / 448 (IEEE), floored at 1e-12;
 *                q = nearest code of fp32(w) / s, ties to the even code, |.| >= 448 -> +-448.
 *     q uint8 [M,K], scale fp32 [M].
 *   INT4 per group of 128 consecutive elements of a row:
 *                s = bf16(amax / 7) (fp32 division rounded to bf16), floored at 1e-12;
 *                q = clamp(round_half_even(fp32(w) / s), -8, 7);
 *     q uint8 [M,K/2], byte i = (q[2i] & 15) | (q[2i+1] & 15) << 4; scale fp32 [M,K/128].
 * Matvecs: y[j] = sum_k dequant(w)[j,k] * x[k], x fp32 [K] (finite), y fp32 [M];
 * FP8 accumulates in fp32, INT4 forms exact integer products of x's 55-bit
 * fixed-point digits on the int8 matrix cores and sums them in fp64; 16-byte
 * aligned x and w; K <= 16384 and K % 16 == 0 (FP8) or
 * K % 128 == 0 (INT4). The _repeat forms are the steady-state form of
 * mq_int8_gemv_repeat (reps matvecs over n_copies copies copy_stride bytes
 * apart, y [n_copies, M]). */
int mq_quantize_fp8_rows_bf16(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream);
int mq_quantize_int4_groups_bf16(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream);
int mq_fp8_gemv(const float* x, const uint8_t* w, const float* scale, float* y, int M, int K, hipStream_t stream);
int mq_int4_gemv(const float* x, const uint8_t* w, const float* scale, float* y, int M, int K, hipStream_t stream);
int mq_fp8_gemv_repeat(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies,
                       const float* scale, float* y, int M, int K, int reps, hipStream_t stream);
int mq_int4_gemv_repeat(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies,
                        const float* scale, float* y, int M, int K, int reps, hipStream_t stream);

/* bench_int8.py:19-24: per-row symmetric int8.
 *   amax = max_k |w[j,k]|               (bf16, exact)
 *   s    = bf16(amax / 127)             (bf16 division), widened to fp32, clamped to >= 1e-12
 *   q    = clamp(round_half_even(fp32(w) / s), -128, 127)
 * w bf16 [M,K] (uint16 bits), q int8 [M,K], scale fp32 [M]. */
int mq_quantize_per_channel_bf16(const void* w_bf16, int M, int K,
                                 int8_t* q, float* scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MEGAQWEN_A10_H */
