// Host-side declarations shared between the kernel translation units and the
// C-ABI layer (api.hip). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/megaqwen_a10.h"

namespace mq {

// Records a message for mq_last_error() and returns `status`.
int set_error(int status, const char* fmt, ...);
// MQ_OK, or MQ_ERR_HIP with the pending launch error recorded.
int check_launch(const char* what);

int launch_quantize(const void* w_bf16, int M, int K, int8_t* q, float* scale, hipStream_t stream);
int launch_quantize_fp8(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream);
int launch_quantize_int4(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream);
int launch_fp8_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                    int M, int K, int reps, hipStream_t stream);
int launch_int4_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale, float* y,
                     int M, int K, int reps, hipStream_t stream);
int launch_int8_gemv(const float* x, const int8_t* w, const float* scale, float* y, int M, int K,
                     hipStream_t stream);
int launch_int8_gemv_repeat(const float* x, const int8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                            float* y, int M, int K, int reps, hipStream_t stream);

// Workspace header at the start of every decode workspace (256 bytes).
struct WsHeader {
    uint32_t epoch;        // step counter; tags are derived from it (starts at 1)
    uint32_t abort_flag;   // set by a kernel whose bounded wait expired
    uint32_t done[2];      // workgroups finished with the LM head, per step parity
    uint64_t best[2];      // packed (ordered logit, ~token) maximum, per step parity
    uint32_t xsteps;       // steps run by the XCD-aware kernel (parity tags of its packed words)
    uint32_t bsteps;       // steps run by the batched kernel (parity tags of its packed words)
    uint32_t batch;        // sequences per step of the batched kernel (0 until its first step)
    uint32_t asteps;       // steps run by the async-wave kernel (parity tags of its packed words)
    uint32_t pad[52];
};
static_assert(sizeof(WsHeader) == 256, "workspace header is 256 bytes");

struct DecodeShape {
    int H, I, NQ, NKV, D, V;
    bool fp8 = false;          // one-byte weights are FP8 E4M3 codes (with per-row scales), not int8
    bool int4 = false;         // layer projections INT4 per group of 128 (the LM head INT8 per row)
};

size_t decode_workspace_bytes(const DecodeShape& s);
// Kernel variant: 0 = automatic (XCD-aware when the workgroups of each residue
// class g mod 8 share one XCD), 1 = single-level exchange kernel, 2 = XCD-aware.
int set_decode_variant(int variant);
// 1: the persistent kernels are launched cooperatively (co-residency guaranteed by the
// runtime, about 10 us more per launch); 0 (default): plain launches.
int set_cooperative_launch(int on);
int decode_variant_in_use(const DecodeShape& s, bool int8);
// the kernel a step attending over cache_len positions uses (or minus a refusal's status)
int decode_variant_for(const DecodeShape& s, bool int8, int cache_len);
// After an in-kernel placement failure: use the single-level kernel from now on.
void mark_xcd_unusable();
// Several decode steps in one launch: step i's input is tokens[i] (device memory) for
// i < n_forced and the previous step's output after that; tokens_out[i - (n_forced - 1)]
// receives the output of every step from the last forced one on.
struct GenPlan {
    const int* tokens;
    int n_forced;
    int n_steps;
    int* tokens_out;
};
// Launches one decode step (several with a plan); `int8` selects the weight format. When
// status_out is non-null the last step's token publisher also stores the abort flag there
// (0 = completed).
int launch_decode(const mq_decode_args& a, const DecodeShape& s, bool int8, hipStream_t stream,
                  uint32_t* status_out = nullptr, const GenPlan* plan = nullptr);
// Byte offset in the workspace of a multi-step launch's forced input tokens (room for
// kDecodeMaxForced of them, whichever kernel runs the launch), and the longest cache the
// async-wave kernel attends over.
constexpr int kDecodeMaxForced = 32768;
size_t decode_token_offset(const DecodeShape& s);
int decode_async_max_len();
int decode_async_split_min(int attn_split_min);
// True when the workgroups of each residue class g mod 8 run on one XCD (checked once per device).
bool xcd_placement_ok();

// Prompt-batched prefill (prefill.hip): INT8 Qwen3-0.6B shape. The workspace of a chunk of
// max_tokens positions, the positions a workspace of `bytes` holds per chunk, and the
// launches that write the K/V cache rows of tokens[0, n_tokens) (host array) at positions
// d.position + i.
size_t prefill_workspace_bytes(int max_tokens);
int prefill_capacity(size_t bytes);
int launch_prefill(const mq_decode_args& d, const int* tokens, int n_tokens, void* ws, size_t ws_bytes,
                   hipStream_t stream);
// After the prefill launches on `stream` (synchronises it): MQ_ERR_TIMEOUT if a grid barrier of the
// last chunk expired, else MQ_OK.
int prefill_check(void* ws, size_t ws_bytes, hipStream_t stream);

// Batched INT8 decode (decode_batch.hip).
size_t decode_batch_workspace_bytes(const DecodeShape& s);
int launch_decode_batch(const mq_batch_args& a, const DecodeShape& s, hipStream_t stream);

}  // namespace mq
