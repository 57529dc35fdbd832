// C-ABI entry points (include/megaqwen_a10.h): argument validation before any
// launch, status codes, per-thread error messages, the library-owned
// workspaces behind the reference-signature launchers, and workspace reset.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>

#include "internal.h"

namespace mq {

static thread_local char g_err[512] = "";

// Every public entry point starts with an empty message, so after a void
// launcher returns, an empty mq_last_error() means it was accepted.
static void clear_error() { g_err[0] = 0; }

int set_error(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
    return MQ_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int shape_of(const mq_model_dims* d, DecodeShape* s) {
    if (d == nullptr) {
        *s = DecodeShape{1024, 3072, 16, 8, 128, 151936};
        return MQ_OK;
    }
    *s = DecodeShape{d->hidden_size, d->intermediate_size, d->num_q_heads, d->num_kv_heads, d->head_dim,
                     d->vocab_size};
    if (s->NQ != 16 || s->NKV != 8 || s->D != 128)
        return set_error(MQ_ERR_UNSUPPORTED, "only 16 query heads, 8 KV heads of dim 128 are compiled (got %d/%d/%d)",
                         s->NQ, s->NKV, s->D);
    if (!((s->H == 1024 && s->I == 3072) || (s->H == 2048 && s->I == 6144)))
        return set_error(MQ_ERR_UNSUPPORTED, "no kernel for hidden %d / intermediate %d", s->H, s->I);
    if (s->V < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "vocab_size %d < 1", s->V);
    return MQ_OK;
}

__global__ void ws_init_kernel(uint64_t* ws, size_t words) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
        ws[i] = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) reinterpret_cast<WsHeader*>(ws)->epoch = 1u;
}

// Whether [p, p + need) lies inside the device allocation that holds p. A best-effort
// guard for arguments that arrive without sizes (the reference-signature launchers
// pass bare pointers): a pointer the runtime cannot place is not rejected, and a
// tensor carved out of a larger allocation is only checked against that allocation's
// end. The last few results are kept per thread, so a decode loop that passes the
// same buffers every step asks the runtime once.
static bool in_allocation(const void* p, size_t need) {
    struct Seen { const void* p; size_t need; bool ok; };
    static thread_local Seen seen[16];
    static thread_local unsigned next = 0;
    for (const Seen& e : seen)
        if (e.p == p && e.need == need) return e.ok;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    bool ok = true;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) == hipSuccess && base != nullptr)
        ok = reinterpret_cast<uintptr_t>(p) + need <= reinterpret_cast<uintptr_t>(base) + size;
    else
        (void)hipGetLastError();
    seen[next++ % 16] = Seen{p, need, ok};
    return ok;
}

static int validate_decode(const mq_decode_args* a, bool int8, DecodeShape* s) {
    if (a == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "args is NULL");
    int st = shape_of(a->dims, s);
    if (st != MQ_OK) return st;
    if (a->num_layers < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "num_layers %d < 1", a->num_layers);
    if (a->max_seq_len < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "max_seq_len %d < 1", a->max_seq_len);
    if (a->input_token_id < 0 || a->input_token_id >= s->V)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "input_token_id %d outside [0, %d)", a->input_token_id, s->V);
    if (a->position < 0 || a->position >= a->max_seq_len)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "position %d outside [0, max_seq_len=%d)", a->position, a->max_seq_len);
    if (a->cache_len != a->position + 1)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "cache_len %d != position + 1 (%d)", a->cache_len, a->position + 1);
    if (!(a->temperature >= 0.0f) || a->temperature == INFINITY)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "temperature %g is not a finite value >= 0", (double)a->temperature);
    if (!a->output_token_id || !a->embed_weight || !a->layer_weights || !a->final_norm_weight ||
        !a->lm_head_weight || !a->cos_table || !a->sin_table || !a->k_cache || !a->v_cache)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
    if (int8 && (!a->scales || !a->lm_head_scale))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "int8 decode needs scales and lm_head_scale");
    if (!aligned16(a->lm_head_weight) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "lm_head_weight and the KV caches must be 16-byte aligned");
    if (!a->workspace || a->workspace_bytes < decode_workspace_bytes(*s))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace of %zu bytes needed, %zu given",
                         decode_workspace_bytes(*s), a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned16(a->workspace)) return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    const size_t HV = (size_t)s->H * (size_t)s->V;
    const size_t cache = (size_t)a->num_layers * s->NKV * a->max_seq_len * s->D * 2;
    const size_t table = (size_t)a->max_seq_len * s->D * 2;
    if (!in_allocation(a->embed_weight, HV * 2) || !in_allocation(a->lm_head_weight, HV * (int8 ? 1 : 2)) ||
        (int8 && !in_allocation(a->lm_head_scale, (size_t)s->V * 4)))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "embed_weight / lm_head_weight hold fewer than vocab_size = %d rows "
                         "of %d (set the model dims; the reference-signature launchers assume Qwen3-0.6B unless "
                         "mq_reference_set_dims says otherwise)", s->V, s->H);
    if (!in_allocation(a->k_cache, cache) || !in_allocation(a->v_cache, cache))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the KV caches hold fewer than num_layers x %d x max_seq_len x %d "
                         "bf16 values", s->NKV, s->D);
    if (!in_allocation(a->cos_table, table) || !in_allocation(a->sin_table, table))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the RoPE tables hold fewer than max_seq_len rows of %d", s->D);
    return MQ_OK;
}

// Library-owned workspace per device for the reference-signature launchers,
// with a pinned host word into which every step's token publisher stores the
// step's abort flag (0 = completed). The reference's caller reads each token
// back (bench_int8.py:218), so by the next call the word holds the previous
// step's outcome; a failed step is then reported through mq_last_error(), its
// workspace re-initialised (and the single-level kernel selected if a
// workgroup ran on an unexpected XCD) before the new step is launched.
struct DeviceWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    volatile uint32_t* status = nullptr;
};
static std::mutex g_ws_mu;
static DeviceWorkspace g_ws[64];
static std::atomic<unsigned int> g_ref_spin{0};   // spin limit of the reference-signature launchers (0 = default)
// model dims of the reference-signature launchers (their signature has none); unset = Qwen3-0.6B
static std::mutex g_ref_mu;
static bool g_ref_has_dims = false;
static mq_model_dims g_ref_dims;

// The reference launchers' dims for this call (copied into *store; NULL when unset).
static const mq_model_dims* reference_dims(mq_model_dims* store) {
    std::lock_guard<std::mutex> lk(g_ref_mu);
    if (!g_ref_has_dims) return nullptr;
    *store = g_ref_dims;
    return store;
}

static int default_workspace(const mq_model_dims* dims, hipStream_t stream, void** out, size_t* bytes,
                             uint32_t** status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(MQ_ERR_HIP, "hipGetDevice failed");
    DecodeShape s;
    int st0 = shape_of(dims, &s);
    if (st0 != MQ_OK) return st0;
    const size_t need = decode_workspace_bytes(s);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    DeviceWorkspace& w = g_ws[dev];
    if (w.ptr != nullptr && w.bytes < need) {
        // larger dims than before: a new workspace (hipFree waits for the steps using the old one)
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
    }
    if (w.ptr == nullptr) {
        if (w.status == nullptr) {
            void* st_word = nullptr;
            if (hipHostMalloc(&st_word, sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
                return set_error(MQ_ERR_OUT_OF_MEMORY, "hipHostMalloc of the step status word failed");
            w.status = static_cast<volatile uint32_t*>(st_word);
        }
        if (hipMalloc(&w.ptr, need) != hipSuccess) {
            w.ptr = nullptr;
            return set_error(MQ_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) for the decode workspace failed", need);
        }
        w.bytes = need;
        *w.status = 0u;
        hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint64_t*>(w.ptr),
                           need / 8);
        int st = check_launch("ws_init_kernel");
        if (st != MQ_OK) return st;
    } else if (*w.status != 0u) {
        // the previous step on this workspace failed: recover before this one
        const uint32_t flag = *w.status;
        *w.status = 0u;
        if (flag == 2u) mark_xcd_unusable();
        hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint64_t*>(w.ptr),
                           w.bytes / 8);
        int st = check_launch("ws_init_kernel");
        if (st != MQ_OK) return st;
        set_error(MQ_ERR_TIMEOUT, "the previous step failed (%s; its token is -1); the workspace was re-initialised "
                                  "and this step launched",
                  flag == 2u ? "a workgroup ran on an unexpected XCD, the single-level kernel is selected"
                             : "a bounded wait in the decode kernel expired");
    }
    *out = w.ptr;
    *bytes = w.bytes;
    *status = const_cast<uint32_t*>(w.status);
    return MQ_OK;
}

// ---- allocation-free decode step --------------------------------------------------------
// A file-scope device array serves as the workspace of mq_int8_decode_step_noalloc,
// one copy per device. Host code uses the per-device address from
// hipGetSymbolAddress (taken once per device on the first call there), never the
// array's name, which on the host is only a stand-in for the symbol.
constexpr size_t kStaticScratchBytes = 4u << 20;   // 4 MiB per device
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static int static_scratch(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(MQ_ERR_HIP, "hipGetDevice failed");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return set_error(MQ_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MQ_OK;
}

// One step of a reference-signature launcher: validation and launch with the
// library-owned status word. A message left by default_workspace() (the
// previous step's failure) stays visible unless this step's own validation or
// launch fails.
static void reference_step(const mq_decode_args* a, bool int8, uint32_t* status, hipStream_t stream) {
    char pending[sizeof(g_err)];
    memcpy(pending, g_err, sizeof(g_err));
    DecodeShape s;
    int st = validate_decode(a, int8, &s);
    if (st == MQ_OK) st = launch_decode(*a, s, int8, stream, status);
    if (st == MQ_OK) memcpy(g_err, pending, sizeof(g_err));
}

}  // namespace mq

using namespace mq;

extern "C" {

int mq_abi_version(void) { return 3; }

const char* mq_last_error(void) { return g_err; }

size_t mq_decode_workspace_bytes(const mq_model_dims* dims) {
    clear_error();
    DecodeShape s;
    if (shape_of(dims, &s) != MQ_OK) return 0;
    return decode_workspace_bytes(s);
}

int mq_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
    clear_error();
    if (!workspace || workspace_bytes < sizeof(WsHeader) || (workspace_bytes % 8) != 0 || !aligned16(workspace))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace must be >= %zu bytes, a multiple of 8, 16-byte aligned",
                         sizeof(WsHeader));
    hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint64_t*>(workspace),
                       workspace_bytes / 8);
    return check_launch("ws_init_kernel");
}

int mq_int8_decode_step(const mq_decode_args* args, hipStream_t stream) {
    clear_error();
    DecodeShape s;
    int st = validate_decode(args, true, &s);
    if (st != MQ_OK) return st;
    return launch_decode(*args, s, true, stream);
}

int mq_fp8_decode_step(const mq_decode_args* args, hipStream_t stream) {
    clear_error();
    DecodeShape s;
    int st = validate_decode(args, true, &s);
    if (st != MQ_OK) return st;
    s.fp8 = true;
    return launch_decode(*args, s, true, stream);
}

int mq_int4_decode_step(const mq_decode_args* args, hipStream_t stream) {
    clear_error();
    DecodeShape s;
    int st = validate_decode(args, true, &s);
    if (st != MQ_OK) return st;
    s.int4 = true;
    return launch_decode(*args, s, true, stream);
}

int mq_bf16_decode_step(const mq_decode_args* args, hipStream_t stream) {
    clear_error();
    DecodeShape s;
    int st = validate_decode(args, false, &s);
    if (st != MQ_OK) return st;
    return launch_decode(*args, s, false, stream);
}

int mq_int8_decode_step_noalloc(const mq_decode_args* args, hipStream_t stream) {
    clear_error();
    if (args == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "args is NULL");
    DecodeShape s;
    int st = shape_of(args->dims, &s);
    if (st != MQ_OK) return st;
    const size_t need = decode_workspace_bytes(s);
    if (need > kStaticScratchBytes)
        return set_error(MQ_ERR_UNSUPPORTED, "these dims need a %zu-byte workspace; the static scratch holds %zu", need,
                         kStaticScratchBytes);
    void* ws = nullptr;
    st = static_scratch(&ws);
    if (st != MQ_OK) return st;
    mq_decode_args a = *args;
    a.workspace = ws;
    a.workspace_bytes = need;
    st = validate_decode(&a, true, &s);
    if (st != MQ_OK) return st;
    // every call starts from a cleared scratch (a fill kernel on the caller's stream), so
    // nothing a previous call left there, a failed step's state included, carries over
    hipLaunchKernelGGL(ws_init_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint64_t*>(ws), need / 8);
    st = check_launch("ws_init_kernel");
    if (st != MQ_OK) return st;
    return launch_decode(a, s, true, stream);
}

// Several steps in one launch (mq_generate_args), any weight format: the async-wave kernel
// within its range, else the XCD-aware kernel's multi-step instantiation.
static int decode_generate(const mq_decode_args* args, const mq_generate_args* gen, bool int8, bool fp8,
                           hipStream_t stream, bool int4 = false) {
    if (args == nullptr || gen == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "args is NULL");
    if (gen->prompt_tokens == nullptr || gen->output_tokens == nullptr)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "prompt_tokens and output_tokens must be non-NULL");
    if (gen->n_forced < 1 || gen->n_generate < 1)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "n_forced %d and n_generate %d must be >= 1", gen->n_forced,
                         gen->n_generate);
    DecodeShape s;
    int st = validate_decode(args, int8, &s);
    if (st != MQ_OK) return st;
    s.fp8 = fp8;
    s.int4 = int4;
    if (args->input_token_id != gen->prompt_tokens[0])
        return set_error(MQ_ERR_INVALID_ARGUMENT, "input_token_id %d != prompt_tokens[0] %d", args->input_token_id,
                         gen->prompt_tokens[0]);
    const int64_t n_steps = (int64_t)gen->n_forced + gen->n_generate - 1;
    if (args->position + n_steps > args->max_seq_len)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "position %d + %lld steps exceed max_seq_len %d", args->position,
                         (long long)n_steps, args->max_seq_len);
    if (n_steps > kDecodeMaxForced)
        return set_error(MQ_ERR_UNSUPPORTED, "%lld steps in one launch: at most %d", (long long)n_steps,
                         kDecodeMaxForced);
    for (int i = 0; i < gen->n_forced; ++i)
        if (gen->prompt_tokens[i] < 0 || gen->prompt_tokens[i] >= s.V)
            return set_error(MQ_ERR_INVALID_ARGUMENT, "prompt_tokens[%d] = %d outside [0, %d)", i, gen->prompt_tokens[i], s.V);
    int* dev_tokens = reinterpret_cast<int*>(static_cast<uint8_t*>(args->workspace) + decode_token_offset(s));
    const hipError_t e = hipMemcpyAsync(dev_tokens, gen->prompt_tokens, (size_t)gen->n_forced * sizeof(int),
                                        hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "hipMemcpyAsync(prompt tokens): %s", hipGetErrorString(e));
    const GenPlan plan{dev_tokens, gen->n_forced, (int)n_steps, gen->output_tokens};
    return launch_decode(*args, s, int8, stream, nullptr, &plan);
}

int mq_int8_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream) {
    clear_error();
    return decode_generate(args, gen, true, false, stream);
}

int mq_bf16_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream) {
    clear_error();
    return decode_generate(args, gen, false, false, stream);
}

int mq_fp8_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream) {
    clear_error();
    return decode_generate(args, gen, true, true, stream);
}

int mq_int4_decode_generate(const mq_decode_args* args, const mq_generate_args* gen, hipStream_t stream) {
    clear_error();
    return decode_generate(args, gen, true, false, stream, true);
}

size_t mq_prefill_workspace_bytes(const mq_model_dims* dims, int max_tokens) {
    clear_error();
    DecodeShape s;
    if (shape_of(dims, &s) != MQ_OK) return 0;
    if (s.H != 1024 || s.I != 3072) {
        set_error(MQ_ERR_UNSUPPORTED, "the prefill is compiled for hidden 1024 / intermediate 3072 only");
        return 0;
    }
    if (max_tokens < 1) {
        set_error(MQ_ERR_INVALID_ARGUMENT, "max_tokens %d < 1", max_tokens);
        return 0;
    }
    return prefill_workspace_bytes(max_tokens);
}

int mq_int8_prefill(const mq_decode_args* a, const int* tokens, int n_tokens, void* workspace,
                    size_t workspace_bytes, hipStream_t stream) {
    clear_error();
    if (a == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "args is NULL");
    DecodeShape s;
    int st = shape_of(a->dims, &s);
    if (st != MQ_OK) return st;
    if (s.H != 1024 || s.I != 3072)
        return set_error(MQ_ERR_UNSUPPORTED, "the prefill is compiled for hidden 1024 / intermediate 3072 only");
    if (a->num_layers < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "num_layers %d < 1", a->num_layers);
    if (a->max_seq_len < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "max_seq_len %d < 1", a->max_seq_len);
    if (n_tokens < 0) return set_error(MQ_ERR_INVALID_ARGUMENT, "n_tokens %d < 0", n_tokens);
    if (n_tokens == 0) return MQ_OK;
    if (tokens == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "tokens is NULL");
    if (a->position < 0 || (int64_t)a->position + n_tokens > a->max_seq_len)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "positions [%d, %lld) outside [0, max_seq_len=%d)", a->position,
                         (long long)a->position + n_tokens, a->max_seq_len);
    for (int i = 0; i < n_tokens; ++i)
        if (tokens[i] < 0 || tokens[i] >= s.V)
            return set_error(MQ_ERR_INVALID_ARGUMENT, "tokens[%d] = %d outside [0, %d)", i, tokens[i], s.V);
    if (!a->embed_weight || !a->layer_weights || !a->scales || !a->cos_table || !a->sin_table || !a->k_cache ||
        !a->v_cache)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "a required pointer is NULL");
    if (!aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->embed_weight))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "embed_weight and the KV caches must be 16-byte aligned");
    if (!workspace || !aligned16(workspace))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the prefill workspace must be non-NULL and 16-byte aligned");
    if (prefill_capacity(workspace_bytes) < 1)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "a prefill workspace of %zu bytes is below the %zu of one chunk",
                         workspace_bytes, prefill_workspace_bytes(1));
    const size_t cache = (size_t)a->num_layers * s.NKV * a->max_seq_len * s.D * 2;
    const size_t table = (size_t)a->max_seq_len * s.D * 2;
    if (!in_allocation(a->embed_weight, (size_t)s.H * s.V * 2))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "embed_weight holds fewer than vocab_size = %d rows of %d", s.V, s.H);
    if (!in_allocation(a->k_cache, cache) || !in_allocation(a->v_cache, cache))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the KV caches hold fewer than num_layers x %d x max_seq_len x %d "
                         "bf16 values", s.NKV, s.D);
    if (!in_allocation(a->cos_table, table) || !in_allocation(a->sin_table, table))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the RoPE tables hold fewer than max_seq_len rows of %d", s.D);
    if (!in_allocation(workspace, workspace_bytes))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "the prefill workspace is smaller than workspace_bytes");
    return launch_prefill(*a, tokens, n_tokens, workspace, workspace_bytes, stream);
}

int mq_prefill_check(void* workspace, size_t workspace_bytes, hipStream_t stream) {
    clear_error();
    if (!workspace) return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace is NULL");
    return prefill_check(workspace, workspace_bytes, stream);
}

int mq_wait_host_token(const volatile int* token, int sentinel, unsigned int timeout_us) {
    clear_error();
    if (!token) return set_error(MQ_ERR_INVALID_ARGUMENT, "token is NULL");
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned int n = 0;; ++n) {
        if (*token != sentinel) return MQ_OK;
        if ((n & 1023u) == 1023u &&
            std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(timeout_us))
            return set_error(MQ_ERR_TIMEOUT, "no token after %u us", timeout_us);
    }
}

int mq_decode_check(void* workspace, hipStream_t stream) {
    clear_error();
    if (!workspace) return set_error(MQ_ERR_INVALID_ARGUMENT, "workspace is NULL");
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    uint32_t flag = 0;
    e = hipMemcpy(&flag, static_cast<uint8_t*>(workspace) + offsetof(WsHeader, abort_flag), sizeof(flag),
                  hipMemcpyDeviceToHost);
    if (e != hipSuccess) return set_error(MQ_ERR_HIP, "hipMemcpy: %s", hipGetErrorString(e));
    if (flag == 2) {
        mark_xcd_unusable();
        return set_error(MQ_ERR_TIMEOUT, "a workgroup ran on an unexpected XCD; the XCD-aware kernel is disabled for "
                                         "this device, re-initialise the workspace and repeat the step");
    }
    if (flag == 3)
        return set_error(MQ_ERR_TIMEOUT, "the workspace was used with another batch size; re-initialise it");
    if (flag != 0)
        return set_error(MQ_ERR_TIMEOUT, "a bounded wait in the decode kernel expired; re-initialise the workspace");
    return MQ_OK;
}

size_t mq_batch_workspace_bytes(const mq_model_dims* dims) {
    clear_error();
    DecodeShape s{2048, 6144, 16, 8, 128, 151936};
    if (dims != nullptr && shape_of(dims, &s) != MQ_OK) return 0;
    const size_t n = decode_batch_workspace_bytes(s);
    if (n == 0) set_error(MQ_ERR_UNSUPPORTED, "no batched decode kernel for hidden %d / intermediate %d", s.H, s.I);
    return n;
}

int mq_int8_decode_batch_step(const mq_batch_args* args, hipStream_t stream) {
    clear_error();
    if (args == nullptr) return set_error(MQ_ERR_INVALID_ARGUMENT, "args is NULL");
    DecodeShape s{2048, 6144, 16, 8, 128, 151936};
    if (args->dims != nullptr) {
        const int st = shape_of(args->dims, &s);
        if (st != MQ_OK) return st;
    }
    if (args->max_seq_len < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "max_seq_len %d < 1", args->max_seq_len);
    if (!aligned16(args->lm_head_weight) || !aligned16(args->k_cache) || !aligned16(args->v_cache) ||
        !aligned16(args->workspace) || !aligned16(args->embed_weight))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "weights, KV caches and workspace must be 16-byte aligned");
    return launch_decode_batch(*args, s, stream);
}

void mq_reference_set_spin_limit(unsigned int polls) {
    clear_error();
    g_ref_spin = polls;
}

int mq_reference_set_dims(const mq_model_dims* dims) {
    clear_error();
    if (dims != nullptr) {
        DecodeShape s;
        const int st = shape_of(dims, &s);
        if (st != MQ_OK) return st;
    }
    std::lock_guard<std::mutex> lk(g_ref_mu);
    g_ref_has_dims = dims != nullptr;
    if (dims != nullptr) g_ref_dims = *dims;
    return MQ_OK;
}

int mq_decode_set_variant(int variant) {
    clear_error();
    return set_decode_variant(variant);
}

int mq_decode_set_cooperative(int enable) {
    clear_error();
    return set_cooperative_launch(enable);
}

int mq_decode_variant(const mq_model_dims* dims, int int8) {
    clear_error();
    DecodeShape s;
    int st = shape_of(dims, &s);
    if (st != MQ_OK) return -st;
    return decode_variant_in_use(s, int8 != 0);            // the variant, or minus the refusal's status
}

int mq_decode_variant_at(const mq_model_dims* dims, int int8, int cache_len) {
    clear_error();
    DecodeShape s;
    int st = shape_of(dims, &s);
    if (st != MQ_OK) return -st;
    if (cache_len < 1) return -set_error(MQ_ERR_INVALID_ARGUMENT, "cache_len %d < 1", cache_len);
    return decode_variant_for(s, int8 != 0, cache_len);
}

void launch_a10_int8_decode(int input_token_id, int* output_token_id, const void* embed_weight,
                            const LayerWeights* layer_weights, const void* final_norm_weight,
                            const void* lm_head_weight, const float* lm_head_scale, const void* cos_table,
                            const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                            void* g_activations, void* g_residual, void* g_q, void* g_k, void* g_v,
                            void* g_attn_out, void* g_mlp_intermediate, void* g_normalized,
                            void* block_max_vals, void* block_max_idxs, int num_layers, int position,
                            int cache_len, int max_seq_len, float attn_scale, const ScalePointers* scales,
                            hipStream_t stream) {
    clear_error();
    mq_decode_args a;
    memset(&a, 0, sizeof(a));
    uint32_t* status = nullptr;
    mq_model_dims dims;
    a.dims = reference_dims(&dims);
    if (default_workspace(a.dims, stream, &a.workspace, &a.workspace_bytes, &status) != MQ_OK) return;
    a.input_token_id = input_token_id;
    a.output_token_id = output_token_id;
    a.embed_weight = embed_weight;
    a.layer_weights = layer_weights;
    a.scales = scales;
    a.final_norm_weight = final_norm_weight;
    a.lm_head_weight = lm_head_weight;
    a.lm_head_scale = lm_head_scale;
    a.cos_table = cos_table;
    a.sin_table = sin_table;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.hidden_buffer = hidden_buffer;
    a.g_activations = g_activations;
    a.g_residual = g_residual;
    a.g_q = g_q;
    a.g_k = g_k;
    a.g_v = g_v;
    a.g_attn_out = g_attn_out;
    a.g_mlp_intermediate = g_mlp_intermediate;
    a.g_normalized = g_normalized;
    a.block_max_vals = block_max_vals;
    a.block_max_idxs = block_max_idxs;
    a.num_layers = num_layers;
    a.position = position;
    a.cache_len = cache_len;
    a.max_seq_len = max_seq_len;
    a.attn_scale = attn_scale;
    a.spin_limit = g_ref_spin.load();
    reference_step(&a, true, status, stream);
}

void launch_a10_decode(int input_token_id, int* output_token_id, const void* embed_weight,
                       const LayerWeights* layer_weights, const void* final_norm_weight, const void* lm_head_weight,
                       const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                       void* hidden_buffer, void* g_activations, void* g_residual, void* g_q, void* g_k, void* g_v,
                       void* g_attn_out, void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
                       void* block_max_idxs, int num_layers, int position, int cache_len, int max_seq_len,
                       float attn_scale, hipStream_t stream) {
    clear_error();
    mq_decode_args a;
    memset(&a, 0, sizeof(a));
    uint32_t* status = nullptr;
    mq_model_dims dims;
    a.dims = reference_dims(&dims);
    if (default_workspace(a.dims, stream, &a.workspace, &a.workspace_bytes, &status) != MQ_OK) return;
    a.input_token_id = input_token_id;
    a.output_token_id = output_token_id;
    a.embed_weight = embed_weight;
    a.layer_weights = layer_weights;
    a.final_norm_weight = final_norm_weight;
    a.lm_head_weight = lm_head_weight;
    a.cos_table = cos_table;
    a.sin_table = sin_table;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.hidden_buffer = hidden_buffer;
    a.g_activations = g_activations;
    a.g_residual = g_residual;
    a.g_q = g_q;
    a.g_k = g_k;
    a.g_v = g_v;
    a.g_attn_out = g_attn_out;
    a.g_mlp_intermediate = g_mlp_intermediate;
    a.g_normalized = g_normalized;
    a.block_max_vals = block_max_vals;
    a.block_max_idxs = block_max_idxs;
    a.num_layers = num_layers;
    a.position = position;
    a.cache_len = cache_len;
    a.max_seq_len = max_seq_len;
    a.attn_scale = attn_scale;
    a.spin_limit = g_ref_spin.load();
    reference_step(&a, false, status, stream);
}

int mq_int8_gemv(const float* x, const int8_t* w, const float* scale, float* y, int M, int K, hipStream_t stream) {
    clear_error();
    if (!x || !w || !scale || !y) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < 1 || K > 16384 || (K % 16) != 0)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and 16 <= K <= 16384 with K %% 16 == 0 (M=%d K=%d)", M, K);
    if (!aligned16(w) || !aligned16(x)) return set_error(MQ_ERR_INVALID_ARGUMENT, "x and w must be 16-byte aligned");
    return launch_int8_gemv(x, w, scale, y, M, K, stream);
}

int mq_int8_gemv_repeat(const float* x, const int8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                        float* y, int M, int K, int reps, hipStream_t stream) {
    clear_error();
    if (!x || !w || !scale || !y) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < 1 || K > 16384 || (K % 16) != 0)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and 16 <= K <= 16384 with K %% 16 == 0 (M=%d K=%d)", M, K);
    if (n_copies < 1 || reps < 1 || (int64_t)reps * M >= ((int64_t)1 << 31))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need n_copies >= 1, reps >= 1 and reps * M < 2^31 (n_copies=%d reps=%d)",
                         n_copies, reps);
    if (n_copies > 1 && (copy_stride < (int64_t)M * K || (copy_stride % 16) != 0))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "copy_stride %lld must be a multiple of 16 and >= M * K",
                         (long long)copy_stride);
    if (!aligned16(w) || !aligned16(x)) return set_error(MQ_ERR_INVALID_ARGUMENT, "x and w must be 16-byte aligned");
    return launch_int8_gemv_repeat(x, w, n_copies > 1 ? copy_stride : 0, n_copies, scale, y, M, K, reps, stream);
}

int mq_quantize_per_channel_bf16(const void* w_bf16, int M, int K, int8_t* q, float* scale, hipStream_t stream) {
    clear_error();
    if (!w_bf16 || !q || !scale) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and K >= 1 (M=%d K=%d)", M, K);
    return launch_quantize(w_bf16, M, K, q, scale, stream);
}

// ---- other weight formats ----------------------------------------------------------------
int mq_quantize_fp8_rows_bf16(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream) {
    clear_error();
    if (!w_bf16 || !q || !scale) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < 1) return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and K >= 1 (M=%d K=%d)", M, K);
    return launch_quantize_fp8(w_bf16, M, K, q, scale, stream);
}

int mq_quantize_int4_groups_bf16(const void* w_bf16, int M, int K, uint8_t* q, float* scale, hipStream_t stream) {
    clear_error();
    if (!w_bf16 || !q || !scale) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < 128 || (K % 128) != 0)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and K a positive multiple of 128 (M=%d K=%d)", M, K);
    return launch_quantize_int4(w_bf16, M, K, q, scale, stream);
}

// Shared checks of the FP8 / INT4 matvecs; `kmul` is the row-length multiple (16 / 128),
// `row_bytes` the bytes of one weight row.
static int check_fmt_gemv(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                          const float* y, int M, int K, int reps, int kmul, int64_t row_bytes) {
    if (!x || !w || !scale || !y) return set_error(MQ_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (M < 1 || K < kmul || K > 16384 || (K % kmul) != 0)
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need M >= 1 and %d <= K <= 16384 with K %% %d == 0 (M=%d K=%d)",
                         kmul, kmul, M, K);
    if (n_copies < 1 || reps < 1 || (int64_t)reps * M >= ((int64_t)1 << 31))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "need n_copies >= 1, reps >= 1 and reps * M < 2^31 (n_copies=%d reps=%d)",
                         n_copies, reps);
    if (n_copies > 1 && (copy_stride < (int64_t)M * row_bytes || (copy_stride % 16) != 0))
        return set_error(MQ_ERR_INVALID_ARGUMENT, "copy_stride %lld must be a multiple of 16 and >= M * row bytes",
                         (long long)copy_stride);
    if (!aligned16(w) || !aligned16(x)) return set_error(MQ_ERR_INVALID_ARGUMENT, "x and w must be 16-byte aligned");
    return MQ_OK;
}

int mq_fp8_gemv_repeat(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                       float* y, int M, int K, int reps, hipStream_t stream) {
    clear_error();
    const int st = check_fmt_gemv(x, w, copy_stride, n_copies, scale, y, M, K, reps, 16, K);
    if (st != MQ_OK) return st;
    return launch_fp8_gemv(x, w, n_copies > 1 ? copy_stride : 0, n_copies, scale, y, M, K, reps, stream);
}

int mq_fp8_gemv(const float* x, const uint8_t* w, const float* scale, float* y, int M, int K, hipStream_t stream) {
    return mq_fp8_gemv_repeat(x, w, 0, 1, scale, y, M, K, 1, stream);
}

int mq_int4_gemv_repeat(const float* x, const uint8_t* w, int64_t copy_stride, int n_copies, const float* scale,
                        float* y, int M, int K, int reps, hipStream_t stream) {
    clear_error();
    const int st = check_fmt_gemv(x, w, copy_stride, n_copies, scale, y, M, K, reps, 128, K / 2);
    if (st != MQ_OK) return st;
    return launch_int4_gemv(x, w, n_copies > 1 ? copy_stride : 0, n_copies, scale, y, M, K, reps, stream);
}

int mq_int4_gemv(const float* x, const uint8_t* w, const float* scale, float* y, int M, int K, hipStream_t stream) {
    return mq_int4_gemv_repeat(x, w, 0, 1, scale, y, M, K, 1, stream);
}

}  // extern "C"
