// SPDX-License-Identifier: MIT
//
// The C ABI of libdbs_hip.so (include/dbs_cuda.h, include/dbs_hip.h):
// argument checks, workspace planning and kernel launches on the caller's
// stream. Statuses, limits and validation rules follow the reference's
// device ABI (reference cuda/dbs_cuda.cu:1254-1271, 1596-1949).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <mutex>
#include <vector>
#include <cstdlib>
#include <cstring>
#include <limits>

#include "dbs_cuda.h"
#include "dbs_hip.h"
#include "engine.hpp"
#include "host_entry.hpp"

using namespace dbs_hip;

// ---------------------------------------------------------------------------
// Optional launch timing (dbs_hip_profile_*)
// ---------------------------------------------------------------------------

namespace {

struct PendingTiming {
    int kind;
    hipEvent_t start;
    hipEvent_t stop;
};

std::atomic<int> g_profile{0};
std::mutex g_profile_mutex;
std::vector<PendingTiming> g_pending;
double g_total_ms[kKindCount] = {};
int64_t g_launches[kKindCount] = {};

// Folds completed timings into the totals (waits for their stop events).
void drain_pending() {
    for (const PendingTiming& t : g_pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(t.stop) == hipSuccess && hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess) {
            g_total_ms[t.kind] += ms;
            g_launches[t.kind] += 1;
        }
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    g_pending.clear();
    (void)hipGetLastError();
}

}  // namespace

namespace dbs_hip {

KernelTimer::KernelTimer(int kind, hipStream_t stream) : kind_(kind), stream_(stream) {
    if (g_profile.load(std::memory_order_relaxed) == 0) return;
    if (hipEventCreate(&start_) != hipSuccess || hipEventCreate(&stop_) != hipSuccess ||
        hipEventRecord(start_, stream_) != hipSuccess) {
        if (start_) (void)hipEventDestroy(start_);
        if (stop_) (void)hipEventDestroy(stop_);
        start_ = stop_ = nullptr;
        (void)hipGetLastError();
    }
}

KernelTimer::~KernelTimer() {
    if (!start_) return;
    if (hipEventRecord(stop_, stream_) != hipSuccess) {
        (void)hipEventDestroy(start_);
        (void)hipEventDestroy(stop_);
        (void)hipGetLastError();
        return;
    }
    std::lock_guard<std::mutex> lock(g_profile_mutex);
    g_pending.push_back(PendingTiming{kind_, start_, stop_});
}

}  // namespace dbs_hip

namespace {

// dbs_cuda_set_synchronization's flag; the environment can also ask for a
// synchronisation after every call (DBS_CUDA_SYNC_CHECK=1, or the legacy
// DBS_CUDA_DEBUG_SYNC=1), read on every call as the reference does
// (reference cuda/dbs_cuda.cu:1226-1231).
std::atomic<int> g_sync{0};

bool sync_requested() {
    if (g_sync.load(std::memory_order_relaxed) != 0) return true;
    const char* v = std::getenv("DBS_CUDA_SYNC_CHECK");
    const char* legacy = std::getenv("DBS_CUDA_DEBUG_SYNC");
    return (v && v[0] == '1') || (legacy && legacy[0] == '1');
}

int status_of(hipError_t e) {
    if (e == hipSuccess) return DBS_CUDA_STATUS_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return DBS_CUDA_STATUS_OUT_OF_MEMORY;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return DBS_CUDA_STATUS_UNAVAILABLE;
    return DBS_CUDA_STATUS_LAUNCH_FAILED;
}

int finish(hipStream_t stream, hipError_t e) {
    if (e == hipSuccess && sync_requested()) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) (void)hipGetLastError();
    return status_of(e);
}

// finish() for a decode: when the call synchronises, an overlapped decode
// whose select pass gave up a wait (fault word set) reports a failed launch;
// asynchronous callers see it as invalid_input[b] == 2.
int finish_decode(hipStream_t stream, hipError_t e, const int32_t* fault) {
    if (e != hipSuccess || !sync_requested()) return finish(stream, e);
    e = hipStreamSynchronize(stream);
    int32_t host = 0;
    if (e == hipSuccess && fault) e = hipMemcpy(&host, fault, sizeof(host), hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return status_of(e);
    }
    return host != 0 ? DBS_CUDA_STATUS_LAUNCH_FAILED : DBS_CUDA_STATUS_OK;
}

// finish_decode() that always synchronises: for a caller that asked for the
// fault word of a decode whose workspace the call allocated itself.
int finish_decode_sync(hipStream_t stream, hipError_t e, const int32_t* fault) {
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    int32_t host = 0;
    if (e == hipSuccess && fault) e = hipMemcpy(&host, fault, sizeof(host), hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return status_of(e);
    }
    return host != 0 ? DBS_CUDA_STATUS_LAUNCH_FAILED : DBS_CUDA_STATUS_OK;
}

bool valid_dtype(int d) { return d == DBS_CUDA_DTYPE_F32 || d == DBS_CUDA_DTYPE_F16 || d == DBS_CUDA_DTYPE_BF16; }

// Shape and option checks (reference cuda/dbs_cuda.cu:1254-1271). Candidate
// indices p * V + v must fit in int32.
bool valid_args(const DBSCudaDecodeArgs* a) {
    if (!a) return false;
    if (a->batch_size <= 0 || a->steps <= 0 || a->beam_size <= 0 || a->vocab_size <= 0) return false;
    if (a->beam_size > DBS_CUDA_MAX_BEAM) return false;
    if (a->eos_token < -1 || a->eos_token >= a->vocab_size) return false;
    if (a->min_length < 0) return false;
    if (!std::isfinite(a->length_penalty_alpha) || a->length_penalty_alpha < 0.0f) return false;
    if (!std::isfinite(a->repetition_penalty) || a->repetition_penalty < 0.0f) return false;
    if (a->reserved0 != 0) return false;
    if (static_cast<int64_t>(a->beam_size) * a->vocab_size > std::numeric_limits<int32_t>::max()) return false;
    const double elements = static_cast<double>(a->batch_size) * a->steps * a->beam_size * a->vocab_size;
    return elements < 9.0e18;
}

bool has_per_example(const DBSCudaDecodeArgs& a) {
    return a.steps_per_example || a.beam_sizes_per_example || a.eos_tokens_per_example || a.min_lengths_per_example;
}

bool constrained(const DBSCudaDecodeArgs& a) { return a.no_repeat_ngram_size > 0 || a.repetition_penalty > 1.0f; }

bool valid_options(const DBSCudaSearchOptions* o, const DBSCudaDecodeArgs& a) {
    if (!o) return true;
    if (o->reserved0 != 0) return false;
    for (int i = 0; i < 4; ++i)
        if (o->reserved[i]) return false;
    if (o->extra_eos_count < 0 || o->extra_eos_count > DBS_CUDA_MAX_EXTRA_EOS) return false;
    if (o->extra_eos_count > 0 && a.eos_token < 0 && !a.eos_tokens_per_example) return false;
    for (int i = 0; i < o->extra_eos_count; ++i)
        if (o->extra_eos_tokens[i] < 0 || o->extra_eos_tokens[i] >= a.vocab_size) return false;
    return true;
}

// The EOS tokens: the scalar one with the extra ones, or with per-example EOS
// tokens the extra ones only (each example adds its own).
void fill_eos(DecodeParams& p, const DBSCudaDecodeArgs& a, const DBSCudaSearchOptions* o) {
    p.eos = a.eos_token;
    p.n_eos = 0;
    p.eos_pe = a.eos_tokens_per_example;
    p.minlen_pe = a.min_lengths_per_example;
    p.beam_pe = a.beam_sizes_per_example;
    if (a.eos_token < 0 && !a.eos_tokens_per_example) return;
    int32_t set[kMaxEos];
    int n = 0;
    if (!a.eos_tokens_per_example) set[n++] = a.eos_token;
    if (o)
        for (int i = 0; i < o->extra_eos_count; ++i) set[n++] = o->extra_eos_tokens[i];
    // sort, unique (reference src/decoder.cpp:57-63)
    for (int i = 1; i < n; ++i) {
        const int32_t v = set[i];
        int j = i - 1;
        while (j >= 0 && set[j] > v) {
            set[j + 1] = set[j];
            --j;
        }
        set[j + 1] = v;
    }
    for (int i = 0; i < n; ++i)
        if (p.n_eos == 0 || p.eos_set[p.n_eos - 1] != set[i]) p.eos_set[p.n_eos++] = set[i];
}

// Stream-ordered scratch: the caller's, or allocated and released on the stream.
struct Scratch {
    void* ptr = nullptr;
    bool owned = false;
    hipStream_t stream = nullptr;
    hipError_t acquire(void* ws, int64_t ws_bytes, size_t need, hipStream_t s, bool* too_small) {
        stream = s;
        *too_small = false;
        if (ws) {
            // the workspace holds 16-byte words: it must be 16-byte aligned
            if (ws_bytes < static_cast<int64_t>(need) || reinterpret_cast<uintptr_t>(ws) % 16 != 0) {
                *too_small = true;
                return hipSuccess;
            }
            ptr = ws;
            return hipSuccess;
        }
        owned = true;
        return hipMallocAsync(&ptr, need, s);
    }
    ~Scratch() {
        if (owned && ptr) (void)hipFreeAsync(ptr, stream);
    }
};

// Device-side range check of the per-example arrays, read back once
// (synchronizes the stream); status is 4 bytes of device scratch.
int check_per_example(const DBSCudaDecodeArgs& a, int32_t* status, hipStream_t stream) {
    if (!has_per_example(a)) return DBS_CUDA_STATUS_OK;
    hipError_t e = launch_check_examples(a.steps_per_example, a.beam_sizes_per_example, a.eos_tokens_per_example,
                                         a.min_lengths_per_example, a.batch_size, a.steps, a.beam_size, a.vocab_size,
                                         status, stream);
    int32_t host = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&host, status, sizeof(host), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return finish(stream, e);
    return host != 0 ? DBS_CUDA_STATUS_INVALID_ARGUMENT : DBS_CUDA_STATUS_OK;
}

void set_pool(DecodeParams& p, const PoolOutputs* pool) {
    if (!pool || pool->mult <= 0) return;
    p.pool_mult = pool->mult;
    p.pool_parents = pool->parents;
    p.pool_tokens = pool->tokens;
    p.pool_lengths = pool->lengths;
    p.pool_scores = pool->scores;
    p.pool_raw = pool->raw_scores;
    p.pool_flp = pool->from_logprob;
}

int decode_common(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                  const DBSCudaSearchOptions* options, const uint8_t* banned_pe, const DBSCudaDecodeOutputs* outputs,
                  float* row_lse, void* workspace, int64_t workspace_bytes, void* stream_ptr,
                  bool allow_overlap = true, int32_t* first_invalid = nullptr, int32_t** fault_out = nullptr,
                  const int32_t* forced = nullptr, const PoolOutputs* pool = nullptr) {
    if (!inputs || !valid_dtype(data_type) || !valid_args(args) || !outputs || !outputs->final_scores)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (!valid_options(options, *args)) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const bool cons = constrained(a);
    const int pool_mult = pool ? pool->mult : 0;
    if (pool_mult < 0 || static_cast<int64_t>(pool_mult) * a.beam_size > DBS_CUDA_MAX_BEAM)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DecodeLayout L =
        decode_layout(a.batch_size, a.steps, a.beam_size, a.vocab_size, cons, false, 0, pool_mult * a.beam_size);
    bool too_small = false;
    Scratch scratch;
    hipError_t e = scratch.acquire(workspace, workspace_bytes, L.total, stream, &too_small);
    if (too_small) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (e != hipSuccess) return finish(stream, e);
    char* ws = static_cast<char*>(scratch.ptr);

    const int checked = check_per_example(a, reinterpret_cast<int32_t*>(ws + L.off_rowinfo), stream);
    if (checked != DBS_CUDA_STATUS_OK) return checked;

    DecodeParams p{};
    p.x = inputs;
    p.dtype = data_type;
    p.from_logits = from_logits ? 1 : 0;
    p.B = a.batch_size;
    p.T = a.steps;
    p.K = a.beam_size;
    p.V = a.vocab_size;
    fill_eos(p, a, options);
    p.min_length = a.min_length;
    p.alpha = a.length_penalty_alpha;
    p.ngram = a.no_repeat_ngram_size > 0 ? a.no_repeat_ngram_size : 0;
    p.penalise = a.repetition_penalty > 1.0f ? 1 : 0;
    p.log_rep = p.penalise ? std::log(a.repetition_penalty) : 0.0f;
    p.constrained = cons ? 1 : 0;
    p.M = L.M;
    p.use_tau = L.use_tau;
    p.steps = a.steps_per_example;
    p.banned = a.banned_tokens;
    p.banned_pe = banned_pe;
    p.forced = forced;
    set_pool(p, pool);
    p.rowinfo = reinterpret_cast<RowInfo*>(ws + L.off_rowinfo);
    p.shortlist = reinterpret_cast<ShortEntry*>(ws + L.off_short);
    p.prefix = reinterpret_cast<int32_t*>(ws + L.off_prefix);
    p.blocked = reinterpret_cast<int32_t*>(ws + L.off_blocked);
    p.prefix_cap = L.prefix_cap;
    p.final_scores = outputs->final_scores;
    p.final_raw = outputs->final_raw_scores;
    p.final_lengths = outputs->final_lengths;
    p.tokens = outputs->tokens;
    p.parents = outputs->parents;
    p.lengths = outputs->lengths;
    p.scores = outputs->scores;
    p.raw_scores = outputs->raw_scores;
    p.from_logprob = outputs->from_logprob;
    p.invalid = outputs->invalid_input;
    p.row_lse = row_lse;
    p.first_invalid = first_invalid;
    int32_t* fault = nullptr;
    e = launch_decode(p, L, stream, ws, &fault, allow_overlap);
    // the fault word lives in the workspace: handed out only where that is
    // the caller's (an allocated one is released when the call returns)
    if (fault_out) *fault_out = (e == hipSuccess && workspace) ? fault : nullptr;
    if (fault_out && !workspace) return finish_decode_sync(stream, e, fault);
    return finish_decode(stream, e, fault);
}

int step_common(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                const DBSCudaSearchOptions* options, const DBSCudaBeamState* state,
                const DBSCudaDecodeOutputs* outputs, float* row_lse, void* workspace, int64_t workspace_bytes,
                void* stream_ptr, const int32_t* forced = nullptr, const PoolOutputs* pool = nullptr,
                const uint8_t* row_mask = nullptr) {
    if (!inputs || !valid_dtype(data_type) || !valid_args(args) || !state || !outputs)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (!valid_options(options, *args)) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    if (a.steps != 1 || a.steps_per_example) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (!state->raw_scores || !state->lengths || !state->finished || state->prefix_stride < 0 || state->reserved0 != 0)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const bool cons = constrained(a);
    if (cons && state->prefix_stride > 0 && !state->prefixes) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const int pool_mult = pool ? pool->mult : 0;
    if (pool_mult < 0 || static_cast<int64_t>(pool_mult) * a.beam_size > DBS_CUDA_MAX_BEAM)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    DecodeLayout L = decode_layout(a.batch_size, 1, a.beam_size, a.vocab_size, cons, true, state->prefix_stride,
                                   pool_mult * a.beam_size);
    if (row_mask) L.M = 0;  // filtered rows are read in full
    bool too_small = false;
    Scratch scratch;
    hipError_t e = scratch.acquire(workspace, workspace_bytes, L.total, stream, &too_small);
    if (too_small) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (e != hipSuccess) return finish(stream, e);
    char* ws = static_cast<char*>(scratch.ptr);
    const int checked = check_per_example(a, reinterpret_cast<int32_t*>(ws + L.off_rowinfo), stream);
    if (checked != DBS_CUDA_STATUS_OK) return checked;

    DecodeParams p{};
    p.x = inputs;
    p.dtype = data_type;
    p.from_logits = from_logits ? 1 : 0;
    p.B = a.batch_size;
    p.T = 1;
    p.K = a.beam_size;
    p.V = a.vocab_size;
    fill_eos(p, a, options);
    p.min_length = a.min_length;
    p.alpha = a.length_penalty_alpha;
    p.ngram = a.no_repeat_ngram_size > 0 ? a.no_repeat_ngram_size : 0;
    p.penalise = a.repetition_penalty > 1.0f ? 1 : 0;
    p.log_rep = p.penalise ? std::log(a.repetition_penalty) : 0.0f;
    p.constrained = cons ? 1 : 0;
    p.M = L.M;
    p.use_tau = 0;
    p.banned = a.banned_tokens;
    p.forced = forced;
    p.row_mask = row_mask;
    set_pool(p, pool);
    p.rowinfo = reinterpret_cast<RowInfo*>(ws + L.off_rowinfo);
    p.shortlist = reinterpret_cast<ShortEntry*>(ws + L.off_short);
    p.blocked = reinterpret_cast<int32_t*>(ws + L.off_blocked);
    p.prefix_cap = L.prefix_cap;
    p.final_scores = outputs->final_scores;
    p.final_raw = outputs->final_scores ? outputs->final_raw_scores : nullptr;
    p.final_lengths = outputs->final_scores ? outputs->final_lengths : nullptr;
    p.tokens = outputs->tokens;
    p.parents = outputs->parents;
    p.lengths = outputs->lengths;
    p.scores = outputs->scores;
    p.raw_scores = outputs->raw_scores;
    p.from_logprob = outputs->from_logprob;
    p.invalid = outputs->invalid_input;
    p.row_lse = row_lse;
    p.step_mode = 1;
    p.st_raw = state->raw_scores;
    p.st_len = state->lengths;
    p.st_fin = state->finished;
    p.st_prefix = state->prefix_stride > 0 ? state->prefixes : nullptr;
    p.st_stride = state->prefix_stride;
    int32_t* fault = nullptr;
    e = launch_decode(p, L, stream, ws, &fault, true);
    return finish_decode(stream, e, fault);
}

void set_pool_grads(BackwardParams& p, const PoolGrads* pool) {
    if (!pool || pool->P <= 0 || !pool->d) return;
    p.P = pool->P;
    p.pool_parents = pool->parents;
    p.pool_tokens = pool->tokens;
    p.pool_flp = pool->from_logprob;
    p.pool_d = pool->d;
}

// mode: 0 writes the gradient everywhere, 1 accumulates into float32, 2
// writes only the rows that receive an entry (the buffer holds zeros).
int backward_common(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, void* out, int out_type,
                    int mode, void* workspace, int64_t workspace_bytes, void* stream_ptr,
                    const PoolGrads* pool = nullptr) {
    if (!valid_args(args) || !in || !out) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (!in->parents || !in->tokens || !in->lengths || !in->from_logprob) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (in->reserved0 != 0) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    for (int i = 0; i < 4; ++i)
        if (in->reserved[i]) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (in->logits && (!in->row_lse || !valid_dtype(in->logits_type))) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const size_t need = backward_workspace_bytes(a.batch_size, a.steps, a.beam_size) + 256;
    bool too_small = false;
    Scratch scratch;
    hipError_t e = scratch.acquire(workspace, workspace_bytes, need, stream, &too_small);
    if (too_small) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (e != hipSuccess) return finish(stream, e);
    char* ws = static_cast<char*>(scratch.ptr);

    const int checked = check_per_example(
        a, reinterpret_cast<int32_t*>(ws + backward_workspace_bytes(a.batch_size, a.steps, a.beam_size)), stream);
    if (checked != DBS_CUDA_STATUS_OK) return checked;
    BackwardParams p{};
    p.B = a.batch_size;
    p.T = a.steps;
    p.K = a.beam_size;
    p.V = a.vocab_size;
    p.alpha = a.length_penalty_alpha;
    p.steps = a.steps_per_example;
    p.beams = a.beam_sizes_per_example;
    p.parents = in->parents;
    p.tokens = in->tokens;
    p.lengths = in->lengths;
    p.from_logprob = in->from_logprob;
    p.g_final = in->grad_final_scores;
    p.g_final_raw = in->grad_final_raw_scores;
    p.g_scores = in->grad_scores;
    p.g_raw = in->grad_raw_scores;
    p.logits = in->logits;
    p.logits_type = in->logits_type;
    p.row_lse = in->row_lse;
    p.draws = reinterpret_cast<float*>(ws);
    p.out = out;
    p.out_type = out_type;
    p.accumulate = mode;
    set_pool_grads(p, pool);
    e = launch_path_walk(p, stream);
    if (e == hipSuccess) e = launch_dense_gradient(p, stream);
    return finish(stream, e);
}

}  // namespace

// Entry points for the host ABI (host_abi.cpp), inside the library.
namespace dbs_hip {

int decode_for_host(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                    const DBSCudaSearchOptions* options, const uint8_t* banned_per_example,
                    const DBSCudaDecodeOutputs* outputs, float* row_lse, int32_t* first_invalid,
                    const int32_t* forced, const PoolOutputs* pool, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream, int32_t** fault) {
    return decode_common(inputs, data_type, from_logits, args, options, banned_per_example, outputs, row_lse,
                         workspace, workspace_bytes, stream, true, first_invalid, fault, forced, pool);
}

int step_for_host(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                  const DBSCudaSearchOptions* options, const DBSCudaBeamState* state,
                  const DBSCudaDecodeOutputs* outputs, float* row_lse, const int32_t* forced,
                  const PoolOutputs* pool, const uint8_t* row_mask, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream) {
    return step_common(inputs, data_type, from_logits, args, options, state, outputs, row_lse, workspace,
                       workspace_bytes, stream, forced, pool, row_mask);
}

int64_t workspace_for_host(const DBSCudaDecodeArgs* args, int pool_mult, int step_mode, int prefix_stride) {
    if (!valid_args(args) || pool_mult < 0 || static_cast<int64_t>(pool_mult) * args->beam_size > DBS_CUDA_MAX_BEAM)
        return -1;
    if (step_mode && (args->steps != 1 || args->steps_per_example || prefix_stride < 0)) return -1;
    return static_cast<int64_t>(decode_layout(args->batch_size, step_mode ? 1 : args->steps, args->beam_size,
                                              args->vocab_size, constrained(*args), step_mode != 0,
                                              step_mode ? prefix_stride : 0, pool_mult * args->beam_size)
                                    .total);
}

int backward_dense_for_host(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, const PoolGrads* pool,
                            float* grad, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
    return backward_common(args, in, grad, DBS_HIP_GRAD_F32, 0, workspace, workspace_bytes, stream, pool);
}

int path_draws_for_host(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, const PoolGrads* pool,
                        float* draws, hipStream_t stream) {
    if (!valid_args(args) || !in || !draws || !in->parents || !in->tokens || !in->lengths || !in->from_logprob)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    BackwardParams p{};
    p.B = a.batch_size;
    p.T = a.steps;
    p.K = a.beam_size;
    p.V = a.vocab_size;
    p.alpha = a.length_penalty_alpha;
    p.steps = a.steps_per_example;
    p.parents = in->parents;
    p.tokens = in->tokens;
    p.lengths = in->lengths;
    p.from_logprob = in->from_logprob;
    p.g_final = in->grad_final_scores;
    p.g_final_raw = in->grad_final_raw_scores;
    p.g_scores = in->grad_scores;
    p.g_raw = in->grad_raw_scores;
    p.draws = draws;
    set_pool_grads(p, pool);
    return finish(stream, launch_path_walk(p, stream));
}

}  // namespace dbs_hip

namespace {

// ---------------------------------------------------------------------------
// The decode that allocates nothing (dbs_hip_decode_noalloc)
// ---------------------------------------------------------------------------

// Its workspace: a static device array, one copy per GPU the library runs on
// (held until the process ends), shared by every call on that GPU. In host
// code the name is only a stand-in: the kernels get each device's address
// from hipGetSymbolAddress, taken once per device with that device current.
__device__ __align__(256) unsigned char scratch[DBS_HIP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// The current device's scratch address (set up on the device's first call).
hipError_t scratch_address(void** out) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace

extern "C" {

DBS_CUDA_EXPORT int dbs_cuda_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n > 0 ? 1 : 0;
}

DBS_CUDA_EXPORT const char* dbs_cuda_status_string(int status) {
    switch (status) {
        case DBS_CUDA_STATUS_OK: return "ok";
        case DBS_CUDA_STATUS_UNAVAILABLE: return "no usable GPU";
        case DBS_CUDA_STATUS_INVALID_ARGUMENT: return "invalid argument";
        case DBS_CUDA_STATUS_LAUNCH_FAILED: return "kernel launch failed";
        case DBS_CUDA_STATUS_OUT_OF_MEMORY: return "out of device memory";
        case DBS_HIP_STATUS_SCRATCH_LIMIT:
            return "the decode needs more than the static scratch of dbs_hip_decode_noalloc "
                   "(DBS_HIP_NOALLOC_SCRATCH_BYTES); call dbs_hip_decode_ex3 with a workspace";
        default: return "unknown status";
    }
}

DBS_CUDA_EXPORT int dbs_cuda_set_synchronization(int synchronize) {
    if (synchronize != 0 && synchronize != 1) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    g_sync.store(synchronize, std::memory_order_relaxed);
    return DBS_CUDA_STATUS_OK;
}

DBS_CUDA_EXPORT int dbs_cuda_get_synchronization(void) { return g_sync.load(std::memory_order_relaxed); }

DBS_CUDA_EXPORT int64_t dbs_cuda_decode_workspace_size(const DBSCudaDecodeArgs* args) {
    if (!valid_args(args)) return -1;
    return static_cast<int64_t>(
        decode_layout(args->batch_size, args->steps, args->beam_size, args->vocab_size, constrained(*args), false, 0)
            .total);
}

DBS_CUDA_EXPORT int64_t dbs_cuda_backward_workspace_size(const DBSCudaDecodeArgs* args) {
    if (!valid_args(args)) return -1;
    return static_cast<int64_t>(backward_workspace_bytes(args->batch_size, args->steps, args->beam_size) + 256);
}

DBS_CUDA_EXPORT int64_t dbs_cuda_decode_step_workspace_size(const DBSCudaDecodeArgs* args, int prefix_stride) {
    if (!valid_args(args) || args->steps != 1 || args->steps_per_example ||
        prefix_stride < 0)
        return -1;
    return static_cast<int64_t>(decode_layout(args->batch_size, 1, args->beam_size, args->vocab_size,
                                              constrained(*args), true, prefix_stride)
                                    .total);
}

DBS_CUDA_EXPORT int dbs_cuda_decode(const float* log_probs, const DBSCudaDecodeArgs* args,
                                    const DBSCudaDecodeOutputs* outputs, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
    return decode_common(log_probs, DBS_CUDA_DTYPE_F32, 0, args, nullptr, nullptr, outputs, nullptr, workspace,
                         workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_decode_ex(const void* inputs, int data_type, int from_logits,
                                       const DBSCudaDecodeArgs* args, const DBSCudaDecodeOutputs* outputs,
                                       float* row_lse, void* workspace, int64_t workspace_bytes, void* stream) {
    return decode_common(inputs, data_type, from_logits, args, nullptr, nullptr, outputs, row_lse, workspace,
                         workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_decode_ex2(const void* inputs, int data_type, int from_logits,
                                        const DBSCudaDecodeArgs* args, const DBSCudaSearchOptions* options,
                                        const DBSCudaDecodeOutputs* outputs, float* row_lse, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
    return decode_common(inputs, data_type, from_logits, args, options, nullptr, outputs, row_lse, workspace,
                         workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_hip_decode_ex3(const void* inputs, int data_type, int from_logits,
                                       const DBSCudaDecodeArgs* args, const DBSCudaSearchOptions* options,
                                       const uint8_t* banned_per_example, const DBSCudaDecodeOutputs* outputs,
                                       float* row_lse, void* workspace, int64_t workspace_bytes, void* stream) {
    return decode_common(inputs, data_type, from_logits, args, options, banned_per_example, outputs, row_lse,
                         workspace, workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_hip_decode_ex4(const void* inputs, int data_type, int from_logits,
                                       const DBSCudaDecodeArgs* args, const DBSCudaSearchOptions* options,
                                       const uint8_t* banned_per_example, const DBSCudaDecodeOutputs* outputs,
                                       float* row_lse, void* workspace, int64_t workspace_bytes,
                                       int32_t** fault_word, void* stream) {
    if (!fault_word) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    *fault_word = nullptr;
    return decode_common(inputs, data_type, from_logits, args, options, banned_per_example, outputs, row_lse,
                         workspace, workspace_bytes, stream, true, nullptr, fault_word);
}

DBS_CUDA_EXPORT int dbs_hip_decode_read_back(const void* src, int64_t bytes, void* dst, const int32_t* fault_word,
                                             void* stream) {
    if (bytes < 0 || (bytes > 0 && (!src || !dst))) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const hipError_t e = decode_read_back(src, static_cast<size_t>(bytes), dst, fault_word,
                                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) (void)hipGetLastError();
    return status_of(e);
}

DBS_CUDA_EXPORT int dbs_hip_decode_noalloc(const void* inputs, int data_type, int from_logits,
                                           const DBSCudaDecodeArgs* args, const DBSCudaSearchOptions* options,
                                           const uint8_t* banned_per_example, const DBSCudaDecodeOutputs* outputs,
                                           float* row_lse, void* stream) {
    if (!inputs || !valid_dtype(data_type) || !valid_args(args) || !outputs || !outputs->final_scores)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    if (!valid_options(options, *args)) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    const DecodeLayout L =
        decode_layout(a.batch_size, a.steps, a.beam_size, a.vocab_size, constrained(a), false, 0);
    if (L.total > static_cast<size_t>(DBS_HIP_NOALLOC_SCRATCH_BYTES)) return DBS_HIP_STATUS_SCRATCH_LIMIT;
    void* ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return status_of(e);
    }
    // the passes one after the other on the caller's stream: no second
    // stream or event is created, and nothing in the scratch needs clearing
    return decode_common(inputs, data_type, from_logits, args, options, banned_per_example, outputs, row_lse, ws,
                         DBS_HIP_NOALLOC_SCRATCH_BYTES, stream, false);
}

DBS_CUDA_EXPORT int dbs_cuda_decode_step(const float* log_probs, const DBSCudaDecodeArgs* args,
                                         const DBSCudaBeamState* state, const DBSCudaDecodeOutputs* outputs,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
    return step_common(log_probs, DBS_CUDA_DTYPE_F32, 0, args, nullptr, state, outputs, nullptr, workspace,
                       workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_decode_step_ex(const void* inputs, int data_type, int from_logits,
                                            const DBSCudaDecodeArgs* args, const DBSCudaBeamState* state,
                                            const DBSCudaDecodeOutputs* outputs, float* row_lse, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
    return step_common(inputs, data_type, from_logits, args, nullptr, state, outputs, row_lse, workspace,
                       workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_decode_step_ex2(const void* inputs, int data_type, int from_logits,
                                             const DBSCudaDecodeArgs* args, const DBSCudaSearchOptions* options,
                                             const DBSCudaBeamState* state, const DBSCudaDecodeOutputs* outputs,
                                             float* row_lse, void* workspace, int64_t workspace_bytes, void* stream) {
    return step_common(inputs, data_type, from_logits, args, options, state, outputs, row_lse, workspace,
                       workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_backward(const DBSCudaDecodeArgs* args, const int32_t* parents, const int32_t* tokens,
                                      const int32_t* lengths, const uint8_t* from_logprob,
                                      const float* grad_final_scores, float* grad_log_probs, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
    if (!grad_final_scores) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    DBSCudaBackwardInputs in{};
    in.parents = parents;
    in.tokens = tokens;
    in.lengths = lengths;
    in.from_logprob = from_logprob;
    in.grad_final_scores = grad_final_scores;
    return backward_common(args, &in, grad_log_probs, 0, 1, workspace, workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_backward_ex(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* inputs,
                                         float* grad_inputs, void* workspace, int64_t workspace_bytes, void* stream) {
    return backward_common(args, inputs, grad_inputs, 0, 1, workspace, workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_hip_backward_dense(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* inputs,
                                           void* grad_out, int grad_type, void* workspace, int64_t workspace_bytes,
                                           void* stream) {
    const int mode = (grad_type & DBS_HIP_GRAD_ZEROED) ? 2 : 0;
    grad_type &= ~DBS_HIP_GRAD_ZEROED;
    if (grad_type != DBS_HIP_GRAD_F32 && grad_type != DBS_HIP_GRAD_F16 && grad_type != DBS_HIP_GRAD_BF16)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    return backward_common(args, inputs, grad_out, grad_type, mode, workspace, workspace_bytes, stream);
}

DBS_CUDA_EXPORT int dbs_cuda_length_penalty(const int32_t* lengths, int64_t count, float alpha, float* out,
                                            void* stream_ptr) {
    if (count < 0 || (count > 0 && (!lengths || !out)) || !std::isfinite(alpha) || alpha < 0.0f)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream, launch_length_penalty(lengths, count, alpha, out, stream));
}

DBS_CUDA_EXPORT int dbs_cuda_path_gradient(const DBSCudaDecodeArgs* args, const int32_t* parents,
                                           const int32_t* tokens, const int32_t* lengths,
                                           const uint8_t* from_logprob, const float* grad_final_scores, float* draws,
                                           void* stream_ptr) {
    if (!valid_args(args) || !parents || !tokens || !lengths || !from_logprob || !grad_final_scores || !draws)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    const DBSCudaDecodeArgs& a = *args;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (has_per_example(a)) {
        Scratch scratch;
        bool too_small = false;
        hipError_t e = scratch.acquire(nullptr, 0, 256, stream, &too_small);
        if (e != hipSuccess) return finish(stream, e);
        const int checked = check_per_example(a, static_cast<int32_t*>(scratch.ptr), stream);
        if (checked != DBS_CUDA_STATUS_OK) return checked;
    }
    BackwardParams p{};
    p.B = a.batch_size;
    p.T = a.steps;
    p.K = a.beam_size;
    p.V = a.vocab_size;
    p.alpha = a.length_penalty_alpha;
    p.steps = a.steps_per_example;
    p.beams = a.beam_sizes_per_example;
    p.parents = parents;
    p.tokens = tokens;
    p.lengths = lengths;
    p.from_logprob = from_logprob;
    p.g_final = grad_final_scores;
    p.draws = draws;
    return finish(stream, launch_path_walk(p, stream));
}

DBS_CUDA_EXPORT int dbs_hip_set_decode_overlap(int on) {
    if (on < -1 || on > 1) return -2;
    return dbs_hip::g_overlap.exchange(on);
}

DBS_CUDA_EXPORT int dbs_hip_set_row_pass(int kind) {
    if (kind < -1 || kind > 5 || kind == 4) return -2;
    return dbs_hip::g_row_pass_kind.exchange(kind);
}

DBS_CUDA_EXPORT int dbs_hip_set_select_pass(int kind) {
    if (kind < 0 || kind > 1) return -2;
    return dbs_hip::g_select_kind.exchange(kind);
}

DBS_CUDA_EXPORT int dbs_hip_profile_enable(int on) {
    if (on != 0 && on != 1) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_profile_mutex);
    drain_pending();
    for (int i = 0; i < kKindCount; ++i) {
        g_total_ms[i] = 0.0;
        g_launches[i] = 0;
    }
    g_profile.store(on, std::memory_order_relaxed);
    if (rescan_counter(1, nullptr) != hipSuccess) (void)hipGetLastError();
    if (wait_timeout_counter(1, nullptr) != hipSuccess) (void)hipGetLastError();
    return DBS_CUDA_STATUS_OK;
}

DBS_CUDA_EXPORT int dbs_hip_profile_read(int kernel, double* total_ms, int64_t* launches) {
    if (kernel < 0 || kernel > kKindCount + 1 || !total_ms || !launches) return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_profile_mutex);
    drain_pending();
    if (kernel >= kKindCount) {
        // rows the select pass had to rescan in full / overlapped-decode waits
        // that gave up, since profiling was enabled
        unsigned long long n = 0;
        const hipError_t e = kernel == kKindCount ? rescan_counter(0, &n) : wait_timeout_counter(0, &n);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return DBS_CUDA_STATUS_LAUNCH_FAILED;
        }
        *total_ms = 0.0;
        *launches = static_cast<int64_t>(n);
        return DBS_CUDA_STATUS_OK;
    }
    *total_ms = g_total_ms[kernel];
    *launches = g_launches[kernel];
    return DBS_CUDA_STATUS_OK;
}

DBS_CUDA_EXPORT int dbs_hip_backtrack(const int32_t* tokens, const int32_t* parents, const int32_t* steps_per_example,
                                      int batch_size, int steps, int beam_size, int64_t* sequences, void* stream_ptr) {
    if (!tokens || !parents || !sequences || batch_size <= 0 || steps <= 0 || beam_size <= 0 ||
        beam_size > DBS_CUDA_MAX_BEAM)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream,
                  launch_backtrack(tokens, parents, steps_per_example, batch_size, steps, beam_size, sequences, stream));
}

DBS_CUDA_EXPORT int dbs_hip_widen_trace(const int32_t* final_lengths, const int32_t* tokens, const int32_t* parents,
                                        const int32_t* lengths, const uint8_t* from_logprob,
                                        const int32_t* steps_per_example, int batch_size, int steps, int beam_size,
                                        int64_t* final_lengths64, int64_t* tokens64, int64_t* parents64,
                                        int64_t* lengths64, uint8_t* from_logprob_bool, int64_t* steps64,
                                        void* stream_ptr) {
    if (!final_lengths || !tokens || !parents || !lengths || !from_logprob || !final_lengths64 || !tokens64 ||
        !parents64 || !lengths64 || !from_logprob_bool || !steps64 || batch_size <= 0 || steps <= 0 ||
        beam_size <= 0)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    WidenTrace w{};
    w.final_len = final_lengths;
    w.tokens = tokens;
    w.parents = parents;
    w.lengths = lengths;
    w.flp = from_logprob;
    w.steps = steps_per_example;
    w.final_len64 = final_lengths64;
    w.tokens64 = tokens64;
    w.parents64 = parents64;
    w.lengths64 = lengths64;
    w.flp_bool = from_logprob_bool;
    w.steps64 = steps64;
    w.n_final = static_cast<int64_t>(batch_size) * beam_size;
    w.n_trace = w.n_final * steps;
    w.n_steps = batch_size;
    w.T = steps;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream, launch_widen_trace(w, stream));
}

DBS_CUDA_EXPORT int dbs_hip_backtrack_i64(const int64_t* tokens, const int64_t* parents,
                                          const int64_t* steps_per_example, int batch_size, int steps, int beam_size,
                                          int64_t* sequences, void* stream_ptr) {
    if (!tokens || !parents || !sequences || batch_size <= 0 || steps <= 0 || beam_size <= 0 ||
        beam_size > DBS_CUDA_MAX_BEAM)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream, launch_backtrack(tokens, parents, steps_per_example, nullptr, batch_size, steps, beam_size,
                                           sequences, stream));
}

DBS_CUDA_EXPORT int dbs_hip_search_sequences(const int64_t* tokens, const int64_t* parents,
                                             const int64_t* steps_per_example, const int64_t* final_lengths,
                                             int batch_size, int steps, int beam_size, int64_t* sequences,
                                             void* stream_ptr) {
    if (!tokens || !parents || !final_lengths || !sequences || batch_size <= 0 || steps <= 0 || beam_size <= 0 ||
        beam_size > DBS_CUDA_MAX_BEAM)
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream, launch_backtrack(tokens, parents, steps_per_example, final_lengths, batch_size, steps,
                                           beam_size, sequences, stream));
}

DBS_CUDA_EXPORT int dbs_hip_minimum_risk(const float* scores, const float* costs, int batch_size, int beam_size,
                                         float temperature, int reduction, float* risk, float* loss,
                                         float* grad_factor, void* stream_ptr) {
    if (!scores || !costs || !risk || !grad_factor || batch_size <= 0 || beam_size <= 0 ||
        !(temperature > 0.0f) || !(temperature < kInf) || reduction < 0 || reduction > 2 ||
        (reduction != 0 && !loss))
        return DBS_CUDA_STATUS_INVALID_ARGUMENT;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    return finish(stream, launch_risk(scores, costs, batch_size, beam_size, temperature, reduction, risk, loss,
                                      grad_factor, stream));
}

}  // extern "C"
