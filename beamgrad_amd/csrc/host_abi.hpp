// SPDX-License-Identifier: MIT
//
// Shared parts of the libdbs host C ABI (include/dbs.h) served by the HIP
// engine: the decoder handle, its device buffers, error and status handling,
// and the two drivers every entry point goes through, a decode of a batch
// and the per-slot path gradients of a trace, both with host arrays in and
// out (host_abi.cpp defines them; host_results.cpp builds the result,
// backward, model-step, statistics and workspace entry points on them).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <limits>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "dbs.h"

namespace dbs_host {

// Device buffers of one handle, by purpose; grown on demand, freed with the
// handle.
enum Slot : int {
    kInputs, kBanned, kBannedPe, kSteps, kBeams, kEos, kMinLengths, kFinalScores, kFinalRaw, kFinalLengths, kTokens,
    kParents, kLengths, kScores, kRawScores, kFromLogprob, kRowLse, kFirstInvalid, kWorkspace, kGradFinal,
    kGradFinalRaw, kGradScores, kGradRaw, kDraws, kDense, kState, kForced, kPoolParents, kPoolTokens,
    kPoolLengths, kPoolScores, kPoolRaw, kPoolFromLogprob, kPoolD, kRowMask, kSlotCount
};

struct Arena {
    void* ptr[kSlotCount] = {};
    size_t size[kSlotCount] = {};

    void* get(Slot s, size_t bytes);
    void release();
};

// Device bytes the library holds in handle buffers (dbs_allocator_byte_count)
// and the buffer allocations made (dbs_allocator_call_count).
extern std::atomic<int64_t> g_device_bytes;
extern std::atomic<int64_t> g_device_allocations;

}  // namespace dbs_host

struct DBSDecoderHandle {
    // options after their defaults (reference src/c_api.cpp:160-189)
    int beam_size = 8;
    int eos_token = -1;
    float alpha = 0.0f;
    int min_length = 0;
    int validate = 0;
    int pool_multiplier = 0;
    float selected_temperature = 1.0f;
    float soft_topk_temperature = 0.25f;
    float soft_topk_tolerance = 1.0e-4f;
    int soft_topk_max_iters = 48;
    int64_t max_dense_gradient_elements = 100000000;
    std::vector<int32_t> extra_eos;

    std::mutex error_mutex;
    std::string error;

    std::mutex stats_mutex;
    DBSStatsC stats{};
    std::atomic<uint64_t> seed{0};

    std::mutex run_mutex;  // one GPU call at a time on a handle
    dbs_host::Arena arena;
    // host arrays the handle builds for a copy to the device (they outlive
    // the asynchronous copy; guarded by run_mutex)
    std::vector<int32_t> staged_forced;
    hipStream_t stream = nullptr;
    int device = -1;

    ~DBSDecoderHandle() {
        arena.release();
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace dbs_host {

// The value DBSStatsC::last_kernel reports for this library (the reference's
// codes are its CPU paths, 0-4): the HIP engine.
constexpr int kKernelHip = 5;

void need(bool ok, const char* message);
size_t mul(size_t a, size_t b, const char* what);
// An input error of one example, prefixed as the reference's batch functions
// do (reference src/c_api.cpp:264-267).
[[noreturn]] void example_error(int b, const std::string& what);

// Records an error (thread and handle) with its DBSStatsC category: 0 none,
// 1 invalid argument, 2 runtime, 3 allocation, 4 overflow.
void record(DBSDecoderHandle* h, const std::string& message, int category);
const char* last_thread_error();

// Runs body and turns its exceptions into the ABI's statuses as the
// reference does (reference src/c_api.cpp:78-101); a success clears the
// recorded errors.
template <class Body>
int run(DBSDecoderHandle* h, Body&& body) {
    try {
        body();
        record(h, std::string(), 0);
        return DBS_OK;
    } catch (const std::invalid_argument& e) {
        record(h, e.what(), 1);
        return DBS_ERROR_INVALID_ARGUMENT;
    } catch (const std::overflow_error& e) {
        record(h, e.what(), 4);
        return DBS_ERROR_INVALID_ARGUMENT;
    } catch (const std::length_error& e) {
        record(h, e.what(), 4);
        return DBS_ERROR_INVALID_ARGUMENT;
    } catch (const std::bad_alloc&) {
        record(h, "out of memory", 3);
        return DBS_ERROR_RUNTIME;
    } catch (const std::exception& e) {
        record(h, e.what(), 2);
        return DBS_ERROR_RUNTIME;
    } catch (...) {
        record(h, "unknown exception", 2);
        return DBS_ERROR_UNKNOWN;
    }
}

void hip_check(hipError_t e, const char* what);
void engine_check(int status, const char* what);

// The handle's stream on the calling thread's device (set up on first use;
// a change of device drops the buffers of the previous one).
hipStream_t stream_of(DBSDecoderHandle* h);

template <class T>
T* upload(DBSDecoderHandle* h, Slot s, const T* host, size_t count, hipStream_t st) {
    if (!host) return nullptr;
    T* d = static_cast<T*>(h->arena.get(s, sizeof(T) * count));
    hip_check(hipMemcpyAsync(d, host, sizeof(T) * count, hipMemcpyHostToDevice, st), "copy to the device");
    return d;
}

template <class T>
T* device_out(DBSDecoderHandle* h, Slot s, const T* host, size_t count) {
    return host ? static_cast<T*>(h->arena.get(s, sizeof(T) * count)) : nullptr;
}

template <class T>
void download(T* host, const T* dev, size_t count, hipStream_t st) {
    if (host && dev) hip_check(hipMemcpyAsync(host, dev, sizeof(T) * count, hipMemcpyDeviceToHost, st), "copy back");
}

size_t dtype_bytes(int data_type);
void check_dtype(int data_type);

// Steps of each example (reference src/c_api.cpp:269-279).
std::vector<int32_t> steps_of(const int32_t* steps_per_example, int B, int T);

// The engine's own limits (device ABI): K <= DBS_CUDA_MAX_BEAM, candidate
// indices K * V within int32, at most DBS_CUDA_MAX_EXTRA_EOS extra EOS tokens.
void check_engine_limits(const DBSDecoderHandle* h, int K, int V);

// One decode of a batch [B, T, K, V] on the handle's GPU, host arrays in and
// out; the arguments were checked by the caller. Per-example arrays (steps,
// beams, EOS tokens, minimum lengths, banned masks [B, V]) may be null. With
// the handle's validate_inputs, the first example whose search read a row
// holding NaN or +inf raises (" (step t, beam k)" after the reference's
// text, prefixed with the example where `batch_errors`).
struct DecodeJob {
    const void* inputs = nullptr;
    int data_type = DBS_DTYPE_F32;
    bool from_logits = false;
    int B = 0, T = 0, K = 0, V = 0;
    const int32_t* steps = nullptr;
    const int32_t* beams = nullptr;
    const int32_t* eos = nullptr;
    const int32_t* min_lengths = nullptr;
    const uint8_t* banned = nullptr;     // [V], every example
    const uint8_t* banned_pe = nullptr;  // [B, V]
    // forced tokens: example b's step t reads forced[b * forced_stride + t]
    // (stride 0: one [T] array for every example), for t below its steps
    const int32_t* forced = nullptr;
    size_t forced_stride = 0;
    int min_length = 0;
    int ngram = 0;
    float repetition_penalty = 1.0f;
    bool batch_errors = true;
    // outputs ([B, K] and [B, T, K]); final_scores is required
    float* final_scores = nullptr;
    float* final_raw = nullptr;
    int32_t* final_lengths = nullptr;
    int32_t* tokens = nullptr;
    int32_t* parents = nullptr;
    int32_t* lengths = nullptr;
    float* scores = nullptr;
    float* raw_scores = nullptr;
    uint8_t* from_logprob = nullptr;
    float* row_lse = nullptr;
    // the relaxed pool ([B, T, pool_mult * K]; pool_mult 0: none)
    int pool_mult = 0;
    int32_t* pool_parents = nullptr;
    int32_t* pool_tokens = nullptr;
    int32_t* pool_lengths = nullptr;
    float* pool_scores = nullptr;
    float* pool_raw = nullptr;
    uint8_t* pool_from_logprob = nullptr;
};
void run_decode(DBSDecoderHandle* h, const DecodeJob& job);

// dbs_decode_batch_into(_ex) with a token filter (host_results.cpp): each
// example decoded step by step on the device step API, the filter's
// verdicts for each step's rows asked on the host in the reference's call
// order (reference src/decoder.cpp:259-282).
void decode_batch_filtered(DBSDecoderHandle* h, const void* inputs, int data_type, bool from_logits, int B, int T,
                           int V, const std::vector<int32_t>& steps_b, const DBSAdvancedConstraintsC* cons,
                           const DBSDecodeOutputsC* out, const DBSDecodeOutputsExC* ex);

// The relaxed pool's size for beam K and multiplier m (reference
// src/decoder.cpp:410-416), refused past what the HIP engine keeps per step.
int pool_size_of(int K, int m);

// Gradients of a trace's outputs; any may be null.
struct Grads {
    const float* final_scores = nullptr;  // [B, K]
    const float* final_raw = nullptr;     // [B, K]
    const float* scores = nullptr;        // [B, T, K]
    const float* raw = nullptr;           // [B, T, K]
};

// Relaxed-pool entries of a backward, host arrays [B, T, P] (P 0: none):
// the pool trace and each entry's raw-score gradient d.
struct PoolTerms {
    int P = 0;
    const int32_t* parents = nullptr;
    const int32_t* tokens = nullptr;
    const int32_t* lengths = nullptr;
    const uint8_t* from_logprob = nullptr;
    std::vector<float> d;
};

// d of the pool entries of one example's T steps (reference
// src/decoder.cpp:617-657): the relaxed weights' term (r: the forward's
// relaxed weights, gr: their gradient, [T, P] or null; soft_temperature the
// forward's), then the pool score and raw-score gradients (or null); 0 for
// dead entries.
void pool_entry_grads(int T, int P, float alpha, float soft_temperature, const int32_t* parents,
                      const int32_t* lengths, const float* r, const float* gr, const float* g_scores,
                      const float* g_raw, float* d);

// The checks of a trace handed to a backward (reference src/decoder.cpp:
// 947-985): indexes in range over each example's own steps, the pool
// trace's after the trace's.
void check_trace(int B, int T, int K, int V, const std::vector<int32_t>& steps_b, const int32_t* parents,
                 const int32_t* tokens, const int32_t* lengths, const PoolTerms* pool = nullptr);

// The per-slot path gradients [B, T, K] of a checked trace (host arrays) on
// the handle's GPU: slot (b, t, k) gets the raw-score gradient its selected
// entry receives (reference src/decoder.cpp:540-610), 0 where it has none;
// the pool entries' d join their parents' incoming gradients.
std::vector<float> path_draws(DBSDecoderHandle* h, int B, int T, int K, int V, float alpha,
                              const int32_t* steps_per_example, const int32_t* parents, const int32_t* tokens,
                              const int32_t* lengths, const uint8_t* from_logprob, const Grads& g,
                              const PoolTerms* pool = nullptr);

// The log-prob entries of step t of example b (selected slots' draws, then
// the pool entries' d, each merged per entry from 0 in that order; reference
// src/decoder.cpp:668-683): (index into the example's [T, K, V], value),
// increasing index.
std::vector<std::pair<int64_t, float>> step_entries(int T, int K, int V, int b, int t, const std::vector<float>& draws,
                                                    const int32_t* parents, const int32_t* tokens,
                                                    const uint8_t* from_logprob, const PoolTerms* pool);

// DBSStatsC bookkeeping (reference src/c_api.cpp:117-158).
void stats_decode(DBSDecoderHandle* h, int64_t elapsed_ns, int64_t selected, int64_t pool, int64_t logprobs,
                  int64_t allocation_bytes, bool model_step);
void stats_backward(DBSDecoderHandle* h, int64_t elapsed_ns, bool sparse, int64_t sparse_count);

}  // namespace dbs_host
