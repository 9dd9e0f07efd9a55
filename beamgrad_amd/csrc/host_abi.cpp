// SPDX-License-Identifier: MIT
//
// The libdbs host C ABI (include/dbs.h) served by the HIP engine: decoder
// handles and the batch entry points of the reference's host library
// (reference src/c_api.cpp:312-400, 700-983), with host arrays in and out,
// and the two drivers the other entry points (host_results.cpp) share.
//
// A call checks its arguments as the reference does, with the same status
// and error text, stages the host arrays into device buffers owned by the
// handle (kept between calls, grown on demand), runs the device decode or
// path walk on the handle's stream, and copies the results back. The
// backward accumulates into the caller's host buffer exactly where the
// reference's does: the log-prob entries on the beams' paths (from the
// per-slot path gradients), or, from logits, the whole rows on those paths
// (from the device's log-softmax gradient rows, computed a bounded chunk of
// examples at a time).
#include "host_abi.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <exception>

#include "dbs_cuda.h"
#include "dbs_hip.h"
#include "host_entry.hpp"
#include "numerics.hpp"

namespace dbs_host {

std::atomic<int64_t> g_device_bytes{0};
std::atomic<int64_t> g_device_allocations{0};

namespace {
thread_local std::string t_error;  // the calling thread's latest error
}  // namespace

void* Arena::get(Slot s, size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (size[s] < bytes) {
        if (ptr[s]) {
            (void)hipFree(ptr[s]);
            g_device_bytes -= static_cast<int64_t>(size[s]);
        }
        ptr[s] = nullptr;
        size[s] = 0;
        if (hipMalloc(&ptr[s], bytes) != hipSuccess) {
            (void)hipGetLastError();
            ptr[s] = nullptr;
            throw std::bad_alloc();
        }
        size[s] = bytes;
        g_device_bytes += static_cast<int64_t>(bytes);
        ++g_device_allocations;
    }
    return ptr[s];
}

void Arena::release() {
    for (int i = 0; i < kSlotCount; ++i) {
        if (ptr[i]) {
            (void)hipFree(ptr[i]);
            g_device_bytes -= static_cast<int64_t>(size[i]);
        }
        ptr[i] = nullptr;
        size[i] = 0;
    }
}

void need(bool ok, const char* message) {
    if (!ok) throw std::invalid_argument(message);
}

size_t mul(size_t a, size_t b, const char* what) {
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a) throw std::overflow_error(what);
    return a * b;
}

void example_error(int b, const std::string& what) {
    throw std::invalid_argument("example " + std::to_string(b) + ": " + what);
}

void record(DBSDecoderHandle* h, const std::string& message, int category) {
    t_error = message;
    if (h) {
        {
            std::lock_guard<std::mutex> lock(h->error_mutex);
            h->error = message;
        }
        if (category != 0) {
            std::lock_guard<std::mutex> lock(h->stats_mutex);
            h->stats.last_error_category = category;
        }
    }
}

const char* last_thread_error() { return t_error.c_str(); }

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void engine_check(int status, const char* what) {
    if (status == DBS_CUDA_STATUS_OK) return;
    if (status == DBS_CUDA_STATUS_OUT_OF_MEMORY) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + dbs_cuda_status_string(status));
}

hipStream_t stream_of(DBSDecoderHandle* h) {
    int device = 0;
    hip_check(hipGetDevice(&device), "no usable GPU");
    if (h->stream && h->device != device) {
        h->arena.release();
        (void)hipStreamDestroy(h->stream);
        h->stream = nullptr;
    }
    if (!h->stream) {
        hip_check(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), "stream creation");
        h->device = device;
    }
    return h->stream;
}

size_t dtype_bytes(int data_type) { return data_type == DBS_DTYPE_F32 ? 4 : 2; }

void check_dtype(int data_type) {
    need(data_type == DBS_DTYPE_F32 || data_type == DBS_DTYPE_F16 || data_type == DBS_DTYPE_BF16,
         "unsupported DBS data type");
}

std::vector<int32_t> steps_of(const int32_t* steps_per_example, int B, int T) {
    std::vector<int32_t> out(static_cast<size_t>(B), T);
    if (!steps_per_example) return out;
    for (int b = 0; b < B; ++b) {
        if (steps_per_example[b] < 1 || steps_per_example[b] > T)
            throw std::invalid_argument("steps_per_example[" + std::to_string(b) + "] must be in [1, steps]");
        out[static_cast<size_t>(b)] = steps_per_example[b];
    }
    return out;
}

void check_engine_limits(const DBSDecoderHandle* h, int K, int V) {
    if (K > DBS_CUDA_MAX_BEAM || static_cast<int64_t>(K) * V > std::numeric_limits<int32_t>::max())
        throw std::invalid_argument("beam_size " + std::to_string(K) + " with vocab_size " + std::to_string(V) +
                                    " is beyond the HIP engine (beam_size <= " + std::to_string(DBS_CUDA_MAX_BEAM) +
                                    ", beam_size * vocab_size < 2^31)");
    if (h->extra_eos.size() > static_cast<size_t>(DBS_CUDA_MAX_EXTRA_EOS))
        throw std::invalid_argument("more than " + std::to_string(DBS_CUDA_MAX_EXTRA_EOS) +
                                    " extra EOS tokens are beyond the HIP engine");
}

int pool_size_of(int K, int m) {
    if (m <= 0) return 0;
    const int64_t P = static_cast<int64_t>(K) * m;
    if (P > DBS_CUDA_MAX_BEAM)
        throw std::invalid_argument("a relaxed pool of " + std::to_string(P) + " candidates (beam_size * " +
                                    "relaxed_pool_multiplier) is beyond the HIP engine (at most " +
                                    std::to_string(DBS_CUDA_MAX_BEAM) + ")");
    return static_cast<int>(P);
}

void run_decode(DBSDecoderHandle* h, const DecodeJob& j) {
    const int B = j.B, T = j.T, K = j.K, V = j.V;
    check_engine_limits(h, K, V);
    const int P = pool_size_of(K, j.pool_mult);
    const size_t BK = static_cast<size_t>(B) * K;
    const size_t BTK = mul(BK, static_cast<size_t>(T), "batch size overflow");
    const size_t elements = mul(BTK, static_cast<size_t>(V), "batch size overflow");

    std::lock_guard<std::mutex> lock(h->run_mutex);
    const hipStream_t st = stream_of(h);
    const void* x = upload(h, kInputs, static_cast<const unsigned char*>(j.inputs), elements * dtype_bytes(j.data_type),
                           st);
    DBSCudaDecodeArgs a{};
    a.batch_size = B;
    a.steps = T;
    a.beam_size = K;
    a.vocab_size = V;
    a.eos_token = h->eos_token;
    a.min_length = j.min_length;
    a.length_penalty_alpha = h->alpha;
    a.no_repeat_ngram_size = j.ngram;
    a.repetition_penalty = j.repetition_penalty;
    a.steps_per_example = upload(h, kSteps, j.steps, static_cast<size_t>(B), st);
    a.beam_sizes_per_example = upload(h, kBeams, j.beams, static_cast<size_t>(B), st);
    a.eos_tokens_per_example = upload(h, kEos, j.eos, static_cast<size_t>(B), st);
    a.min_lengths_per_example = upload(h, kMinLengths, j.min_lengths, static_cast<size_t>(B), st);
    a.banned_tokens = upload(h, kBanned, j.banned, static_cast<size_t>(V), st);
    const uint8_t* banned_pe = upload(h, kBannedPe, j.banned_pe, mul(static_cast<size_t>(B), V, "banned size"), st);
    // forced tokens as the device reads them: [B, T], -1 past an example's
    // steps; none at all when no step is forced (the decode keeps every
    // select pass open to it)
    std::vector<int32_t>& forced_bt = h->staged_forced;
    bool any_forced = false;
    if (j.forced) {
        const std::vector<int32_t> steps_b = steps_of(j.steps, B, T);
        forced_bt.assign(mul(static_cast<size_t>(B), static_cast<size_t>(T), "forced size"), -1);
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < steps_b[static_cast<size_t>(b)]; ++t) {
                const int32_t f = j.forced[static_cast<size_t>(b) * j.forced_stride + t];
                forced_bt[static_cast<size_t>(b) * T + t] = f;
                any_forced = any_forced || f >= 0;
            }
    }
    const int32_t* forced = upload(h, kForced, any_forced ? forced_bt.data() : nullptr, forced_bt.size(), st);
    DBSCudaSearchOptions opts{};
    opts.extra_eos_count = static_cast<int>(h->extra_eos.size());
    for (size_t i = 0; i < h->extra_eos.size(); ++i) opts.extra_eos_tokens[i] = h->extra_eos[i];

    DBSCudaDecodeOutputs o{};
    o.final_scores = device_out(h, kFinalScores, j.final_scores, BK);
    o.final_raw_scores = device_out(h, kFinalRaw, j.final_raw, BK);
    o.final_lengths = device_out(h, kFinalLengths, j.final_lengths, BK);
    o.tokens = device_out(h, kTokens, j.tokens, BTK);
    o.parents = device_out(h, kParents, j.parents, BTK);
    o.lengths = device_out(h, kLengths, j.lengths, BTK);
    o.scores = device_out(h, kScores, j.scores, BTK);
    o.raw_scores = device_out(h, kRawScores, j.raw_scores, BTK);
    o.from_logprob = device_out(h, kFromLogprob, j.from_logprob, BTK);
    float* row_lse = device_out(h, kRowLse, j.row_lse, BTK);
    const size_t BTP = static_cast<size_t>(B) * T * static_cast<size_t>(P);
    dbs_hip::PoolOutputs pool;
    if (P > 0) {
        pool.mult = j.pool_mult;
        pool.parents = device_out(h, kPoolParents, j.pool_parents, BTP);
        pool.tokens = device_out(h, kPoolTokens, j.pool_tokens, BTP);
        pool.lengths = device_out(h, kPoolLengths, j.pool_lengths, BTP);
        pool.scores = device_out(h, kPoolScores, j.pool_scores, BTP);
        pool.raw_scores = device_out(h, kPoolRaw, j.pool_raw, BTP);
        pool.from_logprob = device_out(h, kPoolFromLogprob, j.pool_from_logprob, BTP);
    }
    int32_t* first_invalid =
        h->validate ? static_cast<int32_t*>(h->arena.get(kFirstInvalid, sizeof(int32_t) * static_cast<size_t>(B)))
                    : nullptr;
    const int64_t ws_bytes = dbs_hip::workspace_for_host(&a, pool.mult, 0, 0);
    need(ws_bytes > 0, "invalid decode arguments");
    void* ws = h->arena.get(kWorkspace, static_cast<size_t>(ws_bytes));
    int32_t* fault = nullptr;
    engine_check(dbs_hip::decode_for_host(x, j.data_type, j.from_logits ? 1 : 0, &a, &opts, banned_pe, &o, row_lse,
                                          first_invalid, forced, P > 0 ? &pool : nullptr, ws, ws_bytes, st, &fault),
                 "HIP decode");
    int32_t gave_up = 0;
    if (fault) download(&gave_up, fault, 1, st);
    std::vector<int32_t> bad;
    if (first_invalid) {
        bad.resize(static_cast<size_t>(B));
        download(bad.data(), first_invalid, bad.size(), st);
    }
    download(j.final_scores, o.final_scores, BK, st);
    download(j.final_raw, o.final_raw_scores, BK, st);
    download(j.final_lengths, o.final_lengths, BK, st);
    download(j.tokens, o.tokens, BTK, st);
    download(j.parents, o.parents, BTK, st);
    download(j.lengths, o.lengths, BTK, st);
    download(j.scores, o.scores, BTK, st);
    download(j.raw_scores, o.raw_scores, BTK, st);
    download(j.from_logprob, o.from_logprob, BTK, st);
    download(j.row_lse, row_lse, BTK, st);
    if (P > 0) {
        download(j.pool_parents, pool.parents, BTP, st);
        download(j.pool_tokens, pool.tokens, BTP, st);
        download(j.pool_lengths, pool.lengths, BTP, st);
        download(j.pool_scores, pool.scores, BTP, st);
        download(j.pool_raw, pool.raw_scores, BTP, st);
        download(j.pool_from_logprob, pool.from_logprob, BTP, st);
    }
    hip_check(hipStreamSynchronize(st), "HIP decode");
    // the overlapped select pass gave up waiting for rows of the row pass
    // (bounded at 2 s; only when something starves or serialises the
    // kernels): the traces of those examples are padding
    if (gave_up != 0)
        throw std::runtime_error(
            "HIP decode: the select pass gave up waiting for the row pass (the GPU was starved or its kernels were "
            "serialised); the trace is incomplete");
    // validate_inputs: the first example whose search read a NaN/+inf row,
    // reported at that row (reference src/decoder.cpp:143-171)
    for (int b = 0; b < static_cast<int>(bad.size()); ++b) {
        if (bad[static_cast<size_t>(b)] < 0) continue;
        const int t = bad[static_cast<size_t>(b)] / K, k = bad[static_cast<size_t>(b)] % K;
        const std::string what = std::string(j.from_logits ? "logits contain NaN or +inf"
                                                            : "log_probs contains NaN or +inf") +
                                 " (step " + std::to_string(t) + ", beam " + std::to_string(k) + ")";
        if (j.batch_errors) example_error(b, what);
        throw std::invalid_argument(what);
    }
}

void check_trace(int B, int T, int K, int V, const std::vector<int32_t>& steps_b, const int32_t* parents,
                 const int32_t* tokens, const int32_t* lengths, const PoolTerms* pool) {
    for (int b = 0; b < B; ++b) {
        const size_t base = static_cast<size_t>(b) * T * K;
        const size_t n = static_cast<size_t>(steps_b[static_cast<size_t>(b)]) * K;
        for (size_t i = base; i < base + n; ++i) {
            if (parents[i] < -1 || parents[i] >= K || tokens[i] < -1 || tokens[i] >= V || lengths[i] < 0)
                example_error(b, "decode trace is out of range (parents, tokens or lengths)");
        }
        if (!pool || pool->P <= 0) continue;
        const size_t pbase = static_cast<size_t>(b) * T * pool->P;
        const size_t np = static_cast<size_t>(steps_b[static_cast<size_t>(b)]) * pool->P;
        for (size_t i = pbase; i < pbase + np; ++i) {
            if (pool->parents[i] < -1 || pool->parents[i] >= K || pool->tokens[i] < -1 || pool->tokens[i] >= V ||
                pool->lengths[i] < 0)
                example_error(b, "pool trace is out of range (parents, tokens or lengths)");
        }
    }
}

void pool_entry_grads(int T, int P, float alpha, float soft_temperature, const int32_t* parents,
                      const int32_t* lengths, const float* r, const float* gr, const float* g_scores,
                      const float* g_raw, float* d) {
    constexpr float kEps = 1.0e-12f;
    for (int t = 0; t < T; ++t) {
        const size_t base = static_cast<size_t>(t) * P;
        // the relaxed weights' implicit gradient through the bisected
        // threshold: a_p (gr_p - sum(gr a) / sum(a)) / temperature, a = r (1 - r)
        bool relaxed = false;
        float center = 0.0f, inv_temp = 0.0f;
        if (r && gr) {
            float denom = 0.0f, numer = 0.0f;
            for (int p = 0; p < P; ++p) {
                const float a = r[base + p] * (1.0f - r[base + p]);
                denom += a;
                numer += gr[base + p] * a;
            }
            if (denom > kEps) {
                relaxed = true;
                center = numer / denom;
                inv_temp = 1.0f / soft_temperature;
            }
        }
        for (int p = 0; p < P; ++p) {
            const size_t i = base + static_cast<size_t>(p);
            d[i] = 0.0f;
            if (parents[i] < 0) continue;
            float drank = 0.0f;
            if (relaxed) {
                const float a = r[i] * (1.0f - r[i]);
                drank += a * inv_temp * (gr[i] - center);
            }
            if (g_scores) drank += g_scores[i];
            const float inv_penalty = 1.0f / dbs_hip::length_penalty(std::max(1, static_cast<int>(lengths[i])), alpha);
            float v = drank * inv_penalty;
            if (g_raw) v += g_raw[i];
            d[i] = v;
        }
    }
}

std::vector<std::pair<int64_t, float>> step_entries(int T, int K, int V, int b, int t, const std::vector<float>& draws,
                                                    const int32_t* parents, const int32_t* tokens,
                                                    const uint8_t* from_logprob, const PoolTerms* pool) {
    std::vector<std::pair<int64_t, float>> raw;  // in the order the reference produces them
    auto index = [&](int parent, int token) {
        return (static_cast<int64_t>(t) * K + parent) * static_cast<int64_t>(V) + token;
    };
    const size_t base = (static_cast<size_t>(b) * T + t) * K;
    for (int k = 0; k < K; ++k) {
        const size_t i = base + static_cast<size_t>(k);
        if (draws[i] == 0.0f || parents[i] < 0 || !from_logprob[i] || tokens[i] < 0) continue;
        raw.emplace_back(index(parents[i], tokens[i]), draws[i]);
    }
    if (pool && pool->P > 0) {
        const size_t pbase = (static_cast<size_t>(b) * T + t) * pool->P;
        for (int p = 0; p < pool->P; ++p) {
            const size_t i = pbase + static_cast<size_t>(p);
            if (pool->d[i] == 0.0f || pool->parents[i] < 0 || !pool->from_logprob[i] || pool->tokens[i] < 0) continue;
            raw.emplace_back(index(pool->parents[i], pool->tokens[i]), pool->d[i]);
        }
    }
    std::stable_sort(raw.begin(), raw.end(), [](const auto& x, const auto& y) { return x.first < y.first; });
    std::vector<std::pair<int64_t, float>> merged;
    for (size_t i = 0; i < raw.size();) {
        float v = 0.0f;
        size_t j = i;
        for (; j < raw.size() && raw[j].first == raw[i].first; ++j) v += raw[j].second;
        merged.emplace_back(raw[i].first, v);
        i = j;
    }
    return merged;
}

namespace {

DBSCudaDecodeArgs trace_args(int B, int T, int K, int V, float alpha) {
    DBSCudaDecodeArgs a{};
    a.batch_size = B;
    a.steps = T;
    a.beam_size = K;
    a.vocab_size = V;
    a.eos_token = -1;
    a.length_penalty_alpha = alpha;
    a.repetition_penalty = 1.0f;
    return a;
}

}  // namespace

std::vector<float> path_draws(DBSDecoderHandle* h, int B, int T, int K, int V, float alpha,
                              const int32_t* steps_per_example, const int32_t* parents, const int32_t* tokens,
                              const int32_t* lengths, const uint8_t* from_logprob, const Grads& g,
                              const PoolTerms* pool) {
    check_engine_limits(h, K, V);
    const size_t BK = static_cast<size_t>(B) * K, BTK = BK * static_cast<size_t>(T);
    std::lock_guard<std::mutex> lock(h->run_mutex);
    const hipStream_t st = stream_of(h);
    DBSCudaDecodeArgs a = trace_args(B, T, K, V, alpha);
    a.steps_per_example = upload(h, kSteps, steps_per_example, static_cast<size_t>(B), st);
    DBSCudaBackwardInputs in{};
    in.parents = upload(h, kParents, parents, BTK, st);
    in.tokens = upload(h, kTokens, tokens, BTK, st);
    in.lengths = upload(h, kLengths, lengths, BTK, st);
    in.from_logprob = upload(h, kFromLogprob, from_logprob, BTK, st);
    in.grad_final_scores = upload(h, kGradFinal, g.final_scores, BK, st);
    in.grad_final_raw_scores = upload(h, kGradFinalRaw, g.final_raw, BK, st);
    in.grad_scores = upload(h, kGradScores, g.scores, BTK, st);
    in.grad_raw_scores = upload(h, kGradRaw, g.raw, BTK, st);
    float* draws_d = static_cast<float*>(h->arena.get(kDraws, sizeof(float) * BTK));
    dbs_hip::PoolGrads pg;
    if (pool && pool->P > 0) {
        const size_t BTP = static_cast<size_t>(B) * T * static_cast<size_t>(pool->P);
        pg.P = pool->P;
        pg.parents = upload(h, kPoolParents, pool->parents, BTP, st);
        pg.tokens = upload(h, kPoolTokens, pool->tokens, BTP, st);
        pg.from_logprob = upload(h, kPoolFromLogprob, pool->from_logprob, BTP, st);
        pg.d = upload(h, kPoolD, pool->d.data(), BTP, st);
    }
    engine_check(dbs_hip::path_draws_for_host(&a, &in, pg.P > 0 ? &pg : nullptr, draws_d, st), "HIP path gradient");
    std::vector<float> draws(BTK);
    download(draws.data(), draws_d, BTK, st);
    hip_check(hipStreamSynchronize(st), "HIP path gradient");
    return draws;
}

void stats_decode(DBSDecoderHandle* h, int64_t elapsed_ns, int64_t selected, int64_t pool, int64_t logprobs,
                  int64_t allocation_bytes, bool model_step) {
    std::lock_guard<std::mutex> lock(h->stats_mutex);
    h->stats.abi_version = DBS_ABI_VERSION;
    h->stats.last_kernel = kKernelHip;
    h->stats.used_batch_threads = 1;
    h->stats.used_model_step_callback = model_step ? 1 : 0;
    h->stats.last_decode_ns = elapsed_ns;
    h->stats.last_selected_count = selected;
    h->stats.last_pool_count = pool;
    h->stats.last_logprob_count = logprobs;
    h->stats.last_allocation_bytes = allocation_bytes;
    h->stats.last_error_category = 0;
}

void stats_backward(DBSDecoderHandle* h, int64_t elapsed_ns, bool sparse, int64_t sparse_count) {
    std::lock_guard<std::mutex> lock(h->stats_mutex);
    h->stats.abi_version = DBS_ABI_VERSION;
    h->stats.used_sparse_backward = sparse ? 1 : 0;
    h->stats.used_dense_backward = sparse ? 0 : 1;
    h->stats.last_backward_ns = elapsed_ns;
    h->stats.last_sparse_grad_count = sparse_count;
    h->stats.last_error_category = 0;
}

namespace {

int64_t ns_since(std::chrono::steady_clock::time_point start) {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - start).count();
}

// dbs_decode_batch_into(_ex) (reference src/c_api.cpp:703-800); ex may be null.
void decode_batch(DBSDecoderHandle* h, const void* inputs, int data_type, bool from_logits, int B, int T, int V,
                  const int32_t* steps_per_example, const DBSAdvancedConstraintsC* cons,
                  const DBSDecodeOutputsC* out, const DBSDecodeOutputsExC* ex) {
    need(h != nullptr, "decoder handle cannot be null");
    check_dtype(data_type);
    need(inputs != nullptr, "log_probs cannot be null");
    need(out != nullptr && out->final_scores != nullptr, "outputs and outputs->final_scores cannot be null");
    need(B > 0 && T > 0 && V > 0, "batch_size, steps and vocab_size must be positive");
    const bool pool = ex && (ex->pool_parents || ex->pool_tokens || ex->pool_lengths || ex->pool_scores ||
                             ex->pool_raw_scores || ex->pool_from_logprob);
    if (ex) {
        need(!ex->reserved[0] && !ex->reserved[1] && !ex->reserved[2] && !ex->reserved[3],
             "reserved fields must be NULL");
        need(!pool || h->pool_multiplier > 0, "pool outputs need a relaxed pool: set relaxed_pool_multiplier >= 1");
    }
    const auto start = std::chrono::steady_clock::now();
    const int K = h->beam_size;
    const size_t trace = mul(static_cast<size_t>(T), static_cast<size_t>(K), "batch stride overflow");
    const size_t per_example = mul(trace, static_cast<size_t>(V), "batch stride overflow");
    (void)mul(per_example, static_cast<size_t>(B), "batch size overflow");
    (void)mul(per_example, dtype_bytes(data_type), "batch stride overflow");
    const std::vector<int32_t> steps_b = steps_of(steps_per_example, B, T);

    // What the reference's decoder checks per example (reference
    // src/decoder.cpp:385-406, 779-793); the options are shared, so example
    // 0 is the first to fail.
    const int min_length = cons && cons->min_length >= 0 ? cons->min_length : h->min_length;
    const float rep = cons ? (cons->repetition_penalty > 0.0f ? cons->repetition_penalty : 1.0f) : 1.0f;
    if (h->eos_token >= V) example_error(0, "eos_token is outside the vocabulary");
    for (int32_t tok : h->extra_eos)
        if (tok >= V) example_error(0, "an extra EOS token is outside the vocabulary");
    if (cons && cons->forced_tokens) {
        // the shared array, as far as each example's own steps read it
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < steps_b[static_cast<size_t>(b)]; ++t)
                if (cons->forced_tokens[t] >= V) example_error(b, "forced token is outside the vocabulary");
    }
    if (cons && (!(rep > 0.0f) || !std::isfinite(rep)))
        example_error(0, "repetition_penalty must be finite and positive (1 disables it)");
    if (cons && cons->token_filter) {
        check_engine_limits(h, K, V);
        decode_batch_filtered(h, inputs, data_type, from_logits, B, T, V, steps_b, cons, out, ex);
    } else {
        DecodeJob j;
    j.inputs = inputs;
    j.data_type = data_type;
    j.from_logits = from_logits;
    j.B = B;
    j.T = T;
    j.K = K;
    j.V = V;
    j.steps = steps_per_example;
    j.banned = cons ? cons->banned_tokens : nullptr;
    j.forced = cons ? cons->forced_tokens : nullptr;
    j.min_length = min_length;
    j.ngram = cons && cons->no_repeat_ngram_size > 0 ? cons->no_repeat_ngram_size : 0;
    j.repetition_penalty = rep;
    j.final_scores = out->final_scores;
    j.final_raw = out->final_raw_scores;
    j.final_lengths = out->final_lengths;
    j.tokens = out->tokens;
    j.parents = out->parents;
    j.lengths = out->lengths;
    j.scores = out->scores;
    j.raw_scores = out->raw_scores;
    j.from_logprob = out->from_logprob;
    j.row_lse = ex ? ex->row_lse : nullptr;
    if (pool) {
        j.pool_mult = h->pool_multiplier;
        j.pool_parents = ex->pool_parents;
        j.pool_tokens = ex->pool_tokens;
        j.pool_lengths = ex->pool_lengths;
        j.pool_scores = ex->pool_scores;
        j.pool_raw = ex->pool_raw_scores;
        j.pool_from_logprob = ex->pool_from_logprob;
    }
    run_decode(h, j);
    }
    const int64_t selected = static_cast<int64_t>(B) * static_cast<int64_t>(trace);
    {
        std::lock_guard<std::mutex> lock(h->stats_mutex);
        h->stats.abi_version = DBS_ABI_VERSION;
        h->stats.last_kernel = kKernelHip;
        h->stats.used_batch_threads = 1;
        h->stats.used_model_step_callback = 0;
        h->stats.last_decode_ns = ns_since(start);
        h->stats.last_selected_count = selected;
        h->stats.last_pool_count = 0;
        h->stats.last_logprob_count = selected * V;
        h->stats.last_allocation_bytes = 0;
        h->stats.last_error_category = 0;
    }
}

// Device buffers a chunk of examples of the from-logits backward may take:
// the logits and a float32 gradient of its rows. Test knob
// DBS_HIP_TEST_BACKWARD_CHUNK_BYTES sets a smaller bound (one example per
// chunk at least).
size_t backward_chunk_bytes() {
    const char* env = std::getenv("DBS_HIP_TEST_BACKWARD_CHUNK_BYTES");
    if (env && env[0]) {
        const long long v = std::atoll(env);
        if (v > 0) return static_cast<size_t>(v);
    }
    return size_t{1} << 30;
}

// The backward of a batch into the host buffer grad [B, T, K, V] (+=): the
// per-slot path gradients from the device, then the entries they name, or
// with logits the device's gradient rows of every (example, step, parent)
// row that an entry lands in.
void backward_batch(DBSDecoderHandle* h, int B, int T, int V, const int32_t* steps_per_example,
                    const int32_t* parents, const int32_t* tokens, const int32_t* lengths, const uint8_t* flp,
                    const Grads& g, const void* logits, int logits_type, const float* row_lse, float* grad,
                    PoolTerms* pool, const float* g_pool_scores, const float* g_pool_raw) {
    const auto start = std::chrono::steady_clock::now();
    const int K = h->beam_size;
    const size_t trace = mul(static_cast<size_t>(T), static_cast<size_t>(K), "batch stride overflow");
    const size_t row_block = mul(trace, static_cast<size_t>(V), "batch stride overflow");
    (void)mul(row_block, static_cast<size_t>(B), "batch size overflow");
    const std::vector<int32_t> steps_b = steps_of(steps_per_example, B, T);
    const bool with_pool = pool && pool->P > 0;
    if (with_pool) {
        need(pool->P <= DBS_CUDA_MAX_BEAM, "a relaxed pool of more than 1024 candidates is beyond the HIP engine");
        (void)mul(mul(static_cast<size_t>(T), static_cast<size_t>(pool->P), "batch stride overflow"),
                  static_cast<size_t>(B), "batch size overflow");
    }
    check_trace(B, T, K, V, steps_b, parents, tokens, lengths, with_pool ? pool : nullptr);
    if (with_pool) {
        // each example's pool entries over its own steps (0 past them)
        const size_t TP = static_cast<size_t>(T) * pool->P;
        pool->d.assign(TP * static_cast<size_t>(B), 0.0f);
        for (int b = 0; b < B; ++b) {
            const size_t off = static_cast<size_t>(b) * TP;
            pool_entry_grads(steps_b[static_cast<size_t>(b)], pool->P, h->alpha, h->soft_topk_temperature,
                             pool->parents + off, pool->lengths + off, nullptr, nullptr,
                             g_pool_scores ? g_pool_scores + off : nullptr, g_pool_raw ? g_pool_raw + off : nullptr,
                             pool->d.data() + off);
        }
    }
    const std::vector<float> draws = path_draws(h, B, T, K, V, h->alpha, steps_per_example, parents, tokens, lengths,
                                                flp, g, with_pool ? pool : nullptr);
    const size_t BTK = static_cast<size_t>(B) * trace;

    // (b, t, parent) row and token of every slot with an entry: distinct
    // slots of one step select distinct (parent, token) pairs, so each entry
    // is one slot's draw (reference src/decoder.cpp:540-548, 668-683)
    auto entry_of = [&](size_t i, size_t& row, int& token) -> bool {
        if (draws[i] == 0.0f || parents[i] < 0 || !flp[i] || tokens[i] < 0) return false;
        const size_t bt = i / static_cast<size_t>(K);  // b * T + t
        row = bt * static_cast<size_t>(K) + static_cast<size_t>(parents[i]);
        token = tokens[i];
        return true;
    };
    // the pool entries' (b, t, parent) rows: entries of their own
    auto pool_row_of = [&](size_t i, size_t& row) -> bool {
        if (pool->d[i] == 0.0f || pool->parents[i] < 0 || !pool->from_logprob[i] || pool->tokens[i] < 0) return false;
        const size_t bt = i / static_cast<size_t>(pool->P);
        row = bt * static_cast<size_t>(K) + static_cast<size_t>(pool->parents[i]);
        return true;
    };
    if (!logits && !with_pool) {
        for (size_t i = 0; i < BTK; ++i) {
            size_t row = 0;
            int token = 0;
            if (entry_of(i, row, token)) grad[row * static_cast<size_t>(V) + static_cast<size_t>(token)] += draws[i];
        }
    } else if (!logits) {
        // each entry merged from 0 (the step's selected draw, then its pool
        // entries'), then added (reference src/c_api.cpp:948-951)
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < steps_b[static_cast<size_t>(b)]; ++t)
                for (const auto& e : step_entries(T, K, V, b, t, draws, parents, tokens, flp, pool))
                    grad[static_cast<size_t>(b) * row_block + static_cast<size_t>(e.first)] += e.second;
    } else {
        // From logits: the device writes each gradient row (g - softmax(row) *
        // sum(g), entries summed in token order; zero rows elsewhere), a
        // chunk of examples at a time, and the rows with an entry are added
        // here in full (reference src/decoder.hpp:212-242).
        const size_t example_bytes = mul(row_block, dtype_bytes(logits_type) + sizeof(float), "batch stride overflow");
        const int chunk =
            static_cast<int>(std::max<size_t>(1, std::min<size_t>(B, backward_chunk_bytes() / example_bytes)));
        std::lock_guard<std::mutex> lock(h->run_mutex);
        const hipStream_t st = stream_of(h);
        for (int b0 = 0; b0 < B; b0 += chunk) {
            const int nb = std::min(chunk, B - b0);
            const size_t off = static_cast<size_t>(b0) * trace;  // first [b, t, k] slot of the chunk
            std::vector<size_t> rows;
            for (size_t i = off; i < off + static_cast<size_t>(nb) * trace; ++i) {
                size_t row = 0;
                int token = 0;
                if (entry_of(i, row, token)) rows.push_back(row);
            }
            const size_t pstride = with_pool ? static_cast<size_t>(T) * pool->P : 0;
            const size_t poff = static_cast<size_t>(b0) * pstride, npool = static_cast<size_t>(nb) * pstride;
            for (size_t i = poff; i < poff + npool; ++i) {
                size_t row = 0;
                if (pool_row_of(i, row)) rows.push_back(row);
            }
            if (rows.empty()) continue;
            std::sort(rows.begin(), rows.end());
            rows.erase(std::unique(rows.begin(), rows.end()), rows.end());
            const size_t nslots = static_cast<size_t>(nb) * trace;
            DBSCudaDecodeArgs a = trace_args(nb, T, K, V, h->alpha);
            a.steps_per_example = upload(h, kSteps, steps_per_example ? steps_per_example + b0 : nullptr,
                                         static_cast<size_t>(nb), st);
            DBSCudaBackwardInputs in{};
            in.parents = upload(h, kParents, parents + off, nslots, st);
            in.tokens = upload(h, kTokens, tokens + off, nslots, st);
            in.lengths = upload(h, kLengths, lengths + off, nslots, st);
            in.from_logprob = upload(h, kFromLogprob, flp + off, nslots, st);
            const size_t fin = static_cast<size_t>(b0) * K, nfin = static_cast<size_t>(nb) * K;
            in.grad_final_scores = upload(h, kGradFinal, g.final_scores ? g.final_scores + fin : nullptr, nfin, st);
            in.grad_final_raw_scores = upload(h, kGradFinalRaw, g.final_raw ? g.final_raw + fin : nullptr, nfin, st);
            in.grad_scores = upload(h, kGradScores, g.scores ? g.scores + off : nullptr, nslots, st);
            in.grad_raw_scores = upload(h, kGradRaw, g.raw ? g.raw + off : nullptr, nslots, st);
            in.logits = upload(h, kInputs, static_cast<const unsigned char*>(logits) + off * V * dtype_bytes(logits_type),
                               nslots * V * dtype_bytes(logits_type), st);
            in.logits_type = logits_type;
            in.row_lse = upload(h, kRowLse, row_lse + off, nslots, st);
            float* dense = static_cast<float*>(h->arena.get(kDense, sizeof(float) * nslots * static_cast<size_t>(V)));
            const int64_t ws_bytes = dbs_cuda_backward_workspace_size(&a);
            need(ws_bytes > 0, "invalid backward arguments");
            void* ws = h->arena.get(kWorkspace, static_cast<size_t>(ws_bytes));
            dbs_hip::PoolGrads pg;
            if (with_pool) {
                pg.P = pool->P;
                pg.parents = upload(h, kPoolParents, pool->parents + poff, npool, st);
                pg.tokens = upload(h, kPoolTokens, pool->tokens + poff, npool, st);
                pg.from_logprob = upload(h, kPoolFromLogprob, pool->from_logprob + poff, npool, st);
                pg.d = upload(h, kPoolD, pool->d.data() + poff, npool, st);
            }
            engine_check(dbs_hip::backward_dense_for_host(&a, &in, with_pool ? &pg : nullptr, dense, ws, ws_bytes, st),
                         "HIP backward");
            std::vector<float> buf(rows.size() * static_cast<size_t>(V));
            for (size_t r = 0; r < rows.size(); ++r)
                download(buf.data() + r * V, dense + (rows[r] - off) * V, static_cast<size_t>(V), st);
            hip_check(hipStreamSynchronize(st), "HIP backward");
            for (size_t r = 0; r < rows.size(); ++r) {
                float* dst = grad + rows[r] * static_cast<size_t>(V);
                const float* src = buf.data() + r * static_cast<size_t>(V);
                for (int v = 0; v < V; ++v) dst[v] += src[v];
            }
        }
    }
    std::lock_guard<std::mutex> lock(h->stats_mutex);
    h->stats.used_sparse_backward = 0;
    h->stats.used_dense_backward = 1;
    h->stats.last_backward_ns = ns_since(start);
    h->stats.last_sparse_grad_count = 0;
    h->stats.last_error_category = 0;
}

}  // namespace
}  // namespace dbs_host

using namespace dbs_host;

extern "C" {

DBS_EXPORT int dbs_abi_version(void) { return DBS_ABI_VERSION; }

DBS_EXPORT const char* dbs_version_string(void) { return "2.3.0"; }

DBS_EXPORT const char* dbs_last_global_error(void) { return last_thread_error(); }

DBS_EXPORT const char* dbs_selected_kernel_name(void) { return "hip-gfx950"; }

// Options and their defaults as the reference (reference src/c_api.cpp:
// 160-189, src/decoder.cpp:697-721).
DBS_EXPORT int dbs_create_ex(DBSOptionsC o, DBSDecoderHandle** out_handle) {
    if (out_handle) *out_handle = nullptr;
    return run(nullptr, [&] {
        need(out_handle != nullptr, "out_handle cannot be null");
        auto finite_non_negative = [](float x) { return std::isfinite(x) && x >= 0.0f; };
        need(o.beam_size >= 0, "beam_size cannot be negative");
        need(o.eos_token >= -1, "eos_token must be -1 (disabled) or a token id");
        need(finite_non_negative(o.selected_temperature),
             "selected_temperature must be finite and non-negative (0 selects the default)");
        need(finite_non_negative(o.soft_topk_temperature),
             "soft_topk_temperature must be finite and non-negative (0 selects the default)");
        need(o.relaxed_pool_multiplier >= 0, "relaxed_pool_multiplier cannot be negative");
        need(o.vocab_block >= 0, "vocab_block cannot be negative");
        need(finite_non_negative(o.length_penalty_alpha), "length_penalty_alpha must be finite and non-negative");
        need(finite_non_negative(o.soft_topk_tolerance),
             "soft_topk_tolerance must be finite and non-negative (0 selects the default)");
        need(o.soft_topk_max_iters >= 0, "soft_topk_max_iters cannot be negative");
        need(o.min_length >= 0, "min_length cannot be negative");
        need(o.max_dense_gradient_elements >= 0, "max_dense_gradient_elements cannot be negative");
        auto* h = new DBSDecoderHandle;
        h->beam_size = o.beam_size > 0 ? o.beam_size : 8;
        h->eos_token = o.eos_token;
        h->alpha = o.length_penalty_alpha;
        h->min_length = o.min_length;
        h->validate = o.validate_inputs != 0 ? 1 : 0;
        h->pool_multiplier = o.relaxed_pool_multiplier;
        if (o.selected_temperature > 0.0f) h->selected_temperature = o.selected_temperature;
        if (o.soft_topk_temperature > 0.0f) h->soft_topk_temperature = o.soft_topk_temperature;
        if (o.soft_topk_tolerance > 0.0f) h->soft_topk_tolerance = o.soft_topk_tolerance;
        if (o.soft_topk_max_iters > 0) h->soft_topk_max_iters = o.soft_topk_max_iters;
        if (o.max_dense_gradient_elements > 0) h->max_dense_gradient_elements = o.max_dense_gradient_elements;
        h->stats.abi_version = DBS_ABI_VERSION;
        h->stats.last_kernel = kKernelHip;
        *out_handle = h;
    });
}

DBS_EXPORT DBSDecoderHandle* dbs_create(DBSOptionsC options) {
    DBSDecoderHandle* h = nullptr;
    return dbs_create_ex(options, &h) == DBS_OK ? h : nullptr;
}

DBS_EXPORT void dbs_destroy(DBSDecoderHandle* handle) { delete handle; }

DBS_EXPORT const char* dbs_last_error(DBSDecoderHandle* handle) {
    if (!handle) return dbs_last_global_error();
    // a per-thread copy, so the pointer stays valid while other threads
    // record errors on the handle
    static thread_local std::string copy;
    std::lock_guard<std::mutex> lock(handle->error_mutex);
    copy = handle->error;
    return copy.c_str();
}

// reference src/c_api.cpp:368-379, src/decoder.cpp:701-706
DBS_EXPORT int dbs_set_extra_eos_tokens(DBSDecoderHandle* handle, const int32_t* tokens, int count) {
    return run(handle, [&] {
        need(handle != nullptr, "decoder handle cannot be null");
        need(count >= 0 && (count == 0 || tokens != nullptr), "tokens cannot be null when count > 0");
        for (int i = 0; i < count; ++i) need(tokens[i] >= 0, "extra EOS tokens must be token ids");
        need(count == 0 || handle->eos_token >= 0,
             "extra EOS tokens need EOS handling: set eos_token to one of the EOS tokens");
        std::lock_guard<std::mutex> lock(handle->run_mutex);
        handle->extra_eos.assign(tokens, tokens + count);
    });
}

DBS_EXPORT int dbs_decode_batch_into(DBSDecoderHandle* handle, const float* log_probs, int batch_size, int steps,
                                     int vocab_size, const int32_t* steps_per_example,
                                     const DBSAdvancedConstraintsC* constraints, int num_threads,
                                     const DBSDecodeOutputsC* outputs) {
    (void)num_threads;
    return run(handle, [&] {
        decode_batch(handle, log_probs, DBS_DTYPE_F32, false, batch_size, steps, vocab_size, steps_per_example,
                     constraints, outputs, nullptr);
    });
}

DBS_EXPORT int dbs_decode_batch_into_ex(DBSDecoderHandle* handle, const void* inputs, int data_type, int from_logits,
                                        int batch_size, int steps, int vocab_size, const int32_t* steps_per_example,
                                        const DBSAdvancedConstraintsC* constraints, int num_threads,
                                        const DBSDecodeOutputsExC* outputs) {
    (void)num_threads;
    return run(handle, [&] {
        need(outputs != nullptr, "outputs cannot be null");
        decode_batch(handle, inputs, data_type, from_logits != 0, batch_size, steps, vocab_size, steps_per_example,
                     constraints, &outputs->base, outputs);
    });
}

DBS_EXPORT int dbs_backward_batch_into(DBSDecoderHandle* handle, int batch_size, int steps, int vocab_size,
                                       const int32_t* steps_per_example, const int32_t* parents,
                                       const int32_t* tokens, const int32_t* lengths, const uint8_t* from_logprob,
                                       const float* grad_final_scores, int num_threads, float* grad_log_probs) {
    (void)num_threads;
    return run(handle, [&] {
        need(handle != nullptr, "decoder handle cannot be null");
        need(parents && tokens && lengths && from_logprob,
             "parents, tokens, lengths and from_logprob cannot be null");
        need(grad_final_scores && grad_log_probs, "grad_final_scores and grad_log_probs cannot be null");
        need(batch_size > 0 && steps > 0 && vocab_size > 0, "batch_size, steps and vocab_size must be positive");
        Grads g;
        g.final_scores = grad_final_scores;
        backward_batch(handle, batch_size, steps, vocab_size, steps_per_example, parents, tokens, lengths,
                       from_logprob, g, nullptr, 0, nullptr, grad_log_probs, nullptr, nullptr, nullptr);
    });
}

DBS_EXPORT int dbs_backward_batch_into_ex(DBSDecoderHandle* handle, const DBSBackwardInputsC* in, int num_threads,
                                          float* grad_inputs) {
    (void)num_threads;
    return run(handle, [&] {
        need(handle != nullptr, "decoder handle cannot be null");
        need(in != nullptr && grad_inputs != nullptr, "inputs and grad_inputs cannot be null");
        need(!in->reserved[0] && !in->reserved[1] && !in->reserved[2] && !in->reserved[3],
             "reserved fields must be NULL");
        need(in->parents && in->tokens && in->lengths && in->from_logprob,
             "parents, tokens, lengths and from_logprob cannot be null");
        need(in->batch_size > 0 && in->steps > 0 && in->vocab_size > 0 && in->pool_size >= 0,
             "batch_size, steps and vocab_size must be positive and pool_size non-negative");
        const bool pool_grads = in->grad_pool_scores || in->grad_pool_raw_scores;
        need(!pool_grads || (in->pool_size > 0 && in->pool_parents && in->pool_tokens && in->pool_lengths &&
                             in->pool_from_logprob),
             "pool gradients need pool_size > 0 and the pool trace");
        if (in->logits) {
            check_dtype(in->logits_type);
            need(in->row_lse != nullptr, "row_lse cannot be null with logits");
        }
        Grads g;
        g.final_scores = in->grad_final_scores;
        g.final_raw = in->grad_final_raw_scores;
        g.scores = in->grad_scores;
        g.raw = in->grad_raw_scores;
        PoolTerms pool;
        if (pool_grads) {
            pool.P = in->pool_size;
            pool.parents = in->pool_parents;
            pool.tokens = in->pool_tokens;
            pool.lengths = in->pool_lengths;
            pool.from_logprob = in->pool_from_logprob;
        }
        backward_batch(handle, in->batch_size, in->steps, in->vocab_size, in->steps_per_example, in->parents,
                       in->tokens, in->lengths, in->from_logprob, g, in->logits, in->logits_type, in->row_lse,
                       grad_inputs, pool_grads ? &pool : nullptr, in->grad_pool_scores, in->grad_pool_raw_scores);
    });
}

}  // extern "C"
