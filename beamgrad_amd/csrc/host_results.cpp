// SPDX-License-Identifier: MIT
//
// The result-object half of the libdbs host C ABI (include/dbs.h) served by
// the HIP engine: decodes into result handles (one example, a batch, a batch
// with per-example options, and model-in-the-loop decodes that call the
// caller's model once per step), the backward of a result into a dense or
// sparse gradient handle, the accessors, statistics, workspaces and the
// remaining queries (reference src/c_api.cpp:312-1347, src/decoder.cpp:
// 697-945).
//
// Every decode runs on the GPU through the drivers of host_abi.cpp (a
// model-step decode runs the device step API once per step); the host only
// stages arrays, derives the selected-beam softmax weights of each step from
// the selected scores, and turns the device's per-slot path gradients into
// the reference's gradient layouts. What the engine does not serve (the
// relaxed pool, token-filter callbacks) is refused with
// DBS_ERROR_INVALID_ARGUMENT and a message naming it.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <memory>

#include "dbs_cuda.h"
#include "host_abi.hpp"
#include "host_entry.hpp"
#include "numerics.hpp"

struct DBSResultHandle {
    int steps = 0;
    int beam_size = 0;
    int vocab_size = 0;
    float alpha = 0.0f;
    float selected_temperature = 1.0f;
    std::vector<int32_t> parents, tokens, lengths;  // [T * K]
    std::vector<float> raw_scores, scores, weights;  // [T * K]
    std::vector<uint8_t> from_logprob;               // [T * K]
    std::vector<float> final_raw_scores, final_scores;  // [K]
    // the relaxed pool: P candidates a step (0: none), with their soft top-K
    // inclusion weights
    int pool_size = 0;
    float soft_topk_temperature = 0.25f;
    std::vector<int32_t> pool_parents, pool_tokens, pool_lengths;      // [T * P]
    std::vector<float> pool_raw_scores, pool_scores, relaxed_weights;  // [T * P]
    std::vector<uint8_t> pool_from_logprob;                            // [T * P]
};

struct DBSBatchResultHandle {
    std::vector<DBSResultHandle> results;
};

struct DBSBackwardHandle {
    bool sparse = false;
    std::vector<float> grad_log_probs;  // [T * K * V] (dense)
    std::vector<float> grad_initial_scores;  // [K]
    std::vector<int64_t> sparse_indices;  // flattened [T * K * V] positions, increasing
    std::vector<float> sparse_values;
};

struct DBSWorkspaceHandle {
    std::mutex mutex;
    std::vector<float> f32;
    std::vector<int32_t> i32;
};

using namespace dbs_host;

namespace {

constexpr float kNegInf = -std::numeric_limits<float>::infinity();

int64_t ns_since(std::chrono::steady_clock::time_point start) {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - start).count();
}

// The selected beams' softmax weights of one step: softmax(score / temperature)
// over the live beams (score above -1e30), 0 for the others and for a step
// without live beams; exp as the decode's exact exp of a non-positive value
// (reference src/kernels_scalar.cpp:277-302, operation for operation).
void softmax_selected(const float* scores, float* out, int n, float temperature) {
    constexpr float kNegGuard = -1.0e30f;
    std::fill(out, out + n, 0.0f);
    float maxv = kNegInf;
    for (int i = 0; i < n; ++i)
        if (scores[i] > kNegGuard) maxv = std::max(maxv, scores[i] / temperature);
    if (!std::isfinite(maxv)) return;
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        if (scores[i] > kNegGuard) {
            out[i] = dbs_hip::exp_nonpositive(scores[i] / temperature - maxv);
            sum += out[i];
        }
    }
    if (!(sum > 0.0f) || !std::isfinite(sum)) {
        std::fill(out, out + n, 0.0f);
        return;
    }
    const float inv_sum = 1.0f / sum;
    for (int i = 0; i < n; ++i) out[i] *= inv_sum;
}

// The soft top-k inclusion weights of one step's pool (reference
// src/kernels_scalar.cpp:28-45, 298-364): sigmoid((s - theta) / temperature)
// for every live candidate, theta bisected (as an offset from the best
// score) until the weights sum to k within the tolerance, or theta is
// bracketed to tolerance * temperature or to a few ulps; the reference's
// operations in its order, with its exp, so the weights are its bits.
constexpr float kPoolGuard = -1.0e30f;  // scores at or below it are dead entries

float det_sigmoid(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + dbs_hip::exp_nonpositive(-x));
    const float e = dbs_hip::exp_nonpositive(x);
    return e / (1.0f + e);
}

float inclusion_sum(const float* s, int n, float ref, float offset, float temperature) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i)
        if (s[i] > kPoolGuard) sum += det_sigmoid(((s[i] - ref) - offset) / temperature);
    return sum;
}

void soft_topk_weights(const float* s, float* w, int n, int k, float temperature, float tolerance, int max_iters) {
    std::fill(w, w + n, 0.0f);
    int live = 0;
    float lo_s = std::numeric_limits<float>::infinity(), hi_s = -std::numeric_limits<float>::infinity();
    for (int i = 0; i < n; ++i) {
        if (!(s[i] > kPoolGuard)) continue;
        ++live;
        lo_s = std::min(lo_s, s[i]);
        hi_s = std::max(hi_s, s[i]);
    }
    if (live == 0 || k <= 0) return;
    if (k >= live) {
        for (int i = 0; i < n; ++i) w[i] = s[i] > kPoolGuard ? 1.0f : 0.0f;
        return;
    }
    const float ref = hi_s;
    float lo = (lo_s - ref) - 80.0f * temperature;
    float hi = 80.0f * temperature;
    const float bracket = tolerance * temperature;
    for (int it = 0; it < max_iters; ++it) {
        const float mid = 0.5f * (lo + hi);
        const float err = inclusion_sum(s, n, ref, mid, temperature) - static_cast<float>(k);
        const float ulps = 4.0f * std::numeric_limits<float>::epsilon() * std::fabs(mid);
        if (std::fabs(err) <= tolerance || hi - lo <= std::max(bracket, ulps)) {
            lo = hi = mid;
            break;
        }
        (err > 0.0f ? lo : hi) = mid;
    }
    const float offset = 0.5f * (lo + hi);
    for (int i = 0; i < n; ++i) w[i] = s[i] > kPoolGuard ? det_sigmoid(((s[i] - ref) - offset) / temperature) : 0.0f;
}

// A step's pool from the device (P entries of a [.., Pmax] row) into the
// result at step t, with its inclusion weights over the result's K beams.
void put_pool_step(DBSResultHandle& r, const DBSDecoderHandle& h, int t, const int32_t* par, const int32_t* tok,
                   const int32_t* len, const float* sc, const float* raw, const uint8_t* flp) {
    const int P = r.pool_size;
    const size_t dst = static_cast<size_t>(t) * P;
    std::copy_n(par, P, r.pool_parents.begin() + dst);
    std::copy_n(tok, P, r.pool_tokens.begin() + dst);
    std::copy_n(len, P, r.pool_lengths.begin() + dst);
    std::copy_n(sc, P, r.pool_scores.begin() + dst);
    std::copy_n(raw, P, r.pool_raw_scores.begin() + dst);
    std::copy_n(flp, P, r.pool_from_logprob.begin() + dst);
    soft_topk_weights(r.pool_scores.data() + dst, r.relaxed_weights.data() + dst, P, r.beam_size,
                      h.soft_topk_temperature, h.soft_topk_tolerance, h.soft_topk_max_iters);
}

// A result's pool arrays for `steps` steps of P candidates.
void size_pool(DBSResultHandle& r, const DBSDecoderHandle& h, int steps, int P) {
    r.pool_size = P;
    r.soft_topk_temperature = h.soft_topk_temperature;
    const size_t n = static_cast<size_t>(steps) * static_cast<size_t>(P);
    r.pool_parents.assign(n, -1);
    r.pool_tokens.assign(n, -1);
    r.pool_lengths.assign(n, 0);
    r.pool_scores.assign(n, kNegInf);
    r.pool_raw_scores.assign(n, kNegInf);
    r.relaxed_weights.assign(n, 0.0f);
    r.pool_from_logprob.assign(n, 0);
}

DBSDecoderHandle& handle_of(DBSDecoderHandle* h) {
    need(h != nullptr, "decoder handle cannot be null");
    return *h;
}

// A decode's constraints as the decoder reads them (reference
// src/c_api.cpp:191-203, src/decoder.cpp:385-406); the GPU serves banned
// tokens, forced tokens, min_length, n-gram blocking and the repetition
// penalty.
struct Constraints {
    const uint8_t* banned = nullptr;
    const int32_t* forced = nullptr;
    int min_length = -1;
    float repetition_penalty = 1.0f;
    int ngram = 0;
    bool filter = false;
    DBSTokenFilterFn filter_fn = nullptr;
    void* filter_user = nullptr;
    int batch_index = 0;
};

Constraints constraints_of(const DBSAdvancedConstraintsC* c) {
    Constraints out;
    if (!c) return out;
    out.banned = c->banned_tokens;
    out.forced = c->forced_tokens;
    out.min_length = c->min_length;
    out.repetition_penalty = c->repetition_penalty > 0.0f ? c->repetition_penalty : 1.0f;
    out.ngram = c->no_repeat_ngram_size;
    out.filter = c->token_filter != nullptr;
    out.filter_fn = c->token_filter;
    out.filter_user = c->token_filter_user_data;
    out.batch_index = c->batch_index;
    return out;
}

// check_decode_args of the reference decoder for one decode of `steps`
// steps with beam K (its texts, in its order).
void check_decode_args(const DBSDecoderHandle& h, int K, int eos, int steps, int V, const Constraints* c) {
    need(steps > 0, "steps must be positive");
    need(V > 0, "vocab_size must be positive");
    need(eos < V, "eos_token is outside the vocabulary");
    for (int32_t token : h.extra_eos) need(token < V, "an extra EOS token is outside the vocabulary");
    if (c) {
        if (c->forced) {
            for (int t = 0; t < steps; ++t) need(c->forced[t] < V, "forced token is outside the vocabulary");
        }
        need(c->repetition_penalty > 0.0f && std::isfinite(c->repetition_penalty),
             "repetition_penalty must be finite and positive (1 disables it)");
    }
    const size_t selected = mul(static_cast<size_t>(steps), static_cast<size_t>(K), "result size overflow");
    (void)mul(selected, static_cast<size_t>(V), "log-prob tensor size overflow");
}

// The token filter's verdicts for step t (reference src/decoder.cpp:
// 131-167, 196-282, in its call order): for each read beam in order (a
// finite score, not a finished beam carried; from logits, a row with a
// finite entry), each token in order that passes the forced, banned,
// minimum-length and n-gram checks goes to the filter with the beam's
// prefix (prefix [K, stride], len[k] tokens each); mask[k * V + v] = 1
// where the filter refused it. With validate_inputs, a read row holding NaN
// or +inf raises where the reference's scan raises: from logits before the
// row's calls, from log-probs after them.
void filter_step(const DBSDecoderHandle& h, const Constraints& c, int t, int V, bool from_logits, const float* rows,
                 const std::vector<float>& raw, const std::vector<uint8_t>& finished,
                 const std::vector<int32_t>& len, const std::vector<int32_t>& prefix, int stride, int min_length,
                 std::vector<uint8_t>& mask) {
    const int K = h.beam_size, eos = h.eos_token;
    auto is_eos = [&](int v) {
        if (eos < 0) return false;
        return v == eos || std::find(h.extra_eos.begin(), h.extra_eos.end(), v) != h.extra_eos.end();
    };
    const int forced = c.forced ? c.forced[t] : -1;
    mask.assign(static_cast<size_t>(K) * V, 0);
    std::vector<uint8_t> blocked(static_cast<size_t>(V));
    const auto where = [&](int k) { return " (step " + std::to_string(t) + ", beam " + std::to_string(k) + ")"; };
    for (int k = 0; k < K; ++k) {
        const size_t ki = static_cast<size_t>(k);
        if (!std::isfinite(raw[ki]) || (eos >= 0 && finished[ki])) continue;
        const float* row = rows + ki * static_cast<size_t>(V);
        bool invalid = false, finite = false;
        for (int v = 0; v < V; ++v) {
            if (!(row[v] < std::numeric_limits<float>::infinity())) invalid = true;
            else if (row[v] > kNegInf) finite = true;
        }
        if (from_logits) {
            if (invalid && h.validate) throw std::invalid_argument("logits contain NaN or +inf" + where(k));
            if (!finite) continue;  // no finite logit: the row is not scanned
        }
        const int L = len[ki];
        const int32_t* pre = prefix.data() + ki * static_cast<size_t>(stride);
        std::fill(blocked.begin(), blocked.end(), 0);
        const int n = c.ngram;
        auto block = [&](int32_t tok) {
            if (tok >= 0 && tok < V) blocked[static_cast<size_t>(tok)] = 1;
        };
        if (n == 1) {
            for (int i = 0; i < L; ++i) block(pre[i]);
        } else if (n > 1 && L >= n - 1) {
            const int tail = L - (n - 1);
            for (int i = 0; i + n <= L; ++i) {
                bool same = true;
                for (int j = 0; j < n - 1 && same; ++j) same = pre[i + j] == pre[tail + j];
                if (same) block(pre[i + n - 1]);
            }
        }
        const bool mask_eos = L + 1 < min_length;
        for (int v = 0; v < V; ++v) {
            if (forced >= 0 && v != forced) continue;
            if (c.banned && c.banned[v]) continue;
            if (mask_eos && is_eos(v)) continue;
            if (blocked[static_cast<size_t>(v)]) continue;
            if (c.filter_fn(c.filter_user, c.batch_index, t, k, L > 0 ? pre : nullptr, L, v) == 0)
                mask[ki * static_cast<size_t>(V) + static_cast<size_t>(v)] = 1;
        }
        if (!from_logits && invalid && h.validate) throw std::invalid_argument("log_probs contains NaN or +inf" + where(k));
    }
}

// What the HIP engine does not serve, after the reference's own checks.
void check_served(const DBSDecoderHandle& h, const Constraints* c) {
    (void)h;
    (void)c;
}

// Host copies of a decode's relaxed pool [B, T, mult * Kmax].
struct PoolHost {
    int mult = 0;
    std::vector<int32_t> parents, tokens, lengths;
    std::vector<float> scores, raw;
    std::vector<uint8_t> flp;
};

// Result b of a [B, T, Kmax] trace: its first `steps` steps and `beams`
// slots, with the selected-beam weights of each step (and its pool).
void fill_result(DBSResultHandle& r, const DBSDecoderHandle& h, int steps, int beams, int V, int T, int Kmax, int b,
                 const std::vector<int32_t>& parents, const std::vector<int32_t>& tokens,
                 const std::vector<int32_t>& lengths, const std::vector<float>& raw, const std::vector<float>& scores,
                 const std::vector<uint8_t>& flp, const std::vector<float>& final_raw,
                 const std::vector<float>& final_scores, const PoolHost* pool) {
    r.steps = steps;
    r.beam_size = beams;
    r.vocab_size = V;
    r.alpha = h.alpha;
    r.selected_temperature = h.selected_temperature;
    const size_t n = static_cast<size_t>(steps) * beams;
    r.parents.resize(n);
    r.tokens.resize(n);
    r.lengths.resize(n);
    r.raw_scores.resize(n);
    r.scores.resize(n);
    r.weights.resize(n);
    r.from_logprob.resize(n);
    for (int t = 0; t < steps; ++t) {
        const size_t src = (static_cast<size_t>(b) * T + t) * Kmax, dst = static_cast<size_t>(t) * beams;
        std::copy_n(parents.begin() + src, beams, r.parents.begin() + dst);
        std::copy_n(tokens.begin() + src, beams, r.tokens.begin() + dst);
        std::copy_n(lengths.begin() + src, beams, r.lengths.begin() + dst);
        std::copy_n(raw.begin() + src, beams, r.raw_scores.begin() + dst);
        std::copy_n(scores.begin() + src, beams, r.scores.begin() + dst);
        std::copy_n(flp.begin() + src, beams, r.from_logprob.begin() + dst);
        softmax_selected(r.scores.data() + dst, r.weights.data() + dst, beams, h.selected_temperature);
    }
    if (pool) {
        // the example's pool: the first beams * m of each step's row
        size_pool(r, h, steps, beams * pool->mult);
        const size_t Pmax = static_cast<size_t>(Kmax) * pool->mult;
        for (int t = 0; t < steps; ++t) {
            const size_t src = (static_cast<size_t>(b) * T + t) * Pmax;
            put_pool_step(r, h, t, pool->parents.data() + src, pool->tokens.data() + src, pool->lengths.data() + src,
                          pool->scores.data() + src, pool->raw.data() + src, pool->flp.data() + src);
        }
    }
    const size_t fsrc = static_cast<size_t>(b) * Kmax;
    r.final_raw_scores.assign(final_raw.begin() + fsrc, final_raw.begin() + fsrc + beams);
    r.final_scores.assign(final_scores.begin() + fsrc, final_scores.begin() + fsrc + beams);
}

// The bytes of a result's trace and pool arrays (reference src/c_api.cpp:
// 124-129 counts these).
int64_t result_bytes(const DBSResultHandle& r) {
    return static_cast<int64_t>(r.parents.size() * 3 * sizeof(int32_t) + r.raw_scores.size() * 3 * sizeof(float) +
                                r.pool_parents.size() * 3 * sizeof(int32_t) +
                                r.pool_scores.size() * 3 * sizeof(float));
}

// One decode of B examples [B, T, K, V] of log-probabilities into results:
// the handle's options, optional per-example steps, beams, EOS tokens,
// minimum lengths and banned masks [B, V].
struct BatchSpec {
    const void* inputs = nullptr;
    int data_type = DBS_DTYPE_F32;
    int B = 0, T = 0, K = 0, V = 0;
    const int32_t* steps = nullptr;
    const int32_t* beams = nullptr;
    const int32_t* eos = nullptr;
    const int32_t* min_lengths = nullptr;
    const uint8_t* banned_pe = nullptr;
    const int32_t* forced_pe = nullptr;  // [B, T] forced tokens per example
    const Constraints* cons = nullptr;  // every example
    bool batch_errors = true;
};

std::vector<DBSResultHandle> decode_results(DBSDecoderHandle& h, const BatchSpec& s) {
    const size_t BK = static_cast<size_t>(s.B) * s.K, BTK = BK * static_cast<size_t>(s.T);
    std::vector<int32_t> parents(BTK), tokens(BTK), lengths(BTK);
    std::vector<float> raw(BTK), scores(BTK), final_raw(BK), final_scores(BK);
    std::vector<uint8_t> flp(BTK);
    DecodeJob j;
    j.inputs = s.inputs;
    j.data_type = s.data_type;
    j.B = s.B;
    j.T = s.T;
    j.K = s.K;
    j.V = s.V;
    j.steps = s.steps;
    j.beams = s.beams;
    j.eos = s.eos;
    j.min_lengths = s.min_lengths;
    j.banned_pe = s.banned_pe;
    j.min_length = s.cons && s.cons->min_length >= 0 ? s.cons->min_length : h.min_length;
    j.banned = s.cons ? s.cons->banned : nullptr;
    j.forced = s.cons ? s.cons->forced : s.forced_pe;
    j.forced_stride = s.cons ? 0 : static_cast<size_t>(s.T);
    j.ngram = s.cons && s.cons->ngram > 0 ? s.cons->ngram : 0;
    j.repetition_penalty = s.cons ? s.cons->repetition_penalty : 1.0f;
    j.batch_errors = s.batch_errors;
    j.final_scores = final_scores.data();
    j.final_raw = final_raw.data();
    j.tokens = tokens.data();
    j.parents = parents.data();
    j.lengths = lengths.data();
    j.scores = scores.data();
    j.raw_scores = raw.data();
    j.from_logprob = flp.data();
    PoolHost pool;
    if (h.pool_multiplier > 0) {
        const size_t BTP = BTK * static_cast<size_t>(pool_size_of(s.K, h.pool_multiplier) / s.K);
        pool.mult = h.pool_multiplier;
        pool.parents.resize(BTP);
        pool.tokens.resize(BTP);
        pool.lengths.resize(BTP);
        pool.scores.resize(BTP);
        pool.raw.resize(BTP);
        pool.flp.resize(BTP);
        j.pool_mult = pool.mult;
        j.pool_parents = pool.parents.data();
        j.pool_tokens = pool.tokens.data();
        j.pool_lengths = pool.lengths.data();
        j.pool_scores = pool.scores.data();
        j.pool_raw = pool.raw.data();
        j.pool_from_logprob = pool.flp.data();
    }
    run_decode(&h, j);
    std::vector<DBSResultHandle> out(static_cast<size_t>(s.B));
    for (int b = 0; b < s.B; ++b) {
        fill_result(out[static_cast<size_t>(b)], h, s.steps ? s.steps[b] : s.T, s.beams ? s.beams[b] : s.K, s.V, s.T,
                    s.K, b, parents, tokens, lengths, raw, scores, flp, final_raw, final_scores,
                    pool.mult > 0 ? &pool : nullptr);
    }
    return out;
}

void record_result_stats(DBSDecoderHandle& h, const DBSResultHandle& r, int64_t ns, bool model_step,
                         int64_t extra_bytes = 0) {
    const int64_t selected = static_cast<int64_t>(r.steps) * r.beam_size;
    stats_decode(&h, ns, selected, static_cast<int64_t>(r.steps) * r.pool_size, selected * r.vocab_size,
                 result_bytes(r) + extra_bytes, model_step);
}

// ---------------------------------------------------------------------------
// Model-in-the-loop decode: the caller's model gives each step's [K, V] rows
// ---------------------------------------------------------------------------

// The beams entering a step, as a model-step callback sees them (reference
// src/decoder.cpp:837-901).
struct StepView {
    int step = 0;
    const int32_t* parents;
    const int32_t* tokens;
    const int32_t* lengths;
    const float* scores;
    const float* raw_scores;
    const uint8_t* finished;
    const int32_t* prefixes;  // [K, step]
};

// Runs `steps` steps with rows from fill(view, rows) on the GPU step API:
// the state (raw scores, lengths, finished flags and token prefixes) stays
// on the device between steps, each step's rows (pre-filled with -inf) are
// copied in and its selection copied back.
// How a step-by-step decode reads its rows: from logits (row_lse: host
// [steps, K] or null, 0 for rows not read).
struct StepRows {
    bool from_logits = false;
    float* row_lse = nullptr;
    int32_t* final_lengths = nullptr;  // host [K] or null
};

template <class Fill>
DBSResultHandle decode_model_steps(DBSDecoderHandle& h, int steps, int V, const Constraints* c, Fill&& fill,
                                   int64_t* rows_bytes, const StepRows& how = StepRows{}) {
    const int K = h.beam_size;
    check_decode_args(h, K, h.eos_token, steps, V, c);
    check_served(h, c);
    check_engine_limits(&h, K, V);
    const size_t row_block = static_cast<size_t>(K) * V;
    const size_t prefix_size = mul(static_cast<size_t>(K), static_cast<size_t>(steps), "prefix size overflow");

    DBSResultHandle r;
    r.steps = steps;
    r.beam_size = K;
    r.vocab_size = V;
    r.alpha = h.alpha;
    r.selected_temperature = h.selected_temperature;
    const size_t n = static_cast<size_t>(steps) * K;
    r.parents.assign(n, -1);
    r.tokens.assign(n, -1);
    r.lengths.assign(n, 0);
    r.raw_scores.assign(n, kNegInf);
    r.scores.assign(n, kNegInf);
    r.weights.assign(n, 0.0f);
    r.from_logprob.assign(n, 0);

    // the search state: beam 0 live at step 0
    std::vector<float> raw(static_cast<size_t>(K), kNegInf);
    raw[0] = 0.0f;
    std::vector<int32_t> len(static_cast<size_t>(K), 0), parents(static_cast<size_t>(K), -1),
        tokens(static_cast<size_t>(K), -1);
    std::vector<uint8_t> finished(static_cast<size_t>(K), 0);
    // token prefixes as the search keeps them (the tokens each beam took from
    // a row, its length long) for the device, and as the callback sees them
    // (every step's token, -1 on a dead path)
    std::vector<int32_t> search_prefix(prefix_size, -1), next_search(prefix_size, -1);
    std::vector<int32_t> view_prefix(prefix_size, -1), next_view(prefix_size, -1);
    std::vector<float> scores(static_cast<size_t>(K));
    std::vector<float> rows;

    const int min_length = c && c->min_length >= 0 ? c->min_length : h.min_length;
    // full prefixes: for the constraints, and for a token filter's calls
    const bool constrained = c && (c->ngram > 0 || c->repetition_penalty > 1.0f || c->filter);
    std::vector<uint8_t> filter_mask;
    DBSCudaDecodeArgs a{};
    a.batch_size = 1;
    a.steps = 1;
    a.beam_size = K;
    a.vocab_size = V;
    a.eos_token = h.eos_token;
    a.min_length = min_length;
    a.length_penalty_alpha = h.alpha;
    a.no_repeat_ngram_size = c && c->ngram > 0 ? c->ngram : 0;
    a.repetition_penalty = c ? c->repetition_penalty : 1.0f;
    DBSCudaSearchOptions opts{};
    opts.extra_eos_count = static_cast<int>(h.extra_eos.size());
    for (size_t i = 0; i < h.extra_eos.size(); ++i) opts.extra_eos_tokens[i] = h.extra_eos[i];
    // the relaxed pool of each step (reference src/decoder.cpp:849)
    const int P = pool_size_of(K, h.pool_multiplier);
    if (P > 0) size_pool(r, h, steps, P);
    std::vector<int32_t> pool_par(static_cast<size_t>(P)), pool_tok(static_cast<size_t>(P)),
        pool_len(static_cast<size_t>(P));
    std::vector<float> pool_sc(static_cast<size_t>(P)), pool_raw(static_cast<size_t>(P));
    std::vector<uint8_t> pool_flp(static_cast<size_t>(P));
    const int64_t ws_bytes = dbs_hip::workspace_for_host(&a, P > 0 ? h.pool_multiplier : 0, 1, steps);
    need(ws_bytes > 0, "invalid decode arguments");

    for (int t = 0; t < steps; ++t) {
        if (t > 0) {
            const size_t width = static_cast<size_t>(t - 1);
            for (int k = 0; k < K; ++k) {
                const int32_t p = parents[static_cast<size_t>(k)];
                int32_t* row = next_view.data() + static_cast<size_t>(k) * t;
                if (p >= 0) std::copy_n(view_prefix.data() + static_cast<size_t>(p) * width, width, row);
                else std::fill_n(row, width, -1);
                row[width] = tokens[static_cast<size_t>(k)];
            }
            view_prefix.swap(next_view);
        }
        for (int k = 0; k < K; ++k) {
            const int l = std::max(1, static_cast<int>(len[static_cast<size_t>(k)]));
            scores[static_cast<size_t>(k)] = raw[static_cast<size_t>(k)] / dbs_hip::length_penalty(l, h.alpha);
        }
        StepView view{t, parents.data(), tokens.data(), len.data(), scores.data(), raw.data(), finished.data(),
                      view_prefix.data()};
        rows.assign(row_block, kNegInf);
        fill(view, rows.data());
        if (c && c->filter)
            filter_step(h, *c, t, V, how.from_logits, rows.data(), raw, finished, len, search_prefix, steps,
                        min_length, filter_mask);

        std::vector<int32_t> out_tok(static_cast<size_t>(K)), out_par(static_cast<size_t>(K));
        std::vector<float> out_score(static_cast<size_t>(K));
        std::vector<uint8_t> out_flp(static_cast<size_t>(K));
        uint8_t invalid = 0;
        {
            std::lock_guard<std::mutex> lock(h.run_mutex);
            const hipStream_t st = stream_of(&h);
            const float* rows_d = upload(&h, kInputs, rows.data(), row_block, st);
            a.banned_tokens = upload(&h, kBanned, c ? c->banned : nullptr, static_cast<size_t>(V), st);
            char* state = static_cast<char*>(h.arena.get(kState, K * 9 + 16 + prefix_size * sizeof(int32_t)));
            float* raw_d = reinterpret_cast<float*>(state);
            int32_t* len_d = reinterpret_cast<int32_t*>(state + 4 * K);
            int32_t* prefix_d = reinterpret_cast<int32_t*>(state + 8 * K);
            uint8_t* fin_d = reinterpret_cast<uint8_t*>(state + 8 * K + prefix_size * sizeof(int32_t));
            hip_check(hipMemcpyAsync(raw_d, raw.data(), 4 * K, hipMemcpyHostToDevice, st), "copy to the device");
            hip_check(hipMemcpyAsync(len_d, len.data(), 4 * K, hipMemcpyHostToDevice, st), "copy to the device");
            hip_check(hipMemcpyAsync(fin_d, finished.data(), K, hipMemcpyHostToDevice, st), "copy to the device");
            hip_check(hipMemcpyAsync(prefix_d, search_prefix.data(), prefix_size * sizeof(int32_t),
                                     hipMemcpyHostToDevice, st),
                      "copy to the device");
            DBSCudaBeamState bs{};
            bs.raw_scores = raw_d;
            bs.lengths = len_d;
            bs.finished = fin_d;
            bs.prefixes = prefix_d;
            bs.prefix_stride = steps;
            DBSCudaDecodeOutputs o{};
            o.tokens = static_cast<int32_t*>(h.arena.get(kTokens, 4 * K));
            o.parents = static_cast<int32_t*>(h.arena.get(kParents, 4 * K));
            o.scores = static_cast<float*>(h.arena.get(kScores, 4 * K));
            o.from_logprob = static_cast<uint8_t*>(h.arena.get(kFromLogprob, K));
            o.invalid_input = h.validate ? static_cast<uint8_t*>(h.arena.get(kFirstInvalid, 16)) : nullptr;
            void* ws = h.arena.get(kWorkspace, static_cast<size_t>(ws_bytes));
            // this step's forced token, if any (reference src/decoder.cpp:125)
            const int32_t* forced_d = nullptr;
            if (c && c->forced && c->forced[t] >= 0) {
                h.staged_forced.assign(1, c->forced[t]);
                forced_d = upload(&h, kForced, h.staged_forced.data(), 1, st);
            }
            dbs_hip::PoolOutputs pool;
            if (P > 0) {
                pool.mult = h.pool_multiplier;
                pool.parents = static_cast<int32_t*>(h.arena.get(kPoolParents, 4 * static_cast<size_t>(P)));
                pool.tokens = static_cast<int32_t*>(h.arena.get(kPoolTokens, 4 * static_cast<size_t>(P)));
                pool.lengths = static_cast<int32_t*>(h.arena.get(kPoolLengths, 4 * static_cast<size_t>(P)));
                pool.scores = static_cast<float*>(h.arena.get(kPoolScores, 4 * static_cast<size_t>(P)));
                pool.raw_scores = static_cast<float*>(h.arena.get(kPoolRaw, 4 * static_cast<size_t>(P)));
                pool.from_logprob = static_cast<uint8_t*>(h.arena.get(kPoolFromLogprob, static_cast<size_t>(P)));
            }
            const uint8_t* mask_d =
                c && c->filter ? upload(&h, kRowMask, filter_mask.data(), filter_mask.size(), st) : nullptr;
            float* lse_d = how.row_lse ? static_cast<float*>(h.arena.get(kRowLse, 4 * static_cast<size_t>(K))) : nullptr;
            engine_check(dbs_hip::step_for_host(rows_d, DBS_CUDA_DTYPE_F32, how.from_logits ? 1 : 0, &a, &opts, &bs,
                                                &o, lse_d, forced_d, P > 0 ? &pool : nullptr, mask_d, ws, ws_bytes,
                                                st),
                         "HIP decode step");
            if (lse_d) download(how.row_lse + static_cast<size_t>(t) * K, lse_d, static_cast<size_t>(K), st);
            if (P > 0) {
                download(pool_par.data(), pool.parents, pool_par.size(), st);
                download(pool_tok.data(), pool.tokens, pool_tok.size(), st);
                download(pool_len.data(), pool.lengths, pool_len.size(), st);
                download(pool_sc.data(), pool.scores, pool_sc.size(), st);
                download(pool_raw.data(), pool.raw_scores, pool_raw.size(), st);
                download(pool_flp.data(), pool.from_logprob, pool_flp.size(), st);
            }
            download(out_tok.data(), o.tokens, K, st);
            download(out_par.data(), o.parents, K, st);
            download(out_score.data(), o.scores, K, st);
            download(out_flp.data(), o.from_logprob, K, st);
            download(raw.data(), raw_d, K, st);
            download(len.data(), len_d, K, st);
            download(finished.data(), fin_d, K, st);
            if (o.invalid_input) download(&invalid, o.invalid_input, 1, st);
            hip_check(hipStreamSynchronize(st), "HIP decode step");
        }
        if (invalid) {
            // the first beam read whose row holds NaN or +inf (reference
            // src/decoder.cpp:127-171: every read row is checked whole)
            for (int k = 0; k < K; ++k) {
                const bool read = std::isfinite(view.raw_scores[k]) && !(h.eos_token >= 0 && view.finished[k]);
                if (!read) continue;
                const float* row = rows.data() + static_cast<size_t>(k) * V;
                for (int v = 0; v < V; ++v) {
                    if (!(row[v] < std::numeric_limits<float>::infinity()))
                        throw std::invalid_argument(std::string(how.from_logits ? "logits contain NaN or +inf"
                                                                                : "log_probs contains NaN or +inf") +
                                                    " (step " + std::to_string(t) + ", beam " + std::to_string(k) +
                                                    ")");
                }
            }
        }
        // the step's selection, and the prefixes it extends
        const size_t base = static_cast<size_t>(t) * K;
        for (int k = 0; k < K; ++k) {
            const size_t i = static_cast<size_t>(k);
            r.parents[base + i] = out_par[i];
            r.tokens[base + i] = out_tok[i];
            r.lengths[base + i] = len[i];
            r.raw_scores[base + i] = raw[i];
            r.scores[base + i] = out_score[i];
            r.from_logprob[base + i] = out_flp[i];
            if (constrained) {
                int32_t* dst = next_search.data() + i * steps;
                std::fill_n(dst, steps, -1);
                const int p = out_par[i];
                if (p >= 0) {
                    std::copy_n(search_prefix.data() + static_cast<size_t>(p) * steps, steps, dst);
                    const int l = len[i];
                    if (out_flp[i] && out_tok[i] >= 0 && l >= 1 && l <= steps) dst[l - 1] = out_tok[i];
                }
            } else {
                // the carried token of a finished beam is read at its length
                int32_t* dst = next_search.data() + i * steps;
                std::fill_n(dst, steps, -1);
                const int l = len[i];
                if (out_par[i] >= 0 && l >= 1 && l <= steps) dst[l - 1] = out_tok[i];
            }
        }
        search_prefix.swap(next_search);
        softmax_selected(r.scores.data() + base, r.weights.data() + base, K, h.selected_temperature);
        if (P > 0)
            put_pool_step(r, h, t, pool_par.data(), pool_tok.data(), pool_len.data(), pool_sc.data(), pool_raw.data(),
                          pool_flp.data());
        parents = out_par;
        tokens = out_tok;
    }
    r.final_raw_scores.resize(static_cast<size_t>(K));
    r.final_scores.resize(static_cast<size_t>(K));
    for (int k = 0; k < K; ++k) {
        const size_t i = static_cast<size_t>(k);
        const int l = std::max(1, static_cast<int>(len[i]));
        r.final_scores[i] = raw[i] / dbs_hip::length_penalty(l, h.alpha);
        r.final_raw_scores[i] = raw[i];
        if (how.final_lengths) how.final_lengths[i] = len[i];
    }
    *rows_bytes = static_cast<int64_t>(rows.capacity() * sizeof(float));
    return r;
}

// ---------------------------------------------------------------------------
// Backward of a result
// ---------------------------------------------------------------------------

// The surrogate backward of one result (reference src/decoder.cpp:
// 540-663): the selected-beam weight gradients become per-slot score
// gradients w_k (gw_k - sum_j w_j gw_j) / temperature (the reference's
// first term of each slot's rank gradient), the device walks the paths with
// them and the final-score gradients, and its per-slot path gradients are
// the entries of the gradient and, at step 0, of the initial scores.
DBSBackwardHandle backward_of(DBSDecoderHandle& h, const DBSResultHandle& r, const float* gw, const float* grw,
                              const float* gf, bool sparse) {
    const int T = r.steps, K = r.beam_size, V = r.vocab_size;
    const size_t selected = mul(static_cast<size_t>(T), static_cast<size_t>(K), "selected gradient size overflow");
    const size_t dense = mul(selected, static_cast<size_t>(V), "dense gradient size overflow");
    if (!sparse && dense > static_cast<size_t>(h.max_dense_gradient_elements))
        throw std::length_error("dense gradient allocation exceeds max_dense_gradient_elements; use sparse backward");
    need(!grw || r.pool_size > 0,
         "relaxed-pool gradients need a relaxed pool: create the decoder with relaxed_pool_multiplier >= 1");
    // the relaxed weights' gradient enters as the pool entries' d
    PoolTerms pool;
    if (grw) {
        pool.P = r.pool_size;
        pool.parents = r.pool_parents.data();
        pool.tokens = r.pool_tokens.data();
        pool.lengths = r.pool_lengths.data();
        pool.from_logprob = r.pool_from_logprob.data();
        pool.d.resize(static_cast<size_t>(T) * static_cast<size_t>(pool.P));
        pool_entry_grads(T, pool.P, r.alpha, r.soft_topk_temperature, pool.parents, pool.lengths,
                         r.relaxed_weights.data(), grw, nullptr, nullptr, pool.d.data());
    }
    std::vector<float> g_scores;
    if (gw) {
        g_scores.assign(selected, 0.0f);
        for (int t = 0; t < T; ++t) {
            const size_t base = static_cast<size_t>(t) * K;
            const float* w = r.weights.data() + base;
            float dot = 0.0f;
            for (int k = 0; k < K; ++k) dot += w[k] * gw[base + k];
            for (int k = 0; k < K; ++k) g_scores[base + k] = (w[k] * (gw[base + k] - dot)) / r.selected_temperature;
        }
    }
    Grads g;
    g.final_scores = gf;
    g.scores = gw ? g_scores.data() : nullptr;
    const int32_t steps[1] = {T};
    const PoolTerms* pool_p = pool.P > 0 ? &pool : nullptr;
    std::vector<float> draws;
    if (gw || gf || pool_p)
        draws = path_draws(&h, 1, T, K, V, r.alpha, steps, r.parents.data(), r.tokens.data(), r.lengths.data(),
                           r.from_logprob.data(), g, pool_p);
    else
        draws.assign(selected, 0.0f);

    DBSBackwardHandle out;
    out.sparse = sparse;
    // the initial beams' gradient: step 0's selected draws, then its pool
    // entries' d (reference src/decoder.cpp:566-662)
    out.grad_initial_scores.assign(static_cast<size_t>(K), 0.0f);
    for (int k = 0; k < K; ++k) {
        const float d = draws[static_cast<size_t>(k)];
        const int p = r.parents[static_cast<size_t>(k)];
        if (p >= 0 && d != 0.0f) out.grad_initial_scores[static_cast<size_t>(p)] += d;
    }
    if (pool_p && T > 0) {
        for (int j = 0; j < pool.P; ++j) {
            const float d = pool.d[static_cast<size_t>(j)];
            const int p = pool.parents[j];
            if (p >= 0 && d != 0.0f) out.grad_initial_scores[static_cast<size_t>(p)] += d;
        }
    }
    // the log-prob entries, merged per entry in the reference's order
    if (!sparse) out.grad_log_probs.assign(dense, 0.0f);
    for (int t = 0; t < T; ++t) {
        for (const auto& e : step_entries(T, K, V, 0, t, draws, r.parents.data(), r.tokens.data(),
                                          r.from_logprob.data(), pool_p)) {
            if (sparse) {
                out.sparse_indices.push_back(e.first);
                out.sparse_values.push_back(e.second);
            } else {
                out.grad_log_probs[static_cast<size_t>(e.first)] += e.second;
            }
        }
    }
    return out;
}

int backward_entry(DBSDecoderHandle* handle, const DBSResultHandle* result, const float* gw, const float* grw,
                   const float* gf, DBSBackwardHandle** out_backward, bool sparse) {
    if (out_backward) *out_backward = nullptr;
    return run(handle, [&] {
        need(out_backward != nullptr, "out_backward cannot be null");
        need(result != nullptr, "result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        const auto start = std::chrono::steady_clock::now();
        auto b = std::make_unique<DBSBackwardHandle>(backward_of(h, *result, gw, grw, gf, sparse));
        stats_backward(&h, ns_since(start), sparse, static_cast<int64_t>(b->sparse_values.size()));
        *out_backward = b.release();
    });
}

template <class T>
const T* data_or_null(const std::vector<T>& v) {
    return v.empty() ? nullptr : v.data();
}

bool cpu_has(const char* feature) {
#if (defined(__x86_64__) || defined(__i386__)) && !defined(__HIP_DEVICE_COMPILE__)
    __builtin_cpu_init();
    if (std::string(feature) == "avx512") return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
    if (std::string(feature) == "avx2") return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    if (std::string(feature) == "sse42") return __builtin_cpu_supports("sse4.2");
#endif
    (void)feature;
    return false;
}

}  // namespace

namespace dbs_host {

void decode_batch_filtered(DBSDecoderHandle* hp, const void* inputs, int data_type, bool from_logits, int B, int T,
                           int V, const std::vector<int32_t>& steps_b, const DBSAdvancedConstraintsC* cons,
                           const DBSDecodeOutputsC* out, const DBSDecodeOutputsExC* ex) {
    DBSDecoderHandle& h = *hp;
    const int K = h.beam_size;
    const size_t block = static_cast<size_t>(K) * static_cast<size_t>(V);
    const size_t esize = dtype_bytes(data_type);
    const int P = ex && (ex->pool_parents || ex->pool_tokens || ex->pool_lengths || ex->pool_scores ||
                         ex->pool_raw_scores || ex->pool_from_logprob)
                      ? pool_size_of(K, h.pool_multiplier)
                      : 0;
    std::vector<float> lse;
    std::vector<int32_t> final_len(static_cast<size_t>(K));
    for (int b = 0; b < B; ++b) {
        const int steps = steps_b[static_cast<size_t>(b)];
        Constraints c = constraints_of(cons);
        c.batch_index = b;  // reference src/c_api.cpp:782-786
        const unsigned char* x = static_cast<const unsigned char*>(inputs) + static_cast<size_t>(b) * T * block * esize;
        StepRows how;
        how.from_logits = from_logits;
        lse.assign(static_cast<size_t>(steps) * K, 0.0f);
        how.row_lse = ex && ex->row_lse && from_logits ? lse.data() : nullptr;
        how.final_lengths = final_len.data();
        int64_t rows_bytes = 0;
        DBSResultHandle r;
        try {
            r = decode_model_steps(
                h, steps, V, &c,
                [&](const StepView& v, float* rows) {
                    const unsigned char* src = x + static_cast<size_t>(v.step) * block * esize;
                    if (data_type == DBS_DTYPE_F32) {
                        std::memcpy(rows, src, block * sizeof(float));
                        return;
                    }
                    const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
                    for (size_t i = 0; i < block; ++i)
                        rows[i] = data_type == DBS_DTYPE_F16 ? dbs_hip::half_to_f32(s16[i]) : dbs_hip::bf16_to_f32(s16[i]);
                },
                &rows_bytes, how);
        } catch (const std::invalid_argument& e) {
            example_error(b, e.what());
        }
        // the example's trace, padded past its steps (reference src/c_api.cpp:739-781)
        for (int t = 0; t < T; ++t) {
            for (int k = 0; k < K; ++k) {
                const size_t o = (static_cast<size_t>(b) * T + t) * K + k, i = static_cast<size_t>(t) * K + k;
                const bool live = t < steps;
                if (out->tokens) out->tokens[o] = live ? r.tokens[i] : -1;
                if (out->parents) out->parents[o] = live ? r.parents[i] : -1;
                if (out->lengths) out->lengths[o] = live ? r.lengths[i] : 0;
                if (out->scores) out->scores[o] = live ? r.scores[i] : kNegInf;
                if (out->raw_scores) out->raw_scores[o] = live ? r.raw_scores[i] : kNegInf;
                if (out->from_logprob) out->from_logprob[o] = live ? r.from_logprob[i] : 0;
                if (ex && ex->row_lse) ex->row_lse[o] = live && how.row_lse ? lse[i] : 0.0f;
            }
            for (int q = 0; q < P; ++q) {
                const size_t o = (static_cast<size_t>(b) * T + t) * P + q, i = static_cast<size_t>(t) * P + q;
                const bool live = t < steps;
                if (ex->pool_parents) ex->pool_parents[o] = live ? r.pool_parents[i] : -1;
                if (ex->pool_tokens) ex->pool_tokens[o] = live ? r.pool_tokens[i] : -1;
                if (ex->pool_lengths) ex->pool_lengths[o] = live ? r.pool_lengths[i] : 0;
                if (ex->pool_scores) ex->pool_scores[o] = live ? r.pool_scores[i] : kNegInf;
                if (ex->pool_raw_scores) ex->pool_raw_scores[o] = live ? r.pool_raw_scores[i] : kNegInf;
                if (ex->pool_from_logprob) ex->pool_from_logprob[o] = live ? r.pool_from_logprob[i] : 0;
            }
        }
        for (int k = 0; k < K; ++k) {
            const size_t o = static_cast<size_t>(b) * K + k;
            out->final_scores[o] = r.final_scores[static_cast<size_t>(k)];
            if (out->final_raw_scores) out->final_raw_scores[o] = r.final_raw_scores[static_cast<size_t>(k)];
            if (out->final_lengths) out->final_lengths[o] = final_len[static_cast<size_t>(k)];
        }
    }
}

}  // namespace dbs_host

extern "C" {

// ---- decodes into result handles (reference src/c_api.cpp:402-700) ----

DBS_EXPORT int dbs_decode_constrained_ex(DBSDecoderHandle* handle, const float* log_probs, int steps, int vocab_size,
                                         const DBSAdvancedConstraintsC* constraints, DBSResultHandle** out_result) {
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        const auto start = std::chrono::steady_clock::now();
        const Constraints c = constraints_of(constraints);
        const Constraints* cp = constraints ? &c : nullptr;
        need(log_probs != nullptr, "log_probs cannot be null");
        check_decode_args(h, h.beam_size, h.eos_token, steps, vocab_size, cp);
        check_served(h, cp);
        if (cp && cp->filter) {
            // a token filter: step by step, its verdicts from the host
            const size_t block = static_cast<size_t>(h.beam_size) * static_cast<size_t>(vocab_size);
            int64_t rows_bytes = 0;
            auto r = std::make_unique<DBSResultHandle>(decode_model_steps(
                h, steps, vocab_size, cp,
                [&](const StepView& v, float* rows) {
                    std::copy_n(log_probs + static_cast<size_t>(v.step) * block, block, rows);
                },
                &rows_bytes));
            record_result_stats(h, *r, ns_since(start), false);
            *out_result = r.release();
            return;
        }
        BatchSpec s;
        s.inputs = log_probs;
        s.B = 1;
        s.T = steps;
        s.K = h.beam_size;
        s.V = vocab_size;
        s.cons = cp;
        s.batch_errors = false;
        auto r = std::make_unique<DBSResultHandle>(std::move(decode_results(h, s)[0]));
        record_result_stats(h, *r, ns_since(start), false);
        *out_result = r.release();
    });
}

DBS_EXPORT int dbs_decode(DBSDecoderHandle* handle, const float* log_probs, int steps, int vocab_size,
                          DBSResultHandle** out_result) {
    return dbs_decode_constrained_ex(handle, log_probs, steps, vocab_size, nullptr, out_result);
}

DBS_EXPORT int dbs_decode_constrained(DBSDecoderHandle* handle, const float* log_probs, int steps, int vocab_size,
                                      const uint8_t* banned_tokens, const int32_t* forced_tokens, int min_length,
                                      DBSResultHandle** out_result) {
    DBSAdvancedConstraintsC c{};
    c.banned_tokens = banned_tokens;
    c.forced_tokens = forced_tokens;
    c.min_length = min_length;
    c.repetition_penalty = 1.0f;
    return dbs_decode_constrained_ex(handle, log_probs, steps, vocab_size, &c, out_result);
}

DBS_EXPORT int dbs_decode_typed(DBSDecoderHandle* handle, const void* log_probs, int data_type, int steps,
                                int vocab_size, DBSResultHandle** out_result) {
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        check_dtype(data_type);
        const auto start = std::chrono::steady_clock::now();
        need(log_probs != nullptr, "log_probs cannot be null");
        check_decode_args(h, h.beam_size, h.eos_token, steps, vocab_size, nullptr);
        check_served(h, nullptr);
        BatchSpec s;
        s.inputs = log_probs;
        s.data_type = data_type;
        s.B = 1;
        s.T = steps;
        s.K = h.beam_size;
        s.V = vocab_size;
        s.batch_errors = false;
        auto r = std::make_unique<DBSResultHandle>(std::move(decode_results(h, s)[0]));
        record_result_stats(h, *r, ns_since(start), false);
        *out_result = r.release();
    });
}

DBS_EXPORT int dbs_decode_batch_typed(DBSDecoderHandle* handle, const void* log_probs, int data_type, int batch_size,
                                      int steps, int vocab_size, int num_threads, DBSBatchResultHandle** out_result) {
    (void)num_threads;
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        check_dtype(data_type);
        need(log_probs != nullptr, "log_probs cannot be null");
        need(batch_size > 0 && steps > 0 && vocab_size > 0, "batch_size, steps and vocab_size must be positive");
        const auto start = std::chrono::steady_clock::now();
        const size_t stride = mul(mul(static_cast<size_t>(steps), static_cast<size_t>(h.beam_size),
                                      "batch stride overflow"),
                                  static_cast<size_t>(vocab_size), "batch stride overflow");
        (void)mul(stride, static_cast<size_t>(batch_size), "batch size overflow");
        (void)mul(stride, dtype_bytes(data_type), "batch stride overflow");
        try {
            check_decode_args(h, h.beam_size, h.eos_token, steps, vocab_size, nullptr);
        } catch (const std::invalid_argument& e) {
            example_error(0, e.what());  // the options are shared: example 0 fails first
        }
        check_served(h, nullptr);
        BatchSpec s;
        s.inputs = log_probs;
        s.data_type = data_type;
        s.B = batch_size;
        s.T = steps;
        s.K = h.beam_size;
        s.V = vocab_size;
        auto br = std::make_unique<DBSBatchResultHandle>();
        br->results = decode_results(h, s);
        record_result_stats(h, br->results.front(), ns_since(start), false);
        *out_result = br.release();
    });
}

DBS_EXPORT int dbs_decode_batch(DBSDecoderHandle* handle, const float* log_probs, int batch_size, int steps,
                                int vocab_size, int num_threads, DBSBatchResultHandle** out_result) {
    return dbs_decode_batch_typed(handle, log_probs, DBS_DTYPE_F32, batch_size, steps, vocab_size, num_threads,
                                  out_result);
}

DBS_EXPORT int dbs_decode_batch_variable(DBSDecoderHandle* handle, const float* log_probs, int batch_size,
                                         int max_steps, int max_beam_size, int vocab_size,
                                         const int32_t* steps_per_example, const int32_t* beam_sizes_per_example,
                                         const int32_t* eos_tokens_per_example,
                                         const int32_t* min_lengths_per_example,
                                         const uint8_t* banned_tokens_per_example,
                                         const int32_t* forced_tokens_per_example, int num_threads,
                                         DBSBatchResultHandle** out_result) {
    (void)num_threads;
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        need(log_probs != nullptr, "log_probs cannot be null");
        need(batch_size > 0 && max_steps > 0 && max_beam_size > 0 && vocab_size > 0,
             "batch_size, max_steps, max_beam_size and vocab_size must be positive");
        const auto start = std::chrono::steady_clock::now();
        const size_t step_stride = mul(static_cast<size_t>(max_beam_size), static_cast<size_t>(vocab_size),
                                       "variable batch stride overflow");
        const size_t input_stride = mul(step_stride, static_cast<size_t>(max_steps), "variable batch stride overflow");
        (void)mul(input_stride, static_cast<size_t>(batch_size), "variable batch size overflow");
        // every example's own options and constraints, checked as the
        // reference's per-example decoders do (reference src/c_api.cpp:
        // 659-690, src/decoder.cpp:697-721, 385-406), the first failing
        // example reported
        std::vector<int32_t> steps_b(static_cast<size_t>(batch_size)), beams_b(static_cast<size_t>(batch_size)),
            eos_b(static_cast<size_t>(batch_size)), min_b(static_cast<size_t>(batch_size));
        for (int b = 0; b < batch_size; ++b) {
            try {
                const int st = steps_per_example ? steps_per_example[b] : max_steps;
                const int beam = beam_sizes_per_example ? beam_sizes_per_example[b] : h.beam_size;
                need(st > 0 && st <= max_steps, "per-example steps must be in [1, max_steps]");
                need(beam > 0 && beam <= max_beam_size, "per-example beam size must be in [1, max_beam_size]");
                const int eos = eos_tokens_per_example ? eos_tokens_per_example[b] : h.eos_token;
                need(eos >= -1, "eos_token must be -1 (disabled) or a token id");
                need(h.extra_eos.empty() || eos >= 0,
                     "extra EOS tokens need EOS handling: set eos_token to one of the EOS tokens");
                Constraints c;
                c.forced = forced_tokens_per_example ? forced_tokens_per_example + static_cast<size_t>(b) * max_steps
                                                     : nullptr;
                check_decode_args(h, beam, eos, st, vocab_size, &c);
                steps_b[static_cast<size_t>(b)] = st;
                beams_b[static_cast<size_t>(b)] = beam;
                eos_b[static_cast<size_t>(b)] = eos;
                min_b[static_cast<size_t>(b)] = min_lengths_per_example ? std::max(0, min_lengths_per_example[b])
                                                                        : h.min_length;
            } catch (const std::invalid_argument& e) {
                example_error(b, e.what());
            }
        }
        check_served(h, nullptr);
        BatchSpec s;
        s.inputs = log_probs;
        s.B = batch_size;
        s.T = max_steps;
        s.K = max_beam_size;
        s.V = vocab_size;
        s.steps = steps_b.data();
        s.beams = beams_b.data();
        s.eos = eos_b.data();
        s.min_lengths = min_b.data();
        s.banned_pe = banned_tokens_per_example;
        s.forced_pe = forced_tokens_per_example;
        auto br = std::make_unique<DBSBatchResultHandle>();
        br->results = decode_results(h, s);
        record_result_stats(h, br->results.front(), ns_since(start), false);
        *out_result = br.release();
    });
}

// ---- model-in-the-loop decodes (reference src/c_api.cpp:281-300, 513-606) ----

DBS_EXPORT int dbs_decode_model_steps_with_workspace(DBSDecoderHandle* handle, DBSWorkspaceHandle* workspace,
                                                     DBSModelStepFn step_fn, void* user_data, int batch_index,
                                                     int steps, int vocab_size, DBSResultHandle** out_result) {
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(workspace != nullptr, "workspace cannot be null");
        need(step_fn != nullptr, "model step callback cannot be null");
        std::lock_guard<std::mutex> lock(workspace->mutex);
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        const auto start = std::chrono::steady_clock::now();
        std::vector<float> zeros;
        int64_t rows_bytes = 0;
        DBSResultHandle r = decode_model_steps(h, steps, vocab_size, nullptr, [&](const StepView& v, float* rows) {
            // this callback sees the previous tokens and scores (0 at step 0)
            const float* scores = v.scores;
            if (v.step == 0) {
                zeros.assign(static_cast<size_t>(h.beam_size), 0.0f);
                scores = zeros.data();
            }
            if (step_fn(user_data, batch_index, v.step, v.tokens, scores, h.beam_size, vocab_size, rows) != 0)
                throw std::runtime_error("model step callback returned non-zero status");
        }, &rows_bytes);
        workspace->f32.reserve(static_cast<size_t>(rows_bytes) / sizeof(float));
        auto out = std::make_unique<DBSResultHandle>(std::move(r));
        record_result_stats(h, *out, ns_since(start), true, rows_bytes);
        *out_result = out.release();
    });
}

DBS_EXPORT int dbs_decode_model_steps(DBSDecoderHandle* handle, DBSModelStepFn step_fn, void* user_data,
                                      int batch_index, int steps, int vocab_size, DBSResultHandle** out_result) {
    DBSWorkspaceHandle local;
    return dbs_decode_model_steps_with_workspace(handle, &local, step_fn, user_data, batch_index, steps, vocab_size,
                                                 out_result);
}

DBS_EXPORT int dbs_decode_model_steps_ex(DBSDecoderHandle* handle, DBSModelStepExFn step_fn, void* user_data,
                                         int batch_index, int steps, int vocab_size,
                                         const DBSAdvancedConstraintsC* constraints, DBSResultHandle** out_result) {
    if (out_result) *out_result = nullptr;
    return run(handle, [&] {
        need(step_fn != nullptr, "model step callback cannot be null");
        need(out_result != nullptr, "out_result cannot be null");
        DBSDecoderHandle& h = handle_of(handle);
        const auto start = std::chrono::steady_clock::now();
        Constraints c = constraints_of(constraints);
        c.batch_index = batch_index;  // what a token filter is told (reference src/c_api.cpp:592-596)
        int64_t rows_bytes = 0;
        DBSResultHandle r = decode_model_steps(h, steps, vocab_size, constraints ? &c : nullptr,
                                               [&](const StepView& v, float* rows) {
            DBSModelStepInfoC info{};
            info.batch_index = batch_index;
            info.step = v.step;
            info.beam_size = h.beam_size;
            info.vocab_size = vocab_size;
            info.parents = v.parents;
            info.tokens = v.tokens;
            info.lengths = v.lengths;
            info.scores = v.scores;
            info.raw_scores = v.raw_scores;
            info.finished = v.finished;
            info.prefixes = v.prefixes;
            if (step_fn(user_data, &info, rows) != 0)
                throw std::runtime_error("model step callback returned non-zero status");
        }, &rows_bytes);
        auto out = std::make_unique<DBSResultHandle>(std::move(r));
        record_result_stats(h, *out, ns_since(start), true, rows_bytes);
        *out_result = out.release();
    });
}

// ---- backward of a result (reference src/c_api.cpp:985-1049) ----

DBS_EXPORT int dbs_backward_dense(DBSDecoderHandle* handle, const DBSResultHandle* result,
                                  const float* grad_selected_weights, const float* grad_relaxed_weights,
                                  const float* grad_final_scores, DBSBackwardHandle** out_backward) {
    return backward_entry(handle, result, grad_selected_weights, grad_relaxed_weights, grad_final_scores,
                          out_backward, false);
}

DBS_EXPORT int dbs_backward_sparse(DBSDecoderHandle* handle, const DBSResultHandle* result,
                                   const float* grad_selected_weights, const float* grad_relaxed_weights,
                                   const float* grad_final_scores, DBSBackwardHandle** out_backward) {
    return backward_entry(handle, result, grad_selected_weights, grad_relaxed_weights, grad_final_scores,
                          out_backward, true);
}

DBS_EXPORT int dbs_backward(DBSDecoderHandle* handle, const DBSResultHandle* result,
                            const float* grad_selected_weights, const float* grad_relaxed_weights,
                            const float* grad_final_scores, DBSBackwardHandle** out_backward) {
    return dbs_backward_sparse(handle, result, grad_selected_weights, grad_relaxed_weights, grad_final_scores,
                               out_backward);
}

DBS_EXPORT int dbs_backward_default(DBSDecoderHandle* handle, const DBSResultHandle* result,
                                    const float* grad_selected_weights, const float* grad_relaxed_weights,
                                    const float* grad_final_scores, DBSBackwardHandle** out_backward) {
    return dbs_backward_sparse(handle, result, grad_selected_weights, grad_relaxed_weights, grad_final_scores,
                               out_backward);
}

// ---- handles and accessors ----

DBS_EXPORT void dbs_free_result(DBSResultHandle* result) { delete result; }
DBS_EXPORT void dbs_free_batch_result(DBSBatchResultHandle* result) { delete result; }
DBS_EXPORT void dbs_free_backward(DBSBackwardHandle* result) { delete result; }

DBS_EXPORT int dbs_batch_result_size(const DBSBatchResultHandle* result) {
    return result ? static_cast<int>(result->results.size()) : 0;
}

DBS_EXPORT const DBSResultHandle* dbs_batch_result_at(const DBSBatchResultHandle* result, int batch_index) {
    if (!result || batch_index < 0 || batch_index >= static_cast<int>(result->results.size())) return nullptr;
    return &result->results[static_cast<size_t>(batch_index)];
}

DBS_EXPORT int dbs_result_steps(const DBSResultHandle* r) { return r ? r->steps : 0; }
DBS_EXPORT int dbs_result_beam_size(const DBSResultHandle* r) { return r ? r->beam_size : 0; }
DBS_EXPORT int dbs_result_vocab_size(const DBSResultHandle* r) { return r ? r->vocab_size : 0; }
DBS_EXPORT int dbs_result_pool_size(const DBSResultHandle* r) { return r ? r->pool_size : 0; }
DBS_EXPORT const int32_t* dbs_result_tokens(const DBSResultHandle* r) { return r ? data_or_null(r->tokens) : nullptr; }
DBS_EXPORT const int32_t* dbs_result_parents(const DBSResultHandle* r) {
    return r ? data_or_null(r->parents) : nullptr;
}
DBS_EXPORT const int32_t* dbs_result_lengths(const DBSResultHandle* r) {
    return r ? data_or_null(r->lengths) : nullptr;
}
DBS_EXPORT const float* dbs_result_scores(const DBSResultHandle* r) { return r ? data_or_null(r->scores) : nullptr; }
DBS_EXPORT const float* dbs_result_raw_scores(const DBSResultHandle* r) {
    return r ? data_or_null(r->raw_scores) : nullptr;
}
DBS_EXPORT const float* dbs_result_weights(const DBSResultHandle* r) { return r ? data_or_null(r->weights) : nullptr; }
DBS_EXPORT const float* dbs_result_final_scores(const DBSResultHandle* r) {
    return r ? data_or_null(r->final_scores) : nullptr;
}
DBS_EXPORT const float* dbs_result_final_raw_scores(const DBSResultHandle* r) {
    return r ? data_or_null(r->final_raw_scores) : nullptr;
}
// the relaxed pool's arrays (NULL without a pool)
DBS_EXPORT const float* dbs_result_relaxed_weights(const DBSResultHandle* r) {
    return r ? data_or_null(r->relaxed_weights) : nullptr;
}
DBS_EXPORT const int32_t* dbs_result_pool_tokens(const DBSResultHandle* r) {
    return r ? data_or_null(r->pool_tokens) : nullptr;
}
DBS_EXPORT const int32_t* dbs_result_pool_parents(const DBSResultHandle* r) {
    return r ? data_or_null(r->pool_parents) : nullptr;
}
DBS_EXPORT const int32_t* dbs_result_pool_lengths(const DBSResultHandle* r) {
    return r ? data_or_null(r->pool_lengths) : nullptr;
}
DBS_EXPORT const float* dbs_result_pool_scores(const DBSResultHandle* r) {
    return r ? data_or_null(r->pool_scores) : nullptr;
}
DBS_EXPORT const float* dbs_result_pool_raw_scores(const DBSResultHandle* r) {
    return r ? data_or_null(r->pool_raw_scores) : nullptr;
}

DBS_EXPORT const float* dbs_backward_grad_log_probs(const DBSBackwardHandle* b) {
    return b ? data_or_null(b->grad_log_probs) : nullptr;
}
DBS_EXPORT const float* dbs_backward_grad_initial_scores(const DBSBackwardHandle* b) {
    return b ? data_or_null(b->grad_initial_scores) : nullptr;
}
DBS_EXPORT const int64_t* dbs_backward_sparse_logprob_indices(const DBSBackwardHandle* b) {
    return b ? data_or_null(b->sparse_indices) : nullptr;
}
DBS_EXPORT const float* dbs_backward_sparse_logprob_values(const DBSBackwardHandle* b) {
    return b ? data_or_null(b->sparse_values) : nullptr;
}
DBS_EXPORT int64_t dbs_backward_sparse_logprob_count(const DBSBackwardHandle* b) {
    return b ? static_cast<int64_t>(b->sparse_values.size()) : 0;
}
DBS_EXPORT int dbs_backward_is_sparse(const DBSBackwardHandle* b) { return b && b->sparse ? 1 : 0; }

DBS_EXPORT int64_t dbs_result_selected_count(const DBSResultHandle* r) {
    return r ? static_cast<int64_t>(r->steps) * r->beam_size : 0;
}
DBS_EXPORT int64_t dbs_result_pool_count(const DBSResultHandle* r) {
    return r ? static_cast<int64_t>(r->steps) * r->pool_size : 0;
}
DBS_EXPORT int64_t dbs_result_logprob_count(const DBSResultHandle* r) {
    return r ? static_cast<int64_t>(r->steps) * r->beam_size * r->vocab_size : 0;
}
DBS_EXPORT int64_t dbs_backward_grad_log_probs_count(const DBSResultHandle* r) { return dbs_result_logprob_count(r); }
DBS_EXPORT int64_t dbs_backward_grad_initial_scores_count(const DBSResultHandle* r) { return r ? r->beam_size : 0; }

DBS_EXPORT int64_t dbs_result_eos_count(const DBSResultHandle* r, int eos_token) {
    if (!r || eos_token < 0) return 0;
    return static_cast<int64_t>(std::count(r->tokens.begin(), r->tokens.end(), eos_token));
}

// 0 when every step's beams are in the search's strict candidate order,
// -3 for scores out of order, -4 for a tie broken out of order, -1 for NULL
// (reference src/c_api.cpp:1195-1211; the order is the decode's own).
DBS_EXPORT int dbs_result_validate_deterministic_order(const DBSResultHandle* r) {
    if (!r) return -1;
    const int T = r->steps, K = r->beam_size;
    for (int t = 0; t < T; ++t) {
        for (int k = 1; k < K; ++k) {
            const size_t p = static_cast<size_t>(t) * K + static_cast<size_t>(k - 1), c = p + 1;
            const dbs_hip::Cand a{r->scores[p], r->raw_scores[p], r->parents[p], r->tokens[p], r->lengths[p],
                                  r->from_logprob[p]};
            const dbs_hip::Cand b{r->scores[c], r->raw_scores[c], r->parents[c], r->tokens[c], r->lengths[c],
                                  r->from_logprob[c]};
            if (!dbs_hip::before(b, a)) continue;
            return b.score > a.score ? -3 : -4;
        }
    }
    return 0;
}

DBS_EXPORT int dbs_result_summary_json(const DBSResultHandle* r, int eos_token, char* out_json,
                                       int64_t out_json_capacity) {
    if (!r || !out_json || out_json_capacity <= 0) {
        record(nullptr, "result and out_json cannot be null, and the capacity must be positive", 1);
        return DBS_ERROR_INVALID_ARGUMENT;
    }
    int min_len = r->lengths.empty() ? 0 : std::numeric_limits<int>::max();
    int max_len = 0;
    for (int32_t len : r->lengths) {
        min_len = std::min(min_len, static_cast<int>(len));
        max_len = std::max(max_len, static_cast<int>(len));
    }
    float min_final = r->final_scores.empty() ? 0.0f : r->final_scores[0];
    float max_final = min_final;
    for (float s : r->final_scores) {
        min_final = std::min(min_final, s);
        max_final = std::max(max_final, s);
    }
    const int n = std::snprintf(
        out_json, static_cast<size_t>(out_json_capacity),
        "{\"abi_version\":%d,\"steps\":%d,\"beam_size\":%d,\"vocab_size\":%d,\"selected_count\":%lld,"
        "\"pool_count\":%lld,\"eos_token\":%d,\"eos_count\":%lld,\"min_length\":%d,\"max_length\":%d,"
        "\"min_final_score\":%.9g,\"max_final_score\":%.9g,\"deterministic_order\":%d}",
        DBS_ABI_VERSION, r->steps, r->beam_size, r->vocab_size,
        static_cast<long long>(dbs_result_selected_count(r)), static_cast<long long>(dbs_result_pool_count(r)),
        eos_token,
        static_cast<long long>(dbs_result_eos_count(r, eos_token)), min_len, max_len, static_cast<double>(min_final),
        static_cast<double>(max_final), dbs_result_validate_deterministic_order(r) == 0 ? 1 : 0);
    if (n < 0) {
        record(nullptr, "formatting the summary failed", 2);
        return DBS_ERROR_RUNTIME;
    }
    return n < out_json_capacity ? 0 : 1;
}

// ---- statistics, determinism, allocator and host queries ----

DBS_EXPORT int dbs_get_stats(DBSDecoderHandle* handle, DBSStatsC* out_stats) {
    return run(nullptr, [&] {
        need(handle != nullptr && out_stats != nullptr, "handle and out_stats cannot be null");
        std::lock_guard<std::mutex> lock(handle->stats_mutex);
        *out_stats = handle->stats;
        out_stats->total_allocator_calls = g_device_allocations.load(std::memory_order_relaxed);
        out_stats->total_allocator_bytes = g_device_bytes.load(std::memory_order_relaxed);
    });
}

DBS_EXPORT int dbs_get_stats_json(DBSDecoderHandle* handle, char* out_json, int64_t out_json_capacity) {
    if (!handle || !out_json || out_json_capacity <= 0) {
        record(nullptr, "handle and out_json cannot be null, and the capacity must be positive", 1);
        return DBS_ERROR_INVALID_ARGUMENT;
    }
    DBSStatsC s{};
    const int rc = dbs_get_stats(handle, &s);
    if (rc != DBS_OK) return rc;
    const int n = std::snprintf(
        out_json, static_cast<size_t>(out_json_capacity),
        "{\"abi_version\":%d,\"kernel\":\"%s\",\"used_sparse_backward\":%d,\"used_dense_backward\":%d,"
        "\"batch_threads\":%d,\"model_step\":%d,\"last_error_category\":%d,\"decode_ns\":%lld,\"backward_ns\":%lld,"
        "\"allocation_bytes\":%lld,\"selected_count\":%lld,\"pool_count\":%lld,\"logprob_count\":%lld,"
        "\"sparse_grad_count\":%lld,\"allocator_calls\":%lld,\"allocator_bytes\":%lld}",
        s.abi_version, "hip-gfx950", s.used_sparse_backward, s.used_dense_backward, s.used_batch_threads,
        s.used_model_step_callback, s.last_error_category, static_cast<long long>(s.last_decode_ns),
        static_cast<long long>(s.last_backward_ns), static_cast<long long>(s.last_allocation_bytes),
        static_cast<long long>(s.last_selected_count), static_cast<long long>(s.last_pool_count),
        static_cast<long long>(s.last_logprob_count), static_cast<long long>(s.last_sparse_grad_count),
        static_cast<long long>(s.total_allocator_calls), static_cast<long long>(s.total_allocator_bytes));
    if (n < 0) {
        record(nullptr, "formatting stats failed", 2);
        return DBS_ERROR_RUNTIME;
    }
    return n < out_json_capacity ? 0 : 1;
}

DBS_EXPORT void dbs_reset_stats(DBSDecoderHandle* handle) {
    if (!handle) return;
    std::lock_guard<std::mutex> lock(handle->stats_mutex);
    handle->stats = DBSStatsC{};
    handle->stats.abi_version = DBS_ABI_VERSION;
    handle->stats.last_kernel = kKernelHip;
}

// Decoding uses no randomness and a strict total order over candidates.
DBS_EXPORT int dbs_is_deterministic(void) { return 1; }

DBS_EXPORT int dbs_set_deterministic_seed(DBSDecoderHandle* handle, uint64_t seed) {
    return run(nullptr, [&] {
        need(handle != nullptr, "handle cannot be null");
        handle->seed.store(seed, std::memory_order_relaxed);
    });
}

DBS_EXPORT uint64_t dbs_get_deterministic_seed(DBSDecoderHandle* handle) {
    return handle ? handle->seed.load(std::memory_order_relaxed) : 0;
}

// The library's allocator statistics are its handles' device buffers: the
// allocations made since the last reset, and the bytes held now (a gauge).
DBS_EXPORT void dbs_allocator_counters_reset(void) { g_device_allocations.store(0, std::memory_order_relaxed); }
DBS_EXPORT int64_t dbs_allocator_call_count(void) { return g_device_allocations.load(std::memory_order_relaxed); }
DBS_EXPORT int64_t dbs_allocator_byte_count(void) { return g_device_bytes.load(std::memory_order_relaxed); }

// The host CPU's vector extensions (the reference picks its kernels by them;
// this library decodes on the GPU whatever they are).
DBS_EXPORT int dbs_has_avx512(void) { return cpu_has("avx512") ? 1 : 0; }
DBS_EXPORT int dbs_has_avx2(void) { return cpu_has("avx2") ? 1 : 0; }
DBS_EXPORT int dbs_has_sse42(void) { return cpu_has("sse42") ? 1 : 0; }
DBS_EXPORT int dbs_has_neon(void) { return 0; }

// ---- workspaces (the model-step decodes' host row buffer) ----

DBS_EXPORT int dbs_workspace_create(DBSWorkspaceHandle** out_workspace) {
    if (out_workspace) *out_workspace = nullptr;
    return run(nullptr, [&] {
        need(out_workspace != nullptr, "out_workspace cannot be null");
        *out_workspace = new DBSWorkspaceHandle;
    });
}

DBS_EXPORT void dbs_workspace_destroy(DBSWorkspaceHandle* workspace) { delete workspace; }

DBS_EXPORT int dbs_workspace_reserve(DBSWorkspaceHandle* workspace, int64_t float_count, int64_t int_count) {
    return run(nullptr, [&] {
        need(workspace != nullptr, "workspace cannot be null");
        need(float_count >= 0 && int_count >= 0, "reserve counts cannot be negative");
        std::lock_guard<std::mutex> lock(workspace->mutex);
        workspace->f32.reserve(static_cast<size_t>(float_count));
        workspace->i32.reserve(static_cast<size_t>(int_count));
    });
}

DBS_EXPORT int64_t dbs_workspace_allocated_bytes(DBSWorkspaceHandle* workspace) {
    if (!workspace) return 0;
    std::lock_guard<std::mutex> lock(workspace->mutex);
    return static_cast<int64_t>(workspace->f32.capacity() * sizeof(float) + workspace->i32.capacity() * sizeof(int32_t));
}

}  // extern "C"
