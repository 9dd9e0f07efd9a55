// SPDX-License-Identifier: MIT
//
// Internal interface between the C ABI (api.hip) and the kernels of
// libdbs_hip (decode.hip, backward.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stddef.h>
#include <stdint.h>

#include "numerics.hpp"

namespace dbs_hip {

// Kernel kinds of the optional launch timer (dbs_hip_profile_* in dbs_hip.h).
enum KernelKind : int { kKindRowPass = 0, kKindSelect = 1, kKindPathWalk = 2, kKindDense = 3, kKindBacktrack = 4,
                        kKindCount = 5 };

// Brackets the launches made in its scope with HIP events on `stream` when
// profiling is on; the durations are read back by dbs_hip_profile_read.
class KernelTimer {
public:
    KernelTimer(int kind, hipStream_t stream);
    ~KernelTimer();
    KernelTimer(const KernelTimer&) = delete;
    KernelTimer& operator=(const KernelTimer&) = delete;

private:
    int kind_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
    hipEvent_t stop_ = nullptr;
};

constexpr int kMaxEos = 17;          // eos_token + 16 extra EOS tokens
constexpr int kRowThreads = 64;      // one wavefront per row in the row pass
constexpr int kLanes = 256;          // lanes of the fixed logsumexp fold order
constexpr int kSurvivorCap = 512;    // row-pass candidates kept per row before overflow
constexpr int kSelectThreads = 256;  // one workgroup per example in the select pass
constexpr int kRound = kSelectThreads;      // candidates offered per collector round (one per thread)

// Per-row result of the row pass. In the overlapped decode every 8-byte
// half of it, and every shortlist entry, is published as one 64-bit atomic
// word whose upper half carries a non-zero tag (count + 2, invalid + 1,
// token + 1) over a workspace cleared before the row pass: a reader that
// sees the tag has the whole word, so no ordering between words is needed.
struct RowInfo {
    float lse;     // logsumexp of the row (from logits), else 0
    int32_t count; // shortlist entries; -1: no usable shortlist (the select pass rescans the row)
    float bound;   // upper bound on the log-prob of every allowed token not in the shortlist (-inf: none)
    uint32_t invalid;  // the row holds NaN or +inf
};

struct ShortEntry {
    float lp;
    int32_t token;
};

// Everything the decode kernels read; passed by value.
struct DecodeParams {
    const void* x;            // [B, T, K, V] (decode) or [B, K, V] (step)
    int dtype;
    int from_logits;
    int B, T, K, V;
    int eos;                  // -1: no EOS handling (eos_pe null)
    int n_eos;                // size of eos_set (0 when eos < 0)
    int32_t eos_set[kMaxEos]; // every EOS token, sorted, distinct (with eos_pe: the extra EOS tokens only)
    int min_length;
    // per example (reference include/dbs_cuda.h:80-85; null: the scalars above)
    const int32_t* beam_pe;   // device [B] beams in [1, K]: slots past them stay empty
    const int32_t* eos_pe;    // device [B] EOS token in [-1, V); the extra EOS tokens count only where >= 0
    const int32_t* minlen_pe; // device [B] minimum length >= 0
    float alpha;
    int ngram;
    int penalise;
    float log_rep;            // logf(repetition_penalty) when penalise
    int constrained;          // ngram > 0 || penalise
    int M;                    // shortlist length; 0: every read row is rescanned
    int use_tau;              // prefilter by the K-th shortlist candidate of each row
    const int32_t* steps;     // device [B] or null
    const uint8_t* banned;    // device [V] or null
    const uint8_t* banned_pe; // device [B, V] or null
    // device [B, T] (step mode: [B]) or null: an entry >= 0 is the one token
    // a read beam may take at that step (reference src/decoder.cpp:125)
    const int32_t* forced;
    // step mode, device [B, K, V] or null: 1 where a token filter refused
    // the token for that row (reference src/decoder.cpp:259-282); every read
    // row is then read in full by the select pass (no shortlists)
    const uint8_t* row_mask;
    // Relaxed pool (reference src/decoder.cpp:40, 294-306): with pool_mult
    // m >= 1 each step keeps the best m * beams candidates of an example, its
    // pool, of which the first beams are the selection. Outputs [B, T, m * K]
    // (any may be null); entries past the kept ones, and steps past an
    // example's own, are dead (parent and token -1, length 0, -inf scores).
    int pool_mult;
    int32_t* pool_parents;
    int32_t* pool_tokens;
    int32_t* pool_lengths;
    float* pool_scores;
    float* pool_raw;
    uint8_t* pool_flp;
    RowInfo* rowinfo;         // [rows]
    ShortEntry* shortlist;    // [rows, M]
    int32_t* prefix;          // [B, 2, K, P] when constrained and not kept in LDS (P = prefix capacity)
    int32_t* blocked;         // [B, K, P] n-gram-blocked tokens when not kept in LDS
    int prefix_cap;
    // outputs (any may be null except final_scores in decode mode)
    float* final_scores;
    float* final_raw;
    int32_t* final_lengths;
    int32_t* tokens;
    int32_t* parents;
    int32_t* lengths;
    float* scores;
    float* raw_scores;
    uint8_t* from_logprob;
    uint8_t* invalid;
    float* row_lse;
    // step mode: one step from an explicit state ([B, K] arrays, updated in place)
    int step_mode;
    float* st_raw;
    int32_t* st_len;
    uint8_t* st_fin;
    const int32_t* st_prefix;  // [B, K, st_stride]
    int st_stride;
    // Overlapped decode (null: the select pass runs after the row pass): the
    // row pass hands out rows step-major through row_ticket and counts the
    // finished rows of each (example, step) in step_done [B, T]; the select
    // pass waits for a step's count, then reads the step's tagged words
    // (waiting on any not yet written).
    int32_t* step_done;
    unsigned long long* row_ticket;
    int reserve_cus;  // CUs the persistent row-pass kernels leave free (the select pass's workgroups)
    int select_hold;  // the select pass claims its SIMDs' registers (beside a row pass of one workgroup per row)
    // A select-pass wait that gives up (bounded by wait_ticks of the 100 MHz
    // counter) sets *fault and marks its example invalid (2); the example's
    // remaining steps are written as padding. wait_extra raises the count a
    // wait needs (a test knob: the count is then never reached).
    int32_t* fault;
    unsigned long long wait_ticks;
    int wait_extra;
    // Split launch of a select pass started before its row pass (null: one
    // launch): the early launch (early = 1) takes example b only once the
    // row pass has counted its first row within early_ticks, and marks it in
    // claimed [B]; the late launch, submitted after the row pass, takes the
    // examples left. Two streams that share one hardware queue run the three
    // launches in submission order: the early launch then takes none, and no
    // wait depends on a launch queued behind it.
    int32_t* claimed;
    int early;
    unsigned long long early_ticks;
    // optional [B]: the first row holding NaN or +inf that example b's search
    // read, as t * K + k in reading order, or -1 (the host ABI's error text)
    int32_t* first_invalid;
};

// LDS plan of the select pass (byte offsets into its dynamic shared memory).
struct SelectLayout {
    int sort_cap;        // collector capacity (a power of two)
    int pen_len;         // length-penalty table entries (T + 2; 0 in step mode)
    size_t off_buf, off_rbuf, off_key, off_f32, off_i32, off_sl, off_prefix, off_blk, off_sig;
    int prefix_in_lds;   // the prefixes live in LDS (else in the workspace)
    int blk_in_lds;      // the n-gram-blocked lists live in LDS (else in the workspace)
    int sig_in_lds;      // the prefixes' token signatures are kept (LDS; needs the prefixes in LDS)
    int sig_words;       // 32-bit words per signature (256 or 64)
    size_t smem;
};

struct DecodeLayout {
    int M;
    int use_tau;
    int prefix_cap;
    SelectLayout sel;
    size_t off_rowinfo, off_short, off_prefix, off_blocked, off_sync, total;
};

// keep: candidates a step keeps per example (0: K; the relaxed pool keeps
// more), which sizes the shortlists and the select pass's collector.
DecodeLayout decode_layout(int B, int T, int K, int V, bool constrained, bool step_mode, int prefix_stride,
                           int keep = 0);
SelectLayout select_layout(int B, int T, int K, int M, bool constrained, bool step_mode, int prefix_cap,
                           int keep = 0);

// Queues the decode (or one step) on `stream` with workspace ws; returns a
// hipError_t.
// *fault: the overlapped decode's fault word in the workspace (non-zero once
// a select-pass wait gave up), or null when the passes ran one after the other
// (always so when allow_overlap is false).
hipError_t launch_decode(const DecodeParams& p, const DecodeLayout& L, hipStream_t stream, char* ws,
                         int32_t** fault, bool allow_overlap);
size_t sync_bytes(int B, int T);           // overlapped-decode counters in the workspace
extern std::atomic<int> g_overlap;         // dbs_hip_set_decode_overlap
hipError_t launch_row_pass(const DecodeParams& p, hipStream_t stream);
// Whether launch_row_pass would run one of the persistent (one workgroup per
// CU) row passes for p.
bool row_pass_persistent(const DecodeParams& p);
// Row pass that keeps each row on chip (16-bit rows, V % 8 == 0, 16-byte
// aligned, V <= 155648); launch_row_pass uses it when eligible.
bool row_resident_eligible(const DecodeParams& p);
hipError_t launch_row_resident(const DecodeParams& p, int64_t rows, hipStream_t stream);
bool row_pipe_eligible(const DecodeParams& p);
// bfloat16 logits, both segments of a 512-thread workgroup relaying (row_relay.hip)
bool row_relay_eligible(const DecodeParams& p);
// The relay row pass is the default for the rows it fills (it always folds
// its full register capacity, so shorter rows take the resident pass).
bool row_relay_preferred(const DecodeParams& p);
hipError_t launch_row_relay(const DecodeParams& p, int64_t rows, hipStream_t stream);
bool row_logprob_eligible(const DecodeParams& p);
hipError_t launch_row_logprob(const DecodeParams& p, int64_t rows, hipStream_t stream);
extern std::atomic<int> g_row_pass_kind;  // dbs_hip_set_row_pass
hipError_t launch_row_pipe(const DecodeParams& p, int64_t rows, hipStream_t stream);
hipError_t launch_select(const DecodeParams& p, const SelectLayout& L, hipStream_t stream);
// The select pass runs one wavefront per example (narrow, unconstrained
// decodes with shortlists) instead of one workgroup; dbs_hip_set_select_pass
// (g_select_kind 1) keeps the workgroup pass.
bool select_narrow(const DecodeParams& p);
extern std::atomic<int> g_select_kind;
// CUs the overlapped decode leaves free for the select pass.
int select_reserve_cus(const DecodeParams& p);

// Rows the select pass rescanned in full (reset = 1 clears the count).
hipError_t rescan_counter(int reset, unsigned long long* value);
// Select-pass waits for a step that gave up (the overlapped decode's bounded
// wait; nonzero means results may be wrong). reset / read like rescan_counter.
hipError_t wait_timeout_counter(int reset, unsigned long long* value);

// Elementwise helpers.

// A decode trace's int32 / uint8 outputs widened for torch (int64, bool), and
// the per-example steps (T where steps is null).
struct WidenTrace {
    const int32_t *final_len, *tokens, *parents, *lengths, *steps;
    const uint8_t* flp;
    int64_t *final_len64, *tokens64, *parents64, *lengths64, *steps64;
    uint8_t* flp_bool;
    int64_t n_final, n_trace, n_steps;
    int T;
};
hipError_t launch_widen_trace(const WidenTrace& w, hipStream_t stream);
// The read-back that ends a decode: `bytes` bytes at `src` (written only by
// the decode's select pass: its flags or its fault word) copied to `dst` on
// the host through pinned memory, waiting for nothing else. After an
// overlapped decode (`fault`: its fault word; it must be the last one this
// thread launched) the copy runs on the select pass's stream right behind it,
// so the wait skips the hop back to `stream` and work queued there since;
// otherwise it runs on `stream`.
hipError_t decode_read_back(const void* src, size_t bytes, void* dst, const int32_t* fault, hipStream_t stream);
hipError_t launch_length_penalty(const int32_t* lengths, int64_t n, float alpha, float* out, hipStream_t stream);
hipError_t launch_check_steps(const int32_t* steps, int B, int T, int32_t* status, hipStream_t stream);
// Range check of every per-example array (steps in [1, T], beams in [1, K],
// EOS in [-1, V), minimum lengths >= 0): status 0 when all pass.
hipError_t launch_check_examples(const int32_t* steps, const int32_t* beams, const int32_t* eos,
                                 const int32_t* min_lengths, int B, int T, int K, int V, int32_t* status,
                                 hipStream_t stream);

// Backward.
struct BackwardParams {
    int B, T, K, V;
    float alpha;
    const int32_t* steps;
    const int32_t* beams;  // device [B] beams per example, or null (K)
    const int32_t* parents;
    const int32_t* tokens;
    const int32_t* lengths;
    const uint8_t* from_logprob;
    const float* g_final;
    const float* g_final_raw;
    const float* g_scores;
    const float* g_raw;
    const void* logits;
    int logits_type;
    const float* row_lse;
    float* draws;      // [B, T, K] per-slot entry gradients (workspace or caller output)
    void* out;         // [B, T, K, V]
    int out_type;      // 0 f32, 1 f16, 2 bf16
    int accumulate;    // 1: out += g (f32 only); 0: out = 0 + g everywhere; 2: only rows with an entry (out holds 0)
    // Relaxed-pool entries [B, T, P] (pool_d null: none; reference
    // src/decoder.cpp:617-657): each entry's raw-score gradient d, added to
    // its parent's incoming gradient after the selected children (in entry
    // order), and to its log-prob entry when it came from one.
    int P;
    const int32_t* pool_parents;
    const int32_t* pool_tokens;
    const uint8_t* pool_flp;
    const float* pool_d;
};

size_t backward_workspace_bytes(int B, int T, int K);
hipError_t launch_path_walk(const BackwardParams& p, hipStream_t stream);
hipError_t launch_dense_gradient(const BackwardParams& p, hipStream_t stream);
hipError_t launch_backtrack(const int32_t* tokens, const int32_t* parents, const int32_t* steps, int B, int T, int K,
                            int64_t* seq, hipStream_t stream);
hipError_t launch_backtrack(const int64_t* tokens, const int64_t* parents, const int64_t* steps,
                            const int64_t* lengths, int B, int T, int K,
                            int64_t* seq, hipStream_t stream);
// The minimum-risk loss of scores [B, K] under costs [B, K]: risk [B], with
// reduction 1 (mean) or 2 (sum) also *loss, and the gradient factor [B, K]
// (d loss / d score_bk: d risk_b / d score_bk, over B for the mean).
hipError_t launch_risk(const float* scores, const float* costs, int B, int K, float temperature, int reduction,
                       float* risk, float* loss, float* factor, hipStream_t stream);

}  // namespace dbs_hip
