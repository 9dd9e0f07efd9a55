/* SPDX-License-Identifier: MIT
 *
 * libdbs host C ABI, as served by libdbs_hip.so: the batch entry points of
 * the reference's host library (reference include/dbs.h), with host arrays
 * in and out, computed on the GPU. Declarations, struct layouts, constants
 * and status codes are the reference's, so a C, cgo or ctypes caller of the
 * reference's libdbs links this library instead and keeps its code.
 *
 * Conventions (reference include/dbs.h:5-28):
 *   - DBS_OK (0) on success, else DBS_ERROR_INVALID_ARGUMENT (-1) for bad
 *     arguments or inputs (including NaN/+inf in a row the search reads when
 *     the handle validates inputs), DBS_ERROR_RUNTIME (-2) for failures during
 *     the computation (device errors, out of memory), DBS_ERROR_UNKNOWN (-3).
 *     A failing call records a message for dbs_last_global_error() (per
 *     thread) and dbs_last_error(handle).
 *   - Handles returned through out-parameters belong to the caller
 *     (dbs_destroy).
 *   - Arrays are dense, row-major host memory: inputs [B, T, K, V] indexed
 *     ((b*T + t)*K + k)*V + v; traces [B, T, K].
 *   - A decoder handle may be shared between threads; calls on one handle run
 *     one at a time on the GPU.
 *
 * All 81 functions of the reference's ABI are exported. What the GPU engine
 * does not serve is refused with DBS_ERROR_INVALID_ARGUMENT and a message
 * naming it: only what is beyond the engine's sizes (pools of more than
 * 1024 candidates, beams above 1024). Token-filter callbacks are served: a
 * decode with a filter runs step by step on the device, the filter asked on
 * the host in the reference's call order. The relaxed pool is served: the pool outputs of the batch
 * decodes into caller arrays, the pool and soft top-k inclusion weights of
 * result handles, and the pool's gradients (grad_relaxed_weights,
 * grad_pool_scores, grad_pool_raw_scores). Forced tokens (an entry >= 0: the one token a read beam may take at that
 * step) are served by every decode that takes them: the batch decodes into
 * caller arrays, the result-handle decodes and the model-step decodes.
 */
#pragma once

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define DBS_EXPORT __attribute__((visibility("default")))
#else
#define DBS_EXPORT
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/dbs.h:51-59 */
#define DBS_ABI_VERSION 10
#define DBS_VERSION_MAJOR 2
#define DBS_VERSION_MINOR 3
#define DBS_VERSION_PATCH 0

#define DBS_OK 0
#define DBS_ERROR_INVALID_ARGUMENT (-1)
#define DBS_ERROR_RUNTIME (-2)
#define DBS_ERROR_UNKNOWN (-3)

/* Decoder options (reference include/dbs.h:61-79). A zero field selects the
 * default in brackets; negative or non-finite values are rejected by
 * dbs_create_ex(). eos_token and validate_inputs take 0 literally. */
typedef struct DBSOptionsC {
    int beam_size;                       /* K [8] */
    int eos_token;                       /* -1: no EOS handling */
    float selected_temperature;          /* softmax temperature of the selected-beam weights [1.0] */
    float soft_topk_temperature;         /* [0.25] soft top-k weights of the pool */
    int relaxed_pool_multiplier;         /* [0] m: pool of m * K candidates a step (<= 1024) */
    int vocab_block;                     /* ignored */
    float length_penalty_alpha;          /* GNMT ((5 + len) / 6)^alpha; 0 disables [0] */
    float soft_topk_tolerance;           /* [1e-4] */
    int soft_topk_max_iters;             /* [48] */
    int min_length;                      /* EOS masked below this length [0] */
    int validate_inputs;                 /* non-zero: NaN/+inf in a row the search reads is an error */
    int64_t max_dense_gradient_elements; /* cap on T*K*V for dbs_backward_dense() [1e8] */
    int reserved0;
    int reserved1;
} DBSOptionsC;

typedef struct DBSDecoderHandle DBSDecoderHandle;
typedef struct DBSResultHandle DBSResultHandle;
typedef struct DBSBackwardHandle DBSBackwardHandle;
typedef struct DBSBatchResultHandle DBSBatchResultHandle;
typedef struct DBSWorkspaceHandle DBSWorkspaceHandle;

/* Model-step callback of dbs_decode_model_steps (reference include/dbs.h:
 * 87-101): fills out_log_probs [K, V] for `step` from the tokens the beams
 * emitted at step - 1 and their length-penalised scores (-1 and 0 at step
 * 0); 0 on success. */
typedef int (*DBSModelStepFn)(
    void* user_data,
    int batch_index,
    int step,
    const int32_t* prev_tokens,
    const float* prev_scores,
    int beam_size,
    int vocab_size,
    float* out_log_probs);

/* The beams entering a model step (reference include/dbs.h:103-121): slot k
 * is the k-th best hypothesis after step - 1; parents[k] the slot it
 * extends. Pointers are valid during the callback only. */
typedef struct DBSModelStepInfoC {
    int batch_index;
    int step;
    int beam_size;
    int vocab_size;
    const int32_t* parents;       /* [K] (-1 at step 0 and for dead slots) */
    const int32_t* tokens;        /* [K] token emitted at step - 1 (-1 at step 0) */
    const int32_t* lengths;       /* [K] */
    const float* scores;          /* [K] length-penalised scores */
    const float* raw_scores;      /* [K] cumulative log-probabilities */
    const uint8_t* finished;      /* [K] non-zero once the beam emitted EOS (its row is not read) */
    const int32_t* prefixes;      /* [K * step] the tokens of each beam's path */
    const void* reserved[4];
} DBSModelStepInfoC;

/* Fills out_log_probs [K, V] (pre-filled with -inf) for the beams `info`
 * describes; any non-zero return aborts the decode with DBS_ERROR_RUNTIME
 * (reference include/dbs.h:123-127). */
typedef int (*DBSModelStepExFn)(void* user_data, const DBSModelStepInfoC* info, float* out_log_probs);

/* Token filter callback of the reference (reference include/dbs.h:129-137):
 * called for each read beam in order and each token in order that passes
 * the forced, banned, minimum-length and n-gram checks, with the beam's
 * prefix; 0 refuses the token. */
typedef int (*DBSTokenFilterFn)(
    void* user_data,
    int batch_index,
    int step,
    int parent_beam,
    const int32_t* prefix_tokens,
    int prefix_len,
    int token);

/* Constraints shared by every example of a batch (reference
 * include/dbs.h:139-148). */
typedef struct DBSAdvancedConstraintsC {
    const uint8_t* banned_tokens;        /* [V] or NULL: non-zero bans the token */
    const int32_t* forced_tokens;        /* [T] or NULL: an entry >= 0 (< V) forces that token at step t */
    int min_length;                      /* negative: the handle's min_length */
    float repetition_penalty;            /* <= 1 disables; 0 (zero-initialised) means 1 */
    int no_repeat_ngram_size;            /* <= 0 disables */
    DBSTokenFilterFn token_filter;       /* NULL, or a filter (batch decodes: told the example's index) */
    void* token_filter_user_data;
    int batch_index;                     /* ignored by the batch functions */
} DBSAdvancedConstraintsC;

/* Caller-owned outputs of dbs_decode_batch_into (reference include/dbs.h:
 * 150-163). final_scores is required, the rest may be NULL. Steps past an
 * example's own step count hold token/parent -1, length 0, -inf scores and
 * from_logprob 0. */
typedef struct DBSDecodeOutputsC {
    float* final_scores;                 /* [B, K] */
    float* final_raw_scores;             /* [B, K] */
    int32_t* final_lengths;              /* [B, K] */
    int32_t* tokens;                     /* [B, T, K] */
    int32_t* parents;                    /* [B, T, K] */
    int32_t* lengths;                    /* [B, T, K] */
    float* scores;                       /* [B, T, K] length-penalised ranking scores */
    float* raw_scores;                   /* [B, T, K] cumulative log-probabilities */
    uint8_t* from_logprob;               /* [B, T, K] 0 for EOS carry-forward and padding slots */
} DBSDecodeOutputsC;

/* Per-handle statistics (reference include/dbs.h:165-184). last_kernel is 5
 * here (the GPU engine; the reference's 0-4 name its CPU paths); the
 * allocator totals count the device buffers this library's handles hold. */
typedef struct DBSStatsC {
    int abi_version;
    int last_kernel;
    int used_sparse_backward;
    int used_dense_backward;
    int used_batch_threads;
    int used_model_step_callback;
    int last_error_category;           /* 0 none, 1 invalid argument, 2 runtime, 3 allocation, 4 overflow */
    int64_t last_decode_ns;
    int64_t last_backward_ns;
    int64_t last_allocation_bytes;
    int64_t last_selected_count;
    int64_t last_pool_count;
    int64_t last_logprob_count;
    int64_t last_sparse_grad_count;
    int64_t total_allocator_calls;
    int64_t total_allocator_bytes;
    int64_t reserved_stats0;
    int64_t reserved_stats1;
} DBSStatsC;

/* Element types (reference include/dbs.h:186-190). */
typedef enum DBSDataTypeC {
    DBS_DTYPE_F32 = 0,
    DBS_DTYPE_F16 = 1,
    DBS_DTYPE_BF16 = 2
} DBSDataTypeC;

DBS_EXPORT int dbs_abi_version(void);
DBS_EXPORT const char* dbs_version_string(void);
DBS_EXPORT const char* dbs_last_global_error(void);

/* Handles (reference include/dbs.h:192-205). */
DBS_EXPORT int dbs_create_ex(DBSOptionsC options, DBSDecoderHandle** out_handle);
DBS_EXPORT DBSDecoderHandle* dbs_create(DBSOptionsC options);
DBS_EXPORT void dbs_destroy(DBSDecoderHandle* handle);
DBS_EXPORT const char* dbs_last_error(DBSDecoderHandle* handle);
/* More EOS tokens besides options.eos_token (which must be >= 0); count 0
 * removes them (reference include/dbs.h:206-213). */
DBS_EXPORT int dbs_set_extra_eos_tokens(DBSDecoderHandle* handle, const int32_t* tokens, int count);

/* Decodes float32 log-probs [B, T, K, V] into caller-owned arrays (reference
 * include/dbs.h:298-314). steps_per_example [B] (values in [1, T]) or NULL;
 * constraints apply to every example. num_threads is accepted for source
 * compatibility (the GPU decodes every example at once). */
DBS_EXPORT int dbs_decode_batch_into(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int batch_size,
    int steps,
    int vocab_size,
    const int32_t* steps_per_example,
    const DBSAdvancedConstraintsC* constraints,
    int num_threads,
    const DBSDecodeOutputsC* outputs);

/* Final-score gradient of a batch decoded with the same handle and shapes,
 * accumulated (+=) into grad_log_probs [B, T, K, V] (reference
 * include/dbs.h:316-333): only the log-prob entries on the beams' paths
 * change. */
DBS_EXPORT int dbs_backward_batch_into(
    DBSDecoderHandle* handle,
    int batch_size,
    int steps,
    int vocab_size,
    const int32_t* steps_per_example,
    const int32_t* parents,
    const int32_t* tokens,
    const int32_t* lengths,
    const uint8_t* from_logprob,
    const float* grad_final_scores,
    int num_threads,
    float* grad_log_probs);

/* Extended outputs (reference include/dbs.h:335-349). The pool arrays
 * [B, T, relaxed_pool_multiplier * K] (any may be NULL; one asked for needs a
 * relaxed_pool_multiplier >= 1) get each step's best m * K candidates, the
 * selection first, dead entries (parent and token -1, length 0, -inf scores)
 * past the candidates and past an example's steps; row_lse gets, with
 * from_logits, the logsumexp of each row the search read and 0 elsewhere. */
typedef struct DBSDecodeOutputsExC {
    DBSDecodeOutputsC base;
    int32_t* pool_parents;
    int32_t* pool_tokens;
    int32_t* pool_lengths;
    float* pool_scores;
    float* pool_raw_scores;
    uint8_t* pool_from_logprob;
    float* row_lse;                      /* [B, T, K] */
    void* reserved[4];                   /* must be NULL */
} DBSDecodeOutputsExC;

/* dbs_decode_batch_into for inputs of any DBSDataTypeC, and with from_logits
 * non-zero for logits, normalised per row read exactly as the reference does
 * (reference include/dbs.h:351-368). */
DBS_EXPORT int dbs_decode_batch_into_ex(
    DBSDecoderHandle* handle,
    const void* inputs,
    int data_type,
    int from_logits,
    int batch_size,
    int steps,
    int vocab_size,
    const int32_t* steps_per_example,
    const DBSAdvancedConstraintsC* constraints,
    int num_threads,
    const DBSDecodeOutputsExC* outputs);

/* Inputs of dbs_backward_batch_into_ex (reference include/dbs.h:370-397).
 * pool_size must be 0 and the pool arrays NULL here. */
typedef struct DBSBackwardInputsC {
    int batch_size;
    int steps;
    int vocab_size;
    int pool_size;
    const int32_t* steps_per_example;    /* [B] or NULL */
    const int32_t* parents;              /* [B, T, K] */
    const int32_t* tokens;
    const int32_t* lengths;
    const uint8_t* from_logprob;
    const int32_t* pool_parents;
    const int32_t* pool_tokens;
    const int32_t* pool_lengths;
    const uint8_t* pool_from_logprob;
    const float* grad_final_scores;      /* [B, K] or NULL */
    const float* grad_final_raw_scores;  /* [B, K] or NULL */
    const float* grad_scores;            /* [B, T, K] or NULL */
    const float* grad_raw_scores;        /* [B, T, K] or NULL */
    const float* grad_pool_scores;       /* must be NULL */
    const float* grad_pool_raw_scores;   /* must be NULL */
    const void* logits;                  /* [B, T, K, V] of logits_type, or NULL (log-prob decode) */
    int logits_type;
    const float* row_lse;                /* [B, T, K] the decode's row_lse, with logits */
    void* reserved[4];                   /* must be NULL */
} DBSBackwardInputsC;

/* The surrogate gradient of sum(grad_x * x) over the outputs given,
 * accumulated (+=) into grad_inputs [B, T, K, V] float32 (reference
 * include/dbs.h:399-410); with logits every row on a beam's path gets the
 * log-softmax gradient g - softmax(row) * sum(g) in full. */
DBS_EXPORT int dbs_backward_batch_into_ex(
    DBSDecoderHandle* handle,
    const DBSBackwardInputsC* inputs,
    int num_threads,
    float* grad_inputs);

/* Name of the compute path ("hip-gfx950"; the reference names its CPU
 * kernel, reference include/dbs.h:527). */
DBS_EXPORT const char* dbs_selected_kernel_name(void);

/* ---- Workspaces (reference include/dbs.h:196-199): the host row buffer of
 * the model-step decodes. ---- */
DBS_EXPORT int dbs_workspace_create(DBSWorkspaceHandle** out_workspace);
DBS_EXPORT void dbs_workspace_destroy(DBSWorkspaceHandle* workspace);
DBS_EXPORT int dbs_workspace_reserve(DBSWorkspaceHandle* workspace, int64_t float_count, int64_t int_count);
DBS_EXPORT int64_t dbs_workspace_allocated_bytes(DBSWorkspaceHandle* workspace);

/* ---- Decodes of log-probabilities into result handles (reference
 * include/dbs.h:215-299, 412-437). One example: log_probs [T, K, V]; a
 * batch: [B, T, K, V]; dbs_decode_batch_variable: [B, max_steps,
 * max_beam_size, V] with per-example steps, beam sizes, EOS tokens, minimum
 * lengths, banned masks [B, V] and forced tokens [B, max_steps] (an entry
 * >= 0 forces that token). Each result holds the trace, the selected-beam
 * softmax weights of every step and the final scores. num_threads is
 * accepted and ignored (the GPU decodes every example at once). ---- */
DBS_EXPORT int dbs_decode(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int steps,
    int vocab_size,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_typed(
    DBSDecoderHandle* handle,
    const void* log_probs,
    int data_type,
    int steps,
    int vocab_size,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_batch_typed(
    DBSDecoderHandle* handle,
    const void* log_probs,
    int data_type,
    int batch_size,
    int steps,
    int vocab_size,
    int num_threads,
    DBSBatchResultHandle** out_result);

DBS_EXPORT int dbs_decode_constrained(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int steps,
    int vocab_size,
    const uint8_t* banned_tokens,
    const int32_t* forced_tokens,
    int min_length,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_constrained_ex(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int steps,
    int vocab_size,
    const DBSAdvancedConstraintsC* constraints,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_batch(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int batch_size,
    int steps,
    int vocab_size,
    int num_threads,
    DBSBatchResultHandle** out_result);

DBS_EXPORT int dbs_decode_batch_variable(
    DBSDecoderHandle* handle,
    const float* log_probs,
    int batch_size,
    int max_steps,
    int max_beam_size,
    int vocab_size,
    const int32_t* steps_per_example,
    const int32_t* beam_sizes_per_example,
    const int32_t* eos_tokens_per_example,
    const int32_t* min_lengths_per_example,
    const uint8_t* banned_tokens_per_example,
    const int32_t* forced_tokens_per_example,
    int num_threads,
    DBSBatchResultHandle** out_result);

/* ---- Model-in-the-loop decodes (reference include/dbs.h:254-298): the
 * callback gives each step's [K, V] rows; each step's selection runs on the
 * GPU (one device step per callback). ---- */
DBS_EXPORT int dbs_decode_model_steps(
    DBSDecoderHandle* handle,
    DBSModelStepFn step_fn,
    void* user_data,
    int batch_index,
    int steps,
    int vocab_size,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_model_steps_with_workspace(
    DBSDecoderHandle* handle,
    DBSWorkspaceHandle* workspace,
    DBSModelStepFn step_fn,
    void* user_data,
    int batch_index,
    int steps,
    int vocab_size,
    DBSResultHandle** out_result);

DBS_EXPORT int dbs_decode_model_steps_ex(
    DBSDecoderHandle* handle,
    DBSModelStepExFn step_fn,
    void* user_data,
    int batch_index,
    int steps,
    int vocab_size,
    const DBSAdvancedConstraintsC* constraints,
    DBSResultHandle** out_result);

/* ---- Backward of a result (reference include/dbs.h:439-473): the gradient
 * w.r.t. the log-probabilities [T, K, V] of the selected-beam weight
 * gradients [T, K] and final-score gradients [K] (either may be NULL), dense
 * (capped by max_dense_gradient_elements) or as sorted sparse entries
 * (dbs_backward and dbs_backward_default), and the gradient w.r.t. the
 * initial beam scores [K]. grad_relaxed_weights must be NULL (no pool). ---- */
DBS_EXPORT int dbs_backward(
    DBSDecoderHandle* handle,
    const DBSResultHandle* result,
    const float* grad_selected_weights,
    const float* grad_relaxed_weights,
    const float* grad_final_scores,
    DBSBackwardHandle** out_backward);

DBS_EXPORT int dbs_backward_dense(
    DBSDecoderHandle* handle,
    const DBSResultHandle* result,
    const float* grad_selected_weights,
    const float* grad_relaxed_weights,
    const float* grad_final_scores,
    DBSBackwardHandle** out_backward);

DBS_EXPORT int dbs_backward_sparse(
    DBSDecoderHandle* handle,
    const DBSResultHandle* result,
    const float* grad_selected_weights,
    const float* grad_relaxed_weights,
    const float* grad_final_scores,
    DBSBackwardHandle** out_backward);

DBS_EXPORT int dbs_backward_default(
    DBSDecoderHandle* handle,
    const DBSResultHandle* result,
    const float* grad_selected_weights,
    const float* grad_relaxed_weights,
    const float* grad_final_scores,
    DBSBackwardHandle** out_backward);

DBS_EXPORT void dbs_free_result(DBSResultHandle* result);
DBS_EXPORT void dbs_free_batch_result(DBSBatchResultHandle* result);
DBS_EXPORT void dbs_free_backward(DBSBackwardHandle* result);

/* ---- Accessors (reference include/dbs.h:475-521). Pointers are borrowed
 * from the handle; NULL for a NULL handle or an empty array. ---- */
DBS_EXPORT int dbs_batch_result_size(const DBSBatchResultHandle* result);
DBS_EXPORT const DBSResultHandle* dbs_batch_result_at(const DBSBatchResultHandle* result, int batch_index);

DBS_EXPORT int dbs_result_steps(const DBSResultHandle* result);
DBS_EXPORT int dbs_result_beam_size(const DBSResultHandle* result);
DBS_EXPORT int dbs_result_vocab_size(const DBSResultHandle* result);
DBS_EXPORT int dbs_result_pool_size(const DBSResultHandle* result);

DBS_EXPORT const int32_t* dbs_result_tokens(const DBSResultHandle* result);
DBS_EXPORT const int32_t* dbs_result_parents(const DBSResultHandle* result);
DBS_EXPORT const int32_t* dbs_result_lengths(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_scores(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_raw_scores(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_weights(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_final_scores(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_final_raw_scores(const DBSResultHandle* result);

DBS_EXPORT const float* dbs_result_relaxed_weights(const DBSResultHandle* result);
DBS_EXPORT const int32_t* dbs_result_pool_tokens(const DBSResultHandle* result);
DBS_EXPORT const int32_t* dbs_result_pool_parents(const DBSResultHandle* result);
DBS_EXPORT const int32_t* dbs_result_pool_lengths(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_pool_scores(const DBSResultHandle* result);
DBS_EXPORT const float* dbs_result_pool_raw_scores(const DBSResultHandle* result);

DBS_EXPORT const float* dbs_backward_grad_log_probs(const DBSBackwardHandle* result);
DBS_EXPORT const float* dbs_backward_grad_initial_scores(const DBSBackwardHandle* result);
DBS_EXPORT const int64_t* dbs_backward_sparse_logprob_indices(const DBSBackwardHandle* result);
DBS_EXPORT const float* dbs_backward_sparse_logprob_values(const DBSBackwardHandle* result);
DBS_EXPORT int64_t dbs_backward_sparse_logprob_count(const DBSBackwardHandle* result);
DBS_EXPORT int dbs_backward_is_sparse(const DBSBackwardHandle* result);

DBS_EXPORT int64_t dbs_result_selected_count(const DBSResultHandle* result);
DBS_EXPORT int64_t dbs_result_pool_count(const DBSResultHandle* result);
DBS_EXPORT int64_t dbs_result_logprob_count(const DBSResultHandle* result);
DBS_EXPORT int64_t dbs_backward_grad_log_probs_count(const DBSResultHandle* result);
DBS_EXPORT int64_t dbs_backward_grad_initial_scores_count(const DBSResultHandle* result);

DBS_EXPORT int64_t dbs_result_eos_count(const DBSResultHandle* result, int eos_token);
/* 0 if every step's beams follow the candidate order, -3 for scores out of
 * order, -4 for a tie broken out of order, -1 for NULL. */
DBS_EXPORT int dbs_result_validate_deterministic_order(const DBSResultHandle* result);
DBS_EXPORT int dbs_result_summary_json(const DBSResultHandle* result, int eos_token, char* out_json,
                                       int64_t out_json_capacity);

/* ---- Host queries, statistics and determinism (reference include/dbs.h:
 * 523-545). dbs_has_* report the host CPU's extensions. ---- */
DBS_EXPORT int dbs_has_avx512(void);
DBS_EXPORT int dbs_has_avx2(void);
DBS_EXPORT int dbs_has_sse42(void);
DBS_EXPORT int dbs_has_neon(void);
DBS_EXPORT int dbs_get_stats(DBSDecoderHandle* handle, DBSStatsC* out_stats);
DBS_EXPORT int dbs_get_stats_json(DBSDecoderHandle* handle, char* out_json, int64_t out_json_capacity);
/* Always 1: no randomness, and a strict total order over candidates. */
DBS_EXPORT int dbs_is_deterministic(void);
/* A per-handle seed kept for ABI compatibility; nothing reads it. */
DBS_EXPORT int dbs_set_deterministic_seed(DBSDecoderHandle* handle, uint64_t seed);
DBS_EXPORT uint64_t dbs_get_deterministic_seed(DBSDecoderHandle* handle);
DBS_EXPORT void dbs_allocator_counters_reset(void);
DBS_EXPORT int64_t dbs_allocator_call_count(void);
DBS_EXPORT int64_t dbs_allocator_byte_count(void);
DBS_EXPORT void dbs_reset_stats(DBSDecoderHandle* handle);

#ifdef __cplusplus
}
#endif
