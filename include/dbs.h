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
 * Only what the batch entry points need is declared here; the reference's
 * result handles, sparse backward, statistics, model-step callbacks, token
 * filters, forced tokens and relaxed pool are not served by this library.
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
    float selected_temperature;          /* [1.0] (selected-beam weights: not served) */
    float soft_topk_temperature;         /* [0.25] (relaxed pool: not served) */
    int relaxed_pool_multiplier;         /* [0] (relaxed pool: not served) */
    int vocab_block;                     /* ignored */
    float length_penalty_alpha;          /* GNMT ((5 + len) / 6)^alpha; 0 disables [0] */
    float soft_topk_tolerance;           /* [1e-4] (relaxed pool: not served) */
    int soft_topk_max_iters;             /* [48] (relaxed pool: not served) */
    int min_length;                      /* EOS masked below this length [0] */
    int validate_inputs;                 /* non-zero: NaN/+inf in a row the search reads is an error */
    int64_t max_dense_gradient_elements; /* [1e8] (dense single-example backward: not served) */
    int reserved0;
    int reserved1;
} DBSOptionsC;

typedef struct DBSDecoderHandle DBSDecoderHandle;

/* Token filter callback of the reference (reference include/dbs.h:129-137).
 * Declared for the layout of DBSAdvancedConstraintsC; a non-NULL filter is
 * rejected here (a per-candidate host callback has no place in a GPU scan). */
typedef int (*DBSTokenFilterFn)(
    void* user_data,
    int batch_index,
    int step,
    int parent_beam,
    const int32_t* prefix_tokens,
    int prefix_len,
    int token);

/* Constraints shared by every example of a batch (reference
 * include/dbs.h:139-148). forced_tokens and token_filter must be NULL here. */
typedef struct DBSAdvancedConstraintsC {
    const uint8_t* banned_tokens;        /* [V] or NULL: non-zero bans the token */
    const int32_t* forced_tokens;        /* must be NULL */
    int min_length;                      /* negative: the handle's min_length */
    float repetition_penalty;            /* <= 1 disables; 0 (zero-initialised) means 1 */
    int no_repeat_ngram_size;            /* <= 0 disables */
    DBSTokenFilterFn token_filter;       /* must be NULL */
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

/* Extended outputs (reference include/dbs.h:335-349). The pool arrays must be
 * NULL here (the relaxed pool is not served); row_lse gets, with from_logits,
 * the logsumexp of each row the search read and 0 elsewhere. */
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

#ifdef __cplusplus
}
#endif
