/* SPDX-License-Identifier: MIT
 *
 * Device C ABI of the beam-search engine, implemented for AMD Instinct MI355X
 * (gfx950) by libdbs_hip.so. It is the drop-in for the reference's
 * libdbs_cuda: every declaration below keeps the reference's name, argument
 * order, struct layout and constants (reference include/dbs_cuda.h), so a
 * program written against that header links against libdbs_hip unchanged.
 *
 * Conventions (reference include/dbs_cuda.h:26-36):
 *   - tensor pointers are device pointers to dense row-major data: inputs
 *     [B, T, K, V], per-step outputs [B, T, K], per-beam outputs [B, K];
 *   - work is queued on `stream` (a hipStream_t; NULL = the default stream)
 *     and calls return a status; nothing throws across the ABI;
 *   - `workspace` is caller-owned device memory of at least the size the
 *     matching *_workspace_size() returns, or NULL (then the library
 *     allocates and frees it stream-ordered);
 *   - per-example arrays are validated on the device, which synchronizes the
 *     stream once;
 *   - backward outputs accumulate (+=) into the caller's buffer.
 * The only process-wide state is the synchronization flag, so calls are
 * reentrant across threads and streams.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define DBS_CUDA_EXPORT __attribute__((visibility("default")))
#else
#define DBS_CUDA_EXPORT
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (reference include/dbs_cuda.h:60-64). */
#define DBS_CUDA_STATUS_OK 0
#define DBS_CUDA_STATUS_UNAVAILABLE 1      /* no usable GPU */
#define DBS_CUDA_STATUS_INVALID_ARGUMENT 2
#define DBS_CUDA_STATUS_LAUNCH_FAILED 3
#define DBS_CUDA_STATUS_OUT_OF_MEMORY 4

/* Largest supported beam size (reference include/dbs_cuda.h:67). */
#define DBS_CUDA_MAX_BEAM 1024

/* Problem description (reference include/dbs_cuda.h:69-87). */
typedef struct DBSCudaDecodeArgs {
    int batch_size;               /* B */
    int steps;                    /* T (the maximum with steps_per_example) */
    int beam_size;                /* K, also the beam stride of every tensor */
    int vocab_size;               /* V */
    int eos_token;                /* -1 disables EOS handling */
    int min_length;               /* EOS masked below this hypothesis length */
    float length_penalty_alpha;   /* GNMT ((5 + len) / 6)^alpha; 0 disables */
    int no_repeat_ngram_size;     /* n > 0 blocks repeats of the beam's n-grams */
    float repetition_penalty;     /* > 1: prefix tokens lose log(penalty) */
    int reserved0;                /* must be 0 */
    const int32_t* steps_per_example;       /* device int32 [B] in [1, T], or NULL */
    const int32_t* beam_sizes_per_example;  /* device int32 [B] in [1, K], or NULL */
    const int32_t* eos_tokens_per_example;  /* device int32 [B] in [-1, V), or NULL */
    const int32_t* min_lengths_per_example; /* device int32 [B] >= 0, or NULL */
    const uint8_t* banned_tokens; /* device [V], non-zero bans the token in every example, or NULL */
} DBSCudaDecodeArgs;

/* Decode outputs (reference include/dbs_cuda.h:89-100). */
typedef struct DBSCudaDecodeOutputs {
    float* final_scores;          /* required [B, K] */
    float* final_raw_scores;      /* [B, K] or NULL */
    int32_t* final_lengths;       /* [B, K] or NULL */
    int32_t* tokens;              /* [B, T, K] or NULL */
    int32_t* parents;             /* [B, T, K] or NULL */
    int32_t* lengths;             /* [B, T, K] or NULL */
    float* scores;                /* [B, T, K] or NULL */
    float* raw_scores;            /* [B, T, K] or NULL */
    uint8_t* from_logprob;        /* [B, T, K] or NULL */
    uint8_t* invalid_input;       /* [B] or NULL: 1 if a row the search read held NaN or +inf */
} DBSCudaDecodeOutputs;

/* Replaces reference include/dbs_cuda.h:102-103. */
DBS_CUDA_EXPORT int dbs_cuda_available(void);
DBS_CUDA_EXPORT const char* dbs_cuda_status_string(int status);

/* 1: synchronize the stream after every call; 0: asynchronous (default, or
 * DBS_CUDA_SYNC_CHECK=1 in the environment). Replaces include/dbs_cuda.h:106-107. */
DBS_CUDA_EXPORT int dbs_cuda_set_synchronization(int synchronize);
DBS_CUDA_EXPORT int dbs_cuda_get_synchronization(void);

/* Workspace bytes, or a negative value for invalid arguments.
 * Replaces include/dbs_cuda.h:111-112. */
DBS_CUDA_EXPORT int64_t dbs_cuda_decode_workspace_size(const DBSCudaDecodeArgs* args);
DBS_CUDA_EXPORT int64_t dbs_cuda_backward_workspace_size(const DBSCudaDecodeArgs* args);

/* Hard beam search over float32 log-probs. Replaces include/dbs_cuda.h:122-128. */
DBS_CUDA_EXPORT int dbs_cuda_decode(
    const float* log_probs,
    const DBSCudaDecodeArgs* args,
    const DBSCudaDecodeOutputs* outputs,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Beam state between steps of the step API (reference include/dbs_cuda.h:145-154). */
typedef struct DBSCudaBeamState {
    float* raw_scores;          /* [B, K], updated in place */
    int32_t* lengths;           /* [B, K], updated in place */
    uint8_t* finished;          /* [B, K], updated in place */
    const int32_t* prefixes;    /* [B, K, prefix_stride] tokens of each beam (read with constraints) */
    int prefix_stride;
    int reserved0;              /* must be 0 */
} DBSCudaBeamState;

/* Replaces include/dbs_cuda.h:158-175. */
DBS_CUDA_EXPORT int64_t dbs_cuda_decode_step_workspace_size(const DBSCudaDecodeArgs* args, int prefix_stride);
DBS_CUDA_EXPORT int dbs_cuda_decode_step(
    const float* log_probs,
    const DBSCudaDecodeArgs* args,
    const DBSCudaBeamState* state,
    const DBSCudaDecodeOutputs* outputs,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Final-score surrogate gradient, accumulated into grad_log_probs [B, T, K, V].
 * Replaces include/dbs_cuda.h:184-194. */
DBS_CUDA_EXPORT int dbs_cuda_backward(
    const DBSCudaDecodeArgs* args,
    const int32_t* parents,
    const int32_t* tokens,
    const int32_t* lengths,
    const uint8_t* from_logprob,
    const float* grad_final_scores,
    float* grad_log_probs,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Element types (reference include/dbs_cuda.h:197-199). */
#define DBS_CUDA_DTYPE_F32 0
#define DBS_CUDA_DTYPE_F16 1
#define DBS_CUDA_DTYPE_BF16 2

/* Decode of f32/f16/bf16 rows, log-probs or logits (normalised on the fly);
 * row_lse [B, T, K] (optional) gets the logsumexp of every row read, 0
 * elsewhere. Replaces include/dbs_cuda.h:211-220. */
DBS_CUDA_EXPORT int dbs_cuda_decode_ex(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Replaces include/dbs_cuda.h:224-234. */
DBS_CUDA_EXPORT int dbs_cuda_decode_step_ex(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaBeamState* state,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Backward inputs (reference include/dbs_cuda.h:239-253). */
typedef struct DBSCudaBackwardInputs {
    const int32_t* parents;              /* [B, T, K] */
    const int32_t* tokens;               /* [B, T, K] */
    const int32_t* lengths;              /* [B, T, K] */
    const uint8_t* from_logprob;         /* [B, T, K] */
    const float* grad_final_scores;      /* [B, K] or NULL */
    const float* grad_final_raw_scores;  /* [B, K] or NULL */
    const float* grad_scores;            /* [B, T, K] or NULL */
    const float* grad_raw_scores;        /* [B, T, K] or NULL */
    const void* logits;                  /* [B, T, K, V] when decoded from logits, else NULL */
    int logits_type;                     /* DBS_CUDA_DTYPE_* */
    int reserved0;                       /* must be 0 */
    const float* row_lse;                /* [B, T, K], required with logits */
    void* reserved[4];                   /* must be NULL */
} DBSCudaBackwardInputs;

/* Surrogate gradient of the given outputs, accumulated into grad_inputs.
 * Replaces include/dbs_cuda.h:262-268. */
DBS_CUDA_EXPORT int dbs_cuda_backward_ex(
    const DBSCudaDecodeArgs* args,
    const DBSCudaBackwardInputs* inputs,
    float* grad_inputs,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Search options of the _ex2 functions (reference include/dbs_cuda.h:271-284). */
#define DBS_CUDA_MAX_EXTRA_EOS 16
typedef struct DBSCudaSearchOptions {
    int extra_eos_count;
    int32_t extra_eos_tokens[DBS_CUDA_MAX_EXTRA_EOS];
    int reserved0;        /* must be 0 */
    void* reserved[4];    /* must be NULL */
} DBSCudaSearchOptions;

/* Replaces include/dbs_cuda.h:288-298. */
DBS_CUDA_EXPORT int dbs_cuda_decode_ex2(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaSearchOptions* options,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Replaces include/dbs_cuda.h:304-315. */
DBS_CUDA_EXPORT int dbs_cuda_decode_step_ex2(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaSearchOptions* options,
    const DBSCudaBeamState* state,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* out[i] = GNMT penalty of lengths[i]. Replaces include/dbs_cuda.h:319. */
DBS_CUDA_EXPORT int dbs_cuda_length_penalty(const int32_t* lengths, int64_t count, float alpha, float* out, void* stream);

/* draws [B, T, K]: gradient of the log-prob entry each slot used.
 * Replaces include/dbs_cuda.h:326-334. */
DBS_CUDA_EXPORT int dbs_cuda_path_gradient(
    const DBSCudaDecodeArgs* args,
    const int32_t* parents,
    const int32_t* tokens,
    const int32_t* lengths,
    const uint8_t* from_logprob,
    const float* grad_final_scores,
    float* draws,
    void* stream);

#ifdef __cplusplus
}
#endif
