/* SPDX-License-Identifier: MIT
 *
 * CPU oracle for the beamgrad decode/backward path: a plain-C restatement of
 * the reference algorithm, used ONLY as the checker in tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. Nothing in the
 * product (beamgrad_amd/) links, loads or calls it.
 *
 * Every function names the reference file:line it restates. How each is
 * pinned (tests/test_oracle.py; "_ref" = the reference's own CPU library built
 * from its sources by oracle/Makefile):
 *   orc_f16_to_f32, orc_bf16_to_f32  all 65536 patterns vs the closed form
 *   orc_log_ge1, orc_exp_ge0         vs math.log / math.exp (series error)
 *   orc_length_penalty               <= 1 ulp of pow, integer-alpha squaring,
 *                                    saturation; _ref decodes
 *   orc_exp_nonpositive              vs math.exp; _ref from-logits decodes
 *   orc_row_stats                    vs a float64 logsumexp; _ref row_lse bits
 *   orc_softmax_probability          _ref logits backward bits; finite differences
 *   orc_decode                       _ref bits on random cases (ties, -inf,
 *                                    NaN flags, EOS, n-gram, banned), committed
 *                                    golden fixtures, known answers, exhaustive
 *                                    beams, greedy K = 1
 *   orc_backward                     _ref bits, golden fixtures, finite differences
 *   orc_path_gradient                draws scattered == _ref dense gradient
 *   orc_backtrack                    the reference's path property test
 * No function is left unpinned.
 */
#ifndef DBS_ORACLE_H
#define DBS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2

/* Numerics (src/half.hpp, src/logits.hpp, src/penalty.hpp). */
float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t h);
double orc_log_ge1(double x);
double orc_exp_ge0(double y);
float orc_length_penalty(int length, float alpha);
float orc_exp_nonpositive(float x);
/* max over entries < +inf, logsumexp (-inf when no entry is finite), NaN/+inf flag. */
void orc_row_stats(const float* row, int vocab, float* max_out, float* lse_out, int* invalid_out);
float orc_softmax_probability(float x, float lse);

typedef struct OrcDecodeArgs {
    int batch_size, steps, beam_size, vocab_size;
    int dtype;                        /* ORC_F32 / ORC_F16 / ORC_BF16 */
    int from_logits;
    int eos_token;                    /* -1 disables EOS handling */
    const int32_t* extra_eos;         /* extra EOS ids (need eos_token >= 0) */
    int extra_eos_count;
    int min_length;
    float length_penalty_alpha;
    int no_repeat_ngram_size;
    float repetition_penalty;         /* <= 1 disables */
    const int32_t* steps_per_example; /* [B] or NULL */
    const uint8_t* banned;            /* [V] or NULL, shared by every example */
    const uint8_t* banned_per_example;/* [B, V] or NULL (OR-ed with banned) */
    int num_threads;                  /* <= 0: one thread */
} OrcDecodeArgs;

typedef struct OrcDecodeOutputs {
    float* final_scores;     /* [B, K] */
    float* final_raw_scores; /* [B, K] */
    int32_t* final_lengths;  /* [B, K] */
    int32_t* tokens;         /* [B, T, K] */
    int32_t* parents;        /* [B, T, K] */
    int32_t* lengths;        /* [B, T, K] */
    float* scores;           /* [B, T, K] */
    float* raw_scores;       /* [B, T, K] */
    uint8_t* from_logprob;   /* [B, T, K] */
    float* row_lse;          /* [B, T, K]: lse of rows read (from logits), 0 elsewhere */
    uint8_t* invalid;        /* [B]: a row the search read held NaN or +inf */
    uint8_t* row_read;       /* [B, T, K] or NULL: 1 where the search read the row */
} OrcDecodeOutputs;

/* Returns 0, or -1 for invalid arguments. Invalid (NaN/+inf) entries are
 * reported per example and never selected, as with validate_inputs = 0. */
int orc_decode(const void* inputs, const OrcDecodeArgs* args, const OrcDecodeOutputs* out);

typedef struct OrcBackwardArgs {
    int batch_size, steps, beam_size, vocab_size;
    float length_penalty_alpha;
    const int32_t* steps_per_example; /* [B] or NULL */
    const int32_t* parents;           /* [B, T, K] */
    const int32_t* tokens;
    const int32_t* lengths;
    const uint8_t* from_logprob;
    const float* grad_final_scores;     /* [B, K] or NULL */
    const float* grad_final_raw_scores; /* [B, K] or NULL */
    const float* grad_scores;           /* [B, T, K] or NULL */
    const float* grad_raw_scores;       /* [B, T, K] or NULL */
    const void* logits;                 /* [B, T, K, V] or NULL */
    int logits_dtype;
    const float* row_lse;               /* [B, T, K], with logits */
    int num_threads;
} OrcBackwardArgs;

/* Accumulates (+=) the surrogate gradient into grad [B, T, K, V] (float32).
 * Returns 0, or -1 for invalid arguments / an out-of-range trace. */
int orc_backward(const OrcBackwardArgs* args, float* grad);

/* draws [B, T, K]: the gradient of the log-prob entry each selected slot used. */
int orc_path_gradient(const OrcBackwardArgs* args, float* draws);

void orc_length_penalty_array(const int32_t* lengths, int64_t count, float alpha, float* out);

/* sequences [B, K, T] (int64) of the final beams; -1 past an example's steps and for dead beams. */
void orc_backtrack(const int32_t* tokens, const int32_t* parents, const int32_t* steps_per_example,
                   int batch_size, int steps, int beam_size, int64_t* sequences);

#ifdef __cplusplus
}
#endif

#endif
