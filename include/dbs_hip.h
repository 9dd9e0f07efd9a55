/* SPDX-License-Identifier: MIT
 *
 * Additive entry points of libdbs_hip.so beyond the reference's device ABI
 * (include/dbs_cuda.h). None changes an existing layout; each says which
 * reference interface it extends.
 */
#pragma once

#include "dbs_cuda.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dbs_cuda_decode_ex2 with a per-example banned-token mask: banned_per_example
 * is device uint8 [B, V] (non-zero bans token v in example b), OR-ed with
 * args->banned_tokens. The reference takes only one [V] mask on the device
 * (reference include/dbs_cuda.h:86); its CPU path bans per example through
 * separate dbs_decode_batch_into_ex calls (reference include/dbs.h:339-368). */
DBS_CUDA_EXPORT int dbs_hip_decode_ex3(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaSearchOptions* options,
    const uint8_t* banned_per_example,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* dbs_hip_decode_ex3 that also says where the decode records a select-pass
 * wait that gave up, so that an asynchronous caller can tell an incomplete
 * trace from a good one without validate flags. *fault_word is set to a
 * device int32 inside `workspace` that is non-zero, once `stream` has passed
 * the decode, if a wait of the overlapped decode gave up (those examples'
 * traces are padding; invalid_input[b] == 2 where flags were given), or to
 * NULL when the decode ran its passes one after the other (nothing can give
 * up) or failed to launch. The word is valid until the workspace is reused.
 * Without a caller workspace (workspace == NULL) the call synchronises,
 * returns DBS_CUDA_STATUS_LAUNCH_FAILED for a wait that gave up and sets
 * *fault_word to NULL. No counterpart in the reference, whose CUDA engine
 * has no overlapped passes (reference include/dbs_cuda.h:299-315 is the
 * decode it extends). */
DBS_CUDA_EXPORT int dbs_hip_decode_ex4(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaSearchOptions* options,
    const uint8_t* banned_per_example,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* workspace,
    int64_t workspace_bytes,
    int32_t** fault_word,
    void* stream);

/* The read-back that ends a decode of dbs_hip_decode_ex4 on `stream`: copies
 * `bytes` bytes at `src` -- the decode's invalid_input flags or its
 * *fault_word, which only its select pass writes -- to `dst` on the host and
 * returns once they are there. Given the fault word of the overlapped decode
 * the calling thread launched last, the copy runs on that decode's second
 * stream right behind its select pass, so the wait covers neither the hop back
 * to `stream` nor work queued on `stream` after the decode; with
 * fault_word == NULL (or any other decode) it runs on `stream` and waits for
 * it. Returns a status. No counterpart in the reference, whose CUDA op reads
 * its flags back with a copy on the caller's stream (reference
 * python/csrc/cuda_ops.cpp:177-184). */
DBS_CUDA_EXPORT int dbs_hip_decode_read_back(
    const void* src,
    int64_t bytes,
    void* dst,
    const int32_t* fault_word,
    void* stream);

/* dbs_hip_decode_ex3 without a workspace argument and without any device
 * allocation, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The workspace is a static device array of
 * DBS_HIP_NOALLOC_SCRATCH_BYTES per GPU, held from the library's first use on
 * that GPU until the process ends and shared by every call on it: calls that
 * overlap on one GPU (two streams, two threads) race on it and must be
 * serialised by the caller. A decode whose workspace
 * (dbs_cuda_decode_workspace_size) exceeds the maximum returns
 * DBS_HIP_STATUS_SCRATCH_LIMIT without launching anything. The passes run one
 * after the other on `stream` (no second stream or event is created). With
 * per-example arrays the call synchronises the stream once, as
 * dbs_cuda_decode_ex2 does. */
#define DBS_HIP_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)
#define DBS_HIP_STATUS_SCRATCH_LIMIT 5
DBS_CUDA_EXPORT int dbs_hip_decode_noalloc(
    const void* inputs,
    int data_type,
    int from_logits,
    const DBSCudaDecodeArgs* args,
    const DBSCudaSearchOptions* options,
    const uint8_t* banned_per_example,
    const DBSCudaDecodeOutputs* outputs,
    float* row_lse,
    void* stream);

/* Output element types of dbs_hip_backward_dense. */
#define DBS_HIP_GRAD_F32 0
#define DBS_HIP_GRAD_F16 1
#define DBS_HIP_GRAD_BF16 2
/* OR-ed into grad_type: grad_out already holds zeros (e.g. cleared while the
 * host was busy between the decode and its backward), and only the rows
 * [b, t, q] that receive an entry are written, each as the call without the
 * flag writes it; every other row is left as it is. Same result as the call
 * without the flag on that buffer. */
#define DBS_HIP_GRAD_ZEROED 0x100

/* The gradient of dbs_cuda_backward_ex written, not accumulated: every
 * element of grad_out [B, T, K, V] is stored once, as 0 + g rounded to
 * grad_type (round to nearest even), so the caller needs no zero-fill and no
 * separate cast. Equals zero-filling a float32 buffer, calling
 * dbs_cuda_backward_ex (reference include/dbs_cuda.h:262-268) and converting
 * the result with a round-to-nearest-even cast (reference
 * python/beamgrad/_torch.py:289). Workspace: dbs_cuda_backward_workspace_size. */
DBS_CUDA_EXPORT int dbs_hip_backward_dense(
    const DBSCudaDecodeArgs* args,
    const DBSCudaBackwardInputs* inputs,
    void* grad_out,
    int grad_type,
    void* workspace,
    int64_t workspace_bytes,
    void* stream);

/* Token sequences of the final beams, following parent pointers from the last
 * step: sequences [B, K, T] (int64); steps past steps_per_example[b] and dead
 * beams hold -1. One launch; replaces the T-step torch loop of the reference's
 * backtrack (reference python/beamgrad/_torch.py:582-606). tokens and parents
 * are int32 [B, T, K]; steps_per_example is device int32 [B] or NULL. */
DBS_CUDA_EXPORT int dbs_hip_backtrack(
    const int32_t* tokens,
    const int32_t* parents,
    const int32_t* steps_per_example,
    int batch_size,
    int steps,
    int beam_size,
    int64_t* sequences,
    void* stream);

/* dbs_hip_backtrack with int64 tokens, parents and steps_per_example (the
 * dtype torch hands the trace to the caller in), so the caller converts
 * nothing before the launch. No counterpart in the reference (its backtrack
 * is the torch loop named above). */
DBS_CUDA_EXPORT int dbs_hip_backtrack_i64(
    const int64_t* tokens,
    const int64_t* parents,
    const int64_t* steps_per_example,
    int batch_size,
    int steps,
    int beam_size,
    int64_t* sequences,
    void* stream);

/* The sequences a search returns (reference python/beamgrad/_search.py:
 * 258-311): dbs_hip_backtrack_i64's [B, K, T] tokens with, besides, -1 at
 * and past each final beam's length (final_lengths int64 [B, K]). One launch. */
DBS_CUDA_EXPORT int dbs_hip_search_sequences(
    const int64_t* tokens,
    const int64_t* parents,
    const int64_t* steps_per_example,
    const int64_t* final_lengths,
    int batch_size,
    int steps,
    int beam_size,
    int64_t* sequences,
    void* stream);

/* The minimum-risk loss of the final beams (the objective of reference
 * python/beamgrad/losses.py:139-169): for each example b, risk[b] =
 * sum_k p_k c_k with p = softmax(scores[b] / temperature) over its live beams
 * (finite scores; dead beams get no probability and their costs are not
 * used). reduction 0: the loss is risk [B]; 1: *loss is their mean, 2: their
 * sum (added in index order). grad_factor[b, k] = d loss / d scores[b, k] =
 * p_k (c_k - risk[b]) / temperature, over B for the mean (0 for dead beams).
 * An example without a live beam has risk 0. scores and costs are float32
 * [B, K] on the device; temperature finite and positive; loss may be null
 * for reduction 0. One launch for B <= 1024 and K <= 64, else two. */
DBS_CUDA_EXPORT int dbs_hip_minimum_risk(
    const float* scores,
    const float* costs,
    int batch_size,
    int beam_size,
    float temperature,
    int reduction,
    float* risk,
    float* loss,
    float* grad_factor,
    void* stream);

/* A decode trace's outputs in the dtypes torch returns them in, in one
 * launch: final_lengths [B, K], tokens, parents and lengths [B, T, K] as
 * int64, from_logprob [B, T, K] as 0/1 bytes (torch bool), and the
 * per-example steps [B] as int64 (steps where steps_per_example is null).
 * No counterpart in the reference (its Python wrapper converts each output
 * with its own torch operation); for the torch operator beamgrad::decode_trace. */
DBS_CUDA_EXPORT int dbs_hip_widen_trace(
    const int32_t* final_lengths,
    const int32_t* tokens,
    const int32_t* parents,
    const int32_t* lengths,
    const uint8_t* from_logprob,
    const int32_t* steps_per_example,
    int batch_size,
    int steps,
    int beam_size,
    int64_t* final_lengths64,
    int64_t* tokens64,
    int64_t* parents64,
    int64_t* lengths64,
    uint8_t* from_logprob_bool,
    int64_t* steps64,
    void* stream);

/* Launch timing for measurement tools (no counterpart in the reference).
 * With profiling on, every kernel the library launches is bracketed by HIP
 * events on the caller's stream, and its duration is summed per kernel kind:
 * 0 row pass, 1 select, 2 path walk, 3 dense gradient, 4 backtrack; kind 5
 * returns (in launches) the rows the select pass rescanned in full and kind 6
 * the overlapped-decode waits that gave up (always 0 unless something else
 * failed).
 * dbs_hip_profile_enable(on) clears the sums; dbs_hip_profile_read waits for
 * the recorded events and returns the sum (milliseconds) and the number of
 * launches of one kind. Off by default; costs two event records per launch. */
DBS_CUDA_EXPORT int dbs_hip_profile_enable(int on);
DBS_CUDA_EXPORT int dbs_hip_profile_read(int kernel, double* total_ms, int64_t* launches);

/* Row-pass kernel choice for tests and measurements (no counterpart in the
 * reference; every choice gives the same results): -1 automatic (the
 * default: for log-prob rows the one-read log-prob kernel where it applies;
 * else, for bfloat16 logits rows of 116481 to 155648 entries, the relay
 * kernel; else the resident 16-bit kernel where it applies, else the
 * pipelined 16-bit kernel, else the two-pass kernel), 0 two-pass, 1 resident
 * 16-bit (V % 8 == 0, 16-byte aligned rows), 2 pipelined 16-bit (any V), 3
 * one-read log-prob rows (any dtype, rows up to 163824 bytes), 5 relay for
 * bfloat16 logits (V % 8 == 0, 16-byte aligned rows, V <= 155648); 4 is not
 * a kernel (-2). A kernel that does not apply to a decode falls back to the
 * two-pass one. Returns the previous choice, or -2 for an invalid
 * argument. */
DBS_CUDA_EXPORT int dbs_hip_set_row_pass(int kind);

/* Whether a multi-step decode runs its select pass alongside the row pass, on
 * a second stream that the caller's stream then waits for (no counterpart in
 * the reference; the results are the same either way): -1 automatic (the
 * default: constrained decodes, whose select pass is as long as the row
 * pass), 1 always, 0 never (the select pass after the row pass on the
 * caller's stream). Applies when at most half the CUs would be left to the
 * select pass (one per example for the workgroup pass, one per four examples
 * for the one-wavefront pass). Returns the previous setting, or -2 for an
 * invalid argument. */
DBS_CUDA_EXPORT int dbs_hip_set_decode_overlap(int on);

/* The select pass of a decode (no counterpart in the reference; the results
 * are the same either way): 0 automatic (the default: one wavefront per
 * example for decodes of at most 16 beams with shortlists, with n-gram
 * blocking of n >= 2 and/or a repetition penalty too where their prefixes
 * fit the wavefront's LDS; one 256-thread workgroup per example otherwise),
 * 1 always the workgroup pass.
 * Returns the previous setting, or -2 for an invalid argument. */
DBS_CUDA_EXPORT int dbs_hip_set_select_pass(int kind);

#ifdef __cplusplus
}
#endif
