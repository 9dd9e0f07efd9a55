// SPDX-License-Identifier: MIT
//
// Device entry points that the host ABI (host_abi.cpp) drives, inside
// libdbs_hip: the device ABI's decode with one more output, and the path
// walk alone.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "dbs_cuda.h"

namespace dbs_hip {

// Relaxed-pool outputs of a decode or step (reference src/decoder.cpp:
// 294-306): with mult m >= 1 each step keeps the best m * beams candidates of
// an example, the selection first; device arrays [B, T, m * K] (any may be
// null), dead entries past the kept ones and past an example's steps.
struct PoolOutputs {
    int mult = 0;
    int32_t* parents = nullptr;
    int32_t* tokens = nullptr;
    int32_t* lengths = nullptr;
    float* scores = nullptr;
    float* raw_scores = nullptr;
    uint8_t* from_logprob = nullptr;
};

// Relaxed-pool entries of a backward (reference src/decoder.cpp:617-657):
// device arrays [B, T, P]; d is each entry's raw-score gradient (computed on
// the host from the pool gradients), added to its parent's incoming gradient
// after the selected children and, for an entry from a log-prob, to that
// entry.
struct PoolGrads {
    int P = 0;
    const int32_t* parents = nullptr;
    const int32_t* tokens = nullptr;
    const uint8_t* from_logprob = nullptr;
    const float* d = nullptr;
};

// Workspace bytes of decode_for_host (step_mode 0) or step_for_host
// (step_mode 1, prefix_stride as dbs_cuda_decode_step_workspace_size) with a
// relaxed pool of pool_mult (0: none); -1 for invalid arguments.
int64_t workspace_for_host(const DBSCudaDecodeArgs* args, int pool_mult, int step_mode, int prefix_stride);

// dbs_hip_decode_ex3 (per-example banned masks [B, V] or null), plus
// first_invalid (device int32 [B] or null): the first row holding NaN or
// +inf that example b's search read, t * K + k in reading order, or -1;
// forced (device int32 [B, T] or null): an entry >= 0 (and < V) is the one
// token a read beam of example b may take at step t (reference
// src/decoder.cpp:125, src/kernels_scalar.cpp:16-26); and *fault, as
// dbs_hip_decode_ex4's fault word (the workspace is the caller's). Returns a
// DBS_CUDA_STATUS_*.
int decode_for_host(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                    const DBSCudaSearchOptions* options, const uint8_t* banned_per_example,
                    const DBSCudaDecodeOutputs* outputs, float* row_lse, int32_t* first_invalid,
                    const int32_t* forced, const PoolOutputs* pool, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream, int32_t** fault);

// dbs_cuda_decode_step_ex2 (row_lse: device [B, K] or null) with forced
// (device int32 [B] or null): an entry >= 0 (and < V) is the one token a
// read beam of example b may take at this step; a relaxed pool (null:
// none); and row_mask (device [B, K, V] or null): 1 where a token filter
// refused the token for that row. Returns a DBS_CUDA_STATUS_*.
int step_for_host(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                  const DBSCudaSearchOptions* options, const DBSCudaBeamState* state,
                  const DBSCudaDecodeOutputs* outputs, float* row_lse, const int32_t* forced,
                  const PoolOutputs* pool, const uint8_t* row_mask, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream);

// The per-slot path gradients draws [B, T, K] of the surrogate backward for
// every gradient input of `in` (final scores, final raw scores, scores, raw
// scores; logits are not read) and the relaxed-pool entries (pool may be
// null): slot (b, t, k) gets the gradient of the log-prob entry it selected,
// 0 where it selected none. Returns a DBS_CUDA_STATUS_*.
int path_draws_for_host(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, const PoolGrads* pool,
                        float* draws, hipStream_t stream);

// dbs_hip_backward_dense into a float32 gradient [B, T, K, V] written fresh,
// with relaxed-pool entries (pool may be null). Returns a DBS_CUDA_STATUS_*.
int backward_dense_for_host(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, const PoolGrads* pool,
                            float* grad, void* workspace, int64_t workspace_bytes, hipStream_t stream);

}  // namespace dbs_hip
