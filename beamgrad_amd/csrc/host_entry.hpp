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
                    const int32_t* forced, void* workspace, int64_t workspace_bytes, hipStream_t stream,
                    int32_t** fault);

// dbs_cuda_decode_step_ex2 with forced (device int32 [B] or null): an entry
// >= 0 (and < V) is the one token a read beam of example b may take at this
// step. Returns a DBS_CUDA_STATUS_*.
int step_for_host(const void* inputs, int data_type, int from_logits, const DBSCudaDecodeArgs* args,
                  const DBSCudaSearchOptions* options, const DBSCudaBeamState* state,
                  const DBSCudaDecodeOutputs* outputs, const int32_t* forced, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream);

// The per-slot path gradients draws [B, T, K] of the surrogate backward for
// every gradient input of `in` (final scores, final raw scores, scores, raw
// scores; logits are not read): slot (b, t, k) gets the gradient of the
// log-prob entry it selected, 0 where it selected none. Returns a
// DBS_CUDA_STATUS_*.
int path_draws_for_host(const DBSCudaDecodeArgs* args, const DBSCudaBackwardInputs* in, float* draws,
                        hipStream_t stream);

}  // namespace dbs_hip
