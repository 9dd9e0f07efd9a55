// SPDX-License-Identifier: MIT
//
// Device helpers shared by the row pass and the select pass.
#pragma once

#include <hip/hip_runtime.h>

#include "engine.hpp"

namespace dbs_hip {

// Monotone map of a float to uint32 (-0 and +0 map together).
__device__ __forceinline__ uint32_t ordered_key(float x) {
    if (x == 0.0f) x = 0.0f;
    const uint32_t u = f32_bits(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int DT>
__device__ __forceinline__ float load_one(const void* base, int64_t i) {
    if constexpr (DT == 0) {
        return static_cast<const float*>(base)[i];
    } else if constexpr (DT == 1) {
        return half_to_f32(static_cast<const uint16_t*>(base)[i]);
    } else {
        return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
    }
}

__device__ __forceinline__ bool is_eos_tok(const DecodeParams& p, int32_t v) {
    for (int i = 0; i < p.n_eos; ++i)
        if (p.eos_set[i] == v) return true;
    return false;
}

// Statically excluded tokens of a row: banned (shared or per example) and the
// EOS tokens while the new length is below min_length.
__device__ __forceinline__ bool static_masked(const DecodeParams& p, int b, int v, bool mask_eos) {
    if (p.banned && p.banned[v]) return true;
    if (p.banned_pe && p.banned_pe[static_cast<int64_t>(b) * p.V + v]) return true;
    if (mask_eos && is_eos_tok(p, v)) return true;
    return false;
}

__device__ __forceinline__ int example_steps(const DecodeParams& p, int b) { return p.steps ? p.steps[b] : p.T; }

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

}  // namespace dbs_hip
