// SPDX-License-Identifier: MIT
//
// The decode of libdbs_hip for gfx950, as two launches:
//
//  1. the row pass (row_pass.hip) streams every row the search may read
//     from HBM, independently of the selection, and leaves per row the
//     NaN/+inf flag, the exact logsumexp (from logits) and a shortlist of the
//     best tokens with a bound on the rest;
//  2. the select pass (select.hip) walks the steps of each example over the
//     shortlists under the reference's total order, rescanning a row in full
//     whenever its bound could still change the selection, so the result is
//     the reference's bit for bit.
//
// This file plans the workspace and queues the two launches, plus the small
// elementwise helpers of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "engine.hpp"

namespace dbs_hip {

namespace {

__global__ void fill_f32_kernel(float* dst, float value, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t j = i; j < n; j += stride) dst[j] = value;
}

__global__ void length_penalty_kernel(const int32_t* lengths, int64_t n, float alpha, float* out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t j = i; j < n; j += stride) out[j] = length_penalty(lengths[j], alpha);
}

__global__ void check_steps_kernel(const int32_t* steps, int B, int T, int32_t* status) {
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    for (int i = static_cast<int>(threadIdx.x); i < B; i += static_cast<int>(blockDim.x))
        if (steps[i] < 1 || steps[i] > T) atomicOr(&bad, 1);
    __syncthreads();
    if (threadIdx.x == 0) status[0] = bad;
}

}  // namespace

DecodeLayout decode_layout(int B, int T, int K, int V, bool constrained, bool step_mode, int prefix_stride) {
    DecodeLayout L{};
    // Shortlist length: K plus a margin, while the row pass can pick its
    // threshold from the row's 256 lane maxima; wider beams rescan every row.
    int M = K <= 64 ? ((K + 16 + 7) / 8) * 8 : 0;
    if (const char* env = std::getenv("DBS_HIP_SHORTLIST")) {
        // testing knob: 0 forces full rescans, a small value forces fallbacks
        const int m = std::atoi(env);
        if (m >= 0 && m <= 256) M = m;
    }
    L.M = M;
    L.use_tau = (!constrained && !step_mode && M > 0) ? 1 : 0;
    L.prefix_cap = step_mode ? prefix_stride : T + 1;
    L.sel = select_layout(B, T, K, M, constrained, step_mode, L.prefix_cap);
    const int64_t rows = step_mode ? static_cast<int64_t>(B) * K : static_cast<int64_t>(B) * T * K;
    auto align = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t off = 0;
    L.off_rowinfo = off;
    off = align(off + sizeof(RowInfo) * static_cast<size_t>(rows));
    L.off_short = off;
    off = align(off + sizeof(ShortEntry) * static_cast<size_t>(rows) * static_cast<size_t>(M));
    L.off_prefix = off;
    if (constrained && !step_mode && !L.sel.prefix_in_lds)
        off = align(off + sizeof(int32_t) * 2 * static_cast<size_t>(B) * K * L.prefix_cap);
    L.off_blocked = off;
    if (constrained && !L.sel.blk_in_lds)
        off = align(off + sizeof(int32_t) * static_cast<size_t>(B) * K * (L.prefix_cap > 0 ? L.prefix_cap : 1));
    L.total = off == 0 ? 256 : off;
    (void)V;
    return L;
}

hipError_t launch_decode(const DecodeParams& p, const DecodeLayout& L, hipStream_t stream) {
    hipError_t e = launch_row_pass(p, stream);
    if (e != hipSuccess) return e;
    return launch_select(p, L.sel, stream);
}

hipError_t launch_fill_f32(float* dst, float value, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(fill_f32_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                       stream, dst, value, n);
    return hipGetLastError();
}

hipError_t launch_length_penalty(const int32_t* lengths, int64_t n, float alpha, float* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(length_penalty_kernel, dim3(static_cast<unsigned>(blocks < 4096 ? blocks : 4096)), dim3(256),
                       0, stream, lengths, n, alpha, out);
    return hipGetLastError();
}

hipError_t launch_check_steps(const int32_t* steps, int B, int T, int32_t* status, hipStream_t stream) {
    hipLaunchKernelGGL(check_steps_kernel, dim3(1), dim3(256), 0, stream, steps, B, T, status);
    return hipGetLastError();
}

}  // namespace dbs_hip
