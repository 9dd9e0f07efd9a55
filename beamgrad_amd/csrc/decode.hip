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

#include <atomic>
#include <cstdlib>
#include <mutex>

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

// Range check of the per-example arrays (reference cuda/dbs_cuda.cu:376-385);
// one workgroup, status[0] = 0 when every entry passes.
__global__ void check_examples_kernel(const int32_t* steps, const int32_t* beams, const int32_t* eos,
                                      const int32_t* min_lengths, int B, int T, int K, int V, int32_t* status) {
    __shared__ int bad;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    for (int i = static_cast<int>(threadIdx.x); i < B; i += static_cast<int>(blockDim.x)) {
        const bool ok = (!steps || (steps[i] >= 1 && steps[i] <= T)) && (!beams || (beams[i] >= 1 && beams[i] <= K)) &&
                        (!eos || (eos[i] >= -1 && eos[i] < V)) && (!min_lengths || min_lengths[i] >= 0);
        if (!ok) atomicOr(&bad, 1);
    }
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
    L.off_sync = off;
    if (!step_mode) off = align(off + sync_bytes(B, T));
    L.total = off == 0 ? 256 : off;
    (void)V;
    return L;
}

std::atomic<int> g_overlap{-1};

namespace {

// The second stream of the overlapped decode and its two events, per device
// (default priority; created on first use, kept until the process ends).
struct Aux {
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, done = nullptr;
    int cus = 0;
};
Aux g_aux[64];
std::mutex g_aux_mutex;

hipError_t aux_for(int device, Aux*& out) {
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    Aux& a = g_aux[device];
    if (!a.stream) {
        hipError_t e = hipDeviceGetAttribute(&a.cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&a.start, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&a.done, hipEventDisableTiming);
        if (e != hipSuccess) {
            a.stream = nullptr;
            return e;
        }
    }
    out = &a;
    return hipSuccess;
}

}  // namespace

size_t sync_bytes(int B, int T) {
    return ((sizeof(int32_t) * static_cast<size_t>(B) * static_cast<size_t>(T) + 7) & ~static_cast<size_t>(7)) +
           sizeof(unsigned long long);
}

// The row pass, then the select pass. With several steps and at most half
// the CUs taken by the select pass's workgroups (one per example), the select
// pass can run alongside on a second stream, following the row pass step by
// step: the row pass is queued first and never waits on the select pass, and
// its rows are handed out by ticket, so it always progresses on the CUs left.
// By default constrained decodes (n-gram blocking, repetition penalty) do,
// whose select pass is as long as the row pass, and decodes whose row pass is
// one of the persistent kernels (16-bit rows kept on chip), which lose only
// the B CUs they leave free (MI355X: C2 2.00 -> 1.89 ms, C5 forward 2.35 ->
// 1.75 ms). The one-read log-prob kernel runs several workgroups per CU and
// loses more than the overlap saves (C4 3.03 -> 3.58 ms), so it does not.
hipError_t launch_decode(const DecodeParams& p0, const DecodeLayout& L, hipStream_t stream, char* ws) {
    DecodeParams p = p0;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_aux_mutex);
    Aux* aux = nullptr;
    const int mode = g_overlap.load(std::memory_order_relaxed);
    const bool want =
        !p.step_mode && p.T > 1 && (mode == 1 || (mode == -1 && (p.constrained || row_pass_persistent(p))));
    if (want) {
        e = aux_for(device, aux);
        if (e != hipSuccess) return e;
    }
    if (!want || 2 * p.B > aux->cus) {
        e = launch_row_pass(p, stream);
        if (e != hipSuccess) return e;
        return launch_select(p, L.sel, stream);
    }
    char* sync = ws + L.off_sync;
    p.step_done = reinterpret_cast<int32_t*>(sync);
    p.row_ticket = reinterpret_cast<unsigned long long*>(sync + sync_bytes(p.B, p.T) - sizeof(unsigned long long));
    p.reserve_cus = p.B;  // a persistent row pass would otherwise hold every CU until it ends
    e = launch_fill_f32(reinterpret_cast<float*>(sync), 0.0f, static_cast<int64_t>(sync_bytes(p.B, p.T) / 4), stream);
    if (e == hipSuccess) e = hipEventRecord(aux->start, stream);
    if (e == hipSuccess) e = launch_row_pass(p, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(aux->stream, aux->start, 0);
    if (e == hipSuccess) e = launch_select(p, L.sel, aux->stream);
    if (e == hipSuccess) e = hipEventRecord(aux->done, aux->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, aux->done, 0);
    return e;
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
    return launch_check_examples(steps, nullptr, nullptr, nullptr, B, T, 1, 1, status, stream);
}

hipError_t launch_check_examples(const int32_t* steps, const int32_t* beams, const int32_t* eos,
                                 const int32_t* min_lengths, int B, int T, int K, int V, int32_t* status,
                                 hipStream_t stream) {
    hipLaunchKernelGGL(check_examples_kernel, dim3(1), dim3(256), 0, stream, steps, beams, eos, min_lengths, B, T, K,
                       V, status);
    return hipGetLastError();
}

}  // namespace dbs_hip
