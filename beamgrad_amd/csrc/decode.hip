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
#include <cstring>
#include <mutex>

#include "engine.hpp"

namespace dbs_hip {

namespace {

// Zeroes up to three byte ranges in one launch (each 4-byte aligned and a
// multiple of 4 bytes long; 16-byte stores where a range allows them).
struct ClearRanges {
    char* ptr[3];
    int64_t bytes[3];
    int n;
};

__global__ __launch_bounds__(256) void clear_ranges_kernel(ClearRanges c) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (int r = 0; r < c.n; ++r) {
        char* const dst = c.ptr[r];
        const int64_t bytes = c.bytes[r];
        if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0 && (bytes & 15) == 0) {
            uint4* d4 = reinterpret_cast<uint4*>(dst);
            for (int64_t i = first; i < bytes / 16; i += stride) d4[i] = make_uint4(0u, 0u, 0u, 0u);
        } else {
            uint32_t* d1 = reinterpret_cast<uint32_t*>(dst);
            for (int64_t i = first; i < bytes / 4; i += stride) d1[i] = 0u;
        }
    }
}

hipError_t launch_clear_ranges(const ClearRanges& c, hipStream_t stream) {
    int64_t most = 0;
    for (int r = 0; r < c.n; ++r) most = c.bytes[r] / 16 > most ? c.bytes[r] / 16 : most;
    if (c.n == 0) return hipSuccess;
    const int64_t blocks = (most + 255) / 256;
    hipLaunchKernelGGL(clear_ranges_kernel, dim3(static_cast<unsigned>(blocks < 1 ? 1 : (blocks < 4096 ? blocks : 4096))),
                       dim3(256), 0, stream, c);
    return hipGetLastError();
}

// The decode trace in the dtypes torch returns it in: the int32 indices as
// int64, the from-log-prob flags as bool, and the per-example steps (T where
// none were given), in one launch.
__global__ __launch_bounds__(256) void widen_trace_kernel(WidenTrace w) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (int64_t i = first; i < w.n_trace; i += stride) {
        w.tokens64[i] = w.tokens[i];
        w.parents64[i] = w.parents[i];
        w.lengths64[i] = w.lengths[i];
        w.flp_bool[i] = w.flp[i] != 0 ? 1 : 0;
    }
    for (int64_t i = first; i < w.n_final; i += stride) w.final_len64[i] = w.final_len[i];
    for (int64_t i = first; i < w.n_steps; i += stride) w.steps64[i] = w.steps ? w.steps[i] : w.T;
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

DecodeLayout decode_layout(int B, int T, int K, int V, bool constrained, bool step_mode, int prefix_stride,
                           int keep) {
    DecodeLayout L{};
    // Shortlist length: the candidates kept per step (K, or the relaxed
    // pool) plus a margin, while the row pass can pick its threshold from the
    // row's 256 lane maxima; more rescan every row.
    const int kept = keep > 0 ? keep : K;
    int M = kept <= 64 ? ((kept + 16 + 7) / 8) * 8 : 0;
    if (const char* env = std::getenv("DBS_HIP_SHORTLIST")) {
        // testing knob: 0 forces full rescans, a small value forces fallbacks
        const int m = std::atoi(env);
        if (m >= 0 && m <= 256) M = m;
    }
    L.M = M;
    L.use_tau = (!constrained && !step_mode && M > 0 && kept == K) ? 1 : 0;
    L.prefix_cap = step_mode ? prefix_stride : T + 1;
    L.sel = select_layout(B, T, K, M, constrained, step_mode, L.prefix_cap, kept);
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
    L.total = off;
    (void)V;
    return L;
}

std::atomic<int> g_overlap{-1};

namespace {

// The second stream of the overlapped decode and its two events, one set per
// (device, caller stream): callers on different streams never share one, so
// their decodes do not serialise. Default priority; created on first use.
// The table holds kMaxAux sets; once it is full, the set a new caller stream
// gets is the least recently used one of its device, rebound to it (the
// callers that shared it then serialise their select passes on its stream,
// still in order), or, with none on its device, the least recently used one
// of any device, its stream and events made anew on this device.
struct Aux {
    int device = -1;
    hipStream_t caller = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, done = nullptr;
    int cus = 0;
    uint64_t last_use = 0;
    uint64_t epoch = 0;  // changes whenever `stream` is destroyed and created anew
    std::mutex mutex;    // one decode's enqueue sequence (or read-back) at a time on this set
};
constexpr int kMaxAux = 64;
Aux g_aux[kMaxAux];
int g_aux_used = 0;
uint64_t g_aux_clock = 0;
std::mutex g_aux_mutex;  // guards the table, not the launches
uint64_t g_aux_epoch = 0;

// The overlapped decode this thread launched last: the set and the stream its
// select pass ran on (for the read-back that ends it).
struct LastOverlap {
    const int32_t* fault = nullptr;
    Aux* set = nullptr;
    hipStream_t stream = nullptr;
    uint64_t epoch = 0;
};
thread_local LastOverlap t_last_overlap;

// Pinned host memory for read-backs, per thread (a copy into pageable memory
// goes through the runtime's own staging and costs ~10 us more per call).
struct Staging {
    void* ptr = nullptr;
    size_t cap = 0;
};
thread_local Staging t_staging;

// Stream, events and CU count of a set on `device` (current).
hipError_t aux_create(Aux& a, int device) {
    a.stream = nullptr;
    a.start = a.done = nullptr;
    hipError_t e = hipDeviceGetAttribute(&a.cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&a.start, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&a.done, hipEventDisableTiming);
    a.epoch = ++g_aux_epoch;
    if (e != hipSuccess) {
        if (a.stream) (void)hipStreamDestroy(a.stream);
        if (a.start) (void)hipEventDestroy(a.start);
        a.stream = nullptr;
        a.start = a.done = nullptr;
        a.device = -1;
        return e;
    }
    a.device = device;
    return hipSuccess;
}

// The caller's set (created, or taken over from the least recently used
// one, on first use).
hipError_t aux_for(int device, hipStream_t caller, Aux*& out) {
    out = nullptr;
    std::lock_guard<std::mutex> lock(g_aux_mutex);
    const uint64_t now = ++g_aux_clock;
    for (int i = 0; i < g_aux_used; ++i) {
        if (g_aux[i].device == device && g_aux[i].caller == caller) {
            g_aux[i].last_use = now;
            out = &g_aux[i];
            return hipSuccess;
        }
    }
    if (g_aux_used < kMaxAux) {
        Aux& a = g_aux[g_aux_used];
        const hipError_t e = aux_create(a, device);
        if (e != hipSuccess) return e;
        a.caller = caller;
        a.last_use = now;
        ++g_aux_used;
        out = &a;
        return hipSuccess;
    }
    Aux* same = nullptr;
    Aux* any = nullptr;
    for (int i = 0; i < kMaxAux; ++i) {
        Aux& a = g_aux[i];
        if (a.device == device && (!same || a.last_use < same->last_use)) same = &a;
        if (!any || a.last_use < any->last_use) any = &a;
    }
    if (same) {
        same->caller = caller;
        same->last_use = now;
        out = same;
        return hipSuccess;
    }
    // no set on this device: the oldest one moves here (its stream finishes
    // the work already queued on it before it is destroyed)
    std::lock_guard<std::mutex> busy(any->mutex);
    if (any->stream) (void)hipStreamDestroy(any->stream);
    if (any->start) (void)hipEventDestroy(any->start);
    if (any->done) (void)hipEventDestroy(any->done);
    const hipError_t e = aux_create(*any, device);
    if (e != hipSuccess) return e;
    any->caller = caller;
    any->last_use = now;
    out = any;
    return hipSuccess;
}

// Bound of one select-pass wait: 2 s of the 100 MHz real-time counter. Test
// knob DBS_HIP_TEST_WAIT_GIVE_UP=1: every wait needs one row more than the
// row pass ever counts and gives up after 10 us, so the error path runs with
// every kernel exiting normally.
void wait_policy(DecodeParams& p) {
    p.wait_ticks = 200000000ull;
    p.wait_extra = 0;
    const char* env = std::getenv("DBS_HIP_TEST_WAIT_GIVE_UP");
    if (env && env[0] == '1') {
        p.wait_ticks = 1000ull;
        p.wait_extra = 1;
    }
}

}  // namespace

size_t sync_bytes(int B, int T) {
    // [B, T] step counts, the fault word (padded to 8 bytes), the row ticket,
    // the split launch's claims [B]
    return ((sizeof(int32_t) * static_cast<size_t>(B) * static_cast<size_t>(T) + 7) & ~static_cast<size_t>(7)) + 8 +
           sizeof(unsigned long long) + sizeof(int32_t) * static_cast<size_t>(B);
}

// The row pass, then the select pass. With several steps and at most half
// the CUs taken by the select pass's workgroups (one per example), the select
// pass can run alongside on a second stream, following the row pass step by
// step: the row pass is queued first and never waits on the select pass, and
// its rows are handed out by ticket, so it always progresses on the CUs left.
// By default constrained decodes (n-gram blocking, repetition penalty) do,
// whose select pass is as long as the row pass; decodes whose row pass is
// one of the persistent kernels (16-bit rows kept on chip), which lose only
// the CUs they leave free (MI355X: C2 2.00 -> 1.89 ms, C5 forward 2.35 ->
// 1.75 ms); and decodes with the workgroup select pass beside the one-read
// log-prob kernel (one workgroup per row) when at most one example per 8 CUs
// lets the select pass hold its CUs (C4 2.73 -> 2.13 ms; shared CUs made it
// 3.53 ms).
// *fault: the overlapped decode's fault word (non-zero once a select-pass
// wait gave up), else null.
hipError_t launch_decode(const DecodeParams& p0, const DecodeLayout& L, hipStream_t stream, char* ws,
                         int32_t** fault, bool allow_overlap) {
    DecodeParams p = p0;
    *fault = nullptr;
    // Row indices are 31-bit on the device.
    const int64_t rows = static_cast<int64_t>(p.B) * (p.step_mode ? 1 : p.T) * p.K;
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    Aux* aux = nullptr;
    const int mode = g_overlap.load(std::memory_order_relaxed);
    bool want = allow_overlap && !p.step_mode && p.T > 1 &&
                (mode == 1 || (mode == -1 && (p.constrained || row_pass_persistent(p) || !select_narrow(p))));
    // Under stream capture the two passes run one after the other: a graph
    // may start its branches in any order, and a select pass started before
    // the row pass would wait for rows nobody is producing.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (want && hipStreamIsCapturing(stream, &capture) == hipSuccess && capture != hipStreamCaptureStatusNone)
        want = false;
    if (want) {
        e = aux_for(device, stream, aux);
        if (e != hipSuccess) return e;
    }
    const int reserve = select_reserve_cus(p);
    const bool persistent = row_pass_persistent(p);
    // Beside a row pass of one workgroup per row, a select pass of at most
    // one workgroup per 8 CUs holds its CUs (select_hold: the workgroup pass,
    // and the one-wavefront pass of a constrained decode); a larger one
    // shares them. An unconstrained decode overlaps such a row pass only
    // when its select pass holds its CUs (shared, its steps ran ~3x slower
    // than alone).
    const bool hold = !persistent && aux && 8 * reserve <= aux->cus;
    if (aux && mode == -1 && !p.constrained && !persistent && !hold) aux = nullptr;
    // One launch zeroes the row logsumexps (rows the search does not read keep
    // 0) and, in the overlapped decode, the counters and the RowInfo and
    // shortlist words (tag 0: not written).
    ClearRanges clear{};
    if (p.row_lse) {
        clear.ptr[clear.n] = reinterpret_cast<char*>(p.row_lse);
        clear.bytes[clear.n++] = static_cast<int64_t>(sizeof(float)) * rows;
    }
    if (!aux || 2 * reserve > aux->cus) {
        e = launch_clear_ranges(clear, stream);
        if (e == hipSuccess) e = launch_row_pass(p, stream);
        if (e != hipSuccess) return e;
        return launch_select(p, L.sel, stream);
    }
    char* sync = ws + L.off_sync;
    const size_t counts = (sizeof(int32_t) * static_cast<size_t>(p.B) * static_cast<size_t>(p.T) + 7) & ~static_cast<size_t>(7);
    p.step_done = reinterpret_cast<int32_t*>(sync);
    p.fault = reinterpret_cast<int32_t*>(sync + counts);
    p.row_ticket = reinterpret_cast<unsigned long long*>(sync + counts + 8);
    int32_t* claimed = reinterpret_cast<int32_t*>(sync + counts + 8 + sizeof(unsigned long long));
    p.reserve_cus = reserve;  // a persistent row pass would otherwise hold every CU until it ends
    wait_policy(p);
    std::lock_guard<std::mutex> lock(aux->mutex);
    // (the workspace ranges rounded up to 16 bytes, inside the workspace)
    clear.ptr[clear.n] = sync;
    clear.bytes[clear.n++] = static_cast<int64_t>((sync_bytes(p.B, p.T) + 15) & ~static_cast<size_t>(15));
    clear.ptr[clear.n] = ws + L.off_rowinfo;
    clear.bytes[clear.n++] = static_cast<int64_t>((L.off_prefix - L.off_rowinfo + 15) & ~static_cast<size_t>(15));
    e = launch_clear_ranges(clear, stream);
    if (e == hipSuccess) e = hipEventRecord(aux->start, stream);
    // A persistent row pass is launched first: its grid leaves the select
    // pass's CUs free. A row pass of one workgroup per row would fill every
    // CU before the select pass's workgroups are placed, so the select pass
    // goes first there, split in two launches (DecodeParams::claimed): the
    // early one before the row pass takes the examples whose first row comes
    // within 200 us, the late one after it takes the rest. The streams are
    // not guaranteed to run at once (HIP maps streams onto a few hardware
    // queues, shared once there are more streams), and no select-pass wait
    // may depend on a launch submitted after it.
    p.select_hold = hold ? 1 : 0;
    if (e == hipSuccess && persistent) e = launch_row_pass(p, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(aux->stream, aux->start, 0);
    if (persistent) {
        if (e == hipSuccess) e = launch_select(p, L.sel, aux->stream);
    } else {
        DecodeParams early = p;
        early.claimed = claimed;
        early.early = 1;
        early.early_ticks = 20000;  // 200 us of the 100 MHz counter
        if (e == hipSuccess) e = launch_select(early, L.sel, aux->stream);
        if (e == hipSuccess) e = launch_row_pass(p, stream);
        DecodeParams late = early;
        late.early = 0;
        if (e == hipSuccess) e = launch_select(late, L.sel, aux->stream);
    }
    if (e == hipSuccess) e = hipEventRecord(aux->done, aux->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, aux->done, 0);
    if (e == hipSuccess) {
        *fault = p.fault;
        t_last_overlap = LastOverlap{p.fault, aux, aux->stream, aux->epoch};
    }
    return e;
}

hipError_t decode_read_back(const void* src, size_t bytes, void* dst, const int32_t* fault, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    Staging& st = t_staging;
    if (st.cap < bytes) {
        // no copy is pending into the old buffer: every read-back waits for its copy
        if (st.ptr) (void)hipHostFree(st.ptr);
        st.ptr = nullptr;
        st.cap = 0;
        const size_t cap = bytes < 4096 ? 4096 : bytes;
        const hipError_t e = hipHostMalloc(&st.ptr, cap, hipHostMallocDefault);
        if (e != hipSuccess) {
            st.ptr = nullptr;
            return e;
        }
        st.cap = cap;
    }
    // The select pass's stream, when `fault` is the last overlapped decode of
    // this thread and that stream still exists (its set's mutex, held until
    // the copy has landed, keeps it from being destroyed); else `stream`.
    const LastOverlap last = t_last_overlap;
    std::unique_lock<std::mutex> held;
    hipStream_t on = stream;
    if (fault && last.fault == fault && last.set) {
        std::lock_guard<std::mutex> table(g_aux_mutex);
        if (last.set->epoch == last.epoch && last.set->stream == last.stream) {
            held = std::unique_lock<std::mutex>(last.set->mutex);
            on = last.stream;
        }
    }
    hipError_t e = hipMemcpyAsync(st.ptr, src, bytes, hipMemcpyDeviceToHost, on);
    if (e == hipSuccess) e = hipStreamSynchronize(on);
    if (e == hipSuccess) std::memcpy(dst, st.ptr, bytes);
    return e;
}


hipError_t launch_widen_trace(const WidenTrace& w, hipStream_t stream) {
    const int64_t n = w.n_trace > w.n_final ? (w.n_trace > w.n_steps ? w.n_trace : w.n_steps)
                                            : (w.n_final > w.n_steps ? w.n_final : w.n_steps);
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(widen_trace_kernel, dim3(static_cast<unsigned>(blocks < 2048 ? blocks : 2048)), dim3(256), 0,
                       stream, w);
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
