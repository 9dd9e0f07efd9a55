// SPDX-License-Identifier: MIT
//
// The row pass of the decode: every row the search may read is streamed from
// HBM independently of the selection, so the whole chip works on all B*T*K
// rows at once. Per row it produces the NaN/+inf flag, the exact logsumexp
// (from logits: the reference's fixed 256-lane fold order, reference
// src/logits.hpp:42-50, src/kernels_scalar.cpp:48-66), and a shortlist: the
// best M allowed tokens by (log-prob desc, token asc) with an upper bound on
// every allowed token left out, which the select pass uses to prove its
// selection exact.
#include <hip/hip_runtime.h>

#include <atomic>

#include "device_common.hpp"

namespace dbs_hip {

namespace {

// Four consecutive elements starting at v (v multiple of 4). VEC: the row
// start is aligned and V % 4 == 0, so one 16-byte (f32) or 8-byte (16-bit)
// load covers them; otherwise element loads with bounds checks.
template <int DT, bool VEC>
__device__ __forceinline__ void load4(const void* row, int v, int V, float (&x)[4], bool (&in)[4]) {
    if constexpr (VEC) {
        const bool ok = v < V;
#pragma unroll
        for (int e = 0; e < 4; ++e) in[e] = ok;
        if (!ok) {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = 0.0f;
            return;
        }
        if constexpr (DT == 0) {
            const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + v);
            x[0] = q.x; x[1] = q.y; x[2] = q.z; x[3] = q.w;
        } else {
            const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(row) + v);
            const uint16_t h[4] = {static_cast<uint16_t>(q.x & 0xffffu), static_cast<uint16_t>(q.x >> 16),
                                   static_cast<uint16_t>(q.y & 0xffffu), static_cast<uint16_t>(q.y >> 16)};
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = DT == 1 ? half_to_f32(h[e]) : bf16_to_f32(h[e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            in[e] = v + e < V;
            x[e] = in[e] ? load_one<DT>(row, v + e) : 0.0f;
        }
    }
}

// ---------------------------------------------------------------------------
// Row pass
// ---------------------------------------------------------------------------

// One row (one wavefront): row r, read by the search for example b with new
// length new_len.
template <int DT, bool LOGITS, bool VEC>
__device__ void row_pass_one(const DecodeParams& p, int64_t r, int b, int new_len, uint64_t* s_key, float* s_x,
                             int& s_count) {
    const int lane = static_cast<int>(threadIdx.x);
    const int V = p.V;
    const bool mask_eos = new_len < min_length_of(p, b);
    const size_t esz = DT == 0 ? 4 : 2;
    const char* row = static_cast<const char*>(p.x) + static_cast<size_t>(r) * static_cast<size_t>(V) * esz;
    const int nq = (V + kLanes - 1) / kLanes;
    const int M = p.M;

    // Pass 1: row maximum over x < +inf, lane maxima, NaN/+inf flag.
    float lmax[4] = {-kInf, -kInf, -kInf, -kInf};
    bool bad = false;
    for (int q = 0; q < nq; ++q) {
        const int v = q * kLanes + 4 * lane;
        float x[4];
        bool in[4];
        load4<DT, VEC>(row, v, V, x, in);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!in[e]) continue;
            if (!(x[e] < kInf)) bad = true;
            else if (x[e] > lmax[e]) lmax[e] = x[e];
        }
    }
    const float rmax = wave_max(fmaxf(fmaxf(lmax[0], lmax[1]), fmaxf(lmax[2], lmax[3])));
    const bool any_bad = __any(bad);

    // Shortlist threshold: the M-th largest lane maximum (M <= 256), so at
    // least M elements are >= theta.
    float theta = -kInf;
    if (M > 0) {
        const float a[4] = {lmax[0], lmax[1], lmax[2], lmax[3]};
        theta = shortlist_threshold(a, M);
    }
    if (lane == 0) s_count = 0;
    __syncthreads();

    // Pass 2: logsumexp lanes (lane j = v mod 256 folds in increasing v) and
    // the survivors x >= theta among the allowed finite tokens.
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool do_lse = LOGITS && rmax > -kInf;
    if (M > 0 || do_lse) {
        for (int q = 0; q < nq; ++q) {
            const int v = q * kLanes + 4 * lane;
            float x[4];
            bool in[4];
            load4<DT, VEC>(row, v, V, x, in);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (!in[e]) continue;
                const bool finite = x[e] < kInf && x[e] > -kInf;
                if (LOGITS && do_lse && finite) acc[e] = acc[e] + exp_nonpositive(x[e] - rmax);
                if (M > 0 && finite && x[e] >= theta && !static_masked(p, b, v + e, mask_eos)) {
                    const int slot = atomicAdd(&s_count, 1);
                    if (slot < kSurvivorCap) {
                        s_key[slot] = survivor_key(x[e], v + e);
                        s_x[slot] = x[e];
                    }
                }
            }
        }
    }

    float lse = 0.0f;
    if (LOGITS) {
        if (do_lse) {
            lse = logsumexp_from(rmax, lane_tree_sum(acc, lane));
        } else {
            lse = -kInf;
        }
    }
    __syncthreads();

    finish_row_wave<LOGITS, false>(p, r, lse, theta, any_bad, s_key, s_x, s_count, lane, b, mask_eos);
}

template <int DT, bool LOGITS, bool VEC>
__global__ __launch_bounds__(kRowThreads) void row_pass_kernel(DecodeParams p) {
    __shared__ uint64_t s_key[kSurvivorCap];
    __shared__ float s_x[kSurvivorCap];
    __shared__ int s_count;
    const int64_t r = row_of_ticket(p, blockIdx.x);
    int b, new_len;
    if (!row_is_read(p, r, b, new_len)) return;
    row_pass_one<DT, LOGITS, VEC>(p, r, b, new_len, s_key, s_x, s_count);
}

}  // namespace

std::atomic<int> g_row_pass_kind{-1};

bool row_pass_persistent(const DecodeParams& p) {
    const int kind = g_row_pass_kind.load(std::memory_order_relaxed);
    if ((kind == -1 || kind == 3) && row_logprob_eligible(p)) return false;
    if ((kind == 5 || (kind == -1 && row_relay_preferred(p))) && row_relay_eligible(p)) return true;
    if ((kind == -1 || kind == 1) && row_resident_eligible(p)) return true;
    return (kind == -1 || kind == 2) && row_pipe_eligible(p);
}

hipError_t launch_row_pass(const DecodeParams& p, hipStream_t stream) {
    const int64_t rows = p.step_mode ? static_cast<int64_t>(p.B) * p.K : static_cast<int64_t>(p.B) * p.T * p.K;
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    const size_t esz = p.dtype == 0 ? 4 : 2;
    const bool vec = (p.V % 4 == 0) && (reinterpret_cast<uintptr_t>(p.x) % (4 * esz) == 0);
    KernelTimer timer(kKindRowPass, stream);
    const int kind = g_row_pass_kind.load(std::memory_order_relaxed);
    if ((kind == -1 || kind == 3) && row_logprob_eligible(p)) return launch_row_logprob(p, rows, stream);
    if ((kind == 5 || (kind == -1 && row_relay_preferred(p))) && row_relay_eligible(p))
        return launch_row_relay(p, rows, stream);
    if ((kind == -1 || kind == 1) && row_resident_eligible(p)) return launch_row_resident(p, rows, stream);
    if ((kind == -1 || kind == 2) && row_pipe_eligible(p)) return launch_row_pipe(p, rows, stream);
    const dim3 grid(static_cast<unsigned>(rows));
#define DBS_ROW_PASS(DT, LG)                                                                                 \
    do {                                                                                                     \
        if (vec) hipLaunchKernelGGL((row_pass_kernel<DT, LG, true>), grid, dim3(kRowThreads), 0, stream, p); \
        else hipLaunchKernelGGL((row_pass_kernel<DT, LG, false>), grid, dim3(kRowThreads), 0, stream, p);    \
    } while (0)
    if (p.from_logits) {
        if (p.dtype == 0) DBS_ROW_PASS(0, true);
        else if (p.dtype == 1) DBS_ROW_PASS(1, true);
        else DBS_ROW_PASS(2, true);
    } else {
        if (p.dtype == 0) DBS_ROW_PASS(0, false);
        else if (p.dtype == 1) DBS_ROW_PASS(1, false);
        else DBS_ROW_PASS(2, false);
    }
#undef DBS_ROW_PASS
    return hipGetLastError();
}

}  // namespace dbs_hip
