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

// Bitonic sort (descending) of the 256 lane maxima held 4 per thread
// (element i = 4 * lane + e) across one wavefront.
__device__ __forceinline__ void sort256_desc(float (&a)[4], int lane) {
    for (int k = 2; k <= 256; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j >= 4) {
                const int lj = j >> 2;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float other = __shfl_xor(a[e], lj);
                    const int i = 4 * lane + e;
                    const bool desc = (i & k) == 0;
                    const bool is_lo = (i & j) == 0;
                    a[e] = (is_lo == desc) ? fmaxf(a[e], other) : fminf(a[e], other);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * lane + e;
                    if ((i & j) == 0) {
                        const int e2 = e + j;
                        const bool desc = (i & k) == 0;
                        const float lo = a[e], hi = a[e2];
                        const bool swap = desc ? (hi > lo) : (lo > hi);
                        if (swap) {
                            a[e] = hi;
                            a[e2] = lo;
                        }
                    }
                }
            }
        }
    }
}


template <int DT, bool LOGITS, bool VEC>
__global__ __launch_bounds__(kRowThreads) void row_pass_kernel(DecodeParams p) {
    __shared__ uint64_t s_key[kSurvivorCap];
    __shared__ float s_x[kSurvivorCap];
    __shared__ int s_count;

    const int lane = static_cast<int>(threadIdx.x);
    const int64_t r = blockIdx.x;
    const int K = p.K, V = p.V;
    int b, t, k, new_len;
    if (p.step_mode) {
        b = static_cast<int>(r / K);
        k = static_cast<int>(r % K);
        t = 0;
        const float praw = p.st_raw[r];
        if (!(praw < kInf && praw > -kInf)) return;           // dead beam: not read
        if (p.eos >= 0 && p.st_fin[r]) return;               // finished: not read
        new_len = p.st_len[r] + 1;
    } else {
        b = static_cast<int>(r / (static_cast<int64_t>(p.T) * K));
        t = static_cast<int>((r / K) % p.T);
        k = static_cast<int>(r % K);
        if (t >= example_steps(p, b) || (t == 0 && k != 0)) return;  // never read
        new_len = t + 1;  // every unfinished live beam has length t at step t
    }
    const bool mask_eos = new_len < p.min_length;
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
        float a[4] = {lmax[0], lmax[1], lmax[2], lmax[3]};
        sort256_desc(a, lane);
        const int idx = M - 1;
        const float mine = a[idx & 3];
        theta = __shfl(mine, idx >> 2);
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
                        s_key[slot] = (static_cast<uint64_t>(ordered_key(x[e])) << 32) |
                                      static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(v + e));
                        s_x[slot] = x[e];
                    }
                }
            }
        }
    }

    float lse = 0.0f;
    if (LOGITS) {
        if (do_lse) {
            // pairwise tree over the 256 lanes: lane j += lane j + s, s = 128 .. 1
            for (int s = 128; s >= 4; s >>= 1) {
                const int d = s >> 2;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float other = __shfl_down(acc[e], d);
                    if (4 * lane + e < s) acc[e] = acc[e] + other;
                }
            }
            acc[0] = acc[0] + acc[2];
            acc[1] = acc[1] + acc[3];
            acc[0] = acc[0] + acc[1];
            const float sum = __shfl(acc[0], 0);
            lse = logsumexp_from(rmax, sum);
        } else {
            lse = -kInf;
        }
    }
    __syncthreads();

    RowInfo info;
    info.lse = lse;
    info.invalid = any_bad ? 1u : 0u;
    info.bound = -kInf;
    info.count = 0;
    if (M > 0 && !(LOGITS && lse == -kInf)) {
        const int n = s_count;
        if (n > kSurvivorCap) {
            info.count = -1;
        } else {
            int np = 1;
            while (np < n) np <<= 1;
            for (int i = n + lane; i < np; i += kRowThreads) s_key[i] = 0;
            __syncthreads();
            // bitonic sort of (key, x) descending
            for (int kk = 2; kk <= np; kk <<= 1) {
                for (int j = kk >> 1; j > 0; j >>= 1) {
                    for (int i = lane; i < np; i += kRowThreads) {
                        const int partner = i ^ j;
                        if (partner > i) {
                            const bool desc = (i & kk) == 0;
                            const uint64_t ki = s_key[i], kp = s_key[partner];
                            if (desc ? (kp > ki) : (ki > kp)) {
                                s_key[i] = kp;
                                s_key[partner] = ki;
                                const float xi = s_x[i];
                                s_x[i] = s_x[partner];
                                s_x[partner] = xi;
                            }
                        }
                    }
                    __syncthreads();
                }
            }
            const int cnt = n < M ? n : M;
            ShortEntry* out = p.shortlist + r * M;
            for (int i = lane; i < cnt; i += kRowThreads) {
                const float x = s_x[i];
                const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(s_key[i] & 0xffffffffu));
                out[i].lp = LOGITS ? x - lse : x;
                out[i].token = tok;
            }
            float bx = n > M ? s_x[M] : theta;
            info.count = cnt;
            info.bound = (bx > -kInf) ? (LOGITS ? bx - lse : bx) : -kInf;
        }
    }
    if (lane == 0) p.rowinfo[r] = info;
}


}  // namespace

hipError_t launch_row_pass(const DecodeParams& p, hipStream_t stream) {
    const int64_t rows = p.step_mode ? static_cast<int64_t>(p.B) * p.K : static_cast<int64_t>(p.B) * p.T * p.K;
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    const size_t esz = p.dtype == 0 ? 4 : 2;
    const bool vec = (p.V % 4 == 0) && (reinterpret_cast<uintptr_t>(p.x) % (4 * esz) == 0);
    const dim3 grid(static_cast<unsigned>(rows));
    KernelTimer timer(kKindRowPass, stream);
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
