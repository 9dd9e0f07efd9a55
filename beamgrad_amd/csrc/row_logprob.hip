// SPDX-License-Identifier: MIT
//
// One-read row pass for decodes that take log-probabilities (not logits).
//
// Such a row has no logsumexp to fold (reference src/decoder.cpp:122-187
// reads the log-prob itself); the row pass only flags NaN / +inf and keeps
// the shortlist: the best M allowed tokens by (log-prob desc, token asc) and
// an upper bound on every allowed token left out (the row scan of reference
// src/kernels.hpp:54-140, src/kernels_scalar.cpp:16-79, restated as a
// threshold and a survivor list). Both need the row twice — the threshold
// from the whole row, then the survivors above it — so the row stays in
// VGPRs in between and is read from HBM once:
//
//   * one 256-thread workgroup per row; the row is cut into 16-byte blocks
//     aligned in memory (the first may start before the row, the last end
//     after it; a block holding a row byte never crosses a page), and thread
//     t loads blocks t, t + 256, ... with one buffer load each, all in
//     flight at once; several workgroups share a CU, so one row's loads
//     overlap the others' work;
//   * elements outside the row (and blocks past its end, read as zeros by the
//     clipped buffer view) become -inf, which changes neither the maximum,
//     the flag nor the survivors;
//   * each thread takes the maximum of its elements and the NaN / +inf flag
//     (packed 16-bit integer max/min over the raw patterns for 16-bit rows);
//     theta is the M-th largest of the 256 thread maxima, so at least M
//     elements are >= theta;
//   * the survivors (finite, allowed, x >= theta) are taken from the
//     registers; each survivor's rank among them (a count of the survivors
//     before it) places it in the shortlist, every thread ranking some.
//
// A row with NaN or +inf keeps no shortlist (the select pass reads such a row
// in full), as in the other row passes.
#include <hip/hip_runtime.h>

#include "row_helpers.hpp"

namespace dbs_hip {

namespace {

constexpr int kLpThreads = 256;
constexpr int kLpMaxBlocks = 40;  // 16-byte blocks per thread, at most
constexpr int kLpBlockCap = 512;  // blocks holding survivors, at most (else the row is read in full)

// Element i of a block as f32. binary16 goes through the hardware conversion,
// exact for every finite value and the infinities (denormals are kept); a NaN
// never reaches a shortlist (the row is flagged and read in full instead), so
// its payload does not matter here.
template <int DT>
__device__ __forceinline__ float element_of(const v4u32& d, int i) {
    if constexpr (DT == 0) {
        return bits_f32(d[i]);
    } else if constexpr (DT == 1) {
        const uint16_t h = static_cast<uint16_t>((d[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        return static_cast<float>(__builtin_bit_cast(_Float16, h));
    } else {
        return pattern_value<DT>((d[i >> 1] >> (16 * (i & 1))) & 0xffffu);
    }
}

template <int DT>
__device__ __forceinline__ void set_neg_inf(v4u32& d, int i) {
    if constexpr (DT == 0) {
        d[i] = 0xff800000u;
    } else {
        const uint32_t ninf = DT == 1 ? 0xfc00u : 0xff80u;
        const int sh = 16 * (i & 1);
        d[i >> 1] = (d[i >> 1] & ~(0xffffu << sh)) | (ninf << sh);
    }
}

template <int DT, int C>
__global__ __launch_bounds__(kLpThreads) void row_logprob_kernel(DecodeParams p) {
    __shared__ uint64_t s_key[kSurvivorCap];
    __shared__ float s_x[kSurvivorCap];
    __shared__ float s_tmax[kLpThreads];
    __shared__ v4u32 s_blk[kLpBlockCap];
    __shared__ int s_blk_v0[kLpBlockCap];
    __shared__ int s_count;
    __shared__ int s_nblk;
    __shared__ int s_bad;
    __shared__ float s_theta;
    __shared__ float s_bound;

    const int tid = static_cast<int>(threadIdx.x);
    const int64_t r = row_of_ticket(p, blockIdx.x);
    int b, new_len;
    if (!row_is_read(p, r, b, new_len)) return;
    const bool mask_eos = new_len < min_length_of(p, b);
    const int V = p.V;
    const int M = p.M;
    constexpr int esz = DT == 0 ? 4 : 2;
    constexpr int epb = 16 / esz;  // elements per block

    // Blocks aligned in memory: block q holds elements q * epb - lead_e ...
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(p.x) + static_cast<uintptr_t>(r) * V * esz;
    const int lead = static_cast<int>(a0 & 15u);
    const int lead_e = lead / esz;
    const int nblk = (lead + V * esz + 15) >> 4;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(a0 - lead), 0, 16 * nblk, 0x00020000);

    if (tid == 0) {
        s_count = 0;
        s_nblk = 0;
        s_bad = 0;
    }
    v4u32 d[C];
#pragma unroll
    for (int c = 0; c < C; ++c) d[c] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * tid, 4096 * c, 0);

    // Elements outside the row become -inf.
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int v0 = (c * kLpThreads + tid) * epb - lead_e;
        if (v0 < 0 || v0 + epb > V) {
#pragma unroll
            for (int i = 0; i < epb; ++i)
                if (v0 + i < 0 || v0 + i >= V) set_neg_inf<DT>(d[c], i);
        }
    }

    // Thread maximum over x < +inf and the NaN / +inf flag.
    float tmax = -kInf;
    bool bad = false;
    if constexpr (DT == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = bits_f32(d[c][i]);
                bad = bad || __builtin_amdgcn_classf(x, 0x203);  // sNaN, qNaN, +inf
                tmax = fmaxf(tmax, x);
            }
        }
    } else {
        // Signed max/min and unsigned max of the raw patterns: the largest
        // value is the largest non-negative pattern, else the smallest
        // (most negative) signed one; a signed max >= +inf's pattern flags
        // +inf or a positive NaN, an unsigned max above -inf's a negative NaN.
        uint32_t smax = 0x80008000u, smin = 0x7fff7fffu, umax = 0u;
#pragma unroll
        for (int c = 0; c < C; ++c) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                smax = pk_max_i16(smax, d[c][i]);
                smin = pk_min_i16(smin, d[c][i]);
                umax = pk_max_u16(umax, d[c][i]);
            }
        }
        const int pos_inf = DT == 1 ? 0x7c00 : 0x7f80;
        const uint32_t neg_inf = DT == 1 ? 0xfc00u : 0xff80u;
        int best = -32768;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int16_t hmax = static_cast<int16_t>(smax >> (16 * h));
            const int16_t hmin = static_cast<int16_t>(smin >> (16 * h));
            bad = bad || hmax >= pos_inf || ((umax >> (16 * h)) & 0xffffu) > neg_inf;
            best = max(best, key16(static_cast<uint16_t>(hmax >= 0 ? hmax : hmin)));
        }
        tmax = pattern_value<DT>(key_pattern(best));
    }
    s_tmax[tid] = tmax;
    if (__any(bad) && (tid & 63) == 0) s_bad = 1;
    __syncthreads();

    const bool any_bad = s_bad != 0;
    if (M > 0 && !any_bad && tid < 64) {
        float a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = s_tmax[4 * tid + e];
        const float th = shortlist_threshold(a, tid, M);
        if (tid == 0) s_theta = th;
    }
    __syncthreads();
    const float theta = (M > 0 && !any_bad) ? s_theta : -kInf;
    const bool full = M > 0 && !(theta > -kInf);  // no shortlist: every element would survive

    // Survivors: finite, allowed, x >= theta. Only threads whose maximum
    // reaches theta hold any: their blocks whose maximum reaches it are
    // copied to LDS, and the workgroup then takes the survivors from there.
    if (M > 0 && !full && tmax >= theta) {
        // (an opaque copy: the block starts are recomputed here rather than
        // kept in registers from the edge test above)
        int vt = tid * epb - lead_e;
        asm volatile("" : "+v"(vt));
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float bm = -kInf;
#pragma unroll
            for (int i = 0; i < epb; ++i) bm = fmaxf(bm, element_of<DT>(d[c], i));
            if (bm >= theta) {
                const int slot = atomicAdd(&s_nblk, 1);
                if (slot < kLpBlockCap) {
                    s_blk[slot] = d[c];
                    s_blk_v0[slot] = vt + c * kLpThreads * epb;
                }
            }
        }
    }
    __syncthreads();
    const int nblk_hit = s_nblk;
    const bool keep = M > 0 && !full && nblk_hit <= kLpBlockCap;
    if (keep) {
        for (int i = tid; i < nblk_hit; i += kLpThreads) {
            const v4u32 blk = s_blk[i];
            const int v0 = s_blk_v0[i];
#pragma unroll
            for (int e = 0; e < epb; ++e) {
                const float x = element_of<DT>(blk, e);
                if (x >= theta && x < kInf && !static_masked(p, b, v0 + e, mask_eos)) {
                    const int slot = atomicAdd(&s_count, 1);
                    if (slot < kSurvivorCap) {
                        s_key[slot] = survivor_key(x, v0 + e);
                        s_x[slot] = x;
                    }
                }
            }
        }
    }
    __syncthreads();

    // The shortlist: each survivor's rank is the number of survivors before
    // it (keys are distinct); ranks below M are written in place, rank M is
    // the bound on the rest.
    const bool coherent = p.step_done != nullptr;
    const int n = s_count;
    const bool listed = keep && n <= kSurvivorCap;
    if (listed) {
        ShortEntry* out = p.shortlist + r * M;
        for (int i = tid; i < n; i += kLpThreads) {
            const uint64_t ki = s_key[i];
            int rank = 0;
            int j = 0;
            for (; j + 4 <= n; j += 4) {
                const uint64_t k0 = s_key[j], k1 = s_key[j + 1], k2 = s_key[j + 2], k3 = s_key[j + 3];
                rank += static_cast<int>(k0 > ki) + static_cast<int>(k1 > ki) + static_cast<int>(k2 > ki) +
                        static_cast<int>(k3 > ki);
            }
            for (; j < n; ++j) rank += static_cast<int>(s_key[j] > ki);
            if (rank < M) {
                const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(ki & 0xffffffffu));
                publish_entry(out, rank, s_x[i], tok, coherent);
            } else if (rank == M) {
                s_bound = s_x[i];
            }
        }
    }
    __syncthreads();
    if (tid < 64) {
        RowInfo info;
        info.lse = 0.0f;
        info.invalid = any_bad ? 1u : 0u;
        info.bound = -kInf;
        info.count = 0;
        if (M > 0) {
            if (listed) {
                info.count = n < M ? n : M;
                info.bound = n > M ? s_bound : theta;
            } else {
                info.count = -1;
            }
        }
        if (tid == 0) publish_rowinfo(p.rowinfo + r, info, coherent);
        signal_row_done(p, r, tid);
    }
}

// Blocks per thread for a row of V elements (the first block may start up to
// 15 bytes before the row).
int logprob_blocks(const DecodeParams& p) {
    const int64_t esz = p.dtype == 0 ? 4 : 2;
    const int64_t nblk = (15 + static_cast<int64_t>(p.V) * esz + 15) / 16;
    return static_cast<int>((nblk + kLpThreads - 1) / kLpThreads);
}

}  // namespace

bool row_logprob_eligible(const DecodeParams& p) {
    if (p.from_logits) return false;
    if (p.M > 256) return false;
    return logprob_blocks(p) <= kLpMaxBlocks;
}

hipError_t launch_row_logprob(const DecodeParams& p, int64_t rows, hipStream_t stream) {
    const int need = logprob_blocks(p);
    const dim3 grid(static_cast<unsigned>(rows));
#define DBS_LP_CASE(CB)                                                                                          \
    if (need <= CB) {                                                                                            \
        if (p.dtype == 0) hipLaunchKernelGGL((row_logprob_kernel<0, CB>), grid, dim3(kLpThreads), 0, stream, p); \
        else if (p.dtype == 1) hipLaunchKernelGGL((row_logprob_kernel<1, CB>), grid, dim3(kLpThreads), 0, stream, p); \
        else hipLaunchKernelGGL((row_logprob_kernel<2, CB>), grid, dim3(kLpThreads), 0, stream, p);             \
        return hipGetLastError();                                                                                \
    }
    DBS_LP_CASE(2)
    DBS_LP_CASE(4)
    DBS_LP_CASE(8)
    DBS_LP_CASE(12)
    DBS_LP_CASE(16)
    DBS_LP_CASE(20)
    DBS_LP_CASE(24)
    DBS_LP_CASE(28)
    DBS_LP_CASE(32)
    DBS_LP_CASE(40)
#undef DBS_LP_CASE
    return hipErrorInvalidValue;
}

}  // namespace dbs_hip
