// SPDX-License-Identifier: MIT
//
// Device helpers shared by the row-pass kernels and the select pass.
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

// Element i of a device array (per-example options, masks, beam state), read
// as global memory (a generic pointer compiles to flat loads, which may also
// touch LDS) and waited for right here, on the path that reads it: a load
// left outstanding where paths join makes the compiler wait for every
// outstanding global access at the next use of its register, which in the
// streaming row pass would drain the LDS-DMA loads in flight on every row.
template <class T>
__device__ __forceinline__ T gload(const T* a, int64_t i) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 1, "32-bit or byte elements");
    const T x = ((const __attribute__((address_space(1))) T*)a)[i];
    uint32_t u;
    if constexpr (sizeof(T) == 4) {
        __builtin_memcpy(&u, &x, 4);
    } else {
        u = static_cast<uint32_t>(x);
    }
    asm volatile("" : "+v"(u));
    if constexpr (sizeof(T) == 4) {
        T y;
        __builtin_memcpy(&y, &u, 4);
        return y;
    } else {
        return static_cast<T>(u);
    }
}

__device__ __forceinline__ bool in_eos_set(const DecodeParams& p, int32_t v) {
    for (int i = 0; i < p.n_eos; ++i)
        if (p.eos_set[i] == v) return true;
    return false;
}

// Options of example b: its EOS token (-1: none), minimum length and beams
// (reference cuda/dbs_cuda.cu:148-155 reads the same per-example arrays).
__device__ __forceinline__ int eos_of(const DecodeParams& p, int b) { return p.eos_pe ? gload(p.eos_pe, b) : p.eos; }
__device__ __forceinline__ int min_length_of(const DecodeParams& p, int b) {
    return p.minlen_pe ? gload(p.minlen_pe, b) : p.min_length;
}
__device__ __forceinline__ int beams_of(const DecodeParams& p, int b) { return p.beam_pe ? gload(p.beam_pe, b) : p.K; }

// Whether token v ends a hypothesis of example b: its EOS token or an extra
// one, where the example has EOS handling at all.
__device__ __forceinline__ bool is_eos_of(const DecodeParams& p, int b, int32_t v) {
    if (!p.eos_pe) return in_eos_set(p, v);  // the set holds the EOS token and the extra ones
    const int e = gload(p.eos_pe, b);
    return e >= 0 && (v == e || in_eos_set(p, v));
}

// Statically excluded tokens of a row: banned (shared or per example) and the
// EOS tokens while the new length is below min_length.
__device__ __forceinline__ bool static_masked(const DecodeParams& p, int b, int v, bool mask_eos) {
    if (p.banned && gload(p.banned, v)) return true;
    if (p.banned_pe && gload(p.banned_pe, static_cast<int64_t>(b) * p.V + v)) return true;
    if (mask_eos && is_eos_of(p, b, v)) return true;
    return false;
}

__device__ __forceinline__ int example_steps(const DecodeParams& p, int b) { return p.steps ? gload(p.steps, b) : p.T; }

__device__ __forceinline__ int wave_sum(int v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wavefront by DPP moves (row
// shifts, then the row broadcasts of lanes 15 and 31): six dependent adds,
// no LDS.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
    return x;
}

// The same maximum by DPP row shifts and row broadcasts (no LDS round trips):
// lane 63 ends with the maximum of all lanes, read back into every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
    const int lo = static_cast<int>(0xff800000u);  // -inf
    int x = static_cast<int>(f32_bits(v));
    auto step = [&](int y) { x = static_cast<int>(f32_bits(fmaxf(bits_f32(static_cast<uint32_t>(x)), bits_f32(static_cast<uint32_t>(y))))); };
    step(__builtin_amdgcn_update_dpp(lo, x, 0x111, 0xf, 0xf, false));  // row_shr:1
    step(__builtin_amdgcn_update_dpp(lo, x, 0x112, 0xf, 0xf, false));  // row_shr:2
    step(__builtin_amdgcn_update_dpp(lo, x, 0x114, 0xf, 0xf, false));  // row_shr:4
    step(__builtin_amdgcn_update_dpp(lo, x, 0x118, 0xf, 0xf, false));  // row_shr:8
    step(__builtin_amdgcn_update_dpp(lo, x, 0x142, 0xa, 0xf, false));  // row_bcast:15 into rows 1, 3
    step(__builtin_amdgcn_update_dpp(lo, x, 0x143, 0xc, 0xf, false));  // row_bcast:31 into rows 2, 3
    return bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(x, 63)));
}

// Workgroup barrier for LDS data only: the wavefront's LDS operations have
// completed; its global loads and stores may still be in flight across it
// (the barrier orders nothing in global memory).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Orders the LDS accesses of one wavefront (its lanes run in lockstep and the
// LDS serves a wavefront's requests in issue order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Whether the search may read row r, with its example and the length a token
// taken from it gives (decode: row (b, t, k) is read only for t < steps[b],
// and at t = 0 only beam 0; step: live, unfinished beams). Row indices fit in
// 31 bits (launch_decode refuses more rows), so the quotients are 32-bit.
__device__ __forceinline__ bool row_is_read(const DecodeParams& p, int64_t r, int& b, int& new_len) {
    const uint32_t r32 = static_cast<uint32_t>(r), K32 = static_cast<uint32_t>(p.K);
    const uint32_t bt = r32 / K32;
    const int k = static_cast<int>(r32 - bt * K32);
    if (p.step_mode) {
        b = static_cast<int>(bt);
        if (k >= beams_of(p, b)) return false;  // past the example's beams
        const float praw = gload(p.st_raw, r);
        if (!(praw < kInf && praw > -kInf)) return false;  // dead beam
        if (eos_of(p, b) >= 0 && gload(p.st_fin, r)) return false;  // finished
        new_len = gload(p.st_len, r) + 1;
        return true;
    }
    b = static_cast<int>(bt / static_cast<uint32_t>(p.T));
    const int t = static_cast<int>(bt - static_cast<uint32_t>(b) * static_cast<uint32_t>(p.T));
    if (t >= example_steps(p, b) || (t == 0 && k != 0) || k >= beams_of(p, b)) return false;
    new_len = t + 1;  // every unfinished live beam has length t at step t
    return true;
}

// The row a processing index q < rows stands for: step-major (every example's
// step t before step t + 1) in the overlapped decode, so the select pass can
// follow the row pass step by step; the index itself otherwise.
__device__ __forceinline__ int64_t row_of_ticket(const DecodeParams& p, int64_t q) {
    if (!p.step_done) return q;
    const uint32_t q32 = static_cast<uint32_t>(q), K = static_cast<uint32_t>(p.K), B = static_cast<uint32_t>(p.B);
    const uint32_t bt = q32 / K, k = q32 - bt * K;
    const uint32_t t = bt / B, b = bt - t * B;
    return static_cast<int64_t>((b * static_cast<uint32_t>(p.T) + t) * K + k);
}

// The next processing index of a persistent row-pass workgroup: its own
// stride without tickets, else the next ticket (thread-uniform; call from one
// thread and share).
__device__ __forceinline__ int64_t take_ticket(const DecodeParams& p, int64_t after, int64_t stride) {
    if (!p.row_ticket) return after + stride;
    // (an opaque per-lane offset of 0: the compiler's wavefront-wide atomic
    // combining would wait for the result right away)
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    return static_cast<int64_t>(
        __hip_atomic_fetch_add(p.row_ticket + zero, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Words of the overlapped decode (the row pass's RowInfo and shortlists, read
// by the select pass while the row pass still runs) are 64-bit device-scope
// atomics, each validated by its own tag (upper half non-zero once written,
// over a cleared workspace): coherent across the XCDs' L2 caches word by
// word, with no cache write-back or invalidation and no ordering between
// words. Otherwise plain stores (the select pass starts after the row pass).
__device__ __forceinline__ void publish_word(uint32_t* dst, uint32_t lo, uint32_t hi, bool coherent) {
    if (coherent) {
        const unsigned long long w = (static_cast<unsigned long long>(hi) << 32) | lo;
        __hip_atomic_store(reinterpret_cast<unsigned long long*>(dst), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        dst[0] = lo;
        dst[1] = hi;
    }
}

// Entry i of a shortlist: token + 1 is the overlapped decode's tag.
__device__ __forceinline__ void publish_entry(ShortEntry* out, int i, float lp, int32_t tok, bool coherent) {
    publish_word(reinterpret_cast<uint32_t*>(out + i), f32_bits(lp),
                 static_cast<uint32_t>(coherent ? tok + 1 : tok), coherent);
}

// A row's RowInfo: count + 2 and invalid + 1 are the overlapped decode's tags.
__device__ __forceinline__ void publish_rowinfo(RowInfo* dst, const RowInfo& info, bool coherent) {
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
    publish_word(d, f32_bits(info.lse), static_cast<uint32_t>(coherent ? info.count + 2 : info.count), coherent);
    publish_word(d + 2, f32_bits(info.bound), coherent ? info.invalid + 1u : info.invalid, coherent);
}

// Reads one tagged word; false while it is not written yet.
__device__ __forceinline__ bool read_tagged(const uint32_t* src, uint32_t& lo, uint32_t& hi) {
    const unsigned long long w =
        __hip_atomic_load(reinterpret_cast<const unsigned long long*>(src), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lo = static_cast<uint32_t>(w);
    hi = static_cast<uint32_t>(w >> 32);
    return hi != 0u;
}

// Row r's RowInfo and shortlist words are stored: count the row for its
// step. The count only tells the select pass when to start reading the step;
// each word it reads proves itself by its tag. One wavefront.
__device__ __forceinline__ void signal_row_done(const DecodeParams& p, int64_t r, int lane) {
    if (!p.step_done) return;
    if (lane == 0) {
        const int64_t bt = r / p.K;  // b * T + t
        __hip_atomic_fetch_add(p.step_done + bt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The key of the M-th largest of 256 keys held 4 per lane across one
// wavefront (1 <= M <= 256, keys below 2^BITS), by a radix select from the
// most significant bit: each round counts, with ballots, the keys that agree
// with the bits decided so far and have the next bit set, and keeps that half
// when it holds at least the rank still sought. Exact, ties included, and the
// same in every lane; no LDS and no lane exchange besides the ballots.
template <int BITS>
__device__ __forceinline__ uint32_t mth_largest_key(const uint32_t (&k)[4], int M) {
    uint32_t prefix = 0;
    int need = M;
#pragma unroll
    for (int bit = BITS - 1; bit >= 0; --bit) {
        const uint32_t want = (prefix >> bit) | 1u;
        int c = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) c += __popcll(__ballot((k[e] >> bit) == want));
        if (c >= need) {
            prefix |= 1u << bit;
        } else {
            need -= c;
        }
    }
    return prefix;
}

// Inverse of ordered_key (+0 for the key of zero).
__device__ __forceinline__ float key_value(uint32_t k) {
    return bits_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// The M-th largest of 256 lane maxima held 4 per lane (M <= 256, none NaN):
// at least M elements of the row are >= it.
__device__ __forceinline__ float shortlist_threshold(const float (&a)[4], int M) {
    uint32_t k[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) k[e] = ordered_key(a[e]);
    return key_value(mth_largest_key<32>(k, M));
}

// lane + d's value of v for the lanes < d (d = 1, 2, 4, 8: DPP row shifts;
// 16, 32: the gfx950 permlane swaps), without a trip through the LDS;
// other lanes get unspecified values.
template <int D>
__device__ __forceinline__ float from_lane_above(float v) {
    const int u = static_cast<int>(f32_bits(v));
    int r;
    if constexpr (D == 32) {
        r = static_cast<int>(__builtin_amdgcn_permlane32_swap(u, u, false, false)[1]);
    } else if constexpr (D == 16) {
        r = static_cast<int>(__builtin_amdgcn_permlane16_swap(u, u, false, false)[1]);
    } else {
        static_assert(D == 1 || D == 2 || D == 4 || D == 8, "row shift");
        r = __builtin_amdgcn_update_dpp(0, u, 0x100 + D, 0xf, 0xf, false);  // row_shl:D
    }
    return bits_f32(static_cast<uint32_t>(r));
}

// Combination of the 256 logsumexp lane sums held 4 per lane (lane j = 4 *
// lane + e), pairwise with strides 128, 64, ..., 1: lane j += lane j + s
// (reference src/kernels.hpp:196-202). The whole wavefront calls it.
template <int D>
__device__ __forceinline__ void lane_tree_step(float (&acc)[4], int lane) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float other = from_lane_above<D>(acc[e]);
        if (lane < D) acc[e] = acc[e] + other;  // 4 lane + e < 4 D
    }
}
__device__ __forceinline__ float lane_tree_sum(float (&acc)[4], int lane) {
    lane_tree_step<32>(acc, lane);
    lane_tree_step<16>(acc, lane);
    lane_tree_step<8>(acc, lane);
    lane_tree_step<4>(acc, lane);
    lane_tree_step<2>(acc, lane);
    lane_tree_step<1>(acc, lane);
    acc[0] = acc[0] + acc[2];
    acc[1] = acc[1] + acc[3];
    acc[0] = acc[0] + acc[1];
    return bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(acc[0])), 0)));
}

// Survivor key: value descending, then token ascending.
__device__ __forceinline__ uint64_t survivor_key(float x, int v) {
    return (static_cast<uint64_t>(ordered_key(x)) << 32) |
           static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(v));
}

constexpr int kRankSurvivors = 128;  // up to this many survivors are placed by rank, else sorted

// One wavefront: orders the n row survivors (finite x >= theta) kept in LDS
// and writes the row's shortlist (the best M allowed tokens by value desc,
// token asc, as log-probs) and RowInfo: the bound on every allowed token left
// out is the (M+1)-th allowed survivor, else theta. FILTER: the survivors may
// include statically masked tokens (banned, EOS below min_length of example
// b), which are dropped here (key 0 sorts last).
template <bool LOGITS, bool FILTER>
__device__ void finish_row_wave(const DecodeParams& p, int64_t r, float lse, float theta, bool any_bad,
                                uint64_t* s_key, float* s_x, int n, int lane, int b, bool mask_eos,
                                bool signal = true) {
    const int M = p.M;
    const bool coherent = p.step_done != nullptr;
    RowInfo info;
    info.lse = lse;
    info.invalid = any_bad ? 1u : 0u;
    info.bound = -kInf;
    info.count = 0;
    if (M > 0 && !(LOGITS && lse == -kInf)) {
        if (n > kSurvivorCap) {
            info.count = -1;
        } else {
            int np = 1;
            while (np < n) np <<= 1;
            int dropped = 0;
            if constexpr (FILTER) {
                for (int i0 = 0; i0 < n; i0 += 64) {
                    const int i = i0 + lane;
                    bool drop = false;
                    if (i < n) {
                        const int v = static_cast<int>(0xffffffffu - static_cast<uint32_t>(s_key[i] & 0xffffffffu));
                        drop = static_masked(p, b, v, mask_eos);
                        if (drop) s_key[i] = 0;
                    }
                    dropped += __popcll(__ballot(drop));
                }
            }
            n -= dropped;
            const int cnt = n < M ? n : M;
            ShortEntry* out = p.shortlist + r * M;
            float bx = theta;
            if (n + dropped <= kRankSurvivors) {
                // Few survivors: each lane ranks its own by counting the keys
                // above it (keys are distinct; dropped ones are 0) and writes
                // it in place; rank M is the bound.
                const int nall = n + dropped;
                wave_sync();
                int bound_lane = -1;
                float bound_x = -kInf;
                for (int i0 = 0; i0 < nall; i0 += 64) {
                    const int i = i0 + lane;
                    const uint64_t ki = i < nall ? s_key[i] : 0;
                    int rank = 0;
                    int jj = 0;
                    for (; jj + 8 <= nall; jj += 8) {  // eight keys in flight
                        uint64_t kk[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) kk[u] = s_key[jj + u];
#pragma unroll
                        for (int u = 0; u < 8; ++u) rank += static_cast<int>(kk[u] > ki);
                    }
                    for (; jj < nall; ++jj) rank += static_cast<int>(s_key[jj] > ki);
                    const bool live = i < nall && ki != 0;
                    const float x = live ? s_x[i] : 0.0f;
                    if (live && rank < M) {
                        const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(ki & 0xffffffffu));
                        publish_entry(out, rank, LOGITS ? x - lse : x, tok, coherent);
                    }
                    const uint64_t at_m = __ballot(live && rank == M);
                    if (at_m != 0) {
                        bound_lane = __ffsll(static_cast<long long>(at_m)) - 1;
                        bound_x = __shfl(x, bound_lane);
                    }
                }
                if (n > M) bx = bound_x;
            } else {
                for (int i = n + dropped + lane; i < np; i += 64) s_key[i] = 0;
                wave_sync();
                for (int kk = 2; kk <= np; kk <<= 1) {
                    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
                        for (int i = lane; i < np; i += 64) {
                            const int partner = i ^ jj;
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
                        wave_sync();
                    }
                }
                for (int i = lane; i < cnt; i += 64) {
                    const float x = s_x[i];
                    const int32_t tok = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(s_key[i] & 0xffffffffu));
                    publish_entry(out, i, LOGITS ? x - lse : x, tok, coherent);
                }
                if (n > M) bx = s_x[M];
            }
            info.count = cnt;
            info.bound = (bx > -kInf) ? (LOGITS ? bx - lse : bx) : -kInf;
        }
    }
    if (lane == 0) publish_rowinfo(p.rowinfo + r, info, coherent);
    if (signal) signal_row_done(p, r, lane);  // else the caller signals later
}

}  // namespace dbs_hip
