// SPDX-License-Identifier: MIT
//
// The select pass of the decode: one workgroup per example walks the T steps
// (or the one step of the step API) over the row pass's shortlists.
//
// Per step it stages the step's row statistics and shortlists in LDS, builds
// the candidates (EOS carry-forward; shortlist entries with n-gram blocking
// and the repetition penalty), keeps the best K in an LDS collector under the
// reference's total order (reference src/common.hpp:269-302), and then proves
// the selection exact: a row whose bound could still beat the K-th selected
// candidate is rescanned in full from HBM. The trace, the beam state and the
// prefixes advance as in reference src/decoder.cpp:122-187, 314-350.
#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace dbs_hip {

namespace {

// Rows rescanned since the last reset (read through dbs_hip_profile_read).
__device__ unsigned long long g_rescanned_rows;
// Waits for a step of the overlapped decode that gave up (should stay 0).
__device__ unsigned long long g_wait_timeouts;

constexpr int kStageTags = 8;  // tagged shortlist loads per thread in flight (workgroup pass, overlapped decode)

// Overlapped decode: waits until the row pass has counted every row of
// example b's step t: one at step 0, else one per beam of the example (the
// row pass reads, and counts, exactly those rows). The count is a relaxed
// hint of when to start reading: each word read afterwards is checked by its
// own tag (wait_tagged). Every wait is bounded (p.wait_ticks of the 100 MHz
// real-time counter; a whole row pass takes milliseconds): the row pass
// never waits on the select pass, so the bound only keeps a fault elsewhere
// from hanging the workgroup. One thread; false when the wait gave up.
__device__ __forceinline__ bool wait_step_rows(const DecodeParams& p, int b, int t) {
    const int need = (t == 0 ? 1 : beams_of(p, b)) + p.wait_extra;
    const int32_t* cnt = p.step_done + static_cast<int64_t>(b) * p.T + t;
    if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need) return true;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
        __builtin_amdgcn_s_sleep(4);
        if (__builtin_amdgcn_s_memrealtime() - t0 > p.wait_ticks) {
            atomicAdd(&g_wait_timeouts, 1ull);
            return false;
        }
    }
    return true;
}

// Split launch of the overlapped decode: whether this launch decodes example
// b. The early launch waits for the example's first row at most
// p.early_ticks and then claims it; the late launch takes what the early one
// left. One thread.
__device__ __forceinline__ bool claim_example(const DecodeParams& p, int b) {
    if (!p.early) return __hip_atomic_load(p.claimed + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
    const int need = 1 + p.wait_extra;
    const int32_t* cnt = p.step_done + static_cast<int64_t>(b) * p.T;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
        __builtin_amdgcn_s_sleep(4);
        if (__builtin_amdgcn_s_memrealtime() - t0 > p.early_ticks) return false;
    }
    __hip_atomic_store(p.claimed + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Overlapped decode: one tagged word of the row pass (RowInfo half or
// shortlist entry), waited for while its tag is 0; false when the wait gave
// up (bounded like wait_step_rows).
__device__ __forceinline__ bool wait_tagged(const DecodeParams& p, const uint32_t* src, uint32_t& lo, uint32_t& hi) {
    if (read_tagged(src, lo, hi)) return true;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (!read_tagged(src, lo, hi)) {
        __builtin_amdgcn_s_sleep(2);
        if (__builtin_amdgcn_s_memrealtime() - t0 > p.wait_ticks) {
            atomicAdd(&g_wait_timeouts, 1ull);
            return false;
        }
    }
    return true;
}

constexpr int kRescanBuf = 512;   // candidates of one rescanned row kept before falling back
constexpr int kRescanPerThread = 16;
constexpr int kTauHead = 2;       // entries per row behind the second tau bound
constexpr int kWideBeam = 16;     // beams from which the wide-beam paths pay off
constexpr int kPfRegs = 12;       // 16-byte prefetch registers per thread (K * M <= 6144)
constexpr int kSigWordsMax = 256;  // words of a beam's prefix signature (8192 bits; 2048 when LDS is short)
constexpr int kScoreFilterMaxK = 32;  // beams up to which a rank compaction first ranks by score alone

struct Lds {
    Cand* buf;        // [sort_cap] the collector
    Cand* rbuf;       // [kRescanBuf] one rescanned row's candidates
    uint4* key;       // [2 * kRankMax] candidate keys of a rank compaction (kRankMax used)
    int32_t* part;    // [kSelectThreads] partial ranks (or score keys)
    int32_t* surv;    // [64] candidates left by the score pass of a rank compaction
    int32_t* nsurv;   // [1] how many
    float* raw;       // [K] beams after the previous step
    float* nraw;      // [K] beams after this step (also scratch)
    float* rbound;    // [K]
    float* pen;       // [pen_len] length penalty by length
    float* inv;       // [pen_len] 1 / penalty
    int32_t* len;
    int32_t* nlen;
    int32_t* last;
    int32_t* nlast;
    int32_t* ended;
    int32_t* nended;
    int32_t* rcount;  // [K] shortlist entries of the beam's row (-2 not read, -1 no shortlist, -3 failed check)
    int32_t* plen;    // [2K] prefix lengths
    int32_t* nblk;    // [K] n-gram-blocked tokens of each beam
    ShortEntry* sl;   // [K, M + 1] the step's shortlists (see sl_at)
    int32_t* prefix;  // [2, K, P] (LDS) or the example's slice of the workspace
    int32_t* blk;     // [K, P] (LDS) or workspace
    uint32_t* sig;    // [2, K, sig_words] (LDS) prefix signatures, or null
    int sig_words;
    int V;            // vocabulary size (the keys' token field)
    int sig_shift;    // 32 - log2(32 sig_words): hash bits kept
};

// The select pass's barriers order LDS only (lds_barrier): a step's global
// loads (the next step's prefetch) and its trace stores stay in flight across
// them. The beams' prefixes and n-gram-blocked lists live in global memory
// when LDS cannot hold them (long constrained decodes); the barriers after
// they are written then also wait for global memory.
__device__ __forceinline__ void step_barrier(bool lists_global) {
    if (lists_global) __syncthreads();
    else lds_barrier();
}

struct State {
    int gave_up;  // a wait of the overlapped decode gave up
    int first_bad;  // the first invalid row read (t * K + k), else INT_MAX
    int count;
    int any_fail;
    int rcount;
    int overflow;
    uint32_t invalid;
    float tau;
    Cand thr;
};

// Entry i of beam k's shortlist in LDS. Wide beams pad the rows to M + 1
// entries, so the lanes of a wavefront reading entry i of consecutive beams
// spread over the banks.
__device__ __forceinline__ int sl_stride(int K, int M) { return K >= kWideBeam ? M + 1 : M; }
__device__ __forceinline__ int sl_at(int k, int i, int S) { return k * S + i; }

__device__ __forceinline__ float pen_of(const Lds& s, int pen_len, int l, float alpha) {
    const int c = l > 1 ? l : 1;
    return c < pen_len ? s.pen[c] : length_penalty(c, alpha);
}

__device__ __forceinline__ float inv_of(const Lds& s, int pen_len, int l, float alpha) {
    const int c = l > 1 ? l : 1;
    return c < pen_len ? s.inv[c] : 1.0f / length_penalty(c, alpha);
}

struct PrefixView {
    const int32_t* tok;
    int len;
    const uint32_t* sig;  // two bits set for every token of tok[0, len) (a superset filter), or null
    int sig_shift;
};

// The two signature bits of token v: multiplicative hashes to 32 - shift bits.
__device__ __forceinline__ uint32_t sig_bit0(int v, int shift) { return (static_cast<uint32_t>(v) * 0x9E3779B1u) >> shift; }
__device__ __forceinline__ uint32_t sig_bit1(int v, int shift) { return (static_cast<uint32_t>(v) * 0x85EBCA77u + 0x165667B1u) >> shift; }

__device__ __forceinline__ PrefixView prefix_of(const DecodeParams& p, const Lds& s, int b, int k, int cur) {
    if (p.step_mode) {
        const int l = s.len[k];
        const int L = l < 0 ? 0 : (l < p.st_stride ? l : p.st_stride);
        return PrefixView{p.st_prefix + (static_cast<int64_t>(b) * p.K + k) * p.st_stride, L, nullptr, 0};
    }
    return PrefixView{s.prefix + (static_cast<int64_t>(cur) * p.K + k) * p.prefix_cap, s.plen[cur * p.K + k],
                      s.sig ? s.sig + (cur * p.K + k) * s.sig_words : nullptr, s.sig_shift};
}

// Membership of v in a[0, n): eight independent loads in flight per round
// (the list is in LDS or global memory; its latency, not its length, bounds
// the scan).
__device__ __forceinline__ bool in_list(const int32_t* a, int n, int v) {
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        int32_t t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = a[i + u];
        bool hit = false;
#pragma unroll
        for (int u = 0; u < 8; ++u) hit = hit | (t[u] == v);
        if (hit) return true;
    }
    bool hit = false;
    for (; i < n; ++i) hit = hit | (a[i] == v);
    return hit;
}

// Membership of v in a prefix: the signature rules most tokens out with one
// read; the rest are searched.
__device__ __forceinline__ bool in_prefix(const PrefixView& pre, int v) {
    if (pre.sig) {
        const uint32_t h0 = sig_bit0(v, pre.sig_shift), h1 = sig_bit1(v, pre.sig_shift);
        if ((((pre.sig[h0 >> 5] >> (h0 & 31u)) & (pre.sig[h1 >> 5] >> (h1 & 31u))) & 1u) == 0u) return false;
    }
    return in_list(pre.tok, pre.len, v);
}

// The candidate of token v (finite log-prob lp, statically allowed) in the
// row of beam k; false when n-gram blocking removes it. A token of the prefix
// pays the repetition penalty: raw = p + (lp - log(rep)) (reference
// src/decoder.cpp:196-258).
__device__ __forceinline__ bool make_cand(const DecodeParams& p, const Lds& s, const PrefixView& pre, int k,
                                          float praw, float inv_pen, int v, int new_len, float lp, Cand& c) {
    float value = lp;
    if (p.constrained) {
        if (p.ngram == 1) {
            if (in_prefix(pre, v)) return false;
        } else if (p.ngram > 1 && in_list(s.blk + static_cast<int64_t>(k) * p.prefix_cap, s.nblk[k], v)) {
            return false;
        }
        if (p.penalise && in_prefix(pre, v)) value = lp - p.log_rep;
    }
    const float raw = praw + value;
    c = Cand{raw * inv_pen, raw, k, v, new_len, 1};
    return true;
}

__device__ __forceinline__ void sort_cands(Cand* buf, int np) {
    const int tid = static_cast<int>(threadIdx.x);
    for (int kk = 2; kk <= np; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < np; i += kSelectThreads) {
                const int partner = i ^ j;
                if (partner > i) {
                    const bool desc = (i & kk) == 0;
                    const Cand a = buf[i], c = buf[partner];
                    if (desc ? before(c, a) : before(a, c)) {
                        buf[i] = c;
                        buf[partner] = a;
                    }
                }
            }
            lds_barrier();
        }
    }
}

// Collector sizes up to this are compacted by a parallel rank (larger ones by
// the bitonic sort).
constexpr int kRankMax = kSelectThreads;

// The candidate at collector index idx as a 96-bit integer that is larger
// exactly when the candidate comes earlier in the total order, least
// significant word first: (parent, token) as parent * V + token (asc), raw,
// score (desc; no NaN reaches the collector). No two candidates of a
// collector share (parent, token) (a carried beam is not expanded, a rescan
// first drops its row's shortlisted candidates), so length and from_logprob
// never decide; K * V < 2^31 (the argument checks). Dead sentinels (parent
// -1) rank below every other candidate by score and raw (a candidate is
// admitted only if it ranks before the sentinel) and among themselves by
// index, lower first.
__device__ __forceinline__ uint4 cand_key(const Cand& c, int idx, int V) {
    const uint32_t low = c.parent >= 0 ? static_cast<uint32_t>(c.parent) * static_cast<uint32_t>(V) +
                                             static_cast<uint32_t>(c.token)
                                       : static_cast<uint32_t>(idx);
    return make_uint4(0xffffffffu - low, ordered_key(c.raw), ordered_key(c.score), 0u);
}

// rank += (96-bit key j > key i): the borrow out of i - j, kept in VCC
// through the subtraction.
__device__ __forceinline__ void count_above96(int& rank, uint32_t i0, uint32_t i1, uint32_t i2, uint32_t j0,
                                              uint32_t j1, uint32_t j2) {
    uint32_t t;
    asm("v_sub_co_u32 %0, vcc, %2, %5\n\t"
        "v_subb_co_u32 %0, vcc, %3, %6, vcc\n\t"
        "v_subb_co_u32 %0, vcc, %4, %7, vcc\n\t"
        "v_addc_co_u32 %1, vcc, 0, %1, vcc"
        : "=&v"(t), "+v"(rank)
        : "v"(i0), "v"(i1), "v"(i2), "v"(j0), "v"(j1), "v"(j2)
        : "vcc");
}
__device__ __forceinline__ void count_before(int& rank, const uint4& i, const uint4& j) {
    count_above96(rank, i.x, i.y, i.z, j.x, j.y, j.z);
}

// rank += (64-bit key (hi, lo) j > key i): the borrow out of i - j.
__device__ __forceinline__ void count_above64(int& rank, uint32_t ilo, uint32_t ihi, uint32_t jlo, uint32_t jhi) {
    uint32_t t;
    asm("v_sub_co_u32 %0, vcc, %2, %4\n\t"
        "v_subb_co_u32 %0, vcc, %3, %5, vcc\n\t"
        "v_addc_co_u32 %1, vcc, 0, %1, vcc"
        : "=&v"(t), "+v"(rank)
        : "v"(ilo), "v"(ihi), "v"(jlo), "v"(jhi)
        : "vcc");
}

// Keeps the best K of n <= kRankMax collected candidates, in order: every
// candidate's rank is the number of keys above its own, counted by up to four
// waves per candidate over disjoint ranges of the others, and the candidates
// of rank < K move to their rank.
// Past one wavefront of candidates (few beams), a pass over the scores alone
// (the keys' most significant word) comes first: a candidate with K or more
// scores strictly above its own ranks K or later. Every candidate ranked
// before a remaining one has a score at least as high and so remains too:
// the remaining candidates' ranks among themselves are their ranks among all,
// and when at most 64 remain one wavefront ranks them.
__device__ __forceinline__ void compact_by_rank(Lds& s, State& st, int K, int n) {
    const int tid = static_cast<int>(threadIdx.x);
    const int n4 = (n + 3) & ~3;
    const bool by_score = n > 64 && K <= kScoreFilterMaxK;
    Cand c = dead_cand();
    if (tid < n4) {
        if (tid < n) {
            c = s.buf[tid];
            s.key[tid] = cand_key(c, tid, s.V);
        } else {
            s.key[tid] = make_uint4(0u, 0u, 0u, 0u);  // below every key
        }
        if (by_score) s.part[tid] = static_cast<int32_t>(tid < n ? ordered_key(c.score) : 0u);
    }
    if (by_score && tid == 0) s.nsurv[0] = 0;
    lds_barrier();
    if (by_score) {
        if (tid < n) {
            const uint32_t mine = ordered_key(c.score);
            const uint4* sk = reinterpret_cast<const uint4*>(s.part);
            int above = 0;
            int j = 0;
            for (; j + 4 <= n4 / 4; j += 4) {  // four reads in flight
                uint4 w[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) w[u] = sk[j + u];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    above += (w[u].x > mine) + (w[u].y > mine) + (w[u].z > mine) + (w[u].w > mine);
            }
            for (; j < n4 / 4; ++j) {
                const uint4 w = sk[j];
                above += (w.x > mine) + (w.y > mine) + (w.z > mine) + (w.w > mine);
            }
            if (above < K) {
                const int slot = atomicAdd(s.nsurv, 1);
                if (slot < 64) s.surv[slot] = tid;
            }
        }
        lds_barrier();
        const int ns = __builtin_amdgcn_readfirstlane(s.nsurv[0]);
        if (ns <= 64) {
            if (tid < ns) {
                const int i = s.surv[tid];
                const Cand ci = s.buf[i];
                const uint4 ki = s.key[i];
                int rank = 0;
                for (int j = 0; j < ns; ++j) count_before(rank, ki, s.key[s.surv[j]]);
                if (rank < K) s.buf[rank] = ci;
                if (rank == K - 1 && before(ci, st.thr)) st.thr = ci;
            }
            if (tid == 0) st.count = n < K ? n : K;
            lds_barrier();
            return;
        }
        // many equal scores: every candidate is ranked
    }
    // wave w counts for candidates 64 gi + lane over the gj-th part of the others
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int groups = (n + 63) >> 6;
    const int parts = groups == 1 ? 4 : (groups == 2 ? 2 : 1);
    const int gi = w / parts, gj = w - gi * parts;
    int part = 0;
    if (gi < groups) {
        const int i = 64 * gi + lane;
        const uint4 ki = s.key[i];
        const int span = ((n4 / parts) + 3) & ~3;
        const int j0 = gj * span;
        const int j1 = j0 + span < n4 ? j0 + span : n4;
        int j = j0;
        for (; j + 8 <= j1; j += 8) {  // eight keys in flight
            uint4 w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = s.key[j + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) count_before(part, ki, w[u]);
        }
        for (; j < j1; j += 4) {
            const uint4 a = s.key[j], b2 = s.key[j + 1], c2 = s.key[j + 2], d = s.key[j + 3];
            count_before(part, ki, a);
            count_before(part, ki, b2);
            count_before(part, ki, c2);
            count_before(part, ki, d);
        }
    }
    s.part[tid] = part;
    lds_barrier();
    if (tid < n) {
        const int gi_t = tid >> 6;
        int rank = 0;
        for (int g = 0; g < parts; ++g) rank += s.part[(gi_t * parts + g) * 64 + (tid & 63)];
        if (rank < K) s.buf[rank] = c;
        if (rank == K - 1 && before(c, st.thr)) st.thr = c;
    }
    if (tid == 0) st.count = n < K ? n : K;
    lds_barrier();
}

// Sorts the collected candidates, keeps the best K, and raises the admission
// threshold to the K-th kept one when that is better.
__device__ __forceinline__ void compact(Lds& s, State& st, int K) {
    lds_barrier();
    const int n = __builtin_amdgcn_readfirstlane(st.count);
    if (n <= kRankMax) {
        compact_by_rank(s, st, K, n);
        return;
    }
    int np = 1;
    while (np < n) np <<= 1;
    for (int i = n + static_cast<int>(threadIdx.x); i < np; i += kSelectThreads) s.buf[i] = dead_cand();
    lds_barrier();
    sort_cands(s.buf, np);
    if (threadIdx.x == 0) {
        st.count = n < K ? n : K;
        if (st.count == K && before(s.buf[K - 1], st.thr)) st.thr = s.buf[K - 1];
    }
    lds_barrier();
}

// Admits c unless it ranks after the threshold (a candidate offered earlier,
// or the dead sentinel). Equal admits: after a rescan removed the threshold's
// own row from the collector, the threshold itself must come back.
__device__ __forceinline__ void offer(Lds& s, State& st, const Cand& c) {
    if (before(st.thr, c)) return;
    const int slot = atomicAdd(&st.count, 1);
    s.buf[slot] = c;
}

__device__ __forceinline__ void end_round(Lds& s, State& st, int K, int sort_cap) {
    lds_barrier();
    if (st.count > sort_cap - kSelectThreads) compact(s, st, K);
}

// Every candidate of row `row` (beam k) that does not rank after the
// threshold: gathered into the rescan buffer in one sweep, then offered to the
// collector. A buffer overflow (a row with very many candidates at the
// threshold) falls back to offering round by round.
template <int DT, bool LOGITS>
__device__ __forceinline__ void rescan_row(const DecodeParams& p, Lds& s, State& st, int b, int k, int64_t row, float lse,
                           float praw, float inv_pen, int new_len, const PrefixView& pre, int sort_cap, int keep) {
    const bool mask_eos = new_len < min_length_of(p, b);
    const int V = p.V;
    const int tid = static_cast<int>(threadIdx.x);
    const size_t esz = DT == 0 ? 4 : 2;
    const char* base = static_cast<const char*>(p.x) + static_cast<size_t>(row) * static_cast<size_t>(V) * esz;
    if (tid == 0) {
        st.rcount = 0;
        st.overflow = 0;
    }
    lds_barrier();
    const Cand thr = st.thr;
    for (int v0 = 0; v0 < V; v0 += kSelectThreads * kRescanPerThread) {
        float xs[kRescanPerThread];
#pragma unroll
        for (int j = 0; j < kRescanPerThread; ++j) {
            const int v = v0 + j * kSelectThreads + tid;
            xs[j] = v < V ? load_one<DT>(base, v) : -kInf;
        }
#pragma unroll
        for (int j = 0; j < kRescanPerThread; ++j) {
            const int v = v0 + j * kSelectThreads + tid;
            const float lp = LOGITS ? xs[j] - lse : xs[j];
            if (v >= V || !(lp < kInf) || lp == -kInf) continue;
            const float raw0 = praw + lp;
            const Cand c0{raw0 * inv_pen, raw0, k, v, new_len, 1};
            if (before(thr, c0)) continue;  // penalties only lower a candidate
            if (static_masked(p, b, v, mask_eos)) continue;
            if (p.row_mask && gload(p.row_mask, row * V + v)) continue;
            Cand c;
            if (!make_cand(p, s, pre, k, praw, inv_pen, v, new_len, lp, c)) continue;
            if (before(thr, c)) continue;
            const int slot = atomicAdd(&st.rcount, 1);
            if (slot < kRescanBuf) s.rbuf[slot] = c;
            else st.overflow = 1;
        }
    }
    lds_barrier();
    if (!st.overflow) {
        const int n = st.rcount;
        for (int r0 = 0; r0 < n; r0 += kSelectThreads) {
            if (r0 + tid < n) offer(s, st, s.rbuf[r0 + tid]);
            end_round(s, st, keep, sort_cap);
        }
        return;
    }
    // very many candidates at the threshold: offer the row round by round
    for (int v0 = 0; v0 < V; v0 += kSelectThreads) {
        const int v = v0 + tid;
        if (v < V) {
            const float x = load_one<DT>(base, v);
            const float lp = LOGITS ? x - lse : x;
            if ((lp < kInf) && lp != -kInf && !static_masked(p, b, v, mask_eos) &&
                !(p.row_mask && gload(p.row_mask, row * V + v))) {
                Cand c;
                if (make_cand(p, s, pre, k, praw, inv_pen, v, new_len, lp, c)) offer(s, st, c);
            }
        }
        end_round(s, st, keep, sort_cap);
    }
}

// PF: the next step's RowInfo and shortlists are prefetched into registers
// (chosen on the host: prefetch_fits); a separate instantiation, so the other
// paths keep their register budget.
// HOLD: the kernel claims every accumulation register (a clobber of a255),
// so no wavefront of another kernel fits on its SIMDs beside it: launched
// before a row pass of one workgroup per row, it keeps its CUs to itself
// (registers it never uses; its own occupancy, one wavefront per SIMD, is
// unchanged).
template <int DT, bool LOGITS, bool PF, bool HOLD = false>
__global__ __launch_bounds__(kSelectThreads) void select_kernel(DecodeParams p, SelectLayout L) {
    if constexpr (HOLD) asm volatile("" ::: "a255");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ State st;
    if (p.claimed) {
        __shared__ int s_claim;
        if (threadIdx.x == 0) s_claim = claim_example(p, static_cast<int>(blockIdx.x)) ? 1 : 0;
        __syncthreads();
        if (s_claim == 0) return;
    }
    const int K = p.K, T = p.T, M = p.M;
    const int SL = sl_stride(K, M);
    const int b = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);

    Lds s;
    s.buf = reinterpret_cast<Cand*>(smem + L.off_buf);
    s.rbuf = reinterpret_cast<Cand*>(smem + L.off_rbuf);
    s.key = reinterpret_cast<uint4*>(smem + L.off_key);
    s.part = reinterpret_cast<int32_t*>(smem + L.off_key + sizeof(uint4) * 2 * kRankMax);
    s.surv = s.part + kSelectThreads;
    s.nsurv = s.surv + 64;
    float* f = reinterpret_cast<float*>(smem + L.off_f32);
    s.raw = f;
    s.nraw = f + K;
    s.rbound = f + 2 * K;
    s.pen = f + 3 * K;
    s.inv = f + 3 * K + L.pen_len;
    int32_t* q = reinterpret_cast<int32_t*>(smem + L.off_i32);
    s.len = q;
    s.nlen = q + K;
    s.last = q + 2 * K;
    s.nlast = q + 3 * K;
    s.ended = q + 4 * K;
    s.nended = q + 5 * K;
    s.rcount = q + 6 * K;
    s.plen = q + 7 * K;
    s.nblk = q + 9 * K;
    s.sl = reinterpret_cast<ShortEntry*>(smem + L.off_sl);
    s.prefix = L.prefix_in_lds ? reinterpret_cast<int32_t*>(smem + L.off_prefix)
                               : p.prefix + static_cast<int64_t>(b) * 2 * K * p.prefix_cap;
    s.blk = L.blk_in_lds ? reinterpret_cast<int32_t*>(smem + L.off_blk)
                         : p.blocked + static_cast<int64_t>(b) * K * p.prefix_cap;
    s.sig = L.sig_in_lds && !p.step_mode ? reinterpret_cast<uint32_t*>(smem + L.off_sig) : nullptr;
    s.sig_words = L.sig_words;
    s.V = p.V;
    s.sig_shift = L.sig_words == kSigWordsMax ? 19 : 21;
    const bool lists_global = p.constrained && (!L.prefix_in_lds || !L.blk_in_lds);

    const int steps_b = p.step_mode ? 1 : example_steps(p, b);
    // this example's beams (slots past them stay empty) and EOS token
    const int Kb = beams_of(p, b), eos_b = eos_of(p, b);
    const int T_loop = p.step_mode ? 1 : T;
    const int pen_len = L.pen_len;
    // candidates the collector keeps (the beams, or the relaxed pool), and
    // how many of them are the example's
    const int KP = p.pool_mult > 0 ? K * p.pool_mult : K;
    const int Nb = p.pool_mult > 0 ? Kb * p.pool_mult : Kb;
    for (int l = tid; l < pen_len; l += kSelectThreads) {
        const float pl = length_penalty(l, p.alpha);
        s.pen[l] = pl;
        s.inv[l] = 1.0f / pl;
    }
    // Initial state (reference src/decoder.cpp:46-56) or the caller's (:84-103).
    for (int k = tid; k < K; k += kSelectThreads) {
        if (p.step_mode) {
            const int64_t i = static_cast<int64_t>(b) * K + k;
            s.raw[k] = k < Kb ? p.st_raw[i] : -kInf;
            s.len[k] = p.st_len[i];
            s.ended[k] = p.st_fin[i] != 0;
            const int l = p.st_len[i];
            s.last[k] = (p.st_prefix && l >= 1 && l <= p.st_stride) ? p.st_prefix[i * p.st_stride + (l - 1)] : -1;
        } else {
            s.raw[k] = k == 0 ? 0.0f : -kInf;
            s.len[k] = 0;
            s.ended[k] = 0;
            s.last[k] = -1;
        }
        s.plen[k] = 0;
        s.plen[K + k] = 0;
    }
    if (s.sig)
        for (int i = tid; i < 2 * K * s.sig_words; i += kSelectThreads) s.sig[i] = 0u;
    if (tid == 0) {
        st.invalid = 0;
        st.gave_up = 0;
        st.first_bad = 0x7fffffff;
    }
    lds_barrier();

    // Prefetch (the row pass has finished before this kernel: not the
    // overlapped decode): the next step's RowInfo and shortlists sit at fixed
    // addresses (rows (b, t + 1, k) of every slot), so their loads are issued
    // into registers as soon as a step's own are staged, and land while the
    // step runs.
    constexpr int kPf = PF ? kPfRegs : 1;
    uint4 pf_sl[kPf];
    uint4 pf_info = make_uint4(0u, 0u, 0u, 0u);
    bool have_pf = false;
    auto prefetch = [&](int t_next) {
        const int64_t base = (static_cast<int64_t>(b) * T + t_next) * K;
        if (tid < K) pf_info = reinterpret_cast<const uint4*>(p.rowinfo)[base + tid];
        const uint4* src4 = reinterpret_cast<const uint4*>(p.shortlist + base * M);
        const int n4 = K * M / 2;
#pragma unroll
        for (int u = 0; u < kPf; ++u)
            if (tid + u * kSelectThreads < n4) pf_sl[u] = src4[tid + u * kSelectThreads];
    };

    // Pool entry i of the step starting at pool0 (reference src/decoder.cpp:294-306).
    auto put_pool = [&](int64_t i, const Cand& c) {
        if (p.pool_parents) p.pool_parents[i] = c.parent;
        if (p.pool_tokens) p.pool_tokens[i] = c.token;
        if (p.pool_lengths) p.pool_lengths[i] = c.length;
        if (p.pool_scores) p.pool_scores[i] = c.score;
        if (p.pool_raw) p.pool_raw[i] = c.raw;
        if (p.pool_flp) p.pool_flp[i] = static_cast<uint8_t>(c.flp);
    };
    // A padding step (reference src/c_api.cpp:764-781): no token, no parent.
    auto pad_step = [&](int64_t trace0) {
        for (int k = tid; k < K; k += kSelectThreads) {
            if (p.tokens) p.tokens[trace0 + k] = -1;
            if (p.parents) p.parents[trace0 + k] = -1;
            if (p.lengths) p.lengths[trace0 + k] = 0;
            if (p.scores) p.scores[trace0 + k] = -kInf;
            if (p.raw_scores) p.raw_scores[trace0 + k] = -kInf;
            if (p.from_logprob) p.from_logprob[trace0 + k] = 0;
        }
        if (p.pool_mult > 0) {
            const int64_t pool0 = trace0 / K * KP;
            for (int q = tid; q < KP; q += kSelectThreads) put_pool(pool0 + q, dead_cand());
        }
    };

    int cur = 0;
    for (int t = 0; t < T_loop; ++t) {
        const int64_t trace0 = (static_cast<int64_t>(b) * T + t) * K;  // step mode: T == 1
        if (t >= steps_b) {
            pad_step(trace0);
            continue;
        }
        if (tid == 0) {
            st.count = 0;
            st.any_fail = 0;
            st.tau = -kInf;
            st.thr = dead_cand();
        }
        if (p.step_done) {
            // The row pass runs alongside: wait for this step's rows. After a
            // wait gives up, nothing more of the workspace is read: the
            // example's remaining steps are padding and it is reported
            // invalid.
            if (tid == 0 && !st.gave_up && !wait_step_rows(p, b, t)) st.gave_up = 1;
            lds_barrier();
            if (st.gave_up) {
                pad_step(trace0);
                continue;
            }
        }
        const bool coherent = p.step_done != nullptr;
        // Stage the step: row statistics of the rows read, the shortlists,
        // and the n-gram-blocked tokens of each beam.
        for (int k = tid; k < K; k += kSelectThreads) {
            const float praw = s.raw[k];
            const bool live = praw < kInf && praw > -kInf;
            const bool carried = live && eos_b >= 0 && s.ended[k];
            int cnt = -2;
            float bound = -kInf;
            if (live && !carried) {
                RowInfo info;
                if (have_pf) {
                    __builtin_memcpy(&info, &pf_info, sizeof(info));  // k == tid
                } else if (!coherent) {
                    info = p.rowinfo[trace0 + k];
                } else {
                    // the two tagged words (count + 2, invalid + 1), both
                    // loads issued before either is waited for
                    const uint32_t* src = reinterpret_cast<const uint32_t*>(p.rowinfo + trace0 + k);
                    uint32_t lo0 = 0, hi0 = 2, lo1 = 0, hi1 = 1;
                    (void)read_tagged(src, lo0, hi0);
                    (void)read_tagged(src + 2, lo1, hi1);
                    if ((hi0 == 0u && !wait_tagged(p, src, lo0, hi0)) || (hi1 == 0u && !wait_tagged(p, src + 2, lo1, hi1))) {
                        atomicOr(&st.gave_up, 1);
                        lo0 = lo1 = 0;
                        hi0 = 2;
                        hi1 = 1;
                    }
                    info.lse = bits_f32(lo0);
                    info.count = static_cast<int32_t>(hi0) - 2;
                    info.bound = bits_f32(lo1);
                    info.invalid = hi1 - 1u;
                }
                if (info.invalid) {
                    atomicOr(&st.invalid, 1u);
                    atomicMin(&st.first_bad, t * K + k);  // steps in order, beams in order within one
                }
                if (p.row_lse && LOGITS) p.row_lse[trace0 + k] = info.lse;
                cnt = M > 0 ? info.count : -1;
                bound = info.bound;
                s.nraw[k] = info.lse;  // the row's logsumexp, kept for a rescan
            }
            s.rcount[k] = cnt;
            s.rbound[k] = bound;
            if (p.constrained && p.ngram > 1) s.nblk[k] = 0;
        }
        if (coherent) {
            // a shortlist is read only as far as its row's count
            lds_barrier();
            if (st.gave_up) {
                pad_step(trace0);
                continue;
            }
        }
        if (have_pf) {
            const int n4 = K * M / 2;
#pragma unroll
            for (int u = 0; u < kPf; ++u) {
                const int q = tid + u * kSelectThreads;
                if (q < n4) {
                    const int k = (2 * q) / M, i = 2 * q - k * M;
                    uint2* dst = reinterpret_cast<uint2*>(s.sl + sl_at(k, i, SL));
                    dst[0] = make_uint2(pf_sl[u].x, pf_sl[u].y);
                    dst[1] = make_uint2(pf_sl[u].z, pf_sl[u].w);
                }
            }
        } else if (M > 0) {
            const ShortEntry* src = p.shortlist + trace0 * M;
            if (!coherent && (M & 1) == 0 && K * M >= kWideBeam * 16) {
                // 16-byte loads (two entries of one row: with M even the rows'
                // shortlists start 16-byte aligned), eight in flight per
                // thread
                const uint4* src4 = reinterpret_cast<const uint4*>(src);
                const int n4 = K * M / 2;
                for (int i0 = tid; i0 < n4; i0 += 8 * kSelectThreads) {
                    uint4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (i0 + u * kSelectThreads < n4) v[u] = src4[i0 + u * kSelectThreads];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int q = i0 + u * kSelectThreads;
                        if (q < n4) {
                            const int k = (2 * q) / M, i = 2 * q - k * M;
                            uint2* dst = reinterpret_cast<uint2*>(s.sl + sl_at(k, i, SL));
                            dst[0] = make_uint2(v[u].x, v[u].y);
                            dst[1] = make_uint2(v[u].z, v[u].w);
                        }
                    }
                }
            } else if (coherent) {
                // The entries the row pass wrote (tag token + 1): eight tagged
                // loads per thread issued together (every one made, from a
                // clamped index), then each entry not yet written waited for.
                const uint32_t* src32 = reinterpret_cast<const uint32_t*>(src);
                const int n = K * M;
                for (int i0 = tid; i0 < n; i0 += kStageTags * kSelectThreads) {
                    uint32_t lo[kStageTags], hi[kStageTags];
#pragma unroll
                    for (int u = 0; u < kStageTags; ++u) {
                        const int i = i0 + u * kSelectThreads;
                        (void)read_tagged(src32 + 2 * (i < n ? i : n - 1), lo[u], hi[u]);
                    }
#pragma unroll
                    for (int u = 0; u < kStageTags; ++u) {
                        const int i = i0 + u * kSelectThreads;
                        if (i >= n) continue;
                        const int k = i / M, j = i - k * M;
                        // a word not yet written is waited for only within its
                        // row's count (the rest are never written)
                        if (hi[u] == 0u) {
                            if (j >= s.rcount[k]) continue;
                            if (!wait_tagged(p, src32 + 2 * i, lo[u], hi[u])) {
                                atomicOr(&st.gave_up, 1);
                                hi[u] = 1;
                            }
                        }
                        ShortEntry e;
                        e.lp = bits_f32(lo[u]);
                        e.token = static_cast<int32_t>(hi[u]) - 1;
                        s.sl[SL == M ? i : sl_at(k, j, SL)] = e;
                    }
                }
            } else {
                for (int i = tid; i < K * M; i += kSelectThreads) s.sl[SL == M ? i : sl_at(i / M, i % M, SL)] = src[i];
            }
        }
        // this step's rows are staged: the next step's loads go out now
        if constexpr (PF) {
            have_pf = t + 1 < steps_b;
            if (have_pf) prefetch(t + 1);
        }
        lds_barrier();
        if (coherent && st.gave_up) {
            pad_step(trace0);
            continue;
        }
        if (p.constrained && p.ngram > 1) {
            // n-gram blocking (reference src/decoder.cpp:196-230): for each
            // read beam, the tokens that followed an earlier occurrence of its
            // last n - 1 tokens; one thread per (beam, prefix position), the
            // list in any order (it is only searched)
            // (a decode's prefixes hold at most t tokens at step t)
            const int n = p.ngram, P = p.prefix_cap, Pt = p.step_mode ? P : min(P, t);
            for (int item = tid; item < K * Pt; item += kSelectThreads) {
                const int k = item / Pt, i = item - k * Pt;
                if (s.rcount[k] == -2) continue;
                const PrefixView pre = prefix_of(p, s, b, k, cur);
                if (i + n > pre.len) continue;
                const int tail = pre.len - (n - 1);
                bool same = true;
                for (int j = 0; j < n - 1; ++j) same = same & (pre.tok[i + j] == pre.tok[tail + j]);
                if (same) {
                    const int slot = atomicAdd(&s.nblk[k], 1);
                    s.blk[static_cast<int64_t>(k) * P + slot] = pre.tok[i + n - 1];
                }
            }
            step_barrier(lists_global);
        }
        // a forced step (uniform over the workgroup): no shortlist is used
        const int forced = p.forced ? gload(p.forced, static_cast<int64_t>(b) * T + t) : -1;
        if (p.use_tau && forced < 0) {
            // Lower bounds of the K-th best expanded raw (unconstrained: raw =
            // fl(p + lp), monotone in lp; every beam expanded has the same
            // length, so this step's shortlisted candidates rank by raw).
            // (a) The first K entries of a shortlist are real candidates with
            // raw >= fl(p + lp_K): at least K reach the largest such value.
            if (tid < 64) {
                float best = -kInf;
                for (int k = tid; k < K; k += 64)
                    if (s.rcount[k] >= K) best = fmaxf(best, s.raw[k] + s.sl[sl_at(k, K - 1, SL)].lp);
                best = wave_max_dpp(best);
                if (tid == 0) st.tau = best;
            }
            // (b) Wide beams: the K-th largest raw among the first kTauHead
            // entries of every row: at least K real candidates reach it.
            // Ranked as 64-bit keys (ordered value bits, then the lower index
            // first), two per broadcast read.
            const int nv = K * kTauHead;  // <= 128 (K <= 64 with a shortlist), even
            uint2* vk = reinterpret_cast<uint2*>(s.key);
            float v = -kInf;
            if (K >= kWideBeam && tid < nv) {
                const int k = tid / kTauHead, i = tid - k * kTauHead;
                v = i < s.rcount[k] ? s.raw[k] + s.sl[sl_at(k, i, SL)].lp : -kInf;
                vk[tid] = make_uint2(0xffffffffu - static_cast<uint32_t>(tid), ordered_key(v));
            }
            if (K >= kWideBeam) lds_barrier();  // (a) and the keys are in
            if (K >= kWideBeam && tid < nv) {
                const uint32_t mlo = 0xffffffffu - static_cast<uint32_t>(tid), mhi = ordered_key(v);
                const uint4* w4 = reinterpret_cast<const uint4*>(vk);
                int rank = 0;
                int j2 = 0;
                for (; j2 + 4 <= nv / 2; j2 += 4) {  // four reads in flight
                    uint4 w[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) w[u] = w4[j2 + u];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        count_above64(rank, mlo, mhi, w[u].x, w[u].y);
                        count_above64(rank, mlo, mhi, w[u].z, w[u].w);
                    }
                }
                for (; j2 < nv / 2; ++j2) {
                    const uint4 w = w4[j2];
                    count_above64(rank, mlo, mhi, w.x, w.y);
                    count_above64(rank, mlo, mhi, w.z, w.w);
                }
                if (rank == K - 1 && v > st.tau) st.tau = v;
            }
            lds_barrier();
        }

        // Carried-forward beams (reference src/decoder.cpp:131-139).
        for (int k = tid; k < K; k += kSelectThreads) {
            const float praw = s.raw[k];
            const bool live = praw < kInf && praw > -kInf;
            if (live && eos_b >= 0 && s.ended[k]) {
                const int l = s.len[k] > 1 ? s.len[k] : 1;
                const int32_t last = s.last[k];
                const Cand c{praw / pen_of(s, pen_len, l, p.alpha), praw, k, is_eos_of(p, b, last) ? last : eos_b, l,
                             0};
                offer(s, st, c);
            }
        }
        if (forced >= 0) {
            // A forced step (reference src/decoder.cpp:125-167,
            // src/kernels_scalar.cpp:16-26): a read beam's one candidate is
            // the forced token, under every check another candidate meets (a
            // finite log-prob, banned tokens, the EOS mask below min_length,
            // n-gram blocking, the repetition penalty). At most K of them
            // join the carried beams: 2K <= sort_cap. (The host refuses forced
            // tokens outside the vocabulary; the bound keeps the read in the
            // row regardless.)
            for (int k = tid; k < K; k += kSelectThreads) {
                if (s.rcount[k] == -2 || forced >= p.V) continue;
                const int64_t row = p.step_mode ? static_cast<int64_t>(b) * K + k : trace0 + k;
                const float x = load_one<DT>(static_cast<const char*>(p.x) +
                                                 static_cast<size_t>(row) * static_cast<size_t>(p.V) * (DT == 0 ? 4 : 2),
                                             forced);
                const float lp = LOGITS ? x - s.nraw[k] : x;
                const int new_len = s.len[k] + 1;
                if (!(lp < kInf) || lp == -kInf || static_masked(p, b, forced, new_len < min_length_of(p, b))) continue;
                if (p.row_mask && gload(p.row_mask, row * p.V + forced)) continue;
                Cand c;
                if (make_cand(p, s, prefix_of(p, s, b, k, cur), k, s.raw[k], inv_of(s, pen_len, new_len, p.alpha),
                              forced, new_len, lp, c))
                    offer(s, st, c);
            }
        }
        // (at most K offers: the first round of shortlisted offers joins them
        // unless the one-pass path below needs the count)
        if (M > 0 && p.use_tau && K >= kWideBeam && forced < 0) end_round(s, st, KP, L.sort_cap);

        // Shortlisted candidates. Unconstrained wide beams: few reach tau, and
        // when they fit the collector beside what it holds, they are offered
        // in one pass without compaction rounds.
        // A shortlist is sorted (log-prob desc), so the entries reaching tau
        // are a prefix of it: one thread per beam measures its prefix, then
        // offers it.
        bool one_pass = false;
        if (M > 0 && p.use_tau && K >= kWideBeam && forced < 0) {
            // (K <= 64 with a shortlist: lane k of wavefront 0 measures beam
            // k's prefix, eight entries a round; a lane scan places the
            // prefixes at consecutive collector slots, and the four
            // wavefronts copy them, lane k for beam k)
            if (tid < 64) {
                const float tau = st.tau;
                const int k = tid;
                int n = 0;
                if (k < K) {
                    const float praw = s.raw[k];
                    const int cnt = s.rcount[k];
                    for (;;) {
                        int reach = 0;
#pragma unroll
                        for (int u = 0; u < 8; ++u)
                            reach += (n + u < cnt && !(praw + s.sl[sl_at(k, n + u, SL)].lp < tau)) ? 1 : 0;
                        n += reach;
                        if (reach < 8) break;
                    }
                }
                const int incl = wave_inclusive_sum(n);
                const int total = __builtin_amdgcn_readlane(incl, 63);
                const int base = st.count;
                s.part[k] = base + incl - n;  // beam k's first collector slot
                s.part[64 + k] = n;
                if (tid == 0) st.rcount = base + total <= L.sort_cap ? base + total : -1;
            }
            lds_barrier();
            one_pass = st.rcount >= 0;
            if (one_pass) {
                const int k = tid & 63, w = tid >> 6;
                const int n = k < K ? s.part[64 + k] : 0;
                if (n > w) {
                    const int slot0 = s.part[k];
                    const float praw = s.raw[k];
                    const int new_len = s.len[k] + 1;
                    const float inv = inv_of(s, pen_len, new_len, p.alpha);
                    for (int i = w; i < n; i += 4) {
                        const ShortEntry e = s.sl[sl_at(k, i, SL)];
                        const float raw = praw + e.lp;
                        s.buf[slot0 + i] = Cand{raw * inv, raw, k, e.token, new_len, 1};
                    }
                }
                if (tid == 0) st.count = st.rcount;
            }
        }
        if (M > 0 && !one_pass && forced < 0) {
            const float tau = st.tau;
            for (int base = 0; base < K * M; base += kSelectThreads) {
                const int item = base + tid;
                if (item < K * M) {
                    const int k = item / M;
                    const int i = item - k * M;
                    if (i < s.rcount[k]) {
                        const ShortEntry e = s.sl[sl_at(k, i, SL)];
                        const float praw = s.raw[k];
                        if (!(praw + e.lp < tau)) {
                            const int new_len = s.len[k] + 1;
                            const PrefixView pre = prefix_of(p, s, b, k, cur);
                            Cand c;
                            if (make_cand(p, s, pre, k, praw, inv_of(s, pen_len, new_len, p.alpha), e.token, new_len,
                                          e.lp, c))
                                offer(s, st, c);
                        }
                    }
                }
                end_round(s, st, KP, L.sort_cap);
            }
        }
        compact(s, st, KP);

        // Exactness: every candidate left out of a row's shortlist has raw <=
        // fl(p + bound); a row passes when the K-th selected candidate ranks
        // strictly before that bound's score and raw.
        for (int k = tid; k < K; k += kSelectThreads) {
            const int cnt = s.rcount[k];
            if (cnt == -2 || forced >= 0) continue;  // a forced step read its rows whole
            bool fail = cnt < 0;
            if (!fail && s.rbound[k] > -kInf) {
                const float X = s.raw[k] + s.rbound[k];
                if (X > -kInf) {
                    const float SX = X * inv_of(s, pen_len, s.len[k] + 1, p.alpha);
                    const Cand kth = st.count >= Nb ? s.buf[Nb - 1] : dead_cand();
                    fail = !((kth.score > SX) || (kth.score == SX && kth.raw > X));
                }
            }
            if (fail) {
                s.rcount[k] = -3;
                atomicOr(&st.any_fail, 1);
            }
        }
        lds_barrier();
        if (st.any_fail) {
            for (int k = 0; k < K; ++k) {
                if (s.rcount[k] != -3) continue;
                if (tid == 0) atomicAdd(&g_rescanned_rows, 1ull);
                // drop the row's shortlisted candidates, then offer the whole row
                for (int i = tid; i < st.count; i += kSelectThreads)
                    if (s.buf[i].parent == k && s.buf[i].flp) s.buf[i] = dead_cand();
                lds_barrier();
                const float praw = s.raw[k];
                const int new_len = s.len[k] + 1;
                const int64_t row = p.step_mode ? static_cast<int64_t>(b) * K + k : trace0 + k;
                const PrefixView pre = prefix_of(p, s, b, k, cur);
                rescan_row<DT, LOGITS>(p, s, st, b, k, row, LOGITS ? s.nraw[k] : 0.0f, praw,
                                       inv_of(s, pen_len, new_len, p.alpha), new_len, pre, L.sort_cap, KP);
            }
            compact(s, st, KP);
        }

        // Selection (reference src/decoder.cpp:314-350): the example's best Kb.
        const int nsel = st.count < Kb ? st.count : Kb;
        for (int k = tid; k < K; k += kSelectThreads) {
            const Cand c = k < nsel ? s.buf[k] : dead_cand();
            const int64_t o = trace0 + k;
            if (p.tokens) p.tokens[o] = c.token;
            if (p.parents) p.parents[o] = c.parent;
            if (p.lengths) p.lengths[o] = c.length;
            if (p.scores) p.scores[o] = c.score;
            if (p.raw_scores) p.raw_scores[o] = c.raw;
            if (p.from_logprob) p.from_logprob[o] = static_cast<uint8_t>(c.flp);
            s.nraw[k] = c.raw;
            s.nlen[k] = c.length;
            s.nlast[k] = c.token;
            s.nended[k] = c.parent >= 0 ? (s.ended[c.parent] || is_eos_of(p, b, c.token)) : 0;
            if (p.constrained && !p.step_mode) {
                const int nxt = cur ^ 1;
                s.plen[nxt * K + k] =
                    c.parent >= 0 ? s.plen[cur * K + c.parent] + ((c.flp && c.token >= 0) ? 1 : 0) : 0;
            }
        }
        if (p.pool_mult > 0) {
            // the pool: the example's best Nb, the selection first
            const int npool = st.count < Nb ? st.count : Nb;
            const int64_t pool0 = trace0 / K * KP;
            for (int q = tid; q < KP; q += kSelectThreads) put_pool(pool0 + q, q < npool ? s.buf[q] : dead_cand());
        }
        lds_barrier();
        if (p.constrained && !p.step_mode) {
            // each selected beam: its parent's prefix, then its token, and
            // the signature of both (one pass over every beam's positions)
            const int nxt = cur ^ 1;
            const int P = p.prefix_cap;
            const int Pc = min(P, t + 1);  // the new prefixes' length, at most
            const int W = s.sig ? s.sig_words : 0, W4 = W / 4;  // signatures copied 16 bytes an item
            const int PW = Pc > W4 ? Pc : W4;
            for (int item = tid; item < K * PW; item += kSelectThreads) {
                const int k = item / PW, i = item - k * PW;
                const Cand c = k < nsel ? s.buf[k] : dead_cand();
                if (i < W4) {
                    uint4 w = make_uint4(0u, 0u, 0u, 0u);
                    if (c.parent >= 0) {
                        w = reinterpret_cast<const uint4*>(s.sig + (cur * K + c.parent) * W)[i];
                        if (c.flp && c.token >= 0) {
                            auto set = [&](uint32_t h) {
                                if (static_cast<int>(h >> 7) != i) return;
                                const uint32_t m = 1u << (h & 31u);
                                switch ((h >> 5) & 3u) {
                                    case 0: w.x |= m; break;
                                    case 1: w.y |= m; break;
                                    case 2: w.z |= m; break;
                                    default: w.w |= m; break;
                                }
                            };
                            set(sig_bit0(c.token, s.sig_shift));
                            set(sig_bit1(c.token, s.sig_shift));
                        }
                    }
                    reinterpret_cast<uint4*>(s.sig + (nxt * K + k) * W)[i] = w;
                }
                if (i >= Pc || c.parent < 0) continue;
                const int Lp = s.plen[cur * K + c.parent];
                int32_t* dst = s.prefix + (static_cast<int64_t>(nxt) * K + k) * P;
                if (i < Lp) dst[i] = s.prefix[(static_cast<int64_t>(cur) * K + c.parent) * P + i];
                else if (i == Lp && c.flp && c.token >= 0) dst[Lp] = c.token;
            }
            cur = nxt;
        }
        for (int k = tid; k < K; k += kSelectThreads) {
            s.raw[k] = s.nraw[k];
            s.len[k] = s.nlen[k];
            s.last[k] = s.nlast[k];
            s.ended[k] = s.nended[k];
        }
        step_barrier(lists_global);
    }

    if (st.gave_up) {
        // no hypothesis survives an abandoned decode
        for (int k = tid; k < K; k += kSelectThreads) {
            s.raw[k] = -kInf;
            s.len[k] = 0;
        }
        if (tid == 0 && p.fault) __hip_atomic_store(p.fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_barrier();
    }
    // Final scores (reference src/decoder.cpp:179-187) and the state (step mode).
    for (int k = tid; k < K; k += kSelectThreads) {
        const int64_t i = static_cast<int64_t>(b) * K + k;
        if (p.final_scores) p.final_scores[i] = s.raw[k] / pen_of(s, pen_len, s.len[k], p.alpha);
        if (p.final_raw) p.final_raw[i] = s.raw[k];
        if (p.final_lengths) p.final_lengths[i] = s.len[k];
        if (p.step_mode) {
            p.st_raw[i] = s.raw[k];
            p.st_len[i] = s.len[k];
            p.st_fin[i] = static_cast<uint8_t>(s.ended[k] != 0);
        }
    }
    // 1: a row the search read holds NaN or +inf; 2: the decode of the
    // example did not complete (an overlapped wait gave up)
    if (tid == 0 && p.invalid) p.invalid[b] = static_cast<uint8_t>(st.gave_up ? 2 : (st.invalid != 0 ? 1 : 0));
    if (tid == 0 && p.first_invalid) p.first_invalid[b] = st.first_bad == 0x7fffffff ? -1 : st.first_bad;
}

// ---------------------------------------------------------------------------
// The narrow select pass: decodes with at most kNarrowMaxK beams and
// shortlists, not the step API and not n = 1 blocking, take one wavefront
// per example, up to kNarrowWaves examples per workgroup (a CU
// beside a persistent row pass takes one workgroup of the select pass at a
// time, so the overlapped decode leaves about B / kNarrowWaves CUs to it,
// the same number on each XCD). Lane k holds beam
// k's state in registers, and a step has no workgroup barrier and few LDS
// round trips:
//   * RowInfo of each read row (lane k) and the shortlists (LDS);
//   * tau, the largest fl(p_k + lp) over the K-th entries of the beams'
//     shortlists (as in the workgroup pass): at least K candidates reach it,
//     so none below it is selected;
//   * the survivors, each beam's entries that reach tau (a prefix of its
//     shortlist: fl(p_k + lp) is monotone in lp), and the carried-forward
//     beams. Up to 64 are ranked in the lanes (the count of candidates before
//     each one); more go through a running list of the best Kb in lanes
//     0 .. Kb - 1 (insertion in order, as keep_best);
//   * the workgroup pass's exactness check; when a row fails it, the
//     selection is redone through the running list from the passing rows'
//     survivors, the carried-forward beams and every token of the failing
//     rows (the candidate set only grows, so rows that passed still pass);
//   * the trace and the next state.
// With constraints (CON: n-gram blocking of n >= 2, a repetition penalty)
// each beam's prefix lives in LDS with a 32 W-bit signature (two hashed bits
// per token), both double-buffered and rebuilt from the parent's at every
// step; each step lists a read beam's n-gram-blocked tokens (one lane per
// prefix position), and every candidate takes make_cand's value (blocked:
// none; in the prefix: lp - log(rep)). Constraints only lower a value, so the
// row pass's bound still covers every token left out, and tau counts on K of
// a row's first K + nblk entries (a blocked token is one entry at most),
// each worth at least lp - log(rep).
// The kept set is the best Kb of the same candidates under the same total
// order as the workgroup pass, so the trace is the same bit for bit.
constexpr int kNarrowMaxK = 16;       // the running list lives in one 16-lane DPP row
constexpr int kNarrowPf = 4;          // 16-byte prefetch registers per lane (K * M <= 512)
constexpr int kNarrowPenCap = 1024;   // lengths with a penalty in LDS (larger ones are computed)
constexpr int kNarrowRescanUnroll = 16;
constexpr int kNarrowTagLoads = 4;    // tagged shortlist loads per lane in flight (overlapped decode)
constexpr int kNarrowWaves = 4;       // examples (wavefronts) per workgroup, at most: one workgroup per CU
constexpr int kXcds = 8;              // MI355X: 8 XCDs of 32 CUs
constexpr int kNarrowWaveLds = 24576; // LDS per wavefront, at most (else the workgroup pass)

// Lane j's candidate, wave-uniform.
__device__ __forceinline__ Cand lane_cand(const Cand& c, int j) {
    Cand r;
    r.score = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(c.score)), j)));
    r.raw = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(f32_bits(c.raw)), j)));
    r.parent = __builtin_amdgcn_readlane(c.parent, j);
    r.token = __builtin_amdgcn_readlane(c.token, j);
    r.length = __builtin_amdgcn_readlane(c.length, j);
    r.flp = __builtin_amdgcn_readlane(c.flp, j);
    return r;
}

// The value of lane - 1 (row_shr:1 within a 16-lane row; lane 0 keeps x).
__device__ __forceinline__ int from_lane_below(int x) { return __builtin_amdgcn_update_dpp(x, x, 0x111, 0xf, 0xf, false); }

// The running list: lanes [0, n) hold the best candidates so far, best first
// (dead past what it holds); thr is its last entry (wave-uniform). c
// (wave-uniform) goes in when it ranks before thr.
__device__ __forceinline__ void list_insert(Cand& top, Cand& thr, const Cand& c, int n, int lane) {
    if (!before(c, thr)) return;
    const bool above = lane < n && before(top, c);
    const int pos = __popcll(__builtin_amdgcn_ballot_w64(above));  // the list is sorted: a prefix stays
    Cand prev;
    prev.score = bits_f32(static_cast<uint32_t>(from_lane_below(static_cast<int>(f32_bits(top.score)))));
    prev.raw = bits_f32(static_cast<uint32_t>(from_lane_below(static_cast<int>(f32_bits(top.raw)))));
    prev.parent = from_lane_below(top.parent);
    prev.token = from_lane_below(top.token);
    prev.length = from_lane_below(top.length);
    prev.flp = from_lane_below(top.flp);
    if (lane == pos) top = c;
    else if (lane > pos) top = prev;
    thr = lane_cand(top, n - 1);
}

// Offers every lane's candidate where `offer` is set, in lane order.
__device__ __forceinline__ void list_offer(Cand& top, Cand& thr, const Cand& c, bool offer, int n, int lane) {
    uint64_t m = __builtin_amdgcn_ballot_w64(offer && before(c, thr));
    while (m != 0) {
        const int j = __ffsll(static_cast<long long>(m)) - 1;
        m &= m - 1;
        list_insert(top, thr, lane_cand(c, j), n, lane);
    }
}

// The overlapped decode's words of one step for one wavefront: the step's row
// count (lane 0; a hint of when to read), lane k's RowInfo words and the
// first 64 kNarrowTagLoads shortlist words. Every load is made, from a
// clamped address (a load under a branch is waited for inside it), and the
// caller drops what it does not need; a word not yet written has tag 0.
struct TagWords {
    int have;
    uint32_t ilo0, ihi0, ilo1, ihi1;
    uint32_t lo[kNarrowTagLoads], hi[kNarrowTagLoads];
};

__device__ __forceinline__ void issue_tagged(const DecodeParams& p, int b, int t, int lane, TagWords& w) {
    const int K = p.K, M = p.M;
    const int64_t tr0 = (static_cast<int64_t>(b) * p.T + t) * K;
    w.have = 0;
    if (lane == 0)
        w.have = __hip_atomic_load(p.step_done + static_cast<int64_t>(b) * p.T + t, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t* info32 = reinterpret_cast<const uint32_t*>(p.rowinfo + tr0 + (lane < K ? lane : 0));
    (void)read_tagged(info32, w.ilo0, w.ihi0);
    (void)read_tagged(info32 + 2, w.ilo1, w.ihi1);
    const uint32_t* sl32 = reinterpret_cast<const uint32_t*>(p.shortlist + tr0 * M);
#pragma unroll
    for (int u = 0; u < kNarrowTagLoads; ++u) {
        const int q = 64 * u + lane;
        (void)read_tagged(sl32 + 2 * (q < K * M ? q : K * M - 1), w.lo[u], w.hi[u]);
    }
}

// HOLD: as the workgroup pass's (every register of its SIMDs claimed, so
// no row-pass wavefront joins a CU that holds one of its workgroups).
template <int DT, bool LOGITS, bool PF, bool CON, bool HOLD = false>
__global__ __launch_bounds__(64 * kNarrowWaves) void select_narrow_kernel(DecodeParams p, int pen_len, int wave_bytes,
                                                                         int sig_words) {
    if constexpr (HOLD) asm volatile("" ::: "a255");
    extern __shared__ __align__(16) unsigned char smem_all[];
    const int K = p.K, T = p.T, M = p.M, V = p.V;
    // up to kNarrowWaves examples per workgroup, one per wavefront, each with
    // its own LDS; the wavefronts never wait for each other
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int b = static_cast<int>(blockIdx.x) * (static_cast<int>(blockDim.x) >> 6) + wave;
    const int lane = static_cast<int>(threadIdx.x) & 63;
    if (b >= p.B) return;
    if (p.claimed) {
        int mine = 1;
        if (lane == 0) mine = claim_example(p, b) ? 1 : 0;
        if (__builtin_amdgcn_readfirstlane(mine) == 0) return;
    }
    unsigned char* smem = smem_all + static_cast<size_t>(wave) * wave_bytes;
    uint4* s_key = reinterpret_cast<uint4*>(smem);                   // [64] rank keys
    ShortEntry* s_sl = reinterpret_cast<ShortEntry*>(smem + 1024);  // [K * M], beam k's list at k * M
    Cand* s_cand = reinterpret_cast<Cand*>(smem + 1024 + sizeof(ShortEntry) * static_cast<size_t>(K) * M);  // [64]
    float* s_pen = reinterpret_cast<float*>(s_cand + 64);  // [pen_len]
    float* s_inv = s_pen + pen_len;                        // [pen_len]
    // Constraints (n-gram blocking, repetition penalty): the beams' prefixes,
    // signatures of their tokens and of their (n - 1)-grams but the last (two
    // buffers each: the step's and the next), each read beam's
    // n-gram-blocked tokens, and per beam its read state and next prefix.
    const int P = p.prefix_cap, P4 = (P + 3) & ~3, W = sig_words;  // prefix rows P4 words apart (16-byte aligned)
    uint32_t* s_sig = reinterpret_cast<uint32_t*>(
        smem + ((1024 + sizeof(ShortEntry) * static_cast<size_t>(K) * M + sizeof(Cand) * 64 +
                 2 * sizeof(float) * static_cast<size_t>(pen_len) + 15) & ~static_cast<size_t>(15)));  // [2][K][W]
    uint32_t* s_gsig = s_sig + 2 * K * W;                             // [2][K][W]
    int32_t* s_pre = reinterpret_cast<int32_t*>(s_gsig + 2 * K * W);  // [2][K][P4]
    int32_t* s_blk = s_pre + 2 * K * P4;                             // [K][P]
    int32_t* s_nblk = s_blk + K * P;                                 // [K]
    int32_t* s_plen = s_nblk + K;                                    // [K] prefix length of a read beam, else -1
    int4* s_next = reinterpret_cast<int4*>(((reinterpret_cast<uintptr_t>(s_plen + K)) + 15) & ~static_cast<uintptr_t>(15));  // [K]
    uint32_t* s_gnew = reinterpret_cast<uint32_t*>(s_next + K);  // [K] the (n - 1)-gram a new beam's signature takes
    const int sig_shift = 32 - (31 - __builtin_clz(32 * static_cast<uint32_t>(W > 0 ? W : 1)));
    int cur = 0;  // the step's prefix buffer
    for (int l = lane; l < pen_len; l += 64) {
        const float pl = length_penalty(l, p.alpha);
        s_pen[l] = pl;
        s_inv[l] = 1.0f / pl;
    }
    auto pen_at = [&](int l) {
        const int c = l > 1 ? l : 1;
        return c < pen_len ? s_pen[c] : length_penalty(c, p.alpha);
    };
    auto inv_at = [&](int l) {
        const int c = l > 1 ? l : 1;
        return c < pen_len ? s_inv[c] : 1.0f / length_penalty(c, p.alpha);
    };
    const int steps_b = example_steps(p, b);
    const int Kb = beams_of(p, b), eos_b = eos_of(p, b);
    const bool coherent = p.step_done != nullptr;
    const bool beam = lane < K;
    const Cand dead = dead_cand();

    // beam `lane`'s state (reference src/decoder.cpp:46-56)
    float raw = lane == 0 ? 0.0f : -kInf;
    int len = 0, last = -1;
    bool ended = false;
    bool gave_up = false, any_invalid = false;
    int first_bad = 0x7fffffff;

    // the next step's RowInfo and shortlists (all rows written before this
    // kernel started: not the overlapped decode)
    // (four named registers: an array here would be kept in scratch memory)
    static_assert(kNarrowPf == 4, "four prefetch registers");
    uint4 pf0 = make_uint4(0u, 0u, 0u, 0u), pf1 = pf0, pf2 = pf0, pf3 = pf0, pf_info = pf0;
    auto prefetch = [&](int tn) __attribute__((always_inline)) {
        const int64_t base = (static_cast<int64_t>(b) * T + tn) * K;
        if (beam) pf_info = reinterpret_cast<const uint4*>(p.rowinfo)[base + lane];
        const uint4* src4 = reinterpret_cast<const uint4*>(p.shortlist + base * M);
        const int n4 = K * M / 2;
        if (lane < n4) pf0 = src4[lane];
        if (lane + 64 < n4) pf1 = src4[lane + 64];
        if (lane + 128 < n4) pf2 = src4[lane + 128];
        if (lane + 192 < n4) pf3 = src4[lane + 192];
    };
    bool have_pf = false;
    if constexpr (PF) {
        have_pf = steps_b > 0;
        if (have_pf) prefetch(0);
    }
    // A step's trace is stored during the next step and its row logsumexps
    // later in the same step, just after the next step's loads go out: stores
    // count in vmcnt like loads, so a wait for a loaded value also waits for
    // every store issued before that load.
    int64_t pend_o = -1;  // the pending trace slot (lanes < K), or none
    Cand pend_c = dead;
    bool pend_lse = false;
    int64_t pend_lse_o = 0;
    float pend_lse_v = 0.0f;
    auto flush = [&]() __attribute__((always_inline)) {
        if (pend_lse) p.row_lse[pend_lse_o] = pend_lse_v;
        if (pend_o >= 0) {
            if (p.tokens) p.tokens[pend_o] = pend_c.token;
            if (p.parents) p.parents[pend_o] = pend_c.parent;
            if (p.lengths) p.lengths[pend_o] = pend_c.length;
            if (p.scores) p.scores[pend_o] = pend_c.score;
            if (p.raw_scores) p.raw_scores[pend_o] = pend_c.raw;
            if (p.from_logprob) p.from_logprob[pend_o] = static_cast<uint8_t>(pend_c.flp);
        }
        pend_lse = false;
        pend_o = -1;
    };
    // overlapped decode: a step's words, loaded a step ahead (spec) while the
    // rows are already written, else at the step
    TagWords tw;
    bool spec = false;
    // Constraints: membership of v in beam k's prefix of length lk (the
    // step's buffer; its signature rules most tokens out with two bits), and
    // the value of token v's log-prob lp in beam k's row (make_cand's rules:
    // false when n-gram blocking removes it, the penalty when it repeats).
    auto in_pre = [&](int k, int lk, int v) -> bool {
        const uint32_t* sg = s_sig + (cur * K + k) * W;
        const uint32_t h0 = sig_bit0(v, sig_shift), h1 = sig_bit1(v, sig_shift);
        if ((((sg[h0 >> 5] >> (h0 & 31u)) & (sg[h1 >> 5] >> (h1 & 31u))) & 1u) == 0u) return false;
        return in_list(s_pre + (cur * K + k) * P4, lk, v);
    };
    auto constrain = [&](int k, int lk, int nbk, int v, float lp, float& val) -> bool {
        if (p.ngram > 1 && in_list(s_blk + k * P, nbk, v)) return false;
        val = (p.penalise && in_pre(k, lk, v)) ? lp - p.log_rep : lp;
        return true;
    };
    if constexpr (CON) {
        for (int i = lane; i < K * W; i += 64) {  // every prefix starts empty
            s_sig[i] = 0u;
            s_gsig[i] = 0u;
        }
    }
    // A beam's last n - 1 tokens (its tail), hashed (FNV-1a over the tokens),
    // when it has them: the n-gram list is built only where the tail occurred
    // before, and the tail joins the signature when the beam grows.
    uint32_t tail_h = 0u;
    bool tail_v = false;
    wave_sync();

    for (int t = 0; t < T; ++t) {
        const int64_t trace0 = (static_cast<int64_t>(b) * T + t) * K;
        bool pad = t >= steps_b || gave_up;
        const bool live = beam && raw < kInf && raw > -kInf;
        const bool carried = live && eos_b >= 0 && ended;
        bool read = !pad && live && !carried;
        int cnt = -2;
        float bound = -kInf, lse = 0.0f;
        bool bad = false, lost = false;
        // Overlapped decode: the step's row count (a hint of when to read),
        // the read rows' RowInfo words and the first shortlist words are
        // loaded together, so a step whose rows are all written costs one
        // round trip; a word not yet written (tag 0) is waited for after.
        const uint32_t* sl32 = reinterpret_cast<const uint32_t*>(p.shortlist + trace0 * M);
        uint32_t* const tlo = tw.lo;
        uint32_t* const thi = tw.hi;
        uint32_t& ilo0 = tw.ilo0;
        uint32_t& ihi0 = tw.ihi0;
        uint32_t& ilo1 = tw.ilo1;
        uint32_t& ihi1 = tw.ihi1;
        if (!pad && coherent) {
            // this step's words: loaded during the last step, or now
            if (!spec) issue_tagged(p, b, t, lane, tw);
            spec = false;
            const int need = (t == 0 ? 1 : Kb) + p.wait_extra;
            if (__builtin_amdgcn_readfirstlane(tw.have) < need) {
                int ok = 1;
                if (lane == 0) ok = wait_step_rows(p, b, t) ? 1 : 0;
                if (__builtin_amdgcn_readfirstlane(ok) == 0) {
                    gave_up = pad = true;
                    read = false;
                }
            }
        }
        if (read) {
            RowInfo info;
            if (have_pf) {
                __builtin_memcpy(&info, &pf_info, sizeof(info));
            } else if (!coherent) {
                info = p.rowinfo[trace0 + lane];
            } else {
                // the two tagged words (count + 2, invalid + 1)
                const uint32_t* info32 = reinterpret_cast<const uint32_t*>(p.rowinfo + trace0 + lane);
                bool ok = ihi0 != 0u || wait_tagged(p, info32, ilo0, ihi0);
                ok = ok && (ihi1 != 0u || wait_tagged(p, info32 + 2, ilo1, ihi1));
                if (!ok) {
                    lost = true;
                    ilo0 = ilo1 = 0;
                    ihi0 = 2;
                    ihi1 = 1;
                }
                info.lse = bits_f32(ilo0);
                info.count = static_cast<int32_t>(ihi0) - 2;
                info.bound = bits_f32(ilo1);
                info.invalid = ihi1 - 1u;
            }
            bad = info.invalid != 0;
            if (p.row_lse && LOGITS) {
                pend_lse = true;
                pend_lse_o = trace0 + lane;
                pend_lse_v = info.lse;
            }
            lse = info.lse;
            cnt = M > 0 ? info.count : -1;
            bound = info.bound;
        }
        const uint64_t bad_m = __builtin_amdgcn_ballot_w64(bad);
        if (bad_m != 0) {
            any_invalid = true;
            const int at = t * K + (__ffsll(static_cast<long long>(bad_m)) - 1);  // steps in order, beams in order
            first_bad = at < first_bad ? at : first_bad;
        }
        if (__builtin_amdgcn_ballot_w64(lost) != 0) gave_up = pad = true;
        if (pad) {
            flush();
            // a padding step (reference src/c_api.cpp:764-781): no token, no parent
            if (beam) {
                if (p.tokens) p.tokens[trace0 + lane] = -1;
                if (p.parents) p.parents[trace0 + lane] = -1;
                if (p.lengths) p.lengths[trace0 + lane] = 0;
                if (p.scores) p.scores[trace0 + lane] = -kInf;
                if (p.raw_scores) p.raw_scores[trace0 + lane] = -kInf;
                if (p.from_logprob) p.from_logprob[trace0 + lane] = 0;
            }
            continue;
        }

        // the shortlists into LDS (an entry past its row's count is never read)
        const ShortEntry* src = p.shortlist + trace0 * M;
        if (have_pf) {
            const int n4 = K * M / 2;
            uint4* dst4 = reinterpret_cast<uint4*>(s_sl);
            if (lane < n4) dst4[lane] = pf0;
            if (lane + 64 < n4) dst4[lane + 64] = pf1;
            if (lane + 128 < n4) dst4[lane + 128] = pf2;
            if (lane + 192 < n4) dst4[lane + 192] = pf3;
        } else if (!coherent) {
            for (int q0 = 0; q0 < K * M; q0 += 8 * 64) {
                ShortEntry e[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {  // clamped: every load in flight at once
                    const int q = q0 + 64 * u + lane;
                    e[u] = src[q < K * M ? q : K * M - 1];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (q0 + 64 * u + lane < K * M) s_sl[q0 + 64 * u + lane] = e[u];
            }
        } else {
            // the entries the row pass wrote (tag token + 1): the first
            // 64 kNarrowTagLoads were loaded with the RowInfo, the rest are
            // loaded now, kNarrowTagLoads per lane in flight; an entry not
            // yet written is waited for
            // (words written are stored as they are; only when one is not
            // is each lane's row count looked up, to wait for the words
            // within it)
            bool lost_e = false;
            for (int q0 = 0; q0 < K * M; q0 += 64 * kNarrowTagLoads) {
                if (q0 > 0) {
#pragma unroll
                    for (int u = 0; u < kNarrowTagLoads; ++u) {
                        const int q = q0 + 64 * u + lane;
                        (void)read_tagged(sl32 + 2 * (q < K * M ? q : K * M - 1), tlo[u], thi[u]);
                    }
                }
                bool missing = false;
#pragma unroll
                for (int u = 0; u < kNarrowTagLoads; ++u) {
                    const int q = q0 + 64 * u + lane;
                    if (q >= K * M) continue;
                    if (thi[u] != 0u) s_sl[q] = ShortEntry{bits_f32(tlo[u]), static_cast<int32_t>(thi[u]) - 1};
                    else missing = true;
                }
                if (__builtin_amdgcn_ballot_w64(missing) != 0) {
#pragma unroll
                    for (int u = 0; u < kNarrowTagLoads; ++u) {
                        const int q = q0 + 64 * u + lane;
                        const int k = q / M;
                        const int cq = __shfl(cnt, k < K ? k : 0);  // every lane: the shuffle reads other lanes
                        if (q >= K * M || q - k * M >= cq || thi[u] != 0u) continue;
                        if (!wait_tagged(p, sl32 + 2 * q, tlo[u], thi[u])) {
                            lost_e = true;
                            thi[u] = 1;
                        }
                        s_sl[q] = ShortEntry{bits_f32(tlo[u]), static_cast<int32_t>(thi[u]) - 1};
                    }
                }
            }
            if (__builtin_amdgcn_ballot_w64(lost_e) != 0) {
                gave_up = true;
                flush();
                if (beam) {
                    if (p.tokens) p.tokens[trace0 + lane] = -1;
                    if (p.parents) p.parents[trace0 + lane] = -1;
                    if (p.lengths) p.lengths[trace0 + lane] = 0;
                    if (p.scores) p.scores[trace0 + lane] = -kInf;
                    if (p.raw_scores) p.raw_scores[trace0 + lane] = -kInf;
                    if (p.from_logprob) p.from_logprob[trace0 + lane] = 0;
                }
                wave_sync();
                continue;
            }
        }
        // this step's rows are staged: the next step's loads go out, then
        // the pending stores (after the loads, so that waiting for the loads
        // never waits for them)
        if constexpr (PF) {
            have_pf = t + 1 < steps_b;
            if (have_pf) prefetch(t + 1);
        }
        if (coherent && t + 1 < steps_b) {
            issue_tagged(p, b, t + 1, lane, tw);
            spec = true;
        }
        flush();
        wave_sync();

        // Constraints: each read beam's n-gram-blocked tokens, the tokens
        // that followed an earlier occurrence of its last n - 1 tokens (one
        // lane per (beam, prefix position); a read beam's prefix holds t
        // tokens)
        int nblk = 0;
        if constexpr (CON) {
            bool need = false;
            if (p.ngram > 1) {
                // the tail, and whether it ended an earlier (n - 1)-gram of
                // the prefix (the signature of those; a hit is checked in full)
                const int n = p.ngram;
                tail_v = read && len >= n - 1;
                tail_h = 0x811C9DC5u;
                if (tail_v) {
                    const int32_t* pre = s_pre + (cur * K + lane) * P4;
                    for (int q = len - (n - 1); q < len; ++q)
                        tail_h = (tail_h ^ static_cast<uint32_t>(pre[q])) * 0x01000193u;
                    if (len >= n) {
                        const uint32_t* gs = s_gsig + (cur * K + lane) * W;
                        const uint32_t h0 = sig_bit0(static_cast<int>(tail_h), sig_shift);
                        const uint32_t h1 = sig_bit1(static_cast<int>(tail_h), sig_shift);
                        need = (((gs[h0 >> 5] >> (h0 & 31u)) & (gs[h1 >> 5] >> (h1 & 31u))) & 1u) != 0u;
                    }
                }
            }
            if (beam) s_plen[lane] = need ? len : -1;
            if (__builtin_amdgcn_ballot_w64(need) != 0) {
                if (beam) s_nblk[lane] = 0;
                wave_sync();
                // item = (beam k, position i); eight items per lane a round,
                // every read of a round in flight together
                // (beam k's positions at a power-of-two stride 2^ps >= t: no
                // division)
                const int n = p.ngram, Pt = min(P, t);
                const int ps = Pt > 1 ? 32 - __builtin_clz(static_cast<uint32_t>(Pt - 1)) : 0, total = K << ps;
                for (int j0 = 0; j0 < total; j0 += 8 * 64) {
                    int kk[8], ii[8], tl[8];
                    bool on[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int j = j0 + 64 * u + lane;
                        const int jc = j < total ? j : 0;
                        kk[u] = jc >> ps;
                        ii[u] = jc & ((1 << ps) - 1);
                        const int Lk = s_plen[kk[u]];
                        on[u] = j < total && ii[u] + n <= Lk;  // (a beam not read: -1)
                        tl[u] = on[u] ? Lk - (n - 1) : 0;
                    }
                    bool same[8] = {true, true, true, true, true, true, true, true};
                    for (int q = 0; q < n - 1; ++q) {
                        int32_t a[8], c[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            const int32_t* pre = s_pre + (cur * K + kk[u]) * P4;
                            a[u] = pre[on[u] ? ii[u] + q : 0];
                            c[u] = pre[tl[u] + q];
                        }
#pragma unroll
                        for (int u = 0; u < 8; ++u) same[u] = same[u] && a[u] == c[u];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        if (on[u] && same[u]) {
                            const int slot = atomicAdd(&s_nblk[kk[u]], 1);
                            s_blk[kk[u] * P + slot] = s_pre[(cur * K + kk[u]) * P4 + ii[u] + n - 1];
                        }
                    }
                }
                wave_sync();
                nblk = beam ? s_nblk[lane] : 0;
            }
        }

        // tau (every expanded beam has the same length, so this step's
        // shortlisted candidates rank by raw): at least K candidates reach it
        const int new_len = len + 1;
        const float inv = inv_at(new_len);
        float tv = -kInf;
        if constexpr (CON) {
            // K of a row's first K + nblk entries are not blocked (a blocked
            // token is at most one entry), each worth at least its log-prob
            // less the penalty
            if (read && cnt >= K + nblk) {
                const float lpk = s_sl[lane * M + (K - 1 + nblk)].lp;
                tv = raw + (p.penalise ? lpk - p.log_rep : lpk);
            }
        } else {
            if (read && cnt >= K) tv = raw + s_sl[lane * M + (K - 1)].lp;
        }
        const float tau = wave_max_dpp(tv);
        // survivors of beam `lane`: a prefix of its shortlist
        int ns = 0;
        if (read) {
            for (;;) {  // four entries a round, their reads in flight together
                float lp4[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) lp4[u] = ns + u < cnt ? s_sl[lane * M + ns + u].lp : -kInf;
                int reach = 0;
                bool on = true;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    on = on && ns + u < cnt && !(raw + lp4[u] < tau);
                    reach += on ? 1 : 0;
                }
                ns += reach;
                if (reach < 4) break;
            }
        }
        // the carried-forward candidate (reference src/decoder.cpp:131-139)
        Cand carry = dead;
        if (carried) {
            const int l = len > 1 ? len : 1;
            carry = Cand{raw / pen_at(l), raw, lane, is_eos_of(p, b, last) ? last : eos_b, l, 0};
        }
        const uint64_t carried_m = __builtin_amdgcn_ballot_w64(carried);
        const int incl = wave_inclusive_sum(ns);
        const int nsurv = __builtin_amdgcn_readlane(incl, 63);
        const int ncand = nsurv + static_cast<int>(__popcll(carried_m));

        // the selection: the best Kb candidates, lane k holding the k-th
        Cand sel = dead;
        int nsel = 0;
        // survivor s (< nsurv) as a candidate: beam k with s in [off_k,
        // off_k + ns_k). Every lane calls it (the shuffles read other lanes).
        auto survivor = [&](int s) -> Cand {
            int k = 0;
            for (int kk = 1; kk < K; ++kk)
                if (s >= __builtin_amdgcn_readlane(incl - ns, kk)) k = kk;
            const int i = s - __shfl(incl - ns, k);
            const ShortEntry e = s_sl[k * M + i];
            const int lk = __shfl(len, k), nbk = __shfl(nblk, k);
            float val = e.lp;
            bool ok = true;
            if constexpr (CON) ok = constrain(k, lk, nbk, e.token, e.lp, val);
            const float r = __shfl(raw, k) + val;
            const float ik = __shfl(inv, k);
            const int nlk = __shfl(new_len, k);
            return ok ? Cand{r * ik, r, k, e.token, nlk, 1} : dead;
        };
        if (ncand <= 64) {
            // one candidate per lane, ranked by the count of those before it:
            // lane L < nsurv takes survivor L (of beam k, the last beam whose
            // survivors start at or before L), read from the shortlist;
            // lanes [nsurv, ncand) take the carried beams in beam order
            const int excl = incl - ns;
            int k = 0;
            for (int kk = 1; kk < K; ++kk)
                if (lane >= __builtin_amdgcn_readlane(excl, kk)) k = kk;
            const int ik0 = lane - __shfl(excl, k);
            const ShortEntry e = s_sl[k * M + (lane < nsurv ? ik0 : 0)];
            const float rk = __shfl(raw, k), ivk = __shfl(inv, k);
            const int nlk = __shfl(new_len, k);
            Cand c = dead;
            if (lane < nsurv) {
                if constexpr (CON) {
                    // the log-prob in the score field: the constraints are
                    // applied below, one candidate per lane
                    c = Cand{e.lp, 0.0f, k, e.token, nlk, 1};
                } else {
                    const float r = rk + e.lp;
                    c = Cand{r * ivk, r, k, e.token, nlk, 1};
                }
            }
            if (carried_m != 0) {
                // the (lane - nsurv)-th carried beam
                int src = 0, seen = 0;
                for (int kk = 0; kk < K; ++kk) {
                    if (((carried_m >> kk) & 1ull) == 0) continue;
                    if (seen == lane - nsurv) src = kk;
                    ++seen;
                }
                Cand cb;
                cb.score = bits_f32(static_cast<uint32_t>(__shfl(static_cast<int>(f32_bits(carry.score)), src)));
                cb.raw = bits_f32(static_cast<uint32_t>(__shfl(static_cast<int>(f32_bits(carry.raw)), src)));
                cb.parent = __shfl(carry.parent, src);
                cb.token = __shfl(carry.token, src);
                cb.length = __shfl(carry.length, src);
                cb.flp = __shfl(carry.flp, src);
                if (lane >= nsurv && lane < ncand) c = cb;
            }
            if constexpr (CON) {
                const bool surv = lane < nsurv;  // (the carried-forward beams follow the survivors)
                const int k = surv ? c.parent : 0;
                const float pr = __shfl(raw, k), pi = __shfl(inv, k);
                const int lk = __shfl(len, k), nbk = __shfl(nblk, k);
                if (surv) {
                    float val = c.score;
                    if (constrain(k, lk, nbk, c.token, c.score, val)) {
                        const float r = pr + val;
                        c.score = r * pi;
                        c.raw = r;
                    } else {
                        c = dead;
                    }
                }
            }
            const bool valid = lane < ncand && before(c, dead);
            // Its key, larger exactly when the candidate comes earlier in the
            // total order: score, raw, then (parent, token), which no two of
            // a step's candidates share (a carried beam is not expanded), so
            // length and flp never decide. Parents < 64, tokens < 2^24.
            const uint32_t k2 = ordered_key(c.score), k1 = ordered_key(c.raw);
            const uint32_t k0 = 0xffffffffu - ((static_cast<uint32_t>(c.parent) << 24) |
                                               (static_cast<uint32_t>(c.token) & 0xffffffu));
            s_key[lane] = make_uint4(k0, k1, k2, 0u);
            wave_sync();
            int rank = 0;
            int j = 0;
            for (; j + 4 <= ncand; j += 4) {  // four broadcast reads in flight
                uint4 w[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) w[u] = s_key[j + u];
#pragma unroll
                for (int u = 0; u < 4; ++u) count_above96(rank, k0, k1, k2, w[u].x, w[u].y, w[u].z);
            }
            for (; j < ncand; ++j) {
                const uint4 w = s_key[j];
                count_above96(rank, k0, k1, k2, w.x, w.y, w.z);
            }
            nsel = static_cast<int>(__popcll(__builtin_amdgcn_ballot_w64(valid)));
            nsel = nsel < Kb ? nsel : Kb;
            // each selected candidate to the lane of its rank (lanes not
            // selected write lane 63, which holds no selection: Kb <= 16)
            const int to = 4 * ((valid && rank < Kb) ? rank : 63);
            Cand sc;
            sc.score = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_ds_permute(to, static_cast<int>(f32_bits(c.score)))));
            sc.raw = bits_f32(static_cast<uint32_t>(__builtin_amdgcn_ds_permute(to, static_cast<int>(f32_bits(c.raw)))));
            sc.parent = __builtin_amdgcn_ds_permute(to, c.parent);
            sc.token = __builtin_amdgcn_ds_permute(to, c.token);
            sc.length = __builtin_amdgcn_ds_permute(to, c.length);
            sc.flp = __builtin_amdgcn_ds_permute(to, c.flp);
            if (lane < nsel) sel = sc;
            wave_sync();  // the keys' LDS may be reused
        } else {
            Cand thr = dead;
            for (int s0 = 0; s0 < nsurv; s0 += 64) {
                const bool has = s0 + lane < nsurv;
                const Cand c = survivor(has ? s0 + lane : nsurv - 1);
                list_offer(sel, thr, c, has, Kb, lane);
            }
            list_offer(sel, thr, carry, carried, Kb, lane);
            nsel = static_cast<int>(__popcll(__builtin_amdgcn_ballot_w64(lane < Kb && before(sel, dead))));
        }

        // Exactness: every candidate left out of a row's shortlist has raw <=
        // fl(p + bound); a row passes when the Kb-th selected candidate ranks
        // strictly before that bound's score and raw.
        {
            const Cand kth = nsel >= Kb ? lane_cand(sel, Kb - 1) : dead;
            bool fail = false;
            if (read) {
                fail = cnt < 0;
                if (!fail && bound > -kInf) {
                    const float X = raw + bound;
                    if (X > -kInf) {
                        const float SX = X * inv;
                        fail = !((kth.score > SX) || (kth.score == SX && kth.raw > X));
                    }
                }
            }
            const uint64_t fail_m = __builtin_amdgcn_ballot_w64(fail);
            if (fail_m != 0) {
                if (lane == 0) atomicAdd(&g_rescanned_rows, static_cast<unsigned long long>(__popcll(fail_m)));
                // the passing rows' survivors, the carried-forward beams,
                // then every token of each failing row
                Cand thr = dead;
                sel = dead;
                for (int s0 = 0; s0 < nsurv; s0 += 64) {
                    const bool has = s0 + lane < nsurv;
                    const Cand c = survivor(has ? s0 + lane : nsurv - 1);  // parent in [0, K)
                    list_offer(sel, thr, c, has && ((fail_m >> c.parent) & 1ull) == 0, Kb, lane);
                }
                list_offer(sel, thr, carry, carried, Kb, lane);
                const int min_len = min_length_of(p, b);
                const size_t esz = DT == 0 ? 4 : 2;
                for (uint64_t m = fail_m; m != 0; m &= m - 1) {
                    // beam k's values, in every lane
                    const int k = __ffsll(static_cast<long long>(m)) - 1;
                    const float praw = __shfl(raw, k), lse_k = __shfl(lse, k), inv_k = __shfl(inv, k);
                    const int nl = __shfl(new_len, k), lk = __shfl(len, k), nbk = __shfl(nblk, k);
                    const bool mask_eos = nl < min_len;
                    const char* base = static_cast<const char*>(p.x) +
                                       static_cast<size_t>(trace0 + k) * static_cast<size_t>(V) * esz;
                    for (int v0 = 0; v0 < V; v0 += 64 * kNarrowRescanUnroll) {
                        float xs[kNarrowRescanUnroll];
#pragma unroll
                        for (int u = 0; u < kNarrowRescanUnroll; ++u) {
                            const int v = v0 + 64 * u + lane;
                            xs[u] = v < V ? load_one<DT>(base, v) : -kInf;
                        }
#pragma unroll
                        for (int u = 0; u < kNarrowRescanUnroll; ++u) {
                            const int v = v0 + 64 * u + lane;
                            const float lp = LOGITS ? xs[u] - lse_k : xs[u];
                            bool ok = v < V && lp < kInf && lp != -kInf;
                            float val = lp;
                            if constexpr (CON) ok = ok && constrain(k, lk, nbk, v, lp, val);
                            const float r = praw + val;
                            const Cand c{r * inv_k, r, k, v, nl, 1};
                            const bool offer = ok && before(c, thr) && !static_masked(p, b, v, mask_eos);
                            list_offer(sel, thr, c, offer, Kb, lane);
                        }
                    }
                }
                nsel = static_cast<int>(__popcll(__builtin_amdgcn_ballot_w64(lane < Kb && before(sel, dead))));
            }
        }

        // Selection (reference src/decoder.cpp:314-350): the trace and the
        // next state of each slot
        const Cand c = lane < nsel ? sel : dead;
        if (beam) {
            pend_o = trace0 + lane;
            pend_c = c;
        }
        if constexpr (CON) {
            // each selected beam: its parent's prefix, then its token, and the
            // signature of both, into the other buffer
            const int par = c.parent;
            const int len_par = __shfl(len, par >= 0 ? par : 0);
            const uint32_t gh_par = static_cast<uint32_t>(__shfl(static_cast<int>(tail_h), par >= 0 ? par : 0));
            const int gv_par = __shfl(tail_v ? 1 : 0, par >= 0 ? par : 0);
            const bool grows = par >= 0 && c.flp && c.token >= 0;
            if (beam) {
                s_next[lane] = make_int4(par, grows ? c.token : -1, par >= 0 ? len_par : 0, grows && gv_par ? 1 : 0);
                s_gnew[lane] = gh_par;
            }
            wave_sync();
            const int nxt = cur ^ 1;
            const int Lc = min(P, t + 1);  // the new prefixes' length, at most
            // 16 bytes an item: the parent's prefix (its appended token's
            // word is written over after), then its signature with the
            // token's two bits; four items per lane a round, their reads in
            // flight together
            // (each beam's chunks at power-of-two strides: no division)
            const int C4 = (Lc + 3) >> 2, W4 = W / 4;
            const int cs = C4 > 1 ? 32 - __builtin_clz(static_cast<uint32_t>(C4 - 1)) : 0;
            const int ws = 31 - __builtin_clz(static_cast<uint32_t>(W4));
            // the (n - 1)-gram signatures follow the token signatures
            const int ns = K << ws, np = K << cs, total = np + (p.ngram > 1 ? 2 : 1) * ns;
            uint4* const s_pre4 = reinterpret_cast<uint4*>(s_pre);
            uint4* const s_sig4 = reinterpret_cast<uint4*>(s_sig);
            for (int j0 = 0; j0 < total; j0 += 5 * 64) {
                int dst[5];
                bool isp[5];
                uint4 v[5];
#pragma unroll
                for (int u = 0; u < 5; ++u) {
                    const int j = j0 + 64 * u + lane;
                    const int jc = j < total ? j : 0;
                    isp[u] = jc < np;
                    const bool isg = jc >= np + ns;  // an (n - 1)-gram signature chunk
                    const int jj = isp[u] ? jc : jc - np - (isg ? ns : 0), sh = isp[u] ? cs : ws;
                    const int k = jj >> sh, q = jj & ((1 << sh) - 1);
                    const int4 nx = s_next[k];
                    const int pk = nx.x >= 0 ? nx.x : 0;
                    if (isp[u]) {
                        dst[u] = j < total && nx.x >= 0 && q < C4 ? ((nxt * K + k) * P4 >> 2) + q : -1;
                        v[u] = s_pre4[((cur * K + pk) * P4 >> 2) + (q < C4 ? q : 0)];
                    } else {
                        // (s_gsig is s_sig + 2 K W words: the same buffers, 2 K W4 chunks on)
                        const int g4 = isg ? 2 * K * W4 : 0;
                        dst[u] = j < total ? g4 + (nxt * K + k) * W4 + q : -1;
                        v[u] = s_sig4[g4 + (cur * K + pk) * W4 + q];
                        if (nx.x < 0) v[u] = make_uint4(0u, 0u, 0u, 0u);
                        const bool add = isg ? nx.w != 0 : nx.x >= 0 && nx.y >= 0;
                        if (add) {
                            const int hv = isg ? static_cast<int>(s_gnew[k]) : nx.y;
                            const uint32_t hs[2] = {sig_bit0(hv, sig_shift), sig_bit1(hv, sig_shift)};
#pragma unroll
                            for (int h2 = 0; h2 < 2; ++h2) {
                                const uint32_t h = hs[h2];
                                if (static_cast<int>(h >> 7) != q) continue;
                                const uint32_t m = 1u << (h & 31u);
                                switch ((h >> 5) & 3u) {
                                    case 0: v[u].x |= m; break;
                                    case 1: v[u].y |= m; break;
                                    case 2: v[u].z |= m; break;
                                    default: v[u].w |= m; break;
                                }
                            }
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < 5; ++u)
                    if (dst[u] >= 0) (isp[u] ? s_pre4 : s_sig4)[dst[u]] = v[u];
            }
            wave_sync();
            if (beam && par >= 0 && c.flp && c.token >= 0) s_pre[(nxt * K + lane) * P4 + len_par] = c.token;
            wave_sync();
            cur = nxt;
        }
        const int parent_ended = __shfl(ended ? 1 : 0, c.parent >= 0 ? c.parent : 0);
        ended = c.parent >= 0 && (parent_ended != 0 || is_eos_of(p, b, c.token));
        raw = c.raw;
        len = c.length;
        last = c.token;
        wave_sync();
    }
    flush();

    if (gave_up) {
        // no hypothesis survives an abandoned decode
        raw = -kInf;
        len = 0;
        if (lane == 0 && p.fault) __hip_atomic_store(p.fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Final scores (reference src/decoder.cpp:179-187).
    if (beam) {
        const int64_t i = static_cast<int64_t>(b) * K + lane;
        if (p.final_scores) p.final_scores[i] = raw / pen_at(len);
        if (p.final_raw) p.final_raw[i] = raw;
        if (p.final_lengths) p.final_lengths[i] = len;
    }
    // 1: a row the search read holds NaN or +inf; 2: the decode of the
    // example did not complete (an overlapped wait gave up)
    if (lane == 0 && p.invalid) p.invalid[b] = static_cast<uint8_t>(gave_up ? 2 : (any_invalid ? 1 : 0));
    if (lane == 0 && p.first_invalid) p.first_invalid[b] = first_bad == 0x7fffffff ? -1 : first_bad;
}

// The prefetch needs the row pass finished before the select pass starts (not
// the overlapped decode, whose rows land while it runs) and a step's
// shortlists within the prefetch registers, as 16-byte pairs of entries.
bool prefetch_fits(const DecodeParams& p) {
    return p.step_done == nullptr && !p.step_mode && p.M > 0 && (p.M & 1) == 0 && p.K <= kSelectThreads &&
           p.K * p.M <= 2 * kPfRegs * kSelectThreads;
}

template <int DT, bool LOGITS, bool PF, bool HOLD = false>
hipError_t launch_select_variant(const DecodeParams& p, const SelectLayout& L, hipStream_t stream) {
    if (L.smem > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&select_kernel<DT, LOGITS, PF, HOLD>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(L.smem));
        if (e != hipSuccess) return e;
    }
    KernelTimer timer(kKindSelect, stream);
    hipLaunchKernelGGL((select_kernel<DT, LOGITS, PF, HOLD>), dim3(p.B), dim3(kSelectThreads), L.smem, stream, p, L);
    return hipGetLastError();
}

// Workgroups of the narrow pass: a multiple of kXcds (workgroups are dealt
// to the XCDs in turn, and a persistent row pass of CUs - groups workgroups
// leaves groups / kXcds CUs free on each), up to kNarrowWaves examples each.
int narrow_groups(int B) { return kXcds * ((B + kXcds * kNarrowWaves - 1) / (kXcds * kNarrowWaves)); }
int narrow_per_group(int B) {
    const int g = narrow_groups(B);
    return (B + g - 1) / g;
}

int narrow_pen_len(const DecodeParams& p) { return p.T + 2 < kNarrowPenCap ? p.T + 2 : kNarrowPenCap; }

// One wavefront's LDS: rank keys, shortlists, candidates, penalty tables;
// with constraints also signatures of W words per beam, prefixes, n-gram
// lists and per-beam state (the kernel's layout).
size_t narrow_wave_bytes(const DecodeParams& p, int W) {
    const size_t K = static_cast<size_t>(p.K), P = static_cast<size_t>(p.prefix_cap);
    size_t n = 1024 + sizeof(ShortEntry) * K * static_cast<size_t>(p.M) + sizeof(Cand) * 64 +
               2 * sizeof(float) * static_cast<size_t>(narrow_pen_len(p));
    n = (n + 15) & ~static_cast<size_t>(15);
    if (p.constrained) {
        const size_t P4 = (P + 3) & ~static_cast<size_t>(3);
        n += sizeof(uint32_t) * 4 * K * static_cast<size_t>(W) + sizeof(int32_t) * (2 * K * P4 + K * P + 2 * K);
        n = ((n + 15) & ~static_cast<size_t>(15)) + sizeof(int4) * K + sizeof(uint32_t) * K;
    }
    return (n + 15) & ~static_cast<size_t>(15);
}

// Signature words per beam of a constrained decode (the most of 64, 32, 16
// that fit one wavefront's LDS), else 0; 0 for an unconstrained one.
int narrow_sig_words(const DecodeParams& p) {
    if (!p.constrained) return 0;
    for (int W = 64; W >= 16; W /= 2)
        if (narrow_wave_bytes(p, W) <= static_cast<size_t>(kNarrowWaveLds)) return W;
    return 0;
}

template <int DT, bool LOGITS, bool CON>
hipError_t launch_select_narrow(const DecodeParams& p, hipStream_t stream) {
    const int pen_len = narrow_pen_len(p);
    const int W = narrow_sig_words(p);
    const int wave_bytes = static_cast<int>(narrow_wave_bytes(p, W));
    // prefetch: rows all written before the kernel starts, shortlists as
    // 16-byte pairs of entries within the prefetch registers
    const bool pf = p.step_done == nullptr && (p.M & 1) == 0 && p.K * p.M <= 2 * 64 * kNarrowPf;
    KernelTimer timer(kKindSelect, stream);
    const int per = narrow_per_group(p.B);
    const dim3 grid((p.B + per - 1) / per), block(64 * per);
    const size_t smem = static_cast<size_t>(wave_bytes) * per;
    if (smem > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(pf ? &select_narrow_kernel<DT, LOGITS, true, CON>
                                                                           : &select_narrow_kernel<DT, LOGITS, false, CON>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
        if (e == hipSuccess && CON)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&select_narrow_kernel<DT, LOGITS, false, true, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
        if (e != hipSuccess) return e;
    }
    // beside a row pass of one workgroup per row: constrained decodes hold
    // their CUs (p.select_hold)
    if (CON && p.select_hold)
        hipLaunchKernelGGL((select_narrow_kernel<DT, LOGITS, false, true, true>), grid, block, smem, stream, p, pen_len,
                           wave_bytes, W);
    else if (pf)
        hipLaunchKernelGGL((select_narrow_kernel<DT, LOGITS, true, CON>), grid, block, smem, stream, p, pen_len,
                           wave_bytes, W);
    else
        hipLaunchKernelGGL((select_narrow_kernel<DT, LOGITS, false, CON>), grid, block, smem, stream, p, pen_len,
                           wave_bytes, W);
    return hipGetLastError();
}

template <int DT, bool LOGITS>
hipError_t launch_select_typed(const DecodeParams& p, const SelectLayout& L, hipStream_t stream) {
    if (select_narrow(p))
        return p.constrained ? launch_select_narrow<DT, LOGITS, true>(p, stream)
                             : launch_select_narrow<DT, LOGITS, false>(p, stream);
    if (p.select_hold) return launch_select_variant<DT, LOGITS, false, true>(p, L, stream);
    return prefetch_fits(p) ? launch_select_variant<DT, LOGITS, true>(p, L, stream)
                            : launch_select_variant<DT, LOGITS, false>(p, L, stream);
}

}  // namespace

std::atomic<int> g_select_kind{0};

bool select_narrow(const DecodeParams& p) {
    if (g_select_kind.load(std::memory_order_relaxed) == 1) return false;
    if (p.step_mode || p.forced || p.pool_mult > 0 || p.M <= 0 || p.K > kNarrowMaxK || p.V > (1 << 24)) return false;
    // constrained: n-gram blocking of n >= 2 and/or a repetition penalty
    // (n = 1 blocking would drop most of a long prefix's shortlist entries)
    if (p.constrained) return p.ngram != 1 && narrow_sig_words(p) > 0;
    return p.use_tau && narrow_wave_bytes(p, 0) <= static_cast<size_t>(kNarrowWaveLds);
}

int select_reserve_cus(const DecodeParams& p) {
    return select_narrow(p) ? narrow_groups(p.B) : p.B;
}

SelectLayout select_layout(int B, int T, int K, int M, bool constrained, bool step_mode, int prefix_cap, int keep) {
    (void)B;
    SelectLayout L{};
    int sc = 1;
    while (sc < (keep > K ? keep : K) + 2 * kSelectThreads) sc <<= 1;
    L.sort_cap = sc;
    L.pen_len = step_mode ? 0 : T + 2;
    auto align = [](size_t x) { return (x + 15) & ~static_cast<size_t>(15); };
    size_t off = 0;
    L.off_buf = off;
    off = align(off + sizeof(Cand) * static_cast<size_t>(sc));
    L.off_rbuf = off;
    off = align(off + sizeof(Cand) * kRescanBuf);
    L.off_key = off;
    off = align(off + sizeof(uint4) * 2 * kRankMax + sizeof(int32_t) * (kSelectThreads + 64 + 1));
    L.off_f32 = off;
    off = align(off + sizeof(float) * (3 * static_cast<size_t>(K) + 2 * static_cast<size_t>(L.pen_len)));
    L.off_i32 = off;
    off = align(off + sizeof(int32_t) * 10 * static_cast<size_t>(K));
    L.off_sl = off;
    off = align(off + sizeof(ShortEntry) * static_cast<size_t>(K) * static_cast<size_t>(K >= kWideBeam ? M + 1 : M));
    const size_t prefix_bytes = sizeof(int32_t) * 2 * static_cast<size_t>(K) * static_cast<size_t>(prefix_cap);
    const size_t blk_bytes = sizeof(int32_t) * static_cast<size_t>(K) * static_cast<size_t>(prefix_cap);
    const size_t budget = 150 * 1024;
    L.prefix_in_lds = 0;
    L.blk_in_lds = 0;
    if (constrained && !step_mode && off + prefix_bytes <= budget) {
        L.prefix_in_lds = 1;
        L.off_prefix = off;
        off = align(off + prefix_bytes);
    }
    if (constrained && off + blk_bytes <= budget) {
        L.blk_in_lds = 1;
        L.off_blk = off;
        off = align(off + blk_bytes);
    }
    L.sig_in_lds = 0;
    L.sig_words = 0;
    for (int words = kSigWordsMax; words >= kSigWordsMax / 4 && !L.sig_in_lds; words /= 4) {
        const size_t sig_bytes = sizeof(uint32_t) * 2 * static_cast<size_t>(K) * words;
        if (L.prefix_in_lds && off + sig_bytes <= budget) {
            L.sig_in_lds = 1;
            L.sig_words = words;
            L.off_sig = off;
            off = align(off + sig_bytes);
        }
    }
    L.smem = off;
    return L;
}

hipError_t launch_select(const DecodeParams& p, const SelectLayout& L, hipStream_t stream) {
    if (p.from_logits) {
        switch (p.dtype) {
            case 0: return launch_select_typed<0, true>(p, L, stream);
            case 1: return launch_select_typed<1, true>(p, L, stream);
            default: return launch_select_typed<2, true>(p, L, stream);
        }
    }
    switch (p.dtype) {
        case 0: return launch_select_typed<0, false>(p, L, stream);
        case 1: return launch_select_typed<1, false>(p, L, stream);
        default: return launch_select_typed<2, false>(p, L, stream);
    }
}

hipError_t wait_timeout_counter(int reset, unsigned long long* value) {
    if (reset) {
        const unsigned long long zero = 0;
        return hipMemcpyToSymbol(HIP_SYMBOL(g_wait_timeouts), &zero, sizeof(zero));
    }
    return hipMemcpyFromSymbol(value, HIP_SYMBOL(g_wait_timeouts), sizeof(*value));
}

hipError_t rescan_counter(int reset, unsigned long long* value) {
    if (reset) {
        const unsigned long long zero = 0;
        return hipMemcpyToSymbol(HIP_SYMBOL(g_rescanned_rows), &zero, sizeof(zero));
    }
    return hipMemcpyFromSymbol(value, HIP_SYMBOL(g_rescanned_rows), sizeof(*value));
}

}  // namespace dbs_hip
