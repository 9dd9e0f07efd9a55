// SPDX-License-Identifier: MIT
//
// Decode kernels of libdbs_hip for gfx950.
//
// The search runs as two launches:
//
//  1. row_pass: every row the search may read is streamed from HBM by one
//     wavefront, independently of the selection, so the whole chip works on
//     all B*T*K rows at once. Per row it produces the NaN/+inf flag, the exact
//     logsumexp (from logits), and a shortlist: the best M allowed tokens by
//     (log-prob desc, token asc) plus an upper bound on every allowed token
//     left out.
//  2. select: one workgroup per example walks the T steps. Each step builds
//     the candidates (EOS carry-forward, shortlist entries with n-gram
//     blocking and the repetition penalty), keeps the best K under the
//     reference's total order, and proves the result exact: a row whose
//     bound could still beat the K-th selected candidate is rescanned in full
//     from HBM. So the selection always equals the reference's, and the
//     rescans are rare.
//
// Exactness rests on: all candidates expanded at one step extend beams of one
// length (ranked by raw score, which is monotone in log-prob), the fixed
// 256-lane fold order of the logsumexp (reference src/logits.hpp:42-50,
// src/kernels_scalar.cpp:48-66), and IEEE operations in the reference's order
// (reference src/decoder.cpp:122-187, src/kernels.hpp:113-122).
#include <hip/hip_runtime.h>

#include "engine.hpp"

namespace dbs_hip {

namespace {

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

__device__ __forceinline__ int example_steps(const DecodeParams& p, int b) {
    return p.steps ? p.steps[b] : p.T;
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

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
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

// ---------------------------------------------------------------------------
// Select pass
// ---------------------------------------------------------------------------

struct SelectShared {
    Cand* buf;        // [sort_cap]
    float* raw;       // [K] beams after the previous step
    int32_t* len;
    int32_t* last;
    int32_t* ended;
    float* nraw;      // [K] beams after this step
    int32_t* nlen;
    int32_t* nlast;
    int32_t* nended;
    int32_t* rcount;  // [K] shortlist entries of the beam's row (-2: row not read)
    float* rbound;    // [K]
    int32_t* plen;    // [2 * K] prefix lengths
};

struct SelectState {
    int count;
    int any_fail;
    uint32_t invalid;
    float tau;
    Cand thr;
};

template <int DT>
__device__ __forceinline__ float load_row_elem(const DecodeParams& p, int64_t row, int v) {
    const size_t esz = DT == 0 ? 4 : 2;
    const char* base = static_cast<const char*>(p.x) + static_cast<size_t>(row) * static_cast<size_t>(p.V) * esz;
    return load_one<DT>(base, v);
}

// The prefix of beam k (tokens of its path) in the current buffer.
struct PrefixView {
    const int32_t* tok;
    int len;
};

__device__ __forceinline__ PrefixView prefix_of(const DecodeParams& p, const SelectShared& sh, int b, int k, int cur) {
    if (p.step_mode) {
        const int L = sh.len[k] < 0 ? 0 : (sh.len[k] < p.st_stride ? sh.len[k] : p.st_stride);
        return PrefixView{p.st_prefix + (static_cast<int64_t>(b) * p.K + k) * p.st_stride, L};
    }
    const int64_t base = ((static_cast<int64_t>(cur) * p.B + b) * p.K + k) * p.prefix_cap;
    return PrefixView{p.prefix + base, sh.plen[cur * p.K + k]};
}

// Would token v repeat an n-gram of the prefix (reference src/decoder.cpp:213-226)?
__device__ __forceinline__ bool ngram_blocked(const DecodeParams& p, const PrefixView& pre, int v) {
    const int n = p.ngram;
    const int L = pre.len;
    if (n <= 0) return false;
    if (n == 1) {
        for (int i = 0; i < L; ++i)
            if (pre.tok[i] == v) return true;
        return false;
    }
    if (L < n - 1) return false;
    const int tail = L - (n - 1);
    for (int i = 0; i + n <= L; ++i) {
        if (pre.tok[i + n - 1] != v) continue;
        bool same = true;
        for (int j = 0; j < n - 1 && same; ++j) same = pre.tok[i + j] == pre.tok[tail + j];
        if (same) return true;
    }
    return false;
}

__device__ __forceinline__ bool in_prefix(const PrefixView& pre, int v) {
    for (int i = 0; i < pre.len; ++i)
        if (pre.tok[i] == v) return true;
    return false;
}

// Candidate of token v with log-prob lp (finite, statically allowed) in the
// row of beam k; returns false when n-gram blocking removes it. The raw score
// is p + lp, or p + (lp - log(rep)) for a token of the prefix
// (reference src/decoder.cpp:243-253).
__device__ __forceinline__ bool make_cand(const DecodeParams& p, const PrefixView& pre, float praw, float inv_pen,
                                          int k, int v, int new_len, float lp, Cand& c) {
    float value = lp;
    if (p.constrained) {
        if (ngram_blocked(p, pre, v)) return false;
        if (p.penalise && in_prefix(pre, v)) value = lp - p.log_rep;
    }
    const float raw = praw + value;
    c = Cand{raw * inv_pen, raw, k, v, new_len, 1};
    return true;
}

__device__ void bitonic_sort_cands(Cand* buf, int np) {
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
            __syncthreads();
        }
    }
}

// Sorts the collected candidates and keeps the best K; raises the admission
// threshold to the K-th kept candidate when that is better.
__device__ void compact(SelectShared& sh, SelectState& st, int K) {
    __syncthreads();
    const int n = st.count;
    int np = 1;
    while (np < n) np <<= 1;
    for (int i = n + static_cast<int>(threadIdx.x); i < np; i += kSelectThreads) sh.buf[i] = dead_cand();
    __syncthreads();
    bitonic_sort_cands(sh.buf, np);
    if (threadIdx.x == 0) {
        st.count = n < K ? n : K;
        if (st.count == K && before(sh.buf[K - 1], st.thr)) st.thr = sh.buf[K - 1];
    }
    __syncthreads();
}

// Admits c unless it ranks after the threshold. The threshold is a candidate
// that was offered earlier (or the dead sentinel); admitting an equal one
// matters after a rescan removed the threshold's own row from the buffer.
__device__ __forceinline__ void offer(SelectShared& sh, SelectState& st, const Cand& c) {
    if (before(st.thr, c)) return;
    const int slot = atomicAdd(&st.count, 1);
    sh.buf[slot] = c;
}

__device__ __forceinline__ void end_round(SelectShared& sh, SelectState& st, int K, int sort_cap) {
    __syncthreads();
    if (st.count > sort_cap - kRound) compact(sh, st, K);
}

// Full scan of row `row` (beam k) against the admission threshold.
template <int DT, bool LOGITS>
__device__ void rescan_row(const DecodeParams& p, SelectShared& sh, SelectState& st, int b, int k, int64_t row,
                           float lse, float praw, float inv_pen, int new_len, const PrefixView& pre, int sort_cap) {
    const bool mask_eos = new_len < p.min_length;
    const int V = p.V;
    for (int base = 0; base < V; base += kRound) {
        {
            const int v = base + static_cast<int>(threadIdx.x);
            if (v < V) {
                const float x = load_row_elem<DT>(p, row, v);
                const float lp = LOGITS ? x - lse : x;
                Cand c;
                if ((lp < kInf) && lp != -kInf && !static_masked(p, b, v, mask_eos)) {
                    const float raw0 = praw + lp;
                    const Cand c0{raw0 * inv_pen, raw0, k, v, new_len, 1};
                    // penalties only lower a candidate, so one ranking after the
                    // threshold unpenalised is out
                    if (!before(st.thr, c0) && make_cand(p, pre, praw, inv_pen, k, v, new_len, lp, c)) offer(sh, st, c);
                }
            }
        }
        end_round(sh, st, p.K, sort_cap);
    }
}

template <int DT, bool LOGITS>
__global__ __launch_bounds__(kSelectThreads) void select_kernel(DecodeParams p, int sort_cap) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = p.K, T = p.T;
    const int b = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);

    SelectShared sh;
    unsigned char* ptr = smem;
    sh.buf = reinterpret_cast<Cand*>(ptr);
    ptr += sizeof(Cand) * sort_cap;
    sh.raw = reinterpret_cast<float*>(ptr); ptr += 4 * K;
    sh.nraw = reinterpret_cast<float*>(ptr); ptr += 4 * K;
    sh.rbound = reinterpret_cast<float*>(ptr); ptr += 4 * K;
    sh.len = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.nlen = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.last = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.nlast = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.ended = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.nended = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.rcount = reinterpret_cast<int32_t*>(ptr); ptr += 4 * K;
    sh.plen = reinterpret_cast<int32_t*>(ptr); ptr += 8 * K;
    __shared__ SelectState st;

    const int steps_b = p.step_mode ? 1 : example_steps(p, b);
    const int T_loop = p.step_mode ? 1 : T;

    // Initial state (reference src/decoder.cpp:46-56) or the caller's (:84-103).
    for (int k = tid; k < K; k += kSelectThreads) {
        if (p.step_mode) {
            const int64_t i = static_cast<int64_t>(b) * K + k;
            sh.raw[k] = p.st_raw[i];
            sh.len[k] = p.st_len[i];
            sh.ended[k] = p.st_fin[i] != 0;
            const int L = p.st_len[i];
            sh.last[k] = (p.st_prefix && L >= 1 && L <= p.st_stride) ? p.st_prefix[i * p.st_stride + (L - 1)] : -1;
        } else {
            sh.raw[k] = k == 0 ? 0.0f : -kInf;
            sh.len[k] = 0;
            sh.ended[k] = 0;
            sh.last[k] = -1;
        }
        sh.plen[k] = 0;
        sh.plen[K + k] = 0;
    }
    if (tid == 0) st.invalid = 0;
    __syncthreads();

    int cur = 0;  // prefix buffer holding the current beams
    for (int t = 0; t < T_loop; ++t) {
        const int64_t trace0 = (static_cast<int64_t>(b) * T + t) * K;  // step mode: T == 1
        if (t >= steps_b) {
            // padding step (reference src/c_api.cpp:764-781)
            for (int k = tid; k < K; k += kSelectThreads) {
                if (p.tokens) p.tokens[trace0 + k] = -1;
                if (p.parents) p.parents[trace0 + k] = -1;
                if (p.lengths) p.lengths[trace0 + k] = 0;
                if (p.scores) p.scores[trace0 + k] = -kInf;
                if (p.raw_scores) p.raw_scores[trace0 + k] = -kInf;
                if (p.from_logprob) p.from_logprob[trace0 + k] = 0;
            }
            continue;
        }
        if (tid == 0) {
            st.count = 0;
            st.any_fail = 0;
            st.tau = -kInf;
            st.thr = dead_cand();
        }
        // Rows this step reads, their stats, and the prefilter.
        for (int k = tid; k < K; k += kSelectThreads) {
            const float praw = sh.raw[k];
            const bool live = praw < kInf && praw > -kInf;
            const bool carried = live && p.eos >= 0 && sh.ended[k];
            int cnt = -2;
            float bound = -kInf;
            if (live && !carried) {
                const RowInfo info = p.rowinfo[trace0 + k];
                if (info.invalid) atomicOr(&st.invalid, 1u);
                if (p.row_lse && LOGITS) p.row_lse[trace0 + k] = info.lse;
                cnt = (p.M > 0) ? info.count : -1;
                bound = info.bound;
            }
            sh.rcount[k] = cnt;
            sh.rbound[k] = bound;
        }
        __syncthreads();
        if (p.use_tau) {
            // The first K entries of a row's shortlist are real candidates with
            // raw >= fl(p + lp_K) (raw is monotone in lp), so at least K
            // expanded candidates reach the largest such value over the rows.
            for (int k = tid; k < K; k += kSelectThreads)
                sh.nraw[k] = sh.rcount[k] >= K ? sh.raw[k] + p.shortlist[(trace0 + k) * p.M + (K - 1)].lp : -kInf;
            __syncthreads();
            if (tid < 64) {
                float best = -kInf;
                for (int k = tid; k < K; k += 64) best = fmaxf(best, sh.nraw[k]);
                best = wave_max(best);
                if (tid == 0) st.tau = best;
            }
            __syncthreads();
        }

        // Carried-forward beams (reference src/decoder.cpp:131-139).
        for (int k = tid; k < K; k += kSelectThreads) {
            const float praw = sh.raw[k];
            const bool live = praw < kInf && praw > -kInf;
            if (live && p.eos >= 0 && sh.ended[k]) {
                const int l = sh.len[k] > 1 ? sh.len[k] : 1;
                const int32_t last = sh.last[k];
                const Cand c{praw / length_penalty(l, p.alpha), praw, k, is_eos_tok(p, last) ? last : p.eos, l, 0};
                offer(sh, st, c);
            }
        }
        end_round(sh, st, K, sort_cap);

        // Shortlist candidates.
        if (p.M > 0) {
            const int64_t total = static_cast<int64_t>(K) * p.M;
            for (int64_t base = 0; base < total; base += kRound) {
                const int64_t item = base + tid;
                if (item < total) {
                    const int k = static_cast<int>(item / p.M);
                    const int i = static_cast<int>(item % p.M);
                    if (i < sh.rcount[k]) {
                        const ShortEntry e = p.shortlist[(trace0 + k) * p.M + i];
                        const float praw = sh.raw[k];
                        if (!(praw + e.lp < st.tau)) {
                            const int new_len = sh.len[k] + 1;
                            const float inv_pen = 1.0f / length_penalty(new_len, p.alpha);
                            const PrefixView pre = prefix_of(p, sh, b, k, cur);
                            Cand c;
                            if (make_cand(p, pre, praw, inv_pen, k, e.token, new_len, e.lp, c)) offer(sh, st, c);
                        }
                    }
                }
                end_round(sh, st, K, sort_cap);
            }
        }
        compact(sh, st, K);

        // Exactness check of every shortlisted row; rows without a usable
        // shortlist (or without shortlists at all) always fail.
        for (int k = tid; k < K; k += kSelectThreads) {
            const int cnt = sh.rcount[k];
            if (cnt == -2) continue;
            bool fail = cnt < 0;
            if (!fail && sh.rbound[k] > -kInf) {
                const float X = sh.raw[k] + sh.rbound[k];
                if (X > -kInf) {
                    const float inv_pen = 1.0f / length_penalty(sh.len[k] + 1, p.alpha);
                    const float SX = X * inv_pen;
                    const Cand kth = st.count >= K ? sh.buf[K - 1] : dead_cand();
                    fail = !((kth.score > SX) || (kth.score == SX && kth.raw > X));
                }
            }
            if (fail) {
                sh.rcount[k] = -3;
                atomicOr(&st.any_fail, 1);
            }
        }
        __syncthreads();
        if (st.any_fail) {
            for (int k = 0; k < K; ++k) {
                if (sh.rcount[k] != -3) continue;
                // drop the row's shortlisted candidates, then offer the whole row
                for (int i = tid; i < st.count; i += kSelectThreads)
                    if (sh.buf[i].parent == k && sh.buf[i].flp) sh.buf[i] = dead_cand();
                __syncthreads();
                const float praw = sh.raw[k];
                const int new_len = sh.len[k] + 1;
                const float inv_pen = 1.0f / length_penalty(new_len, p.alpha);
                const float lse = LOGITS ? p.rowinfo[trace0 + k].lse : 0.0f;
                const int64_t row = p.step_mode ? static_cast<int64_t>(b) * K + k : trace0 + k;
                const PrefixView pre = prefix_of(p, sh, b, k, cur);
                rescan_row<DT, LOGITS>(p, sh, st, b, k, row, lse, praw, inv_pen, new_len, pre, sort_cap);
            }
            compact(sh, st, K);
        }

        // Selection (reference src/decoder.cpp:314-350).
        const int nsel = st.count;
        for (int k = tid; k < K; k += kSelectThreads) {
            const Cand c = k < nsel ? sh.buf[k] : dead_cand();
            const int64_t o = trace0 + k;
            if (p.tokens) p.tokens[o] = c.token;
            if (p.parents) p.parents[o] = c.parent;
            if (p.lengths) p.lengths[o] = c.length;
            if (p.scores) p.scores[o] = c.score;
            if (p.raw_scores) p.raw_scores[o] = c.raw;
            if (p.from_logprob) p.from_logprob[o] = static_cast<uint8_t>(c.flp);
            sh.nraw[k] = c.raw;
            sh.nlen[k] = c.length;
            sh.nlast[k] = c.token;
            sh.nended[k] = c.parent >= 0 ? (sh.ended[c.parent] || is_eos_tok(p, c.token)) : 0;
            if (p.constrained && !p.step_mode) {
                const int nxt = cur ^ 1;
                sh.plen[nxt * K + k] = c.parent >= 0 ? sh.plen[cur * K + c.parent] + ((c.flp && c.token >= 0) ? 1 : 0) : 0;
            }
        }
        __syncthreads();
        if (p.constrained && !p.step_mode) {
            // copy each selected beam's parent prefix, then append its token
            const int nxt = cur ^ 1;
            const int P = p.prefix_cap;
            for (int k = 0; k < K; ++k) {
                const Cand c = k < nsel ? sh.buf[k] : dead_cand();
                if (c.parent < 0) continue;
                const int L = sh.plen[cur * K + c.parent];
                const int32_t* src = p.prefix + ((static_cast<int64_t>(cur) * p.B + b) * K + c.parent) * P;
                int32_t* dst = p.prefix + ((static_cast<int64_t>(nxt) * p.B + b) * K + k) * P;
                for (int i = tid; i < L; i += kSelectThreads) dst[i] = src[i];
                if (tid == 0 && c.flp && c.token >= 0) dst[L] = c.token;
            }
            cur = nxt;
        }
        for (int k = tid; k < K; k += kSelectThreads) {
            sh.raw[k] = sh.nraw[k];
            sh.len[k] = sh.nlen[k];
            sh.last[k] = sh.nlast[k];
            sh.ended[k] = sh.nended[k];
        }
        __syncthreads();
    }

    // Final scores (reference src/decoder.cpp:179-187) and the state (step mode).
    for (int k = tid; k < K; k += kSelectThreads) {
        const int64_t i = static_cast<int64_t>(b) * K + k;
        const int l = sh.len[k] > 1 ? sh.len[k] : 1;
        if (p.final_scores) p.final_scores[i] = sh.raw[k] / length_penalty(l, p.alpha);
        if (p.final_raw) p.final_raw[i] = sh.raw[k];
        if (p.final_lengths) p.final_lengths[i] = sh.len[k];
        if (p.step_mode) {
            p.st_raw[i] = sh.raw[k];
            p.st_len[i] = sh.len[k];
            p.st_fin[i] = static_cast<uint8_t>(sh.ended[k] != 0);
        }
    }
    if (tid == 0 && p.invalid) p.invalid[b] = static_cast<uint8_t>(st.invalid != 0);
}

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

template <int DT, bool LOGITS>
hipError_t launch_typed(const DecodeParams& p, const DecodeLayout& L, hipStream_t stream, bool vec) {
    const int64_t rows = p.step_mode ? static_cast<int64_t>(p.B) * p.K : static_cast<int64_t>(p.B) * p.T * p.K;
    if (rows > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(rows));
    {
        KernelTimer timer(kKindRowPass, stream);
        if (vec) {
            hipLaunchKernelGGL((row_pass_kernel<DT, LOGITS, true>), grid, dim3(kRowThreads), 0, stream, p);
        } else {
            hipLaunchKernelGGL((row_pass_kernel<DT, LOGITS, false>), grid, dim3(kRowThreads), 0, stream, p);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (L.smem_bytes > 64 * 1024) {
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&select_kernel<DT, LOGITS>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(L.smem_bytes));
        if (e != hipSuccess) return e;
    }
    {
        KernelTimer timer(kKindSelect, stream);
        hipLaunchKernelGGL((select_kernel<DT, LOGITS>), dim3(p.B), dim3(kSelectThreads), L.smem_bytes, stream, p,
                           L.sort_cap);
    }
    return hipGetLastError();
}

}  // namespace

DecodeLayout decode_layout(int B, int T, int K, int V, bool constrained, bool step_mode, int prefix_stride) {
    DecodeLayout L{};
    // Shortlist length: K plus a margin, while the row pass can pick a
    // threshold from its 256 lane maxima; wider beams rescan every row.
    int M = K <= 64 ? ((K + 16 + 7) / 8) * 8 : 0;
    if (const char* env = getenv("DBS_HIP_SHORTLIST")) {
        // testing knob: 0 forces full rescans, a small value forces fallbacks
        const int m = atoi(env);
        if (m >= 0 && m <= 256) M = m;
    }
    L.M = M;
    L.use_tau = (!constrained && !step_mode && M > 0) ? 1 : 0;
    int sc = 1;
    while (sc < K + 2 * kRound) sc <<= 1;
    L.sort_cap = sc;
    L.smem_bytes = sizeof(Cand) * static_cast<size_t>(sc) + static_cast<size_t>(K) * 4 * 12;
    const int64_t rows = step_mode ? static_cast<int64_t>(B) * K : static_cast<int64_t>(B) * T * K;
    auto align = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    size_t off = 0;
    L.off_rowinfo = off;
    off = align(off + sizeof(RowInfo) * static_cast<size_t>(rows));
    L.off_short = off;
    off = align(off + sizeof(ShortEntry) * static_cast<size_t>(rows) * static_cast<size_t>(M));
    L.off_prefix = off;
    L.prefix_cap = step_mode ? prefix_stride : T + 1;
    if (constrained && !step_mode) off = align(off + sizeof(int32_t) * 2 * static_cast<size_t>(B) * K * (T + 1));
    L.total = off == 0 ? 256 : off;
    (void)V;
    return L;
}

hipError_t launch_decode(const DecodeParams& p, const DecodeLayout& L, hipStream_t stream) {
    const size_t esz = p.dtype == 0 ? 4 : 2;
    const bool vec = (p.V % 4 == 0) && (reinterpret_cast<uintptr_t>(p.x) % (4 * esz) == 0);
    if (p.from_logits) {
        switch (p.dtype) {
            case 0: return launch_typed<0, true>(p, L, stream, vec);
            case 1: return launch_typed<1, true>(p, L, stream, vec);
            default: return launch_typed<2, true>(p, L, stream, vec);
        }
    }
    switch (p.dtype) {
        case 0: return launch_typed<0, false>(p, L, stream, vec);
        case 1: return launch_typed<1, false>(p, L, stream, vec);
        default: return launch_typed<2, false>(p, L, stream, vec);
    }
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
